"""Shape and scalar parameters of the LayerNorm case.

Reference defaults (cases/layernorm/config.py:9-12): B = LN_B (4096),
D = LN_D (1024), EPS = 1e-5, DTYPE = "float32".  LN_PARAMS selects the
distribution of gamma / beta: "reference" (N(0,1), reference.py:28-29) or
"baseline" (gamma = 1 + 0.1 N(0,1), beta = 0.1 N(0,1), this build's
acceptance workload).
"""

import os

B = int(os.environ.get("LN_B", "4096"))
D = int(os.environ.get("LN_D", "1024"))
EPS = 1e-5
DTYPE = "float32"
PARAMS = os.environ.get("LN_PARAMS", "reference")

BASELINE_B = 8192
BASELINE_D = 4096
