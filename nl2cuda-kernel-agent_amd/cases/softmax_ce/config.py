"""Shape parameters of the softmax cross-entropy case.

Reference defaults (cases/softmax_ce/config.py:8-10): B = SMCE_B (8192),
C = SMCE_C (1024), DTYPE = "float32" (labels are always int64).
BENCH_SHAPES are the shapes this build measures: the reference default and
a large-vocabulary shape.
"""

import os

B = int(os.environ.get("SMCE_B", "8192"))
C = int(os.environ.get("SMCE_C", "1024"))
DTYPE = "float32"

BENCH_SHAPES = ((8192, 1024), (4096, 8192))
