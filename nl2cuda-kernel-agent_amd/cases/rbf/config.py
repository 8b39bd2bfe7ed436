"""Shape and scalar parameters of the RBF case.

Reference defaults (cases/rbf/config.py:11-17): N = M = RBF_SIZE (2048),
D = 64, GAMMA = 1/64, DTYPE = "float32".  Added knobs: RBF_D, RBF_GAMMA and
RBF_INPUT_SCALE (the standard deviation of X and Y); the acceptance
workloads of this build use gamma = 0.5 and scale 1/sqrt(64)
(BASELINE_GAMMA / BASELINE_SCALE below).
"""

import os

_SIZE = int(os.environ.get("RBF_SIZE", "2048"))

N = _SIZE
M = _SIZE
D = int(os.environ.get("RBF_D", "64"))
GAMMA = float(os.environ.get("RBF_GAMMA", str(1.0 / 64.0)))
INPUT_SCALE = float(os.environ.get("RBF_INPUT_SCALE", "1.0"))
DTYPE = "float32"

BASELINE_GAMMA = 0.5
BASELINE_SCALE = 1.0 / 8.0
BASELINE_SIZES = (2048, 4096, 8192)
