"""Shape parameters of the cosine-similarity case.

Reference defaults (cases/cosine_sim/config.py:5-8): N = COS_N (2048),
M = COS_M (2048), D = COS_D (64), DTYPE = "float32"; eps = 1e-8 is the case
parameter (cases/cosine_sim/__init__.py:16-24).  BENCH_SIZES are the square
sizes this build measures (the reference default and the RBF acceptance
size, which shares the tile engine).
"""

import os

N = int(os.environ.get("COS_N", "2048"))
M = int(os.environ.get("COS_M", "2048"))
D = int(os.environ.get("COS_D", "64"))
DTYPE = "float32"
EPS = 1e-8

BENCH_SIZES = (2048, 4096)
