"""Shape parameters of the L2-norm-scale case.

Reference defaults (cases/l2norm_scale/config.py:4-8): N = L2N_N (16384),
D = L2N_D (1024), EPS = L2N_EPS (1e-6), DTYPE = "float32".  BENCH_SHAPES
are the shapes this build measures: the reference default and the
LayerNorm acceptance shape (the two cases share their kernels).
"""

import os

N = int(os.environ.get("L2N_N", "16384"))
D = int(os.environ.get("L2N_D", "1024"))
EPS = float(os.environ.get("L2N_EPS", "1e-6"))
DTYPE = "float32"

BENCH_SHAPES = ((16384, 1024), (8192, 4096))
