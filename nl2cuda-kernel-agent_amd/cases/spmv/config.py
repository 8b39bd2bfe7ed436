"""Shape parameters of the CSR SpMM / SpMV case.

Reference defaults (cases/spmv/config.py:6-10): M = SPMV_M (4096), K =
SPMV_K (4096), D = SPMV_D (64), NNZ_PER_ROW = SPMV_NNZ_PER_ROW (64), DTYPE =
"float32", int64 indices, columns drawn with replacement (reference.py:26-51).

BASELINE_* is this build's acceptance workload: A 2^20 x 2^20, int32
row_ptr / col_idx, power-law row lengths (Zipf s = 1.5 clipped to
[1, 4096], rescaled to mean 16, total nnz exactly 16 * 2^20; recipe in
reference.zipf_row_lengths), per-row sorted unique columns ~ U[0, K), fp32
vals / x / dy ~ N(0, 1), D = 1.
"""

import os

M = int(os.environ.get("SPMV_M", "4096"))
K = int(os.environ.get("SPMV_K", "4096"))
D = int(os.environ.get("SPMV_D", "64"))
NNZ_PER_ROW = int(os.environ.get("SPMV_NNZ_PER_ROW", "64"))
DTYPE = "float32"

BASELINE_M = BASELINE_K = 1 << 20
BASELINE_D = 1
BASELINE_MEAN = 16
ZIPF_S = 1.5
MAX_ROW = 4096
