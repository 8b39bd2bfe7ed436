"""Shape parameters of the scan case.

Reference defaults (cases/scan/config.py:4-6): B = SCAN_B (4096), D = 4096,
DTYPE = "float32".  This build also reads SCAN_D (the reference kernel only
handles D == 4096; this one handles any D >= 1) and SCAN_DIST, the input
distribution: "reference" (N(0,1), reference.py:12-22) or "baseline"
(U(-1, 1), the acceptance workload).  BASELINE_* are the acceptance shapes:
x [64, 65536] fp32, and int32 ~ U[-1000, 1000] (forward only, bit-exact).
"""

import os

B = int(os.environ.get("SCAN_B", "4096"))
D = int(os.environ.get("SCAN_D", "4096"))
DTYPE = "float32"
DIST = os.environ.get("SCAN_DIST", "reference")

BASELINE_B = 64
BASELINE_D = 65536
INT_LOW, INT_HIGH = -1000, 1000
