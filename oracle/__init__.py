"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithms of the reference's hot path
(SilenceWanna/nl2cuda-kernel-agent, cases/rbf, cases/layernorm, cases/scan,
cases/spmv) so the HIP kernels can be checked against them.  Only tests/,
__graft_entry__.smoke() and the cpu_baseline leg of bench.py may import it,
and only as the checker or the reported CPU baseline -- never as a product
path.  The package (nl2cuda-kernel-agent_amd/) never imports it.

Modules (each function cites the reference file:line it restates):
  rbf.py        float64 closed form, broadcast brute force, the reference's
                naive loops, and the op-for-op torch CPU path
  layernorm.py  float64 forward/backward and the torch CPU path
  scan.py       exact int64 / float64 prefix sums and the torch CPU path
  spmv.py       float64 CSR products, the Zipf row-length recipe, torch CPU path
  native.py     ctypes bindings of csrc/oracle.c (C restatement, built into
                oracle/lib/liboracle.so by oracle/Makefile) and of
                oracle/_ref/librbf_ref.so, which `make -C oracle ref` builds
                from the reference's own cases/rbf/delivery/rbf_test.cu
                (through ref/rbf_ref_cpu.cpp) when /root/reference exists

How each function is pinned is listed in the module docstrings; functions
without an independent pin say "parity unpinned".
"""
