"""Drop-in replacement for the reference engine's `kernels` package, decode-matmul path only.

Put the directory holding this package on sys.path, as the reference puts engine/ there, and
import the modules the engine imports (reference engine/engine.py:57-58):

    from kernels import fp8
    from kernels.gemv import gemv, gemv_m1, gemv_swiglu, gemv_m1_swiglu, gemv_rows, gemv_tma

The compute runs in libkrq.so (hand-written gfx950 HIP kernels behind the C ABI of
include/krq.h); these modules keep the reference's Python signatures, output contracts and
exception types.
"""
