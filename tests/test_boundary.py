"""Host-side checks of the drop-in boundary that need no GPU: the C-ABI library loads and exports
every symbol include/krq.h declares, argument validation maps to the reference's exception
types, and nothing silently runs on the CPU."""

import ctypes
import os
import re

import pytest
import torch

from kernels import _lib as L
from kernels import fp8, gemv as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "krq.h")).read()
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(krq_\w+)\s*\(", text, re.M))


def test_library_exports_every_header_symbol():
    lib = L.lib()
    declared = header_symbols()
    assert declared == set(L.EXPORTS), declared ^ set(L.EXPORTS)
    for name in declared:
        assert hasattr(lib, name)
    assert lib.krq_version().decode().startswith("krq")
    # the per-block stamps exist only in the timeline build (build_lib.py --timeline)
    assert not hasattr(lib, "krq_timeline_read")


def test_workspace_sizes_are_host_only():
    lib = L.lib()
    assert lib.krq_lmhead_ws_bytes(16, 151936) >= 256 + 16 * 8 * (151936 // 64)
    assert lib.krq_act_scale_ws_floats(16, 2560) >= 1


def _null():
    return ctypes.c_void_p(0)


def test_invalid_arguments_fail_before_any_launch():
    lib = L.lib()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation rejects the call first
    # M out of range
    rc = lib.krq_gemv_fp8(p, 0, p, None, 0, p, 1, p, 1, 0, 64, 256, 1, 0, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"M=0" in lib.krq_last_error()
    # K/split not a multiple of 64
    rc = lib.krq_gemv_fp8(p, 0, p, None, 0, p, 1, p, 1, 1, 64, 200, 1, 0, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"K_SPLIT" in lib.krq_last_error()
    # in-kernel per-token scaling takes one row; static scaling needs x_inv
    rc = lib.krq_gemv_fp8(p, 1, None, None, 0, p, 1, p, 1, 2, 64, 256, 1, 0, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"M == 1" in lib.krq_last_error()
    rc = lib.krq_gemv_fp8(p, 2, p, None, 0, p, 1, p, 1, 2, 64, 256, 1, 0, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"x_inv" in lib.krq_last_error()
    # split > 1 without the partials output
    rc = lib.krq_gemv_bf16(p, p, 0, 1, 64, 256, 2, 0, p, _null())
    assert rc == L.KRQ_EINVAL
    # persistent BF16 GEMV: at least one program, whole 32-element K tiles
    rc = lib.krq_gemv_bf16_rows(p, p, 1, 64, 256, 0, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"programs=0" in lib.krq_last_error()
    rc = lib.krq_gemv_bf16_rows(p, p, 1, 64, 200, 4, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"multiple of 32" in lib.krq_last_error()
    # tiled activations take the matrix-core kernel; their quantizer needs K % 64 == 0
    rc = lib.krq_gemv_fp8(p, L.X_FP8_TILED, p, None, 0, p, 1, p, 1, 1, 64, 256, 1, 0, 2, p, _null())
    assert rc == L.KRQ_EINVAL and b"tiled activations" in lib.krq_last_error()
    # the activation scale with its cast: every pointer, a real shape
    rc = lib.krq_act_scale_cast_fp8(p, 16, 2560, 1.0, p, p, p, None, p, _null())
    assert rc == L.KRQ_EINVAL and b"null pointer" in lib.krq_last_error()
    rc = lib.krq_act_scale_cast_fp8(p, 0, 2560, 1.0, p, p, p, p, p, _null())
    assert rc == L.KRQ_EINVAL and b"bad shape" in lib.krq_last_error()
    rc = lib.krq_quant_rows_tiled(p, 16, 100, p, p, _null())
    assert rc == L.KRQ_EINVAL and b"K=100" in lib.krq_last_error()
    rc = lib.krq_quant_rows_tiled(p, 16, 16384 + 64, p, p, _null())
    assert rc == L.KRQ_EINVAL and b"K at most 16384" in lib.krq_last_error()
    rc = lib.krq_rmsnorm_quant_rows_tiled(p, p, p, 1e-6, 2, 2576, p, p, _null())
    assert rc == L.KRQ_EINVAL and b"multiple of 64" in lib.krq_last_error()
    # the tiled e4m3 lm_head rows need their per-row scales
    rc = lib.krq_lmhead_argmax(p, None, 1, p, L.LM_FP8_TILED_H, 1, p, 1, 16, 1024, 256, None, p, 1 << 20, p,
                               _null())
    assert rc == L.KRQ_EINVAL and b"h_scale" in lib.krq_last_error()
    # the allocation-free lm_head: its argument checks, then its scratch limit, before any HIP call
    rc = lib.krq_lmhead_argmax_noalloc(p, None, 1, p, L.LM_FP8_TILED_H, 1, p, 1, 16, 1024, 256, None, p,
                                       _null())
    assert rc == L.KRQ_EINVAL and b"h_scale" in lib.krq_last_error()
    assert lib.krq_lmhead_ws_bytes(32, 262144) == L.LMHEAD_SCRATCH_BYTES
    rc = lib.krq_lmhead_argmax_noalloc(p, p, 1, p, L.LM_FP8, 1, p, 1, 32, 262144 + 16, 2560, None, p, _null())
    assert rc == L.KRQ_EINVAL and b"scratch maximum of 4194304" in lib.krq_last_error()
    # null pointers
    rc = lib.krq_quant_fp8_rows(None, 16, 64, 64, p, None, p, _null())
    assert rc == L.KRQ_EINVAL
    # workspace too small
    rc = lib.krq_lmhead_argmax(p, None, 0, p, 0, 0, None, 0, 1, 1024, 256, None, p, 8, p, _null())
    assert rc == L.KRQ_EINVAL and b"workspace" in lib.krq_last_error()
    with pytest.raises(ValueError):
        L.call("krq_pack_fp8", p, 17, 64, p, _null())
    # fused MLP: one-row in-kernel scaling only; staging limit
    rc = lib.krq_mlp_fp8(p, 1, None, p, 1, p, 1, p, p, 1, 2, 2560, 9728, 4, p, p, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"M == 1" in lib.krq_last_error()
    rc = lib.krq_mlp_fp8(p, 0, p, p, 1, p, 1, p, p, 1, 32, 2560, 9728, 1, p, p, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"raise split" in lib.krq_last_error()
    # fused BF16 GEMV: residual epilogue needs its buffers; slices that do not fit are refused
    rc = lib.krq_gemv_bf16_fused(p, p, 0, 1, 2560, 4096, 4, L.OUT_RESIDUAL, None, None, 1e-6,
                                 None, None, None, None, p, _null())
    assert rc == L.KRQ_EINVAL and b"res_in" in lib.krq_last_error()
    rc = lib.krq_gemv_bf16_fused(p, p, 0, 16, 19456, 2560, 1, L.OUT_SWIGLU, p, p, 1e-6,
                                 None, None, None, None, p, _null())
    assert rc == L.KRQ_EINVAL and b"krq_rmsnorm_rows" in lib.krq_last_error()
    assert lib.krq_gemv_fused_fits(1, 6144, 2560, 2, L.OUT_PARTIAL, 1) == 1
    assert lib.krq_gemv_fused_fits(16, 19456, 2560, 1, L.OUT_SWIGLU, 1) == 0
    # fused FP8 GEMV: something to fuse; RMSNorm needs bf16 activations; per-token in-kernel
    # scaling takes one row; the residual epilogue needs its buffers
    args = (p, 1, None, None, 0, p, 1, p, 1)
    rc = lib.krq_gemv_fp8_fused(*args, 1, 6144, 2560, 2, L.OUT_PARTIAL, None, None, 1e-6, None, None, None,
                                None, p, _null())
    assert rc == L.KRQ_EINVAL and b"krq_gemv_fp8" in lib.krq_last_error()
    rc = lib.krq_gemv_fp8_fused(p, 0, p, None, 0, p, 1, p, 1, 1, 6144, 2560, 2, L.OUT_PARTIAL, p, p, 1e-6,
                                None, None, None, None, p, _null())
    assert rc == L.KRQ_EINVAL and b"bf16 activations" in lib.krq_last_error()
    rc = lib.krq_gemv_fp8_fused(*args, 2, 6144, 2560, 2, L.OUT_PARTIAL, p, p, 1e-6, None, None, None,
                                None, p, _null())
    assert rc == L.KRQ_EINVAL and b"M == 1" in lib.krq_last_error()
    # (split 2: at M = 1 the four-split residual runs folded and needs no counters)
    rc = lib.krq_gemv_fp8_fused(*args, 1, 2560, 4096, 2, L.OUT_RESIDUAL, None, None, 1e-6, p, p, p, None,
                                p, _null())
    assert rc == L.KRQ_EINVAL and b"cnt" in lib.krq_last_error()
    rc = lib.krq_gemv_fp8_fused(*args, 1, 2560, 4096, 4, L.OUT_RESIDUAL, p, p, 1e-6, p, p, p, p, p, _null())
    assert rc == L.KRQ_EINVAL and b"in one call" in lib.krq_last_error()
    assert lib.krq_gemv_fp8_fused_fits(1, 6144, 2560, 2, L.OUT_PARTIAL, L.X_BF16_DYN, 1) == 1
    assert lib.krq_gemv_fp8_fused_fits(16, 6144, 2560, 2, L.OUT_PARTIAL, L.X_BF16_DYN, 1) == 0
    assert lib.krq_gemv_fp8_fused_fits(4, 6144, 2560, 2, L.OUT_PARTIAL, L.X_BF16_STATIC, 1) == 1
    assert lib.krq_gemv_fp8_fused_fits(16, 6144, 2560, 2, L.OUT_PARTIAL, L.X_BF16_STATIC, 1) == 0
    assert lib.krq_gemv_fp8_fused_fits(32, 19456, 2560, 1, L.OUT_SWIGLU, L.X_BF16_STATIC, 1) == 0
    assert lib.krq_gemv_fp8_fused_fits(1, 2560, 9728, 4, L.OUT_RESIDUAL, L.X_FP8, 0) == 1
    rc = lib.krq_rmsnorm_quant_rows(p, p, p, 1e-6, 1, 16384 + 16, p, p, _null())
    assert rc == L.KRQ_EINVAL and b"at most 16384" in lib.krq_last_error()
    rc = lib.krq_rmsnorm_rows(p, p, p, 1e-6, 1, 20000, p, _null())
    assert rc == L.KRQ_EINVAL and b"at most 16384" in lib.krq_last_error()
    # prefill GEMM: N and K multiples of 128; bf16 activations need their inverse scale
    rc = lib.krq_gemm_fp8(p, L.X_FP8, p, None, 0, p, p, 1, 256, 200, 256, p, _null())
    assert rc == L.KRQ_EINVAL and b"multiples of 128" in lib.krq_last_error()
    rc = lib.krq_gemm_fp8(p, L.X_BF16_STATIC, p, None, 0, p, p, 1, 256, 256, 256, p, _null())
    assert rc == L.KRQ_EINVAL and b"x_inv" in lib.krq_last_error()
    rc = lib.krq_gemm_fp8(p, L.X_BF16_DYN, p, p, 0, p, p, 1, 256, 256, 256, p, _null())
    assert rc == L.KRQ_EINVAL and b"x_kind" in lib.krq_last_error()
    # the workspace form: the same checks, and a size that disagrees with its pointer is refused;
    # no split (0 bytes) where the ring kernels do not run (bf16 activations, K below 256)
    rc = lib.krq_gemm_fp8_ws(p, L.X_FP8, p, None, 0, p, p, 1, 256, 200, 256, p, 0, p, _null())
    assert rc == L.KRQ_EINVAL and b"multiples of 128" in lib.krq_last_error()
    rc = lib.krq_gemm_fp8_ws(p, L.X_FP8, p, None, 0, p, p, 1, 256, 256, 256, None, 1024, p, _null())
    assert rc == L.KRQ_EINVAL and b"workspace" in lib.krq_last_error()
    rc = lib.krq_gemm_fp8_ws(p, L.X_FP8, p, None, 0, p, p, 1, 256, 256, 256, p, -1, p, _null())
    assert rc == L.KRQ_EINVAL and b"workspace" in lib.krq_last_error()
    assert lib.krq_gemm_fp8_ws_bytes(L.X_BF16_STATIC, 256, 2560, 9728) == 0
    assert lib.krq_gemm_fp8_ws_bytes(L.X_FP8, 256, 2560, 128) == 0
    assert lib.krq_gemm_fp8_ws_bytes(L.X_FP8, 256, 200, 9728) == 0


def test_fused_buffers_and_mlp_contracts():
    from kernels.fused_gemv import FusedLayerBuffers
    from kernels.mlp import PersistentMLP
    b = FusedLayerBuffers(4, 2560, 151936, "cpu")
    assert b.res.shape == (2, 4, 2560) and b.res.dtype == torch.bfloat16
    assert b.ss.shape == (2, 4, 160) and b.cnt.shape == (151936 // 8,)
    pm = PersistentMLP(1, 2560, 9728, "cpu")
    assert pm.ctl.numel() == L.lib().krq_mlp_ctl_words() and int(pm.ctl.abs().sum()) == 0
    with pytest.raises(AssertionError):
        PersistentMLP(1, 2560, 9728 + 16, "cpu")          # the reference's chunk contract
    with pytest.raises(ValueError):
        pm(torch.zeros(1, 2560, dtype=torch.bfloat16), torch.zeros(1), torch.zeros(1))


def test_no_cpu_path():
    w = torch.zeros(16, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fp8.quantize(w)
    with pytest.raises(RuntimeError, match="ROCm device"):
        G.gemv(torch.zeros(1, 64, dtype=torch.bfloat16), w)


def test_reference_helpers():
    assert G._bm(1) == 16 and G._bm(16) == 16 and G._bm(17) == 32 and G._bm(32) == 32
    with pytest.raises(ValueError):
        G._prune(G._CONFIGS, {"K_SPLIT": 48, "N": 64})
    assert G._prune(G._CONFIGS, {"K": 64, "N": 32})
    with pytest.raises(ValueError):
        G.gemv_tma(torch.zeros(1, 64), torch.zeros(64, 64))
    with pytest.raises(AssertionError):
        G.gemv_m1(torch.zeros(2, 64, dtype=torch.bfloat16), torch.zeros(16, 64, dtype=torch.bfloat16))
    assert fp8.FP8_MAX == 448.0
    q = fp8.FP8Weight(torch.zeros(1), torch.ones(()), None)
    w8, s = q
    assert isinstance(q, tuple) and q.tiled is None and s.item() == 1.0


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with a message before touching a device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_fused_and_gemm_wrappers_refuse_cpu_tensors():
    from kernels import fused_gemv as FG
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    w = torch.zeros(32, 256, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        FG.gemv_fused(x, w, 1)
    q = fp8.FP8Weight(torch.zeros(128, 256, dtype=torch.float8_e4m3fn), torch.ones(()), None)
    with pytest.raises(RuntimeError, match="ROCm device"):
        FG.gemv_fused(x, q, 1, ep=(x, x, x, x))
    with pytest.raises(RuntimeError, match="ROCm device"):
        fp8.gemm_fp8(torch.zeros(64, 256, dtype=torch.float8_e4m3fn), q, xs=torch.ones(1))
