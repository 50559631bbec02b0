"""BF16 skinny-GEMM ("GEMV") kernels for decode: y[M, N] = x[M, K] @ W[N, K]^T.

Drop-in for the reference's engine/kernels/gemv.py (signatures and output contracts of gemv,
gemv_m1, gemv_swiglu, gemv_m1_swiglu, gemv_rows, gemv_tma at gemv.py:137-411), computed by the
HIP kernels of libkrq.so: matrix cores (v_mfma_f32_16x16x32_bf16) for M > 1, vector ALUs with
cross-lane reductions for M == 1. split == 1 returns bf16 [M, N]; split > 1 returns the fp32
split-K partials [split, M, N], to be summed in order and rounded once by the consumer
(reference engine/kernels/ops.py:29-39). The gate/up projection computes both halves in one
pass and applies SwiGLU in the epilogue: bf16(bf16(silu(bf16 g)) * bf16 u).
"""

import torch

from . import _lib as L

_DOT_F32 = False
# The HIP kernels have one tile shape: 16 output columns x 64 bytes of K per matrix-core step.
# Kept under the reference's names (fused_gemv.py:26 and experiments/i8.py:8 import them).
_CONFIGS = [{"BN": 16, "BK": 32}]
MAX_ROWS = 32


def _bm(M):
    return max(16, 1 << (max(1, M) - 1).bit_length())


def _prune(configs, named_args, **kwargs):
    """Configs whose tile divides K_SPLIT and N; ValueError if none (reference gemv.py:34-40)."""
    ks = named_args.get("K_SPLIT", named_args.get("K"))
    n = named_args.get("N", named_args.get("I"))
    ok = [c for c in configs if ks % c["BK"] == 0 and n % c["BN"] == 0]
    if not ok:
        raise ValueError(f"no config divides K_SPLIT={ks}, N={n}")
    return ok


def pack(w):
    """Attach to the bf16 weight w [N, K] (N % 16 == 0, K % 32 == 0) a copy in the tiled layout
    the kernels stream fastest (w.krq_tiled); later gemv*/lm-head calls on w read it. Returns w.
    The reference has no counterpart: it is the load-time packing step for bf16 weights (the
    tied lm_head), like the tiled copy fp8.quantize makes for FP8 weights."""
    L.require_device(w)
    if w.dtype != torch.bfloat16 or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("pack expects a contiguous bf16 [N, K] tensor")
    N, K = w.shape
    t = torch.empty((N * K * 2,), device=w.device, dtype=torch.uint8)
    L.call("krq_pack_fp8", L.ptr(w), N, 2 * K, L.ptr(t), L.stream(w))
    w.krq_tiled = t
    w.krq_tiled_version = w._version
    return w


def _weight(w):
    """(pointer tensor, layout) of the bf16 weight the kernels read: the tiled copy pack() made,
    unless w has been modified in place since (its version counter moved), in which case the copy
    is dropped and w itself is read."""
    t = getattr(w, "krq_tiled", None)
    if t is not None:
        if getattr(w, "krq_tiled_version", None) == w._version:
            return t, L.W_TILED
        w.krq_tiled = None
    return (w if w.is_contiguous() else w.contiguous()), L.W_ROWMAJOR


def _launch(x, w, split, mode):
    L.require_device(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("gemv expects bf16 x and w")
    x = x.contiguous()
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"x [{M}, {K}] and w {tuple(w.shape)} do not match")
    w, layout = _weight(w)

    def one(xc):
        m = xc.shape[0]
        if mode == L.OUT_PARTIAL:
            out = torch.empty((split, m, N), device=x.device, dtype=torch.float32)
        else:
            out = torch.empty((m, N // 2 if mode == L.OUT_SWIGLU else N), device=x.device,
                              dtype=torch.bfloat16)
        L.call("krq_gemv_bf16", L.ptr(xc), L.ptr(w), layout, m, N, K, split, mode, L.ptr(out), L.stream(x))
        return out

    if M <= MAX_ROWS:
        return one(x)
    return torch.cat([one(x[m0:m0 + MAX_ROWS]) for m0 in range(0, M, MAX_ROWS)], dim=-2)


def gemv(x, w, split=1):
    """x [M, K] bf16, w [N, K] bf16. split == 1: returns bf16 [M, N].
    split > 1: returns fp32 partials [split, M, N] (sum them, then round)."""
    M, K = x.shape
    assert K % split == 0
    return _launch(x, w, split, L.OUT_BF16 if split == 1 else L.OUT_PARTIAL)


def gemv_swiglu(x, w_gu):
    """x [M, K], w_gu [2I, K] = [gate; up] -> bf16(silu(gate) * up) [M, I]."""
    return _launch(x, w_gu, 1, L.OUT_SWIGLU)


def gemv_m1(x, w, split=1):
    """Same contract as gemv() for a single row."""
    M, K = x.shape
    assert M == 1 and K % split == 0
    return _launch(x, w, split, L.OUT_BF16 if split == 1 else L.OUT_PARTIAL)


def gemv_m1_swiglu(x, w_gu):
    M, K = x.shape
    assert M == 1
    return _launch(x, w_gu, 1, L.OUT_SWIGLU)


def gemv_rows(x, w, programs, swiglu=False, bn=16, bk=256, num_warps=4):
    """Persistent GEMV over `programs` programs (reference gemv.py:334-348); bf16 [M, N] out
    (N = I and SwiGLU applied if swiglu, with w = [gate; up]). Workgroup p of exactly `programs`
    owns output rows [p N / programs, (p + 1) N / programs) over the full K, in 16-row chunks
    (the reference's bn default). bn, bk and num_warps are the Triton kernel's tile sizes and warp
    count; the HIP kernel sizes its waves from the rows a workgroup owns, so they are accepted for
    the signature and change nothing. Every output row is summed by one wave in one order: the
    result is the same for every `programs`. Reads the row-major bf16 w (not a packed copy)."""
    L.require_device(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("gemv_rows expects bf16 x and w")
    x = x.contiguous()
    w = w if w.is_contiguous() else w.contiguous()
    M, K = x.shape
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"x [{M}, {K}] and w {tuple(w.shape)} do not match")
    if swiglu and w.shape[0] % 2:
        raise ValueError("gemv_rows(swiglu=True) expects w = [gate; up] with an even row count")
    N = w.shape[0] // 2 if swiglu else w.shape[0]
    programs = int(programs)

    def one(xc):
        out = torch.empty((xc.shape[0], N), device=x.device, dtype=torch.bfloat16)
        L.call("krq_gemv_bf16_rows", L.ptr(xc), L.ptr(w), xc.shape[0], N, K, programs, int(bool(swiglu)),
               L.ptr(out), L.stream(x))
        return out

    if M <= MAX_ROWS:
        return one(x)
    return torch.cat([one(x[m0:m0 + MAX_ROWS]) for m0 in range(0, M, MAX_ROWS)], dim=0)


def gemv_tma(x, w, split=1):
    """Hopper TMA descriptor GEMV in the reference (gemv.py:398-411). CDNA4 has no tensor
    memory accelerator; like the reference on an untileable shape, this raises ValueError, which
    the engine's candidate loop records as unavailable (engine/engine.py:898-899)."""
    raise ValueError("gemv_tma: TMA descriptors are a Hopper feature; not available on gfx950")
