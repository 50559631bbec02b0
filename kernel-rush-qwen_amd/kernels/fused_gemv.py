"""Decode GEMVs with the residual add and RMSNorm folded in (HIP kernel k_gemv_fused of libkrq.so),
so a decoder layer is four GEMV launches plus attention.

Drop-in for the reference's engine/kernels/fused_gemv.py - FusedLayerBuffers(M, H, n_max, device),
gemv_fused(x, w, split, *, norm, zero_ss, ep, eps), gemv_swiglu_fused(x, w_gu, *, norm, zero_ss,
eps) - as the engine calls them (engine/engine.py:209, :940-962), with the same rounding points:
  norm=(ln_w, ss):  x rows are normalized on the fly, h = bf16(bf16(x * rstd) * ln_w) with
                    rstd = rsqrt(ss / K + eps) (Qwen3RMSNorm);
  ep=(res_in, res_out, ss_out, cnt):
                    y = bf16(x @ w^T, split partials summed in split order),
                    res_out = bf16(res_in + y), ss_out <- sums of squares of res_out; returns None.

The sums of squares are kept the MI355X way: ss is [M, K/16], one partial per 16-column tile of the
producer, summed in a fixed order by the consumer, where the reference accumulates an [M] vector
with atomic adds (same-address device atomics serialize on MI355X). FusedLayerBuffers allocates ss
in that shape; the engine only hands ss[0] / ss[1] back to these functions. Every producer
overwrites all of its tiles, so zero_ss (the reference's reset of the next accumulator) is
accepted and has nothing to do. At M = 1 the normalizing kernels hold the whole row and sum its
squares themselves, so ss is neither read there nor needed from the producer: the FP8 residual
GEMVs at M = 1 run folded (N / 4 workgroups, each four output columns over the four quarters of K,
the four-split sums bit for bit without a cross-workgroup reduction) and write no ss.

When a block's normalized K slice does not fit the kernel's LDS staging (large M x K/split), the
rows are normalized by krq_rmsnorm_rows first and the GEMV runs on the result: two launches, same
arithmetic.

FP8 weights (an FP8Weight from kernels.fp8.quantize / quantize_weight, as the reference's FP8 engine
holds them) take the FP8 form of the same kernels (krq_gemv_fp8_fused): the normalized rows are
scaled and quantized in the prologue - per token over the normalized row at M = 1, or with the
static inverse scale of a SharedScale / ActScale `a` at any M - and the residual epilogue sums the
scaled split partials. Rows the prologue cannot stage (M > 1 with per-token scales) go through
krq_rmsnorm_quant_rows first (the values of quant_rows(rmsnorm(x))).
"""

import torch

from . import _lib as L
from . import fp8 as _fp8
from . import gemv as _gemv

MAX_ROWS = 32
# K splits the residual epilogue runs with (None: the caller's split). Its output has no split
# partials, so the decomposition is free; on MI355X one K pass with four waves per block costs at
# most ~0.8 us more than split 4 (O: the same), while the split-K last-arriver reduction costs
# three memory round trips (~3 us) at the tail of the launch.
EP_SPLIT = 1
# FP8 weights at M = 1: the residual epilogue runs with four splits, folded into N / 4 workgroups
# (krq_gemv_fp8_fused; no split partials, no counters); 0: EP_SPLIT as at M > 1.
FOLD_SPLIT = 4


class FusedLayerBuffers:
    """Residual ping-pong rows, per-tile sum-of-squares partials and split-K counters for one M."""

    def __init__(self, M, H, n_max, device):
        self.res = torch.zeros((2, M, H), device=device, dtype=torch.bfloat16)
        self.ss = torch.zeros((2, M, H // 16), device=device, dtype=torch.float32)
        self.cnt = torch.zeros((n_max // 8,), device=device, dtype=torch.int32)


def _check(x, w):
    L.require_device(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("fused GEMVs expect bf16 x and w")
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(w.shape)} do not match")
    if x.shape[0] > MAX_ROWS:
        raise ValueError(f"fused GEMVs take at most {MAX_ROWS} rows, got {x.shape[0]}")


def _norm_args(x, N, norm, mode, split):
    """(x, ln, ss) for the launch: the RMSNorm in the kernel when its slice fits, else rows
    normalized by a separate launch and no norm in the GEMV."""
    if norm is None:
        return x, None, None
    ln, ss = _check_norm(x, norm)
    M, K = x.shape
    if L.lib().krq_gemv_fused_fits(M, N, K, split, mode, 1):
        return x, ln, ss
    return None, ln, ss


def _rmsnorm(x, ln, ss, eps):
    h = torch.empty_like(x)
    L.call("krq_rmsnorm_rows", L.ptr(x), L.ptr(ss), L.ptr(ln), eps, x.shape[0], x.shape[1], L.ptr(h), L.stream(x))
    return h


def _launch(x, w, split, mode, norm, ep, eps, out):
    M, K = x.shape
    N = w.shape[0]
    xin, ln, ss = _norm_args(x, N, norm, mode, split)
    if xin is None:  # normalize first, then the plain fused launch
        xin, ln, ss = _rmsnorm(x, ln, ss, eps), None, None
    wt, layout = _gemv._weight(w)
    res_in = res_out = ss_out = cnt = None
    if ep is not None:
        res_in, res_out, ss_out, cnt = _check_ep(ep, M, N, split)
    L.call("krq_gemv_bf16_fused", L.ptr(xin), L.ptr(wt), layout, M, N, K, split, mode, L.ptr(ln), L.ptr(ss),
           float(eps), L.ptr(res_in), L.ptr(res_out), L.ptr(ss_out), L.ptr(cnt), L.ptr(out), L.stream(x))
    return out


def _is_fp8(w):
    return isinstance(w, tuple) and len(w) >= 2 and w[0].dtype == torch.float8_e4m3fn


def _check_ep(ep, M, N, split):
    res_in, res_out, ss_out, cnt = ep
    L.require_device(res_in, res_out, ss_out, cnt)
    if ss_out.numel() != M * (N // 16) or res_in.numel() != M * N or res_out.numel() != M * N:
        raise ValueError("ep=(res_in [M, N], res_out [M, N], ss_out [M, N/16], cnt) from FusedLayerBuffers")
    if split > 1 and cnt.numel() < N // 16:
        raise ValueError(f"cnt holds {cnt.numel()} counters, needs {N // 16}")
    return ep


def _check_norm(x, norm):
    ln, ss = norm
    M, K = x.shape
    L.require_device(ln, ss)
    if ln.dtype != torch.bfloat16 or ln.numel() != K or ss.dtype != torch.float32 or ss.numel() != M * (K // 16):
        raise ValueError("norm=(ln [K] bf16, ss [M, K/16] fp32 from FusedLayerBuffers.ss)")
    return ln, ss


def _launch_fp8(x, q, split, mode, norm, ep, eps, a, out):
    """One krq_gemv_fp8_fused launch, or the two-launch forms when the prologue cannot stage x."""
    w, layout, ws, (N, K) = _fp8._weight_operand(q)
    M = x.shape[0]
    wpr = 1 if ws.numel() > 1 else 0
    if norm is not None and ep is not None:
        raise ValueError("FP8 fused GEMVs take the RMSNorm prologue or the residual epilogue, not both")
    ln = ss = None
    if norm is not None:
        ln, ss = _check_norm(x, norm)
    res_in = res_out = ss_out = cnt = None
    if ep is not None:
        res_in, res_out, ss_out, cnt = _check_ep(ep, M, N, split)
    fits = L.lib().krq_gemv_fp8_fused_fits
    kind = L.X_BF16_STATIC if a is not None else L.X_BF16_DYN
    if not fits(M, N, K, split, mode, kind, 1 if norm is not None else 0):
        # stage outside: normalize (and quantize) the rows first, then e4m3 activations, row-major
        # or (from fp8.TILED_MIN_ROWS rows) in the tiled activation layout, as fp8's GEMVs choose
        tiled = K % 64 == 0 and K <= _fp8.TILED_ROWS_MAX_K and M >= _fp8.TILED_MIN_ROWS
        if norm is not None:
            if tiled and a is None:
                x8 = torch.empty(((M + 15) // 16 * 16 * K,), device=x.device, dtype=torch.uint8)
                xs = torch.empty((M,), device=x.device, dtype=torch.float32)
                L.call("krq_rmsnorm_quant_rows_tiled", L.ptr(x), L.ptr(ss), L.ptr(ln), float(eps), M, K,
                       L.ptr(x8), L.ptr(xs), L.stream(x))
                return _fp8.gemv_fp8_tiled_launch(x8, xs, q, M, split, mode, out)
            if tiled:
                x8t = _fp8.cast_tiled(_rmsnorm(x, ln, ss, eps), a)
                return _fp8.gemv_fp8_tiled_launch(x8t, a.scale.reshape(1), q, M, split, mode, out)
            if a is None:
                x8 = torch.empty((M, K), device=x.device, dtype=torch.float8_e4m3fn)
                xs = torch.empty((M,), device=x.device, dtype=torch.float32)
                L.call("krq_rmsnorm_quant_rows", L.ptr(x), L.ptr(ss), L.ptr(ln), float(eps), M, K, L.ptr(x8),
                       L.ptr(xs), L.stream(x))
            else:
                x8, xs = _fp8._cast(_rmsnorm(x, ln, ss, eps), a), a.scale.reshape(1)
            return _fp8.gemv_fp8_launch(x8, xs, q, split, mode, L.ALGO_MFMA, out)
        if tiled:
            x8, xs = _fp8._tiled_operand(x, a)
            kind, xin, x_scale, x_inv = L.X_FP8_TILED, x8, xs.reshape(-1), None
        else:
            x8, xs = _fp8._activation_fp8(x, a, None)
            kind, xin, x_scale, x_inv = L.X_FP8, x8, xs, None
    elif a is not None:
        xin, x_scale, x_inv = x, a.scale.reshape(1), a.inv.reshape(1)
    else:
        xin, x_scale, x_inv = x, None, None
    xpr = 1 if (x_scale is not None and x_scale.numel() == M and M > 1) else 0
    L.require_device(x_scale, x_inv)
    L.call("krq_gemv_fp8_fused", L.ptr(xin), kind, L.ptr(x_scale), L.ptr(x_inv), xpr, L.ptr(w), layout, L.ptr(ws),
           wpr, M, N, K, split, mode, L.ptr(ln), L.ptr(ss), float(eps), L.ptr(res_in), L.ptr(res_out),
           L.ptr(ss_out), L.ptr(cnt), L.ptr(out), L.stream(x))
    return out


def _fp8_fused(x, q, split, mode, norm, ep, eps, a):
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError("fused FP8 GEMVs expect bf16 x [M, K]")
    L.require_device(x)
    x = x.contiguous()
    M, K = x.shape
    N = q[0].shape[0]
    if q[0].shape[1] != K:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(q[0].shape)} do not match")
    if M > MAX_ROWS:
        raise ValueError(f"fused GEMVs take at most {MAX_ROWS} rows, got {M}")
    if norm is None and ep is None:  # nothing to fuse: the plain FP8 GEMV
        if mode == L.OUT_SWIGLU:
            return _fp8.gemv_swiglu_fp8(x, q, a)
        return _fp8.gemv_fp8(x, q, split, a)
    if mode == L.OUT_RESIDUAL:
        folded = M == 1 and split == 4  # (the folded launch: no split partials)
        part = torch.empty((split, M, N), device=x.device, dtype=torch.float32) if split > 1 and not folded else None
        _launch_fp8(x, q, split, mode, norm, ep, eps, a, part)
        return None
    if mode == L.OUT_PARTIAL:
        out = torch.empty((split, M, N), device=x.device, dtype=torch.float32)
    else:
        out = torch.empty((M, N // 2 if mode == L.OUT_SWIGLU else N), device=x.device, dtype=torch.bfloat16)
    return _launch_fp8(x, q, split, mode, norm, ep, eps, a, out)


def gemv_fused(x, w, split, *, norm=None, zero_ss=None, ep=None, eps=1e-6, a=None):
    """x [M, K] bf16, w [N, K] bf16 or an FP8Weight.
    norm=(ln_w, ss_in): normalise x rows on the fly.
    zero_ss: accepted; the per-tile sums need no reset (every producer overwrites them).
    ep=(res_in, res_out, ss_out, cnt): residual epilogue; returns None. Runs with EP_SPLIT K
    splits (default one pass) whatever `split` says, or, for FP8 weights at M = 1, FOLD_SPLIT
    folded (ss_out then untouched: one-row consumers sum their row): y is the full fp32 sum.
    a (FP8 weights only): ActScale / SharedScale for static activation scaling; per token if None.
    Otherwise returns bf16 [M, N] (split 1) or fp32 partials [split, M, N]."""
    assert x.shape[-1] % split == 0
    if (ep is not None and FOLD_SPLIT and _is_fp8(w) and x.dim() == 2 and x.shape[0] == 1
            and x.shape[1] % (64 * FOLD_SPLIT) == 0):
        split = FOLD_SPLIT
    elif ep is not None and EP_SPLIT is not None:
        split = EP_SPLIT
    if _is_fp8(w):
        mode = L.OUT_RESIDUAL if ep is not None else (L.OUT_PARTIAL if split > 1 else L.OUT_BF16)
        return _fp8_fused(x, w, split, mode, norm, ep, eps, a)
    if a is not None:
        raise ValueError("activation scales apply to FP8 weights only")
    _check(x, w)
    M, K = x.shape
    N = w.shape[0]
    if ep is not None:
        part = torch.empty((split, M, N), device=x.device, dtype=torch.float32) if split > 1 else None
        _launch(x, w, split, L.OUT_RESIDUAL, norm, ep, eps, part)
        return None
    if split > 1:
        out = torch.empty((split, M, N), device=x.device, dtype=torch.float32)
        return _launch(x, w, split, L.OUT_PARTIAL, norm, None, eps, out)
    out = torch.empty((M, N), device=x.device, dtype=torch.bfloat16)
    return _launch(x, w, 1, L.OUT_BF16, norm, None, eps, out)


def gemv_swiglu_fused(x, w_gu, *, norm=None, zero_ss=None, eps=1e-6, a=None):
    """x [M, K], w_gu [2I, K] = [gate; up] (bf16 or an FP8Weight) -> bf16(silu(gate) * up) [M, I],
    with the optional RMSNorm prologue (and, for FP8 weights, activation scaling) of gemv_fused."""
    if _is_fp8(w_gu):
        return _fp8_fused(x, w_gu, 1, L.OUT_SWIGLU, norm, None, eps, a)
    if a is not None:
        raise ValueError("activation scales apply to FP8 weights only")
    _check(x, w_gu)
    M = x.shape[0]
    out = torch.empty((M, w_gu.shape[0] // 2), device=x.device, dtype=torch.bfloat16)
    return _launch(x, w_gu, 1, L.OUT_SWIGLU, norm, None, eps, out)
