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
accepted and has nothing to do.

When a block's normalized K slice does not fit the kernel's LDS staging (large M x K/split), the
rows are normalized by krq_rmsnorm_rows first and the GEMV runs on the result: two launches, same
arithmetic.
"""

import torch

from . import _lib as L
from . import gemv as _gemv

MAX_ROWS = 32


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


def _norm_args(x, norm, mode, split):
    """(x, ln, ss) for the launch: the RMSNorm in the kernel when its slice fits, else rows
    normalized by a separate launch and no norm in the GEMV."""
    if norm is None:
        return x, None, None
    ln, ss = norm
    M, K = x.shape
    L.require_device(ln, ss)
    if ln.dtype != torch.bfloat16 or ln.numel() != K or ss.dtype != torch.float32 or ss.numel() != M * (K // 16):
        raise ValueError("norm=(ln [K] bf16, ss [M, K/16] fp32 from FusedLayerBuffers.ss)")
    if L.lib().krq_gemv_fused_fits(M, K, split, mode, 1):
        return x, ln, ss
    return None, ln, ss


def _rmsnorm(x, ln, ss, eps):
    h = torch.empty_like(x)
    L.call("krq_rmsnorm_rows", L.ptr(x), L.ptr(ss), L.ptr(ln), eps, x.shape[0], x.shape[1], L.ptr(h), L.stream(x))
    return h


def _launch(x, w, split, mode, norm, ep, eps, out):
    M, K = x.shape
    N = w.shape[0]
    xin, ln, ss = _norm_args(x, norm, mode, split)
    if xin is None:  # normalize first, then the plain fused launch
        xin, ln, ss = _rmsnorm(x, ln, ss, eps), None, None
    wt, layout = _gemv._weight(w)
    res_in = res_out = ss_out = cnt = None
    if ep is not None:
        res_in, res_out, ss_out, cnt = ep
        L.require_device(res_in, res_out, ss_out, cnt)
        if ss_out.numel() != M * (N // 16) or res_in.numel() != M * N or res_out.numel() != M * N:
            raise ValueError("ep=(res_in [M, N], res_out [M, N], ss_out [M, N/16], cnt) from FusedLayerBuffers")
        if split > 1 and cnt.numel() < N // 16:
            raise ValueError(f"cnt holds {cnt.numel()} counters, needs {N // 16}")
    L.call("krq_gemv_bf16_fused", L.ptr(xin), L.ptr(wt), layout, M, N, K, split, mode, L.ptr(ln), L.ptr(ss),
           float(eps), L.ptr(res_in), L.ptr(res_out), L.ptr(ss_out), L.ptr(cnt), L.ptr(out), L.stream(x))
    return out


def gemv_fused(x, w, split, *, norm=None, zero_ss=None, ep=None, eps=1e-6):
    """x [M, K] bf16, w [N, K] bf16.
    norm=(ln_w, ss_in): normalise x rows on the fly.
    zero_ss: accepted; the per-tile sums need no reset (every producer overwrites them).
    ep=(res_in, res_out, ss_out, cnt): residual epilogue; returns None.
    Otherwise returns bf16 [M, N] (split 1) or fp32 partials [split, M, N]."""
    _check(x, w)
    M, K = x.shape
    N = w.shape[0]
    assert K % split == 0
    if ep is not None:
        part = torch.empty((split, M, N), device=x.device, dtype=torch.float32) if split > 1 else None
        _launch(x, w, split, L.OUT_RESIDUAL, norm, ep, eps, part)
        return None
    if split > 1:
        out = torch.empty((split, M, N), device=x.device, dtype=torch.float32)
        return _launch(x, w, split, L.OUT_PARTIAL, norm, None, eps, out)
    out = torch.empty((M, N), device=x.device, dtype=torch.bfloat16)
    return _launch(x, w, 1, L.OUT_BF16, norm, None, eps, out)


def gemv_swiglu_fused(x, w_gu, *, norm=None, zero_ss=None, eps=1e-6):
    """x [M, K], w_gu [2I, K] = [gate; up] -> bf16(silu(gate) * up) [M, I], with the optional
    RMSNorm prologue of gemv_fused."""
    _check(x, w_gu)
    M = x.shape[0]
    out = torch.empty((M, w_gu.shape[0] // 2), device=x.device, dtype=torch.bfloat16)
    return _launch(x, w_gu, 1, L.OUT_SWIGLU, norm, None, eps, out)
