"""FP8 (OCP e4m3) decode matmuls on MI355X: quantizers, activation scales, the scaled cast, and
the dequant-fused skinny GEMM/GEMV that replaces torch._scaled_mm at decode sizes.

Drop-in for the reference's engine/kernels/fp8.py (signatures of quantize_weight, ActScale,
SharedScale, linear_fp8, pick_cast, FP8_MAX, HEADROOM kept as at fp8.py:13-106), plus the
per-channel / per-token family its experiments call (experiments/modal_fp8.py:59-85): quantize,
quant_rows, gemv_fp8, gemv_swiglu_fp8.

Numerics (every quantized byte is the OCP e4m3 round-to-nearest-even of the clamped value, as
torch's float8_e4m3fn cast gives):
  quantize_weight  scale = max(max|w|, 1e-12) / 448;  w8 = e4m3(clamp(w / scale, +-448))
  quantize         the same per output row (scale [N])
  ActScale         amax = max(max|x|, 1e-6) * headroom; inv = 448 / amax; scale = amax / 448
  quant_rows       ActScale per row, then x8 = e4m3(clamp(x * inv[m], +-448)); xs = scale [M, 1]
                   (quant_rows_tiled: the same bytes in the tiled activation layout)
  gemv_fp8 et al.  y = (sum_k x8 w8) * x_scale * w_scale with fp32 accumulation
Quantized weights carry, beside the reference's row-major [N, K] bytes, a copy in the GEMV
kernels' tiled layout (FP8Weight.tiled).
"""

import os

import torch

from . import _lib as L

FP8_MAX = 448.0
HEADROOM = float(os.environ.get("ENGINE_FP8_HEADROOM", "4"))
DECODE_MAX_ROWS = 32  # rows handled by one launch of the skinny kernels
# From this many rows linear_fp8 runs gemm_fp8: per Qwen3-4B decoder layer (the four projections)
# it takes 0.80x-0.995x hipBLASLt's time on MI355X from M = 128 to 4096, and 1.09x at M = 64.
PREFILL_MIN_ROWS = 128


class FP8Weight(tuple):
    """(w8, scale) as the reference returns it - w8 the row-major float8_e4m3fn [N, K] matrix,
    scale fp32 0-d (per tensor) or [N] (per output channel) - with the same bytes in the tiled
    layout of include/krq.h as .tiled (uint8 [N*K], or None when N % 16 or K % 64)."""

    def __new__(cls, w8, scale, tiled=None):
        self = super().__new__(cls, (w8, scale))
        self.tiled = tiled
        return self


def _check_weight(w):
    L.require_device(w)
    if w.dim() != 2 or w.dtype != torch.bfloat16:
        raise ValueError(f"expected a bf16 [N, K] weight, got {w.dtype} {tuple(w.shape)}")
    return w if w.stride(1) == 1 else w.contiguous()


def _weight_out(w, tiled):
    N, K = w.shape
    w8 = torch.empty((N, K), device=w.device, dtype=torch.float8_e4m3fn)
    t = None
    if tiled and N % 16 == 0 and K % 64 == 0:
        t = torch.empty((N * K,), device=w.device, dtype=torch.uint8)
    return w8, t


@torch.no_grad()
def quantize_weight(w, tiled=True):
    """w [N, K] bf16 -> (w8 [N, K] float8_e4m3fn, scale fp32 scalar), w ~= w8 * scale.
    Reference: engine/kernels/fp8.py:17-23."""
    w = _check_weight(w)
    N, K = w.shape
    w8, t = _weight_out(w, tiled)
    scale = torch.empty((), device=w.device, dtype=torch.float32)
    ws = torch.empty((N,), device=w.device, dtype=torch.float32)
    L.call("krq_quant_fp8_tensor", L.ptr(w), N, K, w.stride(0), L.ptr(ws), L.ptr(w8), L.ptr(t),
           L.ptr(scale), L.stream(w))
    return FP8Weight(w8, scale, t)


@torch.no_grad()
def quantize(w, tiled=True):
    """w [N, K] bf16 -> (w8 [N, K] float8_e4m3fn, scale fp32 [N]), w ~= w8 * scale[:, None].
    Per-output-channel form called by the reference's experiments/modal_fp8.py:59-60."""
    w = _check_weight(w)
    N, K = w.shape
    w8, t = _weight_out(w, tiled)
    scale = torch.empty((N,), device=w.device, dtype=torch.float32)
    L.call("krq_quant_fp8_rows", L.ptr(w), N, K, w.stride(0), L.ptr(w8), L.ptr(t), L.ptr(scale),
           L.stream(w))
    return FP8Weight(w8, scale, t)


def _rows(x):
    L.require_device(x)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"expected bf16 activations, got {x.dtype}")
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    return x2.contiguous()


class ActScale:
    """Activation scale for one call: x8 = clamp(x * inv), x ~= x8 * scale.
    Computed on device from this tensor's own range (no sync, graph-safe).
    Reference: engine/kernels/fp8.py:26-35."""

    def __init__(self, x, headroom=1.0):
        x2 = _rows(x)
        M, K = x2.shape
        dev = x2.device
        self.amax = torch.empty((), device=dev, dtype=torch.float32)
        self.inv = torch.empty((1,), device=dev, dtype=torch.float32)
        self.scale = torch.empty((), device=dev, dtype=torch.float32)
        ws = torch.empty((max(1, L.lib().krq_act_scale_ws_floats(M, K)),), device=dev,
                         dtype=torch.float32)
        L.call("krq_act_scale", L.ptr(x2), M, K, 0, float(headroom), L.ptr(self.amax),
               L.ptr(self.inv), L.ptr(self.scale), L.ptr(ws), L.stream(x2))


class SharedScale:
    """Scale slots living in caller-owned device tensors (read by decode graphs).
    Reference: engine/kernels/fp8.py:90-94."""

    def __init__(self, inv, scale):
        self.inv, self.scale = inv, scale


def quant_rows(x):
    """Per-token dynamic FP8: x [M, K] bf16 -> (x8 [M, K] float8_e4m3fn, xs fp32 [M, 1]) with
    x ~= x8 * xs, the operands of torch._scaled_mm(x8, w8.t(), scale_a=xs, ...) in the
    reference's experiments/modal_fp8.py:84-85."""
    x2 = _rows(x)
    M, K = x2.shape
    x8 = torch.empty((M, K), device=x2.device, dtype=torch.float8_e4m3fn)
    xs = torch.empty((M, 1), device=x2.device, dtype=torch.float32)
    L.call("krq_quant_rows", L.ptr(x2), M, K, L.ptr(x8), L.ptr(xs), L.stream(x2))
    return x8, xs


def quant_rows_tiled(x):
    """quant_rows with the e4m3 rows in the tiled activation layout the FP8 GEMV reads as
    X_FP8_TILED: the M rows padded with zero rows to MP = 16 * ceil(M / 16), in 16-row x 64-byte
    tiles (the tiling of FP8Weight.tiled), so each matrix-core operand load is one contiguous KiB.
    Returns (x8t uint8 [MP * K], xs fp32 [M, 1]); the bytes are quant_rows' bytes, permuted."""
    x2 = _rows(x)
    M, K = x2.shape
    mp = (M + 15) // 16 * 16
    x8t = torch.empty((mp * K,), device=x2.device, dtype=torch.uint8)
    xs = torch.empty((M, 1), device=x2.device, dtype=torch.float32)
    L.call("krq_quant_rows_tiled", L.ptr(x2), M, K, L.ptr(x8t), L.ptr(xs), L.stream(x2))
    return x8t, xs


def cast_tiled(x, a):
    """_cast(x, a) in the tiled activation layout of quant_rows_tiled (krq_cast_fp8_tiled): the
    static- or per-call-scale rows for the GEMV on X_FP8_TILED (from TILED_MIN_ROWS to 32 rows).
    Returns uint8 [16 * ceil(M / 16) * K]; the bytes are _cast's, permuted, pad rows zero."""
    x2 = _rows(x)
    M, K = x2.shape
    L.require_device(a.inv)
    mp = (M + 15) // 16 * 16
    x8t = torch.empty((mp * K,), device=x2.device, dtype=torch.uint8)
    L.call("krq_cast_fp8_tiled", L.ptr(x2), M, K, L.ptr(a.inv.reshape(1)), L.ptr(x8t), L.stream(x2))
    return x8t


def _cast_hip(x, a):
    x2 = _rows(x)
    M, K = x2.shape
    L.require_device(a.inv)
    y = torch.empty(x.shape, device=x.device, dtype=torch.float8_e4m3fn)
    L.call("krq_cast_fp8", L.ptr(x2), M, K, L.ptr(a.inv), 0, L.ptr(y), L.stream(x2))
    return y


def _act_scale_cast(x, headroom=1.0):
    """(ActScale(x, headroom), _cast_hip(x, a)) through krq_act_scale_cast_fp8: the same scale and
    bytes, one launch fewer (the fold of the partial maxima runs inside the cast)."""
    x2 = _rows(x)
    M, K = x2.shape
    dev = x2.device
    a = ActScale.__new__(ActScale)
    a.amax = torch.empty((), device=dev, dtype=torch.float32)
    a.inv = torch.empty((1,), device=dev, dtype=torch.float32)
    a.scale = torch.empty((), device=dev, dtype=torch.float32)
    ws = torch.empty((max(1, L.lib().krq_act_scale_ws_floats(M, K)),), device=dev, dtype=torch.float32)
    y = torch.empty(x.shape, device=x.device, dtype=torch.float8_e4m3fn)
    L.call("krq_act_scale_cast_fp8", L.ptr(x2), M, K, float(headroom), L.ptr(a.amax), L.ptr(a.inv),
           L.ptr(a.scale), L.ptr(ws), L.ptr(y), L.stream(x2))
    return a, y


def _cast_torch(x, a):
    return (x.float() * a.inv).clamp_(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)


_cast = _cast_hip


def pick_cast(log):
    """Validate the HIP cast against torch's cast on this GPU (bit-exact) and report both
    timings. Keeps the HIP cast when every byte matches; otherwise falls back to the torch cast
    and says so, as the reference does on a failed check (engine/kernels/fp8.py:62-87)."""
    global _cast
    _cast = _cast_hip
    try:
        x = torch.randn((4096, 2560), device="cuda", dtype=torch.bfloat16) * 3
        a = ActScale(x)
        ref = _cast_torch(x, a).view(torch.uint8)
        got = _cast_hip(x, a).view(torch.uint8)
        bad = int((ref != got).sum().item())
        ts = {}
        for name, fn in (("torch", _cast_torch), ("hip", _cast_hip)):
            fn(x, a)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                fn(x, a)
            e1.record()
            e1.synchronize()
            ts[name] = e0.elapsed_time(e1) / 5
        if bad:
            _cast = _cast_torch
        log(f"fp8 cast: {ts} mismatched bytes={bad} -> {_cast.__name__}")
    except Exception as e:  # pragma: no cover - mirrors the reference's guarded check
        log(f"fp8 hip cast check failed: {e!r}")


# ---------------------------------------------------------------------------------------------
# skinny GEMM / GEMV
# ---------------------------------------------------------------------------------------------
def _weight_operand(q):
    w8, ws = q[0], q[1]
    tiled = getattr(q, "tiled", None)
    L.require_device(w8, ws)
    if ws.dtype != torch.float32:
        raise ValueError("weight scale must be fp32")
    if tiled is not None:
        return tiled, L.W_TILED, ws, w8.shape
    if w8.dtype != torch.float8_e4m3fn or w8.dim() != 2 or not w8.is_contiguous():
        raise ValueError("expected a contiguous float8_e4m3fn [N, K] weight")
    return w8, L.W_ROWMAJOR, ws, w8.shape


FUSED_MAX_ELEMS = 8 * 64 * 64  # activation slice the GEMV can quantize in its prologue (static scale)
TILED_ROWS_MAX_K = 16384  # longest row krq_quant_rows_tiled takes (its vector kernel's register tile)
FUSED_MAX_ELEMS_DYN = 8 * 64 * 32  # row the GEMV can scale per token itself (M == 1)


def _gemv(xin, x_kind, x_scale, x_inv, M, q, split, mode, algo, out):
    w, layout, ws, (N, K) = _weight_operand(q)
    L.require_device(xin, x_scale, x_inv)
    xpr = 1 if (x_scale is not None and x_scale.numel() == M and M > 1) else 0
    wpr = 1 if ws.numel() > 1 else 0
    if out is None:
        if mode == L.OUT_PARTIAL:
            out = torch.empty((split, M, N), device=xin.device, dtype=torch.float32)
        else:
            out = torch.empty((M, N // 2 if mode == L.OUT_SWIGLU else N), device=xin.device,
                              dtype=torch.bfloat16)
    L.call("krq_gemv_fp8", L.ptr(xin), x_kind, L.ptr(x_scale), L.ptr(x_inv), xpr, L.ptr(w), layout,
           L.ptr(ws), wpr, M, N, K, split, mode, algo, L.ptr(out), L.stream(xin))
    return out


def gemv_fp8_launch(x8, xs, q, split=1, mode=L.OUT_BF16, algo=L.ALGO_AUTO, out=None):
    """One launch of the FP8 GEMV kernel on already-quantized activations.
    x8 float8_e4m3fn [M, K] (M <= 32); xs fp32 with 1 (per tensor) or M (per token) values;
    q = quantize(W) or quantize_weight(W). Returns out (allocated when None): bf16 [M, N],
    fp32 partials [split, M, N], or bf16 [M, N/2] for mode OUT_SWIGLU."""
    K = q[0].shape[1]
    M = x8.shape[0]
    if x8.dtype != torch.float8_e4m3fn or x8.dim() != 2 or x8.shape[1] != K or not x8.is_contiguous():
        raise ValueError(f"x8 must be a contiguous float8_e4m3fn [M, {K}] tensor")
    if xs.dtype != torch.float32 or xs.numel() not in (1, M):
        raise ValueError("xs must be fp32 with 1 or M values")
    return _gemv(x8, L.X_FP8, xs.reshape(-1), None, M, q, split, mode, algo, out)


def gemv_fp8_tiled_launch(x8t, xs, q, M, split=1, mode=L.OUT_BF16, out=None):
    """One launch of the FP8 GEMV (matrix-core kernel) on M rows of e4m3 activations in the tiled
    layout of quant_rows_tiled (x8t: 16 * ceil(M / 16) * K bytes) with their scales xs (1 or M
    values). Returns out as gemv_fp8_launch."""
    K = q[0].shape[1]
    mp = (M + 15) // 16 * 16
    if x8t.dtype != torch.uint8 or x8t.numel() != mp * K or not x8t.is_contiguous():
        raise ValueError(f"x8t must be a contiguous uint8 tensor of {mp * K} bytes (quant_rows_tiled)")
    if xs.dtype != torch.float32 or xs.numel() not in (1, M):
        raise ValueError("xs must be fp32 with 1 or M values")
    return _gemv(x8t, L.X_FP8_TILED, xs.reshape(-1), None, M, q, split, mode, L.ALGO_MFMA, out)


def gemv_fp8_bf16_launch(x, q, split=1, mode=L.OUT_BF16, a=None, algo=L.ALGO_AUTO, out=None):
    """One launch of the FP8 GEMV kernel on bf16 activations quantized inside the kernel:
    per token (M == 1, a is None) or with the inverse scale of an ActScale / SharedScale a."""
    x = _rows(x)
    M = x.shape[0]
    if a is None:
        return _gemv(x, L.X_BF16_DYN, None, None, M, q, split, mode, algo, out)
    return _gemv(x, L.X_BF16_STATIC, a.scale.reshape(1), a.inv.reshape(1), M, q, split, mode, algo, out)


def _fits_fused(x, split, a):
    """One row quantized in the GEMV's prologue (its activation wave). More rows with a given
    scale are cast first (row-major, or tiled from TILED_MIN_ROWS): quantizing them in the prologue
    measured slower on MI355X at every M > 1 (split 1, us, prologue / cast + GEMV): QKV M = 4
    9.19 / 6.92, M = 8 10.62 / 7.19; gate_up M = 4 15.78 / 11.33, M = 8 23.66 / 11.90."""
    M, K = x.shape
    if x.dtype != torch.bfloat16 or M != 1 or K % 64:
        return False
    if a is None:
        return K <= FUSED_MAX_ELEMS_DYN
    return K // split <= FUSED_MAX_ELEMS


def _activation_fp8(x, a, xs):
    """(x8, x_scale) for the GEMV when it does not quantize in its prologue: x8 given (fp8
    dtype) with xs; a static or per-call ActScale a (cast kernel); or per-token scales
    (quant_rows kernel)."""
    if x.dtype == torch.float8_e4m3fn:
        if xs is None:
            raise ValueError("float8 activations need their scale xs")
        return x.contiguous(), xs.reshape(-1).contiguous()
    if a is not None:
        return _cast(x, a), a.scale.reshape(1)
    x8, s = quant_rows(x)
    return x8, s.reshape(-1)


# From this many rows the GEMV reads tiled e4m3 rows (padded to 16-row tiles); below, row-major ones.
# Measured on MI355X (graph of 72 launches over 12 weight sets, per-token scales with the decode
# splits / a given scale at split 1), row-major against tiled, us: QKV M = 12 7.28 / 7.40, M = 16
# 7.52 / 7.40; gate_up M = 4 12.64 / 13.47, M = 16 14.19 / 13.70; down M = 4 9.70 / 10.35, M = 16
# 11.24 / 10.83; given scale M = 8 QKV 7.19 / 7.60, M = 16 8.25 / 7.68, M = 32 10.47 / 9.29.
TILED_MIN_ROWS = 13


def _tiled_rows(x, a, xs, algo):
    """bf16 rows at TILED_MIN_ROWS <= M <= 32 go through quant_rows_tiled (scaled per token) or
    cast_tiled (a given scale) and the GEMV on tiled activations (the operands of quant_rows / _cast
    + the row-major e4m3 GEMV, with contiguous loads); fewer rows, and rows longer than the tiled
    kernels take, use the row-major kernels."""
    M, K = x.shape
    return (xs is None and x.dtype == torch.bfloat16 and TILED_MIN_ROWS <= M <= DECODE_MAX_ROWS
            and K % 64 == 0 and K <= TILED_ROWS_MAX_K and algo != L.ALGO_VALU)


def _tiled_operand(x, a):
    """(x8 tiled, x_scale) for _tiled_rows inputs: per token, or with the given scale."""
    if a is None:
        return quant_rows_tiled(x)
    return cast_tiled(x, a), a.scale.reshape(1)


def _chunked(x8, xs, fn):
    M = x8.shape[0]
    if M <= DECODE_MAX_ROWS:
        return fn(x8, xs)
    outs = []
    for m0 in range(0, M, DECODE_MAX_ROWS):
        m1 = min(M, m0 + DECODE_MAX_ROWS)
        outs.append(fn(x8[m0:m1], xs[m0:m1] if xs.numel() == M else xs))
    return torch.cat(outs, dim=-2)


def gemv_fp8(x, q, split=1, a=None, xs=None, algo=L.ALGO_AUTO):
    """FP8 counterpart of kernels.gemv.gemv: x [M, K] bf16 (or float8_e4m3fn with xs), q from
    quantize / quantize_weight. split == 1: bf16 [M, N]; split > 1: fp32 partials [split, M, N]
    whose in-order sum is the product. Activations are scaled per token unless an ActScale /
    SharedScale `a` is given. Called as fp8.gemv_fp8(x, q, split) by the reference's
    experiments/modal_fp8.py:69."""
    M, K = x.shape
    assert K % split == 0
    mode = L.OUT_BF16 if split == 1 else L.OUT_PARTIAL
    if xs is None and _fits_fused(x, split, a):
        return gemv_fp8_bf16_launch(x, q, split, mode, a, algo)
    if _tiled_rows(x, a, xs, algo):
        x8t, s = _tiled_operand(x, a)
        return gemv_fp8_tiled_launch(x8t, s, q, M, split, mode)
    x8, s = _activation_fp8(x, a, xs)
    return _chunked(x8, s, lambda xc, sc: gemv_fp8_launch(xc, sc, q, split, mode, algo))


def gemv_swiglu_fp8(x, q, a=None, xs=None, algo=L.ALGO_AUTO):
    """FP8 counterpart of kernels.gemv.gemv_swiglu: q quantizes w_gu [2I, K] = [gate; up];
    returns bf16(bf16(silu(bf16 g)) * bf16 u) [M, I]. Called as fp8.gemv_swiglu_fp8(x, q) by the
    reference's experiments/modal_fp8.py:67."""
    if xs is None and _fits_fused(x, 1, a):
        return gemv_fp8_bf16_launch(x, q, 1, L.OUT_SWIGLU, a, algo)
    if _tiled_rows(x, a, xs, algo):
        x8t, s = _tiled_operand(x, a)
        return gemv_fp8_tiled_launch(x8t, s, q, x.shape[0], 1, L.OUT_SWIGLU)
    x8, s = _activation_fp8(x, a, xs)
    return _chunked(x8, s, lambda xc, sc: gemv_fp8_launch(xc, sc, q, 1, L.OUT_SWIGLU, algo))


def swiglu_cast_fp8(x, q, out_a, a=None, xs=None):
    """gemv_swiglu_fp8(x, q, a, xs) cast for the next projection in the same launch
    (krq_gemv_swiglu_fp8_cast): the SwiGLU epilogue writes e4m3(clamp(act * out_a.inv, +-448)) of
    its bf16 act in the tiled activation layout of quant_rows_tiled, i.e. the bytes of
    _cast(act, out_a) permuted, with no bf16 act stored and no cast launch. out_a is the next
    projection's ActScale / SharedScale (device inv and scale), as the engine's static-scale decode
    MLP passes it to linear_fp8 (engine/engine.py:977-981). M <= 32. Returns (x8_tiled uint8
    [16 ceil(M / 16) * I], scale fp32 [1]) for gemv_fp8_tiled_launch."""
    w, layout, ws, (N, K) = _weight_operand(q)
    M = x.shape[0]
    if M > DECODE_MAX_ROWS or x.shape[1] != K:
        raise ValueError(f"swiglu_cast_fp8: x {tuple(x.shape)} against w [{N}, {K}] (M <= {DECODE_MAX_ROWS})")
    if N % 128:
        raise ValueError(f"swiglu_cast_fp8: the activation width {N // 2} must be a multiple of 64")
    if xs is None and _fits_fused(x, 1, a):
        xin = _rows(x)
        kind, x_scale, x_inv = (L.X_BF16_DYN, None, None) if a is None else \
            (L.X_BF16_STATIC, a.scale.reshape(1), a.inv.reshape(1))
    elif _tiled_rows(x, a, xs, L.ALGO_AUTO):
        xin, x_scale = _tiled_operand(x, a)
        kind, x_inv = L.X_FP8_TILED, None
    else:
        xin, x_scale = _activation_fp8(x, a, xs)
        kind, x_inv = L.X_FP8, None
    L.require_device(xin, x_scale, x_inv, out_a.inv)
    xpr = 1 if (x_scale is not None and x_scale.numel() == M and M > 1) else 0
    MP = 16 * ((M + 15) // 16)
    x8t = torch.empty((MP * (N // 2),), device=x.device, dtype=torch.uint8)
    L.call("krq_gemv_swiglu_fp8_cast", L.ptr(xin), kind, L.ptr(x_scale), L.ptr(x_inv), xpr, L.ptr(w), layout,
           L.ptr(ws), 1 if ws.numel() > 1 else 0, M, N, K, L.ptr(out_a.inv.reshape(1)), L.ptr(x8t), L.stream(x))
    return x8t, out_a.scale.reshape(1)


def gemm_fp8(x, q, a=None, xs=None):
    """Prefill FP8 GEMM (krq_gemm_fp8_ws): bf16 [M, N] = bf16(x8 . w8^T * x_scale[m] * w_scale[n]),
    the product torch._scaled_mm gives linear_fp8 (engine/kernels/fp8.py:105-106).
    x is bf16 [M, K] with an ActScale / SharedScale `a`, or float8_e4m3fn [M, K] with its scale xs
    (1 or M values); q from quantize_weight / quantize, N and K multiples of 128. bf16 rows are cast
    once (krq_cast_fp8) and multiplied by the e4m3 kernels where those run (K >= 256), else the
    cast is fused into the 128 x 128 kernel's A staging; both give the bytes of the reference's
    cast followed by the e4m3 product."""
    w8, ws = q[0], q[1]
    L.require_device(x, w8, ws)
    if w8.dtype != torch.float8_e4m3fn or w8.dim() != 2 or not w8.is_contiguous():
        raise ValueError("expected a contiguous float8_e4m3fn [N, K] weight")
    N, K = w8.shape
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x {tuple(x.shape)} does not match w8 {tuple(w8.shape)}")
    M = x.shape[0]
    if x.dtype == torch.float8_e4m3fn:
        if xs is None or xs.dtype != torch.float32 or xs.numel() not in (1, M):
            raise ValueError("float8 activations need their fp32 scale xs (1 or M values)")
        kind, xin, x_scale, x_inv = L.X_FP8, x.contiguous(), xs.reshape(-1).contiguous(), None
    else:
        if a is None:
            raise ValueError("bf16 activations need an ActScale / SharedScale a")
        if K % 128 == 0 and K >= 256:
            return gemm_fp8(_cast_hip(_rows(x), a), q, xs=a.scale.reshape(1))
        kind, xin, x_scale, x_inv = L.X_BF16_STATIC, _rows(x), a.scale.reshape(1), a.inv.reshape(1)
    L.require_device(x_scale, x_inv)
    xpr = 1 if (x_scale.numel() == M and M > 1) else 0
    out = torch.empty((M, N), device=x.device, dtype=torch.bfloat16)
    nbytes = L.lib().krq_gemm_fp8_ws_bytes(kind, M, N, K)
    if nbytes < 0:
        raise RuntimeError("krq_gemm_fp8_ws_bytes: device query failed")
    work = torch.empty(nbytes, device=x.device, dtype=torch.uint8) if nbytes else None
    L.call("krq_gemm_fp8_ws", L.ptr(xin), kind, L.ptr(x_scale), L.ptr(x_inv), xpr, L.ptr(w8), L.ptr(ws),
           1 if ws.numel() > 1 else 0, M, N, K, L.ptr(work), nbytes, L.ptr(out), L.stream(xin))
    return out


def linear_fp8(x, q, a=None, amax_out=None):
    """bf16 [M, N] ~= x @ W^T with q = quantize_weight(W); a = given scale, or
    None to scale by this tensor's own range (running max kept in amax_out).
    Reference: engine/kernels/fp8.py:97-106. Decode sizes (M <= 32) run the HIP GEMV; prefill
    rows from PREFILL_MIN_ROWS up run this library's GEMM (gemm_fp8) where its e4m3 kernels take
    the weight (N and K multiples of 128, K >= 256); the rest keep the reference's library GEMM,
    torch._scaled_mm (hipBLASLt on ROCm)."""
    w8, ws = q[0], q[1]
    x8 = None
    if a is None:
        if x.dim() == 2 and x.shape[0] > DECODE_MAX_ROWS and _cast is _cast_hip:
            a, x8 = _act_scale_cast(x)
        else:
            a = ActScale(x)
        if amax_out is not None:
            amax_out.copy_(torch.maximum(amax_out, a.amax.reshape(1)))
    if x8 is None and _fits_fused(x, 1, a):
        return gemv_fp8_bf16_launch(x, q, 1, L.OUT_BF16, a)
    if x8 is None and _tiled_rows(x, a, None, L.ALGO_AUTO):
        return gemv_fp8_tiled_launch(cast_tiled(x, a), a.scale.reshape(1), q, x.shape[0], 1, L.OUT_BF16)
    if x8 is None:
        x8 = _cast(x, a)
    if x.shape[0] <= DECODE_MAX_ROWS:
        return gemv_fp8_launch(x8, a.scale.reshape(1), q, 1, L.OUT_BF16)
    if x.shape[0] >= PREFILL_MIN_ROWS and _ring_gemm_fits(w8):
        return gemm_fp8(x8, q, xs=a.scale.reshape(1))
    return torch._scaled_mm(x8, w8.t(), scale_a=a.scale, scale_b=ws, out_dtype=torch.bfloat16)


def _ring_gemm_fits(w8):
    """The weight shapes gemm_fp8 multiplies with its ring kernels on e4m3 rows."""
    return (w8.dtype == torch.float8_e4m3fn and w8.dim() == 2 and w8.is_contiguous() and w8.shape[0] % 128 == 0
            and w8.shape[1] % 128 == 0 and w8.shape[1] >= 256)
