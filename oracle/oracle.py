"""CPU oracle of the FP8 decode-matmul path - TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (or, for cpu_baseline, as the timed CPU restatement). The product package
(kernel-rush-qwen_amd/kernels) never imports it and has no CPU path.

A numpy restatement of the reference's algorithms (file:line of /root/reference on each
function). bf16 tensors are handled as uint16 bit patterns, e4m3 tensors as uint8 codes, so
every rounding step is explicit.

How each function is pinned (tests/test_oracle.py; tests/golden/):
  e4m3_encode     all 65,536 bf16 patterns and 2M random / tie-point fp32 values against torch's
                  float8_e4m3fn cast (library routine), plus known answers from the OCP spec.
  e4m3_decode     all 256 codes against torch's float8_e4m3fn -> float32.
  quantize_weight,
  quantize        against torch evaluating the reference expressions on CPU (scalar_div="cpu");
                  invariants (max |w8| = 448 per non-zero row / tensor, half-ulp error bound,
                  signed zero); the device form (scalar_div="device") against torch on the GPU
                  (tests/test_gpu_parity.py).
  act_scale, cast,
  quant_rows      as above, against torch evaluating fp8.py:30-35 and :55-56.
  fp8_matmul      exact: float64 BLAS product checked equal to an int64 product of the integer
                  codes; against torch._scaled_mm (CPU) within fp32-accumulation tolerance.
  bf16_matmul     against torch float64 matmul.
  swiglu          against torch.nn.functional.silu in fp32 (at most 1 bf16 ulp, rare).
  mlp_fp8         composition of the pinned functions above; its split partials are checked to
                  sum to the unsplit product, and act to equal swiglu of the gate/up product.
  rmsnorm_rows    torch evaluating Qwen3RMSNorm's expression (fp32 rsqrt of the mean square,
  tile_sumsq,     bf16 casts) on the CPU; residual_add and tile_sumsq against torch's bf16 add
  residual_add    and a float64 sum of squares.
  argmax_lowest   against torch.argmax with planted ties.
  tile / untile   against an element-by-element loop over the layout definition.
"""

import numpy as np

FP8_MAX = np.float32(448.0)
_ONE = np.float32(1.0)


# ---------------------------------------------------------------------------------------------
# bit-level conversions
# ---------------------------------------------------------------------------------------------
def bf16_to_f32(u16):
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """fp32 -> bf16 bits, round to nearest even, NaN kept quiet (torch's .to(bfloat16))."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def round_bf16(f):
    return bf16_to_f32(f32_to_bf16(f))


def e4m3_encode(f):
    """fp32 -> OCP E4M3 (fn) code: round to nearest even; magnitudes rounding beyond 448, NaN and
    inf -> NaN code 0x7F (with sign). Restates torch's float8_e4m3fn cast, which the reference
    uses at engine/kernels/fp8.py:22, :56 (and the Triton cast at :44-45)."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    u = f.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    nan = a >= 0x7F800000
    e = a >> 23
    sub = e < 121
    q_sub = np.rint(a.view(np.float32) * np.float32(512.0)).astype(np.uint32)
    code = ((e - np.uint32(120)) << 3) | ((a >> 20) & 7)
    rem = a & np.uint32(0xFFFFF)
    code = code + ((rem > 0x80000) | ((rem == 0x80000) & ((code & 1) == 1))).astype(np.uint32)
    code = np.where(code > 0x7E, np.uint32(0x7F), code)
    res = np.where(sub, q_sub, code)
    res = np.where(nan, np.uint32(0x7F), res)
    return (res | sign).astype(np.uint8)


def _decode_table():
    t = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 3) & 0xF, b & 7
        if e == 15 and m == 7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * m * 2.0 ** -9
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_VALUES = _decode_table()


def e4m3_decode(codes):
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


# ---------------------------------------------------------------------------------------------
# scale arithmetic. The reference's expressions `amax / FP8_MAX` divide a tensor by a Python
# scalar: torch's CPU kernel divides (IEEE); its device kernels multiply by the fp32 reciprocal
# of the scalar. `FP8_MAX / amax` is Tensor.__rtruediv__ = reciprocal() * 448 on both.
# ---------------------------------------------------------------------------------------------
def div448(a, scalar_div="device"):
    a = np.asarray(a, dtype=np.float32)
    if scalar_div == "cpu":
        return (a / FP8_MAX).astype(np.float32)
    return (a * (_ONE / FP8_MAX)).astype(np.float32)


def inv_from_amax(a):
    a = np.asarray(a, dtype=np.float32)
    return ((_ONE / a) * FP8_MAX).astype(np.float32)


def _clamp_encode(v):
    return e4m3_encode(np.clip(np.asarray(v, dtype=np.float32), -FP8_MAX, FP8_MAX))


# ---------------------------------------------------------------------------------------------
# quantizers
# ---------------------------------------------------------------------------------------------
def quantize_weight(w_u16, scalar_div="device"):
    """Per-tensor: engine/kernels/fp8.py:17-23.
    scale = max(max|w|, 1e-12) / 448; w8 = e4m3(clamp(w / scale, +-448)). Returns (w8, scale)."""
    wf = bf16_to_f32(w_u16)
    amax = np.maximum(np.abs(wf).max(), np.float32(1e-12))
    scale = div448(amax, scalar_div)
    return _clamp_encode(wf / scale), np.float32(scale)


def quantize(w_u16, scalar_div="device"):
    """Per output channel, the form experiments/modal_fp8.py:59-60 calls (row formula
    experiments/modal_fq.py:62-63, clamp convention experiments/i8.py:11-17).
    Returns (w8 [N, K], scale [N])."""
    wf = bf16_to_f32(w_u16)
    amax = np.maximum(np.abs(wf).max(axis=1), np.float32(1e-12))
    scale = div448(amax, scalar_div)
    return _clamp_encode(wf / scale[:, None]), scale


def act_scale(x_u16, headroom=1.0, per_row=False, scalar_div="device"):
    """ActScale, engine/kernels/fp8.py:26-35: amax = max(max|x|, 1e-6) * headroom;
    inv = 448 / amax; scale = amax / 448. Returns (amax, inv, scale) (per row if per_row)."""
    xf = bf16_to_f32(x_u16).reshape(-1, np.shape(x_u16)[-1])
    m = np.abs(xf).max(axis=1) if per_row else np.abs(xf).max()
    amax = (np.maximum(m, np.float32(1e-6)) * np.float32(headroom)).astype(np.float32)
    return amax, inv_from_amax(amax), div448(amax, scalar_div)


def cast(x_u16, inv, per_row=False):
    """_cast_torch / _cast_kernel, engine/kernels/fp8.py:38-56: e4m3(clamp(x * inv, +-448))."""
    xf = bf16_to_f32(x_u16)
    inv = np.asarray(inv, dtype=np.float32)
    if per_row:
        return _clamp_encode(xf * inv.reshape(-1, 1))
    return _clamp_encode(xf * inv.reshape(()))


def quant_rows(x_u16, scalar_div="device"):
    """Per-token quantization (experiments/modal_fp8.py:84-85): ActScale per row + cast.
    Returns (x8 [M, K], xs [M])."""
    _, inv, scale = act_scale(x_u16, 1.0, per_row=True, scalar_div=scalar_div)
    return cast(x_u16, inv, per_row=True), scale


# ---------------------------------------------------------------------------------------------
# matmuls
# ---------------------------------------------------------------------------------------------
def fp8_matmul(x8, xs, w8, ws):
    """torch._scaled_mm(x8, w8.t(), scale_a=xs, scale_b=ws) semantics (engine/kernels/fp8.py:105-106,
    experiments/modal_fp8.py:85) with the sum computed exactly: every e4m3 value is k * 2^-9,
    |k| < 2^18, so each product is a multiple of 2^-18 below 2^36 units and any sum of up to 2^14
    of them stays below 2^50 units - exact in float64 whatever the order.
    Returns (acc float64 [M, N] exact sum, y float64 = acc * xs[m] * ws[n])."""
    acc = e4m3_decode(x8).astype(np.float64) @ e4m3_decode(w8).astype(np.float64).T
    xs = np.asarray(xs, dtype=np.float64).reshape(-1, 1) if np.size(xs) > 1 else np.float64(np.asarray(xs).reshape(()))
    ws = np.asarray(ws, dtype=np.float64).reshape(1, -1) if np.size(ws) > 1 else np.float64(np.asarray(ws).reshape(()))
    return acc, acc * xs * ws


def fp8_matmul_int(x8, w8):
    """The same sum in int64 on the integer codes k (value = k * 2^-9); used to pin fp8_matmul."""
    kx = np.rint(e4m3_decode(x8).astype(np.float64) * 512).astype(np.int64)
    kw = np.rint(e4m3_decode(w8).astype(np.float64) * 512).astype(np.int64)
    return kx @ kw.T  # units of 2^-18


def bf16_matmul(x_u16, w_u16):
    """x[M, K] . w[N, K]^T of bf16 values in float64 (products exact, sum error ~2^-53 relative):
    the fp32-accumulate GEMV of engine/kernels/gemv.py:43-88 up to accumulation order."""
    return bf16_to_f32(x_u16).astype(np.float64) @ bf16_to_f32(w_u16).astype(np.float64).T


def swiglu(acc_g, acc_u):
    """Epilogue of engine/kernels/gemv.py:125-130 (= silu_mul, ops.py:164-172):
    g = bf16(acc_g); u = bf16(acc_u); s = bf16(g / (1 + exp(-g))); out = bf16(s * u), in fp32."""
    g = round_bf16(np.asarray(acc_g, dtype=np.float32))
    u = round_bf16(np.asarray(acc_u, dtype=np.float32))
    with np.errstate(over="ignore"):
        s = round_bf16((g / (_ONE + np.exp(-g))).astype(np.float32))
    return f32_to_bf16((s * u).astype(np.float32))


def argmax_lowest(logits):
    """torch.argmax over the last axis: the first (lowest) index of the maximum
    (engine/engine.py:1022; tie rule of engine/kernels/mega.py:412-419)."""
    return np.argmax(np.asarray(logits), axis=-1)


def mlp_fp8(h_u16, wgu8, gs, wd8, ds, split):
    """Fused decode MLP, engine/kernels/mlp.py:30-85 (phase 1 SwiGLU of the gate/up GEMV, phase 2
    the down GEMV as fp32 split-K partials), with the FP8 quantization of linear_fp8 / quant_rows
    applied to both GEMVs: per-token h, per-token act (amax over the whole act row).
    wgu8 [2I, H] and wd8 [H, I] e4m3 codes with per-row (or per-tensor) scales gs, ds.
    Returns (act u16 [M, I], partials float64 [split, M, H]); the partials sum to the unsplit
    product of the same quantized act."""
    I = wgu8.shape[0] // 2
    x8, xs = quant_rows(h_u16)
    gs = np.broadcast_to(np.asarray(gs, dtype=np.float32).reshape(-1), (2 * I,))
    _, full = fp8_matmul(x8, xs, wgu8, gs)
    act = swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32))
    a8, as_ = quant_rows(act)
    ks = I // split
    parts = [fp8_matmul(a8[:, s * ks:(s + 1) * ks], as_, wd8[:, s * ks:(s + 1) * ks], ds)[1]
             for s in range(split)]
    return act, np.stack(parts)


def tile_sumsq(x_u16):
    """Per-16-column sums of squares of bf16 rows, [M, N/16] float64: the fused residual
    epilogue's partials (the reference accumulates their sum per row, fused_gemv.py:104-105)."""
    xf = bf16_to_f32(x_u16).astype(np.float64)
    M, N = xf.shape
    return (xf * xf).reshape(M, N // 16, 16).sum(-1)


def rmsnorm_rows(x_u16, ss, ln_u16, eps):
    """RMSNorm with the reference's cast points (fused_gemv.py:39-45 = Qwen3RMSNorm):
    rstd = rsqrt(ss / K + eps) in fp32, h = bf16(bf16(x * rstd) * w_ln). ss [M]: sums of squares."""
    K = x_u16.shape[1]
    ms = (np.asarray(ss, dtype=np.float32) / np.float32(K) + np.float32(eps)).astype(np.float32)
    rstd = (_ONE / np.sqrt(ms)).astype(np.float32)
    xr = round_bf16((bf16_to_f32(x_u16) * rstd[:, None]).astype(np.float32))
    return f32_to_bf16((xr * bf16_to_f32(ln_u16)[None, :]).astype(np.float32))


def residual_add(y, res_u16):
    """Residual epilogue (fused_gemv.py:97-105): y (the GEMV's fp32 sum) rounds to bf16, is added
    to the residual in fp32 and rounded: x_new = bf16(res + bf16(y)). Returns x_new (uint16)."""
    yb = round_bf16(np.asarray(y, dtype=np.float32))
    return f32_to_bf16((bf16_to_f32(res_u16) + yb).astype(np.float32))


# ---------------------------------------------------------------------------------------------
# tiled layout of include/krq.h
# ---------------------------------------------------------------------------------------------
def tile(w8):
    """[N, K] bytes -> flat tiled bytes: tiles of 16 rows x 64 bytes in tile-row-major order;
    inside a tile lane 16*g + r holds row r, bytes 16*g .. 16*g+15."""
    N, K = w8.shape
    v = np.asarray(w8).reshape(N // 16, 16, K // 64, 4, 16)   # rb, r, t, g, j
    return np.ascontiguousarray(v.transpose(0, 2, 3, 1, 4)).reshape(-1)


def untile(flat, N, K):
    v = np.asarray(flat).reshape(N // 16, K // 64, 4, 16, 16)  # rb, t, g, r, j
    return np.ascontiguousarray(v.transpose(0, 3, 1, 2, 4)).reshape(N, K)


# ---------------------------------------------------------------------------------------------
# the reference's CPU path, for the reported baseline (bench.py cpu_baseline)
# ---------------------------------------------------------------------------------------------
def torch_dequant_matmul(x8, xs, w8, ws):
    """"torch dequant+matmul" on CPU: bf16(((w8.float() * ws[:, None]) @ (x8.float() * xs).T).T),
    the dequantization of experiments/modal_fp8.py:60 followed by an fp32 matmul. Takes torch CPU
    tensors (x8, w8 float8_e4m3fn; xs [M, 1], ws [N] fp32)."""
    import torch
    w = w8.float() * ws[:, None]
    x = x8.float() * xs
    return (w @ x.T).T.to(torch.bfloat16)
