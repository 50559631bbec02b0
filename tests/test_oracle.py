"""Pins of the CPU oracle (oracle/oracle.py) against library routines, closed forms, invariants
and brute force. The reference ships no golden vectors for this path (its tests/ hold only an
API-client test), so these checks - chosen so that a dropped term, a wrong rounding mode, a
transposed operand or a wrong index fails one of them - are what the oracle rests on."""

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def torch_e4m3(f32):
    return torch.from_numpy(np.ascontiguousarray(f32, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


# ---------------------------------------------------------------------------------------------
# e4m3 encoder / decoder
# ---------------------------------------------------------------------------------------------
def test_encode_all_bf16_patterns_match_torch():
    f = O.bf16_to_f32(np.arange(65536, dtype=np.uint16))
    assert np.array_equal(O.e4m3_encode(f), torch_e4m3(f))


@pytest.mark.parametrize("inv", [1.0, 3.0, 0.0123, 448.0 / 3.1, 1e6, 2.0 ** -12])
def test_encode_scaled_bf16_patterns_match_torch(inv):
    with np.errstate(over="ignore", invalid="ignore"):
        f = O.bf16_to_f32(np.arange(65536, dtype=np.uint16)) * np.float32(inv)
    assert np.array_equal(O.e4m3_encode(f), torch_e4m3(f))


def test_encode_random_and_tie_points_match_torch():
    rng = np.random.default_rng(0)
    r = rng.standard_normal(1_000_000).astype(np.float32) * np.float32(60)
    sub = rng.uniform(-2 ** -6, 2 ** -6, 300_000).astype(np.float32)
    # exact midpoints between adjacent e4m3 values (ties) and their fp32 neighbours
    vals = np.unique(np.abs(O.E4M3_VALUES[np.isfinite(O.E4M3_VALUES)]))
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    ties = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                           np.float32([448, 464, 464.0001, 479.9, 480, 500, 1e30])])
    f = np.concatenate([r, sub, ties, -ties])
    assert np.array_equal(O.e4m3_encode(f), torch_e4m3(f))


def test_encode_known_answers():
    """Closed forms from the OCP E4M3 definition (bias 7, 3 mantissa bits, max 448)."""
    cases = [(0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (1.0625, 0x38), (1.1875, 0x3A), (17.0, 0x58),
             (448.0, 0x7E), (464.0, 0x7E), (500.0, 0x7F), (2.0 ** -9, 0x01), (2.0 ** -10, 0x00),
             (1e-3, 0x01), (2.0 ** -6, 0x08), (-1e-4, 0x80), (0.875 * 2 ** -6, 0x07),
             (15 * 2 ** -10, 0x08), (-2.5, 0xC2)]
    for v, code in cases:
        assert O.e4m3_encode(np.float32([v]))[0] == code, v
    assert O.e4m3_encode(np.float32([np.nan]))[0] & 0x7F == 0x7F
    assert O.e4m3_encode(np.float32([np.inf]))[0] == 0x7F


def test_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok])
    # round trip on every finite code
    assert np.array_equal(O.e4m3_encode(got[ok]), codes[ok])


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.standard_normal(500_000).astype(np.float32) * 100,
                        O.bf16_to_f32(np.arange(65536, dtype=np.uint16)) * np.float32(1.0000001)])
    ref = bf16_bits(torch.from_numpy(f).to(torch.bfloat16))
    got = O.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], ref[~nan])


# ---------------------------------------------------------------------------------------------
# quantizers against the reference's torch expressions (evaluated by torch on the CPU)
# ---------------------------------------------------------------------------------------------
def weight(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)


def test_quantize_weight_matches_reference_expression():
    w = weight(512, 640, 0)
    wf = w.float()                                                   # fp8.py:20-22
    scale = (wf.abs().max().clamp_min(1e-12) / 448.0).reshape(())
    w8 = (wf / scale).clamp_(-448.0, 448.0).to(torch.float8_e4m3fn)
    r8, rs = O.quantize_weight(bf16_bits(w), scalar_div="cpu")
    assert rs == scale.item()
    assert np.array_equal(r8, w8.view(torch.uint8).numpy())


def test_quantize_per_channel_matches_reference_expression():
    w = weight(256, 384, 1)
    w[3] = 0
    wf = w.float()                                                   # modal_fq.py:62-63, i8.py:15
    s = wf.abs().amax(1).clamp_min(1e-12) / 448.0
    w8 = (wf / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    r8, rs = O.quantize(bf16_bits(w), scalar_div="cpu")
    assert np.array_equal(rs, s.numpy())
    assert np.array_equal(r8, w8.view(torch.uint8).numpy())


def test_quantizer_invariants():
    w = weight(200, 300, 2)
    w[5] = 0
    w[6, :10] = -1e-30
    r8, rs = O.quantize(bf16_bits(w))
    vals = O.e4m3_decode(r8)
    amax_rows = np.abs(vals).max(axis=1)
    nz = np.abs(O.bf16_to_f32(bf16_bits(w))).max(axis=1) > 0
    assert np.all(amax_rows[nz] == 448.0)          # the row max maps onto 448 exactly
    assert np.all(vals[5] == 0) and rs[5] == np.float32(1e-12) * (np.float32(1) / np.float32(448))
    assert np.all(r8[6, :10] == 0x80)              # tiny negatives -> signed zero
    # |w - w8*s| <= half an e4m3 ulp (in scaled units) of w/s
    wf = O.bf16_to_f32(bf16_bits(w)).astype(np.float64)
    y = wf / rs[:, None].astype(np.float64)
    e = np.floor(np.log2(np.maximum(np.abs(y), 2.0 ** -6)))
    half_ulp = 2.0 ** (e - 3) / 2
    assert np.all(np.abs(y - vals) <= half_ulp * (1 + 1e-6))


def test_scalar_division_forms_differ_and_are_pinned():
    a = np.float32(np.random.default_rng(3).uniform(1e-3, 8, 1_000_000))
    t = torch.from_numpy(a)
    assert np.array_equal((t / 448.0).numpy(), O.div448(a, "cpu"))
    assert np.array_equal((448.0 / t).numpy(), O.inv_from_amax(a))
    # the device form really is a different rounding for some inputs (pinned on the GPU)
    assert not np.array_equal(O.div448(a, "cpu"), O.div448(a, "device"))


def test_act_scale_and_cast_match_reference_expression():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(16, 2560, generator=g) * 3).to(torch.bfloat16)
    mn, mx = torch.aminmax(x)                                       # fp8.py:31-35
    amax = torch.maximum(-mn, mx).float().clamp_min(1e-6) * 2.0
    inv = (448.0 / amax).reshape(1)
    scale = (amax / 448.0).reshape(())
    ra, ri, rs = O.act_scale(bf16_bits(x), headroom=2.0, scalar_div="cpu")
    assert ra == amax.item() and ri == inv.item() and rs == scale.item()
    x8 = (x.float() * inv).clamp_(-448.0, 448.0).to(torch.float8_e4m3fn)  # fp8.py:55-56
    assert np.array_equal(O.cast(bf16_bits(x), ri), x8.view(torch.uint8).numpy())


def test_quant_rows_per_token():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 512, generator=g).to(torch.bfloat16)
    x[2] = 0
    x8, xs = O.quant_rows(bf16_bits(x), scalar_div="cpu")
    for m in range(8):
        a, i, s = O.act_scale(bf16_bits(x[m:m + 1]), scalar_div="cpu")
        assert xs[m] == s
        assert np.array_equal(x8[m], O.cast(bf16_bits(x[m:m + 1]), i)[0])
    assert xs[2] == np.float32(1e-6) / np.float32(448)
    v = O.e4m3_decode(x8)
    assert np.all(np.abs(v[[0, 1, 3]]).max(axis=1) == 448.0)


# ---------------------------------------------------------------------------------------------
# matmuls
# ---------------------------------------------------------------------------------------------
def test_fp8_matmul_is_exact():
    rng = np.random.default_rng(6)
    fin = np.flatnonzero(np.isfinite(O.E4M3_VALUES)).astype(np.uint8)
    x8 = rng.choice(fin, (4, 9728))
    w8 = rng.choice(fin, (64, 9728))
    x8[0, :] = 0x7E          # extreme magnitudes: 448 * 448 * 9728 still exact
    w8[0, :] = 0x7E
    acc, _ = O.fp8_matmul(x8, np.float32(1), w8, np.float32(1))
    exact = O.fp8_matmul_int(x8, w8)
    assert np.array_equal(acc * 2.0 ** 18, exact.astype(np.float64))
    assert acc[0, 0] == 448.0 * 448.0 * 9728


def test_fp8_matmul_matches_torch_scaled_mm():
    rng = np.random.default_rng(7)
    M, N, K = 16, 96, 2560
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    xb, wb = O.f32_to_bf16(x), O.f32_to_bf16(w)
    x8, xs = O.quant_rows(xb, scalar_div="cpu")
    w8, ws = O.quantize(wb, scalar_div="cpu")
    acc, y = O.fp8_matmul(x8, xs, w8, ws)
    one = torch.ones((), dtype=torch.float32)
    # CPU _scaled_mm takes per-tensor scales only: unit scales give the fp32-accumulated sum,
    # then a per-tensor call checks the scale application
    raw = torch._scaled_mm(torch.from_numpy(x8).view(torch.float8_e4m3fn),
                           torch.from_numpy(w8).view(torch.float8_e4m3fn).t(),
                           scale_a=one, scale_b=one, out_dtype=torch.float32).double().numpy()
    assert np.abs(acc - raw).max() <= 1e-5 * np.abs(acc).max()
    sa, sb = torch.tensor(float(xs[0]), dtype=torch.float32), torch.tensor(float(ws[0]), dtype=torch.float32)
    ref = torch._scaled_mm(torch.from_numpy(x8).view(torch.float8_e4m3fn),
                           torch.from_numpy(w8).view(torch.float8_e4m3fn).t(),
                           scale_a=sa, scale_b=sb, out_dtype=torch.float32).double().numpy()
    _, y1 = O.fp8_matmul(x8, xs[0], w8, ws[0])
    assert np.abs(y1 - ref).max() <= 1e-5 * np.abs(y1).max()
    assert np.allclose(y, acc * xs.astype(np.float64)[:, None] * ws.astype(np.float64)[None, :], rtol=1e-15)
    assert not np.allclose(y, y * ws.max() / ws.min(), rtol=1e-2)


def test_bf16_matmul_and_torch():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(3, 256, generator=g).to(torch.bfloat16)
    w = (torch.randn(40, 256, generator=g) * 0.02).to(torch.bfloat16)
    ref = (x.double() @ w.double().T).numpy()
    assert np.allclose(O.bf16_matmul(bf16_bits(x), bf16_bits(w)), ref, rtol=0, atol=1e-12)


def test_swiglu_epilogue_vs_torch_silu():
    rng = np.random.default_rng(9)
    g = (rng.standard_normal(200_000) * 4).astype(np.float32)
    u = (rng.standard_normal(200_000) * 4).astype(np.float32)
    got = O.bf16_to_f32(O.swiglu(g, u))
    gt = torch.from_numpy(g).to(torch.bfloat16).float()
    ut = torch.from_numpy(u).to(torch.bfloat16).float()
    ref = (F.silu(gt).to(torch.bfloat16).float() * ut).to(torch.bfloat16).float().numpy()
    diff = got != ref
    assert diff.mean() < 1e-3
    # where they differ it is by one bf16 rounding step of the product
    assert np.all(np.abs(got - ref)[diff] <= np.abs(ref[diff]) * 2 ** -6)


def test_mlp_fp8_composition():
    """mlp_fp8 against an independent torch evaluation of the same steps (torch casts, F.silu,
    float64 products of dequantized values), and the split invariant: partials sum to the
    unsplit product of the quantized act."""
    g = torch.Generator().manual_seed(12)
    M, H, I, S = 3, 256, 512, 4
    h = torch.randn(M, H, generator=g).to(torch.bfloat16)
    wgu = (torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16)
    gu8, gs = O.quantize(bf16_bits(wgu), scalar_div="cpu")
    d8, ds = O.quantize(bf16_bits(wd), scalar_div="cpu")
    act, parts = O.mlp_fp8(bf16_bits(h), gu8, gs, d8, ds, S)
    assert act.shape == (M, I) and parts.shape == (S, M, H)

    def tq(x):   # per-token quantization in torch: (dequantized values, scale)
        amax = x.float().abs().amax(-1, keepdim=True).clamp_min(1e-6)
        x8 = (x.float() * (448.0 / amax)).clamp(-448, 448).to(torch.float8_e4m3fn)
        return x8.double(), (amax / 448.0).double()

    def deq(w8, s):
        return torch.from_numpy(w8).view(torch.float8_e4m3fn).double() * torch.from_numpy(s).double()[:, None]

    hx, hs = tq(h)
    full = (hx @ deq(gu8, gs).T) * hs
    gg = full[:, :I].float().to(torch.bfloat16).float()
    uu = full[:, I:].float().to(torch.bfloat16).float()
    act_t = (F.silu(gg).to(torch.bfloat16).float() * uu).to(torch.bfloat16)
    got = O.bf16_to_f32(act)
    ref = act_t.float().numpy()
    assert np.mean(got != ref) < 1e-2
    assert np.abs(got - ref).max() <= 2 ** -6 * np.abs(ref).max()
    ax, asc = tq(act_t)
    ref_out = ((ax @ deq(d8, ds).T) * asc).numpy()
    assert np.abs(parts.sum(0) - ref_out).max() <= 2e-2 * np.abs(ref_out).max()
    a8, as_ = O.quant_rows(act)
    _, unsplit = O.fp8_matmul(a8, as_, d8, ds)
    assert np.allclose(parts.sum(0), unsplit, rtol=1e-12, atol=1e-12 * np.abs(unsplit).max())
    # gate and up swapped is a different function
    swapped = np.concatenate([gu8[I:], gu8[:I]])
    act_sw, _ = O.mlp_fp8(bf16_bits(h), swapped, np.concatenate([gs[I:], gs[:I]]), d8, ds, S)
    assert not np.allclose(O.bf16_to_f32(act_sw), got, rtol=1e-2)


def test_argmax_lowest_index():
    v = np.float32([[1, 5, 5, 2], [7, 7, 7, 7], [-np.inf, -1, -1, -3]])
    assert O.argmax_lowest(v).tolist() == [1, 0, 1]
    t = torch.from_numpy(v)
    assert O.argmax_lowest(v).tolist() == torch.argmax(t, -1).tolist()


# ---------------------------------------------------------------------------------------------
# tiled layout
# ---------------------------------------------------------------------------------------------
def test_tile_layout_definition_and_inverse():
    N, K = 48, 192
    w8 = np.arange(N * K, dtype=np.int64).reshape(N, K)
    flat = O.tile(w8)
    for n in range(N):
        for k in range(K):
            tile = (n // 16) * (K // 64) + k // 64
            lane = 16 * ((k % 64) // 16) + n % 16
            assert flat[(tile * 64 + lane) * 16 + k % 16] == w8[n, k]
    assert np.array_equal(O.untile(flat, N, K), w8)


def test_golden_cast_table():
    """The committed fixture (torch's float8_e4m3fn cast of every bf16 pattern, written by
    tests/golden/make_golden.py) still matches the oracle."""
    path = os.path.join(GOLDEN, "e4m3_of_bf16.npy")
    table = np.load(path)
    assert table.shape == (65536,) and table.dtype == np.uint8
    assert np.array_equal(table, O.e4m3_encode(O.bf16_to_f32(np.arange(65536, dtype=np.uint16))))


def test_golden_small_cases():
    data = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    x8, xs = O.quant_rows(data["x"])
    w8, ws = O.quantize(data["w"])
    assert np.array_equal(x8, data["x8"]) and np.array_equal(xs, data["xs"])
    assert np.array_equal(w8, data["w8"]) and np.array_equal(ws, data["ws"])
    _, y = O.fp8_matmul(x8, xs, w8, ws)
    assert np.array_equal(O.f32_to_bf16(y.astype(np.float32)), data["y_bf16"])


def test_rmsnorm_and_residual_epilogue():
    """The fused GEMV's prologue / epilogue arithmetic against torch evaluating Qwen3RMSNorm's own
    expression and a bf16 residual add (CPU)."""
    g = torch.Generator().manual_seed(13)
    M, K = 3, 2560
    res = torch.randn(M, K, generator=g).to(torch.bfloat16)
    y = torch.randn(M, K, generator=g) * 0.5
    ln = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    xn = O.residual_add(y.numpy(), bf16_bits(res))
    ref_xn = (res.float() + y.to(torch.bfloat16).float()).to(torch.bfloat16)
    assert np.array_equal(xn, bf16_bits(ref_xn))
    ss_t = O.tile_sumsq(xn)
    assert ss_t.shape == (M, K // 16)
    xf = ref_xn.double()
    assert np.allclose(ss_t.sum(1), (xf * xf).sum(1).numpy(), rtol=1e-12)
    for m, t in ((0, 0), (1, 7), (2, K // 16 - 1)):  # tile t = columns 16t .. 16t + 15 of row m
        assert ss_t[m, t] == float((xf[m, 16 * t:16 * t + 16] ** 2).sum())
    eps = 1e-6
    h = O.rmsnorm_rows(xn, ss_t.sum(1), bf16_bits(ln), eps)
    xt = ref_xn.float()
    var = xt.pow(2).mean(-1, keepdim=True)
    ref_h = ln * (xt * torch.rsqrt(var + eps)).to(torch.bfloat16)
    got, ref = O.bf16_to_f32(h), ref_h.float().numpy()
    assert np.mean(got != ref) < 1e-3   # rsqrt / mean rounding may move a value by one bf16 step
    assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max()
    # a dropped weight or a wrong mean divisor is caught
    assert not np.allclose(O.bf16_to_f32(O.rmsnorm_rows(xn, ss_t.sum(1), bf16_bits(torch.ones(K, dtype=torch.bfloat16)), eps)), ref, rtol=1e-2)
    assert not np.allclose(O.bf16_to_f32(O.rmsnorm_rows(xn, 2 * ss_t.sum(1), bf16_bits(ln), eps)), ref, rtol=1e-2)
