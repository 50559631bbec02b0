"""Parity of the HIP path (through the C ABI, via the kernels package) with the CPU oracle.

Integer/byte work (quantizers, casts, packing, argmax indices) must be bit-exact. GEMM outputs
must satisfy max|y - ref| <= 1e-2 * max|ref| (the normalisation of the reference's own check,
engine/engine.py:876) against the exact oracle of the same FP8 semantics; the measured error is
printed. Seeds follow the measurement plan: W ~ N(0, 0.02), x ~ N(0, 1), bf16.
"""

import numpy as np
import pytest
import torch

from kernels import _lib as L
from kernels import fp8, lmhead
from kernels.gemv import gemv, gemv_m1, gemv_m1_swiglu, gemv_rows, gemv_swiglu
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _same_plan(K, split):
    """The one-row kernel with its activation wave streams weights with the e4m3 kernel's waves
    when a block's steps all fit in flight at once (at most 16 steps of 128 bytes)."""
    return (K // split // 64 + 1) // 2 <= 16


QKV, O_PROJ, GATE_UP, DOWN = (6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)


def u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


def weight(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)


def act(M, K, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, K, generator=g) * scale).to(torch.bfloat16)


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


# ---------------------------------------------------------------------------------------------
# casts and scale arithmetic
# ---------------------------------------------------------------------------------------------
def test_torch_device_scale_arithmetic(dev):
    """Pins the oracle's device form of the reference's scale expressions on this GPU:
    tensor / 448.0 multiplies by fp32(1/448); 448.0 / tensor is reciprocal() * 448."""
    a = torch.rand(1 << 20, generator=torch.Generator().manual_seed(3)) * 8 + 1e-3
    d = a.to(dev)
    got_div = (d / fp8.FP8_MAX).cpu().numpy()
    got_rdiv = (fp8.FP8_MAX / d).cpu().numpy()
    an = a.numpy()
    assert np.array_equal(got_div, O.div448(an, "device"))
    assert np.array_equal(got_rdiv, O.inv_from_amax(an))


@pytest.mark.parametrize("inv", [1.0, 3.0, 0.0123, 448.0 / 3.1])
def test_cast_all_bf16_patterns(dev, inv):
    bits = np.arange(65536, dtype=np.uint16)
    x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).reshape(256, 256)
    a = fp8.SharedScale(torch.tensor([inv], dtype=torch.float32, device=dev), None)
    got = u8(fp8._cast_hip(x.to(dev), a))
    ref_torch = u8((x.float() * torch.tensor([inv], dtype=torch.float32)).clamp(-448, 448).to(torch.float8_e4m3fn))
    assert np.array_equal(got, O.cast(bits.reshape(256, 256), np.float32(inv)))
    assert np.array_equal(got, ref_torch)
    dev_ref = u8(fp8._cast_torch(x.to(dev), a))
    assert np.array_equal(got, dev_ref)


def test_act_scale_and_cast(dev):
    x = act(16, 2560, 5, 3.0)
    a = fp8.ActScale(x.to(dev))
    amax, inv, scale = O.act_scale(u16(x))
    assert a.amax.shape == () and a.inv.shape == (1,) and a.scale.shape == ()
    assert a.amax.item() == amax and a.inv.item() == inv and a.scale.item() == scale
    # the reference expression evaluated by torch on this device
    xd = x.to(dev)
    mn, mx = torch.aminmax(xd)
    am = torch.maximum(-mn, mx).float().clamp_min(1e-6) * 1.0
    assert torch.equal(am, a.amax) and torch.equal((fp8.FP8_MAX / am).reshape(1), a.inv)
    assert torch.equal((am / fp8.FP8_MAX).reshape(()), a.scale)
    assert np.array_equal(u8(fp8._cast_hip(xd, a)), O.cast(u16(x), inv))
    # headroom and an all-zero tensor (clamp_min(1e-6))
    a4 = fp8.ActScale(xd, headroom=4.0)
    assert a4.amax.item() == O.act_scale(u16(x), 4.0)[0]
    z = fp8.ActScale(torch.zeros(2, 64, dtype=torch.bfloat16, device=dev))
    assert z.amax.item() == np.float32(1e-6)


# 512-thread kernel (K % 16 == 0, up to its 16,384 maximum), 8-value chunk kernel (K % 16 == 8),
# scalar kernel (K % 8 != 0, and rows longer than the vector kernels hold)
@pytest.mark.parametrize("M,K", [(1, 2560), (16, 9728), (32, 4096), (3, 64), (2, 16384), (2, 200), (3, 100),
                                 (1, 20000)])
def test_quant_rows(dev, M, K):
    x = act(M, K, 7 + M)
    x[0, 0] = 0.0
    x8, xs = fp8.quant_rows(x.to(dev))
    r8, rs = O.quant_rows(u16(x))
    assert xs.shape == (M, 1)
    assert np.array_equal(u8(x8), r8)
    assert np.array_equal(xs.cpu().numpy().reshape(-1), rs)


# ---------------------------------------------------------------------------------------------
# weight quantizers and packing
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,K", [(64, 256), QKV, (48, 200)])
def test_quantize_per_channel(dev, N, K):
    w = weight(N, K, 11)
    w[1] = 0.0            # zero row: scale = 1e-12 / 448
    w[2, :7] = -1e-30     # bf16 denormal-ish negatives -> signed zero codes
    q = fp8.quantize(w.to(dev))
    r8, rs = O.quantize(u16(w))
    assert np.array_equal(u8(q[0]), r8)
    assert np.array_equal(q[1].cpu().numpy(), rs)
    if N % 16 == 0 and K % 64 == 0:
        assert np.array_equal(q.tiled.cpu().numpy(), O.tile(r8))
    else:
        assert q.tiled is None
    # the per-row expression (experiments/modal_fq.py:62-63 with the i8.py clamp) in torch on device
    wf = w.to(dev).float()
    s = wf.abs().amax(1).clamp_min(1e-12) / fp8.FP8_MAX
    ref = (wf / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(s, q[1])
    assert torch.equal(ref.view(torch.uint8), q[0].view(torch.uint8))


@pytest.mark.parametrize("N,K", [(64, 256), QKV])
def test_quantize_weight_per_tensor(dev, N, K):
    w = weight(N, K, 13)
    q = fp8.quantize_weight(w.to(dev))
    r8, rs = O.quantize_weight(u16(w))
    assert q[1].shape == ()
    assert q[1].item() == rs
    assert np.array_equal(u8(q[0]), r8)
    # engine/kernels/fp8.py:20-23 evaluated by torch on this device
    wf = w.to(dev).float()
    scale = (wf.abs().max().clamp_min(1e-12) / fp8.FP8_MAX).reshape(())
    ref = (wf / scale).clamp_(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(scale, q[1])
    assert torch.equal(ref.view(torch.uint8), q[0].view(torch.uint8))


def test_pack_unpack_roundtrip(dev):
    N, K = 256, 1280
    w8 = torch.randint(0, 256, (N, K), dtype=torch.uint8, generator=torch.Generator().manual_seed(1))
    wd = w8.to(dev)
    t = torch.empty(N * K, dtype=torch.uint8, device=dev)
    back = torch.empty_like(wd)
    s = L.stream(wd)
    L.call("krq_pack_fp8", L.ptr(wd), N, K, L.ptr(t), s)
    L.call("krq_unpack_fp8", L.ptr(t), N, K, L.ptr(back), s)
    assert np.array_equal(t.cpu().numpy(), O.tile(w8.numpy()))
    assert torch.equal(back, wd)


# ---------------------------------------------------------------------------------------------
# FP8 GEMV / skinny GEMM
# ---------------------------------------------------------------------------------------------
def _fp8_case(N, K, M, seed):
    w = weight(N, K, 1000 + seed)
    x = act(M, K, 2000 + seed)
    return w, x


SHAPES = {"qkv": QKV, "o": O_PROJ, "down": DOWN, "small": (64, 384)}
SEEDS = {"qkv": 0, "o": 1, "down": 3, "small": 5, "odd": 6}


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("M", [1, 2, 16, 23, 32])  # 23: the two-row-tile rings with a ragged second tile
def test_gemv_fp8(dev, name, M):
    N, K = SHAPES[name]
    w, x = _fp8_case(N, K, M, SEEDS[name])
    q = fp8.quantize(w.to(dev))
    r8, rs = O.quantize(u16(w))
    x8r, xsr = O.quant_rows(u16(x))
    _, yref = O.fp8_matmul(x8r, xsr, r8, rs)
    xd = x.to(dev)
    for split in (1, 2, 4):
        if (K // split) % 64:
            continue
        y = fp8.gemv_fp8(xd, q, split)
        if split > 1:
            assert y.shape == (split, M, N) and y.dtype == torch.float32
            y = _sum_partials(y)
        else:
            assert y.shape == (M, N) and y.dtype == torch.bfloat16
            y = y.float().cpu().numpy()
        e = rel_err(y, yref)
        print(f"{name} M={M} split={split}: max-rel {e:.2e}")
        assert e <= TOL


@pytest.mark.parametrize("M", [16, 32])
def test_gemv_paired_row_blocks(dev, M):
    """Grids of >= 4096 row blocks x splits run the paired-row-block kernels (two 16-column
    blocks per workgroup sharing the activation loads): FP8 and BF16, bf16 and partial outputs,
    both layouts."""
    N, K = 65536, 256
    w, x = _fp8_case(N, K, M, 61)
    wd, xd = w.to(dev), x.to(dev)
    q = fp8.quantize(wd)
    r8, rs = O.quantize(u16(w))
    x8r, xsr = O.quant_rows(u16(x))
    _, yref = O.fp8_matmul(x8r, xsr, r8, rs)
    for qq in (q, fp8.FP8Weight(q[0], q[1], None)):
        assert rel_err(fp8.gemv_fp8(xd, qq, 1).float().cpu().numpy(), yref) <= TOL
        assert rel_err(_sum_partials(fp8.gemv_fp8(xd, qq, 2)), yref) <= TOL
    bref = O.bf16_matmul(u16(x), u16(w))
    assert rel_err(gemv(xd, wd, 1).float().cpu().numpy(), bref) <= TOL
    assert rel_err(_sum_partials(gemv(xd, wd, 2)), bref) <= TOL


def _sum_partials(p):
    """The consumer's rule (engine/kernels/ops.py:35-38): fp32 sum in split order, then bf16."""
    acc = p[0].float().clone()
    for s in range(1, p.shape[0]):
        acc += p[s]
    return acc.to(torch.bfloat16).float().cpu().numpy()


@pytest.mark.parametrize("layout", ["tiled", "rowmajor"])
@pytest.mark.parametrize("algo", [L.ALGO_MFMA, L.ALGO_VALU])
def test_gemv_fp8_layouts_and_algos(dev, layout, algo):
    N, K = QKV
    w, x = _fp8_case(N, K, 1, 42)
    q = fp8.quantize(w.to(dev))
    if layout == "rowmajor":
        q = fp8.FP8Weight(q[0], q[1], None)
    x8, xs = fp8.quant_rows(x.to(dev))
    outs = []
    for split, mode in ((1, L.OUT_BF16), (2, L.OUT_PARTIAL), (5, L.OUT_PARTIAL)):
        y = fp8.gemv_fp8_launch(x8, xs, q, split, mode, algo)
        outs.append(y.float().cpu().numpy() if split == 1 else _sum_partials(y))
    r8, rs = O.quantize(u16(w))
    _, yref = O.fp8_matmul(u8(x8), xs.cpu().numpy(), r8, rs)
    for y in outs:
        assert rel_err(y, yref) <= TOL


# (5 and 12: row-major e4m3 rows; 16, 23, 32: tiled; all but 1 the multi-row mixed launch, its
# half-pair blocks first)
@pytest.mark.parametrize("M", [1, 5, 12, 16, 23, 32])
def test_gemv_swiglu_fp8(dev, M):
    N, K = GATE_UP
    I = N // 2
    w, x = _fp8_case(N, K, M, 2)
    q = fp8.quantize(w.to(dev))
    y = fp8.gemv_swiglu_fp8(x.to(dev), q)
    assert y.shape == (M, I) and y.dtype == torch.bfloat16
    r8, rs = O.quantize(u16(w))
    x8r, xsr = O.quant_rows(u16(x))
    _, full = O.fp8_matmul(x8r, xsr, r8, rs)
    ref = O.bf16_to_f32(O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32)))
    e = rel_err(y.float().cpu().numpy(), ref)
    print(f"gate_up swiglu M={M}: max-rel {e:.2e}")
    assert e <= TOL
    if M == 1:
        yv = fp8.gemv_swiglu_fp8(x.to(dev), q, algo=L.ALGO_VALU)
        assert rel_err(yv.float().cpu().numpy(), ref) <= TOL


def test_gemv_fp8_per_tensor_static_scale(dev):
    """The shipped decode form: per-tensor weights and a static SharedScale
    (engine/engine.py:977-981 through linear_fp8)."""
    N, K = DOWN
    w, x = _fp8_case(N, K, 16, 3)
    q = fp8.quantize_weight(w.to(dev))
    inv = torch.tensor([448.0 / 5.0], device=dev)
    sc = torch.tensor(5.0 / 448.0, device=dev)
    y = fp8.linear_fp8(x.to(dev), q, fp8.SharedScale(inv, sc))
    r8, rs = O.quantize_weight(u16(w))
    x8r = O.cast(u16(x), np.float32(448.0 / 5.0))
    _, yref = O.fp8_matmul(x8r, np.float32(5.0 / 448.0), r8, rs)
    assert rel_err(y.float().cpu().numpy(), yref) <= TOL
    # dynamic per-call scale, running amax kept
    amax_out = torch.zeros(1, device=dev)
    y2 = fp8.linear_fp8(x.to(dev), q, amax_out=amax_out)
    am, inv2, s2 = O.act_scale(u16(x))
    assert amax_out.item() == am
    _, yref2 = O.fp8_matmul(O.cast(u16(x), inv2), s2, r8, rs)
    assert rel_err(y2.float().cpu().numpy(), yref2) <= TOL


def test_gemv_fp8_rejects_bad_shapes(dev):
    w = weight(64, 200, 1).to(dev)
    q = fp8.quantize(w)
    with pytest.raises(ValueError):
        fp8.gemv_fp8(act(1, 200, 1).to(dev), q)   # K % 64 != 0
    q2 = fp8.quantize(weight(64, 256, 1).to(dev))
    with pytest.raises(AssertionError):
        fp8.gemv_fp8(act(1, 256, 1).to(dev), q2, split=3)


# ---------------------------------------------------------------------------------------------
# BF16 GEMV family
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M", [1, 4, 16, 32])
def test_gemv_bf16(dev, M):
    N, K = QKV
    w, x = weight(N, K, 21), act(M, K, 22)
    ref = O.bf16_matmul(u16(x), u16(w))
    wd, xd = w.to(dev), x.to(dev)
    y = gemv(xd, wd)
    assert rel_err(y.float().cpu().numpy(), ref) <= TOL
    p = gemv(xd, wd, 4)
    assert p.shape == (4, M, N)
    assert rel_err(_sum_partials(p), ref) <= TOL
    assert rel_err(gemv_rows(xd, wd, 256).float().cpu().numpy(), ref) <= TOL
    if M == 1:
        assert rel_err(gemv_m1(xd, wd, 2).sum(0).float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M", [1, 16])
def test_gemv_swiglu_bf16(dev, M):
    N, K = 2 * 1024, 2560
    I = N // 2
    w, x = weight(N, K, 31), act(M, K, 32)
    full = O.bf16_matmul(u16(x), u16(w))
    ref = O.bf16_to_f32(O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32)))
    y = gemv_swiglu(x.to(dev), w.to(dev))
    assert rel_err(y.float().cpu().numpy(), ref) <= TOL
    if M == 1:
        assert rel_err(gemv_m1_swiglu(x.to(dev), w.to(dev)).float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M", [1, 16])
def test_gemv_swiglu_bf16_gate_up_shape(dev, M):
    """The BF16 SwiGLU GEMV at Qwen3-4B's real gate_up [19456 x 2560] (gate rows first)."""
    N, K = GATE_UP
    I = N // 2
    w, x = weight(N, K, 33), act(M, K, 34)
    full = O.bf16_matmul(u16(x), u16(w))
    ref = O.bf16_to_f32(O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32)))
    y = gemv_swiglu(x.to(dev), w.to(dev))
    assert y.shape == (M, I)
    e = rel_err(y.float().cpu().numpy(), ref)
    print(f"bf16 swiglu [19456x2560] M={M}: max-rel {e:.2e}")
    assert e <= TOL
    if M == 1:
        assert torch.equal(gemv_m1_swiglu(x.to(dev), w.to(dev)), y)


@pytest.mark.parametrize("M", [1, 5, 16, 32])
@pytest.mark.parametrize("N,K,swiglu", [(6144, 2560, False), (100, 320, False), (2 * 1000, 2560, True)])
def test_gemv_rows_programs(dev, M, N, K, swiglu):
    """gemv_rows (reference gemv.py:270-348): workgroup p of exactly `programs` owns output rows
    [p N / programs, (p + 1) N / programs). Against the oracle at every programs count, including
    ranges that do not start on a 16-row boundary, more programs than rows and N not a multiple of
    16; and bit-identical across programs counts (one wave sums each row in one order)."""
    w, x = weight(N, K, 41 + M), act(M, K, 42 + M)
    full = O.bf16_matmul(u16(x), u16(w))
    if swiglu:
        I = N // 2
        ref = O.bf16_to_f32(O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32)))
    else:
        ref = full
    wd, xd = w.to(dev), x.to(dev)
    first = None
    for programs in (1, 7, 132, 256, 264, 512, N + 3):
        y = gemv_rows(xd, wd, programs, swiglu=swiglu)
        assert y.shape == ref.shape and y.dtype == torch.bfloat16
        assert rel_err(y.float().cpu().numpy(), ref) <= TOL, programs
        if first is None:
            first = y
        else:
            assert torch.equal(y, first), programs


def silu_mul_input(M, K, seed):
    """The down projection's input of BASELINE C2/C3: bf16(bf16(silu(g)) * u) of g, u ~ N(0, 1)
    bf16 pairs, rounded as engine/kernels/ops.py:171-172 rounds it (bench.py's make_inputs)."""
    g = torch.Generator().manual_seed(seed)
    gg = torch.randn(M, K, generator=g).to(torch.bfloat16).float()
    uu = torch.randn(M, K, generator=g).to(torch.bfloat16).float()
    s = (gg / (1.0 + torch.exp(-gg))).to(torch.bfloat16).float()
    return (s * uu).to(torch.bfloat16)


@pytest.mark.parametrize("M", [1, 16, 32])
def test_down_projection_on_swiglu_input(dev, M):
    """down [2560 x 9728] at split 4 (the engine's split) on the SwiGLU-shaped input the bench
    uses: heavier-tailed than N(0, 1), so the per-token scale and the e4m3 subnormals carry more
    of the row. Quantized bytes bit-exact, partials' in-order sum within the parity bar."""
    N, K = DOWN
    w = weight(N, K, 1003)
    x = silu_mul_input(M, K, 2003)
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    x8, xs = fp8.quant_rows(xd)
    x8r, xsr = O.quant_rows(u16(x))
    assert np.array_equal(u8(x8), x8r) and np.array_equal(xs.cpu().numpy().reshape(-1), xsr)
    r8, rs = O.quantize(u16(w))
    _, yref = O.fp8_matmul(x8r, xsr, r8, rs)
    y = _sum_partials(fp8.gemv_fp8(xd, q, 4))
    e = rel_err(y, yref)
    print(f"down on silu*u M={M}: max-rel {e:.2e}; e4m3 subnormal codes {np.mean((x8r & 0x78) == 0):.3f}")
    assert e <= TOL


def test_pick_cast_accepts_bit_exact_hip_cast(dev):
    """pick_cast (engine.py:502 calls it once at load) validates the HIP cast against torch's on
    this GPU and keeps it only when every byte matches (the reference accepts maxdiff <= 32,
    engine/kernels/fp8.py:82-84; here zero mismatches are required) and logs both timings."""
    logs = []
    fp8.pick_cast(logs.append)
    assert len(logs) == 1 and "mismatched bytes=0" in logs[0] and "-> _cast_hip" in logs[0], logs
    assert fp8._cast is fp8._cast_hip
    print(logs[0])


# ---------------------------------------------------------------------------------------------
# LM head + argmax
# ---------------------------------------------------------------------------------------------
def test_lmhead_ties_lowest_index(dev):
    V, K = 4096, 256
    E = torch.zeros(V, K, dtype=torch.bfloat16)
    for j in (3000, 17, 2049, 4095):      # four identical best rows
        E[j, :] = 0.5
    h = torch.ones(2, K, dtype=torch.bfloat16)
    idx = lmhead.lm_head_argmax(h.to(dev), E.to(dev)).cpu().numpy()
    assert idx.tolist() == [17, 17]


def test_lmhead_nan_is_max(dev):
    """torch.argmax (engine.py:1021-1022) and the oracle's numpy argmax take NaN as the maximum and
    return its first index: a NaN logit row wins over every number; all-NaN logits give index 0."""
    V, K = 4096, 256
    E = weight(V, K, 21)
    for j in (3000, 123):                 # two NaN logit rows
        E[j, :] = float("nan")
    h = act(2, K, 22)
    idx = lmhead.lm_head_argmax(h.to(dev), E.to(dev)).cpu().numpy()
    ref = O.argmax_lowest(h.float().numpy() @ E.float().numpy().T)
    assert ref.tolist() == [123, 123] and idx.tolist() == [123, 123]
    hn = h.clone()
    hn[1, 7] = float("nan")               # row 1: every logit NaN
    q = fp8.quantize(weight(V, K, 23).to(dev))
    idx8 = lmhead.lm_head_argmax(hn.to(dev), q).cpu().numpy()
    assert idx8[1] == 0
    assert idx8[0] == lmhead.lm_head_argmax(h.to(dev), q).cpu().numpy()[0]  # row 0 untouched


# ---------------------------------------------------------------------------------------------
# graph replay and determinism
# ---------------------------------------------------------------------------------------------
def test_graph_replay_matches_eager(dev):
    N, K = QKV
    w, x = _fp8_case(N, K, 16, 9)
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    E = weight(8192, 2560, 8).to(dev)
    h = act(16, 2560, 9).to(dev)
    eager_y = fp8.gemv_fp8(xd, q, 2).clone()
    eager_i = lmhead.lm_head_argmax(h, E).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fp8.gemv_fp8(xd, q, 2)
        lmhead.lm_head_argmax(h, E)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gy = fp8.gemv_fp8(xd, q, 2)
        gi = lmhead.lm_head_argmax(h, E)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gy, eager_y)
        assert torch.equal(gi, eager_i)
        lmhead.lm_head_argmax(h, E)   # eager work between replays
        torch.cuda.synchronize()


def test_deterministic(dev):
    N, K = DOWN
    w, x = _fp8_case(N, K, 32, 4)
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    a = fp8.gemv_fp8(xd, q, 4)
    b = fp8.gemv_fp8(xd, q, 4)
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------------------------
# in-kernel activation quantization: identical to quantizing first
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["qkv", "o", "down"])
@pytest.mark.parametrize("algo", [L.ALGO_MFMA, L.ALGO_VALU])
def test_fused_dynamic_quant_matches_two_kernel_path(dev, name, algo):
    N, K = SHAPES[name]
    w, x = _fp8_case(N, K, 1, SEEDS[name])
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    x8, xs = fp8.quant_rows(xd)
    r8, rs = O.quantize(u16(w))
    _, yref = O.fp8_matmul(u8(x8), xs.cpu().numpy(), r8, rs)
    for split in (1, 2, 4, 8):
        mode = L.OUT_BF16 if split == 1 else L.OUT_PARTIAL
        fused = fp8.gemv_fp8_bf16_launch(xd, q, split, mode, None, algo)
        two = fp8.gemv_fp8_launch(x8, xs, q, split, mode, algo)
        if _same_plan(K, split):
            # the same operands in the same launch shape give the same bits
            assert torch.equal(fused, two), (name, split)
        # without it the launch shape (and so the fp32 summation order) may differ
        f = fused.float().cpu().numpy() if split == 1 else _sum_partials(fused)
        t = two.float().cpu().numpy() if split == 1 else _sum_partials(two)
        assert rel_err(f, t) <= 1e-2 and rel_err(f, yref) <= TOL, (name, split)
    sw = fp8.gemv_fp8_bf16_launch(xd, fp8.quantize(weight(2 * 1024, K, 5).to(dev)), 1, L.OUT_SWIGLU, None, algo)
    assert sw.shape == (1, 1024)


@pytest.mark.parametrize("algo", [L.ALGO_MFMA, L.ALGO_VALU])
def test_dynamic_quant_rounds_overshoot_to_448(dev, algo):
    """fp32 amax * fl(fl(1 / amax) * 448) exceeds 448 for some bf16 amax values (by one ulp). The
    one-row quantizer of the GEMV converts without the clamp, so the hardware convert must round
    that to 448 (code 0x7E), as the reference's clamp-then-cast does: the GEMV equals the clamped
    two-kernel path bit for bit, and nothing turns into NaN."""
    u = (np.arange(0x3F80, 0x4100, dtype=np.uint32) << 16).view(np.float32)  # bf16 values in [1, 8)
    inv = (np.float32(1) / u).astype(np.float32) * np.float32(448)
    over = u[(u * inv).astype(np.float32) > np.float32(448)]
    assert over.size > 0
    a = float(over[len(over) // 2])
    N, K = QKV
    w, x = _fp8_case(N, K, 1, 23)
    x = (x.float() * (a / 8)).to(torch.bfloat16)
    x[0, 5], x[0, 1234] = a, -a
    assert float(x.float().abs().max()) == a
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    x8, xs = fp8.quant_rows(xd)
    assert u8(x8)[0, 5] == 0x7E and u8(x8)[0, 1234] == 0xFE
    for split, mode in ((1, L.OUT_BF16), (2, L.OUT_PARTIAL), (4, L.OUT_PARTIAL)):
        fused = fp8.gemv_fp8_bf16_launch(xd, q, split, mode, None, algo)
        assert bool(torch.isfinite(fused).all())
        if _same_plan(K, split):
            assert torch.equal(fused, fp8.gemv_fp8_launch(x8, xs, q, split, mode, algo)), split


@pytest.mark.parametrize("M", [1, 2, 5, 16, 17, 32])
@pytest.mark.parametrize("K", [64, 2560, 9728])
def test_quant_rows_tiled(dev, M, K):
    """quant_rows_tiled writes quant_rows' bytes in the tiled activation layout: the oracle's rows,
    padded with zero rows to a multiple of 16, through the weights' tiling (O.tile), bit for bit;
    the scales equal quant_rows'."""
    x = act(M, K, 300 + M + K)
    x8t, xs = fp8.quant_rows_tiled(x.to(dev))
    r8, rs = O.quant_rows(u16(x))
    mp = (M + 15) // 16 * 16
    pad = np.zeros((mp, K), dtype=np.uint8)
    pad[:M] = r8
    assert np.array_equal(x8t.cpu().numpy(), O.tile(pad).reshape(-1))
    assert np.array_equal(xs.cpu().numpy().reshape(-1), rs.reshape(-1))


@pytest.mark.parametrize("M", [2, 5, 16, 17, 32])
@pytest.mark.parametrize("K", [64, 2560, 9728])
def test_cast_tiled(dev, M, K):
    """cast_tiled (krq_cast_fp8_tiled) writes _cast's bytes with a given scale in the tiled
    activation layout: the oracle's cast rows, padded with zero rows to a multiple of 16, through
    O.tile, bit for bit, with clamped codes and a NaN among them."""
    x = act(M, K, 400 + M + K)
    x[M - 1, K // 2] = float("nan")
    a = fp8.SharedScale(torch.tensor([448.0 / 2.0], device=dev), torch.tensor(2.0 / 448.0, device=dev))
    x8t = fp8.cast_tiled(x.to(dev), a)
    mp = (M + 15) // 16 * 16
    pad = np.zeros((mp, K), dtype=np.uint8)
    pad[:M] = O.cast(u16(x), np.float32(448.0 / 2.0))
    assert np.array_equal(x8t.cpu().numpy(), O.tile(pad).reshape(-1))


@pytest.mark.parametrize("M", [4, 12, 13, 16, 23])
def test_static_scale_multi_row_routes(dev, M):
    """A given scale at 1 < M <= 32 (the engine's FP8 decode, engine/engine.py:977-981): linear_fp8,
    gemv_fp8 (partials) and gemv_swiglu_fp8 cast the rows first - row-major below TILED_MIN_ROWS,
    tiled (cast_tiled) from there - and run that GEMV: the same bits as those launches called
    directly, within the bar of the oracle."""
    a = fp8.SharedScale(torch.tensor([448.0 / 5.0], device=dev), torch.tensor(5.0 / 448.0, device=dev))
    sc = a.scale.reshape(1)

    def direct(xd, q, split, mode):
        if M >= fp8.TILED_MIN_ROWS:
            return fp8.gemv_fp8_tiled_launch(fp8.cast_tiled(xd, a), sc, q, M, split, mode)
        return fp8.gemv_fp8_launch(fp8._cast_hip(xd, a), sc, q, split, mode)

    for name, split in (("qkv", 2), ("down", 4)):
        N, K = SHAPES[name]
        w, x = _fp8_case(N, K, M, 70 + SEEDS[name])
        q = fp8.quantize_weight(w.to(dev))
        xd = x.to(dev)
        y = fp8.linear_fp8(xd, q, a)
        assert torch.equal(y, direct(xd, q, 1, L.OUT_BF16))
        p = fp8.gemv_fp8(xd, q, split, a)
        assert torch.equal(p, direct(xd, q, split, L.OUT_PARTIAL))
        r8, rs = O.quantize_weight(u16(w))
        _, yref = O.fp8_matmul(O.cast(u16(x), np.float32(448.0 / 5.0)), np.float32(5.0 / 448.0), r8, rs)
        assert rel_err(y.float().cpu().numpy(), yref) <= TOL
        assert rel_err(_sum_partials(p), yref) <= TOL
    N, K = GATE_UP
    w, x = _fp8_case(N, K, M, 77)
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    assert torch.equal(fp8.gemv_swiglu_fp8(xd, q, a), direct(xd, q, 1, L.OUT_SWIGLU))


# ("odd": five row blocks, not a multiple of the wide blocks' four, so the 16-column plan runs)
TILED_SHAPES = {"qkv": (QKV, (1, 2)), "o": (O_PROJ, (4,)), "down": (DOWN, (4,)), "small": ((64, 384), (1, 2)),
                "odd": ((80, 640), (1, 5))}


@pytest.mark.parametrize("name", list(TILED_SHAPES))
@pytest.mark.parametrize("M", [2, 5, 16, 17, 32])
def test_gemv_on_tiled_activations(dev, name, M):
    """The FP8 GEMV reading tiled activations (quant_rows_tiled) equals the GEMV reading the same
    e4m3 rows row-major (quant_rows) bit for bit: the same operands through the same launch plan;
    gemv_fp8 takes this path for bf16 rows at 1 < M <= 32, and it meets the parity bar."""
    (N, K), splits = TILED_SHAPES[name]
    w, x = _fp8_case(N, K, M, 80 + SEEDS[name])
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    x8, xs = fp8.quant_rows(xd)
    x8t, xst = fp8.quant_rows_tiled(xd)
    r8, rs = O.quantize(u16(w))
    x8r, xsr = O.quant_rows(u16(x))
    _, yref = O.fp8_matmul(x8r, xsr, r8, rs)
    for split in splits:
        mode = L.OUT_BF16 if split == 1 else L.OUT_PARTIAL
        t = fp8.gemv_fp8_tiled_launch(x8t, xst, q, M, split, mode)
        r = fp8.gemv_fp8_launch(x8, xs, q, split, mode)
        assert torch.equal(t, r), (name, M, split)
        y = fp8.gemv_fp8(xd, q, split)
        assert torch.equal(y, t), (name, M, split)
        f = t.float().cpu().numpy() if split == 1 else _sum_partials(t)
        assert rel_err(f, yref) <= TOL, (name, M, split)
    qs = fp8.quantize(weight(2 * 1024, K, 81).to(dev))
    sw = fp8.gemv_swiglu_fp8(xd, qs)
    assert torch.equal(sw, fp8.gemv_fp8_launch(x8, xs, qs, 1, L.OUT_SWIGLU)), (name, M)


@pytest.mark.parametrize("M", [17, 32])
@pytest.mark.parametrize("scales", ["channel", "tensor", "static"])
def test_gate_up_tiled_rows_match_row_major(dev, M, scales):
    """gate_up at 16 < M <= 32 at its real shape (608 column blocks: the mixed launch of two-matrix
    and half-pair blocks): bf16 rows through the tiled e4m3 operand (quant_rows_tiled or
    cast_tiled) give the act of the row-major e4m3 rows bit for bit, with per-channel, per-tensor
    and static scales, and meet the oracle's bar."""
    N, K = GATE_UP
    w, x = _fp8_case(N, K, M, 96)
    wd, xd = w.to(dev), x.to(dev)
    q = fp8.quantize_weight(wd) if scales == "tensor" else fp8.quantize(wd)
    if scales == "static":
        a = fp8.ActScale(xd)
        y = fp8.gemv_swiglu_fp8(xd, q, a)
        x8, xs = fp8._cast(xd, a), a.scale.reshape(1)
    else:
        y = fp8.gemv_swiglu_fp8(xd, q)
        x8, xs = fp8.quant_rows(xd)
    assert torch.equal(y, fp8.gemv_fp8_launch(x8, xs, q, 1, L.OUT_SWIGLU)), (M, scales)
    I = N // 2
    r8, rs = O.quantize_weight(u16(w)) if scales == "tensor" else O.quantize(u16(w))
    if scales == "static":
        am, inv, sc = O.act_scale(u16(x))
        x8r, xsr = O.cast(u16(x), inv), sc
    else:
        x8r, xsr = O.quant_rows(u16(x))
    _, full = O.fp8_matmul(x8r, xsr, r8, rs)
    ref = O.bf16_to_f32(O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32)))
    assert rel_err(y.float().cpu().numpy(), ref) <= TOL, (M, scales)


@pytest.mark.parametrize("static", [False, True])
def test_wide_one_row_blocks_match_one_row_launch(dev, static):
    """QKV at M = 1 runs the wide one-row blocks (four row blocks per workgroup share one activation
    wave). The same weight's first 6,128 rows (383 row blocks, not a multiple of four) run the
    one-row launch with the same plan (one weight wave holding all ten steps beside the activation
    wave); per-channel quantization gives those rows the same bytes and scales, so the shared
    output columns must be equal bit for bit, for per-token and static activation scales."""
    N, K = QKV
    w, x = _fp8_case(N, K, 1, 95)
    wd, xd = w.to(dev), x.to(dev)
    q, q_cut = fp8.quantize(wd), fp8.quantize(wd[:N - 16].contiguous())
    assert torch.equal(q_cut[0], q[0][:N - 16]) and torch.equal(q_cut[1], q[1][:N - 16])
    a = fp8.ActScale(xd) if static else None
    for split in (1, 2):
        y = fp8.gemv_fp8(xd, q, split, a)
        y_cut = fp8.gemv_fp8(xd, q_cut, split, a)
        assert torch.equal(y[..., :N - 16], y_cut), (static, split)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_fused_static_quant_matches_cast_path(dev, M):
    N, K = O_PROJ
    w, x = _fp8_case(N, K, M, 17)
    q = fp8.quantize_weight(w.to(dev))
    xd = x.to(dev)
    a = fp8.SharedScale(torch.tensor([448.0 / 4.5], device=dev), torch.tensor(4.5 / 448.0, device=dev))
    x8 = fp8._cast_hip(xd, a)
    for split in (4, 8):
        fused = fp8.gemv_fp8_bf16_launch(xd, q, split, L.OUT_PARTIAL, a)
        two = fp8.gemv_fp8_launch(x8, a.scale.reshape(1), q, split, L.OUT_PARTIAL)
        assert torch.equal(fused, two), split
    r8, rs = O.quantize_weight(u16(w))
    _, yref = O.fp8_matmul(O.cast(u16(x), np.float32(448.0 / 4.5)), np.float32(4.5 / 448.0), r8, rs)
    assert rel_err(_sum_partials(fused), yref) <= TOL


@pytest.mark.parametrize("name", ["qkv", "o", "down"])
@pytest.mark.parametrize("algo", [L.ALGO_MFMA, L.ALGO_VALU])
def test_one_row_static_quant_with_clamping(dev, name, algo):
    """One row, static inverse scale small enough that ~5% of the products clamp at +-448: the
    in-kernel quantization (the one-row activation wave) equals the reference's cast followed by
    the e4m3 GEMV, bit for bit where the launch shapes match, and the SwiGLU variant too."""
    N, K = SHAPES[name]
    w, x = _fp8_case(N, K, 1, 40 + SEEDS[name])
    q = fp8.quantize(w.to(dev))
    xd = x.to(dev)
    a = fp8.SharedScale(torch.tensor([448.0 / 2.0], device=dev), torch.tensor(2.0 / 448.0, device=dev))
    x8 = fp8._cast_hip(xd, a)
    assert (u8(x8) & 0x7F == 0x7E).mean() > 0.02  # many clamped codes
    for split in (1, 2, 4, 8):
        mode = L.OUT_BF16 if split == 1 else L.OUT_PARTIAL
        fused = fp8.gemv_fp8_bf16_launch(xd, q, split, mode, a, algo)
        two = fp8.gemv_fp8_launch(x8, a.scale.reshape(1), q, split, mode, algo)
        if _same_plan(K, split):
            assert torch.equal(fused, two), split
        f = fused.float().cpu().numpy() if split == 1 else _sum_partials(fused)
        t = two.float().cpu().numpy() if split == 1 else _sum_partials(two)
        assert rel_err(f, t) <= 1e-2, split
    qs = fp8.quantize(weight(2 * 1024, K, 6).to(dev))
    sw = fp8.gemv_fp8_bf16_launch(xd, qs, 1, L.OUT_SWIGLU, a, algo)
    sw2 = fp8.gemv_fp8_launch(x8, a.scale.reshape(1), qs, 1, L.OUT_SWIGLU, algo)
    assert torch.equal(sw, sw2)  # the two-matrix block always streams with two weight waves


def test_fused_quant_rejects_oversized_slices(dev):
    w = weight(64, 9728, 1).to(dev)
    q = fp8.quantize(w)
    a = fp8.SharedScale(torch.ones(1, device=dev), torch.ones((), device=dev))
    with pytest.raises(ValueError, match="too large"):
        fp8.gemv_fp8_bf16_launch(act(16, 9728, 1).to(dev), q, 1, L.OUT_BF16, a)
    # the public entry point routes such shapes through the cast kernel instead
    y = fp8.gemv_fp8(act(16, 9728, 1).to(dev), q, 1, a=a)
    assert y.shape == (16, 64)


def test_bf16_tiled_layout_matches_rowmajor(dev):
    from kernels import gemv as G
    N, K = 2048, 2560
    w, x1, x16 = weight(N, K, 41), act(1, K, 42), act(16, K, 43)
    wr = w.to(dev)
    ref1, ref16 = G.gemv(x1.to(dev), wr).clone(), G.gemv(x16.to(dev), wr, 4).clone()
    wt = G.pack(w.to(dev))
    assert np.array_equal(wt.krq_tiled.cpu().numpy(), O.tile(u16(w).view(np.uint8).reshape(N, 2 * K)))
    assert torch.equal(G.gemv(x1.to(dev), wt), ref1)
    assert torch.equal(G.gemv(x16.to(dev), wt, 4), ref16)
    assert torch.equal(G.gemv_swiglu(x16.to(dev), wt), G.gemv_swiglu(x16.to(dev), wr))
    # an in-place change after pack(): the stale tiled copy is not read
    wt.mul_(2)
    wr.mul_(2)
    assert torch.equal(G.gemv(x16.to(dev), wt, 4), G.gemv(x16.to(dev), wr, 4))
    assert getattr(wt, "krq_tiled", None) is None


@pytest.mark.parametrize("M", [1, 16])
def test_lmhead_bf16_tiled(dev, M):
    from kernels import gemv as G
    V, K = 151936, 2560
    E, h = weight(V, K, 7), act(M, K, 100 + M)
    Ed = E.to(dev)
    idx_r, lg_r = lmhead.lm_head_argmax(h.to(dev), Ed, return_logits=True)
    G.pack(Ed)
    idx_t, lg_t = lmhead.lm_head_argmax(h.to(dev), Ed, return_logits=True)
    assert torch.equal(idx_t, idx_r) and torch.equal(lg_t, lg_r)


@pytest.mark.parametrize("K", [16448, 16512])
def test_rows_longer_than_tiled_kernels_fall_back(dev, K):
    """M = 16 rows longer than krq_quant_rows_tiled takes (K > fp8.TILED_ROWS_MAX_K) go through
    the row-major quant_rows + e4m3 GEMV instead of raising: gemv_fp8 at every split that tiles K,
    and the per-channel FP8 lm_head (ids and bf16 logits against the oracle)."""
    assert K > fp8.TILED_ROWS_MAX_K
    M, N = 16, 64
    w, x = weight(N, K, 41), act(M, K, 42)
    q = fp8.quantize(w.to(dev))
    r8, rs = O.quantize(u16(w))
    x8r, xsr = O.quant_rows(u16(x))
    _, yref = O.fp8_matmul(x8r, xsr, r8, rs)
    xd = x.to(dev)
    for split in (1, 2):
        if (K // split) % 64:
            continue
        y = fp8.gemv_fp8(xd, q, split)
        y = _sum_partials(y) if split > 1 else y.float().cpu().numpy()
        e = rel_err(y, yref)
        print(f"K={K} M={M} split={split}: max-rel {e:.2e}")
        assert e <= TOL
    idx, lg = lmhead.lm_head_argmax(xd, q, return_logits=True)
    assert rel_err(lg.float().cpu().numpy(), yref) <= TOL
    ref_ids = O.argmax_lowest(O.bf16_to_f32(u16(lg)).reshape(M, N))  # the fold over its own logits
    assert np.array_equal(idx.cpu().numpy(), ref_ids)
