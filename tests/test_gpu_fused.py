"""Fused BF16 decode GEMVs (kernels.fused_gemv over krq_gemv_bf16_fused / krq_rmsnorm_rows) against
the CPU oracle: the RMSNorm prologue, the residual epilogue with split-K last-arriver reduction,
the per-tile sums of squares, and an engine-shaped layer fragment (engine/engine.py:953-961).
GEMV outputs: max|y - ref| <= 1e-2 * max|ref|; residual rows and ss within the same bar."""

import numpy as np
import pytest
import torch

from kernels import gemv as G
from kernels.fused_gemv import FusedLayerBuffers, gemv_fused, gemv_swiglu_fused
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2
H, I, NQKV, V = 2560, 9728, 6144, 151936
EPS = 1e-6


def u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def sum_partials(p):
    acc = p[0].float().clone()
    for s in range(1, p.shape[0]):
        acc += p[s]
    return acc.to(torch.bfloat16).float().cpu().numpy()


@pytest.mark.parametrize("M", [1, 4, 16])
def test_plain_outputs_match_gemv(dev, M):
    w, x = bf((NQKV, H), 1, 0.02), bf((M, H), 2)
    ref = O.bf16_matmul(u16(x), u16(w))
    xd, wd = x.to(dev), w.to(dev)
    assert rel_err(gemv_fused(xd, wd, 1).float().cpu().numpy(), ref) <= TOL
    assert rel_err(sum_partials(gemv_fused(xd, wd, 2)), ref) <= TOL


@pytest.mark.parametrize("M,K,N,split,swiglu", [(1, H, NQKV, 2, False), (16, H, NQKV, 2, False),
                                                (4, H, NQKV, 2, False), (1, H, 2 * I, 1, True),
                                                (4, H, 2 * I, 1, True), (16, H, 2 * I, 1, True),
                                                (4, H, V, 1, False)])
def test_rmsnorm_prologue(dev, M, K, N, split, swiglu):
    """norm=(ln, ss): includes shapes whose normalized slice fits the in-kernel staging and ones that
    take the separate row-normalization launch (M=16 with the full K=2560 slice)."""
    x = bf((M, K), 10 + M)
    w = bf((N, K), 11, 0.02)
    ln = (1 + 0.1 * torch.randn(K, generator=torch.Generator().manual_seed(12))).to(torch.bfloat16)
    ss_t = O.tile_sumsq(u16(x)).astype(np.float32)           # as a residual epilogue leaves it
    h = O.rmsnorm_rows(u16(x), ss_t.astype(np.float64).sum(1), u16(ln), EPS)
    full = O.bf16_matmul(h, u16(w))
    xd, wd, lnd = x.to(dev), w.to(dev), ln.to(dev)
    ssd = torch.from_numpy(ss_t).to(dev)
    if swiglu:
        got = gemv_swiglu_fused(xd, wd, norm=(lnd, ssd), eps=EPS).float().cpu().numpy()
        ref = O.bf16_to_f32(O.swiglu(full[:, :N // 2].astype(np.float32), full[:, N // 2:].astype(np.float32)))
    else:
        y = gemv_fused(xd, wd, split, norm=(lnd, ssd), eps=EPS)
        got = sum_partials(y) if split > 1 else y.float().cpu().numpy()
        ref = full
    e = rel_err(got, ref)
    print(f"norm M={M} N={N} split={split}: max-rel {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("M,split,protocol", [(1, 4, True), (16, 4, True), (1, 1, False), (32, 2, True),
                                              (16, 4, False)])
def test_residual_epilogue(dev, monkeypatch, M, split, protocol):
    """ep=(res_in, res_out, ss_out, cnt): res_out = bf16(res_in + bf16(y)), ss_out per 16-column
    tile; the split counters are back at zero afterwards (twice in a row). protocol: the caller's
    split with the last-arriver reduction (EP_SPLIT None) instead of the default single K pass."""
    from kernels import fused_gemv as FG
    if protocol:
        monkeypatch.setattr(FG, "EP_SPLIT", None)
    K = 4096
    a, w, res = bf((M, K), 20), bf((H, K), 21, 0.02), bf((M, H), 22)
    y = O.bf16_matmul(u16(a), u16(w))
    ref_res = O.residual_add(y, u16(res))
    ref_ss = O.tile_sumsq(ref_res)
    bufs = FusedLayerBuffers(M, H, V, dev)
    res_in = res.to(dev)
    for _ in range(2):
        out = gemv_fused(a.to(dev), w.to(dev), split, ep=(res_in, bufs.res[1], bufs.ss[1], bufs.cnt))
        assert out is None
        torch.cuda.synchronize()
        got = bufs.res[1].float().cpu().numpy()
        mism = float(np.mean(got != O.bf16_to_f32(ref_res)))
        assert rel_err(got, O.bf16_to_f32(ref_res)) <= TOL and mism < 0.02
        assert rel_err(bufs.ss[1].cpu().numpy(), ref_ss) <= TOL
        assert int(bufs.cnt.abs().sum()) == 0


def test_layer_fragment_like_the_engine(dev):
    """o (ep) -> gate_up (norm, SwiGLU) -> down (ep) -> next layer's qkv (norm), as
    engine/engine.py:955-959 chains them, against the unfused oracle sequence."""
    M = 1
    cur, a = bf((M, H), 30), bf((M, 4096), 31)
    wo, wgu, wd, wqkv = bf((H, 4096), 32, 0.02), bf((2 * I, H), 33, 0.02), bf((H, I), 34, 0.02), bf((NQKV, H), 35, 0.02)
    ln2 = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(36))).to(torch.bfloat16)
    ln1 = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(37))).to(torch.bfloat16)
    # oracle
    res_b = O.residual_add(O.bf16_matmul(u16(a), u16(wo)), u16(cur))
    h2 = O.rmsnorm_rows(res_b, O.tile_sumsq(res_b).sum(1), u16(ln2), EPS)
    full = O.bf16_matmul(h2, u16(wgu))
    act = O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32))
    res_a = O.residual_add(O.bf16_matmul(act, u16(wd)), res_b)
    h1 = O.rmsnorm_rows(res_a, O.tile_sumsq(res_a).sum(1), u16(ln1), EPS)
    qkv_ref = O.bf16_matmul(h1, u16(wqkv))
    # fused
    bufs = FusedLayerBuffers(M, H, V, dev)
    res_a_d, res_b_d = bufs.res[0], bufs.res[1]
    ss_a, ss_b = bufs.ss[0], bufs.ss[1]
    d = lambda t: t.to(dev)
    gemv_fused(d(a), d(wo), 4, ep=(d(cur), res_b_d, ss_b, bufs.cnt))
    act_d = gemv_swiglu_fused(res_b_d, d(wgu), norm=(d(ln2), ss_b), zero_ss=ss_a, eps=EPS)
    gemv_fused(act_d, d(wd), 4, ep=(res_b_d, res_a_d, ss_a, bufs.cnt))
    qkv = gemv_fused(res_a_d, d(wqkv), 2, norm=(d(ln1), ss_a), zero_ss=ss_b, eps=EPS)
    assert rel_err(res_b_d.float().cpu().numpy(), O.bf16_to_f32(res_b)) <= TOL
    assert rel_err(act_d.float().cpu().numpy(), O.bf16_to_f32(act)) <= TOL
    assert rel_err(res_a_d.float().cpu().numpy(), O.bf16_to_f32(res_a)) <= TOL
    e = rel_err(sum_partials(qkv), qkv_ref)
    print(f"layer fragment: qkv max-rel {e:.2e}")
    assert e <= TOL


def test_fused_graph_replays(dev, monkeypatch):
    """The residual epilogue's counters reset themselves: replays match eager, with eager calls
    in between (split-K protocol: EP_SPLIT None)."""
    from kernels import fused_gemv as FG
    monkeypatch.setattr(FG, "EP_SPLIT", None)
    M = 4
    a, w, res = bf((M, 4096), 40), bf((H, 4096), 41, 0.02), bf((M, H), 42)
    ad, wd, rd = a.to(dev), w.to(dev), res.to(dev)
    bufs = FusedLayerBuffers(M, H, V, dev)
    gemv_fused(ad, wd, 4, ep=(rd, bufs.res[1], bufs.ss[1], bufs.cnt))
    eager_res, eager_ss = bufs.res[1].clone(), bufs.ss[1].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gemv_fused(ad, wd, 4, ep=(rd, bufs.res[1], bufs.ss[1], bufs.cnt))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gemv_fused(ad, wd, 4, ep=(rd, bufs.res[1], bufs.ss[1], bufs.cnt))
    for _ in range(3):
        bufs.res[1].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(bufs.res[1], eager_res) and torch.equal(bufs.ss[1], eager_ss)
        gemv_fused(ad, wd, 4, ep=(rd, bufs.res[1], bufs.ss[1], bufs.cnt))
    assert int(bufs.cnt.abs().sum()) == 0
    del g


def test_packed_weights(dev):
    """gemv.pack (tiled bf16 copy) is read by the fused kernels too."""
    M = 1
    w, x = bf((NQKV, H), 50, 0.02), bf((M, H), 51)
    ref = O.bf16_matmul(u16(x), u16(w))
    wd = G.pack(w.to(dev))
    assert rel_err(gemv_fused(x.to(dev), wd, 1).float().cpu().numpy(), ref) <= TOL


def test_packfile_rebuilds_tiled_copy_on_device(dev, tmp_path):
    """fp8.quantize on the GPU -> packfile (row-major bytes only) -> load onto the GPU: the tiled
    copy rebuilt by krq_pack_fp8 equals the quantizer's, and the GEMV gives identical bits."""
    from kernels import fp8, packfile
    w, x = bf((NQKV, H), 60, 0.02), bf((1, H), 61)
    q = fp8.quantize(w.to(dev))
    p = str(tmp_path / "w.safetensors")
    packfile.save_fp8(p, {"qkv": q})
    r = packfile.load_fp8(p, device=dev)["qkv"]
    assert torch.equal(r.tiled, q.tiled) and torch.equal(r[1], q[1])
    assert torch.equal(fp8.gemv_fp8(x.to(dev), r, 2), fp8.gemv_fp8(x.to(dev), q, 2))


# ---------------------------------------------------------------------------------------------
# FP8 weights (krq_gemv_fp8_fused, krq_rmsnorm_quant_rows)
# ---------------------------------------------------------------------------------------------
def _fp8_oracle(h_u16, q, split=1, inv=None, scale=None):
    """Oracle of one FP8 GEMV on bf16 rows h: per-token quant_rows (inv None) or the static cast,
    then the exact product; returns the float64 [split, M, N] scaled partials."""
    w8 = q[0].cpu().view(torch.uint8).numpy()
    ws = q[1].cpu().numpy()
    if inv is None:
        x8, xs = O.quant_rows(h_u16)
    else:
        x8, xs = O.cast(h_u16, np.float32(inv)), np.float32(scale)
    K = h_u16.shape[1]
    ks = K // split
    return np.stack([O.fp8_matmul(x8[:, s * ks:(s + 1) * ks], xs, w8[:, s * ks:(s + 1) * ks], ws)[1]
                     for s in range(split)])


def _norm_inputs(M, K, seed):
    x = bf((M, K), seed)
    ln = (1 + 0.1 * torch.randn(K, generator=torch.Generator().manual_seed(seed + 1))).to(torch.bfloat16)
    ss = O.tile_sumsq(u16(x)).astype(np.float32)
    h = O.rmsnorm_rows(u16(x), ss.astype(np.float64).sum(1), u16(ln), EPS)
    return x, ln, ss, h


@pytest.mark.parametrize("M,N,split,swiglu", [(1, NQKV, 2, False), (1, 2 * I, 1, True), (16, NQKV, 2, False),
                                              (16, 2 * I, 1, True), (32, NQKV, 1, False)])
def test_fp8_rmsnorm_prologue_per_token(dev, M, N, split, swiglu):
    """norm=(ln, ss) with per-token scales: in the GEMV prologue at M = 1, krq_rmsnorm_quant_rows
    first at M > 1. Bit-identical to rmsnorm_rows -> the plain FP8 GEMV, and within the bar of the
    oracle (quant_rows of the normalized rows, exact FP8 product)."""
    from kernels import fp8 as F
    from kernels import fused_gemv as FG
    x, ln, ss, h = _norm_inputs(M, H, 70 + M)
    q = F.quantize(bf((N, H), 71, 0.02).to(dev))
    xd, lnd, ssd = x.to(dev), ln.to(dev), torch.from_numpy(ss).to(dev)
    hd = FG._rmsnorm(xd, lnd, ssd, EPS)
    if swiglu:
        got = gemv_swiglu_fused(xd, q, norm=(lnd, ssd), eps=EPS)
        two = F.gemv_swiglu_fp8(hd, q)
        full = _fp8_oracle(h, q)[0]
        ref = O.bf16_to_f32(O.swiglu(full[:, :N // 2].astype(np.float32), full[:, N // 2:].astype(np.float32)))
        gotn = got.float().cpu().numpy()
    else:
        got = gemv_fused(xd, q, split, norm=(lnd, ssd), eps=EPS)
        two = F.gemv_fp8(hd, q, split)
        ref = _fp8_oracle(h, q, split).sum(0)
        gotn = sum_partials(got) if split > 1 else got.float().cpu().numpy()
    assert torch.equal(got, two), "fused prologue differs from rmsnorm_rows + gemv_fp8"
    e = rel_err(gotn, ref)
    print(f"fp8 norm M={M} N={N} split={split}: max-rel {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("M,K", [(1, H), (3, H), (32, H), (2, I), (5, 16384)])
def test_rmsnorm_quant_rows_is_quant_rows_of_rmsnorm(dev, M, K):
    """krq_rmsnorm_quant_rows = quant_rows(krq_rmsnorm_rows(x)) bit for bit (both row-kernel
    variants: K <= 4096 and longer rows); krq_rmsnorm_rows within one bf16 rounding of the
    oracle's RMSNorm (rsqrt against 1 / sqrt)."""
    from kernels import fp8 as F
    from kernels import fused_gemv as FG
    from kernels import _lib as L
    x, ln, ss, h = _norm_inputs(M, K, 80 + M)
    xd, lnd, ssd = x.to(dev), ln.to(dev), torch.from_numpy(ss).to(dev)
    x8 = torch.empty((M, K), device=dev, dtype=torch.float8_e4m3fn)
    xs = torch.empty((M,), device=dev, dtype=torch.float32)
    L.call("krq_rmsnorm_quant_rows", L.ptr(xd), L.ptr(ssd), L.ptr(lnd), EPS, M, K, L.ptr(x8), L.ptr(xs), L.stream(xd))
    hd = FG._rmsnorm(xd, lnd, ssd, EPS)
    r8, rs = F.quant_rows(hd)
    assert torch.equal(x8.view(torch.uint8), r8.view(torch.uint8)) and torch.equal(xs, rs.reshape(-1))
    got = O.bf16_to_f32(u16(hd)).astype(np.float64)
    want = O.bf16_to_f32(h).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)
    assert np.mean(got != want) < 0.05


@pytest.mark.parametrize("M,K", [(1, H), (3, H), (17, H), (2, I), (5, 16384)])
def test_rmsnorm_quant_rows_tiled(dev, M, K):
    """krq_rmsnorm_quant_rows_tiled writes krq_rmsnorm_quant_rows' bytes in the tiled activation
    layout: the rows, padded with zero rows to a multiple of 16, through the weights' tiling
    (O.tile), bit for bit, with the same scales."""
    from kernels import _lib as L
    x, ln, ss, _ = _norm_inputs(M, K, 90 + M)
    xd, lnd, ssd = x.to(dev), ln.to(dev), torch.from_numpy(ss).to(dev)
    x8 = torch.empty((M, K), device=dev, dtype=torch.float8_e4m3fn)
    xs = torch.empty((M,), device=dev, dtype=torch.float32)
    L.call("krq_rmsnorm_quant_rows", L.ptr(xd), L.ptr(ssd), L.ptr(lnd), EPS, M, K, L.ptr(x8), L.ptr(xs), L.stream(xd))
    mp = (M + 15) // 16 * 16
    x8t = torch.empty((mp * K,), device=dev, dtype=torch.uint8)
    xst = torch.empty((M,), device=dev, dtype=torch.float32)
    L.call("krq_rmsnorm_quant_rows_tiled", L.ptr(xd), L.ptr(ssd), L.ptr(lnd), EPS, M, K, L.ptr(x8t), L.ptr(xst),
           L.stream(xd))
    pad = np.zeros((mp, K), dtype=np.uint8)
    pad[:M] = x8.view(torch.uint8).cpu().numpy()
    assert np.array_equal(x8t.cpu().numpy(), O.tile(pad).reshape(-1))
    assert torch.equal(xst, xs)


@pytest.mark.parametrize("M,N,split,swiglu", [(1, NQKV, 2, False), (4, NQKV, 2, False), (4, 2 * I, 1, True),
                                              (16, NQKV, 2, False), (32, 2 * I, 1, True)])
def test_fp8_rmsnorm_prologue_static_scale(dev, M, N, split, swiglu):
    """norm with a static SharedScale a (the reference engine's decode-FP8 form): normalized rows
    cast with a.inv in the prologue; against the oracle's cast of the normalized rows."""
    from kernels import fp8 as F
    x, ln, ss, h = _norm_inputs(M, H, 90 + M)
    q = F.quantize(bf((N, H), 91, 0.02).to(dev))
    xd, lnd, ssd = x.to(dev), ln.to(dev), torch.from_numpy(ss).to(dev)
    amax = float(np.abs(O.bf16_to_f32(h)).max()) * 1.5
    inv = torch.tensor([448.0 / amax], device=dev)
    scale = torch.tensor(amax / 448.0, device=dev)
    a = F.SharedScale(inv, scale)
    if swiglu:
        got = gemv_swiglu_fused(xd, q, norm=(lnd, ssd), eps=EPS, a=a).float().cpu().numpy()
        full = _fp8_oracle(h, q, 1, inv.item(), scale.item())[0]
        ref = O.bf16_to_f32(O.swiglu(full[:, :N // 2].astype(np.float32), full[:, N // 2:].astype(np.float32)))
    else:
        y = gemv_fused(xd, q, split, norm=(lnd, ssd), eps=EPS, a=a)
        got = sum_partials(y) if split > 1 else y.float().cpu().numpy()
        ref = _fp8_oracle(h, q, split, inv.item(), scale.item()).sum(0)
    e = rel_err(got, ref)
    print(f"fp8 norm static M={M} N={N}: max-rel {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("M,split,static,protocol,K,rowmajor",
                         [(1, 4, False, True, 4096, False), (1, 4, False, False, 4096, False),
                          (1, 1, False, True, 4096, False), (1, 4, False, True, I, False),
                          (1, 4, True, True, I, False), (1, 4, False, True, 4096, True), (1, 2, True, False, 1024, True),
                          (16, 4, False, True, 4096, False), (16, 4, False, False, 4096, False),
                          (32, 2, False, True, 4096, False), (4, 4, True, True, 4096, False),
                          (4, 1, True, False, 4096, False)])
def test_fp8_residual_epilogue(dev, monkeypatch, M, split, static, protocol, K, rowmajor):
    """ep=(res_in, res_out, ss_out, cnt) on FP8 weights: res_out equals bf16(res_in + bf16(y)) bit
    for bit, y being the plain GEMV's output for the same K decomposition (the in-order sum of its
    scaled split partials with the split-K protocol, EP_SPLIT None; its one-pass output with the
    default single pass; at M = 1 always the four-split sum, which the folded launch computes
    without cross-workgroup sums), ss_out its per-tile sums of squares (M > 1; at M = 1 the folded
    launch leaves ss_out alone), and the counters are zero again (twice in a row); the oracle
    bounds the whole. K = 9,728 is the down projection (its one-row activation wave of 20 chunks
    per lane, two weight waves); row-major weights take the folded launch's row-major addressing."""
    from kernels import fp8 as F
    from kernels import fused_gemv as FG
    if protocol:
        monkeypatch.setattr(FG, "EP_SPLIT", None)
    ref_split = FG.FOLD_SPLIT if M == 1 else (split if protocol else 1)  # the call passes `split` either way
    a_, res = bf((M, K), 100 + M), bf((M, H), 101)
    q = F.quantize(bf((H, K), 102, 0.02).to(dev))
    if rowmajor:
        q = F.FP8Weight(q[0], q[1], None)
    ad, rd = a_.to(dev), res.to(dev)
    sa = None
    if static:
        sa = F.ActScale(ad)
    bufs = FusedLayerBuffers(M, H, V, dev)
    p = F.gemv_fp8(ad, q, ref_split, sa)
    if ref_split > 1:  # the partials summed in split order, then rounded
        y = p[0].clone()
        for s in range(1, ref_split):
            y += p[s]
        p = y.to(torch.bfloat16)
    want = (rd.float() + p.float()).to(torch.bfloat16)
    bufs.ss[1].fill_(-1.0)
    for _ in range(2):
        assert gemv_fused(ad, q, split, ep=(rd, bufs.res[1], bufs.ss[1], bufs.cnt), a=sa) is None
        torch.cuda.synchronize()
        assert torch.equal(bufs.res[1], want), "residual epilogue differs from the partials path"
        if M > 1:
            assert rel_err(bufs.ss[1].cpu().numpy(), O.tile_sumsq(u16(want))) <= 1e-5
        else:
            assert bool((bufs.ss[1] == -1.0).all()), "the folded launch wrote ss_out"
        assert int(bufs.cnt.abs().sum()) == 0
    if static:
        ref_y = _fp8_oracle(u16(a_), q, 1, sa.inv.item(), sa.scale.item()).sum(0)
    else:
        ref_y = _fp8_oracle(u16(a_), q).sum(0)
    ref = O.bf16_to_f32(O.residual_add(ref_y, u16(res)))
    assert rel_err(bufs.res[1].float().cpu().numpy(), ref) <= TOL


def test_fp8_layer_fragment_like_the_engine(dev):
    """o (ep) -> gate_up (norm, SwiGLU) -> down (ep) -> next qkv (norm) on FP8 weights with
    per-token scales at M = 1. Each stage is checked against the oracle on the inputs that stage
    actually received (the previous stage's GPU output): chaining two independent runs would
    compound re-quantization, since a one-ulp change of a residual element can move the per-token
    amax and with it every e4m3 code of the next stage."""
    from kernels import fp8 as F
    M = 1
    cur, a_ = bf((M, H), 110), bf((M, 4096), 111)
    ws = {n: bf(s, 112 + i, 0.02) for i, (n, s) in enumerate([("o", (H, 4096)), ("gu", (2 * I, H)),
                                                               ("down", (H, I)), ("qkv", (NQKV, H))])}
    q = {n: F.quantize(w.to(dev)) for n, w in ws.items()}
    ln2 = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(120))).to(torch.bfloat16)
    ln1 = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(121))).to(torch.bfloat16)
    bufs = FusedLayerBuffers(M, H, V, dev)
    d = lambda t: t.to(dev)
    gemv_fused(d(a_), q["o"], 4, ep=(d(cur), bufs.res[1], bufs.ss[1], bufs.cnt))
    act_d = gemv_swiglu_fused(bufs.res[1], q["gu"], norm=(d(ln2), bufs.ss[1]), eps=EPS)
    gemv_fused(act_d, q["down"], 4, ep=(bufs.res[1], bufs.res[0], bufs.ss[0], bufs.cnt))
    qkv = gemv_fused(bufs.res[0], q["qkv"], 2, norm=(d(ln1), bufs.ss[0]), eps=EPS)
    res_b, act, res_a = u16(bufs.res[1]), u16(act_d), u16(bufs.res[0])
    # stage by stage
    ref_b = O.residual_add(_fp8_oracle(u16(a_), q["o"]).sum(0), u16(cur))
    h2 = O.rmsnorm_rows(res_b, O.tile_sumsq(res_b).sum(1), u16(ln2), EPS)
    full = _fp8_oracle(h2, q["gu"])[0]
    ref_act = O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32))
    ref_a = O.residual_add(_fp8_oracle(act, q["down"]).sum(0), res_b)
    h1 = O.rmsnorm_rows(res_a, O.tile_sumsq(res_a).sum(1), u16(ln1), EPS)
    qkv_ref = _fp8_oracle(h1, q["qkv"], 2).sum(0)
    errs = [rel_err(O.bf16_to_f32(res_b), O.bf16_to_f32(ref_b)), rel_err(O.bf16_to_f32(act), O.bf16_to_f32(ref_act)),
            rel_err(O.bf16_to_f32(res_a), O.bf16_to_f32(ref_a)), rel_err(sum_partials(qkv), qkv_ref)]
    print("fp8 layer fragment, per stage max-rel: " + " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) <= TOL


@pytest.mark.parametrize("protocol", [True, False])
def test_fp8_fused_graph_replays(dev, monkeypatch, protocol):
    """FP8 residual epilogue and RMSNorm prologue captured in a graph: replays equal eager, with
    eager calls in between, and the counters stay zero (with and without the split-K protocol)."""
    from kernels import fp8 as F
    from kernels import fused_gemv as FG
    if protocol:
        monkeypatch.setattr(FG, "EP_SPLIT", None)
    M = 1
    a_, res = bf((M, 4096), 130), bf((M, H), 131)
    q_o = F.quantize(bf((H, 4096), 132, 0.02).to(dev))
    q_qkv = F.quantize(bf((NQKV, H), 133, 0.02).to(dev))
    ln = torch.ones(H, dtype=torch.bfloat16, device=dev)
    ad, rd = a_.to(dev), res.to(dev)
    bufs = FusedLayerBuffers(M, H, V, dev)
    out = {}

    def step():
        gemv_fused(ad, q_o, 4, ep=(rd, bufs.res[1], bufs.ss[1], bufs.cnt))
        out["qkv"] = gemv_fused(bufs.res[1], q_qkv, 2, norm=(ln, bufs.ss[1]), eps=EPS)

    step()
    torch.cuda.synchronize()
    eager_res, eager_qkv = bufs.res[1].clone(), out["qkv"].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    graph_qkv = out["qkv"]
    for _ in range(3):
        bufs.res[1].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(bufs.res[1], eager_res) and torch.equal(graph_qkv, eager_qkv)
        step()
    assert int(bufs.cnt.abs().sum()) == 0
    del g


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rmsnorm_rounding_all_bf16_products(dev, seed):
    """The RMSNorm's bf16 roundings (a hardware fp32 -> bf16 convert) against the oracle's round to
    nearest even: with partials summing to exactly K and eps = 0, rstd = 1 and h = bf16(x * ln), an
    exact fp32 product rounded once; x runs over all 65,536 bf16 patterns (ties, overflow to inf,
    subnormal products), ln over random finite patterns. NaN inputs only need to stay NaN."""
    from kernels import _lib as L
    M, K = 16, 4096
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(M, K)
    g = torch.Generator().manual_seed(300 + seed)
    lnb = torch.randint(0, 65536, (K,), generator=g, dtype=torch.int32).to(torch.int16)
    lnb = torch.where((lnb.int() & 0x7F80) == 0x7F80, lnb & 0x3FFF, lnb)  # finite ln
    ln = lnb.view(torch.bfloat16)
    ss = torch.full((M, K // 16), 16.0, dtype=torch.float32)
    xd, lnd, ssd = x.to(dev), ln.to(dev), ss.to(dev)
    h = torch.empty_like(xd)
    L.call("krq_rmsnorm_rows", L.ptr(xd), L.ptr(ssd), L.ptr(lnd), 0.0, M, K, L.ptr(h), L.stream(xd))
    got = u16(h)
    with np.errstate(over="ignore", invalid="ignore"):
        want = O.f32_to_bf16((O.bf16_to_f32(u16(x)) * O.bf16_to_f32(u16(ln))[None, :]).astype(np.float32))
    nan_w = np.isnan(O.bf16_to_f32(want))
    assert np.array_equal(np.isnan(O.bf16_to_f32(got)), nan_w)
    bad = (got != want) & ~nan_w
    assert not bad.any(), f"{int(bad.sum())} mismatches, first x={u16(x)[bad][:4]} got={got[bad][:4]} want={want[bad][:4]}"
