"""Fused decode MLP (kernels.mlp.PersistentMLP(one_launch=True) over krq_mlp_fp8) against the CPU
oracle and the two-launch path (gemv_swiglu_fp8 then the per-token-scaled down GEMV). Outputs are fp32 split-K
partials [S, M, H]; the bar is max|y - ref| <= 1e-2 * max|ref| per split and summed."""

import numpy as np
import pytest
import torch

from kernels import _lib as L
from kernels import fp8
from kernels.mlp import PersistentMLP
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2
H, I = 2560, 9728


def u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _step(b, d):
    """bf16 bit patterns moved d steps away from zero (d = -1 toward zero), zero kept."""
    mag = (b & 0x7FFF).astype(np.int32)
    moved = np.clip(mag + d, 0, 0x7F7F)
    return ((b & 0x8000) | np.where(mag == 0, 0, moved)).astype(np.uint16)


def swiglu_within_one_step(got, pre):
    """got [M, I] fp32 act values; pre [M, 2I] exact gate/up sums. True where got equals the
    oracle SwiGLU of some (g, u) whose bf16 patterns are within one step of bf16(pre)."""
    I = got.shape[1]
    gb = O.f32_to_bf16(pre[:, :I].astype(np.float32))
    ub = O.f32_to_bf16(pre[:, I:].astype(np.float32))
    ok = np.zeros(got.shape, dtype=bool)
    for dg in (-1, 0, 1):
        for du in (-1, 0, 1):
            cand = O.bf16_to_f32(O.swiglu(O.bf16_to_f32(_step(gb, dg)), O.bf16_to_f32(_step(ub, du))))
            ok |= cand == got
    return ok


def case(M, h_, i_, seed):
    g = torch.Generator().manual_seed(seed)
    wgu = (torch.randn(2 * i_, h_, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(h_, i_, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, h_, generator=g).to(torch.bfloat16)
    return wgu, wd, x


@pytest.mark.parametrize("M,S", [(1, 4), (16, 4), (32, 8)])
def test_mlp_fp8_vs_oracle(dev, M, S):
    wgu, wd, x = case(M, H, I, 40 + M)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    pm = PersistentMLP(M, H, I, dev, split=S, one_launch=True)
    out = pm(x.to(dev), qgu, qd)
    assert out.shape == (S, M, H) and out.dtype == torch.float32
    act_ref, parts = O.mlp_fp8(u16(x), u8(qgu[0]), qgu[1].cpu().numpy(), u8(qd[0]),
                               qd[1].cpu().numpy(), S)
    x8r, xsr = O.quant_rows(u16(x))
    _, act_pre = O.fp8_matmul(x8r, xsr, u8(qgu[0]), qgu[1].cpu().numpy())
    got_act = pm.act.float().cpu().numpy()
    ref_act = O.bf16_to_f32(act_ref)
    mism = float(np.mean(got_act != ref_act))
    y = out.cpu().numpy()
    e_parts = max(rel_err(y[s], parts[s]) for s in range(S))
    e_sum = rel_err(y.sum(0), parts.sum(0))
    print(f"mlp M={M} S={S}: act mismatches {mism:.2e}, act max-rel {rel_err(got_act, ref_act):.2e}, "
          f"partials max-rel {e_parts:.2e}, sum max-rel {e_sum:.2e}")
    # act = bf16(bf16(silu(bf16 g)) * bf16 u) of sums that the FP8 matrix cores accumulate with an
    # error of ~3e-7 (median; 2.3e-6 max) of sum|products| (measured; the oracle's sums are exact),
    # so for ~2% of columns g or u rounds to a neighbouring bf16 value - by one step except where
    # cancellation leaves the sum small against that error
    assert mism < 0.05 and rel_err(got_act, ref_act) <= TOL
    unexplained = float(np.mean(~swiglu_within_one_step(got_act, act_pre)))
    print(f"  act not explained by one-step g/u roundings: {unexplained:.2e}")
    assert unexplained < 1e-2
    assert np.all(np.abs(got_act - ref_act) <= 2 ** -5 * np.abs(ref_act) + 2 ** -10 * np.abs(ref_act).max())
    assert e_parts <= TOL and e_sum <= TOL
    assert not pm.failed()


@pytest.mark.parametrize("M", [1, 16])
def test_mlp_fp8_matches_two_launch_path(dev, M):
    wgu, wd, x = case(M, H, I, 50 + M)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    xd = x.to(dev)
    pm = PersistentMLP(M, H, I, dev, one_launch=True)
    out = pm(xd, qgu, qd)
    a = fp8.gemv_swiglu_fp8(xd, qgu)
    sep = fp8.gemv_fp8(a, qd, 4)
    ga, sa = pm.act.float().cpu().numpy(), a.float().cpu().numpy()
    assert np.mean(ga != sa) < 1e-3 and rel_err(ga, sa) <= TOL
    assert rel_err(out.sum(0).cpu().numpy(), sep.sum(0).cpu().numpy()) <= TOL


@pytest.mark.parametrize("programs", [1, 3, 256, 100000])
def test_mlp_any_block_count_same_result(dev, programs):
    """One block, a few, one per CU, or more than the device holds (clamped): every launch
    finishes and gives identical bits (an item's arithmetic does not depend on which block runs
    it), and leaves the control words zero."""
    M, h_, i_ = 16, 512, 1024
    wgu, wd, x = case(M, h_, i_, 60)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    xd = x.to(dev)
    ref = PersistentMLP(M, h_, i_, dev, one_launch=True)(xd, qgu, qd)
    pm = PersistentMLP(M, h_, i_, dev, programs=programs, one_launch=True)
    out = pm(xd, qgu, qd)
    assert torch.equal(out, ref)
    assert not pm.failed() and int(pm.ctl.abs().sum()) == 0


def test_mlp_rowmajor_equals_tiled(dev):
    M = 1
    wgu, wd, x = case(M, H, I, 70)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    rgu, rd = fp8.FP8Weight(qgu[0], qgu[1], None), fp8.FP8Weight(qd[0], qd[1], None)
    xd = x.to(dev)
    pm = PersistentMLP(M, H, I, dev, one_launch=True)
    a = pm(xd, qgu, qd)
    b = pm(xd, rgu, rd)
    assert torch.equal(a, b)


def test_mlp_counters_reset_across_calls_and_graph_replays(dev):
    M = 1
    wgu, wd, x = case(M, H, I, 80)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    xd = x.to(dev)
    pm = PersistentMLP(M, H, I, dev, one_launch=True)
    first = pm(xd, qgu, qd).clone()
    for _ in range(3):
        assert torch.equal(pm(xd, qgu, qd), first)
    assert int(pm.ctl.abs().sum()) == 0
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pm(xd, qgu, qd)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = pm(xd, qgu, qd)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        # eager work between replays
        assert torch.equal(pm(xd, qgu, qd), first)
    assert not pm.failed() and int(pm.ctl.abs().sum()) == 0
    del g


@pytest.mark.parametrize("M", [1, 16])
def test_mlp_bf16_weights(dev, M):
    """BF16 weights (the reference engine's call, engine/engine.py:911-915): the same contract,
    fp32 partials [S, M, H] whose in-order sum is the product, against the oracle (bf16 matmul,
    SwiGLU rounding chain, bf16 matmul)."""
    from kernels import gemv as G
    g = torch.Generator().manual_seed(500 + M)
    h = torch.randn(M, H, generator=g).to(torch.bfloat16)
    wgu = (torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16)
    pm = PersistentMLP(M, H, I, dev)
    out = pm(h.to(dev), wgu.to(dev), wd.to(dev))
    assert out.shape == (4, M, H) and out.dtype == torch.float32
    full = O.bf16_matmul(u16(h), u16(wgu))
    act = O.swiglu(full[:, :I].astype(np.float32), full[:, I:].astype(np.float32))
    ref = O.bf16_matmul(act, u16(wd))
    assert rel_err(pm.act.float().cpu().numpy(), O.bf16_to_f32(act)) <= TOL
    y = out[0].clone()
    for s in range(1, 4):
        y += out[s]
    assert rel_err(y.cpu().numpy(), ref) <= TOL
    # the same kernels as the two GEMV calls
    assert torch.equal(out, G.gemv(G.gemv_swiglu(h.to(dev), wgu.to(dev)), wd.to(dev), 4))


@pytest.mark.parametrize("M", [1, 16])
def test_mlp_default_is_the_two_launch_pair(dev, M):
    """PersistentMLP's default form for FP8 weights is the two GEMV launches: bit-identical to
    calling them directly."""
    wgu, wd, x = case(M, H, I, 90 + M)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    xd = x.to(dev)
    out = PersistentMLP(M, H, I, dev)(xd, qgu, qd)
    assert torch.equal(out, fp8.gemv_fp8(fp8.gemv_swiglu_fp8(xd, qgu), qd, 4))


def test_mlp_wait_timeout_poisons_partials(dev):
    """A phase-1 wait that gives up (forced from the host with a bound of 0 polls) sets the error
    word and makes that block's partials NaN; every other partial equals the good launch's. The
    kernel still ends (every wait is bounded) and the next launch is good again."""
    M, h_, i_ = 16, 512, 1024
    wgu, wd, x = case(M, h_, i_, 61)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    xd = x.to(dev)
    good = PersistentMLP(M, h_, i_, dev, one_launch=True)(xd, qgu, qd)
    pm = PersistentMLP(M, h_, i_, dev, one_launch=True)
    out = pm(xd, qgu, qd, max_polls=0)
    torch.cuda.synchronize()
    nan = torch.isnan(out)
    print(f"timed-out partials: {int(nan.sum())} of {out.numel()}, flagged {pm.failed()}")
    assert torch.equal(out[~nan], good[~nan])
    assert pm.failed() == bool(nan.any())
    pm.ctl.zero_()
    assert torch.equal(pm(xd, qgu, qd), good) and not pm.failed()


def _shared(t, headroom):
    """A SharedScale slot pair filled the engine's way: the tensor's amax times a headroom
    (engine.py:666-668 takes the prefill amax x FP8_DECODE_HEADROOM)."""
    a = fp8.ActScale(t, headroom=headroom)
    return fp8.SharedScale(a.inv.clone(), a.scale.clone())


@pytest.mark.parametrize("M", [1, 4, 16, 32])
@pytest.mark.parametrize("sites", ["static", "per_token", "per_channel"])
def test_swiglu_cast_is_the_cast_of_act(dev, M, sites):
    """fp8.swiglu_cast_fp8 writes, bit for bit, the tiled permutation (pad rows zero) of
    _cast(act, a_down), where act is gemv_swiglu_fp8's bf16 output on the same operands: the down
    input of the engine's static-scale decode MLP (engine.py:977-981) without the bf16 act or a
    cast launch. With a_down's headroom below 1 some of act clamps to +-448. Then
    mlp.mlp_fp8_static equals the down GEMV on those rows and the exact oracle of that product."""
    from kernels.mlp import mlp_fp8_static
    wgu, wd, x = case(M, H, I, 900 + M)
    wq = fp8.quantize if sites == "per_channel" else fp8.quantize_weight
    q_gu, q_d = wq(wgu.to(dev)), wq(wd.to(dev))
    xd = x.to(dev)
    a_gu = None if sites == "per_token" else _shared(xd, 2.0)
    act = fp8.gemv_swiglu_fp8(xd, q_gu, a=a_gu)
    for headroom in (2.0, 0.25):
        a_d = _shared(act, headroom)
        x8t, sc = fp8.swiglu_cast_fp8(xd, q_gu, a_d, a=a_gu)
        ref8 = u8(fp8._cast(act, a_d))
        MP = 16 * ((M + 15) // 16)
        padded = np.zeros((MP, I), dtype=np.uint8)
        padded[:M] = ref8
        assert np.array_equal(u8(x8t), O.tile(padded)), headroom
        assert np.array_equal(ref8, O.cast(u16(act), np.float32(a_d.inv.item())))
        for split in (1, 4):
            y = mlp_fp8_static(xd, q_gu, q_d, a_gu, a_d, split)
            mode = L.OUT_BF16 if split == 1 else L.OUT_PARTIAL
            assert torch.equal(y, fp8.gemv_fp8_tiled_launch(x8t, sc, q_d, M, split, mode))
            yf = y.float().cpu().numpy() if split == 1 else y.double().sum(0).cpu().numpy()
            _, yref = O.fp8_matmul(ref8, np.float32(sc.item()), u8(q_d[0]), q_d[1].cpu().numpy())
            assert rel_err(yf, yref) <= TOL, (headroom, split)


# ---- the chained form: gate_up and down in one launch at M == 1 (krq_mlp_chain_fp8) ----

# (H, I, split): Qwen3-4B (mixed gate_up plan, 19 steps per down split), a grid below one block
# per CU, and an odd tile count per split (23 tiles: the last step's high tile masked)
CHAIN_SHAPES = [(H, I, 4), (1024, 3072, 2), (512, 1472, 1)]



@pytest.mark.parametrize("h_,i_,S", CHAIN_SHAPES)
def test_mlp_chain_matches_pair_and_oracle(dev, h_, i_, S):
    """Two different rows in a row (a stale line of the first call's act would show in the
    second): act bit-identical to the two-launch pair's, partials equal to the pair's to fp32
    rounding (a down block sums two weight waves where the standalone GEMV may use one), the last
    call within the oracle's bar; the control words are zero after every call."""
    wgu, wd, _ = case(1, h_, i_, 110)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    pm = PersistentMLP(1, h_, i_, dev, split=S, chunk=64, chained=True)
    g = torch.Generator().manual_seed(111)
    for call in range(2):
        x = (torch.randn(1, h_, generator=g) * (1 + 3 * call)).to(torch.bfloat16)
        xd = x.to(dev)
        out = pm(xd, qgu, qd)
        a = fp8.gemv_swiglu_fp8(xd, qgu)
        sep = fp8.gemv_fp8_bf16_launch(a, qd, S, L.OUT_PARTIAL, None, L.ALGO_AUTO)  # (fp32 also at S = 1)
        torch.cuda.synchronize()
        assert out.shape == (S, 1, h_) and out.dtype == torch.float32
        assert torch.equal(pm.act, a), f"call {call}: act differs from the SwiGLU GEMV's"
        y, ys = out.cpu().numpy(), sep.cpu().numpy()
        e_pair = max(rel_err(y[s], ys[s]) for s in range(S))
        print(f"chain H={h_} I={i_} S={S} call {call}: partials vs pair max-rel {e_pair:.2e}, "
              f"bit-equal {float(np.mean(y == ys)):.3f}")
        assert e_pair <= 1e-5
        assert not pm.failed() and int(pm.ctl.abs().sum()) == 0
    act_ref, parts = O.mlp_fp8(u16(x), u8(qgu[0]), qgu[1].cpu().numpy(), u8(qd[0]), qd[1].cpu().numpy(), S)
    e_parts = max(rel_err(y[s], parts[s]) for s in range(S))
    assert rel_err(pm.act.float().cpu().numpy(), O.bf16_to_f32(act_ref)) <= TOL
    assert e_parts <= TOL and rel_err(y.sum(0), parts.sum(0)) <= TOL


def test_mlp_chain_graph_replays(dev):
    """Replays of a captured chained launch, with a new row copied in between and eager calls
    between replays: every replay equals the eager result for its row (the control words reset
    themselves, and act is read from memory, not from a line cached by an earlier replay)."""
    wgu, wd, _ = case(1, H, I, 120)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    g = torch.Generator().manual_seed(121)
    xs = [torch.randn(1, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
    pm = PersistentMLP(1, H, I, dev, chained=True)
    eager = [pm(x, qgu, qd).clone() for x in xs]
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pm(static_x, qgu, qd)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out = pm(static_x, qgu, qd)
    for r in range(6):
        static_x.copy_(xs[r % 3])
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[r % 3]), r
        assert torch.equal(pm(xs[(r + 1) % 3], qgu, qd), eager[(r + 1) % 3]), r
    assert not pm.failed() and int(pm.ctl.abs().sum()) == 0
    del gr


def test_mlp_chain_wait_timeout_poisons_partials(dev):
    """Waits bounded at one poll (forced from the host): a down block that gives up sets the
    error word and writes NaN partials; every other partial equals the good launch's; the launch
    ends. After zero_ctl() the next launch is good again and leaves the words zero."""
    wgu, wd, x = case(1, H, I, 130)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    xd = x.to(dev)
    pm = PersistentMLP(1, H, I, dev, chained=True)
    good = pm(xd, qgu, qd).clone()
    out = pm(xd, qgu, qd, max_polls=1)
    torch.cuda.synchronize()
    nan = torch.isnan(out)
    print(f"timed-out partials: {int(nan.sum())} of {out.numel()}, flagged {pm.failed()}")
    assert torch.equal(out[~nan], good[~nan])
    assert pm.failed() == bool(nan.any())
    pm.zero_ctl()
    assert torch.equal(pm(xd, qgu, qd), good) and not pm.failed()
    assert int(pm.ctl.abs().sum()) == 0


def test_mlp_chain_rejects_bad_plans(dev):
    """M > 1, row-major weights and splits past the ring raise instead of launching."""
    wgu, wd, x = case(1, 512, 3072, 140)
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    with pytest.raises(ValueError, match="M == 1"):
        PersistentMLP(2, 512, 3072, dev, chained=True)(torch.cat([x, x]).to(dev), qgu, qd)
    pm = PersistentMLP(1, 512, 3072, dev, split=1, chained=True)  # 24 steps of 128 in one split
    with pytest.raises(ValueError, match="ring"):
        pm(x.to(dev), qgu, qd)
    rgu, rd = fp8.FP8Weight(qgu[0], qgu[1], None), fp8.FP8Weight(qd[0], qd[1], None)
    with pytest.raises(ValueError, match="tiled"):
        PersistentMLP(1, 512, 3072, dev, split=2, chained=True)(x.to(dev), rgu, rd)


# ---- the chained form on BF16 weights (krq_mlp_chain_bf16), any M ----

# (M, H, I, split, packed): Qwen3-4B at one row (vector-ALU blocks, mixed gate_up plan), four,
# sixteen and 32 rows (two row tiles), on tiled and row-major weights; a grid below one block per
# CU with four down waves beside two gate_up waves; an odd step count per split
CHAIN_BF16_CASES = [(1, H, I, 4, True), (1, H, I, 4, False), (4, H, I, 4, True), (16, H, I, 4, True),
                    (32, H, I, 4, False), (1, 1024, 3072, 2, True), (3, 512, 1472, 1, False)]


def bf16_case(M, h_, i_, seed, packed):
    from kernels import gemv as G
    wgu, wd, _ = case(M, h_, i_, seed)
    wgu, wd = wgu.to("cuda"), wd.to("cuda")
    if packed:
        G.pack(wgu)
        G.pack(wd)
    return wgu, wd


@pytest.mark.parametrize("M,h_,i_,S,packed", CHAIN_BF16_CASES)
def test_mlp_chain_bf16_matches_pair(dev, M, h_, i_, S, packed):
    """Two different row sets in a row: act and the partials bit-identical to the two BF16 GEMV
    launches (each stage runs its standalone plan), the control words zero after every call, and
    the last call within the oracle's bar (bf16 matmul, SwiGLU rounding chain, bf16 matmul)."""
    from kernels import gemv as G
    wgu, wd = bf16_case(M, h_, i_, 600 + M, packed)
    pm = PersistentMLP(M, h_, i_, dev, split=S, chunk=64, chained=True)
    g = torch.Generator().manual_seed(601 + M)
    for call in range(2):
        x = (torch.randn(M, h_, generator=g) * (1 + 3 * call)).to(torch.bfloat16)
        xd = x.to(dev)
        out = pm(xd, wgu, wd)
        a = G.gemv_swiglu(xd, wgu)
        sep = G.gemv(a, wd, S) if S > 1 else G._launch(a, wd, 1, L.OUT_PARTIAL)
        torch.cuda.synchronize()
        assert out.shape == (S, M, h_) and out.dtype == torch.float32
        assert torch.equal(pm.act, a), f"call {call}: act differs from the SwiGLU GEMV's"
        assert torch.equal(out, sep), f"call {call}: partials differ from the down GEMV's"
        assert not pm.failed() and int(pm.ctl.abs().sum()) == 0
    full = O.bf16_matmul(u16(x), u16(wgu))
    act = O.swiglu(full[:, :i_].astype(np.float32), full[:, i_:].astype(np.float32))
    ref = O.bf16_matmul(act, u16(wd))
    assert rel_err(pm.act.float().cpu().numpy(), O.bf16_to_f32(act)) <= TOL
    assert rel_err(out.double().sum(0).cpu().numpy(), ref) <= TOL


def test_mlp_bf16_one_launch_is_the_chain(dev):
    """one_launch=True on BF16 weights runs the chained launch: the pair's partials, one launch."""
    from kernels import gemv as G
    wgu, wd = bf16_case(1, H, I, 610, True)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(611)).to(torch.bfloat16).to(dev)
    pm = PersistentMLP(1, H, I, dev, one_launch=True)
    out = pm(x, wgu, wd)
    assert torch.equal(out, G.gemv(G.gemv_swiglu(x, wgu), wd, 4))
    assert not pm.failed() and int(pm.ctl.abs().sum()) == 0


def test_mlp_chain_bf16_graph_replays(dev):
    """Replays of a captured BF16 chained launch with a new row copied in between and eager calls
    between replays: every replay equals the eager result for its row."""
    wgu, wd = bf16_case(1, H, I, 620, True)
    g = torch.Generator().manual_seed(621)
    xs = [torch.randn(1, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
    pm = PersistentMLP(1, H, I, dev, chained=True)
    eager = [pm(x, wgu, wd).clone() for x in xs]
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pm(static_x, wgu, wd)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out = pm(static_x, wgu, wd)
    for r in range(6):
        static_x.copy_(xs[r % 3])
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[r % 3]), r
        assert torch.equal(pm(xs[(r + 1) % 3], wgu, wd), eager[(r + 1) % 3]), r
    assert not pm.failed() and int(pm.ctl.abs().sum()) == 0
    del gr


def test_mlp_chain_bf16_wait_timeout_poisons_partials(dev):
    """Waits bounded at one poll (forced from the host): a down block that gives up sets the error
    word and writes NaN partials, every other partial equals the good launch's, and the launch
    ends; after zero_ctl() the next launch is good again."""
    wgu, wd = bf16_case(1, H, I, 630, True)
    xd = torch.randn(1, H, generator=torch.Generator().manual_seed(631)).to(torch.bfloat16).to(dev)
    pm = PersistentMLP(1, H, I, dev, chained=True)
    good = pm(xd, wgu, wd).clone()
    out = pm(xd, wgu, wd, max_polls=1)
    torch.cuda.synchronize()
    nan = torch.isnan(out)
    print(f"bf16 timed-out partials: {int(nan.sum())} of {out.numel()}, flagged {pm.failed()}")
    assert torch.equal(out[~nan], good[~nan])
    assert pm.failed() == bool(nan.any())
    pm.zero_ctl()
    assert torch.equal(pm(xd, wgu, wd), good) and not pm.failed()
    assert int(pm.ctl.abs().sum()) == 0


def test_mlp_chain_bf16_rejects_bad_plans(dev):
    """A down grid the standalone GEMV would pair (4096 blocks above 4 rows) and mixed layouts
    raise instead of launching."""
    from kernels import gemv as G
    with pytest.raises(ValueError):
        PersistentMLP(1, H, I, dev, chained=True, one_launch=True)
    h_, i_ = 16384, 256
    wgu, wd = bf16_case(8, h_, i_, 640, False)
    x = torch.zeros(8, h_, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="4096"):
        PersistentMLP(8, h_, i_, dev, split=4, chunk=64, chained=True)(x, wgu, wd)
    G.pack(wgu)
    with pytest.raises(ValueError, match="layout"):
        PersistentMLP(8, h_, i_, dev, split=4, chunk=64, chained=True)(x, wgu, wd)
