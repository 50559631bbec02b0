"""NaN and inf in quantizer inputs: every max-based scale must propagate them as the reference's
torch reductions do (engine/kernels/fp8.py:21 `wf.abs().max()`, :31-32 `torch.aminmax` +
`torch.maximum`, the per-row `amax(1)` of experiments/modal_fq.py:46-47, :62-63, each floored
with `clamp_min`, which keeps NaN).

  NaN in a row (or tensor)  -> amax NaN, scale NaN, inv NaN, every byte of it a NaN code, and a
                               GEMV output row of NaN;
  +-inf in a row            -> amax inf, scale inf, inv 0: finite elements quantize to signed
                               zeros, the inf element to a NaN code (inf / inf, inf * 0).

Comparisons are NaN-aware: a NaN scale equals a NaN scale, and an e4m3 NaN code (S.1111.111)
equals a NaN code of either sign, because the sign a NaN picks up from a multiply or divide
depends on operand order and on the host (x86 makes the default NaN negative, the GPU
positive); every other scale and byte must be equal bit for bit. Rows without a planted value
must equal the quantization of the same rows with nothing planted.
"""

import numpy as np
import pytest
import torch

from kernels import fp8, lmhead
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NAN, INF = float("nan"), float("inf")


def u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


def weight(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)


def act(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(torch.bfloat16)


def assert_codes(got, ref):
    got, ref = np.asarray(got, np.uint8), np.asarray(ref, np.uint8)
    gn, rn = (got & 0x7F) == 0x7F, (ref & 0x7F) == 0x7F
    assert np.array_equal(gn, rn), f"NaN codes at different places ({int(gn.sum())} vs {int(rn.sum())})"
    assert np.array_equal(got[~gn], ref[~rn])


def assert_f32(got, ref):
    got = np.asarray(got, np.float32).reshape(-1)
    ref = np.asarray(ref, np.float32).reshape(-1)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN at different places: {got} vs {ref}"
    assert np.array_equal(got[~gn].view(np.uint32), ref[~rn].view(np.uint32))


# rows: 3 holds a NaN, 5 a +inf, 9 a -inf
PLANT = {3: NAN, 5: INF, 9: -INF}


def planted(t, where=PLANT, col=17):
    t = t.clone()
    for r, v in where.items():
        if r < t.shape[0]:
            t[r, min(col + r, t.shape[1] - 1)] = v
    return t


# ---------------------------------------------------------------------------------------------
# weight quantizers
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,K", [(64, 2560), (48, 200)])  # vector kernel, scalar kernel
def test_quantize_per_channel_nan_inf(dev, N, K):
    clean = weight(N, K, 31)
    w = planted(clean)
    q = fp8.quantize(w.to(dev))
    r8, rs = O.quantize(u16(w))
    assert_codes(u8(q[0]), r8)
    assert_f32(q[1].cpu().numpy(), rs)
    s = q[1].cpu().numpy()
    assert np.isnan(s[3]) and s[5] == np.inf and s[9] == np.inf
    assert np.all((u8(q[0][3]) & 0x7F) == 0x7F)
    # the reference expression evaluated by torch on this device
    wf = w.to(dev).float()
    sd = wf.abs().amax(1).clamp_min(1e-12) / fp8.FP8_MAX
    ref = (wf / sd[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert_f32(q[1].cpu().numpy(), sd.cpu().numpy())
    assert_codes(u8(q[0]), u8(ref))
    # other rows as without the planted values
    qc = fp8.quantize(clean.to(dev))
    keep = [r for r in range(N) if r not in PLANT]
    assert np.array_equal(u8(q[0])[keep], u8(qc[0])[keep])
    assert np.array_equal(q[1].cpu().numpy()[keep], qc[1].cpu().numpy()[keep])
    if q.tiled is not None:
        assert_codes(q.tiled.cpu().numpy(), O.tile(r8))


@pytest.mark.parametrize("v", [NAN, INF, -INF])
@pytest.mark.parametrize("N,K", [(64, 2560), (48, 200)])
def test_quantize_weight_per_tensor_nan_inf(dev, v, N, K):
    w = weight(N, K, 33)
    w[7, 11] = v
    q = fp8.quantize_weight(w.to(dev))
    r8, rs = O.quantize_weight(u16(w))
    assert_f32(q[1].cpu().numpy(), rs)
    assert_codes(u8(q[0]), r8)
    wf = w.to(dev).float()
    scale = (wf.abs().max().clamp_min(1e-12) / fp8.FP8_MAX).reshape(())
    ref = (wf / scale).clamp_(-448, 448).to(torch.float8_e4m3fn)
    assert_f32(q[1].cpu().numpy(), scale.cpu().numpy())
    assert_codes(u8(q[0]), u8(ref))
    if v != v:
        assert np.all((u8(q[0]) & 0x7F) == 0x7F)
    else:
        b = u8(q[0])
        assert (b[7, 11] & 0x7F) == 0x7F and np.count_nonzero(b & 0x7F) == 1   # signed zeros elsewhere


# ---------------------------------------------------------------------------------------------
# activation scales and per-token quantization
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("v", [NAN, INF, -INF])
def test_act_scale_nan_inf(dev, v):
    x = act(16, 2560, 35)
    x[4, 100] = v
    xd = x.to(dev)
    a = fp8.ActScale(xd)
    amax, inv, scale = O.act_scale(u16(x))
    assert_f32(a.amax.cpu().numpy(), amax)
    assert_f32(a.inv.cpu().numpy(), inv)
    assert_f32(a.scale.cpu().numpy(), scale)
    mn, mx = torch.aminmax(xd)
    am = torch.maximum(-mn, mx).float().clamp_min(1e-6)
    assert_f32(a.amax.cpu().numpy(), am.cpu().numpy())
    assert_f32(a.inv.cpu().numpy(), (fp8.FP8_MAX / am).cpu().numpy())
    assert_codes(u8(fp8._cast_hip(xd, a)), O.cast(u16(x), inv))
    assert_codes(u8(fp8._cast_hip(xd, a)), u8(fp8._cast_torch(xd, a)))


@pytest.mark.parametrize("v", [None, NAN, INF, -INF])
@pytest.mark.parametrize("M,K", [(40, 2560), (300, 9728), (33, 100), (64, 4104)])
def test_act_scale_cast_is_act_scale_then_cast(dev, M, K, v):
    """linear_fp8's first steps without a given scale (engine/kernels/fp8.py:97-104) in two
    launches (krq_act_scale_cast_fp8: the vector maximum pass, then the cast folding the partial
    maxima itself; M K % 8 != 0 takes the scalar passes): the scale and bytes of ActScale then
    _cast_hip, and of the oracle, NaN and inf included."""
    x = act(M, K, 36 + M)
    if v is not None:
        x[M // 2, K // 3] = v
    xd = x.to(dev)
    a, y = fp8._act_scale_cast(xd)
    a2 = fp8.ActScale(xd)
    assert_f32(a.amax.cpu().numpy(), a2.amax.cpu().numpy())
    assert_f32(a.inv.cpu().numpy(), a2.inv.cpu().numpy())
    assert_f32(a.scale.cpu().numpy(), a2.scale.cpu().numpy())
    assert_codes(u8(y), u8(fp8._cast_hip(xd, a2)))
    amax, inv, scale = O.act_scale(u16(x))
    assert_f32(a.amax.cpu().numpy(), amax)
    assert_f32(a.scale.cpu().numpy(), scale)
    assert_codes(u8(y), O.cast(u16(x), inv))


# 512-thread kernel (K % 16 == 0), 8-value chunk kernel (K % 16 == 8), scalar kernel (K % 8 != 0,
# and rows longer than the vector kernels hold)
@pytest.mark.parametrize("M,K", [(16, 2560), (12, 200), (11, 100), (10, 20000)])
def test_quant_rows_nan_inf(dev, M, K):
    clean = act(M, K, 37 + K)
    x = planted(clean)
    x8, xs = fp8.quant_rows(x.to(dev))
    r8, rs = O.quant_rows(u16(x))
    assert_codes(u8(x8), r8)
    assert_f32(xs.cpu().numpy(), rs)
    s = xs.cpu().numpy().reshape(-1)
    assert np.isnan(s[3]) and s[5] == np.inf and s[9] == np.inf
    c8, cs = fp8.quant_rows(clean.to(dev))
    keep = [r for r in range(M) if r not in PLANT]
    assert np.array_equal(u8(x8)[keep], u8(c8)[keep])
    assert np.array_equal(s[keep], cs.cpu().numpy().reshape(-1)[keep])


@pytest.mark.parametrize("M", [10, 16, 20])
def test_quant_rows_tiled_nan_inf(dev, M):
    K = 2560
    x = planted(act(M, K, 39 + M))
    x8t, xs = fp8.quant_rows_tiled(x.to(dev))
    r8, rs = O.quant_rows(u16(x))
    mp = (M + 15) // 16 * 16
    pad = np.zeros((mp, K), dtype=np.uint8)
    pad[:M] = r8
    assert_codes(x8t.cpu().numpy(), O.tile(pad))
    assert_f32(xs.cpu().numpy(), rs)


# ---------------------------------------------------------------------------------------------
# GEMVs that quantize their activations themselves
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,K,split", [(6144, 2560, 1), (6144, 2560, 2), (2560, 9728, 4), (64, 384, 1)])
@pytest.mark.parametrize("v", [NAN, INF])
def test_one_row_gemv_nan_inf(dev, N, K, split, v):
    """M = 1 with bf16 input: the per-token scale is taken inside the GEMV (the activation wave at
    the Qwen3-4B shapes, every wave's shared prologue on the small grid). A NaN or inf in the row
    makes the whole output NaN, as quant_rows + the exact product does."""
    w = weight(N, K, 41)
    x = act(1, K, 43)
    x[0, K // 3] = v
    q = fp8.quantize(w.to(dev))
    y = fp8.gemv_fp8(x.to(dev), q, split)
    x8r, xsr = O.quant_rows(u16(x))
    with np.errstate(invalid="ignore"):
        _, yref = O.fp8_matmul(x8r, xsr, u8(q[0]), q[1].cpu().numpy())
    assert np.all(np.isnan(yref))
    assert torch.isnan(y).all()


def test_swiglu_gemv_nan_row(dev):
    w = weight(19456, 2560, 45)
    x = act(1, 2560, 47)
    x[0, 5] = NAN
    q = fp8.quantize(w.to(dev))
    assert torch.isnan(fp8.gemv_swiglu_fp8(x.to(dev), q)).all()


@pytest.mark.parametrize("M", [2, 16, 32])
def test_multi_row_gemv_nan_row(dev, M):
    """1 < M <= 32 (quant_rows_tiled, then the GEMV on the tiled rows): the planted row's outputs
    are NaN, every other row meets the parity bar against the exact oracle."""
    N, K = 6144, 2560
    w = weight(N, K, 49)
    x = act(M, K, 51)
    bad = M - 1
    x[bad, 7] = NAN
    q = fp8.quantize(w.to(dev))
    y = fp8.gemv_fp8(x.to(dev), q).float().cpu().numpy()
    x8r, xsr = O.quant_rows(u16(x))
    with np.errstate(invalid="ignore"):
        _, yref = O.fp8_matmul(x8r, xsr, u8(q[0]), q[1].cpu().numpy())
    assert np.all(np.isnan(y[bad])) and np.all(np.isnan(yref[bad]))
    good = [m for m in range(M) if m != bad]
    assert not np.isnan(y[good]).any()
    err = np.abs(y[good] - yref[good]).max() / np.abs(yref[good]).max()
    assert err <= 1e-2


def test_rmsnorm_quant_rows_nan(dev):
    """krq_rmsnorm_quant_rows: a NaN in the normalized row makes its scale NaN and its bytes NaN
    codes (the amax over h keeps NaN); other rows are unchanged."""
    from kernels import _lib as L
    M, K, EPS = 4, 2560, 1e-6
    g = torch.Generator().manual_seed(53)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ln = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    ss = O.tile_sumsq(u16(x)).astype(np.float32)
    xn = x.clone()
    xn[2, 30] = NAN   # the partials stay those of the clean row: only the NaN element differs
    outs = []
    for xx in (x, xn):
        xd, lnd, ssd = xx.to(dev), ln.to(dev), torch.from_numpy(ss).to(dev)
        x8 = torch.empty((M, K), device=dev, dtype=torch.float8_e4m3fn)
        xs = torch.empty((M,), device=dev, dtype=torch.float32)
        L.call("krq_rmsnorm_quant_rows", L.ptr(xd), L.ptr(ssd), L.ptr(lnd), EPS, M, K, L.ptr(x8), L.ptr(xs),
               L.stream(xd))
        outs.append((u8(x8), xs.cpu().numpy()))
    (c8, cs), (n8, ns) = outs
    assert np.isnan(ns[2]) and np.all((n8[2] & 0x7F) == 0x7F)
    keep = [0, 1, 3]
    assert np.array_equal(n8[keep], c8[keep]) and np.array_equal(ns[keep], cs[keep])


def test_mlp_one_launch_nan_row(dev):
    """The one-launch MLP's in-kernel per-token scale (M = 1) keeps NaN: every partial is NaN."""
    from kernels.mlp import PersistentMLP
    H, I = 2560, 9728
    g = torch.Generator().manual_seed(55)
    wgu = (torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(1, H, generator=g).to(torch.bfloat16)
    x[0, 9] = NAN
    qgu, qd = fp8.quantize(wgu.to(dev)), fp8.quantize(wd.to(dev))
    pm = PersistentMLP(1, H, I, dev, one_launch=True)
    out = pm(x.to(dev), qgu, qd)
    assert torch.isnan(out).all() and torch.isnan(pm.act.float()).all()
    assert not pm.failed()


def test_fp8_lm_head_nan_row_argmax_first(dev):
    """A NaN hidden row makes every logit NaN; torch.argmax then returns the first index, 0."""
    V, K = 4096, 2560
    E = weight(V, K, 57)
    h = act(1, K, 59)
    h[0, 3] = NAN
    q = fp8.quantize(E.to(dev))
    idx, logits = lmhead.lm_head_argmax(h.to(dev), q, return_logits=True)
    assert torch.isnan(logits.float()).all()
    assert idx.item() == 0 == torch.argmax(logits.float(), -1).item()
