"""The full decode-step weight stream of BASELINE config 5, captured into one hipGraph: 36 layers x
(QKV split 2, O split 4, gate_up SwiGLU, down split 4) FP8 GEMVs with per-channel weights and
per-token activation scales, then the BF16 tied lm_head with argmax (the engine's step order,
engine/engine.py:1010-1022). Every replay must equal the eager step bit for bit, with eager work
and synchronizations between replays; the first layer's outputs also meet the parity bar against
the oracle."""

import numpy as np
import pytest
import torch

from kernels import fp8, lmhead
from kernels import gemv as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

H, I, NQKV, NQD, V = 2560, 9728, 6144, 4096, 151936
LAYERS = 36
PROJ = [("qkv", NQKV, H, 2), ("o", H, NQD, 4), ("gate_up", 2 * I, H, 1), ("down", H, I, 4)]


def u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


@pytest.fixture(scope="module")
def model(dev):
    g = torch.Generator(device=dev)
    layers = []
    for li in range(LAYERS):
        Lw = {}
        for p, (name, N, K, _) in enumerate(PROJ):
            g.manual_seed(1000 + 10 * li + p)
            Lw[name] = fp8.quantize((torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16))
        layers.append(Lw)
    g.manual_seed(7)
    E = G.pack((torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16))
    return layers, E


def _inputs(dev, M):
    xs = {}
    for p, (name, N, K, _) in enumerate(PROJ):
        xs[name] = torch.randn(M, K, generator=torch.Generator().manual_seed(2000 + p)).to(torch.bfloat16).to(dev)
    h = torch.randn(M, H, generator=torch.Generator().manual_seed(100 + M)).to(torch.bfloat16).to(dev)
    return xs, h


def _step(layers, E, xs, h):
    outs = []
    for Lw in layers:
        for name, N, K, split in PROJ:
            if name == "gate_up":
                outs.append(fp8.gemv_swiglu_fp8(xs[name], Lw[name]))
            else:
                outs.append(fp8.gemv_fp8(xs[name], Lw[name], split))
    outs.append(lmhead.lm_head_argmax(h, E))
    return outs


@pytest.mark.parametrize("M", [1, 16])
def test_full_step_graph_replays_equal_eager(dev, model, M):
    layers, E = model
    xs, h = _inputs(dev, M)
    eager = [t.clone() for t in _step(layers, E, xs, h)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _step(layers, E, xs, h)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = _step(layers, E, xs, h)
    assert len(captured) == 4 * LAYERS + 1
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(captured, eager)):
            assert torch.equal(a, b), f"replay {r}: output {i} differs from eager"
        _step(layers, E, xs, h)   # eager work between replays
        torch.cuda.synchronize()
    del g
    # layer 0 against the oracle (per-token scales, exact FP8 product, the consumer's split sum)
    for p, (name, N, K, split) in enumerate(PROJ):
        q = layers[0][name]
        x8r, xsr = O.quant_rows(u16(xs[name]))
        _, yref = O.fp8_matmul(x8r, xsr, u8(q[0]), q[1].cpu().numpy())
        got = eager[p]
        if name == "gate_up":
            yref = O.bf16_to_f32(O.swiglu(yref[:, :I].astype(np.float32), yref[:, I:].astype(np.float32)))
            y = got.float().cpu().numpy()
        else:
            acc = got[0].clone()
            for k in range(1, split):
                acc += got[k]
            y = acc.to(torch.bfloat16).float().cpu().numpy()
        e = float(np.abs(y - yref).max() / np.abs(yref).max())
        print(f"step M={M} layer 0 {name}: max-rel {e:.2e}")
        assert e <= 1e-2
