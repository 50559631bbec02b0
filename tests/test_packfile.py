"""On-disk pre-packed FP8 format (kernels/packfile.py): bit-exact round trip of the canonical
row-major bytes, scales and tiled copies; digest and format checks (CPU, no GPU needed)."""

import numpy as np
import pytest
import torch

from kernels import packfile
from kernels.fp8 import FP8Weight
from oracle import oracle as O


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def cpu_weight(N, K, seed, per_row=True):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    r8, rs = O.quantize(bf16_bits(w)) if per_row else O.quantize_weight(bf16_bits(w))
    w8 = torch.from_numpy(r8.copy()).view(torch.float8_e4m3fn)
    sc = torch.from_numpy(np.asarray(rs, dtype=np.float32).copy()).reshape(-1 if per_row else ())
    return FP8Weight(w8, sc, torch.from_numpy(O.tile(r8)))


def test_round_trip_bit_exact(tmp_path):
    ws = {"qkv": cpu_weight(64, 256, 0), "o": cpu_weight(32, 128, 1, per_row=False)}
    p = str(tmp_path / "w.safetensors")
    packfile.save_fp8(p, ws, meta={"model": "synthetic", "layers": 1}, tiled=True)
    assert packfile.read_meta(p) == {"model": "synthetic", "layers": 1}
    got = packfile.load_fp8(p, tiled=True)
    assert set(got) == {"qkv", "o"}
    for k, q in ws.items():
        g = got[k]
        assert torch.equal(g[0].view(torch.uint8), q[0].view(torch.uint8))
        assert torch.equal(g[1], q[1]) and g[1].shape == q[1].shape
        assert torch.equal(g.tiled, q.tiled)
        assert np.array_equal(O.untile(g.tiled.numpy(), *q[0].shape), q[0].view(torch.uint8).numpy())
    untiled = packfile.load_fp8(p, tiled=False)
    assert untiled["qkv"].tiled is None


def test_digest_and_format_checks(tmp_path):
    p = str(tmp_path / "w.safetensors")
    packfile.save_fp8(p, {"down": cpu_weight(32, 256, 2)})
    raw = bytearray(open(p, "rb").read())
    raw[-100] ^= 0x01                       # one bit of the tensor data
    bad = str(tmp_path / "bad.safetensors")
    open(bad, "wb").write(bytes(raw))
    with pytest.raises(ValueError, match="SHA-256"):
        packfile.load_fp8(bad, tiled=False)
    packfile.load_fp8(bad, tiled=False, verify=False)   # still readable when asked not to check
    with pytest.raises(RuntimeError, match="ROCm device"):
        packfile.load_fp8(p)                # rebuilding the tiled copy needs the GPU
    from safetensors.torch import save_file
    other = str(tmp_path / "other.safetensors")
    save_file({"x.w8": torch.zeros(2, 2, dtype=torch.uint8)}, other, metadata={"format": "something"})
    with pytest.raises(ValueError, match="not a krq-fp8"):
        packfile.load_fp8(other)
    with pytest.raises(ValueError):
        packfile.save_fp8(p, {"a.b": cpu_weight(16, 64, 3)})
