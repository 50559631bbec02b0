"""krq_lmhead_argmax_noalloc (candidates in the library's per-GPU scratch array) against
krq_lmhead_argmax (candidates in a caller workspace), both through the C ABI: the same kernels on
the same operands, so token ids and bf16 logits must match bit for bit. Each weight kind takes two
calls in a row, the second smaller, so the second runs over what the first left in the scratch."""

import ctypes

import pytest
import torch

from kernels import _lib as L
from kernels import fp8, lmhead
from kernels import gemv as G

pytestmark = pytest.mark.gpu

K = 2560
VOCAB = 151936  # Qwen3


def _operands(h, w, kind):
    """(h, h_scale, h_per_row, w, w_kind, layout, w_scale, w_per_row) as lm_head_argmax passes them."""
    if kind == "bf16":
        wt, layout = G._weight(w)
        return h.contiguous(), None, 0, wt, L.LM_BF16, layout, None, 0
    q = fp8.quantize(w) if kind == "fp8_channel" else fp8.quantize_weight(w)
    hin, hsc, hpr, wk = lmhead._fp8_operands(h, q, None, "tiled")
    wt, layout = (q.tiled, L.W_TILED) if q.tiled is not None else (q[0], L.W_ROWMAJOR)
    wpr = 1 if q[1].numel() == w.shape[0] else 0
    return hin, hsc, hpr, wt, wk, layout, q[1], wpr


def _call(noalloc, ops, M, V, with_logits=True):
    hin, hsc, hpr, wt, wk, layout, wsc, wpr = ops
    dev = hin.device
    idx = torch.full((M,), -1, device=dev, dtype=torch.int64)
    logits = torch.empty((M, V), device=dev, dtype=torch.bfloat16) if with_logits else None
    head = (L.ptr(hin), L.ptr(hsc), hpr, L.ptr(wt), wk, layout, L.ptr(wsc), wpr, M, V, K, L.ptr(logits))
    if noalloc:
        L.call("krq_lmhead_argmax_noalloc", *head, L.ptr(idx), L.stream(hin))
    else:
        ws = torch.empty((int(L.lib().krq_lmhead_ws_bytes(M, V)),), device=dev, dtype=torch.uint8)
        L.call("krq_lmhead_argmax", *head, L.ptr(ws), ws.numel(), L.ptr(idx), L.stream(hin))
    torch.cuda.synchronize()
    return idx, logits


def _case(dev, kind, M, V, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (torch.randn(V, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    h = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    return _operands(h, w, kind)


# (kind, (M, V) of the first call, (M, V) of the second, smaller call)
CASES = [
    ("fp8_channel", (16, VOCAB), (4, 32768)),     # tiled e4m3 rows, per-token scales
    ("fp8_channel", (1, VOCAB), (1, 4096)),       # bf16 row scaled inside the GEMV
    ("fp8_tensor", (32, VOCAB), (8, 65536)),      # one ActScale over h
    ("bf16", (8, VOCAB), (2, 1024)),
    ("fp8_channel", (32, 262144), (31, 262128)),  # the scratch maximum exactly, then just below
]


@pytest.mark.parametrize("kind,first,second", CASES)
def test_noalloc_matches_workspace_entry_point(dev, kind, first, second):
    for i, (M, V) in enumerate((first, second)):
        print(f"[noalloc] {kind} call {i + 1}: M={M} V={V} K={K}", flush=True)
        assert L.lib().krq_lmhead_ws_bytes(M, V) <= L.LMHEAD_SCRATCH_BYTES
        ops = _case(dev, kind, M, V, 17 + 7 * i + M)
        ref_idx, ref_logits = _call(False, ops, M, V)
        idx, logits = _call(True, ops, M, V)
        assert torch.equal(idx, ref_idx), (kind, M, V)
        assert torch.equal(logits.view(torch.int16), ref_logits.view(torch.int16)), (kind, M, V)
        assert int(idx.min()) >= 0 and int(idx.max()) < V
        # without the logits output: the same ids
        idx2, _ = _call(True, ops, M, V, with_logits=False)
        assert torch.equal(idx2, ref_idx), (kind, M, V)


def test_noalloc_refuses_sizes_beyond_its_scratch(dev):
    lib = L.lib()
    p = ctypes.c_void_p(4096)  # never dereferenced: the size check refuses the call first
    M, V = 32, 262144 + 16
    assert lib.krq_lmhead_ws_bytes(M, V) > L.LMHEAD_SCRATCH_BYTES
    rc = lib.krq_lmhead_argmax_noalloc(p, p, 1, p, L.LM_FP8, L.W_TILED, p, 1, M, V, K, None, p, None)
    assert rc == L.KRQ_EINVAL and b"scratch maximum" in lib.krq_last_error()
