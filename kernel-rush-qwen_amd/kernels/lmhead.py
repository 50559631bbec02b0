"""LM head GEMV fused with greedy argmax (a GEMV launch with an argmax epilogue plus a fold).

Reference semantics: logits = gemv(h, lm_head, 1) (bf16) then torch.argmax(logits, -1)
(engine/engine.py:1021-1022), i.e. the lowest index among the largest bf16-rounded logits; the
reference's fused form keeps the same rule (engine/kernels/mega.py:412-436). The FP8 variant
scales activations per token (inside the GEMV at M == 1, else fp8.quant_rows_tiled, the rows in
the tiled activation layout) and uses per-channel weights (fp8.quantize).
"""

import torch

from . import _lib as L
from . import fp8 as _fp8
from . import gemv as _gemv


def lm_head_argmax(h, w, return_logits=False, h_layout="tiled"):
    """h [M, K] bf16 (M <= 32); w the tied embedding, bf16 [V, K], or an FP8Weight from
    fp8.quantize (per-channel scales). Returns int64 [M] token ids, or (ids, bf16 logits [M, V])
    with return_logits=True. h_layout ("tiled" or "rowmajor"): how the FP8 head's quantized rows
    are laid out at M > 1 (the same operands either way; tiled loads are contiguous)."""
    L.require_device(h)
    M, K = h.shape
    if isinstance(w, tuple):
        w8, ws = w[0], w[1]
        tiled = getattr(w, "tiled", None)
        V = w8.shape[0]
        if ws.numel() != V:
            raise ValueError("the FP8 lm head needs per-channel scales (fp8.quantize)")
        if M == 1:   # per-token scale computed inside the GEMV
            hin, hsc, wk = _fp8._rows(h), None, L.LM_FP8
        elif K % 64 == 0 and h_layout == "tiled":  # e4m3 rows in the tiled activation layout
            h8, hs = _fp8.quant_rows_tiled(h)
            hin, hsc, wk = h8, hs.reshape(-1), L.LM_FP8_TILED_H
        else:
            h8, hs = _fp8.quant_rows(h)
            hin, hsc, wk = h8, hs.reshape(-1), L.LM_FP8
        wt, layout = (tiled, L.W_TILED) if tiled is not None else (w8, L.W_ROWMAJOR)
        wsc = ws
    else:
        if h.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise ValueError("the bf16 lm head expects bf16 h and w")
        V = w.shape[0]
        wt, layout = _gemv._weight(w)
        hin, hsc, wk, wsc = h.contiguous(), None, L.LM_BF16, None
    L.require_device(wt)
    if M > 32:
        raise ValueError(f"lm_head_argmax: M={M} > 32")
    idx = torch.empty((M,), device=h.device, dtype=torch.int64)
    logits = torch.empty((M, V), device=h.device, dtype=torch.bfloat16) if return_logits else None
    ws_buf = torch.empty((int(L.lib().krq_lmhead_ws_bytes(M, V)),), device=h.device, dtype=torch.uint8)
    L.call("krq_lmhead_argmax", L.ptr(hin), L.ptr(hsc), L.ptr(wt), wk, layout, L.ptr(wsc), M, V, K,
           L.ptr(logits), L.ptr(ws_buf), ws_buf.numel(), L.ptr(idx), L.stream(h))
    return (idx, logits) if return_logits else idx
