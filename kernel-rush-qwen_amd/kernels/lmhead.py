"""LM head GEMV fused with greedy argmax (a GEMV launch with an argmax epilogue plus a fold).

Reference semantics: logits = gemv(h, lm_head, 1) (bf16) then torch.argmax(logits, -1)
(engine/engine.py:1021-1022), i.e. the lowest index among the largest bf16-rounded logits; the
reference's fused form keeps the same rule (engine/kernels/mega.py:412-436).

FP8 heads take the activation scaling of the weight's form:
  per-channel weights (fp8.quantize, BASELINE's per-channel lm_head): h scaled per token, inside
      the GEMV at M == 1, else by fp8.quant_rows (row-major rows) or, from fp8.TILED_MIN_ROWS,
      fp8.quant_rows_tiled (rows in the tiled activation layout);
  per-tensor weights (fp8.quantize_weight, the engine's lm8 = quantize_weight(lm_head),
      engine.py:504-505): exactly linear_fp8(h, lm8) followed by torch.argmax (engine.py:989,
      :1022) - one ActScale over all of h (at M == 1 the same as per token, so inside the GEMV),
      or the given ActScale / SharedScale `a`.
"""

import torch

from . import _lib as L
from . import fp8 as _fp8
from . import gemv as _gemv


def _fp8_operands(h, w, a, h_layout):
    """(h operand, h scale, h_per_row, weight kind) for an FP8 head."""
    M, K = h.shape
    V = w[0].shape[0]
    ws = w[1]
    if ws.numel() not in (1, V):
        raise ValueError("the FP8 lm head needs per-channel or per-tensor weight scales")
    if a is not None:            # a given scale: linear_fp8(h, q, a)
        h8 = _fp8._cast(_fp8._rows(h), a)
        return h8, a.scale.reshape(1), 0, L.LM_FP8
    if M == 1:                   # per token == per tensor: scaled inside the GEMV
        return _fp8._rows(h), None, 0, L.LM_FP8
    if ws.numel() == 1:          # linear_fp8's own ActScale over the whole of h
        a = _fp8.ActScale(h)
        return _fp8._cast(_fp8._rows(h), a), a.scale.reshape(1), 0, L.LM_FP8
    tiled = h_layout == "tiled" or (h_layout == "auto" and M >= _fp8.TILED_MIN_ROWS)
    if K % 64 == 0 and K <= _fp8.TILED_ROWS_MAX_K and tiled:   # tiled e4m3 rows
        h8, hs = _fp8.quant_rows_tiled(h)
        return h8, hs.reshape(-1), 1, L.LM_FP8_TILED_H
    h8, hs = _fp8.quant_rows(h)
    return h8, hs.reshape(-1), 1, L.LM_FP8


def lm_head_argmax(h, w, return_logits=False, h_layout="auto", a=None):
    """h [M, K] bf16 (M <= 32); w the tied embedding, bf16 [V, K], or an FP8Weight from
    fp8.quantize (per channel) or fp8.quantize_weight (per tensor). Returns int64 [M] token ids,
    or (ids, bf16 logits [M, V]) with return_logits=True. h_layout ("auto", "tiled" or
    "rowmajor"): how a per-channel FP8 head's per-token rows are laid out at M > 1 (the same
    operands either way); "auto" takes tiled rows from fp8.TILED_MIN_ROWS (measured on MI355X at
    V = 151,936, us tiled / row-major: M = 2 68.4 / 63.8, M = 8 72.9 / 71.5, M = 12 75.5 / 75.4,
    M = 16 77.5 / 80.7). a: an ActScale / SharedScale for the FP8 head's activations (as
    linear_fp8 takes), instead of the scaling described in the module docstring."""
    L.require_device(h)
    M, K = h.shape
    if M > 32:
        raise ValueError(f"lm_head_argmax: M={M} > 32")
    if isinstance(w, tuple):
        w8, ws = w[0], w[1]
        tiled = getattr(w, "tiled", None)
        V = w8.shape[0]
        hin, hsc, hpr, wk = _fp8_operands(h, w, a, h_layout)
        wt, layout = (tiled, L.W_TILED) if tiled is not None else (w8, L.W_ROWMAJOR)
        wsc, wpr = ws, 1 if ws.numel() == V and V > 1 else 0
    else:
        if h.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise ValueError("the bf16 lm head expects bf16 h and w")
        V = w.shape[0]
        wt, layout = _gemv._weight(w)
        hin, hsc, hpr, wk, wsc, wpr = h.contiguous(), None, 0, L.LM_BF16, None, 0
    L.require_device(wt)
    idx = torch.empty((M,), device=h.device, dtype=torch.int64)
    logits = torch.empty((M, V), device=h.device, dtype=torch.bfloat16) if return_logits else None
    ws_buf = torch.empty((int(L.lib().krq_lmhead_ws_bytes(M, V)),), device=h.device, dtype=torch.uint8)
    L.call("krq_lmhead_argmax", L.ptr(hin), L.ptr(hsc), hpr, L.ptr(wt), wk, layout, L.ptr(wsc), wpr, M, V, K,
           L.ptr(logits), L.ptr(ws_buf), ws_buf.numel(), L.ptr(idx), L.stream(h))
    return (idx, logits) if return_logits else idx
