"""Persistent fused decode MLP: act = SwiGLU(h @ [gate; up]^T), then the fp32 split-K partials of
the down projection.

Drop-in for the reference's engine/kernels/mlp.py: PersistentMLP(M, H, I, device, programs,
split=4, bn=16, bn2=16, chunk=512) and __call__(h, w_gu, w_down) -> fp32 [split, M, H], summed
in split order by the consumer (engine/engine.py:911-915, :1015; ops.py:29-39). Weights are the
FP8Weight tuples of fp8.quantize (per-channel e4m3) and activations are scaled per token, as
linear_fp8 / quant_rows do: at M == 1 the kernel scales h itself, at larger M fp8.quant_rows runs
first; the SwiGLU activations are re-quantized per token inside the kernel once all of them exist.

Two forms give the same contract. By default both phases are separate GEMV launches
(fp8.gemv_swiglu_fp8 then fp8.gemv_fp8 for FP8 weights, kernels.gemv for BF16 weights): on MI355X
that pair measured faster than one persistent launch (17.2 against 31 us at M = 1, 26.7 against
55 us at M = 16 for FP8 weights), because the cross-XCD handoff between the phases costs more than
a launch boundary. one_launch=True runs both phases in one launch of the HIP kernel k_mlp_fp8
(libkrq.so, krq_mlp_fp8; FP8 weights only): `programs` is then the number of blocks, as in the
reference; the library clamps it to the blocks the device holds at once (so spin-waits cannot
deadlock), and `programs=None` takes one per CU. Its control words are zeroed here once and left
zeroed by every launch; a block whose phase-1 wait gives up writes NaN partials, and failed()
reports it.

chained=True (M == 1, tiled FP8 weights) runs the two-launch pair's kernels as one launch of
k_mlp_chain_fp8 (krq_mlp_chain_fp8): the down workgroups issue their weight loads, then wait for
every gate_up workgroup's act through arrival counters polled by scalar loads, and read act with
coherent loads. act is bit-identical to the pair's; the partials equal the pair's to fp32
rounding (the down blocks sum two weight waves). A wait that gives up makes that block's
partials NaN and failed() reports it; zero_ctl() then clears the control words.

For BF16 weights, one_launch=True or chained=True (any M) runs the chained launch of the BF16
GEMVs, k_mlp_chain_bf16 (krq_mlp_chain_bf16): each stage keeps its standalone launch's plan, so
act and the partials are the two-launch pair's, bit for bit; waits, failed() and zero_ctl() as
above.
"""

import torch

from . import _lib as L
from . import fp8 as _fp8
from . import gemv as _gemv


class PersistentMLP:
    """Workspace for one M. Call with (h [M, H] bf16, w_gu [2I, H], w_down [H, I]) as FP8Weight."""

    CHAIN_POLLS = 1 << 20  # bound on the chained form's wait: about a second of polls

    def __init__(self, M, H, I, device, programs=None, split=4, bn=16, bn2=16, chunk=512,
                 one_launch=False, chained=False):
        # the reference's shape contract (engine/kernels/mlp.py:100-103)
        assert I % chunk == 0 and chunk % bn == 0 and I % split == 0
        assert (I // split) % 64 == 0 and H % bn2 == 0
        if bn != 16 or bn2 != 16:
            raise ValueError("the HIP kernel's row blocks are 16 columns (bn = bn2 = 16)")
        if not 1 <= M <= 32:
            raise ValueError(f"PersistentMLP: M={M} outside 1..32")
        self.M, self.H, self.I, self.G = M, H, I, programs
        self.split, self.bn, self.bn2, self.chunk = split, bn, bn2, chunk
        self.one_launch = one_launch
        if chained and one_launch:
            raise ValueError("PersistentMLP: the chained form excludes one_launch")
        self.chained = chained
        words = L.lib().krq_mlp_ctl_words()
        self._mlp_err = int(words) - 1  # krq_mlp_fp8's error word: its last control word
        if chained or one_launch:  # (one_launch with BF16 weights runs the chained form)
            words = max(int(words), int(L.lib().krq_mlp_chain_ctl_words()))
        self.ctl = torch.zeros((int(words),), device=device, dtype=torch.int32)
        self.act = None   # bf16 [M, I] SwiGLU activations of the last call
        self._err = self._mlp_err  # the error word of the form that ran last

    def _bf16(self, h, w_gu, w_down, max_polls):
        H, I, S = self.H, self.I, self.split
        if tuple(w_gu.shape) != (2 * I, H) or tuple(w_down.shape) != (H, I):
            raise ValueError(f"PersistentMLP: weights {tuple(w_gu.shape)} / {tuple(w_down.shape)} do not "
                             f"match H={H}, I={I}")
        h2 = _fp8._rows(h)
        M = h2.shape[0]
        if M != self.M:
            raise ValueError(f"PersistentMLP built for M={self.M}, called with M={M}")
        if not (self.chained or self.one_launch):
            act = _gemv.gemv_swiglu(h2, w_gu)
            self.act = act
            return _gemv.gemv(act, w_down, S)
        L.require_device(h2, w_gu, w_down)
        gu, lay_gu = _gemv._weight(w_gu)
        dn, lay_dn = _gemv._weight(w_down)
        if lay_gu != lay_dn:
            raise ValueError("PersistentMLP: gate/up and down weights must share a layout (pack both or neither)")
        act = torch.empty((M, I), device=h.device, dtype=torch.bfloat16)
        out = torch.empty((S, M, H), device=h.device, dtype=torch.float32)
        self._err = self.CHAIN_ERR
        L.call("krq_mlp_chain_bf16", L.ptr(h2), L.ptr(gu), L.ptr(dn), lay_gu, M, H, I, S, L.ptr(act),
               L.ptr(self.ctl), int(self.CHAIN_POLLS if max_polls is None else max_polls), L.ptr(out), L.stream(h))
        self.act = act
        return out

    def __call__(self, h, w_gu, w_down, max_polls=None):
        """max_polls (one-launch form): bound on the phase-1 wait's polls (default: about a
        second's worth); a small value forces the timeout path, for tests."""
        if isinstance(w_gu, torch.Tensor) and isinstance(w_down, torch.Tensor):
            if w_gu.dtype != torch.bfloat16 or w_down.dtype != torch.bfloat16:
                raise ValueError("PersistentMLP: weights are FP8Weight tuples or bf16 tensors")
            return self._bf16(h, w_gu, w_down, max_polls)
        if not (isinstance(w_gu, tuple) and isinstance(w_down, tuple)):
            raise ValueError("PersistentMLP: weights are FP8Weight tuples or bf16 tensors")
        H, I, S = self.H, self.I, self.split
        gu, lay_gu, gs, gshape = _fp8._weight_operand(w_gu)
        dn, lay_dn, ds, dshape = _fp8._weight_operand(w_down)
        if tuple(gshape) != (2 * I, H) or tuple(dshape) != (H, I):
            raise ValueError(f"PersistentMLP: weights {tuple(gshape)} / {tuple(dshape)} do not match "
                             f"H={H}, I={I}")
        if lay_gu != lay_dn:
            raise ValueError("PersistentMLP: gate/up and down weights must share a layout")
        g_pr = 1 if gs.numel() == 2 * I else 0
        d_pr = 1 if ds.numel() == H else 0
        if gs.numel() not in (1, 2 * I) or ds.numel() not in (1, H):
            raise ValueError("PersistentMLP: weight scales must be per tensor or per row")
        h2 = _fp8._rows(h)
        M = h2.shape[0]
        if M != self.M:
            raise ValueError(f"PersistentMLP built for M={self.M}, called with M={M}")
        if self.chained:
            if M != 1:
                raise ValueError("PersistentMLP: the chained form of FP8 weights takes M == 1")
            if lay_gu != L.W_TILED:
                raise ValueError("PersistentMLP: the chained form takes tiled weights")
            self._err = self.CHAIN_ERR
            act = torch.empty((1, I), device=h.device, dtype=torch.bfloat16)
            out = torch.empty((S, 1, H), device=h.device, dtype=torch.float32)
            L.call("krq_mlp_chain_fp8", L.ptr(h2), L.ptr(gu), L.ptr(gs), g_pr, L.ptr(dn), L.ptr(ds), d_pr,
                   H, I, S, L.ptr(act), L.ptr(self.ctl), int(self.CHAIN_POLLS if max_polls is None else max_polls),
                   L.ptr(out), L.stream(h))
            self.act = act
            return out
        if not self.one_launch:
            act = _fp8.gemv_swiglu_fp8(h2, w_gu)
            self.act = act
            return _fp8.gemv_fp8(act, w_down, S)
        self._err = self._mlp_err
        if M == 1:
            xin, kind, xs = h2, L.X_BF16_DYN, None
        else:
            xin, xs = _fp8.quant_rows(h2)
            kind, xs = L.X_FP8, xs.reshape(-1)
        act = torch.empty((M, I), device=h.device, dtype=torch.bfloat16)
        out = torch.empty((S, M, H), device=h.device, dtype=torch.float32)
        if max_polls is None:
            L.call("krq_mlp_fp8", L.ptr(xin), kind, L.ptr(xs), L.ptr(gu), lay_gu, L.ptr(gs), g_pr,
                   L.ptr(dn), L.ptr(ds), d_pr, M, H, I, S, L.ptr(act), L.ptr(self.ctl),
                   int(self.G or 0), L.ptr(out), L.stream(h))
        else:
            L.call("krq_mlp_fp8_bounded", L.ptr(xin), kind, L.ptr(xs), L.ptr(gu), lay_gu, L.ptr(gs), g_pr,
                   L.ptr(dn), L.ptr(ds), d_pr, M, H, I, S, L.ptr(act), L.ptr(self.ctl),
                   int(self.G or 0), int(max_polls), L.ptr(out), L.stream(h))
        self.act = act
        return out

    def failed(self):
        """True if a one-launch or chained call flagged a wait that timed out (its partials are
        NaN); synchronizes the device."""
        return bool(self.ctl[self._err].item())

    CHAIN_ERR = 513  # the chained form's error word (after 8 groups of 64 words and the exit count)

    def zero_ctl(self):
        """Clear the control words (needed after a wait gave up; every good launch leaves them
        zero)."""
        self.ctl.zero_()


def mlp_fp8_static(h, gu8, down8, a_gu, a_down, split=1):
    """The engine's static-scale FP8 decode MLP (engine/engine.py:977-981 with both sites in FP8):
    linear_fp8(silu_mul(linear_fp8(h, gu8, a_gu)), down8, a_down), in two launches: the SwiGLU
    GEMV with the down input's cast in its epilogue (fp8.swiglu_cast_fp8), then the down GEMV on
    those tiled e4m3 rows. h bf16 [M, H] (M <= 32); gu8 / down8 from quantize_weight or quantize
    (gu8 = [gate; up]); a_gu / a_down the sites' SharedScale (or ActScale). split == 1: bf16
    [M, H]; split > 1: fp32 partials [split, M, H]. The SwiGLU sums come from the two-matrix
    kernel rather than linear_fp8's [M, 2I] GEMV plus silu_mul, so the result equals the engine's
    within the GEMM tolerance; the cast of act is bit-identical."""
    x8t, sc = _fp8.swiglu_cast_fp8(h, gu8, a_down, a=a_gu)
    return _fp8.gemv_fp8_tiled_launch(x8t, sc, down8, h.shape[0], split,
                                      L.OUT_BF16 if split == 1 else L.OUT_PARTIAL)
