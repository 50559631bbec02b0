"""ctypes binding of libkrq.so, the gfx950 HIP extension (C ABI declared in include/krq.h).

The library is loaded after torch, so its libamdhip64.so.7 dependency binds to the HIP runtime
torch already loaded and the kernels share torch's device context and streams. Nothing here
falls back to another implementation: without the built library, or with tensors that are not on
a ROCm device, every entry point raises.
"""

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkrq.so")

KRQ_OK, KRQ_EINVAL, KRQ_EHIP = 0, -1, -2
OUT_BF16, OUT_PARTIAL, OUT_SWIGLU, OUT_RESIDUAL = 0, 1, 2, 4
W_ROWMAJOR, W_TILED = 0, 1
LM_BF16, LM_FP8, LM_FP8_TILED_H = 0, 1, 2
ALGO_AUTO, ALGO_MFMA, ALGO_VALU = 0, 1, 2
X_FP8, X_BF16_DYN, X_BF16_STATIC, X_FP8_TILED = 0, 1, 2, 3
LMHEAD_SCRATCH_BYTES = 4194304  # KRQ_LMHEAD_SCRATCH_BYTES

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# every symbol of include/krq.h: name -> (restype, argtypes)
EXPORTS = {
    "krq_quant_fp8_rows": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "krq_quant_fp8_tensor": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "krq_act_scale": (_i32, [_vp, _i64, _i64, _i32, _f32, _vp, _vp, _vp, _vp, _vp]),
    "krq_act_scale_ws_floats": (_i64, [_i64, _i64]),
    "krq_cast_fp8": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp, _vp]),
    "krq_act_scale_cast_fp8": (_i32, [_vp, _i64, _i64, _f32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "krq_quant_rows": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "krq_quant_rows_tiled": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "krq_cast_fp8_tiled": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "krq_gemv_fp8": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64,
                            _i32, _i32, _i32, _vp, _vp]),
    "krq_gemv_swiglu_fp8_cast": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64,
                                        _vp, _vp, _vp]),
    "krq_gemv_bf16": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp]),
    "krq_gemv_bf16_rows": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp, _vp]),
    "krq_lmhead_argmax": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _i64, _i64, _i64, _vp, _vp,
                                 _i64, _vp, _vp]),
    "krq_lmhead_ws_bytes": (_i64, [_i64, _i64]),
    "krq_lmhead_argmax_noalloc": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _i64, _i64, _i64, _vp,
                                         _vp, _vp]),
    "krq_mlp_fp8": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64,
                           _i32, _vp, _vp, _i32, _vp, _vp]),
    "krq_mlp_fp8_bounded": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _i32, _i64, _i64,
                                   _i64, _i32, _vp, _vp, _i32, ctypes.c_uint32, _vp, _vp]),
    "krq_mlp_ctl_words": (_i64, []),
    "krq_mlp_chain_fp8": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i32, _vp, _vp,
                                 ctypes.c_uint32, _vp, _vp]),
    "krq_mlp_chain_ctl_words": (_i64, []),
    "krq_mlp_chain_bf16": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, ctypes.c_uint32, _vp,
                                  _vp]),
    "krq_gemv_bf16_fused": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _f32, _vp,
                                   _vp, _vp, _vp, _vp, _vp]),
    "krq_gemv_fused_fits": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "krq_rmsnorm_rows": (_i32, [_vp, _vp, _vp, _f32, _i64, _i64, _vp, _vp]),
    "krq_gemv_fp8_fused": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _i32,
                                  _i32, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "krq_gemv_fp8_fused_fits": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32, _i32]),
    "krq_rmsnorm_quant_rows": (_i32, [_vp, _vp, _vp, _f32, _i64, _i64, _vp, _vp, _vp]),
    "krq_rmsnorm_quant_rows_tiled": (_i32, [_vp, _vp, _vp, _f32, _i64, _i64, _vp, _vp, _vp]),
    "krq_gemm_fp8": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _vp]),
    "krq_gemm_fp8_ws": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "krq_gemm_fp8_ws_bytes": (_i64, [_i32, _i64, _i64, _i64]),
    "krq_pack_fp8": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "krq_unpack_fp8": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "krq_version": (ctypes.c_char_p, []),
    "krq_last_error": (ctypes.c_char_p, []),
}

_lib = None


def lib():
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"krq: HIP extension {LIB_PATH} is not built "
                               "(run __graft_entry__.build()); there is no fallback path")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def call(name, *args):
    """Call a status-returning entry point; map KRQ_EINVAL to ValueError, others to RuntimeError."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != KRQ_OK:
        msg = (L.krq_last_error() or b"").decode(errors="replace")
        if rc == KRQ_EINVAL:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("krq kernels run on a ROCm device only; got a tensor on "
                               f"{t.device} (there is no CPU path)")
