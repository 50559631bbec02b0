// LM head GEMV fused with greedy argmax (M <= 32), two launches:
//   1. the skinny GEMV (gemv_fp8.hip / gemv_bf16.hip) with the argmax epilogue: logits are rounded
//      to bf16 (optionally stored) and every 16-column row block writes, per token row, its
//      largest logit and the lowest index holding it;
//   2. k_argmax_fold: one block per token row folds the row blocks' candidates in the same
//      order-free way (largest value, then lowest index) into idx_out.
// The launch boundary makes the candidates visible to the fold: no atomics, counters or fences,
// so graph replays need no reset and the result does not depend on block scheduling.
// Reference semantics: logits = bf16(h . E^T), torch.argmax (first maximum) - engine/engine.py:
// 1021-1022; fused form engine/kernels/mega.py:396-441.
#include <atomic>
#include <mutex>

#include "gemv_common.h"

using namespace krq;

namespace {

constexpr int kFoldThreads = 1024;
constexpr int kFoldPer = 10;  // candidates per thread per batch (V = 151,936: one batch)

// The candidate (v, i) as one unsigned 64-bit key whose order is better()'s: the high word maps v
// to an order-preserving integer (NaN above everything, -0 as +0), the low word is ~i (the lower
// index wins a tie).
KRQ_DEV uint64_t fold_key(Best b) {
  uint32_t hi;
  if (b.v != b.v) {
    hi = 0xffffffffu;
  } else {
    const uint32_t u = b.v == 0.0f ? 0u : __float_as_uint(b.v);
    hi = (u >> 31) ? ~u : (u | 0x80000000u);
  }
  return (static_cast<uint64_t>(hi) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(b.i));
}

template <int CTRL>
KRQ_DEV uint64_t dpp_max_u64(uint64_t k) {
  const uint32_t hi = static_cast<uint32_t>(k >> 32), lo = static_cast<uint32_t>(k);
  const uint32_t oh = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(hi), CTRL, 0xf, 0xf, false));
  const uint32_t ol = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(lo), CTRL, 0xf, 0xf, false));
  const uint64_t o = (static_cast<uint64_t>(oh) << 32) | ol;
  return o > k ? o : k;
}

// max of the key over each row of 16 lanes (every lane of the row ends with it)
KRQ_DEV uint64_t row16_max_u64(uint64_t k) {
  k = dpp_max_u64<0xB1>(k);   // quad_perm(1,0,3,2): lane ^ 1
  k = dpp_max_u64<0x4E>(k);   // quad_perm(2,3,0,1): lane ^ 2
  k = dpp_max_u64<0x141>(k);  // row_half_mirror: the other quad of each 8
  return dpp_max_u64<0x140>(k);  // row_mirror: the other half of each 16
}

KRQ_DEV uint64_t readlane_u64(uint64_t k, int l) {
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(k >> 32), l);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(k), l);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One block per token row (its [nrb] candidates are contiguous, so each wave's load is 512 bytes of
// whole lines): every candidate load of a batch is issued before the first is used (one memory
// round trip), the keys are reduced with DPP steps inside each wave and across the
// block's 16 waves by wave 0.
__global__ __launch_bounds__(kFoldThreads) void k_argmax_fold(const Best* __restrict__ cand, int64_t nrb,
                                                              int M, int64_t* __restrict__ idx_out) {
  __shared__ uint64_t wk[kFoldThreads / 64];
  const int m = blockIdx.x, lane = threadIdx.x & 63;
  const Best* __restrict__ row = cand + (int64_t)m * nrb;  // token row m's candidates, contiguous
  uint64_t best = 0;  // below every candidate's key
  for (int64_t base = 0; base < nrb; base += (int64_t)kFoldPer * kFoldThreads) {
    Best c[kFoldPer];
#pragma unroll
    for (int q = 0; q < kFoldPer; ++q) {
      const int64_t rb = min(base + threadIdx.x + (int64_t)q * kFoldThreads, nrb - 1);  // clamped, valid
      c[q] = row[rb];
    }
#pragma unroll
    for (int q = 0; q < kFoldPer; ++q) {
      const uint64_t k = fold_key(c[q]);
      if (base + threadIdx.x + (int64_t)q * kFoldThreads < nrb && k > best) best = k;
    }
  }
  best = row16_max_u64(best);
  uint64_t w = readlane_u64(best, 0);
#pragma unroll
  for (int l = 16; l < 64; l += 16) {
    const uint64_t o = readlane_u64(best, l);
    w = o > w ? o : w;
  }
  if (lane == 0) wk[threadIdx.x >> 6] = w;
  __syncthreads();
  if (threadIdx.x < 64) {
    uint64_t k = wk[lane & (kFoldThreads / 64 - 1)];  // 16 waves: lanes 0..15 of each row
    k = row16_max_u64(k);
    if (threadIdx.x == 0) {
      const uint32_t i = ~static_cast<uint32_t>(k);
      idx_out[m] = i >= 0x7fffffffu ? 0 : static_cast<int64_t>(i);
    }
  }
}

}  // namespace

extern "C" int64_t krq_lmhead_ws_bytes(int64_t M, int64_t V) {
  return (V / 16) * M * (int64_t)sizeof(Best);
}

namespace {

// Argument checks of both entry points (all but the workspace).
int lmhead_check(const void* h, const float* h_scale, const void* w, int w_kind, int w_layout,
                 const float* w_scale, int64_t M, int64_t V, const int64_t* idx_out) {
  KRQ_REQUIRE(h && w && idx_out, "lmhead_argmax: null pointer");
  KRQ_REQUIRE(M >= 1 && M <= 32, "lmhead_argmax: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(w_kind == KRQ_LM_BF16 || w_kind == KRQ_LM_FP8 || w_kind == KRQ_LM_FP8_TILED_H,
              "lmhead_argmax: bad weight kind %d", w_kind);
  KRQ_REQUIRE(w_kind != KRQ_LM_FP8_TILED_H || h_scale, "lmhead_argmax: tiled e4m3 h needs h_scale");
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "lmhead_argmax: bad layout %d", w_layout);
  KRQ_REQUIRE(w_kind == KRQ_LM_BF16 || w_scale, "lmhead_argmax: FP8 weights need w_scale");
  KRQ_REQUIRE(w_kind == KRQ_LM_BF16 || h_scale || M == 1,
              "lmhead_argmax: bf16 activations with FP8 weights are scaled in the kernel for M == 1 only");
  KRQ_REQUIRE(V > 0 && V % 16 == 0 && V <= 0x7fffffff, "lmhead_argmax: V=%lld must be a positive multiple of 16",
              (long long)V);
  return KRQ_OK;
}

// The two launches into the candidate buffer ws (krq_lmhead_ws_bytes(M, V) bytes, all of which the
// GEMV writes before the fold reads them: nothing needs clearing between calls).
int lmhead_launch(const void* h, const float* h_scale, int h_per_row, const void* w, int w_kind, int w_layout,
                  const float* w_scale, int w_per_row, int64_t M, int64_t V, int64_t K, void* logits, void* ws,
                  int64_t* idx_out, void* stream) {
  int rc;
  if (w_kind == KRQ_LM_BF16)
    rc = gemv_bf16_run(h, w, w_layout, M, V, K, 1, kOutArgmax, logits, ws, stream);
  else if (h_scale)
    rc = gemv_fp8_run(h, w_kind == KRQ_LM_FP8_TILED_H ? KRQ_X_FP8_TILED : KRQ_X_FP8, h_scale, nullptr,
                      h_per_row != 0 && M > 1, w, w_layout, w_scale, w_per_row != 0, M, V, K, 1, kOutArgmax, 0,
                      logits, ws, stream);
  else
    rc = gemv_fp8_run(h, KRQ_X_BF16_DYN, nullptr, nullptr, 0, w, w_layout, w_scale, w_per_row != 0, M, V, K, 1,
                      kOutArgmax, 0, logits, ws, stream);
  if (rc != KRQ_OK) return rc;
  hipLaunchKernelGGL(k_argmax_fold, dim3(static_cast<unsigned>(M)), dim3(kFoldThreads), 0,
                     (hipStream_t)stream, reinterpret_cast<const Best*>(ws), V / 16, static_cast<int>(M),
                     idx_out);
  return krq_check_launch("lmhead_argmax");
}

}  // namespace

extern "C" int krq_lmhead_argmax(const void* h, const float* h_scale, int h_per_row, const void* w,
                                 int w_kind, int w_layout, const float* w_scale, int w_per_row, int64_t M,
                                 int64_t V, int64_t K, void* logits, void* ws, int64_t ws_bytes,
                                 int64_t* idx_out, void* stream) {
  const int rc = lmhead_check(h, h_scale, w, w_kind, w_layout, w_scale, M, V, idx_out);
  if (rc != KRQ_OK) return rc;
  KRQ_REQUIRE(ws, "lmhead_argmax: null pointer");
  KRQ_REQUIRE(ws_bytes >= krq_lmhead_ws_bytes(M, V), "lmhead_argmax: workspace of %lld bytes < %lld",
              (long long)ws_bytes, (long long)krq_lmhead_ws_bytes(M, V));
  return lmhead_launch(h, h_scale, h_per_row, w, w_kind, w_layout, w_scale, w_per_row, M, V, K, logits, ws,
                       idx_out, stream);
}

// ---------------------------------------------------------------------------------------------
// Allocation-free variant: the candidates live in `scratch`, which the code object carries, so the
// call allocates nothing. Each GPU holds its own copy (at its own address) from the library's first
// use on it until the process ends. In host code `scratch` names a host-side stand-in: kernels get
// the address hipGetSymbolAddress returns for the current device, never the array's name.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[KRQ_LMHEAD_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];  // device address of `scratch` per device; null until resolved
std::mutex g_scratch_mu;

// The address of this device's `scratch`, resolved on the first call on the device (with it
// current) and kept.
int scratch_address(int dev, void** out) {
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        krq_set_error("lmhead_argmax_noalloc: hipGetSymbolAddress on device %d: %s", dev,
                      e != hipSuccess ? hipGetErrorString(e) : "null address");
        return KRQ_EHIP;
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return KRQ_OK;
}

}  // namespace

extern "C" int krq_lmhead_argmax_noalloc(const void* h, const float* h_scale, int h_per_row, const void* w,
                                         int w_kind, int w_layout, const float* w_scale, int w_per_row,
                                         int64_t M, int64_t V, int64_t K, void* logits, int64_t* idx_out,
                                         void* stream) {
  int rc = lmhead_check(h, h_scale, w, w_kind, w_layout, w_scale, M, V, idx_out);
  if (rc != KRQ_OK) return rc;
  KRQ_REQUIRE(krq_lmhead_ws_bytes(M, V) <= KRQ_LMHEAD_SCRATCH_BYTES,
              "lmhead_argmax_noalloc: M=%lld, V=%lld need %lld bytes of candidates, above the scratch "
              "maximum of %d (use krq_lmhead_argmax with a workspace)",
              (long long)M, (long long)V, (long long)krq_lmhead_ws_bytes(M, V), KRQ_LMHEAD_SCRATCH_BYTES);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    krq_set_error("lmhead_argmax_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return KRQ_EHIP;
  }
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) {
      krq_set_error("lmhead_argmax_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
      return KRQ_EHIP;
    }
    KRQ_REQUIRE(sdev == dev, "lmhead_argmax_noalloc: stream on device %d while device %d is current", (int)sdev,
                dev);
  }
  KRQ_REQUIRE(dev >= 0 && dev < kMaxDevices, "lmhead_argmax_noalloc: device %d beyond %d", dev, kMaxDevices);
  void* ws = nullptr;
  rc = scratch_address(dev, &ws);
  if (rc != KRQ_OK) return rc;
  return lmhead_launch(h, h_scale, h_per_row, w, w_kind, w_layout, w_scale, w_per_row, M, V, K, logits, ws,
                       idx_out, stream);
}
