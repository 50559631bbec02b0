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
#include "gemv_common.h"

using namespace krq;

namespace {

constexpr int kFoldThreads = 1024;

__global__ __launch_bounds__(kFoldThreads) void k_argmax_fold(const Best* __restrict__ cand, int64_t nrb,
                                                              int M, int64_t* __restrict__ idx_out) {
  __shared__ Best wb[kFoldThreads / 64];
  const int m = blockIdx.x;
  Best b{-INFINITY, 0x7fffffff};
  // four independent loads in flight per thread per round
  for (int64_t rb0 = threadIdx.x; rb0 < nrb; rb0 += 4 * kFoldThreads) {
    Best c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t rb = rb0 + (int64_t)q * kFoldThreads;
      c[q] = rb < nrb ? cand[rb * M + m] : Best{-INFINITY, 0x7fffffff};
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (better(c[q].v, c[q].i, b.v, b.i)) b = c[q];
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const Best c = shfl_best(b, o);
    if (better(c.v, c.i, b.v, b.i)) b = c;
  }
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFoldThreads / 64; ++w)
      if (better(wb[w].v, wb[w].i, b.v, b.i)) b = wb[w];
    idx_out[m] = b.i == 0x7fffffff ? 0 : b.i;
  }
}

}  // namespace

extern "C" int64_t krq_lmhead_ws_bytes(int64_t M, int64_t V) {
  return (V / 16) * M * (int64_t)sizeof(Best);
}

extern "C" int krq_lmhead_argmax(const void* h, const float* h_scale, const void* w, int w_kind,
                                 int w_layout, const float* w_scale, int64_t M, int64_t V, int64_t K,
                                 void* logits, void* ws, int64_t ws_bytes, int64_t* idx_out,
                                 void* stream) {
  KRQ_REQUIRE(h && w && ws && idx_out, "lmhead_argmax: null pointer");
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
  KRQ_REQUIRE(ws_bytes >= krq_lmhead_ws_bytes(M, V), "lmhead_argmax: workspace of %lld bytes < %lld",
              (long long)ws_bytes, (long long)krq_lmhead_ws_bytes(M, V));
  int rc;
  if (w_kind == KRQ_LM_BF16)
    rc = gemv_bf16_run(h, w, w_layout, M, V, K, 1, kOutArgmax, logits, ws, stream);
  else if (h_scale)
    rc = gemv_fp8_run(h, w_kind == KRQ_LM_FP8_TILED_H ? KRQ_X_FP8_TILED : KRQ_X_FP8, h_scale, nullptr, M > 1, w,
                      w_layout, w_scale, 1, M, V, K, 1, kOutArgmax, 0, logits, ws, stream);
  else
    rc = gemv_fp8_run(h, KRQ_X_BF16_DYN, nullptr, nullptr, 0, w, w_layout, w_scale, 1, M, V, K, 1,
                      kOutArgmax, 0, logits, ws, stream);
  if (rc != KRQ_OK) return rc;
  hipLaunchKernelGGL(k_argmax_fold, dim3(static_cast<unsigned>(M)), dim3(kFoldThreads), 0,
                     (hipStream_t)stream, reinterpret_cast<const Best*>(ws), V / 16, static_cast<int>(M),
                     idx_out);
  return krq_check_launch("lmhead_argmax");
}
