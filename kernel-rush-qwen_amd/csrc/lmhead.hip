// LM head GEMV fused with greedy argmax (M <= 32), two launches:
//   1. the skinny GEMV (gemv_fp8.hip / gemv_bf16.hip) with the argmax epilogue: logits are rounded
//      to bf16 (optionally stored) and every 16-column row block writes, per token row, its
//      largest logit and the lowest index holding it; or, for FP8 weights on tiled e4m3 rows of
//      h (M <= 16), the persistent k_lmhead_fp8_persist, whose waves each write one candidate per
//      token row for all of their row blocks;
//   2. k_argmax_fold: one block per token row folds the candidates in the same order-free way
//      (largest value, then lowest index) into idx_out.
// The launch boundary makes the candidates visible to the fold: no atomics, counters or fences,
// so graph replays need no reset and the result does not depend on block scheduling.
// Reference semantics: logits = bf16(h . E^T), torch.argmax (first maximum) - engine/engine.py:
// 1021-1022; fused form engine/kernels/mega.py:396-441.
#include <algorithm>
#include <atomic>
#include <type_traits>
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

// The candidate of a 64-bit key (fold_key's inverse; a NaN comes back as the default NaN). Key 0,
// below every candidate's, comes back as (-inf, 0x7fffffff), which every real candidate beats.
KRQ_DEV Best key_best(uint64_t k) {
  if (k == 0) return Best{-INFINITY, 0x7fffffff};
  const uint32_t hi = static_cast<uint32_t>(k >> 32);
  const float v = hi == 0xffffffffu ? __builtin_nanf("") : __uint_as_float((hi >> 31) ? (hi & 0x7fffffffu) : ~hi);
  return Best{v, static_cast<int>(~static_cast<uint32_t>(k))};
}

// ---------------------------------------------------------------------------------------------
// Persistent FP8 lm head over the tiled e4m3 rows of h (KRQ_LM_FP8_TILED_H, M <= 16, one 16-row
// tile): a grid of a few hundred workgroups, each of which copies the whole tile row of h (K / 64
// tiles of 1 KB) into LDS once and then streams only weights. The one-launch-per-row-block kernel
// (k_gemv_fp8, paired row blocks) instead loads each block's activation tiles from L2 beside its
// weights: 4,748 blocks x 40 KB, half as many bytes again as the 389 MB of FP8 weights.
// Wave w of workgroup b takes row blocks gw, gw + GW, ... (gw = b * kPersistWaves + w, GW = the
// grid's waves) and streams their steps (two 64-byte tiles each) through a ring of U slots that
// runs on from one row block into the next. The products of even and odd steps go to two
// accumulators, summed as (0 + even) + odd: the sums of the paired kernel, whose two waves take
// the even and the odd steps, so the logits are the same bit for bit. After a row block's last
// step the wave rounds its 16 x M logits to bf16 (optionally stores them) and keeps, per token,
// the best (value, index) key so far; at the end it writes one candidate per token, [M][GW], which
// k_argmax_fold reduces as it reduces the row blocks' candidates.
// ---------------------------------------------------------------------------------------------
constexpr int kPersistWaves = 4;
constexpr int kPersistBlocks = 512;  // two per compute unit (LDS: 16 K bytes each)
constexpr int kPersistMaxK = 16 * kPersistWaves * 64;  // h's tile row in 16 chunks per thread, 64 KB
constexpr int kPersistMaxRows = 16;  // row blocks per wave (V = 151,936 on 2,048 waves: 5)

template <int U, int STG>
__global__ __launch_bounds__(kPersistWaves * 64) void k_lmhead_fp8_persist(
    const uint8_t* __restrict__ x8t, const float* __restrict__ xsc, int x_per_row, const uint8_t* __restrict__ w8,
    const float* __restrict__ wsc, int w_per_row, int M, int64_t V, int K, uint16_t* __restrict__ logits,
    Best* __restrict__ cand) {
  static_assert(U % 2 == 0, "even slots: slot u holds steps of u's parity");
  // the tile row of h, as laid out in memory, then [kPersistWaves][kPersistMaxRows][16] column scales
  extern __shared__ __align__(16) uint8_t xl[];
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int kt = K >> 6, nsteps = kt >> 1;  // (the host checks nsteps % U == 0)
  const int64_t nrb = V >> 4;
  const int64_t gw = (int64_t)blockIdx.x * kPersistWaves + wave, GW = (int64_t)gridDim.x * kPersistWaves;
  const int mine = gw < nrb ? static_cast<int>((nrb - 1 - gw) / GW) + 1 : 0;  // row blocks of this wave
  const int iters = mine * (nsteps / U);

  // h's tile row (kt * 64 chunks of 16 bytes, STG per thread; from L2 after the first workgroups):
  // loaded first, stored into LDS once the first steps of the ring are in flight
  const int chunks = kt * 64;
  uint4 hv[STG];
#pragma unroll
  for (int q = 0; q < STG; ++q)
    hv[q] = ld16(x8t + 16 * (int64_t)min(static_cast<int>(threadIdx.x) + q * kPersistWaves * 64, chunks - 1));
  __builtin_amdgcn_sched_barrier(0);  // (issued before the ring)
  float xs_r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xs_r[i] = xsc[min(4 * g + i, M - 1) * x_per_row];  // (x_per_row: 0 or 1)
  // the column scales of the wave's row blocks (lane c: column c; w_per_row 0 or 1), for the table
  // in LDS that the row blocks' ends read (a load inside the loop, behind the branch of a row
  // block's end, makes the compiler drain the whole ring there)
  float wcols[kPersistMaxRows];
#pragma unroll
  for (int j = 0; j < kPersistMaxRows; ++j)
    wcols[j] = wsc[(min(gw + (int64_t)min(j, max(mine - 1, 0)) * GW, nrb - 1) * 16 + c) * w_per_row];

  // the ring: iteration `it` holds steps s0 .. s0 + U - 1 of this wave's row block j
  uint4 wl[U], wh[U];
  int ld_j = 0, ld_s = 0;  // the next iteration to load
  auto load_iter = [&](int u) {
    const int64_t rb = mine > 0 ? gw + (int64_t)min(ld_j, mine - 1) * GW : 0;
    const uint8_t* p = w8 + ((rb * kt + 2 * (ld_s + u)) * 64 + lane) * 16;
    wl[u] = ld16nt(p);
    wh[u] = ld16nt(p + 1024);
  };
  auto advance = [&]() {
    ld_s += U;
    if (ld_s == nsteps) {
      ld_s = 0;
      ++ld_j;
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  // the ring's first steps, issued last and in slot order, as every later iteration issues them (so
  // the wait before each matrix instruction counts the same loads on the first pass as on the rest)
#pragma unroll
  for (int u = 0; u < U; ++u) {
    load_iter(u);
    __builtin_amdgcn_sched_barrier(0);
  }
  advance();
#pragma unroll
  for (int q = 0; q < STG; ++q) {
    const int i = static_cast<int>(threadIdx.x) + q * kPersistWaves * 64;
    if (i < chunks) *reinterpret_cast<uint4*>(xl + 16 * i) = hv[q];
  }
  float* wtab = reinterpret_cast<float*>(xl + 16 * (size_t)K) + wave * kPersistMaxRows * 16;
  if (lane < 16) {
#pragma unroll
    for (int j = 0; j < kPersistMaxRows; ++j) wtab[j * 16 + c] = wcols[j];
  }
  __syncthreads();
  if (mine == 0) {  // (not reached: the host keeps the grid's waves within the row blocks)
    if (c == 0)
      for (int i = 0; i < 4; ++i)
        if (4 * g + i < M) cand[(int64_t)(4 * g + i) * GW + gw] = key_best(0);
    return;
  }

  v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  uint64_t best[4] = {0, 0, 0, 0};
  int cj = 0, cs = 0;  // the iteration being consumed
  // one iteration: consume the U slots (refilling each with the next iteration's step unless this
  // is the last), then, after a row block's last step, its logits and the running best per token
  auto iteration = [&](auto refill) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = cs + u;
      const uint4 xa = *reinterpret_cast<const uint4*>(xl + ((2 * st) * 64 + lane) * 16);
      const uint4 xb = *reinterpret_cast<const uint4*>(xl + ((2 * st + 1) * 64 + lane) * 16);
      const v8i A = pack_v8i(xa, xb), B = pack_v8i(wl[u], wh[u]);
      if (u & 1)
        acc1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc1, 0, 0, 0, 0, 0, 0);
      else
        acc0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc0, 0, 0, 0, 0, 0, 0);
      if constexpr (decltype(refill)::value) load_iter(u);
    }
    if constexpr (decltype(refill)::value) advance();
    cs += U;
    if (cs == nsteps) {
      const int64_t rb = gw + (int64_t)cj * GW;
      const int64_t n = rb * 16 + c;
      const float wcol = wtab[cj * 16 + c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        float a = 0.0f;
        a += acc0[i];
        a += acc1[i];
        const uint16_t yb = f32_to_bf16(a * (m < M ? xs_r[i] : 0.0f) * wcol);
        if (m < M) {
          if (logits) logits[(int64_t)m * V + n] = yb;
          const uint64_t k = fold_key(Best{bf16_to_f32(yb), static_cast<int>(n)});
          best[i] = k > best[i] ? k : best[i];
        }
      }
      acc0 = v4f{0.f, 0.f, 0.f, 0.f};
      acc1 = v4f{0.f, 0.f, 0.f, 0.f};
      cs = 0;
      ++cj;
    }
  };
  for (int it = 0; it + 1 < iters; ++it) iteration(std::true_type{});
  iteration(std::false_type{});  // (iters >= 1: this wave has a row block)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint64_t k = row16_max_u64(best[i]);
    if (c == 0 && 4 * g + i < M) cand[(int64_t)(4 * g + i) * GW + gw] = key_best(k);
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
  // tiled e4m3 h and tiled weights, one row tile, h's tile row within LDS, steps a multiple of the
  // ring: the persistent kernel (k_lmhead_fp8_persist), its candidates [M][its waves]
  const int64_t nrb = V / 16, nsteps = K / 128;
  const int ring = nsteps % 10 == 0 ? 10 : nsteps % 8 == 0 ? 8 : 0;
  // at most one wave per row block: ncand <= nrb candidates per token fit krq_lmhead_ws_bytes
  const int64_t blocks = std::min<int64_t>(kPersistBlocks, nrb / kPersistWaves);
  const int64_t ncand = blocks * kPersistWaves;
  if (w_kind == KRQ_LM_FP8_TILED_H && w_layout == KRQ_W_TILED && M <= 16 && blocks > 0 && K % 128 == 0 &&
      K <= kPersistMaxK && ring > 0 && (nrb + ncand - 1) / ncand <= kPersistMaxRows && aligned16(h) &&
      aligned16(w)) {
    // h's tile row, then each wave's table of column scales
    const size_t smem = 16 * (size_t)K + sizeof(float) * kPersistWaves * kPersistMaxRows * 16;
    hipStream_t s = (hipStream_t)stream;
#define KRQ_PERSIST(UV, SV)                                                                                     \
  hipLaunchKernelGGL((k_lmhead_fp8_persist<UV, SV>), dim3(static_cast<unsigned>(blocks)), dim3(kPersistWaves * 64), \
                     smem, s, (const uint8_t*)h, h_scale, h_per_row != 0 && M > 1 ? 1 : 0, (const uint8_t*)w,    \
                     w_scale, w_per_row != 0 ? 1 : 0, static_cast<int>(M), V, static_cast<int>(K), (uint16_t*)logits, \
                     reinterpret_cast<Best*>(ws))
    // h's tile row: K 16-byte chunks over the workgroup's threads
    const bool small = K <= 10 * kPersistWaves * 64;
    if (ring == 10 && small)
      KRQ_PERSIST(10, 10);
    else if (ring == 10)
      KRQ_PERSIST(10, 16);
    else if (small)
      KRQ_PERSIST(8, 10);
    else
      KRQ_PERSIST(8, 16);
#undef KRQ_PERSIST
    hipLaunchKernelGGL(k_argmax_fold, dim3(static_cast<unsigned>(M)), dim3(kFoldThreads), 0, s,
                       reinterpret_cast<const Best*>(ws), ncand, static_cast<int>(M), idx_out);
    return krq_check_launch("lmhead_argmax");
  }
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
