// FP8 skinny GEMM / GEMV (M <= 32) entry points: y = (x8 . w8^T) * x_scale[m] * w_scale[n], fp32
// accumulate. The kernel template and its activation kinds: gemv_fp8_kernel.h; layout, step and
// epilogue conventions: gemv_common.h.
#include "gemv_fp8_kernel.h"

#include <algorithm>

using namespace krq;

namespace krq {
int plan_waves(int nsteps, int P, int U, int64_t blocks, bool act_wave) {
  if (nsteps < 2) return 1;
  // measured on MI355X at the Qwen3-4B shapes: a single-matrix block takes just enough waves for
  // all of its steps to be in flight at once (one memory round trip), up to 4; when that is not
  // enough, two waves, unless the grid has fewer blocks than the chip has CUs x 2 (the single-pass
  // O and down, 160 blocks: 5.07 / 8.74 us with 4 waves against 6.50 / 8.75 with 2 at M = 1),
  // where four keep more loads in flight. The two-matrix SwiGLU block takes two waves. Beside an
  // activation wave (one-row kernel), three instead of two (four waves in all): down 7.68 -> 7.16
  // us and the FP8 lm_head 64.7 -> 63.1 us at M = 1. With the deep rings (U of 8, 10 or 20 beside
  // the activation wave) the same rule gives one wave for up to U steps and two for up to 2U.
  // Multi-row blocks (two-slot rings) on a grid smaller than the chip (the one-pass residual GEMVs,
  // 160 blocks) take up to eight waves: O + residual 8.49 -> 7.99 us, down + residual 13.32 ->
  // 12.29 at M = 16 (at M = 1 four waves stay faster: 6.20 against 7.10 us for O).
  const int w = (nsteps + U - 1) / U;
  if (P != 1) return 2;
  if (w <= 4) return w;
  if (U == 2 && blocks < kCUs) return min(w, 8);
  if (blocks < 512) return 4;
  return act_wave ? 3 : 2;
}

// Ring of the multi-row matrix-core blocks (1 < M <= 16, one row block per workgroup): every step
// of the block in flight at once. Up to 10 steps of one matrix: one weight wave of 8 or 10 slots,
// which also writes its outputs straight from its accumulators; otherwise waves of 5 slots, at most
// four. Measured at M = 16 on tiled e4m3 rows (graph of 72 launches over 36 layers), against the
// earlier two-slot rings: QKV (10 steps) 5.55 -> 4.85 us, gate_up (20 steps, two matrices)
// 11.28 -> 11.17, down (19 steps) 7.56 -> 7.44, O (8 steps) 4.51 -> 4.53.
void rows_ring(int nsteps, int P, int* u, int* nw) {
  if (P == 1 && nsteps <= 8) {
    *u = 8;
    *nw = 1;
  } else if (P == 1 && nsteps <= 10) {
    *u = 10;
    *nw = 1;
  } else {
    *u = 5;
    *nw = min((nsteps + 4) / 5, 4);
  }
}
}  // namespace krq

namespace {

#define KRQ_GEMV_ARGS xb, x_scale, x_inv, x_per_row, wb, w_scale, w_per_row, m, NO, K, kts, out, aux


// one bf16 row: MT 1, no pairing; awc = chunks per lane of the activation wave (0: none); u = step
// slots per weight wave: 4, or (activation wave, tiled matrix-core kernels) 8, 10 or 20 for one
// matrix, 5 for the two-matrix SwiGLU block
template <int MODE, int LAYOUT, int XK, int ALGO>
void launch_row(int awc, int u, dim3 grid, dim3 block, size_t smem, hipStream_t s, const uint8_t* xb,
                const float* x_scale, const float* x_inv, int x_per_row, const uint8_t* wb,
                const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K, int kts, void* out,
                void* aux) {
  constexpr bool deep = LAYOUT == KRQ_W_TILED && ALGO == 1 && MODE != kOutArgmax;
  constexpr bool one = MODE != KRQ_OUT_SWIGLU;
  constexpr int U20 = deep && one ? kBigU : 4, U10 = deep && one ? kDeepU : 4, U8 = deep && one ? kMidU : 4;
  constexpr int U5 = deep && !one ? kSwiU : 4;
#define KRQ_ROW_U(AWC)                                                                                         \
  if (deep && one && u == kBigU)                                                                               \
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, ALGO, U20, 1, AWC>), grid, block, smem, s, KRQ_GEMV_ARGS); \
  else if (deep && one && u == kDeepU)                                                                         \
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, ALGO, U10, 1, AWC>), grid, block, smem, s, KRQ_GEMV_ARGS); \
  else if (deep && one && u == kMidU)                                                                          \
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, ALGO, U8, 1, AWC>), grid, block, smem, s, KRQ_GEMV_ARGS); \
  else if (deep && !one && u == kSwiU)                                                                         \
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, ALGO, U5, 1, AWC>), grid, block, smem, s, KRQ_GEMV_ARGS); \
  else                                                                                                         \
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, ALGO, 4, 1, AWC>), grid, block, smem, s, KRQ_GEMV_ARGS);
  if (awc == kAwRow) {
    KRQ_ROW_U(kAwRow)
  } else if (awc == kAwSmall) {
    KRQ_ROW_U(kAwSmall)
  } else if (awc == kAwLarge) {
    KRQ_ROW_U(kAwLarge)
  } else {
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, ALGO, 4, 1, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  }
#undef KRQ_ROW_U
}

// 1 < M <= 32 on e4m3 rows (tiled or row-major), one row block per workgroup, rows_ring's slots; MT
// 16-row tiles (2 above M = 16)
template <int MODE, int LAYOUT, int XK, int MT>
void launch_rows(int u, dim3 grid, dim3 block, size_t smem, hipStream_t s, const uint8_t* xb,
                 const float* x_scale, const float* x_inv, int x_per_row, const uint8_t* wb,
                 const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K, int kts, void* out,
                 void* aux) {
  constexpr bool one = MODE != KRQ_OUT_SWIGLU;
  if constexpr (XK == KRQ_X_FP8 || XK == KRQ_X_FP8_TILED) {
    if (MT == 1 && one && u == 10)
      hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, one ? 10 : 5, 1, 0>), grid, block, smem, s,
                         KRQ_GEMV_ARGS);
    else if (MT == 1 && one && u == 8)
      hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, one ? 8 : 5, 1, 0>), grid, block, smem, s,
                         KRQ_GEMV_ARGS);
    else
      hipLaunchKernelGGL((k_gemv_fp8<MT, MODE, LAYOUT, XK, 1, 5, 1, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  }
}

template <int MODE, int LAYOUT, int XK>
int launch(int algo, int pb, int awc, int u, bool rows, int M, dim3 grid, int nthreads, size_t smem,
           hipStream_t s, const uint8_t* xb, const float* x_scale, const float* x_inv, int x_per_row,
           const uint8_t* wb, const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K, int kts,
           void* out, void* aux) {
  const dim3 block(nthreads);
  constexpr int PB2 = MODE == KRQ_OUT_SWIGLU ? 1 : 2;  // no paired variant of the SwiGLU kernel
  if (rows) {
    if (M > 16)
      launch_rows<MODE, LAYOUT, XK, 2>(u, grid, block, smem, s, KRQ_GEMV_ARGS);
    else
      launch_rows<MODE, LAYOUT, XK, 1>(u, grid, block, smem, s, KRQ_GEMV_ARGS);
    return 0;
  }
  if constexpr (XK == KRQ_X_BF16_DYN) {  // (M == 1)
    if (algo == 2)
      launch_row<MODE, LAYOUT, XK, 2>(awc, u, grid, block, smem, s, KRQ_GEMV_ARGS);
    else
      launch_row<MODE, LAYOUT, XK, 1>(awc, u, grid, block, smem, s, KRQ_GEMV_ARGS);
    return 0;
  }
  if constexpr (XK == KRQ_X_BF16_STATIC) {
    if (awc > 0) {  // (M == 1)
      if (algo == 2)
        launch_row<MODE, LAYOUT, XK, 2>(awc, u, grid, block, smem, s, KRQ_GEMV_ARGS);
      else
        launch_row<MODE, LAYOUT, XK, 1>(awc, u, grid, block, smem, s, KRQ_GEMV_ARGS);
      return 0;
    }
  }
  if (algo == 2) {
    if constexpr (XK != KRQ_X_FP8_TILED)  // (rejected by the caller)
      hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 2, 4, 1, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  } else if (M <= 4) {
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, 4, 1, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  } else if (M <= 16 && pb == 2) {
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, 2, PB2, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  } else if (M <= 16) {
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, 2, 1, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  } else if (pb == 2) {
    hipLaunchKernelGGL((k_gemv_fp8<2, MODE, LAYOUT, XK, 1, 2, PB2, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  } else {
    hipLaunchKernelGGL((k_gemv_fp8<2, MODE, LAYOUT, XK, 1, 2, 1, 0>), grid, block, smem, s, KRQ_GEMV_ARGS);
  }
  return 0;
}

template <int MODE, int LAYOUT>
void launch_xk(int xk, int algo, int pb, int awc, int u, bool rows, int M, dim3 grid, int nthreads, size_t smem,
               hipStream_t s, const uint8_t* xb, const float* x_scale, const float* x_inv, int x_per_row,
               const uint8_t* wb, const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K, int kts,
               void* out, void* aux) {
#define KRQ_XK_ARGS algo, pb, awc, u, rows, M, grid, nthreads, smem, s, KRQ_GEMV_ARGS
  if (xk == KRQ_X_FP8)
    launch<MODE, LAYOUT, KRQ_X_FP8>(KRQ_XK_ARGS);
  else if (xk == KRQ_X_FP8_TILED)
    launch<MODE, LAYOUT, KRQ_X_FP8_TILED>(KRQ_XK_ARGS);
  else if (xk == KRQ_X_BF16_DYN)
    launch<MODE, LAYOUT, KRQ_X_BF16_DYN>(KRQ_XK_ARGS);
  else
    launch<MODE, LAYOUT, KRQ_X_BF16_STATIC>(KRQ_XK_ARGS);
#undef KRQ_XK_ARGS
}

// The SwiGLU as k_gemv_fp8_swiglu_mixed (nfull two-matrix blocks, then half-pair blocks) for the
// kernels the plan picked: the one-row kernel beside its activation wave (five-slot rings) or the
// multi-row ring on e4m3 rows (one or two 16-row tiles). False for any other plan, which keeps the
// plain launch. With two row tiles the block takes 228 VGPRs, so two fit per CU and the launch's
// last blocks run in a second round: as half-pair blocks that round is half as long (gate_up at
// M = 32: 13.1 -> 12.7 us).
template <int XK>
bool launch_swiglu_mixed(int awc, int u, bool rows, int M, int nfull, dim3 grid, int nthreads, size_t smem,
                         hipStream_t s, const uint8_t* xb, const float* x_scale, const float* x_inv, int x_per_row,
                         const uint8_t* wb, const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K,
                         int kts, void* out, void* aux) {
  const dim3 block(nthreads);
  if constexpr (XK == KRQ_X_FP8 || XK == KRQ_X_FP8_TILED) {
    if (!rows || u != 5) return false;
    // (multi-row blocks: the half blocks first; at M = 16 gate_up 10.65 -> 10.52 us, the C3 step
    // 37.07 -> 36.95; at M = 32 even within noise)
    if (M > 16)
      hipLaunchKernelGGL((k_gemv_fp8_swiglu_mixed<KRQ_W_TILED, XK, 1, 5, 0, 2>), grid, block, smem, s, KRQ_GEMV_ARGS,
                         nfull, 1);
    else
      hipLaunchKernelGGL((k_gemv_fp8_swiglu_mixed<KRQ_W_TILED, XK, 1, 5, 0>), grid, block, smem, s, KRQ_GEMV_ARGS,
                         nfull, 1);
  } else {
    if (M != 1 || u != kSwiU) return false;
    if (awc == kAwRow)
      hipLaunchKernelGGL((k_gemv_fp8_swiglu_mixed<KRQ_W_TILED, XK, 1, kSwiU, kAwRow>), grid, block, smem, s,
                         KRQ_GEMV_ARGS, nfull, 0);
    else if (awc == kAwSmall)
      hipLaunchKernelGGL((k_gemv_fp8_swiglu_mixed<KRQ_W_TILED, XK, 1, kSwiU, kAwSmall>), grid, block, smem, s,
                         KRQ_GEMV_ARGS, nfull, 0);
    else if (awc == kAwLarge)
      hipLaunchKernelGGL((k_gemv_fp8_swiglu_mixed<KRQ_W_TILED, XK, 1, kSwiU, kAwLarge>), grid, block, smem, s,
                         KRQ_GEMV_ARGS, nfull, 0);
    else
      return false;
  }
  return true;
}

// ---------------------------------------------------------------------------------------------
// Wide blocks at 1 < M <= 32 (MT activation row tiles) on tiled e4m3 rows and tiled weights. At
// M = 32 a 16-column block brings two activation bytes from L2 per weight byte. Here a workgroup
// owns kWideRb adjacent row blocks (one per wave, 64 output columns) of one K split: its waves copy
// the split's activation tiles (MT x kts KB) into LDS once with direct-to-LDS loads, and each wave
// then streams only its row block's weights through a ring of U step slots, reading the A operand
// from LDS. The sums are those of the one-row-block launch the plan would otherwise run with NS
// waves (step j in wave j % NS, the waves' sums added in wave order): here step j goes to
// accumulator set j % NS of the one wave, and the sets are added in the same order, so the
// outputs are the same bit for bit. Every output is written from the wave that owns it.
constexpr int kWideRb = 4;

// 32-bit LDS address of a pointer into a __shared__ array (wave-uniform)
KRQ_DEV uint32_t wide_lds_addr(const uint8_t* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)p)));
}

// global_load_lds_dwordx4: 16 bytes per lane from base + 16 lane into LDS at l + 16 lane. From inline
// assembly, so the compiler does not count it: the kernel waits for these loads itself, and issues
// them before every other load (vector memory loads complete in order, so the compiler's own waits
// for later loads stay correct).
KRQ_DEV void wide_dma(const uint8_t* base, uint32_t l, int lane) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(16u * lane), "s"(base)
               : "memory", "m0");
}

template <int MODE, int U, int TL, int NS, int MT>
__global__ __launch_bounds__(kWideRb * 64) void k_gemv_wide32(const uint8_t* __restrict__ x, const float* __restrict__ xsc,
                                                              int x_per_row, const uint8_t* __restrict__ w8,
                                                              const float* __restrict__ wsc, int w_per_row, int M,
                                                              int64_t NO, int64_t K, int kts, void* __restrict__ out) {
  static_assert(MODE == KRQ_OUT_PARTIAL || MODE == KRQ_OUT_BF16 || MODE == KRQ_OUT_SWIGLU, "wide block modes");
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  static_assert(2 * P * U < 64, "vmcnt range");
  static_assert(U % NS == 0, "slot u feeds set u % NS");
  __shared__ __align__(1024) uint8_t xt[TL * 1024];  // tile (mt, t) of the split at (mt kts + t) KB
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int r = lane & 15, g = lane >> 4;
  const int sidx = blockIdx.y;
  const int64_t rb = (int64_t)blockIdx.x * kWideRb + wave;
  const int64_t tbase = (int64_t)sidx * kts, ktiles = K >> 6;
  const int nsteps = (kts + 1) >> 1;
  KRQ_STAMP(0, threadIdx.x == 0);

  // the split's activation tiles into LDS (the oldest loads of every wave)
  const uint32_t lx = wide_lds_addr(xt);
  for (int i = wave; i < MT * kts; i += kWideRb) {
    const int mt = i >= kts ? 1 : 0, t = i - mt * kts;
    wide_dma(x + ((int64_t)mt * ktiles + tbase + t) * 1024, lx + 1024u * static_cast<uint32_t>(i), lane);
  }
  // the epilogue's weight and row scales, loaded now (behind the tiles, ahead of the ring: the
  // tiles' wait below covers them) so their latency is not paid after the loop
  const int64_t n = rb * 16 + r;
  const float wg = wsc[w_per_row ? n : 0];
  const float wu = P == 2 ? wsc[w_per_row ? NO + n : 0] : 0.0f;
  float xs[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[mt][i] = xsc[x_per_row ? min(mt * 16 + 4 * g + i, M - 1) : 0];
  // the weight ring: slot u holds step u, then u + U, ...; a slot past the last step reloads it
  // (masked where consumed)
  uint4 wl[P][U], wh[P][U];
  auto load_slot = [&](int u, int cc) {
    const int j = min(cc, nsteps - 1);
    const int64_t t0 = tbase + 2 * j, t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t rr = p == 1 ? rb + (NO >> 4) : rb;
      wl[p][u] = ld16nt(w_addr<KRQ_W_TILED>(w8, rr, t0, K, lane));
      wh[p][u] = ld16nt(w_addr<KRQ_W_TILED>(w8, rr, t1, K, lane));
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) {
    load_slot(u, u);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the tiles have landed once at most the ring's loads are outstanding; then a barrier that
  // orders the LDS writes only (a full fence would wait for the whole ring)
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * P * U) : "memory");
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  KRQ_STAMP(1, threadIdx.x == 0);

  v4f acc[P][NS][MT];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int q = 0; q < NS; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[p][q][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](int u, int cc) {
    const int j = min(cc, nsteps - 1);
    const bool ok = cc < nsteps, hi = ok && (2 * j + 1 < kts);
    v8i A[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint8_t* xr = xt + (mt * kts) * 1024 + lane * 16;
      const uint4 lo = *reinterpret_cast<const uint4*>(xr + (2 * j) * 1024);
      const uint4 hh = sel4(2 * j + 1 < kts, *reinterpret_cast<const uint4*>(xr + min(2 * j + 1, kts - 1) * 1024));
      A[mt] = pack_v8i(lo, hh);
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const v8i B = pack_v8i(sel4(ok, wl[p][u]), sel4(hi, wh[p][u]));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[p][u % NS][mt] =
            __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[mt], B, acc[p][u % NS][mt], 0, 0, 0, 0, 0, 0);
    }
  };
  int base = 0;
  for (; base + U < nsteps; base += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      consume(u, base + u);
      load_slot(u, base + u + U);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) consume(u, base + u);
  KRQ_STAMP(2, threadIdx.x == 0);

  // the sets in wave order (from zero, as the epilogue sums the waves; one set: as is)
  v4f sum[P][MT];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (NS == 1) {
        sum[p][mt] = acc[p][0][mt];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float a = 0.0f;
#pragma unroll
          for (int q = 0; q < NS; ++q) a += acc[p][q][mt][i];
          sum[p][mt][i] = a;
        }
      }
    }
  // element i of lane l: row 16 mt + 4 (l / 16) + i, column 16 rb + l % 16
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = mt * 16 + 4 * g + i;
      if (m >= M) continue;
      if constexpr (MODE == KRQ_OUT_PARTIAL) {
        reinterpret_cast<float*>(out)[((int64_t)sidx * M + m) * NO + n] = sum[0][mt][i] * xs[mt][i] * wg;
      } else if constexpr (MODE == KRQ_OUT_BF16) {
        reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = f32_to_bf16(sum[0][mt][i] * xs[mt][i] * wg);
      } else {
        const float gg = round_bf16(sum[0][mt][i] * xs[mt][i] * wg);
        const float uu = round_bf16(sum[1][mt][i] * xs[mt][i] * wu);
        const float sl = round_bf16(gg / (1.0f + expf(-gg)));
        reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = f32_to_bf16(sl * uu);
      }
    }
  KRQ_STAMP(3, threadIdx.x == 0);
}

// The wide-block launch when it applies (1 < M <= 32, tiled e4m3 rows and tiled weights, the
// plain output modes, one row block per block in the plan (pb 1) and ns <= 4 waves per row block,
// row blocks a multiple of kWideRb, the split's tiles within LDS); false otherwise.
bool launch_wide32(int M, int mode, int x_kind, int w_layout, int algo, const void* aux, int pb, int ns, int64_t NO,
                   int split, int kts, hipStream_t s, const uint8_t* xb, const float* x_scale, int x_per_row,
                   const uint8_t* wb, const float* w_scale, int w_per_row, int64_t K, void* out) {
  // (at M = 16, graph-timed: down 7.48 -> 7.03 us, QKV 4.87 -> 4.66, O 4.52 -> 4.20 with eight
  // slots for its eight steps; ten, two of them masked, measured 4.57)
  if (M < 2 || M > 32 || x_kind != KRQ_X_FP8_TILED || w_layout != KRQ_W_TILED || algo != 1 || pb != 1) return false;
  // (the two-matrix SwiGLU block measured slower wide: gate_up 12.7 -> 15.1 us at 254 VGPRs)
  if (!(mode == KRQ_OUT_PARTIAL || mode == KRQ_OUT_BF16)) return false;
  const int mt = M > 16 ? 2 : 1;  // activation row tiles
  if ((NO / 16) % kWideRb != 0 || mt * kts > 96 || ns < 1 || ns > 4) return false;
  const dim3 grid(static_cast<unsigned>(NO / 16 / kWideRb), static_cast<unsigned>(split)), block(kWideRb * 64);
  const int m = M;
  // slots: a multiple of the sets, ten at most (two-matrix blocks take 254 VGPRs with ten); one
  // set over at most eight steps: eight. Four sets (down, 19 steps per split): four slots, one per
  // set (graph-timed, same box, alternating: down at M = 16 6.80 -> 6.33 us, at M = 32 8.21 ->
  // 7.44; rings of 12 and 20 at M = 16 measured 7.1 and 7.2). Two sets (QKV at M = 32): four
  // slots, 5.84 -> 5.63 us (two slots 6.33)
#define KRQ_WIDE(MODE_, U_, TL_, NS_)                                                                              \
  if (M > 16)                                                                                                   \
    hipLaunchKernelGGL((k_gemv_wide32<MODE_, U_, TL_, NS_, 2>), grid, block, 0, s, xb, x_scale, x_per_row, wb,      \
                       w_scale, w_per_row, m, NO, K, kts, out);                                                     \
  else                                                                                                            \
    hipLaunchKernelGGL((k_gemv_wide32<MODE_, U_, TL_, NS_, 1>), grid, block, 0, s, xb, x_scale, x_per_row, wb,      \
                       w_scale, w_per_row, m, NO, K, kts, out)
#define KRQ_WIDE_TL(MODE_, U_, NS_)                  \
  if (mt * kts <= 48) KRQ_WIDE(MODE_, U_, 48, NS_);    \
  else KRQ_WIDE(MODE_, U_, 96, NS_);
#define KRQ_WIDE_U(MODE_)                                 \
  if (ns == 1 && kts <= 16) { KRQ_WIDE_TL(MODE_, 8, 1) }   \
  else if (ns == 1) { KRQ_WIDE_TL(MODE_, 10, 1) }          \
  else if (ns == 2) { KRQ_WIDE_TL(MODE_, 4, 2) }          \
  else if (ns == 3) { KRQ_WIDE_TL(MODE_, 9, 3) }           \
  else { KRQ_WIDE_TL(MODE_, 4, 4) }
  if (mode == KRQ_OUT_PARTIAL) {
    KRQ_WIDE_U(KRQ_OUT_PARTIAL)
  } else {
    KRQ_WIDE_U(KRQ_OUT_BF16)
  }
#undef KRQ_WIDE_U
#undef KRQ_WIDE_TL
#undef KRQ_WIDE
  return true;
}

// ---------------------------------------------------------------------------------------------
// Wide one-row blocks (M = 1, bf16 activations scaled in the kernel, tiled weights): a workgroup
// owns RB adjacent row blocks of one K split, one weight wave each holding every step of its row
// block in a ring of U slots, and one activation wave that scales and quantizes the split's slice
// into LDS once for all of them (the one-row launch's activation wave does it once per row block:
// at K = 9,728 that is the whole bf16 row read per 16 output columns). Each row block's products,
// their order and the output arithmetic are those of the one-row launch with one weight wave per
// row block, so the outputs are the same bit for bit.
template <int MODE, int XK, int U, int AWC, int RB>
__global__ __launch_bounds__((RB + 1) * 64) void k_gemv_wide1(const uint8_t* __restrict__ x,
                                                             const float* __restrict__ xsc,
                                                             const float* __restrict__ xinv,
                                                             const uint8_t* __restrict__ w8,
                                                             const float* __restrict__ wsc, int w_per_row,
                                                             int64_t NO, int64_t K, int kts, void* __restrict__ out) {
  static_assert(MODE == KRQ_OUT_PARTIAL || MODE == KRQ_OUT_BF16, "wide one-row modes");
  static_assert(XK == KRQ_X_BF16_DYN || XK == KRQ_X_BF16_STATIC, "bf16 activations scaled in the kernel");
  static_assert(2 * U < 64, "vmcnt range");
  extern __shared__ __align__(16) uint8_t xq[];  // the split's e4m3 slice (ks bytes), then its scale
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int sidx = blockIdx.y;
  const int ks = kts * 64;
  const int64_t k0 = (int64_t)sidx * ks, tbase = (int64_t)sidx * kts;
  const int nsteps = (kts + 1) >> 1;
  float* xs_l = reinterpret_cast<float*>(xq + ks);
  KRQ_STAMP(0, threadIdx.x == 0);
  if (wave == RB) {
    activation_wave<XK, AWC, false, false>(x, xsc, xinv, K, k0, ks, lane, xq, xs_l, FusedArgs{});
    KRQ_STAMP(1, lane == 0);
    // the slice and its scale are in LDS (a barrier that orders LDS only: the weight waves' rings
    // stay in flight)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    return;
  }
  const int r = lane & 15, g = lane >> 4;
  const int64_t rb = (int64_t)blockIdx.x * RB + wave;
  const float ws = wsc[w_per_row ? rb * 16 + r : 0];  // (read now, not after the loop)
  // the weight ring: slot u holds step u, then u + U, ...; a slot past the last step reloads it
  // (masked where consumed)
  uint4 wl[U], wh[U];
  auto load_slot = [&](int u, int cc) {
    const int j = min(cc, nsteps - 1);
    const int64_t t0 = tbase + 2 * j, t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
    wl[u] = ld16nt(w_addr<KRQ_W_TILED>(w8, rb, t0, K, lane));
    wh[u] = ld16nt(w_addr<KRQ_W_TILED>(w8, rb, t1, K, lane));
  };
#pragma unroll
  for (int u = 0; u < U; ++u) {
    load_slot(u, u);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  // A: every row is the one activation row (lane 16 g + r: bytes 16 g .. 16 g + 15 of the step's
  // 64-byte chunks), as in the one-row launch
  auto consume = [&](int u, int cc) {
    const int j = min(cc, nsteps - 1);
    const bool ok = cc < nsteps, hi = ok && (2 * j + 1 < kts);
    const uint8_t* xr = xq + g * 16;
    const uint4 lo = *reinterpret_cast<const uint4*>(xr + (2 * j) * 64);
    const uint4 hh = sel4(2 * j + 1 < kts, *reinterpret_cast<const uint4*>(xr + min(2 * j + 1, kts - 1) * 64));
    const v8i B = pack_v8i(sel4(ok, wl[u]), sel4(hi, wh[u]));
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(pack_v8i(lo, hh), B, acc, 0, 0, 0, 0, 0, 0);
  };
  int base = 0;
  for (; base + U < nsteps; base += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      consume(u, base + u);
      load_slot(u, base + u + U);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) consume(u, base + u);
  KRQ_STAMP(2, threadIdx.x == 0);
  // row 0 of the product: element 0 of lanes 0-15, column 16 rb + lane
  if (g == 0) {
    const int64_t n = rb * 16 + r;
    const float y = acc[0] * xs_l[0] * ws;
    if constexpr (MODE == KRQ_OUT_BF16)
      reinterpret_cast<uint16_t*>(out)[n] = f32_to_bf16(y);
    else
      reinterpret_cast<float*>(out)[(int64_t)sidx * NO + n] = y;
  }
  KRQ_STAMP(3, threadIdx.x == 0);
}

constexpr int kWide1Rb = 4;

// The wide one-row launch when it applies (M = 1, bf16 activations with the plan's activation
// wave, tiled weights, the plain output modes, a plan of one weight wave per row block holding
// all of its steps, row blocks a multiple of kWide1Rb); false otherwise.
bool launch_wide1(int M, int mode, int x_kind, int w_layout, int algo, int pb, int nw, int awc, int u, int64_t NO,
                  int split, int kts, hipStream_t s, const uint8_t* xb, const float* x_scale, const float* x_inv,
                  const uint8_t* wb, const float* w_scale, int w_per_row, int64_t K, void* out) {
  if (M != 1 || awc <= 0 || algo != 1 || w_layout != KRQ_W_TILED || pb != 1 || nw != 1) return false;
  if (!(mode == KRQ_OUT_PARTIAL || mode == KRQ_OUT_BF16)) return false;
  if (!(x_kind == KRQ_X_BF16_DYN || x_kind == KRQ_X_BF16_STATIC)) return false;
  if ((NO / 16) % kWide1Rb != 0 || !(u == kMidU || u == kDeepU || u == kBigU)) return false;
  // at most 96 KB of weights per workgroup: the wide launch uses one workgroup per CU on fewer CUs,
  // so a CU streams more bytes than in the one-row launch. Measured (graph of 72 launches, same box,
  // alternating): QKV 4.53 -> 4.27 us (80 KB), O 3.99 -> 3.85 (64 KB), down 6.34 -> 6.83 (152 KB).
  if ((int64_t)kWide1Rb * 16 * kts * 64 > 96 * 1024) return false;
  // and splits of more than 16 tiles (QKV, not O): alone each gains, but in the decode step O right
  // after QKV on the wide blocks costs more than both gain (C5 at M = 1, same box, alternating:
  // 1,038.5 us per step with neither, 1,038.3 with QKV, 1,035.8 with O, 1,059.7 with both; the
  // kernel trace shows an extra ~3.7 us gap before O when both run wide)
  if (kts <= 16) return false;
  if (!(awc == kAwRow || awc == kAwSmall || awc == kAwLarge)) return false;
  const dim3 grid(static_cast<unsigned>(NO / 16 / kWide1Rb), static_cast<unsigned>(split)), block((kWide1Rb + 1) * 64);
  const size_t smem = (size_t)kts * 64 + 16;
#define KRQ_W1(MODE_, XK_, U_, AWC_)                                                                        \
  hipLaunchKernelGGL((k_gemv_wide1<MODE_, XK_, U_, AWC_, kWide1Rb>), grid, block, smem, s, xb, x_scale, x_inv, \
                     wb, w_scale, w_per_row, NO, K, kts, out)
#define KRQ_W1_AWC(MODE_, XK_, U_)                      \
  if (awc == kAwRow) { KRQ_W1(MODE_, XK_, U_, kAwRow); }     \
  else if (awc == kAwSmall) { KRQ_W1(MODE_, XK_, U_, kAwSmall); } \
  else { KRQ_W1(MODE_, XK_, U_, kAwLarge); }
#define KRQ_W1_U(MODE_, XK_)                              \
  if (u == kMidU) { KRQ_W1_AWC(MODE_, XK_, kMidU) }         \
  else if (u == kDeepU) { KRQ_W1_AWC(MODE_, XK_, kDeepU) }  \
  else { KRQ_W1_AWC(MODE_, XK_, kBigU) }
  if (x_kind == KRQ_X_BF16_DYN) {
    if (mode == KRQ_OUT_PARTIAL) { KRQ_W1_U(KRQ_OUT_PARTIAL, KRQ_X_BF16_DYN) }
    else { KRQ_W1_U(KRQ_OUT_BF16, KRQ_X_BF16_DYN) }
  } else {
    if (mode == KRQ_OUT_PARTIAL) { KRQ_W1_U(KRQ_OUT_PARTIAL, KRQ_X_BF16_STATIC) }
    else { KRQ_W1_U(KRQ_OUT_BF16, KRQ_X_BF16_STATIC) }
  }
#undef KRQ_W1_U
#undef KRQ_W1_AWC
#undef KRQ_W1
  return true;
}

// Activation-wave chunks per lane holding `span` bf16 elements (0: too long for one wave).
int aw_chunks(int64_t span) {
  return span <= 512 * kAwRow ? kAwRow : span <= 512 * kAwSmall ? kAwSmall : span <= 512 * kAwLarge ? kAwLarge : 0;
}

}  // namespace

int krq::gemv_fp8_run(const void* x, int x_kind, const float* x_scale, const float* x_inv,
                      int x_per_row, const void* w8, int w_layout, const float* w_scale,
                      int w_per_row, int64_t M, int64_t N, int64_t K, int split, int mode,
                      int algo, void* out, void* aux, void* stream) {
  KRQ_REQUIRE(x && w8 && w_scale && (out || mode == kOutArgmax) && (aux || mode != kOutArgmax),
              "gemv_fp8: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w8), "gemv_fp8: x and w8 must be 16-byte aligned");
  KRQ_REQUIRE(x_kind >= KRQ_X_FP8 && x_kind <= KRQ_X_FP8_TILED, "gemv_fp8: bad x_kind %d", x_kind);
  KRQ_REQUIRE(x_kind == KRQ_X_BF16_DYN || x_scale, "gemv_fp8: x_scale is required");
  KRQ_REQUIRE(x_kind != KRQ_X_BF16_STATIC || x_inv, "gemv_fp8: x_inv is required");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_fp8: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(N > 0 && K > 0 && split >= 1, "gemv_fp8: bad shape N=%lld K=%lld split=%d",
              (long long)N, (long long)K, split);
  KRQ_REQUIRE(K % split == 0 && (K / split) % 64 == 0,
              "gemv_fp8: no tiling divides K_SPLIT (K=%lld split=%d; K/split must be a multiple of 64)",
              (long long)K, split);
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "gemv_fp8: bad layout %d", w_layout);
  KRQ_REQUIRE(mode >= KRQ_OUT_BF16 && mode <= kOutArgmax, "gemv_fp8: bad mode %d", mode);
  KRQ_REQUIRE(algo >= 0 && algo <= 2, "gemv_fp8: bad algo %d", algo);
  KRQ_REQUIRE(algo != 2 || M == 1, "gemv_fp8: the vector-ALU kernel takes M == 1 only");
  KRQ_REQUIRE(algo != 2 || x_kind != KRQ_X_FP8_TILED, "gemv_fp8: tiled activations take the matrix-core kernel");
  // In-kernel per-token scaling takes one row. (Scaling M > 1 rows per token inside the GEMV means
  // every workgroup reads the whole bf16 rows for their amax: at M = 16 the QKV / O / gate_up steps
  // measured ~14 us each that way against 4.8 + 2.5 us for quant_rows_tiled and the GEMV.)
  KRQ_REQUIRE(x_kind != KRQ_X_BF16_DYN || M == 1, "gemv_fp8: in-kernel per-token scaling takes M == 1");
  KRQ_REQUIRE(mode == KRQ_OUT_PARTIAL || split == 1, "gemv_fp8: split %d needs the partials output", split);
  KRQ_REQUIRE(mode != kOutArgmax || N <= 0x7fffffff, "gemv_fp8: N=%lld too large for int indices", (long long)N);
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  KRQ_REQUIRE(NO % 16 == 0 && (mode != KRQ_OUT_SWIGLU || N % 2 == 0),
              "gemv_fp8: no tiling divides N=%lld (output columns must be a multiple of 16)", (long long)N);
  KRQ_REQUIRE(NO / 16 <= 0x7fffffff && split <= 65535, "gemv_fp8: grid too large");
  if (algo == 0) algo = 1;
  const int kts = static_cast<int>(K / split / 64);
  const int ks = kts * 64;
  const int nsteps = (kts + 1) / 2;
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w8;
  const int m = static_cast<int>(M);
  hipStream_t s = (hipStream_t)stream;
  // Paired row blocks for the multi-row matrix-core kernels. Measured: pairing halves the blocks,
  // which costs the Qwen3-4B projections (640-768 blocks) more than the saved activation reads
  // gain; the lm_head (9,496 blocks) gains 10-15%.
  const int pb = (mode != KRQ_OUT_SWIGLU && algo != 2 && M > 4 && (NO / 16) % 2 == 0 &&
                  (NO / 16) * split >= 4096) ? 2 : 1;
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : pb;
  const int MT = (algo == 2 || M <= 16) ? 1 : 2;
  const int64_t blocks = NO / 16 / pb * split;
  // Multi-row blocks on e4m3 rows (1 < M <= 16, one row block per workgroup, matrix cores) take
  // rows_ring. So do 16 < M <= 32 (two row tiles) on splits of more than 8 steps, with five-slot
  // waves (ten slots with two row tiles spill): at M = 32 QKV 6.99 -> 6.67 us, gate_up 13.70 ->
  // 13.12, down 9.82 -> 9.51, while O (8 steps) lost with it (5.77 -> 6.49 with one wave of 8
  // slots, 6.39 with two of 5) and keeps the ring of two.
  const bool rows = M > 1 && (M <= 16 || (M <= 32 && (nsteps > 8 || mode == KRQ_OUT_SWIGLU))) && pb == 1 &&
                    algo == 1 && (x_kind == KRQ_X_FP8 || x_kind == KRQ_X_FP8_TILED);
  int awc = 0, u = 0, nw = 0, na = 0;
  if (rows) {
    rows_ring(nsteps, P, &u, &nw);
    if (M > 16 && u > 5) {
      u = 5;
      nw = (nsteps + 4) / 5;
    }
  } else {
    // one-row kind: an activation wave holding the whole row (K <= 10240), else every wave takes
    // part in the prologue. Measured at M = 1: QKV 5.92 -> 5.29 us, O 5.15 -> 4.41, down 7.91 ->
    // 7.16, FP8 lm_head 64.9 -> 63.1; the SwiGLU GEMV 11.24 -> 10.86 with the five-slot ring below
    // (with four slots the activation wave did not pay: 11.45). With static scales (M == 1) the
    // wave quantizes the slice alone.
    if (x_kind == KRQ_X_BF16_DYN) awc = aw_chunks(K);
    if (x_kind == KRQ_X_BF16_STATIC && M == 1) awc = aw_chunks(ks);
    // With fewer blocks than CUs each block's prologue is its CU's critical path, and spreading it
    // over all waves is faster (the one-pass residual GEMVs, 160 blocks: O 6.21 against 6.65 us).
    if (blocks < kCUs) awc = 0;
    na = awc > 0 ? 1 : 0;
    // Deep ring beside the activation wave (tiled single-matrix matrix-core kernels): each weight
    // wave holds all of its steps in flight at once, one memory round trip and no masked slots.
    // Measured at M = 1 (graph of 72 launches over 36 layers): QKV (10 steps, one wave of 10)
    // 5.24 -> 4.84 us, O (8 steps, one wave of 8) 4.38 -> 4.25, down (19 steps) two waves of 10
    // 7.51 -> 6.90, then one wave of 20 (which also writes its outputs straight from its
    // accumulators) 6.68 -> 6.33; rings of 8 for 10 steps (two rounds) or 12 (masked slots) measured
    // slower. The two-matrix SwiGLU block (four loads a step) takes five slots with two weight
    // waves (ten slots, given the registers by launch bounds of its three waves, measured slower:
    // 10.51 -> 11.00 us). The lm_head (argmax epilogue, 9,496 blocks) keeps four slots: 63.1
    // against 64.4 us.
    u = (algo == 2 || M <= 4) ? 4 : 2;
    if (awc > 0 && algo == 1 && w_layout == KRQ_W_TILED && mode != kOutArgmax)
      u = mode == KRQ_OUT_SWIGLU ? kSwiU : nsteps <= kMidU ? kMidU : nsteps <= kDeepU ? kDeepU
                                                               : nsteps <= kBigU ? kBigU : kDeepU;
    nw = plan_waves(nsteps, P, u, blocks, awc > 0);
    // the other fused prologues hold at most kXChunks 16-byte chunks per thread
    int64_t xchunks = 0;
    if (x_kind == KRQ_X_BF16_DYN && awc == 0) xchunks = (K + 7) / 8;
    if (x_kind == KRQ_X_BF16_STATIC && awc == 0) xchunks = M * (ks / 8);
    const int xc = x_kind == KRQ_X_BF16_DYN ? kXChunksDyn : kXChunks;
    while ((int64_t)nw * 64 * xc < xchunks && nw < kMaxThreads / 64) ++nw;
    KRQ_REQUIRE((int64_t)nw * 64 * xc >= xchunks,
                "gemv_fp8: activation slice of %lld elements too large for in-kernel quantization",
                (long long)(xchunks * 8));
    if (awc > 0) nw = min(nw, kMaxThreads / 64 - 1);
  }
  // one row with the activation wave: four row blocks per workgroup share its slice
  if (launch_wide1(m, mode, x_kind, w_layout, algo, pb, nw, awc, u, NO, split, kts, s, xb, x_scale, x_inv, wb,
                   w_scale, w_per_row, K, out))
    return krq_check_launch("gemv_fp8");
  // 1 < M <= 32 on tiled rows: the wide-block kernel, with this plan's waves as its sets
  if (launch_wide32(m, mode, x_kind, w_layout, algo, aux, pb, nw, NO, split, kts, s, xb, x_scale, x_per_row, wb,
                    w_scale, w_per_row, K, out))
    return krq_check_launch("gemv_fp8");
  // LDS: the weight waves' partial sums, then the bf16 kinds' quantized slice [M][ks]
  const size_t slice = x_kind == KRQ_X_FP8 || x_kind == KRQ_X_FP8_TILED ? 0 : (size_t)M * ks;
  const size_t smem = (size_t)nw * P * MT * 256 * sizeof(float) + slice;
  const dim3 grid(static_cast<unsigned>(NO / 16 / pb), static_cast<unsigned>(split));
  const int nthreads = (nw + na) * 64;
  // A SwiGLU grid of column blocks a little over a multiple of the CUs (gate_up: 608 = 2 x 256 +
  // 96) runs its last ones as half-pair blocks in the same launch, so no CU streams a third full
  // block (same steps per wave, so the same output bits).
  if (mode == KRQ_OUT_SWIGLU && algo == 1 && w_layout == KRQ_W_TILED) {
    const int64_t nrbs = NO / 16, rem = nrbs % kCUs;
    if (nrbs > 2 * kCUs && rem != 0 && 2 * rem <= kCUs) {
      const int nfull = static_cast<int>(nrbs - rem);
      const dim3 gm(static_cast<unsigned>(nfull + 2 * rem), 1);
#define KRQ_MIXED(XKV)                                                                                         \
  launch_swiglu_mixed<XKV>(awc, u, rows, m, nfull, gm, nthreads, smem, s, xb, x_scale, x_inv, x_per_row, wb, \
                           w_scale, w_per_row, m, NO, K, kts, out, aux)
      bool ok = false;
      if (x_kind == KRQ_X_FP8) ok = KRQ_MIXED(KRQ_X_FP8);
      else if (x_kind == KRQ_X_FP8_TILED) ok = KRQ_MIXED(KRQ_X_FP8_TILED);
      else if (x_kind == KRQ_X_BF16_DYN) ok = KRQ_MIXED(KRQ_X_BF16_DYN);
      else ok = KRQ_MIXED(KRQ_X_BF16_STATIC);
#undef KRQ_MIXED
      if (ok) return krq_check_launch("gemv_fp8");
    }
  }
#define KRQ_FP8_CASE(MODE, LAYOUT)                                                                          \
  launch_xk<MODE, LAYOUT>(x_kind, algo, pb, awc, u, rows, m, grid, nthreads, smem, s, xb, x_scale, x_inv, \
                          x_per_row, wb, w_scale, w_per_row, m, NO, K, kts, out, aux)
  if (w_layout == KRQ_W_TILED) {
    if (mode == KRQ_OUT_BF16) KRQ_FP8_CASE(KRQ_OUT_BF16, KRQ_W_TILED);
    else if (mode == KRQ_OUT_PARTIAL) KRQ_FP8_CASE(KRQ_OUT_PARTIAL, KRQ_W_TILED);
    else if (mode == KRQ_OUT_SWIGLU) KRQ_FP8_CASE(KRQ_OUT_SWIGLU, KRQ_W_TILED);
    else KRQ_FP8_CASE(kOutArgmax, KRQ_W_TILED);
  } else {
    if (mode == KRQ_OUT_BF16) KRQ_FP8_CASE(KRQ_OUT_BF16, KRQ_W_ROWMAJOR);
    else if (mode == KRQ_OUT_PARTIAL) KRQ_FP8_CASE(KRQ_OUT_PARTIAL, KRQ_W_ROWMAJOR);
    else if (mode == KRQ_OUT_SWIGLU) KRQ_FP8_CASE(KRQ_OUT_SWIGLU, KRQ_W_ROWMAJOR);
    else KRQ_FP8_CASE(kOutArgmax, KRQ_W_ROWMAJOR);
  }
#undef KRQ_FP8_CASE
  return krq_check_launch("gemv_fp8");
}

extern "C" int krq_gemv_fp8(const void* x, int x_kind, const float* x_scale, const float* x_inv,
                            int x_per_row, const void* w8, int w_layout, const float* w_scale,
                            int w_per_row, int64_t M, int64_t N, int64_t K, int split, int mode,
                            int algo, void* out, void* stream) {
  KRQ_REQUIRE(mode >= KRQ_OUT_BF16 && mode <= KRQ_OUT_SWIGLU, "gemv_fp8: bad mode %d", mode);
  return gemv_fp8_run(x, x_kind, x_scale, x_inv, x_per_row, w8, w_layout, w_scale, w_per_row, M, N,
                      K, split, mode, algo, out, nullptr, stream);
}

extern "C" int krq_gemv_swiglu_fp8_cast(const void* x, int x_kind, const float* x_scale, const float* x_inv,
                                        int x_per_row, const void* w8, int w_layout, const float* w_scale,
                                        int w_per_row, int64_t M, int64_t N, int64_t K, const float* out_inv,
                                        void* x8_tiled, void* stream) {
  KRQ_REQUIRE(out_inv && x8_tiled, "gemv_swiglu_fp8_cast: null pointer");
  KRQ_REQUIRE(N > 0 && N % 128 == 0,
              "gemv_swiglu_fp8_cast: N=%lld: the activation width N/2 must be a multiple of 64", (long long)N);
  return gemv_fp8_run(x, x_kind, x_scale, x_inv, x_per_row, w8, w_layout, w_scale, w_per_row, M, N, K, 1,
                      KRQ_OUT_SWIGLU, 0, x8_tiled, const_cast<float*>(out_inv), stream);
}

// The chained FP8 MLP at M = 1 (k_mlp_chain_fp8): act = SwiGLU(x . Wgu^T) and the split-K partials
// of act . Wd^T in one launch, the down blocks streaming their weights before act is complete.
extern "C" int krq_mlp_chain_fp8(const void* x, const void* w_gu, const float* gu_scale, int gu_per_row,
                                 const void* w_down, const float* down_scale, int down_per_row, int64_t H, int64_t I,
                                 int split, void* act, uint32_t* ctl, uint32_t max_polls, void* out, void* stream) {
  KRQ_REQUIRE(x && w_gu && gu_scale && w_down && down_scale && act && ctl && out, "mlp_chain_fp8: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w_gu) && aligned16(w_down) && aligned16(act),
              "mlp_chain_fp8: x, weights and act must be 16-byte aligned");
  KRQ_REQUIRE(H > 0 && I > 0 && H % 64 == 0 && I % 64 == 0 && split >= 1 && I % split == 0 && (I / split) % 64 == 0,
              "mlp_chain_fp8: shape H=%lld I=%lld split=%d (H, I and I/split multiples of 64)", (long long)H,
              (long long)I, split);
  KRQ_REQUIRE(H <= 512 * kAwLarge && I <= 512 * kAwLarge, "mlp_chain_fp8: rows longer than %d elements",
              512 * kAwLarge);
  KRQ_REQUIRE(max_polls > 0, "mlp_chain_fp8: max_polls must be positive");
  const int awg = aw_chunks(H), awd = aw_chunks(I);
  // gate_up: the SwiGLU launch's plan (two-matrix blocks, the last ones as half-pair blocks)
  const int64_t nrbs = I / 16, rem = nrbs % kCUs;
  const bool mixed = nrbs > 2 * kCUs && rem != 0 && 2 * rem <= kCUs;
  const int64_t nfull = mixed ? nrbs - rem : nrbs, n_first = mixed ? nfull + 2 * rem : nrbs;
  const int64_t nrb2 = H / 16, n_second = nrb2 * split;
  KRQ_REQUIRE(n_first + n_second <= 0x7fffffff, "mlp_chain_fp8: grid too large");
  // down: two weight waves of kDeepU slots, every step of the split in flight before the wait for
  // act. (The standalone down GEMV's single wave of kBigU slots would take the chained kernel to
  // 256 VGPRs, two waves per SIMD, and two resident blocks per CU instead of four.) The partial
  // sums are those of two waves, so they differ from the standalone GEMV's in fp32 rounding only.
  constexpr int NWG = 2, NWD = 2;
  const int kts_g = static_cast<int>(H / 64), kts_d = static_cast<int>(I / split / 64);
  KRQ_REQUIRE((kts_d + 1) / 2 <= NWD * kDeepU,
              "mlp_chain_fp8: down's split of I/split=%lld elements exceeds the ring (at most %d steps of 128)",
              (long long)(I / split), NWD * kDeepU);
  // LDS: the larger stage's partial sums and quantized slice
  const size_t smem = std::max((size_t)NWG * 2 * 256 * sizeof(float) + (size_t)H,
                               (size_t)NWD * 256 * sizeof(float) + (size_t)(I / split));
  FusedArgs fa{};
  fa.cnt = ctl;
  fa.max_polls = max_polls;
  fa.n_first = static_cast<int>(n_first);
  fa.n_second = static_cast<int>(n_second);
  const dim3 grid(static_cast<unsigned>(n_first + n_second)), block((NWG + 1) * 64);
  hipStream_t s = (hipStream_t)stream;
#define KRQ_CHAIN(AG, AD)                                                                                            \
  hipLaunchKernelGGL((k_mlp_chain_fp8<kSwiU, AG, kDeepU, AD, NWG, NWD>), grid, block, smem, s, (const uint8_t*)x,    \
                     (const uint8_t*)w_gu, gu_scale, gu_per_row, (const uint8_t*)w_down, down_scale, down_per_row, I, H, \
                     kts_g, kts_d, static_cast<int>(nfull), static_cast<int>(nrb2), (uint16_t*)act, (float*)out, fa)
#define KRQ_CHAIN_D(AG)                     \
  if (awd == kAwRow) KRQ_CHAIN(AG, kAwRow); \
  else if (awd == kAwSmall) KRQ_CHAIN(AG, kAwSmall); \
  else KRQ_CHAIN(AG, kAwLarge);
  if (awg == kAwRow) {
    KRQ_CHAIN_D(kAwRow)
  } else if (awg == kAwSmall) {
    KRQ_CHAIN_D(kAwSmall)
  } else {
    KRQ_CHAIN_D(kAwLarge)
  }
#undef KRQ_CHAIN_D
#undef KRQ_CHAIN
  return krq_check_launch("mlp_chain_fp8");
}

extern "C" int64_t krq_mlp_chain_ctl_words(void) { return kChainWords; }

#ifdef KRQ_TIMELINE
// Timeline build only: copy the stamps of this file's GEMV kernels (8 slots per block, block
// index blockIdx.y * gridDim.x + blockIdx.x) to host memory; the stamp clock's rate in kHz.
extern "C" int krq_timeline_read(void* dst, int64_t bytes) {
  if (bytes < 0 || bytes > (int64_t)sizeof(krq_timeline)) return KRQ_EINVAL;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(krq_timeline), (size_t)bytes, 0, hipMemcpyDeviceToHost) == hipSuccess
             ? KRQ_OK
             : KRQ_EHIP;
}
extern "C" int krq_timeline_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return 0;
  return khz;
}
#endif
