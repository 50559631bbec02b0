// BF16 decode GEMVs with the residual add and RMSNorm folded in, so a decoder layer is four GEMV
// launches plus attention (reference engine/kernels/fused_gemv.py:1-17, :48-167; engine/engine.py
// :940-962). Same rounding points as the reference:
//   NORM prologue   rstd[m] = rsqrt(ss[m] / K + eps); h = bf16(bf16(x * rstd) * w_ln)
//   residual        y = bf16(sum of the split partials, in split order);
//   epilogue        x_new = bf16(res_in + y) -> res_out;  ss_out[m] += x_new^2 over the columns
//
// MI355X form of the sum of squares. Device-scope atomics on one address serialize (~12 ns each),
// so instead of one accumulator per row that every 16-column tile adds into, each tile writes its
// own partial: ss is [M][T] (T = N / 16 tiles of the producer = K / 16 of the consumer). The
// consumer's prologue sums a row's T partials in a fixed order (deterministic; the reference's
// atomic order is not). Every producer overwrites all T slots, so nothing needs zeroing. At M = 1
// the consumer sums its row itself instead (gemv_common.h, sumsq8) and reads no ss_in.
//
// Split-K with the residual epilogue: each split writes its partial tile with write-through
// (agent-scope) stores, waits for them, then bumps the tile's counter; the split that brings it to
// S sums the S partials in split order and finishes the tile, then zeroes the counter for the next
// launch. Counters are per tile (distinct addresses), so at most S atomics meet on one address.
//
// With the RMSNorm the prologue stages the block's K slice of x, normalized, in LDS once, and the
// main loop reads its matrix-core / vector-ALU operands from there; without it the operands come
// from global memory with the weights, as in gemv_bf16.hip. Loads of the prologue and of the weight
// ring are issued unconditionally at clamped addresses (see gemv_fp8.hip).
#include "gemv_common.h"

#include <stdlib.h>

using namespace krq;

namespace {

constexpr int kXC = 8;           // 16-byte x chunks per thread in the prologue
constexpr int kSC = 8;           // sum-of-squares partials per thread in the prologue
constexpr int kMaxNT = 512;

template <int MT, int MODE, int LAYOUT, int ALGO, int U, bool NORM>
__global__ __launch_bounds__(kMaxNT) void k_gemv_fused(const uint8_t* __restrict__ x,
                                                       const uint8_t* __restrict__ w, int M, int64_t NO,
                                                       int64_t K, int kts, void* __restrict__ out,
                                                       FusedArgs fa) {
  extern __shared__ __align__(16) float red[];  // nw*P*MT*256 floats | (NORM) x slice bf16 [M][ks], ss [M][T]
  __shared__ float rstd_s[32], ones[32];
  __shared__ uint32_t last_s;
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  const int NT = blockDim.x, nw = NT >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t rb = blockIdx.x, rbu = rb + (NO >> 4);
  const int sidx = blockIdx.y, S = gridDim.y;
  const int nsteps = (kts + 1) >> 1;
  const int64_t tbase = (int64_t)sidx * kts;
  const int64_t rowb = 2 * K;
  const int ks = kts * 32;  // bf16 elements of this split
  const int64_t k0 = (int64_t)sidx * ks;
  const int cpr = ks >> 3;  // 16-byte chunks per row of the slice
  const int T = (int)(K >> 4);
  const int jcount = wave < nsteps ? (nsteps - wave + nw - 1) / nw : 0;
  uint8_t* hq = reinterpret_cast<uint8_t*>(red + nw * P * MT * 256);
  float* sst = reinterpret_cast<float*>(hq + (size_t)M * ks * 2);
  if (threadIdx.x < 32) ones[threadIdx.x] = 1.0f;
  // ROWSUM (the one-row kernel, M == 1): the prologue loads the whole row and sums it itself
  constexpr bool ROWSUM = NORM && ALGO == 2;
  const int nch = (int)(K >> 3);  // 16-byte chunks of a row

  // ---- prologue part 1 (RMSNorm): x slice (ROWSUM: the row) and norm inputs ahead of the weights ----
  uint4 xv[kXC], lv[kXC];
  float sv[kSC];
  if (ROWSUM) {
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int64_t e = 8 * (int64_t)min((int)threadIdx.x + c * NT, nch - 1);
      xv[c] = ld16(x + 2 * e);
      lv[c] = ld16(reinterpret_cast<const uint8_t*>(fa.ln) + 2 * e);
    }
  } else if (NORM) {
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int idx = min((int)threadIdx.x + c * NT, M * cpr - 1);
      const int m = idx / cpr, ch = idx - m * cpr;
      xv[c] = ld16(x + 2 * ((int64_t)m * K + k0 + 8 * ch));
      lv[c] = ld16(reinterpret_cast<const uint8_t*>(fa.ln) + 2 * (k0 + 8 * ch));
    }
#pragma unroll
    for (int c = 0; c < kSC; ++c) sv[c] = fa.ss_in[min((int)threadIdx.x + c * NT, M * T - 1)];
  }

  // ---- weight ring (a slot past a wave's last step reloads that step, masked where consumed) ----
  v4f acc[MT], accu[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    accu[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  float s0 = 0.f, s1 = 0.f, q0 = 0.f, q1 = 0.f;
  uint4 wl[U], wh[U], ul[U], uh[U], xl[U][MT], xh[U][MT];
  auto load_slot = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const int64_t t0 = tbase + 2 * j;
    const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
    wl[u] = ld16nt(w_addr<LAYOUT>(w, rb, t0, rowb, lane));
    wh[u] = ld16nt(w_addr<LAYOUT>(w, rb, t1, rowb, lane));
    if (P == 2) {
      ul[u] = ld16nt(w_addr<LAYOUT>(w, rbu, t0, rowb, lane));
      uh[u] = ld16nt(w_addr<LAYOUT>(w, rbu, t1, rowb, lane));
    }
    if (!NORM) {  // operands straight from x (rows m >= M read row M - 1; never written out)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
        const uint8_t* xr = x + (int64_t)m * rowb + g * 16;
        xl[u][mt] = ld16(xr + t0 * 64);
        xh[u][mt] = ld16(xr + t1 * 64);
      }
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) load_slot(u, u);
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue part 2: per-row rstd (NORM), then the (normalized) slice into LDS ----
  if (ROWSUM) {  // the row's chunk sums, then the canonical sum over them
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int i = threadIdx.x + c * NT;
      if (i < nch) sst[i] = sumsq8(xv[c]);
    }
    __syncthreads();
    row_rstd(sst, 1, nch, K, fa.eps, rstd_s);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int64_t e = 8 * (int64_t)(threadIdx.x + c * NT);
      if (e >= k0 && e < k0 + ks) *reinterpret_cast<uint4*>(hq + 2 * (e - k0)) = norm8(xv[c], lv[c], rstd_s[0]);
    }
    __syncthreads();
  } else if (NORM) {
#pragma unroll
    for (int c = 0; c < kSC; ++c) {
      const int i = threadIdx.x + c * NT;
      if (i < M * T) sst[i] = sv[c];
    }
    __syncthreads();
    row_rstd(sst, M, T, K, fa.eps, rstd_s);
    __syncthreads();
  }
  if (NORM && !ROWSUM) {
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int idx = threadIdx.x + c * NT;
      if (idx < M * cpr) {
        const int m = idx / cpr, ch = idx - m * cpr;
        *reinterpret_cast<uint4*>(hq + 2 * ((int64_t)m * ks + 8 * ch)) = norm8(xv[c], lv[c], rstd_s[m]);
      }
    }
    __syncthreads();
  }

  // ---- main loop: operands from the staged slice ----
  auto consume_slot = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const bool ok = cc < jcount, hi = ok && (2 * j + 1 < kts);
    const uint4 bl = sel4(ok, wl[u]), bh = sel4(hi, wh[u]);
    uint4 al[MT], ah[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (NORM) {
        const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
        const uint8_t* hr = hq + 2 * ((int64_t)m * ks + 8 * g);
        al[mt] = *reinterpret_cast<const uint4*>(hr + (2 * j) * 64);
        ah[mt] = sel4(2 * j + 1 < kts, *reinterpret_cast<const uint4*>(hr + min(2 * j + 1, kts - 1) * 64));
      } else {
        al[mt] = xl[u][mt];
        ah[mt] = xh[u][mt];
      }
    }
    if (ALGO == 2) {
      s0 = dot8_bf16(bl, al[0], s0);
      s1 = dot8_bf16(bh, ah[0], s1);
      if (P == 2) {
        q0 = dot8_bf16(sel4(ok, ul[u]), al[0], q0);
        q1 = dot8_bf16(sel4(hi, uh[u]), ah[0], q1);
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(al[mt]), as_v8bf(bl), acc[mt], 0, 0, 0);
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(ah[mt]), as_v8bf(bh), acc[mt], 0, 0, 0);
      }
      if (P == 2) {
        const uint4 cl = sel4(ok, ul[u]), ch = sel4(hi, uh[u]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(al[mt]), as_v8bf(cl), accu[mt], 0, 0, 0);
          accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(ah[mt]), as_v8bf(ch), accu[mt], 0, 0, 0);
        }
      }
    }
  };
  int base = 0;
  for (; base + U < jcount; base += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      consume_slot(u, base + u);
      load_slot(u, base + u + U);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) consume_slot(u, base + u);
  if (ALGO == 2) {
    float a = s0 + s1, au = q0 + q1;
    a += __shfl_xor(a, 16, kWave);
    a += __shfl_xor(a, 32, kWave);
    au += __shfl_xor(au, 16, kWave);
    au += __shfl_xor(au, 32, kWave);
    acc[0] = v4f{g == 0 ? a : 0.f, 0.f, 0.f, 0.f};
    accu[0] = v4f{g == 0 ? au : 0.f, 0.f, 0.f, 0.f};
  }
  stash<MT, P>(red, wave, lane, acc, accu);
  __syncthreads();
  if constexpr (MODE != kOutResidual) {
    epilogue<MT, MODE, P>(red, 0, nw, M, NO, rb, sidx, ones, ColScales{1.0f, 1.0f}, out, nullptr);
    return;
  }

  residual_epilogue<MT>(red, nw, M, NO, rb, sidx, S, ones, 1.0f, reinterpret_cast<float*>(out), fa, &last_s);
}

// RMSNorm of whole rows for shapes whose slice does not fit the GEMV's LDS staging:
// h = bf16(bf16(x * rstd) * w_ln), rstd from the [M][K/16] sum-of-squares partials (ROWSUM, one
// row: from the row itself).
template <int C, bool ROWSUM>
__global__ __launch_bounds__(kRowThreads) void k_rmsnorm_rows(const uint16_t* __restrict__ x,
                                                              const float* __restrict__ ss_in,
                                                              const uint16_t* __restrict__ ln, float eps, int64_t K,
                                                              uint16_t* __restrict__ h) {
  __shared__ float sst[kRowThreads * C];
  __shared__ float rstd_sh;
  const int m = blockIdx.x;
  uint4 xv[C], lv[C];
  const float rstd = row_prologue<C, ROWSUM>(x, ss_in, ln, eps, K, m, sst, &rstd_sh, xv, lv);
  uint8_t* hr = reinterpret_cast<uint8_t*>(h + m * K);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = 8 * (int64_t)(threadIdx.x + c * kRowThreads);
    if (e < K) *reinterpret_cast<uint4*>(hr + 2 * e) = norm8(xv[c], lv[c], rstd);
  }
}

template <int MODE, int LAYOUT, bool NORM>
void launch(int M, dim3 grid, int nw, size_t smem, hipStream_t s, const uint8_t* x, const uint8_t* w,
            int m, int64_t NO, int64_t K, int kts, void* out, const FusedArgs& fa) {
  const dim3 block(nw * 64);
  if (M == 1)
    hipLaunchKernelGGL((k_gemv_fused<1, MODE, LAYOUT, 2, 4, NORM>), grid, block, smem, s, x, w, m, NO, K, kts, out, fa);
  else if (M <= 4)
    hipLaunchKernelGGL((k_gemv_fused<1, MODE, LAYOUT, 1, 4, NORM>), grid, block, smem, s, x, w, m, NO, K, kts, out, fa);
  else if (M <= 16)
    hipLaunchKernelGGL((k_gemv_fused<1, MODE, LAYOUT, 1, 2, NORM>), grid, block, smem, s, x, w, m, NO, K, kts, out, fa);
  else
    hipLaunchKernelGGL((k_gemv_fused<2, MODE, LAYOUT, 1, 2, NORM>), grid, block, smem, s, x, w, m, NO, K, kts, out, fa);
}

template <int MODE, bool NORM>
void launch_layout(int layout, int M, dim3 grid, int nw, size_t smem, hipStream_t s, const uint8_t* x,
                   const uint8_t* w, int m, int64_t NO, int64_t K, int kts, void* out, const FusedArgs& fa) {
  if (layout == KRQ_W_TILED)
    launch<MODE, KRQ_W_TILED, NORM>(M, grid, nw, smem, s, x, w, m, NO, K, kts, out, fa);
  else
    launch<MODE, KRQ_W_ROWMAJOR, NORM>(M, grid, nw, smem, s, x, w, m, NO, K, kts, out, fa);
}

constexpr size_t kMaxSmem = 60 * 1024;
// Largest bf16 x slice (bytes) a block normalizes in its prologue. Measured on MI355X: at M = 16
// the QKV slice (40 KB) takes 19.0 us in-kernel against 2.6 + 8.4 us for krq_rmsnorm_rows and the
// plain launch; the M = 4 gate/up slice (20 KB) is faster in-kernel (21.4 against 22.0 us).
constexpr int64_t kNormStageMax = 24 * 1024;

// Waves and LDS bytes of a launch; false if the slice (or the sum-of-squares partials) does not fit.
bool plan_fused(int64_t M, int64_t N, int64_t K, int split, int mode, bool norm, int* nw_out, size_t* smem_out) {
  if (M < 1 || M > 32 || split < 1 || K % 16 || K % split || (K / split) % 32) return false;
  const int64_t ks = K / split;
  if (norm && M * ks * 2 > kNormStageMax) return false;
  const int kts = static_cast<int>(ks / 32);
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : 1;
  const int MT = M <= 16 ? 1 : 2;
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  int nw = plan_waves((kts + 1) / 2, P, M <= 4 ? 4 : 2, NO / 16 * split);
  // (one row: the prologue loads and sums the whole row, K / 8 chunks, instead of the partials)
  auto short_of = [&](int w) {
    if (norm && M == 1) return (int64_t)w * 64 * kXC < K / 8;
    return norm && ((int64_t)w * 64 * kXC < M * (ks / 8) || (int64_t)w * 64 * kSC < M * (K / 16));
  };
  while (short_of(nw) && nw < kMaxNT / 64) ++nw;
  if (short_of(nw)) return false;
  const size_t smem = (size_t)nw * P * MT * 256 * sizeof(float) +
                      (norm ? (size_t)M * ks * 2 + (size_t)(M == 1 ? K / 8 : M * (K / 16)) * sizeof(float) : 0);
  if (smem > kMaxSmem) return false;
  *nw_out = nw;
  *smem_out = smem;
  return true;
}

}  // namespace

extern "C" int64_t krq_gemv_fused_fits(int64_t M, int64_t N, int64_t K, int split, int mode, int norm) {
  int nw = 0;
  size_t smem = 0;
  return plan_fused(M, N, K, split, mode, norm != 0, &nw, &smem) ? 1 : 0;
}

extern "C" int krq_gemv_bf16_fused(const void* x, const void* w, int w_layout, int64_t M, int64_t N,
                                   int64_t K, int split, int mode, const void* ln, const float* ss_in,
                                   float eps, const void* res_in, void* res_out, float* ss_out,
                                   uint32_t* cnt, void* out, void* stream) {
  KRQ_REQUIRE(x && w, "gemv_bf16_fused: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w), "gemv_bf16_fused: x and w must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_bf16_fused: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(mode == KRQ_OUT_BF16 || mode == KRQ_OUT_PARTIAL || mode == KRQ_OUT_SWIGLU || mode == kOutResidual,
              "gemv_bf16_fused: bad mode %d", mode);
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "gemv_bf16_fused: bad layout %d", w_layout);
  KRQ_REQUIRE(N > 0 && K > 0 && K % 16 == 0 && split >= 1 && split <= 64 && K % split == 0 && (K / split) % 32 == 0,
              "gemv_bf16_fused: no tiling divides K_SPLIT (K=%lld split=%d)", (long long)K, split);
  KRQ_REQUIRE(mode == KRQ_OUT_PARTIAL || mode == kOutResidual || split == 1,
              "gemv_bf16_fused: split %d needs the partials or residual output", split);
  const bool norm = ln != nullptr;
  KRQ_REQUIRE(!norm || (ss_in && aligned16(ln)), "gemv_bf16_fused: RMSNorm needs ss_in and an aligned ln");
  KRQ_REQUIRE(mode != kOutResidual || (res_in && res_out && ss_out && (split == 1 || (cnt && out))),
              "gemv_bf16_fused: the residual epilogue needs res_in, res_out, ss_out and, for split > 1, "
              "cnt and the partials buffer");
  KRQ_REQUIRE(mode == kOutResidual || out, "gemv_bf16_fused: null output");
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  KRQ_REQUIRE(NO % 16 == 0 && (mode != KRQ_OUT_SWIGLU || N % 2 == 0),
              "gemv_bf16_fused: no tiling divides N=%lld", (long long)N);
  int nw = 0;
  size_t smem = 0;
  KRQ_REQUIRE(plan_fused(M, N, K, split, mode, norm, &nw, &smem),
              "gemv_bf16_fused: M=%lld x K/split=%lld does not fit the staged slice; normalize rows first "
              "(krq_rmsnorm_rows) and call the plain GEMV", (long long)M, (long long)(K / split));
  const int kts = static_cast<int>(K / split / 32);
  const dim3 grid(static_cast<unsigned>(NO / 16), static_cast<unsigned>(split));
  FusedArgs fa{reinterpret_cast<const uint16_t*>(ln), ss_in, eps, reinterpret_cast<const uint16_t*>(res_in),
               reinterpret_cast<uint16_t*>(res_out), ss_out, cnt};
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w;
  const int m = static_cast<int>(M);
  hipStream_t s = (hipStream_t)stream;
#define KRQ_FUSED_CASE(MODE)                                                                                     \
  do {                                                                                                         \
    if (norm) launch_layout<MODE, true>(w_layout, m, grid, nw, smem, s, xb, wb, m, NO, K, kts, out, fa);       \
    else launch_layout<MODE, false>(w_layout, m, grid, nw, smem, s, xb, wb, m, NO, K, kts, out, fa);           \
  } while (0)
  if (mode == KRQ_OUT_BF16) KRQ_FUSED_CASE(KRQ_OUT_BF16);
  else if (mode == KRQ_OUT_PARTIAL) KRQ_FUSED_CASE(KRQ_OUT_PARTIAL);
  else if (mode == KRQ_OUT_SWIGLU) KRQ_FUSED_CASE(KRQ_OUT_SWIGLU);
  else KRQ_FUSED_CASE(kOutResidual);
#undef KRQ_FUSED_CASE
  return krq_check_launch("gemv_bf16_fused");
}

extern "C" int krq_rmsnorm_rows(const void* x, const float* ss_in, const void* ln, float eps, int64_t M,
                                int64_t K, void* h, void* stream) {
  KRQ_REQUIRE(x && ss_in && ln && h, "rmsnorm_rows: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(ln) && aligned16(h), "rmsnorm_rows: x, ln and h must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 0x7fffffff && K > 0 && K % 16 == 0 && K <= kRowMaxK,
              "rmsnorm_rows: bad shape M=%lld K=%lld (K a multiple of 16, at most %d)", (long long)M, (long long)K,
              kRowMaxK);
  // (one row: its sum of squares from the row itself, as every one-row normalizing kernel takes it)
  auto kern = M == 1 ? (K <= kRowSmallK ? k_rmsnorm_rows<2, true> : k_rmsnorm_rows<kRowChunks, true>)
                     : (K <= kRowSmallK ? k_rmsnorm_rows<2, false> : k_rmsnorm_rows<kRowChunks, false>);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(M)), dim3(kRowThreads), 0, (hipStream_t)stream,
                     (const uint16_t*)x, ss_in, (const uint16_t*)ln, eps, K, (uint16_t*)h);
  return krq_check_launch("rmsnorm_rows");
}
