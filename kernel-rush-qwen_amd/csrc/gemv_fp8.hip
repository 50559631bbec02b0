// FP8 skinny GEMM / GEMV (M <= 32): y = (x8 . w8^T) * x_scale[m] * w_scale[n], fp32 accumulate.
// Layout, step and epilogue conventions: gemv_common.h.
//
// Activation kinds (template XK):
//   KRQ_X_FP8          x is e4m3 [M, K] with its scale; matrix-core A operands are loaded from
//                      global memory by the lanes whose row m < M.
//   KRQ_X_BF16_DYN     x is bf16 [1, K]; the block computes the per-token scale itself
//                      (amax over all of K, ActScale arithmetic), quantizes its K slice into LDS.
//   KRQ_X_BF16_STATIC  x is bf16 [M, K] with a given inverse scale (SharedScale / ActScale
//                      inv, per tensor or per row); the block quantizes its K slice into LDS.
// The activation loads of the fused kinds are issued before the first weight batch, so their
// latency (L2 hits) overlaps the weight stream's; quantization uses the hardware e4m3 convert
// after the reference's clamp, which is bit-identical to the software encoder.
#include "gemv_common.h"

#include <stdlib.h>

using namespace krq;

namespace krq {
int plan_waves(int nsteps, int P, int U) {
  static const int env = [] {
    const char* s = getenv("KRQ_GEMV_WAVES");
    return s ? atoi(s) : 0;
  }();
  if (env >= 1 && env <= 8) return env;
  if (nsteps < 2) return 1;
  // measured on MI355X at the Qwen3-4B shapes: a single-matrix block takes just enough waves for
  // all of its steps to be in flight at once (one memory round trip), up to 4; past that, and for
  // the two-matrix SwiGLU block, two waves
  const int w = (nsteps + U - 1) / U;
  return (P == 1 && w <= 4) ? w : 2;
}
}  // namespace krq

namespace {

// 16-byte activation chunks per thread in the fused prologues: every chunk load is issued (see
// the kernel), so the one-row prologue, which reads the whole row for its amax, keeps the count
// small and takes more waves for long rows instead
constexpr int kXChunks = 8;
constexpr int kXChunksDyn = 4;
constexpr int kMaxThreads = 512;

// PB = 2 (MFMA kernels, modes other than SwiGLU): the block owns two adjacent row blocks, so each
// activation load feeds two matrix-core products (at M > 1 the activation slices are as large as
// the weight steps, and every row block re-reads them).
template <int MT, int MODE, int LAYOUT, int XK, int ALGO, int U, int PB>
__global__ __launch_bounds__(kMaxThreads) void k_gemv_fp8(
    const uint8_t* __restrict__ x, const float* __restrict__ xsc, const float* __restrict__ xinv,
    int x_per_row, const uint8_t* __restrict__ w8, const float* __restrict__ wsc, int w_per_row,
    int M, int64_t NO, int64_t K, int kts, void* __restrict__ out, void* __restrict__ aux) {
  extern __shared__ float red[];  // nw*P*MT*256 partial sums, then the e4m3 activation slice
  __shared__ float xs_l[32];
  __shared__ float amax_w[kMaxThreads / 64];
  static_assert(PB == 1 || (MODE != KRQ_OUT_SWIGLU && ALGO != 2), "paired row blocks: MFMA, no SwiGLU");
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : PB;  // weight row blocks streamed per step
  constexpr bool FUSED = XK != KRQ_X_FP8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t rb = (int64_t)blockIdx.x * PB, rbu = MODE == KRQ_OUT_SWIGLU ? rb + (NO >> 4) : rb + 1;
  const int sidx = blockIdx.y;
  const int nsteps = (kts + 1) >> 1;
  const int64_t tbase = (int64_t)sidx * kts;
  const int64_t k0 = tbase * 64;  // first K element of this split
  const int ks = kts * 64;        // K elements of this split
  uint8_t* xq = reinterpret_cast<uint8_t*>(red + nw * P * MT * 256);
  const int jcount = wave < nsteps ? (nsteps - wave + nw - 1) / nw : 0;
  const ColScales cs = load_col_scales<MODE, PB>(wsc, w_per_row, NO, rb);

  // ---- fused activation prologue, part 1: activation loads ahead of the weight stream ----
  // Every load of the prologue and of the step ring is issued unconditionally, at a clamped (valid)
  // address where it is not needed: a branch around a load makes the compiler's wait counts
  // conservative (a full drain, vmcnt(0)) at the join, which serializes the weight stream.
  uint4 xv[kXChunks];
  if (XK == KRQ_X_BF16_DYN) {
#pragma unroll
    for (int c = 0; c < kXChunksDyn; ++c) {
      const int64_t e = 8 * (int64_t)(threadIdx.x + c * blockDim.x);
      xv[c] = ld16(x + 2 * min(e, K - 8));  // chunks past K repeat the last one (same amax)
    }
  } else if (XK == KRQ_X_BF16_STATIC) {
    const int cpr = ks >> 3;  // chunks per row of the slice
#pragma unroll
    for (int c = 0; c < kXChunks; ++c) {
      const int idx = threadIdx.x + c * blockDim.x, m = idx / cpr;
      xv[c] = ld16(x + 2 * ((int64_t)min(m, M - 1) * K + k0 + 8 * (idx - m * cpr)));
    }
  }

  // scale of this thread's activation row, read now so its latency hides under the weight stream
  // (every thread loads and stores it, threads t and t + 32 the same value, so the load is not
  // sunk into a branch after the weight loads)
  const int xrow = min((int)(threadIdx.x & 31), M - 1);
  const float xs_reg = XK != KRQ_X_BF16_DYN ? xsc[x_per_row ? xrow : 0] : 1.0f;

  // ---- weight (and, for e4m3 activations, A operand) loads: a ring of U step slots ----
  uint4 wl[U], wh[U], ul[U], uh[U], xl[U][MT], xh[U][MT];
  // A slot past this wave's last step reloads that step (an address already in flight or cached,
  // so no extra HBM traffic) and is masked where consumed. Rows m >= M read row M - 1: their
  // products land in accumulator rows the epilogue never writes.
  auto load_slot = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const int64_t t0 = tbase + 2 * j;
    const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
    wl[u] = ld16nt(w_addr<LAYOUT>(w8, rb, t0, K, lane));
    wh[u] = ld16nt(w_addr<LAYOUT>(w8, rb, t1, K, lane));
    if (P == 2) {
      ul[u] = ld16nt(w_addr<LAYOUT>(w8, rbu, t0, K, lane));
      uh[u] = ld16nt(w_addr<LAYOUT>(w8, rbu, t1, K, lane));
    }
    if (!FUSED) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
        const uint8_t* xr = x + (int64_t)m * K + g * 16;
        xl[u][mt] = ld16(xr + t0 * 64);
        xh[u][mt] = ld16(xr + t1 * 64);
      }
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) load_slot(u, u);
  __builtin_amdgcn_sched_barrier(0);

  // ---- fused activation prologue, part 2: scale, quantize the slice into LDS ----
  if (XK == KRQ_X_FP8) {
    xs_l[threadIdx.x & 31] = xs_reg;
  } else if (XK == KRQ_X_BF16_DYN) {
    float am = 0.0f;
#pragma unroll
    for (int c = 0; c < kXChunksDyn; ++c) am = absmax8(xv[c], am);
    am = wave_max(am);
    if (lane == 0) amax_w[wave] = am;
    __syncthreads();
    float a = amax_w[0];
    for (int w = 1; w < nw; ++w) a = fmaxf(a, amax_w[w]);
    a = fmaxf(a, 1e-6f);
    const float inv = inv_from_amax(a);
    if (threadIdx.x == 0) xs_l[0] = scale_from_amax(a);
#pragma unroll
    for (int c = 0; c < kXChunksDyn; ++c) {
      const int64_t e = 8 * (int64_t)(threadIdx.x + c * blockDim.x);
      if (e >= k0 && e < k0 + ks) *reinterpret_cast<uint2*>(xq + (e - k0)) = quant8(xv[c], inv);
    }
  } else {
    const int cpr = ks >> 3;
#pragma unroll
    for (int c = 0; c < kXChunks; ++c) {
      const int idx = threadIdx.x + c * blockDim.x, m = idx / cpr;
      if (m < M)
        *reinterpret_cast<uint2*>(xq + (int64_t)m * ks + 8 * (idx - m * cpr)) =
            quant8(xv[c], xinv[x_per_row ? m : 0]);
    }
    xs_l[threadIdx.x & 31] = xs_reg;
  }
  if (FUSED) __syncthreads();

  // ---- main loop: consume slot u (step cc), then refill it with step cc + U ----
  v4f acc[MT], accu[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    accu[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  float s0 = 0.f, s1 = 0.f, q0 = 0.f, q1 = 0.f;  // vector-ALU partial sums
  auto consume_slot = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const bool ok = cc < jcount, hi = ok && (2 * j + 1 < kts);
    if (FUSED) {
      // the quantized slice ends at ks: the high tile of an odd last step is zero (not stale LDS)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
        const uint8_t* xr = xq + (int64_t)m * ks + g * 16;
        xl[u][mt] = *reinterpret_cast<const uint4*>(xr + (2 * j) * 64);
        xh[u][mt] = sel4(2 * j + 1 < kts, *reinterpret_cast<const uint4*>(xr + min(2 * j + 1, kts - 1) * 64));
      }
    }
    const uint4 bl = sel4(ok, wl[u]), bh = sel4(hi, wh[u]);
    if (ALGO == 2) {
      s0 = dot16_fp8(bl, xl[u][0], s0);
      s1 = dot16_fp8(bh, xh[u][0], s1);
      if (P == 2) {
        q0 = dot16_fp8(sel4(ok, ul[u]), xl[u][0], q0);
        q1 = dot16_fp8(sel4(hi, uh[u]), xh[u][0], q1);
      }
    } else {
      const v8i B = pack_v8i(bl, bh);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const v8i A = pack_v8i(xl[u][mt], xh[u][mt]);
        acc[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[mt], 0, 0, 0, 0, 0, 0);
      }
      if (P == 2) {
        const v8i Bu = pack_v8i(sel4(ok, ul[u]), sel4(hi, uh[u]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const v8i A = pack_v8i(xl[u][mt], xh[u][mt]);
          accu[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, Bu, accu[mt], 0, 0, 0, 0, 0, 0);
        }
      }
    }
  };
  // the last batch is peeled off (consume only), so no load sits behind a branch and the first
  // batch's loads stay ahead of everything else
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
    // the four lanes of row r (g = 0..3) hold partial sums of disjoint k: add them; lanes 0..15
    // then carry columns 16*rb + lane in MFMA slot (mt 0, i 0), i.e. output row m = 0
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
  epilogue<MT, MODE, P>(red, 0, nw, M, NO, rb, sidx, xs_l, cs, out, aux);
  if (PB == 2) epilogue<MT, MODE, P>(red, 1, nw, M, NO, rbu, sidx, xs_l, ColScales{cs.u, 1.0f}, out, aux);
}

#define KRQ_GEMV_ARGS xb, x_scale, x_inv, x_per_row, wb, w_scale, w_per_row, m, NO, K, kts, out, aux

template <int MODE, int LAYOUT, int XK>
int launch(int algo, int pb, int M, dim3 grid, int nw, size_t smem, hipStream_t s, const uint8_t* xb,
           const float* x_scale, const float* x_inv, int x_per_row, const uint8_t* wb,
           const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K, int kts, void* out,
           void* aux) {
  const dim3 block(nw * 64);
  constexpr int PB2 = MODE == KRQ_OUT_SWIGLU ? 1 : 2;  // no paired variant of the SwiGLU kernel
  if (algo == 2)
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 2, 4, 1>), grid, block, smem, s, KRQ_GEMV_ARGS);
  else if (M <= 4)
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, 4, 1>), grid, block, smem, s, KRQ_GEMV_ARGS);
  else if (M <= 16 && pb == 2)
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, 2, PB2>), grid, block, smem, s, KRQ_GEMV_ARGS);
  else if (M <= 16)
    hipLaunchKernelGGL((k_gemv_fp8<1, MODE, LAYOUT, XK, 1, 2, 1>), grid, block, smem, s, KRQ_GEMV_ARGS);
  else if (pb == 2)
    hipLaunchKernelGGL((k_gemv_fp8<2, MODE, LAYOUT, XK, 1, 2, PB2>), grid, block, smem, s, KRQ_GEMV_ARGS);
  else
    hipLaunchKernelGGL((k_gemv_fp8<2, MODE, LAYOUT, XK, 1, 2, 1>), grid, block, smem, s, KRQ_GEMV_ARGS);
  return 0;
}

template <int MODE, int LAYOUT>
void launch_xk(int xk, int algo, int pb, int M, dim3 grid, int nw, size_t smem, hipStream_t s,
               const uint8_t* xb, const float* x_scale, const float* x_inv, int x_per_row,
               const uint8_t* wb, const float* w_scale, int w_per_row, int m, int64_t NO,
               int64_t K, int kts, void* out, void* aux) {
  if (xk == KRQ_X_FP8)
    launch<MODE, LAYOUT, KRQ_X_FP8>(algo, pb, M, grid, nw, smem, s, KRQ_GEMV_ARGS);
  else if (xk == KRQ_X_BF16_DYN)
    launch<MODE, LAYOUT, KRQ_X_BF16_DYN>(algo, pb, M, grid, nw, smem, s, KRQ_GEMV_ARGS);
  else
    launch<MODE, LAYOUT, KRQ_X_BF16_STATIC>(algo, pb, M, grid, nw, smem, s, KRQ_GEMV_ARGS);
}

}  // namespace

int krq::gemv_fp8_run(const void* x, int x_kind, const float* x_scale, const float* x_inv,
                      int x_per_row, const void* w8, int w_layout, const float* w_scale,
                      int w_per_row, int64_t M, int64_t N, int64_t K, int split, int mode,
                      int algo, void* out, void* aux, void* stream) {
  KRQ_REQUIRE(x && w8 && w_scale && (out || mode == kOutArgmax) && (aux || mode != kOutArgmax),
              "gemv_fp8: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w8), "gemv_fp8: x and w8 must be 16-byte aligned");
  KRQ_REQUIRE(x_kind >= KRQ_X_FP8 && x_kind <= KRQ_X_BF16_STATIC, "gemv_fp8: bad x_kind %d", x_kind);
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
  // paired row blocks for the multi-row matrix-core kernels (KRQ_GEMV_PAIR=0 turns them off)
  static const bool pair_ok = [] {
    const char* e = getenv("KRQ_GEMV_PAIR");
    return !(e && atoi(e) == 0);
  }();
  // Measured: pairing halves the blocks, which costs the Qwen3-4B projections (640-768 blocks)
  // more than the saved activation reads gain; the lm_head (9,496 blocks) gains 10-15%.
  const int pb = (pair_ok && mode != KRQ_OUT_SWIGLU && algo != 2 && M > 4 && (NO / 16) % 2 == 0 &&
                  (NO / 16) * split >= 4096) ? 2 : 1;
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : pb;
  const int MT = (algo == 2 || M <= 16) ? 1 : 2;
  // step slots per wave of the variant launch() picks
  const int U = (algo == 2 || M <= 4) ? 4 : 2;
  int nw = plan_waves((kts + 1) / 2, P, U);
  // fused prologues hold at most kXChunks 16-byte chunks per thread
  int64_t xchunks = 0;
  if (x_kind == KRQ_X_BF16_DYN) xchunks = (K + 7) / 8;
  if (x_kind == KRQ_X_BF16_STATIC) xchunks = M * (ks / 8);
  const int xc = x_kind == KRQ_X_BF16_DYN ? kXChunksDyn : kXChunks;
  while ((int64_t)nw * 64 * xc < xchunks && nw < kMaxThreads / 64) ++nw;
  KRQ_REQUIRE((int64_t)nw * 64 * xc >= xchunks,
              "gemv_fp8: activation slice of %lld elements too large for in-kernel quantization",
              (long long)(xchunks * 8));
  const size_t smem = (size_t)nw * P * MT * 256 * sizeof(float) +
                      (x_kind == KRQ_X_FP8 ? 0 : (size_t)M * ks);
  const dim3 grid(static_cast<unsigned>(NO / 16 / pb), static_cast<unsigned>(split));
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w8;
  const int m = static_cast<int>(M);
  hipStream_t s = (hipStream_t)stream;
#define KRQ_FP8_CASE(MODE, LAYOUT)                                                                   \
  launch_xk<MODE, LAYOUT>(x_kind, algo, pb, m, grid, nw, smem, s, xb, x_scale, x_inv, x_per_row, wb, \
                          w_scale, w_per_row, m, NO, K, kts, out, aux)
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
