// FP8 decode GEMVs with the RMSNorm prologue and the residual epilogue of the fused BF16 GEMVs
// (reference engine/kernels/fused_gemv.py:1-17, :48-167, carried over to the FP8 weights of
// engine/kernels/fp8.py): a decoder layer on FP8 weights is four GEMV launches plus attention.
//
//   qkv, gate_up   bf16 residual rows in, RMSNorm in the prologue, then the activation scaling of
//                  the plain FP8 GEMV (per token over the normalized row at M = 1, or a static
//                  SharedScale inverse at any M), e4m3 slice in LDS, matrix cores;
//   o, down        any activation kind, residual epilogue: x_new = bf16(res_in + bf16(y)) with y
//                  the in-order sum of the scaled split partials, plus per-tile sums of squares.
// Rows that do not fit the in-kernel staging (M > 1 with per-token scales) are normalized and
// quantized by k_rmsnorm_quant_rows first: one launch, the same values as quant_rows(rmsnorm(x)).
// The kernel template is gemv_fp8_kernel.h's; the fused variants always use the matrix cores.
#include "gemv_fp8_kernel.h"

using namespace krq;

namespace {

constexpr size_t kMaxSmem = 60 * 1024;
// largest bf16 x slice (bytes) a block normalizes in its prologue (as in fused_gemv.hip)
constexpr int64_t kNormStageMax = 24 * 1024;

// RMSNorm + per-token e4m3 quantization of whole rows (one block of NT threads per row, K % 16 == 0,
// K <= kRowMaxK): x8 = e4m3(h * inv), xs = amax(h) / 448 with the ActScale arithmetic of quant_rows
// (amax floored at 1e-6), h = RMSNorm(x) * ln as every normalizing kernel computes it. Each wave
// sums the row's sum-of-squares partials itself in the canonical order (lane l takes t = l, l + 64,
// ..., SC per lane) instead of staging them in LDS, each thread holds 16-value pieces (two 16-byte
// loads of x and of ln, one 16-byte store), and the amax is DPP wave maxima and one barrier.
// Measured on MI355X (fused FP8 layer, M = 16, against 256 threads of 8-value chunks with the
// partials staged in LDS and four barriers): gate_up + RMSNorm 15.01 -> 14.90 us, QKV + RMSNorm
// 9.29 -> 9.09 us. TILED: x8 in the tiled activation layout (tiled_offset), one block per row of
// the M rows padded to a multiple of 16, the pad rows zero. ROWSUM (one row): the row's own chunk
// sums (sumsq8, chunk i = elements 8 i ..) staged in LDS, and each wave takes the canonical sum over
// them instead of over ss_in.
constexpr int kNqThreads = 512;
template <int NT, int SC, bool TILED, bool ROWSUM>
__global__ __launch_bounds__(NT) void k_rmsnorm_quant_rows(const uint16_t* __restrict__ x,
                                                           const float* __restrict__ ss_in,
                                                           const uint16_t* __restrict__ ln, float eps,
                                                           int64_t M, int64_t K, uint8_t* __restrict__ x8,
                                                           float* __restrict__ xs) {
  constexpr int C = kRowMaxK / 16 / NT;
  __shared__ uint32_t red[NT / 64];
  __shared__ float sq[ROWSUM ? kRowMaxK / 8 : 1];
  const int64_t m = blockIdx.x;
  if (TILED && m >= M) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t e = 16 * (int64_t)(threadIdx.x + c * NT);
      if (e < K) *reinterpret_cast<uint4*>(x8 + tiled_offset(m, e, K)) = zero4();
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int T = (int)(K >> 4);
  const uint8_t* xr = reinterpret_cast<const uint8_t*>(x + m * K);
  const uint8_t* lr = reinterpret_cast<const uint8_t*>(ln);
  // every load unconditional, at a clamped address (pieces past K repeat the last piece)
  uint4 v[C][2], lv[C][2];
  float sp[SC];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = min(16 * (int64_t)(threadIdx.x + c * NT), K - 16);
    v[c][0] = ld16(xr + 2 * e);
    v[c][1] = ld16(xr + 2 * e + 16);
    lv[c][0] = ld16(lr + 2 * e);
    lv[c][1] = ld16(lr + 2 * e + 16);
  }
  float a = 0.0f;
  if constexpr (ROWSUM) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int p = threadIdx.x + c * NT;  // piece p: chunks 2 p and 2 p + 1
      if (16 * (int64_t)p < K) {
        sq[2 * p] = sumsq8(v[c][0]);
        sq[2 * p + 1] = sumsq8(v[c][1]);
      }
    }
    __syncthreads();
    for (int t = lane; t < (int)(K >> 3); t += 64) a += sq[t];
  } else {
#pragma unroll
    for (int j = 0; j < SC; ++j) sp[j] = ss_in[m * T + min(lane + 64 * j, T - 1)];
#pragma unroll
    for (int j = 0; j < SC; ++j)
      if (lane + 64 * j < T) a += sp[j];
  }
  const float rstd = rstd_of(a, K, eps);
  uint32_t am = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    v[c][0] = norm8(v[c][0], lv[c][0], rstd);
    v[c][1] = norm8(v[c][1], lv[c][1], rstd);
    if (16 * (int64_t)(threadIdx.x + c * NT) < K) am = absmax8(v[c][1], absmax8(v[c][0], am));
  }
  am = wave_max_u32_dpp(am);
  if (lane == 0) red[threadIdx.x >> 6] = am;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) am = umax32(am, red[i]);
  const float b = clamp_min_nan(as_f32(am), 1e-6f);
  const float iv = inv_from_amax(b);
  if (threadIdx.x == 0) xs[m] = scale_from_amax(b);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = 16 * (int64_t)(threadIdx.x + c * NT);
    if (e < K) {
      const uint2 lo = quant8(v[c][0], iv), hi = quant8(v[c][1], iv);
      *reinterpret_cast<uint4*>(x8 + (TILED ? tiled_offset(m, e, K) : m * K + e)) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }
}

template <bool TILED>
void launch_rmsnorm_quant(int64_t rows, const void* x, const float* ss_in, const void* ln, float eps, int64_t M,
                          int64_t K, void* x8, float* x_scale, hipStream_t s) {
  // SC partials per lane: T = K / 16 <= 64 * SC; one row sums itself (ROWSUM)
  const dim3 g(static_cast<unsigned>(rows)), b(kNqThreads);
  if (M == 1)
    hipLaunchKernelGGL((k_rmsnorm_quant_rows<kNqThreads, 1, TILED, true>), g, b, 0, s, (const uint16_t*)x, ss_in,
                       (const uint16_t*)ln, eps, M, K, (uint8_t*)x8, x_scale);
  else if (K <= 4096)
    hipLaunchKernelGGL((k_rmsnorm_quant_rows<kNqThreads, 4, TILED, false>), g, b, 0, s, (const uint16_t*)x, ss_in,
                       (const uint16_t*)ln, eps, M, K, (uint8_t*)x8, x_scale);
  else
    hipLaunchKernelGGL((k_rmsnorm_quant_rows<kNqThreads, kRowMaxK / 16 / 64, TILED, false>), g, b, 0, s,
                       (const uint16_t*)x, ss_in, (const uint16_t*)ln, eps, M, K, (uint8_t*)x8, x_scale);
}

#define KRQ_FUSED_FP8_ARGS xb, x_scale, x_inv, x_per_row, wb, w_scale, w_per_row, m, NO, K, kts, out, nullptr, fa

// u: step slots of the one-row launches beside the activation wave on the tiled layout (deep rings,
// plan()): 5 for the SwiGLU block, 8 or 10 otherwise; 0 for the default rings
template <int MODE, int LAYOUT, int XK, bool NORM>
void launch(int M, int awc, int u, dim3 grid, int nw, size_t smem, hipStream_t s, const uint8_t* xb,
            const float* x_scale, const float* x_inv, int x_per_row, const uint8_t* wb, const float* w_scale,
            int w_per_row, int m, int64_t NO, int64_t K, int kts, void* out, const FusedArgs& fa) {
  const dim3 block((nw + (awc > 0 ? 1 : 0)) * 64);
  if constexpr (LAYOUT == KRQ_W_TILED) {
    constexpr int DU = MODE == KRQ_OUT_SWIGLU ? kSwiU : kDeepU, MU = MODE == KRQ_OUT_SWIGLU ? kSwiU : kMidU;
    if constexpr (XK == KRQ_X_BF16_DYN || XK == KRQ_X_BF16_STATIC) {
      if (u > 0 && awc == kAwSmall) {
        // the SwiGLU's last column blocks as half-pair blocks, as the plain launch runs them
        const int64_t nrbs = NO / 16, rem = nrbs % kCUs;
        if constexpr (MODE == KRQ_OUT_SWIGLU) {
          if (u == MU && grid.y == 1 && nrbs > 2 * kCUs && rem != 0 && 2 * rem <= kCUs) {
            const int nfull = static_cast<int>(nrbs - rem);
            const dim3 gm(static_cast<unsigned>(nfull + 2 * rem), 1);
            hipLaunchKernelGGL((k_gemv_fp8_fused_swiglu_mixed<LAYOUT, XK, MU, NORM, kAwSmall>), gm, block, smem, s,
                               KRQ_FUSED_FP8_ARGS, nfull);
            return;
          }
        }
        if (u == MU)
          hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, MU, NORM, kAwSmall>), grid, block, smem, s,
                             KRQ_FUSED_FP8_ARGS);
        else
          hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, DU, NORM, kAwSmall>), grid, block, smem, s,
                             KRQ_FUSED_FP8_ARGS);
        return;
      }
      if constexpr (!NORM) {  // (with RMSNorm the wave takes rows of at most 4,096)
        if (u > 0 && awc == kAwLarge) {
          if (u == MU)
            hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, MU, NORM, kAwLarge>), grid, block, smem, s,
                               KRQ_FUSED_FP8_ARGS);
          else
            hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, DU, NORM, kAwLarge>), grid, block, smem, s,
                               KRQ_FUSED_FP8_ARGS);
          return;
        }
      }
    }
  }
  if constexpr (XK == KRQ_X_BF16_DYN || XK == KRQ_X_BF16_STATIC) {
    if (awc == kAwSmall) {
      hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, 4, NORM, kAwSmall>), grid, block, smem, s,
                         KRQ_FUSED_FP8_ARGS);
      return;
    }
    if (!NORM && awc == kAwLarge) {  // (with RMSNorm the wave takes rows of at most 4,096)
      hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, 4, NORM, kAwLarge>), grid, block, smem, s,
                         KRQ_FUSED_FP8_ARGS);
      return;
    }
  }
  if constexpr (NORM && XK == KRQ_X_BF16_DYN) {
    // (not reached: plan() gives a one-row RMSNorm launch the activation wave)
  } else if constexpr (MODE == kOutResidualFold) {  // (one row)
    hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, 4, NORM, 0>), grid, block, smem, s, KRQ_FUSED_FP8_ARGS);
  } else {
    if (M <= 4)
      hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, 4, NORM, 0>), grid, block, smem, s, KRQ_FUSED_FP8_ARGS);
    else if (M <= 16)
      hipLaunchKernelGGL((k_gemv_fp8_fused<1, MODE, LAYOUT, XK, 1, 2, NORM, 0>), grid, block, smem, s, KRQ_FUSED_FP8_ARGS);
    else
      hipLaunchKernelGGL((k_gemv_fp8_fused<2, MODE, LAYOUT, XK, 1, 2, NORM, 0>), grid, block, smem, s, KRQ_FUSED_FP8_ARGS);
  }
}

template <int MODE, int XK, bool NORM>
void launch_layout(int layout, int M, int awc, int u, dim3 grid, int nw, size_t smem, hipStream_t s,
                   const uint8_t* xb, const float* x_scale, const float* x_inv, int x_per_row, const uint8_t* wb,
                   const float* w_scale, int w_per_row, int m, int64_t NO, int64_t K, int kts, void* out,
                   const FusedArgs& fa) {
  if (layout == KRQ_W_TILED)
    launch<MODE, KRQ_W_TILED, XK, NORM>(M, awc, u, grid, nw, smem, s, xb, x_scale, x_inv, x_per_row, wb, w_scale,
                                         w_per_row, m, NO, K, kts, out, fa);
  else  // (the default rings with the planned waves: deep rings are tiled only)
    launch<MODE, KRQ_W_ROWMAJOR, XK, NORM>(M, awc, 0, grid, nw, smem, s, xb, x_scale, x_inv, x_per_row, wb,
                                            w_scale, w_per_row, m, NO, K, kts, out, fa);
}

struct FusedPlan {
  int nw;       // waves that stream weights
  int awc;      // chunks per lane of the activation wave (0: none, every wave runs the prologue)
  int u;        // step slots of the deep ring (tiled layout), 0: the default ring
  size_t smem;  // dynamic LDS bytes
  bool fold;    // the folded one-row residual launch (kOutResidualFold)
};

// One-row launches (M == 1, bf16 activations) get the activation wave of gemv_fp8_kernel.h when
// its registers hold what it loads: the whole row (per-token scale, or RMSNorm, which sums the row
// itself; K <= 4096 with RMSNorm) or the slice (static scale). Grids of fewer blocks than CUs keep
// the shared prologue.
int act_wave_chunks(int64_t M, int64_t K, int64_t ks, int mode, int x_kind, bool norm) {
  if (M != 1 || x_kind == KRQ_X_FP8 || x_kind == KRQ_X_FP8_TILED) return 0;
  if (norm && K > 512 * kAwSmall) return 0;
  const int64_t span = x_kind == KRQ_X_BF16_DYN || norm ? K : ks;
  return span <= 512 * kAwSmall ? kAwSmall : span <= 512 * kAwLarge ? kAwLarge : 0;
}

// Waves and LDS bytes of a fused FP8 launch; false if the prologue's staging does not fit.
bool plan(int64_t M, int64_t N, int64_t K, int split, int mode, int x_kind, bool norm, FusedPlan* out) {
  if (M < 1 || M > 32 || split < 1 || K < 64 || K % split || (K / split) % 64) return false;
  if (norm && (x_kind == KRQ_X_FP8 || x_kind == KRQ_X_FP8_TILED)) return false;
  if (x_kind == KRQ_X_BF16_DYN && M != 1) return false;
  const int64_t ks = K / split;
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : 1;
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  // The residual epilogue at M = 1 over the callers' four splits of bf16 activations runs folded:
  // N / 4 blocks (each four output columns over the four quarters of K, one matrix-core product
  // per step) with this plan's waves and ring, the split launch's sums bit for bit, and no cross-
  // block reduction. Its whole row is quantized into LDS.
  const bool fold = mode == kOutResidual && M == 1 && split == 4 &&
                    (x_kind == KRQ_X_BF16_DYN || x_kind == KRQ_X_BF16_STATIC);
  const int64_t kq = fold ? K : ks;  // elements of the row quantized into LDS
  const int awc = NO / 16 * split >= kCUs ? act_wave_chunks(M, K, kq, mode, x_kind, norm) : 0;
  // a one-row RMSNorm sums the row in the activation wave (no ss_in at M = 1)
  if (norm && M == 1 && awc == 0) return false;
  if (awc == 0 && norm && x_kind == KRQ_X_BF16_STATIC && M * ks * 2 > kNormStageMax) return false;
  const int kts = static_cast<int>(ks / 64);
  const int MT = M <= 16 ? 1 : 2;
  const int nsteps = (kts + 1) / 2;
  int nw = plan_waves(nsteps, P, M <= 4 ? 4 : 2, NO / 16 * split, awc > 0);
  // Deep rings beside the activation wave (tiled layout, M == 1): the plain kernels' rings, 8 or 10
  // slots, 5 for the two-matrix SwiGLU block, which then takes the activation wave too. Measured in
  // the fused FP8 layer at M = 1: gate_up + RMSNorm 11.60 -> 10.46 us, QKV + RMSNorm 6.80 -> 6.56.
  // The one-pass residual GEMVs (fewer blocks than CUs, every wave in the prologue) measured slower
  // with one round of 8- or 10-slot rings (O 6.21 -> 6.64, down 10.39 -> 12.12) and keep four slots.
  int u = 0;
  if (M == 1 && x_kind != KRQ_X_FP8 && awc > 0) {
    u = mode == KRQ_OUT_SWIGLU ? kSwiU : nsteps <= kMidU ? kMidU : kDeepU;
    nw = plan_waves(nsteps, P, u, NO / 16 * split, true);
  }
  bool staged_ss = false;  // the sum-of-squares partials staged in LDS (RMSNorm of M rows)
  if (awc == 0) {
    const int64_t xchunks = x_kind == KRQ_X_BF16_DYN ? (K + 7) / 8 : x_kind == KRQ_X_BF16_STATIC ? M * (kq / 8) : 0;
    const int xc = x_kind == KRQ_X_BF16_DYN ? kXChunksDyn : kXChunks;
    staged_ss = norm && x_kind == KRQ_X_BF16_STATIC;
    auto short_of = [&](int w) {
      return (int64_t)w * 64 * xc < xchunks || (staged_ss && (int64_t)w * 64 * kSsChunks * 4 < M * (K / 16));
    };
    while (short_of(nw) && nw < kMaxThreads / 64) ++nw;
    if (short_of(nw)) return false;
  } else {
    nw = min(nw, kMaxThreads / 64 - 1);
  }
  const size_t smem = (size_t)nw * P * MT * 256 * sizeof(float) +
                      (x_kind == KRQ_X_FP8 || x_kind == KRQ_X_FP8_TILED ? 0 : (size_t)M * kq) +
                      (staged_ss ? (size_t)M * (K / 16) * sizeof(float) : 0);
  if (smem > kMaxSmem) return false;
  *out = FusedPlan{nw, awc, u, smem, fold};
  return true;
}

}  // namespace

extern "C" int64_t krq_gemv_fp8_fused_fits(int64_t M, int64_t N, int64_t K, int split, int mode, int x_kind,
                                           int norm) {
  FusedPlan p;
  return plan(M, N, K, split, mode, x_kind, norm != 0, &p) ? 1 : 0;
}

extern "C" int krq_gemv_fp8_fused(const void* x, int x_kind, const float* x_scale, const float* x_inv,
                                  int x_per_row, const void* w8, int w_layout, const float* w_scale,
                                  int w_per_row, int64_t M, int64_t N, int64_t K, int split, int mode,
                                  const void* ln, const float* ss_in, float eps, const void* res_in,
                                  void* res_out, float* ss_out, uint32_t* cnt, void* out, void* stream) {
  KRQ_REQUIRE(x && w8 && w_scale, "gemv_fp8_fused: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w8), "gemv_fp8_fused: x and w8 must be 16-byte aligned");
  KRQ_REQUIRE(x_kind >= KRQ_X_FP8 && x_kind <= KRQ_X_FP8_TILED, "gemv_fp8_fused: bad x_kind %d", x_kind);
  KRQ_REQUIRE(x_kind == KRQ_X_BF16_DYN || x_scale, "gemv_fp8_fused: x_scale is required");
  KRQ_REQUIRE(x_kind != KRQ_X_BF16_STATIC || x_inv, "gemv_fp8_fused: x_inv is required");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_fp8_fused: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(x_kind != KRQ_X_BF16_DYN || M == 1, "gemv_fp8_fused: in-kernel per-token scaling takes M == 1");
  KRQ_REQUIRE(N > 0 && K >= 64 && split >= 1 && split <= 65535 && K % split == 0 && (K / split) % 64 == 0,
              "gemv_fp8_fused: no tiling divides K_SPLIT (K=%lld split=%d; K/split must be a multiple of 64)",
              (long long)K, split);
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "gemv_fp8_fused: bad layout %d", w_layout);
  KRQ_REQUIRE(mode == KRQ_OUT_BF16 || mode == KRQ_OUT_PARTIAL || mode == KRQ_OUT_SWIGLU || mode == kOutResidual,
              "gemv_fp8_fused: bad mode %d", mode);
  KRQ_REQUIRE(mode == KRQ_OUT_PARTIAL || mode == kOutResidual || split == 1,
              "gemv_fp8_fused: split %d needs the partials or residual output", split);
  const bool norm = ln != nullptr;
  KRQ_REQUIRE(norm || mode == kOutResidual,
              "gemv_fp8_fused: neither RMSNorm (ln) nor the residual epilogue; call krq_gemv_fp8");
  KRQ_REQUIRE(!(norm && mode == kOutResidual), "gemv_fp8_fused: RMSNorm and the residual epilogue in one call");
  KRQ_REQUIRE(!norm || (ss_in && aligned16(ln) && aligned16(ss_in) && x_kind != KRQ_X_FP8 && x_kind != KRQ_X_FP8_TILED),
              "gemv_fp8_fused: RMSNorm needs bf16 activations, ss_in and aligned ln / ss_in");
  // (at M = 1 with four splits of bf16 activations the folded form needs neither cnt nor out)
  const bool one_row4 = M == 1 && split == 4 && (x_kind == KRQ_X_BF16_DYN || x_kind == KRQ_X_BF16_STATIC);
  KRQ_REQUIRE(mode != kOutResidual || (res_in && res_out && ss_out && (split == 1 || one_row4 || (cnt && out))),
              "gemv_fp8_fused: the residual epilogue needs res_in, res_out, ss_out and, for split > 1, "
              "cnt and the partials buffer");
  KRQ_REQUIRE(mode == kOutResidual || out, "gemv_fp8_fused: null output");
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  KRQ_REQUIRE(NO % 16 == 0 && (mode != KRQ_OUT_SWIGLU || N % 2 == 0) && NO / 16 <= 0x7fffffff,
              "gemv_fp8_fused: no tiling divides N=%lld", (long long)N);
  FusedPlan p;
  KRQ_REQUIRE(plan(M, N, K, split, mode, x_kind, norm, &p),
              "gemv_fp8_fused: M=%lld x K/split=%lld does not fit the in-kernel staging; normalize and "
              "quantize rows first (krq_rmsnorm_quant_rows)", (long long)M, (long long)(K / split));
  const int kts = static_cast<int>(K / split / 64);  // (folded: the tiles of one quarter of K)
  const dim3 grid = p.fold ? dim3(static_cast<unsigned>(N / 4), 1)
                           : dim3(static_cast<unsigned>(NO / 16), static_cast<unsigned>(split));
  const FusedArgs fa{reinterpret_cast<const uint16_t*>(ln), ss_in, eps, reinterpret_cast<const uint16_t*>(res_in),
                     reinterpret_cast<uint16_t*>(res_out), ss_out, cnt};
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w8;
  const int m = static_cast<int>(M);
  hipStream_t s = (hipStream_t)stream;
#define KRQ_CASE(MODE, XK, NORM)                                                                          \
  launch_layout<MODE, XK, NORM>(w_layout, m, p.awc, p.u, grid, p.nw, p.smem, s, xb, x_scale, x_inv, x_per_row, wb, w_scale, \
                                w_per_row, m, NO, K, kts, out, fa)
  if (p.fold) {
    if (x_kind == KRQ_X_BF16_DYN) KRQ_CASE(kOutResidualFold, KRQ_X_BF16_DYN, false);
    else KRQ_CASE(kOutResidualFold, KRQ_X_BF16_STATIC, false);
  } else if (mode == kOutResidual) {
    if (x_kind == KRQ_X_FP8) KRQ_CASE(kOutResidual, KRQ_X_FP8, false);
    else if (x_kind == KRQ_X_FP8_TILED) KRQ_CASE(kOutResidual, KRQ_X_FP8_TILED, false);
    else if (x_kind == KRQ_X_BF16_DYN) KRQ_CASE(kOutResidual, KRQ_X_BF16_DYN, false);
    else KRQ_CASE(kOutResidual, KRQ_X_BF16_STATIC, false);
  } else if (x_kind == KRQ_X_BF16_DYN) {
    if (mode == KRQ_OUT_BF16) KRQ_CASE(KRQ_OUT_BF16, KRQ_X_BF16_DYN, true);
    else if (mode == KRQ_OUT_PARTIAL) KRQ_CASE(KRQ_OUT_PARTIAL, KRQ_X_BF16_DYN, true);
    else KRQ_CASE(KRQ_OUT_SWIGLU, KRQ_X_BF16_DYN, true);
  } else {
    if (mode == KRQ_OUT_BF16) KRQ_CASE(KRQ_OUT_BF16, KRQ_X_BF16_STATIC, true);
    else if (mode == KRQ_OUT_PARTIAL) KRQ_CASE(KRQ_OUT_PARTIAL, KRQ_X_BF16_STATIC, true);
    else KRQ_CASE(KRQ_OUT_SWIGLU, KRQ_X_BF16_STATIC, true);
  }
#undef KRQ_CASE
  return krq_check_launch("gemv_fp8_fused");
}

extern "C" int krq_rmsnorm_quant_rows(const void* x, const float* ss_in, const void* ln, float eps, int64_t M,
                                      int64_t K, void* x8, float* x_scale, void* stream) {
  KRQ_REQUIRE(x && ss_in && ln && x8 && x_scale, "rmsnorm_quant_rows: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(ln) && aligned16(x8), "rmsnorm_quant_rows: x, ln and x8 must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 0x7fffffff && K > 0 && K % 16 == 0 && K <= kRowMaxK,
              "rmsnorm_quant_rows: bad shape M=%lld K=%lld (K a multiple of 16, at most %d)", (long long)M,
              (long long)K, kRowMaxK);
  launch_rmsnorm_quant<false>(M, x, ss_in, ln, eps, M, K, x8, x_scale, (hipStream_t)stream);
  return krq_check_launch("rmsnorm_quant_rows");
}

extern "C" int krq_rmsnorm_quant_rows_tiled(const void* x, const float* ss_in, const void* ln, float eps, int64_t M,
                                      int64_t K, void* x8, float* x_scale, void* stream) {
  KRQ_REQUIRE(x && ss_in && ln && x8 && x_scale, "rmsnorm_quant_rows_tiled: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(ln) && aligned16(x8), "rmsnorm_quant_rows_tiled: x, ln and x8 must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 0x7fffffff && K > 0 && K % 16 == 0 && K <= kRowMaxK,
              "rmsnorm_quant_rows_tiled: bad shape M=%lld K=%lld (K a multiple of 16, at most %d)", (long long)M,
              (long long)K, kRowMaxK);
  KRQ_REQUIRE(K % 64 == 0, "rmsnorm_quant_rows_tiled: K=%lld must be a multiple of 64", (long long)K);
  const int64_t mp = (M + 15) / 16 * 16;  // rows padded to whole 16-row tiles
  launch_rmsnorm_quant<true>(mp, x, ss_in, ln, eps, M, K, x8, x_scale, (hipStream_t)stream);
  return krq_check_launch("rmsnorm_quant_rows_tiled");
}
