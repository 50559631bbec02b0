// The FP8 skinny GEMM / GEMV kernel template, shared by the plain entry points (gemv_fp8.hip) and
// the fused ones (fused_fp8.hip): y = (x8 . w8^T) * x_scale[m] * w_scale[n], fp32 accumulate.
// Layout, step and epilogue conventions: gemv_common.h.
//
// Activation kinds (template XK):
//   KRQ_X_FP8          x is e4m3 [M, K] with its scale; matrix-core A operands are loaded from
//                      global memory by the lanes whose row m < M.
//   KRQ_X_FP8_TILED    the same e4m3 rows in the tiled activation layout (krq_quant_rows_tiled:
//                      16-row x 64-byte tiles, lane 16 g + r holding row r's bytes 16 g .. 16 g + 15),
//                      so each A operand load is one contiguous KiB, like the weights'.
//   KRQ_X_BF16_DYN     x is bf16 [1, K]; the block computes the per-token scale itself
//                      (amax over all of K, ActScale arithmetic), quantizes its K slice into LDS.
//   KRQ_X_BF16_STATIC  x is bf16 [M, K] with a given inverse scale (SharedScale / ActScale
//                      inv, per tensor or per row); the block quantizes its K slice into LDS.
// NORM (bf16 kinds only): the bf16 rows are first normalized, h = bf16(bf16(x * rstd) * w_ln)
// with rstd from the [M][K/16] sum-of-squares partials, and h is what gets scaled and quantized
// (the per-token amax of KRQ_X_BF16_DYN is taken over h).
// The activation loads of the fused kinds are issued before the first weight batch, so their
// latency (L2 hits) overlaps the weight stream's; quantization uses the hardware e4m3 convert
// after the reference's clamp, which is bit-identical to the software encoder.
#pragma once

#include "gemv_common.h"

#ifdef KRQ_TIMELINE
// Timeline build only (compiled out of the shipped library): per block of the last launch that
// ran, wall-clock stamps (100 MHz) at entry, activation slice ready, main loop done and outputs
// issued (slots 0-3), and the compute unit it ran on (slot 4, __smid: XCD, shader engine, CU),
// read back with krq_timeline_read. One copy per translation unit.
static __device__ unsigned long long krq_timeline[8 * 65536];
#define KRQ_STAMP(i, who)                                                                          \
  do {                                                                                             \
    const unsigned long long b_ = 8ull * (blockIdx.y * gridDim.x + blockIdx.x);                    \
    if ((who) && b_ < 8ull * 65536) {                                                              \
      krq_timeline[b_ + (i)] = wall_clock64();                                                     \
      if ((i) == 0) krq_timeline[b_ + 4] = __smid();                                               \
    }                                                                                              \
  } while (0)
#else
#define KRQ_STAMP(i, who) \
  do {                    \
  } while (0)
#endif

namespace {
using namespace krq;

// 16-byte activation chunks per thread in the fused prologues: every chunk load is issued (see
// the kernel), so the one-row prologue, which reads the whole row for its amax, keeps the count
// small and takes more waves for long rows instead
constexpr int kXChunks = 8;
constexpr int kXChunksDyn = 4;
// 16-byte (four-partial) sum-of-squares chunks per thread in the RMSNorm prologue (staged rows)
constexpr int kSsChunks = 4;
constexpr int kMaxThreads = 512;
// one-row activation wave: 16-byte chunks per lane (the whole row, K <= 64 * 8 * AWC)
constexpr int kAwSmall = 8, kAwLarge = 20;
// the smallest one-row wave (K <= 2560), so no lane of a short row loads a clamped repeat of its last chunk
constexpr int kAwRow = 5;
// step slots of the deep-ring one-row kernels (a weight wave issues all of its steps at once)
constexpr int kMidU = 8, kDeepU = 10, kSwiU = 5, kBigU = 20;
constexpr int64_t kCUs = 256;  // compute units of the MI355X

// The activation wave of the one-row kernels: one extra wave per block that quantizes the block's
// K slice [k0, k0 + ks) of the bf16 row into LDS, while the other waves only issue their weight
// loads. It issues no weight loads itself, so its row loads are not queued behind its own weight
// stream, and it runs at raised issue priority; the weight waves wait for it at one barrier.
//   KRQ_X_BF16_DYN: loads the whole row, takes its amax (ActScale arithmetic), quantizes the slice.
//   KRQ_X_BF16_STATIC (M = 1): loads the slice and quantizes it with the given inverse scale.
// NORM: the loaded chunks are first normalized, h = bf16(bf16(x * rstd) * w_ln), with rstd from the
// row's own sum of squares in the canonical order (sumsq8 of its chunks; the wave loads the whole
// row, K <= 4096, also for a static scale, and quantizes the slice).
// ORDER: the wave meets the weight waves at a bare s_barrier (no fence, no wait) once all of its
// loads are issued, and the weight waves issue their ring only after it; see gemv_fp8_body.
// CH (second stage of the chained MLP, KRQ_X_BF16_DYN): the row is written in this launch by the
// first stage's workgroups, on every XCD. The wave first polls its replica of the first stage's
// done flag with a scalar load (which does not queue behind the vector memory traffic of the
// weight stream), until it is set or fa.max_polls polls pass; then it reads the row with
// agent-scope (sc1) buffer loads, which read memory instead of a stale line of this XCD's L2. A
// wait that gives up records kChainErr and makes the scale NaN, so every output of the block is
// NaN.
template <int XK, int AWC, bool NORM, bool ORDER, bool CH = false>
KRQ_DEV void activation_wave(const uint8_t* __restrict__ x, const float* __restrict__ xsc,
                             const float* __restrict__ xinv, int64_t K, int64_t k0, int ks, int lane,
                             uint8_t* xq, float* xs_l, const FusedArgs& fa) {
  constexpr int LC = NORM ? AWC : 1;
  static_assert(!CH || (XK == KRQ_X_BF16_DYN && !NORM), "chained stage: one bf16 row scaled per token");
  bool chain_bad = false;
  if constexpr (CH) chain_bad = !chain_wait(fa);
  __builtin_amdgcn_s_setprio(3);
  // FULL (per-token scale, or RMSNorm): chunk i = lane + 64 c of the row holds elements 8i .. 8i + 7
  // (indices past the row repeat its last chunk); otherwise (static scale) the same over the slice
  constexpr bool FULL = XK == KRQ_X_BF16_DYN || NORM;
  const int lo = static_cast<int>(k0 >> 3), n = ks >> 3;
  const int last = FULL ? static_cast<int>(K >> 3) - 1 : n - 1;
  const int64_t e0 = FULL ? 0 : k0;  // first element of chunk 0
  const uint8_t* lnb = reinterpret_cast<const uint8_t*>(fa.ln);
  uint4 v[AWC], lv[LC];
#pragma unroll
  for (int c = 0; c < AWC; ++c) {
    const int64_t e = e0 + 8 * (int64_t)min(lane + 64 * c, last);
    if constexpr (CH) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(x), (short)0,
                                                                          static_cast<int>(2 * K), 0x00020000);
      v[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(2 * e), 0, 16));
    } else {
      v[c] = ld16(x + 2 * e);
    }
    if (NORM) lv[c] = ld16(lnb + 2 * e);
  }
  float inv = 0.0f;
  if (XK == KRQ_X_BF16_STATIC) {
    inv = xinv[0];
    if (lane == 0) xs_l[0] = xsc[0];
  }
  __builtin_amdgcn_sched_barrier(0);  // every row load in flight before the first wait
  if constexpr (ORDER) __builtin_amdgcn_s_barrier();
  if (NORM) {
    float a = 0.0f;  // the row's canonical sum of squares: chunk i = lane + 64 c at lane i % 64
#pragma unroll
    for (int c = 0; c < AWC; ++c)
      if (lane + 64 * c <= last) a += sumsq8(v[c]);
    const float rstd = rstd_of(a, K, fa.eps);
    // only chunks inside the row: the clamped repeats are left raw and kept out of the amax
#pragma unroll
    for (int c = 0; c < AWC; ++c)
      if (lane + 64 * c <= last) v[c] = norm8(v[c], lv[NORM ? c : 0], rstd);
  }
  if (XK == KRQ_X_BF16_DYN) {
    u16x2 mb = {0, 0};
#pragma unroll
    for (int c = 0; c < AWC; ++c)
      if (!NORM || lane + 64 * c <= last) mb = absmax8_bits(v[c], mb);
    float am = clamp_min_nan(as_f32(wave_max_u32_dpp(bits_max_to_u32(mb))), 1e-6f);
    if (CH && chain_bad) am = __builtin_nanf("");
    inv = inv_from_amax(am);
    if (lane == 0) xs_l[0] = scale_from_amax(am);
  }
#pragma unroll
  for (int c = 0; c < AWC; ++c) {
    const int i = lane + 64 * c - (FULL ? lo : 0);  // chunk index inside the slice
    if (static_cast<unsigned>(i) < static_cast<unsigned>(n))
      *reinterpret_cast<uint2*>(xq + 8 * i) =
          XK == KRQ_X_BF16_DYN ? quant8_own_amax(v[c], inv) : quant8_clamped(v[c], inv);
  }
  __builtin_amdgcn_s_setprio(0);
}

// PB = 2 (MFMA kernels, modes other than SwiGLU): the block owns two adjacent row blocks, so each
// activation load feeds two matrix-core products (at M > 1 the activation slices are as large as
// the weight steps, and every row block re-reads them).
// AWC > 0 (one-row kind without RMSNorm): the block's last wave is the activation wave above and
// the others stream weights; AWC = 0: every wave takes part in the activation prologue.
// CHAIN (the chained MLP, k_mlp_chain_fp8): a SwiGLU block writes act through to memory and then
// counts itself into the first-stage counters; a split-K (partials) block is a second-stage
// block whose activation wave waits for the first stage's done flag (activation_wave<..., CH>)
// and which counts its exit, the last one out zeroing the control words (chain_tail). sy >= 0 / nwo > 0: the block's K split and its
// weight-wave count, given (the chained kernel's one-dimensional grid and common block size).
template <int MT, int MODE, int LAYOUT, int XK, int ALGO, int U, int PB, bool NORM, int AWC, bool CHAIN = false>
KRQ_DEV void gemv_fp8_body(const uint8_t* __restrict__ x, const float* __restrict__ xsc,
                           const float* __restrict__ xinv, int x_per_row, const uint8_t* __restrict__ w8,
                           const float* __restrict__ wsc, int w_per_row, int M, int64_t NO, int64_t K,
                           int kts, void* __restrict__ out, void* __restrict__ aux, const FusedArgs& fa,
                           int64_t bx, int sy = -1, int nwo = 0) {
  // nw*P*MT*256 partial sums | e4m3 activation slice [M][ks] | (NORM) sum-of-squares [M][K/16].
  // 16-byte aligned: the slice is read 16 bytes per lane. (Without it the dynamic region starts
  // right after the static variables, at a 4-byte boundary when they total 132 bytes, as in the
  // two-row-tile argmax kernels, and the slice's 8- and 16-byte accesses are misaligned.)
  extern __shared__ __align__(16) float red[];
  __shared__ float xs_l[32], rstd_s[32];
  __shared__ uint32_t amax_w[kMaxThreads / 64];
  __shared__ uint32_t last_s;
  static_assert(PB == 1 || (MODE != KRQ_OUT_SWIGLU && MODE != kOutSwiGluHalf && MODE != kOutResidual && ALGO != 2),
                "paired row blocks: MFMA, no SwiGLU or residual epilogue");
  static_assert(!NORM || (XK != KRQ_X_FP8 && XK != KRQ_X_FP8_TILED), "the RMSNorm prologue takes bf16 activations");
  constexpr bool AW = AWC > 0;
  static_assert(!AW || (XK != KRQ_X_FP8 && XK != KRQ_X_FP8_TILED && MT == 1), "activation wave: one bf16 row");
  static_assert(!NORM || XK != KRQ_X_BF16_DYN || AW, "one-row RMSNorm: the activation wave sums the row");
  static_assert(XK != KRQ_X_FP8_TILED || ALGO != 2, "tiled activations: matrix-core kernels");
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : PB;  // weight row blocks streamed per step
  constexpr bool XT = XK == KRQ_X_FP8_TILED;
  constexpr bool FUSED = XK != KRQ_X_FP8 && !XT;  // bf16 activations quantized into LDS
  // FOLD: folded one-row residual block (kOutResidualFold): bx owns output columns 4 bx .. 4 bx + 3,
  // kts counts the tiles of one quarter of K, and the whole row is quantized into LDS
  constexpr bool FOLD = MODE == kOutResidualFold;
  static_assert(!FOLD || (MT == 1 && PB == 1 && ALGO == 1 && FUSED && !NORM && !CHAIN),
                "folded residual: one row, bf16 activations quantized in the kernel, matrix cores");
  constexpr int SC = kSsChunks;
  // Load order of the RMSNorm activation wave beside a single-matrix ring: the CU returns loads in
  // issue order, so the wave's row, RMSNorm-weight and partials loads, issued while the weight wave
  // issues its ring, land only after most of it. Making the weight waves issue after the activation wave's loads
  // (one bare barrier) took the M = 1 QKV + RMSNorm launch from 6.58 to 5.22 us; the plain one-row
  // kernels (row loads only: QKV 4.71 -> 5.01 us) and the two-round SwiGLU block (gate_up +
  // RMSNorm 10.5 -> 10.75 us) measured slower with it, so they keep issuing at once.
  constexpr bool ORDER = AWC > 0 && NORM && MODE != KRQ_OUT_SWIGLU && MODE != kOutSwiGluHalf;
  // nw = the waves that stream weights (all but the activation wave)
  static_assert(!CHAIN || (MT == 1 && PB == 1 && !NORM &&
                            ((MODE == KRQ_OUT_PARTIAL && AWC > 0 && XK == KRQ_X_BF16_DYN) ||
                             MODE == KRQ_OUT_SWIGLU || MODE == kOutSwiGluHalf)),
                "chained MLP: SwiGLU first stage, per-token partials second stage");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = nwo > 0 ? nwo : (blockDim.x >> 6) - (AW ? 1 : 0);
  const int r = lane & 15, g = lane >> 4;
  // FOLD: blocks b and b ^ 1 read the two halves of every weight line they touch (rows 8 h .. 8 h + 7
  // of a tile, 64 bytes each); workgroups w and w + 8 run on one XCD, so block b = 2 (8 k + x) + h
  // goes to workgroup w = 16 k + 8 h + x and each line is fetched into one L2 (tail: b = w).
  // Measured in the fused FP8 layer at M = 1: O + residual 5.83 -> 5.07 us, down + residual 10.43 ->
  // 9.15 against the identity order.
  const int64_t bxf = FOLD && bx < (NO >> 2) / 16 * 16 ? 2 * (8 * (bx >> 4) + (bx & 7)) + ((bx >> 3) & 1) : bx;
  const int64_t rb = bxf * PB, rbu = MODE == KRQ_OUT_SWIGLU ? rb + (NO >> 4) : rb + 1;
  const int sidx = sy >= 0 ? sy : static_cast<int>(blockIdx.y);
  const int nsteps = (kts + 1) >> 1;
  const int64_t tbase = (int64_t)sidx * kts;
  const int64_t k0 = tbase * 64;  // first K element of this split
  const int ks = (FOLD ? 4 : 1) * kts * 64;  // K elements of this split (FOLD: the whole row)
  const int T = (int)(K >> 4);    // sum-of-squares partials per row
  uint8_t* xq = reinterpret_cast<uint8_t*>(red + nw * P * MT * 256);
  const int jcount = wave < nsteps ? (nsteps - wave + nw - 1) / nw : 0;
  KRQ_STAMP(0, threadIdx.x == 0);
  const ColScales cs = FOLD ? ColScales{1.0f, 1.0f} : load_col_scales<MODE, PB>(wsc, w_per_row, NO, rb);
  // the residual epilogue's residual values, read now so their latency hides under the weight
  // stream (measured in the fused FP8 layer at M = 16: o + residual 7.89 -> 7.80 us, down +
  // residual 11.93 -> 11.85, layer 43.8 -> 43.2; the folded one-row epilogue keeps its loads: down
  // + residual 9.15 -> 10.04 with them moved here, as does the BF16 kernel: o + residual at M = 16
  // 8.58 -> 8.77)
  ResidualPre<MT> rpre{};
  if constexpr (MODE == kOutResidual) rpre = load_residual<MT>(fa, M, NO, rb);

  // ---- fused activation prologue, part 1: activation loads ahead of the weight stream ----
  // Every load of the prologue and of the step ring is issued unconditionally, at a clamped (valid)
  // address where it is not needed: a branch around a load makes the compiler's wait counts
  // conservative (a full drain, vmcnt(0)) at the join, which serializes the weight stream.
  uint4 xv[kXChunks], lv[kXChunks], sv[SC];
  const uint8_t* lnb = reinterpret_cast<const uint8_t*>(fa.ln);
  if (XK == KRQ_X_BF16_DYN && !AW) {
#pragma unroll
    for (int c = 0; c < kXChunksDyn; ++c) {
      const int64_t e = min(8 * (int64_t)(threadIdx.x + c * blockDim.x), K - 8);
      xv[c] = ld16(x + 2 * e);  // chunks past K repeat the last one (same amax)
      if (NORM) lv[c] = ld16(lnb + 2 * e);
    }
  } else if (XK == KRQ_X_BF16_STATIC && !AW) {
    const int cpr = ks >> 3;  // chunks per row of the slice
#pragma unroll
    for (int c = 0; c < kXChunks; ++c) {
      const int idx = threadIdx.x + c * blockDim.x, m = idx / cpr;
      const int64_t e = k0 + 8 * (idx - m * cpr);
      xv[c] = ld16(x + 2 * ((int64_t)min(m, M - 1) * K + e));
      if (NORM) lv[c] = ld16(lnb + 2 * e);
    }
  }
  if (NORM && !AW) {  // (static scale, M rows: the [M][K/16] partials, staged in LDS below)
    const int nss = M * T / 4;  // 16-byte chunks of the partials
#pragma unroll
    for (int c = 0; c < SC; ++c)
      sv[c] = ld16(reinterpret_cast<const uint8_t*>(fa.ss_in) + 16 * min((int)threadIdx.x + c * (int)blockDim.x, nss - 1));
  }

  // a block whose only weight wave writes its outputs from registers (no cross-wave sum)
  constexpr bool DIRECT_OK = MT == 1 && PB == 1 && (MODE == KRQ_OUT_BF16 || MODE == KRQ_OUT_PARTIAL);
  const bool direct = DIRECT_OK && nw == 1;
  // (wave index read as a scalar: the compiler then knows the branch is uniform per wave)
  if (AW && __builtin_amdgcn_readfirstlane(wave) == nw) {
    activation_wave<XK, AW ? AWC : 1, NORM, ORDER, CHAIN && MODE == KRQ_OUT_PARTIAL>(x, xsc, xinv, K, k0, ks, lane, xq,
                                                                                 xs_l, fa);
    KRQ_STAMP(1, lane == 0);
    __syncthreads();  // the slice and its scale are in LDS
    if (direct) return;
  } else {
  // scale of this thread's activation row, read now so its latency hides under the weight stream
  // (every thread loads and stores it, threads t and t + 32 the same value, so the load is not
  // sunk into a branch after the weight loads)
  const int xrow = min((int)(threadIdx.x & 31), M - 1);
  const float xs_reg = XK != KRQ_X_BF16_DYN && !AW ? xsc[x_per_row ? xrow : 0] : 1.0f;

  // ---- weight (and, for e4m3 activations, A operand) loads: a ring of U step slots ----
  if constexpr (ORDER) __builtin_amdgcn_s_barrier();  // the activation wave's loads are issued
  uint4 wl[U], wh[U], ul[U], uh[U], xl[U][MT], xh[U][MT];
  // A slot past this wave's last step reloads that step (an address already in flight or cached,
  // so no extra HBM traffic) and is masked where consumed. Rows m >= M read row M - 1: their
  // products land in accumulator rows the epilogue never writes.
  auto load_slot = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const int64_t t0 = tbase + 2 * j;
    const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
    if constexpr (MODE == kOutSwiGluHalf) {
      wl[u] = ld16nt(w_addr_hp<LAYOUT>(w8, rb, NO, t0, K, lane));
      wh[u] = ld16nt(w_addr_hp<LAYOUT>(w8, rb, NO, t1, K, lane));
    } else if constexpr (FOLD) {
      wl[u] = ld16nt(w_addr_fold<LAYOUT>(w8, rb, K, kts, t0, lane));
      wh[u] = ld16nt(w_addr_fold<LAYOUT>(w8, rb, K, kts, t1, lane));
    } else {
      wl[u] = ld16nt(w_addr<LAYOUT>(w8, rb, t0, K, lane));
      wh[u] = ld16nt(w_addr<LAYOUT>(w8, rb, t1, K, lane));
    }
    if (P == 2) {
      ul[u] = ld16nt(w_addr<LAYOUT>(w8, rbu, t0, K, lane));
      uh[u] = ld16nt(w_addr<LAYOUT>(w8, rbu, t1, K, lane));
    }
    if (!FUSED) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (XT) {  // tile (mt, t) of the activations: this lane's 16 bytes of it
          xl[u][mt] = ld16(x + (((int64_t)mt * (K >> 6) + t0) * 64 + lane) * 16);
          xh[u][mt] = ld16(x + (((int64_t)mt * (K >> 6) + t1) * 64 + lane) * 16);
        } else {
          const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
          const uint8_t* xr = x + (int64_t)m * K + g * 16;
          xl[u][mt] = ld16(xr + t0 * 64);
          xh[u][mt] = ld16(xr + t1 * 64);
        }
      }
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) load_slot(u, u);
  __builtin_amdgcn_sched_barrier(0);

  // ---- RMSNorm (NORM, static scale, M rows): rstd from the partials, then normalize the chunks ----
  if (NORM && !AW) {
    float* sst = reinterpret_cast<float*>(xq + (size_t)M * ks);
    const int nss = M * T / 4;
#pragma unroll
    for (int c = 0; c < SC; ++c) {
      const int i = threadIdx.x + c * blockDim.x;
      if (i < nss) *reinterpret_cast<uint4*>(sst + 4 * i) = sv[c];
    }
    __syncthreads();
    row_rstd(sst, M, T, K, fa.eps, rstd_s);
    __syncthreads();
    {
      const int cpr = ks >> 3;
#pragma unroll
      for (int c = 0; c < kXChunks; ++c) {
        const int m = (threadIdx.x + c * blockDim.x) / cpr;
        xv[c] = norm8(xv[c], lv[c], rstd_s[min(m, M - 1)]);
      }
    }
  }

  // ---- fused activation prologue, part 2: scale, quantize the slice into LDS ----
  if (XK == KRQ_X_FP8 || XT) {
    xs_l[threadIdx.x & 31] = xs_reg;
  } else if (XK == KRQ_X_BF16_DYN) {
    if constexpr (!AW) {  // (with the activation wave, the slice is already in LDS after the barrier below)
      uint32_t am = 0;
#pragma unroll
      for (int c = 0; c < kXChunksDyn; ++c)
        if (!NORM || 8 * (int64_t)(threadIdx.x + c * blockDim.x) < K) am = absmax8(xv[c], am);
      am = wave_max_u32(am);
      if (lane == 0) amax_w[wave] = am;
      __syncthreads();
      uint32_t ab = amax_w[0];
      for (int w = 1; w < nw; ++w) ab = umax32(ab, amax_w[w]);
      const float a = clamp_min_nan(as_f32(ab), 1e-6f);
      const float inv = inv_from_amax(a);
      if (threadIdx.x == 0) xs_l[0] = scale_from_amax(a);
#pragma unroll
      for (int c = 0; c < kXChunksDyn; ++c) {
        const int64_t e = 8 * (int64_t)(threadIdx.x + c * blockDim.x);
        if (e >= k0 && e < k0 + ks) *reinterpret_cast<uint2*>(xq + (e - k0)) = quant8(xv[c], inv);
      }
    }
  } else if constexpr (!AW) {
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
  if constexpr (!AW) KRQ_STAMP(1, threadIdx.x == 0);

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
        if constexpr (FOLD) {  // A row r < 4: quarter r of the row; rows 4..15 zero
          const uint8_t* xr = xq + min(r, 3) * (kts * 64) + g * 16;
          xl[u][mt] = sel4(r < 4, *reinterpret_cast<const uint4*>(xr + (2 * j) * 64));
          xh[u][mt] = sel4(r < 4 && 2 * j + 1 < kts, *reinterpret_cast<const uint4*>(xr + min(2 * j + 1, kts - 1) * 64));
        } else {
          const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
          const uint8_t* xr = xq + (int64_t)m * ks + g * 16;
          xl[u][mt] = *reinterpret_cast<const uint4*>(xr + (2 * j) * 64);
          xh[u][mt] = sel4(2 * j + 1 < kts, *reinterpret_cast<const uint4*>(xr + min(2 * j + 1, kts - 1) * 64));
        }
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
  KRQ_STAMP(2, threadIdx.x == 0);
  if (direct) {
    // lane l, element i holds output row 4 (l / 16) + i, column 16 rb + l % 16 (xs_l is in LDS:
    // written by this wave, or by the activation wave before the barrier above)
    if constexpr (DIRECT_OK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        if (m < M) {
          const int64_t n = rb * 16 + r;
          const float y = acc[0][i] * xs_l[m] * cs.g;
          if (MODE == KRQ_OUT_BF16)
            reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = f32_to_bf16(y);
          else
            reinterpret_cast<float*>(out)[((int64_t)sidx * M + m) * NO + n] = y;
        }
      }
    }
    if constexpr (CHAIN) chain_tail<false>(fa);  // (thread 0 is in this wave)
    KRQ_STAMP(3, threadIdx.x == 0);
    return;
  }
  stash<MT, P>(red, wave, lane, acc, accu);
  }  // weight waves
  __syncthreads();
  if constexpr (MODE == kOutResidual) {
    residual_epilogue<MT>(red, nw, M, NO, rb, sidx, gridDim.y, xs_l, cs.g, reinterpret_cast<float*>(out), fa,
                          &last_s, &rpre);
  } else if constexpr (FOLD) {
    fold_residual_epilogue(red, nw, rb, xs_l, wsc, w_per_row, fa);
  } else {
    epilogue<MT, MODE, P, CHAIN>(red, 0, nw, M, NO, rb, sidx, xs_l, cs, out, aux);
    if (PB == 2) epilogue<MT, MODE, P>(red, 1, nw, M, NO, rbu, sidx, xs_l, ColScales{cs.u, 1.0f}, out, aux);
  }
  if constexpr (CHAIN) chain_tail<MODE != KRQ_OUT_PARTIAL>(fa);
  KRQ_STAMP(3, threadIdx.x == 0);
}

#define KRQ_FP8_KERNEL_PARAMS                                                                             \
  const uint8_t *__restrict__ x, const float *__restrict__ xsc, const float *__restrict__ xinv, int x_per_row, \
      const uint8_t *__restrict__ w8, const float *__restrict__ wsc, int w_per_row, int M, int64_t NO,        \
      int64_t K, int kts, void *__restrict__ out, void *__restrict__ aux

// the plain kernel (gemv_fp8.hip)
template <int MT, int MODE, int LAYOUT, int XK, int ALGO, int U, int PB, int AWC>
__global__ __launch_bounds__(kMaxThreads) void k_gemv_fp8(KRQ_FP8_KERNEL_PARAMS) {
  gemv_fp8_body<MT, MODE, LAYOUT, XK, ALGO, U, PB, false, AWC>(x, xsc, xinv, x_per_row, w8, wsc, w_per_row, M, NO,
                                                               K, kts, out, aux, FusedArgs{}, blockIdx.x);
}

// The SwiGLU launch (MT 16-row tiles) with its last column blocks split in half: nfull two-matrix
// blocks (output columns 16 i .. 16 i + 15) and nh = gridDim.x - nfull half-pair blocks 2 nfull + j
// (columns 8 (2 nfull + j) ..), which stream half the bytes with the same steps per wave.
// Workgroup i runs on compute unit i mod 256, so nfull = 512 puts two full blocks on every CU and
// at most one half block more, instead of a third full block on some CUs. hfirst = 0: workgroups
// below nfull are the full blocks; hfirst = 1: the half blocks come first, so their loads lead
// their CUs' queues (at M = 16 they otherwise issue behind two full blocks' rings and end the
// launch: gate_up 10.65 -> 10.52 us; at M = 1 they end with the full blocks either way).
template <int LAYOUT, int XK, int ALGO, int U, int AWC, int MT = 1>
__global__ __launch_bounds__(kMaxThreads) void k_gemv_fp8_swiglu_mixed(KRQ_FP8_KERNEL_PARAMS, int nfull, int hfirst) {
  const int nh = static_cast<int>(gridDim.x) - nfull, w = static_cast<int>(blockIdx.x);
  const int f = hfirst ? w - nh : w;  // full block index (< 0 or >= nfull: a half block)
  if (f >= 0 && f < nfull)
    gemv_fp8_body<MT, KRQ_OUT_SWIGLU, LAYOUT, XK, ALGO, U, 1, false, AWC>(x, xsc, xinv, x_per_row, w8, wsc, w_per_row,
                                                                         M, NO, K, kts, out, aux, FusedArgs{}, f);
  else
    gemv_fp8_body<MT, kOutSwiGluHalf, LAYOUT, XK, ALGO, U, 1, false, AWC>(x, xsc, xinv, x_per_row, w8, wsc, w_per_row,
                                                                         M, NO, K, kts, out, aux, FusedArgs{},
                                                                         2 * (int64_t)nfull + (hfirst ? w : w - nfull));
}

// The chained FP8 MLP at M = 1 (krq_mlp_chain_fp8): act = SwiGLU(x . Wgu^T) and the split-K
// partials of act . Wd^T in one launch. Workgroups below nfull are gate_up's two-matrix blocks and
// those up to fa.n_first its half-pair blocks (k_gemv_fp8_swiglu_mixed's plan); the rest are
// down's blocks, pair p = w - fa.n_first (row block p % nrb2, split p / nrb2), which issue their
// weight ring and then wait for act (activation_wave<..., CH>). Workgroups are dispatched in index
// order, so every first-stage block has a slot before any second-stage block waits. The block has
// NWG weight waves and the activation wave; a second-stage block uses NWD <= NWG weight waves and
// its waves past the activation wave end at once (a barrier waits for the surviving waves only).
template <int UG, int AWG, int UD, int AWD, int NWG, int NWD>
__global__ __launch_bounds__(kMaxThreads) void k_mlp_chain_fp8(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ wgu, const float* __restrict__ gsc, int g_per_row,
    const uint8_t* __restrict__ wd, const float* __restrict__ dsc, int d_per_row, int64_t I, int64_t H, int kts_g,
    int kts_d, int nfull, int nrb2, uint16_t* __restrict__ act, float* __restrict__ part, FusedArgs fa) {
  static_assert(NWD <= NWG, "the block holds the second stage's waves");
  const int w = static_cast<int>(blockIdx.x);
  if (w < nfull) {
    gemv_fp8_body<1, KRQ_OUT_SWIGLU, KRQ_W_TILED, KRQ_X_BF16_DYN, 1, UG, 1, false, AWG, true>(
        x, nullptr, nullptr, 0, wgu, gsc, g_per_row, 1, I, H, kts_g, act, nullptr, fa, w, 0, NWG);
  } else if (w < fa.n_first) {
    gemv_fp8_body<1, kOutSwiGluHalf, KRQ_W_TILED, KRQ_X_BF16_DYN, 1, UG, 1, false, AWG, true>(
        x, nullptr, nullptr, 0, wgu, gsc, g_per_row, 1, I, H, kts_g, act, nullptr, fa, (int64_t)w + nfull, 0, NWG);
  } else {
    if (__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)) > NWD) return;
    const int p = w - fa.n_first;
    gemv_fp8_body<1, KRQ_OUT_PARTIAL, KRQ_W_TILED, KRQ_X_BF16_DYN, 1, UD, 1, false, AWD, true>(
        reinterpret_cast<const uint8_t*>(act), nullptr, nullptr, 0, wd, dsc, d_per_row, 1, H, I, kts_d, part, nullptr,
        fa, p % nrb2, p / nrb2, NWD);
  }
}

// the fused kernel (fused_fp8.hip): RMSNorm prologue and / or residual epilogue
template <int MT, int MODE, int LAYOUT, int XK, int ALGO, int U, bool NORM, int AWC>
__global__ __launch_bounds__(kMaxThreads) void k_gemv_fp8_fused(KRQ_FP8_KERNEL_PARAMS, FusedArgs fa) {
  gemv_fp8_body<MT, MODE, LAYOUT, XK, ALGO, U, 1, NORM, AWC>(x, xsc, xinv, x_per_row, w8, wsc, w_per_row, M, NO,
                                                             K, kts, out, aux, fa, blockIdx.x);
}


// The fused kernel's SwiGLU with its last column blocks split in half (as k_gemv_fp8_swiglu_mixed).
template <int LAYOUT, int XK, int U, bool NORM, int AWC>
__global__ __launch_bounds__(kMaxThreads) void k_gemv_fp8_fused_swiglu_mixed(KRQ_FP8_KERNEL_PARAMS, FusedArgs fa,
                                                                            int nfull) {
  if (static_cast<int>(blockIdx.x) < nfull)
    gemv_fp8_body<1, KRQ_OUT_SWIGLU, LAYOUT, XK, 1, U, 1, NORM, AWC>(x, xsc, xinv, x_per_row, w8, wsc, w_per_row, M,
                                                                     NO, K, kts, out, aux, fa, blockIdx.x);
  else
    gemv_fp8_body<1, kOutSwiGluHalf, LAYOUT, XK, 1, U, 1, NORM, AWC>(x, xsc, xinv, x_per_row, w8, wsc, w_per_row, M,
                                                                     NO, K, kts, out, aux, fa,
                                                                     (int64_t)blockIdx.x + nfull);
}

}  // namespace
