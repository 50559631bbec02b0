// BF16 skinny GEMM / GEMV (M <= 32): y = x . w^T in fp32. Weights row-major, or tiled: the FP8
// tile permutation of include/krq.h applied to the [N, 2K] byte matrix (16 rows x 32 bf16).
// A step is 64 bf16 of K per weight row (two 32-element tiles, one v_mfma_f32_16x16x32_bf16 each);
// M == 1 runs on the vector ALUs with cross-lane sums. Conventions: gemv_common.h.
#include "gemv_common.h"

#include <stdlib.h>

#include <algorithm>

using namespace krq;

namespace {

// PB = 2 or 4: adjacent row blocks per block sharing the activation loads (as in gemv_fp8.hip;
// 4 for the multi-row lm_head, where every 16-column block re-reads the bf16 rows from L2).
// bx: the column block this workgroup owns (its two-matrix, paired or single row block, or with
// MODE kOutSwiGluHalf its half-pair block).
// CHAIN (the chained BF16 MLP, k_mlp_chain_bf16): a SwiGLU block writes act through to memory and
// counts itself into the first-stage counters; a split-K (partials) block is a second-stage block
// on act, which issues its weight loads, waits for the first stage's done flag (chain_wait; a wait
// that gives up makes the block's partials NaN) and then reads act with agent-scope (sc1) loads,
// and counts its exit. sy >= 0 / nwo > 0: the block's K split and its wave count, given (the
// chained kernel's one-dimensional grid and common block size); waves past nwo end at once.
template <int MT, int MODE, int LAYOUT, int ALGO, int U, int PB, bool CHAIN = false>
KRQ_DEV void gemv_bf16_body(const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int64_t NO,
                            int64_t K, int kts, void* __restrict__ out, void* __restrict__ aux, int64_t bx,
                            int sy = -1, int nwo = 0, const FusedArgs* fa = nullptr) {
  extern __shared__ __align__(16) float red[];
  __shared__ float ones[32];
  static_assert(PB == 1 || (MODE != KRQ_OUT_SWIGLU && ALGO != 2), "paired row blocks: MFMA, no SwiGLU");
  static_assert(PB == 1 || PB == 2 || PB == 4, "one, two or four row blocks per block");
  static_assert(!CHAIN || (PB == 1 && (MODE == KRQ_OUT_SWIGLU || MODE == kOutSwiGluHalf || MODE == KRQ_OUT_PARTIAL)),
                "chained MLP: SwiGLU first stage, partials second stage");
  constexpr bool WAITS = CHAIN && MODE == KRQ_OUT_PARTIAL;  // (second stage)
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : PB;  // weight row blocks streamed per step
  constexpr int NV = MT * 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = nwo > 0 ? nwo : blockDim.x >> 6;
  if (CHAIN && __builtin_amdgcn_readfirstlane(wave) >= nw) return;
  const int r = lane & 15, g = lane >> 4;
  const int64_t rb = bx * PB;
  const int sidx = sy >= 0 ? sy : static_cast<int>(blockIdx.y);
  const int nsteps = (kts + 1) >> 1;
  const int64_t tbase = (int64_t)sidx * kts;
  const int64_t rowb = 2 * K;
  const int jcount = wave < nsteps ? (nsteps - wave + nw - 1) / nw : 0;
  if (threadIdx.x < 32) ones[threadIdx.x] = 1.0f;
  // weight set p: the up half of the SwiGLU, else the p-th row block of this block
  auto rbp = [&](int p) -> int64_t { return MODE == KRQ_OUT_SWIGLU && p == 1 ? rb + (NO >> 4) : rb + p; };

  v4f acc[P][MT];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[p][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  float sv[P][2];  // vector-ALU partial sums (ALGO 2) of the low and high tile of each step
#pragma unroll
  for (int p = 0; p < P; ++p) sv[p][0] = sv[p][1] = 0.f;
  // a ring of U step slots: consume slot u (step cc), then refill it with step cc + U
  uint4 wl[P][U], wh[P][U], xl[U][MT], xh[U][MT];
  // Every slot load is issued unconditionally (a branch around a load makes the compiler drain all
  // outstanding loads at the join): a slot past this wave's last step reloads that step (already
  // in flight or cached) and is masked where consumed; rows m >= M read row M - 1, whose products
  // land in accumulator rows the epilogue never writes.
  // (WAITS: act, written in this launch on every XCD, read with sc1 loads through a buffer resource)
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(x), (short)0, WAITS ? static_cast<int>(M * rowb) : 0, 0x00020000);
  auto load_w = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const int64_t t0 = tbase + 2 * j;
    const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
    if constexpr (MODE == kOutSwiGluHalf) {
      wl[0][u] = ld16nt(w_addr_hp<LAYOUT>(w, rb, NO, t0, rowb, lane));
      wh[0][u] = ld16nt(w_addr_hp<LAYOUT>(w, rb, NO, t1, rowb, lane));
    } else {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        wl[p][u] = ld16nt(w_addr<LAYOUT>(w, rbp(p), t0, rowb, lane));
        wh[p][u] = ld16nt(w_addr<LAYOUT>(w, rbp(p), t1, rowb, lane));
      }
    }
  };
  auto load_x = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const int64_t t0 = tbase + 2 * j;
    const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = ALGO == 2 ? 0 : min(mt * 16 + r, M - 1);
      if constexpr (WAITS) {
        const int o = static_cast<int>((int64_t)m * rowb + g * 16);
        xl[u][mt] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, o + static_cast<int>(t0 * 64), 0, 16));
        xh[u][mt] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, o + static_cast<int>(t1 * 64), 0, 16));
      } else {
        const uint8_t* xr = x + (int64_t)m * rowb + g * 16;
        xl[u][mt] = ld16(xr + t0 * 64);
        xh[u][mt] = ld16(xr + t1 * 64);
      }
    }
  };
  auto load_slot = [&](int u, int cc) {
    load_w(u, cc);
    load_x(u, cc);
  };
  auto consume_slot = [&](int u, int cc) {
    const int j = jcount > 0 ? wave + min(cc, jcount - 1) * nw : 0;
    const bool ok = cc < jcount, hi = ok && (2 * j + 1 < kts);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint4 bl = sel4(ok, wl[p][u]), bh = sel4(hi, wh[p][u]);
      if (ALGO == 2) {
        sv[p][0] = dot8_bf16(bl, xl[u][0], sv[p][0]);
        sv[p][1] = dot8_bf16(bh, xh[u][0], sv[p][1]);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[p][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xl[u][mt]), as_v8bf(bl), acc[p][mt], 0, 0, 0);
          acc[p][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xh[u][mt]), as_v8bf(bh), acc[p][mt], 0, 0, 0);
        }
      }
    }
  };
  bool chain_bad = false;
  if constexpr (WAITS) {  // the weights first, then the wait, then act
#pragma unroll
    for (int u = 0; u < U; ++u) load_w(u, u);
    chain_bad = !chain_wait(*fa);
#pragma unroll
    for (int u = 0; u < U; ++u) load_x(u, u);
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) load_slot(u, u);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the last batch is peeled off (consume only), so no load sits behind a branch and the first
  // batch's loads stay ahead of everything else
  int base = 0;
  if constexpr (WAITS) {
    // One batch peeled off, unconditionally (past jcount it reloads the last step and consumes
    // nothing): the first batch's loads went out weights first, act after the wait, and a loop
    // entered with them in that order waits for every load on its first pass.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      consume_slot(u, u);
      load_slot(u, u + U);
    }
    base = U;
  }
  // One-row single-matrix blocks pin each slot's refill right behind its products: left to itself
  // the compiler moves the batch's loads to its end and waits for the whole ring on every pass.
  // Measured (M = 1, split 1, graph-timed, two alternating runs on one box): QKV 9.37 -> 8.75 us,
  // O 8.35 -> 6.89, the BF16 lm_head 125.5 -> 122.6, down (split 4) and gate_up unchanged within
  // the runs' spread; pinning every slot of the two-matrix SwiGLU block and of the matrix-core
  // rings (M > 1) as well measured slower (gate_up 18.5 -> 19.8 us, M = 16 lm_head 139 -> 152).
  constexpr bool PIN = ALGO == 2 && P == 1;
  for (; base + U < jcount; base += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      consume_slot(u, base + u);
      load_slot(u, base + u + U);
      if constexpr (PIN) __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) consume_slot(u, base + u);
  if (ALGO == 2) {
    // the four lanes of row r (g = 0..3) hold partial sums of disjoint k: add them; lanes 0..15
    // then carry columns 16 rb + lane in MFMA slot (mt 0, i 0), i.e. output row m = 0
#pragma unroll
    for (int p = 0; p < P; ++p) {
      float a = sv[p][0] + sv[p][1];
      a += __shfl_xor(a, 16, kWave);
      a += __shfl_xor(a, 32, kWave);
      acc[p][0] = v4f{g == 0 ? a : 0.f, 0.f, 0.f, 0.f};
    }
  }
  if (WAITS && chain_bad) {  // (the wait gave up: every partial of the block is NaN)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[p][mt] = v4f{NAN, NAN, NAN, NAN};
  }
  // the P accumulator sets of each wave, in the layout epilogue() reads
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(wave * P + p) * NV + mt * 256 + i * 64 + lane] = acc[p][mt][i];
  __syncthreads();
  if (MODE == KRQ_OUT_SWIGLU) {
    epilogue<MT, MODE, P, CHAIN>(red, 0, nw, M, NO, rb, sidx, ones, ColScales{1.0f, 1.0f}, out, aux,
                                 CHAIN ? nw * kWave : 0);
  } else {
#pragma unroll
    for (int p = 0; p < PB; ++p)
      epilogue<MT, MODE, P, CHAIN>(red, p, nw, M, NO, rb + p, sidx, ones, ColScales{1.0f, 1.0f}, out, aux,
                                   CHAIN ? nw * kWave : 0);
  }
  if constexpr (CHAIN) chain_tail<!WAITS>(*fa);
}

template <int MT, int MODE, int LAYOUT, int ALGO, int U, int PB>
__global__ __launch_bounds__(512) void k_gemv_bf16(const uint8_t* __restrict__ x,
                                                  const uint8_t* __restrict__ w, int M, int64_t NO,
                                                  int64_t K, int kts, void* __restrict__ out,
                                                  void* __restrict__ aux) {
  gemv_bf16_body<MT, MODE, LAYOUT, ALGO, U, PB>(x, w, M, NO, K, kts, out, aux, blockIdx.x);
}

// The SwiGLU with its last column blocks split in half, as k_gemv_fp8_swiglu_mixed: workgroups
// below nfull are two-matrix blocks, workgroup nfull + j is half-pair block 2 nfull + j (the same
// steps per wave, so the same output bits).
template <int LAYOUT, int ALGO, int U>
__global__ __launch_bounds__(512) void k_gemv_bf16_swiglu_mixed(const uint8_t* __restrict__ x,
                                                               const uint8_t* __restrict__ w, int M, int64_t NO,
                                                               int64_t K, int kts, void* __restrict__ out,
                                                               void* __restrict__ aux, int nfull) {
  if (static_cast<int>(blockIdx.x) < nfull)
    gemv_bf16_body<1, KRQ_OUT_SWIGLU, LAYOUT, ALGO, U, 1>(x, w, M, NO, K, kts, out, aux, blockIdx.x);
  else
    gemv_bf16_body<1, kOutSwiGluHalf, LAYOUT, ALGO, U, 1>(x, w, M, NO, K, kts, out, aux,
                                                          (int64_t)blockIdx.x + nfull);
}

// The chained BF16 MLP (krq_mlp_chain_bf16): act = SwiGLU(x . Wgu^T) and the split-K partials of
// act . Wd^T in one launch. Workgroups below fa.n_first are the SwiGLU launch's blocks (two-matrix
// blocks below nfull, then half-pair blocks, as k_gemv_bf16_swiglu_mixed, when MT == 1), with
// NWG waves; the rest are the down launch's blocks with NWD waves, block p at row block p % nrb2
// of K split p / nrb2. Each stage keeps the standalone launch's plan, so act and the partials are
// those of the two launches, bit for bit. The block holds max(NWG, NWD) waves; the waves a stage
// does not use end at once (a barrier waits only for the waves that have not ended).
template <int MT, int LAYOUT, int ALGO, int U>
__global__ __launch_bounds__(512) void k_mlp_chain_bf16(const uint8_t* __restrict__ x, const uint8_t* __restrict__ wgu,
                                                       const uint8_t* __restrict__ wd, int M, int64_t I, int64_t H,
                                                       int kts_g, int kts_d, int nfull, int nrb2, int nwg, int nwd,
                                                       uint16_t* __restrict__ act, float* __restrict__ part,
                                                       FusedArgs fa) {
  const int w = static_cast<int>(blockIdx.x);
  if (w < nfull) {
    gemv_bf16_body<MT, KRQ_OUT_SWIGLU, LAYOUT, ALGO, U, 1, true>(x, wgu, M, I, H, kts_g, act, nullptr, w, 0, nwg, &fa);
  } else if (w < fa.n_first) {
    if constexpr (MT == 1)
      gemv_bf16_body<1, kOutSwiGluHalf, LAYOUT, ALGO, U, 1, true>(x, wgu, M, I, H, kts_g, act, nullptr,
                                                                  (int64_t)w + nfull, 0, nwg, &fa);
  } else {
    const int p = w - fa.n_first;
    gemv_bf16_body<MT, KRQ_OUT_PARTIAL, LAYOUT, ALGO, U, 1, true>(reinterpret_cast<const uint8_t*>(act), wd, M, H, I,
                                                                  kts_d, part, nullptr, p % nrb2, p / nrb2, nwd, &fa);
  }
}

// Persistent row partition (the reference's gemv_rows, engine/kernels/gemv.py:270-348): exactly
// G = gridDim.x workgroups; workgroup p owns output rows [p N / G, (p + 1) N / G) over the full K
// and walks them in 16-row chunks, chunk c to wave c mod nw. A chunk streams its rows' whole K
// through a ring of U step slots on the BF16 matrix cores (row-major weights: a chunk may start
// on any row) and writes the rows it owns straight from its accumulators; lanes of rows past the
// workgroup's range reload its last row and store nothing. One wave sums each output row, in one
// order, so the result does not depend on G. P = 2 (SwiGLU): gate rows n, up rows N + n of the
// [2N, K] matrix, bf16(bf16(silu(bf16 g)) * bf16 u) as gemv.py:125-130.
template <int MT, int P, int U>
__global__ __launch_bounds__(512) void k_gemv_bf16_rows(const uint8_t* __restrict__ x,
                                                       const uint8_t* __restrict__ w, int M, int64_t N,
                                                       int64_t K, void* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t G = gridDim.x, pid = blockIdx.x;
  const int64_t r0 = pid * N / G, r1 = (pid + 1) * N / G;
  const int64_t rowb = 2 * K;
  const int kts = static_cast<int>(K >> 5);  // 64-byte (32-element) tiles of a row
  const int nsteps = (kts + 1) >> 1;
  const int64_t nchunks = (r1 - r0 + 15) >> 4;
  const uint8_t* xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xr[mt] = x + (int64_t)min(mt * 16 + r, M - 1) * rowb + g * 16;
  for (int64_t c = wave; c < nchunks; c += nw) {
    const int64_t n0 = r0 + 16 * c, nrow = min(n0 + r, r1 - 1);
    const uint8_t* wg = w + nrow * rowb + g * 16;
    const uint8_t* wu = w + (N + nrow) * rowb + g * 16;  // (P == 2)
    v4f acc[MT], accu[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      accu[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    uint4 wl[U], wh[U], ul[U], uh[U], xl[U][MT], xh[U][MT];
    // every slot load is issued (a slot past the last step reloads it and is masked where consumed)
    auto load_slot = [&](int u, int cc) {
      const int j = min(cc, nsteps - 1);
      const int64_t t0 = 2 * j, t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
      wl[u] = ld16nt(wg + t0 * 64);
      wh[u] = ld16nt(wg + t1 * 64);
      if (P == 2) {
        ul[u] = ld16nt(wu + t0 * 64);
        uh[u] = ld16nt(wu + t1 * 64);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xl[u][mt] = ld16(xr[mt] + t0 * 64);
        xh[u][mt] = ld16(xr[mt] + t1 * 64);
      }
    };
    auto consume_slot = [&](int u, int cc) {
      const int j = min(cc, nsteps - 1);
      const bool ok = cc < nsteps, hi = ok && (2 * j + 1 < kts);
      const uint4 bl = sel4(ok, wl[u]), bh = sel4(hi, wh[u]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xl[u][mt]), as_v8bf(bl), acc[mt], 0, 0, 0);
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xh[u][mt]), as_v8bf(bh), acc[mt], 0, 0, 0);
      }
      if (P == 2) {
        const uint4 cl = sel4(ok, ul[u]), ch = sel4(hi, uh[u]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xl[u][mt]), as_v8bf(cl), accu[mt], 0, 0, 0);
          accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xh[u][mt]), as_v8bf(ch), accu[mt], 0, 0, 0);
        }
      }
    };
#pragma unroll
    for (int u = 0; u < U; ++u) load_slot(u, u);
    __builtin_amdgcn_sched_barrier(0);
    int base = 0;
    for (; base + U < nsteps; base += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        consume_slot(u, base + u);
        load_slot(u, base + u + U);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) consume_slot(u, base + u);
    // lane (g, r), element i of tile mt: output row m = 16 mt + 4 g + i, column n0 + r
    const int64_t n = n0 + r;
    if (n < r1) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mt * 16 + 4 * g + i;
          if (m >= M) continue;
          uint16_t y;
          if (P == 2) {
            const float gg = round_bf16(acc[mt][i]), uu = round_bf16(accu[mt][i]);
            const float sl = round_bf16(gg / (1.0f + expf(-gg)));
            y = f32_to_bf16(sl * uu);
          } else {
            y = f32_to_bf16(acc[mt][i]);
          }
          reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = y;
        }
    }
  }
}

template <int MODE, int LAYOUT>
void launch(int M, int pb, dim3 grid, int nw, size_t smem, hipStream_t s, const uint8_t* x,
            const uint8_t* w, int m, int64_t NO, int64_t K, int kts, void* out, void* aux) {
  const dim3 block(nw * 64);
  constexpr int PB2 = MODE == KRQ_OUT_SWIGLU ? 1 : 2;
  constexpr int PB4 = MODE == kOutArgmax ? 4 : 1;  // (pb is 4 only for the argmax epilogue)
  if (M == 1)
    hipLaunchKernelGGL((k_gemv_bf16<1, MODE, LAYOUT, 2, 4, 1>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
  else if (M <= 4)
    hipLaunchKernelGGL((k_gemv_bf16<1, MODE, LAYOUT, 1, 4, 1>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
  else if (M <= 16 && pb == 4)
    hipLaunchKernelGGL((k_gemv_bf16<1, MODE, LAYOUT, 1, 2, PB4>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
  else if (M <= 16 && pb == 2)
    hipLaunchKernelGGL((k_gemv_bf16<1, MODE, LAYOUT, 1, 2, PB2>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
  else if (M <= 16)
    hipLaunchKernelGGL((k_gemv_bf16<1, MODE, LAYOUT, 1, 2, 1>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
  else if (pb == 2)
    hipLaunchKernelGGL((k_gemv_bf16<2, MODE, LAYOUT, 1, 2, PB2>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
  else
    hipLaunchKernelGGL((k_gemv_bf16<2, MODE, LAYOUT, 1, 2, 1>), grid, block, smem, s, x, w, m, NO, K, kts, out, aux);
}

template <int MODE>
void launch_layout(int layout, int M, int pb, dim3 grid, int nw, size_t smem, hipStream_t s, const uint8_t* x,
                   const uint8_t* w, int m, int64_t NO, int64_t K, int kts, void* out, void* aux) {
  if (layout == KRQ_W_TILED)
    launch<MODE, KRQ_W_TILED>(M, pb, grid, nw, smem, s, x, w, m, NO, K, kts, out, aux);
  else
    launch<MODE, KRQ_W_ROWMAJOR>(M, pb, grid, nw, smem, s, x, w, m, NO, K, kts, out, aux);
}

constexpr int64_t kCUs = 256;  // compute units of the MI355X (workgroup b runs on CU b mod 256)

// k_gemv_bf16_swiglu_mixed for M <= 16 when the SwiGLU's column blocks number a little over a
// multiple of the CUs (gate_up: 608 = 2 x 256 + 96), with the variant launch() would pick; false
// otherwise.
bool launch_swiglu_mixed(int layout, int M, int64_t NO, int nw, size_t smem, hipStream_t s, const uint8_t* x,
                         const uint8_t* w, int64_t K, int kts, void* out) {
  const int64_t nrbs = NO / 16, rem = nrbs % kCUs;
  if (M > 16 || nrbs <= 2 * kCUs || rem == 0 || 2 * rem > kCUs) return false;
  const int nfull = static_cast<int>(nrbs - rem);
  const dim3 grid(static_cast<unsigned>(nfull + 2 * rem), 1), block(nw * 64);
#define KRQ_BF16_MIXED(LAYOUT)                                                                                   \
  if (M == 1)                                                                                                    \
    hipLaunchKernelGGL((k_gemv_bf16_swiglu_mixed<LAYOUT, 2, 4>), grid, block, smem, s, x, w, M, NO, K, kts, out, \
                       nullptr, nfull);                                                                          \
  else if (M <= 4)                                                                                               \
    hipLaunchKernelGGL((k_gemv_bf16_swiglu_mixed<LAYOUT, 1, 4>), grid, block, smem, s, x, w, M, NO, K, kts, out, \
                       nullptr, nfull);                                                                          \
  else                                                                                                           \
    hipLaunchKernelGGL((k_gemv_bf16_swiglu_mixed<LAYOUT, 1, 2>), grid, block, smem, s, x, w, M, NO, K, kts, out, \
                       nullptr, nfull);
  if (layout == KRQ_W_TILED) {
    KRQ_BF16_MIXED(KRQ_W_TILED)
  } else {
    KRQ_BF16_MIXED(KRQ_W_ROWMAJOR)
  }
#undef KRQ_BF16_MIXED
  return true;
}

}  // namespace

int krq::gemv_bf16_run(const void* x, const void* w, int w_layout, int64_t M, int64_t N, int64_t K,
                       int split, int mode, void* out, void* aux, void* stream) {
  KRQ_REQUIRE(x && w && (out || mode == kOutArgmax) && (aux || mode != kOutArgmax),
              "gemv_bf16: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w), "gemv_bf16: x and w must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_bf16: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(N > 0 && K > 0 && split >= 1, "gemv_bf16: bad shape N=%lld K=%lld split=%d",
              (long long)N, (long long)K, split);
  KRQ_REQUIRE(K % split == 0 && (K / split) % 32 == 0,
              "gemv_bf16: no tiling divides K_SPLIT (K=%lld split=%d; K/split must be a multiple of 32)",
              (long long)K, split);
  KRQ_REQUIRE(mode >= KRQ_OUT_BF16 && mode <= kOutArgmax, "gemv_bf16: bad mode %d", mode);
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "gemv_bf16: bad layout %d", w_layout);
  KRQ_REQUIRE(mode == KRQ_OUT_PARTIAL || split == 1, "gemv_bf16: split %d needs the partials output", split);
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  KRQ_REQUIRE(NO % 16 == 0 && (mode != KRQ_OUT_SWIGLU || N % 2 == 0),
              "gemv_bf16: no tiling divides N=%lld (output columns must be a multiple of 16)", (long long)N);
  KRQ_REQUIRE(NO / 16 <= 0x7fffffff && split <= 65535, "gemv_bf16: grid too large");
  const int kts = static_cast<int>(K / split / 32);
  // paired only where halving the blocks still leaves thousands (the lm_head), as in gemv_fp8.hip;
  // the lm_head's argmax launch at 4 < M <= 16 takes four row blocks per block
  int pb = (mode != KRQ_OUT_SWIGLU && M > 4 && (NO / 16) % 2 == 0 &&
            (NO / 16) * split >= 4096) ? 2 : 1;
  if (pb == 2 && mode == kOutArgmax && M <= 16 && (NO / 16) % 4 == 0) pb = 4;
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : pb;
  const int MT = M <= 16 ? 1 : 2;
  const int nw = plan_waves((kts + 1) / 2, P, M <= 4 ? 4 : 2, NO / 16 / pb * split);  // U of launch()'s variant
  const size_t smem = (size_t)nw * P * MT * 256 * sizeof(float);
  const dim3 grid(static_cast<unsigned>(NO / 16 / pb), static_cast<unsigned>(split));
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w;
  const int m = static_cast<int>(M);
  hipStream_t s = (hipStream_t)stream;
  if (mode == KRQ_OUT_BF16) launch_layout<KRQ_OUT_BF16>(w_layout, m, pb, grid, nw, smem, s, xb, wb, m, NO, K, kts, out, aux);
  else if (mode == KRQ_OUT_PARTIAL) launch_layout<KRQ_OUT_PARTIAL>(w_layout, m, pb, grid, nw, smem, s, xb, wb, m, NO, K, kts, out, aux);
  else if (mode == KRQ_OUT_SWIGLU && launch_swiglu_mixed(w_layout, m, NO, nw, smem, s, xb, wb, K, kts, out))
    ;  // the mixed launch below 17 rows on grids a little over a multiple of the CUs
  else if (mode == KRQ_OUT_SWIGLU) launch_layout<KRQ_OUT_SWIGLU>(w_layout, m, pb, grid, nw, smem, s, xb, wb, m, NO, K, kts, out, aux);
  else launch_layout<kOutArgmax>(w_layout, m, pb, grid, nw, smem, s, xb, wb, m, NO, K, kts, out, aux);
  return krq_check_launch("gemv_bf16");
}

extern "C" int krq_gemv_bf16(const void* x, const void* w, int w_layout, int64_t M, int64_t N, int64_t K,
                             int split, int mode, void* out, void* stream) {
  KRQ_REQUIRE(mode >= KRQ_OUT_BF16 && mode <= KRQ_OUT_SWIGLU, "gemv_bf16: bad mode %d", mode);
  return gemv_bf16_run(x, w, w_layout, M, N, K, split, mode, out, nullptr, stream);
}

extern "C" int krq_gemv_bf16_rows(const void* x, const void* w, int64_t M, int64_t N, int64_t K, int programs,
                                  int swiglu, void* out, void* stream) {
  KRQ_REQUIRE(x && w && out, "gemv_rows: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w), "gemv_rows: x and w must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_rows: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(N > 0 && K > 0 && K % 32 == 0,
              "gemv_rows: bad shape N=%lld K=%lld (K must be a positive multiple of 32)", (long long)N,
              (long long)K);
  KRQ_REQUIRE(programs >= 1, "gemv_rows: programs=%d must be at least 1", programs);
  KRQ_REQUIRE(N <= 0x3fffffffffffll / programs, "gemv_rows: N=%lld too large", (long long)N);
  // waves: the most 16-row chunks any workgroup owns (at most 8; more chunks loop)
  const int64_t maxrows = (N + programs - 1) / programs;
  const int nw = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(8, (maxrows + 15) / 16)));
  const dim3 grid(static_cast<unsigned>(programs)), block(nw * 64);
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w;
  const int m = static_cast<int>(M);
  hipStream_t s = (hipStream_t)stream;
  if (swiglu) {
    if (M <= 16)
      hipLaunchKernelGGL((k_gemv_bf16_rows<1, 2, 4>), grid, block, 0, s, xb, wb, m, N, K, out);
    else
      hipLaunchKernelGGL((k_gemv_bf16_rows<2, 2, 4>), grid, block, 0, s, xb, wb, m, N, K, out);
  } else {
    if (M <= 16)
      hipLaunchKernelGGL((k_gemv_bf16_rows<1, 1, 4>), grid, block, 0, s, xb, wb, m, N, K, out);
    else
      hipLaunchKernelGGL((k_gemv_bf16_rows<2, 1, 4>), grid, block, 0, s, xb, wb, m, N, K, out);
  }
  return krq_check_launch("gemv_rows");
}

// The chained BF16 MLP (k_mlp_chain_bf16): both stages of the decode MLP in one launch, each with
// the plan krq_gemv_bf16 gives it (the SwiGLU launch and the split-K partials launch).
extern "C" int krq_mlp_chain_bf16(const void* x, const void* w_gu, const void* w_down, int w_layout, int64_t M,
                                  int64_t H, int64_t I, int split, void* act, uint32_t* ctl, uint32_t max_polls,
                                  void* out, void* stream) {
  KRQ_REQUIRE(x && w_gu && w_down && act && ctl && out, "mlp_chain_bf16: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w_gu) && aligned16(w_down) && aligned16(act),
              "mlp_chain_bf16: x, weights and act must be 16-byte aligned");
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "mlp_chain_bf16: bad layout %d", w_layout);
  KRQ_REQUIRE(M >= 1 && M <= 32, "mlp_chain_bf16: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(H > 0 && I > 0 && H % 32 == 0 && I % 16 == 0 && split >= 1 && I % split == 0 &&
                  (I / split) % 32 == 0,
              "mlp_chain_bf16: shape H=%lld I=%lld split=%d (H and I/split multiples of 32, I of 16)",
              (long long)H, (long long)I, split);
  KRQ_REQUIRE(M * 2 * I <= 0x7fffffff && I / 16 <= 0x7fffffff && split <= 65535,
              "mlp_chain_bf16: shape too large");
  KRQ_REQUIRE(max_polls > 0, "mlp_chain_bf16: max_polls must be positive");
  const int64_t nrb2 = H / 16, n_second = nrb2 * split;
  // the down launch pairs row blocks on grids of thousands of blocks above 4 rows; the chained
  // kernel keeps one row block per block, so it takes only the unpaired plan
  KRQ_REQUIRE(!(M > 4 && nrb2 % 2 == 0 && n_second >= 4096),
              "mlp_chain_bf16: %lld down blocks at M=%lld (the chained form takes fewer than 4096 above 4 rows)",
              (long long)n_second, (long long)M);
  const int U = M <= 4 ? 4 : 2, MT = M <= 16 ? 1 : 2;  // (launch()'s variant)
  const int kts_g = static_cast<int>(H / 32), kts_d = static_cast<int>(I / split / 32);
  // gate_up: the SwiGLU launch's plan (two-matrix blocks, the last ones as half-pair blocks)
  const int64_t nrbs = I / 16, rem = nrbs % kCUs;
  const bool mixed = M <= 16 && nrbs > 2 * kCUs && rem != 0 && 2 * rem <= kCUs;
  const int64_t nfull = mixed ? nrbs - rem : nrbs, n_first = mixed ? nfull + 2 * rem : nrbs;
  KRQ_REQUIRE(n_first + n_second <= 0x7fffffff, "mlp_chain_bf16: grid too large");
  const int nwg = plan_waves((kts_g + 1) / 2, 2, U, nrbs), nwd = plan_waves((kts_d + 1) / 2, 1, U, n_second);
  const int nwb = std::max(nwg, nwd);
  const size_t smem = std::max((size_t)nwg * 2, (size_t)nwd) * MT * 256 * sizeof(float);
  FusedArgs fa{};
  fa.cnt = ctl;
  fa.max_polls = max_polls;
  fa.n_first = static_cast<int>(n_first);
  fa.n_second = static_cast<int>(n_second);
  const dim3 grid(static_cast<unsigned>(n_first + n_second)), block(nwb * 64);
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* gb = (const uint8_t*)w_gu;
  const uint8_t* db = (const uint8_t*)w_down;
  const int m = static_cast<int>(M);
#define KRQ_CHAIN(MT_, LAYOUT, ALGO, U_)                                                                          \
  hipLaunchKernelGGL((k_mlp_chain_bf16<MT_, LAYOUT, ALGO, U_>), grid, block, smem, s, xb, gb, db, m, I, H, kts_g, \
                     kts_d, static_cast<int>(nfull), static_cast<int>(nrb2), nwg, nwd, (uint16_t*)act, (float*)out, fa)
#define KRQ_CHAIN_M(LAYOUT)                          \
  if (M == 1) KRQ_CHAIN(1, LAYOUT, 2, 4);            \
  else if (M <= 4) KRQ_CHAIN(1, LAYOUT, 1, 4);       \
  else if (M <= 16) KRQ_CHAIN(1, LAYOUT, 1, 2);      \
  else KRQ_CHAIN(2, LAYOUT, 1, 2);
  if (w_layout == KRQ_W_TILED) {
    KRQ_CHAIN_M(KRQ_W_TILED)
  } else {
    KRQ_CHAIN_M(KRQ_W_ROWMAJOR)
  }
#undef KRQ_CHAIN_M
#undef KRQ_CHAIN
  return krq_check_launch("mlp_chain_bf16");
}
