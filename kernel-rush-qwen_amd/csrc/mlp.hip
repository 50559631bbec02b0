// Fused decode MLP in one launch (M <= 32): act = SwiGLU(x . Wgu^T) as bf16 [M, I], then the fp32
// split-K partials of act . Wd^T, [S, M, H]. Reference: engine/kernels/mlp.py:22-118
// (PersistentMLP; used by engine/engine.py:906-935 and :1014-1015), here for per-channel FP8
// weights with per-token dynamic activation scales (the quantization of linear_fp8 /
// fp8.quant_rows applied to both GEMVs).
//
// Work items. Phase 1: the I/16 gate/up row blocks (16 SwiGLU columns over all of H each).
// Phase 2: (H/16) x S down items (16 output columns over one K split of I). Block b takes items
// b, b + G, ... of each phase (G blocks, at most as many as the device holds at once, so every
// block a waiting block depends on is running). The down input's per-token scale needs the amax
// of whole act rows, so phase 2 waits for all of phase 1 - but each phase-2 item issues its
// weight loads before it waits, so the down weights stream while phase 1 drains.
//
// Synchronization. Device-scope atomics on one address serialize (~12 ns each, measured), so a
// block publishes once, after its phase-1 items: the running amax of its act rows (atomic max)
// and a count (atomic add), both into one of kGroups groups of control words 256 bytes apart;
// a waiting block polls the kGroups counters and takes the max over the kGroups amax copies.
// act, the amax copies and the counters move with agent-scope relaxed atomics: their stores
// write through to memory and their loads read memory from every XCD; a producer waits for its
// stores to complete before it publishes. No cache writeback or invalidate is needed. The last
// block out (counted per group, then over groups) zeroes the control words again, so graph
// replays need no host reset. A wait is bounded: past max_polls polls (kSpinLimit by default) the
// block sets the error word and goes on with NaN activation scales, so the kernel ends even if the
// device could not hold all G blocks, and every partial that block writes is NaN: a launch whose
// co-residency assumption failed cannot pass as data. (act is complete either way: phase 1 never
// waits.)
#include "gemv_common.h"

#include <stdlib.h>

#include <algorithm>

using namespace krq;

namespace {

// control words (uint32): kGroups groups of 64 words (256 bytes apart) {phase-1 count, exit
// count, amax bits [32]}, then a group of {exit count over groups, ..., error flag (last word)}
constexpr int kGroups = 8, kGroupWords = 64;
enum : int { kDone = 0, kExitG = 1, kAmax = 2, kTop = kGroups * kGroupWords, kExitTop = kTop,
             kCtlWords = kTop + kGroupWords, kErr = kCtlWords - 1 };
constexpr uint32_t kSpinLimit = 1u << 20;  // polls of the phase-1 counter (~1 s) before flagging an error
constexpr int kXC = 4;                     // 16-byte x chunks per thread in the M == 1 prologue

template <int MT, int XK, int LAYOUT, int NW, int U1, int U2>
__global__ __launch_bounds__(NW * 64, 2) void k_mlp_fp8(
    const uint8_t* __restrict__ x, const float* __restrict__ xsc, const uint8_t* __restrict__ wgu,
    const float* __restrict__ gsc, int g_per_row, const uint8_t* __restrict__ wd,
    const float* __restrict__ dsc, int d_per_row, int M, int H, int I, int S, uint16_t* act,
    uint32_t* ctl, float* __restrict__ out, uint32_t max_polls) {
  extern __shared__ __align__(16) uint8_t lds[];  // red | xq1 (M == 1: H bytes) | xq2 (M*ks2)
  __shared__ float xs1[32], xs2[32], inv2[32];
  __shared__ uint32_t amax_w[NW];
  __shared__ uint32_t p1_bad;  // this block's phase-1 wait timed out
  __shared__ uint16_t act_s[32 * 16];
  constexpr int NT = NW * 64, NV = MT * 256;
  const int n1 = I >> 4, n2 = (H >> 4) * S;
  const int kts1 = H >> 6, nst1 = (kts1 + 1) >> 1;
  const int ks2 = I / S, kts2 = ks2 >> 6, nst2 = (kts2 + 1) >> 1;
  const int G = gridDim.x, grp = blockIdx.x % kGroups;
  float* red = reinterpret_cast<float*>(lds);
  uint8_t* xq1 = lds + NW * 2 * NV * sizeof(float);
  uint8_t* xq2 = xq1 + (XK == KRQ_X_BF16_DYN ? H : 0);
  bool have_x = false, p1_seen = false;
  uint32_t amax_loc = 0;  // threads m < M: running amax (mag_bits) of act row m over this block's items

  for (int t = blockIdx.x; t < n1; t += G) {
    // Lane coordinates are re-derived opaquely in every item: otherwise the compiler hoists the
    // per-slot offsets of both phases out of the item loops and keeps them all live (spills).
    int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    asm volatile("" : "+v"(lane));
    asm volatile("" : "+s"(wave));
    const int r = lane & 15, g = lane >> 4;
    {
      // ------------------------------ phase 1: gate/up row block rb ------------------------------
      const int64_t rb = t, rbu = rb + n1;
      const int jc = wave < nst1 ? (nst1 - wave + NW - 1) / NW : 0;
      const int col = (int)(rb * 16) + (threadIdx.x & 15);
      const float cg = gsc[g_per_row ? col : 0], cu = gsc[g_per_row ? I + col : 0];
      uint4 wl[U1], wh[U1], ul[U1], uh[U1], xl[U1][MT], xh[U1][MT];
      uint4 xv[kXC];
      if (XK == KRQ_X_BF16_DYN && !have_x) {
#pragma unroll
        for (int c = 0; c < kXC; ++c) {
          const int e = 8 * (threadIdx.x + c * NT);
          xv[c] = e < H ? ld16(x + 2 * (int64_t)e) : zero4();
        }
      }
      auto load1 = [&](int u, int cc) {
        const int j = wave + min(cc, jc - 1) * NW;
        const int64_t t0 = 2 * j, t1 = (2 * j + 1 < kts1) ? t0 + 1 : t0;
        wl[u] = ld16nt(w_addr<LAYOUT>(wgu, rb, t0, H, lane));
        wh[u] = ld16nt(w_addr<LAYOUT>(wgu, rb, t1, H, lane));
        ul[u] = ld16nt(w_addr<LAYOUT>(wgu, rbu, t0, H, lane));
        uh[u] = ld16nt(w_addr<LAYOUT>(wgu, rbu, t1, H, lane));
        if (XK == KRQ_X_FP8) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + r;
            uint4 lo = zero4(), hi = zero4();
            if (m < M) {
              const uint8_t* xr = x + (int64_t)m * H + g * 16;
              lo = ld16(xr + t0 * 64);
              hi = ld16(xr + t1 * 64);
            }
            xl[u][mt] = lo;
            xh[u][mt] = hi;
          }
        }
      };
      if (jc > 0) {
#pragma unroll
        for (int u = 0; u < U1; ++u) load1(u, u);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (!have_x) {
        if (XK == KRQ_X_BF16_DYN) {
          uint32_t am = 0;
#pragma unroll
          for (int c = 0; c < kXC; ++c) am = absmax8(xv[c], am);
          am = wave_max_u32(am);
          if (lane == 0) amax_w[wave] = am;
          __syncthreads();
          uint32_t ab = amax_w[0];
#pragma unroll
          for (int w = 1; w < NW; ++w) ab = umax32(ab, amax_w[w]);
          const float a = clamp_min_nan(as_f32(ab), 1e-6f);
          const float inv = inv_from_amax(a);
          if (threadIdx.x == 0) xs1[0] = scale_from_amax(a);
#pragma unroll
          for (int c = 0; c < kXC; ++c) {
            const int e = 8 * (threadIdx.x + c * NT);
            if (e < H) *reinterpret_cast<uint2*>(xq1 + e) = quant8(xv[c], inv);
          }
        } else if (threadIdx.x < (unsigned)M) {
          xs1[threadIdx.x] = xsc[threadIdx.x];
        }
        have_x = true;
        __syncthreads();
      }
      v4f acc[MT], accu[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
        accu[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      }
      auto consume1 = [&](int u, int cc) {
        const int j = wave + min(cc, jc - 1) * NW;
        const bool ok = cc < jc, hi = ok && (2 * j + 1 < kts1);
        if (XK == KRQ_X_BF16_DYN) {
          uint4 lo = zero4(), hh = zero4();
          if (r == 0) {
            lo = *reinterpret_cast<const uint4*>(xq1 + g * 16 + (2 * j) * 64);
            if (2 * j + 1 < kts1) hh = *reinterpret_cast<const uint4*>(xq1 + g * 16 + (2 * j + 1) * 64);
          }
          xl[u][0] = lo;
          xh[u][0] = hh;
        }
        const v8i B = pack_v8i(sel4(ok, wl[u]), sel4(hi, wh[u]));
        const v8i Bu = pack_v8i(sel4(ok, ul[u]), sel4(hi, uh[u]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const v8i A = pack_v8i(xl[u][mt], xh[u][mt]);
          acc[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[mt], 0, 0, 0, 0, 0, 0);
          accu[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, Bu, accu[mt], 0, 0, 0, 0, 0, 0);
        }
      };
      for (int base = 0; base < jc; base += U1) {
#pragma unroll
        for (int u = 0; u < U1; ++u) {
          consume1(u, base + u);
          if (base + u + U1 < jc) load1(u, base + u + U1);
        }
      }
      stash<MT, 2>(red, wave, lane, acc, accu);
      __syncthreads();
      // SwiGLU epilogue (rounding of engine/kernels/gemv.py:125-130), staged per row in LDS
      for (int v = threadIdx.x; v < NV; v += NT) {
        const int mt = v >> 8, i = (v >> 6) & 3, ln = v & 63;
        const int m = mt * 16 + 4 * (ln >> 4) + i;
        if (m >= M) continue;
        float a = 0.0f, au = 0.0f;
        for (int w = 0; w < NW; ++w) {
          a += red[(w * 2 + 0) * NV + v];
          au += red[(w * 2 + 1) * NV + v];
        }
        const float gg = round_bf16(a * xs1[m] * cg);
        const float uu = round_bf16(au * xs1[m] * cu);
        const float sl = round_bf16(gg / (1.0f + expf(-gg)));
        act_s[m * 16 + (ln & 15)] = f32_to_bf16(sl * uu);
      }
      __syncthreads();
      if (threadIdx.x < 4u * M) {
        const int m = threadIdx.x >> 2, q = threadIdx.x & 3;
        const uint64_t v = *reinterpret_cast<const uint64_t*>(&act_s[m * 16 + 4 * q]);
        cstore64(reinterpret_cast<uint64_t*>(act + (int64_t)m * I + rb * 16 + 4 * q), v);
      }
      if (threadIdx.x < (unsigned)M) {
#pragma unroll
        for (int c = 0; c < 16; ++c) amax_loc = umax32(amax_loc, mag_bits(bf16_to_f32(act_s[threadIdx.x * 16 + c])));
      }
      __syncthreads();  // red and act_s are rewritten by the next item
    }
  }
  // publish this block's phase 1 (every block counts, with or without items)
  if (threadIdx.x < (unsigned)M) cmax(&ctl[grp * kGroupWords + kAmax + threadIdx.x], amax_loc);
  stores_done();
  __syncthreads();
  if (threadIdx.x == 0) cadd(&ctl[grp * kGroupWords + kDone], 1u);

  for (int it = blockIdx.x; it < n2; it += G) {
    int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    asm volatile("" : "+v"(lane));
    asm volatile("" : "+s"(wave));
    const int r = lane & 15, g = lane >> 4;
    {
      // ------------------------- phase 2: down row block rb2, K split s -------------------------
      const int nrb2 = H >> 4;
      const int64_t rb2 = it % nrb2;
      const int s = it / nrb2;
      const int64_t tb2 = (int64_t)s * kts2;
      const int jc = wave < nst2 ? (nst2 - wave + NW - 1) / NW : 0;
      const float cd = dsc[d_per_row ? (int)(rb2 * 16) + (threadIdx.x & 15) : 0];
      uint4 wl[U2], wh[U2];
      auto load2 = [&](int u, int cc) {
        const int j = wave + min(cc, jc - 1) * NW;
        const int64_t t0 = tb2 + 2 * j, t1 = (2 * j + 1 < kts2) ? t0 + 1 : t0;
        wl[u] = ld16nt(w_addr<LAYOUT>(wd, rb2, t0, I, lane));
        wh[u] = ld16nt(w_addr<LAYOUT>(wd, rb2, t1, I, lane));
      };
      if (jc > 0) {
#pragma unroll
        for (int u = 0; u < U2; ++u) load2(u, u);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (!p1_seen) {
        if (threadIdx.x == 0) {
          uint32_t polls = 0, bad = 0;
          for (;;) {
            uint32_t done = 0;
#pragma unroll
            for (int q = 0; q < kGroups; ++q) done += cload(&ctl[q * kGroupWords + kDone]);
            if (done >= (uint32_t)G) break;
            if (++polls > max_polls) {
              cstore(&ctl[kErr], 1u);
              bad = 1;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
          p1_bad = bad;
        }
        __syncthreads();
        // per-token scales of act (final once phase 1 is done), kept for this block's later items
        if (threadIdx.x < (unsigned)M) {
          uint32_t ab = 0;
#pragma unroll
          for (int q = 0; q < kGroups; ++q) ab = umax32(ab, cload(&ctl[q * kGroupWords + kAmax + threadIdx.x]));
          const float a = p1_bad ? __builtin_nanf("") : clamp_min_nan(as_f32(ab), 1e-6f);
          xs2[threadIdx.x] = scale_from_amax(a);
          inv2[threadIdx.x] = inv_from_amax(a);
        }
        p1_seen = true;
        __syncthreads();
      }
      // act[:, s*ks2 : (s+1)*ks2] -> e4m3 in LDS
      const int cpr = ks2 >> 2, nch = M * cpr;
      const uint64_t* act64 = reinterpret_cast<const uint64_t*>(act);
      for (int b0 = threadIdx.x; b0 < nch; b0 += 4 * NT) {
        uint64_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int idx = b0 + q * NT;
          v[q] = 0;
          if (idx < nch) {
            const int m = idx / cpr, c = idx - m * cpr;
            v[q] = cload64(act64 + (((int64_t)m * I + (int64_t)s * ks2) >> 2) + c);
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int idx = b0 + q * NT;
          if (idx < nch) {
            const int m = idx / cpr, c = idx - m * cpr;
            const float inv = inv2[m];
            const uint32_t lo = (uint32_t)v[q], hi = (uint32_t)(v[q] >> 32);
            *reinterpret_cast<uint32_t*>(xq2 + m * ks2 + 4 * c) =
                cvt4_e4m3(as_f32(lo << 16) * inv, as_f32(lo & 0xffff0000u) * inv,
                          as_f32(hi << 16) * inv, as_f32(hi & 0xffff0000u) * inv);
          }
        }
      }
      __syncthreads();
      v4f acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      auto consume2 = [&](int u, int cc) {
        const int j = wave + min(cc, jc - 1) * NW;
        const bool ok = cc < jc, hi = ok && (2 * j + 1 < kts2);
        const v8i B = pack_v8i(sel4(ok, wl[u]), sel4(hi, wh[u]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + r;
          uint4 lo = zero4(), hh = zero4();
          if (m < M) {
            const uint8_t* xr = xq2 + m * ks2 + g * 16;
            lo = *reinterpret_cast<const uint4*>(xr + (2 * j) * 64);
            if (2 * j + 1 < kts2) hh = *reinterpret_cast<const uint4*>(xr + (2 * j + 1) * 64);
          }
          const v8i A = pack_v8i(lo, hh);
          acc[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[mt], 0, 0, 0, 0, 0, 0);
        }
      };
      for (int base = 0; base < jc; base += U2) {
#pragma unroll
        for (int u = 0; u < U2; ++u) {
          consume2(u, base + u);
          if (base + u + U2 < jc) load2(u, base + u + U2);
        }
      }
      stash<MT, 1>(red, wave, lane, acc, acc);
      __syncthreads();
      for (int v = threadIdx.x; v < NV; v += NT) {
        const int mt = v >> 8, i = (v >> 6) & 3, ln = v & 63;
        const int m = mt * 16 + 4 * (ln >> 4) + i;
        if (m >= M) continue;
        float a = 0.0f;
        for (int w = 0; w < NW; ++w) a += red[w * NV + v];
        out[((int64_t)s * M + m) * H + rb2 * 16 + (ln & 15)] = a * xs2[m] * cd;
      }
      __syncthreads();  // red and xq2 are rewritten by the next item
    }
  }

  // The last block out zeroes the control words (the error flag stays): blocks count out per
  // group, the last of each group counts out over groups.
  if (threadIdx.x == 0) {
    const uint32_t in_grp = (uint32_t)((G - grp + kGroups - 1) / kGroups);
    const uint32_t groups = (uint32_t)(G < kGroups ? G : kGroups);
    if (cadd(&ctl[grp * kGroupWords + kExitG], 1u) == in_grp - 1 &&
        cadd(&ctl[kExitTop], 1u) == groups - 1) {
      for (int q = 0; q < kGroups; ++q) {
        cstore(&ctl[q * kGroupWords + kDone], 0u);
        cstore(&ctl[q * kGroupWords + kExitG], 0u);
        for (int m = 0; m < 32; ++m) cstore(&ctl[q * kGroupWords + kAmax + m], 0u);
      }
      cstore(&ctl[kExitTop], 0u);
    }
  }
}

constexpr int kNW = 4;  // waves per block
// step slots per wave: phase 1 refills its ring once per Qwen3-4B item (5 steps per wave);
// phase 2 holds a whole item (19 steps over 4 waves), so its loads are all issued before the wait
constexpr int kU2 = 5;

// Blocks of one launch: `programs` (or one per CU), clamped to the blocks the device holds at once
// for this kernel and shared-memory size - a phase-2 block waits on every block's phase 1, so all
// of them must be resident - and to the larger phase's item count.
template <typename Kernel>
int grid_blocks(Kernel kernel, size_t smem, int programs, int items, int* G) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kNW * 64, smem) != hipSuccess ||
      cus <= 0 || per_cu <= 0) {
    krq_set_error("mlp_fp8: occupancy query failed");
    return KRQ_EHIP;
  }
  int g = programs > 0 ? programs : cus;
  g = g < cus * per_cu ? g : cus * per_cu;
  *G = g < items ? g : items;
  return KRQ_OK;
}

}  // namespace

extern "C" int64_t krq_mlp_ctl_words(void) { return kCtlWords; }

extern "C" int krq_mlp_fp8_bounded(const void* x, int x_kind, const float* x_scale, const void* w_gu,
                                   int w_layout, const float* gu_scale, int gu_per_row, const void* w_down,
                                   const float* down_scale, int down_per_row, int64_t M, int64_t H,
                                   int64_t I, int split, void* act, uint32_t* ctl, int programs,
                                   uint32_t max_polls, void* out, void* stream) {
  KRQ_REQUIRE(x && w_gu && w_down && gu_scale && down_scale && act && ctl && out, "mlp_fp8: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w_gu) && aligned16(w_down) && aligned16(act),
              "mlp_fp8: x, weights and act must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "mlp_fp8: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(x_kind == KRQ_X_FP8 || (x_kind == KRQ_X_BF16_DYN && M == 1),
              "mlp_fp8: x_kind must be KRQ_X_FP8, or KRQ_X_BF16_DYN with M == 1");
  KRQ_REQUIRE(x_kind != KRQ_X_FP8 || x_scale, "mlp_fp8: x_scale is required for e4m3 x");
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "mlp_fp8: bad layout %d", w_layout);
  KRQ_REQUIRE(split >= 1 && split <= 64, "mlp_fp8: split=%d outside 1..64", split);
  KRQ_REQUIRE(H > 0 && H % 64 == 0 && H <= kNW * 64 * 8 * kXC,
              "mlp_fp8: H=%lld must be a positive multiple of 64, at most %d", (long long)H,
              kNW * 64 * 8 * kXC);
  KRQ_REQUIRE(I > 0 && I % 16 == 0 && I % split == 0 && (I / split) % 64 == 0,
              "mlp_fp8: no tiling divides I=%lld with split %d ((I/split) %% 64 must be 0)", (long long)I, split);
  const int MT = M <= 16 ? 1 : 2;
  const size_t red = (size_t)kNW * 2 * MT * 256 * sizeof(float);
  const size_t smem = red + (x_kind == KRQ_X_BF16_DYN ? (size_t)H : 0) + (size_t)M * (I / split);
  KRQ_REQUIRE(smem <= 60 * 1024, "mlp_fp8: M*I/split = %lld bytes of staged activations is too large; raise split",
              (long long)(M * (I / split)));
  const int items = static_cast<int>(std::max(I / 16, (H / 16) * split));
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* gb = (const uint8_t*)w_gu;
  const uint8_t* db = (const uint8_t*)w_down;
  const int m = (int)M, h = (int)H, ii = (int)I;
#define KRQ_MLP_ARGS xb, x_scale, gb, gu_scale, gu_per_row, db, down_scale, down_per_row, m, h, ii, split, \
                     (uint16_t*)act, ctl, (float*)out, max_polls
#define KRQ_MLP_LAUNCH(MTV, XKV, LAY)                                                           \
  do {                                                                                          \
    auto kern = k_mlp_fp8<MTV, XKV, LAY, kNW, MTV == 1 ? 4 : 3, kU2>;                           \
    int G = 0;                                                                                  \
    const int rc = grid_blocks(kern, smem, programs, items, &G);                                \
    if (rc != KRQ_OK) return rc;                                                                \
    hipLaunchKernelGGL(kern, dim3(G), dim3(kNW * 64), smem, s, KRQ_MLP_ARGS);                   \
  } while (0)
  if (x_kind == KRQ_X_BF16_DYN) {
    if (w_layout == KRQ_W_TILED) KRQ_MLP_LAUNCH(1, KRQ_X_BF16_DYN, KRQ_W_TILED);
    else KRQ_MLP_LAUNCH(1, KRQ_X_BF16_DYN, KRQ_W_ROWMAJOR);
  } else if (MT == 1) {
    if (w_layout == KRQ_W_TILED) KRQ_MLP_LAUNCH(1, KRQ_X_FP8, KRQ_W_TILED);
    else KRQ_MLP_LAUNCH(1, KRQ_X_FP8, KRQ_W_ROWMAJOR);
  } else {
    if (w_layout == KRQ_W_TILED) KRQ_MLP_LAUNCH(2, KRQ_X_FP8, KRQ_W_TILED);
    else KRQ_MLP_LAUNCH(2, KRQ_X_FP8, KRQ_W_ROWMAJOR);
  }
#undef KRQ_MLP_LAUNCH
#undef KRQ_MLP_ARGS
  return krq_check_launch("mlp_fp8");
}

extern "C" int krq_mlp_fp8(const void* x, int x_kind, const float* x_scale, const void* w_gu,
                           int w_layout, const float* gu_scale, int gu_per_row, const void* w_down,
                           const float* down_scale, int down_per_row, int64_t M, int64_t H, int64_t I,
                           int split, void* act, uint32_t* ctl, int programs, void* out,
                           void* stream) {
  return krq_mlp_fp8_bounded(x, x_kind, x_scale, w_gu, w_layout, gu_scale, gu_per_row, w_down, down_scale,
                             down_per_row, M, H, I, split, act, ctl, programs, kSpinLimit, out, stream);
}
