// Skinny GEMM / GEMV kernels of the decode path (gfx950, wave64), M <= 32 rows:
//   y[M, N] = x[M, K] . W[N, K]^T with fp32 accumulation.
//
// Work unit. A "row block" is 16 output columns (16 weight rows). A "step" is 128 bytes of each of
// those 16 weight rows: two 16x64-byte tiles. In a step lane l (r = l % 16, g = l / 16) reads 16
// bytes of weight row r from each tile, at byte 16*g of the tile, and the same bytes (same k) of
// activation row r. The FP8 matrix-core instruction v_mfma_f32_16x16x128_f8f6f4 takes exactly
// this: 32 bytes of A row r and of B column r per lane, with the k order of a lane's bytes the
// same for A and B, so the product is sum_k x[m,k] w[n,k] for any assignment of byte offsets to
// lanes that A and B share. The BF16 kernels use v_mfma_f32_16x16x32_bf16 twice per step.
// Accumulator layout of both instructions: lane l, element i holds C[4*(l/16) + i][l % 16],
// i.e. output row m = 4*g + i (+16 for the second M tile) and column n = 16*rb + r.
//
// Grid. blockIdx.x = row block, blockIdx.y = K split. The steps of one (row block, split) are
// dealt in contiguous chunks to the waves of the block; each wave issues all loads of a chunk of
// U steps before its first matrix instruction, so a block keeps nw*U*2 KiB of weights in
// flight. The waves' partial accumulators are summed in LDS in wave order (deterministic), and
// the epilogue applies the scales, rounds, and writes bf16, fp32 split-K partials, or SwiGLU.
#include "krq_common.h"

using namespace krq;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define KRQ_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      krq_set_error(__VA_ARGS__);     \
      return KRQ_EINVAL;              \
    }                                 \
  } while (0)

namespace {

constexpr int kU = 4;        // steps per load batch
constexpr int kMaxWaves = 16;

KRQ_DEV uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

KRQ_DEV v8i pack_v8i(uint4 a, uint4 b) {
  v8i v;
  v[0] = (int)a.x; v[1] = (int)a.y; v[2] = (int)a.z; v[3] = (int)a.w;
  v[4] = (int)b.x; v[5] = (int)b.y; v[6] = (int)b.z; v[7] = (int)b.w;
  return v;
}

KRQ_DEV v8bf as_v8bf(uint4 a) { return __builtin_bit_cast(v8bf, a); }

KRQ_DEV uint4 sel4(bool keep, uint4 a) {
  uint4 z;
  z.x = keep ? a.x : 0u; z.y = keep ? a.y : 0u; z.z = keep ? a.z : 0u; z.w = keep ? a.w : 0u;
  return z;
}

// Byte address of the 16 bytes lane `lane` reads from weight tile t of row block rb.
// row_bytes = bytes per weight row (K for FP8, 2K for BF16); tiles are 64 bytes wide.
template <int LAYOUT>
KRQ_DEV const uint8_t* w_addr(const uint8_t* w, int64_t rb, int64_t t, int64_t row_bytes, int lane) {
  if (LAYOUT == KRQ_W_TILED) return w + ((rb * (row_bytes >> 6) + t) * 64 + lane) * 16;
  return w + (rb * 16 + (lane & 15)) * row_bytes + t * 64 + (lane >> 4) * 16;
}

// ---------------------------------------------------------------------------------------------
// epilogue shared by every GEMV kernel: red holds nw (waves) x P (parts: 1, or 2 for gate/up) x
// MT x 256 accumulator values in the MFMA lane layout.
// ---------------------------------------------------------------------------------------------
template <int MT, int MODE>
KRQ_DEV void epilogue(const float* red, int nw, int M, int64_t NO, int64_t rb, int split_idx,
                      const float* __restrict__ xsc, int x_per_row, const float* __restrict__ wsc,
                      int w_per_row, void* __restrict__ out) {
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  constexpr int NV = MT * 256;
  for (int v = threadIdx.x; v < NV; v += blockDim.x) {
    const int mt = v >> 8, i = (v >> 6) & 3, ln = v & 63;
    const int m = mt * 16 + 4 * (ln >> 4) + i;
    if (m >= M) continue;
    const int64_t n = rb * 16 + (ln & 15);
    float a = 0.0f, au = 0.0f;
    for (int w = 0; w < nw; ++w) {
      a += red[(w * P + 0) * NV + v];
      if (P == 2) au += red[(w * P + 1) * NV + v];
    }
    const float xs = xsc ? xsc[x_per_row ? m : 0] : 1.0f;
    if (MODE == KRQ_OUT_SWIGLU) {
      const float wg = wsc ? wsc[w_per_row ? n : 0] : 1.0f;
      const float wu = wsc ? wsc[w_per_row ? NO + n : 0] : 1.0f;
      const float gg = round_bf16(a * xs * wg);
      const float uu = round_bf16(au * xs * wu);
      const float sl = round_bf16(gg / (1.0f + expf(-gg)));
      reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = f32_to_bf16(sl * uu);
    } else {
      const float ws = wsc ? wsc[w_per_row ? n : 0] : 1.0f;
      const float y = a * xs * ws;
      if (MODE == KRQ_OUT_BF16)
        reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = f32_to_bf16(y);
      else
        reinterpret_cast<float*>(out)[((int64_t)split_idx * M + m) * NO + n] = y;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// FP8 x FP8 on the matrix cores.
// ---------------------------------------------------------------------------------------------
template <int MT, int MODE, int LAYOUT>
__global__ __launch_bounds__(1024) void k_gemv_fp8_mfma(
    const uint8_t* __restrict__ x8, const float* __restrict__ xsc, int x_per_row,
    const uint8_t* __restrict__ w8, const float* __restrict__ wsc, int w_per_row, int M,
    int64_t NO, int64_t K, int kts, int spw, void* __restrict__ out) {
  extern __shared__ float red[];
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t rb = blockIdx.x, rbu = rb + (NO >> 4);
  const int sidx = blockIdx.y;
  const int nsteps = (kts + 1) >> 1;
  const int j0 = wave * spw, j1 = min(j0 + spw, nsteps);
  const int64_t tbase = (int64_t)sidx * kts;

  v4f acc[MT], accu[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    accu[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  for (int jc = j0; jc < j1; jc += kU) {
    uint4 wl[kU], wh[kU], ul[kU], uh[kU], xl[kU][MT], xh[kU][MT];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = min(jc + u, j1 - 1);
      const int64_t t0 = tbase + 2 * j;
      const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
      wl[u] = ld16(w_addr<LAYOUT>(w8, rb, t0, K, lane));
      wh[u] = ld16(w_addr<LAYOUT>(w8, rb, t1, K, lane));
      if (P == 2) {
        ul[u] = ld16(w_addr<LAYOUT>(w8, rbu, t0, K, lane));
        uh[u] = ld16(w_addr<LAYOUT>(w8, rbu, t1, K, lane));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        const uint8_t* xr = x8 + (int64_t)min(m, M - 1) * K + g * 16;
        xl[u][mt] = sel4(m < M, ld16(xr + t0 * 64));
        xh[u][mt] = sel4(m < M, ld16(xr + t1 * 64));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = jc + u;
      const bool ok = j < j1, hi = ok && (2 * j + 1 < kts);
      const v8i B = pack_v8i(sel4(ok, wl[u]), sel4(hi, wh[u]));
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
  }

  constexpr int NV = MT * 256;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[(wave * P + 0) * NV + mt * 256 + i * 64 + lane] = acc[mt][i];
      if (P == 2) red[(wave * P + 1) * NV + mt * 256 + i * 64 + lane] = accu[mt][i];
    }
  __syncthreads();
  epilogue<MT, MODE>(red, nw, M, NO, rb, sidx, xsc, x_per_row, wsc, w_per_row, out);
}

// ---------------------------------------------------------------------------------------------
// FP8 x FP8, M == 1, on the vector ALUs: each lane converts its 32 weight bytes and the matching
// 32 activation bytes to fp32 and accumulates row r's partial dot product; the four lanes that
// share r (g = 0..3) are summed with two cross-lane shuffles, then the waves in LDS.
// ---------------------------------------------------------------------------------------------
KRQ_DEV float dot4_fp8(uint32_t a, uint32_t b, float acc) {
  const auto a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, false);
  const auto a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, true);
  const auto b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
  const auto b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, true);
  acc = fmaf(a0[0], b0[0], acc);
  acc = fmaf(a0[1], b0[1], acc);
  acc = fmaf(a1[0], b1[0], acc);
  acc = fmaf(a1[1], b1[1], acc);
  return acc;
}

KRQ_DEV float dot16_fp8(uint4 a, uint4 b, float acc) {
  acc = dot4_fp8(a.x, b.x, acc);
  acc = dot4_fp8(a.y, b.y, acc);
  acc = dot4_fp8(a.z, b.z, acc);
  return dot4_fp8(a.w, b.w, acc);
}

template <int MODE, int LAYOUT>
__global__ __launch_bounds__(1024) void k_gemv_fp8_valu(
    const uint8_t* __restrict__ x8, const float* __restrict__ xsc, int x_per_row,
    const uint8_t* __restrict__ w8, const float* __restrict__ wsc, int w_per_row, int M,
    int64_t NO, int64_t K, int kts, int spw, void* __restrict__ out) {
  extern __shared__ float red[];
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int g = lane >> 4;
  const int64_t rb = blockIdx.x, rbu = rb + (NO >> 4);
  const int sidx = blockIdx.y;
  const int nsteps = (kts + 1) >> 1;
  const int j0 = wave * spw, j1 = min(j0 + spw, nsteps);
  const int64_t tbase = (int64_t)sidx * kts;
  float a0 = 0.f, a1 = 0.f, u0 = 0.f, u1 = 0.f;

  for (int jc = j0; jc < j1; jc += kU) {
    uint4 wl[kU], wh[kU], ul[kU], uh[kU], xl[kU], xh[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = min(jc + u, j1 - 1);
      const int64_t t0 = tbase + 2 * j;
      const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
      wl[u] = ld16(w_addr<LAYOUT>(w8, rb, t0, K, lane));
      wh[u] = ld16(w_addr<LAYOUT>(w8, rb, t1, K, lane));
      if (P == 2) {
        ul[u] = ld16(w_addr<LAYOUT>(w8, rbu, t0, K, lane));
        uh[u] = ld16(w_addr<LAYOUT>(w8, rbu, t1, K, lane));
      }
      xl[u] = ld16(x8 + t0 * 64 + g * 16);
      xh[u] = ld16(x8 + t1 * 64 + g * 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = jc + u;
      const bool ok = j < j1, hi = ok && (2 * j + 1 < kts);
      a0 = dot16_fp8(sel4(ok, wl[u]), xl[u], a0);
      a1 = dot16_fp8(sel4(hi, wh[u]), xh[u], a1);
      if (P == 2) {
        u0 = dot16_fp8(sel4(ok, ul[u]), xl[u], u0);
        u1 = dot16_fp8(sel4(hi, uh[u]), xh[u], u1);
      }
    }
  }
  float a = a0 + a1, au = u0 + u1;
  a += __shfl_xor(a, 16, kWave);
  a += __shfl_xor(a, 32, kWave);
  if (P == 2) {
    au += __shfl_xor(au, 16, kWave);
    au += __shfl_xor(au, 32, kWave);
  }
  // lanes 0..15 now hold columns 16*rb + lane in MFMA slot (mt 0, i 0), i.e. output row m = 0
  constexpr int NV = 256;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    red[(wave * P + 0) * NV + i * 64 + lane] = (i == 0 && g == 0) ? a : 0.0f;
    if (P == 2) red[(wave * P + 1) * NV + i * 64 + lane] = (i == 0 && g == 0) ? au : 0.0f;
  }
  __syncthreads();
  epilogue<1, MODE>(red, nw, M, NO, rb, sidx, xsc, x_per_row, wsc, w_per_row, out);
}

// ---------------------------------------------------------------------------------------------
// BF16 x BF16 on the matrix cores (row-major weights). A step is 64 bf16 of K: two 32-element
// tiles, one v_mfma_f32_16x16x32_bf16 each.
// ---------------------------------------------------------------------------------------------
template <int MT, int MODE>
__global__ __launch_bounds__(1024) void k_gemv_bf16_mfma(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int64_t NO, int64_t K,
    int kts, int spw, void* __restrict__ out) {
  extern __shared__ float red[];
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t rb = blockIdx.x, rbu = rb + (NO >> 4);
  const int sidx = blockIdx.y;
  const int nsteps = (kts + 1) >> 1;
  const int j0 = wave * spw, j1 = min(j0 + spw, nsteps);
  const int64_t tbase = (int64_t)sidx * kts;
  const int64_t rowb = 2 * K;

  v4f acc[MT], accu[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    accu[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  for (int jc = j0; jc < j1; jc += kU) {
    uint4 wl[kU], wh[kU], ul[kU], uh[kU], xl[kU][MT], xh[kU][MT];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = min(jc + u, j1 - 1);
      const int64_t t0 = tbase + 2 * j;
      const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
      wl[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rb, t0, rowb, lane));
      wh[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rb, t1, rowb, lane));
      if (P == 2) {
        ul[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rbu, t0, rowb, lane));
        uh[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rbu, t1, rowb, lane));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        const uint8_t* xr = x + (int64_t)min(m, M - 1) * rowb + g * 16;
        xl[u][mt] = sel4(m < M, ld16(xr + t0 * 64));
        xh[u][mt] = sel4(m < M, ld16(xr + t1 * 64));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = jc + u;
      const bool ok = j < j1, hi = ok && (2 * j + 1 < kts);
      const v8bf B0 = as_v8bf(sel4(ok, wl[u])), B1 = as_v8bf(sel4(hi, wh[u]));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xl[u][mt]), B0, acc[mt], 0, 0, 0);
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xh[u][mt]), B1, acc[mt], 0, 0, 0);
      }
      if (P == 2) {
        const v8bf U0 = as_v8bf(sel4(ok, ul[u])), U1 = as_v8bf(sel4(hi, uh[u]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xl[u][mt]), U0, accu[mt], 0, 0, 0);
          accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xh[u][mt]), U1, accu[mt], 0, 0, 0);
        }
      }
    }
  }
  constexpr int NV = MT * 256;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[(wave * P + 0) * NV + mt * 256 + i * 64 + lane] = acc[mt][i];
      if (P == 2) red[(wave * P + 1) * NV + mt * 256 + i * 64 + lane] = accu[mt][i];
    }
  __syncthreads();
  epilogue<MT, MODE>(red, nw, M, NO, rb, sidx, nullptr, 0, nullptr, 0, out);
}

// BF16, M == 1, vector ALUs
KRQ_DEV float dot8_bf16(uint4 a, uint4 b, float acc) {
  const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = fmaf(as_f32(av[q] << 16), as_f32(bv[q] << 16), acc);
    acc = fmaf(as_f32(av[q] & 0xffff0000u), as_f32(bv[q] & 0xffff0000u), acc);
  }
  return acc;
}

template <int MODE>
__global__ __launch_bounds__(1024) void k_gemv_bf16_valu(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int64_t NO, int64_t K,
    int kts, int spw, void* __restrict__ out) {
  extern __shared__ float red[];
  constexpr int P = MODE == KRQ_OUT_SWIGLU ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int g = lane >> 4;
  const int64_t rb = blockIdx.x, rbu = rb + (NO >> 4);
  const int sidx = blockIdx.y;
  const int nsteps = (kts + 1) >> 1;
  const int j0 = wave * spw, j1 = min(j0 + spw, nsteps);
  const int64_t tbase = (int64_t)sidx * kts;
  const int64_t rowb = 2 * K;
  float a0 = 0.f, a1 = 0.f, u0 = 0.f, u1 = 0.f;
  for (int jc = j0; jc < j1; jc += kU) {
    uint4 wl[kU], wh[kU], ul[kU], uh[kU], xl[kU], xh[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = min(jc + u, j1 - 1);
      const int64_t t0 = tbase + 2 * j;
      const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
      wl[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rb, t0, rowb, lane));
      wh[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rb, t1, rowb, lane));
      if (P == 2) {
        ul[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rbu, t0, rowb, lane));
        uh[u] = ld16(w_addr<KRQ_W_ROWMAJOR>(w, rbu, t1, rowb, lane));
      }
      xl[u] = ld16(x + t0 * 64 + g * 16);
      xh[u] = ld16(x + t1 * 64 + g * 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = jc + u;
      const bool ok = j < j1, hi = ok && (2 * j + 1 < kts);
      a0 = dot8_bf16(sel4(ok, wl[u]), xl[u], a0);
      a1 = dot8_bf16(sel4(hi, wh[u]), xh[u], a1);
      if (P == 2) {
        u0 = dot8_bf16(sel4(ok, ul[u]), xl[u], u0);
        u1 = dot8_bf16(sel4(hi, uh[u]), xh[u], u1);
      }
    }
  }
  float a = a0 + a1, au = u0 + u1;
  a += __shfl_xor(a, 16, kWave);
  a += __shfl_xor(a, 32, kWave);
  if (P == 2) {
    au += __shfl_xor(au, 16, kWave);
    au += __shfl_xor(au, 32, kWave);
  }
  constexpr int NV = 256;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    red[(wave * P + 0) * NV + i * 64 + lane] = (i == 0 && g == 0) ? a : 0.0f;
    if (P == 2) red[(wave * P + 1) * NV + i * 64 + lane] = (i == 0 && g == 0) ? au : 0.0f;
  }
  __syncthreads();
  epilogue<1, MODE>(red, nw, M, NO, rb, sidx, nullptr, 0, nullptr, 0, out);
}

// ---------------------------------------------------------------------------------------------
// LM head + greedy argmax (engine/engine.py:1021-1022; fused form engine/kernels/mega.py:396-441).
// Each wave owns row blocks rb = 4*blockIdx.x + wave, stepping by 4*gridDim.x, over the full K.
// logit = bf16(acc [* h_scale[m] * w_scale[n]]); per output row m the block keeps the largest
// logit and, among equal maxima, the lowest vocabulary index. Block results go to the workspace;
// the last block to finish (agent-scope counter) folds them in the same order-free way and
// resets the counter, so graph replays need no host-side reset.
// ---------------------------------------------------------------------------------------------
struct Best {
  float v;
  int i;
};

KRQ_DEV bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

KRQ_DEV Best shfl_best(Best b, int o) {
  Best r;
  r.v = __shfl_xor(b.v, o, kWave);
  r.i = __shfl_xor(b.i, o, kWave);
  return r;
}

constexpr int kLmWaves = 4;
constexpr int kLmHeader = 256;  // bytes before the per-block results (counter word first)

template <int MT, int WK, int LAYOUT, int ALGO>
__global__ __launch_bounds__(kLmWaves * 64) void k_lmhead(
    const uint8_t* __restrict__ h, const float* __restrict__ hsc, const uint8_t* __restrict__ w,
    const float* __restrict__ wsc, int M, int64_t V, int64_t K, uint16_t* __restrict__ logits,
    uint8_t* __restrict__ ws, int64_t* __restrict__ idx_out) {
  __shared__ float sv[kLmWaves][32];
  __shared__ int si[kLmWaves][32];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t nrb = V >> 4;
  const int64_t rowb = WK == KRQ_LM_FP8 ? K : 2 * K;
  const int kts = static_cast<int>(rowb >> 6);  // 64-byte tiles per row
  const int nsteps = (kts + 1) >> 1;

  Best best[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) best[mt][i] = Best{-INFINITY, 0x7fffffff};

  for (int64_t rb = (int64_t)blockIdx.x * kLmWaves + wave; rb < nrb; rb += (int64_t)gridDim.x * kLmWaves) {
    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    float a0 = 0.f, a1 = 0.f;
    for (int jc = 0; jc < nsteps; jc += kU) {
      uint4 wl[kU], wh[kU], xl[kU][MT], xh[kU][MT];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int j = min(jc + u, nsteps - 1);
        const int64_t t0 = 2 * j;
        const int64_t t1 = (2 * j + 1 < kts) ? t0 + 1 : t0;
        wl[u] = ld16(w_addr<LAYOUT>(w, rb, t0, rowb, lane));
        wh[u] = ld16(w_addr<LAYOUT>(w, rb, t1, rowb, lane));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = ALGO == 2 ? 0 : mt * 16 + r;
          const uint8_t* xr = h + (int64_t)min(m, M - 1) * rowb + g * 16;
          xl[u][mt] = sel4(m < M, ld16(xr + t0 * 64));
          xh[u][mt] = sel4(m < M, ld16(xr + t1 * 64));
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int j = jc + u;
        const bool ok = j < nsteps, hi = ok && (2 * j + 1 < kts);
        const uint4 bl = sel4(ok, wl[u]), bh = sel4(hi, wh[u]);
        if (ALGO == 2) {
          if (WK == KRQ_LM_FP8) {
            a0 = dot16_fp8(bl, xl[u][0], a0);
            a1 = dot16_fp8(bh, xh[u][0], a1);
          } else {
            a0 = dot8_bf16(bl, xl[u][0], a0);
            a1 = dot8_bf16(bh, xh[u][0], a1);
          }
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (WK == KRQ_LM_FP8) {
              acc[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                  pack_v8i(xl[u][mt], xh[u][mt]), pack_v8i(bl, bh), acc[mt], 0, 0, 0, 0, 0, 0);
            } else {
              acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xl[u][mt]), as_v8bf(bl), acc[mt], 0, 0, 0);
              acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(xh[u][mt]), as_v8bf(bh), acc[mt], 0, 0, 0);
            }
          }
        }
      }
    }
    if (ALGO == 2) {
      float a = a0 + a1;
      a += __shfl_xor(a, 16, kWave);
      a += __shfl_xor(a, 32, kWave);
      acc[0][0] = g == 0 ? a : 0.0f;
    }
    const int n = static_cast<int>(rb * 16 + r);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mt * 16 + 4 * g + i;
        if (m < M && (ALGO != 2 || i == 0)) {
          float y = acc[mt][i];
          if (WK == KRQ_LM_FP8) y = y * hsc[m] * wsc[n];
          const uint16_t yb = f32_to_bf16(y);
          if (logits) logits[(int64_t)m * V + n] = yb;
          const float yv = bf16_to_f32(yb);
          if (better(yv, n, best[mt][i].v, best[mt][i].i)) best[mt][i] = Best{yv, n};
        }
      }
  }
  // fold the 16 lanes that share g (same output rows), then the waves
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      Best b = best[mt][i];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const Best c = shfl_best(b, o);
        if (better(c.v, c.i, b.v, b.i)) b = c;
      }
      const int m = mt * 16 + 4 * g + i;
      if (r == 0 && m < 32) {
        sv[wave][m] = b.v;
        si[wave][m] = b.i;
      }
    }
  __syncthreads();
  const int G = gridDim.x;
  unsigned* counter = reinterpret_cast<unsigned*>(ws);
  float* bv = reinterpret_cast<float*>(ws + kLmHeader);
  int* bi = reinterpret_cast<int*>(ws + kLmHeader + (size_t)G * M * sizeof(float));
  if (threadIdx.x < (unsigned)M) {
    const int m = threadIdx.x;
    Best b = Best{sv[0][m], si[0][m]};
    for (int wv = 1; wv < kLmWaves; ++wv)
      if (better(sv[wv][m], si[wv][m], b.v, b.i)) b = Best{sv[wv][m], si[wv][m]};
    bv[(size_t)blockIdx.x * M + m] = b.v;
    bi[(size_t)blockIdx.x * M + m] = b.i;
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(G - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int m = 0; m < M; ++m) {
    Best b = Best{-INFINITY, 0x7fffffff};
    for (int blk = threadIdx.x; blk < G; blk += blockDim.x) {
      const float v = __hip_atomic_load(&bv[(size_t)blk * M + m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int i = __hip_atomic_load(&bi[(size_t)blk * M + m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (better(v, i, b.v, b.i)) b = Best{v, i};
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const Best c = shfl_best(b, o);
      if (better(c.v, c.i, b.v, b.i)) b = c;
    }
    __syncthreads();
    if (lane == 0) {
      sv[wave][0] = b.v;
      si[wave][0] = b.i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int wv = 1; wv < kLmWaves; ++wv)
        if (better(sv[wv][0], si[wv][0], b.v, b.i)) b = Best{sv[wv][0], si[wv][0]};
      idx_out[m] = b.i == 0x7fffffff ? 0 : b.i;
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int lm_blocks(int64_t V) { return static_cast<int>(((V >> 4) + kLmWaves - 1) / kLmWaves); }

// ---------------------------------------------------------------------------------------------
// host-side launch planning
// ---------------------------------------------------------------------------------------------
struct Plan {
  int nw, spw;
};

Plan plan_steps(int nsteps, int max_waves) {
  int nw = (nsteps + kU - 1) / kU;
  if (nw < 1) nw = 1;
  if (nw > max_waves) nw = max_waves;
  return Plan{nw, (nsteps + nw - 1) / nw};
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define KRQ_LAUNCH_GEMV(KERNEL, ...)                                                      \
  hipLaunchKernelGGL(KERNEL, grid, dim3(plan.nw * 64), smem, (hipStream_t)stream, __VA_ARGS__)

template <int MT, int MODE, int LAYOUT>
void launch_fp8_mfma(dim3 grid, Plan plan, size_t smem, void* stream, const uint8_t* x8,
                     const float* xsc, int xpr, const uint8_t* w8, const float* wsc, int wpr,
                     int M, int64_t NO, int64_t K, int kts, void* out) {
  KRQ_LAUNCH_GEMV((k_gemv_fp8_mfma<MT, MODE, LAYOUT>), x8, xsc, xpr, w8, wsc, wpr, M, NO, K, kts,
                  plan.spw, out);
}

template <int MODE, int LAYOUT>
void dispatch_fp8(int algo, dim3 grid, Plan plan, size_t smem, void* stream, const uint8_t* x8,
                  const float* xsc, int xpr, const uint8_t* w8, const float* wsc, int wpr, int M,
                  int64_t NO, int64_t K, int kts, void* out) {
  if (algo == 2) {
    KRQ_LAUNCH_GEMV((k_gemv_fp8_valu<MODE, LAYOUT>), x8, xsc, xpr, w8, wsc, wpr, M, NO, K, kts,
                    plan.spw, out);
  } else if (M <= 16) {
    launch_fp8_mfma<1, MODE, LAYOUT>(grid, plan, smem, stream, x8, xsc, xpr, w8, wsc, wpr, M, NO, K,
                                     kts, out);
  } else {
    launch_fp8_mfma<2, MODE, LAYOUT>(grid, plan, smem, stream, x8, xsc, xpr, w8, wsc, wpr, M, NO, K,
                                     kts, out);
  }
}

template <int MODE>
void dispatch_bf16(int algo, dim3 grid, Plan plan, size_t smem, void* stream, const uint8_t* x,
                   const uint8_t* w, int M, int64_t NO, int64_t K, int kts, void* out) {
  if (algo == 2) {
    KRQ_LAUNCH_GEMV((k_gemv_bf16_valu<MODE>), x, w, M, NO, K, kts, plan.spw, out);
  } else if (M <= 16) {
    KRQ_LAUNCH_GEMV((k_gemv_bf16_mfma<1, MODE>), x, w, M, NO, K, kts, plan.spw, out);
  } else {
    KRQ_LAUNCH_GEMV((k_gemv_bf16_mfma<2, MODE>), x, w, M, NO, K, kts, plan.spw, out);
  }
}

}  // namespace

// =============================================================================================
// C ABI
// =============================================================================================
extern "C" int krq_gemv_fp8(const void* x8, const float* x_scale, int x_per_row, const void* w8,
                            int w_layout, const float* w_scale, int w_per_row, int64_t M, int64_t N,
                            int64_t K, int split, int mode, int algo, void* out, void* stream) {
  KRQ_REQUIRE(x8 && w8 && x_scale && w_scale && out, "gemv_fp8: null pointer");
  KRQ_REQUIRE(aligned16(x8) && aligned16(w8), "gemv_fp8: x8 and w8 must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_fp8: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(N > 0 && K > 0 && split >= 1, "gemv_fp8: bad shape N=%lld K=%lld split=%d",
              (long long)N, (long long)K, split);
  KRQ_REQUIRE(K % split == 0 && (K / split) % 64 == 0,
              "gemv_fp8: no tiling divides K_SPLIT (K=%lld split=%d; K/split must be a multiple of 64)",
              (long long)K, split);
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || w_layout == KRQ_W_TILED, "gemv_fp8: bad layout %d", w_layout);
  KRQ_REQUIRE(mode >= KRQ_OUT_BF16 && mode <= KRQ_OUT_SWIGLU, "gemv_fp8: bad mode %d", mode);
  KRQ_REQUIRE(algo >= 0 && algo <= 2, "gemv_fp8: bad algo %d", algo);
  KRQ_REQUIRE(algo != 2 || M == 1, "gemv_fp8: the vector-ALU kernel takes M == 1 only");
  KRQ_REQUIRE(mode == KRQ_OUT_PARTIAL || split == 1, "gemv_fp8: split %d needs the partials output", split);
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  KRQ_REQUIRE(NO % 16 == 0 && (mode != KRQ_OUT_SWIGLU || N % 2 == 0),
              "gemv_fp8: no tiling divides N=%lld (output columns must be a multiple of 16)", (long long)N);
  KRQ_REQUIRE(NO / 16 <= 0x7fffffff && split <= 65535, "gemv_fp8: grid too large");
  if (algo == 0) algo = 1;
  const int kts = static_cast<int>(K / split / 64);
  const Plan plan = plan_steps((kts + 1) / 2, (M > 16 && mode == KRQ_OUT_SWIGLU) ? 8 : kMaxWaves);
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : 1;
  const int MT = (algo == 2 || M <= 16) ? 1 : 2;
  const size_t smem = (size_t)plan.nw * P * MT * 256 * sizeof(float);
  const dim3 grid(static_cast<unsigned>(NO / 16), static_cast<unsigned>(split));
  const uint8_t* xb = (const uint8_t*)x8;
  const uint8_t* wb = (const uint8_t*)w8;
  const int m = static_cast<int>(M);
#define KRQ_FP8_CASE(MODE, LAYOUT)                                                                 \
  dispatch_fp8<MODE, LAYOUT>(algo, grid, plan, smem, stream, xb, x_scale, x_per_row, wb, w_scale, \
                             w_per_row, m, NO, K, kts, out)
  if (w_layout == KRQ_W_TILED) {
    if (mode == KRQ_OUT_BF16) KRQ_FP8_CASE(KRQ_OUT_BF16, KRQ_W_TILED);
    else if (mode == KRQ_OUT_PARTIAL) KRQ_FP8_CASE(KRQ_OUT_PARTIAL, KRQ_W_TILED);
    else KRQ_FP8_CASE(KRQ_OUT_SWIGLU, KRQ_W_TILED);
  } else {
    if (mode == KRQ_OUT_BF16) KRQ_FP8_CASE(KRQ_OUT_BF16, KRQ_W_ROWMAJOR);
    else if (mode == KRQ_OUT_PARTIAL) KRQ_FP8_CASE(KRQ_OUT_PARTIAL, KRQ_W_ROWMAJOR);
    else KRQ_FP8_CASE(KRQ_OUT_SWIGLU, KRQ_W_ROWMAJOR);
  }
#undef KRQ_FP8_CASE
  return krq_check_launch("gemv_fp8");
}

extern "C" int krq_gemv_bf16(const void* x, const void* w, int64_t M, int64_t N, int64_t K, int split,
                             int mode, void* out, void* stream) {
  KRQ_REQUIRE(x && w && out, "gemv_bf16: null pointer");
  KRQ_REQUIRE(aligned16(x) && aligned16(w), "gemv_bf16: x and w must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "gemv_bf16: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(N > 0 && K > 0 && split >= 1, "gemv_bf16: bad shape N=%lld K=%lld split=%d",
              (long long)N, (long long)K, split);
  KRQ_REQUIRE(K % split == 0 && (K / split) % 32 == 0,
              "gemv_bf16: no tiling divides K_SPLIT (K=%lld split=%d; K/split must be a multiple of 32)",
              (long long)K, split);
  KRQ_REQUIRE(mode >= KRQ_OUT_BF16 && mode <= KRQ_OUT_SWIGLU, "gemv_bf16: bad mode %d", mode);
  KRQ_REQUIRE(mode == KRQ_OUT_PARTIAL || split == 1, "gemv_bf16: split %d needs the partials output", split);
  const int64_t NO = mode == KRQ_OUT_SWIGLU ? N / 2 : N;
  KRQ_REQUIRE(NO % 16 == 0 && (mode != KRQ_OUT_SWIGLU || N % 2 == 0),
              "gemv_bf16: no tiling divides N=%lld (output columns must be a multiple of 16)", (long long)N);
  KRQ_REQUIRE(NO / 16 <= 0x7fffffff && split <= 65535, "gemv_bf16: grid too large");
  const int algo = M == 1 ? 2 : 1;
  const int kts = static_cast<int>(K / split / 32);
  const Plan plan = plan_steps((kts + 1) / 2, (M > 16 && mode == KRQ_OUT_SWIGLU) ? 8 : kMaxWaves);
  const int P = mode == KRQ_OUT_SWIGLU ? 2 : 1;
  const int MT = M <= 16 ? 1 : 2;
  const size_t smem = (size_t)plan.nw * P * MT * 256 * sizeof(float);
  const dim3 grid(static_cast<unsigned>(NO / 16), static_cast<unsigned>(split));
  const uint8_t* xb = (const uint8_t*)x;
  const uint8_t* wb = (const uint8_t*)w;
  const int m = static_cast<int>(M);
  if (mode == KRQ_OUT_BF16) dispatch_bf16<KRQ_OUT_BF16>(algo, grid, plan, smem, stream, xb, wb, m, NO, K, kts, out);
  else if (mode == KRQ_OUT_PARTIAL) dispatch_bf16<KRQ_OUT_PARTIAL>(algo, grid, plan, smem, stream, xb, wb, m, NO, K, kts, out);
  else dispatch_bf16<KRQ_OUT_SWIGLU>(algo, grid, plan, smem, stream, xb, wb, m, NO, K, kts, out);
  return krq_check_launch("gemv_bf16");
}

extern "C" int64_t krq_lmhead_ws_bytes(int64_t M, int64_t V) {
  return kLmHeader + (int64_t)lm_blocks(V) * M * (int64_t)(sizeof(float) + sizeof(int));
}

extern "C" int krq_lmhead_argmax(const void* h, const float* h_scale, const void* w, int w_kind,
                                 int w_layout, const float* w_scale, int64_t M, int64_t V, int64_t K,
                                 void* logits, void* ws, int64_t ws_bytes, int64_t* idx_out,
                                 void* stream) {
  KRQ_REQUIRE(h && w && ws && idx_out, "lmhead_argmax: null pointer");
  KRQ_REQUIRE(aligned16(h) && aligned16(w), "lmhead_argmax: h and w must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 32, "lmhead_argmax: M=%lld outside 1..32", (long long)M);
  KRQ_REQUIRE(w_kind == KRQ_LM_BF16 || w_kind == KRQ_LM_FP8, "lmhead_argmax: bad weight kind %d", w_kind);
  KRQ_REQUIRE(w_layout == KRQ_W_ROWMAJOR || (w_kind == KRQ_LM_FP8 && w_layout == KRQ_W_TILED),
              "lmhead_argmax: bad layout %d", w_layout);
  KRQ_REQUIRE(w_kind == KRQ_LM_BF16 || (h_scale && w_scale), "lmhead_argmax: FP8 needs h_scale and w_scale");
  KRQ_REQUIRE(V > 0 && V % 16 == 0 && V <= 0x7fffffff, "lmhead_argmax: V=%lld must be a positive multiple of 16",
              (long long)V);
  KRQ_REQUIRE(K > 0 && (w_kind == KRQ_LM_FP8 ? K % 64 == 0 : K % 32 == 0),
              "lmhead_argmax: no tiling divides K=%lld", (long long)K);
  KRQ_REQUIRE(ws_bytes >= krq_lmhead_ws_bytes(M, V), "lmhead_argmax: workspace of %lld bytes < %lld",
              (long long)ws_bytes, (long long)krq_lmhead_ws_bytes(M, V));
  const dim3 grid(lm_blocks(V)), block(kLmWaves * 64);
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* hb = (const uint8_t*)h;
  const uint8_t* wb = (const uint8_t*)w;
  uint16_t* lg = (uint16_t*)logits;
  uint8_t* wsb = (uint8_t*)ws;
  const int m = static_cast<int>(M);
#define KRQ_LM(MT, WK, LAYOUT, ALGO) \
  hipLaunchKernelGGL((k_lmhead<MT, WK, LAYOUT, ALGO>), grid, block, 0, s, hb, h_scale, wb, w_scale, m, V, K, lg, wsb, idx_out)
  if (w_kind == KRQ_LM_BF16) {
    if (M == 1) KRQ_LM(1, KRQ_LM_BF16, KRQ_W_ROWMAJOR, 2);
    else if (M <= 16) KRQ_LM(1, KRQ_LM_BF16, KRQ_W_ROWMAJOR, 1);
    else KRQ_LM(2, KRQ_LM_BF16, KRQ_W_ROWMAJOR, 1);
  } else if (w_layout == KRQ_W_TILED) {
    if (M <= 16) KRQ_LM(1, KRQ_LM_FP8, KRQ_W_TILED, 1);
    else KRQ_LM(2, KRQ_LM_FP8, KRQ_W_TILED, 1);
  } else {
    if (M <= 16) KRQ_LM(1, KRQ_LM_FP8, KRQ_W_ROWMAJOR, 1);
    else KRQ_LM(2, KRQ_LM_FP8, KRQ_W_ROWMAJOR, 1);
  }
#undef KRQ_LM
  return krq_check_launch("lmhead_argmax");
}
