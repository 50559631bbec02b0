// Quantization kernels of the decode-matmul path (gfx950):
//   weight quantizers (per output channel, per tensor), activation scales (per tensor, per
//   token), the scaled FP8 cast, and the tiled <-> row-major FP8 weight permutations.
// Quantized bytes come from the software OCP E4M3 RNE encoder (krq::clamp_to_e4m3) on the scalar
// paths and from the hardware convert after the same clamp (krq::cvt4_e4m3, bit-identical) on the
// vectorized paths; both equal torch's float8_e4m3fn cast of the same fp32 values.
#include <stdarg.h>
#include <stdio.h>

#include <stdlib.h>
#include "gemv_common.h"

using namespace krq;

// ---------------------------------------------------------------------------------------------
// error plumbing
// ---------------------------------------------------------------------------------------------
static thread_local char g_err[512] = "";

void krq_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int krq_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    krq_set_error("%s: %s", what, hipGetErrorString(e));
    return KRQ_EHIP;
  }
  return KRQ_OK;
}

extern "C" const char* krq_last_error(void) { return g_err; }
extern "C" const char* krq_version(void) { return "krq 0.1.0 gfx950"; }

namespace {

constexpr int kQT = 256;  // threads of the row-wise kernels

// ---------------------------------------------------------------------------------------------
// Weight rows. One block per row n.
//   MODE 0 (per channel): amax -> scale[n] -> cast with IEEE division by scale[n]
//   MODE 1 (per tensor, pass 1): row_amax[n] = amax
//   MODE 2 (per tensor, pass 3): cast with IEEE division by scale[0]
// Reference: engine/kernels/fp8.py:17-23 (per tensor), experiments/i8.py:11-17 and
// experiments/modal_fq.py:62-63 (per row).
// ---------------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(kQT) void k_weight_rows(const uint16_t* __restrict__ w, int64_t K,
                                                     int64_t ldw, uint8_t* __restrict__ w8,
                                                     uint8_t* __restrict__ w8t,
                                                     float* __restrict__ scale,
                                                     float* __restrict__ row_amax) {
  const int64_t n = blockIdx.x;
  const uint16_t* row = w + n * ldw;
  float s;
  if (MODE == 2) {
    s = scale[0];
  } else {
    uint32_t mb = 0;
    for (int64_t k = threadIdx.x; k < K; k += kQT) mb = umax32(mb, mag_bits(bf16_to_f32(row[k])));
    const float m = as_f32(block_max_u32<kQT>(mb));
    if (MODE == 1) {
      if (threadIdx.x == 0) row_amax[n] = m;
      return;
    }
    s = scale_from_amax(clamp_min_nan(m, 1e-12f));
    if (threadIdx.x == 0) scale[n] = s;
  }
  for (int64_t k = threadIdx.x; k < K; k += kQT) {
    const uint8_t q = clamp_to_e4m3(bf16_to_f32(row[k]) / s);
    if (w8) w8[n * K + k] = q;
    if (w8t) w8t[tiled_offset(n, k, K)] = q;
  }
}

// per-tensor pass 2: one block folds the N row maxima into scale0
__global__ __launch_bounds__(1024) void k_fold_scale(const float* __restrict__ row_amax, int64_t N,
                                                     float* __restrict__ scale0) {
  uint32_t mb = 0;
  for (int64_t i = threadIdx.x; i < N; i += 1024) mb = umax32(mb, mag_bits(row_amax[i]));
  const float m = as_f32(block_max_u32<1024>(mb));
  if (threadIdx.x == 0) scale0[0] = scale_from_amax(clamp_min_nan(m, 1e-12f));
}

// ---------------------------------------------------------------------------------------------
// Activation scales (ActScale, engine/kernels/fp8.py:26-35):
//   amax = max(max|x|, 1e-6) * headroom; inv = fp32(1/amax) * 448; scale = amax * fp32(1/448)
// ---------------------------------------------------------------------------------------------
KRQ_DEV void act_finish(float m, float headroom, float* amax, float* inv, float* scale, int64_t i) {
  const float a = clamp_min_nan(m, 1e-6f) * headroom;
  amax[i] = a;
  inv[i] = inv_from_amax(a);
  scale[i] = scale_from_amax(a);
}

// per tensor pass 1: block-strided partial maxima into ws[blockIdx.x]
__global__ __launch_bounds__(kQT) void k_absmax_partial(const uint16_t* __restrict__ x, int64_t n,
                                                        float* __restrict__ ws) {
  uint32_t mb = 0;
  for (int64_t i = blockIdx.x * (int64_t)kQT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kQT)
    mb = umax32(mb, mag_bits(bf16_to_f32(x[i])));
  mb = block_max_u32<kQT>(mb);
  if (threadIdx.x == 0) ws[blockIdx.x] = as_f32(mb);
}

// pass 1 on 16-byte chunks of 8 bf16 (x 16-byte aligned, n8 chunks): four loads in flight per
// thread and a packed 16-bit bit-max (absmax8_bits) - the scalar pass above reads 2 bytes per lane
// per load and streamed at ~1.7 TB/s on MI355X
__global__ __launch_bounds__(kQT) void k_absmax_partial_vec(const uint4* __restrict__ x, int64_t n8,
                                                            float* __restrict__ ws) {
  u16x2 m{0, 0};
  const int64_t stride = (int64_t)gridDim.x * kQT;
  int64_t i = blockIdx.x * (int64_t)kQT + threadIdx.x;
  for (; i + 3 * stride < n8; i += 4 * stride) {
    const uint4 a0 = x[i], a1 = x[i + stride], a2 = x[i + 2 * stride], a3 = x[i + 3 * stride];
    m = absmax8_bits(a3, absmax8_bits(a2, absmax8_bits(a1, absmax8_bits(a0, m))));
  }
  for (; i < n8; i += stride) m = absmax8_bits(x[i], m);
  const uint32_t mb = block_max_u32<kQT>(bits_max_to_u32(m));
  if (threadIdx.x == 0) ws[blockIdx.x] = as_f32(mb);
}

// per tensor in one launch for small tensors (decode rows): one 1,024-thread block takes the whole
// maximum (16-byte chunks when x allows, else 2 bytes per load) and finishes the scale as k_act_fold
__global__ __launch_bounds__(1024) void k_act_scale_small(const uint16_t* __restrict__ x, int64_t n, int vec,
                                                          float headroom, float* amax, float* inv, float* scale) {
  uint32_t mb = 0;
  if (vec) {
    u16x2 m{0, 0};
    for (int64_t i = threadIdx.x; i < n / 8; i += 1024) m = absmax8_bits(reinterpret_cast<const uint4*>(x)[i], m);
    mb = bits_max_to_u32(m);
  } else {
    for (int64_t i = threadIdx.x; i < n; i += 1024) mb = umax32(mb, mag_bits(bf16_to_f32(x[i])));
  }
  mb = block_max_u32<1024>(mb);
  if (threadIdx.x == 0) act_finish(as_f32(mb), headroom, amax, inv, scale, 0);
}

// per tensor pass 2
__global__ __launch_bounds__(1024) void k_act_fold(const float* __restrict__ ws, int g,
                                                   float headroom, float* amax, float* inv,
                                                   float* scale) {
  uint32_t mb = 0;
  for (int i = threadIdx.x; i < g; i += 1024) mb = umax32(mb, mag_bits(ws[i]));
  mb = block_max_u32<1024>(mb);
  if (threadIdx.x == 0) act_finish(as_f32(mb), headroom, amax, inv, scale, 0);
}

// per row: one block per row m; with x8 != nullptr the row is also cast (quant_rows)
__global__ __launch_bounds__(kQT) void k_act_rows(const uint16_t* __restrict__ x, int64_t K,
                                                  float headroom, float* amax, float* inv,
                                                  float* scale, uint8_t* __restrict__ x8) {
  const int64_t r = blockIdx.x;
  const uint16_t* row = x + r * K;
  uint32_t mb = 0;
  for (int64_t k = threadIdx.x; k < K; k += kQT) mb = umax32(mb, mag_bits(bf16_to_f32(row[k])));
  const float a = clamp_min_nan(as_f32(block_max_u32<kQT>(mb)), 1e-6f) * headroom;
  const float iv = inv_from_amax(a);
  if (threadIdx.x == 0) {
    if (amax) amax[r] = a;
    if (inv) inv[r] = iv;
    scale[r] = scale_from_amax(a);
  }
  if (x8)
    for (int64_t k = threadIdx.x; k < K; k += kQT) x8[r * K + k] = clamp_to_e4m3(bf16_to_f32(row[k]) * iv);
}

// ---------------------------------------------------------------------------------------------
// Cast (engine/kernels/fp8.py:38-56): x8 = e4m3(clamp(float(x) * inv, +-448))
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kQT) void k_cast(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                              const float* __restrict__ inv, int per_row,
                                              uint8_t* __restrict__ x8) {
  const int64_t n = M * K;
  for (int64_t i = blockIdx.x * (int64_t)kQT + threadIdx.x; i < n; i += (int64_t)gridDim.x * kQT) {
    const float iv = inv[per_row ? i / K : 0];
    x8[i] = clamp_to_e4m3(bf16_to_f32(x[i]) * iv);
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled <-> row-major: one thread moves one lane's 16 bytes of one tile.
// ---------------------------------------------------------------------------------------------
template <bool PACK>
__global__ __launch_bounds__(kQT) void k_permute(const uint8_t* __restrict__ src, int64_t N, int64_t K,
                                                 uint8_t* __restrict__ dst) {
  const int64_t total = (N >> 4) * (K >> 6) * 64;
  for (int64_t i = blockIdx.x * (int64_t)kQT + threadIdx.x; i < total; i += (int64_t)gridDim.x * kQT) {
    const int64_t tile = i >> 6;
    const int lane = static_cast<int>(i & 63);
    const int64_t kt = K >> 6;
    const int64_t n = (tile / kt) * 16 + (lane & 15);
    const int64_t k = (tile % kt) * 64 + (lane >> 4) * 16;
    const uint4* a = reinterpret_cast<const uint4*>(src + (PACK ? n * K + k : i * 16));
    uint4* b = reinterpret_cast<uint4*>(dst + (PACK ? i * 16 : n * K + k));
    *b = *a;
  }
}

// ---------------------------------------------------------------------------------------------
// Vectorized forms (K % 8 == 0, 16-byte aligned rows, K <= kVecMaxK): each thread keeps its
// 16-byte chunks of the row in registers between the amax pass and the cast.
// ---------------------------------------------------------------------------------------------
constexpr int kVecChunks = 8;
constexpr int64_t kVecMaxK = (int64_t)kVecChunks * 8 * kQT;

KRQ_DEV uint2 quant8_div(uint4 v, float s) {
  uint2 r;
  r.x = cvt4_e4m3(as_f32(v.x << 16) / s, as_f32(v.x & 0xffff0000u) / s, as_f32(v.y << 16) / s,
                  as_f32(v.y & 0xffff0000u) / s);
  r.y = cvt4_e4m3(as_f32(v.z << 16) / s, as_f32(v.z & 0xffff0000u) / s, as_f32(v.w << 16) / s,
                  as_f32(v.w & 0xffff0000u) / s);
  return r;
}

template <int MODE>
__global__ __launch_bounds__(kQT) void k_weight_rows_vec(const uint16_t* __restrict__ w, int64_t K,
                                                         int64_t ldw, uint8_t* __restrict__ w8,
                                                         uint8_t* __restrict__ w8t,
                                                         float* __restrict__ scale,
                                                         float* __restrict__ row_amax) {
  const int64_t n = blockIdx.x;
  const uint8_t* row = reinterpret_cast<const uint8_t*>(w + n * ldw);
  uint4 v[kVecChunks];
  uint32_t mb = 0;
#pragma unroll
  for (int c = 0; c < kVecChunks; ++c) {
    const int64_t e = 8 * (int64_t)(threadIdx.x + c * kQT);
    v[c] = e < K ? ld16nt(row + 2 * e) : zero4();
    mb = absmax8(v[c], mb);
  }
  float s;
  if (MODE == 2) {
    s = scale[0];
  } else {
    const float m = as_f32(block_max_u32<kQT>(mb));
    if (MODE == 1) {
      if (threadIdx.x == 0) row_amax[n] = m;
      return;
    }
    s = scale_from_amax(clamp_min_nan(m, 1e-12f));
    if (threadIdx.x == 0) scale[n] = s;
  }
#pragma unroll
  for (int c = 0; c < kVecChunks; ++c) {
    const int64_t e = 8 * (int64_t)(threadIdx.x + c * kQT);
    if (e < K) {
      const uint2 q = quant8_div(v[c], s);
      if (w8) *reinterpret_cast<uint2*>(w8 + n * K + e) = q;
      if (w8t) *reinterpret_cast<uint2*>(w8t + tiled_offset(n, e, K)) = q;
    }
  }
}

// per-row activation scale (act_scale), and with x8 the per-token cast (quant_rows where K % 16 != 0)
__global__ __launch_bounds__(kQT) void k_act_rows_vec(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                      float headroom, float* amax, float* inv,
                                                      float* scale, uint8_t* __restrict__ x8) {
  const int64_t r = blockIdx.x;
  const uint8_t* row = reinterpret_cast<const uint8_t*>(x + r * K);
  uint4 v[kVecChunks];
  uint32_t mb = 0;
#pragma unroll
  for (int c = 0; c < kVecChunks; ++c) {
    const int64_t e = 8 * (int64_t)(threadIdx.x + c * kQT);
    v[c] = e < K ? ld16(row + 2 * e) : zero4();
    mb = absmax8(v[c], mb);
  }
  const float a = clamp_min_nan(as_f32(block_max_u32<kQT>(mb)), 1e-6f) * headroom;
  const float iv = inv_from_amax(a);
  if (threadIdx.x == 0) {
    if (amax) amax[r] = a;
    if (inv) inv[r] = iv;
    scale[r] = scale_from_amax(a);
  }
  if (x8) {
#pragma unroll
    for (int c = 0; c < kVecChunks; ++c) {
      const int64_t e = 8 * (int64_t)(threadIdx.x + c * kQT);
      if (e < K) *reinterpret_cast<uint2*>(x8 + r * K + e) = quant8(v[c], iv);
    }
  }
}

// quant_rows (K % 16 == 0): 16 values per thread piece (two 16-byte loads, one 16-byte store), the
// row amax as DPP wave maxima and one barrier, 512 threads, one block per row. Measured on MI355X
// (graph of 72 launches, M = 16; K = 2,560 / 4,096 / 9,728): 2.47 / 2.54 / 3.11 us against 2.87 /
// 2.90 / 3.64 for k_act_rows_vec (256 threads, 8-value pieces, shuffle reductions, two barriers);
// 256 and 1,024 threads measured slower.
constexpr int kRowNT = 512;
template <int NT>
__global__ __launch_bounds__(NT) void k_act_rows_fast(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                      float* __restrict__ scale, uint8_t* __restrict__ x8) {
  constexpr int C = static_cast<int>(kVecMaxK / 16 / NT);
  __shared__ uint32_t red[NT / 64];
  const int64_t r = blockIdx.x;
  const uint8_t* row = reinterpret_cast<const uint8_t*>(x + r * K);
  uint4 v[C][2];
  uint32_t mb = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = 16 * (int64_t)(threadIdx.x + c * NT);
    const bool in = e < K;
    v[c][0] = in ? ld16(row + 2 * e) : zero4();
    v[c][1] = in ? ld16(row + 2 * e + 16) : zero4();
    mb = absmax8(v[c][1], absmax8(v[c][0], mb));
  }
  mb = wave_max_u32_dpp(mb);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mb;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) mb = umax32(mb, red[i]);
  const float a = clamp_min_nan(as_f32(mb), 1e-6f);
  const float iv = inv_from_amax(a);
  if (threadIdx.x == 0) scale[r] = scale_from_amax(a);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = 16 * (int64_t)(threadIdx.x + c * NT);
    if (e < K) {
      const uint2 lo = quant8(v[c][0], iv), hi = quant8(v[c][1], iv);
      *reinterpret_cast<uint4*>(x8 + r * K + e) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }
}

// quant_rows_tiled by four-wave workgroups: workgroup (r, g) reads row r whole, wave w taking the
// pieces of slices w + 4 c (c < CW; piece p = lane + 64 (w + 4 c), two 16-byte loads each, every
// load in flight; pieces past the row repeat its last piece), so each lane loads 2 CW chunks instead
// of the whole row's 2 ch. The waves' maxima (DPP within a wave) meet in LDS at one barrier; then
// wave w quantizes slice w + 4 g, which it holds as its chunk c = g, into the tiled layout. Pad rows
// r >= M get zeros. The same arithmetic as k_act_rows_fast (quant_rows: the row's fp32 magnitude
// bits, the ActScale inverse, the hardware convert), so the same bytes and scales, permuted.
// Measured at M = 16 (graph of 72 launches), K = 2,560 / 4,096 / 9,728: 2.40 / 2.46 / 2.67 us,
// against 2.38 / 2.49 / 2.89 for single-wave workgroups that each read the whole row (one
// workgroup per slice), 2.47 / 2.54 / 3.09 for one 512-thread block per row, and 3.21 / 3.69 /
// 6.60 for one single-wave workgroup per row; eight-wave workgroups (two chunks per lane at
// K = 9,728) measured 2.95 there.
template <int CW>
__global__ __launch_bounds__(256) void k_act_rows_wg(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                     float* __restrict__ scale, uint8_t* __restrict__ x8) {
  __shared__ uint32_t wmax[4];
  const int lane = threadIdx.x & 63, w = static_cast<int>(threadIdx.x >> 6), gi = static_cast<int>(blockIdx.y);
  const int64_t r = blockIdx.x;
  const int np = static_cast<int>(K >> 4);
  const int ps = lane + 64 * (w + 4 * gi);  // the piece this lane stores
  if (r >= M) {  // (uniform per workgroup: no barrier below is skipped by part of it)
    if (ps < np) *reinterpret_cast<uint4*>(x8 + tiled_offset(r, 16 * (int64_t)ps, K)) = zero4();
    return;
  }
  const uint8_t* row = reinterpret_cast<const uint8_t*>(x + r * K);
  uint4 v[CW][2];
  uint32_t mb = 0;
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    const int p = min(lane + 64 * (w + 4 * c), np - 1);
    v[c][0] = ld16(row + 32 * (int64_t)p);
    v[c][1] = ld16(row + 32 * (int64_t)p + 16);
  }
#pragma unroll
  for (int c = 0; c < CW; ++c) mb = absmax8(v[c][1], absmax8(v[c][0], mb));
  mb = wave_max_u32_dpp(mb);
  if (lane == 0) wmax[w] = mb;
  __syncthreads();
  mb = umax32(umax32(wmax[0], wmax[1]), umax32(wmax[2], wmax[3]));
  const float a = clamp_min_nan(as_f32(mb), 1e-6f);
  const float iv = inv_from_amax(a);
  if (gi == 0 && threadIdx.x == 0) scale[r] = scale_from_amax(a);
  if (ps < np) {
#pragma unroll
    for (int c = 0; c < CW; ++c)
      if (c == gi) {
        const uint2 lo = quant8(v[c][0], iv), hi = quant8(v[c][1], iv);
        *reinterpret_cast<uint4*>(x8 + tiled_offset(r, 16 * (int64_t)ps, K)) = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
  }
}

// the cast with a given inverse (krq_cast_fp8's bytes) into the tiled activation layout of
// quant_rows_tiled: one block per row of the M rows padded to a multiple of 16, 16 values
// per thread piece, the pad rows written as zeros
template <int NT>
__global__ __launch_bounds__(NT) void k_cast_rows_tiled(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                        const float* __restrict__ inv, uint8_t* __restrict__ x8) {
  constexpr int C = static_cast<int>(kVecMaxK / 16 / NT);
  const int64_t r = blockIdx.x;
  const float iv = inv[0];
  const uint8_t* row = reinterpret_cast<const uint8_t*>(x + r * K);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = 16 * (int64_t)(threadIdx.x + c * NT);
    if (e < K) {
      uint4 o = zero4();
      if (r < M) {
        const uint2 lo = quant8(ld16(row + 2 * e), iv), hi = quant8(ld16(row + 2 * e + 16), iv);
        o = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
      *reinterpret_cast<uint4*>(x8 + tiled_offset(r, e, K)) = o;
    }
  }
}

// cast, one 16-byte chunk (8 values) per thread
__global__ __launch_bounds__(kQT) void k_cast_vec(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                  const float* __restrict__ inv, int per_row,
                                                  uint8_t* __restrict__ x8) {
  const int64_t nch = M * K / 8;
  for (int64_t i = blockIdx.x * (int64_t)kQT + threadIdx.x; i < nch; i += (int64_t)gridDim.x * kQT) {
    const float iv = inv[per_row ? (8 * i) / K : 0];
    *reinterpret_cast<uint2*>(x8 + 8 * i) = quant8(ld16(reinterpret_cast<const uint8_t*>(x) + 16 * i), iv);
  }
}

// pass 2 folded into the cast (linear_fp8 without a given scale): every block reduces the g
// partials itself (g <= kActPartials, 4 KB from L2), finishes the scale as k_act_fold does (block 0
// stores amax, inv, scale) and casts its chunks as k_cast_vec with that inverse - the bytes of
// pass 2 then the cast, one launch fewer
__global__ __launch_bounds__(kQT) void k_cast_fold_vec(const uint16_t* __restrict__ x, int64_t nch,
                                                       const float* __restrict__ ws, int g, float headroom,
                                                       float* amax, float* inv, float* scale,
                                                       uint8_t* __restrict__ x8) {
  uint32_t mb = 0;
  for (int i = threadIdx.x; i < g; i += kQT) mb = umax32(mb, mag_bits(ws[i]));
  const float a = clamp_min_nan(as_f32(block_max_u32<kQT>(mb)), 1e-6f) * headroom;
  const float iv = inv_from_amax(a);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    amax[0] = a;
    inv[0] = iv;
    scale[0] = scale_from_amax(a);
  }
  for (int64_t i = blockIdx.x * (int64_t)kQT + threadIdx.x; i < nch; i += (int64_t)gridDim.x * kQT)
    *reinterpret_cast<uint2*>(x8 + 8 * i) = quant8(ld16(reinterpret_cast<const uint8_t*>(x) + 16 * i), iv);
}

bool vec_ok(const void* p, int64_t K, int64_t ld) {
  return K % 8 == 0 && ld % 8 == 0 && K <= kVecMaxK && aligned16(p);
}

int grid_for(int64_t work, int per_block, int cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<int>(g);
}

}  // namespace

// =============================================================================================
// C ABI
// =============================================================================================
extern "C" int krq_quant_fp8_rows(const void* w_bf16, int64_t N, int64_t K, int64_t ldw, void* w8,
                                  void* w8_tiled, float* scale, void* stream) {
  KRQ_REQUIRE(w_bf16 && scale && (w8 || w8_tiled), "quant_fp8_rows: null pointer");
  KRQ_REQUIRE(N > 0 && K > 0 && ldw >= K, "quant_fp8_rows: bad shape N=%lld K=%lld ldw=%lld",
              (long long)N, (long long)K, (long long)ldw);
  KRQ_REQUIRE(N <= 0x7fffffff, "quant_fp8_rows: N=%lld too large", (long long)N);
  KRQ_REQUIRE(!w8_tiled || (N % 16 == 0 && K % 64 == 0),
              "quant_fp8_rows: tiled layout needs N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)",
              (long long)N, (long long)K);
  const bool vec = vec_ok(w_bf16, K, ldw) && (!w8 || aligned16(w8));
  hipLaunchKernelGGL(vec ? k_weight_rows_vec<0> : k_weight_rows<0>, dim3(static_cast<unsigned>(N)),
                     dim3(kQT), 0, (hipStream_t)stream, (const uint16_t*)w_bf16, K, ldw, (uint8_t*)w8,
                     (uint8_t*)w8_tiled, scale, nullptr);
  return krq_check_launch("quant_fp8_rows");
}

extern "C" int krq_quant_fp8_tensor(const void* w_bf16, int64_t N, int64_t K, int64_t ldw,
                                    float* row_amax_ws, void* w8, void* w8_tiled, float* scale0,
                                    void* stream) {
  KRQ_REQUIRE(w_bf16 && row_amax_ws && scale0 && (w8 || w8_tiled), "quant_fp8_tensor: null pointer");
  KRQ_REQUIRE(N > 0 && K > 0 && ldw >= K, "quant_fp8_tensor: bad shape N=%lld K=%lld ldw=%lld",
              (long long)N, (long long)K, (long long)ldw);
  KRQ_REQUIRE(N <= 0x7fffffff, "quant_fp8_tensor: N=%lld too large", (long long)N);
  KRQ_REQUIRE(!w8_tiled || (N % 16 == 0 && K % 64 == 0),
              "quant_fp8_tensor: tiled layout needs N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)",
              (long long)N, (long long)K);
  hipStream_t s = (hipStream_t)stream;
  const bool vec = vec_ok(w_bf16, K, ldw) && (!w8 || aligned16(w8));
  hipLaunchKernelGGL(vec ? k_weight_rows_vec<1> : k_weight_rows<1>, dim3(static_cast<unsigned>(N)),
                     dim3(kQT), 0, s, (const uint16_t*)w_bf16, K, ldw, nullptr, nullptr, nullptr,
                     row_amax_ws);
  hipLaunchKernelGGL(k_fold_scale, dim3(1), dim3(1024), 0, s, row_amax_ws, N, scale0);
  hipLaunchKernelGGL(vec ? k_weight_rows_vec<2> : k_weight_rows<2>, dim3(static_cast<unsigned>(N)),
                     dim3(kQT), 0, s, (const uint16_t*)w_bf16, K, ldw, (uint8_t*)w8,
                     (uint8_t*)w8_tiled, scale0, nullptr);
  return krq_check_launch("quant_fp8_tensor");
}

static constexpr int kActPartials = 1024;
static constexpr int64_t kActSmall = 65536;  // elements one block takes in one launch (krq_act_scale)

// per-tensor pass 1 into ws[0 .. g): the vector pass where x allows it; returns g
static int absmax_partials(const void* x_bf16, int64_t M, int64_t K, float* ws, hipStream_t s) {
  const int g = grid_for(M * K, kQT * 16, kActPartials);
  if (aligned16(x_bf16) && (M * K) % 8 == 0)
    hipLaunchKernelGGL(k_absmax_partial_vec, dim3(g), dim3(kQT), 0, s, (const uint4*)x_bf16, M * K / 8, ws);
  else
    hipLaunchKernelGGL(k_absmax_partial, dim3(g), dim3(kQT), 0, s, (const uint16_t*)x_bf16, M * K, ws);
  return g;
}

extern "C" int64_t krq_act_scale_ws_floats(int64_t M, int64_t K) {
  return grid_for(M * K, kQT * 16, kActPartials);
}

extern "C" int krq_act_scale(const void* x_bf16, int64_t M, int64_t K, int per_row, float headroom,
                             float* amax, float* inv, float* scale, float* ws, void* stream) {
  KRQ_REQUIRE(x_bf16 && amax && inv && scale, "act_scale: null pointer");
  KRQ_REQUIRE(M > 0 && K > 0, "act_scale: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  hipStream_t s = (hipStream_t)stream;
  if (per_row) {
    KRQ_REQUIRE(M <= 0x7fffffff, "act_scale: M=%lld too large", (long long)M);
    if (vec_ok(x_bf16, K, K))
      hipLaunchKernelGGL(k_act_rows_vec, dim3(static_cast<unsigned>(M)), dim3(kQT), 0, s,
                         (const uint16_t*)x_bf16, M, K, headroom, amax, inv, scale, nullptr);
    else
      hipLaunchKernelGGL(k_act_rows, dim3(static_cast<unsigned>(M)), dim3(kQT), 0, s, (const uint16_t*)x_bf16, K,
                         headroom, amax, inv, scale, nullptr);
  } else {
    KRQ_REQUIRE(ws != nullptr, "act_scale: per-tensor scale needs a workspace");
    if (M * K <= kActSmall) {
      const int vec = aligned16(x_bf16) && (M * K) % 8 == 0;
      hipLaunchKernelGGL(k_act_scale_small, dim3(1), dim3(1024), 0, s, (const uint16_t*)x_bf16, M * K, vec, headroom,
                         amax, inv, scale);
    } else {
      const int g = absmax_partials(x_bf16, M, K, ws, s);
      hipLaunchKernelGGL(k_act_fold, dim3(1), dim3(1024), 0, s, ws, g, headroom, amax, inv, scale);
    }
  }
  return krq_check_launch("act_scale");
}

extern "C" int krq_act_scale_cast_fp8(const void* x_bf16, int64_t M, int64_t K, float headroom, float* amax,
                                      float* inv, float* scale, float* ws, void* x8, void* stream) {
  KRQ_REQUIRE(x_bf16 && amax && inv && scale && ws && x8, "act_scale_cast: null pointer");
  KRQ_REQUIRE(M > 0 && K > 0, "act_scale_cast: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  hipStream_t s = (hipStream_t)stream;
  const int g = absmax_partials(x_bf16, M, K, ws, s);
  if (vec_ok(x_bf16, K, K) && aligned16(x8)) {
    const int gc = grid_for(M * K / 8, kQT, 8192);
    hipLaunchKernelGGL(k_cast_fold_vec, dim3(gc), dim3(kQT), 0, s, (const uint16_t*)x_bf16, M * K / 8, ws, g,
                       headroom, amax, inv, scale, (uint8_t*)x8);
  } else {  // the two passes and the scalar cast
    hipLaunchKernelGGL(k_act_fold, dim3(1), dim3(1024), 0, s, ws, g, headroom, amax, inv, scale);
    const int gc = grid_for(M * K, kQT * 4, 8192);
    hipLaunchKernelGGL(k_cast, dim3(gc), dim3(kQT), 0, s, (const uint16_t*)x_bf16, M, K, inv, 0, (uint8_t*)x8);
  }
  return krq_check_launch("act_scale_cast");
}

extern "C" int krq_cast_fp8(const void* x_bf16, int64_t M, int64_t K, const float* inv, int per_row,
                            void* x8, void* stream) {
  KRQ_REQUIRE(x_bf16 && inv && x8, "cast_fp8: null pointer");
  KRQ_REQUIRE(M > 0 && K > 0, "cast_fp8: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  if (vec_ok(x_bf16, K, K) && aligned16(x8)) {
    const int g = grid_for(M * K / 8, kQT, 8192);
    hipLaunchKernelGGL(k_cast_vec, dim3(g), dim3(kQT), 0, (hipStream_t)stream, (const uint16_t*)x_bf16,
                       M, K, inv, per_row, (uint8_t*)x8);
  } else {
    const int g = grid_for(M * K, kQT * 4, 8192);
    hipLaunchKernelGGL(k_cast, dim3(g), dim3(kQT), 0, (hipStream_t)stream, (const uint16_t*)x_bf16, M,
                       K, inv, per_row, (uint8_t*)x8);
  }
  return krq_check_launch("cast_fp8");
}

extern "C" int krq_quant_rows(const void* x_bf16, int64_t M, int64_t K, void* x8, float* xs,
                              void* stream) {
  KRQ_REQUIRE(x_bf16 && x8 && xs, "quant_rows: null pointer");
  KRQ_REQUIRE(M > 0 && K > 0 && M <= 0x7fffffff, "quant_rows: bad shape M=%lld K=%lld",
              (long long)M, (long long)K);
  if (vec_ok(x_bf16, K, K) && aligned16(x8) && K % 16 == 0)
    hipLaunchKernelGGL((k_act_rows_fast<kRowNT>), dim3(static_cast<unsigned>(M)), dim3(kRowNT), 0,
                       (hipStream_t)stream, (const uint16_t*)x_bf16, M, K, xs, (uint8_t*)x8);
  else if (vec_ok(x_bf16, K, K) && aligned16(x8))
    hipLaunchKernelGGL(k_act_rows_vec, dim3(static_cast<unsigned>(M)), dim3(kQT), 0, (hipStream_t)stream,
                       (const uint16_t*)x_bf16, M, K, 1.0f, nullptr, nullptr, xs, (uint8_t*)x8);
  else
    hipLaunchKernelGGL(k_act_rows, dim3(static_cast<unsigned>(M)), dim3(kQT), 0, (hipStream_t)stream,
                       (const uint16_t*)x_bf16, K, 1.0f, nullptr, nullptr, xs, (uint8_t*)x8);
  return krq_check_launch("quant_rows");
}

extern "C" int krq_quant_rows_tiled(const void* x_bf16, int64_t M, int64_t K, void* x8_tiled, float* xs,
                                    void* stream) {
  KRQ_REQUIRE(x_bf16 && x8_tiled && xs, "quant_rows_tiled: null pointer");
  KRQ_REQUIRE(M > 0 && M <= 0x7fffffe0 && K > 0 && K % 64 == 0,
              "quant_rows_tiled: bad shape M=%lld K=%lld (K a multiple of 64)", (long long)M, (long long)K);
  KRQ_REQUIRE(vec_ok(x_bf16, K, K) && aligned16(x8_tiled),
              "quant_rows_tiled: x and x8_tiled must be 16-byte aligned and K at most %lld", (long long)kVecMaxK);
  const int64_t mp = (M + 15) / 16 * 16;  // rows padded to whole 16-row tiles
  const int np = static_cast<int>(K / 16), ch = (np + 63) / 64;  // pieces per lane of a whole row (<= 16)
  const int cw = (ch + 3) / 4;                                     // chunks per lane of a four-wave workgroup
  const dim3 grid(static_cast<unsigned>(mp), static_cast<unsigned>(cw));
#define KRQ_ROWS_WG(CW)                                                                                        \
  hipLaunchKernelGGL((k_act_rows_wg<CW>), grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x_bf16, M, K, \
                     xs, (uint8_t*)x8_tiled)
  if (cw <= 1) KRQ_ROWS_WG(1);
  else if (cw <= 2) KRQ_ROWS_WG(2);
  else if (cw <= 3) KRQ_ROWS_WG(3);
  else KRQ_ROWS_WG(4);
#undef KRQ_ROWS_WG
  return krq_check_launch("quant_rows_tiled");
}

extern "C" int krq_cast_fp8_tiled(const void* x_bf16, int64_t M, int64_t K, const float* inv, void* x8_tiled,
                                  void* stream) {
  KRQ_REQUIRE(x_bf16 && inv && x8_tiled, "cast_fp8_tiled: null pointer");
  KRQ_REQUIRE(M > 0 && M <= 0x7fffffe0 && K > 0 && K % 64 == 0,
              "cast_fp8_tiled: bad shape M=%lld K=%lld (K a multiple of 64)", (long long)M, (long long)K);
  KRQ_REQUIRE(vec_ok(x_bf16, K, K) && aligned16(x8_tiled),
              "cast_fp8_tiled: x and x8_tiled must be 16-byte aligned and K at most %lld", (long long)kVecMaxK);
  const int64_t mp = (M + 15) / 16 * 16;
  hipLaunchKernelGGL((k_cast_rows_tiled<kRowNT>), dim3(static_cast<unsigned>(mp)), dim3(kRowNT), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, M, K, inv, (uint8_t*)x8_tiled);
  return krq_check_launch("cast_fp8_tiled");
}

extern "C" int krq_pack_fp8(const void* w8_rowmajor, int64_t N, int64_t K, void* w8_tiled,
                            void* stream) {
  KRQ_REQUIRE(w8_rowmajor && w8_tiled, "pack_fp8: null pointer");
  KRQ_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0,
              "pack_fp8: needs N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  const int g = grid_for((N / 16) * (K / 64) * 64, kQT, 65536);
  hipLaunchKernelGGL(k_permute<true>, dim3(g), dim3(kQT), 0, (hipStream_t)stream,
                     (const uint8_t*)w8_rowmajor, N, K, (uint8_t*)w8_tiled);
  return krq_check_launch("pack_fp8");
}

extern "C" int krq_unpack_fp8(const void* w8_tiled, int64_t N, int64_t K, void* w8_rowmajor,
                              void* stream) {
  KRQ_REQUIRE(w8_rowmajor && w8_tiled, "unpack_fp8: null pointer");
  KRQ_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0,
              "unpack_fp8: needs N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  const int g = grid_for((N / 16) * (K / 64) * 64, kQT, 65536);
  hipLaunchKernelGGL(k_permute<false>, dim3(g), dim3(kQT), 0, (hipStream_t)stream,
                     (const uint8_t*)w8_tiled, N, K, (uint8_t*)w8_rowmajor);
  return krq_check_launch("unpack_fp8");
}
