// Shared device helpers for the krq kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/krq.h"

#define KRQ_DEV __device__ __forceinline__
#define KRQ_HD __host__ __device__ __forceinline__

namespace krq {

constexpr int kWave = 64;
constexpr float kFp8Max = 448.0f;

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------------------------
KRQ_HD float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
KRQ_HD uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }

KRQ_HD float bf16_to_f32(uint16_t h) { return as_f32(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even fp32 -> bf16, NaN kept quiet (the rounding torch's .to(bfloat16) does).
KRQ_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

KRQ_HD float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---------------------------------------------------------------------------------------------
// OCP E4M3 ("fn": bias 7, max 448, no inf, NaN = S.1111.111) encoder, written from the OCP
// 8-bit floating point specification: round to nearest, ties to even, over the extended grid;
// a magnitude that rounds beyond 448 becomes NaN (non-saturating, like torch's float8_e4m3fn
// cast). Callers clamp to +-448 first, as the reference does, so NaN only comes from NaN input.
// ---------------------------------------------------------------------------------------------
KRQ_HD uint8_t f32_to_e4m3(float f) {
  const uint32_t u = as_u32(f);
  const uint8_t sign = static_cast<uint8_t>((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return sign | 0x7fu;  // NaN or inf (no inf in e4m3fn)
  const uint32_t e = a >> 23;                  // biased fp32 exponent
  if (e < 121u) {
    // |f| < 2^-6: subnormal grid of step 2^-9. |f| * 2^9 is exact (power-of-two scaling of a
    // value far from the fp32 limits) and below 8, so rint gives the RNE multiple of 2^-9;
    // q == 8 is the smallest normal, code 0x08, which the formula yields unchanged.
    const float s = as_f32(a) * 512.0f;
    return sign | static_cast<uint8_t>(rintf(s));
  }
  // Normal: keep 3 of the 23 mantissa bits, round the remaining 20 to nearest even; a mantissa
  // carry ripples into the exponent by plain addition.
  uint32_t code = ((e - 120u) << 3) | ((a >> 20) & 7u);
  const uint32_t rem = a & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (code & 1u))) code += 1u;
  if (code > 0x7eu) return sign | 0x7fu;  // beyond 448 -> NaN
  return sign | static_cast<uint8_t>(code);
}

// e4m3 -> fp32, exact (every e4m3 value is an fp32 value). Used only off the hot loop.
KRQ_HD float e4m3_to_f32(uint8_t b) {
  const uint32_t sign = static_cast<uint32_t>(b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
  if (e == 15u && m == 7u) return as_f32(sign | 0x7fc00000u);
  if (e == 0u) {
    const float v = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
    return sign ? -v : v;
  }
  return as_f32(sign | ((e + 120u) << 23) | (m << 20));
}

// quantize one value the way every reference cast does: clamp(v, -448, 448) then e4m3.
// fminf/fmaxf would turn NaN into a bound; torch's clamp propagates NaN, so test it first.
KRQ_HD uint8_t clamp_to_e4m3(float v) {
  if (v != v) return f32_to_e4m3(v);
  v = v < -kFp8Max ? -kFp8Max : v;
  v = v > kFp8Max ? kFp8Max : v;
  return f32_to_e4m3(v);
}

// ---------------------------------------------------------------------------------------------
// Scale arithmetic of the reference's torch expressions, as torch's device kernels evaluate them:
//   amax / 448.0        -> amax * fp32(1/448)   (division by a host scalar is a multiply by its
//                                                 fp32 reciprocal in the device binary kernels)
//   448.0 / amax        -> fp32(1/amax) * 448   (Tensor.__rtruediv__ is reciprocal() * other)
//   w.float() / scale   -> IEEE division        (tensor / tensor)
// ---------------------------------------------------------------------------------------------
KRQ_HD float inv448() { return 1.0f / 448.0f; }
KRQ_HD float scale_from_amax(float amax) { return amax * inv448(); }
KRQ_HD float inv_from_amax(float amax) { return (1.0f / amax) * kFp8Max; }

// Byte offset of element (n, k) of an [N, K] FP8 matrix in the tiled layout: 16-row x 64-byte
// tiles in tile-row-major order; inside a tile lane l = 16*((k%64)/16) + (n%16) owns 16 bytes.
KRQ_HD int64_t tiled_offset(int64_t n, int64_t k, int64_t K) {
  const int64_t tile = (n >> 4) * (K >> 6) + (k >> 6);
  const int64_t lane = (((k & 63) >> 4) << 4) | (n & 15);
  return (tile * 64 + lane) * 16 + (k & 15);
}

// ---------------------------------------------------------------------------------------------
// Magnitude maxima that keep NaN. The reference takes every amax with torch reductions that
// propagate NaN (w.abs().max(), torch.aminmax + torch.maximum, amax(1)) and floors it with
// clamp_min, which keeps NaN too; a NaN element therefore makes its row's (or tensor's) scale NaN
// and every quantized byte of it a NaN code. fmaxf drops NaN, so the kernels compare magnitudes as
// fp32 bit patterns with the sign cleared instead: for numbers these order like the values
// (+0 < denormals < normals < +inf), and every NaN pattern lies above +inf, so an unsigned integer
// max returns NaN as soon as one element is NaN. The folded bits are read back with as_f32.
// ---------------------------------------------------------------------------------------------
KRQ_HD uint32_t mag_bits(float f) { return as_u32(f) & 0x7fffffffu; }

// max(a, lo) that keeps a NaN a, as torch's clamp_min does (fmaxf(NaN, lo) would give lo)
KRQ_HD float clamp_min_nan(float a, float lo) { return a != a ? a : fmaxf(a, lo); }

KRQ_DEV uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

// max over the wave; every lane gets it
KRQ_DEV uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = umax32(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o, kWave)));
  return v;
}

template <int CTRL>
KRQ_DEV uint32_t dpp_max_u32(uint32_t a) {
  return umax32(a, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(a), CTRL, 0xf, 0xf, false)));
}

// max over the wave, returned wave-uniform: DPP steps inside each row of 16 lanes (quad swaps, then
// the half-row and row mirrors), then the four row results read as scalars; a few VALU cycles per
// step instead of an LDS-crossbar round trip per shuffle
KRQ_DEV uint32_t wave_max_u32_dpp(uint32_t v) {
  v = dpp_max_u32<0xB1>(v);   // quad_perm(1,0,3,2): lane ^ 1
  v = dpp_max_u32<0x4E>(v);   // quad_perm(2,3,0,1): lane ^ 2
  v = dpp_max_u32<0x141>(v);  // row_half_mirror: the other quad of each 8
  v = dpp_max_u32<0x140>(v);  // row_mirror: the other half of each 16
  const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
  const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
  const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
  const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
  return umax32(umax32(r0, r1), umax32(r2, r3));
}

KRQ_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// max over a block of NT threads (NT a multiple of 64, at most 1024); every thread gets it.
template <int NT>
KRQ_DEV uint32_t block_max_u32(uint32_t v) {
  __shared__ uint32_t red[NT / kWave];
  v = wave_max_u32(v);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  uint32_t r = red[0];
#pragma unroll
  for (int i = 1; i < NT / kWave; ++i) r = umax32(r, red[i]);
  __syncthreads();
  return r;
}

}  // namespace krq

// error reporting shared by the translation units (defined in quant.hip)
void krq_set_error(const char* fmt, ...);
int krq_check_launch(const char* what);
