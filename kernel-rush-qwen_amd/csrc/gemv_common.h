// Device helpers shared by the skinny GEMM / GEMV kernels (gfx950, wave64).
//
// Work unit. A "row block" is 16 output columns (16 weight rows). A "step" is 128 bytes of each of
// those 16 weight rows: two 16 x 64-byte tiles. In a step lane l (r = l % 16, g = l / 16) reads 16
// bytes of weight row r from each tile, at byte 16*g of the tile, and the same bytes (same k) of
// activation row r. The FP8 matrix-core instruction v_mfma_f32_16x16x128_f8f6f4 takes exactly
// this: 32 bytes of A row r and of B column r per lane, with the k order of a lane's bytes the
// same for A and B, so the product is sum_k x[m,k] w[n,k] for any assignment of byte offsets to
// lanes that A and B share. The BF16 kernels use v_mfma_f32_16x16x32_bf16 twice per step.
// Accumulator layout of both instructions: lane l, element i holds C[4*(l/16) + i][l % 16],
// i.e. output row m = 4*g + i (+16 for the second M tile) and column n = 16*rb + r.
//
// Steps of one (row block, K split) are dealt to the waves of a block round-robin (wave w takes
// steps w, w + nw, ...), so at any moment a block's waves read adjacent tiles; each wave issues
// the loads of U steps before its first matrix instruction. Weight loads are non-temporal
// (streamed once, kept out of the caches' reuse set).
#pragma once

#include "krq_common.h"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

#define KRQ_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      krq_set_error(__VA_ARGS__);     \
      return KRQ_EINVAL;              \
    }                                 \
  } while (0)

namespace krq {

constexpr int kU = 4;  // steps per load batch

// Internal output mode (not part of the C ABI's modes): the lm-head epilogue. Logits are rounded
// to bf16 (optionally stored to `out`) and each block writes, per output row m, the largest
// logit of its 16 columns and the lowest column index holding it to `aux` ([M][row block] Best:
// each token row's candidates are contiguous, so the fold reads them as whole lines).
constexpr int kOutArgmax = 3;

// Internal output mode: the SwiGLU of KRQ_OUT_SWIGLU by a half-pair block b, which owns the 8 output
// columns 8 b .. 8 b + 7: one matrix-core B operand holds both weight halves of them (its columns
// 0-7 gate rows 8 b + c, its columns 8-15 the matching up rows NO + 8 b + c), with the steps per wave
// of the two-matrix block, so the sums are the same bit for bit. A SwiGLU launch runs its last
// column blocks this way (k_gemv_fp8_swiglu_mixed) to even out the bytes per compute unit.
constexpr int kOutSwiGluHalf = 5;

// Internal output mode: the residual epilogue of a folded one-row block b (M = 1, split S = 4 of the
// caller), which owns output columns 4 b .. 4 b + 3 over the whole of K. Matrix-core column c of
// the block is output column 4 b + c % 4 over quarter c / 4 of K, and A row q < 4 holds quarter q
// of the activation row (rows 4..15 zero), so quarter q's sum for column j lands in C[q][4 q + j].
// With the waves and steps of the split launch, those are its S partials bit for bit; the block
// sums them in split order and finishes the residual. 4 N / 16 blocks instead of N / 16 one-pass
// blocks (fewer than the CUs at N = 2,560), and no cross-block reduction.
constexpr int kOutResidualFold = 6;

struct Best {
  float v;
  int i;
};

// larger value wins; among equal values the lower index (torch.argmax keeps the first maximum);
// NaN is larger than every number, as in torch.argmax and numpy.argmax
KRQ_DEV bool better(float v, int i, float bv, int bi) {
  const bool n = v != v, bn = bv != bv;
  if (n || bn) return n && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

KRQ_DEV Best shfl_best(Best b, int o) {
  Best r;
  r.v = __shfl_xor(b.v, o, kWave);
  r.i = __shfl_xor(b.i, o, kWave);
  return r;
}

KRQ_DEV uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

KRQ_DEV uint4 ld16nt(const uint8_t* p) {
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

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

KRQ_DEV uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// The same address, held in vector registers the compiler cannot prove uniform.
KRQ_DEV const uint8_t* vgpr_ptr(const uint8_t* p) {
  uint64_t v = reinterpret_cast<uint64_t>(p);
  asm volatile("" : "+v"(v));
  return reinterpret_cast<const uint8_t*>(v);
}

// Byte address of the 16 bytes lane `lane` reads from weight tile t of row block rb.
// row_bytes = bytes per weight row (K for FP8, 2K for BF16); tiles are 64 bytes wide.
template <int LAYOUT>
KRQ_DEV const uint8_t* w_addr(const uint8_t* w, int64_t rb, int64_t t, int64_t row_bytes, int lane) {
  if (LAYOUT == KRQ_W_TILED) return w + ((rb * (row_bytes >> 6) + t) * 64 + lane) * 16;
  return w + (rb * 16 + (lane & 15)) * row_bytes + t * 64 + (lane >> 4) * 16;
}

// The B-operand address of folded one-row block b (kOutResidualFold): lane column c = lane % 16
// reads output row 4 b + c % 4 at tile t of quarter c / 4 of K (qt 64-byte tiles per quarter).
template <int LAYOUT>
KRQ_DEV const uint8_t* w_addr_fold(const uint8_t* w, int64_t b, int64_t K, int qt, int64_t t, int lane) {
  const int c = lane & 15;
  const int64_t row = 4 * b + (c & 3), tk = (int64_t)(c >> 2) * qt + t;  // the row's tile
  if (LAYOUT == KRQ_W_TILED) return w + (((row >> 4) * (K >> 6) + tk) * 64 + (lane & 48) + (row & 15)) * 16;
  return w + row * K + tk * 64 + (lane >> 4) * 16;
}

// The B-operand address of half-pair block b (kOutSwiGluHalf): lane column c < 8 reads gate row
// 8 b + c, c >= 8 the up row NO + 8 b + c - 8; both are row 8 (b % 2) + c % 8 of 16-row block b / 2
// of their matrix, so in the tiled layout a lane reads that row's 16 bytes of the tile.
template <int LAYOUT>
KRQ_DEV const uint8_t* w_addr_hp(const uint8_t* w, int64_t b, int64_t NO, int64_t t, int64_t row_bytes, int lane) {
  const int c = lane & 15;
  const int64_t rbx = (b >> 1) + (c >> 3) * (NO >> 4);
  const int rr = 8 * static_cast<int>(b & 1) + (c & 7);
  if (LAYOUT == KRQ_W_TILED) return w + ((rbx * (row_bytes >> 6) + t) * 64 + (lane & 48) + rr) * 16;
  return w + (rbx * 16 + rr) * row_bytes + t * 64 + (lane >> 4) * 16;
}

// Hardware fp32 -> OCP e4m3 pair conversion after the reference's clamp to +-448. Bit-identical to
// f32_to_e4m3 (round to nearest even) on the clamped range; NaN stays NaN.
KRQ_DEV float clamp448(float v) { return v != v ? v : fminf(fmaxf(v, -kFp8Max), kFp8Max); }

// NaN inputs: the hardware writes an unsigned NaN code; torch's cast keeps the sign (S.1111.111).
KRQ_DEV uint32_t nan_sign(uint32_t p, float v, int shift) {
  const uint32_t u = as_u32(v);
  const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
  const uint32_t code = ((u >> 24) & 0x80u) | 0x7fu;
  return nan ? (p & ~(0xffu << shift)) | (code << shift) : p;
}

KRQ_DEV uint32_t cvt4_e4m3(float a, float b, float c, float d) {
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(a), clamp448(b), 0, false);
  p = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(c), clamp448(d), p, true);
  uint32_t q = static_cast<uint32_t>(p);
  q = nan_sign(q, a, 0);
  q = nan_sign(q, b, 8);
  q = nan_sign(q, c, 16);
  return nan_sign(q, d, 24);
}

// 8 bf16 (one 16-byte chunk) times s -> 8 e4m3 bytes
KRQ_DEV uint2 quant8(uint4 v, float s) {
  uint2 r;
  r.x = cvt4_e4m3(as_f32(v.x << 16) * s, as_f32(v.x & 0xffff0000u) * s, as_f32(v.y << 16) * s,
                  as_f32(v.y & 0xffff0000u) * s);
  r.y = cvt4_e4m3(as_f32(v.z << 16) * s, as_f32(v.z & 0xffff0000u) * s, as_f32(v.w << 16) * s,
                  as_f32(v.w & 0xffff0000u) * s);
  return r;
}

// 8 bf16 times the inverse of their own row's amax -> 8 e4m3 bytes, without the clamp: |x * inv| is
// at most 448.0001 (fp32 rounding of amax * fl(fl(1 / amax) * 448)), which the convert rounds to
// 448 as the clamp would; a NaN element gives a NaN code (its sign does not reach the products)
KRQ_DEV uint2 quant8_own_amax(uint4 v, float s) {
  uint2 r;
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(as_f32(v.x << 16) * s, as_f32(v.x & 0xffff0000u) * s, 0, false);
  r.x = static_cast<uint32_t>(
      __builtin_amdgcn_cvt_pk_fp8_f32(as_f32(v.y << 16) * s, as_f32(v.y & 0xffff0000u) * s, p, true));
  p = __builtin_amdgcn_cvt_pk_fp8_f32(as_f32(v.z << 16) * s, as_f32(v.z & 0xffff0000u) * s, 0, false);
  r.y = static_cast<uint32_t>(
      __builtin_amdgcn_cvt_pk_fp8_f32(as_f32(v.w << 16) * s, as_f32(v.w & 0xffff0000u) * s, p, true));
  return r;
}

// |x| max of 8 bf16 on their bits: |x| orders as its bit pattern (sign cleared), with NaN above
// every number (mag_bits), so a packed 16-bit integer max per 32-bit word suffices; m holds two
// running maxima. Integer work only, which also keeps the compiler from holding fp32 copies of the
// row for the quantization that follows.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
KRQ_DEV u16x2 absmax8_bits(uint4 v, u16x2 m) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[q] & 0x7fff7fffu));
  return m;
}
// the two running maxima as one fp32 magnitude bit pattern (mag_bits of the larger)
KRQ_DEV uint32_t bits_max_to_u32(u16x2 m) { return static_cast<uint32_t>(m.x > m.y ? m.x : m.y) << 16; }

// running |x| max (fp32 magnitude bits, NaN-keeping) of 8 bf16
KRQ_DEV uint32_t absmax8(uint4 v, uint32_t m) {
  return umax32(m, bits_max_to_u32(absmax8_bits(v, u16x2{0, 0})));
}

// 8 bf16 times a given inverse scale -> 8 e4m3 bytes, with the reference's clamp to +-448 (the
// products can exceed it); NaN stays a NaN code (its sign does not reach the products)
KRQ_DEV uint2 quant8_clamped(uint4 v, float s) {
  uint2 r;
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(as_f32(v.x << 16) * s), clamp448(as_f32(v.x & 0xffff0000u) * s), 0,
                                          false);
  r.x = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(as_f32(v.y << 16) * s),
                                                              clamp448(as_f32(v.y & 0xffff0000u) * s), p, true));
  p = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(as_f32(v.z << 16) * s), clamp448(as_f32(v.z & 0xffff0000u) * s), 0,
                                      false);
  r.y = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(as_f32(v.w << 16) * s),
                                                              clamp448(as_f32(v.w & 0xffff0000u) * s), p, true));
  return r;
}

// vector-ALU dot products (M == 1 kernels)
KRQ_DEV float dot4_fp8(uint32_t a, uint32_t b, float acc) {
  const auto a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, false);
  const auto a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, true);
  const auto b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
  const auto b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, true);
  acc = fmaf(a0[0], b0[0], acc);
  acc = fmaf(a0[1], b0[1], acc);
  acc = fmaf(a1[0], b1[0], acc);
  return fmaf(a1[1], b1[1], acc);
}

KRQ_DEV float dot16_fp8(uint4 a, uint4 b, float acc) {
  acc = dot4_fp8(a.x, b.x, acc);
  acc = dot4_fp8(a.y, b.y, acc);
  acc = dot4_fp8(a.z, b.z, acc);
  return dot4_fp8(a.w, b.w, acc);
}

KRQ_DEV float dot8_bf16(uint4 a, uint4 b, float acc) {
  const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = fmaf(as_f32(av[q] << 16), as_f32(bv[q] << 16), acc);
    acc = fmaf(as_f32(av[q] & 0xffff0000u), as_f32(bv[q] & 0xffff0000u), acc);
  }
  return acc;
}

// ---------------------------------------------------------------------------------------------
// Epilogue of every GEMV kernel. red holds nw (waves) x P (1, or 2 for gate/up) x MT x 256
// accumulator values in the MFMA lane layout; xs[m] is row m's activation scale (1 if unscaled).
// Sums the waves in wave order (deterministic), applies scales, rounds, and writes bf16 [M, NO],
// fp32 partials [split, M, NO], or SwiGLU bf16 [M, NO].
// ---------------------------------------------------------------------------------------------
// Weight scales of the columns this thread writes in the epilogue (thread t writes columns
// 16*rb + t % 16), loaded at kernel start so their latency hides under the weight stream
// (wsc must not be null).
struct ColScales {
  float g, u;
};

// g: row block rb; u: its second matrix, the up half (SwiGLU) or row block rb + 1 (paired blocks)
template <int MODE, int PB>
KRQ_DEV ColScales load_col_scales(const float* __restrict__ wsc, int w_per_row, int64_t NO, int64_t rb) {
  ColScales c{1.0f, 1.0f};
  if (MODE == kOutSwiGluHalf) {  // rb = b: the scale of this lane column's gate or up row
    const int col = threadIdx.x & 15;
    c.g = wsc[w_per_row ? (col >> 3) * NO + rb * 8 + (col & 7) : 0];
    return c;
  }
  const int64_t n = rb * 16 + (threadIdx.x & 15);
  c.g = wsc[w_per_row ? n : 0];
  if (MODE == KRQ_OUT_SWIGLU) c.u = wsc[w_per_row ? NO + n : 0];
  else if (PB == 2) c.u = wsc[w_per_row ? n + 16 : 0];
  return c;
}

// a bf16 output element; WT: written through to memory (agent scope), for a reader on another XCD
// in the same launch
template <bool WT>
KRQ_DEV void store_bf16(uint16_t* p, uint16_t v) {
  if constexpr (WT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

// P accumulator sets per wave in red; this call reads set p0 (and p0 + 1 for SwiGLU) and writes
// row block rb. SwiGLU with aux = a device float `inv`: out receives the next projection's input,
// e4m3(clamp(act * inv, +-448)) of the bf16 act, in the tiled activation layout (rows padded to
// 16 MT, pad rows 0; NO % 64 == 0) instead of bf16 act. nt > 0: only threads 0 .. nt - 1 call it
// (the others have ended); by default every thread of the block does.
template <int MT, int MODE, int P, bool WT = false>
KRQ_DEV void epilogue(const float* red, int p0, int nw, int M, int64_t NO, int64_t rb, int split_idx,
                      const float* xs, ColScales cs, void* __restrict__ out, void* __restrict__ aux, int nt = 0) {
  constexpr int NV = MT * 256;
  const bool cast = (MODE == KRQ_OUT_SWIGLU || MODE == kOutSwiGluHalf) && aux != nullptr;
  const float cinv = cast ? *static_cast<const float*>(aux) : 0.0f;
  const int stride = nt > 0 ? nt : static_cast<int>(blockDim.x);
  for (int v = threadIdx.x; v < NV; v += stride) {
    const int mt = v >> 8, i = (v >> 6) & 3, ln = v & 63;
    const int m = mt * 16 + 4 * (ln >> 4) + i;
    const bool valid = m < M;
    const int64_t n = rb * 16 + (ln & 15);
    float a = 0.0f, au = 0.0f;
    for (int w = 0; w < nw; ++w) {
      a += red[(w * P + p0) * NV + v];
      if (MODE == KRQ_OUT_SWIGLU) au += red[(w * P + p0 + 1) * NV + v];
    }
    const float x = valid ? xs[m] : 0.0f;
    if (MODE == kOutSwiGluHalf) {
      // lane column c < 8 holds gate output 8 rb + c of row m, lane column c + 8 its up value: each
      // rounded as KRQ_OUT_SWIGLU rounds it, then the gate lanes combine them
      const float t = round_bf16(a * x * cs.g);
      const float uu = __shfl_xor(t, 8, kWave);
      if (ln & 8) continue;
      const int64_t n8 = rb * 8 + (ln & 7);
      if (cast) {
        uint8_t q = 0;  // pad rows m >= M
        if (valid) {
          const float sl = round_bf16(t / (1.0f + expf(-t)));
          q = clamp_to_e4m3(round_bf16(sl * uu) * cinv);
        }
        const int64_t tile = (int64_t)(m >> 4) * (NO >> 6) + (n8 >> 6);
        reinterpret_cast<uint8_t*>(out)[tile * 1024 + 16 * (16 * ((n8 & 63) >> 4) + (m & 15)) + (n8 & 15)] = q;
      } else if (valid) {
        const float sl = round_bf16(t / (1.0f + expf(-t)));
        store_bf16<WT>(reinterpret_cast<uint16_t*>(out) + (int64_t)m * NO + n8, f32_to_bf16(sl * uu));
      }
      continue;
    }
    if (MODE == kOutArgmax) {
      // the 16 lanes sharing (mt, i, g) hold the 16 columns of one output row: fold them
      Best b{-INFINITY, 0x7fffffff};
      if (valid) {
        const uint16_t yb = f32_to_bf16(a * x * cs.g);
        if (out) reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = yb;
        b = Best{bf16_to_f32(yb), static_cast<int>(n)};
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const Best c = shfl_best(b, o);
        if (better(c.v, c.i, b.v, b.i)) b = c;
      }
      if (valid && (ln & 15) == 0) reinterpret_cast<Best*>(aux)[(int64_t)m * (NO >> 4) + rb] = b;
      continue;
    }
    if (MODE == KRQ_OUT_SWIGLU && cast) {
      uint8_t q = 0;  // pad rows m >= M
      if (valid) {
        const float gg = round_bf16(a * x * cs.g);
        const float uu = round_bf16(au * x * cs.u);
        const float sl = round_bf16(gg / (1.0f + expf(-gg)));
        q = clamp_to_e4m3(round_bf16(sl * uu) * cinv);
      }
      // tile (m / 16, n / 64); lane 16 ((n % 64) / 16) + m % 16 holds bytes n % 16 of row m
      const int64_t tile = (int64_t)(m >> 4) * (NO >> 6) + (n >> 6);
      reinterpret_cast<uint8_t*>(out)[tile * 1024 + 16 * (16 * ((n & 63) >> 4) + (m & 15)) + (n & 15)] = q;
      continue;
    }
    if (!valid) continue;
    if (MODE == KRQ_OUT_SWIGLU) {
      const float gg = round_bf16(a * x * cs.g);
      const float uu = round_bf16(au * x * cs.u);
      const float sl = round_bf16(gg / (1.0f + expf(-gg)));
      store_bf16<WT>(reinterpret_cast<uint16_t*>(out) + (int64_t)m * NO + n, f32_to_bf16(sl * uu));
    } else {
      const float y = a * x * cs.g;
      if (MODE == KRQ_OUT_BF16)
        reinterpret_cast<uint16_t*>(out)[(int64_t)m * NO + n] = f32_to_bf16(y);
      else
        reinterpret_cast<float*>(out)[((int64_t)split_idx * M + m) * NO + n] = y;
    }
  }
}

template <int MT, int P>
KRQ_DEV void stash(float* red, int wave, int lane, const v4f* acc, const v4f* accu) {
  constexpr int NV = MT * 256;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[(wave * P + 0) * NV + mt * 256 + i * 64 + lane] = acc[mt][i];
      if (P == 2) red[(wave * P + 1) * NV + mt * 256 + i * 64 + lane] = accu[mt][i];
    }
}

// ---------------------------------------------------------------------------------------------
// Cross-block data within one launch (fused MLP, residual epilogue). Agent-scope relaxed atomics:
// their stores write through to memory and their loads read memory, on every XCD, so no cache
// writeback or invalidate is needed. A producer calls stores_done() before it signals.
// ---------------------------------------------------------------------------------------------
KRQ_DEV uint32_t cload(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KRQ_DEV uint64_t cload64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KRQ_DEV void cstore(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KRQ_DEV void cstore64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KRQ_DEV uint32_t cadd(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KRQ_DEV void cmax(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// waits until every store and atomic this thread issued has completed
KRQ_DEV void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------------------------------------
// RMSNorm prologue and residual epilogue of the fused GEMVs (reference engine/kernels/
// fused_gemv.py:48-120): h = bf16(bf16(x * rstd) * w_ln), rstd = rsqrt(ss / K + eps) with ss the
// sum of the row's [K/16] per-tile partials; x_new = bf16(res_in + bf16(y)) with per-tile sums of
// squares of x_new.
// ---------------------------------------------------------------------------------------------
constexpr int kOutResidual = KRQ_OUT_RESIDUAL;

struct FusedArgs {
  const uint16_t* ln;  // RMSNorm weight [K] bf16 (null: no RMSNorm prologue)
  const float* ss_in;  // [M][K/16] per-tile sums of squares of x
  float eps;
  const uint16_t* res_in;  // residual epilogue: bf16 [M][N] residual rows
  uint16_t* res_out;       // bf16 [M][N] new residual rows
  float* ss_out;           // [M][N/16] per-tile sums of squares of res_out
  uint32_t* cnt;           // [N/16] split-arrival counters (zero between launches); chained MLP: kChainWords control words
  uint32_t max_polls;      // chained MLP: polls of the first stage's done flag before a block gives up
  int n_first;             // chained MLP: first workgroup index of the second stage
  int n_second;            // chained MLP: workgroups of the second stage
};

// Control words of the chained MLP (uint32, zero between launches). Group g < kChainGroups owns
// the line at word 64 g: [0] first-stage arrivals, [1] second-stage exits. Word kChainArr counts
// the first-stage groups complete, kChainExit the second-stage groups done, and kChainErr records
// a wait that gave up. The first stage's done flag goes to kChainReps replicas kChainRepStride
// words (4,352 bytes) apart from word kChainRep, and a waiting workgroup polls replica
// blockIdx.x % kChainReps: a few hundred workgroups polling one word saturate the memory channel
// that holds it, and every weight stream, which is interleaved over all channels, slows with it
// (measured: the gate_up stage took 240 us instead of 10).
constexpr int kChainGroups = 8, kChainTop = kChainGroups * 64, kChainExit = kChainTop, kChainErr = kChainTop + 1,
              kChainArr = kChainTop + 2, kChainRep = kChainTop + 64, kChainReps = 64, kChainRepStride = 1088,
              kChainWords = kChainRep + kChainReps * kChainRepStride;
static_assert(kChainReps == 64, "one replica per lane of the publishing wave");

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// Two fp32 values rounded to bf16 (nearest even) and packed lo | hi << 16: one hardware convert
// (v_cvt_pk_bf16_f32). Equal to f32_to_bf16 on every non-NaN input; a NaN stays a NaN.
KRQ_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
}

KRQ_DEV uint4 norm8(uint4 xv, uint4 lv, float rstd) {
  const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w}, la[4] = {lv.x, lv.y, lv.z, lv.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t r = pack_bf16x2(as_f32(xa[q] << 16) * rstd, as_f32(xa[q] & 0xffff0000u) * rstd);
    o[q] = pack_bf16x2(as_f32(r << 16) * as_f32(la[q] << 16), as_f32(r & 0xffff0000u) * as_f32(la[q] & 0xffff0000u));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Sum of squares of the 8 bf16 values of a 16-byte chunk, in element order from zero: the partial
// of chunk i (elements 8 i .. 8 i + 7) when a one-row kernel sums its row itself (see below).
KRQ_DEV float sumsq8(uint4 v) {
  const uint32_t a[4] = {v.x, v.y, v.z, v.w};
  float s = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float lo = as_f32(a[q] << 16), hi = as_f32(a[q] & 0xffff0000u);
    s = fmaf(lo, lo, s);
    s = fmaf(hi, hi, s);
  }
  return s;
}

// One row (M = 1): the normalizing kernels take the row's sum of squares from the row itself, as
// the canonical sum below over its K / 8 chunk partials sumsq8 (chunk i at lane i % 64), and read no
// ss_in; at M > 1 they sum the [M][K/16] partials of ss_in. A one-row prologue holds the whole row
// anyway (its per-token amax needs it), so the producer of x needs no sum of squares at M = 1 (the
// folded residual GEMVs, kOutResidualFold, write none).
// The canonical row sum of T sum-of-squares partials, used by every kernel that normalizes (so the
// fused prologues, k_rmsnorm_rows and k_rmsnorm_quant_rows agree bit for bit): lane l adds
// partials t = l, l + 64, l + 128, ... in that order, then the butterfly wave sum (every lane ends
// with the same total). rstd = rsqrt(sum / K + eps).
KRQ_DEV float rstd_of(float lane_sum, int64_t K, float eps) {
  return rsqrtf(wave_sum(lane_sum) / (float)K + eps);
}

// Row kernels (one block of kRowThreads per row, rows of up to kRowMaxK elements): the x and ln
// chunks are loaded into registers first and the row's partials staged in LDS with independent
// loads, so the whole prologue is one memory round trip. C = 16-byte chunks per thread (2 for
// rows of up to 4,096 elements, else kRowChunks).
constexpr int kRowThreads = 256;
constexpr int kRowChunks = 8;
constexpr int kRowMaxK = 8 * kRowThreads * kRowChunks;  // 16,384
constexpr int kRowSmallK = 8 * kRowThreads * 2;         // 4,096

// rstd[m] for m < M from the [M][T] partials staged in LDS (sst): one wave per row.
KRQ_DEV void row_rstd(const float* sst, int M, int T, int64_t K, float eps, float* rstd) {
  const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  for (int m = threadIdx.x >> 6; m < M; m += nw) {
    float a = 0.0f;
    for (int t = lane; t < T; t += 64) a += sst[m * T + t];
    const float r = rstd_of(a, K, eps);
    if (lane == 0) rstd[m] = r;
  }
}

// Row prologue of the row kernels: loads row m's x and ln chunks (chunk c of this thread covers
// elements 8 * (threadIdx.x + c * kRowThreads)), stages the row's T partials in sst and returns
// rstd (every thread). Chunks past K hold a repeat of the last one.
// ROWSUM (one row): the partials are the row's own chunk sums (sumsq8), staged for the same
// canonical sum; sst then holds K / 8 <= kRowThreads * C floats.
template <int C, bool ROWSUM = false>
KRQ_DEV float row_prologue(const uint16_t* __restrict__ x, const float* __restrict__ ss_in,
                           const uint16_t* __restrict__ ln, float eps, int64_t K, int m, float* sst,
                           float* rstd_sh, uint4* xv, uint4* lv) {
  const int T = (int)(K >> 4);
  const uint8_t* xr = reinterpret_cast<const uint8_t*>(x + m * K);
  const uint8_t* lr = reinterpret_cast<const uint8_t*>(ln);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t e = min(8 * (int64_t)(threadIdx.x + c * kRowThreads), K - 8);
    xv[c] = ld16(xr + 2 * e);
    lv[c] = ld16(lr + 2 * e);
  }
  if constexpr (ROWSUM) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int i = threadIdx.x + c * kRowThreads;
      if (8 * (int64_t)i < K) sst[i] = sumsq8(xv[c]);
    }
    __syncthreads();
    row_rstd(sst, 1, (int)(K >> 3), K, eps, rstd_sh);
    __syncthreads();
    return *rstd_sh;
  }
  constexpr int kSp = C / 2;  // partials per thread: T = K / 16 <= kRowThreads * C / 2
  float sp[kSp];
#pragma unroll
  for (int j = 0; j < kSp; ++j) sp[j] = ss_in[(int64_t)m * T + min((int)threadIdx.x + j * kRowThreads, T - 1)];
#pragma unroll
  for (int j = 0; j < kSp; ++j)
    if ((int)threadIdx.x + j * kRowThreads < T) sst[threadIdx.x + j * kRowThreads] = sp[j];
  __syncthreads();
  row_rstd(sst, 1, T, K, eps, rstd_sh);
  __syncthreads();
  return *rstd_sh;
}

// Residual values a thread of row block rb's residual epilogue adds, res_in at the rows and
// columns it finishes (clamped to row M - 1), loaded at kernel start so their latency hides under
// the weight stream.
template <int MT>
struct ResidualPre {
  uint16_t v[MT * 4];
};
template <int MT>
KRQ_DEV ResidualPre<MT> load_residual(const FusedArgs& fa, int M, int64_t NO, int64_t rb) {
  constexpr int NV = MT * 256;
  ResidualPre<MT> p;
  const int NT = blockDim.x;
#pragma unroll
  for (int q = 0; q < MT * 4; ++q) {
    const int v = min((int)threadIdx.x + q * NT, NV - 1);
    const int ln = v & 63, m = (v >> 8) * 16 + 4 * (ln >> 4) + ((v >> 6) & 3);
    p.v[q] = fa.res_in[(int64_t)min(m, M - 1) * NO + rb * 16 + (ln & 15)];
  }
  return p;
}

// Residual epilogue of one row block rb (P == 1 accumulators in red). One split's value is
// (sum over waves) * xs[m] * wsc, as the partials epilogue writes it. With S > 1 splits each split
// writes its partial tile to part [S][M][NO] with write-through stores, waits for them, and bumps
// cnt[rb]; the split that brings the count to S sums the S partials in split order, finishes the
// tile and zeroes the counter. last_s: a shared word. rp: this thread's residual values
// (load_residual), or null to read them here. Called by every thread of the block.
template <int MT>
KRQ_DEV void residual_epilogue(const float* red, int nw, int M, int64_t NO, int64_t rb, int sidx, int S,
                               const float* xs, float wsc, float* part, const FusedArgs& fa,
                               uint32_t* last_s, const ResidualPre<MT>* rp = nullptr) {
  constexpr int NV = MT * 256;
  constexpr int VPT = NV / 64;  // values per thread at most (blockDim.x >= 64)
  const int NT = blockDim.x;
  float av[VPT];
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int v = threadIdx.x + q * NT;
    float a = 0.0f;
    if (v < NV) {
      for (int w2 = 0; w2 < nw; ++w2) a += red[w2 * NV + v];
      const int ln = v & 63, m = (v >> 8) * 16 + 4 * (ln >> 4) + ((v >> 6) & 3);
      a = a * xs[m] * wsc;
    }
    av[q] = a;
  }
  if (S > 1) {
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      const int v = threadIdx.x + q * NT;
      if (v >= NV) continue;
      const int ln = v & 63, m = (v >> 8) * 16 + 4 * (ln >> 4) + ((v >> 6) & 3);
      if (m < M)
        cstore(reinterpret_cast<uint32_t*>(part + ((int64_t)sidx * M + m) * NO + rb * 16 + (ln & 15)), as_u32(av[q]));
    }
    stores_done();
    __syncthreads();
    if (threadIdx.x == 0) *last_s = cadd(&fa.cnt[rb], 1u) == (uint32_t)(S - 1);
    __syncthreads();
    if (!*last_s) return;
  }
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int v = threadIdx.x + q * NT;  // uniform per wave: NT and NV are multiples of 64
    if (v >= NV) continue;
    const int ln = v & 63, m = (v >> 8) * 16 + 4 * (ln >> 4) + ((v >> 6) & 3);
    const int mm = min(m, M - 1);
    const int64_t n = rb * 16 + (ln & 15);
    float y = av[q];
    if (S > 1) {
      y = 0.0f;
      for (int s2 = 0; s2 < S; ++s2)
        y += s2 == sidx ? av[q] : as_f32(cload(reinterpret_cast<const uint32_t*>(part + ((int64_t)s2 * M + mm) * NO + n)));
    }
    const uint16_t rv = rp ? rp->v[q] : fa.res_in[(int64_t)mm * NO + n];
    const float xn = round_bf16(bf16_to_f32(rv) + round_bf16(y));
    if (m < M) fa.res_out[(int64_t)m * NO + n] = f32_to_bf16(xn);
    float sq = xn * xn;  // the 16 lanes sharing (mt, i, g) hold the 16 columns of one row
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) sq += __shfl_xor(sq, o, kWave);
    if (m < M && (ln & 15) == 0) fa.ss_out[(int64_t)m * (NO >> 4) + rb] = sq;
  }
  if (S > 1 && threadIdx.x == 0) cstore(&fa.cnt[rb], 0u);
}

// Residual epilogue of folded one-row block b (kOutResidualFold; P == 1, MT == 1 accumulators in
// red): quarter q's sum for output column 4 b + j is C[q][4 q + j], element q of lane 4 q + j.
// Each quarter is summed over the waves and scaled as residual_epilogue scales a split's value,
// the four are added in split order, and the residual row is finished as there. No sum of squares
// is written (one-row consumers sum their row themselves).
KRQ_DEV void fold_residual_epilogue(const float* red, int nw, int64_t b, const float* xs, const float* wsc,
                                    int w_per_row, const FusedArgs& fa) {
  if (threadIdx.x >= 4) return;
  const int j = threadIdx.x;
  const int64_t n = 4 * b + j;
  const float ws = wsc[w_per_row ? n : 0];
  float y = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float a = 0.0f;
    for (int w2 = 0; w2 < nw; ++w2) a += red[w2 * 256 + q * 64 + 4 * q + j];
    y += a * xs[0] * ws;
  }
  const float xn = round_bf16(bf16_to_f32(fa.res_in[n]) + round_bf16(y));
  fa.res_out[n] = f32_to_bf16(xn);
}

// block of launch planning shared by the GEMV entry points
struct Plan {
  int nw;  // waves per block
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Waves per block for a block of nsteps steps over P weight matrices with U step slots per wave,
// in a grid of `blocks` blocks (act_wave: weight waves beside the one-row kernel's activation
// wave). Overridable (for launch-shape sweeps) by the environment variable KRQ_GEMV_WAVES.
int plan_waves(int nsteps, int P, int U, int64_t blocks, bool act_wave = false);

// Validated launches shared by the C ABI entry points (gemv_fp8.hip, gemv_bf16.hip); mode may
// also be kOutArgmax (then split == 1, aux = [M][N/16] Best, out = optional bf16 logits).
int gemv_fp8_run(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                 const void* w8, int w_layout, const float* w_scale, int w_per_row, int64_t M,
                 int64_t N, int64_t K, int split, int mode, int algo, void* out, void* aux,
                 void* stream);
int gemv_bf16_run(const void* x, const void* w, int w_layout, int64_t M, int64_t N, int64_t K,
                  int split, int mode, void* out, void* aux, void* stream);

// Second stage of a chained MLP: scalar polls (which do not queue behind the vector memory
// traffic of the weight stream) of this workgroup's replica of the first stage's done flag, at
// most fa.max_polls of them. False if it gave up; the error word is then set. Every thread of the
// calling wave calls it.
KRQ_DEV bool chain_wait(const FusedArgs& fa) {
  // (an address held in scalar registers)
  const uint32_t* rep = fa.cnt + kChainRep + kChainRepStride * static_cast<int>(blockIdx.x % kChainReps);
  uint32_t polls = 0, done = 0;
  for (;;) {
    // the load and its wait in one statement, the destination early-clobber (a load in flight
    // still writes its register)
    asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=&s"(done) : "s"(rep) : "memory");
    if (done != 0 || ++polls > fa.max_polls) break;
    __builtin_amdgcn_s_sleep(1);
  }
  if (done == 0 && (threadIdx.x & 63) == 0) cstore(fa.cnt + kChainErr, 1u);
  return done != 0;
}

// End of a chained-MLP block (every thread of the block, or every thread of its wave 0, calls it).
// First stage: once every thread's act stores have completed, one arrival on the block's group
// counter; the group's last arrival counts the group complete, and the last group complete sets
// every replica of the done flag (one store per lane of wave 0). Second stage: one exit on its
// group; the group's last exit counts the group done, and the last group done zeroes every control
// word. By then every second-stage block has passed its wait, so no word is read again in this
// launch. (Counters that only grow, with the launch number published instead of a flag, need no
// zeroing but measured slower: 32 against 19 us per Qwen3-4B MLP.)
template <bool FIRST>
KRQ_DEV void chain_tail(const FusedArgs& fa) {
  const int g = static_cast<int>(blockIdx.x) % kChainGroups;
  const int lane = threadIdx.x & 63;
  // workgroups lo .. hi - 1 whose index is q mod kChainGroups
  auto in_group = [](int q, int lo, int hi) {
    const int first = lo + ((q - lo % kChainGroups) % kChainGroups + kChainGroups) % kChainGroups;
    return first < hi ? (hi - 1 - first) / kChainGroups + 1 : 0;
  };
  auto groups_of = [&](int lo, int hi) {
    int n = 0;
    for (int q = 0; q < kChainGroups; ++q) n += in_group(q, lo, hi) > 0 ? 1 : 0;
    return n;
  };
  if constexpr (FIRST) {
    stores_done();
    __syncthreads();
  }
  if (threadIdx.x >= 64) return;
  uint32_t last = 0;
  if (lane == 0) {
    const int lo = FIRST ? 0 : fa.n_first, hi = FIRST ? fa.n_first : fa.n_first + fa.n_second;
    if (cadd(fa.cnt + 64 * g + (FIRST ? 0 : 1), 1u) == static_cast<uint32_t>(in_group(g, lo, hi) - 1))
      last = cadd(fa.cnt + (FIRST ? kChainArr : kChainExit), 1u) == static_cast<uint32_t>(groups_of(lo, hi) - 1);
  }
  if (!__shfl(last, 0, kWave)) return;
  if constexpr (FIRST) {
    cstore(fa.cnt + kChainRep + kChainRepStride * lane, 1u);
  } else {
    cstore(fa.cnt + kChainRep + kChainRepStride * lane, 0u);
    if (lane < 2 * kChainGroups) cstore(fa.cnt + 64 * (lane >> 1) + (lane & 1), 0u);
    if (lane == 0) {
      cstore(fa.cnt + kChainArr, 0u);
      cstore(fa.cnt + kChainExit, 0u);
    }
  }
}

}  // namespace krq
