// FP8 prefill GEMM (M > 32): y = bf16((x8 . w8^T) * x_scale[m] * w_scale[n]), fp32 accumulate -
// the product the reference computes with torch._scaled_mm in linear_fp8 (engine/kernels/fp8.py
// :97-106) for prefill (engine/engine.py:670-677).
//
// Tiles. A block owns a 128 x 128 output tile and walks K in steps of 128 bytes; its four waves
// each own a 64 x 64 quarter, a 4 x 4 grid of v_mfma_f32_16x16x128_f8f6f4 products (lane l holds
// 32 bytes of row l % 16 of each operand fragment; the k order inside a lane is the same for A
// and B, which is all the product needs - gemv_common.h). The A (activation) and B (weight) tiles
// of a step are staged in LDS with 16 bytes of padding per 128-byte row, so the sixteen rows a
// fragment read touches fall in distinct banks; the next step's tiles are loaded into registers
// while the current one is multiplied.
//
// Activations arrive as e4m3 (KRQ_X_FP8, with their scale) or as bf16 with an inverse scale
// (KRQ_X_BF16_STATIC: ActScale / SharedScale): the block then quantizes its A tile on the way
// into LDS, e4m3(clamp(x * inv)), the reference's cast fused into the GEMM.
#include "gemv_common.h"

using namespace krq;

namespace {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int kThreads = 256;
constexpr int kLds = BK + 16;  // LDS row stride (bytes)

template <int XK>
__global__ __launch_bounds__(kThreads) void k_gemm_fp8(const uint8_t* __restrict__ a, const float* __restrict__ asc,
                                                       const float* __restrict__ ainv, int a_per_row,
                                                       const uint8_t* __restrict__ b, const float* __restrict__ bsc,
                                                       int b_per_row, int M, int N, int K, int tiles_m,
                                                       uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint8_t As[BM * kLds];
  __shared__ __align__(16) uint8_t Bs[BN * kLds];
  constexpr bool ABF = XK == KRQ_X_BF16_STATIC;
  constexpr int AC = ABF ? 8 : 4;  // 16-byte A chunks per thread per step (bf16: twice the bytes)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
  const int nsteps = K / BK;

  // global -> register staging: B chunk c of this thread = row (tid >> 3) + 32 c, bytes 16 (tid & 7);
  // A likewise in e4m3 bytes, or (bf16) row (tid >> 4) + 16 c, elements 8 (tid & 15)
  uint4 ra[AC], rb[4];
  auto load_step = [&](int s) {
    const int64_t k0 = (int64_t)s * BK;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = (tid >> 3) + 32 * c;
      rb[c] = ld16nt(b + (int64_t)(n0 + row) * K + k0 + 16 * (tid & 7));
    }
#pragma unroll
    for (int c = 0; c < AC; ++c) {
      if (ABF) {
        const int row = min(m0 + (tid >> 4) + 16 * c, M - 1);
        ra[c] = ld16(a + 2 * ((int64_t)row * K + k0 + 8 * (tid & 15)));
      } else {
        const int row = min(m0 + (tid >> 3) + 32 * c, M - 1);
        ra[c] = ld16(a + (int64_t)row * K + k0 + 16 * (tid & 7));
      }
    }
  };
  const float inv = ABF ? ainv[0] : 0.0f;
  auto store_step = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<uint4*>(Bs + ((tid >> 3) + 32 * c) * kLds + 16 * (tid & 7)) = rb[c];
#pragma unroll
    for (int c = 0; c < AC; ++c) {
      if (ABF) {
        const int row = (tid >> 4) + 16 * c;
        const float iv = a_per_row ? ainv[min(m0 + row, M - 1)] : inv;
        *reinterpret_cast<uint2*>(As + row * kLds + 8 * (tid & 15)) = quant8(ra[c], iv);
      } else {
        *reinterpret_cast<uint4*>(As + ((tid >> 3) + 32 * c) * kLds + 16 * (tid & 7)) = ra[c];
      }
    }
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  load_step(0);
  for (int s = 0; s < nsteps; ++s) {
    __syncthreads();  // the previous step's fragment reads are done
    store_step();
    __syncthreads();
    load_step(min(s + 1, nsteps - 1));  // the last step reloads itself (unused), keeping loads unconditional
    v8i fb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint8_t* pb = Bs + (wn + 16 * j + r) * kLds + 16 * g;
      fb[j] = pack_v8i(*reinterpret_cast<const uint4*>(pb), *reinterpret_cast<const uint4*>(pb + 64));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // one A fragment live at a time
      const uint8_t* pa = As + (wm + 16 * i + r) * kLds + 16 * g;
      const v8i fa = pack_v8i(*reinterpret_cast<const uint4*>(pa), *reinterpret_cast<const uint4*>(pa + 64));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fa, fb[j], acc[i][j], 0, 0, 0, 0, 0, 0);
    }
  }

  // epilogue: acc[i][j] element e = C[wm + 16 i + 4 g + e][wn + 16 j + r]
  float sa[4][4], sb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) sa[i][e] = asc[a_per_row ? min(m0 + wm + 16 * i + 4 * g + e, M - 1) : 0];
#pragma unroll
  for (int j = 0; j < 4; ++j) sb[j] = bsc[b_per_row ? n0 + wn + 16 * j + r : 0];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + wm + 16 * i + 4 * g + e;
      if (m < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          out[(int64_t)m * N + n0 + wn + 16 * j + r] = f32_to_bf16(acc[i][j][e] * sa[i][e] * sb[j]);
      }
    }
}

}  // namespace

extern "C" int krq_gemm_fp8(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                            const void* w8, const float* w_scale, int w_per_row, int64_t M, int64_t N, int64_t K,
                            void* out, void* stream) {
  KRQ_REQUIRE(x && w8 && w_scale && x_scale && out, "gemm_fp8: null pointer");
  KRQ_REQUIRE(x_kind == KRQ_X_FP8 || x_kind == KRQ_X_BF16_STATIC, "gemm_fp8: x_kind must be FP8 or BF16_STATIC");
  KRQ_REQUIRE(x_kind != KRQ_X_BF16_STATIC || x_inv, "gemm_fp8: x_inv is required");
  KRQ_REQUIRE(aligned16(x) && aligned16(w8), "gemm_fp8: x and w8 must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 0x7fffffff && N > 0 && N <= 0x7fffffff && N % BN == 0 && K > 0 && K <= 0x7fffffff &&
                  K % BK == 0,
              "gemm_fp8: shape M=%lld N=%lld K=%lld (N and K multiples of 128)", (long long)M, (long long)N,
              (long long)K);
  const int tiles_m = static_cast<int>((M + BM - 1) / BM);
  const int64_t blocks = (int64_t)tiles_m * (N / BN);
  KRQ_REQUIRE(blocks <= 0x7fffffff, "gemm_fp8: grid too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t s = (hipStream_t)stream;
  if (x_kind == KRQ_X_FP8)
    hipLaunchKernelGGL(k_gemm_fp8<KRQ_X_FP8>, grid, dim3(kThreads), 0, s, (const uint8_t*)x, x_scale, x_inv, x_per_row,
                       (const uint8_t*)w8, w_scale, w_per_row, (int)M, (int)N, (int)K, tiles_m, (uint16_t*)out);
  else
    hipLaunchKernelGGL(k_gemm_fp8<KRQ_X_BF16_STATIC>, grid, dim3(kThreads), 0, s, (const uint8_t*)x, x_scale, x_inv,
                       x_per_row, (const uint8_t*)w8, w_scale, w_per_row, (int)M, (int)N, (int)K, tiles_m,
                       (uint16_t*)out);
  return krq_check_launch("gemm_fp8");
}
