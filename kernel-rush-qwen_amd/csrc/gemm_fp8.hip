// FP8 prefill GEMM (M > 32): y = bf16((x8 . w8^T) * x_scale[m] * w_scale[n]), fp32 accumulate -
// the product the reference computes with torch._scaled_mm in linear_fp8 (engine/kernels/fp8.py
// :97-106) for prefill (engine/engine.py:670-677).
//
// Two kernels. k_gemm_ring (below) takes e4m3 activations with K >= 256: persistent blocks, an LDS
// ring of direct global->LDS loads, 256 x 256 / 192 x 256 / 128 x 128 / 64 x 64 tiles and split K
// for small grids.
// k_gemm_fp8 takes the rest (K = 128, or bf16 activations cast on the way into LDS): a block owns
// a 128 x 128 output tile and walks K in steps of 128 bytes; its four waves each own a 64 x 64
// quarter, a 4 x 4 grid of v_mfma_f32_16x16x128_f8f6f4 products (lane l holds 32 bytes of row
// l % 16 of each operand fragment; the k order inside a lane is the same for A and B, which is
// all the product needs - gemv_common.h). Its A (activation) and B (weight) tiles of a step are
// staged in LDS with 16 bytes of padding per 128-byte row, so the sixteen rows a fragment read
// touches fall in distinct banks; the next step's tiles are loaded into registers while the
// current one is multiplied. With bf16 activations and an inverse scale (KRQ_X_BF16_STATIC:
// ActScale / SharedScale) the block quantizes its A tile on the way into LDS, e4m3(clamp(x * inv)),
// the reference's cast fused into the GEMM.
#include <type_traits>

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

// ---- ring kernel: e4m3 A, BM x BN tiles fed by an LDS ring of direct (DMA) loads ----
//
// The block's four waves own (BM/2) x (BN/2) quarters, a grid of 32 x 32 outputs each computed by
// v_mfma_f32_32x32x64_f8f6f4 with the B (weight) fragment as its first operand (lane l holds 32
// bytes of row l % 32 of each operand fragment, k bytes 32 (l / 32) .. +31 of the 64-byte stage;
// the product's element e of lane l belongs to first-operand row 8 (e / 4) + 4 (l / 32) + e % 4 and
// second-operand row l % 32). K advances 64 bytes per stage; stages come in pairs whose 128 bytes
// of each row fill one of two LDS pair buffers. Global bytes reach LDS with
// global_load_lds_dwordx4: one instruction writes 1 KB, 8 rows of 128 bytes (whole lines), lane i
// at byte 16 i, so a lane's global address picks which 16-byte chunk of which row lands at that
// position. Chunk c of row r sits at position c ^ ((r >> 1) & 7) of its row: a ds_read_b128 serves
// 16 lanes (256 bytes) per cycle, and the 16 rows those lanes read then start on 16 distinct
// 16-byte bank groups. (With 64-byte rows, one stage per buffer and a chunk taken from row bits
// 1-2, rows r and r + 8 collided and half the LDS cycles were conflicts; loading a line's two
// halves with separate instructions sent both to L2.)
//
// Per pair of stages (2j, 2j + 1): the even stage multiplies from registers and reads the odd
// stage's fragments; the odd stage waits for the next pair's loads, passes a barrier (every wave's
// loads have landed and every wave is done with pair j's buffer), issues the loads of pair j + 2
// into that buffer, reads the next even stage's fragments and multiplies. Past the last stage the
// loads go to a sink (one cached KB, same count).
namespace ring {

constexpr int BK = 64, kThreads = 256;
typedef float v16f __attribute__((ext_vector_type(16)));

// 32-bit LDS address of a pointer into a __shared__ array, as a wave-uniform value
KRQ_DEV uint32_t lds_addr(const uint8_t* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)p)));
}

// global_load_lds_dwordx4: 16 bytes per lane from base + voff into LDS at l + 16 * lane (base
// wave-uniform, voff a 32-bit per-lane byte offset). Issued from inline assembly so that the
// compiler, which cannot tell the ring's buffers apart once a loop holds more of these loads than
// it tracks, does not wait for every load in flight before each LDS read; the kernel waits for
// them itself (wait_vm). Other global loads the compiler adds (spill reloads) only make those
// waits stricter: vector memory operations complete in order.
// (s_nop 0: an LDS DMA reading M0 right after a scalar write of it needs one wait state on this
// generation - the compiler inserts it for its own instructions, not inside assembly)
KRQ_DEV void dma16s(const uint8_t* base, uint32_t voff, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(voff), "s"(base)
               : "memory", "m0");
}

// global_load_lds_dword: 4 bytes per lane from g into LDS at l + 4 * lane (waited for like dma16s)
KRQ_DEV void dma4(const float* g, uint32_t l) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(l), "v"(g) : "memory", "m0");
}

template <int N>
KRQ_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// workgroup barrier ordering LDS accesses only (the ring's global loads are waited for explicitly)
KRQ_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// scheduling pattern of a stage: product U, then its share of the NR fragment reads
template <int U, int NP, int NR>
struct StagePattern {
  static KRQ_DEV void apply() {
    if constexpr (U < NP) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      constexpr int c = (U + 1) * NR / NP - U * NR / NP;
      if constexpr (c > 0) __builtin_amdgcn_sched_group_barrier(0x100, c, 0);
      StagePattern<U + 1, NP, NR>::apply();
    }
  }
};

// PART: each work unit is (tile, split): the tile's products over K / splits bytes of K, written
// as fp32 to plane `split` of ws [splits][M][N] (k_splitk_reduce finishes them); otherwise one
// unit per tile over all of K, written as bf16 with its scales applied.
template <int BM, int BN, int OCC, bool PART>
__global__ __launch_bounds__(kThreads, OCC) void k_gemm_ring(const uint8_t* __restrict__ a, const float* __restrict__ asc,
                                                           int a_per_row, const uint8_t* __restrict__ b,
                                                           const float* __restrict__ bsc, int b_per_row, int M, int N,
                                                           int K, int tiles_m, int tiles, int splits, int ldo,
                                                           float* __restrict__ ws, uint16_t* __restrict__ out) {
  constexpr int kPairBytes = (BM + BN) * 2 * BK;  // two stages: 128 bytes of K per row, A rows then B rows
  __shared__ __align__(1024) uint8_t ring[2 * kPairBytes];
  __shared__ __align__(1024) float scl[2][BM + BN];  // per tile (alternating): row scales, then column scales
  __shared__ __align__(1024) uint8_t sink[1024];     // where the loads of stages past the last one land
  constexpr int FI = BM / 64, FJ = BN / 64;          // 32-row fragments of a wave's quarter
  constexpr int QA = BM / 32, QB = BN / 32;          // 1 KB loads (8 rows x 128 B) per wave per pair
  constexpr int kVm = QA + QB;
  constexpr int NF = FI + FJ;                  // fragments per stage, two 16-byte reads each
  constexpr int kSI = (BM + BN) / 64;          // 64-scale loads per tile
  constexpr int kScl = (kSI + 3) / 4;          // per wave (the surplus goes to the sink)
  constexpr int EB = PART ? 4 : 2;             // output element bytes
  constexpr int RB = BN / 2 * EB;              // bytes per row of a wave's output quarter
  constexpr int CPR = RB / 16;                 // 16-byte chunks per such row
  constexpr int kStores = FI * 32 * CPR / 64;  // 16-byte stores per lane per tile
  constexpr int CR = kPairBytes >= 4 * 32 * RB ? 32 : 16;  // output rows per staging chunk
  static_assert((BM + BN) % 64 == 0, "scale loads");
  static_assert(kVm + kStores < 64, "vmcnt range");
  static_assert(4 * CR * RB <= kPairBytes, "output staging fits one pair buffer");
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, bid = blockIdx.x;
  const int wm = (wave & 1) * (BM / 2), wn = (wave >> 1) * (BN / 2);
  const int nk = K / BK / splits;  // stages of a work unit (even)
  const int units = tiles * splits;

  // This block's k-th work unit (unit u: tile u % tiles, split u / tiles): units in order, tiles
  // M-fastest; in each round of G units the blocks of one XCD (b, b + 8, ...) take a contiguous
  // run of them.
  auto tile_of = [&](int k) {
    const int base = k * G;
    if (base + bid >= units) return -1;
    if ((G & 7) == 0 && units - base >= G) return base + (bid & 7) * (G >> 3) + (bid >> 3);
    return base + bid;
  };

  // load q of this wave covers rows 8 (wave + 4 q) .. + 7 of A (q < QA) or of B, 128 bytes of K
  // each: lane -> row + lane / 8, position lane % 8 of the row. Addresses are a wave-uniform base
  // (the tile's first A or B row, its split's first K byte) plus a 32-bit offset per lane (the
  // operands are below 2 GiB, checked at launch).
  int m0 = 0, n0 = 0, sp = 0;
  const uint8_t* abase = a;
  const uint8_t* bbase = b;
  uint32_t goff[kVm];
  auto set_tile = [&](int u) {
    const int p = u % tiles;
    sp = u / tiles;
    m0 = (p % tiles_m) * BM;
    n0 = (p / tiles_m) * BN;
    const int64_t kb = (int64_t)sp * nk * BK;
    abase = a + (int64_t)m0 * K + kb;
    bbase = b + (int64_t)n0 * K + kb;
    // ln: the lane index made opaque here, so that these offsets are computed per tile instead of
    // hoisted out of the tile loop and kept live across it (they were, and spilled to scratch;
    // without any scratch gate_up at M = 4096 went from 202 to 175 us)
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int row = 8 * (wave + 4 * q) + (ln >> 3);
      goff[q] = static_cast<uint32_t>((min(m0 + row, M - 1) - m0) * K + 16 * ((ln & 7) ^ ((row >> 1) & 7)));
    }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int row = 8 * (wave + 4 * q) + (ln >> 3);
      goff[QA + q] = static_cast<uint32_t>(row * K + 16 * ((ln & 7) ^ ((row >> 1) & 7)));
    }
  };
  const uint32_t lbase = lds_addr(ring) + 1024 * wave, lsink = lds_addr(sink);
  const uint32_t lscl = lds_addr(reinterpret_cast<const uint8_t*>(&scl[0][0]));
  // load q of pair j (stages 2j and 2j + 1) into pair buffer pb, or past the last stage the same
  // count of loads of one cached KB of B into the sink, chosen without a branch so that every
  // odd stage issues the same loads and waits alike
  auto pair_load = [&](int q, int j, int pb) {
    const bool real = 2 * j < nk;
    dma16s(real ? (q < QA ? abase : bbase) + j * 2 * BK : b, real ? goff[q] : 16u * lane,
           real ? lbase + pb * kPairBytes + (q < QA ? 4096 * q : BM * 2 * BK + 4096 * (q - QA)) : lsink);
  };
  // the tile's scales (kScl loads of 64 per wave; a per-tensor scale is loaded by every lane), then
  // its first pair of stages into pair buffer 0
  auto tile_loads = [&](int sb) {
#pragma unroll
    for (int k = 0; k < kScl; ++k) {
      const int li = 4 * k + wave, e = li * 64 + lane;
      dma4(e < BM ? asc + (a_per_row ? min(m0 + e, M - 1) : 0) : bsc + (b_per_row ? min(n0 + e - BM, N - 1) : 0),
           li < kSI ? lscl + 4 * (sb * (BM + BN) + li * 64) : lsink);
    }
#pragma unroll
    for (int q = 0; q < kVm; ++q) pair_load(q, 0, 0);
  };

  // Fragment f (A for f < FI, else B) of stage s: row (lane & 31) of its 32-row block, the 64-byte
  // half s % 2 of the row's 128 bytes, logical chunks 2 (lane >> 5) (hh = 0) and + 1 (hh = 1) of
  // that half. Chunk c (0 .. 7) of row r sits at c ^ ((r >> 1) & 7): the 16 rows a ds_read_b128
  // phase reads then start on 16 distinct 16-byte bank groups.
  const int sw = ((lane & 31) >> 1) & 7;
  int off[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) off[h][hh] = (lane & 31) * 2 * BK + 16 * ((4 * h + 2 * (lane >> 5) + hh) ^ sw);
  uint4 fh[2][NF][2];
  auto read = [&](int set, int f, int hh, int h, int pb) {
    const uint8_t* p =
        ring + pb * kPairBytes + (f < FI ? (wm + 32 * f) * 2 * BK : BM * 2 * BK + (wn + 32 * (f - FI)) * 2 * BK);
    fh[set][f][hh] = *reinterpret_cast<const uint4*>(p + off[h][hh]);
  };
  v16f acc[FI][FJ];

  // One stage s (register set s % 2): its products, the 2 NF reads of stage s + 1's fragments
  // (pair buffer pbn, half (s + 1) % 2) into the other set spread evenly after them, and for an odd
  // stage the loads of the pair after next (stages s + 3 and s + 4) into pair buffer pbl, the one
  // stages s - 1 and s used, spread the same way. An even stage's data arrived with the odd
  // stage's before it, so only odd stages wait and pass a barrier. The last stage reads and loads
  // nothing.
  constexpr int NP = FI * FJ, NR = 2 * NF, NL = kVm;
  auto body = [&](auto par_c, auto loads_c, auto reads_c, int s, int pbn, int pbl) __attribute__((always_inline)) {
    constexpr int set = decltype(par_c)::value;
    constexpr bool LOADS = decltype(loads_c)::value, READS = decltype(reads_c)::value;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int i = u / FJ, j = u % FJ;
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          pack_v8i(fh[set][FI + j][0], fh[set][FI + j][1]), pack_v8i(fh[set][i][0], fh[set][i][1]), acc[i][j], 0, 0,
          0, 0, 0, 0);
      if (LOADS) {
#pragma unroll
        for (int l = u * NL / NP; l < (u + 1) * NL / NP; ++l) pair_load(l, (s + 3) / 2, pbl);
      }
      if (READS) {
#pragma unroll
        for (int r = u * NR / NP; r < (u + 1) * NR / NP; ++r) read(set ^ 1, r >> 1, r & 1, set ^ 1, pbn);
      }
    }
    if (READS) StagePattern<0, NP, NR>::apply();
  };
  using yes = std::true_type;
  using no = std::false_type;
  using even = std::integral_constant<int, 0>;
  using odd = std::integral_constant<int, 1>;

  // Epilogue. acc[i][j] element e of lane l is the output at row m = wm + 32 i + l % 32 and column
  // n = wn + 32 j + 8 (e / 4) + 4 (l / 32) + e % 4 (B is the first product operand): a lane holds
  // four adjacent columns of a row. Pair buffer 1 is idle here (the next tile's first loads fill
  // buffer 0), so each wave stages CR rows of its quarter at a time in its own part of it (rows of
  // BN bytes, 16-byte chunk c of row r at c ^ (r % (BN / 16))), 8 bytes per lane, then reads them
  // back along rows and stores 16 bytes per lane: each store writes whole row segments. The stores
  // drain while the block's next tile runs. Rounding to bf16 is the hardware convert (nearest
  // even, as f32_to_bf16 for every non-NaN value).
  auto epilogue = [&](int cm0, int cn0, int csp, const float* sc) {
    int le = lane;  // opaque for the same reason as in set_tile
    asm volatile("" : "+v"(le));
    uint8_t* tq = ring + kPairBytes + wave * CR * RB;
    const int r = le & 31;
#pragma unroll
    for (int i = 0; i < FI; ++i) {
      const float sav = sc[wm + 32 * i + r];
#pragma unroll
      for (int h = 0; h < 32 / CR; ++h) {
        if (r / CR == h) {
          const int rl = r % CR;
#pragma unroll
          for (int j = 0; j < FJ; ++j)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              if constexpr (PART) {
                const int c = 8 * j + 2 * g4 + (le >> 5);  // 16-byte chunk of the quarter's row
                *reinterpret_cast<float4*>(tq + rl * RB + 16 * (c ^ (rl & (CPR - 1)))) =
                    make_float4(acc[i][j][4 * g4 + 0], acc[i][j][4 * g4 + 1], acc[i][j][4 * g4 + 2],
                                acc[i][j][4 * g4 + 3]);
              } else {
                const int n = wn + 32 * j + 8 * g4 + 4 * (le >> 5);
                const float4 sb4 = *reinterpret_cast<const float4*>(sc + BM + n);
                const uint32_t lo =
                    pack_bf16x2(acc[i][j][4 * g4 + 0] * sav * sb4.x, acc[i][j][4 * g4 + 1] * sav * sb4.y);
                const uint32_t hi =
                    pack_bf16x2(acc[i][j][4 * g4 + 2] * sav * sb4.z, acc[i][j][4 * g4 + 3] * sav * sb4.w);
                const int c = 4 * j + g4;  // 16-byte chunk of the quarter's row
                *reinterpret_cast<uint2*>(tq + rl * RB + 16 * (c ^ (rl & (CPR - 1))) + 8 * (le >> 5)) =
                    make_uint2(lo, hi);
              }
            }
        }
#pragma unroll
        for (int it = 0; it < CR * CPR / 64; ++it) {
          const int rr = it * (64 / CPR) + le / CPR, c = le % CPR;
          const uint4 v = *reinterpret_cast<const uint4*>(tq + rr * RB + 16 * (c ^ (rr & (CPR - 1))));
          const int m = cm0 + wm + 32 * i + CR * h + rr;
          if (m < M) {
            if constexpr (PART)
              *reinterpret_cast<uint4*>(ws + ((int64_t)csp * M + m) * N + cn0 + wn + 4 * c) = v;
            else  // streamed past the caches: nothing reads it back in this launch
              __builtin_nontemporal_store(v4u{v.x, v.y, v.z, v.w},
                                          reinterpret_cast<v4u*>(out + (int64_t)m * ldo + cn0 + wn + 8 * c));
          }
        }
      }
    }
  };

  int p = tile_of(0);
  if (p < 0) return;
  set_tile(p);
  tile_loads(0);
  bool ragged = false;  // the previous tile had rows past M
  for (int k = 0;; ++k) {
    // The second pair goes into buffer 1 once every wave is done with the previous epilogue's
    // staging. In flight, oldest first: the scales and the first pair, the previous tile's stores
    // (k > 0), the second pair. A tile whose rows all lie below M issued exactly kStores stores per
    // lane; one with rows past M may have issued fewer (a wave whose chunk rows are all past M
    // branches around its store), so after such a tile the wait counts only the second pair.
    lds_barrier();
#pragma unroll
    for (int q = 0; q < kVm; ++q) pair_load(q, 1, 1);
    if (k == 0 || ragged) wait_vm<kVm>();
    else wait_vm<kVm + kStores>();
    lds_barrier();
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      read(0, f, 0, 0, 0);
      read(0, f, 1, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int j = 0; j < FJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    const int cm0 = m0, cn0 = n0, csp = sp;
    const int next = tile_of(k + 1);
    for (int s = 0; s < nk - 2; s += 2) {
      const int pb = (s >> 1) & 1;
      body(even{}, no{}, yes{}, s, pb, 0);
      wait_vm<0>();  // the pair of stages s + 2, s + 3
      lds_barrier();
      body(odd{}, yes{}, yes{}, s + 1, pb ^ 1, pb);
    }
    body(even{}, no{}, yes{}, nk - 2, ((nk - 2) >> 1) & 1, 0);
    // last stage: once every wave is past this barrier the ring is free; the next tile starts loading
    lds_barrier();
    if (next >= 0) {
      set_tile(next);
      tile_loads((k + 1) & 1);
    }
    body(odd{}, no{}, no{}, nk - 1, 0, 0);
    epilogue(cm0, cn0, csp, scl[k & 1]);
    ragged = cm0 + BM > M;
    if (next < 0) break;
  }
  wait_vm<0>();  // no load into LDS outlives the block
}

// out[m][n] = bf16((sum over s of ws[s][m][n], s in order) * x_scale[m] * w_scale[n]), four
// columns per thread
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, int splits, int M, int N,
                                                       const float* __restrict__ asc, int a_per_row,
                                                       const float* __restrict__ bsc, int b_per_row,
                                                       uint16_t* __restrict__ out) {
  const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t plane = (int64_t)M * N;
  if (e >= plane) return;
  const int m = static_cast<int>(e / N), n = static_cast<int>(e % N);
  float4 acc = *reinterpret_cast<const float4*>(ws + e);
  for (int sp = 1; sp < splits; ++sp) {
    const float4 v = *reinterpret_cast<const float4*>(ws + sp * plane + e);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  const float sa = asc[a_per_row ? m : 0];
  const float4 sb = b_per_row ? *reinterpret_cast<const float4*>(bsc + n) : make_float4(bsc[0], bsc[0], bsc[0], bsc[0]);
  *reinterpret_cast<uint2*>(out + e) =
      make_uint2(pack_bf16x2(acc.x * sa * sb.x, acc.y * sa * sb.y), pack_bf16x2(acc.z * sa * sb.z, acc.w * sa * sb.w));
}

}  // namespace ring

// 192 x 256 tiles (three 32-row fragments per wave) fill the compute units where 256 x 256 ones
// leave many idle: M = 4096 with N = 2560 gives 220 tiles instead of 160, each 0.75 of the work.
//
// Tile shape of the ring kernel for an e4m3 GEMM, a pure function of the shape and the device's
// compute-unit count. Measured at the Qwen3-4B projections (M = 256 .. 4096): a round of
// 256 x 256 tiles (one block per compute unit) takes about 1.45x as long as a round of two
// 128 x 128 tiles on each compute unit, and does twice their products (gate_up at M = 4096: 175 us
// for 5 rounds; QKV: 68 us for 2 rounds against 76 us for 3 of 128 x 128); 128 x 256 tiles were
// never faster than one of the two. The plan takes the one with fewer estimated round-lengths,
// counting the tiles of the busiest compute unit (128 x 128 ones two at a time). It picks the
// faster of the measured kernels at the shapes of the prefill bench. The 128 x 128 ring kernel also beat the
// register-staged one on grids of 40 tiles (M = 256: O 15.8 against 41.0 us, down 44.8 against
// 93.4), so bm == 0 only where N is not a multiple of 128.
//
// Split K: a 128 x 128 grid of fewer tiles than compute units, with K of at least 8 KB, splits K
// into `splits` equal parts (the most of 8, 4, 2 with an even number of 64-byte stages and at
// least 2 KB of K per part) when the parts then number at least half the compute units and the
// fp32 partials (splits x M x N x 4 bytes, written once and read once) are no more bytes than the
// weights (N x K). Otherwise such a grid runs 64 x 64 tiles, four blocks per compute unit, split by
// the same rules where 128 x 128 ones could not be. Measured (us, Qwen3-4B shapes):
//   down (K = 9728): M = 256 44.5 -> 16.0 + 4.8 (128 x 128 in 4 parts; 27.3 in 2), M = 1024
//     49.3 -> 38.5 (2 parts), M = 128 34.0 -> 15.6 and M = 64 19.1 -> 13.5 (64 x 64 in 4 parts);
//   O (K = 4096) gained from no split: 64 x 64 tiles took M = 256 from 14.4 to 9.9 us, where 2 parts
//     of 64 x 64 took 12.7 and 2 of 128 x 128 16.8; M = 1024 22.6 -> 20.3;
//   QKV (K = 2560) at M = 256: 64 x 64 tiles 11.2 -> 10.2, 2 parts 18.5.
struct RingPlan {
  int bm, bn, occ, splits;
  int tail;  // 256 x 256: whole rounds over the first columns, then 128 x 128 tiles over the rest
};
RingPlan ring_plan(int64_t M, int64_t N, int64_t K, int cus) {
  const int64_t t256 = N % 256 == 0 ? ((M + 255) / 256) * (N / 256) : 0;
  const int64_t t192 = N % 256 == 0 ? ((M + 191) / 192) * (N / 256) : 0;
  const int64_t t128 = N % 128 == 0 ? ((M + 127) / 128) * (N / 128) : 0;
  const double c256 = (double)((t256 + cus - 1) / cus);                   // rounds of 256 x 256
  const double c192 = 0.75 * (double)((t192 + cus - 1) / cus);            // 192-row tiles
  const double c128 = 0.70 * (double)(((t128 + cus - 1) / cus + 1) / 2);  // two blocks per unit
  const bool ok256 = t256 >= cus / 2, ok192 = t192 >= cus / 2;
  // whole rounds of 256 x 256 tiles, when they cover whole columns of tiles, then the rest of the
  // columns in 128 x 128 tiles (two per unit): a partial round of 256 x 256 tiles at up to half the
  // chip costs a whole one, as 128 x 128 tiles 0.7 of one
  const int64_t r256 = t256 / cus, rest = t256 % cus, tm256 = (M + 255) / 256;
  const double ctail = (double)r256 + 0.70 * (double)((2 * rest + cus - 1) / cus);
  const bool tail = r256 >= 1 && rest > 0 && (r256 * cus) % tm256 == 0 && t128 > 0;
  if (ok192 && c192 < c256 && (t128 == 0 || c192 <= c128) && !(tail && ctail < c192)) return {192, 256, 1, 1, 0};
  if (tail && ctail < c256 && ctail < c128) return {256, 256, 1, 1, 1};
  if (ok256 && (t128 == 0 || c256 <= c128)) return {256, 256, 1, 1, 0};
  if (t128 == 0) return {0, 0, 0, 0, 0};
  if (t128 >= cus) return {128, 128, 2, 1, 0};
  // the most parts (8, 4, 2) a grid of `tiles` may split K into, or 1
  auto parts = [&](int64_t tiles) {
    const int64_t nk = K / 64;
    if (K < 8192) return 1;
    for (int sp = 8; sp >= 2; sp /= 2)
      if (nk % (2 * sp) == 0 && K / sp >= 2048 && sp * M * 4 <= K && tiles * sp >= cus / 2) return sp;
    return 1;
  };
  const int s128 = parts(t128);
  if (s128 > 1) return {128, 128, 2, s128, 0};
  return {64, 64, 4, parts(((M + 63) / 64) * (N / 64)), 0};
}

int query_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || *cus <= 0)
    return KRQ_EHIP;
  return KRQ_OK;
}

// the ring kernels take e4m3 activations and K of at least four 64-byte stages
bool ring_fits(int x_kind, int64_t K) { return x_kind == KRQ_X_FP8 && K % 128 == 0 && K >= 256; }

int gemm_run(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row, const void* w8,
             const float* w_scale, int w_per_row, int64_t M, int64_t N, int64_t K, void* ws, int64_t ws_bytes,
             void* out, void* stream) {
  KRQ_REQUIRE(x && w8 && w_scale && x_scale && out, "gemm_fp8: null pointer");
  KRQ_REQUIRE(x_kind == KRQ_X_FP8 || x_kind == KRQ_X_BF16_STATIC, "gemm_fp8: x_kind must be FP8 or BF16_STATIC");
  KRQ_REQUIRE(x_kind != KRQ_X_BF16_STATIC || x_inv, "gemm_fp8: x_inv is required");
  KRQ_REQUIRE(aligned16(x) && aligned16(w8), "gemm_fp8: x and w8 must be 16-byte aligned");
  KRQ_REQUIRE(M >= 1 && M <= 0x7fffffff && N > 0 && N <= 0x7fffffff && N % BN == 0 && K > 0 && K <= 0x7fffffff &&
                  K % BK == 0,
              "gemm_fp8: shape M=%lld N=%lld K=%lld (N and K multiples of 128)", (long long)M, (long long)N,
              (long long)K);
  KRQ_REQUIRE(ws_bytes >= 0 && (ws_bytes == 0 || ws), "gemm_fp8: workspace pointer and size disagree");
  const int tiles_m = static_cast<int>((M + BM - 1) / BM);
  const int64_t blocks = (int64_t)tiles_m * (N / BN);
  KRQ_REQUIRE(blocks <= 0x7fffffff, "gemm_fp8: grid too large");
  hipStream_t s = (hipStream_t)stream;
  if (ring_fits(x_kind, K) && aligned16(out) && M * K < 0x7fffffff && N * K < 0x7fffffff) {
    int cus = 0;
    KRQ_REQUIRE(query_cus(&cus) == KRQ_OK, "gemm_fp8: device query failed");
    RingPlan rp = ring_plan(M, N, K, cus);
    if (rp.splits > 1 && (!aligned16(ws) || ws_bytes < (int64_t)rp.splits * M * N * 4)) rp.splits = 1;
    if (rp.bm > 0) {
      // one launch over columns [n_lo, n_hi) of the output (ldo = N)
#define KRQ_RING(BM_, BN_, OCC_, PART_, n_lo, n_hi)                                                                  \
  do {                                                                                                             \
    const int64_t nn = (n_hi) - (n_lo), tm_ = (M + (BM_)-1) / (BM_), tiles_ = tm_ * (nn / (BN_));                   \
    const int64_t units_ = tiles_ * rp.splits, slots_ = (int64_t)cus * (OCC_);                                     \
    hipLaunchKernelGGL((ring::k_gemm_ring<BM_, BN_, OCC_, PART_>), dim3(static_cast<unsigned>(units_ < slots_ ? units_ : slots_)), \
                       dim3(ring::kThreads), 0, s, (const uint8_t*)x, x_scale, x_per_row,                           \
                       (const uint8_t*)w8 + (n_lo) * K, w_scale + (w_per_row ? (n_lo) : 0), w_per_row, (int)M,     \
                       (int)nn, (int)K, (int)tm_, (int)tiles_, rp.splits, (int)N, (float*)ws,                       \
                       (uint16_t*)out + (n_lo));                                                                   \
  } while (0)
      if (rp.bm == 256 && rp.tail) {
        // the whole rounds' tiles (M-fastest) fill whole columns of tiles: the first n_split columns
        const int64_t tm256 = (M + 255) / 256, rounds = (N / 256) * tm256 / cus;
        const int64_t n_split = rounds * cus / tm256 * 256;
        KRQ_RING(256, 256, 1, false, 0, n_split);
        KRQ_RING(128, 128, 2, false, n_split, N);
      } else if (rp.bm == 256) {
        KRQ_RING(256, 256, 1, false, 0, N);
      } else if (rp.bm == 192) {
        KRQ_RING(192, 256, 1, false, 0, N);
      } else if (rp.bm == 64 && rp.splits == 1) {
        KRQ_RING(64, 64, 4, false, 0, N);
      } else if (rp.bm == 64) {
        KRQ_RING(64, 64, 4, true, 0, N);
        const int64_t threads = M * N / 4;
        hipLaunchKernelGGL(ring::k_splitk_reduce, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s,
                           (const float*)ws, rp.splits, (int)M, (int)N, x_scale, x_per_row, w_scale, w_per_row,
                           (uint16_t*)out);
      } else if (rp.splits == 1) {
        KRQ_RING(128, 128, 2, false, 0, N);
      } else {
        KRQ_RING(128, 128, 2, true, 0, N);
        const int64_t threads = M * N / 4;
        hipLaunchKernelGGL(ring::k_splitk_reduce, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s,
                           (const float*)ws, rp.splits, (int)M, (int)N, x_scale, x_per_row, w_scale, w_per_row,
                           (uint16_t*)out);
      }
#undef KRQ_RING
      return krq_check_launch("gemm_fp8");
    }
  }
  const dim3 grid(static_cast<unsigned>(blocks));
  if (x_kind == KRQ_X_FP8)
    hipLaunchKernelGGL(k_gemm_fp8<KRQ_X_FP8>, grid, dim3(kThreads), 0, s, (const uint8_t*)x, x_scale, x_inv, x_per_row,
                       (const uint8_t*)w8, w_scale, w_per_row, (int)M, (int)N, (int)K, tiles_m, (uint16_t*)out);
  else
    hipLaunchKernelGGL(k_gemm_fp8<KRQ_X_BF16_STATIC>, grid, dim3(kThreads), 0, s, (const uint8_t*)x, x_scale, x_inv,
                       x_per_row, (const uint8_t*)w8, w_scale, w_per_row, (int)M, (int)N, (int)K, tiles_m,
                       (uint16_t*)out);
  return krq_check_launch("gemm_fp8");
}

}  // namespace

extern "C" int krq_gemm_fp8(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                            const void* w8, const float* w_scale, int w_per_row, int64_t M, int64_t N, int64_t K,
                            void* out, void* stream) {
  return gemm_run(x, x_kind, x_scale, x_inv, x_per_row, w8, w_scale, w_per_row, M, N, K, nullptr, 0, out, stream);
}

extern "C" int krq_gemm_fp8_ws(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                               const void* w8, const float* w_scale, int w_per_row, int64_t M, int64_t N, int64_t K,
                               void* ws, int64_t ws_bytes, void* out, void* stream) {
  return gemm_run(x, x_kind, x_scale, x_inv, x_per_row, w8, w_scale, w_per_row, M, N, K, ws, ws_bytes, out, stream);
}

extern "C" int64_t krq_gemm_fp8_ws_bytes(int x_kind, int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N <= 0 || K <= 0 || N % BN != 0 || K % BK != 0 || !ring_fits(x_kind, K)) return 0;
  int cus = 0;
  if (query_cus(&cus) != KRQ_OK) return -1;
  const RingPlan rp = ring_plan(M, N, K, cus);
  return rp.splits > 1 ? (int64_t)rp.splits * M * N * 4 : 0;
}
