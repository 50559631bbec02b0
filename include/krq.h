/*
 * krq.h - C ABI of libkrq.so, the gfx950 (MI355X) decode-matmul path for Qwen3-4B shapes.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and a hipStream_t passed as void*;
 *   - allocates nothing and never synchronises the host, so it can be captured into a hipGraph;
 *   - returns KRQ_OK (0) on success, KRQ_EINVAL for a bad shape or argument (raised as
 *     ValueError / AssertionError by the Python layer, mirroring the reference), or KRQ_EHIP for a
 *     HIP launch error (raised as RuntimeError). krq_last_error() gives the message of the
 *     calling thread's last failure.
 *
 * Data formats:
 *   bf16      - IEEE bfloat16 bit patterns (uint16), row-major.
 *   e4m3      - OCP FP8 E4M3 "fn" bytes (max 448, no infinities, NaN = 0x7F/0xFF), i.e. the
 *               values of torch.float8_e4m3fn.
 *   tiled     - the FP8 weight copy read by the GEMV kernels. A [N, K] matrix is cut into
 *               16-row x 64-byte tiles, stored tile-row-major ([N/16][K/64]); inside a tile,
 *               lane l (0..63) owns the 16 contiguous bytes of row (l % 16), columns
 *               64*t + 16*(l / 16) .. +16. One 64-lane 128-bit load reads one whole tile (1 KiB,
 *               contiguous). Needs N % 16 == 0 and K % 64 == 0. krq_unpack_fp8 inverts it.
 *   partials  - split-K output: fp32 [split, M, N]; the consumer sums slices 0..split-1 in that
 *               order and rounds once to bf16 (reference engine/kernels/ops.py:29-39).
 */
#ifndef KRQ_H
#define KRQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KRQ_OK 0
#define KRQ_EINVAL (-1)
#define KRQ_EHIP (-2)

/* GEMV output modes */
#define KRQ_OUT_BF16 0     /* bf16 [M, N]; split must be 1 */
#define KRQ_OUT_PARTIAL 1  /* fp32 [split, M, N] */
#define KRQ_OUT_SWIGLU 2   /* w = [gate; up] with 2*I rows; bf16 [M, I] = bf16(bf16(silu(g)) * u) */

/* weight layouts for the FP8 GEMV */
#define KRQ_W_ROWMAJOR 0
#define KRQ_W_TILED 1

/* activation kinds of the FP8 GEMV */
#define KRQ_X_FP8 0          /* x is e4m3 [M,K]; x_scale holds its scale (per row or tensor) */
#define KRQ_X_BF16_DYN 1     /* x is bf16 [1,K]; the per-token scale is computed in the kernel */
#define KRQ_X_BF16_STATIC 2  /* x is bf16 [M,K]; quantized with x_inv, scaled by x_scale */
#define KRQ_X_FP8_TILED 3    /* x is e4m3 in the tiled activation layout of krq_quant_rows_tiled,
                                with its scale */

/* lm-head weight kinds */
#define KRQ_LM_BF16 0
#define KRQ_LM_FP8 1
#define KRQ_LM_FP8_TILED_H 2  /* FP8 weights, h e4m3 in the tiled activation layout */

/*
 * Per-output-channel weight quantizer. Replaces the weight-packing step of engine loading
 * (reference engine/engine.py:496-501) with the per-row form the reference's experiments call as
 * fp8.quantize (experiments/modal_fp8.py:59-60; row formula experiments/modal_fq.py:62-63, clamp
 * convention experiments/i8.py:11-17):
 *   amax[n]  = max_k |w[n,k]|;  scale[n] = max(amax[n], 1e-12) * fp32(1/448)
 *   w8[n,k]  = e4m3_rne(clamp(float(w[n,k]) / scale[n], -448, 448))     (IEEE division)
 * w_bf16 rows are ldw elements apart. w8 (row-major [N,K], may be NULL) and w8_tiled (may be
 * NULL) receive the same bytes in the two layouts; at least one must be given.
 */
int krq_quant_fp8_rows(const void* w_bf16, int64_t N, int64_t K, int64_t ldw,
                       void* w8, void* w8_tiled, float* scale, void* stream);

/*
 * Per-tensor weight quantizer: quantize_weight (reference engine/kernels/fp8.py:17-23).
 *   scale0 = max(max|w|, 1e-12) * fp32(1/448);  w8 = e4m3_rne(clamp(float(w) / scale0, +-448))
 * row_amax_ws: caller workspace of N floats (overwritten).
 */
int krq_quant_fp8_tensor(const void* w_bf16, int64_t N, int64_t K, int64_t ldw,
                         float* row_amax_ws, void* w8, void* w8_tiled, float* scale0,
                         void* stream);

/*
 * Activation scale: ActScale (reference engine/kernels/fp8.py:26-35).
 *   amax = max(max|x|, 1e-6) * headroom;  inv = fp32(1/amax) * 448;  scale = amax * fp32(1/448)
 * per_row = 0: one scale for the whole [M,K] tensor (amax, inv, scale hold 1 float each);
 *              ws must hold at least krq_act_scale_ws_floats(M, K) floats.
 * per_row = 1: one scale per row (amax, inv, scale hold M floats each); ws may be NULL.
 */
int krq_act_scale(const void* x_bf16, int64_t M, int64_t K, int per_row, float headroom,
                  float* amax, float* inv, float* scale, float* ws, void* stream);
int64_t krq_act_scale_ws_floats(int64_t M, int64_t K);

/*
 * FP8 cast: _cast_kernel / _cast_torch (reference engine/kernels/fp8.py:38-56).
 *   x8[m,k] = e4m3_rne(clamp(float(x[m,k]) * inv[per_row ? m : 0], -448, 448))
 */
int krq_cast_fp8(const void* x_bf16, int64_t M, int64_t K, const float* inv, int per_row,
                 void* x8, void* stream);

/*
 * krq_act_scale (per tensor) then krq_cast_fp8 with its inverse: the first two steps of linear_fp8
 * without a given scale (reference engine/kernels/fp8.py:97-104: a = ActScale(x), then _cast(x, a)).
 * The same amax, inv, scale and bytes, in two launches where the alignment allows (the fold of the
 * partial maxima runs inside the cast), else three. ws: krq_act_scale_ws_floats(M, K) floats.
 */
int krq_act_scale_cast_fp8(const void* x_bf16, int64_t M, int64_t K, float headroom, float* amax, float* inv,
                           float* scale, float* ws, void* x8, void* stream);

/*
 * Per-token dynamic quantization in one launch: fp8.quant_rows as called by the reference's
 * experiments/modal_fp8.py:84-85 (x8, xs for torch._scaled_mm scale_a); ActScale per row plus
 * the cast above. xs[m] = scale of row m (amax[m]/448 as above).
 */
int krq_quant_rows(const void* x_bf16, int64_t M, int64_t K, void* x8, float* xs, void* stream);

/*
 * krq_quant_rows with the e4m3 rows written in the tiled activation layout the FP8 GEMV reads
 * as KRQ_X_FP8_TILED (no reference counterpart: the same bytes as quant_rows, permuted, for the
 * gemv_fp8 / gemv_swiglu_fp8 calls of experiments/modal_fp8.py:67-69 at M > 1): rows padded to
 * MP = 16 * ceil(M / 16) (pad rows zero), split into 16-row x 64-byte tiles in the order
 * [MP / 16][K / 64]; inside a tile, lane l = 16 g + r holds row r's bytes 16 g .. 16 g + 15.
 * x8_tiled holds MP * K bytes; K % 64 == 0. xs as krq_quant_rows (M values).
 */
int krq_quant_rows_tiled(const void* x_bf16, int64_t M, int64_t K, void* x8_tiled, float* xs, void* stream);
/* krq_cast_fp8 with a given per-tensor inverse (ActScale / SharedScale, the static scales of the
 * engine's FP8 decode, engine/engine.py:977-981 through linear_fp8) written in that tiled layout:
 * the bytes of _cast(x, a) (reference engine/kernels/fp8.py:52-56) permuted, pad rows zero, for the
 * GEMV on KRQ_X_FP8_TILED rows at 1 < M <= 32. Same shape rules as krq_quant_rows_tiled. */
int krq_cast_fp8_tiled(const void* x_bf16, int64_t M, int64_t K, const float* inv, void* x8_tiled, void* stream);

/*
 * FP8 skinny GEMM/GEMV, M <= 32: replaces linear_fp8 -> torch._scaled_mm (reference
 * engine/kernels/fp8.py:97-106) at decode sizes, and supplies gemv_fp8 / gemv_swiglu_fp8 as
 * called by experiments/modal_fp8.py:67-69 under the output contract of gemv / gemv_swiglu
 * (engine/kernels/gemv.py:83-88, :125-130, :137-167).
 *   x8[m,k]  = x (x_kind KRQ_X_FP8), or e4m3(clamp(x[m,k] * inv, +-448)) computed in the kernel:
 *              inv = x_inv[m or 0] (KRQ_X_BF16_STATIC), or the per-token ActScale inverse of row
 *              0 (KRQ_X_BF16_DYN, M == 1; amax over all of K)
 *   acc[m,n] = sum_k x8[m,k] * w8[n,k]   (fp32 accumulate)
 *   y[m,n]   = acc[m,n] * xs[m] * w_scale[n or 0], xs = x_scale[m or 0] or the in-kernel scale
 * w8: e4m3 [N,K] (or [2I,K] for SWIGLU) in layout w_layout.
 * mode KRQ_OUT_BF16 -> bf16 [M,N] (split 1); KRQ_OUT_PARTIAL -> fp32 [split,M,N] of the K-slices
 * [s*K/split, (s+1)*K/split); KRQ_OUT_SWIGLU -> bf16 [M,I] (split 1).
 * Needs N % 16 == 0, K % split == 0 and (K/split) % 64 == 0; the in-kernel kinds need the
 * activation slice to fit a block of at most 8 64-thread waves: K <= 16384 for DYN (2048
 * elements per wave), M*K/split <= 32768 for STATIC (4096 per wave).
 * algo: 0 = automatic, 1 = matrix-core (MFMA) kernel, 2 = vector-ALU kernel (M == 1 only).
 */
int krq_gemv_fp8(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                 const void* w8, int w_layout, const float* w_scale, int w_per_row,
                 int64_t M, int64_t N, int64_t K, int split, int mode, int algo,
                 void* out, void* stream);

/*
 * The FP8 SwiGLU GEMV with the next projection's input cast in its epilogue: the engine's
 * static-scale decode MLP (reference engine/engine.py:977-981) computes
 * act = silu_mul(linear_fp8(h, gu8, a_gu)) (ops.py:164-172) and then linear_fp8(act, down8, a_down),
 * whose first step is _cast(act, a_down) (fp8.py:38-56, :104). Here, in one launch:
 *   act[m,i]    = krq_gemv_fp8's KRQ_OUT_SWIGLU output (bf16), never stored;
 *   x8_tiled    = e4m3(clamp(float(act) * out_inv[0], +-448)) in the tiled activation layout of
 *                 krq_quant_rows_tiled (rows padded to 16 * ceil(M / 16), pad rows 0): the bytes of
 *                 krq_cast_fp8(act, out_inv) permuted into that layout.
 * The down projection then reads x8_tiled as KRQ_X_FP8_TILED with a_down's scale. Arguments as
 * krq_gemv_fp8 (M <= 32, split 1); N = 2I with I % 64 == 0; out_inv: device fp32 [1].
 */
int krq_gemv_swiglu_fp8_cast(const void* x, int x_kind, const float* x_scale, const float* x_inv,
                             int x_per_row, const void* w8, int w_layout, const float* w_scale, int w_per_row,
                             int64_t M, int64_t N, int64_t K, const float* out_inv, void* x8_tiled,
                             void* stream);

/*
 * BF16 skinny GEMM/GEMV, M <= 32: gemv / gemv_m1 / gemv_swiglu / gemv_m1_swiglu
 * (reference engine/kernels/gemv.py:43-266).
 *   acc = x[M,K] . w[N,K]^T in fp32; modes as krq_gemv_fp8.
 * w_layout KRQ_W_ROWMAJOR: bf16 [N,K]; KRQ_W_TILED: the tiled layout above applied to the [N, 2K]
 * byte matrix (made by krq_pack_fp8(w, N, 2K, w_tiled)).
 * Needs N % 16 == 0, K % split == 0 and (K/split) % 32 == 0.
 */
int krq_gemv_bf16(const void* x, const void* w, int w_layout, int64_t M, int64_t N, int64_t K,
                  int split, int mode, void* out, void* stream);

/*
 * Persistent BF16 GEMV: gemv_rows(x, w, programs, swiglu) (reference engine/kernels/gemv.py:334-348,
 * kernel :276-331; the engine's rows1 / rows2 candidates, engine.py:147-148). Exactly `programs`
 * workgroups; workgroup p owns output rows [p N / programs, (p + 1) N / programs) over the full K.
 *   out[M, N] = bf16(x[M,K] . w[N,K]^T), or with swiglu != 0 (w = [gate; up], [2N, K]) the
 *   SwiGLU of gemv_swiglu; w row-major bf16. The result does not depend on `programs`.
 * Needs 1 <= M <= 32, K % 32 == 0, programs >= 1.
 */
int krq_gemv_bf16_rows(const void* x, const void* w, int64_t M, int64_t N, int64_t K, int programs,
                       int swiglu, void* out, void* stream);

/*
 * LM head + greedy argmax: logits = bf16(h . E^T) and idx[m] = lowest index of the maximum bf16
 * logit of row m. Reference: engine/engine.py:1021-1022 (gemv(h, lm_head, 1) then torch.argmax)
 * and the fused form engine/kernels/mega.py:396-441. Two launches (GEMV with an argmax epilogue,
 * then a per-row fold).
 * w_kind KRQ_LM_BF16: h bf16 [M,K], w bf16 [V,K] in w_layout (row-major, or tiled as for
 *                     krq_gemv_bf16); h_scale / w_scale unused.
 * w_kind KRQ_LM_FP8:  w e4m3 [V,K] in w_layout with w_scale[V] (w_per_row = 1, per channel) or
 *                     w_scale[1] (w_per_row = 0, per tensor: the engine's quantize_weight lm8,
 *                     engine.py:504-505); h e4m3 [M,K] with h_scale[M] (h_per_row = 1, per token)
 *                     or h_scale[1] (h_per_row = 0, one scale: linear_fp8's ActScale or a
 *                     SharedScale, engine.py:989), or (h_scale NULL, M == 1) h bf16 [1,K] scaled
 *                     per token inside the kernel; logits as krq_gemv_fp8 KRQ_OUT_BF16.
 * w_kind KRQ_LM_FP8_TILED_H: as KRQ_LM_FP8 with h e4m3 in the tiled activation layout of
 *                     krq_quant_rows_tiled and its h_scale (no reference counterpart: the same
 *                     operands, contiguous loads).
 * logits: optional bf16 [M,V] output (NULL to skip). ws: scratch of at least
 * krq_lmhead_ws_bytes(M, V) bytes (overwritten; calls that overlap must not share it).
 */
int krq_lmhead_argmax(const void* h, const float* h_scale, int h_per_row, const void* w, int w_kind,
                      int w_layout, const float* w_scale, int w_per_row, int64_t M, int64_t V, int64_t K,
                      void* logits, void* ws, int64_t ws_bytes, int64_t* idx_out, void* stream);
int64_t krq_lmhead_ws_bytes(int64_t M, int64_t V);

/*
 * krq_lmhead_argmax without the workspace argument: the call allocates nothing. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Arguments and results are those
 * of krq_lmhead_argmax. The argmax candidates go to a scratch array of KRQ_LMHEAD_SCRATCH_BYTES
 * that the library holds on each GPU it runs on until the process ends; a call whose
 * krq_lmhead_ws_bytes(M, V) exceeds it is refused with KRQ_EINVAL (4 MiB: every M <= 32 at the
 * Qwen3 vocabulary of 151,936). stream must belong to the current device. The first call on a
 * device resolves the array's address there (hipGetSymbolAddress; no allocation): a caller that
 * captures the call into a graph makes one call on that device beforehand. Every call on one GPU
 * shares its array, so calls that overlap on one GPU (two streams, two threads) race.
 */
#define KRQ_LMHEAD_SCRATCH_BYTES 4194304
int krq_lmhead_argmax_noalloc(const void* h, const float* h_scale, int h_per_row, const void* w, int w_kind,
                              int w_layout, const float* w_scale, int w_per_row, int64_t M, int64_t V,
                              int64_t K, void* logits, int64_t* idx_out, void* stream);

/*
 * Fused decode MLP, one launch: replaces PersistentMLP (reference engine/kernels/mlp.py:22-118,
 * called at engine/engine.py:911-915 and :1015) for FP8 weights, M <= 32.
 *   act[m,i]   = SwiGLU as krq_gemv_fp8 KRQ_OUT_SWIGLU of x with w_gu (e4m3 [2I,H] = [gate; up])
 *   out[s,m,h] = fp32 partial of act . w_down^T over i in [s*I/split, (s+1)*I/split), with act
 *                quantized per token (amax of the whole act row, the arithmetic of quant_rows)
 *                and w_down e4m3 [H,I]; the consumer sums the partials in order s = 0..split-1.
 * x: e4m3 [M,H] with x_scale[M] (KRQ_X_FP8), or bf16 [1,H] scaled per token in the kernel
 * (KRQ_X_BF16_DYN, M == 1). Both weights in w_layout with per-row (or per-tensor) scales.
 * act: bf16 [M,I] workspace (also an output: the SwiGLU activations).
 * ctl: krq_mlp_ctl_words() uint32 words, zero before the first call; the kernel leaves them zero
 *      again, except the last word, which it sets to 1 if a block waited too long for phase 1.
 *      Such a block writes NaN to every partial it owns, so an incomplete result never passes
 *      as data. Calls sharing ctl must not overlap.
 * programs: number of blocks (0 = one per CU); clamped to what the device holds at once.
 * Needs H % 64 == 0, I % 16 == 0, (I/split) % 64 == 0 and M*I/split within the kernel's staging
 * limit (raise split for large M).
 */
int krq_mlp_fp8(const void* x, int x_kind, const float* x_scale, const void* w_gu, int w_layout,
                const float* gu_scale, int gu_per_row, const void* w_down, const float* down_scale,
                int down_per_row, int64_t M, int64_t H, int64_t I, int split, void* act,
                uint32_t* ctl, int programs, void* out, void* stream);
/* krq_mlp_fp8 with the phase-1 wait bounded at max_polls polls instead of about a second's worth
 * (no counterpart in the reference: lets a test force the timeout path from the host). */
int krq_mlp_fp8_bounded(const void* x, int x_kind, const float* x_scale, const void* w_gu, int w_layout,
                        const float* gu_scale, int gu_per_row, const void* w_down, const float* down_scale,
                        int down_per_row, int64_t M, int64_t H, int64_t I, int split, void* act,
                        uint32_t* ctl, int programs, uint32_t max_polls, void* out, void* stream);
int64_t krq_mlp_ctl_words(void);

/*
 * The decode MLP at M == 1 in ONE launch, with the result of the default two-launch pair
 * (reference engine/kernels/mlp.py:22-118 PersistentMLP.__call__, as its consumer
 * engine/engine.py:911-915 uses it): act = SwiGLU(x . [gate; up]^T) (bf16 [1, I], bit-identical
 * to krq_gemv_fp8 KRQ_OUT_SWIGLU on the bf16 row), then out = the fp32 [split, 1, H] split-K
 * partials of act . w_down^T with act scaled per token (krq_gemv_fp8, KRQ_X_BF16_DYN).
 * Both weights KRQ_W_TILED with per-row (or per-tensor) scales; x bf16 [1, H].
 * The down workgroups issue their weight loads first and wait in the kernel for every gate_up
 * workgroup's act (a done flag in ctl, polled at most max_polls times, each poll one memory
 * round trip). The partial sums equal krq_gemv_fp8's to fp32 rounding (two weight waves per
 * split instead of one).
 * ctl: krq_mlp_chain_ctl_words() uint32 words, zero before the first call; every launch leaves
 *      them zero again, except word 513, which a wait that gave up sets to 1 (that block's
 *      partials are then NaN; zero ctl again before the next call). Calls sharing ctl must not
 *      overlap.
 * Needs H % 64 == 0, I % 64 == 0, (I/split) % 64 == 0, H and I at most 10240, and at most 20
 * steps of 128 elements per split (I/split <= 2560).
 */
int krq_mlp_chain_fp8(const void* x, const void* w_gu, const float* gu_scale, int gu_per_row,
                      const void* w_down, const float* down_scale, int down_per_row, int64_t H, int64_t I,
                      int split, void* act, uint32_t* ctl, uint32_t max_polls, void* out, void* stream);
int64_t krq_mlp_chain_ctl_words(void);

/*
 * The decode MLP on BF16 weights in ONE launch (reference engine/kernels/mlp.py:22-118
 * PersistentMLP.__call__ with the engine's bf16 weights, engine/engine.py:911-915): act =
 * SwiGLU(x . [gate; up]^T) (bf16 [M, I]) and out = the fp32 [split, M, H] split-K partials of
 * act . w_down^T, bit-identical to krq_gemv_bf16 KRQ_OUT_SWIGLU followed by krq_gemv_bf16
 * KRQ_OUT_PARTIAL: each stage runs the plan krq_gemv_bf16 gives it. x bf16 [M, H] (1 <= M <= 32);
 * w_gu [2I, H] and w_down [H, I] bf16, both in w_layout (KRQ_W_ROWMAJOR, or KRQ_W_TILED copies
 * from krq_pack_fp8 over 2K-byte rows). The down workgroups issue their first weight loads, then
 * wait for every gate_up workgroup's act (ctl and max_polls as krq_mlp_chain_fp8; a wait that
 * gives up sets word 513 and makes that block's partials NaN).
 * Needs H % 32 == 0, I % 16 == 0, (I/split) % 32 == 0, and fewer than 4096 down blocks
 * (H/16 * split) above 4 rows (krq_gemv_bf16 pairs row blocks there).
 */
int krq_mlp_chain_bf16(const void* x, const void* w_gu, const void* w_down, int w_layout, int64_t M, int64_t H,
                       int64_t I, int split, void* act, uint32_t* ctl, uint32_t max_polls, void* out, void* stream);

/*
 * BF16 GEMV with the RMSNorm prologue and the residual epilogue folded in: gemv_fused /
 * gemv_swiglu_fused (reference engine/kernels/fused_gemv.py:48-221, called at
 * engine/engine.py:953-961).
 *   ln != NULL (RMSNorm): x rows are normalized on the fly, h = bf16(bf16(x * rstd) * ln) with
 *                 rstd[m] = rsqrt(sum(ss_in[m][0..K/16)) / K + eps); ss_in is [M][K/16] fp32.
 *                 M == 1: the sum is the row's own sum of squares (every one-row normalizing
 *                 kernel, this one, krq_rmsnorm_rows, krq_rmsnorm_quant_rows(_tiled) and
 *                 krq_gemv_fp8_fused, takes it in one fixed order from x) and ss_in is not read.
 *   mode KRQ_OUT_BF16 / KRQ_OUT_PARTIAL / KRQ_OUT_SWIGLU: as krq_gemv_bf16, into out.
 *   mode KRQ_OUT_RESIDUAL: y = bf16(sum of the split partials in split order);
 *                 res_out = bf16(res_in + y) (bf16 [M][N]); ss_out[m][t] = sum over the 16
 *                 columns of tile t of res_out^2 (fp32 [M][N/16]); nothing is written to out
 *                 except, for split > 1, the fp32 [split][M][N] partials (scratch), and cnt
 *                 ([N/16] uint32, zero before the first call) is left zero again.
 * The per-tile sums of squares replace the reference's per-row atomic accumulator (same-address
 * atomics serialize on MI355X); every producer overwrites all N/16 tiles, so nothing needs zeroing.
 * krq_gemv_fused_fits() tells whether the block's K slice (and ss_in) fits the in-kernel staging;
 * otherwise normalize the rows with krq_rmsnorm_rows and call krq_gemv_bf16. Calls sharing cnt must
 * not overlap.
 */
#define KRQ_OUT_RESIDUAL 4
int krq_gemv_bf16_fused(const void* x, const void* w, int w_layout, int64_t M, int64_t N, int64_t K,
                        int split, int mode, const void* ln, const float* ss_in, float eps,
                        const void* res_in, void* res_out, float* ss_out, uint32_t* cnt, void* out,
                        void* stream);
int64_t krq_gemv_fused_fits(int64_t M, int64_t N, int64_t K, int split, int mode, int norm);
/* h = bf16(bf16(x * rstd) * ln) for whole bf16 rows x [M][K], rstd as above (M == 1: from x). */
int krq_rmsnorm_rows(const void* x, const float* ss_in, const void* ln, float eps, int64_t M, int64_t K,
                     void* h, void* stream);

/*
 * FP8 counterpart of krq_gemv_bf16_fused: the fused-GEMV semantics above (reference
 * engine/kernels/fused_gemv.py:48-167) on the FP8 weights and activation kinds of krq_gemv_fp8
 * (reference engine/kernels/fp8.py:17-106, the linear_fp8 call sites engine/engine.py:649-677).
 *   ln != NULL (RMSNorm; x_kind KRQ_X_BF16_DYN or KRQ_X_BF16_STATIC; modes BF16 / PARTIAL /
 *                 SWIGLU): h = bf16(bf16(x * rstd) * ln) as above, then h is scaled as the
 *                 x_kind says (DYN: per token over the whole normalized row, M == 1; STATIC:
 *                 x_inv / x_scale) and quantized to e4m3 in the kernel.
 *   mode KRQ_OUT_RESIDUAL (ln == NULL; any x_kind): one split's value is the scaled product
 *                 (x8 . w8) * x_scale[m] * w_scale[n], as the partials output holds it; then
 *                 y = bf16(sum over splits in split order) and res_out / ss_out / cnt / out as in
 *                 krq_gemv_bf16_fused. M == 1, split 4, bf16 activations (DYN or STATIC): the
 *                 folded launch (N / 4 workgroups, each four output columns over the four
 *                 quarters of K) computes the same four split values and y bit for bit with no
 *                 cross-workgroup sum; it needs neither cnt nor out and leaves ss_out alone
 *                 (one-row consumers take the sum of squares from the row).
 * krq_gemv_fp8_fused_fits() tells whether the in-kernel staging holds the launch; otherwise use
 * krq_rmsnorm_quant_rows (per token) or krq_rmsnorm_rows + a static cast, then krq_gemv_fp8 /
 * the residual mode with x_kind KRQ_X_FP8. Calls sharing cnt must not overlap.
 */
int krq_gemv_fp8_fused(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                       const void* w8, int w_layout, const float* w_scale, int w_per_row, int64_t M,
                       int64_t N, int64_t K, int split, int mode, const void* ln, const float* ss_in,
                       float eps, const void* res_in, void* res_out, float* ss_out, uint32_t* cnt,
                       void* out, void* stream);
int64_t krq_gemv_fp8_fused_fits(int64_t M, int64_t N, int64_t K, int split, int mode, int x_kind, int norm);
/* RMSNorm then per-token e4m3 quantization of whole rows: x8 [M][K] e4m3 and x_scale [M] equal
 * krq_quant_rows applied to krq_rmsnorm_rows' output (K <= 16384). */
int krq_rmsnorm_quant_rows(const void* x, const float* ss_in, const void* ln, float eps, int64_t M,
                           int64_t K, void* x8, float* x_scale, void* stream);
/* The same with x8 in the tiled activation layout of krq_quant_rows_tiled (16 * ceil(M / 16) rows,
 * pad rows zero; K % 64 == 0), read by the GEMVs as KRQ_X_FP8_TILED. */
int krq_rmsnorm_quant_rows_tiled(const void* x, const float* ss_in, const void* ln, float eps, int64_t M,
                                 int64_t K, void* x8_tiled, float* x_scale, void* stream);

/*
 * FP8 prefill GEMM (M > 32): out bf16 [M, N] = bf16((x8 . w8^T) * x_scale[m or 0] * w_scale[n or 0]),
 * fp32 accumulate - the torch._scaled_mm product of linear_fp8 (reference engine/kernels/fp8.py:
 * 97-106, prefill call site engine/engine.py:670-677). x_kind KRQ_X_FP8: x is e4m3 [M, K];
 * KRQ_X_BF16_STATIC: x is bf16 [M, K], quantized in the kernel as e4m3(clamp(x * x_inv)) (x_inv per
 * tensor, or per row with x_per_row). w8 row-major e4m3 [N, K]. N and K multiples of 128.
 * e4m3 rows with K >= 256 (and out 16-byte aligned) run the persistent ring kernels (256 x 256,
 * 192 x 256, 128 x 128 or 64 x 64 tiles, chosen from the shape and the device's compute units; a
 * partial last round of 256 x 256 tiles as 128 x 128 tiles in a second launch); other inputs a
 * 128 x 128 kernel with register-staged loads.
 */
int krq_gemm_fp8(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                 const void* w8, const float* w_scale, int w_per_row, int64_t M, int64_t N, int64_t K,
                 void* out, void* stream);

/* krq_gemm_fp8 with a caller workspace for split K (the same product, torch._scaled_mm in
 * engine/kernels/fp8.py:105-106): with e4m3 activations and a grid of fewer 128 x 128 tiles than
 * the device has compute units, K is split and fp32 partials go to ws before one more launch sums
 * them in split order and applies the scales. ws: at least krq_gemm_fp8_ws_bytes(x_kind, M, N, K)
 * bytes, 16-byte aligned (overwritten; calls that overlap must not share it); with a smaller ws (or
 * NULL, 0) K is not split. krq_gemm_fp8_ws_bytes returns 0 when no split is planned for the
 * current device and -1 when the device query fails. */
int krq_gemm_fp8_ws(const void* x, int x_kind, const float* x_scale, const float* x_inv, int x_per_row,
                    const void* w8, const float* w_scale, int w_per_row, int64_t M, int64_t N, int64_t K,
                    void* ws, int64_t ws_bytes, void* out, void* stream);
int64_t krq_gemm_fp8_ws_bytes(int x_kind, int64_t M, int64_t N, int64_t K);

/* Tiled <-> row-major weight copies (byte permutations; see "tiled" above). For a bf16 [N, K]
 * matrix pass its [N, 2K] byte view (K -> 2K). */
int krq_pack_fp8(const void* w8_rowmajor, int64_t N, int64_t K, void* w8_tiled, void* stream);
int krq_unpack_fp8(const void* w8_tiled, int64_t N, int64_t K, void* w8_rowmajor, void* stream);

const char* krq_version(void);
const char* krq_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KRQ_H */
