/*
 * tiq.h -- C ABI of libtiq_hip.so, the MI355X (gfx950) quantized-linear
 * library behind gpt2_harness_amd's quantize-and-run API.
 *
 * Conventions shared by every entry point:
 *   - all pointers are device pointers (hipMalloc / torch CUDA tensors) unless
 *     a comment says otherwise; matrices are row-major with an explicit
 *     leading dimension in elements;
 *   - a weight matrix is (rows = N = out_features, cols = K = in_features),
 *     the nn.Linear layout of the reference (model.py:201-204,333-334);
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream);
 *     every call only enqueues work on it and returns;
 *   - no entry point allocates device or host memory, keeps state between
 *     calls, or synchronises; calls on different streams are independent;
 *   - the return value is TIQ_OK (0) or a negative status; tiq_status_string
 *     names it. TIQ_EHIP_BASE - s means hipError_t s from the launch.
 *
 * Reference interfaces each entry point replaces are cited as
 * file:line under /src/transformer_internals of gpt2-harness.
 */
#ifndef TIQ_H
#define TIQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum tiq_status {
    TIQ_OK = 0,
    TIQ_EINVAL = -1,        /* bad size, null pointer, out-of-range argument   */
    TIQ_EBITS = -2,         /* bits outside [2, 8] (quantization.py:98-99)       */
    TIQ_EALIGN = -3,        /* pointer or leading dimension misaligned          */
    TIQ_EUNSUPPORTED = -4,  /* valid request the library has no kernel for     */
    TIQ_EWORKSPACE = -5,    /* workspace too small                              */
    TIQ_ESCRATCH = -6,      /* beyond the fixed scratch of tiq_decode_linear_noalloc */
    TIQ_EHIP_BASE = -1000   /* TIQ_EHIP_BASE - hipError_t                        */
};

enum tiq_dtype { TIQ_F32 = 0, TIQ_BF16 = 1 };

/* Weight storage formats accepted by tiq_linear_fused. */
enum tiq_weight_format {
    TIQ_WF_INT8 = 0,
    TIQ_WF_INT4 = 1,
    TIQ_WF_INT4_GROUPWISE = 2,
    TIQ_WF_F32 = 3,
    /* int8 codes rearranged by tiq_tile_int8 (tiq_decode_linear only) */
    TIQ_WF_INT8_TILED = 4,
    /* fp32 weights rearranged by tiq_tile_f32 (tiq_decode_linear from planes only) */
    TIQ_WF_F32_TILED = 5,
};

/* Activations fused after a linear. */
enum tiq_activation { TIQ_ACT_NONE = 0, TIQ_ACT_GELU_TANH = 1 };

/* Measurement of kernel durations inside a timed run (no counterpart in the
 * reference; for benchmark harnesses). Between tiq_stamp_begin(buf, slots)
 * and tiq_stamp_end every launch of the decode GEMV's direct kernel (int8
 * weights, bf16 activations and outputs) and of the staged prefill GEMM
 * (int8 weights, bf16 output) runs a stamped copy of the kernel that writes,
 * per workgroup g, its entry and exit time on the GPU's 100 MHz real-time
 * counter to buf[s + 4 g] and buf[s + 4 g + 1], and the same two moments on
 * the shader-clock counter to buf[s + 4 g + 2] and buf[s + 4 g + 3] (cycles
 * over real time: the clock the workgroup ran at), s being the launch's
 * first slot; launches beyond `slots` run unstamped. A launch captured in a HIP
 * graph keeps its slots, so every replay rewrites them. buf is a device
 * array of `slots` uint64 (NULL and 0: stamping off). Not thread safe with
 * launches from other threads. tiq_stamp_end turns stamping off and copies
 * up to max_launches (first slot, workgroup count) pairs, in launch order,
 * into the host arrays; it returns the number of stamped launches. */
int tiq_stamp_begin(uint64_t* buf, int64_t slots);
int64_t tiq_stamp_end(int64_t* first_slot, int64_t* workgroups, int64_t max_launches);

/* Library version: one integer, raised with every change of the kernels
 * (measurement records taken with one version name it). */
int tiq_version(void);
/* Static string naming a status code (never NULL). */
const char* tiq_status_string(int status);

/* ------------------------------------------------------------ quantize */

/* quantize_tensor(w, bits, "per_channel")  -- quantization.py:78-116.
 * w (rows, cols) fp32 with leading dim ldw; q (rows, cols) int8 codes with
 * leading dim ldq; scale (rows) fp32. Codes and scales are bit-identical to the
 * reference: scale = max(amax_row / qmax, FLT_MIN) with IEEE division,
 * q = clamp(rint_half_even(w / scale), qmin, qmax). */
int tiq_quantize_per_channel(const float* w, int64_t rows, int64_t cols, int64_t ldw, int bits,
                             int8_t* q, int64_t ldq, float* scale, void* stream);

/* Workspace bytes tiq_quantize_per_tensor needs for `numel` elements. */
size_t tiq_quantize_per_tensor_workspace(int64_t numel);

/* quantize_tensor(w, bits, "per_tensor")  -- quantization.py:78-116, with the
 * single scale written to scale[0]. w and q are contiguous, numel elements. */
int tiq_quantize_per_tensor(const float* w, int64_t numel, int bits, int8_t* q, float* scale,
                            void* workspace, size_t workspace_bytes, void* stream);

/* pack_int4(q)  -- quantization.py:132-149. q: numel int8 codes in [-8, 7];
 * packed: (numel + 1) / 2 bytes, byte j = ((q[2j+1]+8) << 4) | (q[2j]+8), the
 * high nibble of the last byte 0 when numel is odd. */
int tiq_pack_int4(const int8_t* q, int64_t numel, uint8_t* packed, void* stream);

/* unpack_int4(packed, numel)  -- quantization.py:152-158. */
int tiq_unpack_int4(const uint8_t* packed, int64_t numel, int8_t* q, void* stream);

/* pack_int4(quantize_tensor(w, bits, "per_channel")[0]) in one pass, for
 * bits in [2, 4] and an even number of contiguous columns: packed is the
 * reference's flattened row-major nibble layout, rows * cols / 2 bytes, so row
 * r starts at byte r * cols / 2. Odd `cols` returns TIQ_EUNSUPPORTED (use
 * tiq_quantize_per_channel + tiq_pack_int4). */
int tiq_quantize_per_channel_int4_packed(const float* w, int64_t rows, int64_t cols, int bits,
                                         uint8_t* packed, float* scale, void* stream);

/* Group-wise int4 with fp16 scales. No counterpart in the reference (its
 * int4 scales are per row or per tensor); the format is this library's own:
 * groups of `group` consecutive columns (even, >= 2; the last group ragged),
 * scale = fp16_rne(amax_group / 7) with 0 replaced by the smallest positive
 * fp16 and overflow saturated to 65504, codes clamp(rint(w / scale), -8, 7),
 * nibbles per row (low = even column, +8 bias), row stride (cols + 1) / 2
 * bytes, pad nibble 0. scale_f16 is (rows, ceil(cols / group)) fp16 bits. */
int tiq_quantize_groupwise_int4(const float* w, int64_t rows, int64_t cols, int group,
                                uint8_t* packed, uint16_t* scale_f16, void* stream);

/* (q.float() * scale)  -- quantization.py:119-129,197. per_channel != 0
 * reads scale[row], else scale[0]. Output w_hat (rows, cols) contiguous fp32. */
int tiq_dequantize_int8(const int8_t* q, const float* scale, int per_channel, int64_t rows,
                        int64_t cols, float* w_hat, void* stream);
/* The same for the reference nibble layout (rows * cols / 2 bytes, cols even). */
int tiq_dequantize_int4(const uint8_t* packed, const float* scale, int per_channel, int64_t rows,
                        int64_t cols, float* w_hat, void* stream);
/* The same for the group-wise int4 layout above. */
int tiq_dequantize_groupwise_int4(const uint8_t* packed, const uint16_t* scale_f16, int group,
                                  int64_t rows, int64_t cols, float* w_hat, void* stream);

/* -------------------------------------------------------------- linear
 * y[m, n] = sum_k x[m, k] * (q[n, k] * scale[n]) + bias[n]
 * The quantized replacement of the fp32 F.linear on W_hat at model.py:254
 * (c_attn), :319 (attn.c_proj), :352 (c_fc), :355 (mlp.c_proj).
 * x: (M, K) with leading dim ldx, dtype x_dtype (TIQ_F32 or TIQ_BF16);
 * y: (M, N) with leading dim ldy, dtype y_dtype; bias may be NULL;
 * scale: N fp32 (a per-tensor scale is passed as N copies).
 * Accumulation is fp32. Result matches dequantize-then-fp32-matmul within
 * max|y - y_ref| <= 1e-3 * max|y_ref|; with fp32 x the error is at fp32
 * rounding level.
 */

/* Dispatching entry point: picks the decode GEMV (small M) or the MFMA GEMM. */
int tiq_linear_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  const int8_t* q, const float* scale, const float* bias, int64_t N,
                  void* y, int y_dtype, int64_t ldy, void* stream);

/* Workspace bytes tiq_linear_w8_ws needs (0: none). Nonzero for fp32
 * activations with M >= 128 and K % 64 == 0: M * 3K * 2 bytes, rounded up
 * to 256. */
size_t tiq_linear_w8_workspace(int x_dtype, int64_t M, int64_t K);

/* tiq_linear_w8 with a caller workspace -- the same quantized Linear slot
 * (model.py:254,319,352,355), used by the prefill (M = B*T rows) of a model
 * that keeps fp32 activations. With fp32 x and M >= 128 the activations are
 * split exactly into three bf16 planes (x = hi + lo + lo2, written to the
 * workspace) and the product runs on the matrix cores: every product is exact
 * (int8 is exact in bf16), so the result is as accurate as an fp32 GEMM.
 * Other cases behave as tiq_linear_w8. TIQ_EWORKSPACE when the workspace is
 * smaller than tiq_linear_w8_workspace() or not 16-byte aligned. */
int tiq_linear_w8_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                     const int8_t* q, const float* scale, const float* bias, int64_t N,
                     void* y, int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Workspace bytes with which tiq_gemm_w8_ws (and tiq_linear_w8_ws, and with
 * bf16 activations tiq_linear_w4_ws / tiq_linear_w4g_ws) run a product with
 * few output tiles split over K (fp32 partial slices, summed in a fixed order
 * by a second kernel), plus, for fp32 activations, their bf16 planes. 0 when
 * none is needed. Nonzero from M >= 128, and for fp32 activations also from
 * the fewer rows at which tiq_linear_w4_ws takes the planes (M >= 32, or
 * M >= 16 with N >= 2048; the int8 entry points do not use it there). */
size_t tiq_gemm_w8_workspace(int x_dtype, int64_t M, int64_t K, int64_t N);
/* tiq_gemm_w8 with a caller workspace (see tiq_gemm_w8_workspace): the
 * prefill product of the reference's Linears (model.py:254,319,352,355 at
 * M = B * T) on the matrix cores; without enough workspace it runs unsplit,
 * and also with it when the product has 48 or more 128 x 128 tiles and at
 * most 32 k64 steps (the split would be slower; the workspace is then not
 * touched). */
int tiq_gemm_w8_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q, const float* scale,
                   const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Decode GEMV on the vector ALUs: coalesced 128-bit weight loads, dequant in
 * registers, wavefront reductions. Any M (processed in slices of up to 4
 * rows); needs K % 16 == 0 and 16-byte aligned weight rows. */
int tiq_gemv_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                const int8_t* q, const float* scale, const float* bias, int64_t N,
                void* y, int y_dtype, int64_t ldy, void* stream);

/* Prefill GEMM: int8 tiles dequantized to bf16 in LDS, bf16 MFMA, fp32
 * accumulate, scale + bias epilogue. x must be TIQ_BF16; K % 64 == 0. */
int tiq_gemm_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                const int8_t* q, const float* scale, const float* bias, int64_t N,
                void* y, int y_dtype, int64_t ldy, void* stream);

/* tiq_gemm_w8 with an explicit tile configuration, for tests and
 * measurement: 0 = the automatic choice, 1-4 = the LDS-dequant kernel at
 * 128x128 / 256x128 / 128x256 / 256x128 (8 wavefronts) tiles, 10-15 = the
 * register-staged kernel at 256x256 / 256x128 / 128x128 tiles and, with bf16
 * output, 224x256 / 160x256 / 224x128 (128x128 with fp32 output; falls back
 * to the automatic tile when that kernel does not take the shape), 16 = its
 * 128x128 tile with four register staging sets, 17 = 128x128 with the
 * wavefronts side by side along N (bf16 output; else as 12). No
 * counterpart in the reference (same interface as tiq_gemm_w8); the product
 * path never calls it. */
int tiq_gemm_w8_tile(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                     const int8_t* q, const float* scale, const float* bias, int64_t N,
                     void* y, int y_dtype, int64_t ldy, int tile, void* stream);

/* int4 weights in the reference's nibble layout (per-row scale, K even,
 * row n at byte n * K / 2). Same contract as tiq_linear_w8. */
int tiq_linear_w4(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  const uint8_t* packed, const float* scale, const float* bias, int64_t N,
                  void* y, int y_dtype, int64_t ldy, void* stream);

/* int4 weights in the group-wise layout (fp16 scale per group of `group`
 * columns). No counterpart in the reference. */
int tiq_linear_w4g(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                   const uint8_t* packed, const uint16_t* scale_f16, int group,
                   const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                   void* stream);

/* tiq_linear_w4 / tiq_linear_w4g with a caller workspace of
 * tiq_linear_w8_workspace(x_dtype, M, K) bytes: with fp32 x and M >= 128 the
 * activations are split exactly into three bf16 planes there and the product
 * runs on the matrix cores (every product exact, fp32 accumulation; the
 * group-wise format scales each group's partial sum), as tiq_linear_w8_ws
 * does for int8 -- the prefill of a model quantized to int4 (model.py:254,
 * 319,352,355 at M = B*T). With bf16 x, M >= 128 and a workspace of
 * tiq_gemm_w8_workspace(TIQ_BF16, M, K, N) bytes both split a product with few
 * output tiles over K (group-wise: whole groups a split), the fp32 slices
 * summed in a fixed order. Reference-layout int4 (tiq_linear_w4_ws) with fp32
 * x takes the planes from fewer rows too -- M >= 32, or M >= 16 with
 * N >= 2048 -- given a workspace of tiq_gemm_w8_workspace(TIQ_F32, M, K, N)
 * bytes (planes, then the fp32 slices of a product split over K); with a
 * smaller one such a call computes what tiq_linear_w4 computes. Where the
 * GEMM does not take the shape (K % 64, group % 64), and for bf16 x or
 * M < 128 without a workspace, they compute what tiq_linear_w4 /
 * tiq_linear_w4g compute. With fp32 x, M >= 128 and a
 * shape the GEMM takes, the planes need the workspace: TIQ_EWORKSPACE when it
 * is NULL, smaller than tiq_linear_w8_workspace(x_dtype, M, K) or not 16-byte
 * aligned (as tiq_linear_w8_ws). */
int tiq_linear_w4_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                     const uint8_t* packed, const float* scale, const float* bias, int64_t N,
                     void* y, int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
                     void* stream);
int tiq_linear_w4g_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                      const uint8_t* packed, const uint16_t* scale_f16, int group,
                      const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------- decode step
 * Kernels of one GPT-2 decode step (one token per sequence) over a
 * preallocated KV cache whose fill level `pos` is a device int64 scalar, so
 * the step is the same sequence of launches for every token (capturable in a
 * HIP graph). Device-side values (pos, token ids) are range-checked in the
 * kernels: an out-of-range value yields NaN outputs, never an out-of-bounds
 * access.
 */

/* The fused decode linear, for M <= a few rows (the GEMV path):
 *   y = act(LayerNorm(x) @ W^T * scale + bias) + residual
 * Replaces Block.forward's ln_1 -> attn.c_attn, ln_2 -> mlp.c_fc -> gelu_tanh,
 * and the residual adds x + attn(..), x + mlp(..) (model.py:410-427,57-75,
 * 351-355). ln_weight/ln_bias NULL: no LayerNorm (else both given, eps
 * ln_eps, statistics over the K inputs of each row); activation
 * TIQ_ACT_NONE or TIQ_ACT_GELU_TANH; residual NULL or (M, N) with leading dim
 * ld_residual (may alias y: the update is in place). w_format selects the
 * layout of w: TIQ_WF_INT8 / TIQ_WF_INT4 (per-row fp32 scale),
 * TIQ_WF_INT4_GROUPWISE (fp16 group scales), TIQ_WF_F32 (fp32 weights, scale
 * ignored: the unquantized tied lm_head, model.py:585). Needs K % 32 == 0,
 * K * 4 <= 65536 and 16-byte aligned rows; returns TIQ_EUNSUPPORTED otherwise. */
int tiq_linear_fused(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w,
                     int w_format, const float* scale, const uint16_t* scale_f16, int group,
                     const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                     const float* ln_weight, const float* ln_bias, float ln_eps, int activation,
                     const float* residual, int64_t ld_residual, void* stream);

/* Workspace bytes tiq_linear_fused_ws uses for an (M, K) x (N, K) product
 * (0: none). Nonzero for fp32 activations with 5 <= M <= 64 (a batched
 * decode step) and int8 or fp32 weights: the split activations, 32-row tiles
 * x 3K bf16 (ceil(M / 32) * 32 * 3K * 2 bytes, rounded up to 256). N does not
 * change the size today. The contents need no initialisation and are not
 * preserved; calls that share a workspace must not overlap. */
size_t tiq_linear_fused_workspace(int x_dtype, int w_format, int64_t M, int64_t K, int64_t N);

/* tiq_linear_fused with a caller workspace -- the same decode linear of
 * Block.forward (model.py:410-427) and lm_head (model.py:585). For a batched
 * decode step (5 <= M <= 64 rows of fp32 activations, int8 or fp32 weights)
 * the rows are LayerNorm'd (if requested) and split exactly into three bf16
 * planes once, into the workspace, and the product runs on the matrix cores
 * from those planes; without a large enough workspace the same kernels split
 * the rows themselves (more vector work per weight row). Results are
 * fp32-accurate either way. The workspace must be 16-byte aligned. */
int tiq_linear_fused_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w,
                        int w_format, const float* scale, const uint16_t* scale_f16, int group,
                        const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                        const float* ln_weight, const float* ln_bias, float ln_eps, int activation,
                        const float* residual, int64_t ld_residual, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Batched decode-step linear (5 <= M <= 64 fp32 activation rows; int8
 * weights with per-row scale -- row-major (TIQ_WF_INT8) or in the operand
 * tiles of tiq_tile_int8 (TIQ_WF_INT8_TILED, N % 32 == 0) -- or fp32
 * weights) whose K range is split over
 * workgroups: the matrix-core products write fp32 partial sums to the
 * workspace, a second kernel sums them in a fixed order and applies
 *     y = act(LayerNorm(x) @ W^T * scale + bias) + residual
 * (the reference's Linear at model.py:254,319,352,355 with its neighbours at
 * model.py:413-427, as tiq_linear_fused), so that a small matrix still
 * occupies the whole GPU.
 *   Input: fp32 rows x (leading dimension ldx, optional LayerNorm ln_*), or,
 *   when x_planes is not NULL, operand planes written by planes_out of a
 *   previous call with N = this K (x and ln_* are then unused; ln_* must be
 *   NULL).
 *   Output: y (fp32, may be NULL when only planes are wanted; residual may
 *   alias it) and, when planes_out is not NULL, the operand planes of
 *   next_ln(y) (or of y without next_ln_*) for a following call:
 *   tiq_decode_planes_bytes(M, N) bytes, 16-byte aligned, N % 32 == 0.
 *   workspace: at least tiq_decode_linear_workspace(w_format, M, K, N)
 *   bytes, 16-byte aligned; clobbered.
 * No counterpart in the reference (its decode runs one torch op per step). */
size_t tiq_decode_linear_workspace(int w_format, int64_t M, int64_t K, int64_t N);
size_t tiq_decode_planes_bytes(int64_t M, int64_t K);

/* The int8 codes of an (N, K) weight (leading dimension ldw bytes, 16-byte
 * aligned rows) rearranged for tiq_decode_linear with w_format
 * TIQ_WF_INT8_TILED: N * K bytes in 1 KB blocks, block t * (K / 32) + u
 * holding rows 32 t .. 32 t + 31 and columns 32 u .. 32 u + 31 in the order a
 * wavefront's matrix-core operands take them (byte 16 l + j of the block is
 * w[32 t + l % 32][32 u + 16 (l / 32) + j]), so each 64-lane load of the
 * product reads 1 KB of consecutive memory. Needs N % 32 == 0, K % 32 == 0,
 * ldw % 16 == 0 and 16-byte aligned pointers. The scale, results and every
 * other argument of tiq_decode_linear are those of the row-major codes
 * (TIQ_WF_INT8): the products are the same, in the same order. No
 * counterpart in the reference (a device layout of this library). */
int tiq_tile_int8(const int8_t* w, int64_t N, int64_t K, int64_t ldw, int8_t* tiles, void* stream);

/* The fp32 weights of an (N, K) unquantized Linear (the tied lm_head,
 * model.py:585; leading dimension ldw floats, 16-byte aligned rows)
 * rearranged for tiq_decode_linear with w_format TIQ_WF_F32_TILED:
 * tiq_tile_f32_bytes(N, K) bytes (ceil(N / 32) * 32 rows, rows past N zero)
 * in 4 KB blocks, block t * (K / 32) + u holding rows 32 t .. 32 t + 31 and
 * columns 32 u .. 32 u + 31, byte 1024 q + 16 l + 4 j of the block being
 * w[32 t + l % 32][32 u + 16 (l / 32) + 4 q + j], so each 64-lane load of
 * the product reads 1 KB of consecutive memory. Needs K % 32 == 0. With those
 * tiles tiq_decode_linear takes only operand planes in (x_planes, 1..64 rows,
 * K >= 256) and writes only the fp32 rows y (no bias, activation, residual or
 * planes out); it streams the tiles with one workgroup per CU looping over
 * them and gives the same results, bit for bit, as TIQ_WF_F32 on the
 * row-major weights. No counterpart in the reference (a device layout of
 * this library). */
size_t tiq_tile_f32_bytes(int64_t N, int64_t K);
int tiq_tile_f32(const float* w, int64_t N, int64_t K, int64_t ldw, float* tiles, void* stream);
int tiq_decode_linear(const float* x, int64_t ldx, const uint16_t* x_planes, int64_t M, int64_t K, const void* w,
                      int w_format, const float* scale, const float* bias, int64_t N, float* y, int64_t ldy,
                      const float* ln_weight, const float* ln_bias, float ln_eps, int activation,
                      const float* residual, int64_t ld_residual, const float* next_ln_weight,
                      const float* next_ln_bias, float next_ln_eps, uint16_t* planes_out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Bytes of the fixed device scratch of tiq_decode_linear_noalloc (per GPU,
 * held from the library's load until the process ends). */
#define TIQ_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* tiq_decode_linear without a workspace argument: for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid allocation). No counterpart in the reference. Same
 * arguments, kernels and results as tiq_decode_linear; its workspace is a
 * fixed TIQ_NOALLOC_SCRATCH_BYTES array on the device of `stream`, so it
 * allocates nothing and returns TIQ_ESCRATCH (before any launch) when
 * tiq_decode_linear_workspace(w_format, M, K, N) exceeds that size (GPT-2-XL
 * block shapes at M <= 64 need at most 4.1 MB; the tied fp32 head in the
 * row-major TIQ_WF_F32 layout, N = 50257 rows of K = 1600, needs 13.5 MB at
 * M = 64: 0.6 MB of operand planes and one 12.9 MB partial slice; in the
 * TIQ_WF_F32_TILED layout it needs none). Every call on one GPU shares the
 * array: calls that overlap on one GPU (concurrent streams, threads) race.
 * The first call on a device looks up the array's device address
 * (hipGetSymbolAddress); make that call outside stream capture. */
int tiq_decode_linear_noalloc(const float* x, int64_t ldx, const uint16_t* x_planes, int64_t M, int64_t K,
                              const void* w, int w_format, const float* scale, const float* bias, int64_t N,
                              float* y, int64_t ldy, const float* ln_weight, const float* ln_bias, float ln_eps,
                              int activation, const float* residual, int64_t ld_residual,
                              const float* next_ln_weight, const float* next_ln_bias, float next_ln_eps,
                              uint16_t* planes_out, void* stream);

/* Self-attention of one new token per sequence (model.py:248-318 at T = 1,
 * KVCache.update model.py:153-172): qkv is the (batch, (n_head + 2 n_kv_head)
 * * head_dim) output of c_attn (leading dim ld_qkv); its k and v are written
 * into k_cache / v_cache ((batch, n_kv_head, t_max, head_dim) fp32) at slot
 * *pos; the query attends to slots 0..*pos with softmax(q k^T / sqrt(hd));
 * y (batch, n_head * head_dim) gets the head outputs. head_dim must be 64,
 * t_max <= 1024. */
int tiq_decode_attention(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head, int64_t n_kv_head,
                         int64_t head_dim, float* k_cache, float* v_cache, int64_t t_max, const int64_t* pos,
                         float* y, int64_t ldy, void* stream);

/* tiq_decode_attention that also writes its output rows as the operand
 * planes of the following batched decode linear (tiq_decode_linear's
 * x_planes, K = n_head * head_dim; tiq_decode_planes_bytes(batch, K) bytes,
 * 16-byte aligned), saving that linear a split pass. No counterpart in the
 * reference. */
int tiq_decode_attention_planes(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head, int64_t n_kv_head,
                                int64_t head_dim, float* k_cache, float* v_cache, int64_t t_max, const int64_t* pos,
                                float* y, int64_t ldy, uint16_t* planes_out, void* stream);

/* The q, k, v projection and self-attention of one new token per sequence
 * in one call (model.py:254 c_attn at T = 1, then as tiq_decode_attention_planes):
 * x_planes are the operand planes of LayerNorm 1's output (planes_out of a
 * previous tiq_decode_linear with next_ln = ln_1, K = n_embd); w the int8
 * codes of c_attn (TIQ_WF_INT8, rows of n_embd bytes, or TIQ_WF_INT8_TILED),
 * scale / bias (bias may be NULL) its per-output fp32 factors, N = (n_head +
 * 2 n_kv_head) * head_dim outputs. The product runs split over K into fp32
 * partial slices in the workspace, and the attention kernel sums them for
 * its head ((sum of the slices) * scale + bias) instead of a reduction
 * launch; k, v go to the caches at slot *pos, y / planes_out as
 * tiq_decode_attention_planes (planes_out may be NULL). batch <= 64,
 * n_embd % 32 == 0, head_dim 64, t_max <= 1024.
 *   workspace: tiq_decode_qkv_attention_workspace(batch, n_embd, N) bytes,
 *   16-byte aligned, clobbered; that query returns 0 for a shape the call
 *   does not support (then use tiq_decode_linear + tiq_decode_attention_planes).
 * No counterpart in the reference (its attention is a chain of torch ops). */
size_t tiq_decode_qkv_attention_workspace(int64_t batch, int64_t n_embd, int64_t n_qkv);
int tiq_decode_qkv_attention(const uint16_t* x_planes, int64_t batch, int64_t n_embd, const void* w, int w_format,
                             const float* scale, const float* bias, int64_t n_head, int64_t n_kv_head,
                             int64_t head_dim, float* k_cache, float* v_cache, int64_t t_max, const int64_t* pos,
                             float* y, int64_t ldy, uint16_t* planes_out, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Causal self-attention of T queries per (sequence, head) over S = first + T
 * keys (CausalSelfAttention.forward, model.py:284-309, a prompt block or a
 * cached step): query t, at absolute position first + t, attends to keys
 * 0 .. first + t with softmax(q k^T / sqrt(head_dim)) in fp32 (an online
 * softmax over blocks of 64 keys). q (batch, n_head, T, 64), k and v (batch,
 * n_head, S, 64) and y (batch, n_head, T, 64) are addressed through their
 * (batch, head, position) strides in floats with the 64 dims contiguous:
 * the rows of the q, k, v projection, a KV cache's buffers and the (batch,
 * T, n_head * 64) output rows are read and written in place. head_dim must be
 * 64; pointers 16-byte aligned and strides multiples of 4 (TIQ_EALIGN
 * otherwise). No counterpart in the reference (a chain of torch ops there). */
int tiq_prefill_attention(const float* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const float* k, int64_t k_sb,
                          int64_t k_sh, int64_t k_st, const float* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                          int64_t batch, int64_t n_head, int64_t T, int64_t first, int64_t head_dim, float* y,
                          int64_t y_sb, int64_t y_sh, int64_t y_st, void* stream);

/* y = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) elementwise over n fp32
 * values (16-byte aligned; y may alias x): the MLP activation gelu_tanh
 * (model.py:57-75, applied at model.py:354) in one pass instead of the
 * reference's chain of torch ops. */
int tiq_gelu_tanh(const float* x, float* y, int64_t n, void* stream);

/* A quantized Linear over gelu_tanh of fp32 rows: the MLP's
 * c_proj(gelu_tanh(c_fc(x))) of a prefill (model.py:57-75 and the c_proj
 * slot, model.py:355, at M = B * T rows). The activation is applied while x
 * is split into the three exact bf16 planes the matrix cores take, so y is
 * bit for bit what tiq_linear_w8_ws / tiq_linear_w4_ws / tiq_linear_w4g_ws
 * compute on tiq_gelu_tanh(x), without the activation's own read and write of
 * x. w, w_format (TIQ_WF_INT8, TIQ_WF_INT4, TIQ_WF_INT4_GROUPWISE), scale,
 * scale_f16 and group as tiq_linear_fused; x and y fp32; x is only read.
 * Needs M >= 128, K % 64 == 0, x 16-byte aligned with ldx % 4 == 0 and a
 * workspace of tiq_gemm_w8_workspace(TIQ_F32, M, K, N) bytes (at least the
 * planes' M * 3K * 2, else TIQ_EWORKSPACE; with less than the full size a
 * product with few output tiles runs unsplit); TIQ_EUNSUPPORTED for other
 * shapes, for which the caller applies tiq_gelu_tanh and the plain entry
 * point. */
int tiq_linear_gelu_in_ws(const float* x, int64_t M, int64_t K, int64_t ldx, const void* w, int w_format,
                          const float* scale, const uint16_t* scale_f16, int group, const float* bias, int64_t N,
                          float* y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/* x[b] = wte[tokens[b]] + wpe[*pos]  (model.py:561-564 for one position). */
int tiq_embed_tokens(const int64_t* tokens, const int64_t* pos, const float* wte, int64_t vocab,
                     const float* wpe, int64_t n_positions, int64_t batch, int64_t n_embd, float* x,
                     void* stream);

/* Workspace bytes tiq_argmax_rows needs for `rows` rows. */
size_t tiq_argmax_rows_workspace(int64_t rows);

/* out[r] = argmax of row r of x (first index of the maximum; sampling.py:164),
 * rows <= 65535. If ids is not NULL the index is also written to
 * ids[r * ld_ids + *pos + 1] and then *pos is advanced by one (the decode
 * step's last kernel: the new token now sits at the position). */
int tiq_argmax_rows(const float* x, int64_t rows, int64_t cols, int64_t ld, int64_t* out, int64_t* ids,
                    int64_t ld_ids, int64_t* pos, void* workspace, size_t workspace_bytes, void* stream);

/* The tied fp32 head and its argmax for one row (GPT.forward's lm_head,
 * model.py:585, then logits.argmax(-1) and the id append, sampling.py:164-170),
 * reading a bf16 copy of the head: every row's logit is first computed from the
 * bf16 copy in fp32, together with a bound ||x|| row_coef[v] on its distance from
 * the logit of the fp32 weights (row_coef = err + gamma (2 norm + err), err =
 * ||w_v - bf16(w_v)||_2, norm = ||w_v||_2, gamma = C 2^-24 / (1 - C 2^-24): the
 * bf16 rounding by Cauchy-Schwarz plus the rounding of both fp32 dot products
 * in any order), and only the rows whose upper bound reaches the best lower
 * bound of their workgroup are computed again from the fp32 weights; the token
 * is the first index of the maximum of those exact logits (NaN never selected,
 * as tiq_argmax_rows), so it is the argmax of the fp32 logits. x is the row
 * before the final LayerNorm (ln_w, ln_b, ln_eps); n_embd % 16 == 0, n_embd <=
 * 1024, vocab <= 131072; logits receives the bf16 estimates and the exact values
 * of the recomputed rows. out, ids, ld_ids and pos as tiq_argmax_rows. The extra
 * device bytes are the bf16 copy (2 bytes a weight) and one float a row, from
 * tiq_head_screen_prepare. No counterpart in the reference beyond the head and
 * argmax it replaces. */
size_t tiq_head_screen_workspace(int64_t vocab);
/* w_bf16 = round-to-nearest-even bf16 of the (vocab, n_embd) head w (rows of
 * ldw floats) and row_coef[v] = err + gamma (2 norm + err) as above, the norms
 * summed in fp64 and the coefficient rounded up to fp32. */
int tiq_head_screen_prepare(const float* w, int64_t vocab, int64_t n_embd, int64_t ldw, uint16_t* w_bf16,
                            float* row_coef, void* stream);
int tiq_head_argmax_screened(const float* x, int64_t n_embd, const float* ln_w, const float* ln_b, float ln_eps,
                             const uint16_t* w_bf16, const float* w, int64_t ldw, const float* row_coef,
                             int64_t vocab, float* logits, int64_t* out, int64_t* ids, int64_t ld_ids, int64_t* pos,
                             void* workspace, size_t workspace_bytes, void* stream);
/* The same screen from an int8 copy of the head (half the bytes of the bf16
 * copy): w_i8 = rint(w / s) clamped to +-127 with s = row_scale[v] = max|w_v| /
 * 127, each row's estimate s (x . q_v) in fp32, err = ||w_v - s q_v||_2 and
 * gamma = (C + 1) 2^-24 / (1 - (C + 1) 2^-24) (the product by s is one more
 * rounding); vocab <= 262144, the rest as tiq_head_argmax_screened, and the
 * token the argmax of the fp32 logits all the same. The extra device bytes are
 * the int8 copy (1 byte a weight) and two floats a row, from
 * tiq_head_screen_prepare_i8. No counterpart in the reference beyond the head
 * and argmax it replaces. */
int tiq_head_screen_prepare_i8(const float* w, int64_t vocab, int64_t n_embd, int64_t ldw, int8_t* w_i8,
                               float* row_scale, float* row_coef, void* stream);
int tiq_head_argmax_screened_i8(const float* x, int64_t n_embd, const float* ln_w, const float* ln_b, float ln_eps,
                                const int8_t* w_i8, const float* row_scale, const float* w, int64_t ldw,
                                const float* row_coef, int64_t vocab, float* logits, int64_t* out, int64_t* ids,
                                int64_t ld_ids, int64_t* pos, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TIQ_H */
