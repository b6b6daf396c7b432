// Internal launch interfaces shared by the linear entry points.
#pragma once

#include "tiq_common.hpp"

namespace tiq {

// Weight storage formats of a quantized Linear (rows = N outputs, cols = K inputs).
enum WFormat : int {
    kW8 = 0,   // int8 codes, row n at byte n * ldw
    kW4 = 1,   // reference nibble layout, row n at byte n * K / 2 (K even)
    kW4G = 2,  // group-wise nibbles, row n at byte n * ((K + 1) / 2), fp16 group scales
    kF32 = 3,  // fp32 weights (an unquantized Linear such as the tied lm_head), no scale
    kW8T = 4,  // int8 codes in 32 x 32 operand tiles (tiq_tile_int8; batched decode only)
    kF32T = 5, // fp32 weights in 32 x 32 operand tiles (tiq_tile_f32; the batched decode head)
};

// Optional work fused around a decode GEMV: LayerNorm of the activation rows
// before the product, GELU(tanh) after it, and a residual added to the output.
struct Fusion {
    const float* ln_w = nullptr;  // LayerNorm weight (K), enables the prologue
    const float* ln_b = nullptr;  // LayerNorm bias (K)
    float ln_eps = 1e-5f;
    int act = 0;                  // 0 none, 1 gelu_tanh
    const float* res = nullptr;   // residual (M, N) with leading dim ldr, added last
    int64_t ldr = 0;
};

struct LinearArgs {
    const void* x;
    int x_dtype;
    int64_t M, K, ldx;
    const uint8_t* w;
    int64_t ldw;             // bytes between weight rows
    const float* scale;      // per-row fp32 (kW8, kW4)
    const uint16_t* scale16; // per-group fp16 bits (kW4G)
    int group;
    const float* bias;
    int64_t N;
    void* y;
    int y_dtype;
    int64_t ldy;
    hipStream_t stream;
    WFormat fmt;
    Fusion fuse;
    // Period of K in the weight matrix: the GEMM reads weight column k % kw.
    // 0 means K. The fp32-activation path passes K = 3 kw (x split into three
    // bf16 planes laid side by side along K).
    int64_t kw = 0;
    // Optional device workspace (the decode linears stage LayerNorm'd,
    // split activations there when it is large enough).
    void* ws = nullptr;
    size_t ws_bytes = 0;
};

// Measurement (tiq_stamp_begin): 4 * workgroups slots of the stamp buffer for
// the next launch of a stamped kernel, or nullptr when stamping is off or
// the buffer is full (the launch then runs the unstamped kernel).
uint64_t* stamp_slots(int64_t workgroups);

// Validates the common arguments; TIQ_OK when they are consistent.
int check_linear(const LinearArgs& a);

int launch_gemv(const LinearArgs& a);
// Decode GEMV on the matrix cores for 2..16 bf16 rows and int8 weights
// (gemv.hip): whether it takes these arguments, whether the dispatch picks
// it over the direct and batched kernels, and its launch.
bool rows16_supported(const LinearArgs& a);
bool rows16_preferred(const LinearArgs& a);
int launch_rows16(const LinearArgs& a);
int launch_gemm(const LinearArgs& a);
// The GEMM with a given tile configuration: 0 automatic, 1-4 the LDS-dequant
// kernel's tiles (gemm.hip), 10-16 the staged int8 kernel's (256x256, 256x128,
// 128x128; with bf16 output 224x256, 160x256, 224x128; 128x128 with four
// staging sets; with bf16 output 128x128 with the wavefronts along N).
int launch_gemm_tile(const LinearArgs& a, int tile);
// True when the MFMA GEMM has a kernel for these arguments.
bool gemm_supported(const LinearArgs& a);

// Decode linear on the matrix cores for 5..64 rows of fp32 activations
// (skinny.hip): int8 or fp32 weights, with the decode fusions.
constexpr int64_t kSkinnyMinRows = 5;
bool skinny_supported(const LinearArgs& a);
int launch_skinny(const LinearArgs& a);
// Workspace bytes with which it splits the activations once per call.
size_t skinny_workspace(int64_t M, int64_t K);

// Batched decode linear with its K range split over workgroups (skinny.hip):
// the products write fp32 partials, one more kernel sums them, applies the
// epilogue and optionally writes the next linear's LayerNorm'd operand planes
// (planes_out, K' = N). The input is fp32 rows (a.x, with a.fuse.ln_w) or the
// planes of a previous call (x_planes).
int run_decode_linear(const LinearArgs& a, const uint16_t* x_planes, const float* next_ln_w,
                      const float* next_ln_b, float next_eps, uint16_t* planes_out);

// The product of a batched decode linear as raw fp32 partial sums, for a
// consumer that finishes them itself (skinny.hip): slice z of `part` (M x N,
// at part + z M N) holds K units [z U / S, (z + 1) U / S) of x W^T with no
// scale or bias, S = decode_slices_count(M, K, N) <= kMaxSlices. int8
// weights (kW8, kW8T), 1..64 rows, K % 32 == 0 (K <= 4096 with an even
// count of 32-row tiles, else K <= 8192), the operand planes of a previous
// decode linear in.
constexpr int64_t kMaxSlices = 4;

// fp32 weights in operand tiles (skinny.hip): ceil(N / 32) x (K / 32) blocks
// of 4 KB, rows past N zero; byte 1024 q + 16 l + 4 j of block (t, u) holds
// w[32 t + l % 32][32 u + 16 (l / 32) + 4 q + j].
size_t tile_f32_bytes(int64_t N, int64_t K);
int launch_tile_f32(const float* w, int64_t N, int64_t K, int64_t ldw, float* tiles, hipStream_t stream);
int64_t decode_slices_count(int64_t M, int64_t K, int64_t N);
size_t decode_slices_bytes(int64_t M, int64_t K, int64_t N);  // 0: shape not supported
int launch_decode_slices(const LinearArgs& a, const uint16_t* x_planes, float* part);
size_t decode_linear_workspace(int64_t M, int64_t K, int64_t N);
size_t decode_planes_bytes(int64_t M, int64_t K);
// int8 codes (N, K) -> the operand tiles the decode product reads with kW8T.
int launch_tile_int8(const uint8_t* w, int64_t N, int64_t K, int64_t ldw, uint8_t* tiles, hipStream_t stream);

// The register-staged GEMM (gemm_staged.hip; int8 and reference-layout int4
// weights): whether it takes these arguments, its tile choice (0: 256 x 256,
// 1: 256 x 128, 2: 128 x 128; bf16 output also 3: 224 x 256, 4: 160 x 256,
// 5: 224 x 128) and its launch.
bool staged_gemm_supported(const LinearArgs& a);
int staged_gemm_choice(const LinearArgs& a);
int launch_staged_gemm(const LinearArgs& a, int choice);
// Split-K for products with few output tiles: S (1 = none), the workspace
// bytes of its fp32 partial slices, and the launch (TIQ_EUNSUPPORTED when no
// split is planned or the workspace is short: the caller then launches the
// plain kernel).
int64_t staged_splits(int64_t M, int64_t N, int64_t K);
size_t staged_split_workspace(int64_t M, int64_t N, int64_t K);
int launch_staged_gemm_split(const LinearArgs& a, void* ws, size_t ws_bytes);
// y = scale * (sum of the S fp32 slices part[S][M][N], in slice order) + bias
// (scale null: 1), with a's output, bias and stream; N % 4 == 0.
int launch_splitk_reduce(const LinearArgs& a, const float* part, int64_t S, const float* scale);
// Group-wise int4 with bf16 activations split over K (whole groups a split)
// when the 128 x 128 tiles are too few to fill the GPU; the partial slices in
// ws (staged_split_workspace bytes). TIQ_EUNSUPPORTED: no split planned.
int launch_gemm_w4g_split(const LinearArgs& a, void* ws, size_t ws_bytes);
// Group-wise int4 (groups of 128) with bf16 activations on the register-staged
// kernel (gemm_grouped.hip): whether it takes these arguments, and the launch,
// split over K (whole groups, fp32 slices in ws) when its tiles are few and ws
// holds them. TIQ_EUNSUPPORTED when it does not take them.
bool staged_w4g_supported(const LinearArgs& a);
int launch_staged_w4g(const LinearArgs& a, void* ws, size_t ws_bytes);

}  // namespace tiq
