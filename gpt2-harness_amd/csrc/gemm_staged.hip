// Prefill GEMM for large M on the matrix cores (gfx950): int8 weights,
// bf16 activations, the reference's quantized Linears over a whole prompt
// (model.py:254,319,352,355 with M = B*T):
//     y[m, n] = scale[n] * sum_k x[m, k] * q[n, k] + bias[n]
// Built without -amdgpu-mfma-vgpr-form: its 128 x 128 accumulator blocks live
// in AGPRs.
#include <algorithm>

#include "tiq_internal.hpp"

namespace tiq {
namespace {

#include "gemm_staged_kernel.hpp"

template <int BM, int BN, int WMW, int FMT, typename TY, int DEPTH = 2>
int run_staged(const LinearArgs& a) {
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const int64_t slots = 256 * (BM * BN <= 128 * 128 ? 2 : 1);
    const int64_t grid = staged_persist<BM, BN, WMW>() ? std::min(tiles, slots) : tiles;
    // int8 weights with bf16 output have a stamped copy for measurement
    if constexpr (FMT == kW8 && sizeof(TY) == 2) {
        if (uint64_t* sp = stamp_slots(grid)) {
            hipLaunchKernelGGL((gemm_staged<BM, BN, WMW, FMT, TY, true, DEPTH>), dim3((unsigned)grid), dim3(256), 0,
                               a.stream, static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias,
                               static_cast<TY*>(a.y), a.ldy, (int)a.M, (int)a.N, (int)a.K,
                               (int)(a.kw ? a.kw : a.K), nullptr, 0, sp);
            return launch_status();
        }
    }
    hipLaunchKernelGGL((gemm_staged<BM, BN, WMW, FMT, TY, false, DEPTH>), dim3((unsigned)grid), dim3(256), 0, a.stream,
                       static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, static_cast<TY*>(a.y),
                       a.ldy, (int)a.M, (int)a.N, (int)a.K, (int)(a.kw ? a.kw : a.K), nullptr, 0, nullptr);
    return launch_status();
}

bool staged_supported_impl(const LinearArgs& a) {
    if ((a.fmt != kW8 && a.fmt != kW4) || a.x_dtype != TIQ_BF16 || a.K % BK != 0) return false;
    if (a.kw && (a.kw % BK != 0 || a.K % a.kw != 0)) return false;
    const int64_t kw = a.kw ? a.kw : a.K;
    const int unit = a.y_dtype == TIQ_F32 ? 4 : 8;
    if (a.N % unit != 0 || a.ldy % unit != 0 || !aligned(a.y, 16)) return false;
    if (!aligned(a.scale, 16) || (a.bias && !aligned(a.bias, 16))) return false;
    if (!aligned(a.x, 16) || a.ldx % 8 != 0 || !aligned(a.w, 16) || a.ldw % 16 != 0) return false;
    // 32-bit byte offsets from the base pointers
    if ((a.M - 1) * a.ldx * 2 + a.K * 2 > 0xffffffffLL || (a.N - 1) * a.ldw + kw > 0xffffffffLL) return false;
    return true;
}

// Tile choice: rounds of co-resident workgroups (the WMW = 2 256-row tiles and
// every WMW = 1 tile need most of a CU's LDS and registers: one per CU;
// 128x128 tiles fit two, whose rounds overlap: counted in halves) times the
// duration of one round, modelled as step_us per k64 step plus a fixed term
// (prologue, epilogue, launch), both least-squares fits to MI355X timings of
// every tile at the GPT-2-XL Linear shapes with M = 256 / 1024 / 4096 (bf16
// output, operands rotated over six copies, the current kernels: register-fed
// weights in the WMW = 1 tiles, persistent grids; within 16% of every timing
// but the 128x128 tile's at M = 4096, up to 26%), which picks the fastest
// tile at all twelve.
int staged_choice(int64_t M, int64_t N, int64_t K, bool bf16_out) {
    struct Opt { int bm, bn, per_cu; double step_us, fixed_us; };
    // 3-5: the WMW = 1 tiles (bf16 output only)
    static const Opt opts[] = {{256, 256, 1, 1.218, 13.39}, {256, 128, 1, 0.716, 8.16}, {128, 128, 2, 1.029, 3.29},
                               {224, 256, 1, 1.029, 12.40}, {160, 256, 1, 0.862, 9.06}, {224, 128, 1, 0.674, 6.92}};
    const double nk = (double)(K / BK);
    int best = 0;
    double best_t = 1e30;
    for (int o = 0; o < (bf16_out ? 6 : 3); ++o) {
        const int64_t tiles = ((M + opts[o].bm - 1) / opts[o].bm) * ((N + opts[o].bn - 1) / opts[o].bn);
        const int64_t slots = 256 * opts[o].per_cu;
        const double rounds = opts[o].per_cu == 1 ? (double)((tiles + slots - 1) / slots)
                                                  : 0.5 * (double)((2 * tiles + slots - 1) / slots);
        const double t = rounds * (nk * opts[o].step_us + opts[o].fixed_us);
        if (t < best_t) { best_t = t; best = o; }
    }
    return best;
}

// The end of a split-K product: y[m][n] = scale[n] * sum_z part[z][m][n] +
// bias[n] (scale 1 when null: the group-wise slices are scaled already), the
// S slices summed in a fixed order; 4 consecutive outputs a thread.
template <typename TY>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ bias, TY* __restrict__ y,
                                                            int64_t ldy) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= (int64_t)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    const int64_t slice = (int64_t)M * N;
    // the slices eight at a time (S <= 8 in practice: one trip to memory), all
    // requested before any is added (indices clamped instead of a branch, the
    // repeats not added), summed in slice order
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z0 = 0; z0 < S; z0 += 8) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4*>(part + min(z0 + j, S - 1) * slice + i);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool use = z0 + j < S;
            a.x = use ? a.x + v[j].x : a.x;
            a.y = use ? a.y + v[j].y : a.y;
            a.z = use ? a.z + v[j].z : a.z;
            a.w = use ? a.w + v[j].w : a.w;
        }
    }
    const float4 sc = scale ? *reinterpret_cast<const float4*>(scale + n) : make_float4(1.f, 1.f, 1.f, 1.f);
    float4 bi = make_float4(0.f, 0.f, 0.f, 0.f);
    if (bias) bi = *reinterpret_cast<const float4*>(bias + n);
    const float o0 = fmaf(a.x, sc.x, bi.x), o1 = fmaf(a.y, sc.y, bi.y);
    const float o2 = fmaf(a.z, sc.z, bi.z), o3 = fmaf(a.w, sc.w, bi.w);
    TY* yr = y + (int64_t)m * ldy + n;
    if constexpr (sizeof(TY) == 4) {
        *reinterpret_cast<float4*>(yr) = make_float4(o0, o1, o2, o3);
    } else {
        uint2 o;
        o.x = pk_bf16(o0, o1);
        o.y = pk_bf16(o2, o3);
        *reinterpret_cast<uint2*>(yr) = o;
    }
}

}  // namespace

// Split-K plan for products with too few output tiles to fill the GPU:
// 128 x 128 tiles (two workgroups per CU, 512 slots); when they fill less
// than half of the slots, K is split S ways (each split at least four k64
// steps, at most 8 splits). 1: no split.
int64_t staged_splits(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
    if (tiles * 2 >= 512) return 1;
    const int64_t S = std::min<int64_t>(std::min<int64_t>(512 / tiles, (K / BK) / 4), 8);
    return std::max<int64_t>(S, 1);
}

size_t staged_split_workspace(int64_t M, int64_t N, int64_t K) {
    const int64_t S = staged_splits(M, N, K);
    return S > 1 ? (size_t)((S * M * N * 4 + 255) / 256 * 256) : 0;
}

template <int FMT>
int dispatch_staged_f32(const LinearArgs& a, int choice) {
    switch (choice) {
        case 0: return run_staged<256, 256, 2, FMT, float>(a);
        case 1: return run_staged<256, 128, 2, FMT, float>(a);
        case 6: return run_staged<128, 128, 2, FMT, float, 4>(a);
        default: return run_staged<128, 128, 2, FMT, float>(a);
    }
}

template <int FMT>
int dispatch_staged_bf16(const LinearArgs& a, int choice) {
    switch (choice) {
        case 0: return run_staged<256, 256, 2, FMT, uint16_t>(a);
        case 1: return run_staged<256, 128, 2, FMT, uint16_t>(a);
        case 3: return run_staged<224, 256, 1, FMT, uint16_t>(a);
        case 4: return run_staged<160, 256, 1, FMT, uint16_t>(a);
        case 5: return run_staged<224, 128, 1, FMT, uint16_t>(a);
        case 6: return run_staged<128, 128, 2, FMT, uint16_t, 4>(a);
        case 7: return run_staged<128, 128, 1, FMT, uint16_t>(a);
        default: return run_staged<128, 128, 2, FMT, uint16_t>(a);
    }
}


bool staged_gemm_supported(const LinearArgs& a) { return staged_supported_impl(a); }

// 128 x 128 tiles that all fit on the CUs at once (one a CU): with bf16
// output and at most 32 k64 steps, the wavefronts side by side along N (each
// loads its own weight rows into registers, only activations pass through
// LDS): GPT-2-XL shapes with K = 1600, M = 256 .. 2048, 7-22% faster than the
// 2 x 2 and 224-row tiles, bit-identical; else the 2 x 2 copy with four
// staging sets, whose loads go out three k64 steps before they are needed
// (7-9% faster than two sets; at K = 6400 also ahead of the side-by-side
// tile, 53 against 59 us). With more tiles the cost model's choice stands
// (e.g. M = 1024, N = 4800: 224 x 128 tiles, 24.0 against 24.7 us).
int staged_gemm_choice(const LinearArgs& a) {
    const bool one_round = ((a.M + 127) / 128) * ((a.N + 127) / 128) <= 256;
    if (one_round && a.y_dtype == TIQ_BF16 && a.K / BK <= 32) return 7;
    const int c = staged_choice(a.M, a.N, a.K, a.y_dtype == TIQ_BF16);
    return c == 2 && one_round ? 6 : c;
}

int launch_staged_gemm(const LinearArgs& a, int choice) {
    if (!staged_supported_impl(a)) return TIQ_EUNSUPPORTED;
    if (a.fmt == kW4) return a.y_dtype == TIQ_F32 ? dispatch_staged_f32<kW4>(a, choice) : dispatch_staged_bf16<kW4>(a, choice);
    return a.y_dtype == TIQ_F32 ? dispatch_staged_f32<kW8>(a, choice) : dispatch_staged_bf16<kW8>(a, choice);
}

int launch_staged_gemm_split(const LinearArgs& a, void* ws, size_t ws_bytes) {
    if ((a.fmt != kW8 && a.fmt != kW4) || !staged_supported_impl(a)) return TIQ_EUNSUPPORTED;
    // 48 tiles or more and a short K: the slices' trip through memory costs
    // more than the idle CUs (GPT-2-XL at M = 256 with N >= 4800 and at
    // M = 1024 with N = K = 1600: 7-11% slower split; M = 512, N = K = 1600,
    // 52 tiles: 18.7 split against 16.9 us on the side-by-side 128 x 128 tile)
    if (((a.M + 127) / 128) * ((a.N + 127) / 128) >= 48 && a.K / BK <= 32) return TIQ_EUNSUPPORTED;
    const int64_t S = staged_splits(a.M, a.N, a.K);
    const size_t need = staged_split_workspace(a.M, a.N, a.K);
    if (S <= 1 || !ws || ws_bytes < need || !aligned(ws, 16)) return TIQ_EUNSUPPORTED;
    float* part = static_cast<float*>(ws);
    const int64_t tiles = ((a.M + 127) / 128) * ((a.N + 127) / 128);
    // the products: raw fp32 slices [S][M][N] (unit scale, no bias in the kernel)
    const dim3 grid((unsigned)tiles, 1, (unsigned)S);
    if (a.fmt == kW4)
        hipLaunchKernelGGL((gemm_staged<128, 128, 2, kW4, float>), grid, dim3(256), 0, a.stream,
                           static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, part, (int64_t)a.N,
                           (int)a.M, (int)a.N, (int)a.K, (int)(a.kw ? a.kw : a.K), nullptr, 0, nullptr);
    else
        hipLaunchKernelGGL((gemm_staged<128, 128, 2, kW8, float>), grid, dim3(256), 0, a.stream,
                           static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, part, (int64_t)a.N,
                           (int)a.M, (int)a.N, (int)a.K, (int)(a.kw ? a.kw : a.K), nullptr, 0, nullptr);
    int rc = launch_status();
    if (rc != TIQ_OK) return rc;
    return launch_splitk_reduce(a, part, S, a.scale);
}

int launch_splitk_reduce(const LinearArgs& a, const float* part, int64_t S, const float* scale) {
    const int64_t quads = a.M * a.N / 4;
    const dim3 grid((unsigned)((quads + 255) / 256));
    if (a.y_dtype == TIQ_F32)
        hipLaunchKernelGGL(splitk_reduce_kernel<float>, grid, dim3(256), 0, a.stream, part, (int)S, (int)a.M,
                           (int)a.N, scale, a.bias, static_cast<float*>(a.y), a.ldy);
    else
        hipLaunchKernelGGL(splitk_reduce_kernel<uint16_t>, grid, dim3(256), 0, a.stream, part, (int)S, (int)a.M,
                           (int)a.N, scale, a.bias, static_cast<uint16_t*>(a.y), a.ldy);
    return launch_status();
}

}  // namespace tiq
