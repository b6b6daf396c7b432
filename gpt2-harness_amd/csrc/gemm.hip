// Prefill GEMM on the matrix cores (gfx950), for the reference's quantized
// Linears over a whole prompt (model.py:254,319,352,355 with M = B*T):
//     y[m, n] = scale[n] * sum_k x[m, k] * q[n, k] + bias[n]
//
//   * workgroup tile BM x BN over (M, N), BK = 64 columns of K per step;
//     four wavefronts in a 2 x 2 arrangement, each owning a
//     (BM/2) x (BN/2) block of 16 x 16 v_mfma_f32_16x16x32_bf16 tiles;
//   * activations (bf16) and weights (int8 or int4 nibbles) stream from HBM
//     with 128-bit loads; the weight codes are converted to bf16 in registers
//     (exact: every int8 value is a bf16) before they are written to LDS, so
//     the MFMA reads bf16 operands for both sides;
//   * LDS rows are padded by 16 bytes so that the 16 lanes reading one
//     fragment column hit 16 disjoint bank quads;
//   * the next k-step's global loads are issued before the current step's
//     MFMAs (register prefetch), so HBM latency hides behind the matrix cores;
//   * the epilogue multiplies the fp32 accumulators by the per-channel scale
//     and adds the bias, exactly once per output.
#include "tiq_internal.hpp"

namespace tiq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (16-byte pad)
constexpr int kThreads = 256;

// two sign-extended bytes -> two bf16 in one dword (exact)
__device__ __forceinline__ uint32_t bf16x2_of_bytes(uint32_t d, int shift_lo) {
    const float lo = (float)((int32_t)(d << (24 - shift_lo)) >> 24);
    const float hi = (float)((int32_t)(d << (16 - shift_lo)) >> 24);
    return (__float_as_uint(hi) & 0xffff0000u) | (__float_as_uint(lo) >> 16);
}

// 4 int8 codes of a dword -> 4 bf16 (two dwords)
__device__ __forceinline__ uint2 bf16x4_of_i8x4(uint32_t d) {
    return make_uint2(bf16x2_of_bytes(d, 0), bf16x2_of_bytes(d, 16));
}

// two biased nibbles -> two bf16 in one dword
__device__ __forceinline__ uint32_t bf16x2_of_nibbles(uint32_t d, int sh) {
    const float lo = (float)((int32_t)((d >> sh) & 0xfu) - 8);
    const float hi = (float)((int32_t)((d >> (sh + 4)) & 0xfu) - 8);
    return (__float_as_uint(hi) & 0xffff0000u) | (__float_as_uint(lo) >> 16);
}

template <int BM, int BN, int FMT, typename TY>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                        const uint8_t* __restrict__ w, int64_t ldw,
                                                        const float* __restrict__ scale,
                                                        const float* __restrict__ bias, TY* __restrict__ y,
                                                        int64_t ldy, int M, int N, int K) {
    constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
    constexpr int TM = WM / 16, TN = WN / 16;    // MFMA tiles per wave
    constexpr int A_VEC = BM * BK / 8 / kThreads;  // uint4 (8 bf16) per thread
    // weights: int8 -> 16 codes per uint4; int4 -> 32 codes per uint4
    constexpr int CODES = (FMT == kW8) ? 16 : 32;
    constexpr int B_VEC = BN * BK / CODES / kThreads;
    static_assert(A_VEC >= 1 && B_VEC >= 1, "tile too small for the workgroup");

    __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int m_blk = blockIdx.y * BM, n_blk = blockIdx.x * BN;

    // global -> register staging
    uint4 ra[A_VEC], rb[B_VEC];
    auto load_tiles = [&](int k0) {
#pragma unroll
        for (int j = 0; j < A_VEC; ++j) {
            const int i = tid + kThreads * j;
            const int row = i / (BK / 8), c8 = i % (BK / 8);
            int gm = m_blk + row;
            gm = gm < M ? gm : M - 1;
            ra[j] = *reinterpret_cast<const uint4*>(x + (int64_t)gm * ldx + k0 + c8 * 8);
        }
#pragma unroll
        for (int j = 0; j < B_VEC; ++j) {
            const int i = tid + kThreads * j;
            constexpr int PER_ROW = BK / CODES;
            const int row = i / PER_ROW, cc = i % PER_ROW;
            int gn = n_blk + row;
            gn = gn < N ? gn : N - 1;
            const int64_t byte = (FMT == kW8) ? (int64_t)k0 + cc * 16 : (int64_t)(k0 / 2) + cc * 16;
            rb[j] = *reinterpret_cast<const uint4*>(w + (int64_t)gn * ldw + byte);
        }
    };
    auto store_tiles = [&]() {
#pragma unroll
        for (int j = 0; j < A_VEC; ++j) {
            const int i = tid + kThreads * j;
            const int row = i / (BK / 8), c8 = i % (BK / 8);
            *reinterpret_cast<uint4*>(&As[row * LDS_STRIDE + c8 * 8]) = ra[j];
        }
#pragma unroll
        for (int j = 0; j < B_VEC; ++j) {
            const int i = tid + kThreads * j;
            constexpr int PER_ROW = BK / CODES;
            const int row = i / PER_ROW, cc = i % PER_ROW;
            const uint32_t d[4] = {rb[j].x, rb[j].y, rb[j].z, rb[j].w};
            uint16_t* dst = &Bs[row * LDS_STRIDE + cc * CODES];
            if (FMT == kW8) {
                const uint2 a0 = bf16x4_of_i8x4(d[0]), a1 = bf16x4_of_i8x4(d[1]);
                const uint2 a2 = bf16x4_of_i8x4(d[2]), a3 = bf16x4_of_i8x4(d[3]);
                reinterpret_cast<uint4*>(dst)[0] = make_uint4(a0.x, a0.y, a1.x, a1.y);
                reinterpret_cast<uint4*>(dst)[1] = make_uint4(a2.x, a2.y, a3.x, a3.y);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    reinterpret_cast<uint4*>(dst)[q] =
                        make_uint4(bf16x2_of_nibbles(d[q], 0), bf16x2_of_nibbles(d[q], 8),
                                   bf16x2_of_nibbles(d[q], 16), bf16x2_of_nibbles(d[q], 24));
                }
            }
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int frag_row = lane & 15, frag_k = (lane >> 4) * 8;
    load_tiles(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();  // previous step's LDS reads are done
        store_tiles();
        __syncthreads();
        if (k0 + BK < K) load_tiles(k0 + BK);
#pragma unroll
        for (int sub = 0; sub < BK / 32; ++sub) {
            bf16x8 af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(&As[(wm + i * 16 + frag_row) * LDS_STRIDE + sub * 32 + frag_k]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[(wn + j * 16 + frag_row) * LDS_STRIDE + sub * 32 + frag_k]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
    }

    // epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each tile
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n_blk + wn + j * 16 + (lane & 15);
        if (n >= N) continue;
        const float s = scale[n];
        const float b = bias ? bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m_blk + wm + i * 16 + (lane >> 4) * 4 + r;
                if (m < M) {
                    const float v = fmaf(acc[i][j][r], s, b);
                    if constexpr (sizeof(TY) == 4) y[(int64_t)m * ldy + n] = v;
                    else y[(int64_t)m * ldy + n] = f32_to_bf16_bits(v);
                }
            }
        }
    }
}

template <int BM, int BN, int FMT, typename TY>
int run_gemm(const LinearArgs& a) {
    const dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM));
    hipLaunchKernelGGL((gemm_kernel<BM, BN, FMT, TY>), grid, dim3(kThreads), 0, a.stream,
                       static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, static_cast<TY*>(a.y),
                       a.ldy, (int)a.M, (int)a.N, (int)a.K);
    return launch_status();
}

template <int FMT>
int dispatch_gemm(const LinearArgs& a) {
    if (a.y_dtype == TIQ_F32) return run_gemm<128, 128, FMT, float>(a);
    return run_gemm<128, 128, FMT, uint16_t>(a);
}

}  // namespace

bool gemm_supported(const LinearArgs& a) {
    if (a.x_dtype != TIQ_BF16) return false;
    if (a.fmt == kW4G) return false;
    if (a.K % BK != 0) return false;
    if (!aligned(a.x, 16) || a.ldx % 8 != 0) return false;
    if (!aligned(a.w, 16) || a.ldw % 16 != 0) return false;
    if (a.M > 0x7fffffff || a.N > 0x7fffffff || a.K > 0x7fffffff) return false;
    return true;
}

int launch_gemm(const LinearArgs& a) {
    if (!gemm_supported(a)) return TIQ_EUNSUPPORTED;
    if (a.fmt == kW8) return dispatch_gemm<kW8>(a);
    return dispatch_gemm<kW4>(a);
}

}  // namespace tiq
