// Prefill GEMM on the matrix cores (gfx950), for the reference's quantized
// Linears over a whole prompt (model.py:254,319,352,355 with M = B*T):
//     y[m, n] = scale[n] * sum_k x[m, k] * q[n, k] + bias[n]
// This LDS-dequant kernel takes the group-wise int4 products the staged
// kernels (gemm_staged.hip, gemm_grouped.hip) do not: groups other than 128
// columns, and the three-plane fp32-activation path; and, through
// tiq_gemm_w8_tile's tiles 1-4, int8 and reference int4 for tests.
//
//   * workgroup tile BM x BN over (M, N), BK = 64 columns of K per step;
//     WAVES_M x WAVES_N wavefronts, each owning a (BM/WAVES_M) x (BN/WAVES_N)
//     block of 32 x 32 v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulators;
//     measured on this chip the 32 x 32 x 16 form sustains 87% of the bf16
//     peak from one wave per SIMD, the 16 x 16 x 32 form 42%);
//   * activations (bf16) and weights (int8 or int4 nibbles) stream from HBM
//     with 128-bit loads; weight codes are converted to bf16 in registers
//     (exact: every int8 value is a bf16) before they are written to LDS, so
//     the MFMA reads bf16 operands on both sides;
//   * LDS is double buffered: the global loads of step k+1 are in flight
//     while step k's MFMAs run, and their LDS store goes to the other buffer,
//     so each step needs one barrier;
//   * LDS tiles are XOR-swizzled (see gemm32_kernel) so fragment reads and
//     tile stores are free of bank conflicts without padding;
//   * workgroups are renumbered so that the ones sharing an XCD (dispatch
//     order round-robins over the 8 XCDs) take neighbouring tiles, and
//     within an XCD tiles are walked in column groups so the A panel and the
//     weight panel they share stay in that XCD's L2;
//   * the epilogue multiplies the fp32 accumulators by the per-channel scale
//     and adds the bias, exactly once per output.
#include <algorithm>
#include <cstdlib>
#include <utility>

#include "tiq_internal.hpp"

namespace tiq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16 bytes in flight, as plain loads

constexpr int BK = 64;
constexpr int kXcds = 8;

// two sign-extended bytes -> two bf16 in one dword (exact)
__device__ __forceinline__ uint32_t bf16x2_of_bytes(uint32_t d, int shift_lo) {
    const float lo = (float)((int32_t)(d << (24 - shift_lo)) >> 24);
    const float hi = (float)((int32_t)(d << (16 - shift_lo)) >> 24);
    return (__float_as_uint(hi) & 0xffff0000u) | (__float_as_uint(lo) >> 16);
}

// two biased nibbles -> two bf16 in one dword
__device__ __forceinline__ uint32_t bf16x2_of_nibbles(uint32_t d, int sh) {
    const float lo = (float)((int32_t)((d >> sh) & 0xfu) - 8);
    const float hi = (float)((int32_t)((d >> (sh + 4)) & 0xfu) - 8);
    return (__float_as_uint(hi) & 0xffff0000u) | (__float_as_uint(lo) >> 16);
}

// Workgroup id -> (tile_m, tile_n): XCD-contiguous, then column groups of
// GROUP_M row tiles.
__device__ __forceinline__ void tile_of(int& tm, int& tn, int tiles_m, int tiles_n) {
    const int total = tiles_m * tiles_n;
    int id = blockIdx.x;
    if (total % kXcds == 0) {
        const int per = total / kXcds;
        id = (id % kXcds) * per + id / kXcds;
    }
    constexpr int GROUP_M = 8;
    const int group = id / (GROUP_M * tiles_n);
    const int first_m = group * GROUP_M;
    const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
    const int in = id % (GROUP_M * tiles_n);
    tm = first_m + in % gm;
    tn = in / gm;
}

// Version with 32 x 32 x 16 MFMA tiles and an XOR-swizzled LDS layout.
// Each LDS row of a tile holds BK = 64 bf16 (eight 16-byte chunks); chunk c
// of row r is stored at chunk position c ^ (r % 8), so the 32 lanes that read
// one fragment (32 consecutive rows, same logical chunk) and the 8 lanes that
// write one row both touch 8 distinct chunk positions: no bank conflicts and
// no padding, which lets two 128 x 128 workgroups share a CU.
// v_mfma_f32_32x32x16_bf16 operands: lane l holds A[l % 32][8 (l / 32) + 0..7]
// and B[8 (l / 32) + 0..7][l % 32]; result register r of lane l is
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 3); }

// Group-wise int4 (FMT == kW4G): the nibbles are staged exactly as the
// reference layout's, and every group of `group` columns (a multiple of BK, so
// no k step straddles two groups) is accumulated into its own fp32 partial
// sums (MFMA from zero at the group's first step); at the group's last step
// each partial is multiplied by its column's fp16 scale (converted exactly to
// fp32) and added to the running sums, so the result is
//     y[m, n] = sum_g s[n, g] * (sum_{k in g} x[m, k] * q[n, k]) + bias[n]
// with no rounding beyond fp32 accumulation. The last group may be short
// (K = 1600 with group 128: twelve groups of two steps and one of one).
// kw: the period of K in the weight matrix (the GEMM reads weight column
// k % kw): K = 3 kw for fp32 activations split into three bf16 planes laid side
// by side (x = hi + lo + lo2, each product exact), kw = K otherwise. Groups
// restart with every plane.
// Split over K (gridDim.z = S > 1, group-wise int4 with kw = K only): workgroup
// z takes the whole groups [z G / S, (z + 1) G / S) of the G groups and writes
// its fp32 sums (groups already scaled) to slice z of y, without bias; the
// split-K reduction adds the slices in order and the bias.
// f(integral_constant<int, J>) for J = 0 .. sizeof...(J) - 1, in order: a
// register array indexed by J stays in registers whatever the loop passes do.
template <int... J, typename F>
__device__ __forceinline__ void for_each_index(std::integer_sequence<int, J...>, F&& f) {
    (f(std::integral_constant<int, J>{}), ...);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int OCC, int FMT, typename TY>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64, OCC) void gemm32_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, const uint16_t* __restrict__ scale16, int group,
    const float* __restrict__ bias, TY* __restrict__ y, int64_t ldy, int M, int N, int K, int kw) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave tile
    constexpr int TM = WM / 32, TN = WN / 32;            // 32 x 32 MFMA tiles per wave
    constexpr int A_VEC = BM * BK / 8 / NT;              // 16-byte chunks of A per thread
    constexpr int CODES = (FMT == kW8) ? 16 : 32;        // weight codes per 16-byte load
    constexpr bool GROUPED = FMT == kW4G;
    constexpr int B_VEC = BN * BK / CODES / NT;
    constexpr int B_PER_ROW = BK / CODES;
    static_assert(A_VEC >= 1 && B_VEC >= 1 && BM * BK % (8 * NT) == 0 && BN * BK % (CODES * NT) == 0,
                  "tile does not divide over the workgroup");

    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * BK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * BK];

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(tm, tn, tiles_m, tiles_n);
    const int m_blk = tm * BM, n_blk = tn * BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave / WAVES_N) * WM, wn = (wave % WAVES_N) * WN;

    int64_t a_off[A_VEC];
    int a_dst[A_VEC];
#pragma unroll
    for (int j = 0; j < A_VEC; ++j) {
        const int i = tid + NT * j;
        const int row = i / (BK / 8), c8 = i % (BK / 8);
        const int gm = (m_blk + row < M) ? m_blk + row : M - 1;
        a_off[j] = (int64_t)gm * ldx + c8 * 8;
        a_dst[j] = swz(row, c8);
    }
    int64_t b_off[B_VEC];
    int b_row[B_VEC], b_c8[B_VEC];
#pragma unroll
    for (int j = 0; j < B_VEC; ++j) {
        const int i = tid + NT * j;
        const int row = i / B_PER_ROW, cc = i % B_PER_ROW;
        const int gn = (n_blk + row < N) ? n_blk + row : N - 1;
        b_off[j] = (int64_t)gn * ldw + cc * 16;
        b_row[j] = row;
        b_c8[j] = cc * (CODES / 8);  // first 8-column chunk this load fills
    }

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    // group-wise scales: this lane's output columns (one per 32-wide tile
    // column j, clamped for a partial tile) and the group's partial sums
    const int ngroups = GROUPED ? (kw + group - 1) / group : 1;
    int64_t srow[TN];
    floatx16 part[GROUPED ? TM : 1][GROUPED ? TN : 1];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n_blk + wn + j * 32 + (lane & 31);
        srow[j] = (int64_t)(n < N ? n : N - 1) * ngroups;
    }

    const int frag_row = lane & 31, frag_c = lane >> 5;  // row in the tile, chunk within a k16 step
    const int nk = K / BK;
    // this workgroup's k steps [s_begin, s_end): all of K, or whole groups of a split
    int s_begin = 0, s_end = nk;
    if (GROUPED && gridDim.z > 1) {
        const int gsteps = group / BK, G = (nk + gsteps - 1) / gsteps;
        s_begin = (int)blockIdx.z * G / (int)gridDim.z * gsteps;
        s_end = min(((int)blockIdx.z + 1) * G / (int)gridDim.z * gsteps, nk);
    }
    TY* const yz = y + (int64_t)blockIdx.z * M * ldy;
    // A ring of NS register sets: step t's tiles (and, group-wise, its
    // group's scales) are loaded into set (t - s_begin) % NS during step
    // t - NS + 1 and go to LDS at the end of step t - 1, so each load has
    // NS - 2 steps of MFMA work to arrive behind (a 128 x 128 tile's step is
    // short against a trip to HBM). No load sits under a branch inside the
    // unrolled ring: the compiler's wait counts stay exact only where every
    // path issues the same loads.
    constexpr int NS = (OCC >= 2 || BM * BN > 128 * 128) ? 3 : 4;  // within the register budget
    u32x4 ra[NS][A_VEC], rb[NS][B_VEC];
    uint16_t rs[NS][GROUPED ? TN : 1];
    auto load_tiles = [&](auto set_c, int step) __attribute__((always_inline)) {
        constexpr int set = decltype(set_c)::value;
        const int k0 = min(step, s_end - 1) * BK;  // past the end: repeat the last step
        const int kb = (FMT == kW8) ? k0 % kw : (k0 % kw) / 2;
#pragma unroll
        for (int j = 0; j < A_VEC; ++j) ra[set][j] = *reinterpret_cast<const u32x4*>(x + a_off[j] + k0);
#pragma unroll
        for (int j = 0; j < B_VEC; ++j) rb[set][j] = *reinterpret_cast<const u32x4*>(w + b_off[j] + kb);
        if constexpr (GROUPED) {
            const int g = (k0 % kw) / group;
#pragma unroll
            for (int jj = 0; jj < TN; ++jj) rs[set][jj] = scale16[srow[jj] + g];
        }
    };
    auto store_tiles = [&](auto set_c, int buf) __attribute__((always_inline)) {
        constexpr int set = decltype(set_c)::value;
#pragma unroll
        for (int j = 0; j < A_VEC; ++j) *reinterpret_cast<u32x4*>(&As[buf][a_dst[j]]) = ra[set][j];
#pragma unroll
        for (int j = 0; j < B_VEC; ++j) {
            uint16_t* base = &Bs[buf][0];
            const int r_ = b_row[j], c_ = b_c8[j];
            const u32x4 v = rb[set][j];
            if constexpr (FMT == kW8) {
                *reinterpret_cast<uint4*>(base + swz(r_, c_)) =
                    make_uint4(bf16x2_of_bytes(v.x, 0), bf16x2_of_bytes(v.x, 16), bf16x2_of_bytes(v.y, 0),
                               bf16x2_of_bytes(v.y, 16));
                *reinterpret_cast<uint4*>(base + swz(r_, c_ + 1)) =
                    make_uint4(bf16x2_of_bytes(v.z, 0), bf16x2_of_bytes(v.z, 16), bf16x2_of_bytes(v.w, 0),
                               bf16x2_of_bytes(v.w, 16));
            } else {
                const uint32_t d_[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<uint4*>(base + swz(r_, c_ + q)) =
                        make_uint4(bf16x2_of_nibbles(d_[q], 0), bf16x2_of_nibbles(d_[q], 8),
                                   bf16x2_of_nibbles(d_[q], 16), bf16x2_of_nibbles(d_[q], 24));
            }
        }
    };

    // step s (register set j = (s - s_begin) % NS): the loads of step
    // s + NS - 1 go out into set (j + NS - 1) % NS, whose tiles (step s - 1)
    // are in LDS already; step s's MFMAs run on LDS buffer (s - s_begin) % 2;
    // step s + 1's tiles go from set (j + 1) % NS to the other buffer.
    auto iteration = [&](int s, auto j_c) __attribute__((always_inline)) {
        constexpr int j = decltype(j_c)::value;
        const int buf = (s - s_begin) & 1;
        load_tiles(std::integral_constant<int, (j + NS - 1) % NS>{}, s + NS - 1);
        const int sk = (s * BK) % kw;  // the step's first weight column
        if constexpr (GROUPED) {
            if (sk % group == 0) {  // a new group: partial sums from zero
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int jj = 0; jj < TN; ++jj)
#pragma unroll
                        for (int r = 0; r < 16; ++r) part[i][jj][r] = 0.f;
            }
        }
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            bf16x8 af[TM], bfr[TN];
            const int c = 2 * kk + frag_c;
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(&As[buf][swz(wm + i * 32 + frag_row, c)]);
#pragma unroll
            for (int jj = 0; jj < TN; ++jj)
                bfr[jj] = *reinterpret_cast<const bf16x8*>(&Bs[buf][swz(wn + jj * 32 + frag_row, c)]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int jj = 0; jj < TN; ++jj) {
                    if constexpr (GROUPED)
                        part[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[jj], part[i][jj], 0, 0, 0);
                    else
                        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[jj], acc[i][jj], 0, 0, 0);
                }
        }
        if constexpr (GROUPED) {
            if ((sk + BK) % group == 0 || sk + BK == kw || s + 1 == s_end) {  // the group's last step
#pragma unroll
                for (int jj = 0; jj < TN; ++jj) {
                    const float sg = f16_bits_to_f32(rs[j][jj]);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][jj][r] = fmaf(part[i][jj][r], sg, acc[i][jj][r]);
                }
            }
        }
        store_tiles(std::integral_constant<int, (j + 1) % NS>{}, buf ^ 1);
        __syncthreads();
    };

    for_each_index(std::make_integer_sequence<int, NS - 1>{}, [&](auto j) __attribute__((always_inline)) { load_tiles(j, s_begin + j); });
    store_tiles(std::integral_constant<int, 0>{}, 0);
    __syncthreads();
    int s0 = s_begin;
    for (; s0 + NS <= s_end; s0 += NS)
        for_each_index(std::make_integer_sequence<int, NS>{}, [&](auto j) __attribute__((always_inline)) { iteration(s0 + j, j); });
    for_each_index(std::make_integer_sequence<int, NS - 1>{}, [&](auto j) __attribute__((always_inline)) {
        if (s0 + j < s_end) iteration(s0 + j, j);
    });

#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n_blk + wn + j * 32 + (lane & 31);
        if (n >= N) continue;
        const float s = GROUPED ? 1.f : scale[n];
        const float b = bias ? bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m_blk + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M) {
                    const float v = fmaf(acc[i][j][r], s, b);
                    if constexpr (sizeof(TY) == 4) yz[(int64_t)m * ldy + n] = v;
                    else yz[(int64_t)m * ldy + n] = f32_to_bf16_bits(v);
                }
            }
        }
    }
}


template <int BM, int BN, int WMW, int WNW, int OCC, int FMT, typename TY>
int run_gemm32(const LinearArgs& a) {
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm32_kernel<BM, BN, WMW, WNW, OCC, FMT, TY>), dim3((unsigned)tiles), dim3(WMW * WNW * 64),
                       0, a.stream, static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.scale16, a.group,
                       a.bias, static_cast<TY*>(a.y), a.ldy, (int)a.M, (int)a.N, (int)a.K, (int)(a.kw ? a.kw : a.K));
    return launch_status();
}

// Tile configurations (0 = automatic), selectable through tiq_gemm_w8_tile
// for tests and measurement.
template <int FMT, typename TY>
int dispatch_tile(const LinearArgs& a, int tile) {
    switch (tile) {
        case 1: return run_gemm32<128, 128, 2, 2, 1, FMT, TY>(a);
        case 2: return run_gemm32<256, 128, 2, 2, 1, FMT, TY>(a);
        case 3: return run_gemm32<128, 256, 2, 2, 1, FMT, TY>(a);
        case 4:
            if constexpr (FMT == kW8) return run_gemm32<256, 128, 4, 2, 1, FMT, TY>(a);
            else return run_gemm32<256, 128, 2, 2, 1, FMT, TY>(a);
        default: break;
    }
    // 128 x 128 tiles, two workgroups per CU (64 KB of LDS each)
    return run_gemm32<128, 128, 2, 2, 2, FMT, TY>(a);
}

template <int FMT>
int dispatch_gemm(const LinearArgs& a, int tile) {
    if constexpr (FMT == kW4G) {
        if (tile == 0 && staged_w4g_supported(a)) return launch_staged_w4g(a, nullptr, 0);
    }
    if ((tile == 0 || tile >= 10) && staged_gemm_supported(a))
        return launch_staged_gemm(a, tile >= 10 ? tile - 10 : staged_gemm_choice(a));
    if (a.y_dtype == TIQ_F32) return dispatch_tile<FMT, float>(a, tile);
    return dispatch_tile<FMT, uint16_t>(a, tile);
}

}  // namespace

bool gemm_supported(const LinearArgs& a) {
    if (a.x_dtype != TIQ_BF16) return false;
    if (a.fmt == kF32) return false;
    // group-wise int4: whole k steps per group (the GPT-2 group of 128 is two)
    if (a.fmt == kW4G && (a.group % BK != 0 || !aligned(a.scale16, 2))) return false;
    if (a.K % BK != 0) return false;
    if (a.kw && (a.kw % BK != 0 || a.K % a.kw != 0)) return false;
    if (!aligned(a.x, 16) || a.ldx % 8 != 0) return false;
    if (!aligned(a.w, 16) || a.ldw % 16 != 0) return false;
    if (a.M > 0x7fffffff || a.N > 0x7fffffff || a.K > 0x7fffffff) return false;
    return true;
}

int launch_gemm_tile(const LinearArgs& a, int tile) {
    if (!gemm_supported(a)) return TIQ_EUNSUPPORTED;
    if (tile < 0 || (tile > 4 && (tile < 10 || tile > 17))) return TIQ_EINVAL;
    if (a.fmt == kW8) return dispatch_gemm<kW8>(a, tile);
    if (a.fmt == kW4G) return dispatch_gemm<kW4G>(a, tile);
    return dispatch_gemm<kW4>(a, tile);
}

int launch_gemm(const LinearArgs& a) { return launch_gemm_tile(a, 0); }

int launch_gemm_w4g_split(const LinearArgs& a, void* ws, size_t ws_bytes) {
    if (a.fmt != kW4G || a.x_dtype != TIQ_BF16 || (a.kw && a.kw != a.K) || !gemm_supported(a))
        return TIQ_EUNSUPPORTED;
    // the reduction's 16-byte accesses of y and the bias
    const int unit = a.y_dtype == TIQ_F32 ? 4 : 8;
    if (a.N % unit != 0 || a.ldy % unit != 0 || !aligned(a.y, 16) || (a.bias && !aligned(a.bias, 16)))
        return TIQ_EUNSUPPORTED;
    const int64_t gsteps = a.group / BK, G = (a.K / BK + gsteps - 1) / gsteps;
    const int64_t S = std::min<int64_t>(staged_splits(a.M, a.N, a.K), G);  // at least one group a split
    if (S <= 1) return TIQ_EUNSUPPORTED;
    const size_t need = (size_t)(S * a.M * a.N) * 4;
    if (!ws || ws_bytes < need || !aligned(ws, 16) || a.M * a.N * S > 0x7fffffffLL) return TIQ_EUNSUPPORTED;
    float* part = static_cast<float*>(ws);
    const int64_t tiles = ((a.M + 127) / 128) * ((a.N + 127) / 128);
    hipLaunchKernelGGL((gemm32_kernel<128, 128, 2, 2, 2, kW4G, float>), dim3((unsigned)tiles, 1, (unsigned)S),
                       dim3(256), 0, a.stream, static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale,
                       a.scale16, a.group, nullptr, part, (int64_t)a.N, (int)a.M, (int)a.N, (int)a.K, (int)a.K);
    const int rc = launch_status();
    if (rc != TIQ_OK) return rc;
    return launch_splitk_reduce(a, part, S, nullptr);
}

}  // namespace tiq
