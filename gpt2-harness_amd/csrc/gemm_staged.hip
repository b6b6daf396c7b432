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

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int kXcds = 8;

// ------------------------------------------------------------ staged GEMM
// The int8 GEMM used for large M. One workgroup of 4 wavefronts (one per
// SIMD) owns a BM x BN output tile; the wavefronts are laid out WMW x (4 /
// WMW) over it, each owning a (BM / WMW) x (BN * WMW / 4) block of
// 32 x 32 x 16 bf16 MFMA tiles (accumulators in AGPRs). WMW = 2 gives square
// wave blocks (256 x 256, 256 x 128, 128 x 128 tiles); WMW = 1 puts the four
// side by side along N, which admits tile heights that are odd multiples of
// 32 (224 x 256, 160 x 256, 224 x 128): those make the tile count of the
// GPT-2-XL shapes at M = 4096 just under a whole number of rounds of 256 CUs.
//
//   * Staging through registers: every k64 step each thread loads 16-byte
//     chunks of x (bf16) and of the int8 weight rows into one of two register
//     sets; a chunk is written to LDS one step after it was loaded, so global
//     load latency is hidden behind a full step of MFMAs. Weight codes become
//     bf16 once per workgroup, on the LDS store (exact: every int8 is a bf16).
//   * LDS double buffered: 128-byte rows (64 bf16 of K), 16-byte chunks
//     XOR-swizzled by swz8(row) so that fragment reads (32 rows, one chunk)
//     and staging stores (8 threads per row) are free of bank conflicts.
//   * The k64 step is issued as bundles of one MFMA plus a slice of the other
//     work (the next k16's fragment reads, one staging load or store), fenced
//     with sched_barrier and an empty asm memory clobber so that neither the
//     scheduler nor the IR passes regroup them. One barrier per step, placed
//     before the last k16 group, whose fragments are already in registers.
//   * k order: MFMA block b (0..3) of a k64 step takes, in lane (r, h), the 8
//     columns 32 (b / 2) + 16 h + 8 (b % 2) .. + 7 of its row, for both
//     operands (every staged tile sums the same column groups in the same
//     order, so a bf16 result is the rounding of any tile's fp32 result). A
//     lane's 16 consecutive bytes of a row then feed two MFMA blocks.
//   * Weights in registers (WMW = 1, int8): each wavefront owns its weight
//     rows, so it loads them straight from memory in that operand order (16
//     bytes a lane, two k64 steps ahead) and widens them to bf16 one k16 group
//     before their MFMAs; only the activations pass through LDS, which halves
//     the LDS traffic of a step (GPT-2-XL shapes at M = 4096 with K = 1600:
//     5-7% faster; at K = 6400 the 2 x 2 layout stays ahead).
//   * Output through LDS: the accumulators are scaled, biased and converted,
//     written to an XOR-swizzled LDS tile, then stored as whole 16-byte row
//     chunks (a wavefront writes contiguous rows), which costs a few
//     microseconds per tile instead of the tens a scattered 8-byte store of
//     the MFMA register layout costs.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Bijective tile index -> tile map: the tiles are split into 8 contiguous
// ranges, one per XCD (dispatch round-robins workgroups over the XCDs, and a
// persistent workgroup's later indices differ by a multiple of 8), and each
// range is walked in groups of 4 row tiles so that concurrently running
// workgroups of an XCD share x and weight panels in its L2.
__device__ __forceinline__ void staged_tile_of(int i, int& tm, int& tn, int tiles_m, int tiles_n) {
    const int total = tiles_m * tiles_n;
    const int q = total / kXcds, r = total % kXcds;
    const int xcd = i % kXcds, local = i / kXcds;
    const int id = (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
    constexpr int G = 4;
    const int group = id / (G * tiles_n);
    const int first_m = group * G;
    const int gm = (tiles_m - first_m) < G ? (tiles_m - first_m) : G;
    const int in = id % (G * tiles_n);
    tm = first_m + in % gm;
    tn = in / gm;
}

__device__ __forceinline__ uint32_t bf16x2_of_bytes_perm(uint32_t d, int sh) {
    const float lo = (float)((int32_t)(d << (24 - sh)) >> 24);
    const float hi = (float)((int32_t)(d << (16 - sh)) >> 24);
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// the two biased nibbles of byte sh / 8 of d (low = even column) -> two bf16
// in one dword (exact)
__device__ __forceinline__ uint32_t bf16x2_of_nibbles_perm(uint32_t d, int sh) {
    const float lo = (float)((int32_t)((d >> sh) & 0xfu) - 8);
    const float hi = (float)((int32_t)((d >> (sh + 4)) & 0xfu) - 8);
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// FMT: kW8 (int8 codes) or kW4 (the reference's nibbles), per-row scale.
// Nibble rows are staged 8 bytes a thread per k64 step into the same bf16
// LDS layout as int8 rows. (Group-wise int4 runs on gemm32_kernel: folding a
// group's partial tiles into the sums every two k steps drains the MFMA
// pipeline of a 4-wavefront workgroup, and the partial tiles beside the sums
// halve the workgroups a CU holds -- measured slower than that kernel.)
template <int BM, int BN, int WMW, int FMT, typename TY>
__global__ __launch_bounds__(256, 1) void gemm_staged(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, const float* __restrict__ bias, TY* __restrict__ y, int64_t ldy, int M, int N,
    int K, int kw) {
    static_assert(FMT == kW8 || FMT == kW4, "int8 or reference-layout int4 weights");
    constexpr bool WD = WMW == 1 && FMT == kW8;  // weights straight into registers
    constexpr int NT = 256;
    constexpr int WNW = 4 / WMW;
    constexpr int WM = BM / WMW, WN = BN / WNW;
    constexpr int TMm = WM / 32, TNn = WN / 32;
    constexpr int XS = BM * 128, WS = WD ? 0 : BN * 128, STAGE = XS + WS;
    constexpr int XL = BM * 8 / NT, WL = WD ? 0 : BN * 4 / NT, NL = XL + WL;  // staging loads per thread per step
    constexpr int WLD = WD ? 2 * TNn : 0;                                     // direct weight loads per step
    constexpr int NMF = TMm * TNn, NRD = TMm + (WD ? 0 : TNn);                // per k16
    static_assert((WMW == 1 || WMW == 2) && WM % 32 == 0 && WN % 32 == 0, "wave layout");
    static_assert(XL * NT == BM * 8 && WL * NT == (WD ? 0 : BN * 4), "staging split");
    static_assert(NL <= 3 * NMF && NRD <= 2 * NMF && WLD <= NMF, "staging ops and fragment reads per bundle");
    constexpr int UNIT = 16 / (int)sizeof(TY);  // output elements per 16-byte chunk
    constexpr int UNITS = BN / UNIT;            // chunks per output row
    constexpr int OUTB = BM * BN * (int)sizeof(TY);
    // with the weights out of LDS the whole output tile fits in one pass
    constexpr int SMEM = WD && OUTB > 2 * STAGE ? OUTB : 2 * STAGE;
    constexpr int PASSES = (OUTB + SMEM - 1) / SMEM;
    static_assert(PASSES == 1 || (PASSES == 2 && WMW == 2), "output tile passes");
    // a persistent grid (several tiles a workgroup) only where the next tile's
    // first loads fit beside the accumulators without spilling
    constexpr bool PERSIST = NMF * 16 <= 192;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
    __shared__ __attribute__((aligned(16))) float sb_s[2][BN];  // the tile's scale and bias

    // Tiles blockIdx.x, blockIdx.x + gridDim.x, ... (one unless the grid is
    // persistent: fewer workgroups than tiles, one per CU)
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tile = blockIdx.x, tm, tn;
    staged_tile_of(tile, tm, tn, tiles_m, tiles_n);
    int m_blk = tm * BM, n_blk = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave / WNW) * WM, wn = (wave % WNW) * WN;

    // staging: x rows xrow + 32 q (8 threads per row), weight rows wrow + 64 j
    // (4 threads per row); rows are clamped for a partial tile
    const int xrow = tid >> 3, xch = tid & 7;
    const int wrow = tid >> 2, wch = tid & 3;
    const uint32_t ldx2 = (uint32_t)ldx * 2u, ldw1 = (uint32_t)ldw;
    const int xs0 = xrow * 128 + ((xch ^ swz8(xrow)) * 16);
    const int ws00 = XS + wrow * 128 + (((2 * wch) ^ swz8(wrow)) * 16);
    const int ws01 = XS + wrow * 128 + (((2 * wch + 1) ^ swz8(wrow)) * 16);
    u32x4 sx[2][XL], sw[2][WL];
    auto gload = [&](int k0, int p, int q) {
        if (q < XL) {
            const uint32_t off = (uint32_t)min(m_blk + xrow + 32 * q, M - 1) * ldx2 + xch * 16;
            sx[p][q] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(x) + 2 * k0 + off);
        } else {
            const int j = q - XL;
            if constexpr (FMT == kW8) {
                const uint32_t off = (uint32_t)min(n_blk + wrow + 64 * j, N - 1) * ldw1 + wch * 16;
                sw[p][j] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(w) + (k0 % kw) + off);
            } else {  // 16 nibbles: 8 bytes
                const uint32_t off = (uint32_t)min(n_blk + wrow + 64 * j, N - 1) * ldw1 + wch * 8;
                const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(w) + (k0 % kw) / 2 + off);
                sw[p][j] = u32x4{v.x, v.y, 0u, 0u};
            }
        }
    };
    auto lstore = [&](uint8_t* base, int p, int q) {
        if (q < XL) {
            *reinterpret_cast<u32x4*>(base + xs0 + q * 32 * 128) = sx[p][q];
        } else {
            const int j = q - XL;
            const u32x4 v = sw[p][j];
            u32x4 lo, hi;
            if constexpr (FMT == kW8) {
                lo = u32x4{bf16x2_of_bytes_perm(v.x, 0), bf16x2_of_bytes_perm(v.x, 16),
                           bf16x2_of_bytes_perm(v.y, 0), bf16x2_of_bytes_perm(v.y, 16)};
                hi = u32x4{bf16x2_of_bytes_perm(v.z, 0), bf16x2_of_bytes_perm(v.z, 16),
                           bf16x2_of_bytes_perm(v.w, 0), bf16x2_of_bytes_perm(v.w, 16)};
            } else {
                lo = u32x4{bf16x2_of_nibbles_perm(v.x, 0), bf16x2_of_nibbles_perm(v.x, 8),
                           bf16x2_of_nibbles_perm(v.x, 16), bf16x2_of_nibbles_perm(v.x, 24)};
                hi = u32x4{bf16x2_of_nibbles_perm(v.y, 0), bf16x2_of_nibbles_perm(v.y, 8),
                           bf16x2_of_nibbles_perm(v.y, 16), bf16x2_of_nibbles_perm(v.y, 24)};
            }
            *reinterpret_cast<u32x4*>(base + ws00 + j * 64 * 128) = lo;
            *reinterpret_cast<u32x4*>(base + ws01 + j * 64 * 128) = hi;
        }
    };

    // fragments: lane (r, h) reads row base + r, chunk 4 (kk / 2) + 2 h + kk % 2
    // of k16 block kk (the k order above)
    const int r = lane & 31, h = lane >> 5;
    int fo[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) fo[kk] = r * 128 + (((4 * (kk >> 1) + 2 * h + (kk & 1)) ^ swz8(r)) * 16);
    bf16x8 FW[2][TNn], FX[2][TMm];
    constexpr int FWR = WD ? 0 : TNn;  // weight fragments read from LDS
    auto fread = [&](const uint8_t* base, int kk, int set, int q) {
        if (q < FWR) FW[set][q] = *reinterpret_cast<const bf16x8*>(base + XS + (wn + 32 * q) * 128 + fo[kk]);
        else FX[set][q - FWR] = *reinterpret_cast<const bf16x8*>(base + (wm + 32 * (q - FWR)) * 128 + fo[kk]);
    };
    // WD: lane (r, h) of tile i holds bytes 32 j + 16 h .. + 15 (j = 0, 1) of
    // the step's 64 columns of weight row n_blk + wn + 32 i + r (clamped), in
    // two raw sets; block b widens 8 of them to bf16
    u32x4 wr[2][WD ? TNn : 1][2];
    uint32_t wdrow[TNn];
#pragma unroll
    for (int i = 0; i < TNn; ++i) wdrow[i] = (uint32_t)min(n_blk + wn + 32 * i + r, N - 1) * ldw1 + 16 * h;
    auto wload = [&](int k0, int p, int q) {
        if constexpr (WD) {
            const int i = q >> 1, j = q & 1;
            wr[p][i][j] =
                *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(w) + (k0 % kw) + wdrow[i] + 32 * j);
        }
    };
    auto wfrag = [&](int p, int i, int b) {
        if constexpr (WD) {
            const u32x4 v = wr[p][i][b >> 1];
            const uint32_t s0 = (b & 1) ? v.z : v.x, s1 = (b & 1) ? v.w : v.y;
            const u32x4 t = {bf16x2_of_bytes_perm(s0, 0), bf16x2_of_bytes_perm(s0, 16),
                             bf16x2_of_bytes_perm(s1, 0), bf16x2_of_bytes_perm(s1, 16)};
            return __builtin_bit_cast(bf16x8, t);
        } else {
            return FW[0][0];
        }
    };
    // D[n][m] = sum_k w[n][k] x[m][k]: result register q of lane (r, h) holds
    // n = 8 (q / 4) + 4 h + q % 4, m = r of its 32 x 32 tile
    floatx16 acc[TNn][TMm];
    auto mfma_set = [&](int set, int t) {
        const int i = t / TMm, j = t % TMm;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FW[set][i], FX[set][j], acc[i][j], 0, 0, 0);
    };

    // split-K (gridDim.z > 1): workgroup z takes k64 steps [z NK / S, (z + 1) NK / S)
    // and writes raw fp32 partial sums (unit scale, no bias) to slice z of y
    const int NK = K / BK;
    const int s0 = (int)blockIdx.z * NK / (int)gridDim.z;
    const int nk = ((int)blockIdx.z + 1) * NK / (int)gridDim.z - s0;
    const int kbase = s0 * BK;
    const bool split = gridDim.z > 1;
    // A tile's first stage and its epilogue's per-column scale and bias
    // (columns past N repeat the last one), requested together; for the next
    // tile of a persistent workgroup this runs before the current tile's
    // epilogue, so those loads and the epilogue's stores overlap. The second
    // stage follows after the epilogue (its registers would otherwise be live
    // beside the accumulators).
    constexpr int SBN = (BN + NT - 1) / NT;
    float sbr[2][SBN];
    auto begin_tile = [&]() {
#pragma unroll
        for (int q = 0; q < NL; ++q) gload(kbase, 0, q);
#pragma unroll
        for (int q = 0; q < WLD; ++q) wload(kbase, 0, q);
#pragma unroll
        for (int c = 0; c < SBN; ++c) {
            const int n = min(n_blk + min(tid + NT * c, BN - 1), N - 1);
            sbr[0][c] = split ? 1.f : scale[n];
            sbr[1][c] = (bias && !split) ? bias[n] : 0.f;
        }
    };
    begin_tile();
    for (;;) {  // the workgroup's tiles
#pragma unroll
    for (int q = 0; q < NL; ++q) gload(kbase + min(1, nk - 1) * BK, 1, q);
#pragma unroll
    for (int q = 0; q < WLD; ++q) wload(kbase + min(1, nk - 1) * BK, 1, q);
#pragma unroll
    for (int c = 0; c < SBN; ++c)
        if (tid + NT * c < BN) sb_s[0][tid + NT * c] = sbr[0][c], sb_s[1][tid + NT * c] = sbr[1][c];
#pragma unroll
    for (int q = 0; q < NL; ++q) lstore(smem, 0, q);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NRD; ++q) fread(smem, 0, 0, q);
    if constexpr (WD) {
#pragma unroll
        for (int i = 0; i < TNn; ++i) FW[0][i] = wfrag(0, i, 0);
    }
#pragma unroll
    for (int i = 0; i < TNn; ++i)
#pragma unroll
        for (int j = 0; j < TMm; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

    // Step s: MFMAs on buffer s % 2; stage s + 1 (register set (s + 1) % 2)
    // is stored to the other buffer over the first three k16 groups; stage
    // s + 2 is loaded into set s % 2 over all four. Past the last stage the
    // loads repeat it (clamped k), which keeps the loop body one path. WD:
    // raw weight set p (this step's) is widened one k16 group ahead; by the
    // end of the third group it is free and takes step s + 2's weights in the
    // fourth, whose end widens block 0 of raw set p ^ 1 (step s + 1's).
    auto step = [&](int s, int p) {
        uint8_t* cur = smem + (s & 1) * STAGE;
        uint8_t* nxt = smem + ((s + 1) & 1) * STAGE;
        const int k2 = kbase + min(s + 2, nk - 1) * BK;
#pragma unroll
        for (int kk = 0; kk < 3; ++kk) {
            const int set = kk & 1;
#pragma unroll
            for (int t = 0; t < NMF; ++t) {
                mfma_set(set, t);
                if constexpr (NRD <= NMF) {
                    if (t < NRD) fread(cur, kk + 1, set ^ 1, t);
                } else {  // more fragments than MFMAs: spread over the bundles
#pragma unroll
                    for (int q = t * NRD / NMF; q < (t + 1) * NRD / NMF; ++q) fread(cur, kk + 1, set ^ 1, q);
                }
                if constexpr (WD) {
                    if (t < TNn) FW[set ^ 1][t] = wfrag(p, t, kk + 1);
                }
                const int b = kk * NMF + t;
                if ((b + 1) * NL / (3 * NMF) > b * NL / (3 * NMF)) lstore(nxt, p ^ 1, b * NL / (3 * NMF));
                if ((b + 1) * NL / (4 * NMF) > b * NL / (4 * NMF)) gload(k2, p, b * NL / (4 * NMF));
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NMF; ++t) {
            mfma_set(1, t);
            if constexpr (NRD <= NMF) {
                if (t < NRD) fread(nxt, 0, 0, t);
            } else {
#pragma unroll
                for (int q = t * NRD / NMF; q < (t + 1) * NRD / NMF; ++q) fread(nxt, 0, 0, q);
            }
            const int b = 3 * NMF + t;
            if ((b + 1) * NL / (4 * NMF) > b * NL / (4 * NMF)) gload(k2, p, b * NL / (4 * NMF));
            if constexpr (WD) {
                if ((t + 1) * WLD / NMF > t * WLD / NMF) wload(k2, p, t * WLD / NMF);
                if (t == NMF - 1) {
#pragma unroll
                    for (int i = 0; i < TNn; ++i) FW[0][i] = wfrag(p ^ 1, i, 0);
                }
            }
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int s = 0;
    for (; s + 1 < nk; s += 2) {
        step(s, 0);
        step(s + 1, 1);
    }
    if (s < nk) step(s, 0);
    __syncthreads();
    // the next tile's first loads, then this tile's epilogue
    const int em_blk = m_blk, en_blk = n_blk;
    tile += gridDim.x;
    const bool more = PERSIST && tile < tiles_m * tiles_n;
    if (more) {
        staged_tile_of(tile, tm, tn, tiles_m, tiles_n);
        m_blk = tm * BM;
        n_blk = tn * BN;
        if constexpr (WD) {
#pragma unroll
            for (int i = 0; i < TNn; ++i) wdrow[i] = (uint32_t)min(n_blk + wn + 32 * i + r, N - 1) * ldw1 + 16 * h;
        }
        begin_tile();
    }

    // epilogue: scale, bias, convert; LDS tile [rows of the pass][UNITS chunks],
    // chunk u of row m at position u ^ (m % UNITS)
    constexpr int ROWS = BM / PASSES;
    constexpr int ROW_BYTES = BN * (int)sizeof(TY);
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        if (PASSES == 1 || (wm / WM) == pass) {
#pragma unroll
            for (int i = 0; i < TNn; ++i) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int nl = wn + 32 * i + 8 * g + 4 * h;  // 4 consecutive outputs
                    const float4 sc = *reinterpret_cast<const float4*>(&sb_s[0][nl]);
                    const float4 bi = *reinterpret_cast<const float4*>(&sb_s[1][nl]);
#pragma unroll
                    for (int j = 0; j < TMm; ++j) {
                        const int ml = wm + 32 * j + r - pass * ROWS;
                        const float v0 = fmaf(acc[i][j][4 * g + 0], sc.x, bi.x);
                        const float v1 = fmaf(acc[i][j][4 * g + 1], sc.y, bi.y);
                        const float v2 = fmaf(acc[i][j][4 * g + 2], sc.z, bi.z);
                        const float v3 = fmaf(acc[i][j][4 * g + 3], sc.w, bi.w);
                        const int u = nl / UNIT;
                        uint8_t* dst = smem + ml * ROW_BYTES + ((u ^ (ml & (UNITS - 1))) * 16);
                        if constexpr (sizeof(TY) == 4) {
                            *reinterpret_cast<float4*>(dst) = make_float4(v0, v1, v2, v3);
                        } else {
                            // v_cvt_pk_bf16_f32 (round to nearest even, two values an
                            // instruction): the bit-level software rounding cost six
                            // instructions a value, ~60% of a 256 x 256 tile's epilogue
                            uint2 o;
                            o.x = pk_bf16(v0, v1);
                            o.y = pk_bf16(v2, v3);
                            *reinterpret_cast<uint2*>(dst + 8 * (nl % UNIT != 0)) = o;
                        }
                    }
                }
            }
        }
        __syncthreads();
        constexpr int CH = ROWS * UNITS / NT;  // 16-byte chunks per thread
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int idx = tid + NT * c;
            const int ml = idx / UNITS, u = idx % UNITS;
            const int m = em_blk + pass * ROWS + ml, n = en_blk + u * UNIT;
            const u32x4 v = *reinterpret_cast<const u32x4*>(smem + ml * ROW_BYTES + ((u ^ (ml & (UNITS - 1))) * 16));
            // nontemporal: the output is written once and read by a later kernel
            if (m < M && n < N)
                __builtin_nontemporal_store(
                    v, reinterpret_cast<u32x4*>(y + ((int64_t)blockIdx.z * M + m) * ldy + n));
        }
        if (pass + 1 < PASSES) __syncthreads();
    }
    if (!more) break;
    __syncthreads();  // the epilogue's LDS reads are done before the next tile's stores
    }
}

// The kernel's PERSIST condition, on the host: tiles whose accumulators leave
// room for the next tile's first loads run on a persistent grid of one
// workgroup per tile slot (256 CUs x the workgroups a CU holds).
template <int BM, int BN, int WMW>
constexpr bool staged_persist() {
    return (BM / WMW / 32) * (BN * WMW / 4 / 32) * 16 <= 192;
}

template <int BM, int BN, int WMW, int FMT, typename TY>
int run_staged(const LinearArgs& a) {
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const int64_t slots = 256 * (BM * BN <= 128 * 128 ? 2 : 1);
    const int64_t grid = staged_persist<BM, BN, WMW>() ? std::min(tiles, slots) : tiles;
    hipLaunchKernelGGL((gemm_staged<BM, BN, WMW, FMT, TY>), dim3((unsigned)grid), dim3(256), 0, a.stream,
                       static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, static_cast<TY*>(a.y),
                       a.ldy, (int)a.M, (int)a.N, (int)a.K, (int)(a.kw ? a.kw : a.K));
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
        default: return run_staged<128, 128, 2, FMT, uint16_t>(a);
    }
}


bool staged_gemm_supported(const LinearArgs& a) { return staged_supported_impl(a); }

int staged_gemm_choice(const LinearArgs& a) { return staged_choice(a.M, a.N, a.K, a.y_dtype == TIQ_BF16); }

int launch_staged_gemm(const LinearArgs& a, int choice) {
    if (!staged_supported_impl(a)) return TIQ_EUNSUPPORTED;
    if (a.fmt == kW4) return a.y_dtype == TIQ_F32 ? dispatch_staged_f32<kW4>(a, choice) : dispatch_staged_bf16<kW4>(a, choice);
    return a.y_dtype == TIQ_F32 ? dispatch_staged_f32<kW8>(a, choice) : dispatch_staged_bf16<kW8>(a, choice);
}

int launch_staged_gemm_split(const LinearArgs& a, void* ws, size_t ws_bytes) {
    if (a.fmt != kW8 || !staged_supported_impl(a)) return TIQ_EUNSUPPORTED;
    const int64_t S = staged_splits(a.M, a.N, a.K);
    const size_t need = staged_split_workspace(a.M, a.N, a.K);
    if (S <= 1 || !ws || ws_bytes < need || !aligned(ws, 16)) return TIQ_EUNSUPPORTED;
    float* part = static_cast<float*>(ws);
    const int64_t tiles = ((a.M + 127) / 128) * ((a.N + 127) / 128);
    // the products: raw fp32 slices [S][M][N] (unit scale, no bias in the kernel)
    hipLaunchKernelGGL((gemm_staged<128, 128, 2, kW8, float>), dim3((unsigned)tiles, 1, (unsigned)S), dim3(256), 0,
                       a.stream, static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, part,
                       (int64_t)a.N, (int)a.M, (int)a.N, (int)a.K, (int)(a.kw ? a.kw : a.K));
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
