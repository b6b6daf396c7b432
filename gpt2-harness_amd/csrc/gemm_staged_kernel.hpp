// The register-staged MFMA GEMM kernel (gemm_staged) and its tile map,
// shared by gemm_staged.hip (int8 and reference-layout int4 weights) and
// gemm_grouped.hip (group-wise int4).
// Included inside namespace tiq's anonymous namespace of each file.
#pragma once


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

// Nibbles as bf16 times 16: d holds 8 biased nibbles (column 2j in the low
// nibble of byte j, code n - 8); e (even columns) and o (odd columns) get
// each nibble in the high half of a byte with its top bit flipped, which as
// a signed byte is 16 (n - 8). A byte becomes a float in one instruction
// (sub-dword operand select with sign extension), and 16 (n - 8) is exact in
// bf16; the factor 16 is taken out in the epilogue (an exact power of two:
// every partial sum is 16 times the unscaled one, rounded the same way).
__device__ __forceinline__ void nibbles_x16(uint32_t d, uint32_t& e, uint32_t& o) {
    e = ((d << 4) & 0xf0f0f0f0u) ^ 0x80808080u;
    o = (d & 0xf0f0f0f0u) ^ 0x80808080u;
}

// byte k of e and o -> two bf16 in one dword (even column low)
__device__ __forceinline__ uint32_t bf16x2_of_x16(uint32_t e, uint32_t o, int k) {
    const float lo = (float)(int8_t)(e >> (8 * k));
    const float hi = (float)(int8_t)(o >> (8 * k));
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// FMT: kW8 (int8 codes) or kW4 (the reference's nibbles), per-row scale.
// Nibble rows are staged 8 bytes a thread per k64 step into the same bf16
// LDS layout as int8 rows.
// kW4G (group-wise nibbles, groups of 128 columns = two k64 steps, fp16 scale
// per row and group, 1 x 4 layout only, kw = K): the weights go straight into
// registers like int8 ones, 16 bytes (32 columns) a lane per step, so the k
// order is block b, half h -> columns 32 h + 8 b .. + 7. Each group's products
// accumulate into partial tiles (the first MFMA of a group starts them from
// zero); the partial tiles of group g are scaled by their column's fp16 scale
// and added to the sums during group g + 1's first k16 block, one tile before
// each of its MFMAs, so the scaling overlaps the matrix cores' work instead of
// draining them; the last group is folded after the loop. No rounding beyond
// fp32 accumulation. Built with the MFMA accumulators in AGPRs, the partial
// tiles live there and the sums, which only the fold and the epilogue touch,
// in VGPRs.
// STAMP: the measurement copy (per-workgroup entry / exit times to `stamp`).
// DEPTH: register staging sets (2, or up to 4 for the 2 x 2 layouts with the
// weights staged through LDS): a stage's loads are issued DEPTH - 1 steps
// before its LDS store, for tiles whose k64 step is too short to cover a trip
// to memory (few tiles a CU at M = 256 .. 1024).
template <int BM, int BN, int WMW, int FMT, typename TY, bool STAMP = false, int DEPTH = 2>
__global__ __launch_bounds__(256, 1) void gemm_staged(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, const float* __restrict__ bias, TY* __restrict__ y, int64_t ldy, int M, int N,
    int K, int kw, const uint16_t* __restrict__ scale16, int ngroups, uint64_t* stamp) {
    Stamp<STAMP> clock;
    clock.start();
    static_assert(FMT == kW8 || FMT == kW4 || (FMT == kW4G && WMW == 1),
                  "int8 or reference-layout int4 weights; group-wise int4 in the 1 x 4 layout");
    constexpr bool GROUPED = FMT == kW4G;
    constexpr bool WD = WMW == 1 && (FMT == kW8 || GROUPED);  // weights straight into registers
    static_assert(DEPTH == 2 || (!WD && DEPTH >= 2 && DEPTH <= 4), "deeper staging: LDS-staged weights only");
    constexpr int NT = 256;
    constexpr int WNW = 4 / WMW;
    constexpr int WM = BM / WMW, WN = BN / WNW;
    constexpr int TMm = WM / 32, TNn = WN / 32;
    constexpr int XS = BM * 128, WS = WD ? 0 : BN * 128, STAGE = XS + WS;
    constexpr int XL = BM * 8 / NT, WL = WD ? 0 : BN * 4 / NT, NL = XL + WL;  // staging loads per thread per step
    constexpr int WLD = WD ? (GROUPED ? TNn : 2 * TNn) : 0;                   // direct weight loads per step
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
    constexpr bool PERSIST = NMF * 16 <= 192 && !GROUPED;
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
    u32x4 sx[DEPTH][XL], sw[DEPTH][WL];
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
                uint32_t e0, o0, e1, o1;
                nibbles_x16(v.x, e0, o0);
                nibbles_x16(v.y, e1, o1);
                lo = u32x4{bf16x2_of_x16(e0, o0, 0), bf16x2_of_x16(e0, o0, 1), bf16x2_of_x16(e0, o0, 2),
                           bf16x2_of_x16(e0, o0, 3)};
                hi = u32x4{bf16x2_of_x16(e1, o1, 0), bf16x2_of_x16(e1, o1, 1), bf16x2_of_x16(e1, o1, 2),
                           bf16x2_of_x16(e1, o1, 3)};
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
    for (int kk = 0; kk < 4; ++kk) {
        const int chunk = GROUPED ? 4 * h + kk : 4 * (kk >> 1) + 2 * h + (kk & 1);
        fo[kk] = r * 128 + ((chunk ^ swz8(r)) * 16);
    }
    bf16x8 FW[2][TNn], FX[2][TMm];
    constexpr int FWR = WD ? 0 : TNn;  // weight fragments read from LDS
    auto fread = [&](const uint8_t* base, int kk, int set, int q) {
        if (q < FWR) FW[set][q] = *reinterpret_cast<const bf16x8*>(base + XS + (wn + 32 * q) * 128 + fo[kk]);
        else FX[set][q - FWR] = *reinterpret_cast<const bf16x8*>(base + (wm + 32 * (q - FWR)) * 128 + fo[kk]);
    };
    // WD: lane (r, h) of tile i holds bytes 32 j + 16 h .. + 15 (j = 0, 1) of
    // the step's 64 columns of weight row n_blk + wn + 32 i + r (clamped), in
    // two raw sets; block b widens 8 of them to bf16. Group-wise: bytes
    // 16 h .. + 15 of the step's 32 (columns 32 h .. + 31), dword b for block b.
    u32x4 wr[2][WD ? TNn : 1][2];
    uint32_t wdrow[TNn];
#pragma unroll
    for (int i = 0; i < TNn; ++i) wdrow[i] = (uint32_t)min(n_blk + wn + 32 * i + r, N - 1) * ldw1 + 16 * h;
    auto wload = [&](int k0, int p, int q) {
        if constexpr (GROUPED) {
            wr[p][q][0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(w) + k0 / 2 + wdrow[q]);
        } else if constexpr (WD) {
            const int i = q >> 1, j = q & 1;
            wr[p][i][j] =
                *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(w) + (k0 % kw) + wdrow[i] + 32 * j);
        }
    };
    auto wfrag = [&](int p, int i, int b) {  // group-wise: block b of tile i from raw set p
        const u32x4 v = wr[p][i][0];
        const uint32_t d = b == 0 ? v.x : b == 1 ? v.y : b == 2 ? v.z : v.w;
        uint32_t e, o;
        nibbles_x16(d, e, o);
        const u32x4 t = {bf16x2_of_x16(e, o, 0), bf16x2_of_x16(e, o, 1), bf16x2_of_x16(e, o, 2),
                         bf16x2_of_x16(e, o, 3)};
        return __builtin_bit_cast(bf16x8, t);
    };
    // int8 rows in registers: dword d (bf16 pair d) of block b of tile i,
    // widened from raw set p -- a fragment a dword a bundle, so that no bundle
    // carries more vector-ALU work than its MFMA keeps the matrix core busy
    // (160x256: 6% faster than a whole fragment in one bundle)
    constexpr bool SPREAD = WD && !GROUPED;
    auto wpart = [&](int p, int i, int b, int d) -> uint32_t {
        const u32x4 v = wr[p][i][b >> 1];
        const uint32_t s0 = (b & 1) ? v.z : v.x, s1 = (b & 1) ? v.w : v.y;
        return bf16x2_of_bytes_perm(d < 2 ? s0 : s1, (d & 1) * 16);
    };
    u32x4 FWu[2][SPREAD ? TNn : 1];  // the widened fragments [set][tile] as dwords
    static_assert(!SPREAD || 4 * TNn <= NMF, "a widened dword per bundle");
    // D[n][m] = sum_k w[n][k] x[m][k]: result register q of lane (r, h) holds
    // n = 8 (q / 4) + 4 h + q % 4, m = r of its 32 x 32 tile
    floatx16 acc[TNn][TMm];
    // group-wise: the group's partial tiles, the scales of the 16 columns a
    // lane's result registers hold (fp16 bits as loaded, then fp32 for the
    // fold) and those columns' offsets in the scale array (clamped rows)
    floatx16 part[GROUPED ? TNn : 1][GROUPED ? TMm : 1];
    uint16_t sgr[GROUPED ? TNn : 1][16];
    float scf[GROUPED ? TNn : 1][16];
    uint32_t sbase[GROUPED ? TNn : 1];
    auto mfma_set = [&](int set, int t, bool fresh) {
        const int i = t / TMm, j = t % TMm;
        if constexpr (GROUPED) {
            if (fresh) {
                const floatx16 z = {};
                part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FW[set][i], FX[set][j], z, 0, 0, 0);
            } else {
                part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FW[set][i], FX[set][j], part[i][j], 0, 0, 0);
            }
        } else if constexpr (SPREAD) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, FWu[set][i]), FX[set][j],
                                                                acc[i][j], 0, 0, 0);
        } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(FW[set][i], FX[set][j], acc[i][j], 0, 0, 0);
        }
    };
    // sums += partial tile t x its columns' scales (group-wise)
    auto fold = [&](int t) {
        if constexpr (GROUPED) {
            const int i = t / TMm, j = t % TMm;
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = fmaf(part[i][j][q], scf[i][q], acc[i][j][q]);
        }
    };
    // the scales of group g (requested at its first step, used at the next
    // group's first step) and their conversion
    auto sload = [&](int g) {
        if constexpr (GROUPED) {
#pragma unroll
            for (int i = 0; i < TNn; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    sgr[i][q] = *reinterpret_cast<const uint16_t*>(
                        reinterpret_cast<const char*>(scale16) + 2 * (g + (8 * (q >> 2) + (q & 3)) * ngroups) +
                        sbase[i]);
        }
    };
    auto sconvert = [&]() {
        if constexpr (GROUPED) {
#pragma unroll
            for (int i = 0; i < TNn; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) scf[i][q] = f16_bits_to_f32(sgr[i][q]);
        }
    };

    // split-K (gridDim.z > 1): workgroup z takes k64 steps [z NK / S, (z + 1) NK / S)
    // and writes raw fp32 partial sums (unit scale, no bias) to slice z of y
    const int NK = K / BK;
    int s0 = (int)blockIdx.z * NK / (int)gridDim.z;
    int nk = ((int)blockIdx.z + 1) * NK / (int)gridDim.z - s0;
    if constexpr (GROUPED) {  // whole groups (two steps) a split
        const int G2 = (NK + 1) / 2;
        s0 = 2 * ((int)blockIdx.z * G2 / (int)gridDim.z);
        nk = min(2 * (((int)blockIdx.z + 1) * G2 / (int)gridDim.z), NK) - s0;
    }
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
            // nibble codes enter the MFMAs times 16
            constexpr float unit = FMT == kW8 ? 1.f : 0.0625f;
            sbr[0][c] = (split || GROUPED) ? unit : scale[n] * unit;
            sbr[1][c] = (bias && !split) ? bias[n] : 0.f;
        }
    };
    begin_tile();
    for (;;) {  // the workgroup's tiles
#pragma unroll
    for (int d = 1; d < DEPTH; ++d)
#pragma unroll
        for (int q = 0; q < NL; ++q) gload(kbase + min(d, nk - 1) * BK, d, q);
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
    if constexpr (SPREAD) {
#pragma unroll
        for (int i = 0; i < TNn; ++i)
#pragma unroll
            for (int d = 0; d < 4; ++d) FWu[0][i][d] = wpart(0, i, 0, d);
    } else if constexpr (GROUPED) {
#pragma unroll
        for (int i = 0; i < TNn; ++i) FW[0][i] = wfrag(0, i, 0);
    }
#pragma unroll
    for (int i = 0; i < TNn; ++i)
#pragma unroll
        for (int j = 0; j < TMm; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;
    if constexpr (GROUPED) {
        // result register q of lane (r, h) holds column 8 (q / 4) + 4 h + q % 4
        // of its 32-column tile (N % 32 == 0: a tile's columns are all inside
        // or all outside; an outside one reads the last tile's scales); the
        // first fold adds zero partial tiles
#pragma unroll
        for (int i = 0; i < TNn; ++i) {
            sbase[i] = (uint32_t)(min(n_blk + wn + 32 * i, N - 32) + 4 * h) * (uint32_t)ngroups * 2u;
#pragma unroll
            for (int q = 0; q < 16; ++q) sgr[i][q] = 0;
#pragma unroll
            for (int j = 0; j < TMm; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) part[i][j][q] = 0.f;
        }
    }

    // Step s: MFMAs on buffer s % 2; stage s + 1 (register set (s + 1) % DEPTH)
    // is stored to the other buffer over the first three k16 groups; stage
    // s + DEPTH is loaded into set s % DEPTH over all four. Past the last stage the
    // loads repeat it (clamped k), which keeps the loop body one path. WD:
    // raw weight set p (this step's) is widened one k16 group ahead; by the
    // end of the third group it is free and takes step s + 2's weights in the
    // fourth, whose end widens block 0 of raw set p ^ 1 (step s + 1's).
    // Group-wise, p = 0 is a group's first step: the previous group's scales
    // are converted, this group's requested, and the first k16 block folds
    // the previous partial tiles just before restarting each.
    auto step = [&](int s, int p) {
        uint8_t* cur = smem + (s & 1) * STAGE;
        uint8_t* nxt = smem + ((s + 1) & 1) * STAGE;
        const int k2 = kbase + min(s + DEPTH, nk - 1) * BK;
        if (GROUPED && p == 0) {
            sconvert();
            sload((s0 + s) >> 1);
        }
#pragma unroll
        for (int kk = 0; kk < 3; ++kk) {
            const int set = kk & 1;
#pragma unroll
            for (int t = 0; t < NMF; ++t) {
                const bool fresh = GROUPED && p == 0 && kk == 0;
                if (fresh) fold(t);
                mfma_set(set, t, fresh);
                if constexpr (NRD <= NMF) {
                    if (t < NRD) fread(cur, kk + 1, set ^ 1, t);
                } else {  // more fragments than MFMAs: spread over the bundles
#pragma unroll
                    for (int q = t * NRD / NMF; q < (t + 1) * NRD / NMF; ++q) fread(cur, kk + 1, set ^ 1, q);
                }
                if constexpr (SPREAD) {
                    if (t < 4 * TNn) FWu[set ^ 1][t >> 2][t & 3] = wpart(p, t >> 2, kk + 1, t & 3);
                } else if constexpr (GROUPED) {
                    if (t < TNn) FW[set ^ 1][t] = wfrag(p, t, kk + 1);
                }
                const int b = kk * NMF + t;
                if ((b + 1) * NL / (3 * NMF) > b * NL / (3 * NMF)) lstore(nxt, (p + 1) % DEPTH, b * NL / (3 * NMF));
                if ((b + 1) * NL / (4 * NMF) > b * NL / (4 * NMF)) gload(k2, p, b * NL / (4 * NMF));
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NMF; ++t) {
            mfma_set(1, t, false);
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
            }
            // block 0 of the next step (raw set p ^ 1) into set 0, which this
            // group's MFMAs do not read
            if constexpr (SPREAD) {
                if (t < 4 * TNn) FWu[0][t >> 2][t & 3] = wpart(p ^ 1, t >> 2, 0, t & 3);
            } else if constexpr (GROUPED) {
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
    for (; s + DEPTH - 1 < nk; s += DEPTH) {
        step(s, 0);
        step(s + 1, 1);
        if constexpr (DEPTH > 2) step(s + 2, 2);
        if constexpr (DEPTH > 3) step(s + 3, 3);
    }
    if (s < nk) step(s, 0);
    if constexpr (DEPTH > 2) {
        if (s + 1 < nk) step(s + 1, 1);
    }
    if constexpr (DEPTH > 3) {
        if (s + 2 < nk) step(s + 2, 2);
    }
    if constexpr (GROUPED) {  // the last group's partial tiles
        sconvert();
#pragma unroll
        for (int t = 0; t < NMF; ++t) fold(t);
    }
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
    if constexpr (STAMP) __syncthreads();  // every wavefront's stores issued
    clock.finish(stamp, (int64_t)blockIdx.z * gridDim.x + blockIdx.x);
}

// The kernel's PERSIST condition, on the host: tiles whose accumulators leave
// room for the next tile's first loads run on a persistent grid of one
// workgroup per tile slot (256 CUs x the workgroups a CU holds).
template <int BM, int BN, int WMW>
constexpr bool staged_persist() {
    return (BM / WMW / 32) * (BN * WMW / 4 / 32) * 16 <= 192;
}

