// Weight quantize / pack / dequantize kernels (gfx950).
//
// Replaces the torch op chain of the reference's quantize_tensor
// (src/transformer_internals/quantization.py:78-116):
//   abs -> amax -> div -> clamp -> div -> round -> clamp -> to(int8)
// with one pass over HBM: each row is read once into registers, its |max| is
// reduced across the row's wavefronts, and the codes are written from the same
// registers. Codes and scales are bit-identical to the reference: an unsigned
// max on |w| bits (order-free, NaN-propagating), the correctly rounded fp32
// scale divide, codes rint(w / s) (half to even) with the same clamps, where
// the row kernels form w / s as a product with the reciprocal and take the
// division itself wherever the two could round differently (codes4).
//
// Memory: per-channel int8 reads 4*rows*cols bytes and writes rows*cols + 4*rows.
#include "tiq_common.hpp"

namespace tiq {
namespace {

// ------------------------------------------------------------- helpers
// max over each 16-lane row of the wavefront, in every lane of the row
// (DPP moves: pairs, quads, half rows, rows). All 64 lanes must be active.
__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x, uint32_t keep) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)keep, (int)x, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    v = umax(v, dpp_u32<0xB1>(v, 0u));   // quad_perm [1, 0, 3, 2]
    v = umax(v, dpp_u32<0x4E>(v, 0u));   // quad_perm [2, 3, 0, 1]
    v = umax(v, dpp_u32<0x141>(v, 0u));  // row_half_mirror
    v = umax(v, dpp_u32<0x140>(v, 0u));  // row_mirror
    return v;
}
// max over lanes 0-31 in lane 31 and over lanes 32-63 in lane 63
// (row_bcast:15 adds row 0 into row 1 and row 2 into row 3).
__device__ __forceinline__ uint32_t half_max_u32(uint32_t v) {
    v = row16_max_u32(v);
    return umax(v, dpp_u32<0x142, 0xa>(v, v));
}
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
    v = half_max_u32(v);
    v = umax(v, dpp_u32<0x143, 0xc>(v, v));  // row_bcast:31 into rows 2 and 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// v_cvt_i32_f32: round-toward-zero conversion that saturates out-of-range
// values and maps NaN to 0 (defined for every input, unlike a C++ cast).
__device__ __forceinline__ int cvt_i32_sat(float f) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
    return r;
}

// A row as a buffer resource of `bytes` bytes: 16-byte loads past it return
// zeros and make no memory access, so every load of a row is issued without a
// bounds branch (a branch per load makes the compiler wait for each load
// before the next is issued).
typedef float tiq_qf32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ float4 row_load(__amdgpu_buffer_rsrc_t r, int byte_off) {
    const tiq_qf32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    return make_float4(v.x, v.y, v.z, v.w);
}

// Codes of four values, clamp(rint(w / s), qmin, qmax) with w / s the
// correctly rounded quotient, computed as rint(w * inv), inv = 1 / s
// correctly rounded. For |w / s| <= 130 the exact product w * inv is within
// 130 * 2^-23 < 2^-15.9 of the rounded quotient and its own rounding within
// 2^-17, so the rounded product and the quotient round to the same integer
// unless w * inv lies within 2^-14 of a half-integer. Beyond 130 a wrong
// neighbour would still clamp to the same end (qmax <= 127, qmin >= -128),
// and past 2^23 both are the same integer. Only groups of four with a value
// near a half-integer (about one in 2000) take the exact division, so the
// codes equal the per-element division's. Infinite and NaN products give
// the quotient's codes through the saturating conversion (inf -> the clamp
// end, NaN -> 0), whichever branch they take.
__device__ __forceinline__ void codes4(const float4& v, float s, float inv, int qmin, int qmax, int (&c)[4]) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    float t[4], e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        t[k] = __builtin_rintf(x[k] * inv);
        e[k] = fabsf(fabsf(__builtin_fmaf(x[k], inv, -t[k])) - 0.5f);  // exact w*inv - t, rounded once
    }
    const float emin = fminf(fminf(e[0], e[1]), fminf(e[2], e[3]));
    if (!(emin > 0x1p-14f)) {
        asm volatile("");  // a real branch: the divisions run only in waves that need them
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] = __builtin_rintf(x[k] / s);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = max(cvt_i32_sat(t[k]), qmin);
        c[k] = min(q, qmax);
    }
}

// ----------------------------------------------------------- per-channel
// WPR wavefronts per row, 4 / WPR rows per 256-thread workgroup; the row held
// in registers as V float4 per lane (float4 index (sub*64 + lane) + 64*WPR*i
// for wavefront `sub` of the row), so each load instruction reads 1 KB of
// consecutive memory. |max| per wavefront with DPP moves, across the row's
// wavefronts through LDS. Needs cols % 4 == 0 and 16-byte aligned rows.
// Out = int8 codes (PACK == false, 4 codes per 32-bit store) or the
// reference's nibble packing (PACK == true, 2 bytes per float4).
template <int V, int WPR, bool PACK>
__global__ __launch_bounds__(256) void quant_rows_vec(const float* __restrict__ w, int64_t rows,
                                                      int cols, int64_t ldw, float qmin, float qmax,
                                                      uint8_t* __restrict__ out, int64_t ldq,
                                                      float* __restrict__ scale) {
    constexpr int kRows = 4 / WPR;
    __shared__ uint32_t red[4];
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x >> 6, sub = wv % WPR;
    const int64_t row = (int64_t)blockIdx.x * kRows + wv / WPR;
    const bool valid = row < rows;  // wave-uniform; no early return before the barrier
    const __amdgpu_buffer_rsrc_t wr = row_rsrc(w + (valid ? row : 0) * ldw, valid ? cols * 4 : 0);
    const int nv = valid ? cols >> 2 : 0;
    float4 v[V];
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = row_load(wr, (sub * kWave + lane + kWave * WPR * i) * 16);
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const uint32_t a = abs_bits(v[i].x), b = abs_bits(v[i].y), c = abs_bits(v[i].z), d = abs_bits(v[i].w);
        m = umax(m, umax(umax(a, b), umax(c, d)));
    }
    m = wave_max_u32_dpp(m);
    if (WPR > 1) {
        if (lane == 0) red[wv] = m;
        __syncthreads();
        m = red[wv - sub];
#pragma unroll
        for (int j = 1; j < WPR; ++j) m = umax(m, red[wv - sub + j]);
    }
    const float s = scale_from_amax(__uint_as_float(m), qmax);
    const float inv = 1.0f / s;
    if (valid && sub == 0 && lane == 0) scale[row] = s;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int idx = sub * kWave + lane + kWave * WPR * i;
        if (idx < nv) {
            int c[4];
            codes4(v[i], s, inv, (int)qmin, (int)qmax, c);
            if (PACK) {
                const uint16_t b = (uint16_t)(((c[0] + 8) & 0xf) | (((c[1] + 8) & 0xf) << 4) |
                                              (((c[2] + 8) & 0xf) << 8) | (((c[3] + 8) & 0xf) << 12));
                reinterpret_cast<uint16_t*>(out + row * (int64_t)(cols >> 1))[idx] = b;
            } else {
                const uint32_t b = (uint32_t)(c[0] & 0xff) | ((uint32_t)(c[1] & 0xff) << 8) |
                                   ((uint32_t)(c[2] & 0xff) << 16) | ((uint32_t)(c[3] & 0xff) << 24);
                reinterpret_cast<uint32_t*>(out + row * ldq)[idx] = b;
            }
        }
    }
}

// Wavefronts per row for a row of nv float4: the fewest that keep at most 8
// float4 per lane (32 with 4 wavefronts) and give at least 4096 wavefronts
// (4 per SIMD), else the most that fit; 0 when none fits.
int rows_split(int64_t rows, int64_t nv, int* per_lane) {
    int best = 0;
    for (int wpr = 1; wpr <= 4; wpr *= 2) {
        const int64_t pl = (nv + 64 * wpr - 1) / (64 * wpr);
        if (pl > (wpr == 4 ? 32 : 8)) continue;
        best = wpr;
        *per_lane = (int)pl;
        if (rows * wpr >= 4096) break;
    }
    return best;
}

// Any shape / alignment: one workgroup per row, two passes over the row
// (the second pass hits L2). PACK writes the reference nibble layout for an
// even number of columns.
template <bool PACK>
__global__ __launch_bounds__(256) void quant_rows_generic(const float* __restrict__ w, int64_t rows,
                                                          int64_t cols, int64_t ldw, float qmin,
                                                          float qmax, uint8_t* __restrict__ out,
                                                          int64_t ldq, float* __restrict__ scale) {
    __shared__ uint32_t red[256 / kWave];
    const int64_t row = blockIdx.x;
    const float* wr = w + row * ldw;
    uint32_t m = 0;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        uint32_t a = abs_bits(wr[c]);
        m = a > m ? a : m;
    }
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) m = red[i] > m ? red[i] : m;
    const float s = scale_from_amax(__uint_as_float(m), qmax);
    if (threadIdx.x == 0) scale[row] = s;
    if (PACK) {
        uint8_t* orow = out + row * (cols >> 1);
        for (int64_t j = threadIdx.x; j < (cols >> 1); j += blockDim.x) {
            const int lo = code_of(wr[2 * j], s, qmin, qmax) + 8;
            const int hi = code_of(wr[2 * j + 1], s, qmin, qmax) + 8;
            orow[j] = (uint8_t)((lo & 0xf) | ((hi & 0xf) << 4));
        }
    } else {
        int8_t* orow = reinterpret_cast<int8_t*>(out + row * ldq);
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) orow[c] = (int8_t)code_of(wr[c], s, qmin, qmax);
    }
}

int launch_quant_rows(const float* w, int64_t rows, int64_t cols, int64_t ldw, int bits, uint8_t* out,
                      int64_t ldq, float* scale, bool pack, hipStream_t st) {
    const float qmax = (float)((1 << (bits - 1)) - 1), qmin = (float)(-(1 << (bits - 1)));
    const int64_t nv = cols / 4;
    int per_lane = 0;
    const int wpr = rows_split(rows, nv, &per_lane);
    const bool vec = (cols % 4 == 0) && (ldw % 4 == 0) && aligned(w, 16) &&
                     (pack || ((ldq % 4 == 0) && aligned(out, 4))) && (!pack || aligned(out, 2)) && wpr > 0;
    if (!vec) {
        if (pack) hipLaunchKernelGGL(quant_rows_generic<true>, dim3((unsigned)rows), dim3(256), 0, st, w, rows, cols, ldw, qmin, qmax, out, ldq, scale);
        else hipLaunchKernelGGL(quant_rows_generic<false>, dim3((unsigned)rows), dim3(256), 0, st, w, rows, cols, ldw, qmin, qmax, out, ldq, scale);
        return launch_status();
    }
    const int rpb = 4 / wpr;
    const dim3 grid((unsigned)((rows + rpb - 1) / rpb)), block(256);
    const int c = (int)cols;
#define TIQ_QR(V, W)                                                                                              \
    if (wpr == W && per_lane <= V) {                                                                              \
        if (pack) hipLaunchKernelGGL((quant_rows_vec<V, W, true>), grid, block, 0, st, w, rows, c, ldw, qmin, qmax, out, ldq, scale); \
        else hipLaunchKernelGGL((quant_rows_vec<V, W, false>), grid, block, 0, st, w, rows, c, ldw, qmin, qmax, out, ldq, scale);    \
        return launch_status();                                                                                   \
    }
    TIQ_QR(1, 1) TIQ_QR(2, 1) TIQ_QR(4, 1) TIQ_QR(8, 1)
    TIQ_QR(1, 2) TIQ_QR(2, 2) TIQ_QR(4, 2) TIQ_QR(8, 2)
    TIQ_QR(1, 4) TIQ_QR(2, 4) TIQ_QR(4, 4) TIQ_QR(8, 4) TIQ_QR(16, 4) TIQ_QR(32, 4)
#undef TIQ_QR
    return TIQ_EUNSUPPORTED;
}

// ------------------------------------------------------------ per-tensor
// Phase 1: per-workgroup |max| bits into workspace[blockIdx.x].
__global__ __launch_bounds__(256) void amax_partial(const float* __restrict__ w, int64_t n, bool vec,
                                                    uint32_t* __restrict__ partial) {
    __shared__ uint32_t red[4];
    uint32_t m = 0;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t tail = 0;
    if (vec) {
        const float4* w4 = reinterpret_cast<const float4*>(w);
        const int64_t n4 = n >> 2;
        for (int64_t i = tid; i < n4; i += stride) {
            const float4 v = w4[i];
            uint32_t a = abs_bits(v.x), b = abs_bits(v.y), c = abs_bits(v.z), d = abs_bits(v.w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            a = a > c ? a : c;
            m = a > m ? a : m;
        }
        tail = n4 << 2;
    }
    for (int64_t i = tail + tid; i < n; i += stride) {
        const uint32_t a = abs_bits(w[i]);
        m = a > m ? a : m;
    }
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = red[0];
        for (int i = 1; i < 4; ++i) r = red[i] > r ? red[i] : r;
        partial[blockIdx.x] = r;
    }
}

// Phase 2: every workgroup reduces the partials, derives the scale and codes
// its slice.
__global__ __launch_bounds__(256) void quant_flat(const float* __restrict__ w, int64_t n, bool vec,
                                                  const uint32_t* __restrict__ partial, int nparts,
                                                  float qmin, float qmax, int8_t* __restrict__ q,
                                                  float* __restrict__ scale) {
    __shared__ uint32_t red[4];
    uint32_t m = 0;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = partial[i] > m ? partial[i] : m;
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int i = 1; i < 4; ++i) m = red[i] > m ? red[i] : m;
    const float s = scale_from_amax(__uint_as_float(m), qmax);
    if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = s;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t tail = 0;
    if (vec) {
        const float4* w4 = reinterpret_cast<const float4*>(w);
        uint32_t* q4 = reinterpret_cast<uint32_t*>(q);
        const int64_t n4 = n >> 2;
        for (int64_t i = tid; i < n4; i += stride) {
            const float4 v = w4[i];
            const int c0 = code_of(v.x, s, qmin, qmax), c1 = code_of(v.y, s, qmin, qmax);
            const int c2 = code_of(v.z, s, qmin, qmax), c3 = code_of(v.w, s, qmin, qmax);
            q4[i] = (uint32_t)(c0 & 0xff) | ((uint32_t)(c1 & 0xff) << 8) | ((uint32_t)(c2 & 0xff) << 16) |
                    ((uint32_t)(c3 & 0xff) << 24);
        }
        tail = n4 << 2;
    }
    for (int64_t i = tail + tid; i < n; i += stride) q[i] = (int8_t)code_of(w[i], s, qmin, qmax);
}

constexpr int kMaxPartials = 1024;

int partial_blocks(int64_t n) {
    int64_t b = (n + 256 * 16 - 1) / (256 * 16);
    if (b < 1) b = 1;
    if (b > kMaxPartials) b = kMaxPartials;
    return (int)b;
}

// ----------------------------------------------------------- group-wise
// Group-wise int4, group 128, over the flattened (row, group) space: eight
// lanes per group, a wavefront takes 8 * U consecutive groups (U rounds of 8,
// in the same or the next rows). Lane 8 * lg + sl of round u holds float4
// sl + 8 j (j < 4) of group 8 u + lg, so each load instruction reads whole
// 128-byte lines; the group max is a DPP reduction over 8 lanes and the
// scale (two divisions) is computed once per 16 values of a lane. The
// weight is one buffer resource: loads past a group's end (a ragged last
// group) or past the last row go to an offset beyond it and return zeros.
template <int U>
__global__ __launch_bounds__(256) void quant_g128_groups(const float* __restrict__ w, int rows, int cols, int ng,
                                                         uint8_t* __restrict__ packed,
                                                         uint16_t* __restrict__ scale16) {
    const int lane = threadIdx.x & (kWave - 1), sl = lane & 7, lg = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
    const uint32_t gid0 = (uint32_t)wave * 8u * U;  // rows * ng + 64 < 2^31 (checked by the launcher)
    const int r0 = (int)(gid0 / (uint32_t)ng), g0 = (int)(gid0 % (uint32_t)ng);
    const __amdgpu_buffer_rsrc_t wr = row_rsrc(w, rows * cols * 4);
    int r[U], g[U], nq[U];
    uint32_t base[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {  // every group's place first, so all loads issue together
        int gg = g0 + 8 * u + lg, rr = r0;
        while (gg >= ng) {
            gg -= ng;
            ++rr;
        }
        r[u] = rr;
        g[u] = gg;
        nq[u] = rr < rows ? min(32, (cols - gg * 128) >> 2) : 0;  // float4 in the group
        base[u] = ((uint32_t)rr * (uint32_t)cols + (uint32_t)gg * 128u) * 4u;
    }
    float4 v[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int f = sl + 8 * j;
            v[u][j] = row_load(wr, (int)(f < nq[u] ? base[u] + (uint32_t)f * 16u : 0x7ffffff0u));
        }
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first wait
#pragma unroll
    for (int u = 0; u < U; ++u) {
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            m = umax(m, umax(umax(abs_bits(v[u][j].x), abs_bits(v[u][j].y)),
                             umax(abs_bits(v[u][j].z), abs_bits(v[u][j].w))));
        m = umax(m, dpp_u32<0xB1>(m, 0u));   // quad_perm [1, 0, 3, 2]
        m = umax(m, dpp_u32<0x4E>(m, 0u));   // quad_perm [2, 3, 0, 1]
        m = umax(m, dpp_u32<0x141>(m, 0u));  // row_half_mirror: the 8 lanes of the group
        uint16_t h = f32_to_f16_bits(__uint_as_float(m) / 7.0f);
        if (h == 0) h = 1;
        if (h > 0x7bffu) h = 0x7bffu;
        const float s = f16_bits_to_f32(h);
        const float inv = 1.0f / s;
        if (nq[u] > 0) {
            if (sl == 0) scale16[(int64_t)r[u] * ng + g[u]] = h;
            uint16_t* pg = reinterpret_cast<uint16_t*>(packed + (int64_t)r[u] * (cols >> 1) + g[u] * 64);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int f = sl + 8 * j;
                if (f < nq[u]) {
                    int c[4];
                    codes4(v[u][j], s, inv, -8, 7, c);
                    pg[f] = (uint16_t)((c[0] + 8) | ((c[1] + 8) << 4) | ((c[2] + 8) << 8) | ((c[3] + 8) << 12));
                }
            }
        }
    }
}

// Any group / shape: one thread per (row, group).
__global__ __launch_bounds__(256) void quant_groups_generic(const float* __restrict__ w, int64_t rows,
                                                            int64_t cols, int group,
                                                            uint8_t* __restrict__ packed,
                                                            uint16_t* __restrict__ scale16) {
    const int64_t ngroups = (cols + group - 1) / group;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * ngroups) return;
    const int64_t row = t / ngroups, g = t % ngroups;
    const int64_t c0 = g * group, c1 = (c0 + group < cols) ? c0 + group : cols;
    const float* wr = w + row * cols;
    uint32_t m = 0;
    for (int64_t c = c0; c < c1; ++c) {
        const uint32_t a = abs_bits(wr[c]);
        m = a > m ? a : m;
    }
    uint16_t h = f32_to_f16_bits(__uint_as_float(m) / 7.0f);
    if (h == 0) h = 1;
    if (h > 0x7bffu) h = 0x7bffu;
    scale16[t] = h;
    const float s = f16_bits_to_f32(h);
    uint8_t* prow = packed + row * ((cols + 1) / 2);
    // group is even, so a group owns whole bytes except a ragged odd tail.
    for (int64_t c = c0; c < c1; c += 2) {
        const int lo = code_of(wr[c], s, -8.f, 7.f) + 8;
        const int hi = (c + 1 < c1) ? code_of(wr[c + 1], s, -8.f, 7.f) + 8 : 0;
        prow[c / 2] = (uint8_t)(lo | (hi << 4));
    }
}

// ------------------------------------------------------------ pack/unpack
__global__ __launch_bounds__(256) void pack_int4_kernel(const int8_t* __restrict__ q, int64_t numel,
                                                        uint8_t* __restrict__ packed) {
    const int64_t nbytes = (numel + 1) / 2;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < nbytes;
         j += (int64_t)gridDim.x * blockDim.x) {
        const int lo = q[2 * j] + 8;
        const int hi = (2 * j + 1 < numel) ? q[2 * j + 1] + 8 : 0;
        packed[j] = (uint8_t)(((hi << 4) | lo) & 0xff);
    }
}

__global__ __launch_bounds__(256) void unpack_int4_kernel(const uint8_t* __restrict__ packed, int64_t numel,
                                                          int8_t* __restrict__ q) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t b = packed[i >> 1];
        q[i] = (int8_t)(((i & 1) ? (b >> 4) : (b & 0xf)) - 8);
    }
}

// ------------------------------------------------------------ dequantize
__global__ __launch_bounds__(256) void dequant_int8_kernel(const int8_t* __restrict__ q,
                                                           const float* __restrict__ scale, int per_channel,
                                                           int64_t rows, int64_t cols, float* __restrict__ out) {
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (float)q[i] * scale[per_channel ? i / cols : 0];
}

__global__ __launch_bounds__(256) void dequant_int4_kernel(const uint8_t* __restrict__ packed,
                                                           const float* __restrict__ scale, int per_channel,
                                                           int64_t rows, int64_t cols, float* __restrict__ out) {
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t b = packed[i >> 1];
        const int code = ((i & 1) ? (b >> 4) : (b & 0xf)) - 8;
        out[i] = (float)code * scale[per_channel ? i / cols : 0];
    }
}

__global__ __launch_bounds__(256) void dequant_g4_kernel(const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scale16, int group,
                                                         int64_t rows, int64_t cols, float* __restrict__ out) {
    const int64_t n = rows * cols;
    const int64_t stride = (cols + 1) / 2, ngroups = (cols + group - 1) / group;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / cols, c = i % cols;
        const uint8_t b = packed[r * stride + (c >> 1)];
        const int code = ((c & 1) ? (b >> 4) : (b & 0xf)) - 8;
        out[i] = (float)code * f16_bits_to_f32(scale16[r * ngroups + c / group]);
    }
}

unsigned elementwise_grid(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace
}  // namespace tiq

using namespace tiq;

extern "C" int tiq_quantize_per_channel(const float* w, int64_t rows, int64_t cols, int64_t ldw, int bits,
                                        int8_t* q, int64_t ldq, float* scale, void* stream) {
    if (bits < 2 || bits > 8) return TIQ_EBITS;
    if (rows < 0 || cols < 0 || ldw < cols || ldq < cols) return TIQ_EINVAL;
    if (rows == 0) return TIQ_OK;
    if (!w || !q || !scale || cols == 0) return TIQ_EINVAL;
    if (rows > 0x7fffffffLL) return TIQ_EUNSUPPORTED;
    return launch_quant_rows(w, rows, cols, ldw, bits, reinterpret_cast<uint8_t*>(q), ldq, scale, false,
                             as_stream(stream));
}

extern "C" size_t tiq_quantize_per_tensor_workspace(int64_t numel) {
    return (size_t)partial_blocks(numel < 0 ? 0 : numel) * sizeof(uint32_t);
}

extern "C" int tiq_quantize_per_tensor(const float* w, int64_t numel, int bits, int8_t* q, float* scale,
                                       void* workspace, size_t workspace_bytes, void* stream) {
    if (bits < 2 || bits > 8) return TIQ_EBITS;
    if (numel <= 0 || !w || !q || !scale || !workspace) return TIQ_EINVAL;
    const int parts = partial_blocks(numel);
    if (workspace_bytes < (size_t)parts * sizeof(uint32_t)) return TIQ_EWORKSPACE;
    if (!aligned(workspace, 4)) return TIQ_EALIGN;
    const float qmax = (float)((1 << (bits - 1)) - 1), qmin = (float)(-(1 << (bits - 1)));
    const bool vec = aligned(w, 16) && aligned(q, 4);
    hipStream_t st = as_stream(stream);
    uint32_t* part = reinterpret_cast<uint32_t*>(workspace);
    hipLaunchKernelGGL(amax_partial, dim3(parts), dim3(256), 0, st, w, numel, vec, part);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(quant_flat, dim3(parts), dim3(256), 0, st, w, numel, vec, part, parts, qmin, qmax, q, scale);
    return launch_status();
}

extern "C" int tiq_pack_int4(const int8_t* q, int64_t numel, uint8_t* packed, void* stream) {
    if (numel < 0) return TIQ_EINVAL;
    if (numel == 0) return TIQ_OK;
    if (!q || !packed) return TIQ_EINVAL;
    hipLaunchKernelGGL(pack_int4_kernel, dim3(elementwise_grid((numel + 1) / 2)), dim3(256), 0, as_stream(stream),
                       q, numel, packed);
    return launch_status();
}

extern "C" int tiq_unpack_int4(const uint8_t* packed, int64_t numel, int8_t* q, void* stream) {
    if (numel < 0) return TIQ_EINVAL;
    if (numel == 0) return TIQ_OK;
    if (!q || !packed) return TIQ_EINVAL;
    hipLaunchKernelGGL(unpack_int4_kernel, dim3(elementwise_grid(numel)), dim3(256), 0, as_stream(stream), packed,
                       numel, q);
    return launch_status();
}

extern "C" int tiq_quantize_per_channel_int4_packed(const float* w, int64_t rows, int64_t cols, int bits,
                                                    uint8_t* packed, float* scale, void* stream) {
    if (bits < 2 || bits > 8) return TIQ_EBITS;
    if (bits > 4) return TIQ_EINVAL;
    if (rows < 0 || cols <= 0) return TIQ_EINVAL;
    if (rows == 0) return TIQ_OK;
    if (cols % 2) return TIQ_EUNSUPPORTED;
    if (!w || !packed || !scale) return TIQ_EINVAL;
    if (rows > 0x7fffffffLL) return TIQ_EUNSUPPORTED;
    return launch_quant_rows(w, rows, cols, cols, bits, packed, cols / 2, scale, true, as_stream(stream));
}

extern "C" int tiq_quantize_groupwise_int4(const float* w, int64_t rows, int64_t cols, int group,
                                           uint8_t* packed, uint16_t* scale_f16, void* stream) {
    if (group < 2 || (group & 1)) return TIQ_EINVAL;
    if (rows < 0 || cols <= 0) return TIQ_EINVAL;
    if (rows == 0) return TIQ_OK;
    if (!w || !packed || !scale_f16) return TIQ_EINVAL;
    hipStream_t st = as_stream(stream);
    const int64_t ng = (cols + 127) / 128;
    if (group == 128 && cols % 4 == 0 && aligned(w, 16) && aligned(packed, 2) &&
        (rows + 16) * cols * 4 < 0x7ffffff0LL) {
        const int64_t G = rows * ng;
        const int u = G >= 2048 * 16 ? 2 : 1;
        const int64_t waves = (G + 8 * u - 1) / (8 * u);
        const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
        if (u == 2)
            hipLaunchKernelGGL(quant_g128_groups<2>, grid, block, 0, st, w, (int)rows, (int)cols, (int)ng, packed, scale_f16);
        else
            hipLaunchKernelGGL(quant_g128_groups<1>, grid, block, 0, st, w, (int)rows, (int)cols, (int)ng, packed, scale_f16);
        return launch_status();
    }
    const int64_t ngroups = (cols + group - 1) / group;
    const int64_t threads = rows * ngroups;
    hipLaunchKernelGGL(quant_groups_generic, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, w, rows,
                       cols, group, packed, scale_f16);
    return launch_status();
}

extern "C" int tiq_dequantize_int8(const int8_t* q, const float* scale, int per_channel, int64_t rows, int64_t cols,
                                   float* w_hat, void* stream) {
    if (rows < 0 || cols < 0) return TIQ_EINVAL;
    if (rows * cols == 0) return TIQ_OK;
    if (!q || !scale || !w_hat) return TIQ_EINVAL;
    hipLaunchKernelGGL(dequant_int8_kernel, dim3(elementwise_grid(rows * cols)), dim3(256), 0, as_stream(stream), q,
                       scale, per_channel, rows, cols, w_hat);
    return launch_status();
}

extern "C" int tiq_dequantize_int4(const uint8_t* packed, const float* scale, int per_channel, int64_t rows,
                                   int64_t cols, float* w_hat, void* stream) {
    if (rows < 0 || cols < 0) return TIQ_EINVAL;
    if (rows * cols == 0) return TIQ_OK;
    if (!packed || !scale || !w_hat) return TIQ_EINVAL;
    hipLaunchKernelGGL(dequant_int4_kernel, dim3(elementwise_grid(rows * cols)), dim3(256), 0, as_stream(stream),
                       packed, scale, per_channel, rows, cols, w_hat);
    return launch_status();
}

extern "C" int tiq_dequantize_groupwise_int4(const uint8_t* packed, const uint16_t* scale_f16, int group,
                                             int64_t rows, int64_t cols, float* w_hat, void* stream) {
    if (group < 2 || (group & 1) || rows < 0 || cols < 0) return TIQ_EINVAL;
    if (rows * cols == 0) return TIQ_OK;
    if (!packed || !scale_f16 || !w_hat) return TIQ_EINVAL;
    hipLaunchKernelGGL(dequant_g4_kernel, dim3(elementwise_grid(rows * cols)), dim3(256), 0, as_stream(stream),
                       packed, scale_f16, group, rows, cols, w_hat);
    return launch_status();
}
