// Weight quantize / pack / dequantize kernels (gfx950).
//
// Replaces the torch op chain of the reference's quantize_tensor
// (src/transformer_internals/quantization.py:78-116):
//   abs -> amax -> div -> clamp -> div -> round -> clamp -> to(int8)
// with one pass over HBM: each row is read once into registers, its |max| is
// reduced across the wavefront, and the codes are written from the same
// registers. Codes and scales are bit-identical to the reference because every
// step is the same IEEE operation: an unsigned max on |w| bits (order-free,
// NaN-propagating), the correctly rounded fp32 divide, rint (half to even)
// and the same clamps.
//
// Memory: per-channel int8 reads 4*rows*cols bytes and writes rows*cols + 4*rows.
#include "tiq_common.hpp"

namespace tiq {
namespace {

constexpr int kRowsPerBlock = 4;  // one wavefront per row, four per workgroup

// ----------------------------------------------------------- per-channel
// One wavefront per row, the row held in registers as VPL float4 per lane
// (columns lane*4 + 256*i). Needs cols % 4 == 0 and 16-byte aligned rows.
// Out = int8 codes (PACK == false, 4 codes per 32-bit store) or the
// reference's nibble packing (PACK == true, 2 bytes per float4).
template <int VPL, bool PACK>
__global__ __launch_bounds__(256) void quant_rows_vec(const float* __restrict__ w, int64_t rows,
                                                      int cols, int64_t ldw, float qmin, float qmax,
                                                      uint8_t* __restrict__ out, int64_t ldq,
                                                      float* __restrict__ scale) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float4* wr = reinterpret_cast<const float4*>(w + row * ldw);
    const int nv = cols >> 2;
    float4 v[VPL];
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int idx = lane + kWave * i;
        if (idx < nv) {
            v[i] = wr[idx];
            uint32_t a = abs_bits(v[i].x), b = abs_bits(v[i].y), c = abs_bits(v[i].z), d = abs_bits(v[i].w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            a = a > c ? a : c;
            m = a > m ? a : m;
        }
    }
    m = wave_max_u32(m);
    const float s = scale_from_amax(__uint_as_float(m), qmax);
    if (lane == 0) scale[row] = s;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int idx = lane + kWave * i;
        if (idx < nv) {
            const int c0 = code_of(v[i].x, s, qmin, qmax), c1 = code_of(v[i].y, s, qmin, qmax);
            const int c2 = code_of(v[i].z, s, qmin, qmax), c3 = code_of(v[i].w, s, qmin, qmax);
            if (PACK) {
                const uint16_t b = (uint16_t)(((c0 + 8) & 0xf) | (((c1 + 8) & 0xf) << 4) |
                                              (((c2 + 8) & 0xf) << 8) | (((c3 + 8) & 0xf) << 12));
                reinterpret_cast<uint16_t*>(out + row * (int64_t)(cols >> 1))[idx] = b;
            } else {
                const uint32_t b = (uint32_t)(c0 & 0xff) | ((uint32_t)(c1 & 0xff) << 8) |
                                   ((uint32_t)(c2 & 0xff) << 16) | ((uint32_t)(c3 & 0xff) << 24);
                reinterpret_cast<uint32_t*>(out + row * ldq)[idx] = b;
            }
        }
    }
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
    const bool vec = (cols % 4 == 0) && (ldw % 4 == 0) && aligned(w, 16) &&
                     (pack || ((ldq % 4 == 0) && aligned(out, 4))) && (!pack || aligned(out, 2)) &&
                     cols <= 64 * 4 * 32;
    if (!vec) {
        if (pack) hipLaunchKernelGGL(quant_rows_generic<true>, dim3((unsigned)rows), dim3(256), 0, st, w, rows, cols, ldw, qmin, qmax, out, ldq, scale);
        else hipLaunchKernelGGL(quant_rows_generic<false>, dim3((unsigned)rows), dim3(256), 0, st, w, rows, cols, ldw, qmin, qmax, out, ldq, scale);
        return launch_status();
    }
    const int nv = (int)(cols / 4);
    const int per_lane = (nv + kWave - 1) / kWave;
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)), block(256);
    const int c = (int)cols;
#define TIQ_QR(V)                                                                                             \
    if (per_lane <= V) {                                                                                      \
        if (pack) hipLaunchKernelGGL((quant_rows_vec<V, true>), grid, block, 0, st, w, rows, c, ldw, qmin, qmax, out, ldq, scale); \
        else hipLaunchKernelGGL((quant_rows_vec<V, false>), grid, block, 0, st, w, rows, c, ldw, qmin, qmax, out, ldq, scale);    \
        return launch_status();                                                                               \
    }
    TIQ_QR(1) TIQ_QR(2) TIQ_QR(4) TIQ_QR(8) TIQ_QR(16) TIQ_QR(32)
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
// Group-wise int4, group 128, one wavefront per row: a group is 32 float4,
// i.e. one half of the wavefront in iteration i (lanes 0-31: group 2i,
// lanes 32-63: group 2i+1), so the group max is a half-wave reduction.
template <int VPL>
__global__ __launch_bounds__(256) void quant_g128_vec(const float* __restrict__ w, int64_t rows, int cols,
                                                      uint8_t* __restrict__ packed,
                                                      uint16_t* __restrict__ scale16) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float4* wr = reinterpret_cast<const float4*>(w + row * (int64_t)cols);
    const int nv = cols >> 2;
    const int ngroups = (cols + 127) >> 7;
    uint16_t* prow = reinterpret_cast<uint16_t*>(packed + row * (int64_t)(cols >> 1));
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int idx = lane + kWave * i;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        uint32_t m = 0;
        if (idx < nv) {
            v = wr[idx];
            uint32_t a = abs_bits(v.x), b = abs_bits(v.y), c = abs_bits(v.z), d = abs_bits(v.w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            m = a > c ? a : c;
        }
        m = group_max_u32<32>(m);
        uint16_t h = f32_to_f16_bits(__uint_as_float(m) / 7.0f);
        if (h == 0) h = 1;
        if (h > 0x7bffu) h = 0x7bffu;
        const float s = f16_bits_to_f32(h);
        if (idx < nv) {
            if ((idx & 31) == 0) scale16[row * ngroups + (idx >> 5)] = h;
            const int c0 = code_of(v.x, s, -8.f, 7.f) + 8, c1 = code_of(v.y, s, -8.f, 7.f) + 8;
            const int c2 = code_of(v.z, s, -8.f, 7.f) + 8, c3 = code_of(v.w, s, -8.f, 7.f) + 8;
            prow[idx] = (uint16_t)(c0 | (c1 << 4) | (c2 << 8) | (c3 << 12));
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
    const int64_t nv = cols / 4;
    if (group == 128 && cols % 4 == 0 && aligned(w, 16) && aligned(packed, 2) && nv <= 64 * 32 &&
        rows <= 0x7fffffffLL) {
        const int per_lane = (int)((nv + 63) / 64);
        const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)), block(256);
        const int c = (int)cols;
#define TIQ_QG(V)                                                                                      \
    if (per_lane <= V) {                                                                               \
        hipLaunchKernelGGL((quant_g128_vec<V>), grid, block, 0, st, w, rows, c, packed, scale_f16); \
        return launch_status();                                                                        \
    }
        TIQ_QG(1) TIQ_QG(2) TIQ_QG(4) TIQ_QG(8) TIQ_QG(16) TIQ_QG(32)
#undef TIQ_QG
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
