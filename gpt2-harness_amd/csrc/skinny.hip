// Decode linear for batches of up to 32 rows with fp32 activations, on the
// matrix cores -- the quantized Linears of a batched decode step
// (model.py:254,319,352,355 at T = 1, M = batch) and the fp32 tied lm_head
// (model.py:585), with the same optional fusions as the decode GEMV:
//     y = act(LayerNorm(x) @ W^T * scale + bias) + residual
//
//   * One workgroup of 8 wavefronts owns 32 weight rows (one 32 x 32 MFMA
//     tile of outputs) and 32 activation rows; its wavefronts split K into
//     32-wide units and sum their partial tiles through LDS in a fixed order
//     (results do not depend on timing).
//   * Activations are split exactly into three bf16 planes (x = hi + lo + lo2,
//     the rounding residues are exact in fp32): with int8 weights (exact in
//     bf16) every product the MFMA forms is exact, so the result is as
//     accurate as an fp32 product. fp32 weights are split the same way and
//     the six plane products with combined weight >= 2^-16 are kept (the
//     dropped ones are below fp32 rounding of the sum).
//   * Each wavefront loads its weight slices straight into MFMA operand
//     registers (lane (r, h) holds 16 consecutive K of weight row r), 4 units
//     at a time (2 for fp32 weights), double buffered, and converts them in
//     registers.
//   * LayerNorm statistics (two-pass mean and biased variance, as torch) are
//     computed over the workgroup's activation rows, which needs K covered by
//     one workgroup (at most 2048 with 8 wavefronts of 8 units).
#include "tiq_internal.hpp"

namespace tiq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
// units per load batch: 4 for int8 weights, 2 for fp32 weights (4x the bytes)
template <int WF>
constexpr int chunk_units() { return WF == kW8 ? 4 : 2; }
constexpr int kLnMaxK = kWaves * 8 * 32;

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    const bf16x2 v = __builtin_convertvector(floatx2{a, b}, bf16x2);
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// 8 fp32 values -> three bf16x8 planes with hi + lo + lo2 == v.
__device__ __forceinline__ void split3(const float (&v)[8], bf16x8& p0, bf16x8& p1, bf16x8& p2) {
    u32x4 a, b, c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = v[2 * i], x1 = v[2 * i + 1];
        const uint32_t h = pk_bf16(x0, x1);
        const float r0 = x0 - bf_lo(h), r1 = x1 - bf_hi(h);
        const uint32_t l = pk_bf16(r0, r1);
        const float s0 = r0 - bf_lo(l), s1 = r1 - bf_hi(l);
        a[i] = h;
        b[i] = l;
        c[i] = pk_bf16(s0, s1);
    }
    p0 = __builtin_bit_cast(bf16x8, a);
    p1 = __builtin_bit_cast(bf16x8, b);
    p2 = __builtin_bit_cast(bf16x8, c);
}

__device__ __forceinline__ uint32_t bf16x2_of_bytes(uint32_t d, int sh) {
    const float lo = (float)((int32_t)(d << (24 - sh)) >> 24);
    const float hi = (float)((int32_t)(d << (16 - sh)) >> 24);
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ float gelu_tanh_f(float x) {
    const float k = 0.7978845608028654f;  // sqrt(2 / pi)
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

template <typename TY>
__device__ __forceinline__ void store_out(TY* p, float v) {
    if constexpr (sizeof(TY) == 4) *p = v;
    else *p = f32_to_bf16_bits(v);
}

// WF: kW8 (int8 codes, per-row scale) or kF32 (fp32 weights, no scale).
template <int WF, typename TY>
__global__ __launch_bounds__(kWaves * 64, 1) void skinny_kernel(
    const float* __restrict__ x, int64_t ldx, int M, int K, const uint8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, const float* __restrict__ bias, int N, TY* __restrict__ y, int64_t ldy,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, float ln_eps, int act,
    const float* __restrict__ res, int64_t ldr) {
    constexpr int WB = (WF == kW8) ? 16 : 64;  // weight bytes a lane loads per unit
    constexpr int kChunk = chunk_units<WF>();
    __shared__ float red[kWaves][32][33];      // partial output tiles, rows padded
    __shared__ float stat[kWaves][32];
    __shared__ float mean_s[32], rstd_s[32];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
    const int U = K / 32;
    const int u0 = wave * U / kWaves, u1 = (wave + 1) * U / kWaves;
    const bool xrow_ok = m0 + r < M;
    const float* xr = x + (int64_t)(xrow_ok ? m0 + r : 0) * ldx + 16 * h;  // + 32 u
    const uint8_t* wr = w + (int64_t)min(n0 + r, N - 1) * ldw + WB * h;    // + 2 WB u

    // LayerNorm statistics of the 32 activation rows (two-pass)
    float mu = 0.f, rs = 1.f;
    if (ln_w) {
        float s = 0.f;
        for (int u = u0; u < u1; ++u) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4*>(xr + 32 * u + 4 * q);
                s += (v.x + v.y) + (v.z + v.w);
            }
        }
        s += __shfl_xor(s, 32, 64);
        if (h == 0) stat[wave][r] = s;
        __syncthreads();
        if (threadIdx.x < 32) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < kWaves; ++i) t += stat[i][threadIdx.x];
            mean_s[threadIdx.x] = t / (float)K;
        }
        __syncthreads();
        mu = mean_s[r];
        float d = 0.f;
        for (int u = u0; u < u1; ++u) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4*>(xr + 32 * u + 4 * q);
                const float a = v.x - mu, b = v.y - mu, c = v.z - mu, e = v.w - mu;
                d += (a * a + b * b) + (c * c + e * e);
            }
        }
        d += __shfl_xor(d, 32, 64);
        __syncthreads();
        if (h == 0) stat[wave][r] = d;
        __syncthreads();
        if (threadIdx.x < 32) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < kWaves; ++i) t += stat[i][threadIdx.x];
            rstd_s[threadIdx.x] = 1.0f / sqrtf(t / (float)K + ln_eps);
        }
        __syncthreads();
        rs = rstd_s[r];
    }

    floatx16 acc;
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.f;

    // register batches: kChunk units of activations (16 fp32) and weights
    float xa[2][kChunk][16];
    u32x4 wa[2][kChunk][WB / 16];
    auto load = [&](int b, int ub) {
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
            const int u = ub + c < u1 ? ub + c : u1 - 1;  // past the end: repeat (unused)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4*>(xr + 32 * u + 4 * q);
                xa[b][c][4 * q] = v.x;
                xa[b][c][4 * q + 1] = v.y;
                xa[b][c][4 * q + 2] = v.z;
                xa[b][c][4 * q + 3] = v.w;
            }
#pragma unroll
            for (int q = 0; q < WB / 16; ++q)
                wa[b][c][q] = *reinterpret_cast<const u32x4*>(wr + 2 * WB * u + 16 * q);
        }
    };
    auto compute = [&](int b, int ub) {
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
            if (ub + c >= u1) break;
            const int k0 = 32 * (ub + c) + 16 * h;
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = xrow_ok ? xa[b][c][i] : 0.f;
            if (ln_w) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 g = *reinterpret_cast<const float4*>(ln_w + k0 + 4 * q);
                    const float4 bb = *reinterpret_cast<const float4*>(ln_b + k0 + 4 * q);
                    v[4 * q] = xrow_ok ? (v[4 * q] - mu) * rs * g.x + bb.x : 0.f;
                    v[4 * q + 1] = xrow_ok ? (v[4 * q + 1] - mu) * rs * g.y + bb.y : 0.f;
                    v[4 * q + 2] = xrow_ok ? (v[4 * q + 2] - mu) * rs * g.z + bb.z : 0.f;
                    v[4 * q + 3] = xrow_ok ? (v[4 * q + 3] - mu) * rs * g.w + bb.w : 0.f;
                }
            }
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                float ve[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) ve[i] = v[8 * e + i];
                bf16x8 x0, x1, x2;
                split3(ve, x0, x1, x2);
                if constexpr (WF == kW8) {
                    const u32x4 d = wa[b][c][0];
                    const uint32_t s0 = e == 0 ? d.x : d.z, s1 = e == 0 ? d.y : d.w;
                    const u32x4 wv = {bf16x2_of_bytes(s0, 0), bf16x2_of_bytes(s0, 16), bf16x2_of_bytes(s1, 0),
                                      bf16x2_of_bytes(s1, 16)};
                    const bf16x8 wf = __builtin_bit_cast(bf16x8, wv);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, x0, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, x1, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, x2, acc, 0, 0, 0);
                } else {
                    float wv[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) wv[i] = __uint_as_float(wa[b][c][2 * e + i / 4][i % 4]);
                    bf16x8 w0, w1, w2;
                    split3(wv, w0, w1, w2);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, x0, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, x1, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, x0, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, x2, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, x1, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w2, x0, acc, 0, 0, 0);
                }
            }
        }
    };
    // two register batches, alternating (literal indices keep them in VGPRs)
    if (u0 < u1) load(0, u0);
    for (int ub = u0; ub < u1; ub += 2 * kChunk) {
        if (ub + kChunk < u1) load(1, ub + kChunk);
        compute(0, ub);
        if (ub + kChunk >= u1) break;
        if (ub + 2 * kChunk < u1) load(0, ub + 2 * kChunk);
        compute(1, ub + kChunk);
    }

    // partial tiles -> LDS: register q of lane (r, h) is output row
    // n = 8 (q / 4) + 4 h + q % 4 of the tile, activation row m = r
#pragma unroll
    for (int q = 0; q < 16; ++q) red[wave][r][8 * (q >> 2) + 4 * h + (q & 3)] = acc[q];
    __syncthreads();
    // 1024 outputs, two per thread: m = o / 32, n = o % 32 (a row of y per 32 threads)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int o = threadIdx.x + kWaves * 64 * t;
        const int m = o >> 5, nn = o & 31;
        const int gm = m0 + m, gn = n0 + nn;
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) v += red[i][m][nn];
        if (gm < M && gn < N) {
            if (WF == kW8) v *= scale[gn];
            if (bias) v += bias[gn];
            if (act == 1) v = gelu_tanh_f(v);
            if (res) v += res[(int64_t)gm * ldr + gn];
            store_out<TY>(y + (int64_t)gm * ldy + gn, v);
        }
    }
}

template <int WF, typename TY>
int run_skinny(const LinearArgs& a) {
    const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 31) / 32));
    hipLaunchKernelGGL((skinny_kernel<WF, TY>), grid, dim3(kWaves * 64), 0, a.stream, static_cast<const float*>(a.x),
                       a.ldx, (int)a.M, (int)a.K, a.w, a.ldw, a.scale, a.bias, (int)a.N, static_cast<TY*>(a.y),
                       a.ldy, a.fuse.ln_w, a.fuse.ln_b, a.fuse.ln_eps, a.fuse.act, a.fuse.res, a.fuse.ldr);
    return launch_status();
}

}  // namespace

bool skinny_supported(const LinearArgs& a) {
    if (a.x_dtype != TIQ_F32 || (a.fmt != kW8 && a.fmt != kF32)) return false;
    if (a.M < kSkinnyMinRows || a.M > 64 || a.K % 32 != 0 || a.N > 0x7fffffff) return false;
    if (!aligned(a.x, 16) || a.ldx % 4 != 0 || !aligned(a.w, 16) || a.ldw % 16 != 0) return false;
    if (a.fuse.ln_w && (a.K > kLnMaxK || !aligned(a.fuse.ln_w, 16) || !aligned(a.fuse.ln_b, 16))) return false;
    // the residual may alias y only element for element
    if (a.fuse.res && a.fuse.res != a.y && a.fuse.ldr < a.N) return false;
    return true;
}

int launch_skinny(const LinearArgs& a) {
    if (a.fmt == kW8) return a.y_dtype == TIQ_F32 ? run_skinny<kW8, float>(a) : run_skinny<kW8, uint16_t>(a);
    return a.y_dtype == TIQ_F32 ? run_skinny<kF32, float>(a) : run_skinny<kF32, uint16_t>(a);
}

}  // namespace tiq
