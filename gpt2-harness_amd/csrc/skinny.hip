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
//   * Each wavefront requests all of its weight slices at once, straight into
//     MFMA operand registers (lane (r, h) holds 16 consecutive K of weight
//     row r): the whole matrix is in flight together, which a decode linear
//     (a few MB read once) needs to approach HBM bandwidth. They are converted
//     in registers as the units are consumed.
//   * LayerNorm statistics (two-pass mean and biased variance, as torch) are
//     computed over the workgroup's activation rows, which needs K covered by
//     one workgroup (at most 2048 with 8 wavefronts of 8 units).
#include <algorithm>
#include <utility>

#include "tiq_internal.hpp"

namespace tiq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
// Units (32 K each) a wavefront holds in registers: all of its share of K.
// int8: 25 units (K <= 8 * 25 * 32 = 6400); fp32 weights (4x the bytes): 8.
// int8 codes, row-major or in operand tiles
template <int WF>
constexpr bool is_w8() { return WF == kW8 || WF == kW8T; }
template <int WF>
constexpr int max_units() { return is_w8<WF>() ? 25 : 8; }
// activation units in flight per wavefront (ring): 4, 3 with fp32 weights
template <int WF>
constexpr int ring_units() { return is_w8<WF>() ? 4 : 3; }
// With int8 weights and the plane input, up to kPlUnits units per wavefront
// (K <= 8 * 7 * 32 = 1792) have every activation operand in flight at once;
// longer K streams them through the ring.
constexpr int kPlUnits = 7;
constexpr int kLnMaxK = kWaves * 8 * 32;


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

template <typename TY>
__device__ __forceinline__ void store_out(TY* p, float v) {
    if constexpr (sizeof(TY) == 4) *p = v;
    else *p = f32_to_bf16_bits(v);
}

// LayerNorm (optional) and the exact three-plane split of M activation rows,
// once per linear, into MFMA operand order: for row tile t (32 rows), unit u
// (32 K), plane q and half e, a 1 KB block holds the 16-byte operand of each
// lane l = 32 h + r (row 32 t + r, K = 32 u + 16 h + 8 e + 0..7), so that
// the product kernel reads each operand with one contiguous load.
// One workgroup per row; two-pass mean and biased variance as torch.
template <bool LN>
__global__ __launch_bounds__(256) void ln_split_kernel(const float* __restrict__ x, int64_t ldx, int K,
                                                       const float* __restrict__ ln_w,
                                                       const float* __restrict__ ln_b, float ln_eps,
                                                       uint16_t* __restrict__ x3) {
    __shared__ float part[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)m * ldx;
    float mu = 0.f, rs = 1.f;
    if (LN) {
        float s = 0.f;
        for (int k = 4 * tid; k < K; k += 1024) {
            const float4 v = *reinterpret_cast<const float4*>(xr + k);
            s += (v.x + v.y) + (v.z + v.w);
        }
        s = wave_sum_dpp(s);
        if ((tid & 63) == 0) part[tid >> 6] = s;
        __syncthreads();
        mu = ((part[0] + part[1]) + (part[2] + part[3])) / (float)K;
        __syncthreads();
        float d = 0.f;
        for (int k = 4 * tid; k < K; k += 1024) {
            const float4 v = *reinterpret_cast<const float4*>(xr + k);
            const float a = v.x - mu, b = v.y - mu, c = v.z - mu, e = v.w - mu;
            d += (a * a + b * b) + (c * c + e * e);
        }
        d = wave_sum_dpp(d);
        if ((tid & 63) == 0) part[tid >> 6] = d;
        __syncthreads();
        rs = 1.0f / sqrtf(((part[0] + part[1]) + (part[2] + part[3])) / (float)K + ln_eps);
    }
    const int U = K / 32, t = m >> 5, r = m & 31;
    for (int c = tid; c < K / 8; c += 256) {  // 8 consecutive K per thread: one operand chunk
        const int k = 8 * c, u = k >> 5, h = (k >> 4) & 1, e = (k >> 3) & 1;
        float v[8];
        *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(xr + k);
        *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(xr + k + 4);
        if (LN) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (v[i] - mu) * rs * ln_w[k + i] + ln_b[k + i];
        }
        u32x4 pl[3];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x0 = v[2 * i], x1 = v[2 * i + 1];
            const uint32_t hh = pk_bf16(x0, x1);
            const float r0 = x0 - bf_lo(hh), r1 = x1 - bf_hi(hh);
            const uint32_t l = pk_bf16(r0, r1);
            pl[0][i] = hh;
            pl[1][i] = l;
            pl[2][i] = pk_bf16(r0 - bf_lo(l), r1 - bf_hi(l));
        }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            const int64_t blk = (((int64_t)t * U + u) * 3 + q) * 2 + e;
            *reinterpret_cast<u32x4*>(x3 + (blk * 64 + 32 * h + r) * 8) = pl[q];
        }
    }
}

// The end of a split-K decode linear, one workgroup of NT threads per
// activation row m (256 for rows of up to 2048 columns, else 1024), thread t
// owning the 8 consecutive columns 8 t .. 8 t + 7:
// the S partial rows (row m of slice s at part + (s M + m) ldp) are summed in
// a fixed order (the result does not depend on timing), then scale, bias,
// GELU(tanh) and the residual (which may alias y: every element is read and
// written by one thread) give the output row, stored to y when y is given.
// With PLANES the row is also written as the next linear's operand planes
// (ln_split_kernel's layout, K' = N), after LayerNorm when LN. With S = 1,
// no epilogue and part = fp32 rows, the kernel is a LayerNorm + split pass.
// Every load is issued before any is used (the slices eight at a time, after
// the epilogue operands) and none sits behind a branch (the optional operands
// are compile-time flags): one trip to memory for up to eight slices.
constexpr int kRedThreads = 1024;
constexpr int kRedMaxCols = kRedThreads * 8;
template <bool LN, bool PLANES, bool SC, bool BI, bool RS, int NT>
__global__ __launch_bounds__(NT) void reduce_rows_kernel(const float* __restrict__ part, int64_t ldp, int S, int M,
                                                         int N, const float* __restrict__ scale,
                                                         const float* __restrict__ bias, int act, const float* res,
                                                         int64_t ldr, float* y, int64_t ldy,
                                                         const float* __restrict__ ln_w,
                                                         const float* __restrict__ ln_b, float ln_eps,
                                                         uint16_t* __restrict__ x3) {
    __shared__ float red[NT / 64];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int NC8 = N / 8;
    const bool own = tid < NC8;
    const int n = 8 * min(tid, NC8 - 1);  // a thread past the row repeats its last chunk, unused
    // the epilogue operands first, then the slices (indices clamped, the
    // repeats not added), summed in slice order
    float4 sc[2], bi[2], rs[2], gw[2], gb[2];
    if constexpr (SC) sc[0] = reinterpret_cast<const float4*>(scale + n)[0], sc[1] = reinterpret_cast<const float4*>(scale + n)[1];
    if constexpr (BI) bi[0] = reinterpret_cast<const float4*>(bias + n)[0], bi[1] = reinterpret_cast<const float4*>(bias + n)[1];
    if constexpr (RS) {
        rs[0] = reinterpret_cast<const float4*>(res + (int64_t)m * ldr + n)[0];
        rs[1] = reinterpret_cast<const float4*>(res + (int64_t)m * ldr + n)[1];
    }
    if constexpr (LN) gw[0] = reinterpret_cast<const float4*>(ln_w + n)[0], gw[1] = reinterpret_cast<const float4*>(ln_w + n)[1];
    if constexpr (LN) gb[0] = reinterpret_cast<const float4*>(ln_b + n)[0], gb[1] = reinterpret_cast<const float4*>(ln_b + n)[1];
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int z0 = 0; z0 < S; z0 += 8) {
        float4 p[8][2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float* pr = part + ((int64_t)min(z0 + j, S - 1) * M + m) * ldp + n;
            p[j][0] = reinterpret_cast<const float4*>(pr)[0];
            p[j][1] = reinterpret_cast<const float4*>(pr)[1];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool use = z0 + j < S;
            a[0] = use ? a[0] + p[j][0].x : a[0]; a[1] = use ? a[1] + p[j][0].y : a[1];
            a[2] = use ? a[2] + p[j][0].z : a[2]; a[3] = use ? a[3] + p[j][0].w : a[3];
            a[4] = use ? a[4] + p[j][1].x : a[4]; a[5] = use ? a[5] + p[j][1].y : a[5];
            a[6] = use ? a[6] + p[j][1].z : a[6]; a[7] = use ? a[7] + p[j][1].w : a[7];
        }
    }
    auto lane8 = [](const float4 (&f)[2], int i) { const float4 q = f[i >> 2]; return (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w; };
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float t = a[i];
        if constexpr (SC) t *= lane8(sc, i);
        if constexpr (BI) t += lane8(bi, i);
        v[i] = t;
    }
    apply_act<8>(v, act);
    if constexpr (RS) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += lane8(rs, i);
    }
    if (y && own) {
        float* yr = y + (int64_t)m * ldy + n;
        reinterpret_cast<float4*>(yr)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(yr)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if constexpr (!PLANES) return;
    float mu = 0.f, rstd = 1.f;
    if constexpr (LN) {  // two-pass mean and biased variance over the row, as torch
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += v[i];
        sum = wave_sum_dpp(own ? sum : 0.f);
        if ((tid & 63) == 0) red[tid >> 6] = sum;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) tot += red[w];
        mu = tot / (float)N;
        __syncthreads();
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d += (v[i] - mu) * (v[i] - mu);
        d = wave_sum_dpp(own ? d : 0.f);
        if ((tid & 63) == 0) red[tid >> 6] = d;
        __syncthreads();
        tot = 0.f;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) tot += red[w];
        rstd = 1.0f / sqrtf(tot / (float)N + ln_eps);
    }
    if (!own) return;
    const int U = N / 32, t = m >> 5, r = m & 31;
    const int u = n >> 5, h = (n >> 4) & 1, e = (n >> 3) & 1;
    float x8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (LN) x8[i] = (v[i] - mu) * rstd * lane8(gw, i) + lane8(gb, i);
        else x8[i] = v[i];
    }
    u32x4 pl[3];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = x8[2 * i], x1 = x8[2 * i + 1];
        const uint32_t hh = pk_bf16(x0, x1);
        const float r0 = x0 - bf_lo(hh), r1 = x1 - bf_hi(hh);
        const uint32_t l = pk_bf16(r0, r1);
        pl[0][i] = hh;
        pl[1][i] = l;
        pl[2][i] = pk_bf16(r0 - bf_lo(l), r1 - bf_hi(l));
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const int64_t blk = (((int64_t)t * U + u) * 3 + q) * 2 + e;
        *reinterpret_cast<u32x4*>(x3 + (blk * 64 + 32 * h + r) * 8) = pl[q];
    }
}

// The reduction kernel instance for these operands.
using ReduceFn = void (*)(const float*, int64_t, int, int, int, const float*, const float*, int, const float*,
                          int64_t, float*, int64_t, const float*, const float*, float, uint16_t*);
template <bool LN, bool PLANES, int NT>
ReduceFn reduce_fn(bool sc, bool bi, bool rs) {
    const int k = (sc ? 4 : 0) | (bi ? 2 : 0) | (rs ? 1 : 0);
    switch (k) {
        case 0: return reduce_rows_kernel<LN, PLANES, false, false, false, NT>;
        case 1: return reduce_rows_kernel<LN, PLANES, false, false, true, NT>;
        case 2: return reduce_rows_kernel<LN, PLANES, false, true, false, NT>;
        case 3: return reduce_rows_kernel<LN, PLANES, false, true, true, NT>;
        case 4: return reduce_rows_kernel<LN, PLANES, true, false, false, NT>;
        case 5: return reduce_rows_kernel<LN, PLANES, true, false, true, NT>;
        case 6: return reduce_rows_kernel<LN, PLANES, true, true, false, NT>;
        default: return reduce_rows_kernel<LN, PLANES, true, true, true, NT>;
    }
}

// threads of the reduction workgroup for rows of N columns (8 a thread)
int red_threads(int64_t N) { return N <= 2048 ? 256 : 1024; }

ReduceFn pick_reduce(bool ln, bool planes, bool sc, bool bi, bool rs, int64_t N) {
    if (N <= 2048) {
        if (!planes) return reduce_fn<false, false, 256>(sc, bi, rs);
        return ln ? reduce_fn<true, true, 256>(sc, bi, rs) : reduce_fn<false, true, 256>(sc, bi, rs);
    }
    if (!planes) return reduce_fn<false, false, 1024>(sc, bi, rs);
    return ln ? reduce_fn<true, true, 1024>(sc, bi, rs) : reduce_fn<false, true, 1024>(sc, bi, rs);
}

// WF: kW8 (int8 codes, per-row scale), kW8T (the same codes in the operand
// tiles of tile_int8_kernel: 1 KB per 32 rows x 32 columns, lane-contiguous,
// read with nontemporal loads) or kF32 (fp32 weights, no scale).
// XM: how the activations arrive.
//   kXRows   fp32 rows, LayerNorm'd (optionally) and split here;
//   kXPlanes the three bf16 planes of ln_split_kernel (x is then a uint16_t
//            pointer to the operand-ordered blocks, LayerNorm already applied);
//   kXBf16   bf16 rows (int8 weights only, no LayerNorm): one plane, each
//            int8 x bf16 product exact, one MFMA per 16 K.
enum XMode : int { kXRows = 0, kXPlanes = 1, kXBf16 = 2 };
// bf16 rows: units a wavefront holds, every one in flight at once
// (K <= 8 * 12 * 32 = 3072)
constexpr int kXbUnits = 12;

template <int WF, int XM, typename TY>
__global__ __launch_bounds__(kWaves * 64, 1) void skinny_kernel(
    const float* __restrict__ x, int64_t ldx, int M, int K, const uint8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, const float* __restrict__ bias, int N, TY* y, int64_t ldy,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, float ln_eps, int act,
    const float* res, int64_t ldr, float* __restrict__ part, uint16_t* __restrict__ x3o) {
    // y may alias res (x = x + f(x) in place): neither is __restrict__
    constexpr bool W8 = is_w8<WF>();
    constexpr int WB = W8 ? 16 : 64;  // weight bytes a lane loads per unit
    constexpr bool PL = XM == kXPlanes;
    constexpr int kXp = ring_units<WF>();
    __shared__ float red[kWaves][32][33];      // partial output tiles, rows padded
    __shared__ float stat[kWaves][32];
    __shared__ float mean_s[32], rstd_s[32];
    __shared__ __attribute__((aligned(16))) float gb_s[2][kLnMaxK];  // LayerNorm weight and bias

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
    const int U = K / 32;
    // split-K: workgroup z takes units [z U / S, (z + 1) U / S) of the row,
    // shared out over its wavefronts (S = 1: the whole row)
    const int ub = blockIdx.z * U / gridDim.z, Us = (blockIdx.z + 1) * U / gridDim.z - ub;
    const int u0 = ub + wave * Us / kWaves, u1 = ub + (wave + 1) * Us / kWaves;
    const bool xrow_ok = m0 + r < M;
    const float* xr = x + (int64_t)(xrow_ok ? m0 + r : 0) * ldx + 16 * h;  // + 32 u
    const uint16_t* xbr = reinterpret_cast<const uint16_t*>(x) + (int64_t)(xrow_ok ? m0 + r : 0) * ldx + 16 * h;
    // plane input: this row tile's operand blocks, lane-contiguous
    const uint16_t* x3t = reinterpret_cast<const uint16_t*>(x) + (int64_t)blockIdx.y * (K / 32) * 6 * 64 * 8 + lane * 8;
    // row-major: row n0 + r, + 2 WB u per unit; tiles: this row tile's 1 KB
    // blocks (N % 32 == 0, the host checks), + 1024 u per unit
    const uint8_t* wr = WF == kW8T ? w + (int64_t)blockIdx.x * U * 1024 + lane * 16
                                   : w + (int64_t)min(n0 + r, N - 1) * ldw + WB * h;

    const int cnt = u1 - u0;  // <= kUnits (the host checks K)
    constexpr int kUnits = XM == kXBf16 ? kXbUnits : max_units<WF>();
    // every weight slice of the wavefront is requested first, so the whole
    // matrix is in flight at once (behind the LayerNorm statistics);
    // activations (L2 hits) follow through a ring of kXp unit registers
    u32x4 wreg[kUnits][WB / 16];
#pragma unroll
    for (int c = 0; c < kUnits; ++c)
        if (c < cnt) {
            if constexpr (WF == kW8T) {
                // 1 KB of consecutive memory per load instruction, read once:
                // nontemporal (1.5-1.9 us less per launch on a 7.7-10 MB
                // matrix than row-major codes with the default policy)
                wreg[c][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (int64_t)(u0 + c) * 1024));
            } else {
#pragma unroll
                for (int q = 0; q < WB / 16; ++q)
                    wreg[c][q] = *reinterpret_cast<const u32x4*>(wr + 2 * WB * (u0 + c) + 16 * q);
            }
        }
    // Epilogue operands of this thread's two outputs (column n0 + t % 32,
    // rows m0 + t / 32 and 16 below it), requested with the weights rather
    // than after the reduction, where they would cost another serial trip to
    // HBM. A residual aliasing y is read by the thread that writes the same
    // element.
    const int ep_n = n0 + (threadIdx.x & 31), ep_m = m0 + (threadIdx.x >> 5);
    float ep_scale = 1.f, ep_bias = 0.f, ep_res[2] = {0.f, 0.f};
    if (ep_n < N) {
        if (W8) ep_scale = scale[ep_n];
        if (bias) ep_bias = bias[ep_n];
        if (res) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
                if (ep_m + 16 * t < M) ep_res[t] = res[(int64_t)(ep_m + 16 * t) * ldr + ep_n];
        }
    }
    // planes out: thread t finishes row t / 16, columns n0 + 2 (t % 16) + 0..1
    // (every wavefront takes a share of the GELU)
    float2 pe_scale = make_float2(1.f, 1.f), pe_bias = make_float2(0.f, 0.f);
    if (x3o) {
        const int c2 = n0 + 2 * (threadIdx.x & 15);  // N % 32 == 0 (the host checks): in range
        if (W8) pe_scale = *reinterpret_cast<const float2*>(scale + c2);
        if (bias) pe_bias = *reinterpret_cast<const float2*>(bias + c2);
    }
    // LayerNorm statistics of the 32 activation rows (two-pass); its weight
    // and bias go to LDS (read there, they add no global loads to the unit
    // loop, whose in-order waits would otherwise include the prefetches)
    float mu = 0.f, rs = 1.f;
    if (XM == kXRows && ln_w) {
        for (int i = threadIdx.x; i < K / 4; i += kWaves * 64) {
            reinterpret_cast<float4*>(gb_s[0])[i] = reinterpret_cast<const float4*>(ln_w)[i];
            reinterpret_cast<float4*>(gb_s[1])[i] = reinterpret_cast<const float4*>(ln_b)[i];
        }
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

    // compute one unit: activations v (16 fp32 of row r, K = 32 u + 16 h + 0..15)
    // and the weight registers of the same K
    auto unit = [&](int u, const float (&xv)[16], const u32x4 (&wv)[WB / 16]) {
        const int k0 = 32 * u + 16 * h;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = xrow_ok ? xv[i] : 0.f;
        if (ln_w) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 g = *reinterpret_cast<const float4*>(gb_s[0] + k0 + 4 * q);
                const float4 bb = *reinterpret_cast<const float4*>(gb_s[1] + k0 + 4 * q);
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
            if constexpr (W8) {
                const u32x4 d = wv[0];
                const uint32_t s0 = e == 0 ? d.x : d.z, s1 = e == 0 ? d.y : d.w;
                const u32x4 wq = {bf16x2_of_bytes(s0, 0), bf16x2_of_bytes(s0, 16), bf16x2_of_bytes(s1, 0),
                                  bf16x2_of_bytes(s1, 16)};
                const bf16x8 wf = __builtin_bit_cast(bf16x8, wq);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, x0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, x1, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, x2, acc, 0, 0, 0);
            } else {
                float wf[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) wf[i] = __uint_as_float(wv[2 * e + i / 4][i % 4]);
                bf16x8 w0, w1, w2;
                split3(wf, w0, w1, w2);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, x0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, x1, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, x0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, x2, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, x1, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w2, x0, acc, 0, 0, 0);
            }
        }
    };
    // plane mode: the 6 operand registers of a unit come straight from x3
    auto unit_pl = [&](const u32x4 (&xv)[3][2], const u32x4 (&wv)[WB / 16]) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            bf16x8 xq[3];
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                u32x4 t = xv[q][e];
                if (!xrow_ok) t = u32x4{0u, 0u, 0u, 0u};
                xq[q] = __builtin_bit_cast(bf16x8, t);
            }
            if constexpr (W8) {
                const u32x4 d = wv[0];
                const uint32_t s0 = e == 0 ? d.x : d.z, s1 = e == 0 ? d.y : d.w;
                const u32x4 wq = {bf16x2_of_bytes(s0, 0), bf16x2_of_bytes(s0, 16), bf16x2_of_bytes(s1, 0),
                                  bf16x2_of_bytes(s1, 16)};
                const bf16x8 wf = __builtin_bit_cast(bf16x8, wq);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xq[0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xq[1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xq[2], acc, 0, 0, 0);
            } else {
                float wf[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) wf[i] = __uint_as_float(wv[2 * e + i / 4][i % 4]);
                bf16x8 w0, w1, w2;
                split3(wf, w0, w1, w2);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, xq[0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, xq[1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, xq[0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, xq[2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, xq[1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w2, xq[0], acc, 0, 0, 0);
            }
        }
    };
    auto xload_pl = [&](int u, u32x4 (&xv)[3][2]) {
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
            for (int e = 0; e < 2; ++e)
                xv[q][e] = *reinterpret_cast<const u32x4*>(x3t + (((int64_t)u * 3 + q) * 2 + e) * 64 * 8);
    };
    auto xload = [&](int u, float (&xv)[16]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(xr + 32 * u + 4 * q);
            xv[4 * q] = v.x;
            xv[4 * q + 1] = v.y;
            xv[4 * q + 2] = v.z;
            xv[4 * q + 3] = v.w;
        }
    };

    // bf16 rows: the 16 K of a lane are two operand registers
    auto xload_bf = [&](int u, u32x4 (&xv)[2]) {
        xv[0] = *reinterpret_cast<const u32x4*>(xbr + 32 * u);
        xv[1] = *reinterpret_cast<const u32x4*>(xbr + 32 * u + 8);
    };
    auto unit_bf = [&](const u32x4 (&xv)[2], const u32x4 (&wv)[WB / 16]) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const u32x4 t = xrow_ok ? xv[e] : u32x4{0u, 0u, 0u, 0u};
            const u32x4 d = wv[0];
            const uint32_t s0 = e == 0 ? d.x : d.z, s1 = e == 0 ? d.y : d.w;
            const u32x4 wq = {bf16x2_of_bytes(s0, 0), bf16x2_of_bytes(s0, 16), bf16x2_of_bytes(s1, 0),
                              bf16x2_of_bytes(s1, 16)};
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wq),
                                                          __builtin_bit_cast(bf16x8, t), acc, 0, 0, 0);
        }
    };

    if constexpr (XM == kXBf16) {
        static_assert(WF == kW8, "bf16 rows are taken with row-major int8 weights");
        // every activation unit in flight (the host checks cnt <= kXbUnits)
        u32x4 ball[kXbUnits][2];
#pragma unroll
        for (int c = 0; c < kXbUnits; ++c)
            if (c < cnt) xload_bf(u0 + c, ball[c]);
#pragma unroll
        for (int c = 0; c < kXbUnits; ++c)
            if (c < cnt) unit_bf(ball[c], wreg[c]);
    } else if (PL && W8 && cnt <= kPlUnits) {
        // every activation unit in flight too
        u32x4 pall[kPlUnits][3][2];
#pragma unroll
        for (int c = 0; c < kPlUnits; ++c)
            if (c < cnt) xload_pl(u0 + c, pall[c]);
#pragma unroll
        for (int c = 0; c < kPlUnits; ++c)
            if (c < cnt) unit_pl(pall[c], wreg[c]);
    } else if constexpr (PL) {
        u32x4 pring[kXp][3][2];
#pragma unroll
        for (int c = 0; c < kXp; ++c)
            if (c < cnt) xload_pl(u0 + c, pring[c]);
#pragma unroll
        for (int c = 0; c < kUnits; ++c) {
            if (c < cnt) {
                unit_pl(pring[c % kXp], wreg[c]);
                if (c + kXp < cnt) xload_pl(u0 + c + kXp, pring[c % kXp]);
            }
        }
    } else {
        float xring[kXp][16];
#pragma unroll
        for (int c = 0; c < kXp; ++c)
            if (c < cnt) xload(u0 + c, xring[c]);
#pragma unroll
        for (int c = 0; c < kUnits; ++c) {
            if (c < cnt) {
                unit(u0 + c, xring[c % kXp], wreg[c]);
                if (c + kXp < cnt) xload(u0 + c + kXp, xring[c % kXp]);
            }
        }
    }

    // partial tiles -> LDS: register q of lane (r, h) is output row
    // n = 8 (q / 4) + 4 h + q % 4 of the tile, activation row m = r
#pragma unroll
    for (int q = 0; q < 16; ++q) red[wave][r][8 * (q >> 2) + 4 * h + (q & 3)] = acc[q];
    __syncthreads();
    if (x3o) {
        // The tile as the next linear's operand planes: its 32 columns are
        // unit u = n0 / 32 of that linear's K (= this N), row tile blockIdx.y;
        // rows past M are not written (the consumer zeroes them). Thread t:
        // row m = t / 16, columns 2 c, 2 c + 1 (c = t % 16) -- 4 bytes of the
        // 16-byte operand chunk (8 columns) of each plane.
        const int m = threadIdx.x >> 4, c = threadIdx.x & 15, gm = m0 + m;
        float v[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) t += red[w][m][2 * c + i];
            v[i] = t * (i ? pe_scale.y : pe_scale.x) + (i ? pe_bias.y : pe_bias.x);
        }
        apply_act<2>(v, act);
        if (gm < M) {
            if constexpr (sizeof(TY) == 4) {  // fp32 rows too when asked for
                if (y) *reinterpret_cast<float2*>(y + (int64_t)gm * ldy + n0 + 2 * c) = make_float2(v[0], v[1]);
            }
            const uint32_t hi = pk_bf16(v[0], v[1]);
            const float r0 = v[0] - bf_lo(hi), r1 = v[1] - bf_hi(hi);
            const uint32_t lo = pk_bf16(r0, r1);
            const uint32_t pl[3] = {hi, lo, pk_bf16(r0 - bf_lo(lo), r1 - bf_hi(lo))};
            const int64_t Uo = N / 32, u = blockIdx.x;
            const int g = c >> 2, hh = g >> 1, e = g & 1;
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                const int64_t blk = (((int64_t)blockIdx.y * Uo + u) * 3 + q) * 2 + e;
                *reinterpret_cast<uint32_t*>(x3o + (blk * 64 + 32 * hh + m) * 8 + 2 * (c & 3)) = pl[q];
            }
        }
        return;
    }
    // 1024 outputs, two per thread: m = o / 32, n = o % 32 (a row of y per 32 threads)
    float vsum[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int o = threadIdx.x + kWaves * 64 * t;
        const int m = o >> 5, nn = o & 31;
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) v += red[i][m][nn];
        vsum[t] = v;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int o = threadIdx.x + kWaves * 64 * t;
        const int m = o >> 5, nn = o & 31;
        const int gm = m0 + m, gn = n0 + nn;
        float v = vsum[t];
        if (part) {  // split-K: the raw partial sum; the epilogue runs after the reduction
            if (gm < M && gn < N) part[((int64_t)blockIdx.z * M + gm) * N + gn] = v;
            continue;
        }
        if (gm < M && gn < N) {
            if (W8) v *= ep_scale;
            if (bias) v += ep_bias;
            v = apply_act(v, act);
            if (res) v += ep_res[t];
            store_out<TY>(y + (int64_t)gm * ldy + gn, v);
        }
    }
}

// The product of a split batched decode linear whose output the reduction
// kernel (or the decode attention, for the q, k, v projection) finishes: int8
// weights (row-major or operand tiles), the activation
// planes of the previous call in, raw fp32 partial sums out (slice z of
// `part` holds K units [z U / S, (z + 1) U / S) of every output; scale, bias
// and the rest are applied by the reduction). A workgroup of 8 wavefronts owns
// RT 32-row weight tiles (N rows 32 t0 .. 32 (t0 + RT) - 1) and 32 activation
// rows; its wavefronts split its K units, at most MU each, and every
// activation operand a wavefront loads feeds the MFMAs of all RT tiles. All
// loads are issued at once, activations first; the wavefronts' partial tiles are summed through
// LDS in wavefront order (results do not depend on timing).
template <int WF, int RT, int MU>
__global__ __launch_bounds__(kWaves * 64, 1) void split_product_kernel(const uint16_t* __restrict__ x3, int M, int K,
                                                                      const uint8_t* __restrict__ w, int64_t ldw,
                                                                      int N, float* __restrict__ part) {
    static_assert(WF == kW8 || WF == kW8T, "int8 codes");
    __shared__ float red[kWaves][RT * 32][33];  // partial tiles, rows padded
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
    const int t0 = blockIdx.x * RT, m0 = blockIdx.y * 32;
    const int U = K / 32;
    const int ub = blockIdx.z * U / gridDim.z, Us = (blockIdx.z + 1) * U / gridDim.z - ub;
    const int u0 = ub + wave * Us / kWaves, cnt = ub + (wave + 1) * Us / kWaves - u0;  // <= MU (host checks)
    const bool xrow_ok = m0 + r < M;
    const uint16_t* x3t = x3 + (int64_t)blockIdx.y * U * 6 * 64 * 8 + lane * 8;
    // the activation operands first (L2 hits), then the weights (HBM): a unit's
    // MFMAs then wait for its own weights, not for every weight of the
    // wavefront as they would behind activations requested last (in-order
    // completion)
    u32x4 xv[MU][3][2];
#pragma unroll
    for (int c = 0; c < MU; ++c)
        if (c < cnt) {
#pragma unroll
            for (int q = 0; q < 3; ++q)
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    xv[c][q][e] = *reinterpret_cast<const u32x4*>(x3t + (((int64_t)(u0 + c) * 3 + q) * 2 + e) * 64 * 8);
        }
    u32x4 wreg[MU][RT];
#pragma unroll
    for (int c = 0; c < MU; ++c)
        if (c < cnt) {
#pragma unroll
            for (int j = 0; j < RT; ++j) {
                if constexpr (WF == kW8T) {  // 1 KB of consecutive codes per instruction, read once
                    wreg[c][j] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4*>(w + ((int64_t)(t0 + j) * U + u0 + c) * 1024 + lane * 16));
                } else {  // lane (r, h): 16 codes of row 32 (t0 + j) + r (clamped for a partial tile)
                    wreg[c][j] = *reinterpret_cast<const u32x4*>(w + (int64_t)min(32 * (t0 + j) + r, N - 1) * ldw +
                                                                 32 * (u0 + c) + 16 * h);
                }
            }
        }
    floatx16 acc[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[j][q] = 0.f;
#pragma unroll
    for (int c = 0; c < MU; ++c)
        if (c < cnt) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                bf16x8 xq[3];
#pragma unroll
                for (int q = 0; q < 3; ++q) {
                    u32x4 t = xv[c][q][e];
                    if (!xrow_ok) t = u32x4{0u, 0u, 0u, 0u};
                    xq[q] = __builtin_bit_cast(bf16x8, t);
                }
#pragma unroll
                for (int j = 0; j < RT; ++j) {
                    const u32x4 d = wreg[c][j];
                    const uint32_t s0 = e == 0 ? d.x : d.z, s1 = e == 0 ? d.y : d.w;
                    const u32x4 wq = {bf16x2_of_bytes(s0, 0), bf16x2_of_bytes(s0, 16), bf16x2_of_bytes(s1, 0),
                                      bf16x2_of_bytes(s1, 16)};
                    const bf16x8 wf = __builtin_bit_cast(bf16x8, wq);
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xq[0], acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xq[1], acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xq[2], acc[j], 0, 0, 0);
                }
            }
        }
    // register q of lane (r, h) in tile j: output row n = 32 (t0 + j) + 8 (q / 4)
    // + 4 h + q % 4, activation row m = m0 + r
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) red[wave][32 * j + r][8 * (q >> 2) + 4 * h + (q & 3)] = acc[j][q];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2 * RT; ++t) {  // 1024 outputs a tile, two per thread and tile
        const int o = threadIdx.x + kWaves * 64 * t;
        const int j = o >> 10, m = (o >> 5) & 31, nn = o & 31;
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) v += red[i][32 * j + m][nn];
        const int gm = m0 + m, gn = 32 * (t0 + j) + nn;
        if (gm < M && gn < N) part[((int64_t)blockIdx.z * M + gm) * N + gn] = v;
    }
}

template <int... J, typename F>
__device__ __forceinline__ void for_each_slot(std::integer_sequence<int, J...>, F&& f) {
    (f(std::integral_constant<int, J>{}), ...);
}

// The fp32 head of a batched decode (a 50257 x K tied embedding, far more
// rows than one round of workgroups) from the previous call's operand planes:
// one workgroup per CU loops over the 32-row weight tiles t = blockIdx.x +
// i gridDim.x of its row tile (blockIdx.y); its wavefronts split each tile's
// K into the same unit ranges as skinny_kernel and stream (weights, planes)
// units through a ring of kStreamSlots register slots that runs on across
// tile boundaries, so the next tile's weights are in flight while a tile's
// partial sums are reduced and stored (skinny_kernel holds one workgroup a CU
// and loads a whole tile before computing). Weights in the tiles of
// tile_f32 (1 KB of consecutive memory per load instruction, nontemporal).
// Per unit: the six plane products of the fp32 weights and activations as in
// skinny_kernel, in the same order, and the same fixed-order reduction over
// the wavefronts: the outputs equal skinny_kernel's bit for bit.
// Each wavefront reaches the per-tile barriers once per tile of its
// workgroup whatever its unit count (every wavefront holds >= 1 unit).
constexpr int kStreamSlots = 4;
__global__ __launch_bounds__(kWaves * 64, 1) void stream_f32_kernel(const uint16_t* __restrict__ x3, int M, int K,
                                                                   const uint8_t* __restrict__ wt, int N,
                                                                   float* __restrict__ y, int64_t ldy) {
    constexpr int D = kStreamSlots;
    __shared__ float red[kWaves][32][33];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
    const int U = K / 32, m0 = blockIdx.y * 32;
    const int u0 = wave * U / kWaves, cnt = (wave + 1) * U / kWaves - u0;  // >= 1 (the host checks U >= 8)
    const int T = (N + 31) / 32, G = gridDim.x;
    const int n_my = (T - (int)blockIdx.x + G - 1) / G;  // tiles blockIdx.x + i G < T
    const int L = n_my * cnt;
    const bool xrow_ok = m0 + r < M;
    const uint16_t* x3t = x3 + (int64_t)blockIdx.y * U * 6 * 64 * 8 + lane * 8;
    const uint8_t* wl = wt + lane * 16;
    u32x4 wring[D][4];
    u32x4 xring[D][3][2];
    auto issue = [&](int s, auto slot) __attribute__((always_inline)) {
        constexpr int j = decltype(slot)::value;
        const int i = s / cnt, u = u0 + (s - i * cnt);
        const uint8_t* wb = wl + ((int64_t)((int)blockIdx.x + i * G) * U + u) * 4096;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            wring[j][q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wb + 1024 * q));
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
            for (int e = 0; e < 2; ++e)
                xring[j][q][e] = *reinterpret_cast<const u32x4*>(x3t + (((int64_t)u * 3 + q) * 2 + e) * 64 * 8);
    };
    floatx16 acc;
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.f;
    auto step = [&](int s, auto slot) __attribute__((always_inline)) {
        constexpr int j = decltype(slot)::value;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            bf16x8 xq[3];
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                u32x4 tq = xring[j][q][e];
                if (!xrow_ok) tq = u32x4{0u, 0u, 0u, 0u};
                xq[q] = __builtin_bit_cast(bf16x8, tq);
            }
            float wf[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) wf[i] = __uint_as_float(wring[j][2 * e + i / 4][i % 4]);
            bf16x8 w0, w1, w2;
            split3(wf, w0, w1, w2);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, xq[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, xq[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, xq[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, xq[2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, xq[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w2, xq[0], acc, 0, 0, 0);
        }
        if (s + D < L) issue(s + D, slot);  // the slot's next unit, possibly of the next tile
        const int i = s / cnt;
        if (s - i * cnt == cnt - 1) {  // this wavefront's share of tile i is summed
#pragma unroll
            for (int q = 0; q < 16; ++q) red[wave][r][8 * (q >> 2) + 4 * h + (q & 3)] = acc[q];
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[q] = 0.f;
            __syncthreads();
            const int n0 = 32 * ((int)blockIdx.x + i * G);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {  // 1024 outputs, two per thread, wavefront order
                const int o = threadIdx.x + kWaves * 64 * tt;
                const int m = o >> 5, nn = o & 31;
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) v += red[w][m][nn];
                if (m0 + m < M && n0 + nn < N) y[(int64_t)(m0 + m) * ldy + n0 + nn] = v;
            }
            __syncthreads();  // red is free for the next tile
        }
    };
    for_each_slot(std::make_integer_sequence<int, D>{}, [&](auto slot) __attribute__((always_inline)) {
        if (decltype(slot)::value < L) issue(decltype(slot)::value, slot);
    });
    int s0 = 0;
    for (; s0 + D <= L; s0 += D)
        for_each_slot(std::make_integer_sequence<int, D>{},
                      [&](auto slot) __attribute__((always_inline)) { step(s0 + decltype(slot)::value, slot); });
    for_each_slot(std::make_integer_sequence<int, D>{}, [&](auto slot) __attribute__((always_inline)) {
        if (s0 + decltype(slot)::value < L) step(s0 + decltype(slot)::value, slot);
    });
}

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Workspace: the split activation planes, row tiles x 32 x 3K bf16 in operand order.
size_t planes_bytes(int64_t M, int64_t K) { return round256((size_t)((M + 31) / 32) * 32 * 3 * K * 2); }

template <int WF, typename TY>
int run_skinny(const LinearArgs& a) {
    const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 31) / 32));
    if (a.x_dtype == TIQ_F32 && a.ws && a.ws_bytes >= planes_bytes(a.M, a.K)) {
        // LayerNorm + split once, then the products on the planes
        uint16_t* x3 = static_cast<uint16_t*>(a.ws);
        if (a.fuse.ln_w)
            hipLaunchKernelGGL(ln_split_kernel<true>, dim3((unsigned)a.M), dim3(256), 0, a.stream,
                               static_cast<const float*>(a.x), a.ldx, (int)a.K, a.fuse.ln_w, a.fuse.ln_b,
                               a.fuse.ln_eps, x3);
        else
            hipLaunchKernelGGL(ln_split_kernel<false>, dim3((unsigned)a.M), dim3(256), 0, a.stream,
                               static_cast<const float*>(a.x), a.ldx, (int)a.K, nullptr, nullptr, 0.f, x3);
        int rc = launch_status();
        if (rc != TIQ_OK) return rc;
        hipLaunchKernelGGL((skinny_kernel<WF, kXPlanes, TY>), grid, dim3(kWaves * 64), 0, a.stream,
                           reinterpret_cast<const float*>(x3), (int64_t)0, (int)a.M, (int)a.K, a.w, a.ldw, a.scale,
                           a.bias, (int)a.N, static_cast<TY*>(a.y), a.ldy, nullptr, nullptr, 0.f, a.fuse.act,
                           a.fuse.res, a.fuse.ldr, nullptr, nullptr);
        return launch_status();
    }
    if constexpr (WF == kW8) {
        if (a.x_dtype == TIQ_BF16) {
            hipLaunchKernelGGL((skinny_kernel<kW8, kXBf16, TY>), grid, dim3(kWaves * 64), 0, a.stream,
                               static_cast<const float*>(a.x), a.ldx, (int)a.M, (int)a.K, a.w, a.ldw, a.scale,
                               a.bias, (int)a.N, static_cast<TY*>(a.y), a.ldy, nullptr, nullptr, 0.f, a.fuse.act,
                               a.fuse.res, a.fuse.ldr, nullptr, nullptr);
            return launch_status();
        }
    }
    hipLaunchKernelGGL((skinny_kernel<WF, kXRows, TY>), grid, dim3(kWaves * 64), 0, a.stream,
                       static_cast<const float*>(a.x), a.ldx, (int)a.M, (int)a.K, a.w, a.ldw, a.scale, a.bias,
                       (int)a.N, static_cast<TY*>(a.y), a.ldy, a.fuse.ln_w, a.fuse.ln_b, a.fuse.ln_eps, a.fuse.act,
                       a.fuse.res, a.fuse.ldr, nullptr, nullptr);
    return launch_status();
}

// Splits of a batched decode linear's K range when nothing but the split
// needs the reduction kernel (y rows out, or planes out without LayerNorm or
// residual): about six 32-column units per wavefront, so a split pays for its
// partial sums and the reduction launch only on long rows (6400 columns: four
// splits); with at most 64 output tiles (N <= 2048) two splits.
int64_t decode_splits(int64_t M, int64_t K, int64_t N) {
    (void)M;
    int64_t S = (K / 32) / (kWaves * 6);
    if (S <= 1 && (N + 31) / 32 <= 64 && K / 32 >= 2 * kWaves) S = 2;
    S = std::min<int64_t>(S, (K / 32) / kWaves);
    return std::max<int64_t>(1, std::min<int64_t>(S, 32));
}

// The split of an int8 product whose output the reduction kernel finishes in
// any case (LayerNorm'd planes or a residual follow): split_product_kernel
// with one weight tile a workgroup and K split until about 256 workgroups
// stream the weights, at least one 32-column unit and at most
// kSplitMaxUnits1 a wavefront, at most 16 splits. GPT-2-XL at batch 32:
// attn.c_proj and mlp.c_proj 50 tiles x 5 splits. (Two tiles a workgroup,
// which halves the activation reads per weight byte, measured no faster for
// the product at these shapes and needs twice the splits for the same
// workgroup count, which the reduction pays for: mlp.c_proj 12.4 against
// 11.1 us product + reduction.)
constexpr int kSplitMaxUnits = 4;   // units a wavefront with two tiles a workgroup
constexpr int kSplitMaxUnits1 = 8;  // with one
struct SplitPlan { int64_t S; int RT; };
int split_max_units(int RT) { return RT == 1 ? kSplitMaxUnits1 : kSplitMaxUnits; }
SplitPlan reduce_plan(int64_t M, int64_t K, int64_t N) {
    const int64_t U = K / 32, tiles = (N + 31) / 32, rows = (M + 31) / 32;
    const int64_t groups = tiles * rows;
    int64_t S = std::min<int64_t>(std::max<int64_t>(256 / groups, 1), std::max<int64_t>(U / kWaves, 1));
    S = std::max<int64_t>(S, (U + kWaves * kSplitMaxUnits1 - 1) / (kWaves * kSplitMaxUnits1));
    return {std::min<int64_t>(S, 16), 1};
}

// The split of a product whose raw partial slices its consumer sums itself
// (the q, k, v projection read by the decode attention): two weight tiles a
// workgroup where the tile count is even (each activation operand then feeds
// twice the weights), K split until about 256 workgroups stream the weights,
// at least one unit and at most split_max_units(RT) a wavefront, at most
// kMaxSlices splits (a longer K is refused). GPT-2-XL at batch 32: c_attn 75
// tile pairs x 3 splits (5.9 us against 6.7-7.3 us for one tile a workgroup
// and no split).
SplitPlan slices_plan(int64_t M, int64_t K, int64_t N) {
    const int64_t U = K / 32, tiles = (N + 31) / 32, rows = (M + 31) / 32;
    const int RT = tiles % 2 == 0 ? 2 : 1;
    const int64_t groups = tiles / RT * rows;
    int64_t S = std::min<int64_t>(std::max<int64_t>(256 / groups, 1), std::max<int64_t>(U / kWaves, 1));
    const int64_t mu = split_max_units(RT);
    S = std::max<int64_t>(S, (U + kWaves * mu - 1) / (kWaves * mu));
    return {std::min<int64_t>(S, kMaxSlices), RT};
}

size_t partials_bytes(int64_t M, int64_t K, int64_t N) {
    const int64_t S = std::max<int64_t>(decode_splits(M, K, N), reduce_plan(M, K, N).S);
    return round256((size_t)(S * M * N) * 4);
}

template <int WF, int RT>
int launch_split_product(const LinearArgs& a, const uint16_t* x3, float* part, int64_t S) {
    const dim3 grid((unsigned)((a.N + 31) / 32 / RT), (unsigned)((a.M + 31) / 32), (unsigned)S);
    const int64_t per_wave = ((a.K / 32 + S - 1) / S + kWaves - 1) / kWaves;
    if (per_wave <= 2)
        hipLaunchKernelGGL((split_product_kernel<WF, RT, 2>), grid, dim3(kWaves * 64), 0, a.stream, x3, (int)a.M,
                           (int)a.K, a.w, a.ldw, (int)a.N, part);
    else if (RT == 2 || per_wave <= kSplitMaxUnits)
        hipLaunchKernelGGL((split_product_kernel<WF, RT, kSplitMaxUnits>), grid, dim3(kWaves * 64), 0, a.stream, x3,
                           (int)a.M, (int)a.K, a.w, a.ldw, (int)a.N, part);
    else  // one tile a workgroup: up to kSplitMaxUnits1 units a wavefront
        hipLaunchKernelGGL((split_product_kernel<WF, 1, kSplitMaxUnits1>), grid, dim3(kWaves * 64), 0, a.stream, x3,
                           (int)a.M, (int)a.K, a.w, a.ldw, (int)a.N, part);
    return launch_status();
}

// plan.RT > 0: split_product_kernel with that many tiles a workgroup (int8
// weights, the reduction follows); else skinny_kernel (its own epilogue
// without `part`, raw partial slices with it)
template <int WF>
int run_decode_t(const LinearArgs& a, const uint16_t* x3, const float* next_ln_w, const float* next_ln_b,
                 float next_eps, uint16_t* planes_out, float* part, SplitPlan plan) {
    const int64_t S = plan.S;
    const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 31) / 32), (unsigned)S);
    const float* xp = reinterpret_cast<const float*>(x3);
    if (!part) {  // one split: the product kernel's own epilogue writes y and / or the planes
        hipLaunchKernelGGL((skinny_kernel<WF, kXPlanes, float>), grid, dim3(kWaves * 64), 0, a.stream, xp,
                           (int64_t)0, (int)a.M, (int)a.K, a.w, a.ldw, a.scale, a.bias, (int)a.N,
                           static_cast<float*>(a.y), a.ldy, nullptr, nullptr, 0.f, a.fuse.act, a.fuse.res,
                           a.fuse.ldr, nullptr, planes_out);
        return launch_status();
    }
    int rc = TIQ_OK;
    if constexpr (is_w8<WF>()) {
        if (plan.RT == 2) rc = launch_split_product<WF, 2>(a, x3, part, S);
        else if (plan.RT == 1) rc = launch_split_product<WF, 1>(a, x3, part, S);
    }
    if (plan.RT == 0) {
        hipLaunchKernelGGL((skinny_kernel<WF, kXPlanes, float>), grid, dim3(kWaves * 64), 0, a.stream, xp,
                           (int64_t)0, (int)a.M, (int)a.K, a.w, a.ldw, a.scale, a.bias, (int)a.N,
                           static_cast<float*>(nullptr), (int64_t)0, nullptr, nullptr, 0.f, 0, nullptr, (int64_t)0,
                           part, nullptr);
        rc = launch_status();
    }
    if (rc != TIQ_OK) return rc;
    const float* sc = is_w8<WF>() ? a.scale : nullptr;
    ReduceFn red = pick_reduce(next_ln_w != nullptr, planes_out != nullptr, sc != nullptr, a.bias != nullptr,
                               a.fuse.res != nullptr, a.N);
    hipLaunchKernelGGL(red, dim3((unsigned)a.M), dim3(red_threads(a.N)), 0, a.stream, part, (int64_t)a.N, (int)S,
                       (int)a.M, (int)a.N, sc, a.bias, a.fuse.act, a.fuse.res, a.fuse.ldr, static_cast<float*>(a.y),
                       a.ldy, next_ln_w, next_ln_b, next_eps, planes_out);
    return launch_status();
}

}  // namespace

size_t skinny_workspace(int64_t M, int64_t K) { return planes_bytes(M, K); }

size_t decode_linear_workspace(int64_t M, int64_t K, int64_t N) {
    return planes_bytes(M, K) + partials_bytes(M, K, N);
}

size_t decode_planes_bytes(int64_t M, int64_t K) { return planes_bytes(M, K); }

// fp32 tiles (the head): planes in, fp32 rows out, nothing fused
static int run_decode_f32_tiles(const LinearArgs& a, const uint16_t* x_planes, const float* next_ln_w,
                         uint16_t* planes_out) {
    if (a.M < 1 || a.M > 64 || a.K <= 0 || a.K % 32 != 0 || a.K / 32 < kWaves || a.N <= 0 || a.N > 0x7fffffff - 31)
        return TIQ_EUNSUPPORTED;
    if (!x_planes || a.bias || a.fuse.act || a.fuse.res || next_ln_w || planes_out) return TIQ_EUNSUPPORTED;
    if (!a.y || !a.w) return TIQ_EINVAL;
    if (!aligned(a.w, 16) || !aligned(x_planes, 16)) return TIQ_EALIGN;
    const int64_t T = (a.N + 31) / 32;
    const dim3 grid((unsigned)std::min<int64_t>(T, 256), (unsigned)((a.M + 31) / 32));
    hipLaunchKernelGGL(stream_f32_kernel, grid, dim3(kWaves * 64), 0, a.stream, x_planes, (int)a.M, (int)a.K, a.w,
                       (int)a.N, static_cast<float*>(a.y), a.ldy);
    return launch_status();
}

int run_decode_linear(const LinearArgs& a, const uint16_t* x_planes, const float* next_ln_w,
                      const float* next_ln_b, float next_eps, uint16_t* planes_out) {
    if (a.fmt == kF32T) return run_decode_f32_tiles(a, x_planes, next_ln_w, planes_out);
    if (a.fmt != kW8 && a.fmt != kW8T && a.fmt != kF32) return TIQ_EUNSUPPORTED;
    if (a.M < kSkinnyMinRows || a.M > 64 || a.K <= 0 || a.K % 32 != 0 || a.N <= 0 || a.N > 0x7fffffff)
        return TIQ_EUNSUPPORTED;
    if (a.fmt == kW8T && a.N % 32 != 0) return TIQ_EUNSUPPORTED;  // whole row tiles
    const bool w8 = a.fmt == kW8 || a.fmt == kW8T;
    if ((next_ln_w == nullptr) != (next_ln_b == nullptr) || (next_ln_w && !planes_out)) return TIQ_EINVAL;
    if (!a.y && !planes_out) return TIQ_EINVAL;
    // a row the reduction cannot take (N % 8, N > 8192) without planes out:
    // one split, the product kernel's own epilogue
    const bool red_ok = a.N % 8 == 0 && a.N <= kRedMaxCols;
    // LayerNorm'd planes or a residual after the product: the reduction kernel
    // runs whatever the split, so int8 products split to fill the GPU
    const bool must_reduce = planes_out && (next_ln_w || a.fuse.res || a.N % 32 != 0);
    SplitPlan plan{(red_ok || planes_out) ? decode_splits(a.M, a.K, a.N) : 1, 0};
    if (w8 && must_reduce && red_ok) {
        const SplitPlan p = reduce_plan(a.M, a.K, a.N);
        const int64_t per_wave = ((a.K / 32 + p.S - 1) / p.S + kWaves - 1) / kWaves;
        if (per_wave <= split_max_units(p.RT) && ((a.N + 31) / 32) % p.RT == 0) plan = p;
    }
    const int64_t S = plan.S;
    // planes without a LayerNorm or residual from one split: the product
    // kernel writes them itself (its 32 columns are one unit of the next
    // linear's K), no reduction launch
    const bool product_planes = planes_out && !next_ln_w && !a.fuse.res && S == 1 && a.N % 32 == 0;
    const bool reduce = !product_planes && (S > 1 || planes_out);
    // every wavefront's share of K fits its weight registers
    const int64_t units = ((a.K / 32 + S - 1) / S + kWaves - 1) / kWaves;
    if (plan.RT == 0 && units > (w8 ? max_units<kW8>() : max_units<kF32>())) return TIQ_EUNSUPPORTED;
    if (!aligned(a.w, 16) || a.ldw % 16 != 0) return TIQ_EALIGN;
    if (x_planes ? !aligned(x_planes, 16)
                 : (!a.x || !aligned(a.x, 16) || a.ldx % 4 != 0 ||
                    (a.fuse.ln_w && (!aligned(a.fuse.ln_w, 16) || !aligned(a.fuse.ln_b, 16)))))
        return x_planes || a.x ? TIQ_EALIGN : TIQ_EINVAL;
    if (product_planes &&
        (!aligned(planes_out, 16) || (a.y && (!aligned(a.y, 16) || a.ldy % 4 != 0)) ||
         (w8 && !aligned(a.scale, 16)) || (a.bias && !aligned(a.bias, 16))))
        return TIQ_EALIGN;
    if (reduce) {  // the reduction's 16-byte row accesses and its 8192-column reach
        if (a.N % 8 != 0 || a.N > kRedMaxCols) return TIQ_EUNSUPPORTED;
        if ((a.y && (!aligned(a.y, 16) || a.ldy % 4 != 0)) ||
            (a.fuse.res && (!aligned(a.fuse.res, 16) || a.fuse.ldr % 4 != 0)))
            return TIQ_EALIGN;
        if ((w8 && !aligned(a.scale, 16)) || (a.bias && !aligned(a.bias, 16))) return TIQ_EALIGN;
        if (planes_out && (!aligned(planes_out, 16) || a.N % 32 != 0)) return TIQ_EUNSUPPORTED;
    }
    if (a.fuse.res && a.fuse.res != a.y && a.fuse.ldr < a.N) return TIQ_EINVAL;
    const size_t need = (x_planes ? 0 : planes_bytes(a.M, a.K)) + (reduce ? partials_bytes(a.M, a.K, a.N) : 0);
    if (need && (!a.ws || a.ws_bytes < need || !aligned(a.ws, 16))) return TIQ_EWORKSPACE;
    uint8_t* ws = static_cast<uint8_t*>(a.ws);
    const uint16_t* x3 = x_planes;
    if (!x3) {
        uint16_t* xs = reinterpret_cast<uint16_t*>(ws);
        if (a.K <= kRedMaxCols) {  // LayerNorm + split: the reduction kernel with one slice, no epilogue
            ReduceFn f = pick_reduce(a.fuse.ln_w != nullptr, true, false, false, false, a.K);
            hipLaunchKernelGGL(f, dim3((unsigned)a.M), dim3(red_threads(a.K)), 0, a.stream,
                               static_cast<const float*>(a.x), a.ldx, 1, (int)a.M, (int)a.K, nullptr, nullptr, 0,
                               nullptr, (int64_t)0, nullptr, (int64_t)0, a.fuse.ln_w, a.fuse.ln_b, a.fuse.ln_eps, xs);
        } else if (a.fuse.ln_w) {
            hipLaunchKernelGGL(ln_split_kernel<true>, dim3((unsigned)a.M), dim3(256), 0, a.stream,
                               static_cast<const float*>(a.x), a.ldx, (int)a.K, a.fuse.ln_w, a.fuse.ln_b,
                               a.fuse.ln_eps, xs);
        } else {
            hipLaunchKernelGGL(ln_split_kernel<false>, dim3((unsigned)a.M), dim3(256), 0, a.stream,
                               static_cast<const float*>(a.x), a.ldx, (int)a.K, nullptr, nullptr, 0.f, xs);
        }
        int rc = launch_status();
        if (rc != TIQ_OK) return rc;
        x3 = xs;
        ws += planes_bytes(a.M, a.K);
    }
    float* part = reduce ? reinterpret_cast<float*>(ws) : nullptr;
    if (!part) plan.RT = 0;
    if (a.fmt == kW8) return run_decode_t<kW8>(a, x3, next_ln_w, next_ln_b, next_eps, planes_out, part, plan);
    if (a.fmt == kW8T) return run_decode_t<kW8T>(a, x3, next_ln_w, next_ln_b, next_eps, planes_out, part, plan);
    return run_decode_t<kF32>(a, x3, next_ln_w, next_ln_b, next_eps, planes_out, part, plan);
}

int64_t decode_slices_count(int64_t M, int64_t K, int64_t N) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    return slices_plan(M, K, N).S;
}

// every wavefront's share of K fits its registers within kMaxSlices splits
bool slices_fit(int64_t K, SplitPlan plan) {
    const int64_t per_wave = ((K / 32 + plan.S - 1) / plan.S + kWaves - 1) / kWaves;
    return per_wave <= split_max_units(plan.RT);
}

size_t decode_slices_bytes(int64_t M, int64_t K, int64_t N) {
    if (M <= 0 || M > 64 || K <= 0 || K % 32 != 0 || N <= 0) return 0;
    const SplitPlan plan = slices_plan(M, K, N);
    if (!slices_fit(K, plan)) return 0;
    return round256((size_t)(plan.S * M * N) * 4);
}

int launch_decode_slices(const LinearArgs& a, const uint16_t* x_planes, float* part) {
    if (a.fmt != kW8 && a.fmt != kW8T) return TIQ_EUNSUPPORTED;
    if (a.M < 1 || a.M > 64 || a.K <= 0 || a.K % 32 != 0 || a.N <= 0 || a.N > 0x7fffffff) return TIQ_EUNSUPPORTED;
    if (a.fmt == kW8T && a.N % 32 != 0) return TIQ_EUNSUPPORTED;  // whole row tiles
    if (!x_planes || !part || !a.w) return TIQ_EINVAL;
    if (a.fmt == kW8 && a.ldw < a.K) return TIQ_EINVAL;
    if (!aligned(a.w, 16) || a.ldw % 16 != 0 || !aligned(x_planes, 16) || !aligned(part, 16)) return TIQ_EALIGN;
    const SplitPlan plan = slices_plan(a.M, a.K, a.N);
    if (!slices_fit(a.K, plan)) return TIQ_EUNSUPPORTED;
    if (a.fmt == kW8T)
        return plan.RT == 2 ? launch_split_product<kW8T, 2>(a, x_planes, part, plan.S)
                            : launch_split_product<kW8T, 1>(a, x_planes, part, plan.S);
    return plan.RT == 2 ? launch_split_product<kW8, 2>(a, x_planes, part, plan.S)
                        : launch_split_product<kW8, 1>(a, x_planes, part, plan.S);
}

// One thread per 16 bytes of a tile: block b = (t, u) of (N / 32, K / 32),
// lane l = 32 h + r takes w[32 t + r][32 u + 16 h .. + 15].
__global__ __launch_bounds__(256) void tile_int8_kernel(const uint8_t* __restrict__ w, int64_t ldw, int64_t U,
                                                        int64_t nchunks, uint8_t* __restrict__ tiles) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nchunks) return;
    const int64_t b = i >> 6, t = b / U, u = b - t * U;
    const int l = (int)(i & 63), r = l & 31, h = l >> 5;
    const uint4 v = *reinterpret_cast<const uint4*>(w + (32 * t + r) * ldw + 32 * u + 16 * h);
    *reinterpret_cast<uint4*>(tiles + b * 1024 + l * 16) = v;
}

int launch_tile_int8(const uint8_t* w, int64_t N, int64_t K, int64_t ldw, uint8_t* tiles, hipStream_t stream) {
    if (N < 0 || K < 0) return TIQ_EINVAL;
    if (N == 0 || K == 0) return TIQ_OK;
    if (!w || !tiles || ldw < K) return TIQ_EINVAL;
    if (N % 32 != 0 || K % 32 != 0) return TIQ_EUNSUPPORTED;
    if (!aligned(w, 16) || !aligned(tiles, 16) || ldw % 16 != 0) return TIQ_EALIGN;
    const int64_t nchunks = N * K / 16;
    hipLaunchKernelGGL(tile_int8_kernel, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0, stream, w, ldw, K / 32,
                       nchunks, tiles);
    return launch_status();
}

// One thread per 16 bytes of the fp32 tiles: block b = (t, u) of
// (ceil(N / 32), K / 32), chunk c = 64 q + l of the block holds row 32 t + l % 32,
// columns 32 u + 16 (l / 32) + 4 q .. + 3 (zeros for rows past N).
__global__ __launch_bounds__(256) void tile_f32_kernel(const float* __restrict__ w, int64_t ldw, int64_t N,
                                                       int64_t U, int64_t nchunks, float* __restrict__ tiles) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nchunks) return;
    const int64_t b = i >> 8, t = b / U, u = b - t * U;
    const int c = (int)(i & 255), q = c >> 6, l = c & 63, r = l & 31, h = l >> 5;
    const int64_t row = 32 * t + r;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < N) v = *reinterpret_cast<const float4*>(w + row * ldw + 32 * u + 16 * h + 4 * q);
    reinterpret_cast<float4*>(tiles)[i] = v;
}

size_t tile_f32_bytes(int64_t N, int64_t K) {
    if (N <= 0 || K <= 0 || K % 32 != 0) return 0;
    return (size_t)((N + 31) / 32) * 32 * (size_t)K * 4;
}

int launch_tile_f32(const float* w, int64_t N, int64_t K, int64_t ldw, float* tiles, hipStream_t stream) {
    if (N < 0 || K < 0) return TIQ_EINVAL;
    if (N == 0 || K == 0) return TIQ_OK;
    if (!w || !tiles || ldw < K) return TIQ_EINVAL;
    if (K % 32 != 0) return TIQ_EUNSUPPORTED;
    if (!aligned(w, 16) || !aligned(tiles, 16) || ldw % 4 != 0) return TIQ_EALIGN;
    const int64_t nchunks = (int64_t)(tile_f32_bytes(N, K) / 16);
    hipLaunchKernelGGL(tile_f32_kernel, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0, stream, w, ldw, N,
                       K / 32, nchunks, tiles);
    return launch_status();
}

bool skinny_supported(const LinearArgs& a) {
    if (a.fmt != kW8 && a.fmt != kF32) return false;
    // bf16 rows: int8 weights, no LayerNorm, 16-byte rows
    const bool xbf = a.x_dtype == TIQ_BF16;
    if (xbf && (a.fmt != kW8 || a.fuse.ln_w || a.ldx % 8 != 0)) return false;
    // up to 16 bf16 rows against fewer than 2048 weight rows: too few 32-row
    // tiles to fill the chip (24 workgroups at N = 768); the decode GEMV's
    // direct kernel, tiled four activation rows at a time, is faster there
    if (xbf && a.M <= 16 && a.N < 2048) return false;
    if (!xbf && a.x_dtype != TIQ_F32) return false;
    if (a.M < kSkinnyMinRows || a.M > 64 || a.K % 32 != 0 || a.N > 0x7fffffff) return false;
    const int64_t units = (a.K / 32 + kWaves - 1) / kWaves;
    if (units > (xbf ? kXbUnits : a.fmt == kW8 ? max_units<kW8>() : max_units<kF32>())) return false;
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
