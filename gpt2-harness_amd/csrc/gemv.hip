// Decode GEMV on the vector ALUs (gfx950), for the reference's quantized
// Linears at decode time (model.py:254,319,352,355 with T = 1, M = batch):
//     y[m, n] = scale[n] * sum_k q[n, k] * x[m, k] + bias[n]
//
// The op is bound by the weight stream: N*K bytes of int8 (N*K/2 of int4)
// per call against 2-4*M*K bytes of activations; at decode sizes (0.6-10 MB)
// one launch is about one trip to HBM plus the launch itself. Two kernels:
//
// gemv_direct_kernel (up to 4 rows; the default, with the LayerNorm of fp32
// rows fused for up to 8192 weight rows, and for a tied fp32 head at one
// row): one wavefront per weight row (two or four at one row), every load of
// the workgroup issued before any is
// used -- the row's 16-byte chunks (8 bytes of nibbles for int4: 16 columns
// a lane whatever the format; nontemporal), the activations they multiply
// (straight into registers) and the epilogue operands -- then one
// FMA pass, a wavefront reduction and the store. Rows are dealt to the eight
// XCDs in contiguous blocks.
//
// gemv_kernel (LayerNorm prologue, group-wise int4, rows longer than the
// direct kernel's registers):
//   * a workgroup stages its MT activation rows in LDS once, as fp32 and in
//     "planes" (float4 p of every 16-byte weight chunk stored contiguously
//     over chunks), so lane l's reads of chunk l are consecutive 16-byte LDS
//     words: no bank conflicts;
//   * each wavefront owns R weight rows; lane l streams 16-byte chunks
//     l, l+64, ... of each row (nontemporal global_load_dwordx4, fully
//     coalesced: a wavefront instruction covers 1 KB of one row), four chunks
//     per row in flight, the first ones issued before the activations are
//     staged;
//   * the chunk is dequantized in registers (sign-extended bytes or biased
//     nibbles -> fp32, one v_cvt_f32_i32_sdwa per int8 code) once and reused
//     for all MT activation rows;
//   * per-row partial sums are reduced across the wavefront with DPP lane
//     moves; the per-channel scale and the bias are applied once per
//     output; the group-wise format scales each 32-column chunk's partial sum
//     by its group's fp16 scale.
// gemv_rows16_kernel (4..16 bf16 rows, int8 weights): 16 (or 8, 4) weight
// rows a workgroup on the matrix cores, so the activations are read once per
// block of rows instead of once per row; see the kernel.
//
// Optional fusions for the decode step of a GPT-2 block (model.py:410-427):
// LayerNorm of the staged activation rows (two-pass mean / variance over the
// row held in LDS), GELU(tanh) of the output (model.py:57-75) and a residual
// added to it (x + f(x)), so one launch replaces LayerNorm + Linear + GELU or
// Linear + add. The fp32 weight format serves the unquantized tied lm_head.
// The first two kernels use no MFMA: at M <= 4 the int8->fp32 convert plus M
// FMAs per weight byte stay within the VALU budget of the HBM stream.
#include "tiq_internal.hpp"

namespace tiq {
namespace {

constexpr int kWavesPerBlock = 8;
constexpr int kThreads = kWavesPerBlock * 64;

template <int FMT>
struct Fmt {
    // columns per 16-byte weight chunk
    static constexpr int KC = (FMT == kW8) ? 16 : (FMT == kF32) ? 4 : 32;
};

// The direct kernel's chunk: 16 bytes (16 int8 / 4 fp32 columns), but 8 bytes
// (16 columns) of nibbles, so that an int4 lane carries the activations (and
// LayerNorm operands) of 16 columns, as an int8 lane does, rather than 32:
// twice the lanes each with half the loads and arithmetic on a row.
template <int FMT>
constexpr int direct_kc() { return FMT == kW4 ? 16 : Fmt<FMT>::KC; }
template <int FMT>
constexpr int direct_chunk_bytes() { return FMT == kW4 ? 8 : 16; }

template <typename TX>
__device__ __forceinline__ float4 load_x4(const TX* p);

template <>
__device__ __forceinline__ float4 load_x4<float>(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

template <>
__device__ __forceinline__ float4 load_x4<uint16_t>(const uint16_t* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}

template <typename TY>
__device__ __forceinline__ void store_y(TY* p, float v);

template <>
__device__ __forceinline__ void store_y<float>(float* p, float v) {
    *p = v;
}

template <>
__device__ __forceinline__ void store_y<uint16_t>(uint16_t* p, float v) {
    *p = f32_to_bf16_bits(v);
}

// sum over the 16 columns of an int8 chunk
__device__ __forceinline__ float dot_w8(const uint4& w, const float4* xv) {
    float s = 0.f;
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 xx = xv[j];
        s = fmaf(sbyte_f32<0>(d[j]), xx.x, s);
        s = fmaf(sbyte_f32<1>(d[j]), xx.y, s);
        s = fmaf(sbyte_f32<2>(d[j]), xx.z, s);
        s = fmaf(sbyte_f32<3>(d[j]), xx.w, s);
    }
    return s;
}

// sum over the 32 columns of a nibble chunk (low nibble = even column)
__device__ __forceinline__ float dot_w4(const uint4& w, const float4* xv) {
    float s = 0.f;
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 a = xv[2 * j], b = xv[2 * j + 1];
        s = fmaf(nibble_f32<0>(d[j]), a.x, s);
        s = fmaf(nibble_f32<1>(d[j]), a.y, s);
        s = fmaf(nibble_f32<2>(d[j]), a.z, s);
        s = fmaf(nibble_f32<3>(d[j]), a.w, s);
        s = fmaf(nibble_f32<4>(d[j]), b.x, s);
        s = fmaf(nibble_f32<5>(d[j]), b.y, s);
        s = fmaf(nibble_f32<6>(d[j]), b.z, s);
        s = fmaf(nibble_f32<7>(d[j]), b.w, s);
    }
    return s;
}

// sum over the 16 columns of an 8-byte nibble chunk (w.x, w.y). A nibble n
// moved into the high half of a byte with that byte's top bit flipped is the
// signed byte 16 (n - 8), which becomes a float in one instruction; every
// product and partial sum is then exactly 16 times the one of n - 8 (a power
// of two), and the sum is scaled back once: the same result as converting
// n - 8 directly, in the same column order.
__device__ __forceinline__ float dot_w4h(const uint4& w, const float4* xv) {
    float s = 0.f;
    const uint32_t d[2] = {w.x, w.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float4 a = xv[2 * j], b = xv[2 * j + 1];
        const uint32_t e = ((d[j] << 4) & 0xf0f0f0f0u) ^ 0x80808080u;  // even columns (low nibbles)
        const uint32_t o = (d[j] & 0xf0f0f0f0u) ^ 0x80808080u;         // odd columns
        s = fmaf(sbyte_f32<0>(e), a.x, s);
        s = fmaf(sbyte_f32<0>(o), a.y, s);
        s = fmaf(sbyte_f32<1>(e), a.z, s);
        s = fmaf(sbyte_f32<1>(o), a.w, s);
        s = fmaf(sbyte_f32<2>(e), b.x, s);
        s = fmaf(sbyte_f32<2>(o), b.y, s);
        s = fmaf(sbyte_f32<3>(e), b.z, s);
        s = fmaf(sbyte_f32<3>(o), b.w, s);
    }
    return s * 0.0625f;
}

// sum over the 4 columns of an fp32 chunk
__device__ __forceinline__ float dot_f32(const uint4& w, const float4* xv) {
    const float4 xx = xv[0];
    float s = __uint_as_float(w.x) * xx.x;
    s = fmaf(__uint_as_float(w.y), xx.y, s);
    s = fmaf(__uint_as_float(w.z), xx.z, s);
    return fmaf(__uint_as_float(w.w), xx.w, s);
}

template <int FMT>
__device__ __forceinline__ float dot_chunk(const uint4& w, const float4* xv) {
    if constexpr (FMT == kW8) return dot_w8(w, xv);
    else if constexpr (FMT == kF32) return dot_f32(w, xv);
    else return dot_w4(w, xv);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Bijective map of a workgroup index so that XCD b % 8 (where the hardware
// places workgroup b) owns a contiguous range of the G workgroups.
__device__ __forceinline__ int xcd_block(int b, int G) {
    const int q = G >> 3, r = G & 7, xcd = b & 7, idx = b >> 3;
    return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + idx;
}

// Sum of v over the workgroup, for MT rows at once. red holds MT * 8 floats.
template <int MT>
__device__ __forceinline__ void block_sum(float (&v)[MT], float* red) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float s = wave_sum_dpp(v[m]);
        if (lane == 0) red[m * kWavesPerBlock + wave] = s;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kWavesPerBlock; ++i) s += red[m * kWavesPerBlock + i];
        v[m] = s;
    }
    __syncthreads();
}

template <int MT, int R, int FMT, typename TX, typename TY>
__global__ __launch_bounds__(kThreads) void gemv_kernel(
    const TX* __restrict__ x, int64_t ldx, int M, const uint8_t* __restrict__ w, int64_t ldw,
    const float* __restrict__ scale, const uint16_t* __restrict__ scale16, int group,
    const float* __restrict__ bias, TY* y, int64_t ldy, int N, int K, Fusion fz) {
    constexpr int KC = Fmt<FMT>::KC;
    constexpr int P = KC / 4;  // float4 planes per chunk
    constexpr int U = 4;       // chunks per row in flight per lane
    extern __shared__ float4 xs[];
    __shared__ float red[MT * kWavesPerBlock];
    const int K4 = K >> 2;
    const int NC = K / KC;
    const int m0 = blockIdx.y * MT;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n0 = (xcd_block(blockIdx.x, gridDim.x) * kWavesPerBlock + wave) * R;
    const bool active = n0 < N;  // wave-uniform

    const uint8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = w + (int64_t)((n0 + r < N) ? n0 + r : (active ? n0 : 0)) * ldw;

    // weight chunks c0 + 64u of every row, zero past the end of the row
    uint4 wv[U][R];
    auto load_block = [&](int c0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
#pragma unroll
            for (int r = 0; r < R; ++r)
            {
                // nontemporal: the weights are read once
                const u32x4 t = (c < NC) ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[r] + 16 * (int64_t)c))
                                         : u32x4{0u, 0u, 0u, 0u};
                wv[u][r] = make_uint4(t.x, t.y, t.z, t.w);
            }
        }
    };
    // The first weight block goes out before the activations are staged, so
    // its HBM latency overlaps the staging and the barrier.
    if (active) load_block(lane);

    // The epilogue operands of the output this lane stores (lane r * MT + m
    // stores row n0 + r of activation row m0 + m) are loaded now as well:
    // loaded after the reduction they would cost a second, serial trip to
    // HBM. A residual that aliases y is read here by the lane that later
    // writes the same element, so the early read is safe.
    float ep_scale = 1.f, ep_bias = 0.f, ep_res = 0.f;
    {
        const int r = lane / MT, m = lane - (lane / MT) * MT;
        const int n = n0 + r;
        if (active && r < R && n < N && m0 + m < M) {
            if (FMT == kW8 || FMT == kW4) ep_scale = scale[n];
            if (bias) ep_bias = bias[n];
            if (fz.res) ep_res = fz.res[(int64_t)(m0 + m) * fz.ldr + n];
        }
    }

    // LayerNorm weight and bias of the columns this thread normalizes
    // (k4 = tid, tid + kThreads; rows up to 8 * kThreads columns), requested
    // with the weights so the normalize pass does not wait on them
    constexpr int kLnPre = 2;
    const bool ln_pre = fz.ln_w && K4 <= kLnPre * kThreads;
    float4 gpre[kLnPre], bpre[kLnPre];
    if (ln_pre) {
#pragma unroll
        for (int j = 0; j < kLnPre; ++j) {
            const int k4 = min((int)threadIdx.x + kThreads * j, K4 - 1);
            gpre[j] = reinterpret_cast<const float4*>(fz.ln_w)[k4];
            bpre[j] = reinterpret_cast<const float4*>(fz.ln_b)[k4];
        }
    }

    // stage MT activation rows as fp32 planes: xs[m][p][c]
    float rsum[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) rsum[m] = 0.f;
    for (int t = threadIdx.x; t < MT * K4; t += blockDim.x) {
        const int m = t / K4, k4 = t - m * K4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m0 + m < M) v = load_x4<TX>(x + (int64_t)(m0 + m) * ldx + 4 * k4);
        const int c = k4 / P, p = k4 - c * P;
        xs[m * K4 + p * NC + c] = v;
#pragma unroll
        for (int mm = 0; mm < MT; ++mm)
            if (mm == m) rsum[mm] += (v.x + v.y) + (v.z + v.w);
    }
    if (fz.ln_w) {
        // LayerNorm over each staged row: mean, then the mean squared
        // deviation (biased, as torch), then normalise in place.
        block_sum<MT>(rsum, red);
        float mean[MT], dev[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            mean[m] = rsum[m] / (float)K;
            dev[m] = 0.f;
        }
        for (int t = threadIdx.x; t < MT * K4; t += blockDim.x) {
            const int m = t / K4, k4 = t - m * K4;
            const int c = k4 / P, p = k4 - c * P;
            const float4 v = xs[m * K4 + p * NC + c];
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) {
                if (mm == m) {
                    const float a = v.x - mean[mm], b = v.y - mean[mm], cc = v.z - mean[mm], d = v.w - mean[mm];
                    dev[mm] += (a * a + b * b) + (cc * cc + d * d);
                }
            }
        }
        block_sum<MT>(dev, red);
        float rstd[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) rstd[m] = 1.0f / sqrtf(dev[m] / (float)K + fz.ln_eps);
        if (ln_pre) {
#pragma unroll
            for (int j = 0; j < kLnPre; ++j) {
                const int k4 = (int)threadIdx.x + kThreads * j;
                if (k4 >= K4) break;
                const int c = k4 / P, p = k4 - c * P;
                const float4 g = gpre[j], b = bpre[j];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float4 v = xs[m * K4 + p * NC + c];
                    v.x = (v.x - mean[m]) * rstd[m] * g.x + b.x;
                    v.y = (v.y - mean[m]) * rstd[m] * g.y + b.y;
                    v.z = (v.z - mean[m]) * rstd[m] * g.z + b.z;
                    v.w = (v.w - mean[m]) * rstd[m] * g.w + b.w;
                    if (m0 + m >= M) v = make_float4(0.f, 0.f, 0.f, 0.f);
                    xs[m * K4 + p * NC + c] = v;
                }
            }
        }
        for (int t = ln_pre ? MT * K4 : threadIdx.x; t < MT * K4; t += blockDim.x) {
            const int m = t / K4, k4 = t - m * K4;
            const int c = k4 / P, p = k4 - c * P;
            float4 v = xs[m * K4 + p * NC + c];
            float mu = 0.f, rs = 0.f;
#pragma unroll
            for (int mm = 0; mm < MT; ++mm)
                if (mm == m) {
                    mu = mean[mm];
                    rs = rstd[mm];
                }
            const float4 g = *reinterpret_cast<const float4*>(fz.ln_w + 4 * k4);
            const float4 b = *reinterpret_cast<const float4*>(fz.ln_b + 4 * k4);
            v.x = (v.x - mu) * rs * g.x + b.x;
            v.y = (v.y - mu) * rs * g.y + b.y;
            v.z = (v.z - mu) * rs * g.z + b.z;
            v.w = (v.w - mu) * rs * g.w + b.w;
            if (m0 + m >= M) v = make_float4(0.f, 0.f, 0.f, 0.f);
            xs[m * K4 + p * NC + c] = v;
        }
    }
    __syncthreads();
    if (!active) return;  // after the last barrier

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

    const int ng = (FMT == kW4G) ? (K + group - 1) / group : 0;
    for (int c0 = lane; c0 < NC; c0 += 64 * U) {
        uint4 cur[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) cur[u][r] = wv[u][r];
        if (c0 + 64 * U < NC) load_block(c0 + 64 * U);  // next block in flight during this one's math
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
            if (c >= NC) break;
            float gs[R];
            if (FMT == kW4G) {
                const int g = (c * KC) / group;
#pragma unroll
                for (int r = 0; r < R; ++r)
                    gs[r] = f16_bits_to_f32(scale16[(int64_t)((n0 + r < N) ? n0 + r : n0) * ng + g]);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float4 xv[P];
#pragma unroll
                for (int p = 0; p < P; ++p) xv[p] = xs[m * K4 + p * NC + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float part = dot_chunk<FMT>(cur[u][r], xv);
                    if (FMT == kW4G) acc[r][m] = fmaf(gs[r], part, acc[r][m]);
                    else acc[r][m] += part;
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = wave_sum_dpp(acc[r][m]);

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = n0 + r;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (lane == r * MT + m && n < N && m0 + m < M) {
                float v = acc[r][m];
                if (FMT == kW8 || FMT == kW4) v *= ep_scale;
                if (bias) v += ep_bias;
                v = apply_act(v, fz.act);
                if (fz.res) v += ep_res;
                store_y<TY>(y + (int64_t)(m0 + m) * ldy + n, v);
            }
        }
    }
}

// Direct decode GEMV (no LayerNorm prologue, int8 / int4 / fp32 weights).
// At decode sizes (0.6-10 MB per matrix) a launch costs about one trip to
// HBM plus the launch itself, so this kernel is built to make that trip once:
//   * one wavefront per workgroup, one weight row per wavefront; lane l holds
//     16-byte chunks l, l + 64, ... of the row (UM of them at most);
//   * every load is issued before any is used: the row's chunks
//     (nontemporal: the stream is read once and must not evict what is
//     reused), the activations those chunks multiply (16-32 bytes per chunk
//     and row, straight into registers, no LDS staging and no barrier), and
//     the lane's epilogue operands (scale, bias, residual);
//   * rows are handed to the eight XCDs in contiguous blocks (the hardware
//     deals workgroups round-robin over XCDs), so a 128-byte line of scales or
//     biases is fetched into one XCD's L2 rather than into all eight;
//   * the lane partial sums are reduced across the wavefront with DPP lane
//     moves; lane m stores output (m0 + m, n).
template <typename TX>
__device__ __forceinline__ float4 x4_of(const u32x4& u, int half);

template <>
__device__ __forceinline__ float4 x4_of<uint16_t>(const u32x4& u, int half) {
    const uint32_t a = half ? u.z : u.x, b = half ? u.w : u.y;
    return make_float4(__uint_as_float(a << 16), __uint_as_float(a & 0xffff0000u), __uint_as_float(b << 16),
                       __uint_as_float(b & 0xffff0000u));
}

template <>
__device__ __forceinline__ float4 x4_of<float>(const u32x4& u, int) {
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}

// R weight rows per wavefront (1 or 2) share the activation registers.
// STAMP: the measurement copy (per-workgroup entry / exit times to `stamp`).
template <int MT, int UM, int R, int FMT, typename TX, typename TY, bool LNF, bool STAMP = false>
// The arguments up to M fill the 14 dwords the hardware preloads into SGPRs
// at wave launch (built with kernarg preloading), so the first loads wait on
// no kernarg fetch; the grid size is passed rather than read from the
// dispatch's hidden arguments. The rest is fetched while the weights are in
// flight.
__global__ __launch_bounds__(64) void gemv_direct_kernel(const uint8_t* __restrict__ w,
                                                         const TX* __restrict__ x,
                                                         const float* __restrict__ scale, TY* y, int ldw, int ldx,
                                                         int N, int K, int G, int M, int ldy,
                                                         const float* __restrict__ bias, Fusion fz,
                                                         uint64_t* stamp) {
    Stamp<STAMP> clock;
    clock.start();
    constexpr int KC = direct_kc<FMT>();
    constexpr int CB = direct_chunk_bytes<FMT>();
    constexpr int P = KC / 4;                          // float4 of activations per chunk
    constexpr int XB = KC * (int)sizeof(TX);           // activation bytes per chunk and row
    constexpr int XQ = XB >= 16 ? XB / 16 : 1;         // 16-byte registers holding them
    const int lane = threadIdx.x;
    const int n0 = xcd_block(blockIdx.x, G) * R;  // rows n0 .. n0 + R - 1; past N: row N - 1, not stored
    const int m0 = blockIdx.y * MT;
    const int NC = K / KC;

    // No load sits behind a branch: a lane past the end of the row re-reads
    // the row's last chunk (its product is dropped below; the repeats
    // coalesce into one request). Loads under a branch get merged with their
    // alternative through register moves, which wait for every load issued
    // before them and so serialize the trips to memory.
    u32x4 wv[UM][R];
    auto load_weights = [&]() {
#pragma unroll
        for (int u = 0; u < UM; ++u) {
            const int c = min(lane + 64 * u, NC - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t* src = w + (int64_t)min(n0 + r, N - 1) * ldw + CB * (int64_t)c;
                if constexpr (CB == 8) {
                    const u32x2 h = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src));
                    wv[u][r] = u32x4{h.x, h.y, 0u, 0u};
                } else {
                    wv[u][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                }
            }
        }
    };
    // With a LayerNorm the activations are requested first: a wavefront's
    // loads complete in order, so the statistics (which need only the
    // activations) are computed while the weights are still in flight.
    if constexpr (!LNF) load_weights();
    // activations of the same K range: rows past M repeat row M - 1 (their
    // outputs are not stored)
    u32x4 xv[UM][MT][XQ];
#pragma unroll
    for (int u = 0; u < UM; ++u) {
        const int c = min(lane + 64 * u, NC - 1);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const TX* xr = x + (int64_t)min(m0 + m, M - 1) * ldx + (int64_t)KC * c;
#pragma unroll
            for (int q = 0; q < XQ; ++q) {
                if constexpr (XB >= 16) {
                    xv[u][m][q] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(xr) + 16 * q);
                } else {  // fp32 weights with bf16 activations: 8 bytes
                    const uint2 h = *reinterpret_cast<const uint2*>(xr);
                    xv[u][m][q] = u32x4{h.x, h.y, 0u, 0u};
                }
            }
        }
    }
    if constexpr (LNF) {
        __builtin_amdgcn_sched_barrier(0);
        load_weights();
        __builtin_amdgcn_sched_barrier(0);  // nothing that waits on the argument fetch ahead of them
    }
    // LayerNorm weight and bias of the lane's columns
    float4 gv[LNF ? UM : 1][P], bv[LNF ? UM : 1][P];
    if constexpr (LNF) {
#pragma unroll
        for (int u = 0; u < UM; ++u) {
            const int c = min(lane + 64 * u, NC - 1);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                gv[u][p] = reinterpret_cast<const float4*>(fz.ln_w + (int64_t)KC * c)[p];
                bv[u][p] = reinterpret_cast<const float4*>(fz.ln_b + (int64_t)KC * c)[p];
            }
        }
    }
    // epilogue operands, read by every lane (lane r MT + m keeps those of
    // weight row n0 + r and activation row m0 + m); a residual aliasing y is
    // read by the lane that writes the element
    const int en = min(n0 + min(lane / MT, R - 1), N - 1), em = min(m0 + lane % MT, M - 1);
    const float ep_scale = (FMT == kW8 || FMT == kW4) ? scale[en] : 1.f;
    const float ep_bias = bias ? bias[en] : 0.f;
    float ep_res = 0.f;
    if (fz.res) ep_res = fz.res[(int64_t)em * fz.ldr + en];

    auto x_of = [&](int u, int m, int p) -> float4 {
        if constexpr (sizeof(TX) == 2) return x4_of<TX>(xv[u][m][p / 2], p % 2);
        else return x4_of<TX>(xv[u][m][p], 0);
    };
    // LayerNorm statistics: between them the lanes hold the whole row, so the
    // mean and then the mean squared deviation (biased, as torch) are two
    // wavefront sums over the lanes' own chunks
    float mean[MT], rstd[MT];
    if constexpr (LNF) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float t = 0.f;
#pragma unroll
            for (int u = 0; u < UM; ++u) {
                float cs = 0.f;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const float4 v = x_of(u, m, p);
                    cs += (v.x + v.y) + (v.z + v.w);
                }
                t += lane + 64 * u < NC ? cs : 0.f;
            }
            mean[m] = wave_sum_dpp(t) / (float)K;
            float d = 0.f;
#pragma unroll
            for (int u = 0; u < UM; ++u) {
                float cs = 0.f;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const float4 v = x_of(u, m, p);
                    const float a = v.x - mean[m], b = v.y - mean[m], c = v.z - mean[m], e = v.w - mean[m];
                    cs += (a * a + b * b) + (c * c + e * e);
                }
                d += lane + 64 * u < NC ? cs : 0.f;
            }
            rstd[m] = 1.0f / sqrtf(wave_sum_dpp(d) / (float)K + fz.ln_eps);
        }
    }
    // Keep the epilogue loads in the shadow of the weight loads: left to
    // itself the compiler sinks them into the storing lane's branch, one more
    // trip to memory after the reduction. Pinned after the LayerNorm
    // statistics (an operand of the pin, so that it is not hoisted above
    // them), which so need not wait for the weights; the FMA pass waits for
    // them anyway.
    if constexpr (LNF) asm volatile("" ::"v"(ep_scale), "v"(ep_bias), "v"(ep_res), "v"(rstd[MT - 1]));
    else asm volatile("" ::"v"(ep_scale), "v"(ep_bias), "v"(ep_res));

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
#pragma unroll
    for (int u = 0; u < UM; ++u) {
        const bool own = lane + 64 * u < NC;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float4 xf[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                xf[p] = x_of(u, m, p);
                if constexpr (LNF) {
                    const float4 g = gv[u][p], b = bv[u][p];
                    xf[p].x = (xf[p].x - mean[m]) * rstd[m] * g.x + b.x;
                    xf[p].y = (xf[p].y - mean[m]) * rstd[m] * g.y + b.y;
                    xf[p].z = (xf[p].z - mean[m]) * rstd[m] * g.z + b.z;
                    xf[p].w = (xf[p].w - mean[m]) * rstd[m] * g.w + b.w;
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint4 wc = make_uint4(wv[u][r].x, wv[u][r].y, wv[u][r].z, wv[u][r].w);
                float part;
                if constexpr (FMT == kW4) part = dot_w4h(wc, xf);
                else part = dot_chunk<FMT>(wc, xf);
                acc[r][m] += own ? part : 0.f;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = wave_sum_dpp(acc[r][m]);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (lane == r * MT + m && n0 + r < N && m0 + m < M) {
                float v = acc[r][m] * ep_scale + ep_bias;
                v = apply_act(v, fz.act);
                if (fz.res) v += ep_res;
                store_y<TY>(y + (int64_t)(m0 + m) * ldy + n0 + r, v);
            }
        }
    clock.finish(stamp, (int64_t)blockIdx.y * G + blockIdx.x);
}

// Decode GEMV on the matrix cores for 2..16 bf16 activation rows and int8
// weights: a workgroup takes 16 weight rows and every activation row, so the
// activations are read once per 16 weight rows (the direct kernel reads them
// once per row); its W wavefronts split K into runs of `pw` 64-column pairs.
// For pair p a lane holds the 16 weight bytes of row n0 + l % 16 and the 16
// bf16 of activation row l % 16 at columns 64 p + 16 (l / 16) .. + 15: two
// v_mfma_f32_16x16x32_bf16, A = activations, B = weights (both operands
// take a lane's 8 values from the same columns, so the pairing of columns
// needs no particular order inside the instruction; an int8 code is exact in
// bf16, every product is exact, fp32 sums). Loads go through buffer
// descriptors sized to the 16 weight rows and the M activation rows: a row
// past N or M, or a pair past the wavefront's run, reads zero with no memory
// access and adds exact zeros, so no load is clamped or branched around.
// Lane l ends with D[4 (l / 16) + q][l % 16], q = 0..3 (activation row,
// weight row); the W partial tiles meet in LDS and one thread per output
// sums them in wavefront order and applies scale, bias, activation and
// residual.
typedef __bf16 r16_bf16x8 __attribute__((ext_vector_type(8)));
typedef float r16_floatx4 __attribute__((ext_vector_type(4)));

template <int W, int UP, typename TY>
__global__ __launch_bounds__(64 * W) void gemv_rows16_kernel(const uint8_t* __restrict__ w,
                                                            const uint16_t* __restrict__ x,
                                                            const float* __restrict__ scale, TY* y, int ldw, int ldx,
                                                            int N, int K, int G, int M, int ldy, int pw, int rb,
                                                            const float* __restrict__ bias, Fusion fz) {
    static_assert(W >= 4, "one epilogue thread per output of the 16 x 16 tile");
    __shared__ r16_floatx4 part[W][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int n0 = xcd_block(blockIdx.x, G) * rb;  // weight rows n0 .. n0 + rows - 1
    const int rows = min(rb, N - n0);
    // bytes each descriptor covers; an offset at or past them reads zero (the
    // host keeps both below 2^31 - 256, so offset + 16 does not wrap)
    const int wbytes = (rows - 1) * ldw + K, xbytes = ((M - 1) * ldx + K) * 2;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w) + (int64_t)n0 * ldw, (short)0, wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, xbytes, 0x00020000);
    const int first = wave * pw, cnt = min(pw, K / 64 - first);  // this wavefront's pairs
    u32x4 wq[UP], xa[UP][2];
#pragma unroll
    for (int j = 0; j < UP; ++j) {
        const int k0 = 64 * (first + j) + 16 * g;
        wq[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, j < cnt ? r * ldw + k0 : wbytes, 0, 2);  // nontemporal
    }
#pragma unroll
    for (int j = 0; j < UP; ++j) {
        const int xo = j < cnt ? (r * ldx + 64 * (first + j) + 16 * g) * 2 : xbytes;
        xa[j][0] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        xa[j][1] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
    }
    // epilogue operands of this thread's output (row m = tid / 16, weight row
    // n0 + tid % 16), requested beside the tiles
    const int em = min(tid >> 4, M - 1), en = min(n0 + (tid & 15), N - 1);
    const float ep_scale = scale[en];
    const float ep_bias = bias ? bias[en] : 0.f;
    float ep_res = 0.f;
    if (fz.res) ep_res = fz.res[(int64_t)em * fz.ldr + en];
    asm volatile("" ::"v"(ep_scale), "v"(ep_bias), "v"(ep_res));

    r16_floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < UP; ++j) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint32_t d0 = s ? wq[j].z : wq[j].x, d1 = s ? wq[j].w : wq[j].y;
            const u32x4 b = {bf16x2_of_bytes_perm(d0, 0), bf16x2_of_bytes_perm(d0, 16), bf16x2_of_bytes_perm(d1, 0),
                             bf16x2_of_bytes_perm(d1, 16)};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(r16_bf16x8, xa[j][s]),
                                                          __builtin_bit_cast(r16_bf16x8, b), acc, 0, 0, 0);
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (tid < 256) {
        const int m = tid >> 4, n = tid & 15;
        const float* pf = reinterpret_cast<const float*>(part);
        const int at = (16 * (m >> 2) + n) * 4 + (m & 3);  // lane 16 (m / 4) + n, register m % 4
        float sum = 0.f;
#pragma unroll
        for (int v = 0; v < W; ++v) sum += pf[v * 256 + at];
        if (m < M && n < rows) {
            float o = sum * ep_scale + ep_bias;
            o = apply_act(o, fz.act);
            if (fz.res) o += ep_res;
            store_y<TY>(y + (int64_t)m * ldy + n0 + n, o);
        }
    }
}

// Fallback for any shape or alignment: one wavefront per output (m, n),
// scalar loads.
template <int FMT, typename TX, typename TY>
__global__ __launch_bounds__(256) void gemv_generic(const TX* __restrict__ x, int64_t ldx, int M,
                                                    const uint8_t* __restrict__ w, int64_t ldw,
                                                    const float* __restrict__ scale,
                                                    const uint16_t* __restrict__ scale16, int group,
                                                    const float* __restrict__ bias, TY* __restrict__ y,
                                                    int64_t ldy, int N, int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= (int64_t)M * N) return;
    const int m = (int)(o / N), n = (int)(o % N);
    const uint8_t* wr = w + (int64_t)n * ldw;
    const int64_t ng = (K + group - 1) / group;
    float s = 0.f;
    for (int64_t k = lane; k < K; k += 64) {
        float xv;
        if constexpr (sizeof(TX) == 4) xv = x[(int64_t)m * ldx + k];
        else xv = bf16_bits_to_f32(x[(int64_t)m * ldx + k]);
        float wv;
        if (FMT == kW8) {
            wv = (float)(int8_t)wr[k];
        } else if (FMT == kF32) {
            wv = reinterpret_cast<const float*>(wr)[k];
        } else {
            const uint8_t b = wr[k >> 1];
            wv = (float)((int)((k & 1) ? (b >> 4) : (b & 0xf)) - 8);
            if (FMT == kW4G) wv *= f16_bits_to_f32(scale16[(int64_t)n * ng + k / group]);
        }
        s = fmaf(wv, xv, s);
    }
    s = wave_sum(s);
    if (lane == 0) {
        if (FMT == kW8 || FMT == kW4) s *= scale[n];
        if (bias) s += bias[n];
        store_y<TY>(y + (int64_t)m * ldy + n, s);
    }
}

constexpr size_t kMaxLds = 64 * 1024;

template <int MT, int R, int FMT, typename TX, typename TY>
int run_gemv(const LinearArgs& a) {
    const int N = (int)a.N, K = (int)a.K, M = (int)a.M;
    const size_t lds = (size_t)MT * K * sizeof(float);
    const dim3 grid((unsigned)((N + kWavesPerBlock * R - 1) / (kWavesPerBlock * R)), (unsigned)((M + MT - 1) / MT));
    hipLaunchKernelGGL((gemv_kernel<MT, R, FMT, TX, TY>), grid, dim3(kThreads), lds, a.stream,
                       static_cast<const TX*>(a.x), a.ldx, M, a.w, a.ldw, a.scale, a.scale16, a.group, a.bias,
                       static_cast<TY*>(a.y), a.ldy, N, K, a.fuse);
    return launch_status();
}

// Activation registers of the direct kernel: UM chunks x MT rows x XQ x 4
// VGPRs, kept within 128 so that weights, activations and sums all fit.
template <int MT, int UM, int FMT, typename TX, bool LNF>
constexpr bool direct_fits() {
    constexpr int XB = direct_kc<FMT>() * (int)sizeof(TX);
    // with LayerNorm: fp32 activations, plus the LayerNorm weight and bias of
    // the lane's columns (2 x KC VGPRs a chunk)
    if constexpr (LNF) {
        if (sizeof(TX) != 4) return false;
        return UM * (MT * (XB / 16) * 4 + 2 * direct_kc<FMT>()) <= 160;
    }
    return UM * MT * (XB >= 16 ? XB / 16 : 1) * 4 <= 128;
}

template <int MT, int UM, int R, int FMT, typename TX, typename TY, bool LNF>
bool run_direct(const LinearArgs& a, int& rc) {
    if constexpr (direct_fits<MT, UM, FMT, TX, LNF>()) {
        const int G = (int)((a.N + R - 1) / R);
        const dim3 grid((unsigned)G, (unsigned)((a.M + MT - 1) / MT));
        // int8 weights with bf16 in and out have a stamped copy for measurement
        if constexpr (FMT == kW8 && sizeof(TX) == 2 && sizeof(TY) == 2 && !LNF) {
            if (uint64_t* sp = stamp_slots((int64_t)grid.x * grid.y)) {
                hipLaunchKernelGGL((gemv_direct_kernel<MT, UM, R, FMT, TX, TY, LNF, true>), grid, dim3(64), 0,
                                   a.stream, a.w, static_cast<const TX*>(a.x), a.scale, static_cast<TY*>(a.y),
                                   (int)a.ldw, (int)a.ldx, (int)a.N, (int)a.K, G, (int)a.M, (int)a.ldy, a.bias,
                                   a.fuse, sp);
                rc = launch_status();
                return true;
            }
        }
        hipLaunchKernelGGL((gemv_direct_kernel<MT, UM, R, FMT, TX, TY, LNF>), grid, dim3(64), 0, a.stream, a.w,
                           static_cast<const TX*>(a.x), a.scale, static_cast<TY*>(a.y), (int)a.ldw, (int)a.ldx,
                           (int)a.N, (int)a.K, G, (int)a.M, (int)a.ldy, a.bias, a.fuse, nullptr);
        rc = launch_status();
        return true;
    }
    return false;
}

// Weight rows up to which a wavefront of the direct kernel reads the whole
// activation row and its LayerNorm weight and bias for one or two weight
// rows; above it only a head at one row (four or eight rows a wavefront).
constexpr int64_t kDirectLnMaxRows = 8192;

template <int UM, int FMT, typename TX, typename TY, bool LNF>
bool run_direct_mt(const LinearArgs& a, int& rc) {
    if (a.M == 1) {
        // a tied head behind its LayerNorm (tens of thousands of rows): four
        // fp32 rows or eight rows of codes a wavefront, so each wavefront's
        // read of the activations and the LayerNorm weight and bias (12 bytes
        // a column) serves 16 or 8 bytes a column of weights (GPT-2's 50257 x
        // 768 head: fp32 24-25 us, 6.1-6.4 TB/s, int8 12.1 us, against 36.4
        // and 26.7 us for the LDS-staged kernel)
        if constexpr (LNF)
            if (a.N > kDirectLnMaxRows) return run_direct<1, UM, FMT == kF32 ? 4 : 8, FMT, TX, TY, LNF>(a, rc);
        // two weight rows a wavefront share its activation loads: a gain on
        // wide matrices with short rows (N >= 2048, at most two chunks a
        // lane), a loss on narrow ones, where it halves the wavefronts
        if constexpr (UM <= 2)
            if (a.N >= 2048) return run_direct<1, UM, 2, FMT, TX, TY, LNF>(a, rc);
        return run_direct<1, UM, 1, FMT, TX, TY, LNF>(a, rc);
    }
    if (a.M == 2) return run_direct<2, UM, 1, FMT, TX, TY, LNF>(a, rc);
    return run_direct<4, UM, 1, FMT, TX, TY, LNF>(a, rc);
}

template <int FMT, typename TX, typename TY, bool LNF>
bool run_direct_um(const LinearArgs& a, int& rc) {
    // exactly the chunks a lane needs: a spare round of (clamped, repeated)
    // loads costs address work and registers, 0.1-0.2 us a launch
    switch ((a.K / direct_kc<FMT>() + 63) / 64) {
        case 0:
        case 1: return run_direct_mt<1, FMT, TX, TY, LNF>(a, rc);
        case 2: return run_direct_mt<2, FMT, TX, TY, LNF>(a, rc);
        case 3: return run_direct_mt<3, FMT, TX, TY, LNF>(a, rc);
        case 4: return run_direct_mt<4, FMT, TX, TY, LNF>(a, rc);
        case 5: return run_direct_mt<5, FMT, TX, TY, LNF>(a, rc);
        case 6: return run_direct_mt<6, FMT, TX, TY, LNF>(a, rc);
        case 7: return run_direct_mt<7, FMT, TX, TY, LNF>(a, rc);
        case 8: return run_direct_mt<8, FMT, TX, TY, LNF>(a, rc);
        default: return false;
    }
}


// The direct kernel, when it takes the arguments (no LayerNorm, int8 / int4 /
// fp32 weights, a row of at most 8 chunks per lane, 16-byte activation rows).
template <int FMT, typename TX, typename TY>
bool try_direct(const LinearArgs& a, int& rc) {
    if constexpr (FMT == kW4G) {
        return false;
    } else {
        constexpr int KC = direct_kc<FMT>();
        constexpr size_t XB = KC * sizeof(TX);
        const size_t xa = XB >= 16 ? 16 : XB;
        if (!aligned(a.x, xa) || ((size_t)a.ldx * sizeof(TX)) % xa != 0) return false;
        // the kernel takes its strides and sizes as 32-bit integers
        if (a.ldw > INT32_MAX || a.ldx > INT32_MAX || a.ldy > INT32_MAX || a.N > INT32_MAX) return false;
        if (a.fuse.ln_w) {
            // every wavefront reads the whole row and its LayerNorm weight and
            // bias (12 bytes a column) from L2: worth it while a launch is
            // latency-bound, not for a head of 50257 rows, where that traffic
            // is twelve times the weights' and the LDS-staged kernel shares it
            // (a head at M = 1 is the exception: four or eight weight rows a
            // wavefront share that read)
            if ((a.N > kDirectLnMaxRows && a.M != 1) || !aligned(a.fuse.ln_w, 16) || !aligned(a.fuse.ln_b, 16))
                return false;
            return run_direct_um<FMT, TX, TY, true>(a, rc);
        }
        return run_direct_um<FMT, TX, TY, false>(a, rc);
    }
}

template <int W, int UP, typename TY>
int run_rows16(const LinearArgs& a, int rb = 16) {
    const int P = (int)(a.K / 64), pw = (P + W - 1) / W;
    const int G = (int)((a.N + rb - 1) / rb);
    hipLaunchKernelGGL((gemv_rows16_kernel<W, UP, TY>), dim3((unsigned)G), dim3(64 * W), 0, a.stream, a.w,
                       static_cast<const uint16_t*>(a.x), a.scale, static_cast<TY*>(a.y), (int)a.ldw, (int)a.ldx,
                       (int)a.N, (int)a.K, G, (int)a.M, (int)a.ldy, pw, rb, a.bias, a.fuse);
    return launch_status();
}


// Many wavefronts with short runs: one pair a wavefront up to 16 pairs
// (4, 8, 12 or 16 wavefronts), then 16 wavefronts with 2, 3, 4 or 7 pairs
// each. Weight rows a workgroup: 16 on wide matrices, 8 or 4 on narrower
// ones, so the grid stays near 150 workgroups or more (narrower blocks leave
// MFMA columns zero, which costs no memory traffic). Both from a sweep over
// GPT-2 small and XL shapes at M = 4 / 8 / 16 (graph-timed, cold weights).
template <typename TY>
int dispatch_rows16(const LinearArgs& a) {
    const int64_t P = a.K / 64;
    const int rb = a.N >= 2048 ? 16 : a.N >= 1200 ? 8 : 4;
    if (P <= 4) return run_rows16<4, 1, TY>(a, rb);
    if (P <= 8) return run_rows16<8, 1, TY>(a, rb);
    if (P <= 12) return run_rows16<12, 1, TY>(a, rb);
    if (P <= 16) return run_rows16<16, 1, TY>(a, rb);
    if (P <= 32) return run_rows16<16, 2, TY>(a, rb);
    if (P <= 48) return run_rows16<16, 3, TY>(a, rb);
    if (P <= 64) return run_rows16<16, 4, TY>(a, rb);
    return run_rows16<16, 7, TY>(a, rb);
}

template <int FMT, typename TX, typename TY>
int run_generic(const LinearArgs& a) {
    const int64_t outs = a.M * a.N;
    hipLaunchKernelGGL((gemv_generic<FMT, TX, TY>), dim3((unsigned)((outs + 3) / 4)), dim3(256), 0, a.stream,
                       static_cast<const TX*>(a.x), a.ldx, (int)a.M, a.w, a.ldw, a.scale, a.scale16, a.group,
                       a.bias, static_cast<TY*>(a.y), a.ldy, (int)a.N, a.K);
    return launch_status();
}

template <int FMT, typename TX, typename TY>
int dispatch_fmt(const LinearArgs& a) {
    constexpr int KC = Fmt<FMT>::KC;
    const size_t xb = (a.x_dtype == TIQ_F32) ? 16 : 8;
    const bool fused = a.fuse.ln_w || a.fuse.act || a.fuse.res;
    const bool vec = (a.K % KC == 0) && (a.K % 4 == 0) && aligned(a.w, 16) && (a.ldw % 16 == 0) &&
                     aligned(a.x, xb) && (a.ldx % 4 == 0) && (FMT != kW4G || a.group % KC == 0) &&
                     a.K * sizeof(float) <= kMaxLds && a.N <= 0x7fffffff &&
                     (!a.fuse.ln_w || (aligned(a.fuse.ln_w, 16) && aligned(a.fuse.ln_b, 16)));
    if (!vec) {
        if (fused) return TIQ_EUNSUPPORTED;
        return run_generic<FMT, TX, TY>(a);
    }
    int rc = TIQ_OK;
    if constexpr (FMT == kW8 && sizeof(TX) == 2)
        if (rows16_preferred(a)) return launch_rows16(a);
    // up to 4 rows; up to 16 bf16 rows without fusions on narrow matrices
    // (N < 2048), four rows a tile, where the batched kernel has too few tiles
    const bool direct_rows = a.M <= 4 || (a.M <= 16 && a.N < 2048 && a.x_dtype == TIQ_BF16 && !fused);
    if (direct_rows && try_direct<FMT, TX, TY>(a, rc)) return rc;
    const size_t row_lds = (size_t)a.K * sizeof(float);
    int mt = 4;
    while (mt > 1 && (size_t)mt * row_lds > kMaxLds) mt >>= 1;
    if (a.M < mt) mt = a.M >= 2 ? 2 : 1;
    // two rows per wavefront once the grid has enough wavefronts to fill the chip
    const bool r2 = a.N >= 2048;
    switch (mt) {
        case 4: return r2 ? run_gemv<4, 2, FMT, TX, TY>(a) : run_gemv<4, 1, FMT, TX, TY>(a);
        case 2: return r2 ? run_gemv<2, 2, FMT, TX, TY>(a) : run_gemv<2, 1, FMT, TX, TY>(a);
        default: return r2 ? run_gemv<1, 2, FMT, TX, TY>(a) : run_gemv<1, 1, FMT, TX, TY>(a);
    }
}

template <int FMT>
int dispatch_types(const LinearArgs& a) {
    if (a.x_dtype == TIQ_F32) {
        return a.y_dtype == TIQ_F32 ? dispatch_fmt<FMT, float, float>(a) : dispatch_fmt<FMT, float, uint16_t>(a);
    }
    return a.y_dtype == TIQ_F32 ? dispatch_fmt<FMT, uint16_t, float>(a) : dispatch_fmt<FMT, uint16_t, uint16_t>(a);
}

}  // namespace

bool rows16_supported(const LinearArgs& a) {
    if (a.fmt != kW8 || a.x_dtype != TIQ_BF16 || a.fuse.ln_w || a.M < 2 || a.M > 16) return false;
    if (a.K % 64 != 0 || a.K / 64 > 112 || a.N > 0x7fffffff) return false;
    if (!aligned(a.x, 16) || a.ldx % 8 != 0 || !aligned(a.w, 16) || a.ldw % 16 != 0) return false;
    if (a.fuse.res && a.fuse.res != a.y && a.fuse.ldr < a.N) return false;
    // the descriptors' 32-bit byte offsets: 16 weight rows, M activation rows
    if (15 * a.ldw + a.K > 0x7fffff00LL || ((a.M - 1) * a.ldx + a.K) * 2 > 0x7fffff00LL) return false;
    if (a.ldy > INT32_MAX || a.ldx > INT32_MAX || a.ldw > INT32_MAX) return false;
    return true;
}

// Where it beats the direct kernel and the batched one (graph-timed, cold
// weights, GPT-2 small and XL shapes): from 4 rows on matrices of 1200 rows
// or more, from 9 rows on narrower ones (at 768 rows the direct kernel's
// 768 one-wavefront workgroups win up to 8 rows).
bool rows16_preferred(const LinearArgs& a) {
    if (a.M < 4 || (a.N < 1200 && a.M <= 8)) return false;
    return rows16_supported(a);
}

int launch_rows16(const LinearArgs& a) {
    return a.y_dtype == TIQ_F32 ? dispatch_rows16<float>(a) : dispatch_rows16<uint16_t>(a);
}

int launch_gemv(const LinearArgs& a) {
    switch (a.fmt) {
        case kW8: return dispatch_types<kW8>(a);
        case kW4: return dispatch_types<kW4>(a);
        case kW4G: return dispatch_types<kW4G>(a);
        case kF32: return dispatch_types<kF32>(a);
        // operand-tile layouts are read by the batched decode kernels only
        case kW8T:
        case kF32T: return TIQ_EUNSUPPORTED;
    }
    return TIQ_EINVAL;
}

}  // namespace tiq
