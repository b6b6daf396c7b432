// Decode-step kernels around the quantized Linears (gfx950): one token per
// sequence attends over a preallocated KV cache whose fill level is a device
// scalar, so the whole step can be captured once and replayed per token.
//
//   decode_attention  -- CausalSelfAttention.forward at T = 1 with a cache
//                        (model.py:248-318, KVCache.update model.py:153-172):
//                        the new key / value are written at slot `pos`, the
//                        query attends to slots 0..pos (the causal mask of a
//                        single query at absolute position pos), softmax in
//                        fp32, weighted sum of values;
//   embed_tokens      -- wte(idx) + wpe(pos) (model.py:561-564);
//   argmax_rows       -- logits.argmax(-1) (sampling.py:164), first index of
//                        the maximum, the token also written into the id
//                        buffer at column pos + 1.
#include <cmath>

#include "tiq_internal.hpp"

namespace tiq {
namespace {

constexpr int kHeadDim = 64;    // every released GPT-2 size
constexpr int kMaxSlots = 1024;  // n_positions of GPT-2

// Attention of one query per (sequence, head): a workgroup of kAttWaves
// wavefronts. The cache rows are read through buffer descriptors sized to the
// pos slots written so far: a load past them returns zero with no memory
// access, so no load address depends on pos (one scalar read gates them all,
// no per-load clamps) and no traffic is spent on the empty tail of the cache.
// Slot layout: chunk c covers slots 128 c .. 128 c + 127; wave w takes the
// 16 slots from 128 c + 16 w, four a load instruction (16 lanes x 16 bytes of
// one slot's row: 1 KB of consecutive cache per instruction). The keys of the
// first NCH chunks are requested at launch (and the values too when NCH = 1);
// with two chunks the values are requested as soon as the scores are stored,
// into the keys' registers, so that second trip to memory overlaps the
// softmax. Histories past 128 NCH slots stream one chunk per trip.
constexpr int kAttWaves = 8;
constexpr int kSlotsPerWave = 128 / kAttWaves;
constexpr int kLoadsPerChunk = kSlotsPerWave / 4;

typedef float tiq_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 cache_load(__amdgpu_buffer_rsrc_t r, int byte_off) {
    const tiq_f32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    return make_float4(v.x, v.y, v.z, v.w);
}

// Columns k .. k + 7 of activation row m as the exact three bf16 planes, in
// the operand order of the batched decode linear for K = Kc columns: for row
// tile t = m / 32, unit u = k / 32, plane q and half e = (k / 8) % 2, a 1 KB
// block holds the 16 bytes of lane 32 ((k / 16) % 2) + m % 32.
__device__ __forceinline__ void store_planes(uint16_t* x3, int64_t m, int64_t Kc, int64_t k, const float (&v)[8]) {
    uint32_t pl[3][4];
    split3_words(v, pl);
    const int64_t U = Kc / 32, t = m >> 5, u = k >> 5;
    const int r = (int)(m & 31), hh = (int)((k >> 4) & 1), e = (int)((k >> 3) & 1);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const int64_t blk = ((t * U + u) * 3 + q) * 2 + e;
        *reinterpret_cast<uint4*>(x3 + (blk * 64 + 32 * hh + r) * 8) = make_uint4(pl[q][0], pl[q][1], pl[q][2], pl[q][3]);
    }
}

// WHOLE: the descriptors cover the whole cache (t_max slots) rather than the
// pos filled ones, so the first loads need not wait for pos -- for small caches
// (batch 1), where the unused tail costs less than that wait; the slots past
// pos are dropped where they are used either way.
// SL: qkv holds the n_sl raw partial slices of the q, k, v projection
// (slice z at qkv + z sl_stride, rows of ld_qkv; launch_decode_slices), which
// the kernel finishes for its head: (sum of the slices in slice order) *
// scale + bias, the reduction kernel's arithmetic.
// Grid (head, sequence). The arguments up to t_max are the ones the loads
// need, in the 14 dwords preloaded into SGPRs.
// Eight wavefronts a SIMD (at most 64 VGPRs): four workgroups a CU, so the
// 800 of a GPT-2-XL batch-32 layer are resident at once.
template <int NCH, bool WHOLE, bool SL>
__global__ __launch_bounds__(64 * kAttWaves) __attribute__((amdgpu_waves_per_eu(8))) void decode_attention_kernel(
    const float* __restrict__ qkv, const int64_t* __restrict__ pos_p, float* __restrict__ kc, float* __restrict__ vc,
    int ld_qkv, int H, int Hkv, int group, int t_max, float* __restrict__ y, int64_t ldy,
    uint16_t* __restrict__ x3, int n_sl, int64_t sl_stride, const float* __restrict__ sl_scale,
    const float* __restrict__ sl_bias) {
    constexpr int W = kAttWaves, NI = kLoadsPerChunk;
    __shared__ __align__(16) float qn[kHeadDim];  // read as float4 with slices
    __shared__ float kn[kHeadDim], vn[kHeadDim];
    __shared__ float sc[kMaxSlots];
    __shared__ float red[W];
    __shared__ float4 part[W][4][16];
    __shared__ float ov[kHeadDim];
    const int h = blockIdx.x, b = blockIdx.y;  // no integer division on the way to the first loads
    const int hk = group == 1 ? h : h / group;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row = lane >> 4, d4 = (lane & 15) * 4;  // slot within the load, first of 4 dims
    const float* qr = qkv + (int64_t)b * ld_qkv;
    const int C = H * kHeadDim, KV = Hkv * kHeadDim;
    float* kb = kc + ((int64_t)b * Hkv + hk) * t_max * kHeadDim;
    float* vb = vc + ((int64_t)b * Hkv + hk) * t_max * kHeadDim;

    const int off0 = ((kSlotsPerWave * wave + row) * kHeadDim + d4) * 4;
    auto slot_off = [&](int base, int i) { return off0 + (base + 4 * i) * kHeadDim * 4; };
    // The keys of the first chunk need no position: requested at launch through
    // a descriptor over the first min(t_max, 128) slots (a key past pos gets no
    // score stored), so the read of pos below overlaps them.
    float4 kr[NCH][NI], vr[NCH][NI];
    {
        const int first = (WHOLE ? t_max : min(t_max, 128)) * kHeadDim * 4;
        const __amdgpu_buffer_rsrc_t rk0 = __builtin_amdgcn_make_buffer_rsrc(kb, (short)0, first, 0x00020000);
#pragma unroll
        for (int i = 0; i < NI; ++i) kr[0][i] = cache_load(rk0, slot_off(0, i));
    }
    asm volatile("" ::: "memory");  // keep the read of pos (and its wait) behind those loads
    int64_t pos_in = 0;
    if constexpr (!WHOLE) pos_in = *pos_p;  // the other descriptors need it
    // bytes of slots 0 .. pos - 1 (0 for a position outside the cache)
    const int valid =
        WHOLE ? t_max * kHeadDim * 4 : (pos_in < 0 || pos_in >= t_max ? 0 : (int)pos_in * kHeadDim * 4);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(kb, (short)0, valid, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(vb, (short)0, valid, 0x00020000);
#pragma unroll
    for (int c = 1; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < NI; ++i) kr[c][i] = cache_load(rk, slot_off(128 * c, i));
    if constexpr (NCH == 1) {  // one chunk: its values too, one trip to memory
#pragma unroll
        for (int i = 0; i < NI; ++i) vr[0][i] = cache_load(rv, slot_off(0, i));
    }
    float4 q4;  // with slices, from the finished row in LDS below
    if constexpr (!SL) q4 = *reinterpret_cast<const float4*>(qr + h * kHeadDim + d4);
    if constexpr (WHOLE) pos_in = *pos_p;  // read behind the loads, which do not need it
    // A position outside the cache computes on slot 0, writes nothing to the
    // cache and stores NaN: no branch, so no load is sunk behind the read of pos.
    const bool ok = pos_in >= 0 && pos_in < t_max;
    const int64_t pos = ok ? pos_in : 0;
    if constexpr (SL) {
        if (wave < 3) {  // wavefront 0 the query, 1 the key, 2 the value; every slice requested at once
            const int col = (wave == 0 ? h * kHeadDim : wave == 1 ? C + hk * kHeadDim : C + KV + hk * kHeadDim) + lane;
            float p[kMaxSlices];
#pragma unroll
            for (int z = 0; z < kMaxSlices; ++z) p[z] = qr[(int64_t)min(z, n_sl - 1) * sl_stride + col];
            const float f_sc = sl_scale[col], f_bi = sl_bias ? sl_bias[col] : 0.f;
            float a = 0.f;
#pragma unroll
            for (int z = 0; z < kMaxSlices; ++z)
                if (z < n_sl) a += p[z];
            const float v = a * f_sc + f_bi;
            (wave == 0 ? qn : wave == 1 ? kn : vn)[lane] = v;
            if (wave > 0 && ok && (group == 1 || h % group == 0))  // one writer per kv head
                (wave == 1 ? kb : vb)[pos * kHeadDim + lane] = v;
        }
    } else if (tid < kHeadDim) {
        const float q_new = qr[h * kHeadDim + tid];
        const float k_new = qr[C + hk * kHeadDim + tid];
        const float v_new = qr[C + KV + hk * kHeadDim + tid];
        qn[tid] = q_new;
        kn[tid] = k_new;
        vn[tid] = v_new;
        if (ok && (group == 1 || h % group == 0)) {  // one writer per kv head; no workgroup reads slot pos
            kb[pos * kHeadDim + tid] = k_new;
            vb[pos * kHeadDim + tid] = v_new;
        }
    }
    __syncthreads();
    if constexpr (SL) q4 = *reinterpret_cast<const float4*>(qn + d4);

    // ---- scores of slots < pos (slot pos is the new key) ----
    const float inv_div = 1.0f / sqrtf((float)kHeadDim);  // exactly 1/8
    auto score = [&](int t, const float4& k) {
        float s = fmaf(q4.x, k.x, fmaf(q4.y, k.y, fmaf(q4.z, k.z, q4.w * k.w)));
        s += dpp_move<0xB1>(s);   // the 16 lanes of the slot: lane xor 1,
        s += dpp_move<0x4E>(s);   // xor 2,
        s += dpp_move<0x141>(s);  // half-row mirror,
        s += dpp_move<0x140>(s);  // row mirror: every lane of the row holds the sum
        if ((lane & 15) == 0 && t < pos) sc[t] = s * inv_div;
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < NI; ++i) score(128 * c + kSlotsPerWave * wave + 4 * i + row, kr[c][i]);
    for (int base = 128 * NCH; base < pos; base += 128) {
        float4 kk[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) kk[i] = cache_load(rk, slot_off(base, i));
#pragma unroll
        for (int i = 0; i < NI; ++i) score(base + kSlotsPerWave * wave + 4 * i + row, kk[i]);
    }
    if constexpr (NCH >= 2) {
        asm volatile("" ::: "memory");  // the scores are stored: the keys' registers are free
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int i = 0; i < NI; ++i) vr[c][i] = cache_load(rv, slot_off(128 * c, i));
    }
    if (wave == 0) {  // the new key's score
        const float s = wave_sum_dpp(qn[lane] * kn[lane]);
        if (lane == 0) sc[pos] = s * inv_div;
    }
    __syncthreads();

    // ---- softmax over slots 0..pos ----
    float mx = -INFINITY;
    for (int64_t t = tid; t <= pos; t += 64 * W) mx = fmaxf(mx, sc[t]);
    mx = wave_max_dpp(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < W; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    float sum = 0.f;
    for (int64_t t = tid; t <= pos; t += 64 * W) {
        const float p = expf(sc[t] - mx);
        sc[t] = p;
        sum += p;
    }
    sum = wave_sum_dpp(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = red[0];
#pragma unroll
    for (int w = 1; w < W; ++w) sum += red[w];

    // ---- weighted sum of values: this lane's 4 dims over its slots ----
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](int t, const float4& v) {  // a slot past pos adds nothing, whatever the memory holds
        const bool in = t < pos;
        const float p = in ? sc[t] : 0.f;
        acc.x = in ? fmaf(p, v.x, acc.x) : acc.x;
        acc.y = in ? fmaf(p, v.y, acc.y) : acc.y;
        acc.z = in ? fmaf(p, v.z, acc.z) : acc.z;
        acc.w = in ? fmaf(p, v.w, acc.w) : acc.w;
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < NI; ++i) add(128 * c + kSlotsPerWave * wave + 4 * i + row, vr[c][i]);
    for (int base = 128 * NCH; base < pos; base += 128) {
        float4 vv[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) vv[i] = cache_load(rv, slot_off(base, i));
#pragma unroll
        for (int i = 0; i < NI; ++i) add(base + kSlotsPerWave * wave + 4 * i + row, vv[i]);
    }
    part[wave][row][lane & 15] = acc;
    __syncthreads();
    if (tid < kHeadDim) {  // the new value, then the partial sums of every wave and slot row in order
        const float* pf = reinterpret_cast<const float*>(part);
        float o = sc[pos] * vn[tid];
#pragma unroll
        for (int w = 0; w < W; ++w)
#pragma unroll
            for (int r = 0; r < 4; ++r) o += pf[(w * 4 + r) * 64 + tid];
        const float r = ok ? o / sum : NAN;  // a position outside the cache flags the output
        y[(int64_t)b * ldy + h * kHeadDim + tid] = r;
        ov[tid] = r;
    }
    if (x3) {  // the head's 64 outputs as the operand planes of the output projection
        __syncthreads();
        if (tid < kHeadDim / 8) {
            float o8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o8[i] = ov[8 * tid + i];
            store_planes(x3, b, H * kHeadDim, h * kHeadDim + 8 * tid, o8);
        }
    }
}

__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ tok, const int64_t* __restrict__ pos_p,
                                                    const float* __restrict__ wte, const float* __restrict__ wpe,
                                                    int64_t vocab, int64_t n_pos, int64_t C, float* __restrict__ x) {
    const int b = blockIdx.x;
    const int64_t t = tok[b], p = *pos_p;
    const bool ok = t >= 0 && t < vocab && p >= 0 && p < n_pos;  // ids are device data: checked here
    for (int64_t c = threadIdx.x; c < C; c += blockDim.x) x[b * C + c] = ok ? wte[t * C + c] + wpe[p * C + c] : NAN;
}

// Row maximum in two stages: kArgParts workgroups per row each reduce a slice
// to (value, first index), then one workgroup reduces every row's partials,
// writes the token (and its id slot) and advances the position.
constexpr int kArgParts = 64;

__device__ __forceinline__ void better(float& v, int64_t& i, float ov, int64_t oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ x, int64_t cols, int64_t ld,
                                                             float* __restrict__ pv, int64_t* __restrict__ pi) {
    __shared__ float bv[4];
    __shared__ int64_t bi[4];
    const int64_t r = blockIdx.y;
    const int part = blockIdx.x;
    const int64_t span = (cols + kArgParts - 1) / kArgParts;
    const int64_t c0 = part * span, c1 = (c0 + span < cols) ? c0 + span : cols;
    const float* xr = x + r * ld;
    float v = -INFINITY;
    int64_t idx = c0 < cols ? c0 : 0;
    // four independent loads in flight per thread
    for (int64_t c = c0 + threadIdx.x; c < c1; c += 4 * 256) {
        float a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) a[u] = (c + u * 256 < c1) ? xr[c + u * 256] : -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (a[u] > v) {
                v = a[u];
                idx = c + u * 256;
            }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    if (lane == 0) {
        bv[wave] = v;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 4; ++i) better(v, idx, bv[i], bi[i]);
        pv[r * kArgParts + part] = v;
        pi[r * kArgParts + part] = idx;
    }
}

// One wavefront per row (rows beyond kArgFinalWaves taken in turn), so the
// rows' partials are read together rather than one dependent trip per row.
constexpr int kArgFinalWaves = 16;

__global__ __launch_bounds__(64 * kArgFinalWaves) void argmax_final_kernel(
    const float* __restrict__ pv, const int64_t* __restrict__ pi, int64_t rows, int64_t* __restrict__ out,
    int64_t* __restrict__ ids, int64_t ld_ids, int64_t* __restrict__ pos_p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t col = pos_p ? *pos_p + 1 : 0;
    for (int64_t r = wave; r < rows; r += kArgFinalWaves) {
        float v = pv[r * kArgParts + lane];
        int64_t idx = pi[r * kArgParts + lane];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
        if (lane == 0) {
            out[r] = idx;
            if (ids && col >= 0 && col < ld_ids) ids[r * ld_ids + col] = idx;
        }
    }
    if (pos_p && ids) {
        __syncthreads();  // every wavefront has read the position of this step
        if (threadIdx.x == 0) *pos_p = col;
    }
}


// Causal self-attention of a prompt block (CausalSelfAttention.forward at
// T > 1, model.py:284-309): T queries at absolute positions first .. first +
// T - 1 over the S = first + T cached keys. Grid (query tiles of 64, heads,
// sequences); 128 threads (two wavefronts) per tile, thread (g, c) =
// (tid / 4, tid % 4) holding query rows 2 g and 2 g + 1 of the tile and dims
// 16 c .. 16 c + 15: each 16-byte read of a key or value from LDS feeds both
// rows (eight FMAs). Per block of 64 keys staged in LDS, 16 keys at a time: the rows' scores
// (16-dim partial dots summed over the row's four lanes by quad DPP moves),
// the causal mask (-inf past the query's position), an online softmax in
// fp32 -- the running maximum, the rescale of the partial outputs, the
// running sum -- and the weighted sum of the values. q, k, v and y are read
// and written through (batch, head, position) strides in floats, the 64 dims
// contiguous, so the q, k, v projection's rows, a cache's (B, H, capacity, 64)
// buffers and the (B, T, C) output rows serve directly, with no copy.
constexpr int kPaRows = 64, kPaKeys = 64, kPaSub = 16;
constexpr int kPaR = 2;                         // query rows a lane holds
constexpr int kPaThreads = kPaRows / kPaR * 4;  // four lanes a row group

__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_move<0xB1>(v);  // quad_perm [1, 0, 3, 2]
    v += dpp_move<0x4E>(v);  // quad_perm [2, 3, 0, 1]
    return v;
}

__global__ __launch_bounds__(kPaThreads) void prefill_attention_kernel(
    const float* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_st, const float* __restrict__ k,
    int64_t k_sb, int64_t k_sh, int64_t k_st, const float* __restrict__ v, int64_t v_sb, int64_t v_sh,
    int64_t v_st, int T, int first, float* __restrict__ y, int64_t y_sb, int64_t y_sh, int64_t y_st) {
    __shared__ float4 ks[kPaKeys][kHeadDim / 4 + 1];  // rows padded
    __shared__ float4 vs[kPaKeys][kHeadDim / 4 + 1];
    const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x, g = lane >> 2, c4 = lane & 3;
    const int t0 = tile * kPaRows + kPaR * g;  // rows t0 .. t0 + kPaR - 1 (past T: computed on row T - 1, unstored)
    float qv[kPaR][16];
    int64_t qpos[kPaR];
#pragma unroll
    for (int r = 0; r < kPaR; ++r) {
        const int tq = min(t0 + r, T - 1);
        qpos[r] = (int64_t)first + tq;
        const float4* qr = reinterpret_cast<const float4*>(q + b * q_sb + h * q_sh + tq * q_st + 16 * c4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 f = qr[j];
            qv[r][4 * j] = f.x, qv[r][4 * j + 1] = f.y, qv[r][4 * j + 2] = f.z, qv[r][4 * j + 3] = f.w;
        }
    }
    const float* kb = k + b * k_sb + h * k_sh;
    const float* vb = v + b * v_sb + h * v_sh;
    const int64_t s_end = (int64_t)first + min(T, kPaRows * (tile + 1));  // keys this tile needs
    float mx[kPaR], sum[kPaR], acc[kPaR][16];
#pragma unroll
    for (int r = 0; r < kPaR; ++r) {
        mx[r] = -INFINITY, sum[r] = 0.f;
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[r][d] = 0.f;
    }
    for (int64_t j0 = 0; j0 < s_end; j0 += kPaKeys) {
        __syncthreads();  // the previous block is consumed
#pragma unroll
        for (int u = 0; u < kPaKeys * 16 / kPaThreads; ++u) {  // the block's keys and values, 16 float4 a key
            const int e = lane + kPaThreads * u, kk = e >> 4, dq = e & 15;
            const int64_t slot = j0 + kk < s_end ? j0 + kk : s_end - 1;
            ks[kk][dq] = reinterpret_cast<const float4*>(kb + slot * k_st)[dq];
            vs[kk][dq] = reinterpret_cast<const float4*>(vb + slot * v_st)[dq];
        }
        __syncthreads();
        const int nsub = (int)min<int64_t>(kPaKeys / kPaSub, (s_end - j0 + kPaSub - 1) / kPaSub);
        for (int sb = 0; sb < nsub; ++sb) {
            const int kb0 = sb * kPaSub;
            float sc[kPaR][kPaSub];
#pragma unroll
            for (int kk = 0; kk < kPaSub; ++kk) {
                float d[kPaR];
#pragma unroll
                for (int r = 0; r < kPaR; ++r) d[r] = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 f = ks[kb0 + kk][4 * c4 + j];
#pragma unroll
                    for (int r = 0; r < kPaR; ++r) {
                        d[r] = fmaf(qv[r][4 * j], f.x, d[r]);
                        d[r] = fmaf(qv[r][4 * j + 1], f.y, d[r]);
                        d[r] = fmaf(qv[r][4 * j + 2], f.z, d[r]);
                        d[r] = fmaf(qv[r][4 * j + 3], f.w, d[r]);
                    }
                }
                const int64_t key = j0 + kb0 + kk;
#pragma unroll
                for (int r = 0; r < kPaR; ++r) {
                    const float full = quad_sum(d[r]);
                    sc[r][kk] = key <= qpos[r] ? full * 0.125f : -INFINITY;  // 1 / sqrt(64), exact
                }
            }
#pragma unroll
            for (int r = 0; r < kPaR; ++r) {
                float bm = sc[r][0];
#pragma unroll
                for (int kk = 1; kk < kPaSub; ++kk) bm = fmaxf(bm, sc[r][kk]);
                const float mnew = fmaxf(mx[r], bm);  // finite: key 0 is visible to every query
                const float alpha = expf(mx[r] - mnew);
                // lane c of the row's quad exponentiates keys 4 jj + c, the quad
                // broadcasts them: each exponential computed once
                float pe[kPaSub / 4], ps = 0.f;
#pragma unroll
                for (int jj = 0; jj < kPaSub / 4; ++jj) {
                    const float mine = c4 == 0 ? sc[r][4 * jj] : c4 == 1 ? sc[r][4 * jj + 1]
                                     : c4 == 2 ? sc[r][4 * jj + 2] : sc[r][4 * jj + 3];
                    pe[jj] = expf(mine - mnew);
                    ps += pe[jj];
                }
#pragma unroll
                for (int jj = 0; jj < kPaSub / 4; ++jj) {
                    sc[r][4 * jj] = dpp_move<0x00>(pe[jj]);  // quad_perm [0, 0, 0, 0]
                    sc[r][4 * jj + 1] = dpp_move<0x55>(pe[jj]);
                    sc[r][4 * jj + 2] = dpp_move<0xAA>(pe[jj]);
                    sc[r][4 * jj + 3] = dpp_move<0xFF>(pe[jj]);
                }
                sum[r] = sum[r] * alpha + quad_sum(ps);
                mx[r] = mnew;
#pragma unroll
                for (int d = 0; d < 16; ++d) acc[r][d] *= alpha;
            }
#pragma unroll
            for (int kk = 0; kk < kPaSub; ++kk) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 f = vs[kb0 + kk][4 * c4 + j];
#pragma unroll
                    for (int r = 0; r < kPaR; ++r) {
                        acc[r][4 * j] = fmaf(sc[r][kk], f.x, acc[r][4 * j]);
                        acc[r][4 * j + 1] = fmaf(sc[r][kk], f.y, acc[r][4 * j + 1]);
                        acc[r][4 * j + 2] = fmaf(sc[r][kk], f.z, acc[r][4 * j + 2]);
                        acc[r][4 * j + 3] = fmaf(sc[r][kk], f.w, acc[r][4 * j + 3]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kPaR; ++r) {
        if (t0 + r < T) {
            float4* yr = reinterpret_cast<float4*>(y + b * y_sb + h * y_sh + (int64_t)(t0 + r) * y_st + 16 * c4);
            const float inv = 1.0f / sum[r];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                yr[j] = make_float4(acc[r][4 * j] * inv, acc[r][4 * j + 1] * inv, acc[r][4 * j + 2] * inv,
                                    acc[r][4 * j + 3] * inv);
        }
    }
}

// ------------------------------------------------------------ screened head
// The tied fp32 head and its argmax at one row (GPT.forward's lm_head,
// model.py:585, then logits.argmax(-1), sampling.py:164), reading a bf16 copy
// of the head instead of all of its fp32 rows. Per row v, with x the
// LayerNorm'd row, a_v = x . bf16(w_v) in fp32 and the exact logit e_v =
// x . w_v in fp32 differ by at most
//   |x . (w_v - bf16(w_v))| + gamma (|x| . |w_v| + |x| . |bf16(w_v)|)
//   <= ||x|| (err_v + gamma (2 norm_v + err_v)) = b_v
// (Cauchy-Schwarz; gamma = C u / (1 - C u), u = 2^-24, bounds the rounding of
// a length-C dot product in any order; err_v = ||w_v - bf16(w_v)||_2, norm_v =
// ||w_v||_2; tiq_head_screen_prepare stores the row's coefficient
// err_v + gamma (2 norm_v + err_v), rounded up, so b_v = ||x|| coef_v). Among a
// workgroup's rows, every row with a_v + b_v below L = max (a_u - b_u) has an
// exact logit below the exact logit of the row that attains L, so the
// workgroup's exact maximum is among its rows with a_v + b_v >= L (usually
// one): only those are recomputed from the fp32 weights. The workgroup writes
// (its exact maximum, the first row attaining it) -- the semantics of
// argmax_partial_kernel: NaN never wins, -inf everywhere gives the first row --
// and argmax_parts_kernel reduces the workgroups' pairs. The logits buffer
// holds a_v, and e_v for the recomputed rows.
// I8: the copy is int8 codes q_v with a per-row scale s_v (half the bytes of
// the bf16 copy), a_v = s_v (x . q_v) in fp32 and err_v = ||w_v - s_v q_v||_2;
// the product by s_v is one more rounding, so gamma takes C + 1 for C (the
// same bound otherwise: x . (s_v q_v) is a dot product of C terms plus one
// multiplication).
// Layout: kHsGroups workgroups of kHsWaves wavefronts (two a CU, all resident
// at once); a wavefront takes the chunks gw, gw + W, gw + 2 W, ... of the head
// (4 rows a chunk, 8 for int8 codes: 64 bytes of a lane's columns either way;
// gw its index among the W wavefronts), the next chunk's rows in flight while
// the current one is summed, so the head streams in one pass.
constexpr int kHsWaves = 8, kHsGroups = 512, kHsChunk = 4, kHsMaxChunks = 8;
constexpr int kHsMaxCols = 64 * 16;  // a lane holds 16 columns of the row

__device__ __forceinline__ void better_i32(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

// P: columns a lane (16; 12 for the int8 copy at 768 columns, so that all 64
// lanes work instead of 48).
template <bool I8, int P = 16>
__global__ __launch_bounds__(64 * kHsWaves) __attribute__((amdgpu_waves_per_eu(4))) void head_screen_kernel(
    const float* __restrict__ x, int C, const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
    const void* __restrict__ wq, const float* __restrict__ row_scale, const float* __restrict__ wf, int64_t ldw,
    const float* __restrict__ row_coef, int V, float* __restrict__ logits, float* __restrict__ pv,
    int* __restrict__ pi) {
    constexpr int CH = I8 ? 2 * kHsChunk : kHsChunk;  // rows a chunk
    constexpr int RU = I8 ? 1 : 2;                    // 16-byte loads of a row a lane
    static_assert(P == 16 || (P == 12 && I8), "16 columns a lane, or 12 from the int8 copy");
    __shared__ float4 xs[64][P / 4];  // the LayerNorm'd row, lane l's P columns at xs[l]
    __shared__ float sxn;         // its 2-norm
    __shared__ float lo[kHsWaves];
    __shared__ float bv[kHsWaves];
    __shared__ int bi[kHsWaves];
    __shared__ int nc[kHsWaves];             // candidates of each wavefront
    __shared__ int crow[kHsWaves * 64];      // the workgroup's candidate rows, wavefront by wavefront
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int CK = C / P;
    const bool act = lane < CK;
    const int cl = P * min(lane, CK - 1);  // a lane past the row repeats the last chunk, unused
    const int W = gridDim.x * kHsWaves, gw = blockIdx.x * kHsWaves + wave;
    const int NC = (V + CH - 1) / CH;
    const int nch = gw < NC ? (NC - 1 - gw) / W + 1 : 0;  // this wavefront's chunks (<= kHsMaxChunks)
    auto load = [&](int c, uint4 (&r)[CH][RU]) {  // chunk gw + c W (rows clamped)
        const int row0 = (gw + c * W) * CH;
#pragma unroll
        for (int q = 0; q < CH; ++q) {
            if constexpr (I8) {
                const int8_t* p = static_cast<const int8_t*>(wq) + (int64_t)min(row0 + q, V - 1) * C + cl;
                if constexpr (P == 12) {
                    const uint3 t = *reinterpret_cast<const uint3*>(p);
                    r[q][0] = uint4{t.x, t.y, t.z, 0u};
                } else {
                    r[q][0] = *reinterpret_cast<const uint4*>(p);
                }
            } else {
                const uint16_t* p = static_cast<const uint16_t*>(wq) + (int64_t)min(row0 + q, V - 1) * C + cl;
                r[q][0] = *reinterpret_cast<const uint4*>(p);
                r[q][1] = *reinterpret_cast<const uint4*>(p + 8);
            }
        }
    };
    uint4 buf[2][CH][RU];
    if (nch > 0) load(0, buf[0]);
    if (nch > 1) load(1, buf[1]);
    // lane q + 4 c (int8 copy: 8 q + c) holds row q of chunk c: its bound's
    // inputs requested now
    const int lc = I8 ? (lane & 7) : lane / CH, lq = I8 ? (lane >> 3) : lane % CH;
    const int my_row = (gw + lc * W) * CH + lq;
    const bool mine = lc < nch && my_row < V;
    const int nl = mine ? my_row : 0;
    const float k_l = row_coef[nl];
    const float s_l = I8 ? row_scale[nl] : 1.f;
    if (wave == 0) {  // LayerNorm (two-pass mean and biased variance, as torch) into LDS
        float v[P], g[P], bb[P];
#pragma unroll
        for (int q = 0; q < P / 4; ++q) {
            *reinterpret_cast<float4*>(v + 4 * q) = reinterpret_cast<const float4*>(x + cl)[q];
            *reinterpret_cast<float4*>(g + 4 * q) = reinterpret_cast<const float4*>(ln_w + cl)[q];
            *reinterpret_cast<float4*>(bb + 4 * q) = reinterpret_cast<const float4*>(ln_b + cl)[q];
        }
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < P; ++j) sum += v[j];
        const float mean = wave_sum_dpp(act ? sum : 0.f) / (float)C;
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < P; ++j) d += (v[j] - mean) * (v[j] - mean);
        const float rstd = 1.0f / sqrtf(wave_sum_dpp(act ? d : 0.f) / (float)C + eps);
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            v[j] = (v[j] - mean) * rstd * g[j] + bb[j];
            ss = fmaf(v[j], v[j], ss);
        }
        ss = wave_sum_dpp(act ? ss : 0.f);
        if (act) {
#pragma unroll
            for (int q = 0; q < P / 4; ++q) xs[lane][q] = *reinterpret_cast<const float4*>(v + 4 * q);
        }
        if (lane == 0) sxn = sqrtf(ss);
    }
    __syncthreads();
    float xl[P];
#pragma unroll
    for (int q = 0; q < P / 4; ++q) *reinterpret_cast<float4*>(xl + 4 * q) = xs[act ? lane : 0][q];
    // ||x|| with its own rounding covered (a relative 2^-10 is far above it)
    const float xn = sxn * (1.0f + 0x1p-10f);
    // a_v of this wavefront's rows: the bf16 copy sums each row over the
    // wavefront in turn; the int8 copy, with twice the rows a chunk, sums the
    // chunk's 8 rows at once (halving the rows a lane carries at each of the
    // first three exchanges, then three on one value), after which lane 8 q + c
    // holds row q of chunk c
    float a_l = 0.f;
#pragma unroll
    for (int c = 0; c < kHsMaxChunks; ++c) {
        if (c < nch) {  // uniform across the wavefront
            const uint4 (&r)[CH][RU] = buf[c & 1];
            float sv[CH];
#pragma unroll
            for (int q = 0; q < CH; ++q) {
                float s = 0.f;
                if constexpr (I8) {
                    const uint32_t w32[4] = {r[q][0].x, r[q][0].y, r[q][0].z, r[q][0].w};
#pragma unroll
                    for (int j = 0; j < P / 4; ++j) {
                        s = fmaf(sbyte_f32<0>(w32[j]), xl[4 * j], s);
                        s = fmaf(sbyte_f32<1>(w32[j]), xl[4 * j + 1], s);
                        s = fmaf(sbyte_f32<2>(w32[j]), xl[4 * j + 2], s);
                        s = fmaf(sbyte_f32<3>(w32[j]), xl[4 * j + 3], s);
                    }
                } else {
                    const uint32_t w32[8] = {r[q][0].x, r[q][0].y, r[q][0].z, r[q][0].w,
                                             r[q][RU - 1].x, r[q][RU - 1].y, r[q][RU - 1].z, r[q][RU - 1].w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        s = fmaf(bf_lo(w32[j]), xl[2 * j], s);
                        s = fmaf(bf_hi(w32[j]), xl[2 * j + 1], s);
                    }
                }
                if constexpr (I8) {
                    sv[q] = act ? s : 0.f;
                } else {
                    const float a = wave_sum_dpp(act ? s : 0.f);
                    a_l = lane == q + CH * c ? a : a_l;
                }
            }
            if constexpr (I8) {
                float t4[4], t2[2];
                const bool u5 = lane & 32, u4 = lane & 16, u3 = lane & 8;
#pragma unroll
                for (int j = 0; j < 4; ++j) t4[j] = (u5 ? sv[4 + j] : sv[j]) + __shfl_xor(u5 ? sv[j] : sv[4 + j], 32, 64);
#pragma unroll
                for (int j = 0; j < 2; ++j) t2[j] = (u4 ? t4[2 + j] : t4[j]) + __shfl_xor(u4 ? t4[j] : t4[2 + j], 16, 64);
                float t1 = (u3 ? t2[1] : t2[0]) + __shfl_xor(u3 ? t2[0] : t2[1], 8, 64);
                t1 += __shfl_xor(t1, 4, 64);
                t1 += __shfl_xor(t1, 2, 64);
                t1 += __shfl_xor(t1, 1, 64);
                a_l = (lane & 7) == c ? t1 : a_l;
            }
            if (c + 2 < nch) load(c + 2, buf[c & 1]);  // its registers are free now
        }
    }
    if constexpr (I8) a_l *= s_l;  // x . q_v scaled: one rounding, inside gamma_(C + 1)
    const float b_l = xn * k_l * (1.0f + 0x1p-10f);
    const float hi_l = a_l + b_l;
    if (mine) logits[my_row] = a_l;
    const float low = wave_max_dpp(mine ? a_l - b_l : -INFINITY);
    if (lane == 0) lo[wave] = low;
    __syncthreads();
    float L = lo[0];
#pragma unroll
    for (int w = 1; w < kHsWaves; ++w) L = fmaxf(L, lo[w]);
    // the candidates of this wavefront, recomputed from the fp32 rows
    float best = -INFINITY;
    int bidx = INT32_MAX;
    uint64_t cand = __ballot(mine && hi_l >= L);
    while (cand) {
        const int l = __builtin_ctzll(cand);
        cand &= cand - 1;
        const int n = I8 ? (gw + (l & 7) * W) * CH + (l >> 3) : (gw + (l / CH) * W) * CH + l % CH;
        const float* p = wf + (int64_t)n * ldw + cl;
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < P / 4; ++q) {
            const float4 f = reinterpret_cast<const float4*>(p)[q];
            s = fmaf(f.x, xl[4 * q], s);
            s = fmaf(f.y, xl[4 * q + 1], s);
            s = fmaf(f.z, xl[4 * q + 2], s);
            s = fmaf(f.w, xl[4 * q + 3], s);
        }
        const float e = wave_sum_dpp(act ? s : 0.f);
        if (lane == 0) logits[n] = e;
        better_i32(best, bidx, e, n);
    }
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = bidx;
    }
    __syncthreads();
    if (tid == 0) {
        // no row above -inf: the group's first row, as argmax_partial_kernel
        float v = -INFINITY;
        int i = gw < NC ? gw * CH : INT32_MAX;
#pragma unroll
        for (int w = 0; w < kHsWaves; ++w) better_i32(v, i, bv[w], bi[w]);
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = i;
    }
}

// The workgroups' (maximum, index) pairs of one row reduced to its argmax;
// the token is written to out and to ids at column pos + 1, and pos advanced.
__global__ __launch_bounds__(1024) void argmax_parts_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                            int P, int64_t* __restrict__ out,
                                                            int64_t* __restrict__ ids, int64_t ld_ids,
                                                            int64_t* __restrict__ pos_p) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t col = pos_p ? *pos_p + 1 : 0;
    float v = -INFINITY;
    int idx = INT32_MAX;
    for (int k = tid; k < P; k += 1024) better_i32(v, idx, pv[k], pi[k]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) better_i32(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    if (lane == 0) {
        sv[wave] = v;
        si[wave] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w) better_i32(v, idx, sv[w], si[w]);
        out[0] = idx;
        if (ids && col >= 0 && col < ld_ids) ids[col] = idx;
        if (pos_p && ids) *pos_p = col;
    }
}

// bf16 copy of the head (round to nearest even), and per row the bound
// coefficient err + gamma (2 norm + err) from the 2-norms of w - bf16(w) and of
// w, summed in fp64 and rounded up to fp32.
__device__ __forceinline__ float f32_round_up(double d) {  // d >= 0
    float f = (float)d;
    if ((double)f < d) f = __uint_as_float(__float_as_uint(f) + 1u);  // the next float up
    return f;
}

__global__ __launch_bounds__(256) void head_screen_prepare_kernel(const float* __restrict__ w, int C, int64_t ldw,
                                                                  uint16_t* __restrict__ wb,
                                                                  float* __restrict__ row_coef) {
    __shared__ double red[2][4];
    const int64_t n = blockIdx.x;
    const int tid = threadIdx.x;
    double e2 = 0.0, n2 = 0.0;
    for (int c = tid; c < C; c += 256) {
        const float v = w[n * ldw + c];
        const uint16_t h = f32_to_bf16_bits(v);
        wb[n * C + c] = h;
        const double d = (double)v - (double)bf16_bits_to_f32(h);
        e2 += d * d;
        n2 += (double)v * (double)v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        e2 += __shfl_xor(e2, off, 64);
        n2 += __shfl_xor(n2, off, 64);
    }
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = e2;
        red[1][tid >> 6] = n2;
    }
    __syncthreads();
    if (tid == 0) {
        // the fp64 sums of C squares are within a relative C 2^-53 of the
        // exact ones; one fp64 ulp per term more, rounded up
        const double se = (red[0][0] + red[0][1] + red[0][2] + red[0][3]) * (1.0 + (C + 4) * 0x1p-52);
        const double sn = (red[1][0] + red[1][1] + red[1][2] + red[1][3]) * (1.0 + (C + 4) * 0x1p-52);
        const double err = sqrt(se) * (1.0 + 0x1p-50), nrm = sqrt(sn) * (1.0 + 0x1p-50);
        const double cu = (double)C * 0x1p-24, gamma = cu / (1.0 - cu);
        row_coef[n] = f32_round_up((err + gamma * (2.0 * nrm + err)) * (1.0 + 0x1p-50));
    }
}

// int8 copy of the head for the screen: per row s = max|w| / 127 (0 for a zero
// row), q = rint(w / s) clamped to +-127 (any codes serve: the bound uses their
// actual error), and the coefficient err + gamma_(C + 1) (2 norm + err) from
// the fp64 2-norms of w - s q and of w, rounded up to fp32. A row holding NaN
// gets a NaN coefficient, so it is never a candidate (as in the bf16 copy).
__global__ __launch_bounds__(256) void head_screen_prepare_i8_kernel(const float* __restrict__ w, int C, int64_t ldw,
                                                                     int8_t* __restrict__ wq,
                                                                     float* __restrict__ row_scale,
                                                                     float* __restrict__ row_coef) {
    __shared__ double red[2][4];
    __shared__ float mx[4];
    const int64_t n = blockIdx.x;
    const int tid = threadIdx.x;
    float m = 0.f;
    for (int c = tid; c < C; c += 256) m = fmaxf(m, fabsf(w[n * ldw + c]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) mx[tid >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
    const float sc = amax / 127.f;
    double e2 = 0.0, n2 = 0.0;
    for (int c = tid; c < C; c += 256) {
        const float v = w[n * ldw + c];
        const float qf = sc > 0.f ? fminf(fmaxf(rintf(v / sc), -127.f), 127.f) : 0.f;
        wq[n * C + c] = (int8_t)(int)qf;
        const double d = (double)v - (double)qf * (double)sc;
        e2 += d * d;
        n2 += (double)v * (double)v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        e2 += __shfl_xor(e2, off, 64);
        n2 += __shfl_xor(n2, off, 64);
    }
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = e2;
        red[1][tid >> 6] = n2;
    }
    __syncthreads();
    if (tid == 0) {
        const double se = (red[0][0] + red[0][1] + red[0][2] + red[0][3]) * (1.0 + (C + 4) * 0x1p-52);
        const double sn = (red[1][0] + red[1][1] + red[1][2] + red[1][3]) * (1.0 + (C + 4) * 0x1p-52);
        const double err = sqrt(se) * (1.0 + 0x1p-50), nrm = sqrt(sn) * (1.0 + 0x1p-50);
        const double cu = (double)(C + 1) * 0x1p-24, gamma = cu / (1.0 - cu);
        row_scale[n] = sc;
        row_coef[n] = f32_round_up((err + gamma * (2.0 * nrm + err)) * (1.0 + 0x1p-50));
    }
}

// y = gelu_tanh(x) elementwise (the MLP activation of a prefill, one pass in
// place of the reference's op chain at model.py:57-75): 4 values a thread per
// step of a grid-stride loop; n % 4 tail by the first threads.
__global__ __launch_bounds__(256) void gelu_tanh_kernel(const float* x, float* y, int64_t n) {
    const int64_t n4 = n / 4, stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        float4 v = reinterpret_cast<const float4*>(x)[i];
        v.x = gelu_tanh(v.x);
        v.y = gelu_tanh(v.y);
        v.z = gelu_tanh(v.z);
        v.w = gelu_tanh(v.w);
        reinterpret_cast<float4*>(y)[i] = v;
    }
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t < n - 4 * n4) y[4 * n4 + t] = gelu_tanh(x[4 * n4 + t]);
}
}  // namespace
}  // namespace tiq

using namespace tiq;


// qkv rows, or (n_sl > 0) the raw partial slices of the q, k, v projection
// with its scale and bias
static int decode_attention(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head, int64_t n_kv_head,
                            int64_t head_dim, float* k_cache, float* v_cache, int64_t t_max, const int64_t* pos,
                            float* y, int64_t ldy, uint16_t* planes_out, void* stream, int64_t n_sl = 0,
                            const float* sl_scale = nullptr, const float* sl_bias = nullptr) {
    if (batch < 0 || n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head) return TIQ_EINVAL;
    if (batch == 0) return TIQ_OK;
    if (!qkv || !k_cache || !v_cache || !pos || !y) return TIQ_EINVAL;
    if (head_dim != kHeadDim || t_max <= 0 || t_max > kMaxSlots) return TIQ_EUNSUPPORTED;
    if (ld_qkv < (n_head + 2 * n_kv_head) * head_dim || ldy < n_head * head_dim) return TIQ_EINVAL;
    // the kernel takes the row stride as 32 bits and the sequence as grid row
    if (ld_qkv > INT32_MAX || batch > 65535 || n_head > 65535) return TIQ_EUNSUPPORTED;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || (planes_out && !aligned(planes_out, 16))) return TIQ_EALIGN;
    const dim3 grid((unsigned)n_head, (unsigned)batch), block(64 * kAttWaves);
    // a small cache (keys and values of the layer under 32 MB) is read whole
    const bool whole = batch * n_kv_head * t_max * kHeadDim * 4 * 2 <= (32ll << 20);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, as_stream(stream), qkv, pos, k_cache, v_cache, (int)ld_qkv,
                           (int)n_head, (int)n_kv_head, (int)(n_head / n_kv_head), (int)t_max, y, ldy, planes_out,
                           (int)n_sl, batch * ld_qkv, sl_scale, sl_bias);
    };
    if (n_sl > 0) {
        if (t_max <= 128)
            whole ? launch(decode_attention_kernel<1, true, true>) : launch(decode_attention_kernel<1, false, true>);
        else whole ? launch(decode_attention_kernel<2, true, true>) : launch(decode_attention_kernel<2, false, true>);
    } else if (t_max <= 128) {
        whole ? launch(decode_attention_kernel<1, true, false>) : launch(decode_attention_kernel<1, false, false>);
    } else {
        whole ? launch(decode_attention_kernel<2, true, false>) : launch(decode_attention_kernel<2, false, false>);
    }
    return launch_status();
}

extern "C" int tiq_decode_attention(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head,
                                    int64_t n_kv_head, int64_t head_dim, float* k_cache, float* v_cache,
                                    int64_t t_max, const int64_t* pos, float* y, int64_t ldy, void* stream) {
    return decode_attention(qkv, ld_qkv, batch, n_head, n_kv_head, head_dim, k_cache, v_cache, t_max, pos, y, ldy,
                            nullptr, stream);
}

extern "C" int tiq_decode_attention_planes(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head,
                                           int64_t n_kv_head, int64_t head_dim, float* k_cache, float* v_cache,
                                           int64_t t_max, const int64_t* pos, float* y, int64_t ldy,
                                           uint16_t* planes_out, void* stream) {
    if (!planes_out) return TIQ_EINVAL;
    return decode_attention(qkv, ld_qkv, batch, n_head, n_kv_head, head_dim, k_cache, v_cache, t_max, pos, y, ldy,
                            planes_out, stream);
}

extern "C" size_t tiq_decode_qkv_attention_workspace(int64_t batch, int64_t n_embd, int64_t n_qkv) {
    return decode_slices_bytes(batch, n_embd, n_qkv);
}

extern "C" int tiq_decode_qkv_attention(const uint16_t* x_planes, int64_t batch, int64_t n_embd, const void* w,
                                        int w_format, const float* scale, const float* bias, int64_t n_head,
                                        int64_t n_kv_head, int64_t head_dim, float* k_cache, float* v_cache,
                                        int64_t t_max, const int64_t* pos, float* y, int64_t ldy,
                                        uint16_t* planes_out, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    if (w_format != TIQ_WF_INT8 && w_format != TIQ_WF_INT8_TILED) return TIQ_EUNSUPPORTED;
    if (batch < 0 || n_embd <= 0 || n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head) return TIQ_EINVAL;
    if (batch == 0) return TIQ_OK;
    if (!x_planes || !w || !scale || !k_cache || !v_cache || !pos || !y) return TIQ_EINVAL;
    if (head_dim != kHeadDim || t_max <= 0 || t_max > kMaxSlots) return TIQ_EUNSUPPORTED;
    if (batch > 64 || n_embd % 32 != 0) return TIQ_EUNSUPPORTED;
    if (ldy < n_head * head_dim) return TIQ_EINVAL;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || (planes_out && !aligned(planes_out, 16))) return TIQ_EALIGN;
    const int64_t N = (n_head + 2 * n_kv_head) * head_dim;
    if (N > INT32_MAX) return TIQ_EUNSUPPORTED;
    const size_t need = decode_slices_bytes(batch, n_embd, N);
    if (need == 0) return TIQ_EUNSUPPORTED;  // K beyond the product's splits
    if (!workspace || workspace_bytes < need) return TIQ_EWORKSPACE;
    if (!aligned(workspace, 16)) return TIQ_EALIGN;
    const WFormat fmt = w_format == TIQ_WF_INT8_TILED ? kW8T : kW8;
    LinearArgs a{};
    a.x_dtype = TIQ_F32;
    a.M = batch;
    a.K = n_embd;
    a.w = static_cast<const uint8_t*>(w);
    a.ldw = n_embd;  // row-major codes: rows of K bytes
    a.scale = scale;
    a.bias = bias;
    a.N = N;
    a.y_dtype = TIQ_F32;
    a.stream = as_stream(stream);
    a.fmt = fmt;
    float* part = static_cast<float*>(workspace);
    int rc = launch_decode_slices(a, x_planes, part);
    if (rc != TIQ_OK) return rc;
    return decode_attention(part, N, batch, n_head, n_kv_head, head_dim, k_cache, v_cache, t_max, pos, y, ldy,
                            planes_out, stream, decode_slices_count(batch, n_embd, N), scale, bias);
}

extern "C" int tiq_prefill_attention(const float* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const float* k,
                                     int64_t k_sb, int64_t k_sh, int64_t k_st, const float* v, int64_t v_sb,
                                     int64_t v_sh, int64_t v_st, int64_t batch, int64_t n_head, int64_t T,
                                     int64_t first, int64_t head_dim, float* y, int64_t y_sb, int64_t y_sh,
                                     int64_t y_st, void* stream) {
    if (batch < 0 || n_head <= 0 || T < 0 || first < 0) return TIQ_EINVAL;
    if (batch == 0 || T == 0) return TIQ_OK;
    if (!q || !k || !v || !y) return TIQ_EINVAL;
    if (head_dim != kHeadDim) return TIQ_EUNSUPPORTED;
    if (batch > 65535 || n_head > 65535 || T > INT32_MAX - kPaRows || first > INT32_MAX - T) return TIQ_EUNSUPPORTED;
    const int64_t strides[12] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, y_sb, y_sh, y_st};
    for (int64_t st : strides)
        if (st < 0 || st % 4 != 0) return TIQ_EALIGN;  // 16-byte rows of 4 floats
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(y, 16)) return TIQ_EALIGN;
    const dim3 grid((unsigned)((T + kPaRows - 1) / kPaRows), (unsigned)n_head, (unsigned)batch);
    hipLaunchKernelGGL(prefill_attention_kernel, grid, dim3(kPaThreads), 0, as_stream(stream), q, q_sb, q_sh, q_st, k, k_sb,
                       k_sh, k_st, v, v_sb, v_sh, v_st, (int)T, (int)first, y, y_sb, y_sh, y_st);
    return launch_status();
}

extern "C" int tiq_gelu_tanh(const float* x, float* y, int64_t n, void* stream) {
    if (n < 0) return TIQ_EINVAL;
    if (n == 0) return TIQ_OK;
    if (!x || !y) return TIQ_EINVAL;
    if (!aligned(x, 16) || !aligned(y, 16)) return TIQ_EALIGN;
    int64_t blocks = (n / 4 + 255) / 256;
    blocks = blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks);
    hipLaunchKernelGGL(gelu_tanh_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), x, y, n);
    return launch_status();
}

extern "C" int tiq_embed_tokens(const int64_t* tokens, const int64_t* pos, const float* wte, int64_t vocab,
                                const float* wpe, int64_t n_positions, int64_t batch, int64_t n_embd, float* x,
                                void* stream) {
    if (batch < 0 || n_embd <= 0 || vocab <= 0 || n_positions <= 0) return TIQ_EINVAL;
    if (batch == 0) return TIQ_OK;
    if (!tokens || !pos || !wte || !wpe || !x) return TIQ_EINVAL;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)batch), dim3(256), 0, as_stream(stream), tokens, pos, wte, wpe,
                       vocab, n_positions, n_embd, x);
    return launch_status();
}

extern "C" size_t tiq_head_screen_workspace(int64_t vocab) {
    if (vocab <= 0) return 0;
    return (size_t)kHsGroups * (sizeof(float) + sizeof(int));
}

extern "C" int tiq_head_screen_prepare(const float* w, int64_t vocab, int64_t n_embd, int64_t ldw, uint16_t* w_bf16,
                                       float* row_coef, void* stream) {
    if (vocab <= 0 || n_embd <= 0 || ldw < n_embd) return TIQ_EINVAL;
    if (!w || !w_bf16 || !row_coef) return TIQ_EINVAL;
    if (vocab > INT32_MAX || n_embd > INT32_MAX) return TIQ_EUNSUPPORTED;
    hipLaunchKernelGGL(head_screen_prepare_kernel, dim3((unsigned)vocab), dim3(256), 0, as_stream(stream), w,
                       (int)n_embd, ldw, w_bf16, row_coef);
    return launch_status();
}

extern "C" int tiq_head_screen_prepare_i8(const float* w, int64_t vocab, int64_t n_embd, int64_t ldw, int8_t* w_i8,
                                          float* row_scale, float* row_coef, void* stream) {
    if (vocab <= 0 || n_embd <= 0 || ldw < n_embd) return TIQ_EINVAL;
    if (!w || !w_i8 || !row_scale || !row_coef) return TIQ_EINVAL;
    if (vocab > INT32_MAX || n_embd > INT32_MAX) return TIQ_EUNSUPPORTED;
    hipLaunchKernelGGL(head_screen_prepare_i8_kernel, dim3((unsigned)vocab), dim3(256), 0, as_stream(stream), w,
                       (int)n_embd, ldw, w_i8, row_scale, row_coef);
    return launch_status();
}

static int head_argmax_screened(bool i8, const float* x, int64_t n_embd, const float* ln_w, const float* ln_b,
                                float ln_eps, const void* wq, const float* row_scale, const float* w, int64_t ldw,
                                const float* row_coef, int64_t vocab, float* logits, int64_t* out, int64_t* ids,
                                int64_t ld_ids, int64_t* pos, void* workspace, size_t workspace_bytes,
                                void* stream) {
    if (vocab <= 0 || n_embd <= 0 || ldw < n_embd) return TIQ_EINVAL;
    if (!x || !ln_w || !ln_b || !wq || (i8 && !row_scale) || !w || !row_coef || !logits || !out || (ids && !pos))
        return TIQ_EINVAL;
    if (!workspace) return TIQ_EINVAL;
    // every wavefront's chunks in its registers' reach (GPT-2's 50257 rows: 4 chunks of 4 bf16 rows or 2 of 8
    // int8 rows a wavefront)
    const int64_t rows_max = (int64_t)kHsMaxChunks * (i8 ? 2 * kHsChunk : kHsChunk) * kHsGroups * kHsWaves;
    if (n_embd % 16 != 0 || n_embd > kHsMaxCols || vocab > rows_max) return TIQ_EUNSUPPORTED;
    if (!aligned(x, 16) || !aligned(ln_w, 16) || !aligned(ln_b, 16) || !aligned(wq, 16) || !aligned(w, 16) ||
        ldw % 4 != 0)
        return TIQ_EALIGN;
    if (workspace_bytes < tiq_head_screen_workspace(vocab)) return TIQ_EWORKSPACE;
    if (!aligned(workspace, 4)) return TIQ_EALIGN;
    const int64_t P = kHsGroups;
    float* pv = static_cast<float*>(workspace);
    int* pi = reinterpret_cast<int*>(pv + P);
    hipStream_t st = as_stream(stream);
    if (i8 && n_embd == 768)  // 12 columns a lane: all 64 lanes busy
        hipLaunchKernelGGL((head_screen_kernel<true, 12>), dim3((unsigned)P), dim3(64 * kHsWaves), 0, st, x,
                           (int)n_embd, ln_w, ln_b, ln_eps, wq, row_scale, w, ldw, row_coef, (int)vocab, logits, pv, pi);
    else if (i8)
        hipLaunchKernelGGL(head_screen_kernel<true>, dim3((unsigned)P), dim3(64 * kHsWaves), 0, st, x, (int)n_embd,
                           ln_w, ln_b, ln_eps, wq, row_scale, w, ldw, row_coef, (int)vocab, logits, pv, pi);
    else
        hipLaunchKernelGGL(head_screen_kernel<false>, dim3((unsigned)P), dim3(64 * kHsWaves), 0, st, x, (int)n_embd,
                           ln_w, ln_b, ln_eps, wq, nullptr, w, ldw, row_coef, (int)vocab, logits, pv, pi);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_parts_kernel, dim3(1), dim3(1024), 0, st, pv, pi, (int)P, out, ids, ld_ids, pos);
    return launch_status();
}

extern "C" int tiq_head_argmax_screened(const float* x, int64_t n_embd, const float* ln_w, const float* ln_b,
                                        float ln_eps, const uint16_t* w_bf16, const float* w, int64_t ldw,
                                        const float* row_coef, int64_t vocab, float* logits, int64_t* out,
                                        int64_t* ids, int64_t ld_ids, int64_t* pos, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    return head_argmax_screened(false, x, n_embd, ln_w, ln_b, ln_eps, w_bf16, nullptr, w, ldw, row_coef, vocab,
                                logits, out, ids, ld_ids, pos, workspace, workspace_bytes, stream);
}

extern "C" int tiq_head_argmax_screened_i8(const float* x, int64_t n_embd, const float* ln_w, const float* ln_b,
                                           float ln_eps, const int8_t* w_i8, const float* row_scale, const float* w,
                                           int64_t ldw, const float* row_coef, int64_t vocab, float* logits,
                                           int64_t* out, int64_t* ids, int64_t ld_ids, int64_t* pos,
                                           void* workspace, size_t workspace_bytes, void* stream) {
    return head_argmax_screened(true, x, n_embd, ln_w, ln_b, ln_eps, w_i8, row_scale, w, ldw, row_coef, vocab,
                                logits, out, ids, ld_ids, pos, workspace, workspace_bytes, stream);
}

extern "C" size_t tiq_argmax_rows_workspace(int64_t rows) {
    return (size_t)(rows < 0 ? 0 : rows) * kArgParts * (sizeof(float) + sizeof(int64_t));
}

extern "C" int tiq_argmax_rows(const float* x, int64_t rows, int64_t cols, int64_t ld, int64_t* out, int64_t* ids,
                               int64_t ld_ids, int64_t* pos, void* workspace, size_t workspace_bytes,
                               void* stream) {
    if (rows < 0 || cols <= 0 || ld < cols || rows > 65535) return TIQ_EINVAL;
    if (rows == 0) return TIQ_OK;
    if (!x || !out || (ids && !pos) || !workspace) return TIQ_EINVAL;
    if (workspace_bytes < tiq_argmax_rows_workspace(rows)) return TIQ_EWORKSPACE;
    if (!aligned(workspace, 8)) return TIQ_EALIGN;
    int64_t* pi = reinterpret_cast<int64_t*>(workspace);
    float* pv = reinterpret_cast<float*>(pi + rows * kArgParts);
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgParts, (unsigned)rows), dim3(256), 0, st, x, cols, ld, pv, pi);
    int rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64 * kArgFinalWaves), 0, st, pv, pi, rows, out, ids, ld_ids,
                       pos);
    return launch_status();
}
