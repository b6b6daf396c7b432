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
#include "tiq_internal.hpp"

namespace tiq {
namespace {

constexpr int kHeadDim = 64;    // every released GPT-2 size
constexpr int kMaxSlots = 1024;  // n_positions of GPT-2

// One workgroup (4 wavefronts) per (sequence, head).
__global__ __launch_bounds__(256) void decode_attention_kernel(const float* __restrict__ qkv, int64_t ld_qkv, int H,
                                                               int Hkv, float* __restrict__ kc,
                                                               float* __restrict__ vc, int64_t t_max,
                                                               const int64_t* __restrict__ pos_p,
                                                               float* __restrict__ y, int64_t ldy) {
    __shared__ float qs[kHeadDim], kn[kHeadDim], vn[kHeadDim];
    __shared__ float sc[kMaxSlots];
    __shared__ float red[4];
    __shared__ float part[4][kHeadDim];
    const int b = blockIdx.x / H, h = blockIdx.x % H;
    const int group = H / Hkv, hk = h / group;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t pos = *pos_p;
    if (pos < 0 || pos >= t_max) {  // position outside the cache: flag the output, touch nothing else
        if (tid < kHeadDim) y[(int64_t)b * ldy + h * kHeadDim + tid] = NAN;
        return;
    }
    const float* row = qkv + (int64_t)b * ld_qkv;
    const int C = H * kHeadDim, KV = Hkv * kHeadDim;
    float* kb = kc + ((int64_t)b * Hkv + hk) * t_max * kHeadDim;
    float* vb = vc + ((int64_t)b * Hkv + hk) * t_max * kHeadDim;
    if (tid < kHeadDim) {
        qs[tid] = row[h * kHeadDim + tid];
        kn[tid] = row[C + hk * kHeadDim + tid];
        vn[tid] = row[C + KV + hk * kHeadDim + tid];
        if (h % group == 0) {  // one writer per kv head
            kb[pos * kHeadDim + tid] = kn[tid];
            vb[pos * kHeadDim + tid] = vn[tid];
        }
    }
    __syncthreads();

    // scores: 16 keys per wavefront pass, 4 lanes per key (16 dims each)
    const float inv_div = 1.0f / sqrtf((float)kHeadDim);  // exactly 1/8
    const int qd = (lane & 3) * 16;
    for (int64_t t0 = wave * 16; t0 <= pos; t0 += 64) {
        const int64_t t = t0 + (lane >> 2);
        float s = 0.f;
        if (t <= pos) {
            if (t == pos) {
#pragma unroll
                for (int d = 0; d < 16; ++d) s = fmaf(qs[qd + d], kn[qd + d], s);
            } else {
                const float4* kr = reinterpret_cast<const float4*>(kb + t * kHeadDim + qd);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 k4 = kr[j];
                    s = fmaf(qs[qd + 4 * j], k4.x, s);
                    s = fmaf(qs[qd + 4 * j + 1], k4.y, s);
                    s = fmaf(qs[qd + 4 * j + 2], k4.z, s);
                    s = fmaf(qs[qd + 4 * j + 3], k4.w, s);
                }
            }
        }
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((lane & 3) == 0 && t <= pos) sc[t] = s * inv_div;
    }
    __syncthreads();

    // softmax over slots 0..pos
    float mx = -INFINITY;
    for (int64_t t = tid; t <= pos; t += 256) mx = fmaxf(mx, sc[t]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (int64_t t = tid; t <= pos; t += 256) {
        const float p = expf(sc[t] - mx);
        sc[t] = p;
        sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);

    // weighted sum of values: wavefront w takes slots t = w mod 4, lane = dim
    float acc = 0.f;
    for (int64_t t = wave; t <= pos; t += 4) {
        const float v = (t == pos) ? vn[lane] : vb[t * kHeadDim + lane];
        acc = fmaf(sc[t], v, acc);
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (tid < kHeadDim) {
        const float o = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
        y[(int64_t)b * ldy + h * kHeadDim + tid] = o / sum;
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

__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int64_t cols, int64_t ld,
                                                      int64_t* __restrict__ out, int64_t* __restrict__ ids,
                                                      int64_t ld_ids, const int64_t* __restrict__ pos_p) {
    __shared__ float bv[16];
    __shared__ int64_t bi[16];
    const int64_t r = blockIdx.x;
    const float* xr = x + r * ld;
    float v = -INFINITY;
    int64_t idx = 0;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float a = xr[c];
        if (a > v) {
            v = a;
            idx = c;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int64_t oi = __shfl_xor(idx, off, 64);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    if (lane == 0) {
        bv[wave] = v;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i)
            if (bv[i] > v || (bv[i] == v && bi[i] < idx)) {
                v = bv[i];
                idx = bi[i];
            }
        out[r] = idx;
        if (ids) {
            const int64_t col = *pos_p + 1;
            if (col >= 0 && col < ld_ids) ids[r * ld_ids + col] = idx;
        }
    }
}

}  // namespace
}  // namespace tiq

using namespace tiq;

extern "C" int tiq_decode_attention(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head,
                                    int64_t n_kv_head, int64_t head_dim, float* k_cache, float* v_cache,
                                    int64_t t_max, const int64_t* pos, float* y, int64_t ldy, void* stream) {
    if (batch < 0 || n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head) return TIQ_EINVAL;
    if (batch == 0) return TIQ_OK;
    if (!qkv || !k_cache || !v_cache || !pos || !y) return TIQ_EINVAL;
    if (head_dim != kHeadDim || t_max <= 0 || t_max > kMaxSlots) return TIQ_EUNSUPPORTED;
    if (ld_qkv < (n_head + 2 * n_kv_head) * head_dim || ldy < n_head * head_dim) return TIQ_EINVAL;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16)) return TIQ_EALIGN;
    hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)(batch * n_head)), dim3(256), 0, as_stream(stream), qkv,
                       ld_qkv, (int)n_head, (int)n_kv_head, k_cache, v_cache, t_max, pos, y, ldy);
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

extern "C" int tiq_argmax_rows(const float* x, int64_t rows, int64_t cols, int64_t ld, int64_t* out, int64_t* ids,
                               int64_t ld_ids, const int64_t* pos, void* stream) {
    if (rows < 0 || cols <= 0 || ld < cols) return TIQ_EINVAL;
    if (rows == 0) return TIQ_OK;
    if (!x || !out || (ids && !pos)) return TIQ_EINVAL;
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, as_stream(stream), x, cols, ld, out, ids,
                       ld_ids, pos);
    return launch_status();
}
