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

// One workgroup (4 wavefronts) per (sequence, head). Every global load the
// kernel needs for the first kPre key / value slots (the whole cache at
// GPT-2 decode lengths) is issued before the first barrier, so the kernel
// waits for HBM once; longer histories stream the rest in a second pass.
constexpr int kPreKeys = 128;  // slots whose key rows / values are prefetched

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

__global__ __launch_bounds__(256) void decode_attention_kernel(const float* __restrict__ qkv, int64_t ld_qkv, int H,
                                                               int Hkv, float* __restrict__ kc,
                                                               float* __restrict__ vc, int64_t t_max,
                                                               const int64_t* __restrict__ pos_p,
                                                               float* __restrict__ y, int64_t ldy,
                                                               uint16_t* __restrict__ x3) {
    __shared__ float qs[kHeadDim], kn[kHeadDim], vn[kHeadDim];
    __shared__ float sc[kMaxSlots];
    __shared__ float red[4];
    __shared__ float part[4][kHeadDim];
    __shared__ float ov[kHeadDim];
    const int b = blockIdx.x / H, h = blockIdx.x % H;
    const int group = H / Hkv, hk = h / group;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float* row = qkv + (int64_t)b * ld_qkv;
    const int C = H * kHeadDim, KV = Hkv * kHeadDim;
    float* kb = kc + ((int64_t)b * Hkv + hk) * t_max * kHeadDim;
    float* vb = vc + ((int64_t)b * Hkv + hk) * t_max * kHeadDim;

    // ---- issue every load of the first kPreKeys slots ----
    // No address depends on pos (a device scalar) and no load sits behind a
    // branch: slots are clamped into the cache and the values of slots >= pos
    // are dropped where they are used, so all loads are in flight together.
    const int64_t last = t_max - 1;
    // keys: slot t = (tid / 4) + 64 j, this lane's 16 dims at qd
    const int qd = (lane & 3) * 16;
    const int kslot = (wave * 16) + (lane >> 2);  // 0..63
    float4 kr[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t t = min((int64_t)(kslot + 64 * j), last);
#pragma unroll
        for (int q = 0; q < 4; ++q) kr[j][q] = reinterpret_cast<const float4*>(kb + t * kHeadDim + qd)[q];
    }
    // values: slot t = wave + 4 i, this lane's dim
    float vr[kPreKeys / 4];
#pragma unroll
    for (int i = 0; i < kPreKeys / 4; ++i) vr[i] = vb[min((int64_t)(wave + 4 * i), last) * kHeadDim + lane];
    float q_new = 0.f, k_new = 0.f, v_new = 0.f;
    if (tid < kHeadDim) {
        q_new = row[h * kHeadDim + tid];
        k_new = row[C + hk * kHeadDim + tid];
        v_new = row[C + KV + hk * kHeadDim + tid];
    }
    const int64_t pos = *pos_p;
    if (pos < 0 || pos >= t_max) {  // position outside the cache: flag the output, write nothing else
        if (tid < kHeadDim) y[(int64_t)b * ldy + h * kHeadDim + tid] = NAN;
        if (x3 && tid < kHeadDim / 8) {
            float nan8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) nan8[i] = NAN;
            store_planes(x3, b, H * kHeadDim, h * kHeadDim + 8 * tid, nan8);
        }
        return;
    }
    if (tid < kHeadDim) {
        qs[tid] = q_new;
        kn[tid] = k_new;
        vn[tid] = v_new;
        if (h % group == 0) {  // one writer per kv head
            kb[pos * kHeadDim + tid] = k_new;
            vb[pos * kHeadDim + tid] = v_new;
        }
    }
    __syncthreads();

    // ---- scores ----
    const float inv_div = 1.0f / sqrtf((float)kHeadDim);  // exactly 1/8
    // chunks of kPreKeys slots, this thread's two 64-slot rows each: the first
    // chunk's keys were loaded at the start, a later chunk's are all requested
    // before any is used (one trip to memory per chunk, slots clamped into the
    // cache; only slots < pos count, slot pos is the new key)
    for (int64_t base = 0; base <= pos; base += kPreKeys) {
        float4 kk[2][4];
        if (base == 0) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) kk[j][q] = kr[j][q];
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int64_t t = min(base + kslot + 64 * j, last);
#pragma unroll
                for (int q = 0; q < 4; ++q) kk[j][q] = reinterpret_cast<const float4*>(kb + t * kHeadDim + qd)[q];
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t t = base + kslot + 64 * j;
            float s = 0.f;
            if (t == pos) {
#pragma unroll
                for (int d = 0; d < 16; ++d) s = fmaf(qs[qd + d], kn[qd + d], s);
            } else if (t < pos) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    s = fmaf(qs[qd + 4 * q], kk[j][q].x, s);
                    s = fmaf(qs[qd + 4 * q + 1], kk[j][q].y, s);
                    s = fmaf(qs[qd + 4 * q + 2], kk[j][q].z, s);
                    s = fmaf(qs[qd + 4 * q + 3], kk[j][q].w, s);
                }
            }
            s += dpp_move<0xB1>(s);  // quad_perm [1, 0, 3, 2]: the lane xor 1
            s += dpp_move<0x4E>(s);  // quad_perm [2, 3, 0, 1]: the lane xor 2
            if ((lane & 3) == 0 && t <= pos) sc[t] = s * inv_div;
        }
    }
    __syncthreads();

    // ---- softmax over slots 0..pos ----
    float mx = -INFINITY;
    for (int64_t t = tid; t <= pos; t += 256) mx = fmaxf(mx, sc[t]);
    mx = wave_max_dpp(mx);
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
    sum = wave_sum_dpp(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);

    // ---- weighted sum of values: wavefront w takes slots t = w mod 4, lane = dim ----
    // (in chunks of kPreKeys slots as the scores: the first prefetched, a
    // later chunk's values all requested before any is used)
    float acc = 0.f;
    for (int64_t base = 0; base < pos; base += kPreKeys) {
        float vv[kPreKeys / 4];
        if (base == 0) {
#pragma unroll
            for (int i = 0; i < kPreKeys / 4; ++i) vv[i] = vr[i];
        } else {
#pragma unroll
            for (int i = 0; i < kPreKeys / 4; ++i) vv[i] = vb[min(base + wave + 4 * i, last) * kHeadDim + lane];
        }
#pragma unroll
        for (int i = 0; i < kPreKeys / 4; ++i) {
            const int64_t t = base + wave + 4 * i;
            if (t < pos) acc = fmaf(sc[t], vv[i], acc);
        }
    }
    if ((pos & 3) == wave) acc = fmaf(sc[pos], vn[lane], acc);
    part[wave][lane] = acc;
    __syncthreads();
    if (tid < kHeadDim) {
        const float o = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
        y[(int64_t)b * ldy + h * kHeadDim + tid] = o / sum;
        ov[tid] = o / sum;
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

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pv, const int64_t* __restrict__ pi,
                                                          int64_t rows, int64_t* __restrict__ out,
                                                          int64_t* __restrict__ ids, int64_t ld_ids,
                                                          int64_t* __restrict__ pos_p) {
    const int lane = threadIdx.x;
    const int64_t col = pos_p ? *pos_p + 1 : 0;
    for (int64_t r = 0; r < rows; ++r) {
        float v = pv[r * kArgParts + lane];
        int64_t idx = pi[r * kArgParts + lane];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
        if (lane == 0) {
            out[r] = idx;
            if (ids && col >= 0 && col < ld_ids) ids[r * ld_ids + col] = idx;
        }
    }
    if (lane == 0 && pos_p && ids) *pos_p = col;  // every read of the position in this step came before
}

}  // namespace
}  // namespace tiq

using namespace tiq;

static int decode_attention(const float* qkv, int64_t ld_qkv, int64_t batch, int64_t n_head, int64_t n_kv_head,
                            int64_t head_dim, float* k_cache, float* v_cache, int64_t t_max, const int64_t* pos,
                            float* y, int64_t ldy, uint16_t* planes_out, void* stream) {
    if (batch < 0 || n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head) return TIQ_EINVAL;
    if (batch == 0) return TIQ_OK;
    if (!qkv || !k_cache || !v_cache || !pos || !y) return TIQ_EINVAL;
    if (head_dim != kHeadDim || t_max <= 0 || t_max > kMaxSlots) return TIQ_EUNSUPPORTED;
    if (ld_qkv < (n_head + 2 * n_kv_head) * head_dim || ldy < n_head * head_dim) return TIQ_EINVAL;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || (planes_out && !aligned(planes_out, 16))) return TIQ_EALIGN;
    hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)(batch * n_head)), dim3(256), 0, as_stream(stream), qkv,
                       ld_qkv, (int)n_head, (int)n_kv_head, k_cache, v_cache, t_max, pos, y, ldy, planes_out);
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
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(64), 0, st, pv, pi, rows, out, ids, ld_ids, pos);
    return launch_status();
}
