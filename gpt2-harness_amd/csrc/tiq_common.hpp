// Shared device helpers and host-side launch plumbing for libtiq_hip.so.
// CDNA4 (gfx950) only: 64-lane wavefronts, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "tiq.h"

namespace tiq {

constexpr int kWave = 64;

inline int status_of(hipError_t e) { return e == hipSuccess ? TIQ_OK : TIQ_EHIP_BASE - (int)e; }

// Status of the most recent launch on this thread.
inline int launch_status() { return status_of(hipGetLastError()); }

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------ device helpers

// |x| as raw bits. For non-negative floats integer order is float order and
// every NaN sorts above +inf, so an unsigned max propagates NaN like torch.amax.
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    return v;
}

// Max over aligned groups of `width` lanes (width a power of two <= 64).
template <int Width>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
#pragma unroll
    for (int off = Width / 2; off >= 1; off >>= 1) {
        uint32_t o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// x moved across lanes by DPP control CTRL; lanes of rows outside ROW_MASK
// get `keep` (0 by default).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float x, float keep = 0.f) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(keep), __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wavefront with DPP lane moves (VALU operations,
// no round trips through the LDS crossbar as with shuffles): pairs and quads
// (quad_perm), 8 and 16 lanes (row_half_mirror, row_mirror), then rows 0 -> 1
// and 2 -> 3 (row_bcast:15) and rows 0-1 -> 2-3 (row_bcast:31); lane 63 holds
// the total, which every lane receives. All 64 lanes must be active.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_move<0xB1>(v);        // quad_perm [1, 0, 3, 2]
    v += dpp_move<0x4E>(v);        // quad_perm [2, 3, 0, 1]
    v += dpp_move<0x141>(v);       // row_half_mirror
    v += dpp_move<0x140>(v);       // row_mirror
    v += dpp_move<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_move<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum over the 64 lanes, the same moves as wave_sum_dpp (lanes outside a
// broadcast's rows keep their own value). All 64 lanes must be active.
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    v = fmaxf(v, dpp_move<0x142, 0xa>(v, v));
    v = fmaxf(v, dpp_move<0x143, 0xc>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// (amax / qmax).clamp(min=FLT_MIN) with the IEEE correctly rounded division
// (hipcc keeps fp32 division correctly rounded unless told otherwise; this
// library is never built with fast-math). NaN passes through the clamp.
__device__ __forceinline__ float scale_from_amax(float amax, float qmax) {
    float s = amax / qmax;
    return (s < 1.17549435e-38f) ? 1.17549435e-38f : s;
}

// clamp(rint_half_even(w / s), qmin, qmax) as an int.
__device__ __forceinline__ int code_of(float w, float s, float qmin, float qmax) {
    float r = __builtin_rintf(w / s);
    r = r < qmin ? qmin : r;
    r = r > qmax ? qmax : r;
    return (int)r;
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> fp16 bits, round to nearest even (hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// bf16 packing for the exact three-plane split of fp32 activations:
// x = hi + lo + lo2 with hi = bf16(x), lo = bf16(x - hi), lo2 = bf16(x - hi - lo)
// (round to nearest even; the residues are exact in fp32).
typedef __bf16 tiq_bf16x2 __attribute__((ext_vector_type(2)));
typedef float tiq_floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    const tiq_bf16x2 v = __builtin_convertvector(tiq_floatx2{a, b}, tiq_bf16x2);
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
// The three planes of 8 consecutive values, each as 4 packed bf16 pairs.
__device__ __forceinline__ void split3_words(const float (&x)[8], uint32_t (&pl)[3][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = x[2 * i], x1 = x[2 * i + 1];
        const uint32_t h = pk_bf16(x0, x1);
        const float r0 = x0 - bf_lo(h), r1 = x1 - bf_hi(h);
        const uint32_t l = pk_bf16(r0, r1);
        pl[0][i] = h;
        pl[1][i] = l;
        pl[2][i] = pk_bf16(r0 - bf_lo(l), r1 - bf_hi(l));
    }
}

// Sign-extended byte `i` of a dword, as float.
// Signed bytes sh / 8 and sh / 8 + 1 of d as two bf16 (low half = the lower
// byte): an int8 code is exact in bf16, so the top half of its float is it.
__device__ __forceinline__ uint32_t bf16x2_of_bytes_perm(uint32_t d, int sh) {
    const float lo = (float)((int32_t)(d << (24 - sh)) >> 24);
    const float hi = (float)((int32_t)(d << (16 - sh)) >> 24);
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

template <int I>
__device__ __forceinline__ float sbyte_f32(uint32_t d) {
    return (float)((int32_t)(d << (24 - 8 * I)) >> 24);
}

// Nibble `i` (0..7) of a dword minus the +8 bias, as float.
template <int I>
__device__ __forceinline__ float nibble_f32(uint32_t d) {
    return (float)((int32_t)((d >> (4 * I)) & 0xfu) - 8);
}

// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
__device__ __forceinline__ float gelu_tanh(float x) {
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

// Activation code 1 (GELU) applied to n values behind a real branch. Left to
// itself the compiler evaluates the GELU unconditionally and selects the
// result; those ~45 instructions (two transcendentals) then lengthen every
// wavefront's tail, ~0.2 us per launch of a latency-bound kernel, also when
// no activation is asked for. The empty volatile asm cannot be speculated,
// so the block stays behind the branch.
template <int n>
__device__ __forceinline__ void apply_act(float (&v)[n], int act) {
    if (act == 1) {
        asm volatile("");
#pragma unroll
        for (int i = 0; i < n; ++i) v[i] = gelu_tanh(v[i]);
    }
}
__device__ __forceinline__ float apply_act(float v, int act) {
    float t[1] = {v};
    apply_act<1>(t, act);
    return t[0];
}

// Per-workgroup entry and exit of a measurement launch: slots 4 g and 4 g + 1
// hold workgroup g's entry and exit on the GPU's 100 MHz real-time counter,
// 4 g + 2 and 4 g + 3 the same two moments on the shader-clock counter (its
// ratio to the real time is the clock the workgroup ran at). Off (ON =
// false) the kernel is the product kernel, unchanged.
template <bool ON>
struct Stamp {
    uint64_t t0 = 0, c0 = 0;
    __device__ __forceinline__ void start() {
        if constexpr (ON) {
            t0 = __builtin_amdgcn_s_memrealtime();
            c0 = __builtin_amdgcn_s_memtime();
        }
    }
    // after the workgroup's last store is issued; thread 0 writes the slots
    __device__ __forceinline__ void finish(uint64_t* slots, int64_t wg) {
        if constexpr (ON) {
            const uint64_t c1 = __builtin_amdgcn_s_memtime();
            const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
            if (threadIdx.x == 0 && slots) {
                slots[4 * wg] = t0;
                slots[4 * wg + 1] = t1;
                slots[4 * wg + 2] = c0;
                slots[4 * wg + 3] = c1;
            }
        }
    }
};

}  // namespace tiq
