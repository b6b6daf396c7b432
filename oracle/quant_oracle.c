/*
 * CPU restatement of the reference's weight quantization arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP kernels are
 * compared against; nothing in the shipped library links or calls it.
 *
 * Every function restates, element by element, the torch op chain in
 * src/transformer_internals/quantization.py of the reference:
 *
 *   quantize_tensor   quantization.py:78-116
 *       qmax = 2^(b-1)-1, qmin = -2^(b-1)
 *       amax = |w|.amax(dim=1) (per_channel) or |w|.amax() (per_tensor)
 *       scale = (amax / qmax).clamp(min=FLT_MIN)        IEEE fp32 divide
 *       q = round_half_even(w / scale).clamp(qmin, qmax).to(int8)
 *   pack_int4         quantization.py:132-149
 *       flatten row-major, +8, pad one zero nibble if odd, byte=(odd<<4)|even
 *   unpack_int4       quantization.py:152-158
 *   quantize_dequantize quantization.py:119-129   (q.float() * scale)
 *
 * The group-wise int4 format (groupwise_int4 below) has no counterpart in the
 * reference; it follows the build's own specification: groups of `group`
 * consecutive columns inside a row (the last one ragged), scale_f32 =
 * amax/7, stored as fp16 (round to nearest even, a zero result replaced by the
 * smallest positive fp16, an overflow saturated to 65504), codes
 * rint(w / float(scale_f16)) clamped to [-8, 7], nibbles packed per row with
 * the reference's convention (low nibble = even column, +8 bias), row stride
 * ceil(cols/2) bytes, a pad nibble of 0 when cols is odd.
 *
 * Built with -ffp-contract=off and without -ffast-math: every division is the
 * IEEE correctly rounded one and rintf() rounds half to even under the default
 * rounding mode, which is what torch.div and torch.round compute.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* |x| as raw bits: for non-negative floats integer order equals float order,
 * and every NaN compares above +inf, so the maximum propagates NaN the way
 * torch.amax does. */
static uint32_t abs_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof u);
    return u & 0x7fffffffu;
}

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* (amax / qmax).clamp(min=torch.finfo(float32).tiny)  -- quantization.py:114 */
static float scale_from_amax(float amax, int qmax) {
    float s = amax / (float)qmax;
    if (s < 1.17549435e-38f) s = 1.17549435e-38f; /* NaN compares false: kept */
    return s;
}

/* round(w / scale).clamp(qmin, qmax).to(int8)  -- quantization.py:115 */
static int8_t code_of(float w, float scale, int qmin, int qmax) {
    float r = rintf(w / scale);
    if (r < (float)qmin) r = (float)qmin;
    if (r > (float)qmax) r = (float)qmax;
    return (int8_t)r;
}

int oracle_quantize_per_channel(const float* w, int64_t rows, int64_t cols, int bits,
                                int8_t* q, float* scale) {
    if (bits < 2 || bits > 8) return -1;
    const int qmax = (1 << (bits - 1)) - 1, qmin = -(1 << (bits - 1));
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        uint32_t m = 0;
        for (int64_t c = 0; c < cols; ++c) {
            uint32_t a = abs_bits(row[c]);
            if (a > m) m = a;
        }
        const float s = scale_from_amax(bits_to_float(m), qmax);
        scale[r] = s;
        for (int64_t c = 0; c < cols; ++c) q[r * cols + c] = code_of(row[c], s, qmin, qmax);
    }
    return 0;
}

int oracle_quantize_per_tensor(const float* w, int64_t numel, int bits, int8_t* q,
                               float* scale) {
    if (bits < 2 || bits > 8) return -1;
    const int qmax = (1 << (bits - 1)) - 1, qmin = -(1 << (bits - 1));
    uint32_t m = 0;
    for (int64_t i = 0; i < numel; ++i) {
        uint32_t a = abs_bits(w[i]);
        if (a > m) m = a;
    }
    const float s = scale_from_amax(bits_to_float(m), qmax);
    *scale = s;
    for (int64_t i = 0; i < numel; ++i) q[i] = code_of(w[i], s, qmin, qmax);
    return 0;
}

void oracle_pack_int4(const int8_t* q, int64_t numel, uint8_t* packed) {
    const int64_t nbytes = (numel + 1) / 2;
    for (int64_t j = 0; j < nbytes; ++j) {
        const int lo = q[2 * j] + 8;
        const int hi = (2 * j + 1 < numel) ? q[2 * j + 1] + 8 : 0;
        packed[j] = (uint8_t)(((hi << 4) | lo) & 0xff);
    }
}

void oracle_unpack_int4(const uint8_t* packed, int64_t numel, int8_t* q) {
    for (int64_t i = 0; i < numel; ++i) {
        const uint8_t b = packed[i / 2];
        const int nib = (i & 1) ? (b >> 4) & 0xf : b & 0xf;
        q[i] = (int8_t)(nib - 8);
    }
}

void oracle_dequantize(const int8_t* q, const float* scale, int64_t rows, int64_t cols,
                       int per_channel, float* w_hat) {
    for (int64_t r = 0; r < rows; ++r) {
        const float s = per_channel ? scale[r] : scale[0];
        for (int64_t c = 0; c < cols; ++c) w_hat[r * cols + c] = (float)q[r * cols + c] * s;
    }
}

/* ---- fp16 round-to-nearest-even from fp32, written out on the bits ---- */
uint16_t oracle_f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or NaN */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) /* rounds to >= 65520: overflow to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) { /* normal fp16 range: >= 2^-14 */
        const uint32_t mant = ax & 0x7fffffu;
        uint32_t h = ((ax >> 23) - 112u) << 10 | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) /* below half of the smallest subnormal 2^-24 */
        return (uint16_t)sign;
    /* subnormal fp16: value = m * 2^-24 with m in [0, 1023] */
    const uint32_t e = ax >> 23;            /* biased fp32 exponent, 102..112 */
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;        /* so that result = mant >> shift */
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        const float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 31) return bits_to_float(sign | 0x7f800000u | (m << 13));
    return bits_to_float(sign | ((e + 112u) << 23) | (m << 13));
}

int oracle_quantize_groupwise_int4(const float* w, int64_t rows, int64_t cols, int group,
                                   uint8_t* packed, uint16_t* scale_f16) {
    if (group < 2 || (group & 1)) return -1;
    const int64_t ngroups = (cols + group - 1) / group;
    const int64_t stride = (cols + 1) / 2;
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        uint8_t* prow = packed + r * stride;
        memset(prow, 0, (size_t)stride);
        for (int64_t g = 0; g < ngroups; ++g) {
            const int64_t c0 = g * group;
            const int64_t c1 = (c0 + group < cols) ? c0 + group : cols;
            uint32_t m = 0;
            for (int64_t c = c0; c < c1; ++c) {
                uint32_t a = abs_bits(row[c]);
                if (a > m) m = a;
            }
            uint16_t h = oracle_f32_to_f16_rne(bits_to_float(m) / 7.0f);
            if (h == 0) h = 1;                 /* smallest positive fp16 */
            if (h > 0x7bffu) h = 0x7bffu;      /* saturate at 65504 (NaN too) */
            scale_f16[r * ngroups + g] = h;
            const float s = oracle_f16_to_f32(h);
            for (int64_t c = c0; c < c1; ++c) {
                const int code = code_of(row[c], s, -8, 7) + 8;
                prow[c / 2] |= (uint8_t)((c & 1) ? code << 4 : code);
            }
        }
    }
    return 0;
}
