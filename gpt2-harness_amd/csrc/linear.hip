// Linear entry points of the C ABI: argument checks and the choice between
// the decode GEMV (vector ALUs) and the prefill GEMM (matrix cores).
#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

#include "tiq_internal.hpp"

namespace tiq {

int check_linear(const LinearArgs& a) {
    if (a.x_dtype != TIQ_F32 && a.x_dtype != TIQ_BF16) return TIQ_EINVAL;
    if (a.y_dtype != TIQ_F32 && a.y_dtype != TIQ_BF16) return TIQ_EINVAL;
    if (a.M < 0 || a.N < 0 || a.K < 0) return TIQ_EINVAL;
    if (a.M == 0 || a.N == 0) return TIQ_OK;
    if (a.K == 0) return TIQ_EINVAL;
    if (!a.x || !a.w || !a.y) return TIQ_EINVAL;
    if (a.fmt == kW4G ? !a.scale16 : !a.scale) return TIQ_EINVAL;
    if (a.ldx < a.K || a.ldy < a.N) return TIQ_EINVAL;
    if (a.M > 0x7fffffff || a.N > 0x7fffffff || a.K > 0x7fffffff) return TIQ_EUNSUPPORTED;
    if (a.fmt == kW4 && (a.K % 2)) return TIQ_EINVAL;
    if (a.fmt == kW4G && (a.group < 2 || (a.group & 1))) return TIQ_EINVAL;
    return TIQ_OK;
}

// Measurement state of tiq_stamp_begin / tiq_stamp_end: the caller's stamp
// buffer, the slots handed out so far and, per stamped launch, its first
// slot and workgroup count.
namespace {
struct StampState {
    std::mutex mu;
    uint64_t* base = nullptr;
    int64_t slots = 0, used = 0;
    std::vector<std::pair<int64_t, int64_t>> log;
};
StampState& stamp_state() {
    static StampState st;
    return st;
}
}  // namespace

uint64_t* stamp_slots(int64_t workgroups) {
    StampState& st = stamp_state();
    std::lock_guard<std::mutex> lk(st.mu);
    if (!st.base || workgroups <= 0 || st.used + 4 * workgroups > st.slots) return nullptr;
    uint64_t* p = st.base + st.used;
    st.log.emplace_back(st.used, workgroups);
    st.used += 4 * workgroups;
    return p;
}

namespace {

// Rows of M at and above which the 128 x 128-tile MFMA GEMM beats the
// vector-ALU GEMV (below it the GEMM wastes most of each tile).
constexpr int64_t kGemmMinRows = 128;

// fp32 rows against reference-layout int4 codes take the three-plane
// matrix-core path (split over K where the tiles are few) from 32 rows, or
// from 16 on matrices of 2048 rows or more: below 128 rows there is no
// batched kernel for int4, and the LDS-staged GEMV, four activation rows a
// tile, grows with M (GPT-2 small shapes at M = 64: 18-57 us against 12-19 us
// through the planes; int8 has the batched kernel up to 64 rows).
bool w4_planes_rows(int64_t M, int64_t N) { return M >= 32 || (M >= 16 && N >= 2048); }

LinearArgs make_args(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w, int64_t ldw,
                     const float* scale, const uint16_t* scale16, int group, const float* bias, int64_t N, void* y,
                     int y_dtype, int64_t ldy, void* stream, WFormat fmt) {
    LinearArgs a;
    a.x = x;
    a.x_dtype = x_dtype;
    a.M = M;
    a.K = K;
    a.ldx = ldx;
    a.w = w;
    a.ldw = ldw;
    a.scale = scale;
    a.scale16 = scale16;
    a.group = group;
    a.bias = bias;
    a.N = N;
    a.y = y;
    a.y_dtype = y_dtype;
    a.ldy = ldy;
    a.stream = as_stream(stream);
    a.fmt = fmt;
    return a;
}

// x (M, K) fp32 -> x3 (M, 3K) bf16: [hi | lo | lo2] with hi = rne(x),
// lo = rne(x - hi), lo2 = rne(x - hi - lo). Both differences are exact in fp32
// and lo2 holds the last 8 significant bits, so hi + lo + lo2 == x; an int8
// weight is exact in bf16, so every product the MFMA forms is exact and the
// GEMM over the three planes is as accurate as an fp32 GEMM. gelu: the planes
// of gelu_tanh(x) (the same function as tiq_gelu_tanh's), x read once.
__global__ void split_bf16x3_kernel(const float* __restrict__ x, int64_t ldx, int M, int K,
                                    uint16_t* __restrict__ x3, bool gelu) {
    const int k4 = K / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * k4) return;
    const int m = (int)(i / k4), k = (int)(i % k4) * 4;
    float4 v = *reinterpret_cast<const float4*>(x + (int64_t)m * ldx + k);
    if (gelu) {
        v.x = gelu_tanh(v.x);
        v.y = gelu_tanh(v.y);
        v.z = gelu_tanh(v.z);
        v.w = gelu_tanh(v.w);
    }
    // pairs through v_cvt_pk_bf16_f32 (round to nearest even)
    uint32_t p[3][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float x0 = e ? v.z : v.x, x1 = e ? v.w : v.y;
        const uint32_t hi = pk_bf16(x0, x1);
        const float r0 = x0 - bf_lo(hi), r1 = x1 - bf_hi(hi);
        const uint32_t lo = pk_bf16(r0, r1);
        p[0][e] = hi;
        p[1][e] = lo;
        p[2][e] = pk_bf16(r0 - bf_lo(lo), r1 - bf_hi(lo));
    }
    uint16_t* row = x3 + (int64_t)m * 3 * K + k;
#pragma unroll
    for (int q = 0; q < 3; ++q) *reinterpret_cast<uint2*>(row + (int64_t)q * K) = make_uint2(p[q][0], p[q][1]);
}

size_t split_workspace(int64_t M, int64_t K) { return (size_t)(M * 3 * K * 2 + 255) / 256 * 256; }

// fp32 activations through the matrix cores when a GEMM takes the three-plane
// problem (the staged kernel, else the LDS-dequant one); TIQ_EUNSUPPORTED
// otherwise (the caller falls back). gelu_in: the product takes gelu_tanh(x).
int run_linear_split(const LinearArgs& a, void* ws, size_t ws_bytes, bool gelu_in = false) {
    if (a.x_dtype != TIQ_F32 || a.fmt == kF32 || a.K % 4 != 0) return TIQ_EUNSUPPORTED;
    const bool few = a.M < kGemmMinRows;  // below the GEMM's own row count: int4 from fewer rows
    if (few && !(a.fmt == kW4 && w4_planes_rows(a.M, a.N))) return TIQ_EUNSUPPORTED;
    if (!aligned(a.x, 16) || a.ldx % 4 != 0 || a.M * 3 * a.K > 0x7fffffffLL) return TIQ_EUNSUPPORTED;
    LinearArgs g = a;
    g.x = ws;
    g.x_dtype = TIQ_BF16;
    g.K = 3 * a.K;
    g.ldx = 3 * a.K;
    g.kw = a.K;
    const bool staged = staged_gemm_supported(g);
    if (!staged && !gemm_supported(g)) return TIQ_EUNSUPPORTED;
    if (!ws || ws_bytes < split_workspace(a.M, a.K) || !aligned(ws, 16))
        return few ? TIQ_EUNSUPPORTED : TIQ_EWORKSPACE;  // with fewer rows the GEMV path takes it
    const int64_t n = a.M * (a.K / 4);
    hipLaunchKernelGGL(split_bf16x3_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, a.stream,
                       static_cast<const float*>(a.x), a.ldx, (int)a.M, (int)a.K, static_cast<uint16_t*>(ws),
                       gelu_in);
    int rc = launch_status();
    if (rc != TIQ_OK) return rc;
    if (!staged) return launch_gemm(g);
    // a workspace sized by tiq_gemm_w8_workspace also holds split-K partials
    const size_t planes = split_workspace(a.M, a.K);
    rc = launch_staged_gemm_split(g, static_cast<uint8_t*>(ws) + planes, ws_bytes - planes);
    if (rc != TIQ_EUNSUPPORTED) return rc;
    return launch_staged_gemm(g, staged_gemm_choice(g));
}

int run_linear(const LinearArgs& a) {
    int rc = check_linear(a);
    if (rc != TIQ_OK || a.M == 0 || a.N == 0) return rc;
    if (rows16_preferred(a)) return launch_rows16(a);
    if (skinny_supported(a)) return launch_skinny(a);
    if (a.M >= kGemmMinRows && gemm_supported(a)) return launch_gemm(a);
    return launch_gemv(a);
}

}  // namespace
}  // namespace tiq

using namespace tiq;

extern "C" int tiq_version(void) { return 126; }

extern "C" const char* tiq_status_string(int status) {
    switch (status) {
        case TIQ_OK: return "ok";
        case TIQ_EINVAL: return "invalid argument";
        case TIQ_EBITS: return "bits must be in [2, 8]";
        case TIQ_EALIGN: return "misaligned pointer or leading dimension";
        case TIQ_EUNSUPPORTED: return "unsupported shape or layout";
        case TIQ_EWORKSPACE: return "workspace too small";
        case TIQ_ESCRATCH: return "request exceeds the fixed scratch of the allocation-free entry point";
        default: break;
    }
    if (status <= TIQ_EHIP_BASE) return hipGetErrorString((hipError_t)(TIQ_EHIP_BASE - status));
    return "unknown status";
}

extern "C" int tiq_stamp_begin(uint64_t* buf, int64_t slots) {
    if (slots < 0 || (slots > 0 && !buf)) return TIQ_EINVAL;
    StampState& st = stamp_state();
    std::lock_guard<std::mutex> lk(st.mu);
    st.base = slots ? buf : nullptr;
    st.slots = slots;
    st.used = 0;
    st.log.clear();
    return TIQ_OK;
}

extern "C" int64_t tiq_stamp_end(int64_t* first_slot, int64_t* workgroups, int64_t max_launches) {
    StampState& st = stamp_state();
    std::lock_guard<std::mutex> lk(st.mu);
    const int64_t n = (int64_t)st.log.size();
    for (int64_t i = 0; i < n && i < max_launches; ++i) {
        if (first_slot) first_slot[i] = st.log[i].first;
        if (workgroups) workgroups[i] = st.log[i].second;
    }
    st.base = nullptr;
    st.slots = st.used = 0;
    st.log.clear();
    return n;
}

extern "C" int tiq_linear_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                             const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                             void* stream) {
    return run_linear(make_args(x, x_dtype, M, K, ldx, reinterpret_cast<const uint8_t*>(q), K, scale, nullptr, 0,
                                bias, N, y, y_dtype, ldy, stream, kW8));
}

extern "C" size_t tiq_linear_w8_workspace(int x_dtype, int64_t M, int64_t K) {
    if (x_dtype != TIQ_F32 || M < kGemmMinRows || K <= 0 || K % 64 != 0) return 0;
    return split_workspace(M, K);
}

extern "C" int tiq_linear_w8_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                                const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                                void* workspace, size_t workspace_bytes, void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, reinterpret_cast<const uint8_t*>(q), K, scale, nullptr, 0, bias,
                             N, y, y_dtype, ldy, stream, kW8);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    rc = run_linear_split(a, workspace, workspace_bytes);
    if (rc != TIQ_EUNSUPPORTED) return rc;
    if (a.x_dtype == TIQ_BF16 && M >= kGemmMinRows) {  // bf16 rows: split-K when planned
        rc = launch_staged_gemm_split(a, workspace, workspace_bytes);
        if (rc != TIQ_EUNSUPPORTED) return rc;
    }
    return run_linear(a);
}

extern "C" size_t tiq_gemm_w8_workspace(int x_dtype, int64_t M, int64_t K, int64_t N) {
    if ((x_dtype != TIQ_F32 && x_dtype != TIQ_BF16) || K <= 0 || K % 64 != 0 || N <= 0) return 0;
    if (M < kGemmMinRows && !(x_dtype == TIQ_F32 && w4_planes_rows(M, N))) return 0;
    if (x_dtype == TIQ_F32) return split_workspace(M, K) + staged_split_workspace(M, N, 3 * K);
    return staged_split_workspace(M, N, K);
}

extern "C" int tiq_gemm_w8_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                              const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                              void* workspace, size_t workspace_bytes, void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, reinterpret_cast<const uint8_t*>(q), K, scale, nullptr, 0, bias,
                             N, y, y_dtype, ldy, stream, kW8);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    if (workspace && !aligned(workspace, 16)) return TIQ_EALIGN;
    if (x_dtype == TIQ_F32) {
        rc = run_linear_split(a, workspace, workspace_bytes);
        if (rc != TIQ_EUNSUPPORTED) return rc;
    } else {
        rc = launch_staged_gemm_split(a, workspace, workspace_bytes);
        if (rc != TIQ_EUNSUPPORTED) return rc;
    }
    return launch_gemm(a);
}

extern "C" int tiq_linear_gelu_in_ws(const float* x, int64_t M, int64_t K, int64_t ldx, const void* w, int w_format,
                                     const float* scale, const uint16_t* scale_f16, int group, const float* bias,
                                     int64_t N, float* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    if (w_format != TIQ_WF_INT8 && w_format != TIQ_WF_INT4 && w_format != TIQ_WF_INT4_GROUPWISE) return TIQ_EINVAL;
    const WFormat fmt = (WFormat)w_format;
    const int64_t ldw = fmt == kW8 ? K : fmt == kW4 ? K / 2 : (K + 1) / 2;
    LinearArgs a = make_args(x, TIQ_F32, M, K, ldx, static_cast<const uint8_t*>(w), ldw, scale, scale_f16, group,
                             bias, N, y, TIQ_F32, ldy, stream, fmt);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    if (M < kGemmMinRows || K % 64 != 0) return TIQ_EUNSUPPORTED;
    if (workspace && !aligned(workspace, 16)) return TIQ_EALIGN;
    return run_linear_split(a, workspace, workspace_bytes, true);
}

extern "C" int tiq_gemv_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                           const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                           void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, reinterpret_cast<const uint8_t*>(q), K, scale, nullptr, 0, bias,
                             N, y, y_dtype, ldy, stream, kW8);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    return launch_gemv(a);
}

extern "C" int tiq_gemm_w8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                           const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                           void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, reinterpret_cast<const uint8_t*>(q), K, scale, nullptr, 0, bias,
                             N, y, y_dtype, ldy, stream, kW8);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    return launch_gemm(a);
}

extern "C" int tiq_gemm_w8_tile(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* q,
                                const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                                int tile, void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, reinterpret_cast<const uint8_t*>(q), K, scale, nullptr, 0, bias,
                             N, y, y_dtype, ldy, stream, kW8);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    return launch_gemm_tile(a, tile);
}

extern "C" int tiq_linear_w4(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                             const float* scale, const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                             void* stream) {
    return run_linear(make_args(x, x_dtype, M, K, ldx, packed, K / 2, scale, nullptr, 0, bias, N, y, y_dtype, ldy,
                                stream, kW4));
}

static int linear_fused(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w, int w_format,
                        const float* scale, const uint16_t* scale_f16, int group, const float* bias, int64_t N,
                        void* y, int y_dtype, int64_t ldy, const float* ln_weight, const float* ln_bias,
                        float ln_eps, int activation, const float* residual, int64_t ld_residual, void* workspace,
                        size_t workspace_bytes, void* stream) {
    if (w_format < TIQ_WF_INT8 || w_format > TIQ_WF_F32) return TIQ_EINVAL;
    if (activation != TIQ_ACT_NONE && activation != TIQ_ACT_GELU_TANH) return TIQ_EINVAL;
    if ((ln_weight == nullptr) != (ln_bias == nullptr)) return TIQ_EINVAL;
    if (residual && ld_residual < N) return TIQ_EINVAL;
    const WFormat fmt = (WFormat)w_format;
    const int64_t ldw = fmt == kW8 ? K : fmt == kW4 ? K / 2 : fmt == kW4G ? (K + 1) / 2 : K * 4;
    if (fmt == kF32 && scale == nullptr) scale = reinterpret_cast<const float*>(w);  // unused, keeps checks simple
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, static_cast<const uint8_t*>(w), ldw, scale, scale_f16, group,
                             bias, N, y, y_dtype, ldy, stream, fmt);
    a.fuse.ln_w = ln_weight;
    a.fuse.ln_b = ln_bias;
    a.fuse.ln_eps = ln_eps;
    a.fuse.act = activation;
    a.fuse.res = residual;
    a.fuse.ldr = ld_residual;
    a.ws = workspace;
    a.ws_bytes = workspace_bytes;
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    if (rows16_preferred(a)) return launch_rows16(a);
    if (skinny_supported(a)) return launch_skinny(a);
    return launch_gemv(a);
}

extern "C" int tiq_linear_fused(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w,
                                int w_format, const float* scale, const uint16_t* scale_f16, int group,
                                const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                                const float* ln_weight, const float* ln_bias, float ln_eps, int activation,
                                const float* residual, int64_t ld_residual, void* stream) {
    return linear_fused(x, x_dtype, M, K, ldx, w, w_format, scale, scale_f16, group, bias, N, y, y_dtype, ldy,
                        ln_weight, ln_bias, ln_eps, activation, residual, ld_residual, nullptr, 0, stream);
}

extern "C" size_t tiq_linear_fused_workspace(int x_dtype, int w_format, int64_t M, int64_t K, int64_t N) {
    if (x_dtype != TIQ_F32 || (w_format != TIQ_WF_INT8 && w_format != TIQ_WF_F32)) return 0;
    if (M < kSkinnyMinRows || M > 64 || K <= 0 || K % 32 != 0 || N <= 0) return 0;
    return skinny_workspace(M, K);
}

extern "C" int tiq_linear_fused_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w,
                                   int w_format, const float* scale, const uint16_t* scale_f16, int group,
                                   const float* bias, int64_t N, void* y, int y_dtype, int64_t ldy,
                                   const float* ln_weight, const float* ln_bias, float ln_eps, int activation,
                                   const float* residual, int64_t ld_residual, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    if (workspace && !aligned(workspace, 16)) return TIQ_EALIGN;
    return linear_fused(x, x_dtype, M, K, ldx, w, w_format, scale, scale_f16, group, bias, N, y, y_dtype, ldy,
                        ln_weight, ln_bias, ln_eps, activation, residual, ld_residual, workspace, workspace_bytes,
                        stream);
}

extern "C" int tiq_linear_w4_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                                const uint8_t* packed, const float* scale, const float* bias, int64_t N, void* y,
                                int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, packed, K / 2, scale, nullptr, 0, bias, N, y, y_dtype, ldy,
                             stream, kW4);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    if (workspace && !aligned(workspace, 16)) return TIQ_EALIGN;
    rc = run_linear_split(a, workspace, workspace_bytes);
    if (rc != TIQ_EUNSUPPORTED) return rc;
    if (x_dtype == TIQ_BF16 && M >= kGemmMinRows) {  // bf16 rows: split over K when planned
        rc = launch_staged_gemm_split(a, workspace, workspace_bytes);
        if (rc != TIQ_EUNSUPPORTED) return rc;
    }
    return run_linear(a);
}

extern "C" int tiq_linear_w4g_ws(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                                 const uint8_t* packed, const uint16_t* scale_f16, int group, const float* bias,
                                 int64_t N, void* y, int y_dtype, int64_t ldy, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    LinearArgs a = make_args(x, x_dtype, M, K, ldx, packed, (K + 1) / 2, nullptr, scale_f16, group, bias, N, y,
                             y_dtype, ldy, stream, kW4G);
    int rc = check_linear(a);
    if (rc != TIQ_OK || M == 0 || N == 0) return rc;
    if (workspace && !aligned(workspace, 16)) return TIQ_EALIGN;
    rc = run_linear_split(a, workspace, workspace_bytes);
    if (rc != TIQ_EUNSUPPORTED) return rc;
    if (x_dtype == TIQ_BF16 && M >= kGemmMinRows) {  // bf16 rows: split over K when planned
        rc = launch_staged_w4g(a, workspace, workspace_bytes);
        if (rc != TIQ_EUNSUPPORTED) return rc;
        rc = launch_gemm_w4g_split(a, workspace, workspace_bytes);
        if (rc != TIQ_EUNSUPPORTED) return rc;
    }
    return run_linear(a);
}

extern "C" int tiq_linear_w4g(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* packed,
                              const uint16_t* scale_f16, int group, const float* bias, int64_t N, void* y,
                              int y_dtype, int64_t ldy, void* stream) {
    return run_linear(make_args(x, x_dtype, M, K, ldx, packed, (K + 1) / 2, nullptr, scale_f16, group, bias, N, y,
                                y_dtype, ldy, stream, kW4G));
}

extern "C" size_t tiq_decode_linear_workspace(int w_format, int64_t M, int64_t K, int64_t N) {
    if (w_format == TIQ_WF_F32_TILED) return 0;  // planes in only: nothing staged
    if ((w_format != TIQ_WF_INT8 && w_format != TIQ_WF_INT8_TILED && w_format != TIQ_WF_F32) ||
        M < kSkinnyMinRows || M > 64 || K <= 0 ||
        K % 32 != 0 || N <= 0)
        return 0;
    return decode_linear_workspace(M, K, N);
}

extern "C" int tiq_tile_int8(const int8_t* w, int64_t N, int64_t K, int64_t ldw, int8_t* tiles, void* stream) {
    return launch_tile_int8(reinterpret_cast<const uint8_t*>(w), N, K, ldw, reinterpret_cast<uint8_t*>(tiles),
                            as_stream(stream));
}

extern "C" size_t tiq_tile_f32_bytes(int64_t N, int64_t K) { return tile_f32_bytes(N, K); }

extern "C" int tiq_tile_f32(const float* w, int64_t N, int64_t K, int64_t ldw, float* tiles, void* stream) {
    return launch_tile_f32(w, N, K, ldw, tiles, as_stream(stream));
}

extern "C" size_t tiq_decode_planes_bytes(int64_t M, int64_t K) {
    if (M <= 0 || K <= 0 || K % 32 != 0) return 0;
    return decode_planes_bytes(M, K);
}

// ------------------------------------------- allocation-free decode linear
// tiq_decode_linear_noalloc runs tiq_decode_linear with this fixed array as
// its workspace: TIQ_NOALLOC_SCRATCH_BYTES per GPU, held by the loaded code
// object until the process ends. In host code the array's name only names the
// symbol; its device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and only that address is passed to
// the kernels. Every call on one GPU shares the array (calls that overlap on
// one GPU race); nothing in it needs clearing between calls (the planes and
// the partial slices are written whole before they are read).
static __device__ __align__(256) uint8_t scratch[TIQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// The scratch address on the device that runs `stream`.
int noalloc_scratch(hipStream_t stream, void** out) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return status_of(e);
    int dev = cur;
    if (stream) {
        e = hipStreamGetDevice(stream, &dev);
        if (e != hipSuccess) return status_of(e);
    }
    if (dev < 0 || dev >= kMaxDevices) return TIQ_EUNSUPPORTED;
    void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (p) {
        *out = p;
        return TIQ_OK;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return status_of(e);
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t back = dev != cur ? hipSetDevice(cur) : hipSuccess;
        if (e != hipSuccess) return status_of(e);
        if (back != hipSuccess) return status_of(back);
        if (!p) return TIQ_EINVAL;
        g_scratch_addr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return TIQ_OK;
}

}  // namespace

extern "C" int tiq_decode_linear(const float* x, int64_t ldx, const uint16_t* x_planes, int64_t M, int64_t K,
                                 const void* w, int w_format, const float* scale, const float* bias, int64_t N,
                                 float* y, int64_t ldy, const float* ln_weight, const float* ln_bias, float ln_eps,
                                 int activation, const float* residual, int64_t ld_residual,
                                 const float* next_ln_weight, const float* next_ln_bias, float next_ln_eps,
                                 uint16_t* planes_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (w_format != TIQ_WF_INT8 && w_format != TIQ_WF_INT8_TILED && w_format != TIQ_WF_F32 &&
        w_format != TIQ_WF_F32_TILED)
        return TIQ_EUNSUPPORTED;
    if (activation != TIQ_ACT_NONE && activation != TIQ_ACT_GELU_TANH) return TIQ_EINVAL;
    if ((ln_weight == nullptr) != (ln_bias == nullptr)) return TIQ_EINVAL;
    if (M < 0 || K < 0 || N < 0) return TIQ_EINVAL;
    if (M == 0 || N == 0) return TIQ_OK;
    const bool f32w = w_format == TIQ_WF_F32 || w_format == TIQ_WF_F32_TILED;
    if (!w || (!f32w && !scale)) return TIQ_EINVAL;
    if (x_planes && ln_weight) return TIQ_EINVAL;  // planes already carry their LayerNorm
    if (!x_planes && (!x || ldx < K)) return TIQ_EINVAL;
    if (y && ldy < N) return TIQ_EINVAL;
    if (residual && (!y || ld_residual < N)) return TIQ_EINVAL;
    const WFormat fmt = (WFormat)w_format;
    LinearArgs a = make_args(x, TIQ_F32, M, K, ldx, static_cast<const uint8_t*>(w), fmt == kF32 ? 4 * K : K, scale,
                             nullptr, 0, bias, N, y, TIQ_F32, ldy, stream, fmt);
    a.fuse.ln_w = ln_weight;
    a.fuse.ln_b = ln_bias;
    a.fuse.ln_eps = ln_eps;
    a.fuse.act = activation;
    a.fuse.res = residual;
    a.fuse.ldr = ld_residual;
    a.ws = workspace;
    a.ws_bytes = workspace_bytes;
    return run_decode_linear(a, x_planes, next_ln_weight, next_ln_bias, next_ln_eps, planes_out);
}

extern "C" int tiq_decode_linear_noalloc(const float* x, int64_t ldx, const uint16_t* x_planes, int64_t M,
                                         int64_t K, const void* w, int w_format, const float* scale,
                                         const float* bias, int64_t N, float* y, int64_t ldy,
                                         const float* ln_weight, const float* ln_bias, float ln_eps, int activation,
                                         const float* residual, int64_t ld_residual, const float* next_ln_weight,
                                         const float* next_ln_bias, float next_ln_eps, uint16_t* planes_out,
                                         void* stream) {
    // the workspace tiq_decode_linear may use for this shape, against the fixed
    // array (host arithmetic only: nothing is launched for a refused request)
    if (tiq_decode_linear_workspace(w_format, M, K, N) > TIQ_NOALLOC_SCRATCH_BYTES) return TIQ_ESCRATCH;
    void* ws = nullptr;
    if (M > 0 && N > 0) {
        const int rc = noalloc_scratch(as_stream(stream), &ws);
        if (rc != TIQ_OK) return rc;
    }
    return tiq_decode_linear(x, ldx, x_planes, M, K, w, w_format, scale, bias, N, y, ldy, ln_weight, ln_bias, ln_eps,
                             activation, residual, ld_residual, next_ln_weight, next_ln_bias, next_ln_eps, planes_out,
                             ws, TIQ_NOALLOC_SCRATCH_BYTES, stream);
}
