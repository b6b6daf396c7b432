// Group-wise int4 prefill GEMM on the register-staged kernel (gfx950): the
// library's own group-wise format (nibbles as the reference's int4 rows,
// quantization.py:132-149, one fp16 scale per row and group of 128 columns)
// behind the reference's quantized Linears over a whole prompt
// (model.py:254,319,352,355 with M = B*T):
//     y[m, n] = sum_g s[n, g] * sum_{k in g} x[m, k] * q[n, k] + bias[n]
// Built without -amdgpu-mfma-vgpr-form: the MFMAs accumulate a group's
// partial tiles in AGPRs, and the scaled sums, which only vector instructions
// touch, stay in VGPRs.
#include <algorithm>

#include "tiq_internal.hpp"

namespace tiq {
namespace {

#include "gemm_staged_kernel.hpp"

constexpr int kGroup = 128;  // two k64 steps
constexpr int kBN = 128;

// Tile height: 224 rows, or 128 where 128-row tiles cover M with fewer rows
// than 224-row ones and all fit on the CUs at once (GPT-2-XL shapes: M = 256,
// 256 rows of work instead of 448, 13-22% faster; M = 1024 with N = 1600,
// 4-9% faster).
int w4g_rows(int64_t M, int64_t N) {
    const bool fewer_rows = (M + 127) / 128 * 128 < (M + 223) / 224 * 224;
    return fewer_rows && ((M + 127) / 128) * ((N + kBN - 1) / kBN) <= 256 ? 128 : 224;
}

// One workgroup per tile (the group-wise kernel does not run persistent);
// gridDim.z = S splits of whole groups, fp32 slices without bias when S > 1.
template <int BM, typename TY>
int run_w4g(const LinearArgs& a, TY* y, int64_t ldy, const float* bias, int64_t S) {
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + kBN - 1) / kBN);
    const int ngroups = (int)((a.K + kGroup - 1) / kGroup);
    hipLaunchKernelGGL((gemm_staged<BM, kBN, 1, kW4G, TY>), dim3((unsigned)tiles, 1, (unsigned)S), dim3(256), 0,
                       a.stream, static_cast<const uint16_t*>(a.x), a.ldx, a.w, a.ldw, nullptr, bias, y, ldy,
                       (int)a.M, (int)a.N, (int)a.K, (int)a.K, a.scale16, ngroups, nullptr);
    return launch_status();
}

}  // namespace

bool staged_w4g_supported(const LinearArgs& a) {
    if (a.fmt != kW4G || a.x_dtype != TIQ_BF16 || a.group != kGroup || (a.kw && a.kw != a.K)) return false;
    if (a.K % BK != 0 || a.ldw != a.K / 2) return false;
    const int unit = a.y_dtype == TIQ_F32 ? 4 : 8;
    if (a.N % unit != 0 || a.ldy % unit != 0 || !aligned(a.y, 16)) return false;
    if (a.N % 32 != 0) return false;  // a 32-column tile is all inside N or all outside
    if ((a.bias && !aligned(a.bias, 16)) || !aligned(a.scale16, 2)) return false;
    if (!aligned(a.x, 16) || a.ldx % 8 != 0 || !aligned(a.w, 16) || a.ldw % 16 != 0) return false;
    // 32-bit byte offsets from the base pointers, 32-bit scale offsets
    if ((a.M - 1) * a.ldx * 2 + a.K * 2 > 0xffffffffLL || (a.N - 1) * a.ldw + a.K / 2 > 0xffffffffLL) return false;
    if (a.N * ((a.K + kGroup - 1) / kGroup) * 2 > 0xffffffffLL) return false;
    return true;
}

// Splits of whole groups when the tiles fill less than a round of 256 CUs (at
// most 8, at most one a group, within the workspace); 1: none, also for 96
// tiles or more with at most 32 k64 steps, where the slices' trip through
// memory costs more than the idle CUs (M = 256 and 1024 at K = 1600: 5-9%).
int64_t staged_w4g_splits(int64_t M, int64_t N, int64_t K, size_t ws_bytes) {
    const int bm = w4g_rows(M, N);
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + kBN - 1) / kBN);
    if (tiles >= 96 && K / BK <= 32) return 1;
    const int64_t groups = (K + kGroup - 1) / kGroup;
    int64_t S = std::min<int64_t>(std::min<int64_t>(256 / std::max<int64_t>(tiles, 1), groups), 8);
    S = std::min<int64_t>(S, (int64_t)(ws_bytes / (size_t)(M * N * 4)));
    return std::max<int64_t>(S, 1);
}

int launch_staged_w4g(const LinearArgs& a, void* ws, size_t ws_bytes) {
    if (!staged_w4g_supported(a)) return TIQ_EUNSUPPORTED;
    const int64_t S = (ws && aligned(ws, 16)) ? staged_w4g_splits(a.M, a.N, a.K, ws_bytes) : 1;
    const bool short_m = w4g_rows(a.M, a.N) == 128;
    if (S > 1 && a.M * a.N * S <= 0x7fffffffLL) {
        float* part = static_cast<float*>(ws);
        int rc = short_m ? run_w4g<128, float>(a, part, a.N, nullptr, S) : run_w4g<224, float>(a, part, a.N, nullptr, S);
        if (rc != TIQ_OK) return rc;
        return launch_splitk_reduce(a, part, S, nullptr);
    }
    if (a.y_dtype == TIQ_F32)
        return short_m ? run_w4g<128, float>(a, static_cast<float*>(a.y), a.ldy, a.bias, 1)
                       : run_w4g<224, float>(a, static_cast<float*>(a.y), a.ldy, a.bias, 1);
    return short_m ? run_w4g<128, uint16_t>(a, static_cast<uint16_t*>(a.y), a.ldy, a.bias, 1)
                   : run_w4g<224, uint16_t>(a, static_cast<uint16_t*>(a.y), a.ldy, a.bias, 1);
}

}  // namespace tiq
