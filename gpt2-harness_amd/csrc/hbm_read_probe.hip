// hbm_read_probe: measures what one kernel launch can read from HBM on this
// GPU, as a function of bytes per launch, 16-byte loads in flight per lane
// and grid size, plus the per-launch cost of back-to-back launches (on a
// stream and inside a HIP graph, with an empty kernel for the floor). Buffers
// rotate over a 2 GiB region so every launch reads cold (past the 256 MB
// Infinity Cache). It calibrates the attainable bandwidth the GEMV and
// quantize kernels are judged against; it is not part of libtiq_hip.so.
//   make -C gpt2-harness_amd/csrc probe && gpt2-harness_amd/csrc/bin/hbm_read_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e), __LINE__); exit(1); } } while (0)

// Each thread reads U 16-byte chunks: chunk index = tid + j * nthreads (j < U),
// only if < nchunks. One float per thread written (sum) to keep the loads.
template <int U>
__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ p, long nchunks, float* __restrict__ out) {
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long nthr = (long)gridDim.x * blockDim.x;
    uint4 v[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const long c = tid + j * nthr;
        v[j] = (c < nchunks) ? p[c] : make_uint4(0, 0, 0, 0);
    }
    uint32_t s = 0;
#pragma unroll
    for (int j = 0; j < U; ++j) s ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    // loop for the remainder when the grid is small
    for (long c = tid + U * nthr; c < nchunks; c += nthr) { uint4 t = p[c]; s ^= t.x ^ t.y ^ t.z ^ t.w; }
    if (s == 0x12345678u) out[tid % 1024] = (float)s;  // practically never taken
}

__global__ void empty_kernel(float*) {}

int main() {
    const size_t region = 2ull << 30;  // 2 GiB
    uint4* buf;
    float* out;
    CK(hipMalloc(&buf, region));
    CK(hipMalloc(&out, 1024 * sizeof(float)));
    CK(hipMemset(buf, 1, region));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    const size_t sizes[] = {600000, 1800000, 2400000, 7700000, 10200000, 40000000, 200000000};
    const int waves_per_cu[] = {4, 8, 16, 32};
    for (size_t bytes : sizes) {
        const long nchunks = (long)(bytes / 16);
        for (int U : {1, 2, 4, 8}) {
            for (int wpc : waves_per_cu) {
                long threads = 256L * wpc * 64;      // 256 CUs
                long need = (nchunks + U - 1) / U;   // threads needed for one pass
                if (threads > need) threads = ((need + 255) / 256) * 256;
                const unsigned blocks = (unsigned)(threads / 256);
                const int reps = 40;
                // offsets rotate through the region, each launch cold
                const size_t stride = ((bytes + (1 << 20)) >> 20) << 20;
                const int slots = (int)(region / stride) - 1;
                auto launch = [&](int r) {
                    const uint4* p = buf + (size_t)(r % slots) * (stride / 16);
                    switch (U) {
                        case 1: hipLaunchKernelGGL(read_kernel<1>, dim3(blocks), dim3(256), 0, 0, p, nchunks, out); break;
                        case 2: hipLaunchKernelGGL(read_kernel<2>, dim3(blocks), dim3(256), 0, 0, p, nchunks, out); break;
                        case 4: hipLaunchKernelGGL(read_kernel<4>, dim3(blocks), dim3(256), 0, 0, p, nchunks, out); break;
                        default: hipLaunchKernelGGL(read_kernel<8>, dim3(blocks), dim3(256), 0, 0, p, nchunks, out); break;
                    }
                };
                for (int r = 0; r < 4; ++r) launch(r);
                CK(hipDeviceSynchronize());
                float best = 1e30f, sum = 0.f;
                for (int r = 0; r < reps; ++r) {
                    CK(hipEventRecord(a, 0));
                    launch(r + 7);
                    CK(hipEventRecord(b, 0));
                    CK(hipEventSynchronize(b));
                    float ms;
                    CK(hipEventElapsedTime(&ms, a, b));
                    best = ms < best ? ms : best;
                    sum += ms;
                }
                printf("bytes=%10zu U=%d waves/CU=%2d blocks=%6u  best=%8.2f us (%7.1f GB/s)  mean=%8.2f us (%7.1f GB/s)\n",
                       bytes, U, wpc, blocks, best * 1e3, bytes / (best * 1e-3) / 1e9, sum / reps * 1e3,
                       bytes / (sum / reps * 1e-3) / 1e9);
                fflush(stdout);
            }
        }
    }
    // back-to-back launches in a graph-free stream, no events between: time 200 launches of 1.8 MB
    for (size_t bytes : {1800000ul, 10200000ul}) {
        const long nchunks = (long)(bytes / 16);
        const unsigned blocks = (unsigned)((nchunks + 255) / 256);
        const size_t stride = ((bytes + (1 << 20)) >> 20) << 20;
        const int slots = (int)(region / stride) - 1;
        CK(hipDeviceSynchronize());
        CK(hipEventRecord(a, 0));
        for (int r = 0; r < 200; ++r)
            hipLaunchKernelGGL(read_kernel<1>, dim3(blocks), dim3(256), 0, 0, buf + (size_t)(r % slots) * (stride / 16), nchunks, out);
        CK(hipEventRecord(b, 0));
        CK(hipEventSynchronize(b));
        float ms;
        CK(hipEventElapsedTime(&ms, a, b));
        printf("back-to-back bytes=%zu: %.2f us per launch (%.1f GB/s)\n", bytes, ms * 1e3 / 200, bytes * 200 / (ms * 1e-3) / 1e9);
    }
    // The same inside a HIP graph, as the decode step runs: 240 launches
    // captured back to back, the graph replayed; an empty kernel (the launch
    // floor) and one 16-byte load per thread of 1.8 / 10.2 MB (cold).
    hipStream_t st;
    CK(hipStreamCreate(&st));
    for (size_t bytes : {0ul, 1800000ul, 10200000ul}) {
        const long nchunks = (long)(bytes / 16);
        const unsigned blocks = bytes ? (unsigned)((nchunks + 255) / 256) : 1u;
        const size_t stride = ((bytes + (1 << 20)) >> 20) << 20;
        const int slots = (int)(region / stride) - 1;
        const int L = 240;
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
        for (int r = 0; r < L; ++r) {
            if (bytes == 0) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, st, out);
            else hipLaunchKernelGGL(read_kernel<1>, dim3(blocks), dim3(256), 0, st, buf + (size_t)(r % slots) * (stride / 16), nchunks, out);
        }
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, st));
        CK(hipStreamSynchronize(st));
        float best = 1e30f;
        for (int rep = 0; rep < 5; ++rep) {
            CK(hipEventRecord(a, st));
            CK(hipGraphLaunch(ge, st));
            CK(hipEventRecord(b, st));
            CK(hipEventSynchronize(b));
            float ms;
            CK(hipEventElapsedTime(&ms, a, b));
            best = ms < best ? ms : best;
        }
        printf("graph back-to-back bytes=%zu: %.3f us per launch (%.1f GB/s)\n", bytes, best * 1e3 / L,
               bytes / (best * 1e-3 / L) / 1e9);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    CK(hipStreamDestroy(st));
    CK(hipFree(buf));
    CK(hipFree(out));
    printf("done\n");
    return 0;
}
