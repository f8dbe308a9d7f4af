// trench-gguf_amd/bench/ldlq_update.hip - the LDLQ update kernel alone (k_ldlq_update, the f64 MFMA GEMM).
//
// nmat matrices of 2048 x 7168 (W f32), the block's Es (256 x nmat*2048 f64, k-major) and per-matrix U factors
// (7168 x 7168 f64; `shared` = 1: one U for all) filled with synthetic values; timed with HIP events over 5 launches
// after 2 warm-ups, for three column ranges of block 0: the far update [512, 7168), the next block [256, 512) and
// the right half [3584, 7168). flops = 2 * 256 * rows * columns.
//   usage: ldlq_update [nmat=64] [shared=0]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "../csrc/ldlq.cuh"

__global__ void fill_f64(double *p, size_t n, double s) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = s * (double)((i * 2654435761u) % 1000) / 1000.0 - s / 2;
}
__global__ void fill_f32(float *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = (float)((i * 40503u) % 1000) / 50000.0f;
}

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));            \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

int main(int argc, char **argv) {
    const int64_t nmat = argc > 1 ? atoi(argv[1]) : 64, ne1 = 2048, ne0 = 7168;
    const int shared = argc > 2 ? atoi(argv[2]) : 0;
    if (nmat < 1 || nmat > 64) {
        fprintf(stderr, "nmat must be 1..64\n");
        return 2;
    }
    const size_t nw = (size_t)nmat * ne1 * ne0, nes = (size_t)QK * nmat * ne1;
    const size_t nu = (size_t)(shared ? 1 : nmat) * ne0 * ne0;
    float *W;
    double *Es, *U;
    CHECK(hipMalloc(&W, nw * 4));
    CHECK(hipMalloc(&Es, nes * 8));
    CHECK(hipMalloc(&U, nu * 8));
    hipLaunchKernelGGL(fill_f32, dim3(4096), dim3(256), 0, 0, W, nw);
    hipLaunchKernelGGL(fill_f64, dim3(4096), dim3(256), 0, 0, Es, nes, 0.01);
    hipLaunchKernelGGL(fill_f64, dim3(4096), dim3(256), 0, 0, U, nu, 1.0);
    CHECK(hipDeviceSynchronize());
    const int64_t u_stride = shared ? 0 : ne0 * ne0;
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    const struct {
        int64_t cb, ce;
        const char *name;
    } cases[] = {{512, ne0, "far [512, 7168)"}, {256, 512, "next [256, 512)"}, {3584, ne0, "half [3584, 7168)"}};
    for (const auto &c : cases) {
        const int64_t nt = ((c.ce - c.cb + LDLQ_TN - 1) / LDLQ_TN) * ((ne1 + LDLQ_TM - 1) / LDLQ_TM) * nmat;
        const dim3 grid((unsigned)((nt + 7) / 8 * 8));
        for (int it = 0; it < 2; ++it)
            hipLaunchKernelGGL(k_ldlq_update, grid, dim3(256), 0, 0, W, Es, U, u_stride, nmat, ne1, ne0, (int64_t)0,
                               c.cb, c.ce);
        CHECK(hipDeviceSynchronize());
        const int reps = 5;
        CHECK(hipEventRecord(e0, 0));
        for (int it = 0; it < reps; ++it)
            hipLaunchKernelGGL(k_ldlq_update, grid, dim3(256), 0, 0, W, Es, U, u_stride, nmat, ne1, ne0, (int64_t)0,
                               c.cb, c.ce);
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        ms /= reps;
        const double flops = 2.0 * QK * ne1 * nmat * (double)(c.ce - c.cb);
        printf("%-18s nmat %ld shared U %d: %.3f ms  %.1f TFLOP/s  %.3f of 78.6\n", c.name, (long)nmat, shared, ms,
               flops / ms / 1e9, flops / ms / 1e9 / 78.6);
    }
    CHECK(hipFree(W));
    CHECK(hipFree(Es));
    CHECK(hipFree(U));
    return 0;
}
