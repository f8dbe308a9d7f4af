// trench-gguf_amd/bench/valu_peak.hip - the VALU throughput the roofline is priced against.
//
// Every wave64 of 2048 workgroups x 4 waves runs 8 independent chains of one non-packed 32-bit VALU instruction
// (fp32 add, mul, fma; the integer step (b ^ it) + u, which compiles to one v_xad_u32) for 4096 x 8 iterations; the
// rate is 64 lane-instructions per wave instruction over the event-timed kernel. The search kernels' algorithmic op
// counts are priced against the fp32 rate.
#include <hip/hip_runtime.h>
#include <cstdio>

#define N_IT 4096

template <int OP> __global__ __launch_bounds__(256) void k_chain(float *out, float s) {
    float a[8];
    int b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { a[i] = threadIdx.x * 0.001f + i; b[i] = threadIdx.x + i; }
    for (int it = 0; it < N_IT; ++it) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (OP == 0) a[i] = a[i] + s;
                else if (OP == 1) a[i] = a[i] * s;
                else if (OP == 2) b[i] = (b[i] ^ it) + u;
                else a[i] = fmaf(a[i], s, 0.5f);
            }
        }
    }
    float r = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) r += a[i] + (float)b[i];
    if (r == 123.456f) out[threadIdx.x] = r;      // (never true: keeps the chains live)
}

int main() {
    float *out = nullptr;
    if (hipMalloc(&out, 4096) != hipSuccess) { fprintf(stderr, "no device memory\n"); return 1; }
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    const int wgs = 256 * 8;
    const double lane_instr = (double)wgs * 256 * N_IT * 64;
    const char *name[4] = {"v_add_f32", "v_mul_f32", "v_xad_u32", "v_fma_f32"};
    for (int rep = 0; rep < 2; ++rep) {
        for (int op = 0; op < 4; ++op) {
            if (hipEventRecord(e0) != hipSuccess) return 1;
            if (op == 0) hipLaunchKernelGGL(k_chain<0>, dim3(wgs), dim3(256), 0, 0, out, 1.0001f);
            if (op == 1) hipLaunchKernelGGL(k_chain<1>, dim3(wgs), dim3(256), 0, 0, out, 1.0001f);
            if (op == 2) hipLaunchKernelGGL(k_chain<2>, dim3(wgs), dim3(256), 0, 0, out, 1.0001f);
            if (op == 3) hipLaunchKernelGGL(k_chain<3>, dim3(wgs), dim3(256), 0, 0, out, 1.0001f);
            if (hipEventRecord(e1) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1;
            float ms = 0;
            if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1;
            const double per = 1.0;   // one instruction a step (the int step (b ^ it) + u compiles to one v_xad_u32)
            if (rep) printf("%-16s %8.3f ms  %7.2f T lane-instructions/s\n", name[op], ms,
                            per * lane_instr / (ms * 1e-3) / 1e12);
        }
    }
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) return 1;
    printf("CUs %d, peak engine clock %d kHz\n", p.multiProcessorCount, p.clockRate);
    (void)hipFree(out);
    return 0;
}
