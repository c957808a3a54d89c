// mfma_rate.hip -- issue rate of the gfx950 matrix instructions the prefill GEMM could use
// (a measurement program for the design notes; not part of the library).
//
// Every wave runs four independent accumulator chains of one MFMA kind, 8 waves per SIMD,
// and the time per instruction per SIMD is printed in ns and in cycles of a 2.4 GHz clock.
// Build: hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops
//        mnemocuda_amd/probes/mfma_rate.hip -o mfma_rate
#include <hip/hip_runtime.h>

#include <cstdio>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int kIters = 4096;
constexpr int kThreads = 256;
constexpr int kBlocks = 256 * 8;  // 8 workgroups of 4 waves per CU: 8 waves per SIMD

__global__ void __launch_bounds__(kThreads) f16_16x16x32(float *o, h8 a, h8 b) {
    f4 c[4] = {};
    for (int i = 0; i < kIters; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
    o[blockIdx.x * kThreads + threadIdx.x] = c[0][0] + c[1][1] + c[2][2] + c[3][3];
}
__global__ void __launch_bounds__(kThreads) i8_16x16x64(float *o, i4 a, i4 b) {
    i4 c[4] = {};
    for (int i = 0; i < kIters; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[j], 0, 0, 0);
    o[blockIdx.x * kThreads + threadIdx.x] = (float)(c[0][0] + c[1][1] + c[2][2] + c[3][3]);
}
__global__ void __launch_bounds__(kThreads) i8_16x16x32(float *o, long a, long b) {
    i4 c[4] = {};
    for (int i = 0; i < kIters; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c[j], 0, 0, 0);
    o[blockIdx.x * kThreads + threadIdx.x] = (float)(c[0][0] + c[1][1] + c[2][2] + c[3][3]);
}

int main() {
    float *o = nullptr;
    if (hipMalloc(&o, (size_t)kBlocks * kThreads * sizeof(float)) != hipSuccess) return 1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    int cus = 256;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
    h8 a;
    for (int i = 0; i < 8; i++) a[i] = (_Float16)0.001f;
    const i4 ia = {1, 2, 3, 4};
    auto run = [&](const char *name, int k_depth, auto launch) {
        launch();
        (void)hipDeviceSynchronize();
        (void)hipEventRecord(e0);
        launch();
        (void)hipEventRecord(e1);
        (void)hipEventSynchronize(e1);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        const double instr_per_simd = (double)kBlocks * (kThreads / 64) * 4.0 * kIters / (4.0 * cus);
        const double ns = ms * 1e6 / instr_per_simd;
        printf("%-26s K=%2d per 16x16 tile: %.2f ns = %.1f cycles at 2.4 GHz per instruction per SIMD\n", name,
               k_depth, ns, ns * 2.4);
    };
    run("v_mfma_f32_16x16x32_f16", 32, [&] { f16_16x16x32<<<kBlocks, kThreads>>>(o, a, a); });
    run("v_mfma_i32_16x16x64_i8", 64, [&] { i8_16x16x64<<<kBlocks, kThreads>>>(o, ia, ia); });
    run("v_mfma_i32_16x16x32_i8", 32, [&] { i8_16x16x32<<<kBlocks, kThreads>>>(o, 1, 2); });
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
