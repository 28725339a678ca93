// Sustained FP8 matrix-core rate of the whole gfx950 device: every CU runs
// waves that issue nothing but v_mfma_scale_f32_32x32x64_f8f6f4 (131 072 flop
// each) on operands held in registers, into independent accumulators, with
// no memory traffic, no LDS and no barriers. The result is the FP8 MFMA
// throughput the device sustains under its own power and clock management,
// against the 5.0 PFLOP/s dense peak of the data sheet (2.4 GHz).
//
// Launches: 256 workgroups (one per CU: the 96 KB of LDS each takes keeps a
// second one off the CU) of 4 or 8 waves (1 or 2 waves per SIMD); each wave
// runs `iters` loop iterations of 16 MFMAs (4 accumulators x 4). The wall
// time of a launch comes from hipEvents; launches of growing length show
// whether the rate falls as the device heats (the clock drops under power).
//
// Build: hy-nomas_amd/build.py (build_probes) -> hy-nomas_amd/probes/mfma_fp8_rate
// Run:   hy-nomas_amd/probes/mfma_fp8_rate   (one GPU, a few seconds)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                    \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

constexpr int LDS_BYTES = 96 * 1024;
constexpr double FLOP_PER_MFMA = 2.0 * 32 * 32 * 64;

__global__ void mfma_stream(float* sink, int iters) {
    __shared__ uint8_t lds[LDS_BYTES];  // occupancy only: one workgroup per CU
    const int lane = threadIdx.x & 63;
    i32x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = 0x38383838 ^ (lane * 7 + i);  // finite e4m3 codes, nothing special
        b[i] = 0x30303030 ^ (lane * 3 + i);
    }
    f32x16 acc[4] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[c], 0, 0, 0, 0, 0, 0);
    }
    float s = 0.0f;
    for (int c = 0; c < 4; ++c)
        for (int v = 0; v < 16; ++v) s += acc[c][v];
    if (s == 1234.5f) sink[blockIdx.x] = s + lds[lane];  // keeps the chain alive; never true
}

int main() {
    int dev = 0;
    CHECK(hipSetDevice(dev));
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, dev));
    const int cus = prop.multiProcessorCount;
    float* sink = nullptr;
    CHECK(hipMalloc(&sink, sizeof(float) * cus));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    printf("device %s, %d CUs\n", prop.name, cus);
    printf("%-8s %10s %10s %12s %10s %14s\n", "w/SIMD", "iters", "ms", "TFLOP/s", "of 5.0 PF",
           "MHz at 100 %");
    for (int waves : {4, 8}) {
        // warm-up launch, then launches of growing length
        hipLaunchKernelGGL(mfma_stream, dim3(cus), dim3(64 * waves), 0, 0, sink, 2000);
        CHECK(hipDeviceSynchronize());
        for (int iters : {2000, 20000, 200000}) {
            CHECK(hipEventRecord(e0));
            hipLaunchKernelGGL(mfma_stream, dim3(cus), dim3(64 * waves), 0, 0, sink, iters);
            CHECK(hipEventRecord(e1));
            CHECK(hipEventSynchronize(e1));
            float ms = 0.0f;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            const double mfmas = (double)cus * waves * iters * 16;
            const double tflops = mfmas * FLOP_PER_MFMA / (ms * 1e-3) / 1e12;
            // clock at which one MFMA per SIMD every 64 cycles gives this rate
            const double mhz = mfmas * 64.0 / (cus * 4.0) / (ms * 1e-3) / 1e6;
            printf("%-8d %10d %10.3f %12.1f %9.1f%% %14.0f\n", waves / 4, iters, ms, tflops,
                   100.0 * tflops / 5000.0, mhz);
        }
    }
    CHECK(hipFree(sink));
    return 0;
}
