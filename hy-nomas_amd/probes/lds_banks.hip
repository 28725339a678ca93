// LDS bank-conflict probe for gfx950: one dispatch per (access kind, lane
// address pattern), read with rocprofv3 counters (SQ_LDS_BANK_CONFLICT,
// SQ_LDS_IDX_ACTIVE, SQ_INSTS_LDS_STORE, SQ_INSTS_LDS_LOAD), which give the
// conflict cycles and LDS-busy cycles per instruction of each pattern.
//
// Every dispatch is 256 workgroups of 4 waves; each wave loops 1000 times
// over one LDS instruction at its lane's address (wave w offset by 16 KB) and
// waits for it. Kinds: 16-byte store, 16-byte load, 8-byte store. Patterns
// (lane l of the wave, byte address):
//    0  16 l                                  linear
//    1  272 (l / 8) + 32 (l % 8)              8 lanes per 272-byte row, 32 B apart
//    2  32 l                                  32 B apart
//    3  256 (l / 8) + 32 (l % 8)              the same with 256-byte rows
//    4  272 (l / 8) + 32 (l % 8) + 16 ((l / 8) % 2)
//    5  16 (l % 32) + 512 (l / 32)            two 512-byte halves
//    6  272 (l / 4) + 16 (l % 4)              4 lanes per row, 64 contiguous bytes
//    7  272 (l / 16) + 16 (l % 16)            16 lanes per row, 256 contiguous bytes
//    8  8 l                                   (8-byte store only)
//    9  272 (l % 32) + 16 (l / 32)            one row per lane, lanes 32-63 at +16 B
//   10  272 (l / 8) + 32 ((l % 8) ^ (l / 8))  row-swizzled 32-byte units
//   11  288 (l / 8) + 32 (l % 8)              288-byte rows
//   12  272 k + 32 u, k = 2 (l / 16) + (l / 4) % 2, u = l % 4 + 4 ((l / 8) % 2)
//                                             two keys per 8 lanes (the chunk
//                                             attention's K-tile write)
//
// Build: hy-nomas_amd/build.py (build_probes) -> hy-nomas_amd/probes/lds_banks
// Run:   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS_STORE
//            SQ_INSTS_LDS_LOAD --output-format csv -d <dir> -o p -- hy-nomas_amd/probes/lds_banks
//        (dispatches in the order the program prints them)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                    \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

constexpr int PATTERNS = 13;

// Byte address of lane l under pattern pat (at most 8 464 + 16 bytes; every
// 16-byte access is 16-byte aligned).
__device__ uint32_t addr_of(int pat, uint32_t l) {
    switch (pat) {
    case 0: return l * 16;
    case 1: return (l >> 3) * 272 + (l & 7) * 32;
    case 2: return l * 32;
    case 3: return (l >> 3) * 256 + (l & 7) * 32;
    case 4: return (l >> 3) * 272 + (l & 7) * 32 + ((l >> 3) & 1) * 16;
    case 5: return (l & 31) * 16 + (l >> 5) * 512;
    case 6: return (l >> 2) * 272 + (l & 3) * 16;
    case 7: return (l >> 4) * 272 + (l & 15) * 16;
    case 8: return l * 8;
    case 9: return (l & 31) * 272 + (l >> 5) * 16;
    case 10: return (l >> 3) * 272 + ((l & 7) ^ ((l >> 3) & 7)) * 32;
    case 11: return (l >> 3) * 288 + (l & 7) * 32;
    case 12: return (2 * (l >> 4) + ((l >> 2) & 1)) * 272 + ((l & 3) + 4 * ((l >> 3) & 1)) * 32;
    default: return 0;
    }
}

enum Kind { STORE16 = 0, STORE8 = 1, LOAD16 = 2 };

template <int KIND>
__global__ void lds_kernel(int pat, int iters, float* out) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[65536];
    const uint32_t l = threadIdx.x & 63u;
    const uint32_t a = (uint32_t)(uintptr_t)lds + addr_of(pat, l) + (threadIdx.x >> 6) * 16384u;
    u32x4 d = {threadIdx.x, 1u, 2u, 3u};
    for (int i = 0; i < iters; ++i) {
        if (KIND == STORE16) asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(d) : "memory");
        if (KIND == STORE8) asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(u32x2{d.x, d.y}) : "memory");
        if (KIND == LOAD16) asm volatile("ds_read_b128 %0, %1" : "=v"(d) : "v"(a) : "memory");
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = (float)(d.x + d.y + d.z + d.w);
}

int main() {
    float* out = nullptr;
    CHECK(hipMalloc(&out, 256 * 256 * sizeof(float)));
    const char* kinds[3] = {"16-byte store", "8-byte store", "16-byte load"};
    int n = 0;
    for (int pat = 0; pat < PATTERNS; ++pat) {
        for (int kind : {STORE16, LOAD16, STORE8}) {
            if (kind == STORE8 && pat != 0 && pat != 5 && pat != 8) continue;
            if (kind != STORE8 && pat == 8) continue;
            if (kind == STORE16) hipLaunchKernelGGL(lds_kernel<STORE16>, dim3(256), dim3(256), 0, 0, pat, 1000, out);
            if (kind == STORE8) hipLaunchKernelGGL(lds_kernel<STORE8>, dim3(256), dim3(256), 0, 0, pat, 1000, out);
            if (kind == LOAD16) hipLaunchKernelGGL(lds_kernel<LOAD16>, dim3(256), dim3(256), 0, 0, pat, 1000, out);
            CHECK(hipGetLastError());
            CHECK(hipDeviceSynchronize());
            printf("dispatch %2d: pattern %2d, %s\n", n++, pat, kinds[kind]);
        }
    }
    CHECK(hipFree(out));
    return 0;
}
