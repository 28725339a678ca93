// Issue-rate microbenchmark for gfx950: what one SIMD sustains when a wave's
// instruction stream mixes v_mfma_f32_32x32x16_bf16 with VALU work, and what
// the chunk attention's per-tile slot mix allows at most.
//
// Every kernel runs 256 workgroups (one per CU; the 96 KB of LDS each takes
// keeps a second one off the CU) of 256, 512 or 768 threads, i.e. 1, 2 or 3
// waves per SIMD, for a fixed number of "slots". A slot is one MFMA (or none)
// followed by the VALU instructions of its pattern, fenced with
// sched_barrier so the compiler keeps that order. Reported per SIMD: wall
// nanoseconds per slot (hipEvent timing of the whole launch) and the MFMA
// share of that time against the MFMA-only launch at the same occupancy.
//
// Patterns:
//   mfma            1 MFMA per slot (dependent accumulator chain)
//   valu N          N v_fma_f32 per slot, no MFMA
//   mfma+N          1 MFMA + N v_fma_f32 in the same wave
//   split N         even waves MFMA only, odd waves N v_fma_f32 only
//   tile            the attention's tile in the kernel's order: 8 step-A
//                   slots (MFMA + 2 fma, 2 exp, 1 cvt_pk_f16, 1 dot2), 8
//                   K-write slots (MFMA + fp8 cvt, 2 mul, cvt_pk_bf16, max3),
//                   8 step-A slots, 8 V-write slots (the K-write work + 2
//                   unpack + cvt_pkrtz); each MFMA's A operand read from LDS
//                   two slots ahead, as the kernel does.
//   tile+barrier    the same with a workgroup barrier after every tile, as
//                   the kernel has (its waves then run each phase together).
//   tile+barrier, V^T reads
//                   the same, the write slots' operands read at the V^T
//                   tile's addresses (144-byte rows, 32 rows a block) as the
//                   kernel's PV MFMAs do, the step-A slots' at the K tile's
//                   (272-byte rows).
//   tile+barrier + clump
//                   the same with 16 extra instructions per tile (VALU
//                   v_add_u32 or SALU s_mov_b32), either together at the end
//                   of the tile (as loop control, address arithmetic and
//                   checks gather at the kernel's tile boundary) or spread
//                   one per slot over the first 16 slots.
//   chain           1 MFMA per slot, all into one accumulator (the other
//                   patterns alternate two)
//   tile, kernel dependencies (+ barrier)
//                   the tile with the kernel's register dependencies: the
//                   step-A slots chain their 8 bf16 MFMAs into one S block
//                   and take their exponentials' inputs from the S block of
//                   16 slots before; the write slots issue fp16 MFMAs into
//                   four rotating O blocks and their max3 reads the S block
//                   the step-A chain before them has just produced.
//   op K           8 independent VALU instructions of one kind per slot, no
//                  MFMA (K: v_fma_f32, v_mul_f32, v_exp_f32, v_cvt_pk_bf16_f32,
//                  v_cvt_scalef32_pk_f32_fp8, v_cvt_pk_f16_f32, v_pk_fma_f16,
//                  v_max3_f32): each kind's own issue cost, in ns per
//                  instruction per SIMD.
//   tile+barrier, rotated
//                   the same, with the waves of the workgroup's upper half
//                   (the second wave of each SIMD) starting 8 slots later in
//                   the tile's order, so one wave of a SIMD is in a step-A
//                   phase while the other is in a write phase.
//
// Build: hy-nomas_amd/build.py (build_probes) -> hy-nomas_amd/probes/issue_rates
// Run:   hy-nomas_amd/probes/issue_rates   (one GPU, about a second)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                    \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

constexpr int SLOTS = 32;  // slots per loop iteration (one attention tile per wave)
constexpr int LDS_BYTES = 96 * 1024;

enum Pattern { MFMA = 0, VALU = 1, MFMA_VALU = 2, SPLIT = 3, TILE = 4, TILE_BAR = 5, TILE_BAR_ROT = 6, TILE_BAR_VT = 7, CLUMP_VALU_END = 8, CLUMP_VALU_SPREAD = 9, CLUMP_SALU_END = 10,
               CLUMP_SALU_SPREAD = 11, CHAIN = 12, TILE_DEP = 13, VALU_OP = 14 };

// One instruction of VALU kind K on chain x (the VALU_OP pattern).
constexpr const char* OP_NAMES[8] = {"v_fma_f32", "v_mul_f32", "v_exp_f32", "v_cvt_pk_bf16_f32",
                                     "v_cvt_scalef32_pk_f32_fp8", "v_cvt_pk_f16_f32", "v_pk_fma_f16", "v_max3_f32"};
template <int K>
__device__ __forceinline__ void kind_op(float& x, float c) {
    if (K == 0) asm volatile("v_fma_f32 %0, %0, %1, 0.5" : "+v"(x) : "v"(c));
    if (K == 1) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x) : "v"(c));
    if (K == 2) asm volatile("v_exp_f32 %0, %0" : "+v"(x));
    if (K == 3) asm volatile("v_cvt_pk_bf16_f32 %0, %0, %1" : "+v"(x) : "v"(c));
    if (K == 4) {
        double d;
        asm volatile("v_cvt_scalef32_pk_f32_fp8 %0, %1, 1.0" : "=v"(d) : "v"(x));
        x = __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(uint64_t, d));
    }
    if (K == 5) asm volatile("v_cvt_pk_f16_f32 %0, %0, %1" : "+v"(x) : "v"(c));
    if (K == 6) asm volatile("v_pk_fma_f16 %0, %0, %1, %0" : "+v"(x) : "v"(c));
    if (K == 7) asm volatile("v_max3_f32 %0, %0, %1, 0.5" : "+v"(x) : "v"(c));
}

// 8 chains of VALU kind K per slot, no MFMA.
template <int K>
__device__ __forceinline__ float op_loop(int iters) {
    float x[8];
    for (int i = 0; i < 8; ++i) x[i] = 0.01f * (threadIdx.x + i);
    const float c = 0.999f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
#pragma unroll
            for (int j = 0; j < 8; ++j) kind_op<K>(x[j], c);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float sum = 0.0f;
    for (int i = 0; i < 8; ++i) sum += x[i];
    return sum;
}

__device__ __forceinline__ void fma_op(float& x, float c) { asm volatile("v_fma_f32 %0, %0, %1, 0.5" : "+v"(x) : "v"(c)); }

// The VALU work of one attention slot of kind k (0: step A, 1: K write, 2: V write).
__device__ __forceinline__ void tile_valu(int k, float (&x)[12], float c, uint32_t w) {
    if (k == 0) {
        asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[0]) : "v"(c), "v"(x[8]));
        asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[1]) : "v"(c), "v"(x[8]));
        asm volatile("v_exp_f32 %0, %0" : "+v"(x[0]));
        asm volatile("v_exp_f32 %0, %0" : "+v"(x[1]));
        asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(x[2]) : "v"(x[0]), "v"(x[1]));
        asm volatile("v_dot2c_f32_f16 %0, %1, %2" : "+v"(x[3]) : "v"(x[2]), "v"(x[9]));
    } else {
        asm volatile("v_cvt_scalef32_pk_f32_fp8 %0, %1, 1.0" : "=v"(*reinterpret_cast<double*>(&x[4])) : "v"(w));
        asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[4]) : "v"(c));
        asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[5]) : "v"(c));
        asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(x[6]) : "v"(x[4]), "v"(x[5]));
        if (k == 2) {
            asm volatile("v_lshlrev_b32 %0, 16, %1" : "=v"(x[2]) : "v"(x[6]));
            asm volatile("v_and_b32 %0, 0xffff0000, %1" : "=v"(x[3]) : "v"(x[6]));
            asm volatile("v_cvt_pkrtz_f16_f32 %0, %1, %2" : "=v"(x[9]) : "v"(x[2]), "v"(x[3]));
        }
        asm volatile("v_max3_f32 %0, %0, %1, %2" : "+v"(x[7]) : "v"(x[10]), "v"(x[11]));
    }
}

// Extra instruction of a clump: CK 1 VALU, 2 SALU.
template <int CK>
__device__ __forceinline__ void clump_op(uint32_t (&t)[4], uint32_t (&u)[2], int i) {
    if (CK == 1) asm volatile("v_add_u32 %0, %0, %1" : "+v"(t[i & 3]) : "v"(t[(i + 1) & 3]));
    if (CK == 2) asm volatile("s_mov_b32 %0, %1" : "=s"(u[i & 1]) : "s"(u[(i + 1) & 1]));
}

// The slot loop of one wave role (compile-time: MFMA issued, VALU pattern).
// VK: 0 none, 1 NV x v_fma_f32, 2 the attention slot mix (with LDS operands);
// BAR: a workgroup barrier after each 32-slot tile; ROT: the tile's slot
// kinds taken 8 slots later.
// Always inlined: as a called function it keeps the ABI's register limits and
// spills f[] to scratch, which would be timed with the pattern.
// CK: clump kind (0 none, 1 VALU, 2 SALU), CS: clump spread over slots 0..15
// (else at the tile end).
template <bool MF, int VK, int NV, bool BAR = false, bool ROT = false, bool VT = false, int CK = 0, bool CS = false>
__device__ __forceinline__ float slot_loop(int iters, const uint8_t* lds) {
    f32x16 acc[2];
    for (int a = 0; a < 2; ++a)
        for (int v = 0; v < 16; ++v) acc[a][v] = 0.0f;
    bf16x8 qa, qb;
    for (int i = 0; i < 8; ++i) {
        qa[i] = (__bf16)(0.001f * (threadIdx.x + i));
        qb[i] = (__bf16)(0.002f * i);
    }
    float x[12];
    for (int i = 0; i < 12; ++i) x[i] = 0.01f * (threadIdx.x + i);
    const float c = 0.999f;
    const uint32_t w = 0x38383838u + threadIdx.x;
    uint32_t t[4] = {threadIdx.x, threadIdx.x + 1, threadIdx.x + 2, threadIdx.x + 3};
    uint32_t u[2] = {(uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x), 7u};
    const uint8_t* base = lds + (threadIdx.x & 63) * 272;
    // V^T operand: row (lane % 32) of a 32-row dim block, 16-byte unit lane / 32
    const uint8_t* vbase = lds + 17408 + (threadIdx.x & 31) * 144 + ((threadIdx.x >> 5) & 1) * 16;
    for (int it = 0; it < iters; ++it) {
        bf16x8 f[SLOTS];
        if (VK == 2) {
            f[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base));
            f[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + 32));
        }
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            if (VK == 2 && s + 2 < SLOTS) {
                const int s2 = s + 2;
                const uint8_t* addr = (VT && (s2 & 8)) ? vbase + 64 * ((s2 >> 4) & 1) + 32 * ((s2 >> 2) & 1) +
                                                            (s2 & 3) * 32 * 144
                                                      : base + 32 * (s2 & 7) + 4096 * (s2 >> 3);
                f[s2] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(addr));
            }
            if (MF) acc[s & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(VK == 2 ? f[s] : qa, qb, acc[s & 1], 0, 0, 0);
            if (VK == 1) {
#pragma unroll
                for (int j = 0; j < NV; ++j) fma_op(x[j % 12], c);
            }
            if (VK == 2) {
                const int k = ROT ? (s + 8) & 31 : s;  // kernel order: A, K write, A, V write
                tile_valu((k & 8) == 0 ? 0 : (k & 16) == 0 ? 1 : 2, x, c, w);
            }
            if (CK && CS && s < 16) clump_op<CK>(t, u, s);
            if (CK && !CS && s == SLOTS - 1) {
#pragma unroll
                for (int i = 0; i < 16; ++i) clump_op<CK>(t, u, i);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (BAR) __syncthreads();
    }
    float sum = 0.0f;
    for (int a = 0; a < 2; ++a)
        for (int v = 0; v < 16; ++v) sum += acc[a][v];
    for (int i = 0; i < 12; ++i) sum += x[i];
    sum += (float)(t[0] + t[1] + t[2] + t[3] + u[0] + u[1]);
    return sum;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// The tile with the kernel's register dependencies (see TILE_DEP above).
template <bool BAR>
__device__ __forceinline__ float dep_loop(int iters, const uint8_t* lds) {
    f32x16 sblk[2], o[4];
    for (int a = 0; a < 2; ++a)
        for (int v = 0; v < 16; ++v) sblk[a][v] = 0.001f * v;
    for (int a = 0; a < 4; ++a)
        for (int v = 0; v < 16; ++v) o[a][v] = 0.0f;
    bf16x8 qf;
    f16x8 pf;
    for (int i = 0; i < 8; ++i) {
        qf[i] = (__bf16)(0.001f * (threadIdx.x + i));
        pf[i] = (_Float16)(0.002f * i);
    }
    float x[12];
    for (int i = 0; i < 12; ++i) x[i] = 0.01f * (threadIdx.x + i);
    const float c = 0.999f;
    const uint32_t w = 0x38383838u + threadIdx.x;
    const uint8_t* base = lds + (threadIdx.x & 63) * 272;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // two half tiles: step A (8 slots), then a write step (8 slots)
            bf16x8 f[16];
            f[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base));
            f[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + 32));
            f32x16& sn = sblk[h];      // S block produced by this half's step A
            f32x16& sp = sblk[h ^ 1];  // S block of the previous half (softmax input)
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s + 2 < 16)
                    f[s + 2] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + 32 * ((s + 2) & 7) + 4096 * ((s + 2) >> 3)));
                if (s < 8) {
                    sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[s], qf, s == 0 ? f32x16{} : sn, 0, 0, 0);
                    float a0 = sp[2 * s], a1 = sp[2 * s + 1];
                    asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(a0) : "v"(c), "v"(x[8]));
                    asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(a1) : "v"(c), "v"(x[8]));
                    asm volatile("v_exp_f32 %0, %0" : "+v"(a0));
                    asm volatile("v_exp_f32 %0, %0" : "+v"(a1));
                    asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(x[2]) : "v"(a0), "v"(a1));
                    asm volatile("v_dot2c_f32_f16 %0, %1, %2" : "+v"(x[3]) : "v"(x[2]), "v"(x[9]));
                } else {
                    const int i = s - 8;
                    o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, f[s]), pf, o[i & 3], 0, 0, 0);
                    asm volatile("v_cvt_scalef32_pk_f32_fp8 %0, %1, 1.0" : "=v"(*reinterpret_cast<double*>(&x[4])) : "v"(w));
                    asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[4]) : "v"(c));
                    asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[5]) : "v"(c));
                    asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(x[6]) : "v"(x[4]), "v"(x[5]));
                    if (h == 1) {
                        asm volatile("v_lshlrev_b32 %0, 16, %1" : "=v"(x[2]) : "v"(x[6]));
                        asm volatile("v_and_b32 %0, 0xffff0000, %1" : "=v"(x[3]) : "v"(x[6]));
                        asm volatile("v_cvt_pkrtz_f16_f32 %0, %1, %2" : "=v"(x[9]) : "v"(x[2]), "v"(x[3]));
                    }
                    asm volatile("v_max3_f32 %0, %0, %1, %2" : "+v"(x[7]) : "v"(sn[2 * i]), "v"(sn[2 * i + 1]));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (BAR) __syncthreads();
    }
    float sum = 0.0f;
    for (int a = 0; a < 4; ++a)
        for (int v = 0; v < 16; ++v) sum += o[a][v];
    for (int a = 0; a < 2; ++a)
        for (int v = 0; v < 16; ++v) sum += sblk[a][v];
    for (int i = 0; i < 12; ++i) sum += x[i];
    return sum;
}

// One MFMA per slot into a single accumulator.
__device__ __forceinline__ float chain_loop(int iters) {
    f32x16 acc;
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    bf16x8 qa, qb;
    for (int i = 0; i < 8; ++i) {
        qa[i] = (__bf16)(0.001f * (threadIdx.x + i));
        qb[i] = (__bf16)(0.002f * i);
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, qb, acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float sum = 0.0f;
    for (int v = 0; v < 16; ++v) sum += acc[v];
    return sum;
}

template <int PAT, int NV>
__global__ void issue_kernel(int iters, float* out) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
    for (int i = threadIdx.x; i < LDS_BYTES / 4; i += blockDim.x) reinterpret_cast<uint32_t*>(lds)[i] = 0x3c003c00u ^ i;
    __syncthreads();
    float sum;
    if (PAT == MFMA) sum = slot_loop<true, 0, 0>(iters, lds);
    else if (PAT == VALU) sum = slot_loop<false, 1, NV>(iters, lds);
    else if (PAT == MFMA_VALU) sum = slot_loop<true, 1, NV>(iters, lds);
    else if (PAT == TILE) sum = slot_loop<true, 2, 0>(iters, lds);
    else if (PAT == TILE_BAR) sum = slot_loop<true, 2, 0, true>(iters, lds);
    else if (PAT == TILE_BAR_VT) sum = slot_loop<true, 2, 0, true, false, true>(iters, lds);
    else if (PAT == CHAIN) sum = chain_loop(iters);
    else if (PAT == TILE_DEP) sum = dep_loop<true>(iters, lds);
    else if (PAT == VALU_OP) sum = op_loop<NV>(iters);
    else if (PAT == CLUMP_VALU_END) sum = slot_loop<true, 2, 0, true, false, false, 1, false>(iters, lds);
    else if (PAT == CLUMP_VALU_SPREAD) sum = slot_loop<true, 2, 0, true, false, false, 1, true>(iters, lds);
    else if (PAT == CLUMP_SALU_END) sum = slot_loop<true, 2, 0, true, false, false, 2, false>(iters, lds);
    else if (PAT == CLUMP_SALU_SPREAD) sum = slot_loop<true, 2, 0, true, false, false, 2, true>(iters, lds);
    else if (PAT == TILE_BAR_ROT) {
        if ((__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 2) & 1) sum = slot_loop<true, 2, 0, true, true>(iters, lds);
        else sum = slot_loop<true, 2, 0, true>(iters, lds);
    }
    else if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 1) sum = slot_loop<false, 1, NV>(iters, lds);
    else sum = slot_loop<true, 0, 0>(iters, lds);  // SPLIT: even waves MFMA, odd waves VALU
    out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
}

template <int PAT, int NV>
double run(int threads, float* out) {
    const int blocks = 256, iters = 1000;
    hipLaunchKernelGGL((issue_kernel<PAT, NV>), dim3(blocks), dim3(threads), 0, 0, 1, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    CHECK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL((issue_kernel<PAT, NV>), dim3(blocks), dim3(threads), 0, 0, iters, out);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    // per SIMD slot: every wave of the SIMD runs SLOTS * iters slots
    return ms * 1e6 / (double(SLOTS) * iters * (threads / 256));
}

int main() {
    float* out = nullptr;
    CHECK(hipMalloc(&out, 256 * 768 * sizeof(float)));
    printf("%-40s %6s %12s %10s\n", "pattern", "w/SIMD", "ns/slot", "MFMA share");
    for (int threads : {256, 512, 768}) {
        const int wps = threads / 256;
        const double base = run<MFMA, 0>(threads, out);
        // MFMA share: the MFMA-only launch's time per MFMA over this pattern's
        // (frac: share of the waves that issue MFMAs)
        auto line = [&](const char* name, double ns, bool has_mfma, double frac = 1.0) {
            if (has_mfma)
                printf("%-40s %6d %12.2f %9.1f%%\n", name, wps, ns, 100.0 * base * frac / ns);
            else
                printf("%-40s %6d %12.2f %10s\n", name, wps, ns, "-");
        };
        line("mfma", base, true);
        line("valu 8", run<VALU, 8>(threads, out), false);
        line("chain (one accumulator)", run<CHAIN, 0>(threads, out), true);
        line("mfma+4", run<MFMA_VALU, 4>(threads, out), true);
        line("mfma+8", run<MFMA_VALU, 8>(threads, out), true);
        if (wps > 1) line("split 8 (even: mfma, odd: 8 valu)", run<SPLIT, 8>(threads, out), true, 0.5);
        line("tile (attention slot mix + LDS reads)", run<TILE, 0>(threads, out), true);
        line("tile + barrier per tile", run<TILE_BAR, 0>(threads, out), true);
        line("tile + barrier, V^T reads in write slots", run<TILE_BAR_VT, 0>(threads, out), true);
        if (wps > 1) line("tile + barrier, upper waves rotated", run<TILE_BAR_ROT, 0>(threads, out), true);
        line("tile, kernel dependencies, + barrier", run<TILE_DEP, 0>(threads, out), true);
        line("tile + barrier + 16 VALU at tile end", run<CLUMP_VALU_END, 0>(threads, out), true);
        line("tile + barrier + 16 VALU, 1 per slot", run<CLUMP_VALU_SPREAD, 0>(threads, out), true);
        line("tile + barrier + 16 SALU at tile end", run<CLUMP_SALU_END, 0>(threads, out), true);
        line("tile + barrier + 16 SALU, 1 per slot", run<CLUMP_SALU_SPREAD, 0>(threads, out), true);
    }
    // Per-instruction cost of each VALU kind: slot time / 8.
    printf("\n%-28s %14s %14s %14s\n", "VALU kind (ns per instr)", "1 w/SIMD", "2 w/SIMD", "3 w/SIMD");
    auto op_row = [&](int k, double (*f)(int, float*)) {
        printf("%-28s", OP_NAMES[k]);
        for (int threads : {256, 512, 768}) printf(" %14.3f", f(threads, out) / 8.0);
        printf("\n");
    };
    op_row(0, run<VALU_OP, 0>);
    op_row(1, run<VALU_OP, 1>);
    op_row(2, run<VALU_OP, 2>);
    op_row(3, run<VALU_OP, 3>);
    op_row(4, run<VALU_OP, 4>);
    op_row(5, run<VALU_OP, 5>);
    op_row(6, run<VALU_OP, 6>);
    op_row(7, run<VALU_OP, 7>);
    CHECK(hipFree(out));
    return 0;
}
