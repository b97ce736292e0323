// mgh_common.h — shared device helpers for the gfx950 kernels of the Q8_0 / Q4_K FC path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgh {

typedef int32_t  i32x4  __attribute__((ext_vector_type(4)));
typedef int32_t  i32x16 __attribute__((ext_vector_type(16)));
typedef float    f32x4  __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8  __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4  __attribute__((ext_vector_type(4)));
// dword-aligned 16-byte vector: Q8_0 blocks are 34 bytes, so block pairs start on 4-byte
// (not 16-byte) boundaries; this type tells the compiler exactly that.
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int WAVE = 64;

// fp16 bits -> fp32 (hardware conversion, exact)
__device__ __forceinline__ float h2f(uint32_t bits16) {
    union { uint16_t u; _Float16 h; } c;
    c.u = (uint16_t)bits16;
    return (float)c.h;
}

// GELU in its erf form (not the tanh form), 0.5 v (1 + erf(v / sqrt 2)) (reference mg-opencl.cpp:36-40, mg-cpu.cpp:65),
// with erf from Abramowitz & Stegun, Handbook of Mathematical Functions, eq. 7.1.26 (Hastings):
// for x >= 0, erf(x) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-x^2), t = 1 / (1 + p x),
// |error| <= 1.5e-7. With h = (1 - erf(|v| / sqrt 2)) / 2 (the coefficients a1..a5 carry the
// 1/2): v Phi(v) = v - |v| h for v >= 0 and -|v| h for v < 0, i.e. max(v, 0) - |v| h.
// 14 VALU operations (rcp and exp2 in hardware) against ~45 for the library erff: in the FC
// epilogue of a 3072-wide GELU layer every operation per output shows in the kernel time.
__device__ __forceinline__ float gelu_erf(float v) {
    const float a = fabsf(v);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678f, a, 1.0f));
    const float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 0.5307027145f, -0.7265760135f), 0.7107068705f),
                                        -0.142248368f), 0.127414796f);
    // exp(-v^2 / 2) = exp2(-v^2 log2(e) / 2)
    const float h = poly * __builtin_amdgcn_exp2f(-0.72134752f * v * v);
    return fmaf(-a, h, fmaxf(v, 0.f));
}

// GELU(erf) / SiLU epilogue activation — reference mg-opencl.cpp:36-40
__device__ __forceinline__ float act_fn(float v, int act) {
    if (act == 1) return gelu_erf(v);
    if (act == 2) return v / (1.0f + expf(-v));
    return v;
}

// XOR-swizzled LDS slot for 16-byte piece `j` of row `r` in a tile of `rows` rows.
// Reads of one piece by 32 consecutive rows and writes of 8 consecutive pieces of one row
// both land in distinct 16-byte bank groups.
__device__ __forceinline__ int swz_slot(int j, int r, int rows) {
    return j * rows + (r ^ (j & 7));
}

// Stage hand-over: this wave's DMA up to the newest N instructions has landed and its LDS
// reads are done, then the workgroup barrier. __syncthreads() is not used here: its
// workgroup fence makes the compiler wait for every outstanding LDS DMA (vmcnt(0)), which
// drains the prefetched stages of the ring. The empty asm statements keep the compiler from
// moving memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void stage_sync() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));   // vmcnt(N) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// XCD-aware workgroup remap: the dispatcher sends workgroup i to XCD i % 8. Give each XCD
// a contiguous range of logical tiles so tiles that share operand rows share an L2.
__device__ __forceinline__ int xcd_remap(int bid, int G) {
    const int full = (G / 8) * 8;
    if (bid >= full) return bid;
    return (bid % 8) * (G / 8) + bid / 8;
}

}  // namespace mgh
