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

// GELU(erf) / SiLU epilogue activation — reference mg-opencl.cpp:36-40
__device__ __forceinline__ float act_fn(float v, int act) {
    if (act == 1) return 0.5f * v * (1.0f + erff(v * 0.70710678f));
    if (act == 2) return v / (1.0f + expf(-v));
    return v;
}

// XOR-swizzled LDS slot for 16-byte piece `j` of row `r` in a tile of `rows` rows.
// Reads of one piece by 32 consecutive rows and writes of 8 consecutive pieces of one row
// both land in distinct 16-byte bank groups.
__device__ __forceinline__ int swz_slot(int j, int r, int rows) {
    return j * rows + (r ^ (j & 7));
}

// XCD-aware workgroup remap: the dispatcher sends workgroup i to XCD i % 8. Give each XCD
// a contiguous range of logical tiles so tiles that share operand rows share an L2.
__device__ __forceinline__ int xcd_remap(int bid, int G) {
    const int full = (G / 8) * 8;
    if (bid >= full) return bid;
    return (bid % 8) * (G / 8) + bid / 8;
}

}  // namespace mgh
