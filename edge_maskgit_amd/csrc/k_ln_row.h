// k_ln_row.h — LayerNorm + affine of one row held by one wave (gfx950), shared by the
// LayerNorm kernel and the split-K reduce that feeds a LayerNorm, so both give the same bits.
//
// Semantics: the reference's Norm node with affine (src/mg-cpu/mg-cpu.cpp:105-121 and
// :249-261; GPU twin k_norm_affine, src/mg-opencl/mg-opencl.cpp:705-727):
//   mean = sum(x)/D and var = sum((x-mean)^2)/D in double;
//   inv  = 1 / sqrt((float)var + eps);
//   y    = ((float)(x - mean)) * inv * gamma + beta          (each step rounded to fp32)
// Row layout: D = 256 C; lane l holds the float4 chunks c = 0..C-1 at element 4 (l + 64 c),
// so the 8 lanes of a 32-element block are adjacent (xor-shuffle block reductions).
// EMIT selects the next FC's operand written alongside y:
//   0: none;
//   1: int8-dot operand of k_gemm_qp — the k_quantize_act_q8 rule (mg-opencl.cpp:424-434)
//      applied to y: fp16 codes [rows][D], dx [rows][D/32], int32 code sums s4 [rows][D/32];
//   2: dequant-fp16 operand — y rounded to fp16, unit dx and fp32 block sums of the rounded
//      values in s4 (each nullable).
#pragma once

#include "mgh_common.h"

namespace mgh {

typedef _Float16 ln_f16x4 __attribute__((ext_vector_type(4)));

// xor-butterfly sum of a double over the wave; the two 32-bit halves are shuffled
// explicitly so no overload can narrow the value
__device__ __forceinline__ double ln_shfl_xor_d(double v, int o) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)u, o);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(u >> 32), o);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double ln_wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += ln_shfl_xor_d(v, o);
    return v;
}

template <int C, int EMIT>
__device__ __forceinline__ void ln_affine_row(const f32x4 (&v)[C], int lane, int row,
                                              const float* __restrict__ gamma,
                                              const float* __restrict__ beta, float* __restrict__ y,
                                              float eps, void* __restrict__ codes,
                                              float* __restrict__ dx, void* __restrict__ s4) {
#pragma clang fp contract(off)   // y = v*gamma + beta rounds twice, as in the reference
    constexpr int D = 256 * C;
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < C; c++) s += ((double)v[c].x + (double)v[c].y) + ((double)v[c].z + (double)v[c].w);
    const double mean = ln_wave_sum_d(s) / (double)D;
    double q = 0.0;
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const double d = (double)v[c][e] - mean;
            q += d * d;
        }
    const double var = ln_wave_sum_d(q) / (double)D;
    // 1/sqrt in fp32 with each step correctly rounded, as the reference CPU computes it: the
    // fp32 sqrt and divide are evaluated in double and rounded once to fp32 (exact for sqrt
    // and division since 53 >= 2*24 + 2); the device's fp32 sqrt is not correctly rounded.
    const float sq = (float)sqrt((double)__fadd_rn((float)var, eps));
    const float inv = (float)(1.0 / (double)sq);
    float* yr = y + (size_t)row * D;
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int k = 4 * (lane + 64 * c);
        const f32x4 g = *(const f32x4*)(gamma + k);
        const f32x4 b = *(const f32x4*)(beta + k);
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++)
            o[e] = (float)((double)v[c][e] - mean) * inv * g[e] + b[e];
        __builtin_nontemporal_store(o, (f32x4*)(yr + k));   // streamed: read again a few kernels later
        if (EMIT == 1) {
            // k_quantize_act_q8 on the 32-element block of lanes 8j..8j+7
            float a = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
            a = fmaxf(a, __shfl_xor(a, 1));
            a = fmaxf(a, __shfl_xor(a, 2));
            a = fmaxf(a, __shfl_xor(a, 4));
            const float d = a / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            const int q0 = (int)roundf(o.x * id), q1 = (int)roundf(o.y * id);
            const int q2 = (int)roundf(o.z * id), q3 = (int)roundf(o.w * id);
            int sqc = q0 + q1 + q2 + q3;
            sqc += __shfl_xor(sqc, 1);
            sqc += __shfl_xor(sqc, 2);
            sqc += __shfl_xor(sqc, 4);
            *(ln_f16x4*)((_Float16*)codes + (size_t)row * D + k) =
                ln_f16x4{(_Float16)q0, (_Float16)q1, (_Float16)q2, (_Float16)q3};
            if ((lane & 7) == 0) {
                const size_t blk = (size_t)row * (D / 32) + (k >> 5);
                dx[blk] = d;
                ((int32_t*)s4)[blk] = sqc;
            }
        } else if (EMIT == 2) {
            const ln_f16x4 h = {(_Float16)o.x, (_Float16)o.y, (_Float16)o.z, (_Float16)o.w};
            float su = ((float)h.x + (float)h.y) + ((float)h.z + (float)h.w);
            su += __shfl_xor(su, 1);
            su += __shfl_xor(su, 2);
            su += __shfl_xor(su, 4);
            __builtin_nontemporal_store(h, (ln_f16x4*)((_Float16*)codes + (size_t)row * D + k));
            if ((lane & 7) == 0) {
                const size_t blk = (size_t)row * (D / 32) + (k >> 5);
                if (dx) dx[blk] = 1.0f;
                if (s4) ((float*)s4)[blk] = su;
            }
        }
    }
}

}  // namespace mgh
