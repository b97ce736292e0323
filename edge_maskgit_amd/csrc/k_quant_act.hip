// k_quant_act.hip — per-32-block int8 activation quantizer (gfx950).
//
// Semantics of the reference's k_quantize_q8 (src/mg-opencl/mg-opencl.cpp:424-434):
//   amax = max|x| over the block; d = amax/127; id = d > 0 ? 1/d : 0;
//   dx[block] = d (fp32); qx[i] = round(x[i]*id) with round half away from zero.
// Additionally emits sx[block] = sum of the block's qx (used by the Q4_K min term,
// mg-opencl.cpp:559-563), so the GEMM does not re-sum the activations.
//
// Layout: x [M][K] fp32 row-major, blocks run along K, so the flat block index
// b = m*(K/32) + t addresses x + 32*b, dx[b], sx[b]. Eight lanes own one block, each lane
// one float4 (16-byte coalesced loads); the block max and sum are xor-shuffle reductions
// inside the 8-lane group. HBM-bound: 4 B read and 1.25 B written per element.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

// F16 = false: qx is int8 (the reference layout). F16 = true: the same codes are written as
// fp16 values (exact for |q| <= 127), the operand format of k_gemm_qp.
template <bool F16>
__global__ __launch_bounds__(256) void k_quantize_act_q8(const float* __restrict__ x,
                                                         void* __restrict__ qx,
                                                         float* __restrict__ dx,
                                                         int32_t* __restrict__ sx,
                                                         int64_t nblocks) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int sub = (int)(gid & 7);
    const bool valid = blk < nblocks;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (valid) v = *(const f32x4*)(x + blk * 32 + sub * 4);
    float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    a = fmaxf(a, __shfl_xor(a, 1));
    a = fmaxf(a, __shfl_xor(a, 2));
    a = fmaxf(a, __shfl_xor(a, 4));
    const float d = a / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = (int)roundf(v.x * id);
    const int q1 = (int)roundf(v.y * id);
    const int q2 = (int)roundf(v.z * id);
    const int q3 = (int)roundf(v.w * id);
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (valid) {
        if (F16) {
            typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
            *(f16x4*)((_Float16*)qx + blk * 32 + sub * 4) =
                f16x4{(_Float16)q0, (_Float16)q1, (_Float16)q2, (_Float16)q3};
        } else {
            const uint32_t packed = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                    ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
            *(uint32_t*)((int8_t*)qx + blk * 32 + sub * 4) = packed;
        }
        if (sub == 0) {
            dx[blk] = d;
            if (sx) sx[blk] = s;
        }
    }
}

hipError_t launch_quantize_act_q8(const float* x, int8_t* qx, float* dx, int32_t* sx,
                                  int64_t M, int64_t K, hipStream_t s) {
    const int64_t nblocks = M * (K / 32);
    const int64_t threads = nblocks * 8;
    const int64_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(k_quantize_act_q8<false>, dim3((unsigned)grid), dim3(256), 0, s, x,
                       (void*)qx, dx, sx, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_act_q8_f16(const float* x, _Float16* qx16, float* dx, int32_t* sx,
                                      int64_t M, int64_t K, hipStream_t s) {
    const int64_t nblocks = M * (K / 32);
    const int64_t grid = (nblocks * 8 + 255) / 256;
    hipLaunchKernelGGL(k_quantize_act_q8<true>, dim3((unsigned)grid), dim3(256), 0, s, x,
                       (void*)qx16, dx, sx, nblocks);
    return hipGetLastError();
}

// Activation operand of the dequantize-weights algorithm (MGH_ALGO_DEQ_F16, the reference's
// fp16-slab path k_mul_mat_*_t2_h, mg-opencl.cpp:320-411): x rounded to fp16 (round to
// nearest even, as vstore_half_rte), unit block scales so the packed GEMM's per-block scale
// reduces to the weight scale, and ux[block] = fp32 sum of the rounded values for Q4_K's
// min term (sum_i (d*sc*q_i - dmin*m) * x_i = d*sc*sum_i q_i*x_i - dmin*m*ux).
__global__ __launch_bounds__(256) void k_round_act_f16(const float* __restrict__ x,
                                                       _Float16* __restrict__ x16,
                                                       float* __restrict__ ones,
                                                       float* __restrict__ ux, int64_t nblocks) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int sub = (int)(gid & 7);
    const bool valid = blk < nblocks;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (valid) v = *(const f32x4*)(x + blk * 32 + sub * 4);
    const f16x4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    float s = ((float)h.x + (float)h.y) + ((float)h.z + (float)h.w);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (valid) {
        *(f16x4*)(x16 + blk * 32 + sub * 4) = h;
        if (sub == 0) {
            ones[blk] = 1.0f;
            if (ux) ux[blk] = s;
        }
    }
}

hipError_t launch_round_act_f16(const float* x, _Float16* x16, float* ones, float* ux,
                                int64_t M, int64_t K, hipStream_t s) {
    const int64_t nblocks = M * (K / 32);
    const int64_t grid = (nblocks * 8 + 255) / 256;
    hipLaunchKernelGGL(k_round_act_f16, dim3((unsigned)grid), dim3(256), 0, s, x, x16, ones, ux,
                       nblocks);
    return hipGetLastError();
}

// Graph-capture-safe fill (used instead of hipMemsetAsync).
__global__ __launch_bounds__(256) void k_fill_u32(uint32_t* __restrict__ p, uint32_t v, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * 256;
    for (; i < n; i += stride) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    size_t grid = (n + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)grid), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

}  // namespace mgh
