// k_layernorm.hip — LayerNorm + affine over rows of D (gfx950), optionally emitting the next
// FC layer's activation operand in the same pass.
//
// Semantics: the reference's Norm node with affine (src/mg-cpu/mg-cpu.cpp:105-121 and
// :249-261; GPU twin k_norm_affine, src/mg-opencl/mg-opencl.cpp:705-727):
//   mean = sum(x)/D and var = sum((x-mean)^2)/D in double;
//   inv  = 1 / sqrt((float)var + eps);
//   y    = ((float)(x - mean)) * inv * gamma + beta          (each step rounded to fp32)
// The double statistics follow the reference CPU executor; the sums run in a different
// order, so mean/var can differ in their last double bits and y by at most an fp32 ulp.
// Contraction into FMAs is disabled in the kernel (the reference rounds the product and the
// sum separately), and the sqrt/reciprocal are rounded correctly.
//
// Every LN output in the transformer feeds a quantized FC GEMM (and is kept in fp32 as the
// next residual). EMIT selects the operand written alongside y (k_ln_row.h): none, the
// int8-dot operand of k_gemm_qp, or the fp16-rounded y of the dequantize-fused path.
// Layout: one wave per row (ln_affine_row, shared with the split-K reduce that feeds a
// LayerNorm). HBM-bound: 4 B read + 4 B written per element (+2 + 8/32 B with an emitted
// operand).
#include "mgh_common.h"
#include "mgh_kernels.h"
#include "k_ln_row.h"

namespace mgh {

namespace {

template <int C, int EMIT>
__global__ __launch_bounds__(256) void k_layernorm_affine(const float* __restrict__ x,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta,
                                                          float* __restrict__ y, int rows, float eps,
                                                          void* __restrict__ codes,
                                                          float* __restrict__ dx,
                                                          void* __restrict__ s4) {
    constexpr int D = 256 * C;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;                        // whole wave exits together
    const float* xr = x + (size_t)row * D;
    f32x4 v[C];
#pragma unroll
    for (int c = 0; c < C; c++) v[c] = *(const f32x4*)(xr + 4 * (lane + 64 * c));
    ln_affine_row<C, EMIT>(v, lane, row, gamma, beta, y, eps, codes, dx, s4);
}

template <int EMIT>
hipError_t launch_ln_emit(const float* x, const float* g, const float* b, float* y, int rows, int D,
                          float eps, void* codes, float* dx, void* s4, hipStream_t s) {
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    switch (D / 256) {
#define MGH_LN(CV)                                                                                    \
    case CV:                                                                                          \
        hipLaunchKernelGGL((k_layernorm_affine<CV, EMIT>), grid, block, 0, s, x, g, b, y, rows, eps, \
                           codes, dx, s4);                                                            \
        break;
        MGH_LN(1) MGH_LN(2) MGH_LN(3) MGH_LN(4) MGH_LN(5) MGH_LN(6) MGH_LN(7) MGH_LN(8)
#undef MGH_LN
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_layernorm_affine(const float* x, const float* gamma, const float* beta, float* y,
                                   int rows, int D, float eps, int emit, void* codes, float* dx,
                                   void* s4, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (emit == 1) return launch_ln_emit<1>(x, gamma, beta, y, rows, D, eps, codes, dx, s4, s);
    if (emit == 2) return launch_ln_emit<2>(x, gamma, beta, y, rows, D, eps, codes, dx, s4, s);
    return launch_ln_emit<0>(x, gamma, beta, y, rows, D, eps, codes, dx, s4, s);
}

}  // namespace mgh
