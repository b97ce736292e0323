// k_ops.hip — the remaining F32 graph ops of the reference's GPU runtime (gfx950), so that a
// graph the reference's OpenCLRuntime::compute runs also runs here (src/mg-opencl/mg-opencl.cpp
// :1450-1534): SoftMax, Add/Mul with broadcasting, Scale, Gelu, Silu, and the batched,
// stride-aware F32 MulMat the unfused attention chain uses (k_mul_mat_t, :60-94, 1429-1440).
//
// Numerics follow the reference's CPU executor (src/mg-cpu/mg-cpu.cpp), the repository's
// oracle: fp contraction is off, so every product and sum is rounded as the scalar C++ code
// rounds it.
//  * k_softmax_rows: mx = max(x*scale); e = exp(x*scale - mx); y = e * (1/sum e) (mg-cpu.cpp
//    :88-103). The sum is a wave reduction, not the CPU's sequential loop.
//  * k_binary: out = a (op) b, b broadcast over its size-1 dimensions (mg-cpu.cpp:27-38).
//  * k_unary: scale, exact-erf GELU (mg-cpu.cpp:150-156), SiLU (:158-163), library erf/exp.
//  * k_gemm_f32_batched: out[b3][b2][m][n] = act(sum_k w[k,n,b2',b3'] x[k,m,b2,b3] + bias[n])
//    + resid, w broadcasting over batch dimensions of size 1 (mg-cpu.cpp:48-72). Each output
//    accumulates over k in order with a separate multiply and add, as the CPU loop does, so
//    the raw sums are bit-identical to the reference executor's.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

unsigned grid_of(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (unsigned)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// one wave per row of D values (4 rows per 256-thread workgroup)
__global__ __launch_bounds__(256) void k_softmax_rows(const float* __restrict__ x, int64_t rows, int D,
                                                      float scale, float* __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* r = x + row * D;
    float* o = y + row * D;
    float mx = -INFINITY;
    for (int d = lane; d < D; d += 64) mx = fmaxf(mx, r[d] * scale);
    mx = wave_max(mx);
    float s = 0.0f;
    for (int d = lane; d < D; d += 64) {
        const float t = r[d] * scale;
        const float e = expf(t - mx);
        o[d] = e;
        s += e;
    }
    const float inv = 1.0f / wave_sum(s);
    for (int d = lane; d < D; d += 64) o[d] = o[d] * inv;
}

template <int OP>
__global__ __launch_bounds__(256) void k_binary(const float* __restrict__ a, const float* __restrict__ b,
                                                BinaryArgs p, float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t n = p.ne[0] * p.ne[1] * p.ne[2] * p.ne[3];
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        int64_t r = i;
        const int64_t i0 = r % p.ne[0]; r /= p.ne[0];
        const int64_t i1 = r % p.ne[1]; r /= p.ne[1];
        const int64_t i2 = r % p.ne[2];
        const int64_t i3 = r / p.ne[2];
        const float av = a[i0 * p.as[0] + i1 * p.as[1] + i2 * p.as[2] + i3 * p.as[3]];
        const int64_t j = (p.bne[0] == 1 ? 0 : i0) * p.bs[0] + (p.bne[1] == 1 ? 0 : i1) * p.bs[1] +
                          (p.bne[2] == 1 ? 0 : i2) * p.bs[2] + (p.bne[3] == 1 ? 0 : i3) * p.bs[3];
        out[i] = OP == 1 ? av * b[j] : av + b[j];
    }
}

// op 0: x * s; 1: GELU (erf); 2: SiLU
template <int OP>
__global__ __launch_bounds__(256) void k_unary(const float* __restrict__ x, int64_t n, float s,
                                               float* __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        const float v = x[i];
        if (OP == 0) y[i] = v * s;
        else if (OP == 1) y[i] = 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
        else y[i] = v / (1.0f + expf(-v));
    }
}

// 64 x 64 output tile (n x m) per workgroup, 4 x 4 per thread, K in steps of 16 through LDS
constexpr int BT = 64, BK = 16, BP = BT + 4;

template <int ACT>
__global__ __launch_bounds__(256) void k_gemm_f32_batched(BatchedGemmArgs g) {
#pragma clang fp contract(off)
    __shared__ float Ws[BK][BP];
    __shared__ float Xs[BK][BP];
    const int64_t N = g.N, M = g.M, K = g.K;
    const int64_t tiles_n = (N + BT - 1) / BT;
    const int64_t n0 = (blockIdx.x % tiles_n) * BT, m0 = (blockIdx.x / tiles_n) * BT;
    const int64_t bz = blockIdx.y;
    const int64_t b2 = bz % g.B2, b3 = bz / g.B2;
    const float* wb = g.w + (g.wne2 == 1 ? 0 : b2) * g.ws[2] + (g.wne3 == 1 ? 0 : b3) * g.ws[3];
    const float* xb = g.x + b2 * g.xs[2] + b3 * g.xs[3];
    const int tid = threadIdx.x;
    const int tn = tid & 15, tm = tid >> 4;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = q * 256 + tid;
            const int kk = e % BK, rr = e / BK;
            const int64_t k = k0 + kk;
            const int64_t n = n0 + rr, m = m0 + rr;
            Ws[kk][rr] = (k < K && n < N) ? wb[k * g.ws[0] + n * g.ws[1]] : 0.0f;
            Xs[kk][rr] = (k < K && m < M) ? xb[k * g.xs[0] + m * g.xs[1]] : 0.0f;
        }
        __syncthreads();
        const int kn = (int)(K - k0 < BK ? K - k0 : BK);
        for (int kk = 0; kk < kn; kk++) {
            float wv[4], xv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) wv[i] = Ws[kk][4 * tn + i];
#pragma unroll
            for (int j = 0; j < 4; j++) xv[j] = Xs[kk][4 * tm + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float p = wv[i] * xv[j];
                    acc[i][j] = acc[i][j] + p;
                }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t m = m0 + 4 * tm + j;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t n = n0 + 4 * tn + i;
            if (n >= N) continue;
            float v = acc[i][j];
            if (g.bias) v = v + g.bias[n];
            if (ACT == 1) v = 0.5f * v * (1.0f + erff(v * 0.70710678f));
            else if (ACT == 2) v = v / (1.0f + expf(-v));
            const int64_t idx = (bz * M + m) * N + n;
            if (g.resid) v = v + g.resid[idx];
            g.y[idx] = v;
        }
    }
}

}  // namespace

hipError_t launch_softmax_rows(const float* x, int64_t rows, int D, float scale, float* y, hipStream_t s) {
    if (rows == 0 || D == 0) return hipSuccess;
    hipLaunchKernelGGL(k_softmax_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, rows, D, scale, y);
    return hipGetLastError();
}

hipError_t launch_binary(int op, const float* a, const float* b, const BinaryArgs& p, float* out, hipStream_t s) {
    const int64_t n = p.ne[0] * p.ne[1] * p.ne[2] * p.ne[3];
    if (n == 0) return hipSuccess;
    if (op == 1) hipLaunchKernelGGL(k_binary<1>, dim3(grid_of(n)), dim3(256), 0, s, a, b, p, out);
    else hipLaunchKernelGGL(k_binary<0>, dim3(grid_of(n)), dim3(256), 0, s, a, b, p, out);
    return hipGetLastError();
}

hipError_t launch_unary(int op, const float* x, int64_t n, float sc, float* y, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (op == 1) hipLaunchKernelGGL(k_unary<1>, dim3(grid_of(n)), dim3(256), 0, s, x, n, sc, y);
    else if (op == 2) hipLaunchKernelGGL(k_unary<2>, dim3(grid_of(n)), dim3(256), 0, s, x, n, sc, y);
    else hipLaunchKernelGGL(k_unary<0>, dim3(grid_of(n)), dim3(256), 0, s, x, n, sc, y);
    return hipGetLastError();
}

hipError_t launch_gemm_f32_batched(const BatchedGemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0 || a.B2 * a.B3 == 0) return hipSuccess;
    const int64_t tiles = ((a.N + BT - 1) / BT) * ((a.M + BT - 1) / BT);
    const dim3 grid((unsigned)tiles, (unsigned)(a.B2 * a.B3)), block(256);
    if (a.act == 1) hipLaunchKernelGGL(k_gemm_f32_batched<1>, grid, block, 0, s, a);
    else if (a.act == 2) hipLaunchKernelGGL(k_gemm_f32_batched<2>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(k_gemm_f32_batched<0>, grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace mgh
