// k_gemm_f32.hip — fp32 FC GEMM with the fused epilogue (gfx950): the MLM head tied to the
// fp32 token embedding, and MulMat nodes whose weights are F32.
//
// Semantics: the reference's F32 MulMat (CPU src/mg-cpu/mg-cpu.cpp:48-72, GPU k_mul_mat_t
// src/mg-opencl/mg-opencl.cpp:60-94): y[m][n] = act(sum_k w[n][k] * x[m][k] + bias[n]) +
// resid[m][n], fp32 accumulation (the summation order differs from the reference's
// sequential k loop), epilogue order of mg-opencl.cpp:36-40, 485-491.
//
// gfx950 mapping: v_mfma_f32_16x16x4_f32 (fp32 inputs, fp32 accumulation) on 64 x 64 output
// tiles per 256-thread workgroup (2x2 waves of 2x2 MFMA tiles), K in steps of 32 staged
// through LDS with a register prefetch of the next step. LDS rows are 36 floats so the
// 16-row x 4-column fragment reads hit 64 distinct banks. Weights take the MFMA A role so a
// lane holds four consecutive output columns of one row.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

constexpr int TB = 64;     // output tile (rows of W and of x)
constexpr int KS = 32;     // K step
constexpr int LD = 36;     // LDS row stride (floats)

template <int ACT>
__device__ __forceinline__ float act_f(float v) {
    if (ACT == 1) return gelu_erf(v);
    if (ACT == 2) return v / (1.0f + expf(-v));
    return v;
}

template <int ACT>
__global__ __launch_bounds__(256) void k_gemm_f32(GemmF32Args g) {
    __shared__ __attribute__((aligned(16))) float Ws[TB * LD];
    __shared__ __attribute__((aligned(16))) float Xs[TB * LD];
    const int M = g.M, N = g.N, K = g.K;
    const int tiles_n = (N + TB - 1) / TB;
    const int bt = xcd_remap(blockIdx.x, tiles_n * ((M + TB - 1) / TB));
    const int n0 = (bt % tiles_n) * TB, m0 = (bt / tiles_n) * TB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = (wave & 1) * 32, wm = (wave >> 1) * 32;
    const int l16 = lane & 15, lg = lane >> 4;

    // each thread moves two float4 of each operand per K step: tile row idx/8, column 4*(idx%8)
    const int r0 = tid >> 3, c4 = (tid & 7) * 4;
    const float* wp0 = g.w + (size_t)min(n0 + r0, N - 1) * K + c4;
    const float* wp1 = g.w + (size_t)min(n0 + r0 + 32, N - 1) * K + c4;
    const float* xp0 = g.x + (size_t)min(m0 + r0, M - 1) * K + c4;
    const float* xp1 = g.x + (size_t)min(m0 + r0 + 32, M - 1) * K + c4;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    f32x4 pw0 = *(const f32x4*)wp0, pw1 = *(const f32x4*)wp1;
    f32x4 px0 = *(const f32x4*)xp0, px1 = *(const f32x4*)xp1;
    for (int k0 = 0; k0 < K; k0 += KS) {
        __syncthreads();
        *(f32x4*)&Ws[r0 * LD + c4] = pw0;
        *(f32x4*)&Ws[(r0 + 32) * LD + c4] = pw1;
        *(f32x4*)&Xs[r0 * LD + c4] = px0;
        *(f32x4*)&Xs[(r0 + 32) * LD + c4] = px1;
        __syncthreads();
        if (k0 + KS < K) {
            pw0 = *(const f32x4*)(wp0 + k0 + KS);
            pw1 = *(const f32x4*)(wp1 + k0 + KS);
            px0 = *(const f32x4*)(xp0 + k0 + KS);
            px1 = *(const f32x4*)(xp1 + k0 + KS);
        }
#pragma unroll
        for (int kk = 0; kk < KS; kk += 4) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = Ws[(wn + 16 * i + l16) * LD + kk + lg];
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = Xs[(wm + 16 * j + l16) * LD + kk + lg];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
    // epilogue: register r of tile (i, j) is y[m0+wm+16j+l16][n0+wn+16i+4lg+r]
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int m = m0 + wm + 16 * j + l16;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int n = n0 + wn + 16 * i + 4 * lg + r;
                if (n >= N) continue;
                float v = acc[i][j][r];
                if (g.bias) v += g.bias[n];
                v = act_f<ACT>(v);
                const size_t o = (size_t)m * N + n;
                if (g.resid) v += g.resid[o];
                g.y[o] = v;
            }
    }
}

}  // namespace

hipError_t launch_gemm_f32(const GemmF32Args& a, hipStream_t s) {
    if (a.M == 0) return hipSuccess;
    const int tiles = ((a.N + TB - 1) / TB) * ((a.M + TB - 1) / TB);
    const dim3 grid(tiles), block(256);
    if (a.act == 1) hipLaunchKernelGGL(k_gemm_f32<1>, grid, block, 0, s, a);
    else if (a.act == 2) hipLaunchKernelGGL(k_gemm_f32<2>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(k_gemm_f32<0>, grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace mgh
