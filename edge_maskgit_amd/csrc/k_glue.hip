// k_glue.hip — the small graph ops around the FC path (gfx950): row gather, broadcast add and
// strided (permute) copy. All HBM-bound streaming kernels.
//
//  * k_get_rows: out[i][:] = a[ids[i]][:], a negative id counts from the end
//    (src/mg-cpu/mg-cpu.cpp:74-86; GPU k_get_rows src/mg-opencl/mg-opencl.cpp:667-672); an id
//    still out of range is clamped to the table (the reference reads out of bounds).
//  * k_add_bcast: out[i] = a[i] + b[i mod nb] — the reference's Add, whose src1 is either the
//    same shape or a prefix that repeats over the leading dimensions (a row-vector bias, the
//    positional table over a batch) (mg-tensor.hpp:46, mg-transformer.cpp:44-46).
//  * k_copy4d: out (contiguous, shape ne) = a viewed with element strides st — the Cont of a
//    permuted view (mg-opencl.cpp:940-945), e.g. the head merge of mg-transformer.cpp:84-85.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

__global__ __launch_bounds__(256) void k_get_rows(const float* __restrict__ a, int64_t E, int64_t R,
                                                  const int32_t* __restrict__ ids, int64_t n,
                                                  float* __restrict__ out) {
    const int64_t i = blockIdx.y;                    // output row
    if (i >= n) return;
    int64_t r = ids[i];
    if (r < 0) r += R;
    r = r < 0 ? 0 : (r >= R ? R - 1 : r);            // out-of-range ids are clamped, never read OOB
    const float* src = a + r * E;
    float* dst = out + i * E;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < E; e += (int64_t)gridDim.x * 256)
        dst[e] = src[e];
}

__global__ __launch_bounds__(256) void k_add_bcast(const float* __restrict__ a,
                                                   const float* __restrict__ b, int64_t nb,
                                                   float* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = a[i] + b[i % nb];
}

__global__ __launch_bounds__(256) void k_copy4d(const float* __restrict__ a, CopyArgs c,
                                                float* __restrict__ out) {
    const int64_t n = c.ne[0] * c.ne[1] * c.ne[2] * c.ne[3];
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        int64_t r = i;
        const int64_t i0 = r % c.ne[0]; r /= c.ne[0];
        const int64_t i1 = r % c.ne[1]; r /= c.ne[1];
        const int64_t i2 = r % c.ne[2];
        const int64_t i3 = r / c.ne[2];
        out[i] = a[i0 * c.st[0] + i1 * c.st[1] + i2 * c.st[2] + i3 * c.st[3]];
    }
}

unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (unsigned)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

}  // namespace

hipError_t launch_get_rows(const float* a, int64_t E, int64_t R, const int32_t* ids, int64_t n,
                           float* out, hipStream_t s) {
    if (n == 0 || E == 0) return hipSuccess;
    const dim3 grid((unsigned)((E + 255) / 256 > 16 ? 16 : (E + 255) / 256), (unsigned)n);
    hipLaunchKernelGGL(k_get_rows, grid, dim3(256), 0, s, a, E, R, ids, n, out);
    return hipGetLastError();
}

hipError_t launch_add_bcast(const float* a, const float* b, int64_t nb, float* out, int64_t n,
                            hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_add_bcast, dim3(grid_for(n)), dim3(256), 0, s, a, b, nb, out, n);
    return hipGetLastError();
}

hipError_t launch_copy4d(const float* a, const CopyArgs& c, float* out, hipStream_t s) {
    const int64_t n = c.ne[0] * c.ne[1] * c.ne[2] * c.ne[3];
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_copy4d, dim3(grid_for(n)), dim3(256), 0, s, a, c, out);
    return hipGetLastError();
}

}  // namespace mgh
