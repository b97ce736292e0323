// k_conv_common.h — the conv kernels' shared epilogue (fp32 and int8 convs).
#pragma once
#include "mgh_common.h"

namespace mgh {

// out[row + pp + e] = ((v[e] + bias[oc]) + resid[row + pp + e]) for the e with pp + e < M,
// each addition rounded on its own (the graph's conv node, then its Add nodes); one 16-byte
// store when the four pixels are in range and rows are 16-byte aligned (M % 4 == 0).
// STREAM: a final output, stored non-temporally (the next op reads it from HBM anyway; it
// should not evict the operands still in use); split-K partials, read back at once by the
// reduce, stay cacheable.
template <bool STREAM = true>
__device__ __forceinline__ void conv_store(float* __restrict__ out, const float* __restrict__ bias,
                                           const float* __restrict__ resid, size_t row, int oc, int pp, int M,
                                           f32x4 v) {
#pragma clang fp contract(off)
    if (bias) {
        const float b = bias[oc];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = v[e] + b;
    }
    if (pp + 3 < M && (M & 3) == 0) {
        if (resid) v = v + *(const f32x4*)(resid + row + pp);
        if (STREAM) __builtin_nontemporal_store(v, (f32x4*)(out + row + pp));
        else *(f32x4*)(out + row + pp) = v;
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (pp + e < M) out[row + pp + e] = resid ? v[e] + resid[row + pp + e] : v[e];
    }
}

}  // namespace mgh
