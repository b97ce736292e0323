// graph_cases.h — graphs built with the mg tensor API, shared by the two test harnesses
// (TEST INFRASTRUCTURE ONLY): oracle/ref_harness.cpp compiles them against the reference's
// own headers and runs the reference CPU executor; tests/graph_harness.cpp compiles the same
// text against this repository's include/mg-tensor.hpp and runs HipRuntime. The same source
// building the same graph on both sides is the drop-in check of the graph API.
#pragma once

#include <cmath>
#include <cstdint>

namespace graph_cases {

// sin(0.05 i + phase) * 0.5 over the flat elements: the input recipe of the reference's own
// GPU harness (tools/test-opencl.cpp:12-15)
inline void fill_sin(mg::Tensor* t, float phase) {
    const int64_t n = t->nelements();
    float* p = static_cast<float*>(t->data);
    for (int64_t i = 0; i < n; i++) p[i] = std::sin(0.05f * i + phase) * 0.5f;
}

// The FFN graph of tools/test-opencl.cpp:18-28: mul_mat -> add_bias -> gelu -> mul_mat ->
// add_bias, x {K,S}, W1 {K,F}, W2 {F,K}.
inline mg::Tensor* ffn(mg::Context& c, int64_t K, int64_t S, int64_t F) {
    using namespace mg;
    Tensor* x = c.tensor2d(Type::F32, K, S);  fill_sin(x, 0.1f);
    Tensor* W1 = c.tensor2d(Type::F32, K, F); fill_sin(W1, 0.3f);
    Tensor* b1 = c.tensor1d(Type::F32, F);    fill_sin(b1, 0.7f);
    Tensor* W2 = c.tensor2d(Type::F32, F, K); fill_sin(W2, 0.9f);
    Tensor* b2 = c.tensor1d(Type::F32, K);    fill_sin(b2, 1.3f);
    Tensor* h = add_bias(c, mul_mat(c, W1, x), b1);
    Tensor* g = gelu(c, h);
    return add_bias(c, mul_mat(c, W2, g), b2);
}

// The remaining elementwise / batched ops in one graph (D x R rows, H heads):
//   s  = soft_max(mul_mat(k, q), scale)      batched F32 product over strided head views
//   a  = mul_mat(permute(v, 1, 0, 2, 3), s)   second product on a transposed view
//   m  = mul(a, col)                           Mul broadcast over dims 0 and 2
//   z  = silu(scale(m, 0.75)) + mul(gelu(m), row)
inline mg::Tensor* ops(mg::Context& c, int64_t D, int64_t H, int64_t S, int64_t B) {
    using namespace mg;
    Tensor* q0 = c.tensor3d(Type::F32, D * H, S, B); fill_sin(q0, 0.2f);
    Tensor* k0 = c.tensor3d(Type::F32, D * H, S, B); fill_sin(k0, 0.5f);
    Tensor* v0 = c.tensor3d(Type::F32, D * H, S, B); fill_sin(v0, 0.8f);
    Tensor* q = permute(c, reshape(c, q0, {D, H, S, B}), 0, 2, 1, 3);   // {D,S,H,B}
    Tensor* k = permute(c, reshape(c, k0, {D, H, S, B}), 0, 2, 1, 3);
    Tensor* v = permute(c, reshape(c, v0, {D, H, S, B}), 0, 2, 1, 3);
    Tensor* s = soft_max(c, mul_mat(c, k, q), 1.0f / std::sqrt((float)D));  // {S,S,H,B}
    Tensor* a = mul_mat(c, permute(c, v, 1, 0, 2, 3), s);                    // {D,S,H,B}
    Tensor* col = c.tensor4d(Type::F32, 1, S, 1, B); fill_sin(col, 1.1f);
    Tensor* row = c.tensor1d(Type::F32, D);          fill_sin(row, 1.7f);
    Tensor* m = mul(c, a, col);
    return add(c, silu(c, scale(c, m, 0.75f)), mul(c, gelu(c, m), row));
}

}  // namespace graph_cases
