// graph_harness.cpp — runs the graphs of oracle/graph_cases.h through mg::HipRuntime
// (TEST INFRASTRUCTURE ONLY). The same graph source runs on the reference CPU executor in
// oracle/ref_harness.cpp; tests/test_gpu_graph.py compares the two. Built by
// __graft_entry__.build() into tests/_build/libgraph_harness.so.
#include "mg-hip.hpp"
#include "mg-model.hpp"
#include "mg-tensor.hpp"
#include "mg-vqgan.hpp"

#include "graph_cases.h"
#include "graph_sig.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>

namespace {
std::string g_err;
}

extern "C" {

const char* gh_last_error() { return g_err.c_str(); }

// which 0: ffn(K=a, S=b, F=c); 1: ops(D=a, H=b, S=c, B=d). out receives the final node.
int gh_graph_case(int which, int64_t a, int64_t b, int64_t c, int64_t d, float* out, int64_t out_len) {
    try {
        mg::Context ctx((size_t)512 << 20);
        mg::Tensor* o = which == 0 ? graph_cases::ffn(ctx, a, b, c) : graph_cases::ops(ctx, a, b, c, d);
        if (o->nelements() != out_len) { g_err = "output size mismatch"; return -2; }
        mg::Graph g;
        g.build_forward(o);
        mg::HipRuntime rt;
        rt.compute(g);
        std::memcpy(out, o->data, (size_t)out_len * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// One quantized MulMat node with its fused epilogue, y = act(w . x + bias) + resid, through
// HipRuntime under quant algorithm `algo`: w raw GGUF blocks (wtype 8 = Q8_0, 12 = Q4_K) of
// N rows of K, x {K, M} fp32, bias [N] (nullable), resid {N, M} (nullable); out {N, M}.
int gh_quant_mulmat(int wtype, int64_t N, int64_t K, int64_t M, void* wq, float* x, float* bias, float* resid,
                    int act, int algo, float* out) {
    try {
        mg::Context ctx((size_t)64 << 20);
        const int64_t wne[4] = {K, N, 1, 1};
        mg::Tensor* w = ctx.external(wtype == 8 ? mg::Type::Q8_0 : mg::Type::Q4_K, 2, wne, wq);
        const int64_t xne[4] = {K, M, 1, 1};
        mg::Tensor* xt = ctx.external(mg::Type::F32, 2, xne, x);
        const int64_t bne[4] = {N, 1, 1, 1};
        mg::Tensor* b = bias ? ctx.external(mg::Type::F32, 1, bne, bias) : nullptr;
        const int64_t rne[4] = {N, M, 1, 1};
        mg::Tensor* r = resid ? ctx.external(mg::Type::F32, 2, rne, resid) : nullptr;
        mg::Tensor* y = mg::mul_mat_ex(ctx, w, xt, b, act, r);
        mg::Graph g;
        g.build_forward(y);
        mg::HipRuntime rt;
        rt.set_quant_algo(algo);
        rt.compute(g);
        std::memcpy(out, y->data, (size_t)(N * M) * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// A post-norm pair whose gamma is computed after the FC: y = norm_affine(mul_mat_ex(w, x, bias,
// 0, resid), gamma = scale(g0, gs), beta = b0, eps) through HipRuntime under `algo` (the
// graph order puts the scale node between the FC and the Norm). out {N, M}.
int gh_post_norm_case(int wtype, int64_t N, int64_t K, int64_t M, void* wq, float* x, float* bias, float* resid,
                      float* g0, float gs, float* b0, int algo, float* out) {
    try {
        mg::Context ctx((size_t)64 << 20);
        const int64_t wne[4] = {K, N, 1, 1}, xne[4] = {K, M, 1, 1}, nne[4] = {N, 1, 1, 1}, rne[4] = {N, M, 1, 1};
        mg::Tensor* w = ctx.external(wtype == 8 ? mg::Type::Q8_0 : mg::Type::Q4_K, 2, wne, wq);
        mg::Tensor* fc = mg::mul_mat_ex(ctx, w, ctx.external(mg::Type::F32, 2, xne, x),
                                        ctx.external(mg::Type::F32, 1, nne, bias), 0,
                                        ctx.external(mg::Type::F32, 2, rne, resid));
        mg::Tensor* gamma = mg::scale(ctx, ctx.external(mg::Type::F32, 1, nne, g0), gs);
        mg::Tensor* y = mg::norm_affine(ctx, fc, gamma, ctx.external(mg::Type::F32, 1, nne, b0), 1e-5f);
        mg::Graph g;
        g.build_forward(y);
        mg::HipRuntime rt;
        rt.set_quant_algo(algo);
        rt.compute(g);
        std::memcpy(out, y->data, (size_t)(N * M) * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// Host-only checks of the graph API semantics (no device): returns 0 or the first failed check.
//  1: build_forward starts from an empty node list (reference src/mg-tensor.cpp:241)
//  2: a view whose size-1 dimension carries a non-packed stride is not contiguous
//     (reference src/mg-tensor.cpp:36-43)
//  3: a contiguous tensor and a reshape of it are contiguous; quantized tensors (all strides 0)
//     are contiguous
int gh_api_checks() {
    mg::Context c(1 << 20);
    mg::Tensor* a = c.tensor2d(mg::Type::F32, 8, 4);
    mg::Tensor* b = c.tensor2d(mg::Type::F32, 8, 4);
    mg::Tensor* s1 = mg::add(c, a, b);
    mg::Tensor* s2 = mg::gelu(c, mg::scale(c, a, 2.0f));
    mg::Graph g;
    g.build_forward(s1);
    g.build_forward(s2);
    if (g.nodes.size() != 2 || g.nodes[0]->op != mg::Op::Scale || g.nodes[1] != s2) return 1;
    mg::Tensor* t = c.tensor3d(mg::Type::F32, 8, 1, 4);
    mg::Tensor* p = mg::permute(c, t, 0, 2, 1, 3);      // {8, 4, 1}: dim 2 has stride 32 B
    if (p->ne[2] != 1 || p->is_contiguous()) return 2;
    if (!t->is_contiguous() || !mg::reshape(c, t, {32})->is_contiguous()) return 3;
    const int64_t qne[4] = {256, 2, 1, 1};
    mg::Tensor* q = c.external(mg::Type::Q8_0, 2, qne, nullptr);
    if (!q->is_contiguous()) return 3;
    return 0;
}

// The signature (graph_sig.h) of build_vqgan_decoder's graph for B grids of n_tokens ids
// (ids ne = {n_tokens} for B == 1, {n_tokens, B} otherwise); built, not run (host only).
int64_t gh_vqgan_graph_sig(const char* gguf_path, int64_t n_tokens, int64_t B, int64_t arena_bytes, char* buf,
                           int64_t cap) {
    try {
        mg::Context wctx(64 << 20);
        auto model = mg::Model::load(gguf_path, wctx);
        mg::Context ctx((size_t)arena_bytes);
        mg::Tensor* ids = B == 1 ? ctx.tensor1d(mg::Type::I32, n_tokens) : ctx.tensor2d(mg::Type::I32, n_tokens, B);
        mg::Graph g;
        g.build_forward(mg::build_vqgan_decoder(ctx, *model, ids));
        return graph_sig::copy_out(graph_sig::describe(g), buf, cap);
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

}  // extern "C"
