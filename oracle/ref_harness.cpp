// ref_harness.cpp — C entry points over the reference's own CPU executor (TEST INFRASTRUCTURE).
//
// Linked against the reference sources where they lie (mg-tensor.cpp, mg-cpu/mg-cpu.cpp,
// mg-model.cpp, mg-transformer.cpp, mg-generate.cpp, mg-vqgan.cpp) by oracle/Makefile into oracle/_ref/libmgref.so. Only
// tests and bench.py's cpu_baseline leg load it. Each function builds the same graph the
// reference builds and runs the reference's mg::compute (src/mg-cpu/mg-cpu.cpp:296-298),
// so its results are the reference's F32 CPU semantics, not a restatement.
#include "mg-generate.hpp"
#include "mg-model.hpp"
#include "mg-tensor.hpp"
#include "mg-transformer.hpp"
#include "mg-vqgan.hpp"

#include "graph_cases.h"
#include "graph_sig.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

using namespace mg;

namespace {
std::string g_err;

Tensor* ext2(Context& c, const float* p, int64_t ne0, int64_t ne1) {
    int64_t ne[4] = {ne0, ne1, 1, 1};
    return c.external(Type::F32, 2, ne, const_cast<float*>(p));
}
}  // namespace

extern "C" {

const char* mgref_last_error() { return g_err.c_str(); }

// y[M][N] = act(w[N][K] . x[M][K] + bias) + resid via mul_mat_ex (mg-tensor.cpp:117-123)
int mgref_mul_mat(const float* w, int64_t N, int64_t K, const float* x, int64_t M,
                  const float* bias, int act, const float* resid, float* y) {
    try {
        Context c(64 << 20);
        Tensor* tw = ext2(c, w, K, N);
        Tensor* tx = ext2(c, x, K, M);
        Tensor* tb = nullptr;
        if (bias) { int64_t ne[4] = {N, 1, 1, 1}; tb = c.external(Type::F32, 1, ne, const_cast<float*>(bias)); }
        Tensor* tr = resid ? ext2(c, resid, N, M) : nullptr;
        Tensor* out = mul_mat_ex(c, tw, tx, tb, act, tr);
        Graph g; g.build_forward(out); compute(c, g);
        std::memcpy(y, out->data, (size_t)(M * N) * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// LayerNorm + affine via norm_affine (mg-tensor.cpp:141-147)
int mgref_norm_affine(const float* x, int64_t rows, int64_t D, const float* gamma,
                      const float* beta, float eps, float* y) {
    try {
        Context c(16 << 20);
        Tensor* tx = ext2(c, x, D, rows);
        int64_t ne[4] = {D, 1, 1, 1};
        Tensor* tg = c.external(Type::F32, 1, ne, const_cast<float*>(gamma));
        Tensor* tb = c.external(Type::F32, 1, ne, const_cast<float*>(beta));
        Tensor* out = norm_affine(c, tx, tg, tb, eps);
        Graph g; g.build_forward(out); compute(c, g);
        std::memcpy(y, out->data, (size_t)(rows * D) * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// Attention on q/k/v laid out as the transformer's linear outputs [B][S][H*D]: the same
// reshape({D,H,S,B}) + permute(0,2,1,3) views as mg-transformer.cpp:65-67 feed
// flash_attention (mg-tensor.cpp:186-198). Output is contiguous {D,S,H,B}.
int mgref_attention(const float* q, const float* k, const float* v, int64_t D, int64_t S,
                    int64_t H, int64_t B, float scale, float* o) {
    try {
        Context c(64 << 20);
        int64_t ne[4] = {D * H, S, B, 1};
        auto view = [&](const float* p) {
            Tensor* t = c.external(Type::F32, 3, ne, const_cast<float*>(p));
            return permute(c, reshape(c, t, {D, H, S, B}), 0, 2, 1, 3);
        };
        Tensor* out = flash_attention(c, view(q), view(k), view(v), scale);
        Graph g; g.build_forward(out); compute(c, g);
        std::memcpy(o, out->data, (size_t)(D * S * H * B) * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// Full transformer forward on an F32 GGUF: Model::load + build_transformer + compute
// (the path of tools/verify-transformer.cpp:40-55). tokens [B][S] -> logits [B][S][vocab].
int mgref_transformer_forward(const char* gguf_path, const int32_t* tokens, int64_t S,
                              int64_t B, float* logits, int64_t logits_len) {
    try {
        Context wctx(64 << 20);
        auto model = Model::load(gguf_path, wctx);
        Context ctx((size_t)1 << 30);
        Tensor* tok = ctx.tensor2d(Type::I32, S, B);
        std::memcpy(tok->data, tokens, (size_t)(S * B) * sizeof(int32_t));
        Tensor* out = build_transformer(ctx, *model, tok);
        if (out->nelements() != logits_len) { g_err = "logits size mismatch"; return -2; }
        Graph g; g.build_forward(out); compute(ctx, g);
        std::memcpy(logits, out->data, (size_t)logits_len * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// The graphs of graph_cases.h on the reference CPU executor (the same source HipRuntime runs
// in tests/graph_harness.cpp). which 0: ffn(K=a, S=b, F=c); 1: ops(D=a, H=b, S=c, B=d).
int mgref_graph_case(int which, int64_t a, int64_t b, int64_t c, int64_t d, float* out, int64_t out_len) {
    try {
        Context ctx((size_t)512 << 20);
        Tensor* o = which == 0 ? graph_cases::ffn(ctx, a, b, c) : graph_cases::ops(ctx, a, b, c, d);
        if (o->nelements() != out_len) { g_err = "output size mismatch"; return -2; }
        Graph g; g.build_forward(o); compute(ctx, g);
        std::memcpy(out, o->data, (size_t)out_len * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// The reference's own decoding loop, generate() (src/mg-generate.cpp:39-123), on a GGUF
// model's hyper-parameters, driven through its two hooks: the TransformerFwd hook records the
// tokens of each step's forward (tokens_out [steps][S]) and answers with the caller's logits for
// that step (logits [steps][S][vocab]); the VqganFwd hook captures the final token grid
// (grid_out [n_tokens]) and returns a blank image, so neither the transformer nor the VQGAN runs.
int mgref_generate(const char* gguf_path, int class_id, uint64_t seed, int steps, float temperature,
                   const float* logits, int32_t* tokens_out, int32_t* grid_out) {
    try {
        Context wctx(64 << 20);
        auto model = Model::load(gguf_path, wctx);
        const auto& h = model->hparams();
        const int S = h.n_tokens + 1;
        const size_t per = (size_t)S * h.vocab_size;
        int step = 0;
        TransformerFwd fwd = [&](const int32_t* tok, float* out) {
            if (step >= steps) throw std::runtime_error("more forwards than steps");
            std::memcpy(tokens_out + (size_t)step * S, tok, (size_t)S * sizeof(int32_t));
            std::memcpy(out, logits + (size_t)step * per, per * sizeof(float));
            step++;
        };
        VqganFwd vq = [&](const int32_t* grid, float* img) {
            std::memcpy(grid_out, grid, (size_t)h.n_tokens * sizeof(int32_t));
            std::memset(img, 0, (size_t)h.resolution * h.resolution * 3 * sizeof(float));
        };
        GenConfig cfg;
        cfg.class_id = class_id;
        cfg.steps = steps;
        cfg.seed = seed;
        cfg.temperature = temperature;
        generate(*model, cfg, false, fwd, vq);
        if (step != steps) { g_err = "fewer forwards than steps"; return -2; }
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// conv_2d (mg-tensor.cpp:167-177) on the CPU executor's k_conv_2d (mg-cpu.cpp:165-190):
// in {IW, IH, IC, N}, ker {KW, KH, IC, OC} -> out {OW, OH, OC, N}
int mgref_conv2d(const float* in, int64_t IW, int64_t IH, int64_t IC, int64_t N, const float* ker,
                 int64_t KW, int64_t KH, int64_t OC, int stride, int pad, float* out, int64_t out_len) {
    try {
        Context c((size_t)out_len * 4 + (16 << 20));   // the output node's storage is in the arena
        int64_t ni[4] = {IW, IH, IC, N}, nk[4] = {KW, KH, IC, OC};
        Tensor* ti = c.external(Type::F32, 4, ni, const_cast<float*>(in));
        Tensor* tk = c.external(Type::F32, 4, nk, const_cast<float*>(ker));
        Tensor* o = conv_2d(c, tk, ti, stride, pad);
        if (o->nelements() != out_len) { g_err = "conv2d output size mismatch"; return -2; }
        Graph g; g.build_forward(o); compute(c, g);
        std::memcpy(out, o->data, (size_t)out_len * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// group_norm / group_norm_affine_silu (mg-tensor.cpp:148-163) on the CPU executor
// (mg-cpu.cpp:123-147, 262-276); gamma == NULL: no affine
int mgref_group_norm(const float* x, int64_t W, int64_t H, int64_t C, int64_t N, int groups, float eps,
                     const float* gamma, const float* beta, float* y) {
    try {
        const size_t n = (size_t)(W * H * C * N);
        Context c(n * 4 + (16 << 20));
        int64_t nx[4] = {W, H, C, N}, nc[4] = {C, 1, 1, 1};
        Tensor* tx = c.external(Type::F32, 4, nx, const_cast<float*>(x));
        Tensor* o = gamma ? group_norm_affine_silu(c, tx, c.external(Type::F32, 1, nc, const_cast<float*>(gamma)),
                                                   c.external(Type::F32, 1, nc, const_cast<float*>(beta)), groups, eps)
                          : group_norm(c, tx, groups, eps);
        Graph g; g.build_forward(o); compute(c, g);
        std::memcpy(y, o->data, n * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// upscale (mg-tensor.cpp:179-184, mg-cpu.cpp:192-198)
int mgref_upscale(const float* x, int64_t W, int64_t H, int64_t C, int64_t N, int f, float* y) {
    try {
        const size_t n = (size_t)(W * H * C * N) * f * f;
        Context c(n * 4 + (16 << 20));
        int64_t nx[4] = {W, H, C, N};
        Tensor* o = upscale(c, c.external(Type::F32, 4, nx, const_cast<float*>(x)), f);
        Graph g; g.build_forward(o); compute(c, g);
        std::memcpy(y, o->data, n * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// The reference's VQGAN decode of one token grid: Model::load + build_vqgan_decoder
// (mg-vqgan.cpp:62-110) + the CPU executor, as tools/verify-vqgan.cpp runs it.
// grid [n_tokens] -> image {W, H, 3, 1} (out_len floats). arena_bytes: the graph arena.
int mgref_vqgan_decode(const char* gguf_path, const int32_t* grid, int64_t n_tokens, float* img,
                       int64_t out_len, int64_t arena_bytes) {
    try {
        Context wctx(64 << 20);
        auto model = Model::load(gguf_path, wctx);
        Context ctx((size_t)arena_bytes);
        Tensor* gt = ctx.tensor1d(Type::I32, n_tokens);
        std::memcpy(gt->data, grid, (size_t)n_tokens * sizeof(int32_t));
        Tensor* out = build_vqgan_decoder(ctx, *model, gt);
        if (out->nelements() != out_len) { g_err = "image size mismatch"; return -2; }
        Graph g; g.build_forward(out); compute(ctx, g);
        std::memcpy(img, out->data, (size_t)out_len * sizeof(float));
        return 0;
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

// The signature (graph_sig.h) of the reference builder's decoder graph for one grid of
// n_tokens ids; the graph is built, not run. Returns the signature length.
int64_t mgref_vqgan_graph_sig(const char* gguf_path, int64_t n_tokens, int64_t arena_bytes, char* buf,
                              int64_t cap) {
    try {
        Context wctx(64 << 20);
        auto model = Model::load(gguf_path, wctx);
        Context ctx((size_t)arena_bytes);
        Tensor* gt = ctx.tensor1d(Type::I32, n_tokens);
        Graph g; g.build_forward(build_vqgan_decoder(ctx, *model, gt));
        return graph_sig::copy_out(graph_sig::describe(g), buf, cap);
    } catch (const std::exception& e) { g_err = e.what(); return -1; }
}

}  // extern "C"
