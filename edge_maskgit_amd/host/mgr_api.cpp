// mgr_api.cpp — C entry points (include/mgr.h) over Model + build_transformer + HipRuntime.
#include "mgr.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "mg-hip.hpp"
#include "mgh.h"
#include "mg-model.hpp"
#include "mg-transformer.hpp"
#include "mg-vqgan.hpp"

namespace {
thread_local std::string g_err;

int fail(const std::exception& e) {
    g_err = e.what();
    return -1;
}
}  // namespace

struct mgr_model {
    std::unique_ptr<mg::Context> wctx;     // weight tensors (externals over the mmap)
    std::unique_ptr<mg::Model> model;
    std::unique_ptr<mg::HipRuntime> rt;
    std::unique_ptr<mg::Context> gctx;     // per-forward graph; host data only for the output
    size_t gctx_bytes = 0;
    // device buffers of mgr_generate, grown on demand: tokens, result [B][S] i32, engine
    // states, per-step work
    void* d_tok = nullptr;
    void* d_res = nullptr;
    void* d_state = nullptr;
    void* d_work = nullptr;
    size_t cap_tok = 0, cap_res = 0, cap_state = 0, cap_work = 0;
    // named nodes of the last forward's graph (their host data holds the values after a
    // forward run with MG_DUMP_NAMED set)
    std::vector<const mg::Tensor*> named;
    // the last mgr_forward graph, reused while the batch shape repeats and nothing else has
    // reset the graph context (gctx_epoch counts the resets): only the token ids change
    uint64_t gctx_epoch = 0;
    struct {
        bool valid = false, unfused = false;   // unfused: MG_NO_FLASH_ATTN at build time
        int S = 0, B = 0;
        uint64_t epoch = 0;
        mg::Tensor* tok = nullptr;
        mg::Tensor* out = nullptr;
        mg::Graph graph;
    } fwd;

    ~mgr_model() {
        if (!rt) return;
        mgh_ctx* c = rt->context();
        mgh_sync(c);
        for (void* p : {d_tok, d_res, d_state, d_work})
            if (p) mgh_free(c, p);
    }

    // reserves the graph arena for S x B tokens: graph nodes keep host storage (the
    // reference's Context semantics); the arena is not zero-filled, so only the token ids and
    // the logits pages are ever touched. Per token: each layer's 10 n_embd-wide nodes and its
    // n_ffn-wide node, 5 more n_embd-wide nodes around the layers and the logits (plus
    // alignment slack)
    void reserve_graph(int S, int B) {
        const mg::HParams& h = model->hparams();
        const size_t per_tok = (size_t)h.n_layer * (10 * (size_t)h.n_embd + (size_t)h.n_ffn) +
                               5 * (size_t)h.n_embd + (size_t)h.vocab_size;
        const size_t need = (size_t)S * B * per_tok * 4 + (size_t)(h.n_layer * 16 + 16) * 64 + (64u << 20);
        if (!gctx || gctx_bytes < need) {
            gctx.reset(new mg::Context(need));
            gctx_bytes = need;
        }
        gctx->reset();
        gctx_epoch++;
    }
};

namespace {

// host bytes the VQGAN decoder graph's nodes reserve for B images (each node keeps host
// storage, the reference's Context semantics; the arena is not zero-filled, so only the
// ids and the image pages are ever touched): the nodes of build_vqgan_decoder level by
// level — a res block at most 6 nodes of its wider width, an up-sampling 3 nodes at twice
// the side — plus alignment slack
size_t vqgan_graph_bytes(const mg::HParams& h, int B) {
    int64_t L = 1;
    while (L * L < h.n_tokens) L++;
    const std::vector<int>& mult = h.vq_channel_mult;
    if (mult.empty()) return 64u << 20;
    const int R = h.vq_num_res_blocks;
    int64_t side = L, width = (int64_t)h.vq_filters * mult.back();
    int64_t el = 2 * (int64_t)h.vq_embedding_dim * L * L + 2 * L * L * width + 6 * R * L * L * width;
    for (int i = (int)mult.size() - 1; i >= 0; i--) {
        const int64_t out = (int64_t)h.vq_filters * mult[i];
        el += 6 * R * side * side * std::max(width, out);
        if (R > 0) width = out;
        if (i > 0) {
            side *= 2;
            el += 3 * side * side * width;
        }
    }
    el += side * side * (width + 6);
    const size_t nodes = 64 + 16 * (size_t)(R + 2) * mult.size();
    return (size_t)el * B * 4 + nodes * 64 + (64u << 20);
}

void grow(mgh_ctx* c, void** p, size_t* cap, size_t need) {
    if (*cap >= need) return;
    if (*p && mgh_free(c, *p) != MGH_OK) throw std::runtime_error(mgh_last_error(c));
    *p = nullptr;
    *cap = 0;
    if (mgh_alloc(c, need, p) != MGH_OK) throw std::runtime_error(mgh_last_error(c));
    *cap = need;
}

void check(mgh_ctx* c, int rc) {
    if (rc != MGH_OK) throw std::runtime_error(std::string("mgr: ") + mgh_last_error(c));
}

}  // namespace

extern "C" {

const char* mgr_last_error(void) { return g_err.c_str(); }

int mgr_load(const char* path, int device, int algo, mgr_model** out) {
    if (!path || !out) {
        g_err = "mgr_load: null argument";
        return -1;
    }
    try {
        std::unique_ptr<mgr_model> m(new mgr_model());
        m->wctx.reset(new mg::Context(16 << 20));
        m->model = mg::Model::load(path, *m->wctx);
        m->rt.reset(new mg::HipRuntime(device));
        if (algo) m->rt->set_quant_algo(algo);
        *out = m.release();
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

void mgr_free(mgr_model* m) { delete m; }

int mgr_hparams(const mgr_model* m, int32_t o[7]) {
    if (!m || !o) return -1;
    const mg::HParams& h = m->model->hparams();
    o[0] = h.n_layer; o[1] = h.n_head; o[2] = h.n_embd; o[3] = h.head_dim;
    o[4] = h.vocab_size; o[5] = h.n_positions; o[6] = h.mask_token_id;
    return 0;
}

int mgr_decode_params(const mgr_model* m, int32_t* n_tokens, int32_t* codebook, float* choice_temperature) {
    if (!m) return -1;
    const mg::HParams& h = m->model->hparams();
    if (n_tokens) *n_tokens = h.n_tokens;
    if (codebook) *codebook = h.vq_codebook_size;
    if (choice_temperature) *choice_temperature = h.choice_temperature;
    return 0;
}

const char* mgr_device_name(const mgr_model* m) { return m ? m->rt->device_name().c_str() : ""; }

int mgr_forward(mgr_model* m, const int32_t* tokens, int S, int B, float* logits) {
    if (!m || !tokens || S <= 0 || B <= 0) {
        g_err = "mgr_forward: bad argument";
        return -1;
    }
    try {
        auto& f = m->fwd;
        const bool unfused = std::getenv("MG_NO_FLASH_ATTN") != nullptr;   // read by the builder
        if (!f.valid || f.S != S || f.B != B || f.epoch != m->gctx_epoch || f.unfused != unfused) {
            // build the reference's graph for this batch shape (the same nodes at the same
            // addresses every time, so the runtime reuses its plan as well)
            f.valid = false;
            m->reserve_graph(S, B);
            f.tok = m->gctx->tensor2d(mg::Type::I32, S, B);
            f.out = mg::build_transformer(*m->gctx, *m->model, f.tok);
            f.graph.build_forward(f.out);
            m->named.clear();
            for (const mg::Tensor* t : f.graph.nodes)
                if (!t->name.empty()) m->named.push_back(t);
            f.S = S;
            f.B = B;
            f.epoch = m->gctx_epoch;
            f.unfused = unfused;
            f.valid = true;
        }
        std::memcpy(f.tok->data, tokens, (size_t)S * B * sizeof(int32_t));
        m->rt->invalidate(f.tok);             // new token ids at a reused host address
        // the logits go straight from HBM to the caller's buffer (or stay on the device)
        const void* d = m->rt->compute_device(f.graph);
        mgh_ctx* c = m->rt->context();
        check(c, logits ? mgh_d2h(c, logits, d, f.out->nbytes()) : mgh_sync(c));
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int mgr_image_side(const mgr_model* m) {
    if (!m) return -1;
    const mg::HParams& h = m->model->hparams();
    if (h.n_tokens <= 0 || h.vq_channel_mult.empty()) return 0;
    int64_t L = 1;
    while (L * L < h.n_tokens) L++;
    return (int)(L << (h.vq_channel_mult.size() - 1));   // one 2x up-sampling per level but the last
}

namespace {

// one decoder graph for nb grids (the caller checked the arguments)
void decode_group(mgr_model* m, const int32_t* grids, int nb, float* images) {
    const mg::HParams& h = m->model->hparams();
    const size_t need = vqgan_graph_bytes(h, nb);
    if (!m->gctx || m->gctx_bytes < need) {
        m->gctx.reset(new mg::Context(need));
        m->gctx_bytes = need;
    }
    m->gctx->reset();
    m->gctx_epoch++;
    mg::Tensor* ids = m->gctx->tensor2d(mg::Type::I32, h.n_tokens, nb);
    std::memcpy(ids->data, grids, (size_t)h.n_tokens * nb * sizeof(int32_t));
    mg::Tensor* out = mg::build_vqgan_decoder(*m->gctx, *m->model, ids);
    mg::Graph g;
    g.build_forward(out);
    m->named.clear();
    for (const mg::Tensor* t : g.nodes)
        if (!t->name.empty()) m->named.push_back(t);
    m->rt->invalidate(ids);               // new ids at a reused host address
    const void* d = m->rt->compute_device(g);
    mgh_ctx* c = m->rt->context();
    check(c, images ? mgh_d2h(c, images, d, out->nbytes()) : mgh_sync(c));
}

}  // namespace

int mgr_decode_images(mgr_model* m, const int32_t* grids, int B, float* images) {
    if (!m || !grids || B <= 0) {
        g_err = "mgr_decode_images: bad argument";
        return -1;
    }
    try {
        const mg::HParams& h = m->model->hparams();
        const int side = mgr_image_side(m);
        if (h.n_tokens <= 0 || h.vq_embedding_dim <= 0 || side <= 0)
            throw std::runtime_error("mgr_decode_images: no VQGAN in the model");
        for (int64_t i = 0; i < (int64_t)h.n_tokens * B; i++)
            if (grids[i] < 0 || grids[i] >= h.vq_codebook_size)
                throw std::runtime_error("mgr_decode_images: code id outside the codebook");
        // groups of 8 images: the graph's host arena (untouched node storage, the reference's
        // Context semantics) and the device buffers stay bounded; an image's result does not
        // depend on the images decoded with it
        const size_t per = (size_t)3 * side * side;
        for (int b0 = 0; b0 < B; b0 += 8) {
            const int nb = std::min(8, B - b0);
            decode_group(m, grids + (size_t)b0 * h.n_tokens, nb, images ? images + (size_t)b0 * per : nullptr);
        }
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int mgr_named(const mgr_model* m, const char* name, float* out, int64_t capacity) {
    if (!m || !name) {
        g_err = "mgr_named: null argument";
        return -1;
    }
    for (const mg::Tensor* t : m->named) {
        if (t->name != name) continue;
        const int64_t n = t->nelements();
        if (t->type != mg::Type::F32 || !t->data) {
            g_err = std::string("mgr_named: '") + name + "' has no F32 host data";
            return -1;
        }
        if (out) {
            if (capacity < n) {
                g_err = "mgr_named: output too small";
                return -1;
            }
            std::memcpy(out, t->data, (size_t)n * sizeof(float));
        }
        return (int)n;
    }
    g_err = std::string("mgr_named: no node named '") + name + "' in the last forward";
    return -1;
}

int mgr_generate(mgr_model* m, const int32_t* class_ids, const uint64_t* seeds, int B, int steps,
                 float temperature, int32_t* out_tokens) {
    if (!m || !class_ids || !seeds || !out_tokens || B <= 0 || steps <= 0) {
        g_err = "mgr_generate: bad argument";
        return -1;
    }
    try {
        const mg::HParams& h = m->model->hparams();
        const int CB = h.vq_codebook_size, MASK = h.mask_token_id, S = h.n_tokens + 1;
        if (CB <= 0) throw std::runtime_error("mgr_generate: model has no maskgit.vqgan.codebook_size");
        if (S > h.n_positions) throw std::runtime_error("mgr_generate: n_tokens + 1 exceeds n_positions");
        for (int b = 0; b < B; b++)
            if (class_ids[b] < 0 || class_ids[b] + CB >= h.vocab_size)
                throw std::runtime_error("mgr_generate: class id out of range");
        const float temp = temperature < 0 ? h.choice_temperature : temperature;
        mgh_ctx* c = m->rt->context();
        const size_t ntok = (size_t)B * S * sizeof(int32_t);
        grow(c, &m->d_tok, &m->cap_tok, ntok);
        grow(c, &m->d_res, &m->cap_res, ntok);
        grow(c, &m->d_state, &m->cap_state, mgh_decode_state_bytes(B));
        grow(c, &m->d_work, &m->cap_work, mgh_decode_work_bytes(B, S));

        // class token at position 0, every image position masked (mg-generate.cpp:56-59)
        std::vector<int32_t> tok((size_t)B * S, MASK);
        for (int b = 0; b < B; b++) tok[(size_t)b * S] = class_ids[b] + CB;
        check(c, mgh_h2d(c, m->d_tok, tok.data(), ntok));
        check(c, mgh_decode_init(c, B, seeds, m->d_state));

        // one graph for every step; its token leaf reads the device token buffer
        m->reserve_graph(S, B);
        mg::Tensor* tl = m->gctx->tensor2d(mg::Type::I32, S, B);
        mg::Tensor* out = mg::build_transformer(*m->gctx, *m->model, tl);
        mg::Graph g;
        g.build_forward(out);
        for (int step = 0; step < steps; step++) {
            m->rt->bind_device(tl, m->d_tok);
            const float* logits = (const float*)m->rt->compute_device(g);
            check(c, mgh_decode_step(c, m->d_state, m->d_work, logits, B, S, h.vocab_size, CB, MASK,
                                     h.n_tokens, step, steps, temp, (int32_t*)m->d_tok,
                                     (int32_t*)m->d_res));
        }
        check(c, mgh_d2h(c, tok.data(), m->d_res, ntok));
        for (int b = 0; b < B; b++)
            std::memcpy(out_tokens + (size_t)b * h.n_tokens, tok.data() + (size_t)b * S + 1,
                        (size_t)h.n_tokens * sizeof(int32_t));
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int mgr_generate_images(mgr_model* m, const int32_t* class_ids, const uint64_t* seeds, int B, int steps,
                        float temperature, int32_t* out_tokens, float* images) {
    if (!m || !images || B <= 0) {
        g_err = "mgr_generate_images: bad argument";
        return -1;
    }
    try {
        const int n = m->model->hparams().n_tokens;
        const int side = mgr_image_side(m);
        if (n <= 0 || side <= 0) throw std::runtime_error("mgr_generate_images: the model has no VQGAN decoder");
        std::vector<int32_t> grids((size_t)B * n);
        if (int rc = mgr_generate(m, class_ids, seeds, B, steps, temperature, grids.data())) return rc;
        if (out_tokens) std::memcpy(out_tokens, grids.data(), grids.size() * sizeof(int32_t));
        return mgr_decode_images(m, grids.data(), B, images);
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int mgr_profile_enable(mgr_model* m, int on) {
    if (!m) return -1;
    m->rt->profile_enable(on != 0);
    m->rt->profile_reset();
    return 0;
}

int mgr_profile_report(const mgr_model* m, char* buf, size_t cap) {
    if (!m || !buf || !cap) return -1;
    std::string s;
    for (const mg::OpProfile& p : m->rt->profile_report()) {
        char line[160];
        std::snprintf(line, sizeof line, "%s %d %.4f\n", p.op.c_str(), p.count, p.ms);
        s += line;
    }
    std::snprintf(buf, cap, "%s", s.c_str());
    return 0;
}

int mgr_gguf_info(const char* path, int32_t o[7], int64_t* n_tensors) {
    if (!path || !o) {
        g_err = "mgr_gguf_info: null argument";
        return -1;
    }
    try {
        mg::Context c(16 << 20);
        auto m = mg::Model::load(path, c);
        const mg::HParams& h = m->hparams();
        o[0] = h.n_layer; o[1] = h.n_head; o[2] = h.n_embd; o[3] = h.head_dim;
        o[4] = h.vocab_size; o[5] = h.n_positions; o[6] = h.mask_token_id;
        if (n_tensors) *n_tensors = (int64_t)m->n_tensors();
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int mgr_graph_stats(const char* path, int S, int B, int32_t counts[32]) {
    if (!path || !counts || S <= 0 || B <= 0) {
        g_err = "mgr_graph_stats: bad argument";
        return -1;
    }
    try {
        mg::Context wc(16 << 20);
        auto m = mg::Model::load(path, wc);
        const mg::HParams& h = m->hparams();
        const size_t per_tok = (size_t)h.n_layer * (10 * (size_t)h.n_embd + (size_t)h.n_ffn) +
                               5 * (size_t)h.n_embd + (size_t)h.vocab_size;
        // node storage is reserved, never touched (the arena is not zero-filled)
        mg::Context big((size_t)S * B * per_tok * 4 + (64u << 20));
        mg::Tensor* tok2 = big.tensor2d(mg::Type::I32, S, B);
        std::memset(tok2->data, 0, (size_t)S * B * 4);
        mg::Tensor* out = mg::build_transformer(big, *m, tok2);
        mg::Graph g;
        g.build_forward(out);
        for (int i = 0; i < 32; i++) counts[i] = 0;
        for (const mg::Tensor* t : g.nodes) counts[(int)t->op & 31]++;
        return (int)g.nodes.size();
    } catch (const std::exception& e) {
        return fail(e);
    }
}

}  // extern "C"
