// mg-transformer.cpp — MaskGIT forward graph (the reference's src/mg-transformer.cpp:32-111).
//
// Node sequence, which fixes the numerics and so must match the reference:
//   x = LN_emb(get_rows(token_embd, ids) + pos_embd[:S])
//   per layer l (post-norm):
//     q, k, v = x W + b                     (three FC nodes, fused bias)
//     a = flash_attention(q, k, v) on the {D,S,H,B} head views, merged back to [S*B][H*D]
//         (with MG_NO_FLASH_ATTN set in the environment: the unfused chain
//          softmax(scale * k . q) then v^T . scores, mg-transformer.cpp:55, 75-81)
//     x = LN_attn(a W_o + b_o + x)          (residual fused into the FC epilogue)
//     x = LN_ffn(GELU(x W_up + b_up) W_down + b_down + x)
//   logits = LN_out(GELU(x W_proj + b_proj)) E^T + output.bias   (E = token_embd, F32)
// Tensor names are the GGUF names the reference's converter writes.
#include "mg-transformer.hpp"

#include <cmath>
#include <cstdlib>
#include <stdexcept>
#include <string>

namespace mg {

namespace {

Tensor* fc(Context& c, const Model& m, const std::string& w, const std::string& b, Tensor* x,
           int act = 0, Tensor* resid = nullptr) {
    return mul_mat_ex(c, m.require(w), x, m.require(b), act, resid);
}

Tensor* ln(Context& c, const Model& m, const std::string& p, Tensor* x, float eps) {
    return norm_affine(c, x, m.require(p + ".weight"), m.require(p + ".bias"), eps);
}

// [H*D, S, B] FC output -> {D, S, H, B} head view
Tensor* heads(Context& c, Tensor* t, int64_t D, int64_t H, int64_t S, int64_t B) {
    return permute(c, reshape(c, t, {D, H, S, B}), 0, 2, 1, 3);
}

}  // namespace

Tensor* build_transformer(Context& c, const Model& m, Tensor* ids) {
    const HParams& hp = m.hparams();
    const int64_t S = ids->ne[0], B = ids->ne[1];
    const int64_t E = hp.n_embd, H = hp.n_head, D = hp.head_dim;
    const float eps = hp.ln_eps;
    // the position table is viewed as its first S rows; more positions than it holds would
    // read past the tensor (the reference does not check)
    const Tensor* pe = m.require("pos_embd.weight");
    if (pe->ne[0] != E || S > pe->ne[1])
        throw std::runtime_error("build_transformer: sequence longer than the position table");

    Tensor* tok = get_rows(c, m.require("token_embd.weight"), ids);          // {E, S, B}
    const int64_t pne[MAX_DIMS] = {E, S, 1, 1};
    Tensor* pos = c.external(Type::F32, 2, pne, pe->data);                   // first S rows
    Tensor* x = ln(c, m, "token_embd_norm", add(c, tok, pos), eps);
    x->named("embd_post_norm");
    const bool unfused = std::getenv("MG_NO_FLASH_ATTN") != nullptr;
    const float scale = 1.0f / std::sqrt((float)D);

    for (int l = 0; l < hp.n_layer; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Tensor* q = heads(c, fc(c, m, p + "attn_q.weight", p + "attn_q.bias", x), D, H, S, B);
        Tensor* k = heads(c, fc(c, m, p + "attn_k.weight", p + "attn_k.bias", x), D, H, S, B);
        Tensor* v = heads(c, fc(c, m, p + "attn_v.weight", p + "attn_v.bias", x), D, H, S, B);
        Tensor* a;
        if (!unfused) {
            a = flash_attention(c, q, k, v, scale);                              // {D, S, H, B}
        } else {
            Tensor* sc = soft_max(c, mul_mat(c, k, q), scale);                  // {S keys, S, H, B}
            a = mul_mat(c, permute(c, v, 1, 0, 2, 3), sc);                      // {D, S, H, B}
        }
        a = reshape(c, cont(c, permute(c, a, 0, 2, 1, 3)), {E, S, B});          // heads merged
        x = fc(c, m, p + "attn_o.weight", p + "attn_o.bias", a, 0, x);
        x = ln(c, m, p + "attn_norm", x, eps);
        x->named(p + "attn_post");
        Tensor* f = fc(c, m, p + "ffn_up.weight", p + "ffn_up.bias", x, 1);
        x = fc(c, m, p + "ffn_down.weight", p + "ffn_down.bias", f, 0, x);
        x = ln(c, m, p + "ffn_norm", x, eps);
        x->named(p + "ffn_post");
    }

    Tensor* h = fc(c, m, "output_proj.weight", "output_proj.bias", x, 1);
    h = ln(c, m, "output_norm", h, eps);
    h->named("output_norm");
    Tensor* logits = mul_mat_ex(c, m.require("token_embd.weight"), h, m.require("output.bias"), 0, nullptr);
    logits->named("output_logits");
    return logits;
}

}  // namespace mg
