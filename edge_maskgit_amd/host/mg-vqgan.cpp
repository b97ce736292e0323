// mg-vqgan.cpp — MaskGIT VQGAN decoder graph (the reference's src/mg-vqgan.cpp:62-110).
//
// Node sequence, which fixes the numerics and so follows the reference:
//   f   = cont(permute(reshape(get_rows(codebook, ids), {E, L, L, B}), 2, 0, 1, 3))  {L, L, E, B}
//   x   = conv3x3(f) + b                                      conv_in, E -> filters * mult[last]
//   x   = R res blocks at that width                          res_blocks.0.{0..R-1}
//   for level i = last .. 0 (group j = last - i + 1), width c = filters * mult[i]:
//     x = R res blocks, the first from the previous width     res_blocks.j.{0..R-1}
//     if i > 0: x = conv3x3(upscale2(x)) + b                  res_blocks.j.{R+1}
//   img = conv3x3(gn_silu(x)) + b                             norm_out, conv_out -> 3 channels
// A res block is h = conv3x3(gn_silu(conv3x3(gn_silu(x)))) (no conv bias) and returns h + x,
// or h + conv1x1(h) when the width changes: the shortcut convolves the block's own output h,
// not its input (the quirk of the upstream Decoder the reference reproduces, mg-vqgan.cpp:51-55).
// gn_silu is GroupNorm(32 groups, eps 1e-5) with per-channel affine and SiLU as one node
// (group_norm_affine_silu); a conv bias is an Add of the bias viewed as {1, 1, C, 1}.
// Tensor names are the converter's `vqgan.*` names (tools/convert_to_gguf.py:216-226).
#include "mg-vqgan.hpp"

#include <stdexcept>
#include <string>

namespace mg {

namespace {

// the reference fixes these rather than reading maskgit.vqgan.group_norm_groups
// (mg-vqgan.cpp:14-15): PyTorch's GroupNorm defaults as the upstream decoder used them
constexpr int kGroups = 32;
constexpr float kEps = 1e-5f;

struct DecoderBuilder {
    Context& c;
    const Model& m;

    Tensor* w(const std::string& name) const { return m.require(name); }

    Tensor* channel_view(Tensor* v, int64_t C) { return reshape(c, v, {1, 1, C, 1}); }

    // each GroupNorm, conv (+ bias) and res-block output is named after its weights' prefix
    // (".out" for a block), so MG_DUMP_NAMED can read any of them back
    Tensor* gn_silu(const std::string& p, Tensor* x) {
        return group_norm_affine_silu(c, x, w(p + ".weight"), w(p + ".bias"), kGroups, kEps)->named(p);
    }

    Tensor* conv(const std::string& p, Tensor* x, int pad, bool bias) {
        Tensor* y = conv_2d(c, w(p + ".weight"), x, 1, pad);
        return (bias ? add(c, y, channel_view(w(p + ".bias"), y->ne[2])) : y)->named(p);
    }

    Tensor* res_block(const std::string& p, Tensor* x, int in_ch, int out_ch) {
        Tensor* h = conv(p + "conv0", gn_silu(p + "norm0", x), 1, false);
        h = conv(p + "conv1", gn_silu(p + "norm1", h), 1, false);
        Tensor* shortcut = in_ch == out_ch ? x : conv(p + "conv_res", h, 0, false);
        return add(c, h, shortcut)->named(p + "out");
    }
};

std::string block_prefix(int group, int layer) {
    return "vqgan.decoder.res_blocks." + std::to_string(group) + "." + std::to_string(layer);
}

}  // namespace

Tensor* build_vqgan_decoder(Context& c, const Model& m, Tensor* ids) {
    const HParams& hp = m.hparams();
    const std::vector<int>& mult = hp.vq_channel_mult;
    const int R = hp.vq_num_res_blocks;
    if (mult.empty() || hp.vq_filters <= 0 || R < 0 || hp.vq_embedding_dim <= 0)
        throw std::runtime_error("vqgan: model has no decoder hyper-parameters");
    if (ids->type != Type::I32 || ids->ne[2] != 1 || ids->ne[3] != 1)
        throw std::runtime_error("vqgan: ids must be I32 with ne = {n_tokens} or {n_tokens, B}");
    const int64_t n = ids->ne[0], B = ids->ne[1];
    int64_t L = 1;
    while (L * L < n) L++;                          // latent side (16 for 256 tokens)
    if (L * L != n) throw std::runtime_error("vqgan: the token count must be a square");
    DecoderBuilder d{c, m};

    Tensor* f = get_rows(c, d.w("vqgan.quantizer.codebook.weight"), ids);          // {E, n, B}
    f = reshape(c, f, {(int64_t)hp.vq_embedding_dim, L, L, B});
    Tensor* x = d.conv("vqgan.decoder.conv_in", cont(c, permute(c, f, 2, 0, 1, 3))->named("vqgan.decoder.conv_in.in"), 1, true);

    const int last = (int)mult.size() - 1;
    int width = hp.vq_filters * mult[last];
    for (int l = 0; l < R; l++) x = d.res_block(block_prefix(0, l) + ".", x, width, width);
    for (int i = last; i >= 0; i--) {
        const int group = last - i + 1, out = hp.vq_filters * mult[i];
        for (int l = 0; l < R; l++) {
            x = d.res_block(block_prefix(group, l) + ".", x, width, out);
            width = out;
        }
        if (i > 0) x = d.conv(block_prefix(group, R + 1), upscale(c, x, 2)->named(block_prefix(group, R + 1) + ".in"), 1, true);
    }
    return d.conv("vqgan.decoder.conv_out", d.gn_silu("vqgan.decoder.norm_out", x), 1, true);
}

}  // namespace mg
