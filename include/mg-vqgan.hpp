// mg-vqgan.hpp — the MaskGIT VQGAN decoder forward graph.
//
// Interface of the reference's builder (include/mg-vqgan.hpp:7-13): codebook ids of a token
// grid (I32, ne = {n_tokens}, row-major: index h*L + w of an L x L grid) -> image (F32,
// ne = {W, H, 3, 1}, W innermost), with the reference's node sequence (src/mg-vqgan.cpp:62-110),
// so every runtime that evaluates the reference's graph evaluates this one to the same values.
// Ids with ne = {n_tokens, B} give B images, ne = {W, H, 3, B}: each node then carries the
// whole batch (image b is the same as decoding its grid alone). The implementation
// (edge_maskgit_amd/host/mg-vqgan.cpp) is this project's own.
#pragma once
#include "mg-model.hpp"
#include "mg-tensor.hpp"

namespace mg {

Tensor* build_vqgan_decoder(Context& ctx, const Model& m, Tensor* grid_ids);

}  // namespace mg
