// mg-transformer.hpp — the MaskGIT bidirectional-transformer forward graph.
//
// Interface of the reference's builder (include/mg-transformer.hpp:7-13): token ids
// (I32, ne = {S, B}) -> logits (F32, ne = {vocab_size, S, B}); post-norm layers, flash
// attention, MLM head tied to the token embedding plus output.bias. The implementation
// (edge_maskgit_amd/host/mg-transformer.cpp) is this project's own.
#pragma once
#include "mg-model.hpp"
#include "mg-tensor.hpp"

namespace mg {

Tensor* build_transformer(Context& ctx, const Model& m, Tensor* token_ids);

}  // namespace mg
