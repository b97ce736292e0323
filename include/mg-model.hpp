// mg-model.hpp — GGUF v3 weight file loader (mmap, zero-copy weight tensors).
//
// Interface of the reference's loader (include/mg-model.hpp:16-66, src/mg-model.cpp:139-201):
// Model::load(path, ctx) maps the file and registers every tensor as an external Tensor in
// ctx; hyper-parameters come from the `maskgit.*` metadata keys. The implementation
// (edge_maskgit_amd/host/mg-model.cpp) is this project's own.
#pragma once

#include "mg-tensor.hpp"

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace mg {

struct HParams {
    int n_layer = 0, n_head = 0, n_embd = 0, n_ffn = 0, head_dim = 0;
    int vocab_size = 0, n_tokens = 0, n_positions = 0;
    int mask_token_id = -1;
    float ln_eps = 1e-12f;
    int vq_codebook_size = 0, vq_embedding_dim = 0, vq_filters = 0;
    int vq_num_res_blocks = 0, vq_gn_groups = 32;
    std::vector<int> vq_channel_mult;
    float choice_temperature = 4.5f;
    int resolution = 256;
    std::string arch, name;
    std::string quant = "f32";
};

class Model {
public:
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    static std::unique_ptr<Model> load(const std::string& path, Context& ctx);

    const HParams& hparams() const { return hp_; }
    bool has(const std::string& name) const { return tensors_.count(name) != 0; }
    Tensor* get(const std::string& name) const;       // nullptr when absent
    Tensor* require(const std::string& name) const;   // throws when absent
    size_t n_tensors() const { return tensors_.size(); }
    const std::unordered_map<std::string, Tensor*>& tensors() const { return tensors_; }
    void* mmap_base() const { return base_; }
    size_t mmap_size() const { return size_; }

private:
    Model() = default;
    HParams hp_;
    std::unordered_map<std::string, Tensor*> tensors_;
    void* base_ = nullptr;
    size_t size_ = 0;
    int fd_ = -1;
    friend struct GgufReader;
};

}  // namespace mg
