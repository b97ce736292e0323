// mg-tensor.hpp — the graph/tensor interface this backend executes.
//
// It mirrors the reference's graph API (include/mg-tensor.hpp of chenxugz/edge_maskgit,
// lines 22-168): the same type and op enumerations (same values), the same Tensor fields and
// node-builder functions, so a graph built against either header means the same thing and
// HipRuntime (mg-hip.hpp) can stand in for the reference's OpenCLRuntime. The implementation
// (edge_maskgit_amd/host/mg-tensor.cpp) is this project's own.
//
// Conventions (the reference's, mg-tensor.hpp:3-13):
//  * ne[0] is the innermost, contiguous dimension; a numpy shape [d0, .., dn] is ne reversed.
//  * nb[] are strides in bytes (views may carry any strides).
//  * mul_mat(w, x): w has ne = {K, N} (a Linear weight [N][K]), x has ne = {K, M, ...};
//    the result has ne = {N, M, ...} and result[n, m] = sum_k w[k, n] * x[k, m].
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace mg {

inline constexpr int MAX_DIMS = 4;
inline constexpr int MAX_SRC = 4;         // src0, src1, fused bias (2), fused residual (3)
inline constexpr int MAX_OP_PARAMS = 4;

// element types (values as in the reference; GGUF codes are mapped by the loader)
enum class Type { F32 = 0, F16 = 1, I32 = 2, I8 = 3, I4 = 4, Q8_0 = 5, Q4_K = 6 };

inline constexpr int Q8_0_BLOCK = 32;     // values per Q8_0 block
inline constexpr int Q8_0_BYTES = 34;     // fp16 scale + 32 int8
inline constexpr int Q4_K_BLOCK = 256;    // values per Q4_K super-block
inline constexpr int Q4_K_BYTES = 144;    // fp16 d, dmin + 12 B scales/mins + 128 B nibbles

enum class Op {
    None = 0,
    Add,             // src1 broadcast over its size-1 dims (same shape, bias row, ...)
    Mul,
    Scale,           // fparam[0]
    MulMat,          // src[2] bias {N}, src[3] residual (shape of the output), iparam[0] act
    GetRows,         // gather src0 rows by the I32 indices in src1
    SoftMax,         // over ne[0], fparam[0] scale
    Norm,            // LayerNorm over ne[0], fparam[0] eps; src[1]/src[2] gamma/beta = affine
    GroupNorm,
    Gelu,
    Silu,
    Conv2D,
    Upscale,
    FlashAttention,  // src0 Q, src1 K, src2 V, all {D, S, H, B}; fparam[0] scale
    Reshape,         // views
    View,
    Permute,
    Cont,            // contiguous copy of a view
};

size_t type_size(Type t);

struct Tensor {
    Type type = Type::F32;
    int n_dims = 1;
    int64_t ne[MAX_DIMS] = {1, 1, 1, 1};
    size_t nb[MAX_DIMS] = {0, 0, 0, 0};

    Op op = Op::None;
    Tensor* src[MAX_SRC] = {nullptr, nullptr, nullptr, nullptr};
    int32_t iparam[MAX_OP_PARAMS] = {0, 0, 0, 0};
    float fparam[MAX_OP_PARAMS] = {0, 0, 0, 0};

    void* data = nullptr;      // host storage: the context arena, or external (mmap'd weights)
    bool is_view = false;
    std::string name;

    int64_t nelements() const;
    size_t nbytes() const;
    bool is_contiguous() const;

    float f32(int64_t i) const { return static_cast<const float*>(data)[i]; }
    void set_f32(int64_t i, float v) { static_cast<float*>(data)[i] = v; }
    Tensor* named(const std::string& n) {
        name = n;
        return this;
    }
};

// Owns the Tensor objects (stable addresses) and a bump arena for their host data.
class Context {
public:
    explicit Context(size_t arena_bytes);

    Tensor* tensor(Type t, int n_dims, const int64_t ne[MAX_DIMS]);
    Tensor* tensor1d(Type t, int64_t ne0);
    Tensor* tensor2d(Type t, int64_t ne0, int64_t ne1);
    Tensor* tensor3d(Type t, int64_t ne0, int64_t ne1, int64_t ne2);
    Tensor* tensor4d(Type t, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);
    Tensor* external(Type t, int n_dims, const int64_t ne[MAX_DIMS], void* data);  // no copy

    size_t used() const { return used_; }
    void reset();                        // drop every tensor and rewind the arena
    void* alloc(size_t bytes);           // 32-byte aligned bump allocation

    Tensor* make(Type t, int n_dims, const int64_t ne[MAX_DIMS], Op op, Tensor* s0, Tensor* s1,
                 bool alloc_data);

private:
    std::vector<std::unique_ptr<Tensor>> tensors_;
    std::unique_ptr<uint8_t[]> arena_;   // not zero-filled: untouched pages stay unmapped
    size_t capacity_ = 0;
    size_t used_ = 0;
};

// ---- node builders (evaluation happens in a runtime's compute) ----
Tensor* add(Context&, Tensor* a, Tensor* b);
Tensor* mul(Context&, Tensor* a, Tensor* b);
Tensor* add_bias(Context&, Tensor* a, Tensor* bias);
Tensor* scale(Context&, Tensor* a, float s);
Tensor* mul_mat(Context&, Tensor* w, Tensor* x);
// out = act(w . x + bias) + residual; bias (ne = {N}), act (0 none, 1 GELU, 2 SiLU) and
// residual (shape of out) are each optional
Tensor* mul_mat_ex(Context&, Tensor* w, Tensor* x, Tensor* bias, int act, Tensor* residual);
Tensor* get_rows(Context&, Tensor* a, Tensor* ids);
Tensor* soft_max(Context&, Tensor* a, float scale = 1.0f);
Tensor* norm(Context&, Tensor* a, float eps);
Tensor* norm_affine(Context&, Tensor* a, Tensor* gamma, Tensor* beta, float eps);
Tensor* group_norm(Context&, Tensor* a, int groups, float eps);
Tensor* group_norm_affine_silu(Context&, Tensor* a, Tensor* gamma, Tensor* beta, int groups,
                               float eps);
Tensor* gelu(Context&, Tensor* a);
Tensor* silu(Context&, Tensor* a);
Tensor* conv_2d(Context&, Tensor* kernel, Tensor* input, int stride, int pad);
Tensor* upscale(Context&, Tensor* a, int factor);
Tensor* flash_attention(Context&, Tensor* q, Tensor* k, Tensor* v, float scale);

// zero-copy views
Tensor* reshape(Context&, Tensor* a, std::vector<int64_t> ne);
Tensor* permute(Context&, Tensor* a, int a0, int a1, int a2, int a3);
Tensor* cont(Context&, Tensor* a);

struct Graph {
    std::vector<Tensor*> nodes;          // computed nodes in dependency order
    void build_forward(Tensor* out);
};

}  // namespace mg
