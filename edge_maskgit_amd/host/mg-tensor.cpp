// mg-tensor.cpp — tensors, the host arena, node builders and graph ordering for the graph
// interface of include/mg-tensor.hpp (the reference's graph API, src/mg-tensor.cpp).
#include "mg-tensor.hpp"

#include <unordered_set>

#include <cstdio>
#include <stdexcept>
#include <string>

namespace mg {

namespace {

constexpr size_t kAlign = 32;

void contiguous_strides(Tensor* t) {
    size_t s = type_size(t->type);
    for (int i = 0; i < MAX_DIMS; i++) {
        t->nb[i] = s;
        s *= (size_t)t->ne[i];
    }
}

int dims_of(const int64_t ne[MAX_DIMS]) {
    int n = MAX_DIMS;
    while (n > 1 && ne[n - 1] == 1) n--;
    return n;
}

void require(bool ok, const char* what) {
    if (!ok) throw std::runtime_error(std::string("mg: ") + what);
}

}  // namespace

size_t type_size(Type t) {
    switch (t) {
        case Type::F32: return 4;
        case Type::F16: return 2;
        case Type::I32: return 4;
        case Type::I8: return 1;
        case Type::I4: return 1;
        default: return 0;      // block formats: size only through nbytes()
    }
}

int64_t Tensor::nelements() const { return ne[0] * ne[1] * ne[2] * ne[3]; }

size_t Tensor::nbytes() const {
    const int64_t n = nelements();
    switch (type) {
        case Type::Q8_0: return (size_t)(n / Q8_0_BLOCK) * Q8_0_BYTES;
        case Type::Q4_K: return (size_t)(n / Q4_K_BLOCK) * Q4_K_BYTES;
        case Type::I4: return (size_t)(n + 1) / 2;
        default: return (size_t)n * type_size(type);
    }
}

// Contiguous means every stride equals the packed stride, size-1 dimensions included
// (reference src/mg-tensor.cpp:36-43).
bool Tensor::is_contiguous() const {
    size_t s = type_size(type);
    for (int i = 0; i < MAX_DIMS; i++) {
        if (ne[i] == 0) return true;
        if (nb[i] != s) return false;
        s *= (size_t)ne[i];
    }
    return true;
}

Context::Context(size_t arena_bytes) : arena_(new uint8_t[arena_bytes]), capacity_(arena_bytes) {}

void Context::reset() {
    tensors_.clear();
    used_ = 0;
}

void* Context::alloc(size_t bytes) {
    const size_t at = (used_ + kAlign - 1) & ~(kAlign - 1);
    if (at + bytes > capacity_) {
        std::fprintf(stderr, "[mg::Context] arena full: %zu bytes requested, %zu of %zu used\n", bytes,
                     used_, capacity_);
        throw std::runtime_error("mg::Context arena out of memory");
    }
    used_ = at + bytes;
    return arena_.get() + at;
}

Tensor* Context::make(Type t, int n_dims, const int64_t ne[MAX_DIMS], Op op, Tensor* s0, Tensor* s1,
                      bool alloc_data) {
    tensors_.emplace_back(new Tensor());
    Tensor* x = tensors_.back().get();
    x->type = t;
    x->n_dims = n_dims;
    for (int i = 0; i < MAX_DIMS; i++) x->ne[i] = i < n_dims ? ne[i] : 1;
    contiguous_strides(x);
    x->op = op;
    x->src[0] = s0;
    x->src[1] = s1;
    if (alloc_data) x->data = alloc(x->nbytes());
    return x;
}

Tensor* Context::tensor(Type t, int n_dims, const int64_t ne[MAX_DIMS]) {
    return make(t, n_dims, ne, Op::None, nullptr, nullptr, true);
}
Tensor* Context::tensor1d(Type t, int64_t a) {
    const int64_t ne[MAX_DIMS] = {a, 1, 1, 1};
    return tensor(t, 1, ne);
}
Tensor* Context::tensor2d(Type t, int64_t a, int64_t b) {
    const int64_t ne[MAX_DIMS] = {a, b, 1, 1};
    return tensor(t, 2, ne);
}
Tensor* Context::tensor3d(Type t, int64_t a, int64_t b, int64_t c) {
    const int64_t ne[MAX_DIMS] = {a, b, c, 1};
    return tensor(t, 3, ne);
}
Tensor* Context::tensor4d(Type t, int64_t a, int64_t b, int64_t c, int64_t d) {
    const int64_t ne[MAX_DIMS] = {a, b, c, d};
    return tensor(t, 4, ne);
}
Tensor* Context::external(Type t, int n_dims, const int64_t ne[MAX_DIMS], void* data) {
    Tensor* x = make(t, n_dims, ne, Op::None, nullptr, nullptr, false);
    x->data = data;
    x->is_view = true;
    return x;
}

// ---- node builders ----
namespace {
Tensor* same_shape(Context& c, Op op, Tensor* a, Tensor* b) {
    return c.make(a->type, a->n_dims, a->ne, op, a, b, true);
}
}  // namespace

Tensor* add(Context& c, Tensor* a, Tensor* b) { return same_shape(c, Op::Add, a, b); }
Tensor* mul(Context& c, Tensor* a, Tensor* b) { return same_shape(c, Op::Mul, a, b); }
Tensor* add_bias(Context& c, Tensor* a, Tensor* bias) { return same_shape(c, Op::Add, a, bias); }
Tensor* scale(Context& c, Tensor* a, float s) {
    Tensor* t = same_shape(c, Op::Scale, a, nullptr);
    t->fparam[0] = s;
    return t;
}

Tensor* mul_mat(Context& c, Tensor* w, Tensor* x) {
    require(w->ne[0] == x->ne[0], "mul_mat: inner dimensions differ");
    const int64_t ne[MAX_DIMS] = {w->ne[1], x->ne[1], x->ne[2], x->ne[3]};
    return c.make(Type::F32, dims_of(ne) < 2 ? 2 : dims_of(ne), ne, Op::MulMat, w, x, true);
}

Tensor* mul_mat_ex(Context& c, Tensor* w, Tensor* x, Tensor* bias, int act, Tensor* residual) {
    Tensor* y = mul_mat(c, w, x);
    y->src[2] = bias;
    y->src[3] = residual;
    y->iparam[0] = act;
    return y;
}

Tensor* get_rows(Context& c, Tensor* a, Tensor* ids) {
    const int64_t ne[MAX_DIMS] = {a->ne[0], ids->ne[0], ids->ne[1], 1};
    return c.make(a->type, ne[2] > 1 ? 3 : 2, ne, Op::GetRows, a, ids, true);
}

Tensor* soft_max(Context& c, Tensor* a, float s) {
    Tensor* t = same_shape(c, Op::SoftMax, a, nullptr);
    t->fparam[0] = s;
    return t;
}

Tensor* norm(Context& c, Tensor* a, float eps) {
    Tensor* t = same_shape(c, Op::Norm, a, nullptr);
    t->fparam[0] = eps;
    return t;
}

Tensor* norm_affine(Context& c, Tensor* a, Tensor* gamma, Tensor* beta, float eps) {
    Tensor* t = norm(c, a, eps);
    t->src[1] = gamma;
    t->src[2] = beta;
    return t;
}

Tensor* group_norm(Context& c, Tensor* a, int groups, float eps) {
    Tensor* t = same_shape(c, Op::GroupNorm, a, nullptr);
    t->iparam[0] = groups;
    t->fparam[1] = eps;
    return t;
}

Tensor* group_norm_affine_silu(Context& c, Tensor* a, Tensor* gamma, Tensor* beta, int groups,
                               float eps) {
    Tensor* t = group_norm(c, a, groups, eps);
    t->src[1] = gamma;
    t->src[2] = beta;
    t->iparam[1] = 1;
    return t;
}

Tensor* gelu(Context& c, Tensor* a) { return same_shape(c, Op::Gelu, a, nullptr); }
Tensor* silu(Context& c, Tensor* a) { return same_shape(c, Op::Silu, a, nullptr); }

Tensor* conv_2d(Context& c, Tensor* kernel, Tensor* input, int stride, int pad) {
    const int64_t ow = (input->ne[0] + 2 * pad - kernel->ne[0]) / stride + 1;
    const int64_t oh = (input->ne[1] + 2 * pad - kernel->ne[1]) / stride + 1;
    const int64_t ne[MAX_DIMS] = {ow, oh, kernel->ne[3], input->ne[3]};
    Tensor* t = c.make(Type::F32, 4, ne, Op::Conv2D, kernel, input, true);
    t->iparam[0] = stride;
    t->iparam[1] = pad;
    return t;
}

Tensor* upscale(Context& c, Tensor* a, int factor) {
    const int64_t ne[MAX_DIMS] = {a->ne[0] * factor, a->ne[1] * factor, a->ne[2], a->ne[3]};
    Tensor* t = c.make(a->type, 4, ne, Op::Upscale, a, nullptr, true);
    t->iparam[0] = factor;
    return t;
}

Tensor* flash_attention(Context& c, Tensor* q, Tensor* k, Tensor* v, float scale) {
    for (int i = 0; i < 3; i++)
        require(q->ne[i] == k->ne[i] && q->ne[i] == v->ne[i], "flash_attention: q/k/v shapes differ");
    Tensor* t = c.make(Type::F32, q->n_dims, q->ne, Op::FlashAttention, q, k, true);
    t->src[2] = v;
    t->fparam[0] = scale;
    return t;
}

// ---- views: share the source's storage ----
namespace {
Tensor* view_of(Context& c, Tensor* a, Op op) {
    Tensor* t = c.make(a->type, a->n_dims, a->ne, op, a, nullptr, false);
    for (int i = 0; i < MAX_DIMS; i++) t->nb[i] = a->nb[i];
    t->data = a->data;
    t->is_view = true;
    return t;
}
}  // namespace

Tensor* reshape(Context& c, Tensor* a, std::vector<int64_t> ne) {
    require(a->is_contiguous(), "reshape: source is not contiguous");
    require(!ne.empty() && ne.size() <= (size_t)MAX_DIMS, "reshape: bad rank");
    Tensor* t = view_of(c, a, Op::Reshape);
    t->n_dims = (int)ne.size();
    for (int i = 0; i < MAX_DIMS; i++) t->ne[i] = i < t->n_dims ? ne[i] : 1;
    contiguous_strides(t);
    require(t->nelements() == a->nelements(), "reshape: element count changes");
    return t;
}

Tensor* permute(Context& c, Tensor* a, int a0, int a1, int a2, int a3) {
    const int to[MAX_DIMS] = {a0, a1, a2, a3};
    Tensor* t = view_of(c, a, Op::Permute);
    for (int i = 0; i < MAX_DIMS; i++) {       // source dim i becomes output dim to[i]
        t->ne[to[i]] = a->ne[i];
        t->nb[to[i]] = a->nb[i];
    }
    return t;
}

Tensor* cont(Context& c, Tensor* a) { return c.make(a->type, a->n_dims, a->ne, Op::Cont, a, nullptr, true); }

// ---- graph: post-order walk from the output (leaves are not nodes) ----
namespace {
void visit(std::vector<Tensor*>& order, std::unordered_set<const Tensor*>& seen, Tensor* t) {
    if (!t || t->op == Op::None || !seen.insert(t).second) return;
    for (Tensor* s : t->src) visit(order, seen, s);
    order.push_back(t);
}
}  // namespace

// A graph holds the nodes of one output: building it again starts from an empty list
// (reference src/mg-tensor.cpp:241).
void Graph::build_forward(Tensor* out) {
    nodes.clear();
    std::unordered_set<const Tensor*> seen;      // a set: the transformer graph has ~450 nodes
    seen.reserve(1024);
    visit(nodes, seen, out);
}

}  // namespace mg
