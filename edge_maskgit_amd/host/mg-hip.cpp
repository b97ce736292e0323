// mg-hip.cpp — HipRuntime: the graph walker of the MI355X backend (the role of the
// reference's OpenCLRuntime::compute, src/mg-opencl/mg-opencl.cpp:1354-1656), built on the
// libmgh C ABI (include/mgh.h).
//
// Per compute():
//  1. Plan: every node's storage root (views alias their source), each root's last consumer,
//     the LayerNorm nodes whose output feeds quantized FC layers (fused operand: int8 codes for
//     the int8-dot path, fp16 values for the dequantize-fused path), on the dequantize-fused
//     path the FC groups that share their input (q/k/v: one GEMM) and the attention / FC
//     outputs read only by FCs (stored as fp16), and the
//     flash-attention -> permute -> cont chains (attention writes the merged layout).
//  2. Run the nodes in order; device buffers of computed roots come from a size-bucketed
//     pool and return to it after their last consumer.
//  3. Copy the final node to its host data and wait (the reference's readback, :1622-1642);
//     with MG_DUMP_NAMED set in the environment, every named computed node is also copied to
//     its host data (:1627-1641) — right after it runs, before its buffer can be reused;
//     compute_device() instead keeps the result in HBM for device-side consumers (the
//     decode step) and returns without waiting.
// Leaves are uploaded once per (host address, byte size) and kept; quantized weights are
// packed on upload (mgh_pack_weights for the int8-dot path, mgh_pack_weights_f16 for the
// dequantize-fused path). Supported ops: MulMat (Q8_0, Q4_K; F32 weights, batched and
// strided), Norm (plain or affine), SoftMax, FlashAttention, GetRows, Add, Mul, Scale, Gelu,
// Silu, Cont, Reshape, View, Permute — the ops of the reference's GPU runtime outside the
// VQGAN decoder (mg-opencl.cpp:1367-1534). Any other op throws (:1600-1601).
#include "mg-hip.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <stdexcept>
#include <tuple>
#include <unordered_map>
#include <unordered_set>

#include "mgh.h"

namespace mg {

namespace {

bool is_view_op(Op op) { return op == Op::Reshape || op == Op::View || op == Op::Permute; }

const char* op_name(const Tensor* t) {
    switch (t->op) {
        case Op::MulMat:
            return (t->src[0]->type == Type::Q8_0 || t->src[0]->type == Type::Q4_K) ? "MulMat(q)" : "MulMat(f32)";
        case Op::Norm: return "Norm";
        case Op::SoftMax: return "SoftMax";
        case Op::FlashAttention: return "FlashAttention";
        case Op::GetRows: return "GetRows";
        case Op::Add: return "Add";
        case Op::Mul: return "Mul";
        case Op::Scale: return "Scale";
        case Op::Gelu: return "Gelu";
        case Op::Silu: return "Silu";
        case Op::Cont: return "Cont";
        case Op::GroupNorm: return "GroupNorm";
        case Op::Conv2D: return "Conv2D";
        case Op::Upscale: return "Upscale";
        default: return "Other";
    }
}

}  // namespace

struct HipRuntime::Impl {
    mgh_ctx* ctx = nullptr;
    std::string name;
    // the reference's choice on a device without cl_arm_integer_dot_product (any non-Mali
    // GPU): the dequant-fused path (mg-opencl.cpp:1237-1238, 1400-1423)
    int algo = MGH_ALGO_DEQ_F16;
    bool profiling = false;
    std::map<std::string, std::pair<int, double>> prof;

    // leaf uploads: (host address, bytes, layout) -> device pointer
    std::map<std::tuple<const void*, size_t, int>, void*> leaves;
    // free device buffers by size
    std::multimap<size_t, void*> pool;
    // unit gamma / zero beta per D for plain Norm nodes
    std::map<int64_t, std::pair<void*, void*>> unit_affine;

    // leaves bound to caller-owned device memory for the next compute
    std::unordered_map<const Tensor*, void*> bound;
    // final result of the last compute_device, returned to the pool by the next compute
    void* held = nullptr;

    // row-concatenated weights / biases of fused FC groups, keyed by the members' host data
    std::map<std::vector<const void*>, void*> fused_w, fused_b;

    // per-compute state
    std::unordered_map<const Tensor*, void*> addr;            // device address of a tensor
    std::unordered_map<const Tensor*, int64_t> pitch;         // row pitch of a fused FC output
    std::unordered_map<const Tensor*, const Tensor*> owner;   // fused FC output -> group leader
    struct Codes { void* q = nullptr; void* dx = nullptr; void* sx = nullptr; size_t bytes = 0; };
    std::unordered_map<const Tensor*, Codes> codes;           // fused FC operand of a Norm node

    // Epilogue Adds a VQGAN conv evaluates (bias, then residual) and the last node it writes
    struct ConvFuse {
        const Tensor* bias = nullptr;
        const Tensor* resid = nullptr;
        const Tensor* out = nullptr;
    };
    // What run() decides from the graph's structure alone (consumers, fusions). A graph whose
    // fingerprint (algorithm, and per node its address, op, type, shape, strides, parameters,
    // sources, and the sources' shape and host data when they are leaves) equals the last
    // planned one reuses that plan: rebuilding the same graph into a reset context, as every
    // forward of one batch shape does, gives the same nodes at the same addresses.
    struct Plan {
        bool valid = false;
        std::vector<uint64_t> key;
        std::unordered_map<const Tensor*, int> last;              // root -> last consumer index
        std::unordered_map<const Tensor*, int> fc_uses, other_uses;  // Norm root -> consumer kinds
        std::unordered_map<const Tensor*, const Tensor*> fa_into;    // cont -> its FA source
        std::unordered_map<const Tensor*, const Tensor*> fa_target;  // FA -> cont it writes
        std::vector<std::vector<Tensor*>> groups;
        std::unordered_map<const Tensor*, int> grp_of;
        std::unordered_set<int> grp16;                               // groups stored as fp16
        std::unordered_set<const Tensor*> emit16;
        std::unordered_map<const Tensor*, const Tensor*> ln_pair;    // FC -> its Norm
        std::unordered_map<const Tensor*, ConvFuse> cfuse;           // conv -> its fused Adds
        std::unordered_map<const Tensor*, const Tensor*> absorbed;   // absorbed Add -> its conv
        std::unordered_map<const Tensor*, const Tensor*> owner;      // owner map after planning
    } plan;
    std::vector<uint64_t> key_tmp;

    // true when g matches the last planned graph; otherwise the plan is invalidated and will
    // be rebuilt under g's fingerprint
    bool plan_matches(const Graph& g) {
        std::vector<uint64_t>& k = key_tmp;
        k.clear();
        k.push_back((uint64_t)algo);
        k.push_back(g.nodes.size());
        auto shape = [&](const Tensor* t) {
            k.push_back(((uint64_t)t->op << 32) | (uint64_t)t->type);
            for (int d = 0; d < MAX_DIMS; d++) {
                k.push_back((uint64_t)t->ne[d]);
                k.push_back((uint64_t)t->nb[d]);
            }
        };
        for (const Tensor* t : g.nodes) {
            k.push_back((uint64_t)(uintptr_t)t);
            shape(t);
            for (int j = 0; j < MAX_OP_PARAMS; j++)
                k.push_back(((uint64_t)(uint32_t)t->iparam[j] << 32) | __builtin_bit_cast(uint32_t, t->fparam[j]));
            for (const Tensor* s : t->src) {
                k.push_back((uint64_t)(uintptr_t)s);
                if (s && s->op == Op::None) {
                    shape(s);
                    k.push_back((uint64_t)(uintptr_t)s->data);
                }
            }
        }
        if (plan.valid && k == plan.key) return true;
        plan.valid = false;
        plan.key.swap(k);
        return false;
    }

    void check(int rc) {
        if (rc != MGH_OK) throw std::runtime_error(std::string("HipRuntime: ") + mgh_last_error(ctx));
    }

    void* take(size_t bytes) {
        bytes = (bytes + 255) & ~(size_t)255;
        auto it = pool.lower_bound(bytes);
        if (it != pool.end() && it->first <= bytes + bytes / 4) {  // reuse a buffer up to 25% larger
            void* p = it->second;
            pool.erase(it);
            return p;
        }
        void* p = nullptr;
        check(mgh_alloc(ctx, bytes, &p));
        alloc_size[p] = bytes;
        return p;
    }
    void give(void* p) {
        if (p) pool.emplace(alloc_size.at(p), p);
    }
    std::unordered_map<void*, size_t> alloc_size;

    // the dequantize-fused FC path, on the quantized bytes (MGH_ALGO_DEQ_Q) or on fp16 copies
    bool deq() const { return algo == MGH_ALGO_DEQ_F16 || algo == MGH_ALGO_DEQ_Q; }
    // the dequantize-fused FC entry points for this algorithm's weight form (wt: the GGUF type)
    int fc(int wt, const void* w, int N, int K, const void* x16, int M, const float* b, int act, const float* r,
           float* y) {
        return algo == MGH_ALGO_DEQ_Q ? mgh_gemm_dq(ctx, wt, w, N, K, x16, M, b, act, r, y)
                                      : mgh_gemm_h16(ctx, w, N, K, x16, M, b, act, r, y);
    }
    int fc_y16(int wt, const void* w, int N, int K, const void* x16, int M, const float* b, int act,
               const float* r, void* y16) {
        return algo == MGH_ALGO_DEQ_Q ? mgh_gemm_dq_y16(ctx, wt, w, N, K, x16, M, b, act, r, y16)
                                      : mgh_gemm_h16_y16(ctx, w, N, K, x16, M, b, act, r, y16);
    }
    int fc_f32in(int wt, const void* w, int N, int K, const float* x, int M, const float* b, int act,
                 const float* r, float* y) {
        return algo == MGH_ALGO_DEQ_Q ? mgh_gemm_dq_f32in(ctx, wt, w, N, K, x, M, b, act, r, y)
                                      : mgh_gemm_h16_f32in(ctx, w, N, K, x, M, b, act, r, y);
    }
    int fc_ln(int wt, const void* w, int N, int K, const void* x16, int M, const float* b, int act, const float* r,
              float* y, const float* gamma, const float* beta, float eps, float* y_ln, int emit, void* codes,
              float* dx, void* s4) {
        return algo == MGH_ALGO_DEQ_Q
                   ? mgh_gemm_dq_ln(ctx, wt, w, N, K, x16, M, b, act, r, y, gamma, beta, eps, y_ln, emit, codes, dx, s4)
                   : mgh_gemm_h16_ln(ctx, w, N, K, x16, M, b, act, r, y, gamma, beta, eps, y_ln, emit, codes, dx,
                                     s4);
    }

    // layout 0: the leaf's bytes as stored; 1: quantized weight in the int8-dot packed layout
    // (mgh_pack_weights); 2: quantized weight dequantized into fp16 (mgh_pack_weights_f16);
    // 3: F32 conv kernel {KW, KH, IC, OC} in the tap-major layout (mgh_conv2d_pack_weights);
    // 4: the same kernel quantized per (channel, 32-block) for the int8 conv (mgh_conv2d_i8_pack_weights);
    // 5: quantized weight in the K-loop-dequant layout, GGUF-sized (mgh_pack_weights_dq);
    // 6: quantized weight dequantized into fp32 [N][K] (mgh_dequant_weights_f32)
    void* upload_leaf(const Tensor* t, int layout) {
        const size_t n = t->nbytes();
        const auto key = std::make_tuple((const void*)t->data, n, layout ? 100 * layout + (int)t->type : -1);
        const auto it = leaves.find(key);
        if (it != leaves.end()) return it->second;
        if (!t->data) throw std::runtime_error("HipRuntime: leaf '" + t->name + "' has no host data");
        void* raw = nullptr;
        check(mgh_alloc(ctx, n, &raw));
        check(mgh_h2d(ctx, raw, t->data, n));
        void* d = raw;
        if (layout == 3 || layout == 4) {
            const int KW = (int)t->ne[0], KH = (int)t->ne[1], IC = (int)t->ne[2], OC = (int)t->ne[3];
            if (layout == 3) {
                check(mgh_alloc(ctx, mgh_conv2d_packed_bytes(KW, KH, IC, OC), &d));
                check(mgh_conv2d_pack_weights(ctx, (const float*)raw, KW, KH, IC, OC, (float*)d));
            } else {
                check(mgh_alloc(ctx, mgh_conv2d_i8_weight_bytes(KW, KH, IC, OC), &d));
                check(mgh_conv2d_i8_pack_weights(ctx, (const float*)raw, KW, KH, IC, OC, d));
            }
            check(mgh_free(ctx, raw));
        } else if (layout) {
            const int wt = t->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K;
            const int K = (int)t->ne[0], N = (int)(t->nelements() / t->ne[0]);
            const size_t pb = layout == 2   ? mgh_packed_weight_bytes_f16(N, K)
                              : layout == 5 ? mgh_packed_weight_bytes_dq(wt, N, K)
                              : layout == 6 ? (size_t)N * K * 4
                                            : mgh_packed_weight_bytes(wt, N, K);
            if (!pb) throw std::runtime_error("HipRuntime: unsupported quantized weight shape for '" + t->name + "'");
            check(mgh_alloc(ctx, pb, &d));
            check(layout == 2   ? mgh_pack_weights_f16(ctx, wt, raw, N, K, d)
                  : layout == 5 ? mgh_pack_weights_dq(ctx, wt, raw, N, K, d)
                  : layout == 6 ? mgh_dequant_weights_f32(ctx, wt, raw, N, K, (float*)d)
                                : mgh_pack_weights(ctx, wt, raw, N, K, d));
            check(mgh_free(ctx, raw));
        }
        leaves[key] = d;
        return d;
    }

    const Tensor* root(const Tensor* t) const {
        while (is_view_op(t->op)) t = t->src[0];
        return t;
    }

    // weights of a fused FC group, rows concatenated in member order (cached): fp16 copies, or
    // (MGH_ALGO_DEQ_Q) the K-loop-dequant layout of the stacked blocks -- ggml blocks are
    // row-local, so the members' block bytes back to back are the stacked matrix's
    void* fused_weight(const std::vector<Tensor*>& grp, int K, int64_t Nt) {
        std::vector<const void*> key;
        for (const Tensor* m : grp) key.push_back(m->src[0]->data);
        const auto it = fused_w.find(key);
        if (it != fused_w.end()) return it->second;
        void* d = nullptr;
        if (algo == MGH_ALGO_DEQ_Q) {
            const Tensor* w0 = grp[0]->src[0];
            const int wt = w0->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K;
            size_t total = 0;
            for (const Tensor* m : grp) {
                if (m->src[0]->type != w0->type) throw std::runtime_error("HipRuntime: fused FC weights differ in type");
                total += m->src[0]->nbytes();
            }
            void* raw = nullptr;
            check(mgh_alloc(ctx, total, &raw));
            size_t off = 0;
            for (const Tensor* m : grp) {
                const Tensor* w = m->src[0];
                if (!w->data) throw std::runtime_error("HipRuntime: leaf '" + w->name + "' has no host data");
                check(mgh_h2d(ctx, (char*)raw + off, w->data, w->nbytes()));
                off += w->nbytes();
            }
            const size_t pb = mgh_packed_weight_bytes_dq(wt, (int)Nt, K);
            if (!pb) throw std::runtime_error("HipRuntime: unsupported quantized weight shape for a fused FC group");
            check(mgh_alloc(ctx, pb, &d));
            check(mgh_pack_weights_dq(ctx, wt, raw, (int)Nt, K, d));
            check(mgh_sync(ctx));
            check(mgh_free(ctx, raw));
            return fused_w[key] = d;
        }
        check(mgh_alloc(ctx, mgh_packed_weight_bytes_f16((int)Nt, K), &d));
        int64_t off = 0;
        for (const Tensor* m : grp) {
            const Tensor* w = m->src[0];
            if (!w->data) throw std::runtime_error("HipRuntime: leaf '" + w->name + "' has no host data");
            const int N = (int)w->ne[1];
            void* raw = nullptr;
            check(mgh_alloc(ctx, w->nbytes(), &raw));
            check(mgh_h2d(ctx, raw, w->data, w->nbytes()));
            check(mgh_pack_weights_f16(ctx, w->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K, raw, N, K,
                                       (char*)d + (size_t)off * K * 2));
            check(mgh_sync(ctx));
            check(mgh_free(ctx, raw));
            off += N;
        }
        return fused_w[key] = d;
    }

    // biases of a fused FC group, concatenated (zeros for members without one)
    void* fused_bias(const std::vector<Tensor*>& grp, int64_t Nt) {
        std::vector<const void*> key;
        for (const Tensor* m : grp) key.push_back(m->src[2] ? m->src[2]->data : nullptr);
        const auto it = fused_b.find(key);
        if (it != fused_b.end()) return it->second;
        std::vector<float> h((size_t)Nt, 0.0f);
        int64_t off = 0;
        for (const Tensor* m : grp) {
            const Tensor* b = m->src[2];
            const int64_t N = m->src[0]->ne[1];
            if (b) {
                if (b->type != Type::F32 || b->nelements() != N || !b->data)
                    throw std::runtime_error("HipRuntime: fused FC bias must be F32 [N] with host data");
                std::memcpy(h.data() + off, b->data, (size_t)N * 4);
            }
            off += N;
        }
        void* d = nullptr;
        check(mgh_alloc(ctx, (size_t)Nt * 4, &d));
        check(mgh_h2d(ctx, d, h.data(), (size_t)Nt * 4));
        return fused_b[key] = d;
    }

    // element strides of a view of a fused FC output: whole-row strides scale to the wide pitch
    void widen(const Tensor* v, int64_t st[4]) const {
        const auto p = pitch.find(root(v));
        if (p == pitch.end()) return;
        const int64_t rowlen = root(v)->ne[0];
        for (int i = 0; i < 4; i++)
            if (st[i] >= rowlen && st[i] % rowlen == 0) st[i] = st[i] / rowlen * p->second;
    }

    void* dev(const Tensor* t) {
        if (!t) return nullptr;
        const Tensor* r = root(t);
        if (r->op == Op::None) {
            const auto it = addr.find(r);
            if (it != addr.end()) return it->second;
            const auto b = bound.find(r);
            void* d = b != bound.end() ? b->second : upload_leaf(r, 0);
            addr[r] = d;
            return d;
        }
        const auto it = addr.find(r);
        if (it == addr.end()) throw std::runtime_error("HipRuntime: node used before it was computed");
        return it->second;
    }

    static void elem_strides(const Tensor* t, int64_t st[4]) {
        const size_t es = type_size(t->type);
        for (int i = 0; i < 4; i++) st[i] = (int64_t)(t->nb[i] / es);
    }

    std::pair<void*, void*> unit(int64_t D) {
        auto it = unit_affine.find(D);
        if (it != unit_affine.end()) return it->second;
        std::vector<float> one((size_t)D, 1.0f), zero((size_t)D, 0.0f);
        void *g = nullptr, *b = nullptr;
        check(mgh_alloc(ctx, (size_t)D * 4, &g));
        check(mgh_alloc(ctx, (size_t)D * 4, &b));
        check(mgh_h2d(ctx, g, one.data(), (size_t)D * 4));
        check(mgh_h2d(ctx, b, zero.data(), (size_t)D * 4));
        return unit_affine[D] = {g, b};
    }
};

HipRuntime::HipRuntime() : HipRuntime(0) {}

HipRuntime::HipRuntime(int device) : p_(new Impl()) {
    if (mgh_create(device, &p_->ctx) != MGH_OK)
        throw std::runtime_error("HipRuntime: no gfx950 device at ordinal " + std::to_string(device));
    p_->name = mgh_device_name(p_->ctx);
}

HipRuntime::~HipRuntime() {
    if (!p_ || !p_->ctx) return;
    mgh_sync(p_->ctx);
    for (auto& kv : p_->leaves) mgh_free(p_->ctx, kv.second);
    for (auto& kv : p_->fused_w) mgh_free(p_->ctx, kv.second);
    for (auto& kv : p_->fused_b) mgh_free(p_->ctx, kv.second);
    for (auto& kv : p_->pool) mgh_free(p_->ctx, kv.second);
    if (p_->held) mgh_free(p_->ctx, p_->held);
    for (auto& kv : p_->unit_affine) {
        mgh_free(p_->ctx, kv.second.first);
        mgh_free(p_->ctx, kv.second.second);
    }
    mgh_destroy(p_->ctx);
}

const std::string& HipRuntime::device_name() const { return p_->name; }

void HipRuntime::invalidate(Tensor* t) {
    if (!t) return;
    for (auto it = p_->leaves.begin(); it != p_->leaves.end();) {
        if (std::get<0>(it->first) == t->data) {
            mgh_free(p_->ctx, it->second);
            it = p_->leaves.erase(it);
        } else {
            ++it;
        }
    }
    for (auto* m : {&p_->fused_w, &p_->fused_b})
        for (auto it = m->begin(); it != m->end();) {
            if (std::find(it->first.begin(), it->first.end(), (const void*)t->data) != it->first.end()) {
                mgh_free(p_->ctx, it->second);
                it = m->erase(it);
            } else {
                ++it;
            }
        }
}

bool HipRuntime::import_host_region(void*, size_t) { return false; }

void HipRuntime::profile_enable(bool on) { p_->profiling = on; }
void HipRuntime::profile_reset() { p_->prof.clear(); }
std::vector<OpProfile> HipRuntime::profile_report() const {
    std::vector<OpProfile> r;
    for (auto& kv : p_->prof) r.push_back({kv.first, kv.second.first, kv.second.second});
    std::sort(r.begin(), r.end(), [](const OpProfile& a, const OpProfile& b) { return a.ms > b.ms; });
    return r;
}

void HipRuntime::set_quant_algo(int algo) {
    if (algo != MGH_ALGO_INT8 && algo != MGH_ALGO_DEQ_F16 && algo != MGH_ALGO_DEQ_Q)
        throw std::runtime_error("HipRuntime: quant algo must be 1 (int8), 2 (dequant, fp16 weight copies) or 3 "
                                 "(dequant on the quantized bytes)");
    p_->algo = algo;
}

void HipRuntime::bind_device(const Tensor* t, void* d) {
    if (!t || t->op != Op::None) throw std::runtime_error("HipRuntime::bind_device: needs a leaf tensor");
    p_->bound[t] = d;
}

mgh_ctx* HipRuntime::context() const { return p_->ctx; }

void HipRuntime::compute(Graph& g) { run(g, true); }

const void* HipRuntime::compute_device(Graph& g) { return run(g, false); }

const void* HipRuntime::run(Graph& g, bool readback) {
    Impl& I = *p_;
    if (I.held) {
        I.give(I.held);
        I.held = nullptr;
    }
    if (g.nodes.empty()) {
        I.bound.clear();
        return nullptr;
    }
    I.addr.clear();
    I.codes.clear();
    const int n = (int)g.nodes.size();
    // quantized weights the fused kernels take (mgh_gemm_h16 / _dq / _q_packed: Q8_0 with
    // K % 64 == 0, N % 4 == 0; Q4_K with N % 4 == 0; N <= 2^21); other quantized shapes run the
    // reference's F32 dequant GEMM on weights dequantized once at upload (layout 6)
    auto quant = [](const Tensor* w) {
        if (w->type != Type::Q8_0 && w->type != Type::Q4_K) return false;
        const int64_t K = w->ne[0], N = w->nelements() / w->ne[0];
        return N % 4 == 0 && N <= (int64_t)1 << 21 && (w->type == Type::Q4_K || K % 64 == 0);
    };

    // ---- plan (reused for a graph that matches the last planned one) ----
    Impl::Plan& P = I.plan;
    const bool reuse = I.plan_matches(g);
    auto& last = P.last;
    auto& fc_uses = P.fc_uses;
    auto& other_uses = P.other_uses;
    auto& fa_into = P.fa_into;
    auto& fa_target = P.fa_target;
    auto& groups = P.groups;
    auto& grp_of = P.grp_of;
    auto& grp16 = P.grp16;
    auto& emit16 = P.emit16;
    auto& ln_pair = P.ln_pair;
    auto& cfuse = P.cfuse;
    auto& absorbed = P.absorbed;
    using ConvFuse = Impl::ConvFuse;
    (void)other_uses;
    I.pitch.clear();
    if (reuse) {
        I.owner = P.owner;
    } else {
        I.owner.clear();
        last.clear();
        fc_uses.clear();
        other_uses.clear();
        fa_into.clear();
        fa_target.clear();
        groups.clear();
        grp_of.clear();
        grp16.clear();
        emit16.clear();
        ln_pair.clear();
        cfuse.clear();
        absorbed.clear();
        for (int i = 0; i < n; i++) {
            const Tensor* t = g.nodes[i];
            for (const Tensor* s : t->src) {
                if (!s) continue;
                const Tensor* r = I.root(s);
                last[r] = i;
                if (r->op == Op::Norm && !is_view_op(t->op)) {
                    if (t->op == Op::MulMat && s == t->src[1] && quant(t->src[0])) fc_uses[r]++;
                    else other_uses[r]++;
                }
            }
        }
        // flash attention -> permute(0,2,1,3) -> cont: the attention writes the cont's buffer
        {
            std::unordered_map<const Tensor*, int> uses;
            for (const Tensor* t : g.nodes)
                for (const Tensor* s : t->src)
                    if (s) uses[s]++;
            for (const Tensor* t : g.nodes) {
                if (t->op != Op::Cont) continue;
                const Tensor* p = t->src[0];
                if (p->op != Op::Permute || !p->src[0] || p->src[0]->op != Op::FlashAttention) continue;
                const Tensor* fa = p->src[0];
                // only the head merge permute(0, 2, 1, 3): the attention then writes its output
                // straight into the merged layout; any other view goes through the strided copy
                const bool merge = p->ne[0] == fa->ne[0] && p->ne[1] == fa->ne[2] && p->ne[2] == fa->ne[1] &&
                                   p->ne[3] == fa->ne[3] && p->nb[0] == fa->nb[0] && p->nb[1] == fa->nb[2] &&
                                   p->nb[2] == fa->nb[1] && p->nb[3] == fa->nb[3] && fa->is_contiguous();
                if (merge && uses[fa] == 1 && uses[p] == 1 && fa->type == Type::F32) fa_into[t] = fa;
            }
        }
        for (auto& kv : fa_into) fa_target[kv.second] = kv.first;

        // dequantize-fused path: quantized FCs that read the same activations and feed only the
        // attention (q, k, v: mg-transformer.cpp:59-70) run as one GEMM on row-concatenated
        // weights; each output is a column range of the wide result, which the attention reads
        // through its strides
        if (I.deq()) {
            std::unordered_map<const Tensor*, std::vector<const Tensor*>> cons;   // root -> consumer nodes
            for (const Tensor* t : g.nodes) {
                if (is_view_op(t->op)) continue;
                for (const Tensor* s : t->src)
                    if (s) cons[I.root(s)].push_back(t);
            }
            std::map<std::tuple<const Tensor*, int, int64_t, int>, int> key_grp;
            for (Tensor* t : g.nodes) {
                if (t->op != Op::MulMat || !quant(t->src[0]) || t->src[3] || t != I.root(t)) continue;
                bool fa_only = !cons[t].empty();
                for (const Tensor* c : cons[t]) fa_only = fa_only && c->op == Op::FlashAttention;
                if (!fa_only || t == g.nodes.back()) continue;
                const Tensor* w = t->src[0];
                const auto key = std::make_tuple(I.root(t->src[1]), (int)w->type, w->ne[0], t->iparam[0]);
                auto it = key_grp.find(key);
                if (it == key_grp.end()) {
                    key_grp[key] = (int)groups.size();
                    groups.push_back({t});
                } else {
                    groups[it->second].push_back(t);
                }
            }
            for (size_t gi = 0; gi < groups.size(); gi++) {
                if (groups[gi].size() < 2) continue;
                const Tensor* lead = groups[gi][0];
                for (Tensor* m : groups[gi]) {
                    grp_of[m] = (int)gi;
                    last[lead] = std::max(last[lead], last.count(m) ? last[m] : 0);
                }
            }
            // a group whose attentions can all read fp16 q/k/v (the whole-head kernel: S <= 512,
            // scale > 0, unit d stride, strides and column offsets in multiples of 8 halves) stores its wide
            // output as fp16; the attention would round q/k/v to fp16 on load (same result)
            for (size_t gi = 0; gi < groups.size(); gi++) {
                if (groups[gi].size() < 2) continue;
                bool ok = true;
                int64_t Nt = 0, off = 0;
                for (const Tensor* m : groups[gi]) Nt += m->src[0]->ne[1];
                for (const Tensor* m : groups[gi]) {
                    ok = ok && off % 8 == 0;
                    off += m->src[0]->ne[1];
                    for (const Tensor* c : cons[m]) {
                        const int D = (int)c->src[0]->ne[0], S = (int)c->src[0]->ne[1];
                        ok = ok && S <= 512 && (D == 16 || D == 32 || D == 48 || D == 64) && c->fparam[0] > 0.f;
                        for (int j = 0; j < 3 && ok; j++) {
                            int64_t st[4];
                            Impl::elem_strides(c->src[j], st);
                            const int64_t rowlen = I.root(c->src[j])->ne[0];
                            for (int i = 0; i < 4; i++)
                                if (st[i] >= rowlen && st[i] % rowlen == 0) st[i] = st[i] / rowlen * Nt;
                            ok = ok && st[0] == 1 && st[1] % 8 == 0 && st[2] % 8 == 0 && st[3] % 8 == 0;
                        }
                    }
                }
                if (ok) grp16.insert((int)gi);
            }
        }


        // dequantize-fused path: an attention output or an FC output whose only consumers are
        // dequantize-fused FCs reading it as their activations is stored as fp16 directly (the
        // consumers would round it to fp16 on their way in; the result is identical)
        if (I.deq()) {
            std::unordered_map<const Tensor*, std::vector<const Tensor*>> cons;
            for (const Tensor* t : g.nodes) {
                if (is_view_op(t->op)) continue;
                for (const Tensor* s : t->src)
                    if (s) cons[I.root(s)].push_back(t);
            }
            for (const Tensor* t : g.nodes) {
                if (t == g.nodes.back() || is_view_op(t->op) || grp_of.count(t)) continue;
                const bool fa_out = t->op == Op::Cont && fa_into.count(t);
                const bool fc_out = t->op == Op::MulMat && quant(t->src[0]);
                if (!fa_out && !fc_out) continue;
                bool ok = !cons[t].empty();
                // every consumer reads t only as its activations (not as weight, bias or residual)
                for (const Tensor* c : cons[t])
                    ok = ok && c->op == Op::MulMat && quant(c->src[0]) && I.root(c->src[1]) == t &&
                         I.root(c->src[0]) != t && (!c->src[2] || I.root(c->src[2]) != t) &&
                         (!c->src[3] || I.root(c->src[3]) != t) && c->src[1]->type == Type::F32 &&
                         c->src[1]->is_contiguous();
                if (ok) emit16.insert(t);
            }
        }

        // post-norm pairs (mg-transformer.cpp:88-90, 95-97): a dequantize-fused FC without
        // activation whose only consumer is a Norm over its rows runs as one mgh_gemm_h16_ln call,
        // which for split-K plans (a few hundred rows) normalizes the rows in the reduce, one
        // launch fewer; the Norm node then launches nothing. Same bits as the two nodes apart.
        if (I.deq()) {
            std::unordered_map<const Tensor*, std::vector<const Tensor*>> cons;
            for (const Tensor* t : g.nodes)
                for (const Tensor* s : t->src)
                    if (s) cons[I.root(s)].push_back(t);
            std::unordered_map<const Tensor*, size_t> pos;
            for (size_t i = 0; i < g.nodes.size(); i++) pos[g.nodes[i]] = i;
            // the Norm's gamma / beta are read when the FC runs: they must be leaves or nodes
            // computed before it (a computed gamma between the FC and the Norm would not exist yet)
            auto ready_at = [&](const Tensor* s, const Tensor* fc) {
                if (!s) return true;
                const auto it = pos.find(I.root(s));
                return it == pos.end() || it->second < pos.at(fc);
            };
            for (const Tensor* t : g.nodes) {
                if (t->op != Op::MulMat || !quant(t->src[0]) || grp_of.count(t) || emit16.count(t) ||
                    t == g.nodes.back() || t->iparam[0] != 0)
                    continue;
                const auto& cs = cons[t];
                if (cs.size() != 1 || cs[0]->op != Op::Norm || cs[0]->src[0] != t) continue;
                if (!ready_at(cs[0]->src[1], t) || !ready_at(cs[0]->src[2], t)) continue;
                const int64_t N = t->src[0]->ne[1];
                if (cs[0]->ne[0] != N || N % 256 || N > 2048 || cs[0]->nelements() != t->nelements()) continue;
                ln_pair[t] = cs[0];
            }
        }

        // Conv2D epilogue fusion (the VQGAN decoder, mg-vqgan.cpp:31-55): the Add of a per-channel
        // bias viewed as {1, 1, C, 1} that is a conv's only consumer, and then an Add of a same-shaped
        // tensor computed before the conv (the res block's h + x, or h + conv_res(h)), are evaluated
        // in the conv's epilogue with the same roundings (out = (conv + bias) + resid); the absorbed
        // Add nodes launch nothing and share the conv's buffer
        {
            std::unordered_map<const Tensor*, int> uses, at;
            for (int i = 0; i < n; i++) {
                at[g.nodes[i]] = i;
                for (const Tensor* s : g.nodes[i]->src)
                    if (s) uses[s]++;
            }
            auto f32c = [](const Tensor* x) { return x->type == Type::F32 && x->is_contiguous(); };
            for (int i = 0; i < n; i++) {
                const Tensor* t = g.nodes[i];
                if (t->op == Op::Conv2D) cfuse[t].out = t;
                if (t->op != Op::Add) continue;
                const Tensor* a = t->src[0];
                const Tensor* b = t->src[1];
                // conv (+ bias already absorbed) whose only consumer is this Add, with no residual yet
                auto open_conv = [&](const Tensor* x) -> const Tensor* {
                    if (uses[x] != 1 || !f32c(x)) return nullptr;
                    const Tensor* cv = x->op == Op::Conv2D ? x : (absorbed.count(x) ? absorbed.at(x) : nullptr);
                    if (!cv || cfuse.at(cv).out != x || cfuse.at(cv).resid) return nullptr;
                    return cv;
                };
                const Tensor* cv = open_conv(a);
                const Tensor* rb = I.root(b);
                if (cv && !cfuse.at(cv).bias && cfuse.at(cv).out == cv && rb->op == Op::None && f32c(rb) &&
                    b->ne[0] == 1 && b->ne[1] == 1 && b->ne[2] == a->ne[2] && b->ne[3] == 1 &&
                    rb->nelements() == a->ne[2] && b->is_contiguous()) {
                    cfuse[cv].bias = rb;
                    cfuse[cv].out = t;
                    absorbed[t] = cv;
                    continue;
                }
                if (!std::equal(a->ne, a->ne + 4, b->ne) || !f32c(a) || !f32c(b) || !f32c(t)) continue;
                for (const Tensor* x : {b, a}) {                         // prefer the later operand
                    const Tensor* c2 = open_conv(x);
                    const Tensor* r = I.root(x == a ? b : a);
                    if (!c2 || (r->op != Op::None && (!at.count(r) || at.at(r) >= at.at(c2)))) continue;
                    cfuse[c2].resid = x == a ? b : a;
                    cfuse[c2].out = t;
                    absorbed[t] = c2;
                    break;
                }
            }
            for (auto& kv : cfuse)                                        // the chain shares one buffer
                if (kv.second.out != kv.first) {
                    I.owner[kv.first] = kv.second.out;
                    for (auto& ab : absorbed)
                        if (ab.second == kv.first && ab.first != kv.second.out) I.owner[ab.first] = kv.second.out;
                }
        }

        P.owner = I.owner;
        P.valid = true;
    }
    std::unordered_set<const Tensor*> h16_store;         // nodes whose device data is fp16
    std::unordered_set<const Tensor*> ln_done;           // Norms computed with their FC

    // release roots whose last consumer was node i (never the final output)
    auto release_after = [&](int i, const Tensor* t) {
        for (const Tensor* s : t->src) {
            if (!s) continue;
            const Tensor* r = I.root(s);
            if (r->op == Op::None || r == g.nodes.back() || last.at(r) != i) continue;
            const auto a = I.addr.find(r);
            if (a == I.addr.end() || !a->second) continue;
            if (fa_target.count(r)) continue;                      // shares the cont's buffer
            const auto ow = I.owner.find(r);
            if (ow != I.owner.end() && ow->second != r) continue;   // column range of a fused output
            I.give(a->second);
            a->second = nullptr;
            const auto c = I.codes.find(r);
            if (c != I.codes.end()) {
                I.give(c->second.q);
                I.give(c->second.dx);
                I.give(c->second.sx);
                I.codes.erase(c);
            }
        }
    };

    // MG_DUMP_NAMED: named computed nodes are read back to their host data (mg-opencl.cpp
    // :1627-1641), each right after its kernel, while its buffer is still its own
    const bool dump_named = std::getenv("MG_DUMP_NAMED") != nullptr;

    auto dump_node = [&](const Tensor* d) {
        const auto a = I.addr.find(d);
        if (!d->name.empty() && d->data && a != I.addr.end() && a->second && !h16_store.count(d) &&
            !I.pitch.count(d))
            I.check(mgh_d2h(I.ctx, d->data, a->second, d->nbytes()));
    };
    // a Norm's affine parameters (unit when absent) and the FC operand it emits: int8 codes
    // (flat 32-blocks, so any FC row length that is a multiple of 32 reads the same codes), or
    // for the dequantize-fused path the fp16-rounded y, when a quantized FC reads it
    struct NormOut {
        const float* gamma;
        const float* beta;
        int emit = MGH_EMIT_NONE;
        Impl::Codes cd;
    };
    auto norm_out = [&](const Tensor* t) {
        NormOut o;
        const int D = (int)t->ne[0];
        const int rows = (int)(t->nelements() / D);
        o.gamma = (const float*)I.dev(t->src[1]);
        o.beta = (const float*)I.dev(t->src[2]);
        if (!t->src[1] || !t->src[2]) {
            const auto u = I.unit(D);
            o.gamma = (const float*)u.first;
            o.beta = (const float*)u.second;
        }
        if ((I.algo == MGH_ALGO_INT8 || I.deq()) && fc_uses.count(t)) {
            o.emit = I.algo == MGH_ALGO_INT8 ? MGH_EMIT_INT8 : MGH_EMIT_DEQ_F16;
            const size_t T = (size_t)D / 32;
            o.cd.q = I.take((size_t)rows * D * 2);
            if (o.emit == MGH_EMIT_INT8) {         // the dequant-fused GEMM reads only the fp16 y
                o.cd.dx = I.take((size_t)rows * T * 4);
                o.cd.sx = I.take((size_t)rows * T * 4);
            }
        }
        return o;
    };

    // ---- run ----
    for (int i = 0; i < n; i++) {
        Tensor* t = g.nodes[i];
        if (is_view_op(t->op)) continue;
        if (t->type != Type::F32 && t->op != Op::GetRows)
            throw std::runtime_error("HipRuntime: only F32 results are supported");
        if (grp_of.count(t) && I.addr.count(t)) {                 // computed with its group
            release_after(i, t);
            continue;
        }
        if (ln_done.count(t)) {                                    // normalized with its FC
            if (dump_named) dump_node(t);
            release_after(i, t);
            continue;
        }
        if (absorbed.count(t)) {                                   // evaluated by its conv
            release_after(i, t);
            continue;
        }
        // a cont written by its attention launches nothing: not timed
        const bool timed = I.profiling && !(t->op == Op::Cont && fa_into.count(t));
        if (timed) I.check(mgh_timer_start(I.ctx));

        void* out = nullptr;
        if (grp_of.count(t)) {
            const std::vector<Tensor*>& grp = groups[grp_of.at(t)];
            const Tensor* x = t->src[1];
            if (x->type != Type::F32 || !x->is_contiguous())
                throw std::runtime_error("HipRuntime: MulMat needs a contiguous F32 input");
            const int K = (int)t->src[0]->ne[0];
            const int M = (int)(x->nelements() / K);
            int64_t Nt = 0;
            for (const Tensor* m : grp) Nt += m->src[0]->ne[1];
            void* wp = I.fused_weight(grp, K, Nt);
            const int wt = t->src[0]->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K;
            const float* bias = (const float*)I.fused_bias(grp, Nt);
            const auto c = I.codes.find(I.root(x));
            const bool h16 = c != I.codes.end() && grp16.count(grp_of.at(t));
            out = I.take((size_t)M * Nt * (h16 ? 2 : 4));
            if (h16)
                I.check(I.fc_y16(wt, wp, (int)Nt, K, c->second.q, M, bias, t->iparam[0], nullptr, out));
            else if (c != I.codes.end())
                I.check(I.fc(wt, wp, (int)Nt, K, c->second.q, M, bias, t->iparam[0], nullptr, (float*)out));
            else
                I.check(I.fc_f32in(wt, wp, (int)Nt, K, (const float*)I.dev(x), M, bias, t->iparam[0], nullptr,
                                   (float*)out));
            int64_t off = 0;
            for (const Tensor* m : grp) {
                I.addr[m] = (char*)out + off * (h16 ? 2 : 4);
                I.pitch[m] = Nt;
                I.owner[m] = grp[0];
                if (h16) h16_store.insert(m);
                off += m->src[0]->ne[1];
            }
        } else if (t->op == Op::Cont && fa_into.count(t)) {
            out = I.dev(fa_into.at(t));                         // written by the attention
            I.addr[t] = out;
        } else if (t->op == Op::FlashAttention && fa_target.count(t)) {
            // an fp16-only merged output (emit16) needs no fp32 buffer
            out = emit16.count(fa_target.at(t)) ? nullptr : I.take(fa_target.at(t)->nbytes());
            I.addr[fa_target.at(t)] = out;
            I.addr[t] = out;
        } else if (t->op == Op::MulMat && emit16.count(t) && I.codes.count(I.root(t->src[1]))) {
            out = nullptr;                                      // stored as fp16 only (below)
            I.addr[t] = out;
        } else if (t->op == Op::Conv2D && cfuse.at(t).out != t) {
            out = I.take(cfuse.at(t).out->nbytes());             // written once, by the conv
            I.addr[t] = out;
            I.addr[cfuse.at(t).out] = out;
            for (auto& ab : absorbed)
                if (ab.second == t) I.addr[ab.first] = out;
        } else if (t->op == Op::MulMat && ln_pair.count(t) && I.codes.count(I.root(t->src[1])) &&
                   !(dump_named && !t->name.empty())) {
            // an FC whose only reader is its post-norm: the pair call writes only the Norm's
            // outputs (the FC's own rows stay in the library's scratch, or in registers when
            // the split-K reduce normalizes them)
            out = nullptr;
            I.addr[t] = out;
        } else {
            out = I.take(t->nbytes());
            I.addr[t] = out;
        }

        switch (grp_of.count(t) ? Op::None : t->op) {
            case Op::None:
                break;
            case Op::MulMat: {
                const Tensor* w = t->src[0];
                const Tensor* x = t->src[1];
                if (x->type != Type::F32)
                    throw std::runtime_error("HipRuntime: MulMat needs an F32 input");
                // F32 weights: strided or batched operands (the unfused attention chain), and
                // every product up to 2^28 multiply-adds, take the order-exact kernel (each
                // output sums k in order with separate multiply and add, as the reference CPU
                // executor, so the reference's absolute gates hold: tools/test-opencl.cpp:50);
                // larger contiguous products (the tied MLM head) take the fp32 MFMA GEMM
                const bool f32_exact = w->type == Type::F32 &&
                                       (!x->is_contiguous() || !w->is_contiguous() || w->ne[2] != 1 ||
                                        w->ne[3] != 1 || (double)w->ne[0] * w->ne[1] * (x->nelements() / x->ne[0]) <=
                                                             (double)(1 << 28));
                if (f32_exact) {
                    // the reference's k_mul_mat_t contract (mg-opencl.cpp:60-94, 1429-1440)
                    if (t->src[3] && !t->src[3]->is_contiguous())
                        throw std::runtime_error("HipRuntime: MulMat residual must be contiguous");
                    int64_t wst[4], xst[4];
                    Impl::elem_strides(w, wst);
                    Impl::elem_strides(x, xst);
                    I.check(mgh_gemm_f32_batched(I.ctx, (const float*)I.dev(w), w->ne, wst, (const float*)I.dev(x), x->ne,
                                                 xst, (const float*)I.dev(t->src[2]), t->iparam[0],
                                                 (const float*)I.dev(t->src[3]), (float*)out));
                    break;
                }
                if (!x->is_contiguous())
                    throw std::runtime_error("HipRuntime: MulMat needs a contiguous F32 input");
                const int K = (int)w->ne[0], N = (int)w->ne[1];
                const int M = (int)(x->nelements() / K);     // batch flattened into M
                const float* bias = (const float*)I.dev(t->src[2]);
                const float* resid = (const float*)I.dev(t->src[3]);
                const int act = t->iparam[0];
                if (quant(w) && I.deq()) {
                    void* wp = I.upload_leaf(w, I.algo == MGH_ALGO_DEQ_Q ? 5 : 2);
                    const int wt = w->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K;
                    const auto c = I.codes.find(I.root(x));
                    if (c != I.codes.end() && emit16.count(t)) {
                        Impl::Codes cd;
                        cd.q = I.take((size_t)M * N * 2);
                        I.check(I.fc_y16(wt, wp, N, K, c->second.q, M, bias, act, resid, cd.q));
                        I.codes[t] = cd;
                    } else if (c != I.codes.end() && ln_pair.count(t)) {
                        const Tensor* nr = ln_pair.at(t);
                        void* yl = I.take(nr->nbytes());
                        I.addr[nr] = yl;
                        const NormOut o = norm_out(nr);
                        I.check(I.fc_ln(wt, wp, N, K, c->second.q, M, bias, act, resid, (float*)out, o.gamma,
                                        o.beta, nr->fparam[0], (float*)yl, o.emit, o.cd.q, (float*)o.cd.dx,
                                        o.cd.sx));
                        if (o.emit) I.codes[nr] = o.cd;
                        ln_done.insert(nr);
                    } else if (c != I.codes.end())
                        I.check(I.fc(wt, wp, N, K, c->second.q, M, bias, act, resid, (float*)out));
                    else
                        I.check(I.fc_f32in(wt, wp, N, K, (const float*)I.dev(x), M, bias, act, resid, (float*)out));
                } else if (quant(w)) {
                    void* wp = I.upload_leaf(w, 1);
                    const auto c = I.codes.find(I.root(x));
                    if (c != I.codes.end())
                        I.check(mgh_gemm_q_packed(I.ctx, w->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K,
                                                  wp, N, K, (const uint16_t*)c->second.q, (const float*)c->second.dx,
                                                  (const int32_t*)c->second.sx, M, bias, act, resid, (float*)out));
                    else
                        I.check(mgh_gemm_q_packed_f32in(I.ctx, I.algo,
                                                        w->type == Type::Q8_0 ? MGH_WTYPE_Q8_0 : MGH_WTYPE_Q4_K, wp,
                                                        N, K, (const float*)I.dev(x), M, bias, act, resid,
                                                        (float*)out));
                } else if (w->type == Type::Q8_0 || w->type == Type::Q4_K) {
                    // a quantized shape the fused kernels do not take: the reference's F32
                    // dequant GEMM (k_mul_mat_q8_0_t2 / q4k_t2, mg-opencl.cpp:320-411) on the
                    // weights dequantized once at upload
                    I.check(mgh_gemm_f32(I.ctx, (const float*)I.upload_leaf(w, 6), N, K, (const float*)I.dev(x), M,
                                         bias, act, resid, (float*)out));
                } else if (w->type == Type::F32) {
                    I.check(mgh_gemm_f32(I.ctx, (const float*)I.dev(w), N, K, (const float*)I.dev(x), M, bias,
                                         act, resid, (float*)out));
                } else {
                    throw std::runtime_error("HipRuntime: unsupported MulMat weight type");
                }
                break;
            }
            case Op::Norm: {
                const Tensor* x = t->src[0];
                const int D = (int)t->ne[0];
                const int rows = (int)(t->nelements() / D);
                const NormOut o = norm_out(t);
                I.check(mgh_layernorm_affine(I.ctx, (const float*)I.dev(x), o.gamma, o.beta, rows, D, t->fparam[0],
                                             (float*)out, o.emit, o.cd.q, (float*)o.cd.dx, o.cd.sx));
                if (o.emit) I.codes[t] = o.cd;
                break;
            }
            case Op::FlashAttention: {
                const Tensor* q = t->src[0];
                int64_t st[4], sk[4], sv[4];
                Impl::elem_strides(q, st);
                Impl::elem_strides(t->src[1], sk);
                Impl::elem_strides(t->src[2], sv);
                I.widen(q, st);
                I.widen(t->src[1], sk);
                I.widen(t->src[2], sv);
                if (!std::equal(st, st + 4, sk) || !std::equal(st, st + 4, sv))
                    throw std::runtime_error("HipRuntime: FlashAttention needs q, k, v with equal strides");
                const int D = (int)q->ne[0], S = (int)q->ne[1], H = (int)q->ne[2], B = (int)q->ne[3];
                int64_t ost[4];
                const int64_t* po = nullptr;
                if (fa_target.count(t)) {
                    // output element (d, s, h, b) at its place in the permuted-then-contiguous
                    // layout {D, H, S, B}
                    ost[0] = 1; ost[1] = (int64_t)D * H; ost[2] = D; ost[3] = (int64_t)D * H * S;
                    po = ost;
                }
                const bool in16 = h16_store.count(I.root(q)) && h16_store.count(I.root(t->src[1])) &&
                                  h16_store.count(I.root(t->src[2]));
                if (in16) {
                    const bool o16 = po && emit16.count(fa_target.at(t));
                    Impl::Codes cd;
                    if (o16) cd.q = I.take((size_t)D * S * H * B * 2);
                    I.check(mgh_flash_attn_f16in(I.ctx, I.dev(q), I.dev(t->src[1]), I.dev(t->src[2]), st, D, S, H, B,
                                                 t->fparam[0], o16 ? nullptr : (float*)out, o16 ? cd.q : nullptr, po));
                    if (o16) I.codes[fa_target.at(t)] = cd;
                } else if (po && emit16.count(fa_target.at(t))) {
                    Impl::Codes cd;
                    cd.q = I.take((size_t)D * S * H * B * 2);
                    I.check(mgh_flash_attn_f16kv_o16(I.ctx, (const float*)I.dev(q), (const float*)I.dev(t->src[1]),
                                                     (const float*)I.dev(t->src[2]), st, D, S, H, B, t->fparam[0],
                                                     cd.q, po));
                    I.codes[fa_target.at(t)] = cd;
                } else {
                    I.check(mgh_flash_attn_f16kv(I.ctx, (const float*)I.dev(q), (const float*)I.dev(t->src[1]),
                                                 (const float*)I.dev(t->src[2]), st, D, S, H, B, t->fparam[0],
                                                 (float*)out, po));
                }
                break;
            }
            case Op::GetRows: {
                const Tensor* a = t->src[0];
                const Tensor* ids = t->src[1];
                if (a->type != Type::F32 || ids->type != Type::I32 || !a->is_contiguous() || !ids->is_contiguous())
                    throw std::runtime_error("HipRuntime: GetRows needs an F32 table and I32 ids");
                I.check(mgh_get_rows(I.ctx, (const float*)I.dev(a), a->ne[0], a->nelements() / a->ne[0],
                                     (const int32_t*)I.dev(ids), ids->nelements(), (float*)out));
                break;
            }
            case Op::Add:
            case Op::Mul: {
                // b broadcast over its size-1 dimensions (mg-cpu.cpp:27-38, k_add / k_mul
                // mg-opencl.cpp:947-960)
                const Tensor* a = t->src[0];
                const Tensor* b = t->src[1];
                if (a->type != Type::F32 || b->type != Type::F32)
                    throw std::runtime_error("HipRuntime: Add/Mul need F32 operands");
                bool prefix = a->is_contiguous() && b->is_contiguous(), ones = false;
                for (int d = 0; d < 4; d++) {
                    if (b->ne[d] != t->ne[d] && b->ne[d] != 1)
                        throw std::runtime_error("HipRuntime: Add/Mul operand dims must match or be 1");
                    if (ones) prefix = prefix && b->ne[d] == 1;
                    else if (b->ne[d] != t->ne[d]) ones = true;
                }
                if (t->op == Op::Add && prefix) {   // b repeats as a whole (bias row, position table)
                    I.check(mgh_add(I.ctx, (const float*)I.dev(a), (const float*)I.dev(b), b->nelements(),
                                    (float*)out, a->nelements()));
                } else {
                    int64_t ast[4], bst[4];
                    Impl::elem_strides(a, ast);
                    Impl::elem_strides(b, bst);
                    I.check(mgh_binary(I.ctx, t->op == Op::Mul ? 1 : 0, (const float*)I.dev(a), ast,
                                       (const float*)I.dev(b), b->ne, bst, t->ne, (float*)out));
                }
                break;
            }
            case Op::SoftMax: {
                const Tensor* x = t->src[0];
                if (x->type != Type::F32 || !x->is_contiguous())
                    throw std::runtime_error("HipRuntime: SoftMax needs a contiguous F32 input");
                const int D = (int)t->ne[0];
                I.check(mgh_softmax(I.ctx, (const float*)I.dev(x), t->nelements() / D, D, t->fparam[0], (float*)out));
                break;
            }
            case Op::Scale:
            case Op::Gelu:
            case Op::Silu: {
                const Tensor* x = t->src[0];
                if (x->type != Type::F32 || !x->is_contiguous())
                    throw std::runtime_error("HipRuntime: Scale/Gelu/Silu need a contiguous F32 input");
                if (t->op == Op::Scale)
                    I.check(mgh_scale(I.ctx, (const float*)I.dev(x), t->nelements(), t->fparam[0], (float*)out));
                else
                    I.check(mgh_unary(I.ctx, t->op == Op::Gelu ? MGH_ACT_GELU : MGH_ACT_SILU, (const float*)I.dev(x),
                                      t->nelements(), (float*)out));
                break;
            }
            case Op::Cont: {
                if (fa_into.count(t)) break;                       // already written
                int64_t st[4];
                Impl::elem_strides(t->src[0], st);
                const int64_t ne[4] = {t->ne[0], t->ne[1], t->ne[2], t->ne[3]};
                I.check(mgh_copy_strided(I.ctx, (const float*)I.dev(t->src[0]), ne, st, (float*)out));
                break;
            }
            case Op::Conv2D: {
                // src[0] kernel {KW, KH, IC, OC}, src[1] input {IW, IH, IC, N}; iparam[0] stride,
                // iparam[1] pad (mg-tensor.cpp:167-177, dispatch mg-opencl.cpp:1535-1566)
                const Tensor* k = t->src[0];
                const Tensor* x = t->src[1];
                if (k->type != Type::F32 || x->type != Type::F32 || !k->is_contiguous() || !x->is_contiguous())
                    throw std::runtime_error("HipRuntime: Conv2D needs contiguous F32 kernel and input");
                if (k->ne[2] != x->ne[2] || t->ne[2] != k->ne[3] || t->ne[3] != x->ne[3])
                    throw std::runtime_error("HipRuntime: Conv2D kernel channels must match the input's");
                const int64_t dims[] = {x->ne[0], x->ne[1], x->ne[2], x->ne[3], k->ne[0], k->ne[1], k->ne[3]};
                for (int64_t d : dims)
                    if (d > INT32_MAX) throw std::runtime_error("HipRuntime: Conv2D dimension too large");
                const int KW = (int)k->ne[0], KH = (int)k->ne[1], IC = (int)k->ne[2], OC = (int)k->ne[3];
                const ConvFuse& f = cfuse.at(t);
                if (I.algo == MGH_ALGO_INT8 && k->op == Op::None && !std::getenv("MG_NO_ARM_CONV")) {
                    // the int8 conv, with the int8-dot FC path as in the reference (both follow
                    // cl_arm_integer_dot_product; MG_NO_ARM_CONV keeps the fp32 conv,
                    // mg-opencl.cpp:1237-1242, 1541-1553)
                    I.check(mgh_conv2d_i8(I.ctx, (const float*)I.dev(x), (int)x->ne[0], (int)x->ne[1], IC,
                                          (int)x->ne[3], I.upload_leaf(k, 4), KW, KH, OC, t->iparam[0],
                                          t->iparam[1], (const float*)I.dev(f.bias), (const float*)I.dev(f.resid),
                                          (float*)out));
                    break;
                }
                // tap-major weights packed once per leaf where the packed kernel runs
                const bool pk = k->op == Op::None && mgh_conv2d_packed_bytes(KW, KH, IC, OC) > 0;
                I.check(mgh_conv2d_ex(I.ctx, (const float*)I.dev(x), (int)x->ne[0], (int)x->ne[1], IC, (int)x->ne[3],
                                      pk ? nullptr : (const float*)I.dev(k), pk ? (const float*)I.upload_leaf(k, 3) : nullptr,
                                      KW, KH, OC, t->iparam[0], t->iparam[1], (const float*)I.dev(f.bias),
                                      (const float*)I.dev(f.resid), (float*)out));
                break;
            }
            case Op::GroupNorm: {
                // iparam[0] groups, fparam[1] eps; affine + SiLU when iparam[1] == 1 with gamma and
                // beta in src[1], src[2] (mg-opencl.cpp:1568-1590)
                const Tensor* x = t->src[0];
                if (x->type != Type::F32 || !x->is_contiguous())
                    throw std::runtime_error("HipRuntime: GroupNorm needs a contiguous F32 input");
                const bool fused = t->src[1] && t->src[2] && t->iparam[1] == 1;
                if (fused)
                    for (const Tensor* p : {t->src[1], t->src[2]})
                        if (p->type != Type::F32 || !p->is_contiguous() || p->nelements() != t->ne[2])
                            throw std::runtime_error("HipRuntime: GroupNorm gamma/beta must be F32 [C]");
                for (int d = 0; d < 4; d++)
                    if (t->ne[d] > INT32_MAX) throw std::runtime_error("HipRuntime: GroupNorm dimension too large");
                I.check(mgh_group_norm(I.ctx, (const float*)I.dev(x), (int)t->ne[0], (int)t->ne[1], (int)t->ne[2],
                                       (int)t->ne[3], t->iparam[0], t->fparam[1],
                                       fused ? (const float*)I.dev(t->src[1]) : nullptr,
                                       fused ? (const float*)I.dev(t->src[2]) : nullptr, (float*)out));
                break;
            }
            case Op::Upscale: {
                const Tensor* x = t->src[0];
                if (x->type != Type::F32 || !x->is_contiguous())
                    throw std::runtime_error("HipRuntime: Upscale needs a contiguous F32 input");
                for (int d = 0; d < 4; d++)
                    if (x->ne[d] > INT32_MAX) throw std::runtime_error("HipRuntime: Upscale dimension too large");
                I.check(mgh_upscale(I.ctx, (const float*)I.dev(x), (int)x->ne[0], (int)x->ne[1], (int)x->ne[2],
                                    (int)x->ne[3], t->iparam[0], (float*)out));
                break;
            }
            default:
                throw std::runtime_error(std::string("HipRuntime: unsupported op ") + std::to_string((int)t->op));
        }

        if (timed) {
            float ms = 0.f;
            I.check(mgh_timer_stop(I.ctx, &ms));
            // an FC that also normalized its rows (its Norm node launched nothing) is its own entry
            auto& e = I.prof[ln_pair.count(t) && ln_done.count(ln_pair.at(t)) ? "MulMat(q)+Norm" : op_name(t)];
            e.first++;
            e.second += ms;
        }
        // a conv whose Add nodes were absorbed leaves the chain's last node in its buffer: that
        // node is the one read back (the conv's own value never exists on its own)
        if (dump_named) dump_node(t->op == Op::Conv2D && cfuse.count(t) ? cfuse.at(t).out : t);
        release_after(i, t);
    }

    Tensor* outp = g.nodes.back();
    const Tensor* ro = I.root(outp);
    void* result = I.dev(ro);
    if (readback) {
        if (!outp->data) throw std::runtime_error("HipRuntime: output node has no host storage");
        I.check(mgh_d2h(I.ctx, outp->data, result, outp->nbytes()));
    } else {
        I.held = result;                                           // kept until the next compute
    }
    I.bound.clear();
    for (auto& kv : I.addr)                                        // computed buffers back to the pool
        if (kv.first->op != Op::None && kv.second && kv.second != I.held && !fa_target.count(kv.first) &&
            !(I.owner.count(kv.first) && I.owner.at(kv.first) != kv.first)) {
            I.give(kv.second);
            kv.second = nullptr;
        }
    for (auto& kv : I.codes) {
        I.give(kv.second.q);
        I.give(kv.second.dx);
        I.give(kv.second.sx);
    }
    I.codes.clear();
    I.addr.clear();
    return readback ? nullptr : result;
}

}  // namespace mg
