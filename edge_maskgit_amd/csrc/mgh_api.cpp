// mgh_api.cpp — the C ABI (include/mgh.h): argument validation, contexts, dispatch.
#include "../../include/mgh.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "mgh_kernels.h"

struct mgh_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct mgh_ctx {
    int device = 0;
    bool capturing = false;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::string err;
    std::string name;
    // grow-on-demand activation scratch for mgh_gemm_q_f32in (qx | dx | sx)
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // grow-on-demand split-K workspace of the packed GEMM
    void* qp_ws = nullptr;
    size_t qp_ws_bytes = 0;
    // buffers replaced by a larger one: a captured graph may still reference them, so they
    // are released only with the context
    std::vector<void*> retired;
};

namespace {

int fail(mgh_ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    return code;
}

int hip_fail(mgh_ctx* c, hipError_t e, const char* what) {
    return fail(c, MGH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define MGH_HIP(ctx, expr, what)                                  \
    do {                                                          \
        hipError_t e_ = (expr);                                   \
        if (e_ != hipSuccess) return hip_fail((ctx), e_, (what)); \
    } while (0)

int set_dev(mgh_ctx* c) {
    MGH_HIP(c, hipSetDevice(c->device), "hipSetDevice");
    return MGH_OK;
}

int check_quant_shape(mgh_ctx* c, int wtype, int N, int K, int M) {
    if (wtype != MGH_WTYPE_Q8_0 && wtype != MGH_WTYPE_Q4_K)
        return fail(c, MGH_ERR_ARG, "wtype must be MGH_WTYPE_Q8_0 (8) or MGH_WTYPE_Q4_K (12)");
    if (N <= 0 || K <= 0 || M < 0) return fail(c, MGH_ERR_ARG, "shape must have N>0, K>0, M>=0");
    if (K % 32) return fail(c, MGH_ERR_ARG, "K must be a multiple of 32 (ggml block size)");
    if (wtype == MGH_WTYPE_Q8_0 && K % 64)
        return fail(c, MGH_ERR_UNSUPPORTED, "Q8_0 GEMM needs K % 64 == 0 (dword-aligned block pairs)");
    if (wtype == MGH_WTYPE_Q4_K && K % 256)
        return fail(c, MGH_ERR_ARG, "Q4_K needs K % 256 == 0 (super-block size)");
    return MGH_OK;
}

// Pick the workgroup tile: the larger 128x64 / 64x128 tiles when they still yield >= 2
// workgroups per CU (256 CUs); otherwise 64x64, which maximizes the number of busy SIMDs.
// (128x128 tiles exceed the register file with the scale outer products in flight.)
mgh::TileCfg pick_tile(int M, int N) {
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if (tiles(128, 64) >= 512) return {2, 1};
    if (tiles(64, 128) >= 512) return {1, 2};
    return {1, 1};
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// fp16-code production kernel: K % 256 == 0, N % 4 == 0, 16-byte aligned w/bias/resid/y.

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Grow-on-demand activation scratch (like the reference's qx_buf/dx_buf,
// mg-opencl.cpp:1125-1134). Not allowed while a graph is being captured. The replaced
// buffer is retired, not freed (stream order keeps it valid for queued work and graphs).
int ensure_scratch(mgh_ctx* c, size_t need) {
    if (c->scratch_bytes >= need) return MGH_OK;
    if (c->capturing)
        return fail(c, MGH_ERR_ARG, "activation scratch must grow, which is not allowed during "
                                    "graph capture (run the call once before capturing)");
    need = std::max(need, 2 * c->scratch_bytes);
    if (c->scratch) c->retired.push_back(c->scratch);
    c->scratch = nullptr;
    c->scratch_bytes = 0;
    MGH_HIP(c, hipMalloc(&c->scratch, need), "hipMalloc(scratch)");
    c->scratch_bytes = need;
    return MGH_OK;
}

// Split-K workspace of the packed GEMM (partial tiles).
int ensure_qp_ws(mgh_ctx* c, size_t need) {
    if (c->qp_ws_bytes >= need) return MGH_OK;
    if (c->capturing)
        return fail(c, MGH_ERR_ARG, "split-K workspace must grow, which is not allowed during graph "
                                    "capture (run the call once before capturing)");
    need = std::max(need, 2 * c->qp_ws_bytes);
    if (c->qp_ws) c->retired.push_back(c->qp_ws);
    c->qp_ws = nullptr;
    c->qp_ws_bytes = 0;
    MGH_HIP(c, hipMalloc(&c->qp_ws, need), "hipMalloc(qp_ws)");
    c->qp_ws_bytes = need;
    return MGH_OK;
}

// The packed GEMM with its split-K plan (workspace from the context).
int run_gemm_qp(mgh_ctx* c, int wtype, mgh::GemmArgs a, bool dbg) {
    if (!dbg) {
        const mgh::QpPlan p = mgh::gemm_qp_plan(a.M, a.N, a.K);
        a.splits = p.splits;
        if (p.splits > 1) {
            if (int r = ensure_qp_ws(c, p.ws_bytes)) return r;
            a.ws = (float*)c->qp_ws;
        }
    }
    MGH_HIP(c, mgh::launch_gemm_qp(wtype, a, dbg, c->stream), dbg ? "k_gemm_qp(debug)" : "k_gemm_qp");
    return MGH_OK;
}

// The fp16 dequantize-fused GEMM with its split-K plan (workspace from the context).
int run_gemm_h16(mgh_ctx* c, mgh::GemmH16Args a) {
    if (mgh::use_gemv_h16(a.M, a.K)) {
        MGH_HIP(c, mgh::launch_gemv_h16(a, c->stream), "k_gemv_fc");
        return MGH_OK;
    }
    const mgh::H16Plan p = mgh::gemm_h16_plan(a.M, a.N, a.K, a.xf != nullptr, a.wq);
    a.splits = p.splits;
    if (p.splits > 1) {
        if (int r = ensure_qp_ws(c, p.ws_bytes)) return r;
        a.ws = (float*)c->qp_ws;
    }
    MGH_HIP(c, mgh::launch_gemm_h16(p, a, c->stream), "k_gemm_fc");
    return MGH_OK;
}

int check_h16(mgh_ctx* c, const char* fn, const void* wp, int N, int K, const void* x, int M,
              const float* bias, int act, const float* resid, const float* y, bool y_optional = false) {
    if (N <= 0 || K <= 0 || M < 0) return fail(c, MGH_ERR_ARG, std::string(fn) + ": shape must have N>0, K>0, M>=0");
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "act must be 0 (none), 1 (gelu) or 2 (silu)");
    if (K % 64) return fail(c, MGH_ERR_UNSUPPORTED, std::string(fn) + ": needs K % 64 == 0");
    if (N % 4) return fail(c, MGH_ERR_UNSUPPORTED, std::string(fn) + ": needs N % 4 == 0");
    if (N > mgh::kFcMaxN) return fail(c, MGH_ERR_UNSUPPORTED, std::string(fn) + ": needs N <= 2097152");
    if (M == 0) return MGH_OK;
    if (!wp || !x || (!y && !y_optional)) return fail(c, MGH_ERR_ARG, std::string(fn) + ": null pointer");
    if (!aligned16(wp) || !aligned16(x) || !aligned16(bias) || !aligned16(resid) || !aligned16(y))
        return fail(c, MGH_ERR_ARG, std::string(fn) + ": operands must be 16-byte aligned");
    return MGH_OK;
}


// The raw-block int8-dot GEMM (GGUF blocks as stored, int8 activation codes)
hipError_t launch_gemm(int wtype, const mgh::GemmArgs& a, bool dbg, hipStream_t s) {
    return mgh::launch_gemm_q_i8(wtype, a, pick_tile(a.M, a.N), dbg, s);
}

// Activation operands + packed GEMM on fp32 input, activation scratch at `base`
// (x16/codes [M][K] fp16 | dx [M][T] | sx or ux [M][T]).
int packed_f32in(mgh_ctx* c, int algo, int wtype, const void* wp, int N, int K, const float* x,
                 int M, const float* bias, int act, const float* resid, float* y, char* base) {
    const size_t T = (size_t)K / 32;
    const size_t q_b = round256((size_t)M * K * 2), d_b = round256((size_t)M * T * 4);
    void* q = base;
    float* dx = (float*)(base + q_b);
    void* s4 = base + q_b + d_b;
    mgh::GemmArgs a{};
    a.w = (const uint8_t*)wp; a.qx16 = q; a.dx = dx;
    a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    if (algo == MGH_ALGO_DEQ_F16) {
        MGH_HIP(c, mgh::launch_round_act_f16(x, (_Float16*)q, dx, (float*)s4, M, K, c->stream),
                "k_round_act_f16");
        a.ux = (const float*)s4;
    } else {
        MGH_HIP(c, mgh::launch_quantize_act_q8_f16(x, (_Float16*)q, dx, (int32_t*)s4, M, K, c->stream),
                "k_quantize_act_q8<f16>");
        a.sx = (const int32_t*)s4;
    }
    return run_gemm_qp(c, wtype, a, false);
}

size_t packed_f32in_scratch(int M, int K) {
    const size_t T = (size_t)K / 32;
    return round256((size_t)M * K * 2) + 2 * round256((size_t)M * T * 4);
}

}  // namespace

extern "C" {

int mgh_version(void) { return 1; }

int mgh_create(int device_ordinal, mgh_ctx** out) {
    if (!out) return MGH_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device_ordinal < 0 || device_ordinal >= n)
        return MGH_ERR_NO_DEVICE;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device_ordinal) != hipSuccess) return MGH_ERR_NO_DEVICE;
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) return MGH_ERR_NO_DEVICE;
    mgh_ctx* c = new mgh_ctx();
    c->device = device_ordinal;
    c->name = p.name;
    c->name += " (";
    c->name += p.gcnArchName;
    c->name += ")";
    if (hipSetDevice(device_ordinal) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess) {
        mgh_destroy(c);
        return MGH_ERR_HIP;
    }
    *out = c;
    return MGH_OK;
}

void mgh_destroy(mgh_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->scratch) (void)hipFree(c->scratch);
    if (c->qp_ws) (void)hipFree(c->qp_ws);
    for (void* p : c->retired) (void)hipFree(p);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char* mgh_last_error(const mgh_ctx* c) { return c ? c->err.c_str() : "null context"; }
const char* mgh_device_name(const mgh_ctx* c) { return c ? c->name.c_str() : ""; }

int mgh_alloc(mgh_ctx* c, size_t bytes, void** out) {
    if (!c || !out) return fail(c, MGH_ERR_ARG, "mgh_alloc: null argument");
    if (int r = set_dev(c)) return r;
    *out = nullptr;
    if (bytes == 0) bytes = 256;
    MGH_HIP(c, hipMalloc(out, bytes), "hipMalloc");
    return MGH_OK;
}

int mgh_free(mgh_ctx* c, void* p) {
    if (!c) return MGH_ERR_ARG;
    if (!p) return MGH_OK;
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    MGH_HIP(c, hipFree(p), "hipFree");
    return MGH_OK;
}

int mgh_h2d(mgh_ctx* c, void* d, const void* h, size_t n) {
    if (!c || (n && (!d || !h))) return fail(c, MGH_ERR_ARG, "mgh_h2d: null argument");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    MGH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return MGH_OK;
}

int mgh_d2h(mgh_ctx* c, void* h, const void* d, size_t n) {
    if (!c || (n && (!d || !h))) return fail(c, MGH_ERR_ARG, "mgh_d2h: null argument");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
    MGH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return MGH_OK;
}

int mgh_fill_u32(mgh_ctx* c, void* d, uint32_t v, size_t n) {
    if (!c || (n && !d)) return fail(c, MGH_ERR_ARG, "mgh_fill_u32: null argument");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_fill_u32((uint32_t*)d, v, n, c->stream), "k_fill_u32");
    return MGH_OK;
}

int mgh_sync(mgh_ctx* c) {
    if (!c) return MGH_ERR_ARG;
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return MGH_OK;
}

int mgh_timer_start(mgh_ctx* c) {
    if (!c) return MGH_ERR_ARG;
    MGH_HIP(c, hipEventRecord(c->ev0, c->stream), "hipEventRecord");
    return MGH_OK;
}

int mgh_timer_stop(mgh_ctx* c, float* ms) {
    if (!c || !ms) return fail(c, MGH_ERR_ARG, "mgh_timer_stop: null argument");
    MGH_HIP(c, hipEventRecord(c->ev1, c->stream), "hipEventRecord");
    MGH_HIP(c, hipEventSynchronize(c->ev1), "hipEventSynchronize");
    MGH_HIP(c, hipEventElapsedTime(ms, c->ev0, c->ev1), "hipEventElapsedTime");
    return MGH_OK;
}

int mgh_graph_begin(mgh_ctx* c) {
    if (!c) return MGH_ERR_ARG;
    if (c->capturing) return fail(c, MGH_ERR_ARG, "mgh_graph_begin: already capturing");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    c->capturing = true;
    return MGH_OK;
}

int mgh_graph_end(mgh_ctx* c, mgh_graph** out) {
    if (!c || !out) return fail(c, MGH_ERR_ARG, "mgh_graph_end: null argument");
    if (!c->capturing) return fail(c, MGH_ERR_ARG, "mgh_graph_end: not capturing");
    c->capturing = false;
    mgh_graph* g = new mgh_graph();
    hipError_t e = hipStreamEndCapture(c->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        mgh_graph_destroy(g);
        return hip_fail(c, e, "graph capture/instantiate");
    }
    *out = g;
    return MGH_OK;
}

int mgh_graph_launch(mgh_ctx* c, mgh_graph* g) {
    if (!c || !g || !g->exec) return fail(c, MGH_ERR_ARG, "mgh_graph_launch: null argument");
    MGH_HIP(c, hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
    return MGH_OK;
}

void mgh_graph_destroy(mgh_graph* g) {
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

int mgh_quantize_act_q8(mgh_ctx* c, const float* x, int M, int K, int8_t* qx, float* dx, int32_t* sx) {
    if (!c) return MGH_ERR_ARG;
    if (M < 0 || K <= 0 || K % 32) return fail(c, MGH_ERR_ARG, "quantize_act_q8: need M>=0, K>0, K%32==0");
    if (M == 0) return MGH_OK;
    if (!x || !qx || !dx) return fail(c, MGH_ERR_ARG, "quantize_act_q8: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_quantize_act_q8(x, qx, dx, sx, M, K, c->stream), "k_quantize_act_q8");
    return MGH_OK;
}

int mgh_gemm_q(mgh_ctx* c, int wtype, const void* w, int N, int K, const int8_t* qx,
               const float* dx, const int32_t* sx, int M, const float* bias, int act,
               const float* resid, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_quant_shape(c, wtype, N, K, M)) return r;
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "act must be 0 (none), 1 (gelu) or 2 (silu)");
    if (M == 0) return MGH_OK;
    if (!w || !qx || !dx || !y) return fail(c, MGH_ERR_ARG, "gemm_q: null pointer");
    if (wtype == MGH_WTYPE_Q4_K && !sx) return fail(c, MGH_ERR_ARG, "gemm_q: Q4_K needs block sums sx");
    if (int r = set_dev(c)) return r;
    mgh::GemmArgs a{};
    a.w = (const uint8_t*)w; a.qx = qx; a.dx = dx; a.sx = sx;
    a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    MGH_HIP(c, launch_gemm(wtype, a, false, c->stream), "k_gemm_q_i8");
    return MGH_OK;
}

int mgh_quantize_act_q8_codes16(mgh_ctx* c, const float* x, int M, int K, uint16_t* qx16,
                                float* dx, int32_t* sx) {
    if (!c) return MGH_ERR_ARG;
    if (M < 0 || K <= 0 || K % 32) return fail(c, MGH_ERR_ARG, "quantize_act_q8_codes16: need M>=0, K>0, K%32==0");
    if (M == 0) return MGH_OK;
    if (!x || !qx16 || !dx) return fail(c, MGH_ERR_ARG, "quantize_act_q8_codes16: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_quantize_act_q8_f16(x, (_Float16*)qx16, dx, sx, M, K, c->stream),
            "k_quantize_act_q8<f16>");
    return MGH_OK;
}

size_t mgh_packed_weight_bytes(int wtype, int N, int K) {
    if ((wtype != MGH_WTYPE_Q8_0 && wtype != MGH_WTYPE_Q4_K) || N <= 0 || K <= 0 || K % 32) return 0;
    if (wtype == MGH_WTYPE_Q4_K && K % 256) return 0;
    return mgh::packed_weight_bytes(wtype, N, K);
}

int mgh_pack_weights(mgh_ctx* c, int wtype, const void* w, int N, int K, void* wp) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_quant_shape(c, wtype, N, K, 0)) return r;
    if (!w || !wp) return fail(c, MGH_ERR_ARG, "pack_weights: null pointer");
    if (!aligned16(wp)) return fail(c, MGH_ERR_ARG, "pack_weights: d_packed must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_pack_weights(wtype, w, wp, N, K, c->stream), "k_pack_w");
    return MGH_OK;
}

namespace {
// Packed weights and outputs: shape rules, N % 4 == 0, 16-byte aligned wp/bias/resid/y.
int check_packed_w(mgh_ctx* c, const std::string& f, int wtype, const void* wp, int N, int K, int M,
                   const float* bias, const float* resid, const float* y, bool need_y) {
    if (int r = check_quant_shape(c, wtype, N, K, M)) return r;
    if (M == 0) return MGH_OK;
    if (!wp || (need_y && !y)) return fail(c, MGH_ERR_ARG, f + ": null pointer");
    if (N % 4) return fail(c, MGH_ERR_UNSUPPORTED, f + ": needs N % 4 == 0");
    if (!aligned16(wp) || !aligned16(bias) || !aligned16(resid) || !aligned16(y))
        return fail(c, MGH_ERR_ARG, f + ": d_wp, d_bias, d_resid and d_y must be 16-byte aligned");
    return MGH_OK;
}

// fp16-code activation operands: qx16 16-byte aligned; dx 4-byte aligned (16-byte, with sx,
// for Q4_K, whose min term reads them as float4).
int check_act16(mgh_ctx* c, const std::string& f, int wtype, const uint16_t* qx16, const float* dx,
                const int32_t* sx, bool need_scales) {
    if (!qx16 || (need_scales && !dx)) return fail(c, MGH_ERR_ARG, f + ": null pointer");
    if (need_scales && wtype == MGH_WTYPE_Q4_K && !sx)
        return fail(c, MGH_ERR_ARG, f + ": Q4_K needs block sums sx");
    if (!aligned16(qx16)) return fail(c, MGH_ERR_ARG, f + ": d_qx16 must be 16-byte aligned");
    if (need_scales && (((uintptr_t)dx & 3u) || (wtype == MGH_WTYPE_Q4_K && (!aligned16(dx) || !aligned16(sx)))))
        return fail(c, MGH_ERR_ARG, f + ": d_dx must be 4-byte aligned (16-byte, with d_sx, for Q4_K)");
    return MGH_OK;
}
}  // namespace

int mgh_gemm_q_packed(mgh_ctx* c, int wtype, const void* wp, int N, int K, const uint16_t* qx16,
                      const float* dx, const int32_t* sx, int M, const float* bias, int act,
                      const float* resid, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "act must be 0 (none), 1 (gelu) or 2 (silu)");
    if (int r = check_packed_w(c, "gemm_q_packed", wtype, wp, N, K, M, bias, resid, y, true)) return r;
    if (M == 0) return MGH_OK;
    if (int r = check_act16(c, "gemm_q_packed", wtype, qx16, dx, sx, true)) return r;
    if (int r = set_dev(c)) return r;
    mgh::GemmArgs a{};
    a.w = (const uint8_t*)wp; a.qx16 = qx16; a.dx = dx; a.sx = sx;
    a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    return run_gemm_qp(c, wtype, a, false);
}

int mgh_debug_block_dots_packed(mgh_ctx* c, int wtype, const void* wp, int N, int K,
                                const uint16_t* qx16, int M, int32_t* out) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_packed_w(c, "debug_block_dots_packed", wtype, wp, N, K, M, nullptr, nullptr,
                               nullptr, false)) return r;
    if (M == 0) return MGH_OK;
    if (int r = check_act16(c, "debug_block_dots_packed", wtype, qx16, nullptr, nullptr, false)) return r;
    if (!out) return fail(c, MGH_ERR_ARG, "debug_block_dots_packed: null pointer");
    if (int r = set_dev(c)) return r;
    mgh::GemmArgs a{};
    a.w = (const uint8_t*)wp; a.qx16 = qx16; a.dots = out;
    a.M = M; a.N = N; a.K = K;
    return run_gemm_qp(c, wtype, a, true);
}

int mgh_gemm_q_packed_f32in(mgh_ctx* c, int algo, int wtype, const void* wp, int N, int K,
                            const float* x, int M, const float* bias, int act, const float* resid,
                            float* y) {
    if (!c) return MGH_ERR_ARG;
    if (algo != MGH_ALGO_AUTO && algo != MGH_ALGO_INT8 && algo != MGH_ALGO_DEQ_F16)
        return fail(c, MGH_ERR_ARG, "algo must be MGH_ALGO_AUTO, _INT8 or _DEQ_F16");
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "act must be 0 (none), 1 (gelu) or 2 (silu)");
    // the activation operands are built in aligned context scratch
    if (algo == MGH_ALGO_AUTO) algo = MGH_ALGO_DEQ_F16;
    if (int r = check_packed_w(c, "gemm_q_packed_f32in", wtype, wp, N, K, M, bias, resid, y, true)) return r;
    if (M == 0) return MGH_OK;
    if (!x) return fail(c, MGH_ERR_ARG, "gemm_q_packed_f32in: null pointer");
    if ((uintptr_t)x & 15u) return fail(c, MGH_ERR_ARG, "gemm_q_packed_f32in: d_x must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    if (int r = ensure_scratch(c, packed_f32in_scratch(M, K))) return r;
    return packed_f32in(c, algo, wtype, wp, N, K, x, M, bias, act, resid, y, (char*)c->scratch);
}

int mgh_gemm_q_f32in(mgh_ctx* c, int algo, int wtype, const void* w, int N, int K, const float* x,
                     int M, const float* bias, int act, const float* resid, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_quant_shape(c, wtype, N, K, M)) return r;
    if (algo != MGH_ALGO_AUTO && algo != MGH_ALGO_INT8 && algo != MGH_ALGO_DEQ_F16)
        return fail(c, MGH_ERR_ARG, "algo must be MGH_ALGO_AUTO, _INT8 or _DEQ_F16");
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "act must be 0 (none), 1 (gelu) or 2 (silu)");
    if (algo == MGH_ALGO_AUTO) algo = MGH_ALGO_DEQ_F16;
    if (M == 0) return MGH_OK;
    if (!x || !w || !y) return fail(c, MGH_ERR_ARG, "gemm_q_f32in: null pointer");
    if (int r = set_dev(c)) return r;
    if (algo == MGH_ALGO_DEQ_F16) {
        // weights packed into scratch for this call, then the packed kernel
        if (N % 4 || ((uintptr_t)x & 15u) || !aligned16(bias) || !aligned16(resid) || !aligned16(y))
            return fail(c, MGH_ERR_UNSUPPORTED, "gemm_q_f32in(DEQ_F16) needs N % 4 == 0 and 16-byte "
                                                "aligned x/bias/resid/y");
        const size_t wb = round256(mgh::packed_weight_bytes(wtype, N, K));
        if (int r = ensure_scratch(c, wb + packed_f32in_scratch(M, K))) return r;
        MGH_HIP(c, mgh::launch_pack_weights(wtype, w, c->scratch, N, K, c->stream), "k_pack_w");
        return packed_f32in(c, algo, wtype, c->scratch, N, K, x, M, bias, act, resid, y,
                            (char*)c->scratch + wb);
    }
    const size_t nb = (size_t)K / 32;
    const size_t q_b = round256((size_t)M * K);
    const size_t d_b = round256((size_t)M * nb * 4);
    if (int r = ensure_scratch(c, q_b + 2 * d_b)) return r;
    int8_t* q = (int8_t*)c->scratch;
    float* dx = (float*)((char*)c->scratch + q_b);
    int32_t* sx = (int32_t*)((char*)c->scratch + q_b + d_b);
    if (int r = mgh_quantize_act_q8(c, x, M, K, q, dx, sx)) return r;
    return mgh_gemm_q(c, wtype, w, N, K, q, dx, sx, M, bias, act, resid, y);
}

int mgh_layernorm_affine(mgh_ctx* c, const float* x, const float* g, const float* b, int rows, int D,
                         float eps, float* y, int emit, void* codes, float* dx, void* s4) {
    if (!c) return MGH_ERR_ARG;
    if (rows < 0 || D <= 0) return fail(c, MGH_ERR_ARG, "layernorm_affine: need rows >= 0, D > 0");
    if (D % 256 || D > 2048) return fail(c, MGH_ERR_UNSUPPORTED, "layernorm_affine: needs D % 256 == 0 and D <= 2048");
    if (emit < 0 || emit > 2) return fail(c, MGH_ERR_ARG, "layernorm_affine: emit must be 0, 1 or 2");
    if (rows == 0) return MGH_OK;
    if (!x || !g || !b || !y) return fail(c, MGH_ERR_ARG, "layernorm_affine: null pointer");
    if (emit && (!codes || (emit == 1 && (!dx || !s4))))
        return fail(c, MGH_ERR_ARG, "layernorm_affine: emit needs d_codes (and d_dx, d_s4 for INT8)");
    if (!aligned16(x) || !aligned16(y) || !aligned16(g) || !aligned16(b) || !aligned16(codes) ||
        ((uintptr_t)dx & 3u) || ((uintptr_t)s4 & 3u))
        return fail(c, MGH_ERR_ARG, "layernorm_affine: x/y/gamma/beta/codes must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_layernorm_affine(x, g, b, y, rows, D, eps, emit, codes, dx, s4, c->stream),
            "k_layernorm_affine");
    return MGH_OK;
}

}  // extern "C"

namespace {

int flash_attn(mgh_ctx* c, const void* q, const void* k, const void* v, bool in16, const int64_t st[4], int D,
               int S, int H, int B, float scale, float* o, _Float16* o16, const int64_t ost[4]) {
    if (!c) return MGH_ERR_ARG;
    if (S < 0 || H < 0 || B < 0) return fail(c, MGH_ERR_ARG, "flash_attn: negative shape");
    if (D != 16 && D != 32 && D != 48 && D != 64)
        return fail(c, MGH_ERR_UNSUPPORTED, "flash_attn: D must be 16, 32, 48 or 64");
    if (S == 0 || H == 0 || B == 0) return MGH_OK;
    if (!q || !k || !v || (!o && !o16) || (o && o16) || !st) return fail(c, MGH_ERR_ARG, "flash_attn: null pointer");
    if (H > 65535 || B > 65535) return fail(c, MGH_ERR_UNSUPPORTED, "flash_attn: H and B must be <= 65535");
    if (in16) {
        auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
        if (S > 512 || st[0] != 1 || st[1] % 4 || st[2] % 4 || st[3] % 4 || !al(q) || !al(k) || !al(v) ||
            !(scale > 0.f))
            return fail(c, MGH_ERR_UNSUPPORTED, "flash_attn_f16in: needs S <= 512, unit d stride, other strides "
                                                "multiples of 4, 16-byte aligned q/k/v and scale > 0");
    }
    if (int r = set_dev(c)) return r;
    mgh::FaArgs a{};
    if (in16) {
        a.q16 = (const _Float16*)q; a.k16 = (const _Float16*)k; a.v16 = (const _Float16*)v;
    } else {
        a.q = (const float*)q; a.k = (const float*)k; a.v = (const float*)v;
    }
    a.o = o; a.o16 = o16;
    for (int i = 0; i < 4; i++) a.st[i] = st[i];
    if (ost) {
        for (int i = 0; i < 4; i++) a.os[i] = ost[i];
    } else {
        a.os[0] = 1; a.os[1] = D; a.os[2] = (int64_t)D * S; a.os[3] = (int64_t)D * S * H;
    }
    a.S = S; a.H = H; a.B = B; a.scale = scale;
    MGH_HIP(c, mgh::launch_flash_attn_f16kv(a, D, c->stream), "k_flash_attn_f16kv");
    return MGH_OK;
}

}  // namespace

extern "C" {

int mgh_flash_attn_f16kv(mgh_ctx* c, const float* q, const float* k, const float* v,
                         const int64_t st[4], int D, int S, int H, int B, float scale, float* o,
                         const int64_t ost[4]) {
    return flash_attn(c, q, k, v, false, st, D, S, H, B, scale, o, nullptr, ost);
}

int mgh_flash_attn_f16kv_o16(mgh_ctx* c, const float* q, const float* k, const float* v,
                             const int64_t st[4], int D, int S, int H, int B, float scale, void* o16,
                             const int64_t ost[4]) {
    return flash_attn(c, q, k, v, false, st, D, S, H, B, scale, nullptr, (_Float16*)o16, ost);
}

int mgh_flash_attn_f16in(mgh_ctx* c, const void* q16, const void* k16, const void* v16,
                         const int64_t st[4], int D, int S, int H, int B, float scale, float* o, void* o16,
                         const int64_t ost[4]) {
    return flash_attn(c, q16, k16, v16, true, st, D, S, H, B, scale, o, (_Float16*)o16, ost);
}

int mgh_gemm_f32(mgh_ctx* c, const float* w, int N, int K, const float* x, int M, const float* bias,
                 int act, const float* resid, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (N <= 0 || K <= 0 || M < 0) return fail(c, MGH_ERR_ARG, "gemm_f32: shape must have N>0, K>0, M>=0");
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "act must be 0 (none), 1 (gelu) or 2 (silu)");
    if (K % 32) return fail(c, MGH_ERR_UNSUPPORTED, "gemm_f32: needs K % 32 == 0");
    if (M == 0) return MGH_OK;
    if (!w || !x || !y) return fail(c, MGH_ERR_ARG, "gemm_f32: null pointer");
    if (!aligned16(w) || !aligned16(x)) return fail(c, MGH_ERR_ARG, "gemm_f32: w and x must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    mgh::GemmF32Args a{};
    a.w = w; a.x = x; a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    MGH_HIP(c, mgh::launch_gemm_f32(a, c->stream), "k_gemm_f32");
    return MGH_OK;
}

int mgh_get_rows(mgh_ctx* c, const float* a, int64_t E, int64_t R, const int32_t* ids, int64_t n, float* out) {
    if (!c) return MGH_ERR_ARG;
    if (E < 0 || R <= 0 || n < 0) return fail(c, MGH_ERR_ARG, "get_rows: need E >= 0, R > 0, n >= 0");
    if (n == 0 || E == 0) return MGH_OK;
    if (n > 65535) return fail(c, MGH_ERR_UNSUPPORTED, "get_rows: at most 65535 rows per call");
    if (!a || !ids || !out) return fail(c, MGH_ERR_ARG, "get_rows: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_get_rows(a, E, R, ids, n, out, c->stream), "k_get_rows");
    return MGH_OK;
}

int mgh_add(mgh_ctx* c, const float* a, const float* b, int64_t nb, float* out, int64_t n) {
    if (!c) return MGH_ERR_ARG;
    if (n < 0 || nb <= 0 || (n % nb)) return fail(c, MGH_ERR_ARG, "add: need nb > 0 dividing n");
    if (n == 0) return MGH_OK;
    if (!a || !b || !out) return fail(c, MGH_ERR_ARG, "add: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_add_bcast(a, b, nb, out, n, c->stream), "k_add_bcast");
    return MGH_OK;
}

int mgh_copy_strided(mgh_ctx* c, const float* a, const int64_t ne[4], const int64_t st[4], float* out) {
    if (!c) return MGH_ERR_ARG;
    if (!ne || !st) return fail(c, MGH_ERR_ARG, "copy_strided: null shape");
    mgh::CopyArgs ca{};
    for (int i = 0; i < 4; i++) {
        if (ne[i] <= 0) return fail(c, MGH_ERR_ARG, "copy_strided: shape must be positive");
        ca.ne[i] = ne[i];
        ca.st[i] = st[i];
    }
    if (!a || !out) return fail(c, MGH_ERR_ARG, "copy_strided: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_copy4d(a, ca, out, c->stream), "k_copy4d");
    return MGH_OK;
}

int mgh_softmax(mgh_ctx* c, const float* x, int64_t rows, int D, float scale, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (rows < 0 || D < 0) return fail(c, MGH_ERR_ARG, "softmax: need rows >= 0, D >= 0");
    if (rows == 0 || D == 0) return MGH_OK;
    if (!x || !y) return fail(c, MGH_ERR_ARG, "softmax: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_softmax_rows(x, rows, D, scale, y, c->stream), "k_softmax_rows");
    return MGH_OK;
}

int mgh_binary(mgh_ctx* c, int op, const float* a, const int64_t as[4], const float* b, const int64_t bne[4],
               const int64_t bs[4], const int64_t ne[4], float* out) {
    if (!c) return MGH_ERR_ARG;
    if (op != 0 && op != 1) return fail(c, MGH_ERR_ARG, "binary: op must be 0 (add) or 1 (mul)");
    if (!as || !bne || !bs || !ne) return fail(c, MGH_ERR_ARG, "binary: null shape");
    mgh::BinaryArgs p{};
    for (int i = 0; i < 4; i++) {
        if (ne[i] <= 0) return fail(c, MGH_ERR_ARG, "binary: shape must be positive");
        if (bne[i] != ne[i] && bne[i] != 1) return fail(c, MGH_ERR_ARG, "binary: b dims must equal the output's or be 1");
        p.ne[i] = ne[i];
        p.as[i] = as[i];
        p.bne[i] = bne[i];
        p.bs[i] = bs[i];
    }
    if (!a || !b || !out) return fail(c, MGH_ERR_ARG, "binary: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_binary(op, a, b, p, out, c->stream), "k_binary");
    return MGH_OK;
}

int mgh_scale(mgh_ctx* c, const float* x, int64_t n, float s, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (n < 0) return fail(c, MGH_ERR_ARG, "scale: need n >= 0");
    if (n == 0) return MGH_OK;
    if (!x || !y) return fail(c, MGH_ERR_ARG, "scale: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_unary(0, x, n, s, y, c->stream), "k_unary");
    return MGH_OK;
}

int mgh_unary(mgh_ctx* c, int act, const float* x, int64_t n, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (act != MGH_ACT_GELU && act != MGH_ACT_SILU) return fail(c, MGH_ERR_ARG, "unary: act must be GELU (1) or SiLU (2)");
    if (n < 0) return fail(c, MGH_ERR_ARG, "unary: need n >= 0");
    if (n == 0) return MGH_OK;
    if (!x || !y) return fail(c, MGH_ERR_ARG, "unary: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_unary(act, x, n, 0.0f, y, c->stream), "k_unary");
    return MGH_OK;
}

namespace {

int conv_shape(mgh_ctx* c, int IW, int IH, int IC, int N, int KW, int KH, int OC, int stride, int pad, int64_t* OW,
               int64_t* OH) {
    if (IW <= 0 || IH <= 0 || IC <= 0 || N < 0 || KW <= 0 || KH <= 0 || OC <= 0 || stride <= 0 || pad < 0)
        return fail(c, MGH_ERR_ARG, "conv2d: need positive sizes, stride >= 1, pad >= 0");
    if (IW + 2 * (int64_t)pad < KW || IH + 2 * (int64_t)pad < KH)
        return fail(c, MGH_ERR_ARG, "conv2d: kernel larger than the padded input");
    *OW = ((int64_t)IW + 2 * pad - KW) / stride + 1;
    *OH = ((int64_t)IH + 2 * pad - KH) / stride + 1;
    // grids: pixel tiles of 64 or 128 (or one thread per pixel) in x, N (x splits < 1024) in z
    if ((int64_t)IW * IH > INT32_MAX || *OW * *OH > ((int64_t)1 << 30) || (int64_t)IC * KW * KH > INT32_MAX ||
        (int64_t)N > 65535 || *OW * *OH * N > ((int64_t)1 << 31))
        return fail(c, MGH_ERR_UNSUPPORTED, "conv2d: shape too large");
    return MGH_OK;
}

bool conv_packed_path(int IC, int OC) { return IC % 16 == 0 && OC > 0; }

}  // namespace

int mgh_conv2d_ex(mgh_ctx* c, const float* in, int IW, int IH, int IC, int N, const float* ker, const float* wpk,
                  int KW, int KH, int OC, int stride, int pad, const float* bias, const float* resid, float* out) {
    if (!c) return MGH_ERR_ARG;
    int64_t OW = 0, OH = 0;
    if (int r = conv_shape(c, IW, IH, IC, N, KW, KH, OC, stride, pad, &OW, &OH)) return r;
    if (N == 0) return MGH_OK;
    if (!in || !out || (!ker && !wpk)) return fail(c, MGH_ERR_ARG, "conv2d: null pointer");
    if (!aligned16(out) || (resid && !aligned16(resid)) || (wpk && !aligned16(wpk)))
        return fail(c, MGH_ERR_ARG, "conv2d: d_out, d_resid and d_packed must be 16-byte aligned");
    const bool packed = conv_packed_path(IC, OC);
    if (!ker && !packed)
        return fail(c, MGH_ERR_ARG, "conv2d: this shape runs on the reference-layout kernel: pass d_ker");
    if (int r = set_dev(c)) return r;
    const int M = (int)(OW * OH), K = IC * KW * KH;
    if (!packed) {
        mgh::ConvArgs a{in, ker, out, IW, IH, IC, (int)OW, (int)OH, OC, KW, KH, stride, pad, N, bias, resid};
        MGH_HIP(c, mgh::launch_conv2d_f32(a, c->stream), "k_conv2d_f32");
        return MGH_OK;
    }
    if (!wpk) {                          // tap-major copy of the weights in the context scratch
        if (int r = ensure_scratch(c, (size_t)OC * K * sizeof(float))) return r;
        MGH_HIP(c, mgh::launch_conv_pack(ker, (float*)c->scratch, IC, KW * KH, OC, c->stream), "k_conv_pack");
        wpk = (const float*)c->scratch;
    }
    if (int r = ensure_qp_ws(c, mgh::conv_pk_ws_bytes(M, OC, N, K))) return r;
    mgh::ConvPkArgs a{in, wpk, out, bias, resid, IW, IH, IC, (int)OW, (int)OH, OC, KW, KH, stride, pad, N, 1, K};
    MGH_HIP(c, mgh::launch_conv2d_pk(a, (float*)c->qp_ws, c->stream), "k_conv2d_pk");
    return MGH_OK;
}

int mgh_conv2d(mgh_ctx* c, const float* in, int IW, int IH, int IC, int N, const float* ker, int KW, int KH,
               int OC, int stride, int pad, float* out) {
    if (c && !ker && N > 0) return fail(c, MGH_ERR_ARG, "conv2d: null pointer");
    return mgh_conv2d_ex(c, in, IW, IH, IC, N, ker, nullptr, KW, KH, OC, stride, pad, nullptr, nullptr, out);
}

size_t mgh_conv2d_packed_bytes(int KW, int KH, int IC, int OC) {
    if (KW <= 0 || KH <= 0 || IC <= 0 || OC <= 0 || !conv_packed_path(IC, OC)) return 0;
    return (size_t)KW * KH * IC * OC * sizeof(float);
}

int mgh_conv2d_pack_weights(mgh_ctx* c, const float* ker, int KW, int KH, int IC, int OC, float* wpk) {
    if (!c) return MGH_ERR_ARG;
    if (KW <= 0 || KH <= 0 || IC <= 0 || OC <= 0 || (int64_t)IC * KW * KH > INT32_MAX)
        return fail(c, MGH_ERR_ARG, "conv2d_pack_weights: need positive sizes");
    if (!conv_packed_path(IC, OC))
        return fail(c, MGH_ERR_UNSUPPORTED, "conv2d_pack_weights: the packed kernel needs IC % 16 == 0");
    if (!ker || !wpk) return fail(c, MGH_ERR_ARG, "conv2d_pack_weights: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_conv_pack(ker, wpk, IC, KW * KH, OC, c->stream), "k_conv_pack");
    return MGH_OK;
}

size_t mgh_conv2d_i8_weight_bytes(int KW, int KH, int IC, int OC) {
    if (KW <= 0 || KH <= 0 || IC <= 0 || OC <= 0 || (int64_t)IC * KW * KH > INT32_MAX) return 0;
    return mgh::conv_i8_weight_bytes(IC * KW * KH, OC);
}

int mgh_conv2d_i8_pack_weights(mgh_ctx* c, const float* ker, int KW, int KH, int IC, int OC, void* wq) {
    if (!c) return MGH_ERR_ARG;
    if (!mgh_conv2d_i8_weight_bytes(KW, KH, IC, OC))
        return fail(c, MGH_ERR_ARG, "conv2d_i8_pack_weights: need positive sizes");
    if (!ker || !wq) return fail(c, MGH_ERR_ARG, "conv2d_i8_pack_weights: null pointer");
    if (!aligned16(wq)) return fail(c, MGH_ERR_ARG, "conv2d_i8_pack_weights: d_wq must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_conv_quant_w(ker, wq, IC * KW * KH, OC, c->stream), "k_conv_quant_w");
    return MGH_OK;
}

int mgh_conv2d_i8(mgh_ctx* c, const float* in, int IW, int IH, int IC, int N, const void* wq, int KW, int KH,
                  int OC, int stride, int pad, const float* bias, const float* resid, float* out) {
    if (!c) return MGH_ERR_ARG;
    int64_t OW = 0, OH = 0;
    if (int r = conv_shape(c, IW, IH, IC, N, KW, KH, OC, stride, pad, &OW, &OH)) return r;
    if (N == 0) return MGH_OK;
    if (!in || !wq || !out) return fail(c, MGH_ERR_ARG, "conv2d_i8: null pointer");
    if (!aligned16(out) || !aligned16(wq) || (resid && !aligned16(resid)))
        return fail(c, MGH_ERR_ARG, "conv2d_i8: d_wq, d_out and d_resid must be 16-byte aligned");
    const int M = (int)(OW * OH), K = IC * KW * KH;
    // grids: blocks / 4 (quantize pass) and channel tiles (GEMM pass) in y
    if ((K + 31) / 32 > 4 * 65535 || (OC + 15) / 16 > 65535)
        return fail(c, MGH_ERR_UNSUPPORTED, "conv2d_i8: IC*KW*KH or OC too large");
    if (int r = set_dev(c)) return r;
    int8_t* qa = nullptr;
    float* dxa = nullptr;
    if (!mgh::conv_i8_one_pass(IW, IH, IC, (int)OW, (int)OH, OC, KW, KH, N)) {   // two passes: codes in the workspace
        if (int r = ensure_qp_ws(c, mgh::conv_i8_ws_bytes(M, K, N))) return r;
        qa = (int8_t*)c->qp_ws;
        dxa = (float*)(qa + mgh::conv_i8_ws_codes_bytes(M, K, N));
    }
    const int8_t* qw = (const int8_t*)wq;
    const float* dw = (const float*)((const char*)wq + mgh::conv_i8_codes_bytes(K, OC));
    mgh::ConvI8Args a{in, qw, dw, out, bias, resid, qa, dxa, IW, IH, IC, (int)OW, (int)OH, OC, KW, KH, stride, pad, N};
    MGH_HIP(c, mgh::launch_conv2d_i8(a, c->stream), "k_conv2d_i8");
    return MGH_OK;
}

int mgh_group_norm(mgh_ctx* c, const float* x, int W, int H, int C, int N, int groups, float eps,
                   const float* gamma, const float* beta, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (W <= 0 || H <= 0 || C <= 0 || N < 0 || groups <= 0 || C % groups)
        return fail(c, MGH_ERR_ARG, "group_norm: need positive sizes and C % groups == 0");
    if (!(eps >= 0.0f)) return fail(c, MGH_ERR_ARG, "group_norm: eps must be >= 0");
    if ((gamma == nullptr) != (beta == nullptr))
        return fail(c, MGH_ERR_ARG, "group_norm: gamma and beta go together (affine + SiLU) or not at all");
    // grid: x = one workgroup of 256 per 4096-element chunk of a group, y = groups * N
    if ((int64_t)groups * N > 65535 || (int64_t)W * H * (C / groups) > ((int64_t)1 << 32))
        return fail(c, MGH_ERR_UNSUPPORTED, "group_norm: shape too large");
    if (N == 0) return MGH_OK;
    if (!x || !y) return fail(c, MGH_ERR_ARG, "group_norm: null pointer");
    if (int r = set_dev(c)) return r;
    if (int r = ensure_scratch(c, mgh::group_norm_ws_bytes(W, H, C, N, groups))) return r;
    MGH_HIP(c, mgh::launch_group_norm(x, W, H, C, N, groups, eps, gamma, beta, y, c->scratch, c->stream),
            "k_group_norm");
    return MGH_OK;
}

int mgh_upscale(mgh_ctx* c, const float* x, int W, int H, int C, int N, int factor, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (W <= 0 || H <= 0 || C <= 0 || N < 0 || factor <= 0) return fail(c, MGH_ERR_ARG, "upscale: need positive sizes");
    if ((int64_t)W * factor > INT32_MAX || (int64_t)H * factor > INT32_MAX ||
        (double)W * H * factor * factor * C * N > (double)((int64_t)1 << 31))
        return fail(c, MGH_ERR_UNSUPPORTED, "upscale: shape too large");
    if (N == 0) return MGH_OK;
    if (!x || !y) return fail(c, MGH_ERR_ARG, "upscale: null pointer");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_upscale(x, W, H, (int64_t)C * N, factor, y, c->stream), "k_upscale");
    return MGH_OK;
}

int mgh_gemm_f32_batched(mgh_ctx* c, const float* w, const int64_t wne[4], const int64_t ws[4], const float* x,
                         const int64_t xne[4], const int64_t xs[4], const float* bias, int act, const float* resid,
                         float* y) {
    if (!c) return MGH_ERR_ARG;
    if (!wne || !ws || !xne || !xs) return fail(c, MGH_ERR_ARG, "gemm_f32_batched: null shape");
    if (act < 0 || act > 2) return fail(c, MGH_ERR_ARG, "gemm_f32_batched: act must be 0, 1 or 2");
    for (int i = 0; i < 4; i++)
        if (wne[i] <= 0 || xne[i] <= 0) return fail(c, MGH_ERR_ARG, "gemm_f32_batched: shapes must be positive");
    if (wne[0] != xne[0]) return fail(c, MGH_ERR_ARG, "gemm_f32_batched: w and x must share K (ne[0])");
    if ((wne[2] != 1 && wne[2] != xne[2]) || (wne[3] != 1 && wne[3] != xne[3]))
        return fail(c, MGH_ERR_ARG, "gemm_f32_batched: w batch dims must equal x's or be 1");
    if (xne[2] * xne[3] > 65535) return fail(c, MGH_ERR_UNSUPPORTED, "gemm_f32_batched: at most 65535 batches");
    if (!w || !x || !y) return fail(c, MGH_ERR_ARG, "gemm_f32_batched: null pointer");
    mgh::BatchedGemmArgs a{};
    a.w = w; a.x = x; a.bias = bias; a.resid = resid; a.y = y;
    a.K = wne[0]; a.N = wne[1]; a.M = xne[1]; a.B2 = xne[2]; a.B3 = xne[3];
    a.wne2 = wne[2]; a.wne3 = wne[3];
    for (int i = 0; i < 4; i++) { a.ws[i] = ws[i]; a.xs[i] = xs[i]; }
    a.act = act;
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_gemm_f32_batched(a, c->stream), "k_gemm_f32_batched");
    return MGH_OK;
}

size_t mgh_decode_state_bytes(int B) { return B > 0 ? mgh::decode_state_bytes(B) : 0; }

size_t mgh_decode_work_bytes(int B, int S) { return B > 0 && S > 0 ? mgh::decode_work_bytes(B, S) : 0; }

int mgh_decode_init(mgh_ctx* c, int B, const uint64_t* seeds, void* state) {
    if (!c) return MGH_ERR_ARG;
    if (B <= 0) return fail(c, MGH_ERR_ARG, "decode_init: need B > 0");
    if (!seeds || !state) return fail(c, MGH_ERR_ARG, "decode_init: null pointer");
    if ((uintptr_t)state % 8) return fail(c, MGH_ERR_ARG, "decode_init: state must be 8-byte aligned");
    if (int r = set_dev(c)) return r;
    // seed b goes to word 0 of image b's state block; the kernel expands it in place
    const size_t pitch = mgh::decode_state_bytes(1);
    MGH_HIP(c, hipMemcpy2DAsync(state, pitch, seeds, sizeof(uint64_t), sizeof(uint64_t), (size_t)B,
                                hipMemcpyHostToDevice, c->stream), "decode_init: seed copy");
    MGH_HIP(c, mgh::launch_decode_seed(B, state, c->stream), "k_mt64_seed");
    MGH_HIP(c, hipStreamSynchronize(c->stream), "decode_init");
    return MGH_OK;
}

int mgh_decode_step(mgh_ctx* c, void* state, void* work, const float* logits, int B, int S, int V,
                    int codebook, int mask_id, int n_tokens, int step, int n_steps,
                    float choice_temp, int32_t* tokens, int32_t* result) {
    if (!c) return MGH_ERR_ARG;
    if (B <= 0 || S <= 0 || V <= 0) return fail(c, MGH_ERR_ARG, "decode_step: need B, S, V > 0");
    if (S > 512) return fail(c, MGH_ERR_UNSUPPORTED, "decode_step: at most 512 positions per image");
    if (codebook <= 0 || codebook % 64 || codebook > 1024 || codebook > V)
        return fail(c, MGH_ERR_UNSUPPORTED, "decode_step: codebook must be a multiple of 64, <= 1024 and <= V");
    if (n_steps <= 0 || step < 0 || step >= n_steps)
        return fail(c, MGH_ERR_ARG, "decode_step: need 0 <= step < n_steps");
    if (!state || !work || !logits || !tokens || !result) return fail(c, MGH_ERR_ARG, "decode_step: null pointer");
    if ((uintptr_t)state % 8 || (uintptr_t)work % 256)
        return fail(c, MGH_ERR_ARG, "decode_step: state must be 8-byte and work 256-byte aligned");
    if (int r = set_dev(c)) return r;
    mgh::DecodeArgs a{};
    a.logits = logits; a.tokens = tokens; a.result = result;
    a.B = B; a.S = S; a.V = V; a.CB = codebook; a.mask_id = mask_id; a.n_tokens = n_tokens;
    a.step = step; a.n_steps = n_steps; a.choice_temp = choice_temp;
    MGH_HIP(c, mgh::launch_decode_step(a, state, work, c->stream), "decode_step");
    return MGH_OK;
}

size_t mgh_packed_weight_bytes_f16(int N, int K) {
    return N > 0 && K > 0 ? mgh::packed_weight_bytes_f16(N, K) : 0;
}

int mgh_pack_weights_f16(mgh_ctx* c, int wtype, const void* w, int N, int K, void* wp16) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_quant_shape(c, wtype, N, K, 0)) return r;
    if (!w || !wp16) return fail(c, MGH_ERR_ARG, "pack_weights_f16: null pointer");
    if (!aligned16(wp16)) return fail(c, MGH_ERR_ARG, "pack_weights_f16: output must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_pack_weights_f16(wtype, w, wp16, N, K, c->stream), "k_pack_w16");
    return MGH_OK;
}

int mgh_f32_to_f16(mgh_ctx* c, const float* x, int64_t n, void* x16) {
    if (!c) return MGH_ERR_ARG;
    if (n < 0 || n % 8) return fail(c, MGH_ERR_ARG, "f32_to_f16: n must be a non-negative multiple of 8");
    if (n == 0) return MGH_OK;
    if (!x || !x16 || !aligned16(x) || !aligned16(x16))
        return fail(c, MGH_ERR_ARG, "f32_to_f16: pointers must be non-null and 16-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_f32_to_f16(x, (_Float16*)x16, n, c->stream), "k_f32_to_f16");
    return MGH_OK;
}

}  // extern "C"

namespace {

// The dequantize-fused FC entry points, for either weight form: wq 0 (fp16 [N][K] from
// mgh_pack_weights_f16) or 8 / 12 (the K-loop-dequant layout of mgh_pack_weights_dq).
int gemm_h16_any(mgh_ctx* c, const char* fn, int wq, const void* w, int N, int K, const void* x16, int M,
                 const float* bias, int act, const float* resid, float* y, _Float16* y16) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_h16(c, fn, w, N, K, x16, M, bias, act, resid, y16 ? (const float*)y16 : y)) return r;
    if (M == 0) return MGH_OK;
    if (int r = set_dev(c)) return r;
    mgh::GemmH16Args a{};
    a.x = (const _Float16*)x16; a.w = w; a.wq = wq;
    a.bias = bias; a.resid = resid; a.y = y16 ? nullptr : y; a.y16 = y16;
    a.M = M; a.N = N; a.K = K; a.act = act;
    return run_gemm_h16(c, a);
}

int gemm_h16_ln_any(mgh_ctx* c, const char* fn, int wq, const void* w, int N, int K, const void* x16, int M,
                    const float* bias, int act, const float* resid, float* y, const float* gamma,
                    const float* beta, float eps, float* y_ln, int emit, void* codes, float* dx, void* s4) {
    if (!c) return MGH_ERR_ARG;
    const std::string f(fn);
    // y may be null: then only the LayerNorm's outputs are written (y in the context scratch
    // when the plan runs the FC and the LayerNorm as two launches)
    const bool no_y = y == nullptr;
    if (int r = check_h16(c, fn, w, N, K, x16, M, bias, act, resid, y, true)) return r;
    if (N % 256 || N > 2048) return fail(c, MGH_ERR_UNSUPPORTED, f + ": needs N % 256 == 0 and N <= 2048");
    if (emit < 0 || emit > 2) return fail(c, MGH_ERR_ARG, f + ": emit must be 0, 1 or 2");
    if (M == 0) return MGH_OK;
    if (!gamma || !beta || !y_ln) return fail(c, MGH_ERR_ARG, f + ": null pointer");
    if (emit && (!codes || (emit == 1 && (!dx || !s4))))
        return fail(c, MGH_ERR_ARG, f + ": emit needs d_codes (and d_dx, d_s4 for INT8)");
    if (!aligned16(gamma) || !aligned16(beta) || !aligned16(y_ln) || !aligned16(codes) || ((uintptr_t)dx & 3u) ||
        ((uintptr_t)s4 & 3u))
        return fail(c, MGH_ERR_ARG, f + ": gamma/beta/y_ln/codes must be 16-byte aligned");
    if (int r = set_dev(c)) return r;
    mgh::GemmH16Args a{};
    a.x = (const _Float16*)x16; a.w = w; a.wq = wq;
    a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    const mgh::H16Plan p = mgh::gemm_h16_plan(M, N, K, false, wq);
    if (!mgh::use_gemv_h16(M, K) && p.splits > 1 && act == 0) {
        // the split-K reduce normalizes each row as it leaves: one launch fewer
        if (int r = ensure_qp_ws(c, p.ws_bytes)) return r;
        a.splits = p.splits;
        a.ws = (float*)c->qp_ws;
        const mgh::LnArgs ln{gamma, beta, eps, y_ln, emit, codes, dx, s4};
        MGH_HIP(c, mgh::launch_gemm_h16(p, a, c->stream, &ln), "k_gemm_fc + k_gemm_fc_reduce_ln");
        return MGH_OK;
    }
    if (no_y) {
        if (int r = ensure_scratch(c, round256((size_t)M * N * 4))) return r;
        a.y = y = (float*)c->scratch;
    }
    if (int r = run_gemm_h16(c, a)) return r;
    MGH_HIP(c, mgh::launch_layernorm_affine(y, gamma, beta, y_ln, M, N, eps, emit, codes, dx, s4, c->stream),
            "k_layernorm_affine");
    return MGH_OK;
}

// fp32 activations are rounded to fp16 either inside the GEMM's K loop (the 64-row fp32-operand
// plans) or by a separate pass feeding the fp16-operand plans (128-row tiles): every weight-row
// tile repeats the in-loop rounding, the pass is paid once per call. Measured on the four FC
// shapes at M = 2056 .. 16448 (Q8_0 bytes and fp16 copies): the pass wins from about 4096 x
// 3072 outputs (M = 4097 up-proj: 42.6 against 46.0 us on Q8_0 bytes) and from M = 8192 on
// (QKV 53.7 against 62.3 us), rounding in the loop below that (M = 4097 Q8_0: QKV 32.3 against
// 34.0, out-proj 19.2 against 25.2, down-proj 49.1 against 56.9 us; M = 2056: the four FCs
// 95 against 112 us).
bool round_act_pass(int M, int N) { return M >= 8192 || (M >= 2048 && (int64_t)M * N >= (int64_t)4096 * 3072); }

int gemm_h16_f32in_any(mgh_ctx* c, const char* fn, int wq, const void* w, int N, int K, const float* x, int M,
                       const float* bias, int act, const float* resid, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_h16(c, fn, w, N, K, x, M, bias, act, resid, y)) return r;
    if (M == 0) return MGH_OK;
    if (int r = set_dev(c)) return r;
    mgh::GemmH16Args a{};
    a.w = w; a.wq = wq;
    a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    if (!round_act_pass(M, N)) {
        a.xf = x;                               // rounded while the GEMM reads them
    } else {
        // a rounding pass, then the fp16-operand kernel and its tile plans
        if (int r = ensure_scratch(c, round256((size_t)M * K * 2))) return r;
        MGH_HIP(c, mgh::launch_f32_to_f16(x, (_Float16*)c->scratch, (int64_t)M * K, c->stream), "k_f32_to_f16");
        a.x = (const _Float16*)c->scratch;
    }
    return run_gemm_h16(c, a);
}

int check_dq(mgh_ctx* c, const char* fn, int wtype, int N, int K) {
    if (!c) return MGH_ERR_ARG;
    if (wtype != MGH_WTYPE_Q8_0 && wtype != MGH_WTYPE_Q4_K)
        return fail(c, MGH_ERR_ARG, std::string(fn) + ": wtype must be MGH_WTYPE_Q8_0 (8) or MGH_WTYPE_Q4_K (12)");
    if (wtype == MGH_WTYPE_Q4_K && K % 256 == 0 && K > 0) return MGH_OK;
    if (wtype == MGH_WTYPE_Q4_K) return fail(c, MGH_ERR_ARG, std::string(fn) + ": Q4_K needs K % 256 == 0");
    return MGH_OK;
}

}  // namespace

extern "C" {

int mgh_gemm_h16(mgh_ctx* c, const void* wp16, int N, int K, const void* x16, int M,
                 const float* bias, int act, const float* resid, float* y) {
    return gemm_h16_any(c, "gemm_h16", 0, wp16, N, K, x16, M, bias, act, resid, y, nullptr);
}

int mgh_gemm_h16_y16(mgh_ctx* c, const void* wp16, int N, int K, const void* x16, int M,
                     const float* bias, int act, const float* resid, void* y16) {
    return gemm_h16_any(c, "gemm_h16_y16", 0, wp16, N, K, x16, M, bias, act, resid, nullptr, (_Float16*)y16);
}

int mgh_gemm_h16_ln(mgh_ctx* c, const void* wp16, int N, int K, const void* x16, int M, const float* bias,
                    int act, const float* resid, float* y, const float* gamma, const float* beta, float eps,
                    float* y_ln, int emit, void* codes, float* dx, void* s4) {
    return gemm_h16_ln_any(c, "gemm_h16_ln", 0, wp16, N, K, x16, M, bias, act, resid, y, gamma, beta, eps, y_ln,
                           emit, codes, dx, s4);
}

int mgh_gemm_h16_f32in(mgh_ctx* c, const void* wp16, int N, int K, const float* x, int M,
                       const float* bias, int act, const float* resid, float* y) {
    return gemm_h16_f32in_any(c, "gemm_h16_f32in", 0, wp16, N, K, x, M, bias, act, resid, y);
}

int mgh_dequant_weights_f32(mgh_ctx* c, int wtype, const void* w, int N, int K, float* out) {
    if (!c) return MGH_ERR_ARG;
    if (wtype != MGH_WTYPE_Q8_0 && wtype != MGH_WTYPE_Q4_K)
        return fail(c, MGH_ERR_ARG, "dequant_weights_f32: wtype must be MGH_WTYPE_Q8_0 (8) or MGH_WTYPE_Q4_K (12)");
    if (N <= 0 || K <= 0) return fail(c, MGH_ERR_ARG, "dequant_weights_f32: needs N > 0, K > 0");
    if (K % (wtype == MGH_WTYPE_Q8_0 ? 32 : 256))
        return fail(c, MGH_ERR_ARG, "dequant_weights_f32: K must be a multiple of the block size (32 / 256)");
    if (!w || !out) return fail(c, MGH_ERR_ARG, "dequant_weights_f32: null pointer");
    if ((uintptr_t)out & 3u) return fail(c, MGH_ERR_ARG, "dequant_weights_f32: output must be 4-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_dequant_weights_f32(wtype, w, out, N, K, c->stream), "k_dequant_w32");
    return MGH_OK;
}

size_t mgh_packed_weight_bytes_dq(int wtype, int N, int K) {
    if (N <= 0 || K <= 0 || K % 64) return 0;
    if (wtype == MGH_WTYPE_Q4_K && K % 256) return 0;
    return mgh::packed_weight_bytes_dq(wtype, N, K);
}

int mgh_pack_weights_dq(mgh_ctx* c, int wtype, const void* w, int N, int K, void* wdq) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_quant_shape(c, wtype, N, K, 0)) return r;
    if (int r = check_dq(c, "pack_weights_dq", wtype, N, K)) return r;
    if (!w || !wdq) return fail(c, MGH_ERR_ARG, "pack_weights_dq: null pointer");
    if (!aligned16(wdq) || ((uintptr_t)w & 3u))
        return fail(c, MGH_ERR_ARG, "pack_weights_dq: output must be 16-byte aligned, input 4-byte aligned");
    if (int r = set_dev(c)) return r;
    MGH_HIP(c, mgh::launch_pack_weights_dq(wtype, w, wdq, N, K, c->stream), "k_pack_wdq");
    return MGH_OK;
}

int mgh_gemm_dq(mgh_ctx* c, int wtype, const void* wdq, int N, int K, const void* x16, int M,
                const float* bias, int act, const float* resid, float* y) {
    if (int r = check_dq(c, "gemm_dq", wtype, N, K)) return r;
    return gemm_h16_any(c, "gemm_dq", wtype, wdq, N, K, x16, M, bias, act, resid, y, nullptr);
}

int mgh_gemm_dq_y16(mgh_ctx* c, int wtype, const void* wdq, int N, int K, const void* x16, int M,
                    const float* bias, int act, const float* resid, void* y16) {
    if (int r = check_dq(c, "gemm_dq_y16", wtype, N, K)) return r;
    return gemm_h16_any(c, "gemm_dq_y16", wtype, wdq, N, K, x16, M, bias, act, resid, nullptr, (_Float16*)y16);
}

int mgh_gemm_dq_ln(mgh_ctx* c, int wtype, const void* wdq, int N, int K, const void* x16, int M,
                   const float* bias, int act, const float* resid, float* y, const float* gamma,
                   const float* beta, float eps, float* y_ln, int emit, void* codes, float* dx, void* s4) {
    if (int r = check_dq(c, "gemm_dq_ln", wtype, N, K)) return r;
    return gemm_h16_ln_any(c, "gemm_dq_ln", wtype, wdq, N, K, x16, M, bias, act, resid, y, gamma, beta, eps, y_ln,
                           emit, codes, dx, s4);
}

int mgh_gemm_dq_f32in(mgh_ctx* c, int wtype, const void* wdq, int N, int K, const float* x, int M,
                      const float* bias, int act, const float* resid, float* y) {
    if (int r = check_dq(c, "gemm_dq_f32in", wtype, N, K)) return r;
    return gemm_h16_f32in_any(c, "gemm_dq_f32in", wtype, wdq, N, K, x, M, bias, act, resid, y);
}

int mgh_gemm_h16_f32in_noalloc(mgh_ctx* c, const void* wp16, int N, int K, const float* x, int M,
                               const float* bias, int act, const float* resid, float* y) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_h16(c, "gemm_h16_f32in_noalloc", wp16, N, K, x, M, bias, act, resid, y)) return r;
    if (M == 0) return MGH_OK;
    // the same launches as mgh_gemm_h16_f32in, with the rounded activations (round_act_pass)
    // and the split-K partials placed in the fixed scratch array instead of context buffers
    mgh::GemmH16Args a{};
    a.w = wp16;
    a.bias = bias; a.resid = resid; a.y = y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    if (mgh::use_gemv_h16(M, K)) {               // skinny-M kernel: no scratch at all
        if (int r = set_dev(c)) return r;
        a.xf = x;
        MGH_HIP(c, mgh::launch_gemv_h16(a, c->stream), "k_gemv_fc");
        return MGH_OK;
    }
    const bool round_pass = round_act_pass(M, N);
    const size_t x16_b = round_pass ? round256((size_t)M * K * 2) : 0;
    const mgh::H16Plan p = mgh::gemm_h16_plan(M, N, K, !round_pass, 0);
    const size_t need = x16_b + (p.splits > 1 ? round256(p.ws_bytes) : 0);
    const size_t cap = mgh::noalloc_scratch_bytes();
    if (need > cap)
        return fail(c, MGH_ERR_UNSUPPORTED, "gemm_h16_f32in_noalloc: this shape needs " + std::to_string(need) +
                                                " bytes of scratch, the maximum is " + std::to_string(cap));
    if (int r = set_dev(c)) return r;
    void* base = nullptr;
    MGH_HIP(c, mgh::noalloc_scratch(c->device, &base), "hipGetSymbolAddress(scratch)");
    // calls on other streams of this GPU share the array: run after the previous one
    bool capturing = false;
    MGH_HIP(c, mgh::noalloc_order_begin(c->device, c->stream, &capturing), "noalloc ordering");
    hipError_t e = hipSuccess;
    if (round_pass) {
        e = mgh::launch_f32_to_f16(x, (_Float16*)base, (int64_t)M * K, c->stream);
        a.x = (const _Float16*)base;
    } else {
        a.xf = x;
    }
    a.splits = p.splits;
    if (p.splits > 1) a.ws = (float*)((char*)base + x16_b);
    if (e == hipSuccess) e = mgh::launch_gemm_h16(p, a, c->stream);
    const hipError_t e2 = mgh::noalloc_order_end(c->device, c->stream, capturing);
    MGH_HIP(c, e, "k_gemm_fc (no-allocation entry)");
    MGH_HIP(c, e2, "noalloc ordering");
    return MGH_OK;
}

int mgh_debug_block_dots(mgh_ctx* c, int wtype, const void* w, int N, int K, const int8_t* qx,
                         int M, int32_t* out) {
    if (!c) return MGH_ERR_ARG;
    if (int r = check_quant_shape(c, wtype, N, K, M)) return r;
    if (M == 0) return MGH_OK;
    if (!w || !qx || !out) return fail(c, MGH_ERR_ARG, "debug_block_dots: null pointer");
    if (int r = set_dev(c)) return r;
    mgh::GemmArgs a{};
    a.w = (const uint8_t*)w; a.qx = qx; a.dots = out;
    a.M = M; a.N = N; a.K = K;
    MGH_HIP(c, launch_gemm(wtype, a, true, c->stream), "k_gemm_q_i8(debug)");
    return MGH_OK;
}

}  // extern "C"
