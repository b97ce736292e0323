/* mgh.h — C ABI of the MI355X (gfx950) kernel layer for the edge_maskgit FC hot path.
 *
 * This is the boundary the C++ backend (HipRuntime, include/mg-hip.hpp) and any FFI
 * (ctypes, cgo, ...) bind. It replaces the OpenCL kernel dispatches inside
 * OpenCLRuntime::compute (reference src/mg-opencl/mg-opencl.cpp:1354-1656).
 *
 * Conventions
 *  - Status: every call returns 0 (MGH_OK) or a negative MGH_ERR_*; no exception or
 *    abort crosses the ABI. mgh_last_error() gives the message of the last failure.
 *  - Memory: pointers named d_* are device pointers the caller owns (mgh_alloc/mgh_free
 *    or any hipMalloc'd memory); h_* are host pointers.
 *  - Ordering: compute calls are enqueued on the context's stream and return without
 *    waiting (stream-ordered, like the reference's in-order cl queue). mgh_sync waits.
 *  - Threading: one context per host thread; a context is not thread-safe (the reference
 *    OpenCLRuntime is single-threaded too, mg-opencl.cpp:1108-1212).
 *  - Shapes follow the reference (include/mg-tensor.hpp:3-13): a weight has N rows of K
 *    values (GGUF ne={K,N}) stored as raw ggml blocks, activations are [M][K] row-major,
 *    outputs are [M][N] row-major.
 */
#ifndef MGH_H
#define MGH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mgh_ctx mgh_ctx;

enum {
    MGH_OK = 0,
    MGH_ERR_ARG = -1,          /* invalid argument (null pointer, bad shape, bad enum) */
    MGH_ERR_UNSUPPORTED = -2,  /* valid but not implemented (e.g. K not a multiple of 64) */
    MGH_ERR_HIP = -3,          /* HIP runtime error (message has the HIP error string) */
    MGH_ERR_NO_DEVICE = -4     /* no gfx950 device at that ordinal */
};

/* weight types: the GGUF tensor type codes (reference src/mg-model.cpp:22) */
enum { MGH_WTYPE_F32 = 0, MGH_WTYPE_Q8_0 = 8, MGH_WTYPE_Q4_K = 12 };

/* fused epilogue activations (reference mg-opencl.cpp:36-40) */
enum { MGH_ACT_NONE = 0, MGH_ACT_GELU = 1, MGH_ACT_SILU = 2 };

/* GEMM algorithm for quantized weights. INT8 = per-32 int8 activation codes, exact block
 * dots (the reference's int8-dot path, mg-opencl.cpp:1381-1398); DEQ_F16 = fp16-rounded
 * activations against the dequantized weights, fp32 accumulation (the reference's
 * dequant-fused fp16-slab path, mg-opencl.cpp:1400-1423), on fp16 weight copies made at
 * upload; DEQ_Q = the same product on the Q8_0 / Q4_K bytes themselves, decoded inside the K
 * loop as the reference does (mgh_gemm_dq), with identical results. AUTO = DEQ_F16, the
 * reference's choice on any device without cl_arm_integer_dot_product
 * (mg-opencl.cpp:1237-1238), which includes this one, in its faster weight form. */
enum { MGH_ALGO_AUTO = 0, MGH_ALGO_INT8 = 1, MGH_ALGO_DEQ_F16 = 2, MGH_ALGO_DEQ_Q = 3 };

/* ---- context: replaces OpenCLRuntime::OpenCLRuntime / ~OpenCLRuntime / device_name
 *      (reference include/mg-opencl.hpp:25-31, src/mg-opencl/mg-opencl.cpp:1214-1280) ---- */
int         mgh_create(int device_ordinal, mgh_ctx** out);
void        mgh_destroy(mgh_ctx* ctx);
const char* mgh_last_error(const mgh_ctx* ctx);      /* never NULL; "" after success */
const char* mgh_device_name(const mgh_ctx* ctx);
int         mgh_version(void);

/* ---- device memory: replaces the clCreateBuffer / clEnqueueWriteBuffer /
 *      clEnqueueReadBuffer traffic of OpenCLRuntime::Impl::buf() and the final readback
 *      (mg-opencl.cpp:1172-1206, 1622-1626) ---- */
int mgh_alloc(mgh_ctx* ctx, size_t bytes, void** d_out);
int mgh_free(mgh_ctx* ctx, void* d_ptr);
int mgh_h2d(mgh_ctx* ctx, void* d_dst, const void* h_src, size_t bytes);   /* synchronous */
int mgh_d2h(mgh_ctx* ctx, void* h_dst, const void* d_src, size_t bytes);   /* synchronous */
int mgh_fill_u32(mgh_ctx* ctx, void* d_dst, uint32_t value, size_t n_words); /* kernel fill */
int mgh_sync(mgh_ctx* ctx);                                                  /* clFinish */

/* ---- timing on the context stream (HIP events), for benchmarks ---- */
int mgh_timer_start(mgh_ctx* ctx);
int mgh_timer_stop(mgh_ctx* ctx, float* ms_out);   /* waits for the stop event */

/* ---- HIP graphs: capture a sequence of calls on the context stream and replay it as one
 *      submission (the reference re-enqueues every node each step, mg-opencl.cpp:1362).
 *      Between mgh_graph_begin and mgh_graph_end only stream-ordered compute calls may be
 *      made (no mgh_alloc/mgh_free/mgh_h2d/mgh_d2h/mgh_sync, no scratch growth). ---- */
typedef struct mgh_graph mgh_graph;
int  mgh_graph_begin(mgh_ctx* ctx);
int  mgh_graph_end(mgh_ctx* ctx, mgh_graph** out);
int  mgh_graph_launch(mgh_ctx* ctx, mgh_graph* graph);
void mgh_graph_destroy(mgh_graph* graph);

/* ---- activation quantizer: replaces k_quantize_q8 and its dispatch
 *      (mg-opencl.cpp:424-434, 1381-1389). x [M][K] -> qx [M][K] int8,
 *      dx [M][K/32] fp32 scales, sx [M][K/32] int32 block sums (nullable). K % 32 == 0. */
int mgh_quantize_act_q8(mgh_ctx* ctx, const float* d_x, int M, int K,
                        int8_t* d_qx, float* d_dx, int32_t* d_sx);

/* ---- quantized FC GEMM on pre-quantized activations: replaces k_mul_mat_q8_i8 /
 *      k_mul_mat_q4k_i8 and their dispatch (mg-opencl.cpp:440-590, 1390-1398).
 *      y[M][N] = act(w . x + bias) + resid; bias [N] and resid [M][N] nullable.
 *      Q8_0 needs K % 64 == 0, Q4_K needs K % 256 == 0 and d_sx. ---- */
int mgh_gemm_q(mgh_ctx* ctx, int wtype, const void* d_w, int N, int K,
               const int8_t* d_qx, const float* d_dx, const int32_t* d_sx, int M,
               const float* d_bias, int act, const float* d_resid, float* d_y);

/* ---- the quantizer of mgh_quantize_act_q8 writing its int8 codes as fp16 values (uint16
 *      bit patterns, exact for |q| <= 127): the activation operand of mgh_gemm_q_packed. ---- */
int mgh_quantize_act_q8_codes16(mgh_ctx* ctx, const float* d_x, int M, int K,
                                uint16_t* d_qx16, float* d_dx, int32_t* d_sx);

/* ---- device-native weight layout. The reference's OpenCL runtime uploads each weight
 *      tensor once into a device buffer it caches for the model's lifetime
 *      (mg-opencl.cpp:1172-1206); this backend rewrites the tensor once at that point into
 *      fp16 codes [N][K] | fp32 block scales [K/32][N] (| fp32 block mins [N][K/32] for
 *      Q4_K: dmin*m_j), so the hot GEMM streams whole aligned lines with no block
 *      decoding. mgh_packed_weight_bytes returns the size (0 for an invalid type/shape);
 *      d_packed must be 16-byte aligned. ---- */
size_t mgh_packed_weight_bytes(int wtype, int N, int K);
int    mgh_pack_weights(mgh_ctx* ctx, int wtype, const void* d_w, int N, int K, void* d_packed);

/* ---- quantized FC GEMM on packed weights and fp16-code activations (the production
 *      kernel; replaces k_mul_mat_q8_i8 / k_mul_mat_q4k_i8 and their dispatch,
 *      mg-opencl.cpp:440-590, 1390-1398). Semantics of mgh_gemm_q. Needs Q8_0 K % 64 == 0
 *      or Q4_K K % 256 == 0, N % 4 == 0, 16-byte aligned d_wp/d_qx16/d_bias/d_resid/d_y,
 *      4-byte aligned d_dx (16-byte d_dx and d_sx for Q4_K). ---- */
int mgh_gemm_q_packed(mgh_ctx* ctx, int wtype, const void* d_wp, int N, int K,
                      const uint16_t* d_qx16, const float* d_dx, const int32_t* d_sx, int M,
                      const float* d_bias, int act, const float* d_resid, float* d_y);

/* ---- the whole MulMat(q) node on packed weights and fp32 activations (replaces the node
 *      dispatch mg-opencl.cpp:1367-1428): ALGO_INT8 = per-32 int8 activation codes +
 *      mgh_gemm_q_packed; ALGO_AUTO/DEQ_F16 = activations rounded to fp16 against the dequantized
 *      weights (the reference's fp16-slab path k_mul_mat_*_t2_h, mg-opencl.cpp:320-411),
 *      same kernel. Activation operands live in context scratch (grown on demand, not during
 *      graph capture). Shape/alignment rules of mgh_gemm_q_packed; d_x 16-byte aligned. ---- */
int mgh_gemm_q_packed_f32in(mgh_ctx* ctx, int algo, int wtype, const void* d_wp, int N, int K,
                            const float* d_x, int M, const float* d_bias, int act,
                            const float* d_resid, float* d_y);

/* ---- quantized FC GEMM on fp32 activations: replaces the whole MulMat(q) node
 *      dispatch (mg-opencl.cpp:1367-1428): mgh_quantize_act_q8 + mgh_gemm_q for ALGO_INT8
 *      (activation scratch owned by the context and grown on demand, like the reference's
 *      qx_buf/dx_buf, mg-opencl.cpp:1125-1134), or the weights packed into scratch and one
 *      dequant-fp16 GEMM for ALGO_AUTO/DEQ_F16. Output semantics as mgh_gemm_q. ---- */
int mgh_gemm_q_f32in(mgh_ctx* ctx, int algo, int wtype, const void* d_w, int N, int K,
                     const float* d_x, int M, const float* d_bias, int act,
                     const float* d_resid, float* d_y);

/* LayerNorm-affine output modes: what else mgh_layernorm_affine writes besides y */
enum { MGH_EMIT_NONE = 0, MGH_EMIT_INT8 = 1, MGH_EMIT_DEQ_F16 = 2 };

/* ---- LayerNorm + affine over rows: replaces the Norm(affine) node and its dispatch
 *      (k_norm_affine mg-opencl.cpp:705-727, 1450-1465; CPU mg-cpu.cpp:105-121, 249-261).
 *      x, y [rows][D] fp32 (may alias), gamma/beta [D]; D % 256 == 0, D <= 2048; 16-byte
 *      aligned x/y/gamma/beta/codes. Statistics in double, as the reference CPU executor.
 *      emit = MGH_EMIT_INT8 also writes the next GEMM's operand for y (as
 *      mgh_quantize_act_q8_codes16): d_codes fp16 codes [rows][D], d_dx fp32 and d_s4 int32
 *      [rows][D/32]; MGH_EMIT_DEQ_F16 writes fp16-rounded y, and (each nullable) unit d_dx
 *      and fp32 block sums in d_s4. No reference counterpart for the fused operand (the reference
 *      quantizes in a separate k_quantize_q8 dispatch, mg-opencl.cpp:1381-1389). ---- */
int mgh_layernorm_affine(mgh_ctx* ctx, const float* d_x, const float* d_gamma, const float* d_beta,
                         int rows, int D, float eps, float* d_y, int emit, void* d_codes,
                         float* d_dx, void* d_s4);

/* ---- flash attention with fp16 K/V: replaces k_flash_attention_h and its dispatch
 *      (mg-opencl.cpp:859-937, 1483-1511). q/k/v are {D,S,H,B} views with element strides
 *      strides[4] (d, s, h, b); the output has element strides o_strides[4], or is the
 *      contiguous {D,S,H,B} tensor when o_strides is NULL. D in {16, 32, 48, 64}. ---- */
int mgh_flash_attn_f16kv(mgh_ctx* ctx, const float* d_q, const float* d_k, const float* d_v,
                         const int64_t strides[4], int D, int S, int H, int B, float scale,
                         float* d_o, const int64_t o_strides[4]);
/* the same attention with the output stored rounded to fp16 (the operand of the following
 * dequantize-fused out-projection; no counterpart in the reference, whose FC rounds its fp32
 * input to fp16 — the result is identical) */
int mgh_flash_attn_f16kv_o16(mgh_ctx* ctx, const float* d_q, const float* d_k, const float* d_v,
                             const int64_t strides[4], int D, int S, int H, int B, float scale,
                             void* d_o16, const int64_t o_strides[4]);
/* the same attention on q/k/v already stored as fp16 (the fused QKV FC's fp16 output; no
 * counterpart in the reference, whose k_flash_attention_h rounds its fp32 q/k/v to fp16 on
 * load, mg-opencl.cpp:859-937 — the result is identical). Exactly one of d_o (fp32) and d_o16
 * (fp16) is non-NULL. Needs S <= 512, strides[0] == 1, the other strides multiples of 4,
 * 16-byte aligned q/k/v and scale > 0 (MGH_ERR_UNSUPPORTED otherwise). */
int mgh_flash_attn_f16in(mgh_ctx* ctx, const void* d_q16, const void* d_k16, const void* d_v16,
                         const int64_t strides[4], int D, int S, int H, int B, float scale,
                         float* d_o, void* d_o16, const int64_t o_strides[4]);

/* ---- fp32 GEMM with the fused epilogue (tied MLM head, F32 FC weights): replaces
 *      k_mul_mat_t and its dispatch (mg-opencl.cpp:60-94, 1429-1440).
 *      y[M][N] = act(x . w^T + bias) + resid; w [N][K], x [M][K]; K % 32 == 0, 16-byte
 *      aligned w and x. ---- */
int mgh_gemm_f32(mgh_ctx* ctx, const float* d_w, int N, int K, const float* d_x, int M,
                 const float* d_bias, int act, const float* d_resid, float* d_y);

/* ---- graph glue: GetRows (k_get_rows mg-opencl.cpp:667-672; negative ids count from the end,
 *      out-of-range ids are clamped), Add with a repeating second operand (out[i] = a[i] +
 *      b[i % nb]), and the Cont of a strided view into a contiguous {ne0..ne3} buffer
 *      (k_cont mg-opencl.cpp:940-945). ---- */
int mgh_get_rows(mgh_ctx* ctx, const float* d_a, int64_t E, int64_t R, const int32_t* d_ids,
                 int64_t n, float* d_out);
int mgh_add(mgh_ctx* ctx, const float* d_a, const float* d_b, int64_t nb, float* d_out, int64_t n);
int mgh_copy_strided(mgh_ctx* ctx, const float* d_a, const int64_t ne[4], const int64_t strides[4],
                     float* d_out);

/* ---- the remaining F32 graph ops of the reference's GPU runtime
 *      (mg-opencl.cpp:1450-1534; CPU semantics mg-cpu.cpp:27-38, 40-45, 88-103, 150-163).
 *      Strides are in elements; outputs are contiguous.
 *      mgh_softmax: SoftMax over rows of D contiguous values, y = softmax(x * scale)
 *        (k_soft_max :732-751); x and y may alias.
 *      mgh_binary: out = a + b (op 0, Add) or a * b (op 1, Mul) over shape ne, a read with
 *        a_strides, b of shape b_ne broadcast over its size-1 dimensions (k_add/k_mul
 *        :947-960; the reference needs each b_ne[i] to be ne[i] or 1, so does this).
 *      mgh_scale: y = x * s (Scale, k_scale :961-963).
 *      mgh_unary: y = GELU(x) (act MGH_ACT_GELU, exact erf, k_gelu :964-967) or SiLU
 *        (MGH_ACT_SILU, k_silu :968-971).
 *      mgh_gemm_f32_batched: the stride-aware batched F32 MulMat (k_mul_mat_t :60-94, dispatch
 *        :1429-1440): w {K, N, w_ne[2], w_ne[3]}, x {K, M, B2, B3}; w broadcasts over batch
 *        dimensions of size 1; y [B3][B2][M][N] = act(w . x + bias) + resid. Each output sums
 *        over k in order with separate multiply and add, as the reference CPU executor. ---- */
int mgh_softmax(mgh_ctx* ctx, const float* d_x, int64_t rows, int D, float scale, float* d_y);
int mgh_binary(mgh_ctx* ctx, int op, const float* d_a, const int64_t a_strides[4], const float* d_b,
               const int64_t b_ne[4], const int64_t b_strides[4], const int64_t ne[4], float* d_out);
int mgh_scale(mgh_ctx* ctx, const float* d_x, int64_t n, float s, float* d_y);
int mgh_unary(mgh_ctx* ctx, int act, const float* d_x, int64_t n, float* d_y);
int mgh_gemm_f32_batched(mgh_ctx* ctx, const float* d_w, const int64_t w_ne[4], const int64_t w_strides[4],
                         const float* d_x, const int64_t x_ne[4], const int64_t x_strides[4],
                         const float* d_bias, int act, const float* d_resid, float* d_y);

/* ---- VQGAN decoder ops, layout ne = {W, H, C, N} (W innermost), fp32, contiguous.
 *      mgh_conv2d: the Conv2D node (CPU mg-cpu.cpp:165-190; GPU k_conv2d_t,
 *      mg-opencl.cpp:985-1025, 1535-1566): ker {KW, KH, IC, OC}, out {OW, OH, OC, N} with
 *      OW = (IW + 2 pad - KW) / stride + 1; fp32 products and accumulation; d_out 16-byte aligned.
 *      Kernels: IC % 16 == 0 an fp32-MFMA implicit GEMM over tap-major packed weights (packed
 *      into the context scratch per call, or once by mgh_conv2d_pack_weights; 128 x 128 tiles,
 *      256 x 16 for OC <= 16), with K split across workgroups when one image's output alone
 *      gives too few (per image: results do not depend on the batch); otherwise, for OC <= 8,
 *      one thread per pixel in the reference loop's order (the CPU executor's float operations
 *      exactly), else a 64 x 64 fp32-MFMA implicit GEMM over the reference layout.
 *      mgh_conv2d_ex: the conv node with the decoder's following Add nodes fused:
 *      out = (conv + bias[oc]) + resid, each addition rounded as its own node would (bias [OC]
 *      or null; resid shaped as out, 16-byte aligned, or null); d_packed (optional, from
 *      mgh_conv2d_pack_weights, mgh_conv2d_packed_bytes large) saves the per-call packing,
 *      and for the packed path d_ker may then be null.
 *      mgh_group_norm: the GroupNorm node (mg-cpu.cpp:123-147, 262-276; mg-opencl.cpp:1027-1095,
 *      1568-1590): statistics per (n, group) in double, y = (x - mean) / sqrt(var + eps); with
 *      d_gamma and d_beta [C] also the fused per-channel affine and SiLU (both null: plain).
 *      Scratch from the context. mgh_upscale: nearest-neighbour upscale by factor
 *      (mg-cpu.cpp:192-198, mg-opencl.cpp:1096-1103, 1591-1599). ---- */
int mgh_conv2d(mgh_ctx* ctx, const float* d_in, int IW, int IH, int IC, int N, const float* d_ker,
               int KW, int KH, int OC, int stride, int pad, float* d_out);
int mgh_conv2d_ex(mgh_ctx* ctx, const float* d_in, int IW, int IH, int IC, int N, const float* d_ker,
                  const float* d_packed, int KW, int KH, int OC, int stride, int pad, const float* d_bias,
                  const float* d_resid, float* d_out);
/* bytes of the packed copy (0: the shape does not take the packed kernel) */
size_t mgh_conv2d_packed_bytes(int KW, int KH, int IC, int OC);
int mgh_conv2d_pack_weights(mgh_ctx* ctx, const float* d_ker, int KW, int KH, int IC, int OC, float* d_packed);
/* The int8 conv of the reference's integer-dot devices (k_quantize_conv_w + k_conv2d_i8,
 * mg-opencl.cpp:598-664, 1541-1553): mgh_conv2d_i8_pack_weights quantizes the kernel once per
 * output channel and 32-block of k = (ic*KH + kh)*KW + kw (d = amax/127, round half away from
 * zero; buffer of mgh_conv2d_i8_weight_bytes: int8 codes [ceil(OC/16)][blocks][16][32], then
 * fp32 scales [ceil(OC/16)][blocks][16], zero past OC and K); mgh_conv2d_i8
 * quantizes every output pixel's im2col column per 32-block the same way, sums the exact
 * integer block dots as acc = acc + (dx*dw)*idot in block order (fp32, each operation
 * rounded), then (+ bias[oc]) (+ resid) as mgh_conv2d_ex. The quantized im2col matrix lives
 * in the context's workspace (about 1.13 bytes per output pixel and k, grown on first use). */
size_t mgh_conv2d_i8_weight_bytes(int KW, int KH, int IC, int OC);
int mgh_conv2d_i8_pack_weights(mgh_ctx* ctx, const float* d_ker, int KW, int KH, int IC, int OC, void* d_wq);
int mgh_conv2d_i8(mgh_ctx* ctx, const float* d_in, int IW, int IH, int IC, int N, const void* d_wq, int KW,
                  int KH, int OC, int stride, int pad, const float* d_bias, const float* d_resid, float* d_out);
int mgh_group_norm(mgh_ctx* ctx, const float* d_x, int W, int H, int C, int N, int groups, float eps,
                   const float* d_gamma, const float* d_beta, float* d_y);
int mgh_upscale(mgh_ctx* ctx, const float* d_x, int W, int H, int C, int N, int factor, float* d_y);

/* ---- dequantize-fused fp16 FC path: the reference's fp16-slab dequant GEMMs
 *      k_mul_mat_q8_0_t2_h / k_mul_mat_q4k_t2_h (src/mg-opencl/mg-opencl.cpp:320-411).
 *      mgh_pack_weights_f16 expands raw Q8_0 / Q4_K blocks once into fp16 [N][K]
 *      (w = d*q, resp. (d*sc)*q - dmin*m in fp32, rounded to nearest fp16; buffer size
 *      mgh_packed_weight_bytes_f16). mgh_gemm_h16 computes
 *      y[M][N] = act(x16[M][K] . w16^T + bias) + resid with fp16 activations (for example
 *      from mgh_layernorm_affine with MGH_EMIT_DEQ_F16 or mgh_f32_to_f16) and fp32
 *      accumulation; mgh_gemm_h16_f32in rounds fp32 activations to fp16 first (context
 *      scratch). A few activation rows (M <= 16, or M <= 32 with K <= 1024: decode- and
 *      GEMV-shaped calls) take a skinny-M kernel that streams each weight row once and sums
 *      K slices across waves, the rest the tiled kernel; the same product and rounding.
 *      K % 64 == 0, N % 4 == 0, N <= 2097152, 16-byte aligned operands.
 *      For measurements, the environment variable MGH_FC_PLAN="bm,bn,ns,splits[,K,N]" (read
 *      once per process) replaces the tile plan of the tiled launches; a plan outside the
 *      compiled kernel set makes the call fail. ---- */
size_t mgh_packed_weight_bytes_f16(int N, int K);
int mgh_pack_weights_f16(mgh_ctx* ctx, int wtype, const void* d_w, int N, int K, void* d_wp16);
/* x -> fp16 (round to nearest even); n % 8 == 0 */
int mgh_f32_to_f16(mgh_ctx* ctx, const float* d_x, int64_t n, void* d_x16);
int mgh_gemm_h16(mgh_ctx* ctx, const void* d_wp16, int N, int K, const void* d_x16, int M,
                 const float* d_bias, int act, const float* d_resid, float* d_y);
int mgh_gemm_h16_f32in(mgh_ctx* ctx, const void* d_wp16, int N, int K, const float* d_x, int M,
                       const float* d_bias, int act, const float* d_resid, float* d_y);
/* mgh_gemm_h16_f32in for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): identical launches and
 * results, with the rounded activations and split-K partials in a fixed 64 MiB scratch array
 * the library holds on each GPU it runs on (no hipMalloc/hipFree, no context buffer growth).
 * Shapes whose scratch exceeds 64 MiB return MGH_ERR_UNSUPPORTED before anything runs. All
 * calls on one GPU share that array; the library orders them on the device (each call's
 * launches wait for the previous call's, whatever context or stream made it, through one
 * event per GPU), except under stream capture, where a captured call must not be replayed
 * while another call on the same GPU runs. No counterpart in the reference (its runtime grows
 * scratch buffers on demand, mg-opencl.cpp:1130-1134). */
int mgh_gemm_h16_f32in_noalloc(mgh_ctx* ctx, const void* d_wp16, int N, int K, const float* d_x, int M,
                               const float* d_bias, int act, const float* d_resid, float* d_y);
/* mgh_gemm_h16 followed by mgh_layernorm_affine of its output rows, the pair a post-norm
 * layer runs (reference: the MulMat node with its fused residual, mg-opencl.cpp:320-411, then
 * the Norm(affine) node, :705-727; mg-transformer.cpp:88-90, 95-97): y as mgh_gemm_h16 writes it and
 * d_y_ln, d_codes, d_dx, d_s4 as mgh_layernorm_affine(y) writes them (gamma/beta [N], N % 256
 * == 0, N <= 2048), bit for bit. When the product splits K (a few hundred activation rows)
 * and act is 0, the split-K reduce normalizes each row as it leaves, one launch instead of
 * two. d_y may be NULL when the caller needs only the LayerNorm's outputs: the split-K reduce
 * then skips y's store, and the two-launch form keeps y in the context scratch. No single
 * reference counterpart: the reference runs the two nodes as two dispatches. */
int mgh_gemm_h16_ln(mgh_ctx* ctx, const void* d_wp16, int N, int K, const void* d_x16, int M,
                    const float* d_bias, int act, const float* d_resid, float* d_y, const float* d_gamma,
                    const float* d_beta, float eps, float* d_y_ln, int emit, void* d_codes, float* d_dx,
                    void* d_s4);
/* the same product stored rounded to fp16 (d_y16 [M][N]): the operand of a following
 * dequantize-fused FC (no counterpart in the reference, where the next FC rounds its fp32
 * input; the result is identical) */
int mgh_gemm_h16_y16(mgh_ctx* ctx, const void* d_wp16, int N, int K, const void* d_x16, int M,
                     const float* d_bias, int act, const float* d_resid, void* d_y16);

/* ---- dequantize-fused FC path on the quantized bytes: the same product as mgh_gemm_h16
 *      (the reference's k_mul_mat_q8_0_t2_h / k_mul_mat_q4k_t2_h, mg-opencl.cpp:320-411, which
 *      decode every weight inside the K loop: DEQ_Q8 :386-387, deq_q4k_elem :252-262), reading
 *      the Q8_0 / Q4_K bytes on every call instead of an fp16 copy. mgh_pack_weights_dq
 *      regroups the GGUF blocks once, at upload, into 16-row groups of 64-deep K stages laid
 *      out in MFMA fragment order (Q8_0: int8 codes + fp16 block scales, 1.0625 bytes per
 *      weight; Q4_K: 4-bit values + the raw 16-byte super-block headers, 0.5625 bytes per
 *      weight; rows padded to a multiple of 16; buffer size mgh_packed_weight_bytes_dq). The
 *      kernels decode each weight to d*q, resp. (d*sc)*q - dmin*m rounded once to fp16 -- the
 *      value mgh_pack_weights_f16 stores -- as the MFMA fragments are read, so results equal
 *      mgh_gemm_h16's for the same tile plan. Shapes and alignment as mgh_gemm_h16 (K % 64 == 0,
 *      Q4_K K % 256 == 0, N % 4 == 0, N <= 2097152, 16-byte aligned operands). ---- */
size_t mgh_packed_weight_bytes_dq(int wtype, int N, int K);
/* raw Q8_0 / Q4_K blocks (GGUF layout, any byte alignment) -> fp32 [N][K], the values the
 * reference's dequantizing kernels compute (DEQ_Q8 mg-opencl.cpp:386-387; deq_q4k_elem
 * :252-262): any N >= 1, K a multiple of the block size. HipRuntime runs a quantized MulMat
 * whose shape the tiled kernels do not take (Q8_0 with K % 64 != 0, N % 4 != 0) as the
 * reference's F32 dequant GEMM on these values (k_mul_mat_q8_0_t2, :320-411). */
int mgh_dequant_weights_f32(mgh_ctx* ctx, int wtype, const void* d_w, int N, int K, float* d_out);
int mgh_pack_weights_dq(mgh_ctx* ctx, int wtype, const void* d_w, int N, int K, void* d_wdq);
int mgh_gemm_dq(mgh_ctx* ctx, int wtype, const void* d_wdq, int N, int K, const void* d_x16, int M,
                const float* d_bias, int act, const float* d_resid, float* d_y);
int mgh_gemm_dq_f32in(mgh_ctx* ctx, int wtype, const void* d_wdq, int N, int K, const float* d_x, int M,
                      const float* d_bias, int act, const float* d_resid, float* d_y);
int mgh_gemm_dq_y16(mgh_ctx* ctx, int wtype, const void* d_wdq, int N, int K, const void* d_x16, int M,
                    const float* d_bias, int act, const float* d_resid, void* d_y16);
int mgh_gemm_dq_ln(mgh_ctx* ctx, int wtype, const void* d_wdq, int N, int K, const void* d_x16, int M,
                   const float* d_bias, int act, const float* d_resid, float* d_y, const float* d_gamma,
                   const float* d_beta, float eps, float* d_y_ln, int emit, void* d_codes, float* d_dx,
                   void* d_s4);

/* ---- iterative decoding on the device: one step of the reference's generate() loop,
 *      src/mg-generate.cpp:82-121, for B images whose logits [B][S][V] are already in HBM.
 *      Image b draws from std::mt19937_64(seeds[b]) through uniform_real_distribution<double>
 *      in the reference's order (S categorical draws, then S Gumbel draws per step), samples
 *      every position over the first `codebook` logits (softmax, :89-97), keeps known tokens
 *      (:98-100), applies the cosine schedule with n_tokens unknown positions at the start
 *      (:104-110) and re-masks the lowest-confidence samples (:112-119). `tokens` [B][S] is
 *      updated in place; `result` [B][S] receives the step's samples before re-masking (the
 *      reference's `result`). `state` (mgh_decode_state_bytes, 8-byte aligned) carries the
 *      engines across steps; `work` (mgh_decode_work_bytes, 256-byte aligned) is per-step
 *      scratch. Limits: S <= 512, codebook a multiple of 64 and <= 1024. ---- */
size_t mgh_decode_state_bytes(int B);
size_t mgh_decode_work_bytes(int B, int S);
/* seeds: host array of B seeds; the state is ready when the call returns */
int mgh_decode_init(mgh_ctx* ctx, int B, const uint64_t* seeds, void* d_state);
int mgh_decode_step(mgh_ctx* ctx, void* d_state, void* d_work, const float* d_logits, int B, int S,
                    int V, int codebook, int mask_id, int n_tokens, int step, int n_steps,
                    float choice_temp, int32_t* d_tokens, int32_t* d_result);

/* ---- debug: the int32 per-block dot products exactly as the production GEMM's MFMA
 *      computes them, out[m][n][t] (t = K/32 blocks). The reference has no counterpart;
 *      it exposes the quantity mg-opencl.cpp:472-478 / :571-576 accumulates. ---- */
int mgh_debug_block_dots(mgh_ctx* ctx, int wtype, const void* d_w, int N, int K,
                         const int8_t* d_qx, int M, int32_t* d_out);

/* ---- debug: the block dot products of mgh_gemm_q_packed's MFMA, out[m][n][t] (no
 *      reference counterpart, as mgh_debug_block_dots). ---- */
int mgh_debug_block_dots_packed(mgh_ctx* ctx, int wtype, const void* d_wp, int N, int K,
                                const uint16_t* d_qx16, int M, int32_t* d_out);

#ifdef __cplusplus
}
#endif
#endif /* MGH_H */
