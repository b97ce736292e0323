/* mg_oracle.h — CPU restatement of the reference hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This is the checker, never the product: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The shipped GPU path (edge_maskgit_amd/)
 * never links, loads or falls back to it.
 *
 * Every function restates one piece of chenxugz/edge_maskgit and cites the reference
 * file:line it follows (paths relative to the reference repository root). Arithmetic
 * is written out operation by operation in fp32 (or double where the reference CPU
 * path uses double) and the library is compiled with -ffp-contract=off, so each
 * rounding step is the one written here.
 *
 * Layout conventions (reference include/mg-tensor.hpp:3-13): row-major, a weight is
 * [N rows][K] (GGUF ne={K,N}), an activation x is [M][K], an output y is [M][N].
 */
#ifndef MG_ORACLE_H
#define MG_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MGO_WTYPE_F32 = 0, MGO_WTYPE_Q8_0 = 8, MGO_WTYPE_Q4_K = 12 };

/* ---- IEEE binary16 <-> binary32 (round to nearest even) ---- */
uint16_t mgo_f32_to_f16(float f);
float    mgo_f16_to_f32(uint16_t h);
void     mgo_f32_to_f16_array(const float* x, uint16_t* h, size_t n);
void     mgo_f16_to_f32_array(const uint16_t* h, float* x, size_t n);
/* round every element to the nearest fp16 value and back (used for fp16 K/V) */
void     mgo_round_f16_array(const float* x, float* y, size_t n);

/* ---- weight block formats ---- */
size_t mgo_q8_0_row_bytes(int64_t K);   /* (K/32)*34  */
size_t mgo_q4_k_row_bytes(int64_t K);   /* (K/256)*144 */
/* tools/convert_to_gguf.py:109-124 (quant_q8_0) */
void mgo_quantize_q8_0(const float* w, int64_t N, int64_t K, uint8_t* out);
/* tools/convert_to_gguf.py:68-106 (quant_q4_k) */
void mgo_quantize_q4_k(const float* w, int64_t N, int64_t K, uint8_t* out);
/* src/mg-opencl/mg-opencl.cpp:178-184 (q4k_sm = ggml get_scale_min_k4) */
void mgo_q4k_scale_min(const uint8_t* scales12, int j, uint8_t* sc, uint8_t* m);
/* dequantize to fp32 rows: mg-opencl.cpp:386-387 (DEQ_Q8) and :252-262 (deq_q4k_elem) */
void mgo_dequant(int wtype, const uint8_t* w, int64_t N, int64_t K, float* out);

/* ---- activation quantizer: mg-opencl.cpp:424-434 (k_quantize_q8) ----
 * qx int8 [M][K], dx fp32 [M][K/32]; sx (nullable) int32 [M][K/32] = sum of qx per block */
void mgo_quantize_act_q8(const float* x, int64_t M, int64_t K, int8_t* qx, float* dx, int32_t* sx);

/* ---- exact int32 per-block dot products, out[m][n][t] ----
 * Q8_0: sum_i qw[n,t,i]*qx[m,32t+i] (mg-opencl.cpp:472-478);
 * Q4_K: nibble (0..15) * qx (mg-opencl.cpp:571-576). */
void mgo_block_dots(int wtype, const uint8_t* w, int64_t N, int64_t K,
                    const int8_t* qx, int64_t M, int32_t* out);

/* ---- int8-dot GEMM with fused epilogue ----
 * Q8_0: mg-opencl.cpp:440-494 (k_mul_mat_q8_i8); Q4_K: :504-590 (k_mul_mat_q4k_i8).
 * y[m][n] = act(sum_t scale_t * idot_t + bias[n]) + resid[m][n]; bias/resid nullable. */
void mgo_gemm_q_i8(int wtype, const uint8_t* w, int64_t N, int64_t K,
                   const int8_t* qx, const float* dx, int64_t M,
                   const float* bias, int act, const float* resid, float* y);

/* ---- F32 GEMM with fused epilogue: src/mg-cpu/mg-cpu.cpp:48-72 (k_mul_mat) ----
 * w fp32 [N][K]; sequential k accumulation in fp32. */
void mgo_gemm_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M,
                  const float* bias, int act, const float* resid, float* y);
/* dequantize-then-F32 semantics (the reference's non-arm_dot path, mg-opencl.cpp:1400-1423):
 * mgo_dequant followed by mgo_gemm_f32. */
void mgo_gemm_q_deq_f32(int wtype, const uint8_t* w, int64_t N, int64_t K, const float* x,
                        int64_t M, const float* bias, int act, const float* resid, float* y);

/* epilogue activation: mg-opencl.cpp:36-40, mg-cpu.cpp:64-66 (0 none, 1 erf-GELU, 2 SiLU) */
float mgo_act(float v, int act);

/* ---- LayerNorm + affine: mg-cpu.cpp:105-121 (double stats) + :249-261 (affine) ---- */
void mgo_layernorm_affine(const float* x, const float* gamma, const float* beta,
                          int64_t rows, int64_t D, float eps, float* y);

/* ---- attention: mg-cpu.cpp:211-239 (k_flash_attention) on strided {D,S,H,B} views.
 * strides[4] are element strides of q/k/v (mg-opencl.cpp:1493-1496). f16kv != 0 rounds
 * q, k and v to fp16 first (mg-opencl.cpp:859-937, k_flash_attention_h).
 * Output is contiguous {D,S,H,B}: o[((b*H+h)*S+s)*D+d]. */
void mgo_attention(const float* q, const float* k, const float* v, const int64_t strides[4],
                   int64_t D, int64_t S, int64_t H, int64_t B, float scale, int f16kv, float* o);

/* ---- glue ops ---- */
/* mg-cpu.cpp:74-86 (k_get_rows): rows of a[R][E] by ids; negative id wraps */
void mgo_get_rows(const float* a, int64_t E, int64_t R, const int32_t* ids, int64_t n, float* o);
/* cont(permute({D,S,H,B},0,2,1,3)) -> {D,H,S,B}: mg-transformer.cpp:84-85, mg-cpu.cpp:198-209 */
void mgo_merge_heads(const float* a, int64_t D, int64_t S, int64_t H, int64_t B, float* o);

/* library self-description */
/* VQGAN int8 conv (mg-opencl.cpp:598-664): k_quantize_conv_w quantizes each output channel's
 * weights ker[oc][k] (k = (ic*KH + kh)*KW + kw) per 32-block: qw [OC][nb*32] (zero past K),
 * dw [OC][nb]; k_conv2d_i8 quantizes the gathered im2col column of every output pixel per
 * 32-block of k (zero outside the image and past K) and sums acc = acc + (dx*dw)*idot over the
 * blocks in order; out {OW, OH, OC, N}. */
void mgo_conv_quant_w(const float* ker, int64_t OC, int64_t K, int8_t* qw, float* dw);
void mgo_conv2d_i8(const float* in, int64_t IW, int64_t IH, int64_t IC, int64_t N, const int8_t* qw,
                   const float* dw, int64_t KW, int64_t KH, int64_t OC, int stride, int pad, float* out);

int mgo_version(void);

/* ---- iterative decoding (mg_oracle_decode.cpp; src/mg-generate.cpp:82-121) ----
 * std::mt19937_64 / std::uniform_real_distribution<double> exactly as the reference calls them */
void mgo_mt64_draws(uint64_t seed, int64_t n, uint64_t* out);
void mgo_uniform_draws(uint64_t seed, double a, double b, int64_t n, double* out);
void mgo_decode_step(const float* logits, int B, int S, int V, int CB, int mask_id, int n_tokens,
                     int step, int n_steps, float choice_temp, const uint64_t* seeds,
                     int64_t draws_before, int32_t* tokens, int32_t* result);

#ifdef __cplusplus
}
#endif
#endif
