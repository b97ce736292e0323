// mgh_kernels.h — host-side launchers for the gfx950 kernels (internal to libmgh).
// Every launcher enqueues on `stream`, checks nothing but its own launch status, and
// returns the hipError_t of the launch. Argument validation lives in mgh_api.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgh {

// Arguments of the block-quantized GEMMs. Shapes follow the reference convention
// (include/mg-tensor.hpp:3-13): w has N rows of K weights in ggml blocks, x/qx is [M][K],
// y/resid are [M][N], bias is [N], dx/sx are [M][K/32].
struct GemmArgs {
    const uint8_t* w;
    const int8_t* qx;
    const float* dx;
    const int32_t* sx;
    const void* qx16;      // activation codes as fp16 [M][K] (k_gemm_qp operand)
    const float* x;        // fp32 activations (dequant-f16 path)
    const float* ux;       // Q4_K min-term activation factor [M][K/32] in fp32 (dequant-f16
                           // path: block sums of the fp16 activations); null: dx * sx
    const float* bias;
    const float* resid;
    float* y;
    int32_t* dots;         // debug: [M][N][K/32] int32 block dot products
    float* ws;             // split-K partial tiles (k_gemm_qp, splits > 1)
    int M, N, K;
    int act;
    int splits;            // K splits of k_gemm_qp (0 or 1: none)
};

// Tile configuration chosen by the dispatcher (see mgh_api.cpp: pick_tile()).
struct TileCfg {
    int wm, wn;            // 32x32 MFMA tiles per wave along M and N (2x2 waves per WG)
};

hipError_t launch_quantize_act_q8(const float* x, int8_t* qx, float* dx, int32_t* sx,
                                  int64_t M, int64_t K, hipStream_t s);
hipError_t launch_quantize_act_q8_f16(const float* x, _Float16* qx16, float* dx, int32_t* sx,
                                      int64_t M, int64_t K, hipStream_t s);
hipError_t launch_round_act_f16(const float* x, _Float16* x16, float* ones, float* ux,
                                int64_t M, int64_t K, hipStream_t s);
hipError_t launch_gemm_q_i8(int wtype, const GemmArgs& a, TileCfg t, bool debug_dots,
                            hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s);

// LayerNorm + affine over rows of D (D % 256 == 0, D <= 2048); emit 0: y only, 1: also the
// int8-dot operand (fp16 codes, dx, int32 sx) of y, 2: also the dequant-fp16 operand
// (fp16 y, unit dx, fp32 ux).
hipError_t launch_layernorm_affine(const float* x, const float* gamma, const float* beta, float* y,
                                   int rows, int D, float eps, int emit, void* codes, float* dx,
                                   void* s4, hipStream_t s);

// Flash attention with fp16 K/V over strided {D,S,H,B} views (element strides).
struct FaArgs {
    const float* q;
    const float* k;
    const float* v;
    const _Float16* q16;   // fp16 q/k/v instead of q/k/v when set (whole-head kernel only)
    const _Float16* k16;
    const _Float16* v16;
    float* o;
    _Float16* o16;         // fp16 output instead of o when set
    int64_t st[4];         // q/k/v element strides for d, s, h, b
    int64_t os[4];         // output element strides for d, s, h, b
    int S, H, B;
    float scale;
};
hipError_t launch_flash_attn_f16kv(const FaArgs& a, int D, hipStream_t s);

// fp32 GEMM with the fused epilogue: y[M][N] = act(x[M][K] . w[N][K]^T + bias) + resid.
struct GemmF32Args {
    const float* w;
    const float* x;
    const float* bias;
    const float* resid;
    float* y;
    int M, N, K;
    int act;
};
hipError_t launch_gemm_f32(const GemmF32Args& a, hipStream_t s);

// Graph glue: row gather, broadcast add, strided 4-D copy into a contiguous buffer.
struct CopyArgs {
    int64_t ne[4];         // output shape (contiguous)
    int64_t st[4];         // source element strides
};
hipError_t launch_get_rows(const float* a, int64_t E, int64_t R, const int32_t* ids, int64_t n,
                           float* out, hipStream_t s);
hipError_t launch_add_bcast(const float* a, const float* b, int64_t nb, float* out, int64_t n,
                            hipStream_t s);
hipError_t launch_copy4d(const float* a, const CopyArgs& c, float* out, hipStream_t s);
// Remaining F32 graph ops (k_ops.hip). Element strides throughout; out is contiguous.
struct BinaryArgs {
    int64_t ne[4];         // output shape
    int64_t as[4];         // a strides
    int64_t bne[4];        // b shape (each dim equal to ne or 1: broadcast)
    int64_t bs[4];         // b strides
};
struct BatchedGemmArgs {
    const float* w;        // {K, N, wne2, wne3} with strides ws
    const float* x;        // {K, M, B2, B3} with strides xs
    const float* bias;     // [N] or null
    const float* resid;    // [B3][B2][M][N] or null
    float* y;              // [B3][B2][M][N]
    int64_t K, N, M, B2, B3, wne2, wne3;
    int64_t ws[4], xs[4];
    int act;
};
hipError_t launch_softmax_rows(const float* x, int64_t rows, int D, float scale, float* y, hipStream_t s);
hipError_t launch_binary(int op, const float* a, const float* b, const BinaryArgs& p, float* out, hipStream_t s);
// op 0: y = x * sc; 1: GELU (erf); 2: SiLU
hipError_t launch_unary(int op, const float* x, int64_t n, float sc, float* y, hipStream_t s);
hipError_t launch_gemm_f32_batched(const BatchedGemmArgs& a, hipStream_t s);

// Weight repack (k_pack_w.hip): raw Q8_0/Q4_K -> fp16 codes [N][K] | fp32 scale [K/32][N]
// (| fp32 min [N][K/32] for Q4_K).
size_t packed_weight_bytes(int wtype, int64_t N, int64_t K);
hipError_t launch_pack_weights(int wtype, const void* w, void* out, int N, int K, hipStream_t s);
// GEMM on packed weights (a.w) and fp16-code activations (a.qx16): K % 64 == 0, N % 4 == 0,
// 16-byte aligned w/qx16/bias/resid/y.
hipError_t launch_gemm_qp(int wtype, const GemmArgs& a, bool debug_dots, hipStream_t s);
// Split-K plan of k_gemm_qp for a shape: activation tile rows, number of K splits and the
// bytes of partial tiles the splits write (then reduced by a second, stream-ordered kernel).
struct QpPlan {
    int bm, splits;
    size_t ws_bytes;
};
QpPlan gemm_qp_plan(int M, int N, int K);

// Iterative decoding (k_decode.hip). Per image: mt19937_64 state (312 words + index) in
// `state`; per step 2*S engine outputs, softmax/categorical per position, confidence and
// re-mask per image. The launcher carves draws/sampled/selp out of `work`.
struct DecodeArgs {
    const float* logits;   // [B][S][V]
    int32_t* tokens;       // [B][S] in/out
    int32_t* result;       // [B][S] samples before re-masking
    uint64_t* draws;       // [B][2S]
    int32_t* sampled;      // [B][S]
    float* selp;           // [B][S]
    int B, S, V, CB, mask_id, n_tokens, step, n_steps;
    float choice_temp;
};
size_t decode_state_bytes(int B);
size_t decode_work_bytes(int B, int S);
// seeds are read from word 0 of each image's state block (the caller puts them there)
hipError_t launch_decode_seed(int B, void* state, hipStream_t s);
hipError_t launch_decode_step(DecodeArgs a, void* state, void* work, hipStream_t s);

// Dequantize-fused fp16 path (k_gemm_fc.hip): weights dequantized once into fp16 [N][K],
// fp16 activations, fp32 accumulation, y = act(x . w^T + bias) + resid. K % 64 == 0,
// N % 4 == 0, 16-byte aligned operands.
struct GemmH16Args {
    const _Float16* x;     // [M][K] fp16 activations, or
    const float* xf;       // [M][K] fp32 activations rounded to fp16 in the kernel (x unused)
    const void* w;         // wq 0: fp16 [N][K]; wq 8 / 12: the K-loop-dequant layout of
                           // launch_pack_weights_dq (Q8_0 / Q4_K bytes, GGUF-sized)
    int wq;                // weight form: 0 fp16, 8 Q8_0, 12 Q4_K
    const float* bias;     // [N] or null
    const float* resid;    // [M][N] or null
    float* y;              // [M][N]
    _Float16* y16;         // [M][N] fp16 output instead of y when set
    float* ws;             // split-K partial tiles (H16Plan::ws_bytes)
    int M, N, K, splits, act;
    int ph;                // tile order: panels of ph activation-row tiles (set from the plan)
};
struct H16Plan {
    int bm, bn, wmr;       // activation / weight tile rows, waves along the activation rows
    int splits, ns;        // K splits, K-stage ring depth
    int ph;                // tile order: panel height in activation-row tiles
    size_t ws_bytes;
};
H16Plan gemm_h16_plan(int M, int N, int K, bool xf32, int wq);
// LayerNorm-affine of a GEMM's output rows taken by the split-K reduce (k_gemm_fc_reduce_ln):
// gamma/beta [N] and the LayerNorm outputs as launch_layernorm_affine takes them
struct LnArgs {
    const float* gamma;
    const float* beta;
    float eps;
    float* y;              // [M][N] fp32
    int emit;              // MGH_EMIT_* operand written alongside y
    void* codes;
    float* dx;
    void* s4;
};
size_t packed_weight_bytes_f16(int64_t N, int64_t K);
hipError_t launch_pack_weights_f16(int wtype, const void* w, void* out, int N, int K, hipStream_t s);
// K-loop-dequant weight layout (the operand of the wq = 8 / 12 forms of k_gemm_fc and
// k_gemv_fc): the GGUF bytes regrouped into 16-row groups and 64-deep K stages, so that one
// 16-byte-per-lane DMA moves whole MFMA fragments; the same byte count per weight as the GGUF
// blocks (Q8_0 1.0625, Q4_K 0.5625) for N % 16 == 0, rows padded to a multiple of 16.
//   Q8_0: codes [G][K/64][2][4][16][8] u8 (q + 128), then scales [G][K/64][2][16] fp16
//   Q4_K: nibbles [G][K/64][2][4][16][4] (byte e: element e low, e + 4 high), then the raw
//         16-byte super-block headers (d, dmin, packed 6-bit scales) [G][K/256][16][16]
// with G = ceil(N / 16) row groups; [2][4][16] = K half, 8-wide K slice, row in the group.
// raw Q8_0 / Q4_K blocks -> fp32 [N][K] (any N, K % 32 resp. % 256; any byte alignment)
hipError_t launch_dequant_weights_f32(int wtype, const void* w, float* out, int N, int K, hipStream_t s);
size_t packed_weight_bytes_dq(int wtype, int64_t N, int64_t K);
hipError_t launch_pack_weights_dq(int wtype, const void* w, void* out, int N, int K, hipStream_t s);
hipError_t launch_f32_to_f16(const float* x, _Float16* h, int64_t n, hipStream_t s);
// ln: the split-K reduce also writes the LayerNorm-affine of y's rows (the plan must split K;
// act 0, fp32 y, N % 256 == 0, N <= 2048). N <= kFcMaxN: the tiled epilogue addresses a tile's
// outputs with 32-bit offsets from its origin.
constexpr int kFcMaxN = 1 << 21;
hipError_t launch_gemm_h16(const H16Plan& p, const GemmH16Args& a, hipStream_t s, const LnArgs* ln = nullptr);
// skinny-M form of the same product (1 <= M <= kGemvMaxRows; no workspace), and the rule that
// picks it over the tiled plan
constexpr int kGemvMaxRows = 32;
bool use_gemv_h16(int M, int K);
hipError_t launch_gemv_h16(const GemmH16Args& a, hipStream_t s);

// Scratch of the no-allocation entry point (noalloc.hip): the device address of this device's
// copy of a fixed-size file-scope array, looked up once per device.
// VQGAN decoder ops (k_vqgan.hip); layouts {W, H, C, N}, W innermost, contiguous
struct ConvArgs {
    const float* in;       // {IW, IH, IC, N}
    const float* ker;      // {KW, KH, IC, OC}
    float* out;            // {OW, OH, OC, N}
    int IW, IH, IC, OW, OH, OC, KW, KH, stride, pad, N;
    const float* bias;     // [OC] or null: out = conv + bias
    const float* resid;    // shape of out or null: then + resid
};
constexpr int kConvFewMax = 8;      // OC up to this: the one-thread-per-pixel kernel
// the reference-layout kernels (IC % 16 != 0): one thread per pixel for OC <= kConvFewMax,
// else the 64 x 64 fp32-MFMA implicit GEMM
hipError_t launch_conv2d_f32(const ConvArgs& a, hipStream_t s);

// packed-weight fp32-MFMA implicit GEMM for IC % 16 == 0 (wpk from launch_conv_pack): tiles of
// 128 pixels x 128 channels, or 256 x 16 when OC <= 16 (conv_pk_narrow)
struct ConvPkArgs {
    const float* in;
    const float* wpk;      // [OC][KH][KW][IC]
    float* out;
    const float* bias;
    const float* resid;
    int IW, IH, IC, OW, OH, OC, KW, KH, stride, pad, N;
    int splits, kps;       // set by the launcher
};
struct ConvPkPlan {
    int splits, kps;       // K split into `splits` ranges of kps values (a multiple of 16)
};
bool conv_pk_narrow(int OC);
ConvPkPlan conv_pk_plan(int M, int OC, int K);   // per image: independent of the batch
size_t conv_pk_ws_bytes(int M, int OC, int N, int K);    // split-K partials, 0 without a split
hipError_t launch_conv_pack(const float* ker, float* wpk, int IC, int taps, int OC, hipStream_t s);
hipError_t launch_conv2d_pk(const ConvPkArgs& a, float* ws, hipStream_t s);
// int8 conv (the reference's k_conv2d_i8): weights from launch_conv_quant_w — int8 codes in
// fragment order [ceil(OC/16)][blocks][16][32] (conv_i8_codes_bytes, 256-byte aligned), then
// fp32 scales [ceil(OC/16)][blocks][16]; qa / dxa: the workspace of conv_i8_ws_bytes (the
// im2col codes [N][ceil(M/16)][blocks][16][32], then their scales [N][ceil(M/16)][blocks][16])
struct ConvI8Args {
    const float* in;
    const int8_t* qw;
    const float* dw;
    float* out;
    const float* bias;
    const float* resid;
    int8_t* qa;
    float* dxa;
    int IW, IH, IC, OW, OH, OC, KW, KH, stride, pad, N;
};
size_t conv_i8_codes_bytes(int K, int OC);
size_t conv_i8_weight_bytes(int K, int OC);
size_t conv_i8_ws_codes_bytes(int M, int K, int N);   // the workspace's codes, 256-byte aligned
size_t conv_i8_ws_bytes(int M, int K, int N);
hipError_t launch_conv_quant_w(const float* ker, void* wq, int K, int OC, hipStream_t s);
// true: launch_conv2d_i8 runs the one-pass kernel, which needs no workspace (qa / dxa unused)
bool conv_i8_one_pass(int IW, int IH, int IC, int OW, int OH, int OC, int KW, int KH, int N);
hipError_t launch_conv2d_i8(const ConvI8Args& a, hipStream_t s);
size_t group_norm_ws_bytes(int64_t W, int64_t H, int C, int N, int G);
hipError_t launch_group_norm(const float* x, int64_t W, int64_t H, int C, int N, int G, float eps,
                             const float* gamma, const float* beta, float* y, void* ws, hipStream_t s);
hipError_t launch_upscale(const float* x, int IW, int IH, int64_t CN, int f, float* y, hipStream_t s);

size_t noalloc_scratch_bytes();
hipError_t noalloc_scratch(int device, void** out);
// order a call's launches on `s` after the previous call's on this device (event wait; takes a
// host lock), then (end) record the event after them and release the lock; *capturing: `s` is
// under stream capture, where neither is done. end must follow every successful begin.
hipError_t noalloc_order_begin(int device, hipStream_t s, bool* capturing);
hipError_t noalloc_order_end(int device, hipStream_t s, bool capturing);

}  // namespace mgh
