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
    const void* qx16;      // activation codes as fp16 [M][K] (k_gemm_q_f16x operand)
    const float* x;        // fp32 activations (dequant-f16 path)
    const float* bias;
    const float* resid;
    float* y;
    int32_t* dots;         // debug: [M][N][K/32] int32 block dot products
    int M, N, K;
    int act;
};

// Tile configuration chosen by the dispatcher (see mgh_api.cpp: pick_tile()).
struct TileCfg {
    int wm, wn;            // 32x32 MFMA tiles per wave along M and N (2x2 waves per WG)
};

hipError_t launch_quantize_act_q8(const float* x, int8_t* qx, float* dx, int32_t* sx,
                                  int64_t M, int64_t K, hipStream_t s);
hipError_t launch_quantize_act_q8_f16(const float* x, _Float16* qx16, float* dx, int32_t* sx,
                                      int64_t M, int64_t K, hipStream_t s);
hipError_t launch_i8_to_f16(const int8_t* q, _Float16* h, size_t n, hipStream_t s);
hipError_t launch_gemm_q_i8(int wtype, const GemmArgs& a, TileCfg t, bool debug_dots,
                            hipStream_t s);
// Production kernel for K % 256 == 0, N % 4 == 0, 16-byte aligned operands: fp16-code
// activations (qx16), 16x16x32 fp16 MFMA block dots.
hipError_t launch_gemm_q_f16x(int wtype, const GemmArgs& a, bool debug_dots, hipStream_t s);
// Streamed variant for K % 256 == 0 with 16-byte aligned qx/dx/sx/w (64x64 tiles).
hipError_t launch_gemm_q_i8_s256(int wtype, const GemmArgs& a, bool debug_dots, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s);

}  // namespace mgh
