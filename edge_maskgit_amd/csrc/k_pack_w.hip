// k_pack_w.hip — one-time repack of GGUF Q8_0 / Q4_K weight tensors into the device-native
// layout the packed GEMM (k_gemm_qp.hip) streams.
//
// The GGUF block formats (reference include/mg-tensor.hpp:3-13, src/mg-model.cpp:22 and the
// block decoders in src/mg-opencl/mg-opencl.cpp:440-494 / :504-590):
//   Q8_0: 34-byte blocks of 32 values {fp16 d; int8 qs[32]};      w = d * q
//   Q4_K: 144-byte super-blocks of 256 {fp16 d, dmin; u8 scales[12]; u8 qs[128]}; sub-block j
//         (32 values) has 6-bit (sc_j, m_j) packed in scales[] and 4-bit q in the low (j even)
//         or high (j odd) nibbles of qs[32*(j/2) .. +32];           w = d*sc_j * q - dmin*m_j
// Packed layout for N rows of K weights, T = K/32 blocks per row (byte offsets):
//   [0, 2NK)              codes  fp16 [N][K]   the integer q (exact in fp16)
//   [2NK, 2NK+4NT)        scale  fp32 [T][N]   Q8_0: d;  Q4_K: d*sc_j (the reference's fp32 product)
//                                              block-major: a K stage's scales of consecutive
//                                              rows are contiguous for the GEMM's stream
//   [2NK+4NT, 2NK+8NT)    min    fp32 [N][T]   Q4_K only: dmin*m_j (read once per output tile)
// The products d*sc_j and dmin*m_j are formed once here in fp32 exactly as the reference
// kernel forms them per use, so the GEMM applies the same fp32 values.
// The GEMM streams fp16 codes and fp32 scales with aligned 16-byte loads straight into LDS;
// the 34-byte Q8_0 blocks and the nibble/6-bit packing of Q4_K never reach the inner loop.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

__device__ __forceinline__ uint32_t f16_bits(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

// One thread per 32-value block: 64 bytes of codes (4 x 16-byte stores) and its scale(s).
template <int WTYPE>
__global__ __launch_bounds__(256) void k_pack_w(const uint8_t* __restrict__ w, uint8_t* __restrict__ out,
                                                int N, int K) {
    const int T = K / 32;
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (int64_t)N * T) return;
    const int64_t n = blk / T;
    const int t = (int)(blk - n * T);
    uint16_t* codes = (uint16_t*)out + n * K + (int64_t)t * 32;
    float* scale = (float*)(out + (size_t)2 * N * K) + (int64_t)t * N + n;
    uint32_t c[16];
    if (WTYPE == 8) {
        const uint8_t* b = w + blk * 34;
        *scale = h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
#pragma unroll
        for (int i = 0; i < 16; i++)
            c[i] = f16_bits((float)(int8_t)b[2 + 2 * i]) | (f16_bits((float)(int8_t)b[3 + 2 * i]) << 16);
    } else {
        const uint8_t* sb = w + (n * (T / 8) + t / 8) * 144;
        const int j = t & 7;
        const uint8_t* sc12 = sb + 4;
        uint32_t sc, mn;
        if (j < 4) {
            sc = sc12[j] & 63u;
            mn = sc12[j + 4] & 63u;
        } else {
            sc = (sc12[j + 4] & 0xFu) | ((uint32_t)(sc12[j - 4] >> 6) << 4);
            mn = (uint32_t)(sc12[j + 4] >> 4) | ((uint32_t)(sc12[j] >> 6) << 4);
        }
        const float d = h2f((uint32_t)sb[0] | ((uint32_t)sb[1] << 8));
        const float dmin = h2f((uint32_t)sb[2] | ((uint32_t)sb[3] << 8));
        *scale = d * (float)sc;
        float* mins = (float*)(out + (size_t)2 * N * K + (size_t)4 * N * T) + blk;
        *mins = dmin * (float)mn;
        const uint8_t* qs = sb + 16 + 32 * (j >> 1);
        const int sh = 4 * (j & 1);
#pragma unroll
        for (int i = 0; i < 16; i++)
            c[i] = f16_bits((float)((qs[2 * i] >> sh) & 15)) | (f16_bits((float)((qs[2 * i + 1] >> sh) & 15)) << 16);
    }
    u32x4* dst = (u32x4*)codes;
#pragma unroll
    for (int i = 0; i < 4; i++) dst[i] = u32x4{c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]};
}

}  // namespace

size_t packed_weight_bytes(int wtype, int64_t N, int64_t K) {
    const int64_t T = K / 32;
    return (size_t)(2 * N * K + 4 * N * T + (wtype == 12 ? 4 * N * T : 0));
}

hipError_t launch_pack_weights(int wtype, const void* w, void* out, int N, int K, hipStream_t s) {
    const int64_t blocks = (int64_t)N * (K / 32);
    if (blocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
    if (wtype == 8)
        hipLaunchKernelGGL(k_pack_w<8>, grid, block, 0, s, (const uint8_t*)w, (uint8_t*)out, N, K);
    else if (wtype == 12)
        hipLaunchKernelGGL(k_pack_w<12>, grid, block, 0, s, (const uint8_t*)w, (uint8_t*)out, N, K);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace mgh
