// k_conv_i8.hip — the reference's int8 conv on gfx950: weight quantization, the quantized
// im2col pass and the block-scaled exact int8 MFMA GEMM (k_quantize_conv_w + k_conv2d_i8,
// src/mg-opencl/mg-opencl.cpp:598-664). Built with MFMA results in VGPRs (-amdgpu-mfma-vgpr-form):
// every block's int32 dots are read once by the scale arithmetic, and accumulation registers
// would cost a v_accvgpr_read per value.
#include <algorithm>

#include "k_conv_common.h"
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

// ---- int8 conv: the reference's k_quantize_conv_w + k_conv2d_i8 (mg-opencl.cpp:598-664) ----
// Codes and scales are kept in the fragment order of v_mfma_i32_16x16x32_i8: a 16 x 32 int8
// tile is 512 contiguous bytes (row r at byte 32r), so lane (l16, lg) reads its operand as the
// 8 bytes at 32*l16 + 8*lg and a wave's load is one contiguous 512-byte run.
//   weights      codes [OT][nb][16][32] int8, scales [OT][nb][16] fp32: channel 16*ot + row,
//                OT = ceil(OC/16); zero codes and scales past OC and past K
//   activations  codes [N][PT][nb][16][32] int8, scales [N][PT][nb][16] fp32 (the call's
//                workspace): pixel 16*pt + row, PT = ceil(M/16); zero past M and past K
// Both are quantized per row and 32-block of k = (ic*KH + kh)*KW + kw: d = amax/127,
// id = d > 0 ? 1/d : 0, code = round(v*id) half away from zero (k_quantize_conv_w :598-607 and
// the quantizer inside k_conv2d_i8 :637-641).

__device__ __forceinline__ uint32_t pack_i8x4(float a, float b, float c, float d) {
    return (uint32_t)(uint8_t)(int8_t)(int)a | (uint32_t)(uint8_t)(int8_t)(int)b << 8 |
           (uint32_t)(uint8_t)(int8_t)(int)c << 16 | (uint32_t)(uint8_t)(int8_t)(int)d << 24;
}

// One thread per (channel, block) of the padded channel range; runs once per weight.
__global__ __launch_bounds__(256) void k_conv_quant_w(const float* __restrict__ ker, int8_t* __restrict__ qw,
                                                      float* __restrict__ dw, int K, int OC, int OT, int nb) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (int64_t)OT * 16 * nb) return;
    const int oc = (int)(gid / nb), b = (int)(gid - (int64_t)oc * nb);
    const int k0 = 32 * b, n = oc < OC ? min(32, K - k0) : 0;
    const float* w = ker + (size_t)(oc < OC ? oc : 0) * K + k0;
    float v[32];
    float amax = 0.f;
    for (int i = 0; i < 32; i++) {
        v[i] = i < n ? w[i] : 0.f;
        amax = fmaxf(amax, fabsf(v[i]));
    }
    const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
    const size_t frag = (size_t)(oc >> 4) * nb + b;
    dw[frag * 16 + (oc & 15)] = d;
    u32x4* q = (u32x4*)(qw + frag * 512 + (oc & 15) * 32);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        u32x4 u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float* x = v + 16 * h + 4 * e;
            u[e] = pack_i8x4(roundf(x[0] * id), roundf(x[1] * id), roundf(x[2] * id), roundf(x[3] * id));
        }
        q[h] = u;
    }
}

// Pass 1: the im2col matrix quantized, one (image, 16-pixel tile, block) fragment per wave and
// four consecutive blocks per workgroup. Lane (l16, lg) gathers the 8 values k = 32b + 8lg ..
// +7 of pixel l16 (zero outside the image and past K), the block max of a pixel is two xor
// shuffles over its four lanes, and the lane stores its 8 codes where the GEMM's lane (l16, lg)
// reads them.
template <int KSZ>
__global__ __launch_bounds__(256) void k_conv_im2col_q8(ConvI8Args a) {
#pragma clang fp contract(off)
    const int KW = KSZ ? KSZ : a.KW, KH = KSZ ? KSZ : a.KH, KK = KW * KH;
    const int M = a.OW * a.OH, K = a.IC * KK, nb = (K + 31) / 32, PT = (M + 15) / 16;
    const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
    const int b = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;                        // whole waves: the kernel has no barriers
    const int pt = blockIdx.x, n = blockIdx.z, p = pt * 16 + l16;
    const bool pv = p < M;
    const int ow = pv ? p % a.OW : 0, oh = pv ? p / a.OW : 0;
    const int iw0 = ow * a.stride - a.pad, ih0 = oh * a.stride - a.pad;
    const size_t plane = (size_t)a.IW * a.IH;
    const float* inb = a.in + (size_t)n * a.IC * plane;
    const int k = 32 * b + 8 * lg;
    int ic = k / KK, t = k - ic * KK, kh = t / KW, kw = t - kh * KW;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int ih = ih0 + kh, iw = iw0 + kw;
        v[j] = pv && k + j < K && ih >= 0 && ih < a.IH && iw >= 0 && iw < a.IW
                   ? inb[(size_t)ic * plane + (size_t)ih * a.IW + iw] : 0.f;
        if (++kw == KW) {
            kw = 0;
            if (++kh == KH) {
                kh = 0;
                ic++;
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
    const size_t frag = ((size_t)n * PT + pt) * nb + b;
    uint2 u;
    u.x = pack_i8x4(roundf(v[0] * id), roundf(v[1] * id), roundf(v[2] * id), roundf(v[3] * id));
    u.y = pack_i8x4(roundf(v[4] * id), roundf(v[5] * id), roundf(v[6] * id), roundf(v[7] * id));
    *(uint2*)(a.qa + frag * 512 + l16 * 32 + 8 * lg) = u;
    if (lg == 0) a.dxa[frag * 16 + l16] = d;
}

// Pass 1 for 1 x 1 and 3 x 3 kernels (per-image input below 2 GiB): one lane per output pixel,
// the 32 values of a block in its registers. A block covers 32 consecutive k = 9*ic + tap
// (3 x 3) or k = ic (1 x 1); for 3 x 3 its (channel, tap) pattern repeats with period 9 blocks,
// so each phase b % 9 has its own fully unrolled body and every tap index is a constant. The
// lane's tap offsets are computed once; a tap outside the image gets offset 0x80000000, past
// the buffer's range, which the raw buffer load returns as 0 (no branch per value). The channel
// offset goes into the load's scalar offset. Rounding: for |y| < 2^23,
// (int)(y + copysign(0x1.fffffep-2f, y)) equals (int)roundf(y) (checked exhaustively over all
// such floats of both signs), three operations instead of roundf's six.
__device__ __forceinline__ int round_half_away(float y) {
#pragma clang fp contract(off)
    return (int)(y + __builtin_copysignf(0x1.fffffep-2f, y));
}

template <int KSZ, int PH, bool FULL>
__device__ __forceinline__ void gather_block(float (&v)[32], __amdgpu_buffer_rsrc_t rs, const uint32_t (&toff)[KSZ * KSZ],
                                             int b, int IC, int plane4) {
    constexpr int KK = KSZ * KSZ, R0 = KK == 1 ? 0 : (32 * PH) % KK;
    const int ic0 = (32 * b - R0) / KK;        // channel of the block's first value
#pragma unroll
    for (int e = 0; e < 32; e++) {
        const int kk = R0 + e, icr = kk / KK, t = kk % KK;
        const int ic = ic0 + icr;
        v[e] = FULL || ic < IC ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)toff[t], ic * plane4, 0))
                               : 0.f;
    }
}

template <int KSZ, int PH>
__device__ __forceinline__ void gather_phase(float (&v)[32], __amdgpu_buffer_rsrc_t rs, const uint32_t (&toff)[KSZ * KSZ],
                                             int b, int IC, int K, int plane4) {
    if (32 * b + 32 <= K) gather_block<KSZ, PH, true>(v, rs, toff, b, IC, plane4);
    else gather_block<KSZ, PH, false>(v, rs, toff, b, IC, plane4);
}

template <int KSZ>
__global__ __launch_bounds__(256) void k_conv_im2col_q8p(ConvI8Args a, int bpw) {
#pragma clang fp contract(off)
    constexpr int KK = KSZ * KSZ;
    const int M = a.OW * a.OH, K = a.IC * KK, nb = (K + 31) / 32, PT = (M + 15) / 16;
    const int p = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    const int n = blockIdx.z, b0 = blockIdx.y * bpw, b1 = min(nb, b0 + bpw);
    const bool pv = p < M;
    const int ow = pv ? p % a.OW : 0, oh = pv ? p / a.OW : 0;
    const int iw0 = ow * a.stride - a.pad, ih0 = oh * a.stride - a.pad;
    uint32_t toff[KK];
#pragma unroll
    for (int kh = 0; kh < KSZ; kh++)
#pragma unroll
        for (int kw = 0; kw < KSZ; kw++) {
            const int ih = ih0 + kh, iw = iw0 + kw;
            toff[kh * KSZ + kw] = pv && ih >= 0 && ih < a.IH && iw >= 0 && iw < a.IW
                                      ? (uint32_t)(ih * a.IW + iw) * 4u : 0x80000000u;
        }
    const int plane = a.IW * a.IH;                     // IC * plane * 4 < 2^31 (host check)
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.in + (size_t)n * a.IC * plane), (short)0, a.IC * plane * 4, 0x00020000);
    const bool st = p < 16 * PT;                       // rows of the workspace's last tile
    for (int b = b0; b < b1; b++) {
        float v[32];
        if (KK == 1) {
            gather_phase<KSZ, 0>(v, rs, toff, b, a.IC, K, plane * 4);
        } else {
            switch (b % 9) {
                case 0: gather_phase<KSZ, 0>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 1: gather_phase<KSZ, 1>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 2: gather_phase<KSZ, 2>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 3: gather_phase<KSZ, 3>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 4: gather_phase<KSZ, 4>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 5: gather_phase<KSZ, 5>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 6: gather_phase<KSZ, 6>(v, rs, toff, b, a.IC, K, plane * 4); break;
                case 7: gather_phase<KSZ, 7>(v, rs, toff, b, a.IC, K, plane * 4); break;
                default: gather_phase<KSZ, 8>(v, rs, toff, b, a.IC, K, plane * 4); break;
            }
        }
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(v[e]));
        const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
        u32x4 q[2];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float* x = v + 16 * h + 4 * w;
                q[h][w] = (uint32_t)(uint8_t)round_half_away(x[0] * id) |
                          (uint32_t)(uint8_t)round_half_away(x[1] * id) << 8 |
                          (uint32_t)(uint8_t)round_half_away(x[2] * id) << 16 |
                          (uint32_t)(uint8_t)round_half_away(x[3] * id) << 24;
            }
        if (st) {
            const size_t frag = ((size_t)n * PT + (p >> 4)) * nb + b;
            u32x4* dst = (u32x4*)(a.qa + frag * 512 + (p & 15) * 32);
            __builtin_nontemporal_store(q[0], dst);
            __builtin_nontemporal_store(q[1], dst + 1);
            __builtin_nontemporal_store(d, a.dxa + frag * 16 + (p & 15));
        }
    }
}

// One pass (layers with many output pixels and >= 128 channels): a wave computes 64 output
// pixels x 16*CT channels, quantizing its own im2col rows as k_conv_im2col_q8p does (lane =
// pixel, the block's 32 values in registers, the next block's gathered while this one's
// arithmetic runs) and handing the codes to the MFMA fragments through 2 KB of wave-private
// LDS (each lane writes its pixel's 32 codes as one row, then reads its 8-byte fragment
// pieces), then the same block-scaled exact GEMM as k_conv_i8_gemm. No workspace round trip:
// the codes never reach HBM. Same codes and arithmetic, hence bit-identical results.
template <int KSZ, int CT>
__global__ __launch_bounds__(64) void k_conv_i8_fused(ConvI8Args a) {
#pragma clang fp contract(off)
    constexpr int KK = KSZ * KSZ;
    const int M = a.OW * a.OH, K = a.IC * KK, nb = (K + 31) / 32, OT = (a.OC + 15) / 16;
    const int lane = threadIdx.x, l16 = lane & 15, lg = lane >> 4;
    const int p = blockIdx.x * 64 + lane, ot0 = blockIdx.y * CT, n = blockIdx.z;
    const bool pv = p < M;
    const int ow = pv ? p % a.OW : 0, oh = pv ? p / a.OW : 0;
    const int iw0 = ow * a.stride - a.pad, ih0 = oh * a.stride - a.pad;
    uint32_t toff[KK];
#pragma unroll
    for (int kh = 0; kh < KSZ; kh++)
#pragma unroll
        for (int kw = 0; kw < KSZ; kw++) {
            const int ih = ih0 + kh, iw = iw0 + kw;
            toff[kh * KSZ + kw] = pv && ih >= 0 && ih < a.IH && iw >= 0 && iw < a.IW
                                      ? (uint32_t)(ih * a.IW + iw) * 4u : 0x80000000u;
        }
    const int plane = a.IW * a.IH;                     // IC * plane * 4 < 2^31 (host check)
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.in + (size_t)n * a.IC * plane), (short)0, a.IC * plane * 4, 0x00020000);
    __shared__ __attribute__((aligned(16))) int8_t cs[64 * 32];   // [pixel][32 codes]
    __shared__ __attribute__((aligned(16))) float dsc[64];        // the pixels' block scales
    const int aoff = l16 * 32 + 8 * lg;
    size_t bf[CT];
#pragma unroll
    for (int j = 0; j < CT; j++) bf[j] = (size_t)min(ot0 + j, OT - 1) * nb;
    f32x4 acc[4][CT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < CT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto gather = [&](float (&v)[32], int b) {
        if (KK == 1) {
            gather_phase<KSZ, 0>(v, rs, toff, b, a.IC, K, plane * 4);
            return;
        }
        switch (b % 9) {
            case 0: gather_phase<KSZ, 0>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 1: gather_phase<KSZ, 1>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 2: gather_phase<KSZ, 2>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 3: gather_phase<KSZ, 3>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 4: gather_phase<KSZ, 4>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 5: gather_phase<KSZ, 5>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 6: gather_phase<KSZ, 6>(v, rs, toff, b, a.IC, K, plane * 4); break;
            case 7: gather_phase<KSZ, 7>(v, rs, toff, b, a.IC, K, plane * 4); break;
            default: gather_phase<KSZ, 8>(v, rs, toff, b, a.IC, K, plane * 4); break;
        }
    };
    float v[32];
    gather(v, 0);
    for (int b = 0; b < nb; b++) {
        int64_t B[CT];
        float W[CT];
#pragma unroll
        for (int j = 0; j < CT; j++) {
            B[j] = *(const int64_t*)(a.qw + (bf[j] + b) * 512 + aoff);
            W[j] = a.dw[(bf[j] + b) * 16 + l16];
        }
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(v[e]));
        const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
        u32x4 q[2];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float* x = v + 16 * h + 4 * w;
                q[h][w] = (uint32_t)(uint8_t)round_half_away(x[0] * id) |
                          (uint32_t)(uint8_t)round_half_away(x[1] * id) << 8 |
                          (uint32_t)(uint8_t)round_half_away(x[2] * id) << 16 |
                          (uint32_t)(uint8_t)round_half_away(x[3] * id) << 24;
            }
        if (b + 1 < nb) gather(v, b + 1);
        __syncthreads();                               // the previous block's fragments are read
        *(u32x4*)&cs[lane * 32] = q[0];
        *(u32x4*)&cs[lane * 32 + 16] = q[1];
        dsc[lane] = d;
        __syncthreads();
        int64_t A[4];
        f32x4 X[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            A[i] = *(const int64_t*)&cs[(16 * i + l16) * 32 + 8 * lg];
            X[i] = *(const f32x4*)&dsc[16 * i + 4 * lg];
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < CT; j++) {
                const i32x4 I = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[i], B[j], i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float sc = X[i][r] * W[j];
                    acc[i][j][r] = acc[i][j][r] + sc * (float)I[r];
                }
            }
    }
    // register r of tile (i, j): pixel 64*blockIdx.x + 16i + 4lg + r, channel 16*(ot0 + j) + l16
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < CT; j++) {
            const int oc = 16 * (ot0 + j) + l16;
            if (oc >= a.OC) continue;
            conv_store(a.out, a.bias, a.resid, ((size_t)n * a.OC + oc) * M, oc, blockIdx.x * 64 + 16 * i + 4 * lg, M,
                       acc[i][j]);
        }
}

// Pass 2: one wave computes RT x CT tiles of 16 pixels x 16 channels straight from the
// fragment-ordered codes (no LDS, no barriers). Per block, one v_mfma_i32_16x16x32_i8 per tile
// gives the exact int32 block dots and acc = acc + (dx*dw)*(float)idot, each operation rounded
// to fp32, blocks in order: the reference's `acc += dcm*dwl[nL]*(float)idot` as written (:651).
// The operands of block b + D are loaded while block b is computed (D register stages).
template <int RT, int CT, int D>
__global__ __launch_bounds__(64) void k_conv_i8_gemm(ConvI8Args a) {
#pragma clang fp contract(off)
    const int M = a.OW * a.OH, K = a.IC * a.KW * a.KH, nb = (K + 31) / 32;
    const int PT = (M + 15) / 16, OT = (a.OC + 15) / 16;
    const int lane = threadIdx.x, l16 = lane & 15, lg = lane >> 4;
    const int pt0 = blockIdx.x * RT, ot0 = blockIdx.y * CT, n = blockIdx.z;
    const int aoff = l16 * 32 + 8 * lg;
    // tiles past the edge re-read the last tile in range; their sums are never stored
    size_t af[RT], bf[CT];
#pragma unroll
    for (int i = 0; i < RT; i++) af[i] = ((size_t)n * PT + min(pt0 + i, PT - 1)) * nb;
#pragma unroll
    for (int j = 0; j < CT; j++) bf[j] = (size_t)min(ot0 + j, OT - 1) * nb;

    struct Stage {
        int64_t A[RT];
        f32x4 X[RT];
        int64_t B[CT];
        float W[CT];
    };
    // block b of the ring; past the last block the stage re-reads the last block's codes with
    // zero scales, so its products are +-0 and leave acc unchanged (acc starts at +0 and is
    // never -0), and the ring runs without branches (with a branch per stage the compiler's
    // load waits drained the ring)
    // The scales come through raw buffer loads over their tile row's nb * 16 floats; a stage
    // past the last block reads offset 0x80000000, outside that range, which loads 0 (the
    // choice is made on the address, so nothing waits for a load to select its value).
    __amdgpu_buffer_rsrc_t xr[RT], wr[CT];
#pragma unroll
    for (int i = 0; i < RT; i++)
        xr[i] = __builtin_amdgcn_make_buffer_rsrc((void*)(a.dxa + af[i] * 16), (short)0, nb * 64, 0x00020000);
#pragma unroll
    for (int j = 0; j < CT; j++)
        wr[j] = __builtin_amdgcn_make_buffer_rsrc((void*)(a.dw + bf[j] * 16), (short)0, nb * 64, 0x00020000);
    auto load = [&](Stage& s, int b) {
        const bool live = b < nb;
        const int xo = live ? (b * 16 + 4 * lg) * 4 : (int)0x80000000u;
        const int wo = live ? (b * 16 + l16) * 4 : (int)0x80000000u;
        b = min(b, nb - 1);
#pragma unroll
        for (int i = 0; i < RT; i++) {
            s.A[i] = *(const int64_t*)(a.qa + (af[i] + b) * 512 + aoff);
            s.X[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr[i], xo, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < CT; j++) {
            s.B[j] = *(const int64_t*)(a.qw + (bf[j] + b) * 512 + aoff);
            s.W[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr[j], wo, 0, 0));
        }
    };

    f32x4 acc[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int j = 0; j < CT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    Stage st[D];
#pragma unroll
    for (int s = 0; s < D; s++) load(st[s], s);
    for (int b0 = 0; b0 < nb; b0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
#pragma unroll
            for (int i = 0; i < RT; i++)
#pragma unroll
                for (int j = 0; j < CT; j++) {
                    const i32x4 I = __builtin_amdgcn_mfma_i32_16x16x32_i8(st[s].A[i], st[s].B[j],
                                                                           i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float sc = st[s].X[i][r] * st[s].W[j];
                        acc[i][j][r] = acc[i][j][r] + sc * (float)I[r];
                    }
                }
            load(st[s], b0 + s + D);
            // deep rings: keep each stage's loads behind its own arithmetic (hoisted into other
            // registers, they become copies at the loop's back edge, each waiting for its
            // load); 2- and 3-deep rings keep the scheduler free to overlap the stages
            if (D >= 4) __builtin_amdgcn_sched_barrier(0);
        }
    }
    // register r of tile (i, j): pixel 16*(pt0 + i) + 4lg + r, channel 16*(ot0 + j) + l16
#pragma unroll
    for (int i = 0; i < RT; i++) {
        if (pt0 + i >= PT) continue;
#pragma unroll
        for (int j = 0; j < CT; j++) {
            const int oc = 16 * (ot0 + j) + l16;
            if (oc >= a.OC) continue;
            conv_store(a.out, a.bias, a.resid, ((size_t)n * a.OC + oc) * M, oc, 16 * (pt0 + i) + 4 * lg, M,
                       acc[i][j]);
        }
    }
}

}  // namespace

size_t conv_i8_codes_bytes(int K, int OC) {
    return ((size_t)((OC + 15) / 16) * ((K + 31) / 32) * 512 + 255) & ~(size_t)255;
}

size_t conv_i8_weight_bytes(int K, int OC) {
    return conv_i8_codes_bytes(K, OC) + (size_t)((OC + 15) / 16) * ((K + 31) / 32) * 16 * sizeof(float);
}

size_t conv_i8_ws_codes_bytes(int M, int K, int N) {
    return ((size_t)N * ((M + 15) / 16) * ((K + 31) / 32) * 512 + 255) & ~(size_t)255;
}

size_t conv_i8_ws_bytes(int M, int K, int N) {
    return conv_i8_ws_codes_bytes(M, K, N) + (size_t)N * ((M + 15) / 16) * ((K + 31) / 32) * 16 * sizeof(float);
}

hipError_t launch_conv_quant_w(const float* ker, void* wq, int K, int OC, hipStream_t s) {
    const int nb = (K + 31) / 32, OT = (OC + 15) / 16;
    const int64_t total = (int64_t)OT * 16 * nb;
    if (total == 0) return hipSuccess;
    float* dw = (float*)((char*)wq + conv_i8_codes_bytes(K, OC));
    hipLaunchKernelGGL(k_conv_quant_w, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, ker, (int8_t*)wq, dw,
                       K, OC, OT, nb);
    return hipGetLastError();
}

bool conv_i8_one_pass(int IW, int IH, int IC, int OW, int OH, int OC, int KW, int KH, int N) {
    // 3 x 3 or 1 x 1 kernels, >= 8 channel tiles and >= 2048 waves of 64 pixels x 128 channels
    // (measured: 256 x 256 x 128 at 8 images 552 against 803 us for the two passes, 128 x 128,
    // 256 -> 128 at 8 images 244 against 391; at 1024 waves or fewer the two passes win or tie)
    const int64_t waves = ((int64_t)OW * OH + 63) / 64 * (((OC + 15) / 16 + 7) / 8) * N;
    return KW == KH && (KW == 3 || KW == 1) && (int64_t)IC * IW * IH * 4 < ((int64_t)1 << 31) &&
           (OC + 15) / 16 >= 8 && waves >= 2048;
}

hipError_t launch_conv2d_i8(const ConvI8Args& a, hipStream_t s) {
    const int M = a.OW * a.OH;
    if (M == 0 || a.OC == 0 || a.N == 0) return hipSuccess;
    const int K = a.IC * a.KW * a.KH, nb = (K + 31) / 32, PT = (M + 15) / 16, OT = (a.OC + 15) / 16;
    if (conv_i8_one_pass(a.IW, a.IH, a.IC, a.OW, a.OH, a.OC, a.KW, a.KH, a.N)) {
        const dim3 grid((unsigned)((M + 63) / 64), (unsigned)((OT + 7) / 8), (unsigned)a.N), block(64);
        if (a.KW == 3) hipLaunchKernelGGL((k_conv_i8_fused<3, 8>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((k_conv_i8_fused<1, 8>), grid, block, 0, s, a);
        return hipGetLastError();
    }
    const int ks = a.KW == a.KH && (a.KW == 3 || a.KW == 1) ? a.KW : 0;
    if (ks && (int64_t)a.IC * a.IW * a.IH * 4 < ((int64_t)1 << 31)) {
        // blocks per wave: enough (pixel group, block) pairs for >= 4096 waves
        const int64_t groups = (M + 63) / 64, pairs = groups * nb * a.N;
        const int bpw = (int)std::max<int64_t>((nb + 65534) / 65535, std::min<int64_t>(nb, pairs / 4096));
        const dim3 g1((unsigned)((M + 255) / 256), (unsigned)((nb + bpw - 1) / bpw), (unsigned)a.N);
        if (ks == 3) hipLaunchKernelGGL(k_conv_im2col_q8p<3>, g1, dim3(256), 0, s, a, bpw);
        else hipLaunchKernelGGL(k_conv_im2col_q8p<1>, g1, dim3(256), 0, s, a, bpw);
    } else {
        const dim3 g1((unsigned)PT, (unsigned)((nb + 3) / 4), (unsigned)a.N);
        hipLaunchKernelGGL(k_conv_im2col_q8<0>, g1, dim3(256), 0, s, a);
    }
    // Wave tile (16-pixel rows x 16-channel tiles, no more tiles than the operands have) and
    // ring depth, from timings of every variant on the decoder's GEMM shapes at 1 and 8 images
    // (all bit-identical): the largest tile that still gives >= 2048 waves for 4 x 4, >= 1024
    // for the others, else 1 x 1; deeper rings where waves are few (one wave's ring then has
    // to cover a whole memory latency), shallower ones where occupancy hides it.
    static const int cand[][3] = {{4, 4, 2048}, {4, 2, 1024}, {2, 2, 1024}, {4, 1, 1024}, {2, 1, 1024}};
    int rt = 1, ct = 1;
    int64_t waves = (int64_t)PT * OT * a.N;
    for (const auto& c : cand) {
        if (c[0] > PT || c[1] > OT) continue;
        const int64_t w = (int64_t)((PT + c[0] - 1) / c[0]) * ((OT + c[1] - 1) / c[1]) * a.N;
        if (w >= c[2]) {
            rt = c[0];
            ct = c[1];
            waves = w;
            break;
        }
    }
    const dim3 g2((unsigned)((PT + rt - 1) / rt), (unsigned)((OT + ct - 1) / ct), (unsigned)a.N), block(64);
    if (rt == 4 && ct == 4) {
        if (waves >= 8192) hipLaunchKernelGGL((k_conv_i8_gemm<4, 4, 2>), g2, block, 0, s, a);
        else hipLaunchKernelGGL((k_conv_i8_gemm<4, 4, 4>), g2, block, 0, s, a);
    } else if (rt == 4 && ct == 2) {
        hipLaunchKernelGGL((k_conv_i8_gemm<4, 2, 4>), g2, block, 0, s, a);
    } else if (rt == 2 && ct == 2) {
        if (waves > 1024) hipLaunchKernelGGL((k_conv_i8_gemm<2, 2, 4>), g2, block, 0, s, a);
        else hipLaunchKernelGGL((k_conv_i8_gemm<2, 2, 8>), g2, block, 0, s, a);
    } else if (rt == 4) {
        if (waves > 2048) hipLaunchKernelGGL((k_conv_i8_gemm<4, 1, 3>), g2, block, 0, s, a);
        else hipLaunchKernelGGL((k_conv_i8_gemm<4, 1, 6>), g2, block, 0, s, a);
    } else if (rt == 2) {
        hipLaunchKernelGGL((k_conv_i8_gemm<2, 1, 4>), g2, block, 0, s, a);
    } else {
        hipLaunchKernelGGL((k_conv_i8_gemm<1, 1, 8>), g2, block, 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace mgh
