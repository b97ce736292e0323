// k_vqgan.hip — the VQGAN decoder's ops on gfx950: 2-D convolution as an implicit GEMM on
// fp32 MFMA, GroupNorm (+ per-channel affine + SiLU), nearest-neighbour upscale.
//
// Semantics (layout ne = {W, H, C, N}, W innermost, every tensor contiguous):
//  * Conv2D: out[n][oc][oh][ow] = sum over (ic, kh, kw) of ker[oc][ic][kh][kw] *
//    in[n][ic][oh*stride - pad + kh][ow*stride - pad + kw] (zero outside), fp32 products and
//    fp32 accumulation — the reference's CPU executor k_conv_2d (src/mg-cpu/mg-cpu.cpp:165-190)
//    and its non-Mali GPU kernel k_conv2d_t (src/mg-opencl/mg-opencl.cpp:985-1025); only the
//    summation order differs.
//  * GroupNorm over each (n, group of C/G channels): mean and variance in double (two passes,
//    as mg-cpu.cpp:123-147), inv = 1 / sqrt((float)var + eps) with the fp32 sqrt and divide
//    correctly rounded, y = (float)(x - mean) * inv; with the fused affine + SiLU
//    (mg-cpu.cpp:262-276, GPU k_group_norm_affine_silu mg-opencl.cpp:1059-1095): xn = y *
//    gamma[c] + beta[c] (two roundings), out = xn / (1 + exp(-xn)).
//  * Upscale by f: out[n][c][oh][ow] = in[n][c][oh / f][ow / f] (mg-cpu.cpp:192-198).
//
// gfx950 mapping
//  * Conv2D: a workgroup computes 64 output pixels (flattened p = ow + OW*oh) x 64 output
//    channels; K = IC*KH*KW in slabs of 16 (the weights' own order: kw fastest, then kh, then
//    ic). Each thread gathers 4 im2col values (one pixel, four k) and 4 weights per slab into
//    registers one slab ahead, then writes them to a double-buffered LDS tile; four waves of
//    2 x 2 v_mfma_f32_16x16x4_f32 tiles read 1-float fragments (bank-conflict free: a row of
//    16 consecutive pixels or channels). A lane ends with four consecutive pixels of one
//    channel: one 16-byte store.
//  * GroupNorm: the statistics of one (n, group) are split over chunks of 4096 elements, one
//    workgroup each (the reference's one workgroup per group leaves all but 32 CUs idle at
//    the largest resolution); pass 1 writes per-chunk sums, pass 2 per-chunk sums of squared
//    deviations from the mean (each workgroup adds the pass-1 partials in chunk order, so every
//    chunk sees the same mean), and the apply pass derives mean and variance the same way.
//    Partials are summed in a fixed order: results do not depend on scheduling.
#include <algorithm>

#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

constexpr int CBM = 64, CBN = 64, CBK = 16, CPAD = 4;

// out[row + pp + e] = ((v[e] + bias[oc]) + resid[row + pp + e]) for the e with pp + e < M,
// each addition rounded on its own (the graph's conv node, then its Add nodes); one 16-byte
// store when the four pixels are in range and rows are 16-byte aligned (M % 4 == 0)
__device__ __forceinline__ void conv_store(float* __restrict__ out, const float* __restrict__ bias,
                                           const float* __restrict__ resid, size_t row, int oc, int pp, int M,
                                           f32x4 v) {
#pragma clang fp contract(off)
    if (bias) {
        const float b = bias[oc];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = v[e] + b;
    }
    if (pp + 3 < M && (M & 3) == 0) {
        if (resid) v = v + *(const f32x4*)(resid + row + pp);
        *(f32x4*)(out + row + pp) = v;
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (pp + e < M) out[row + pp + e] = resid ? v[e] + resid[row + pp + e] : v[e];
    }
}

// ---- packed-weight implicit GEMM (IC % 16 == 0): K in tap-major order k = (kh*KW + kw)*IC + ic,
// so a 16-wide K slab is one tap and 16 consecutive input channels: the im2col gather needs one
// bounds check per pixel and slab, and its loads step through channel planes.
constexpr int PBM = 128, PBN = 128, PBK = 16, PST = PBK + 4;   // LDS rows padded to 20 floats

// SPLIT: blockIdx.z = image * splits + split; the split's K range [split*kps, +kps) is summed
// into its own partial plane part[split][image][oc][pixel] (no bias or residual), which
// k_conv_reduce adds up in split order
template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void k_conv2d_pk(ConvPkArgs a) {
    __shared__ __attribute__((aligned(16))) float As[2][PBM][PST];   // [pixel][k]
    __shared__ __attribute__((aligned(16))) float Bs[2][PBN][PST];   // [channel][k]
    const int M = a.OW * a.OH, K = a.IC * a.KW * a.KH, OC = a.OC;
    const int z = blockIdx.z;
    const int n = SPLIT ? z / a.splits : z, sp = SPLIT ? z - n * a.splits : 0;
    const int kbeg = sp * a.kps, kend = min(K, kbeg + a.kps);
    const int m0 = blockIdx.x * PBM, n0 = blockIdx.y * PBN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, l16 = lane & 15, lg = lane >> 4;

    // gather roles: pixel pa with channels 8cg..8cg+7 of the slab; weight row bo, k half bh
    const int pa = tid & (PBM - 1), cg = tid >> 7;
    const int p = m0 + pa;
    const bool pv = p < M;
    const int ow = pv ? p % a.OW : 0, oh = pv ? p / a.OW : 0;
    const int iw0 = ow * a.stride - a.pad, ih0 = oh * a.stride - a.pad;
    const size_t plane = (size_t)a.IW * a.IH;
    const float* inb = a.in + ((size_t)n * a.IC + 8 * cg) * plane;
    const int bo = tid >> 1, bh = tid & 1;
    const bool bv = n0 + bo < OC;
    const float* wrow = a.wpk + (size_t)(bv ? n0 + bo : 0) * K + 8 * bh;

    float ra[8];
    f32x4 rb[2];
    auto load = [&](int k0) {
        const int tap = k0 / a.IC, ic0 = k0 - tap * a.IC;
        const int kh = tap / a.KW, kw = tap - kh * a.KW;
        const int ih = ih0 + kh, iw = iw0 + kw;
        if (pv && ih >= 0 && ih < a.IH && iw >= 0 && iw < a.IW) {
            const float* src = inb + (size_t)ic0 * plane + (size_t)ih * a.IW + iw;
#pragma unroll
            for (int j = 0; j < 8; j++) ra[j] = src[j * plane];
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) ra[j] = 0.f;
        }
        if (bv) {
            rb[0] = *(const f32x4*)(wrow + k0);
            rb[1] = *(const f32x4*)(wrow + k0 + 4);
        } else {
            rb[0] = rb[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store = [&](int buf) {
        *(f32x4*)&As[buf][pa][8 * cg] = f32x4{ra[0], ra[1], ra[2], ra[3]};
        *(f32x4*)&As[buf][pa][8 * cg + 4] = f32x4{ra[4], ra[5], ra[6], ra[7]};
        *(f32x4*)&Bs[buf][bo][8 * bh] = rb[0];
        *(f32x4*)&Bs[buf][bo][8 * bh + 4] = rb[1];
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nk = (kend - kbeg) / PBK;
    load(kbeg);
    store(0);
    __syncthreads();
    for (int t = 0; t < nk; t++) {
        const int cur = t & 1;
        if (t + 1 < nk) load(kbeg + (t + 1) * PBK);
        // lane (l16, lg) holds k = 4lg .. 4lg+3 of a row; MFMA step kk contracts k = 4lg + kk
        f32x4 af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const f32x4*)&As[cur][64 * wm + 16 * i + l16][4 * lg];
#pragma unroll
        for (int j = 0; j < 4; j++) bf[j] = *(const f32x4*)&Bs[cur][64 * wn + 16 * j + l16][4 * lg];
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][kk], bf[j][kk], acc[i][j], 0, 0, 0);
        // the other buffer was last read before the previous barrier
        if (t + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }
    // register e of tile (i, j): pixel m0 + 64wm + 16i + 4lg + e, channel n0 + 64wn + 16j + l16
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int oc = n0 + 64 * wn + 16 * j + l16;
        if (oc >= OC) continue;
        const size_t row = ((size_t)(SPLIT ? sp * a.N + n : n) * OC + oc) * M;
#pragma unroll
        for (int i = 0; i < 4; i++)
            conv_store(a.out, SPLIT ? nullptr : a.bias, SPLIT ? nullptr : a.resid, row, oc,
                       m0 + 64 * wm + 16 * i + 4 * lg, M, acc[i][j]);
    }
}

// few output channels (OC <= 16, the 3-channel conv_out) on the same packed weights: a
// workgroup computes 256 pixels x 16 channels, each wave 64 pixels x 16 channels
constexpr int NBM = 256, NBN = 16;

template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void k_conv2d_pkn(ConvPkArgs a) {
    __shared__ __attribute__((aligned(16))) float As[2][NBM][PST];   // [pixel][k]
    __shared__ __attribute__((aligned(16))) float Bs[2][NBN][PST];   // [channel][k]
    const int M = a.OW * a.OH, K = a.IC * a.KW * a.KH, OC = a.OC;
    const int z = blockIdx.z;
    const int n = SPLIT ? z / a.splits : z, sp = SPLIT ? z - n * a.splits : 0;
    const int kbeg = sp * a.kps, kend = min(K, kbeg + a.kps);
    const int m0 = blockIdx.x * NBM, n0 = blockIdx.y * NBN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;

    // gather roles: pixel tid with the slab's 16 channels; threads < 64: weight row tid/4, k 4(tid%4)..
    const int p = m0 + tid;
    const bool pv = p < M;
    const int ow = pv ? p % a.OW : 0, oh = pv ? p / a.OW : 0;
    const int iw0 = ow * a.stride - a.pad, ih0 = oh * a.stride - a.pad;
    const size_t plane = (size_t)a.IW * a.IH;
    const float* inb = a.in + (size_t)n * a.IC * plane;
    const int bo = tid >> 2, bq = tid & 3;
    const bool bload = tid < 4 * NBN, bv = bload && n0 + bo < OC;
    const float* wrow = a.wpk + (size_t)(bv ? n0 + bo : 0) * K + 4 * bq;

    float ra[16];
    f32x4 rb;
    auto load = [&](int k0) {
        const int tap = k0 / a.IC, ic0 = k0 - tap * a.IC;
        const int kh = tap / a.KW, kw = tap - kh * a.KW;
        const int ih = ih0 + kh, iw = iw0 + kw;
        if (pv && ih >= 0 && ih < a.IH && iw >= 0 && iw < a.IW) {
            const float* src = inb + (size_t)ic0 * plane + (size_t)ih * a.IW + iw;
#pragma unroll
            for (int j = 0; j < 16; j++) ra[j] = src[j * plane];
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) ra[j] = 0.f;
        }
        rb = bv ? *(const f32x4*)(wrow + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            *(f32x4*)&As[buf][tid][4 * q] = f32x4{ra[4 * q], ra[4 * q + 1], ra[4 * q + 2], ra[4 * q + 3]};
        if (bload) *(f32x4*)&Bs[buf][bo][4 * bq] = rb;
    };

    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nk = (kend - kbeg) / PBK;
    load(kbeg);
    store(0);
    __syncthreads();
    for (int t = 0; t < nk; t++) {
        const int cur = t & 1;
        if (t + 1 < nk) load(kbeg + (t + 1) * PBK);
        f32x4 af[4];
#pragma unroll
        for (int i = 0; i < 4; i++) af[i] = *(const f32x4*)&As[cur][64 * wave + 16 * i + l16][4 * lg];
        const f32x4 bf = *(const f32x4*)&Bs[cur][l16][4 * lg];
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][kk], bf[kk], acc[i], 0, 0, 0);
        if (t + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }
    const int oc = n0 + l16;
    if (oc >= OC) return;
    const size_t row = ((size_t)(SPLIT ? sp * a.N + n : n) * OC + oc) * M;
#pragma unroll
    for (int i = 0; i < 4; i++)
        conv_store(a.out, SPLIT ? nullptr : a.bias, SPLIT ? nullptr : a.resid, row, oc, m0 + 64 * wave + 16 * i + 4 * lg,
                   M, acc[i]);
}

// out[i] = ((sum over splits in order of part[s][i]) + bias[oc]) + resid[i]
__global__ __launch_bounds__(256) void k_conv_reduce(const float* __restrict__ part, int splits, int64_t total,
                                                     int M, int OC, const float* __restrict__ bias,
                                                     const float* __restrict__ resid, float* __restrict__ out) {
#pragma clang fp contract(off)
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        float v = part[i];
        for (int sp = 1; sp < splits; sp++) v = v + part[(size_t)sp * total + i];
        if (bias) v = v + bias[(i / M) % OC];
        if (resid) v = v + resid[i];
        out[i] = v;
    }
}

// wpk[oc][(kh*KW + kw)*IC + ic] = ker[oc][ic][kh][kw]
__global__ __launch_bounds__(256) void k_conv_pack(const float* __restrict__ ker, float* __restrict__ wpk, int IC,
                                                   int taps, int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t K = (int64_t)IC * taps;
        const int64_t oc = i / K, r = i - oc * K;
        const int64_t tap = r / IC, ic = r - tap * IC;
        wpk[i] = ker[oc * K + ic * taps + tap];
    }
}

// ---- few output channels (OC <= 8, the 3-channel conv_out): one thread per output pixel,
// products and sums in the reference loop's order (ic, kh, kw; out-of-image taps skipped) with
// separate multiply and add — the same float operations as the CPU executor's k_conv_2d.
// KSZ = 3: the input values of ICB channels x 9 taps are loaded before they are summed, so a
// thread has that many loads in flight (a skipped tap keeps the sum by a select, not by adding
// zero); KSZ = 0: any kernel size, one tap at a time.
template <int OCN, int KSZ>
__global__ __launch_bounds__(256) void k_conv2d_few(ConvArgs a) {
#pragma clang fp contract(off)
    constexpr int ICB = 4;
    const int M = a.OW * a.OH;
    const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= (int64_t)M * a.N) return;
    const int n = (int)(gi / M), p = (int)(gi - (int64_t)n * M);
    const int ow = p % a.OW, oh = p / a.OW;
    const int KW = KSZ ? KSZ : a.KW, KH = KSZ ? KSZ : a.KH;
    const int K = a.IC * KH * KW;
    const size_t plane = (size_t)a.IW * a.IH;
    const int ih0 = oh * a.stride - a.pad, iw0 = ow * a.stride - a.pad;
    float acc[OCN];
#pragma unroll
    for (int o = 0; o < OCN; o++) acc[o] = 0.f;
    const float* xn = a.in + (size_t)n * a.IC * plane;
    if (KSZ == 3) {
        bool ok[9];
        int off[9];
#pragma unroll
        for (int t = 0; t < 9; t++) {
            const int ih = ih0 + t / 3, iw = iw0 + t % 3;
            ok[t] = ih >= 0 && ih < a.IH && iw >= 0 && iw < a.IW;
            off[t] = ok[t] ? ih * a.IW + iw : 0;
        }
        for (int ic0 = 0; ic0 < a.IC; ic0 += ICB) {
            float v[ICB][9];
#pragma unroll
            for (int c = 0; c < ICB; c++) {
                const bool cv = ic0 + c < a.IC;
                const float* xin = xn + (size_t)(cv ? ic0 + c : 0) * plane;
#pragma unroll
                for (int t = 0; t < 9; t++) v[c][t] = ok[t] && cv ? xin[off[t]] : 0.f;
            }
#pragma unroll
            for (int c = 0; c < ICB; c++) {
                if (ic0 + c >= a.IC) break;
#pragma unroll
                for (int t = 0; t < 9; t++) {
                    const int k = (ic0 + c) * 9 + t;
#pragma unroll
                    for (int o = 0; o < OCN; o++)
                        if (o < a.OC) {
                            const float s = acc[o] + a.ker[(size_t)o * K + k] * v[c][t];
                            acc[o] = ok[t] ? s : acc[o];
                        }
                }
            }
        }
    } else {
        for (int ic = 0; ic < a.IC; ic++) {
            const float* xin = xn + (size_t)ic * plane;
            for (int kh = 0; kh < KH; kh++) {
                const int ih = ih0 + kh;
                if (ih < 0 || ih >= a.IH) continue;
                for (int kw = 0; kw < KW; kw++) {
                    const int iw = iw0 + kw;
                    if (iw < 0 || iw >= a.IW) continue;
                    const float v = xin[(size_t)ih * a.IW + iw];
                    const int k = (ic * KH + kh) * KW + kw;
#pragma unroll
                    for (int o = 0; o < OCN; o++)
                        if (o < a.OC) acc[o] = acc[o] + a.ker[(size_t)o * K + k] * v;
                }
            }
        }
    }
#pragma unroll
    for (int o = 0; o < OCN; o++) {
        if (o >= a.OC) break;
        const size_t idx = ((size_t)n * a.OC + o) * M + p;
        float v = acc[o];
        if (a.bias) v = v + a.bias[o];
        if (a.resid) v = v + a.resid[idx];
        a.out[idx] = v;
    }
}

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
            dst[0] = q[0];
            dst[1] = q[1];
            a.dxa[frag * 16 + (p & 15)] = d;
        }
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
    auto load = [&](Stage& s, int b) {
#pragma unroll
        for (int i = 0; i < RT; i++) {
            s.A[i] = *(const int64_t*)(a.qa + (af[i] + b) * 512 + aoff);
            s.X[i] = *(const f32x4*)(a.dxa + (af[i] + b) * 16 + 4 * lg);
        }
#pragma unroll
        for (int j = 0; j < CT; j++) {
            s.B[j] = *(const int64_t*)(a.qw + (bf[j] + b) * 512 + aoff);
            s.W[j] = a.dw[(bf[j] + b) * 16 + l16];
        }
    };

    f32x4 acc[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int j = 0; j < CT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    Stage st[D];
#pragma unroll
    for (int s = 0; s < D; s++) load(st[s], min(s, nb - 1));
    for (int b0 = 0; b0 < nb; b0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            if (b0 + s < nb) {
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
            }
            load(st[s], min(b0 + s + D, nb - 1));
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

// KSZ > 0: KW = KH = KSZ known at compile time (the index arithmetic then divides by a
// constant); 0: any kernel size
template <int KSZ>
__global__ __launch_bounds__(256) void k_conv2d_f32(ConvArgs a) {
    __shared__ float As[2][CBK][CBM + CPAD];    // im2col tile: [k][pixel]
    __shared__ float Bs[2][CBK][CBN + CPAD];    // weights: [k][channel]
    const int KW = KSZ ? KSZ : a.KW, KH = KSZ ? KSZ : a.KH;
    const int IW = a.IW, IH = a.IH, OC = a.OC;
    const int M = a.OW * a.OH, K = a.IC * KW * KH;
    const int n = blockIdx.z;
    const int m0 = blockIdx.x * CBM, n0 = blockIdx.y * CBN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, g = lane >> 4;

    // gather roles: im2col values (pixel am, k = ak0 + 4i), weights (k = bk, channel bn0 + 16i)
    const int am = tid & 63, ak0 = tid >> 6;
    const int p = m0 + am;
    const bool pv = p < M;
    const int ow = pv ? p % a.OW : 0, oh = pv ? p / a.OW : 0;
    const int iw0 = ow * a.stride - a.pad, ih0 = oh * a.stride - a.pad;
    const float* inb = a.in + (size_t)n * a.IC * IH * IW;
    const int bk = tid & 15, bn0 = tid >> 4;
    float ra[4], rb[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k = k0 + ak0 + 4 * i;
            float v = 0.f;
            if (pv && k < K) {
                const int kw = k % KW, t = k / KW, kh = t % KH, ic = t / KH;
                const int iw = iw0 + kw, ih = ih0 + kh;
                if (iw >= 0 && iw < IW && ih >= 0 && ih < IH) v = inb[iw + (size_t)IW * (ih + (size_t)IH * ic)];
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int oc = n0 + bn0 + 16 * i, k = k0 + bk;
            rb[i] = oc < OC && k < K ? a.ker[(size_t)oc * K + k] : 0.f;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) As[buf][ak0 + 4 * i][am] = ra[i];
#pragma unroll
        for (int i = 0; i < 4; i++) Bs[buf][bk][bn0 + 16 * i] = rb[i];
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nk = (K + CBK - 1) / CBK;
    load(0);
    store(0);
    __syncthreads();
    for (int t = 0; t < nk; t++) {
        const int cur = t & 1;
        if (t + 1 < nk) load((t + 1) * CBK);
#pragma unroll
        for (int kk = 0; kk < CBK; kk += 4) {
            float av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; i++) av[i] = As[cur][kk + g][32 * wm + 16 * i + r16];
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = Bs[cur][kk + g][32 * wn + 16 * j + r16];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        // the other buffer was last read before the previous barrier
        if (t + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }
    // register e of tile (i, j): pixel m0 + 32wm + 16i + 4g + e, channel n0 + 32wn + 16j + r16
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int oc = n0 + 32 * wn + 16 * j + r16;
        if (oc >= OC) continue;
        const size_t row = ((size_t)n * OC + oc) * M;
#pragma unroll
        for (int i = 0; i < 2; i++)
            conv_store(a.out, a.bias, a.resid, row, oc, m0 + 32 * wm + 16 * i + 4 * g, M, acc[i][j]);
    }
}

constexpr int GN_CHUNK = 4096;

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    // fixed-order reduction: wave butterflies, then the 4 wave sums in wave order; red[4] must
    // not be in use by another reduction of the same block
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)u, o);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(u >> 32), o);
        v += __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// this thread's elements of a 4096-element chunk: VEC, 16-byte groups at 4t + 1024j (j < 4);
// else single elements at t + 256j (j < 16); idx = -1 past the chunk's end
template <bool VEC>
__device__ __forceinline__ int64_t gn_idx(int64_t b, int64_t e, int j) {
    const int64_t i = VEC ? b + 4 * (int64_t)threadIdx.x + 1024 * (j >> 2) + (j & 3) : b + threadIdx.x + 256 * j;
    return i < e ? i : -1;
}

// per chunk of a group: S = sum of x and Q = sum of (x - S/n_c)^2, both in double, from the
// chunk's values held in registers (one read of x)
template <bool VEC>
__global__ __launch_bounds__(256) void k_gn_stats(const float* __restrict__ x, double* __restrict__ part,
                                                  int64_t cnt, int chunks) {
    __shared__ double red[2][4];
    const int chunk = blockIdx.x, ng = blockIdx.y;
    const float* xg = x + (size_t)ng * cnt;
    const int64_t b = (int64_t)chunk * GN_CHUNK, e = min(cnt, b + GN_CHUNK);
    float v[16];
    if (VEC) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int64_t i = b + 4 * (int64_t)threadIdx.x + 1024 * q;
            const f32x4 w = i < e ? *(const f32x4*)(xg + i) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < 4; r++) v[4 * q + r] = w[r];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int64_t i = gn_idx<false>(b, e, j);
            v[j] = i >= 0 ? xg[i] : 0.f;
        }
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 16; j++) s += (double)v[j];           // out-of-chunk values are 0
    const double S = block_sum_d(s, red[0]);
    const double mc = S / (double)(e - b);
    double q = 0.0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const double d = (double)v[j] - mc;
        if (gn_idx<VEC>(b, e, j) >= 0) q += d * d;
    }
    const double Q = block_sum_d(q, red[1]);
    if (threadIdx.x == 0) {
        part[2 * ((size_t)ng * chunks + chunk)] = S;
        part[2 * ((size_t)ng * chunks + chunk) + 1] = Q;
    }
}

// y = (float)(x - mean) * inv (+ affine + SiLU) over one chunk; mean and variance of the group
// from its chunks' (S, Q): mean = sum S / n, n var = sum over chunks of Q_c + n_c (m_c - mean)^2
// (the parallel form of the two-pass sum of squared deviations), each sum in a fixed order
template <bool AFFINE_SILU, bool VEC>
__global__ __launch_bounds__(256) void k_gn_apply(const float* __restrict__ x, const double* __restrict__ part,
                                                  const float* __restrict__ gamma, const float* __restrict__ beta,
                                                  float* __restrict__ y, int64_t cnt, int64_t plane, int cpg,
                                                  int G, int chunks, float eps) {
#pragma clang fp contract(off)   // xn = y*gamma + beta rounds twice, as in the reference
    __shared__ double red[2][4];
    const int chunk = blockIdx.x, ng = blockIdx.y;
    const double* pg = part + 2 * (size_t)ng * chunks;
    double s = 0.0;
    for (int c = threadIdx.x; c < chunks; c += 256) s += pg[2 * c];
    const double mean = block_sum_d(s, red[0]) / (double)cnt;
    double q = 0.0;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        const double nc = (double)min((int64_t)GN_CHUNK, cnt - (int64_t)c * GN_CHUNK);
        const double d = pg[2 * c] / nc - mean;
        q += pg[2 * c + 1] + nc * d * d;
    }
    const double var = block_sum_d(q, red[1]) / (double)cnt;
    // fp32 sqrt and divide, each correctly rounded (evaluated in double, rounded once)
    const float sq = (float)sqrt((double)__fadd_rn((float)var, eps));
    const float inv = (float)(1.0 / (double)sq);
    const float* xg = x + (size_t)ng * cnt;
    float* yg = y + (size_t)ng * cnt;
    const int c0 = (ng % G) * cpg;
    const int64_t b = (int64_t)chunk * GN_CHUNK, e = min(cnt, b + GN_CHUNK);
    auto f = [&](float xv, float g, float bb) {
        float v = (float)((double)xv - mean) * inv;
        if (AFFINE_SILU) {
            v = v * g + bb;
            v = v / (1.0f + expf(-v));
        }
        return v;
    };
    if (VEC) {
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            const int64_t i = b + 4 * (int64_t)threadIdx.x + 1024 * qd;
            if (i >= e) break;
            const f32x4 w = *(const f32x4*)(xg + i);
            const int c = c0 + (int)(i / plane);              // plane % 4 == 0: one channel
            const float g = AFFINE_SILU ? gamma[c] : 0.f, bb = AFFINE_SILU ? beta[c] : 0.f;
            *(f32x4*)(yg + i) = f32x4{f(w[0], g, bb), f(w[1], g, bb), f(w[2], g, bb), f(w[3], g, bb)};
        }
    } else {
        for (int64_t i = b + threadIdx.x; i < e; i += 256) {
            const int c = c0 + (int)(i / plane);
            yg[i] = f(xg[i], AFFINE_SILU ? gamma[c] : 0.f, AFFINE_SILU ? beta[c] : 0.f);
        }
    }
}

__global__ __launch_bounds__(256) void k_upscale(const float* __restrict__ x, float* __restrict__ y, int IW,
                                                 int IH, int f, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int OW = IW * f, OH = IH * f;
    const int ow = (int)(i % OW);
    const int64_t r = i / OW;
    const int oh = (int)(r % OH);
    const int64_t cn = r / OH;
    y[i] = x[(cn * IH + oh / f) * IW + ow / f];
}

}  // namespace

hipError_t launch_conv2d_f32(const ConvArgs& a, hipStream_t s) {
    const int M = a.OW * a.OH;
    if (M == 0 || a.OC == 0 || a.N == 0) return hipSuccess;
    if (a.OC <= kConvFewMax) {
        const int64_t total = (int64_t)M * a.N;
        const dim3 grid((unsigned)((total + 255) / 256));
        const bool k3 = a.KW == 3 && a.KH == 3;
        if (a.OC <= 4) {
            if (k3) hipLaunchKernelGGL((k_conv2d_few<4, 3>), grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL((k_conv2d_few<4, 0>), grid, dim3(256), 0, s, a);
        } else {
            if (k3) hipLaunchKernelGGL((k_conv2d_few<8, 3>), grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL((k_conv2d_few<8, 0>), grid, dim3(256), 0, s, a);
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((M + CBM - 1) / CBM), (unsigned)((a.OC + CBN - 1) / CBN), (unsigned)a.N), block(256);
    if (a.KW == 3 && a.KH == 3) hipLaunchKernelGGL(k_conv2d_f32<3>, grid, block, 0, s, a);
    else if (a.KW == 1 && a.KH == 1) hipLaunchKernelGGL(k_conv2d_f32<1>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(k_conv2d_f32<0>, grid, block, 0, s, a);
    return hipGetLastError();
}

bool conv_pk_narrow(int OC) { return OC <= NBN; }

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

hipError_t launch_conv2d_i8(const ConvI8Args& a, hipStream_t s) {
    const int M = a.OW * a.OH;
    if (M == 0 || a.OC == 0 || a.N == 0) return hipSuccess;
    const int K = a.IC * a.KW * a.KH, nb = (K + 31) / 32, PT = (M + 15) / 16, OT = (a.OC + 15) / 16;
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
    // the largest wave tile (rows x channel tiles, no more tiles than the operands have) that
    // still gives >= 2048 waves; 1 x 1 tiles otherwise
    static const int cand[][2] = {{4, 4}, {4, 2}, {2, 2}, {4, 1}, {2, 1}};
    int rt = 1, ct = 1;
    for (const auto& c : cand) {
        if (c[0] > PT || c[1] > OT) continue;
        if ((int64_t)((PT + c[0] - 1) / c[0]) * ((OT + c[1] - 1) / c[1]) * a.N >= 2048) {
            rt = c[0];
            ct = c[1];
            break;
        }
    }
    const dim3 g2((unsigned)((PT + rt - 1) / rt), (unsigned)((OT + ct - 1) / ct), (unsigned)a.N), block(64);
    if (rt == 4 && ct == 4) hipLaunchKernelGGL((k_conv_i8_gemm<4, 4, 2>), g2, block, 0, s, a);
    else if (rt == 4 && ct == 2) hipLaunchKernelGGL((k_conv_i8_gemm<4, 2, 3>), g2, block, 0, s, a);
    else if (rt == 2 && ct == 2) hipLaunchKernelGGL((k_conv_i8_gemm<2, 2, 4>), g2, block, 0, s, a);
    else if (rt == 4) hipLaunchKernelGGL((k_conv_i8_gemm<4, 1, 3>), g2, block, 0, s, a);
    else if (rt == 2) hipLaunchKernelGGL((k_conv_i8_gemm<2, 1, 4>), g2, block, 0, s, a);
    else hipLaunchKernelGGL((k_conv_i8_gemm<1, 1, 8>), g2, block, 0, s, a);
    return hipGetLastError();
}

ConvPkPlan conv_pk_plan(int M, int OC, int K) {
    // Split K when one image's output tiles give fewer than 384 workgroups: up to about 512
    // workgroups, each split keeping >= 9 16-wide slabs. Measured on the decoder's convs at
    // one image (split targets 128..1024 workgroups): shorter splits lose to their partial
    // planes (16 x 16 x 512 -> 512: 31.5 us at 9 slabs per split, 39.1 at 5; the 8-slab 1x1
    // conv at 128 x 128: 16.7 us unsplit, 30.6 in 4 splits), while the 64-128 px levels want
    // about 512 workgroups. The plan does not depend on the batch, so an image's sums are the
    // same whatever it is batched with.
    ConvPkPlan p{1, K};
    const int bm = conv_pk_narrow(OC) ? NBM : PBM, bn = conv_pk_narrow(OC) ? NBN : PBN;
    const int64_t tiles = (int64_t)((M + bm - 1) / bm) * ((OC + bn - 1) / bn);
    const int slabs = K / PBK;
    const int want = (int)std::min<int64_t>((512 + tiles - 1) / tiles, slabs / 9);
    if (tiles >= 384 || want < 2) return p;
    const int per = (slabs + want - 1) / want;
    p.kps = per * PBK;
    p.splits = (slabs + per - 1) / per;
    return p;
}

// images per split launch: grid z = images x splits stays within 65535
static int conv_pk_group(int N, int splits) { return std::min(N, 65535 / splits); }

size_t conv_pk_ws_bytes(int M, int OC, int N, int K) {
    const ConvPkPlan p = conv_pk_plan(M, OC, K);
    return p.splits > 1 ? (size_t)p.splits * conv_pk_group(N, p.splits) * OC * (size_t)M * sizeof(float) : 0;
}

hipError_t launch_conv_pack(const float* ker, float* wpk, int IC, int taps, int OC, hipStream_t s) {
    const int64_t total = (int64_t)OC * IC * taps;
    if (total == 0) return hipSuccess;
    const int64_t g = std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(k_conv_pack, dim3((unsigned)g), dim3(256), 0, s, ker, wpk, IC, taps, total);
    return hipGetLastError();
}

hipError_t launch_conv2d_pk(const ConvPkArgs& a0, float* ws, hipStream_t s) {
    const int M = a0.OW * a0.OH, K = a0.IC * a0.KW * a0.KH;
    if (M == 0 || a0.OC == 0 || a0.N == 0) return hipSuccess;
    const ConvPkPlan p = conv_pk_plan(M, a0.OC, K);
    ConvPkArgs a = a0;
    a.splits = p.splits;
    a.kps = p.kps;
    const dim3 block(256);
    const bool nar = conv_pk_narrow(a0.OC);
    const unsigned gx = (unsigned)(nar ? (M + NBM - 1) / NBM : (M + PBM - 1) / PBM);
    const unsigned gy = (unsigned)(nar ? (a0.OC + NBN - 1) / NBN : (a0.OC + PBN - 1) / PBN);
    if (p.splits == 1) {
        const dim3 grid(gx, gy, (unsigned)a.N);
        if (nar) hipLaunchKernelGGL(k_conv2d_pkn<false>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(k_conv2d_pk<false>, grid, block, 0, s, a);
        return hipGetLastError();
    }
    // groups of images: partials part[split][image of the group][oc][pixel] in ws, then reduced
    const int G = conv_pk_group(a0.N, p.splits);
    const size_t in_img = (size_t)a0.IC * a0.IW * a0.IH, out_img = (size_t)a0.OC * M;
    for (int n0 = 0; n0 < a0.N; n0 += G) {
        const int g = std::min(G, a0.N - n0);
        a.in = a0.in + n0 * in_img;
        a.out = ws;
        a.N = g;
        const dim3 grid(gx, gy, (unsigned)(g * p.splits));
        if (nar) hipLaunchKernelGGL(k_conv2d_pkn<true>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(k_conv2d_pk<true>, grid, block, 0, s, a);
        const int64_t total = (int64_t)g * out_img;
        const int64_t nb = std::min<int64_t>((total + 255) / 256, 8192);
        hipLaunchKernelGGL(k_conv_reduce, dim3((unsigned)nb), block, 0, s, ws, p.splits, total, M, a.OC, a0.bias,
                           a0.resid ? a0.resid + n0 * out_img : nullptr, a0.out + n0 * out_img);
    }
    return hipGetLastError();
}

size_t group_norm_ws_bytes(int64_t W, int64_t H, int C, int N, int G) {
    const int64_t cnt = W * H * (C / G);
    const int64_t chunks = (cnt + GN_CHUNK - 1) / GN_CHUNK;
    return (size_t)(2 * chunks * G * N) * sizeof(double);
}

hipError_t launch_group_norm(const float* x, int64_t W, int64_t H, int C, int N, int G, float eps,
                             const float* gamma, const float* beta, float* y, void* ws, hipStream_t s) {
    const int cpg = C / G;
    const int64_t plane = W * H, cnt = plane * cpg;
    if (cnt == 0 || N == 0) return hipSuccess;
    const int chunks = (int)((cnt + GN_CHUNK - 1) / GN_CHUNK);
    double* part = (double*)ws;
    const dim3 grid((unsigned)chunks, (unsigned)(G * N)), block(256);
    // 16-byte accesses: planes of 4k elements (a group and a 4-group never straddle channels)
    const bool vec = plane % 4 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0;
    if (vec) hipLaunchKernelGGL(k_gn_stats<true>, grid, block, 0, s, x, part, cnt, chunks);
    else hipLaunchKernelGGL(k_gn_stats<false>, grid, block, 0, s, x, part, cnt, chunks);
#define GN_APPLY(A, V) \
    hipLaunchKernelGGL((k_gn_apply<A, V>), grid, block, 0, s, x, part, gamma, beta, y, cnt, plane, cpg, G, chunks, eps)
    if (gamma) {
        if (vec) GN_APPLY(true, true);
        else GN_APPLY(true, false);
    } else {
        if (vec) GN_APPLY(false, true);
        else GN_APPLY(false, false);
    }
#undef GN_APPLY
    return hipGetLastError();
}

hipError_t launch_upscale(const float* x, int IW, int IH, int64_t CN, int f, float* y, hipStream_t s) {
    const int64_t total = (int64_t)IW * f * IH * f * CN;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_upscale, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, y, IW, IH, f, total);
    return hipGetLastError();
}

}  // namespace mgh
