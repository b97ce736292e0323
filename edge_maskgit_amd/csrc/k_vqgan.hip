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

#include "k_conv_common.h"
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

constexpr int CBM = 64, CBN = 64, CBK = 16, CPAD = 4;

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
            conv_store<!SPLIT>(a.out, SPLIT ? nullptr : a.bias, SPLIT ? nullptr : a.resid, row, oc,
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
        conv_store<!SPLIT>(a.out, SPLIT ? nullptr : a.bias, SPLIT ? nullptr : a.resid, row, oc, m0 + 64 * wave + 16 * i + 4 * lg,
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

// Up-sampling by 2 on even widths (every decoder level): a thread reads two neighbouring
// input values and writes them doubled, {a, a, b, b}, as one 16-byte store into each of the
// two output rows.
__global__ __launch_bounds__(256) void k_upscale2(const float2* __restrict__ x, f32x4* __restrict__ y, int IWh,
                                                  int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const float2 v = x[i];
    const int64_t row = i / IWh;                // input row (c*IH + ih) of an image
    const int j = (int)(i - row * IWh);
    const f32x4 o = {v.x, v.x, v.y, v.y};
    f32x4* out = y + (size_t)row * 2 * IWh + j; // output rows 2*row and 2*row + 1, IWh vectors each
    out[0] = o;
    out[IWh] = o;
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
    if (f == 2 && IW % 2 == 0 && ((uintptr_t)x & 7) == 0 && ((uintptr_t)y & 15) == 0) {
        const int64_t pairs = (int64_t)IW / 2 * IH * CN;
        hipLaunchKernelGGL(k_upscale2, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, (const float2*)x,
                           (f32x4*)y, IW / 2, pairs);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_upscale, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, y, IW, IH, f, total);
    return hipGetLastError();
}

}  // namespace mgh
