// k_flash_attn.hip — fused self-attention with fp16 K/V (gfx950).
//
// Semantics: the reference's k_flash_attention_h (src/mg-opencl/mg-opencl.cpp:859-937) with
// the CPU oracle k_flash_attention (src/mg-cpu/mg-cpu.cpp:211-239) for the math:
//   per (batch b, head h, query s): q, k, v rounded to fp16; score_t = (q . k_t) * scale in
//   fp32; softmax over keys in fp32 (online, max-subtracted); o = sum_t p_t v_t / sum_t p_t.
// Inputs are strided {D, S, H, B} views (element strides st[0..3]); the reference passes
// the q/k/v FC outputs [S*B][H*D] with st = {1, H*D, D, H*D*S} (mg-opencl.cpp:1493-1496).
// The output strides are a parameter too, so the head merge that follows in the reference
// graph (permute + cont, mg-transformer.cpp:84-85) is written directly.
//
// gfx950 mapping (one workgroup = 4 waves = 64 queries of one (b, h); keys in chunks of 64
// staged once per workgroup in LDS as fp16):
//  * Scores as S^T = K . Q^T on v_mfma_f32_16x16x32_f16 (two 16-wide d chunks per
//    instruction, an odd last chunk paired with zeros): fp16 products are exact in fp32, so
//    only the summation order differs from the reference. The S^T accumulator layout (lane
//    = query, registers = 4 consecutive keys) is exactly the A-operand layout of the next
//    product, so P . V needs no data exchange between lanes.
//  * Softmax statistics per query in fp32 (max, running sum), cross-lane over the 4 lane
//    groups; exp is the fp32 expf.
//  * P . V on the same MFMA with P split into fp16 hi + lo parts (two instructions), so the
//    fp32 probabilities are applied to ~2^-22 — the reference multiplies them in fp32.
// LDS rows are padded (K: D+8 halves, V^T: 72 halves) so the fragment reads are
// bank-conflict free.
#include <algorithm>

#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x8 cat8(f16x4 a, f16x4 b) {
    return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// -1.0f as a value the compiler cannot fold: with it, fmaf((float)h, -1, p) for an fp16 h
// is selected as v_fma_mix_f32 (h read as an fp16 half of its register, no conversion), where
// the constant form becomes a conversion and a subtraction. A scalar move, read by VALU
// instructions only.
__device__ __forceinline__ float opaque_neg_one() {
    float m;
    asm("s_mov_b32 %0, 0xbf800000" : "=s"(m));
    return m;
}

constexpr int KT = 64;             // keys per LDS chunk
constexpr int VLD = KT + 8;        // V^T row stride (halves)

template <int DC>
__global__ __launch_bounds__(256) void k_flash_attn_f16kv(FaArgs a) {
    constexpr int D = 16 * DC;
    constexpr int KLD = D + 8;     // K row stride (halves)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[KT * KLD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VLD];

    const int S = a.S;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, lg = lane >> 4;
    const int h = blockIdx.y, b = blockIdx.z;
    const int q0w = blockIdx.x * 64 + wave * 16;
    const bool active = q0w < S;
    const int64_t base = (int64_t)b * a.st[3] + (int64_t)h * a.st[2];

    // Q as the B operand: lane = query q0w + l16, k = d = 16c + 4lg + j
    f16x4 qf[DC];
    {
        const int qi = min(q0w + l16, S - 1);
#pragma unroll
        for (int c = 0; c < DC; c++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                qf[c][j] = (_Float16)a.q[base + (int64_t)qi * a.st[1] + (int64_t)(16 * c + 4 * lg + j) * a.st[0]];
    }

    f32x4 O[DC];
#pragma unroll
    for (int c = 0; c < DC; c++) O[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;          // statistics of query q0w + l16

    for (int k0 = 0; k0 < S; k0 += KT) {
        __syncthreads();                   // the previous chunk is consumed
        for (int idx = tid; idx < KT * D; idx += 256) {
            const int key = idx / D, d = idx - key * D, t = k0 + key;
            float kv = 0.f, vv = 0.f;
            if (t < S) {
                const int64_t off = base + (int64_t)t * a.st[1] + (int64_t)d * a.st[0];
                kv = a.k[off];
                vv = a.v[off];
            }
            Ks[key * KLD + d] = (_Float16)kv;
            Vt[d * VLD + key] = (_Float16)vv;
        }
        __syncthreads();
        if (!active) continue;

        // scores: register r of subtile t holds key k0 + 16t + 4lg + r for query l16
        f32x4 sc[KT / 16];
#pragma unroll
        for (int t = 0; t < KT / 16; t++) {
            // pairs of 16-wide d chunks on the 32-deep MFMA (k = 8lg + j: d = 16(c + j/4) + 4lg +
            // j%4 in both operands); an odd last chunk is paired with zeros (the 16-deep MFMA
            // takes as long, and a 16-deep MFMA accumulating right after a 32-deep one into
            // the same registers gave wrong sums)
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const _Float16* krow = &Ks[(16 * t + l16) * KLD + 4 * lg];
#pragma unroll
            for (int c = 0; c < DC; c += 2) {
                const f16x4 k1 = c + 1 < DC ? *(const f16x4*)(krow + 16 * c + 16) : f16x4{0, 0, 0, 0};
                const f16x4 q1 = c + 1 < DC ? qf[c + 1] : f16x4{0, 0, 0, 0};
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cat8(*(const f16x4*)(krow + 16 * c), k1),
                                                             cat8(qf[c], q1), acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = k0 + 16 * t + 4 * lg + r;
                sc[t][r] = key < S ? acc[r] * a.scale : -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < KT / 16; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, sc[t][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float alpha = expf(m - mn);
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < KT / 16; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = sc[t][r] == -INFINITY ? 0.f : expf(sc[t][r] - mn);
                sc[t][r] = p;
                ps += p;
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = alpha * l + ps;
        m = mn;

        // O rows are queries 4lg + r: rescale by that query's alpha (held by lane 4lg + r)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * lg + r);
#pragma unroll
            for (int c = 0; c < DC; c++) O[c][r] *= ar;
        }
        // O += P . V with P = hi + lo in fp16 (A operand: query l16, keys 16t + 4lg + j)
#pragma unroll
        for (int t = 0; t < KT / 16; t++) {
            f16x4 ph, pl;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                ph[j] = (_Float16)sc[t][j];
                pl[j] = (_Float16)(sc[t][j] - (float)ph[j]);
            }
#pragma unroll
            for (int c = 0; c < DC; c++) {
                const f16x4 vf = *(const f16x4*)&Vt[(16 * c + l16) * VLD + 16 * t + 4 * lg];
                O[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vf, O[c], 0, 0, 0);
                O[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vf, O[c], 0, 0, 0);
            }
        }
    }
    if (!active) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float inv = 1.f / __shfl(l, 4 * lg + r);
        const int qi = q0w + 4 * lg + r;
        if (qi >= S) continue;
        const int64_t ro = (int64_t)b * a.os[3] + (int64_t)h * a.os[2] + (int64_t)qi * a.os[1];
#pragma unroll
        for (int c = 0; c < DC; c++) {
            const int64_t e = ro + (int64_t)(16 * c + l16) * a.os[0];
            if (a.o16) a.o16[e] = (_Float16)(O[c][r] * inv);
            else a.o[e] = O[c][r] * inv;
        }
    }
}


// Whole-head variant for S <= 16*KT: one workgroup per (h, b) stages the head's K (row-major)
// and V (transposed) once in LDS as fp16, then each wave takes 16-query tiles and computes all
// scores of a tile in registers, a plain (not online) max-subtracted softmax over the row —
// the order of the reference CPU kernel — and P . V. K/V are read once per head instead of
// once per query tile (needs unit d stride and 16-byte aligned rows; q/k/v either fp32,
// rounded to fp16 on load, or already fp16). The exponentials use the hardware exp2 on
// log2(e)-scaled scores (relative error ~1e-7, far inside the attention tolerance), with the
// scale folded into one fma. Both products run on v_mfma_f32_16x16x32_f16 (the 16-deep
// instruction takes as many cycles on gfx950): scores over pairs of d chunks, P . V over pairs
// of key tiles (k = 8lg + j maps to key 16(t + j/4) + 4lg + j%4 in both operands, so the score
// registers are the P operand as they stand). The work per tile is VALU-bound (exp, the
// hi/lo split of P), so the VALU is kept to what the math needs: P . V is computed transposed
// (each lane ends with consecutive features of one query: one division, 8/16-byte stores),
// the row sums come from the MFMA on an all-ones operand, the lo part of P takes one
// v_fma_mix_f32 per element, and LDS fragments are read ahead of their MFMAs.
// At most NW waves (a workgroup takes min(NW, ~half the query tiles) waves), so the score
// registers (4 * KT per lane) fit without spilling: 17 key tiles take 9 waves (3 per SIMD,
// 168 registers) only for fp16 q/k/v at D <= 48 with a 17th, partial tile (S = 257 .. 272);
// at D = 64, with fp32 q/k/v (the next tile's Q held as fp32) or for S <= 256 (16 query
// tiles, two per wave) 8 (256 registers per wave, two waves per SIMD); 32 key tiles with
// D >= 48 need more than 256, so there one wave per SIMD
template <int DC, int KT, bool I16, bool TAIL>
constexpr int kHeadWaves = KT <= 17 ? std::min((KT + 1) / 2, DC >= 4 || !I16 || !TAIL ? 8 : 9)
                                    : (KT == 32 && DC >= 3 ? 4 : 8);

// 4 consecutive elements of q/k/v as fp16: rounded from fp32 (RNE) or, with I16, loaded as
// stored (the producer rounded them the same way)
template <bool I16>
__device__ __forceinline__ f16x4 load_h4(const float* p32, const _Float16* p16, int64_t e) {
    if (I16) return *(const f16x4*)(p16 + e);
    const f32x4 v = *(const f32x4*)(p32 + e);
    return f16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}
// 8 consecutive elements (e % 8 == 0): one 16-byte load of fp16 rows when they are 16-byte
// aligned (A16), two 8-byte loads otherwise; fp32 rows as two 16-byte loads, rounded
template <bool I16, bool A16>
__device__ __forceinline__ f16x8 load_h8(const float* p32, const _Float16* p16, int64_t e) {
    if (I16 && A16) return *(const f16x8*)(p16 + e);
    return cat8(load_h4<I16>(p32, p16, e), load_h4<I16>(p32, p16, e + 4));
}

// TAIL: S > 16 (KT - 1), so every key tile but the last is full (no masking there).
// A16: fp16 inputs whose rows start on 16-byte boundaries (element strides multiples of 8).
template <int DC, int KT, bool I16, bool TAIL, bool A16>
__global__ __launch_bounds__(64 * (kHeadWaves<DC, KT, I16, TAIL>)) void k_attn_head(FaArgs a) {
    constexpr int D = 16 * DC;
    // K row stride (halves): an odd number of 16-wide d chunks is padded with one chunk of
    // zeros, the upper half of the last score MFMA's K operand, so it is read, not zeroed
    constexpr int KLD = D + 8;
    constexpr int SP = 16 * KT;        // keys, padded
    constexpr int VT = SP + 8;         // V^T row stride (halves)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[SP * KLD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VT];

    const int S = a.S;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    // XCD-aware placement: workgroup i runs on XCD i % 8, so the logical (query split, head,
    // image) order is remapped into contiguous runs per XCD — each XCD takes whole images, whose
    // q/k/v rows (all heads interleaved in one row) its L2 then fetches once
    const int QS = gridDim.z;
    const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int lid = xcd_remap(lin, gridDim.x * gridDim.y * QS);
    const int zq = lid % QS, hb = lid / QS;
    const int h = hb % gridDim.x, b = hb / gridDim.x;
    const int64_t base = (int64_t)b * a.st[3] + (int64_t)h * a.st[2];

    // The staging is latency-bound (one workgroup per CU at typical shapes), so each round
    // issues all of a thread's K and V loads before it stores any, and the first query tile's
    // Q is requested with them: at the usual shapes one round trip fills LDS.
    // K row-major: a task moves 8 elements of a key row. V transposed: a task loads an
    // 8-key x 8-d block and stores it as eight 16-byte rows of V^T.
    constexpr int DW = D / 8;
    constexpr int KTASK = SP * DW, VTASK = (SP / 8) * DW;
    constexpr int UK = 8;              // K tasks per thread and round (one V task: 8 loads)
    static_assert(KTASK == UK * VTASK, "one V task per UK K tasks");

    const int nqt = (S + 15) / 16;
    const int qstep = nw * gridDim.z;
    int qt = zq * nw + wave;           // query split z takes query tiles z*nw + wave, + qstep, ...
    // Q as the B operand: lane = query 16t + l16, k = d = 16c + 4lg + j
    f16x4 qf[DC];
    auto load_q = [&](int t) {
        const int qi = min(16 * t + l16, S - 1);
        const int64_t qrow = base + (int64_t)qi * a.st[1];
#pragma unroll
        for (int c = 0; c < DC; c++) qf[c] = load_h4<I16>(a.q, a.q16, qrow + 16 * c + 4 * lg);
    };
    if (qt < nqt) load_q(qt);

    // rounds are workgroup-uniform: round r0 takes K tasks UK*r0 .. UK*(r0 + nth) - 1 and V
    // tasks r0 .. r0 + nth - 1
    for (int r0 = 0; r0 < VTASK; r0 += blockDim.x) {
        f16x8 kv[UK], vv[8];
        const f16x8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
        const int iv = r0 + tid, kg = iv / DW, dv = 8 * (iv - kg * DW);
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int idx = UK * r0 + u * blockDim.x + tid;
            const int t = idx / DW, d = 8 * (idx - t * DW);
            kv[u] = z8;
            if (idx < KTASK && t < S) kv[u] = load_h8<I16, A16>(a.k, a.k16, base + (int64_t)t * a.st[1] + d);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int t = 8 * kg + i;
            vv[i] = z8;
            if (iv < VTASK && t < S) vv[i] = load_h8<I16, A16>(a.v, a.v16, base + (int64_t)t * a.st[1] + dv);
        }
#pragma unroll
        for (int u = 0; u < UK; u++) {
            const int idx = UK * r0 + u * blockDim.x + tid;
            const int t = idx / DW, d = 8 * (idx - t * DW);
            if (idx < KTASK) *(f16x8*)&Ks[t * KLD + d] = kv[u];
        }
        if (iv < VTASK) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                *(f16x8*)&Vt[(dv + j) * VT + 8 * kg] = f16x8{vv[0][j], vv[1][j], vv[2][j], vv[3][j],
                                                            vv[4][j], vv[5][j], vv[6][j], vv[7][j]};
        }
    }
    __syncthreads();

    // scores in log2 units: exp(s*scale - max) = exp2(s*scale*log2(e) - max'), evaluated with
    // the hardware exp2 (v_exp_f32, ~1 ulp)
    const float scale2 = a.scale * 1.4426950408889634f;
    // Output rows are written with 8-byte (fp16) or 16-byte (fp32) stores when the features are
    // unit-stride and every row starts 16-byte aligned, element by element otherwise.
    const bool vec = a.os[0] == 1 && ((a.os[1] | a.os[2] | a.os[3]) & 3) == 0 &&
                     ((uintptr_t)(a.o16 ? (const void*)a.o16 : (const void*)a.o) & 15) == 0;
    constexpr int KC = (DC + 1) / 2;   // 32-deep MFMAs per score tile
    constexpr int NPT = (KT + 1) / 2;  // key-tile pairs of P . V (an odd last tile with zeros)
    // LDS fragment prefetch distances (key tiles for K, key-tile pairs for V), as far as the
    // registers allow
    constexpr int PF = KT <= 17 ? (DC <= 3 ? 2 : 0) : (DC <= 2 ? 1 : 0);
    constexpr int PFV = KT <= 17 && DC <= 3 ? 1 : 0;
    // P . V is computed transposed, O^T = V^T . P^T, with row i of the chunk-c V^T fragment
    // holding feature d = 4 DC (i / 4) + 4c + i % 4: O^T register r of chunk c in lane (l16,
    // lg) is then feature 4 DC lg + 4c + r of query q0 + l16, so each lane ends with 4 DC
    // consecutive features of one query and that query's softmax sum.
    const int vrow0 = 4 * DC * (l16 >> 2) + (l16 & 3);
    const float m1 = opaque_neg_one();
    for (; qt < nqt; qt += qstep) {
        const int q0 = 16 * qt;
        // Q as the B operand of the score MFMAs, d chunks in pairs
        f16x8 qb[KC];
#pragma unroll
        for (int i = 0; i < KC; i++)
            qb[i] = cat8(qf[2 * i], 2 * i + 1 < DC ? qf[2 * i + 1] : f16x4{0, 0, 0, 0});
        // scores: register r of key tile t holds key 16t + 4lg + r of query q0 + l16
        f32x4 sc[KT];
        float mx = -INFINITY;
        // pairs of 16-wide d chunks on the 32-deep MFMA (k = 8lg + j: d = 16(c + j/4) + 4lg + j%4
        // in both operands); an odd last chunk is paired with zeros (the 16-deep MFMA takes as
        // long, and a 16-deep MFMA accumulating right after a 32-deep one into the same
        // registers gave wrong sums). Fragments are read PF key tiles ahead.
        f16x8 kf[PF + 1][KC];
        auto kfrag = [&](int t, int i) {
            const _Float16* krow = &Ks[(16 * t + l16) * KLD + 4 * lg + 32 * i];
            return cat8(*(const f16x4*)krow, 2 * i + 1 < DC ? *(const f16x4*)(krow + 16) : f16x4{0, 0, 0, 0});
        };
        auto load_k = [&](int t, f16x8 (&f)[KC]) {
#pragma unroll
            for (int i = 0; i < KC; i++) f[i] = kfrag(t, i);
        };
#pragma unroll
        for (int t = 0; t < PF && t < KT; t++) load_k(t, kf[t]);
#pragma unroll
        for (int t = 0; t < KT; t++) {
            if (PF && t + PF < KT) load_k(t + PF, kf[(t + PF) % (PF + 1)]);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < KC; i++)   // without prefetch, one fragment at a time
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(PF ? kf[t % (PF + 1)][i] : kfrag(t, i), qb[i], acc, 0, 0, 0);
            // raw scores; keys past S are -inf (with TAIL only the last tile holds such keys;
            // otherwise the tiles from key S on, a uniform branch)
            if ((TAIL && t < KT - 1) || 16 * t + 16 <= S) {
                sc[t] = acc;
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) sc[t][r] = 16 * t + 4 * lg + r < S ? acc[r] : -INFINITY;
            }
            // the running max takes the previous tile, whose MFMAs have completed by now
            if (t > 0) {
                mx = fmaxf(fmaxf(mx, sc[t - 1][0]), sc[t - 1][1]);
                mx = fmaxf(fmaxf(mx, sc[t - 1][2]), sc[t - 1][3]);
            }
            __builtin_amdgcn_sched_barrier(0);  // the fragment reads stay PF tiles ahead
        }
        mx = fmaxf(fmaxf(mx, sc[KT - 1][0]), sc[KT - 1][1]);
        mx = fmaxf(fmaxf(mx, sc[KT - 1][2]), sc[KT - 1][3]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // the scores are done with Q: request the next tile's while this one's P . V runs
        if (qt + qstep < nqt) load_q(qt + qstep);
        // scale2 > 0 (checked at launch), so the max of the scaled scores is the scaled max;
        // p = exp2(s * scale2 - max) as one fma, and exp2(-inf) = 0 for the masked keys
        const float mxs = mx * scale2;
#pragma unroll
        for (int t = 0; t < KT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) sc[t][r] = __builtin_amdgcn_exp2f(fmaf(sc[t][r], scale2, -mxs));
        // O^T += V^T . P^T, P = hi + lo in fp16 (B operand: query l16, keys 16t + 4lg + j): hi
        // is P rounded toward zero, lo the exact remainder P - hi rounded toward zero
        // (|P - hi - lo| <= 2^-20 P, or 2^-24 where lo is an fp16 subnormal). The row sums
        // come from the same MFMAs on an all-ones V^T chunk (S1 = 1 . P^T: every register of
        // lane (l16, lg) holds the sum of query l16), so they add exactly the hi + lo that
        // the numerators use.
        f32x4 O[DC], S1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < DC; c++) O[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        const f16x4 z4 = {0, 0, 0, 0};
        const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
        // hi and lo operands of key tiles t, t + 1 (t + 1 = KT: zeros); p - hi is exact in fp32
        // and taken as one v_fma_mix_f32 (m1 = -1) per element
        auto split = [&](int t, f16x8& ph, f16x8& pl) {
            const f32x4 zf = {0.f, 0.f, 0.f, 0.f};
            const f32x4 a = sc[t], b = t + 1 < KT ? sc[t + 1] : zf;
            const auto h0 = __builtin_amdgcn_cvt_pkrtz(a[0], a[1]), h1 = __builtin_amdgcn_cvt_pkrtz(a[2], a[3]);
            const auto h2 = __builtin_amdgcn_cvt_pkrtz(b[0], b[1]), h3 = __builtin_amdgcn_cvt_pkrtz(b[2], b[3]);
            const auto l0 = __builtin_amdgcn_cvt_pkrtz(fmaf((float)h0[0], m1, a[0]), fmaf((float)h0[1], m1, a[1]));
            const auto l1 = __builtin_amdgcn_cvt_pkrtz(fmaf((float)h1[0], m1, a[2]), fmaf((float)h1[1], m1, a[3]));
            const auto l2 = __builtin_amdgcn_cvt_pkrtz(fmaf((float)h2[0], m1, b[0]), fmaf((float)h2[1], m1, b[1]));
            const auto l3 = __builtin_amdgcn_cvt_pkrtz(fmaf((float)h3[0], m1, b[2]), fmaf((float)h3[1], m1, b[3]));
            auto u = [](auto v) { return __builtin_bit_cast(uint32_t, v); };
            ph = __builtin_bit_cast(f16x8, u32x4{u(h0), u(h1), u(h2), u(h3)});
            pl = __builtin_bit_cast(f16x8, u32x4{u(l0), u(l1), u(l2), u(l3)});
        };
        // pairs of key tiles on the 32-deep MFMA (k = 8lg + j: key 16(t + j/4) + 4lg + j%4 in
        // both operands); an odd last tile is paired with zeros. V^T fragments are read PF
        // pairs ahead.
        f16x8 vf[PFV + 1][DC];
        auto vfrag = [&](int p, int c) {
            const _Float16* vrow = &Vt[(vrow0 + 4 * c) * VT + 32 * p + 4 * lg];
            return cat8(*(const f16x4*)vrow, 2 * p + 1 < KT ? *(const f16x4*)(vrow + 16) : z4);
        };
        auto load_v = [&](int p, f16x8 (&f)[DC]) {
#pragma unroll
            for (int c = 0; c < DC; c++) f[c] = vfrag(p, c);
        };
#pragma unroll
        for (int p = 0; p < PFV && p < NPT; p++) load_v(p, vf[p]);
#pragma unroll
        for (int p = 0; p < NPT; p++) {
            if (PFV && p + PFV < NPT) load_v(p + PFV, vf[(p + PFV) % (PFV + 1)]);
            f16x8 ph, pl;
            split(2 * p, ph, pl);
#pragma unroll
            for (int c = 0; c < DC; c++) {
                const f16x8 v = PFV ? vf[p % (PFV + 1)][c] : vfrag(p, c);   // without prefetch, one chunk at a time
                O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v, ph, O[c], 0, 0, 0);
                O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v, pl, O[c], 0, 0, 0);
            }
            S1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ph, S1, 0, 0, 0);
            S1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pl, S1, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);  // the fragment reads stay PFV pairs ahead
        }
        // features 4 DC lg .. 4 DC lg + 4 DC - 1 of query q0 + l16, divided by its row sum
        const float inv = 1.f / S1[0];
        const int qi = q0 + l16;
        if (qi < S) {
            const int64_t ro = (int64_t)b * a.os[3] + (int64_t)h * a.os[2] + (int64_t)qi * a.os[1];
            const int d0 = 4 * DC * lg;
            if (vec) {
#pragma unroll
                for (int c = 0; c < DC; c++) {
                    const f32x4 v = O[c] * inv;
                    if (a.o16)
                        *(f16x4*)(a.o16 + ro + d0 + 4 * c) = f16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                    else
                        *(f32x4*)(a.o + ro + d0 + 4 * c) = v;
                }
            } else {
#pragma unroll
                for (int c = 0; c < DC; c++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int64_t e = ro + (int64_t)(d0 + 4 * c + r) * a.os[0];
                        if (a.o16) a.o16[e] = (_Float16)(O[c][r] * inv);
                        else a.o[e] = O[c][r] * inv;
                    }
            }
        }
    }
}

template <int DC, int KT>
void launch_head_t(const FaArgs& a, hipStream_t s) {
    const int nqt = (a.S + 15) / 16;
    const int64_t heads = (int64_t)a.H * a.B;
    // A head's query tiles spread over qs workgroups (each restaging the head's K/V) while the
    // heads alone give fewer than ~256 workgroups, keeping >= 6 waves per workgroup (staging
    // with fewer threads costs more than the finer split gains); every query's arithmetic is
    // the same either way. Measured at S = 257, 16 heads (cfg4 shapes, fp32 q/k/v): one image
    // 10.8 us (3 workgroups per head) against ~15 us with 2 waves in 9 and 18 us unsplit;
    // 8 images 14.2 against 18.0 us unsplit (2 per head, 9 waves); at 16 images (256 heads)
    // splitting costs (29.4 against 21.4 us), so qs = 1 there, ~2 query tiles per wave.
    // With the staging down to one round trip, four waves per workgroup (one per SIMD) win
    // where that finer split still gives every workgroup its own CU: S = 257, one image 7.4
    // against 8.5 us (3 workgroups of 6 waves), two images 7.6 against 8.7; 3, 5, 6 or 9 waves
    // 8.4-9.8 us at one image.
    int qs = (int)std::max<int64_t>(1, std::min<int64_t>(256 / std::max<int64_t>(heads, 1), (nqt + 5) / 6));
    const bool tail = a.S > 16 * (KT - 1);
    const int maxw = a.q16 ? (tail ? kHeadWaves<DC, KT, true, true> : kHeadWaves<DC, KT, true, false>)
                           : (tail ? kHeadWaves<DC, KT, false, true> : kHeadWaves<DC, KT, false, false>);
    int nw = std::min(maxw, std::max(1, qs > 1 ? (nqt + qs - 1) / qs : (nqt + 1) / 2));
    if (qs > 1 && maxw >= 4 && heads * ((nqt + 3) / 4) <= 256) nw = 4;
    if (qs > 1) qs = (nqt + nw - 1) / nw;
    const dim3 grid((unsigned)a.H, (unsigned)a.B, (unsigned)qs), block((unsigned)(64 * nw));
    // fp16 rows 16-byte aligned (the pointers are, head_ok): one load per 8 elements
    const bool a16 = a.st[1] % 8 == 0 && a.st[2] % 8 == 0 && a.st[3] % 8 == 0;
    if (a.q16 && a16) {
        if (tail) hipLaunchKernelGGL((k_attn_head<DC, KT, true, true, true>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((k_attn_head<DC, KT, true, false, true>), grid, block, 0, s, a);
    } else if (a.q16) {
        if (tail) hipLaunchKernelGGL((k_attn_head<DC, KT, true, true, false>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((k_attn_head<DC, KT, true, false, false>), grid, block, 0, s, a);
    } else {
        if (tail) hipLaunchKernelGGL((k_attn_head<DC, KT, false, true, false>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((k_attn_head<DC, KT, false, false, false>), grid, block, 0, s, a);
    }
}

template <int DC>
hipError_t launch_head(const FaArgs& a, hipStream_t s) {
    const int kt = (a.S + 15) / 16;
    if (kt <= 4) launch_head_t<DC, 4>(a, s);
    else if (kt <= 8) launch_head_t<DC, 8>(a, s);
    else if (kt <= 17) launch_head_t<DC, 17>(a, s);
    else if (kt <= 24) launch_head_t<DC, 24>(a, s);
    else launch_head_t<DC, 32>(a, s);
    return hipGetLastError();
}

bool head_ok(const FaArgs& a, int D) {
    auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const bool ptrs = a.q16 ? al(a.q16) && al(a.k16) && al(a.v16) : al(a.q) && al(a.k) && al(a.v);
    return a.S <= 512 && a.st[0] == 1 && a.st[1] % 4 == 0 && a.st[2] % 4 == 0 && a.st[3] % 4 == 0 &&
           D % 16 == 0 && ptrs && a.H <= 65535 && a.B <= 65535 && a.scale > 0.f;
}

}  // namespace

hipError_t launch_flash_attn_f16kv(const FaArgs& a, int D, hipStream_t s) {
    if (a.S <= 0 || a.H <= 0 || a.B <= 0) return hipSuccess;
    if (a.q16 && !head_ok(a, D)) return hipErrorInvalidValue;   // fp16 inputs: whole-head kernel only
    if (head_ok(a, D)) {
        switch (D) {
            case 16: return launch_head<1>(a, s);
            case 32: return launch_head<2>(a, s);
            case 48: return launch_head<3>(a, s);
            case 64: return launch_head<4>(a, s);
            default: break;
        }
    }
    const dim3 grid((unsigned)((a.S + 63) / 64), (unsigned)a.H, (unsigned)a.B), block(256);
    switch (D) {
        case 16: hipLaunchKernelGGL(k_flash_attn_f16kv<1>, grid, block, 0, s, a); break;
        case 32: hipLaunchKernelGGL(k_flash_attn_f16kv<2>, grid, block, 0, s, a); break;
        case 48: hipLaunchKernelGGL(k_flash_attn_f16kv<3>, grid, block, 0, s, a); break;
        case 64: hipLaunchKernelGGL(k_flash_attn_f16kv<4>, grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mgh
