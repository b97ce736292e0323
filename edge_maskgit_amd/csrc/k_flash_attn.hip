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
// registers are the P operand as they stand).
// at most NW waves (a workgroup takes min(NW, ~half the query tiles) waves), so the score
// registers (4 * KT per lane) fit without spilling
template <int KT>
constexpr int kHeadWaves = KT <= 17 ? (KT + 1) / 2 : 8;

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
__global__ __launch_bounds__(64 * kHeadWaves<KT>) void k_attn_head(FaArgs a) {
    constexpr int D = 16 * DC;
    constexpr int KLD = D + 8;         // K row stride (halves)
    constexpr int SP = 16 * KT;        // keys, padded
    constexpr int VT = SP + 8;         // V^T row stride (halves)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[SP * KLD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VT];

    const int S = a.S;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int h = blockIdx.x, b = blockIdx.y;
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
    int qt = blockIdx.z * nw + wave;   // workgroup z takes query tiles z*nw + wave, + qstep, ...
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
    for (; qt < nqt; qt += qstep) {
        const int q0 = 16 * qt;
        // scores: register r of key tile t holds key 16t + 4lg + r of query q0 + l16
        f32x4 sc[KT];
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < KT; t++) {
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
            // raw scores; keys past S are -inf (with TAIL only the last tile holds such keys)
            if (TAIL && t < KT - 1) {
                sc[t] = acc;
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) sc[t][r] = 16 * t + 4 * lg + r < S ? acc[r] : -INFINITY;
            }
            mx = fmaxf(fmaxf(mx, sc[t][0]), sc[t][1]);
            mx = fmaxf(fmaxf(mx, sc[t][2]), sc[t][3]);
            __builtin_amdgcn_sched_barrier(0);  // keep the K fragment loads per key tile
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // the scores are done with Q: request the next tile's while this one's P . V runs
        if (qt + qstep < nqt) load_q(qt + qstep);
        // scale2 > 0 (checked at launch), so the max of the scaled scores is the scaled max;
        // p = exp2(s * scale2 - max) as one fma, and exp2(-inf) = 0 for the masked keys
        const float mxs = mx * scale2;
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < KT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(fmaf(sc[t][r], scale2, -mxs));
                sc[t][r] = p;
                ps += p;
            }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        // O += P . V, P = hi + lo in fp16 (A operand: query l16, keys 16t + 4lg + j): hi is P
        // rounded toward zero, lo the exact remainder rounded toward zero (|P - hi - lo| <=
        // 2^-20 P)
        f32x4 O[DC];
#pragma unroll
        for (int c = 0; c < DC; c++) O[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto split = [&](int t, f16x4& ph, f16x4& pl) {
            const auto h01 = __builtin_amdgcn_cvt_pkrtz(sc[t][0], sc[t][1]);
            const auto h23 = __builtin_amdgcn_cvt_pkrtz(sc[t][2], sc[t][3]);
            const auto l01 = __builtin_amdgcn_cvt_pkrtz(sc[t][0] - (float)h01[0], sc[t][1] - (float)h01[1]);
            const auto l23 = __builtin_amdgcn_cvt_pkrtz(sc[t][2] - (float)h23[0], sc[t][3] - (float)h23[1]);
            ph = __builtin_bit_cast(f16x4, u32x2{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)});
            pl = __builtin_bit_cast(f16x4, u32x2{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)});
        };
        // pairs of key tiles on the 32-deep MFMA (k = 8lg + j: key 16(t + j/4) + 4lg + j%4 in
        // both operands), an odd last tile on the 16-deep one
#pragma unroll
        for (int t = 0; t + 1 < KT; t += 2) {
            f16x4 ph0, pl0, ph1, pl1;
            split(t, ph0, pl0);
            split(t + 1, ph1, pl1);
            const f16x8 ph = cat8(ph0, ph1), pl = cat8(pl0, pl1);
#pragma unroll
            for (int c = 0; c < DC; c++) {
                const _Float16* vrow = &Vt[(16 * c + l16) * VT + 16 * t + 4 * lg];
                const f16x8 vf = cat8(*(const f16x4*)vrow, *(const f16x4*)(vrow + 16));
                O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vf, O[c], 0, 0, 0);
                O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vf, O[c], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the V fragment loads per key tile pair (registers)
        }
        if (KT % 2) {                          // the odd last tile, paired with zeros
            f16x4 ph, pl;
            split(KT - 1, ph, pl);
            const f16x4 z = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < DC; c++) {
                const f16x8 vf = cat8(*(const f16x4*)&Vt[(16 * c + l16) * VT + 16 * (KT - 1) + 4 * lg], z);
                O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cat8(ph, z), vf, O[c], 0, 0, 0);
                O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cat8(pl, z), vf, O[c], 0, 0, 0);
            }
        }
        // O register r: query q0 + 4lg + r, d = 16c + l16; its row sum sits in lane 4lg + r
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float inv = 1.f / __shfl(ps, 4 * lg + r);
            const int qi = q0 + 4 * lg + r;
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
    int nw = std::min(kHeadWaves<KT>, std::max(1, qs > 1 ? (nqt + qs - 1) / qs : (nqt + 1) / 2));
    if (qs > 1 && kHeadWaves<KT> >= 4 && heads * ((nqt + 3) / 4) <= 256) nw = 4;
    if (qs > 1) qs = (nqt + nw - 1) / nw;
    const dim3 grid((unsigned)a.H, (unsigned)a.B, (unsigned)qs), block((unsigned)(64 * nw));
    const bool tail = a.S > 16 * (KT - 1);
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
