// k_gemm_i8.hip — ggml Q8_0 / Q4_K weights x per-32-block int8 activations on gfx950 MFMA.
//
// Semantics: the reference's int8-dot FC kernels
//   Q8_0  k_mul_mat_q8_i8  (src/mg-opencl/mg-opencl.cpp:440-494)
//   Q4_K  k_mul_mat_q4k_i8 (src/mg-opencl/mg-opencl.cpp:504-590)
// For output (m, n) and every 32-wide K block t:
//   idot = sum_i qw[n,t,i] * qx[m,32t+i]                                  (int32, exact)
//   Q8_0: acc += (dx[m,t] * dw[n,t]) * idot
//   Q4_K: acc += (dx[m,t] * d*sc_j[n]) * idot - (dx[m,t]*sum_i qx[m,32t+i]) * dmin*m_j[n]
// then the fused epilogue y = act(acc + bias[n]) + resid[m,n] (mg-opencl.cpp:485-491).
//
// gfx950 design:
//  * Matrix cores do all three products of a 32x32 output tile and a pair of K blocks:
//      - v_mfma_i32_32x32x32_i8, once per block: K = 32 is exactly one ggml block, so the
//        int32 block dot comes out whole and bit-exact;
//      - v_mfma_f32_32x32x1_2b_f32, once per block pair: two outer products dx (x) dw, i.e.
//        the per-(m,n,block) scale, delivered in the same register layout as the dots;
//      - Q4_K only: v_mfma_f32_32x32x2_f32 accumulates the min-correction term of both
//        blocks, (dx*sum qx) . (dmin*m)^T, into its own accumulator.
//    The VALU is left with one int->float convert and one FMA per output and block.
//  * 256-thread workgroups = 2x2 waves; each wave owns WM x WN 32x32 tiles, so a workgroup
//    covers BM = 64*WM activation rows by BN = 64*WN weight rows.
//  * K advances in steps of KS = 4 blocks. Raw GGUF blocks are streamed from their file
//    layout (no repacking) and de-interleaved in registers: a Q8_0 block pair is 68
//    dword-aligned bytes (quants re-aligned with v_alignbyte), a Q4_K super-block gives its
//    16-byte header and 64 nibble bytes per step. int8 operands sit in LDS as 16-byte pieces
//    under an XOR swizzle: conflict-free for both the coalesced writes and the MFMA reads.
//  * Two LDS stages: global loads for step s+1 are in flight while step s is computed, and
//    a single barrier per step separates the stages. Loads use clamped addresses and carry
//    no data-dependent branches, so no wait is emitted before the compute phase.
//  * Blocks past K (when K/32 is not a multiple of KS) get zero scales, contributing 0.
//  * Workgroups are remapped so each XCD walks a contiguous range of M-major tiles.
//  * DEBUG writes the MFMA's int32 block dots instead of accumulating; that is how the
//    bit-exactness of the block dots is tested.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

typedef float f32x32 __attribute__((ext_vector_type(32)));

constexpr int KS = 4;            // 32-blocks per K step (two block pairs)
constexpr int NTHREADS = 256;

template <int WTYPE, int WM, int WN>
struct Shape {
    static constexpr bool Q4K = WTYPE == 12;
    static constexpr int BM = 64 * WM;
    static constexpr int BN = 64 * WN;
    static constexpr int A_ITEMS = BM * KS * 2 / NTHREADS;                 // 16-B pieces / thread
    static constexpr int B_ITEMS = Q4K ? (BN + NTHREADS - 1) / NTHREADS          // rows
                                       : (BN * 2 + NTHREADS - 1) / NTHREADS;     // block pairs
    static constexpr int B_VECS = Q4K ? 5 : 4;     // 16-byte vectors per item
};

// One LDS stage (one K step).
template <int WTYPE, int WM, int WN>
struct Stage {
    using S = Shape<WTYPE, WM, WN>;
    u32x4 a[S::BM * KS * 2];                // int8 activations, 16-byte pieces, swizzled
    u32x4 b[S::BN * KS * 2];                // int8 weights (Q4_K nibbles as 0..15)
    float sa[KS * S::BM];                   // dx per (block, row); 0 past K
    float sb[KS * S::BN];                   // dw (Q8_0) or d*sc (Q4_K) per (block, row)
    float ua[S::Q4K ? KS * S::BM : 1];      // dx * sum(qx)
    float mb[S::Q4K ? KS * S::BN : 1];      // dmin * m
};

// Registers holding one K step of global data while the previous step is computed. The
// weight bytes stay in whole 16-byte vectors (the load destinations) until the LDS store,
// so the loop carries them without register shuffles that would wait on the loads.
template <int WTYPE, int WM, int WN>
struct Prefetch {
    using S = Shape<WTYPE, WM, WN>;
    u32x4 a[S::A_ITEMS];
    float dxv[KS];
    int32_t sxv[KS];
    u32x4 bv[S::B_ITEMS][S::B_VECS];   // Q8_0: block pair bytes 0..63; Q4_K: header + nibbles
    uint32_t btail[S::B_ITEMS];        // Q8_0: block pair bytes 64..67
};

template <int WTYPE, int WM, int WN, bool SCALES>
__device__ __forceinline__ void load_step(Prefetch<WTYPE, WM, WN>& p, const GemmArgs& g,
                                          int m0, int n0, int t0, int nb) {
    using S = Shape<WTYPE, WM, WN>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < S::A_ITEMS; k++) {
        const int i = tid + k * NTHREADS;
        const int r = i >> 3, piece = i & 7;
        const int t = min(t0 + (piece >> 1), nb - 1);
        const int m = min(m0 + r, g.M - 1);
        p.a[k] = *(const u32x4*)(g.qx + (size_t)m * g.K + (size_t)t * 32 + (piece & 1) * 16);
    }
    if (SCALES && tid < S::BM) {
        const size_t row = (size_t)min(m0 + tid, g.M - 1) * nb;
#pragma unroll
        for (int kb = 0; kb < KS; kb++) {
            const int t = min(t0 + kb, nb - 1);
            p.dxv[kb] = g.dx[row + t];
            if (S::Q4K) p.sxv[kb] = g.sx[row + t];
        }
    }
#pragma unroll
    for (int k = 0; k < S::B_ITEMS; k++) {
        const int i = tid + k * NTHREADS;
        if (!S::Q4K) {
            if (i < S::BN * 2) {
                const int n = min(n0 + (i >> 1), g.N - 1);
                const int t = min(t0 + (i & 1) * 2, nb - 2);
                const uint8_t* src = g.w + ((size_t)n * nb + t) * 34;
#pragma unroll
                for (int q = 0; q < 4; q++) p.bv[k][q] = ((const u32x4a4*)src)[q];
                p.btail[k] = *(const uint32_t*)(src + 64);
            }
        } else {
            if (i < S::BN) {
                const int n = min(n0 + i, g.N - 1);
                const uint8_t* sbp = g.w + ((size_t)n * (nb / 8) + (t0 >> 3)) * 144;
                p.bv[k][0] = *(const u32x4*)sbp;
                const u32x4* nib = (const u32x4*)(sbp + 16 + ((t0 >> 2) & 1) * 64);
#pragma unroll
                for (int q = 0; q < 4; q++) p.bv[k][1 + q] = nib[q];
            }
        }
    }
}

// byte j of the 12-byte Q4_K scale array held in three dwords
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int j) {
    const uint32_t w = j < 4 ? s0 : (j < 8 ? s1 : s2);
    return (w >> (8 * (j & 3))) & 0xffu;
}

template <int WTYPE, int WM, int WN, bool SCALES>
__device__ __forceinline__ void store_step(const Prefetch<WTYPE, WM, WN>& p,
                                           Stage<WTYPE, WM, WN>& st, int t0, int nb) {
    using S = Shape<WTYPE, WM, WN>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < S::A_ITEMS; k++) {
        const int i = tid + k * NTHREADS;
        st.a[swz_slot(i & 7, i >> 3, S::BM)] = p.a[k];
    }
    if (SCALES && tid < S::BM) {
#pragma unroll
        for (int kb = 0; kb < KS; kb++) {
            const bool ok = t0 + kb < nb;
            st.sa[kb * S::BM + tid] = ok ? p.dxv[kb] : 0.0f;
            if (S::Q4K) st.ua[kb * S::BM + tid] = ok ? p.dxv[kb] * (float)p.sxv[kb] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < S::B_ITEMS; k++) {
        const int i = tid + k * NTHREADS;
        uint32_t w[S::Q4K ? 20 : 17];
#pragma unroll
        for (int q = 0; q < S::B_VECS; q++) {
            w[4 * q + 0] = p.bv[k][q].x; w[4 * q + 1] = p.bv[k][q].y;
            w[4 * q + 2] = p.bv[k][q].z; w[4 * q + 3] = p.bv[k][q].w;
        }
        if (!S::Q4K) w[16] = p.btail[k];
        if (!S::Q4K) {
            if (i < S::BN * 2) {
                const int rl = i >> 1, kb0 = (i & 1) * 2;
                const bool ok = t0 + kb0 < nb;
                // even block: fp16 scale in bytes 0-1, quants at bytes 2..33
                u32x4 q0, q1;
                q0.x = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
                q0.y = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
                q0.z = __builtin_amdgcn_alignbyte(w[3], w[2], 2);
                q0.w = __builtin_amdgcn_alignbyte(w[4], w[3], 2);
                q1.x = __builtin_amdgcn_alignbyte(w[5], w[4], 2);
                q1.y = __builtin_amdgcn_alignbyte(w[6], w[5], 2);
                q1.z = __builtin_amdgcn_alignbyte(w[7], w[6], 2);
                q1.w = __builtin_amdgcn_alignbyte(w[8], w[7], 2);
                st.b[swz_slot(kb0 * 2 + 0, rl, S::BN)] = q0;
                st.b[swz_slot(kb0 * 2 + 1, rl, S::BN)] = q1;
                // odd block: fp16 scale in bytes 34-35 (high half of word 8), quants = words 9..16
                st.b[swz_slot(kb0 * 2 + 2, rl, S::BN)] = u32x4{w[9], w[10], w[11], w[12]};
                st.b[swz_slot(kb0 * 2 + 3, rl, S::BN)] = u32x4{w[13], w[14], w[15], w[16]};
                if (SCALES) {
                    st.sb[kb0 * S::BN + rl] = ok ? h2f(w[0] & 0xffffu) : 0.0f;
                    st.sb[(kb0 + 1) * S::BN + rl] = ok ? h2f(w[8] >> 16) : 0.0f;
                }
            }
        } else {
            if (i < S::BN) {
                const float d = h2f(w[0] & 0xffffu), dmin = h2f(w[0] >> 16);
                const int half = (t0 >> 2) & 1;
#pragma unroll
                for (int jj = 0; jj < KS; jj++) {
                    const int j = half * 4 + jj;       // sub-block within the super-block
                    uint32_t sc, mn;
                    if (j < 4) {
                        sc = sbyte(w[1], w[2], w[3], j) & 63u;
                        mn = sbyte(w[1], w[2], w[3], j + 4) & 63u;
                    } else {
                        sc = (sbyte(w[1], w[2], w[3], j + 4) & 0xFu) | ((sbyte(w[1], w[2], w[3], j - 4) >> 6) << 4);
                        mn = (sbyte(w[1], w[2], w[3], j + 4) >> 4) | ((sbyte(w[1], w[2], w[3], j) >> 6) << 4);
                    }
                    if (SCALES) {
                        st.sb[jj * S::BN + i] = d * (float)sc;
                        st.mb[jj * S::BN + i] = dmin * (float)mn;
                    }
                    // nibble group jj>>1 (32 bytes = 8 dwords): low nibbles for even jj
                    const uint32_t* g8 = w + 4 + (jj >> 1) * 8;
                    const int sh = (jj & 1) * 4;
                    u32x4 q0, q1;
                    q0.x = (g8[0] >> sh) & 0x0F0F0F0Fu; q0.y = (g8[1] >> sh) & 0x0F0F0F0Fu;
                    q0.z = (g8[2] >> sh) & 0x0F0F0F0Fu; q0.w = (g8[3] >> sh) & 0x0F0F0F0Fu;
                    q1.x = (g8[4] >> sh) & 0x0F0F0F0Fu; q1.y = (g8[5] >> sh) & 0x0F0F0F0Fu;
                    q1.z = (g8[6] >> sh) & 0x0F0F0F0Fu; q1.w = (g8[7] >> sh) & 0x0F0F0F0Fu;
                    st.b[swz_slot(jj * 2 + 0, i, S::BN)] = q0;
                    st.b[swz_slot(jj * 2 + 1, i, S::BN)] = q1;
                }
            }
        }
    }
}

template <int ACT>
__device__ __forceinline__ float act_t(float v) {
    if (ACT == 1) return gelu_erf(v);
    if (ACT == 2) return v / (1.0f + expf(-v));
    return v;
}

}  // namespace

template <int WTYPE, int WM, int WN, int ACT, bool DEBUG>
__global__ __launch_bounds__(NTHREADS) void k_gemm_q_i8(GemmArgs g) {
    using S = Shape<WTYPE, WM, WN>;
    __shared__ Stage<WTYPE, WM, WN> lds[2];

    const int nb = g.K / 32;
    const int tiles_n = (g.N + S::BN - 1) / S::BN;
    const int tiles = tiles_n * ((g.M + S::BM - 1) / S::BM);
    const int L = xcd_remap(blockIdx.x, tiles);
    const int m0 = (L / tiles_n) * S::BM;
    const int n0 = (L % tiles_n) * S::BN;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * WM * 32;
    const int wn0 = (wave & 1) * WN * 32;
    const int hl = lane >> 5;          // lane half: which 16 bytes of a block / which block of a pair
    const int l32 = lane & 31;

    f32x16 acc[WM][WN], accm[S::Q4K ? WM : 1][S::Q4K ? WN : 1];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    if (S::Q4K) {
#pragma unroll
        for (int i = 0; i < (S::Q4K ? WM : 1); i++)
#pragma unroll
            for (int j = 0; j < (S::Q4K ? WN : 1); j++)
#pragma unroll
                for (int r = 0; r < 16; r++) accm[i][j][r] = 0.0f;
    }

    Prefetch<WTYPE, WM, WN> pf;
    const int steps = (nb + KS - 1) / KS;
    load_step<WTYPE, WM, WN, !DEBUG>(pf, g, m0, n0, 0, nb);
    store_step<WTYPE, WM, WN, !DEBUG>(pf, lds[0], 0, nb);
    __syncthreads();

    for (int s = 0; s < steps; s++) {
        const int t0 = s * KS;
        const Stage<WTYPE, WM, WN>& st = lds[s & 1];
        if (s + 1 < steps) load_step<WTYPE, WM, WN, !DEBUG>(pf, g, m0, n0, t0 + KS, nb);

#pragma unroll
        for (int kp = 0; kp < KS / 2; kp++) {
            const int kb0 = 2 * kp;
            i32x4 af[2][WM], bf[2][WN];
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int i = 0; i < WM; i++)
                    af[h][i] = (i32x4)st.a[swz_slot((kb0 + h) * 2 + hl, wm0 + i * 32 + l32, S::BM)];
#pragma unroll
                for (int j = 0; j < WN; j++)
                    bf[h][j] = (i32x4)st.b[swz_slot((kb0 + h) * 2 + hl, wn0 + j * 32 + l32, S::BN)];
            }
            if (DEBUG) {
#pragma unroll
                for (int i = 0; i < WM; i++)
#pragma unroll
                    for (int j = 0; j < WN; j++)
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const i32x16 z = {};
                            const i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[h][i], bf[h][j], z, 0, 0, 0);
                            const int n = n0 + wn0 + j * 32 + l32;
                            const int t = t0 + kb0 + h;
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
                                if (m < g.M && n < g.N && t < nb)
                                    g.dots[((size_t)m * g.N + n) * nb + t] = I[r];
                            }
                        }
                continue;
            }
            // outer-product operands: lane half hl carries block kb0 + hl
            float sa[WM], sb[WN], ua[S::Q4K ? WM : 1], mb[S::Q4K ? WN : 1];
#pragma unroll
            for (int i = 0; i < WM; i++) {
                sa[i] = st.sa[(kb0 + hl) * S::BM + wm0 + i * 32 + l32];
                if (S::Q4K) ua[i] = st.ua[(kb0 + hl) * S::BM + wm0 + i * 32 + l32];
            }
#pragma unroll
            for (int j = 0; j < WN; j++) {
                sb[j] = st.sb[(kb0 + hl) * S::BN + wn0 + j * 32 + l32];
                if (S::Q4K) mb[j] = -st.mb[(kb0 + hl) * S::BN + wn0 + j * 32 + l32];
            }
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++) {
                    const f32x32 z32 = {};
                    const i32x16 z16 = {};
                    const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sa[i], sb[j], z32, 0, 0, 0);
                    const i32x16 I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0][i], bf[0][j], z16, 0, 0, 0);
                    const i32x16 I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[1][i], bf[1][j], z16, 0, 0, 0);
                    if (S::Q4K)
                        accm[S::Q4K ? i : 0][S::Q4K ? j : 0] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            ua[S::Q4K ? i : 0], mb[S::Q4K ? j : 0], accm[S::Q4K ? i : 0][S::Q4K ? j : 0], 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[i][j][r] = __builtin_fmaf(sc[r], (float)I0[r], acc[i][j][r]);
                        acc[i][j][r] = __builtin_fmaf(sc[16 + r], (float)I1[r], acc[i][j][r]);
                    }
                }
        }

        if (s + 1 < steps) store_step<WTYPE, WM, WN, !DEBUG>(pf, lds[(s + 1) & 1], t0 + KS, nb);
        __syncthreads();
    }
    if (DEBUG) return;

    // fused epilogue: +bias -> act -> +resid (mg-opencl.cpp:485-491)
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = n0 + wn0 + j * 32 + l32;
        if (n >= g.N) continue;
        const float bv = g.bias ? g.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
                if (m >= g.M) continue;
                float v = acc[i][j][r];
                if (S::Q4K) v += accm[S::Q4K ? i : 0][S::Q4K ? j : 0][r];
                v = act_t<ACT>(v + bv);
                const size_t idx = (size_t)m * g.N + n;
                if (g.resid) v += g.resid[idx];
                g.y[idx] = v;
            }
    }
}

template <int WTYPE, int WM, int WN>
static hipError_t launch_cfg(const GemmArgs& a, bool dbg, hipStream_t s) {
    using S = Shape<WTYPE, WM, WN>;
    const int tiles = ((a.M + S::BM - 1) / S::BM) * ((a.N + S::BN - 1) / S::BN);
    const dim3 grid(tiles), block(NTHREADS);
    if (dbg) hipLaunchKernelGGL((k_gemm_q_i8<WTYPE, WM, WN, 0, true>), grid, block, 0, s, a);
    else if (a.act == 1) hipLaunchKernelGGL((k_gemm_q_i8<WTYPE, WM, WN, 1, false>), grid, block, 0, s, a);
    else if (a.act == 2) hipLaunchKernelGGL((k_gemm_q_i8<WTYPE, WM, WN, 2, false>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_gemm_q_i8<WTYPE, WM, WN, 0, false>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int WTYPE>
static hipError_t launch_type(const GemmArgs& a, TileCfg t, bool dbg, hipStream_t s) {
    if (t.wm == 1 && t.wn == 2) return launch_cfg<WTYPE, 1, 2>(a, dbg, s);
    if (t.wm == 2 && t.wn == 1) return launch_cfg<WTYPE, 2, 1>(a, dbg, s);
    if (t.wm == 1 && t.wn == 1) return launch_cfg<WTYPE, 1, 1>(a, dbg, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_q_i8(int wtype, const GemmArgs& a, TileCfg t, bool debug_dots, hipStream_t s) {
    if (wtype == 8) return launch_type<8>(a, t, debug_dots, s);
    if (wtype == 12) return launch_type<12>(a, t, debug_dots, s);
    return hipErrorInvalidValue;
}

}  // namespace mgh
