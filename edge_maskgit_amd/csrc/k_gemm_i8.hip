// k_gemm_i8.hip — ggml Q8_0 / Q4_K weights x per-32-block int8 activations on gfx950 MFMA.
//
// Semantics: the reference's int8-dot FC kernels
//   Q8_0  k_mul_mat_q8_i8  (src/mg-opencl/mg-opencl.cpp:440-494)
//   Q4_K  k_mul_mat_q4k_i8 (src/mg-opencl/mg-opencl.cpp:504-590)
// For output (m, n) and every 32-wide K block t, in order t = 0..K/32-1:
//   idot = sum_i qw[n,t,i] * qx[m,32t+i]                                  (int32, exact)
//   Q8_0: acc += (dw[n,t] * dx[m,t]) * idot
//   Q4_K: acc += (d*sc_j * dx[m,t]) * idot - (dmin*m_j) * (dx[m,t] * sum_i qx[m,32t+i])
// then the fused epilogue y = act(acc + bias[n]) + resid[m,n] (mg-opencl.cpp:485-491).
//
// gfx950 design (not a translation of the OpenCL 16x16-workgroup tiling):
//  * One v_mfma_i32_32x32x32_i8 per (32x32 output tile, K block): its K of 32 is exactly
//    one ggml block, so the int32 block dot comes out of the matrix core whole and the
//    per-block scales are applied in registers (cvt + mul + fma per output per block).
//  * 256-thread workgroups = 2x2 waves; each wave owns WM x WN 32x32 tiles, so a
//    workgroup covers BM = 64*WM rows by BN = 64*WN weight rows.
//  * K advances in steps of KS = 4 blocks (128 K). The raw GGUF blocks are streamed
//    with 16-byte loads straight from their file layout (no repacking) and de-interleaved
//    in registers: a Q8_0 block pair is 68 dword-aligned bytes (scale words + quants via
//    v_alignbyte), a Q4_K super-block contributes its 16-byte header and 64 nibble bytes
//    per step. int8 operands land in LDS in 16-byte pieces under an XOR swizzle, so both
//    the coalesced-order writes and the MFMA-order reads are bank-conflict free.
//  * Global loads for step s+1 are issued before the MFMAs of step s (register prefetch).
//  * Workgroups are remapped so each XCD walks a contiguous range of M-major tiles.
//  * Debug mode writes the MFMA's int32 block dots instead of accumulating, which is how
//    the bit-exactness of the block dots is checked.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

constexpr int KS = 4;            // 32-blocks per K step
constexpr int NTHREADS = 256;

template <int WTYPE, int WM, int WN>
struct GemmI8Shape {
    static constexpr int BM = 64 * WM;
    static constexpr int BN = 64 * WN;
    static constexpr int A_ITEMS = BM * KS * 2 / NTHREADS;          // 16-byte pieces / thread
    static constexpr int B_ITEMS = WTYPE == 8 ? (BN * 2 + NTHREADS - 1) / NTHREADS  // pairs
                                              : (BN + NTHREADS - 1) / NTHREADS;     // rows
    static constexpr int LDS_A = BM * KS * 32;                      // bytes
    static constexpr int LDS_B = BN * KS * 32;
};

// Registers holding one K step of global data, in flight across the MFMA phase.
template <int WTYPE, int WM, int WN>
struct Prefetch {
    using S = GemmI8Shape<WTYPE, WM, WN>;
    u32x4 a[S::A_ITEMS];
    float dxv[KS];
    int32_t sxv[KS];
    uint32_t b[S::B_ITEMS][WTYPE == 8 ? 17 : 20];
};

template <int WTYPE, int WM, int WN, bool SCALES>
__device__ __forceinline__ void load_step(Prefetch<WTYPE, WM, WN>& p, const GemmArgs& g,
                                          int m0, int n0, int t0, int nb) {
    using S = GemmI8Shape<WTYPE, WM, WN>;
    const int tid = threadIdx.x;
    // activations: BM rows x 8 pieces of 16 bytes (4 blocks)
#pragma unroll
    for (int k = 0; k < S::A_ITEMS; k++) {
        const int i = tid + k * NTHREADS;
        const int r = i >> 3, piece = i & 7, kb = piece >> 1;
        const int m = min(m0 + r, g.M - 1);
        if (t0 + kb < nb)
            p.a[k] = *(const u32x4*)(g.qx + (size_t)m * g.K + (size_t)(t0 + kb) * 32 + (piece & 1) * 16);
        else
            p.a[k] = u32x4{0u, 0u, 0u, 0u};
    }
    // activation scales (and block sums for Q4_K): one row per thread. The debug-dots
    // mode has no scales (dx/sx are null) and must not read them.
    if (SCALES && tid < S::BM) {
        const int m = min(m0 + tid, g.M - 1);
#pragma unroll
        for (int kb = 0; kb < KS; kb++) {
            const bool ok = t0 + kb < nb;
            p.dxv[kb] = ok ? g.dx[(size_t)m * nb + t0 + kb] : 0.0f;
            if (WTYPE == 12) p.sxv[kb] = ok ? g.sx[(size_t)m * nb + t0 + kb] : 0;
        }
    }
    // weights
#pragma unroll
    for (int k = 0; k < S::B_ITEMS; k++) {
        if (WTYPE == 8) {
            const int i = tid + k * NTHREADS;       // (row, pair)
            if (i < S::BN * 2) {
                const int n = min(n0 + (i >> 1), g.N - 1);
                const int t = t0 + (i & 1) * 2;
                if (t < nb) {
                    const uint8_t* src = g.w + ((size_t)n * nb + t) * 34;
                    const u32x4a4* s4 = (const u32x4a4*)src;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        u32x4a4 v = s4[q];
                        p.b[k][4 * q + 0] = v.x; p.b[k][4 * q + 1] = v.y;
                        p.b[k][4 * q + 2] = v.z; p.b[k][4 * q + 3] = v.w;
                    }
                    p.b[k][16] = *(const uint32_t*)(src + 64);
                } else {
#pragma unroll
                    for (int q = 0; q < 17; q++) p.b[k][q] = 0u;
                }
            }
        } else {
            const int i = tid + k * NTHREADS;       // row
            if (i < S::BN) {
                const int n = min(n0 + i, g.N - 1);
                const int nsb = nb / 8;
                const uint8_t* sbp = g.w + ((size_t)n * nsb + (t0 >> 3)) * 144;
                const u32x4 hdr = *(const u32x4*)sbp;
                p.b[k][0] = hdr.x; p.b[k][1] = hdr.y; p.b[k][2] = hdr.z; p.b[k][3] = hdr.w;
                const u32x4* nib = (const u32x4*)(sbp + 16 + ((t0 >> 2) & 1) * 64);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    u32x4 v = nib[q];
                    p.b[k][4 + 4 * q + 0] = v.x; p.b[k][4 + 4 * q + 1] = v.y;
                    p.b[k][4 + 4 * q + 2] = v.z; p.b[k][4 + 4 * q + 3] = v.w;
                }
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
__device__ __forceinline__ void store_step(const Prefetch<WTYPE, WM, WN>& p, uint8_t* ldsA,
                                           uint8_t* ldsB, float* sA, float* uA, float* sB,
                                           float* mB, int t0) {
    using S = GemmI8Shape<WTYPE, WM, WN>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < S::A_ITEMS; k++) {
        const int i = tid + k * NTHREADS;
        const int r = i >> 3, piece = i & 7;
        *(u32x4*)(ldsA + swz_slot(piece, r, S::BM) * 16) = p.a[k];
    }
    if (SCALES && tid < S::BM) {
#pragma unroll
        for (int kb = 0; kb < KS; kb++) {
            sA[kb * S::BM + tid] = p.dxv[kb];
            if (WTYPE == 12) uA[kb * S::BM + tid] = p.dxv[kb] * (float)p.sxv[kb];
        }
    }
#pragma unroll
    for (int k = 0; k < S::B_ITEMS; k++) {
        if (WTYPE == 8) {
            const int i = tid + k * NTHREADS;
            if (i < S::BN * 2) {
                const int rl = i >> 1, kb0 = (i & 1) * 2;
                const uint32_t* w = p.b[k];
                // even block: scale in bytes 0-1, quants at bytes 2..33 (2-byte offset)
                u32x4 q0, q1;
                q0.x = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
                q0.y = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
                q0.z = __builtin_amdgcn_alignbyte(w[3], w[2], 2);
                q0.w = __builtin_amdgcn_alignbyte(w[4], w[3], 2);
                q1.x = __builtin_amdgcn_alignbyte(w[5], w[4], 2);
                q1.y = __builtin_amdgcn_alignbyte(w[6], w[5], 2);
                q1.z = __builtin_amdgcn_alignbyte(w[7], w[6], 2);
                q1.w = __builtin_amdgcn_alignbyte(w[8], w[7], 2);
                *(u32x4*)(ldsB + swz_slot(kb0 * 2 + 0, rl, S::BN) * 16) = q0;
                *(u32x4*)(ldsB + swz_slot(kb0 * 2 + 1, rl, S::BN) * 16) = q1;
                // odd block: scale in bytes 34-35 (high half of word 8), quants = words 9..16
                *(u32x4*)(ldsB + swz_slot(kb0 * 2 + 2, rl, S::BN) * 16) = u32x4{w[9], w[10], w[11], w[12]};
                *(u32x4*)(ldsB + swz_slot(kb0 * 2 + 3, rl, S::BN) * 16) = u32x4{w[13], w[14], w[15], w[16]};
                sB[kb0 * S::BN + rl] = h2f(w[0] & 0xffffu);
                sB[(kb0 + 1) * S::BN + rl] = h2f(w[8] >> 16);
            }
        } else {
            const int i = tid + k * NTHREADS;
            if (i < S::BN) {
                const uint32_t* w = p.b[k];
                const float d = h2f(w[0] & 0xffffu), dmin = h2f(w[0] >> 16);
                const int half = (t0 >> 2) & 1;
#pragma unroll
                for (int jj = 0; jj < KS; jj++) {
                    const int j = half * 4 + jj;       // sub-block in the super-block
                    uint32_t sc, mn;
                    if (j < 4) {
                        sc = sbyte(w[1], w[2], w[3], j) & 63u;
                        mn = sbyte(w[1], w[2], w[3], j + 4) & 63u;
                    } else {
                        sc = (sbyte(w[1], w[2], w[3], j + 4) & 0xFu) | ((sbyte(w[1], w[2], w[3], j - 4) >> 6) << 4);
                        mn = (sbyte(w[1], w[2], w[3], j + 4) >> 4) | ((sbyte(w[1], w[2], w[3], j) >> 6) << 4);
                    }
                    sB[jj * S::BN + i] = d * (float)sc;
                    mB[jj * S::BN + i] = dmin * (float)mn;
                    // nibble group jj>>1 (32 bytes = 8 dwords), low nibbles for even jj
                    const uint32_t* g8 = w + 4 + (jj >> 1) * 8;
                    const int sh = (jj & 1) * 4;
                    u32x4 q0, q1;
                    q0.x = (g8[0] >> sh) & 0x0F0F0F0Fu; q0.y = (g8[1] >> sh) & 0x0F0F0F0Fu;
                    q0.z = (g8[2] >> sh) & 0x0F0F0F0Fu; q0.w = (g8[3] >> sh) & 0x0F0F0F0Fu;
                    q1.x = (g8[4] >> sh) & 0x0F0F0F0Fu; q1.y = (g8[5] >> sh) & 0x0F0F0F0Fu;
                    q1.z = (g8[6] >> sh) & 0x0F0F0F0Fu; q1.w = (g8[7] >> sh) & 0x0F0F0F0Fu;
                    *(u32x4*)(ldsB + swz_slot(jj * 2 + 0, i, S::BN) * 16) = q0;
                    *(u32x4*)(ldsB + swz_slot(jj * 2 + 1, i, S::BN) * 16) = q1;
                }
            }
        }
    }
}

}  // namespace

template <int WTYPE, int WM, int WN, bool DEBUG>
__global__ __launch_bounds__(NTHREADS) void k_gemm_q_i8(GemmArgs g) {
    using S = GemmI8Shape<WTYPE, WM, WN>;
    __shared__ __attribute__((aligned(16))) uint8_t ldsA[S::LDS_A];
    __shared__ __attribute__((aligned(16))) uint8_t ldsB[S::LDS_B];
    __shared__ __attribute__((aligned(16))) float sA[KS * S::BM];
    __shared__ __attribute__((aligned(16))) float uA[WTYPE == 12 ? KS * S::BM : 4];
    __shared__ __attribute__((aligned(16))) float sB[KS * S::BN];
    __shared__ __attribute__((aligned(16))) float mB[WTYPE == 12 ? KS * S::BN : 4];

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
    const int hl = lane >> 5;          // which 16-byte half of the block this lane feeds
    const int l32 = lane & 31;

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    Prefetch<WTYPE, WM, WN> pf;
    const int steps = (nb + KS - 1) / KS;
    load_step<WTYPE, WM, WN, !DEBUG>(pf, g, m0, n0, 0, nb);

    for (int s = 0; s < steps; s++) {
        const int t0 = s * KS;
        __syncthreads();
        store_step<WTYPE, WM, WN, !DEBUG>(pf, ldsA, ldsB, sA, uA, sB, mB, t0);
        __syncthreads();
        if (s + 1 < steps) load_step<WTYPE, WM, WN, !DEBUG>(pf, g, m0, n0, t0 + KS, nb);

#pragma unroll
        for (int kb = 0; kb < KS; kb++) {
            if (t0 + kb >= nb) break;
            i32x4 af[WM], bf[WN];
#pragma unroll
            for (int i = 0; i < WM; i++)
                af[i] = *(const i32x4*)(ldsA + swz_slot(kb * 2 + hl, wm0 + i * 32 + l32, S::BM) * 16);
#pragma unroll
            for (int j = 0; j < WN; j++)
                bf[j] = *(const i32x4*)(ldsB + swz_slot(kb * 2 + hl, wn0 + j * 32 + l32, S::BN) * 16);
            if (DEBUG) {
#pragma unroll
                for (int i = 0; i < WM; i++)
#pragma unroll
                    for (int j = 0; j < WN; j++) {
                        const i32x16 z = {};
                        const i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], z, 0, 0, 0);
                        const int n = n0 + wn0 + j * 32 + l32;
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
                            if (m < g.M && n < g.N)
                                g.dots[((size_t)m * g.N + n) * nb + t0 + kb] = I[r];
                        }
                    }
                continue;
            }
            // per-row activation scales of this lane's 16 rows, per-column weight scales
            f32x4 da[WM][4], ua[WM][4];
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int row = wm0 + i * 32 + 8 * q + 4 * hl;
                    da[i][q] = *(const f32x4*)(sA + kb * S::BM + row);
                    if (WTYPE == 12) ua[i][q] = *(const f32x4*)(uA + kb * S::BM + row);
                }
            float db[WN], mb[WN];
#pragma unroll
            for (int j = 0; j < WN; j++) {
                db[j] = sB[kb * S::BN + wn0 + j * 32 + l32];
                if (WTYPE == 12) mb[j] = mB[kb * S::BN + wn0 + j * 32 + l32];
            }
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++) {
                    const i32x16 z = {};
                    const i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float sc = da[i][r >> 2][r & 3] * db[j];
                        acc[i][j][r] = __builtin_fmaf(sc, (float)I[r], acc[i][j][r]);
                        if (WTYPE == 12) acc[i][j][r] = __builtin_fmaf(-mb[j], ua[i][r >> 2][r & 3], acc[i][j][r]);
                    }
                }
        }
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
                float v = acc[i][j][r] + bv;
                v = act_fn(v, g.act);
                const size_t idx = (size_t)m * g.N + n;
                if (g.resid) v += g.resid[idx];
                g.y[idx] = v;
            }
    }
}

template <int WTYPE, int WM, int WN>
static hipError_t launch_cfg(const GemmArgs& a, bool dbg, hipStream_t s) {
    using S = GemmI8Shape<WTYPE, WM, WN>;
    const int tiles = ((a.M + S::BM - 1) / S::BM) * ((a.N + S::BN - 1) / S::BN);
    if (dbg)
        hipLaunchKernelGGL((k_gemm_q_i8<WTYPE, WM, WN, true>), dim3(tiles), dim3(NTHREADS), 0, s, a);
    else
        hipLaunchKernelGGL((k_gemm_q_i8<WTYPE, WM, WN, false>), dim3(tiles), dim3(NTHREADS), 0, s, a);
    return hipGetLastError();
}

template <int WTYPE>
static hipError_t launch_type(const GemmArgs& a, TileCfg t, bool dbg, hipStream_t s) {
    if (t.wm == 2 && t.wn == 2) return launch_cfg<WTYPE, 2, 2>(a, dbg, s);
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
