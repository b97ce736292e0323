// k_gemm_qp.hip — production Q8_0 / Q4_K FC GEMM on pre-packed weights (int8-dot semantics).
//
// Semantics: the reference's int8-dot FC kernels k_mul_mat_q8_i8 / k_mul_mat_q4k_i8
// (src/mg-opencl/mg-opencl.cpp:440-494, :504-590): per 32-wide K block t
//   idot = sum_i qw[n,t,i] * qx[m,32t+i]                         (exact integer)
//   Q8_0: acc += (dw[n,t] * dx[m,t]) * idot
//   Q4_K: acc += (scl[n,t] * dx[m,t]) * idot - (mnl[n,t] * dx[m,t]) * sx[m,t]
// then y = act(acc + bias[n]) + resid[m,n] (mg-opencl.cpp:485-491, :578-589).
//
// Operands (all produced on the device, no host repacking):
//  * weights in the packed layout of k_pack_w.hip: fp16 codes [N][K], fp32 scale [T][N]
//    (T = K/32), and for Q4_K fp32 min [N][T];
//  * activations from k_quantize_act_q8<fp16 codes>: fp16 codes [M][K], dx [M][T], and for
//    Q4_K the int32 block sums sx [M][T];
//  * or, for the dequantize-weights algorithm (the reference's fp16-slab path), from
//    k_round_act_f16: x rounded to fp16, unit dx, and fp32 block sums ux for Q4_K — the same
//    kernel then computes sum_t w_scale[n,t] * (sum_i q * x16) - mins[n,t] * ux[m,t].
//
// gfx950 mapping
//  * Block dots on v_mfma_f32_16x16x32_f16: its K of 32 is one ggml block; the operands are
//    integer codes held exactly in fp16, every partial sum is an integer below 2^24, so
//    the fp32 result is the exact int32 dot.
//  * Scales dw (x) dx from v_mfma_f32_16x16x1_4b_f32: four 16x16 outer products (the four
//    weight-row subtiles of a wave against one activation subtile) per instruction, in the
//    dot's register layout; one fp32 FMA per output and block applies them.
//  * Q4_K's min term sum_t mnl[n,t] * (dx*sx)[m,t] is a K/32-deep fp32 product computed
//    once per tile after the main loop: both factors split into bf16 hi+lo parts and
//    contracted on v_mfma_f32_16x16x32_bf16 (32 blocks per instruction, four cross terms,
//    relative error ~2^-15 of the term).
//  * Weights take the MFMA "A" role, so each lane ends with four consecutive output
//    columns of one row; the epilogue transposes the tile through LDS so it leaves as whole
//    512-byte rows with streaming (non-temporal) stores.
// Data movement: 128 weight rows x BM activation rows per 256-thread workgroup (2x2 waves,
// 64 x BM/2 outputs each), K stage of 64 (two blocks), double-buffered. Every operand —
// codes and scales — moves with global_load_lds (dwordx4 for codes, dword for scales)
// straight into LDS: each code instruction reads 8 whole 128-byte row segments (one cache
// line per 8 lanes), XOR-swizzled so the MFMA fragment reads are bank-conflict free; one
// barrier per stage. The loop body is software-pipelined (see the stage comment below).
#include <algorithm>

#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int NT = 256;
constexpr int BN = 128;            // weight rows (output columns) per workgroup
constexpr int KB = 2;              // blocks per stage
#ifndef MGH_QP_NS128
#define MGH_QP_NS128 3             // ring depth with 128-row activation tiles when every workgroup
#endif                             // has a CU (102 KB LDS, 1 per CU); 2 beyond (68 KB, 2 per CU)
#ifndef MGH_QP_SPLIT_TARGET
#define MGH_QP_SPLIT_TARGET 400    // split-K aims at about this many workgroups
#endif
#ifndef MGH_QP_NS64
#define MGH_QP_NS64 3              // ring depth with 64-row activation tiles (77 KB LDS, 2 per CU)
#endif

template <int BM, int NS>
struct PLds {
    u32x4 w[NS][KB * BN * 4];          // [stage][row][8 swizzled 16-byte chunks] fp16 codes
    u32x4 x[NS][KB * BM * 4];
    float sw[NS][KB * BN];             // [stage][kb][row] weight block scales
    float sx[NS][BM * KB];             // [stage][row][kb] activation block scales
    float pad[64];                     // sink of the scale DMA of waves with no scale rows
};

__device__ __forceinline__ void dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 4, 0, 0);
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt/lgkmcnt unconstrained)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int ACT>
__device__ __forceinline__ float act_x(float v) {
    if (ACT == 1) return gelu_erf(v);
    if (ACT == 2) return v / (1.0f + expf(-v));
    return v;
}

// fp32 -> (hi, lo) bf16 bit patterns (upper 16 bits), v = hi + lo + O(2^-16 |v|).
__device__ __forceinline__ void split_bf16(float v, uint32_t& hi, uint32_t& lo) {
    hi = __builtin_bit_cast(uint32_t, v) & 0xFFFF0000u;
    lo = __builtin_bit_cast(uint32_t, v - __builtin_bit_cast(float, hi)) & 0xFFFF0000u;
}

// eight fp32 -> bf16x8 hi and lo operands
__device__ __forceinline__ void split8(const float (&v)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
        uint32_t h0, l0, h1, l1;
        split_bf16(v[2 * e], h0, l0);
        split_bf16(v[2 * e + 1], h1, l1);
        hi[e] = (h0 >> 16) | h1;
        lo[e] = (l0 >> 16) | l1;
    }
}

// Logical tile -> (first activation row, first weight row): panels of 8 activation tiles,
// activation tile index fastest within a panel.
__device__ __forceinline__ void tile_origin(int lt, int tiles_m, int tiles_n, int bm, int& m0, int& n0) {
    const int panel = lt / (8 * tiles_n);
    const int pm = min(8, tiles_m - panel * 8);
    const int rem = lt - panel * 8 * tiles_n;
    m0 = (panel * 8 + rem % pm) * bm;
    n0 = (rem / pm) * BN;
}

}  // namespace

template <int WTYPE, int ACT, int BM, int NS, bool DEBUG>
__global__ __launch_bounds__(NT, 2) void k_gemm_qp(GemmArgs g) {
    constexpr int J = BM / 32;                   // 16-row activation subtiles per wave
    constexpr int CW = KB * (BN / 16) / 4;       // weight code chunks per wave and stage
    constexpr int CX = KB * (BM / 16) / 4;       // activation code chunks per wave and stage
    constexpr bool Q4K = WTYPE == 12;
    __shared__ PLds<BM, NS> L;

    const int K = g.K, T = K / 32, M = g.M, N = g.N;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    // tile order: XCD-contiguous ranges of logical tiles, walked in panels of 8 activation
    // tiles (activation tile index fastest), so an XCD's L2 holds a compact block of both
    // operands
    // split-K: the splits of one output tile are consecutive logical workgroups
    const int splits = max(g.splits, 1);
    const int lfull = xcd_remap(blockIdx.x, tiles_m * tiles_n * splits);
    const int lt = lfull / splits, ks = lfull - lt * splits;
    int m0, n0;
    tile_origin(lt, tiles_m, tiles_n, BM, m0, n0);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int l16 = lane & 15, lq = lane >> 4;

    const uint8_t* wcodes = g.w;
    const float* wscale = (const float*)(g.w + (size_t)2 * N * K);
    const uint8_t* xcodes = (const uint8_t*)g.qx16;

    // Stage layout of both code operands: row r's 128 bytes of the stage (blocks kb = 0, 1 =
    // eight 16-byte chunks) at LDS slots r*8 + (chunk ^ sw(r)), sw(r) = (r >> 1) & 7. One DMA
    // instruction moves 8 whole rows: lane l reads row 8c + (l >> 3), chunk (l & 7) ^ sw(row)
    // — a full 128-byte line per 8 lanes — and lands lane-linearly in the swizzled slot. An
    // MFMA fragment read (rows r0 + l16, chunk 4*kb + lq) covers the 16 bank groups once per
    // 16 lanes: slot mod 16 = 8*(r & 1) + (chunk ^ sw(r)) is distinct over 16 rows.
    // Rows are clamped in range; their outputs are masked.
    const uint8_t* srcw[CW];
    const uint8_t* srcx[CX];
#pragma unroll
    for (int q = 0; q < CW; q++) {
        const int c = wave + 4 * q;
        const int n = min(n0 + 8 * c + (lane >> 3), N - 1);
        srcw[q] = wcodes + (size_t)n * K * 2 + ((lane & 7) ^ ((4 * c + (lane >> 4)) & 7)) * 16;
    }
#pragma unroll
    for (int q = 0; q < CX; q++) {
        const int c = wave + 4 * q;
        const int m = min(m0 + 8 * c + (lane >> 3), M - 1);
        srcx[q] = xcodes + (size_t)m * K * 2 + ((lane & 7) ^ ((4 * c + (lane >> 4)) & 7)) * 16;
    }
    // weight scales, block-major [T][N]: wave w loads block kb = w >> 1 of rows 64*(w&1) + lane
    const float* srcsw = wscale + (size_t)(wave >> 1) * N + min(n0 + 64 * (wave & 1) + lane, N - 1);
    // activation scales: BM*KB floats, one dword DMA per wave; waves beyond that (BM = 64)
    // load a clamped copy into a pad so every wave issues the same instruction sequence
    const bool has_sx = 64 * wave < BM * KB;
    const float* srcsx = g.dx + (size_t)min(m0 + 32 * wave + (lane >> 1), M - 1) * T + (lane & 1);

    constexpr int NDMA = CW + CX + (DEBUG ? 0 : 2);   // DMA instructions per wave and stage
    auto dma_slot = [&](int d, int st, int s) {
        const size_t cofs = (size_t)s * KB * 64;          // bytes of fp16 codes per stage
        if (d < CW) {
            dma16(srcw[d] + cofs, &L.w[st][(wave + 4 * d) * 64]);
        } else if (d < CW + CX) {
            dma16(srcx[d - CW] + cofs, &L.x[st][(wave + 4 * (d - CW)) * 64]);
        } else if (d == CW + CX) {
            dma4(srcsw + (size_t)s * KB * N, &L.sw[st][64 * wave]);
        } else {
            dma4(srcsx + s * KB, has_sx ? &L.sx[st][64 * wave] : &L.pad[0]);
        }
    };

    f32x4 acc[4][J];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < J; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // NS-deep ring: stages s+1 .. s+NS-2 stay in flight while stage s is computed. Stages
    // past the end re-load the last one into the buffer just freed (never read), so every
    // iteration issues the same NDMA instructions and the vmcnt wait below is exact.
    const int S = T / KB;
    const int s_beg = (int)((int64_t)ks * S / splits), s_end = (int)((int64_t)(ks + 1) * S / splits);
#pragma unroll
    for (int k = 0; k < NS - 1; k++)
#pragma unroll
        for (int d = 0; d < NDMA; d++) dma_slot(d, k, min(s_beg + k, s_end - 1));
    int st = 0;                             // buffer of stage s
    int bn = NS - 1;                        // buffer receiving stage s + NS - 1
    for (int s = s_beg; s < s_end; s++) {
        const int sn = min(s + NS - 1, s_end - 1);
        // my loads of stage s have landed, then everyone's; and stage s-1 is consumed (the
        // debug variant's dot stores also count in vmcnt, so it waits for all)
        if (DEBUG) stage_sync<0>();
        else stage_sync<(NS - 2) * NDMA>();

        const u32x4* W = L.w[st];
        const u32x4* X = L.x[st];
        // MFMA operand: rows r0 + l16 (r0 % 16 == 0), block kb, K chunk lq
        auto frag = [&](const u32x4* B, int r0, int kb) {
            return __builtin_bit_cast(f16x8, B[(r0 + l16) * 8 + ((4 * kb + lq) ^ ((l16 >> 1) & 7))]);
        };
        if (DEBUG) {
#pragma unroll
            for (int d = 0; d < NDMA; d++) dma_slot(d, bn, sn);
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < J; j++) {
                        const f16x8 a = frag(W, 64 * wn + 16 * i, kb);
                        const f16x8 b = frag(X, (BM / 2) * wm + 16 * j, kb);
                        const f32x4 F = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        const int m = m0 + (BM / 2) * wm + 16 * j + l16;
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int n = n0 + 64 * wn + 16 * i + 4 * lq + r;
                            if (m < M && n < N) g.dots[((size_t)m * N + n) * T + s * KB + kb] = (int32_t)F[r];
                        }
                    }
            st = st + 1 == NS ? 0 : st + 1;
            bn = bn + 1 == NS ? 0 : bn + 1;
            continue;
        }

        // Software-pipelined stage: group g = (block kb, activation subtile j) issues the scale
        // outer product and the four block-dot MFMAs of g, then the 16 FMAs of group g-1 (whose
        // MFMAs have finished meanwhile), one or two of the next stage's DMA instructions and
        // the LDS fragment reads of block kb+1, interleaved so the MFMA pipe, the VALU and the
        // address unit stay busy together.
        constexpr int NG = KB * J;
        f32x2 dw2;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) dw2[kb] = L.sw[st][kb * BN + 64 * wn + lane];
        f32x2 dx2[J];
#pragma unroll
        for (int j = 0; j < J; j++) dx2[j] = *(const f32x2*)&L.sx[st][((BM / 2) * wm + 16 * j + l16) * KB];
        f16x8 a[KB][4], b[KB][J];
#pragma unroll
        for (int i = 0; i < 4; i++) a[0][i] = frag(W, 64 * wn + 16 * i, 0);
#pragma unroll
        for (int j = 0; j < J; j++) b[0][j] = frag(X, (BM / 2) * wm + 16 * j, 0);

        f32x16 scp = {};
        f32x4 Fp[4];
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int kb = g / J, j = g % J;
            const f32x16 sc = __builtin_amdgcn_mfma_f32_16x16x1f32(dw2[kb], dx2[j][kb], f32x16{}, 0, 0, 0);
            f32x4 F[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                F[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[kb][i], b[kb][j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            if (g > 0) {
                const int jp = (g - 1) % J;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][jp][r] = __builtin_fmaf(scp[4 * i + r], Fp[i][r], acc[i][jp][r]);
            }
            // fragments of the next block, spread over this block's groups
            if (kb + 1 < KB) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (i % J == j) a[kb + 1][i] = frag(W, 64 * wn + 16 * i, kb + 1);
                b[kb + 1][j] = frag(X, (BM / 2) * wm + 16 * j, kb + 1);
            }
#pragma unroll
            for (int d = 0; d < NDMA; d++)
                if (d % NG == g) dma_slot(d, bn, sn);
            // issue order: scale MFMA, then each dot MFMA followed by 4 FMAs
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
            scp = sc;
#pragma unroll
            for (int i = 0; i < 4; i++) Fp[i] = F[i];
        }
        {
            constexpr int jp = (NG - 1) % J;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[i][jp][r] = __builtin_fmaf(scp[4 * i + r], Fp[i][r], acc[i][jp][r]);
        }
        st = st + 1 == NS ? 0 : st + 1;
        bn = bn + 1 == NS ? 0 : bn + 1;
    }
    wait_vm0();                             // the re-loads past the end must land before exit
    if (DEBUG) return;

    if (Q4K && ks == 0) {               // linear: one split carries the whole min term
        // acc -= sum_t mnl[n,t] * (dx*sx)[m,t]: lane supplies blocks t = 32c + 8*lq + e
        const float* wmin = wscale + (size_t)N * T;
        for (int c = 0; c < T; c += 32) {
            const int t = c + 8 * lq;
            const bool in = t < T;                       // T % 8 == 0: a lane's 8 blocks are all in or out
            u32x4 ah[4], al[4], bh[J], bl[J];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = min(n0 + 64 * wn + 16 * i + l16, N - 1);
                float v[8];
                if (in) {
                    const f32x4 p0 = *(const f32x4*)(wmin + (size_t)n * T + t);
                    const f32x4 p1 = *(const f32x4*)(wmin + (size_t)n * T + t + 4);
#pragma unroll
                    for (int e = 0; e < 4; e++) { v[e] = -p0[e]; v[4 + e] = -p1[e]; }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = 0.f;
                }
                split8(v, ah[i], al[i]);
            }
#pragma unroll
            for (int j = 0; j < J; j++) {
                const int m = min(m0 + (BM / 2) * wm + 16 * j + l16, M - 1);
                float v[8];
                if (in && g.ux) {
                    const f32x4 u0 = *(const f32x4*)(g.ux + (size_t)m * T + t);
                    const f32x4 u1 = *(const f32x4*)(g.ux + (size_t)m * T + t + 4);
#pragma unroll
                    for (int e = 0; e < 4; e++) { v[e] = u0[e]; v[4 + e] = u1[e]; }
                } else if (in) {
                    const f32x4 d0 = *(const f32x4*)(g.dx + (size_t)m * T + t);
                    const f32x4 d1 = *(const f32x4*)(g.dx + (size_t)m * T + t + 4);
                    const i32x4 s0 = *(const i32x4*)(g.sx + (size_t)m * T + t);
                    const i32x4 s1 = *(const i32x4*)(g.sx + (size_t)m * T + t + 4);
#pragma unroll
                    for (int e = 0; e < 4; e++) { v[e] = d0[e] * (float)s0[e]; v[4 + e] = d1[e] * (float)s1[e]; }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = 0.f;
                }
                split8(v, bh[j], bl[j]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < J; j++) {
                    f32x4 a = acc[i][j];
                    a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al[i]), __builtin_bit_cast(bf16x8, bl[j]), a, 0, 0, 0);
                    a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al[i]), __builtin_bit_cast(bf16x8, bh[j]), a, 0, 0, 0);
                    a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[i]), __builtin_bit_cast(bf16x8, bl[j]), a, 0, 0, 0);
                    a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[i]), __builtin_bit_cast(bf16x8, bh[j]), a, 0, 0, 0);
                    acc[i][j] = a;
                }
        }
    }

    // epilogue: the tile leaves through LDS as whole rows (512 bytes per 32 lanes), in two
    // halves of BM/2 rows, with streaming stores; +bias -> act -> +resid (mg-opencl.cpp:485-491)
    // on the way out, or (split-K) the raw partial tile row-major into the workspace, summed in
    // split order by k_gemm_qp_reduce — a fixed order, so results are deterministic
    constexpr int P = BN + 4;                   // padded row pitch (floats)
    constexpr int HR = BM / 2;
    static_assert(HR * P * 4 <= (int)sizeof(PLds<BM, NS>), "transpose buffer fits the ring");
    float* Tt = (float*)&L;
    const int c = 4 * (tid & 31);               // this thread's 4 columns
    const int n = n0 + c;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (splits == 1 && g.bias && n < N) bv = *(const f32x4*)(g.bias + n);
    float* part = splits > 1 ? g.ws + ((size_t)lt * splits + ks) * (size_t)BM * BN : nullptr;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        // with 64-row tiles (the shapes that carry a residual) the half's residual loads go out
        // before the transpose, all at once (one HBM round trip per half, overlapped with the
        // LDS work); 128-row tiles load them in the store loop (no registers to spare)
        constexpr bool PRE = BM == 64;
        f32x4 rv[PRE ? HR / 8 : 1];
#pragma unroll
        for (int p = 0; p < (PRE ? HR / 8 : 0); p++) {
            const int m = m0 + HR * h + 8 * p + (tid >> 5);
            rv[p] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (splits == 1 && g.resid && m < M && n < N) rv[p] = *(const f32x4*)(g.resid + (size_t)m * N + n);
        }
        __syncthreads();                        // ring / previous half no longer read
        if (wm == h) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < J; j++)
                    *(f32x4*)&Tt[(16 * j + l16) * P + 64 * wn + 16 * i + 4 * lq] = acc[i][j];
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < HR / 8; p++) {
            const int r = 8 * p + (tid >> 5);
            const f32x4 v = *(const f32x4*)&Tt[r * P + c];
            if (splits > 1) {
                __builtin_nontemporal_store(v, (f32x4*)(part + (size_t)(HR * h + r) * BN + c));
                continue;
            }
            const int m = m0 + HR * h + r;
            if (m >= M || n >= N) continue;
            f32x4 o = v + bv;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = act_x<ACT>(o[e]);
            const size_t idx = (size_t)m * N + n;
            if (g.resid) o += PRE ? rv[PRE ? p : 0] : *(const f32x4*)(g.resid + idx);
            __builtin_nontemporal_store(o, (f32x4*)(g.y + idx));
        }
    }
}

// Split-K epilogue: one thread per output float4; sums the splits' row-major partial tiles in
// split order, then +bias -> act -> +resid.
template <int ACT, int BM>
__global__ __launch_bounds__(256) void k_gemm_qp_reduce(GemmArgs g) {
    const int M = g.M, N = g.N, splits = g.splits;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const size_t idx4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    constexpr int Q = BM * BN / 4;              // float4s per tile
    const int lt = (int)(idx4 / Q);
    if (lt >= tiles_m * tiles_n) return;
    const int q = (int)(idx4 - (size_t)lt * Q);
    const int r = q / (BN / 4), c = 4 * (q % (BN / 4));
    int m0, n0;
    tile_origin(lt, tiles_m, tiles_n, BM, m0, n0);
    const int m = m0 + r, n = n0 + c;
    if (m >= M || n >= N) return;
    const f32x4* part = (const f32x4*)(g.ws + (size_t)lt * splits * BM * BN) + q;
    const size_t o = (size_t)m * N + n;
    // the first KB partials, the bias and the residual are requested before any is summed (one
    // memory round trip, not one per split); the sum keeps split order
    constexpr int KB = 4;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 p[KB];
#pragma unroll
    for (int k = 0; k < KB; k++) p[k] = k < splits ? __builtin_nontemporal_load(part + (size_t)k * Q) : z;
    const f32x4 bv = g.bias ? *(const f32x4*)(g.bias + n) : z;
    const f32x4 rv = g.resid ? *(const f32x4*)(g.resid + o) : z;
    f32x4 v = p[0];
#pragma unroll
    for (int k = 1; k < KB; k++)
        if (k < splits) v += p[k];
    for (int k = KB; k < splits; k++) v += __builtin_nontemporal_load(part + (size_t)k * Q);
    if (g.bias) v += bv;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = act_x<ACT>(v[e]);
    if (g.resid) v += rv;
    __builtin_nontemporal_store(v, (f32x4*)(g.y + o));
}

int gemm_qp_bm(int M, int N) {
    // 128-row activation tiles unless that leaves most CUs without a workgroup
    const int t128 = ((M + 127) / 128) * ((N + BN - 1) / BN);
    return t128 >= 192 ? 128 : 64;
}

QpPlan gemm_qp_plan(int M, int N, int K) {
    QpPlan p{};
    p.bm = gemm_qp_bm(M, N);
    const int tiles = ((M + p.bm - 1) / p.bm) * ((N + BN - 1) / BN);
    const int S = K / (32 * KB);
    // A workgroup's time is about (its K stages) x (a stage's memory latency) when few tiles
    // run per CU, so shapes with fewer tiles than CUs split K into about
    // MGH_QP_SPLIT_TARGET / tiles parts of >= 8 stages (measured: splitting K = 768 loses,
    // K = 3072 gains 2.1x at M = 1025 and 1.3x at M = 4097).
    p.splits = 1;
    if (tiles < 256)
        p.splits = std::max(1, std::min((MGH_QP_SPLIT_TARGET + tiles / 2) / tiles, S / 8));
    p.ws_bytes = p.splits > 1 ? (size_t)tiles * p.splits * p.bm * BN * 4 : 0;
    return p;
}

template <int BMV, int NSV>
hipError_t launch_gemm_qp_t(int wtype, const GemmArgs& a, bool dbg, hipStream_t s) {
    const int tiles = ((a.M + BMV - 1) / BMV) * ((a.N + BN - 1) / BN) * (dbg ? 1 : std::max(a.splits, 1));
    const dim3 grid(tiles), block(NT);
    GemmArgs b = a;
    if (dbg) b.splits = 1;
#define MGH_LAUNCH(WT)                                                                                 \
    do {                                                                                               \
        if (dbg) hipLaunchKernelGGL((k_gemm_qp<WT, 0, BMV, NSV, true>), grid, block, 0, s, b);         \
        else if (b.act == 1) hipLaunchKernelGGL((k_gemm_qp<WT, 1, BMV, NSV, false>), grid, block, 0, s, b); \
        else if (b.act == 2) hipLaunchKernelGGL((k_gemm_qp<WT, 2, BMV, NSV, false>), grid, block, 0, s, b); \
        else hipLaunchKernelGGL((k_gemm_qp<WT, 0, BMV, NSV, false>), grid, block, 0, s, b);           \
    } while (0)
    if (wtype == 8) MGH_LAUNCH(8);
    else if (wtype == 12) MGH_LAUNCH(12);
    else return hipErrorInvalidValue;
#undef MGH_LAUNCH
    if (!dbg && b.splits > 1) {
        const int rt = ((b.M + BMV - 1) / BMV) * ((b.N + BN - 1) / BN);
        const dim3 rgrid((unsigned)(((size_t)rt * 4 * (BMV / 32) * NT + 255) / 256));
        if (b.act == 1) hipLaunchKernelGGL((k_gemm_qp_reduce<1, BMV>), rgrid, dim3(256), 0, s, b);
        else if (b.act == 2) hipLaunchKernelGGL((k_gemm_qp_reduce<2, BMV>), rgrid, dim3(256), 0, s, b);
        else hipLaunchKernelGGL((k_gemm_qp_reduce<0, BMV>), rgrid, dim3(256), 0, s, b);
    }
    return hipGetLastError();
}

// a.splits > 1 needs a.ws sized by gemm_qp_plan (the caller's plan for this shape).
hipError_t launch_gemm_qp(int wtype, const GemmArgs& a, bool dbg, hipStream_t s) {
    if (gemm_qp_bm(a.M, a.N) == 128) {
        // the 3-deep ring halves the workgroups per CU: only where they all run at once
        // (cfg2 up-proj, 216 tiles: 24.2 -> 21.1 us; at M = 4112 it slowed the int8 forward)
        const int wgs = ((a.M + 127) / 128) * ((a.N + BN - 1) / BN) * (dbg ? 1 : std::max(a.splits, 1));
        if (wgs <= 256) return launch_gemm_qp_t<128, MGH_QP_NS128>(wtype, a, dbg, s);
        return launch_gemm_qp_t<128, 2>(wtype, a, dbg, s);
    }
    return launch_gemm_qp_t<64, MGH_QP_NS64>(wtype, a, dbg, s);
}

}  // namespace mgh
