// k_gemm_q_f16x.hip — production Q8_0 / Q4_K FC GEMM (int8-dot semantics) for K % 256 == 0.
//
// Semantics: the reference's int8-dot FC kernels k_mul_mat_q8_i8 / k_mul_mat_q4k_i8
// (src/mg-opencl/mg-opencl.cpp:440-494, :504-590): per 32-wide K block t
//   idot = sum_i qw[n,t,i] * qx[m,32t+i]                 (exact integer)
//   Q8_0: acc += (dx[m,t] * dw[n,t]) * idot
//   Q4_K: acc += (dx[m,t] * d*sc_j[n]) * idot - (dx[m,t]*sum_i qx[m,32t+i]) * dmin*m_j[n]
// then y = act(acc + bias[n]) + resid[m,n] (mg-opencl.cpp:485-491).
//
// gfx950 mapping (measured: this inner loop runs ~2x faster than int8 MFMA + VALU convert):
//  * Block dots on v_mfma_f32_16x16x32_f16: its K of 32 is one ggml block and its operands
//    are the int8 codes held as fp16 (exact for |q| <= 255). Every partial sum is an
//    integer below 2^24, so the fp32 result equals the int32 dot exactly — the dots stay
//    bit-exact, and no int->float convert is needed.
//  * Per-(n,m,block) scales from v_mfma_f32_16x16x1_4b_f32: four outer products dw (x) dx
//    (four K blocks) per 16x16 tile in one instruction, in the dot's register layout.
//  * VALU: one FMA per output and block. Q4_K's min term is a rank-4 update per step that
//    v_mfma_f32_16x16x4_f32 accumulates into its own accumulator.
//  * Weights play the MFMA "A" role, so each lane ends with 4 consecutive output columns
//    of one row: float4 epilogue loads/stores.
// Data movement:
//  * Activations arrive as fp16 codes (k_quantize_act_q8 with fp16 output) and are moved
//    with global_load_lds_dwordx4 (one 16-byte chunk per lane straight into LDS),
//    double-buffered; row units are XOR-permuted by (row & 7) so the coalesced fill and
//    the MFMA-order reads are both bank-conflict free.
//  * Raw GGUF weight rows (no repacking) are moved the same way — 144 bytes per row and
//    step: a 16-byte aligned window of Q8_0 blocks, or a Q4_K header plus half the nibbles —
//    and unpacked once per workgroup and step into fp16 codes plus block scales
//    (v_alignbyte for the 34-byte blocks, v_perm + packed fp16 add for int8/nibble -> fp16).
// Tile: 64 x 64 outputs per 256-thread workgroup (2x2 waves, each 32x32 = 2x2 MFMA tiles),
// K step 128 (4 blocks), ~60 KB LDS, two workgroups per CU.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int NT = 256;
constexpr int BM = 64, BN = 64;
constexpr int KB = 4;              // blocks per step
constexpr int UNITS = KB * 4;      // 16-byte units of fp16 codes per row and step

template <int WTYPE>
struct XLds {
    static constexpr bool Q4K = WTYPE == 12;
    static constexpr int RAW = Q4K ? 5 : 9;       // 16-byte chunks per weight row and step
    u32x4 a[2][BM * UNITS];                       // activation codes: unit u of row r at r*UNITS + (u ^ (r&7))
    float sa[2][KB * BM];                         // dx per (block, row)
    float ua[2][Q4K ? KB * BM : 1];               // dx * sum(qx)
    u32x4 raw[BN * RAW];                          // weight bytes as stored in the GGUF tensor
    u32x4 b[BN * UNITS];                          // weight codes, same layout as a
    float sb[KB * BN];                            // dw (Q8_0) or d*sc (Q4_K)
    float mb[Q4K ? KB * BN : 1];                  // dmin*m (Q4_K)
};

__device__ __forceinline__ int xslot(int r, int u) { return r * UNITS + (u ^ (r & 7)); }

__device__ __forceinline__ void dma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 16, 0, 0);
}

__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// four int8 (one dword) -> four fp16 codes (two dwords), exact:
// byte b -> fp16 bits 0x64 | (b ^ 0x80) = 1024 + (q + 128), then subtract 1152.
__device__ __forceinline__ uint2 i8x4_to_f16(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const f16x2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const f16x2 l = __builtin_bit_cast(f16x2, lo) + off;
    const f16x2 h = __builtin_bit_cast(f16x2, hi) + off;
    return uint2{__builtin_bit_cast(uint32_t, l), __builtin_bit_cast(uint32_t, h)};
}

// four unsigned bytes 0..15 -> four fp16 codes: 0x64 | b = 1024 + b, then subtract 1024.
__device__ __forceinline__ uint2 u4x4_to_f16(uint32_t w) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
    const f16x2 off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const f16x2 l = __builtin_bit_cast(f16x2, lo) + off;
    const f16x2 h = __builtin_bit_cast(f16x2, hi) + off;
    return uint2{__builtin_bit_cast(uint32_t, l), __builtin_bit_cast(uint32_t, h)};
}

template <int WTYPE>
__device__ __forceinline__ void issue_step(XLds<WTYPE>& L, int st, const GemmArgs& g, int m0,
                                           int n0, int t0, int nb, int wave, int lane) {
    using S = XLds<WTYPE>;
    const uint8_t* qx16 = (const uint8_t*)g.qx16;
#pragma unroll
    for (int k = 0; k < BM * UNITS / 64 / 4; k++) {          // 16 instructions, 4 per wave
        const int q = wave + 4 * k;
        const int slot = q * 64 + lane;
        const int r = slot / UNITS;
        const int u = (slot % UNITS) ^ (r & 7);
        const int m = min(m0 + r, g.M - 1);
        dma16(qx16 + ((size_t)m * g.K + (size_t)(t0 + (u >> 2)) * 32) * 2 + (u & 3) * 16,
              &L.a[st][q * 64]);
    }
    constexpr int RI = BN * S::RAW / 64;                      // 9 (Q8_0) or 5 (Q4_K)
#pragma unroll
    for (int k = 0; k < (RI + 3) / 4; k++) {
        const int q = wave + 4 * k;
        if (q < RI) {
            const int slot = q * 64 + lane;
            const int r = slot / S::RAW;
            const int c = slot - r * S::RAW;
            const int n = min(n0 + r, g.N - 1);
            const uint8_t* src;
            if (S::Q4K) {
                const uint8_t* sbp = g.w + ((size_t)n * (nb / 8) + t0 / 8) * 144;
                src = c == 0 ? sbp : sbp + 16 + ((t0 >> 2) & 1) * 64 + (c - 1) * 16;
            } else {
                // 16-byte aligned 144-byte window holding blocks t0..t0+3 of row n
                src = g.w + ((size_t)n * nb + t0) * 34 - ((t0 >> 2) & 1) * 8 + c * 16;
            }
            dma16(src, &L.raw[q * 64]);
        }
    }
}

template <int WTYPE>
__device__ __forceinline__ void load_scales(f32x4& dv, i32x4& sv, const GemmArgs& g, int m0,
                                            int t0, int nb, int tid) {
    if (tid < BM) {
        const size_t off = (size_t)min(m0 + tid, g.M - 1) * nb + t0;
        dv = *(const f32x4*)(g.dx + off);
        if (WTYPE == 12) sv = *(const i32x4*)(g.sx + off);
    }
}

template <int WTYPE>
__device__ __forceinline__ void store_scales(XLds<WTYPE>& L, int st, f32x4 dv, i32x4 sv, int tid) {
    if (tid < BM) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            L.sa[st][kb * BM + tid] = dv[kb];
            if (WTYPE == 12) L.ua[st][kb * BM + tid] = dv[kb] * (float)sv[kb];
        }
    }
}

__device__ __forceinline__ uint32_t byte_of(u32x4 v, int j) {
    return (v[j >> 2] >> (8 * (j & 3))) & 0xffu;
}

// raw weight rows of this step -> fp16 codes + scales. Item = (row r, block kb).
template <int WTYPE, bool SCALES>
__device__ __forceinline__ void unpack_step(XLds<WTYPE>& L, int t0, int tid) {
    const int r = tid >> 2, kb = tid & 3;
    uint32_t q[8];
    if (WTYPE == 8) {
        const int o = ((t0 >> 2) & 1) * 8;                     // window offset of block t0
        const int bs = o + 34 * kb;                             // block start within the window
        const uint32_t* w = (const uint32_t*)((const uint8_t*)L.raw + r * 144 + (bs & ~3));
        uint32_t d[9];
#pragma unroll
        for (int i = 0; i < 9; i++) d[i] = w[i];
        float scale;
        if ((kb & 1) == 0) {                                    // bs % 4 == 0: scale in bytes 0-1
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], 2);
            scale = h2f(d[0] & 0xffffu);
        } else {                                                // bs % 4 == 2: quants dword-aligned
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = d[i + 1];
            scale = h2f(d[0] >> 16);
        }
        if (SCALES) L.sb[kb * BN + r] = scale;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint2 c0 = i8x4_to_f16(q[2 * i]), c1 = i8x4_to_f16(q[2 * i + 1]);
            L.b[xslot(r, kb * 4 + i)] = u32x4{c0.x, c0.y, c1.x, c1.y};
        }
    } else {
        const u32x4* row = L.raw + r * 5;
        const u32x4 hdr = row[0];
        const u32x4 n0 = row[1 + 2 * (kb >> 1)], n1 = row[2 + 2 * (kb >> 1)];
        const int sh = (kb & 1) * 4;
        q[0] = (n0.x >> sh) & 0x0F0F0F0Fu; q[1] = (n0.y >> sh) & 0x0F0F0F0Fu;
        q[2] = (n0.z >> sh) & 0x0F0F0F0Fu; q[3] = (n0.w >> sh) & 0x0F0F0F0Fu;
        q[4] = (n1.x >> sh) & 0x0F0F0F0Fu; q[5] = (n1.y >> sh) & 0x0F0F0F0Fu;
        q[6] = (n1.z >> sh) & 0x0F0F0F0Fu; q[7] = (n1.w >> sh) & 0x0F0F0F0Fu;
        if (SCALES) {
            const int j = ((t0 >> 2) & 1) * 4 + kb;                   // sub-block in the super-block
            const u32x4 sc12 = u32x4{hdr.y, hdr.z, hdr.w, 0u};
            uint32_t sc, mn;
            if (j < 4) {
                sc = byte_of(sc12, j) & 63u;
                mn = byte_of(sc12, j + 4) & 63u;
            } else {
                sc = (byte_of(sc12, j + 4) & 0xFu) | ((byte_of(sc12, j - 4) >> 6) << 4);
                mn = (byte_of(sc12, j + 4) >> 4) | ((byte_of(sc12, j) >> 6) << 4);
            }
            L.sb[kb * BN + r] = h2f(hdr.x & 0xffffu) * (float)sc;
            L.mb[kb * BN + r] = h2f(hdr.x >> 16) * (float)mn;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint2 c0 = u4x4_to_f16(q[2 * i]), c1 = u4x4_to_f16(q[2 * i + 1]);
            L.b[xslot(r, kb * 4 + i)] = u32x4{c0.x, c0.y, c1.x, c1.y};
        }
    }
}

template <int ACT>
__device__ __forceinline__ float act_x(float v) {
    if (ACT == 1) return gelu_erf(v);
    if (ACT == 2) return v / (1.0f + expf(-v));
    return v;
}

}  // namespace

template <int WTYPE, int ACT, bool DEBUG>
__global__ __launch_bounds__(NT, 2) void k_gemm_q_f16x(GemmArgs g) {
    using S = XLds<WTYPE>;
    __shared__ S L;

    const int nb = g.K / 32;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_n * ((g.M + BM - 1) / BM);
    const int T = xcd_remap(blockIdx.x, tiles);
    const int m0 = (T / tiles_n) * BM;
    const int n0 = (T % tiles_n) * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wn0 = (wave & 1) * 32, wm0 = (wave >> 1) * 32;
    const int l16 = lane & 15, lq = lane >> 4;

    f32x4 acc[2][2], accm[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            accm[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    const int steps = nb / KB;
    f32x4 dv = {0.f, 0.f, 0.f, 0.f};
    i32x4 sv = {0, 0, 0, 0};
    issue_step<WTYPE>(L, 0, g, m0, n0, 0, nb, wave, lane);
    if (!DEBUG) load_scales<WTYPE>(dv, sv, g, m0, 0, nb, tid);

    for (int s = 0; s < steps; s++) {
        const int st = s & 1;
        const int t0 = s * KB;
        wait_vm0();
        if (!DEBUG) store_scales<WTYPE>(L, st, dv, sv, tid);
        __syncthreads();                        // activations, raw weights, scales of step s ready
        unpack_step<WTYPE, !DEBUG>(L, t0, tid);
        __syncthreads();                        // weight codes ready; raw buffer free
        if (s + 1 < steps) {
            issue_step<WTYPE>(L, st ^ 1, g, m0, n0, t0 + KB, nb, wave, lane);
            if (!DEBUG) load_scales<WTYPE>(dv, sv, g, m0, t0 + KB, nb, tid);
        }

        // fragments: weights (MFMA A, rows n) and activations (MFMA B, cols m), 4 blocks
        f16x8 wf[KB][2], xf[KB][2];
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int rn = wn0 + 16 * i + l16, rm = wm0 + 16 * i + l16;
                wf[kb][i] = __builtin_bit_cast(f16x8, L.b[xslot(rn, kb * 4 + lq)]);
                xf[kb][i] = __builtin_bit_cast(f16x8, L.a[st][xslot(rm, kb * 4 + lq)]);
            }
        if (DEBUG) {
#pragma unroll
            for (int tn = 0; tn < 2; tn++)
#pragma unroll
                for (int tm = 0; tm < 2; tm++)
#pragma unroll
                    for (int kb = 0; kb < KB; kb++) {
                        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                        const f32x4 F = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[kb][tn], xf[kb][tm], z, 0, 0, 0);
                        const int m = m0 + wm0 + 16 * tm + l16;
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int n = n0 + wn0 + 16 * tn + 4 * lq + r;
                            if (m < g.M && n < g.N) g.dots[((size_t)m * g.N + n) * nb + t0 + kb] = (int32_t)F[r];
                        }
                    }
            continue;
        }
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int rn = wn0 + 16 * tn + l16;
            const float sbv = L.sb[lq * BN + rn];
            const float mbv = S::Q4K ? -L.mb[lq * BN + rn] : 0.0f;
#pragma unroll
            for (int tm = 0; tm < 2; tm++) {
                const int rm = wm0 + 16 * tm + l16;
                const float sav = L.sa[st][lq * BM + rm];
                const f32x16 z16 = {};
                const f32x16 sc = __builtin_amdgcn_mfma_f32_16x16x1f32(sbv, sav, z16, 0, 0, 0);
                if (S::Q4K) {
                    const float uav = L.ua[st][lq * BM + rm];
                    accm[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(mbv, uav, accm[tn][tm], 0, 0, 0);
                }
#pragma unroll
                for (int kb = 0; kb < KB; kb++) {
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    const f32x4 F = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[kb][tn], xf[kb][tm], z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[tn][tm][r] = __builtin_fmaf(sc[4 * kb + r], F[r], acc[tn][tm][r]);
                }
            }
        }
    }
    if (DEBUG) return;

    // epilogue: lane holds y[m][n..n+3]; +bias -> act -> +resid (mg-opencl.cpp:485-491)
#pragma unroll
    for (int tn = 0; tn < 2; tn++) {
        const int n = n0 + wn0 + 16 * tn + 4 * lq;
        if (n >= g.N) continue;
        const f32x4 bv = g.bias ? *(const f32x4*)(g.bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tm = 0; tm < 2; tm++) {
            const int m = m0 + wm0 + 16 * tm + l16;
            if (m >= g.M) continue;
            const size_t idx = (size_t)m * g.N + n;
            f32x4 v = acc[tn][tm];
            if (S::Q4K) v += accm[tn][tm];
            v += bv;
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = act_x<ACT>(v[r]);
            if (g.resid) v += *(const f32x4*)(g.resid + idx);
            *(f32x4*)(g.y + idx) = v;
        }
    }
}

hipError_t launch_gemm_q_f16x(int wtype, const GemmArgs& a, bool dbg, hipStream_t s) {
    const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const dim3 grid(tiles), block(NT);
#define MGH_LAUNCH(WT)                                                                              \
    do {                                                                                            \
        if (dbg) hipLaunchKernelGGL((k_gemm_q_f16x<WT, 0, true>), grid, block, 0, s, a);            \
        else if (a.act == 1) hipLaunchKernelGGL((k_gemm_q_f16x<WT, 1, false>), grid, block, 0, s, a); \
        else if (a.act == 2) hipLaunchKernelGGL((k_gemm_q_f16x<WT, 2, false>), grid, block, 0, s, a); \
        else hipLaunchKernelGGL((k_gemm_q_f16x<WT, 0, false>), grid, block, 0, s, a);              \
    } while (0)
    if (wtype == 8) MGH_LAUNCH(8);
    else if (wtype == 12) MGH_LAUNCH(12);
    else return hipErrorInvalidValue;
#undef MGH_LAUNCH
    return hipGetLastError();
}

}  // namespace mgh
