// k_gemm_i8_stream.hip — streamed Q8_0 / Q4_K x int8-activation GEMM for K % 256 == 0.
//
// Same arithmetic as k_gemm_i8.hip (the reference's k_mul_mat_q8_i8 / k_mul_mat_q4k_i8,
// src/mg-opencl/mg-opencl.cpp:440-494 and :504-590): per 32-wide K block an exact int32 dot
// on v_mfma_i32_32x32x32_i8, the per-(m,n,block) scale dx*dw from
// v_mfma_f32_32x32x1_2b_f32 outer products, one cvt + one FMA per output and block on the
// VALU, and for Q4_K the min term accumulated by v_mfma_f32_32x32x2_f32.
//
// What differs is how operands reach LDS, built for HBM/L2 latency rather than ALU work:
//  * K steps are 256 wide (8 blocks), so one step of a weight row is 272 contiguous,
//    16-byte aligned bytes of Q8_0 blocks (17 chunks) or one 144-byte Q4_K super-block
//    (9 chunks), whenever K % 256 == 0.
//  * Activations and raw weight rows are fetched with global_load_lds_dwordx4: each lane
//    moves one 16-byte chunk straight into LDS, no VGPRs, 64 consecutive chunks per
//    instruction, consecutive lanes on consecutive bytes (fully coalesced). Activation rows
//    land with their 16 chunks XOR-permuted by (row & 7), which keeps the fill coalesced
//    and the MFMA-order reads bank-conflict free.
//  * After each step lands, the workgroup unpacks the raw weight rows once in LDS (Q8_0
//    block pairs realigned with v_alignbyte; Q4_K nibbles split, 6-bit scales/mins decoded)
//    into an int8 tile plus per-block scales; the four waves then read MFMA operands from it.
//  * Activation tiles and their scales are double-buffered: loads for step s+1 are issued
//    right after the unpack of step s and complete under the MFMAs of step s.
// Tile: 64 x 64 outputs per 256-thread workgroup (2x2 waves of one 32x32 tile each); about
// 71 KB of LDS, two workgroups per CU.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int NT = 256;
constexpr int BM = 64, BN = 64;
constexpr int KB = 8;                       // 32-blocks per step
constexpr int A_SLOTS = BM * 16;            // 16-byte chunks of a 64 x 256-byte activation tile

template <int WTYPE>
struct SLds {
    static constexpr bool Q4K = WTYPE == 12;
    static constexpr int RAW_CHUNKS = Q4K ? 9 : 17;     // 16-byte chunks per weight row and step
    u32x4 a[2][A_SLOTS];                    // activations, row-major, chunk j of row r at r*16 + (j ^ (r&7))
    float sa[2][KB * BM];                   // dx per (block, row)
    float ua[2][Q4K ? KB * BM : 1];         // dx * sum(qx) (Q4_K)
    u32x4 raw[BN * RAW_CHUNKS];             // weight rows as stored in the GGUF tensor
    u32x4 b[KB * 2 * BN];                   // unpacked int8 weights, piece j of row r at j*BN + (r ^ (j&7))
    float sb[KB * BN];                      // dw (Q8_0) or d*sc (Q4_K) per (block, row)
    float mb[Q4K ? KB * BN : 1];            // dmin*m (Q4_K)
};

__device__ __forceinline__ void dma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 16, 0, 0);
}

// vmcnt(0): every global load of this wave, including direct-to-LDS ones, has landed.
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <int WTYPE>
__device__ __forceinline__ void issue_step(SLds<WTYPE>& L, int stage, const GemmArgs& g,
                                           int m0, int n0, int t0, int nb, int wave, int lane) {
    using S = SLds<WTYPE>;
    // activations: 16 instructions of 64 chunks, wave w issues q = w, w+4, w+8, w+12
#pragma unroll
    for (int k = 0; k < A_SLOTS / 64 / 4; k++) {
        const int q = wave + 4 * k;
        const int slot = q * 64 + lane;
        const int r = slot >> 4;
        const int j = (slot & 15) ^ (r & 7);
        const int m = min(m0 + r, g.M - 1);
        dma16(g.qx + (size_t)m * g.K + (size_t)t0 * 32 + j * 16, &L.a[stage][q * 64]);
    }
    // raw weight rows
    constexpr int RAW_INSTR = BN * S::RAW_CHUNKS / 64;
#pragma unroll
    for (int k = 0; k < (RAW_INSTR + 3) / 4; k++) {
        const int q = wave + 4 * k;
        if (q < RAW_INSTR) {
            const int slot = q * 64 + lane;
            const int r = slot / S::RAW_CHUNKS;
            const int c = slot - r * S::RAW_CHUNKS;
            const int n = min(n0 + r, g.N - 1);
            const uint8_t* row = S::Q4K ? g.w + ((size_t)n * (nb / 8) + t0 / 8) * 144
                                        : g.w + ((size_t)n * nb + t0) * 34;
            dma16(row + c * 16, &L.raw[q * 64]);
        }
    }
}

template <int WTYPE>
__device__ __forceinline__ void load_scales(f32x4 (&dv)[2], i32x4 (&sv)[2], const GemmArgs& g,
                                            int m0, int t0, int nb, int tid) {
    if (tid < BM) {
        const size_t off = (size_t)min(m0 + tid, g.M - 1) * nb + t0;
        dv[0] = *(const f32x4*)(g.dx + off);
        dv[1] = *(const f32x4*)(g.dx + off + 4);
        if (WTYPE == 12) {
            sv[0] = *(const i32x4*)(g.sx + off);
            sv[1] = *(const i32x4*)(g.sx + off + 4);
        }
    }
}

template <int WTYPE>
__device__ __forceinline__ void store_scales(SLds<WTYPE>& L, int stage, const f32x4 (&dv)[2],
                                             const i32x4 (&sv)[2], int tid) {
    if (tid < BM) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const float d = dv[kb >> 2][kb & 3];
            L.sa[stage][kb * BM + tid] = d;
            if (WTYPE == 12) L.ua[stage][kb * BM + tid] = d * (float)sv[kb >> 2][kb & 3];
        }
    }
}

__device__ __forceinline__ uint32_t byte_of(u32x4 v, int j) {
    const uint32_t w = v[j >> 2];
    return (w >> (8 * (j & 3))) & 0xffu;
}

// Unpack the raw weight rows of the current step into the int8 tile and block scales.
template <int WTYPE>
__device__ __forceinline__ void unpack_step(SLds<WTYPE>& L, int tid) {
    const int r = tid >> 2, p = tid & 3;
    if (WTYPE == 8) {
        // item (row r, block pair p): raw bytes [68p, 68p+68) of the row's 272-byte slab
        const uint32_t* src = (const uint32_t*)((const uint8_t*)L.raw + r * 272 + 68 * p);
        uint32_t w[17];
#pragma unroll
        for (int i = 0; i < 17; i++) w[i] = src[i];
        u32x4 q0, q1;
        q0.x = __builtin_amdgcn_alignbyte(w[1], w[0], 2);
        q0.y = __builtin_amdgcn_alignbyte(w[2], w[1], 2);
        q0.z = __builtin_amdgcn_alignbyte(w[3], w[2], 2);
        q0.w = __builtin_amdgcn_alignbyte(w[4], w[3], 2);
        q1.x = __builtin_amdgcn_alignbyte(w[5], w[4], 2);
        q1.y = __builtin_amdgcn_alignbyte(w[6], w[5], 2);
        q1.z = __builtin_amdgcn_alignbyte(w[7], w[6], 2);
        q1.w = __builtin_amdgcn_alignbyte(w[8], w[7], 2);
        const int kb0 = 2 * p;
        L.b[swz_slot(kb0 * 2 + 0, r, BN)] = q0;
        L.b[swz_slot(kb0 * 2 + 1, r, BN)] = q1;
        L.b[swz_slot(kb0 * 2 + 2, r, BN)] = u32x4{w[9], w[10], w[11], w[12]};
        L.b[swz_slot(kb0 * 2 + 3, r, BN)] = u32x4{w[13], w[14], w[15], w[16]};
        L.sb[kb0 * BN + r] = h2f(w[0] & 0xffffu);
        L.sb[(kb0 + 1) * BN + r] = h2f(w[8] >> 16);
    } else {
        // item (row r, nibble group g = p): sub-blocks 2g (low nibbles) and 2g+1 (high)
        const u32x4* src = L.raw + r * 9;
        const u32x4 hdr = src[0];
        const u32x4 n0 = src[1 + 2 * p], n1 = src[2 + 2 * p];
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        const u32x4 sc12 = u32x4{hdr.y, hdr.z, hdr.w, 0u};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int j = 2 * p + h;                 // sub-block = block index within the step
            uint32_t sc, mn;
            if (j < 4) {
                sc = byte_of(sc12, j) & 63u;
                mn = byte_of(sc12, j + 4) & 63u;
            } else {
                sc = (byte_of(sc12, j + 4) & 0xFu) | ((byte_of(sc12, j - 4) >> 6) << 4);
                mn = (byte_of(sc12, j + 4) >> 4) | ((byte_of(sc12, j) >> 6) << 4);
            }
            L.sb[j * BN + r] = d * (float)sc;
            L.mb[j * BN + r] = dmin * (float)mn;
            const int sh = 4 * h;
            L.b[swz_slot(j * 2 + 0, r, BN)] = (n0 >> sh) & 0x0F0F0F0Fu;
            L.b[swz_slot(j * 2 + 1, r, BN)] = (n1 >> sh) & 0x0F0F0F0Fu;
        }
    }
}

template <int ACT>
__device__ __forceinline__ float act_s(float v) {
    if (ACT == 1) return gelu_erf(v);
    if (ACT == 2) return v / (1.0f + expf(-v));
    return v;
}

}  // namespace

template <int WTYPE, int ACT, bool DEBUG>
__global__ __launch_bounds__(NT, 2) void k_gemm_q_i8_s256(GemmArgs g) {
    using S = SLds<WTYPE>;
    __shared__ S L;

    const int nb = g.K / 32;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int tiles = tiles_n * ((g.M + BM - 1) / BM);
    const int T = xcd_remap(blockIdx.x, tiles);
    const int m0 = (T / tiles_n) * BM;
    const int n0 = (T % tiles_n) * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * 32, wn0 = (wave & 1) * 32;
    const int hl = lane >> 5, l32 = lane & 31;

    f32x16 acc, accm;
#pragma unroll
    for (int r = 0; r < 16; r++) { acc[r] = 0.0f; accm[r] = 0.0f; }

    const int steps = nb / KB;
    f32x4 dv[2];
    i32x4 sv[2];
    issue_step<WTYPE>(L, 0, g, m0, n0, 0, nb, wave, lane);
    if (!DEBUG) load_scales<WTYPE>(dv, sv, g, m0, 0, nb, tid);

    for (int s = 0; s < steps; s++) {
        const int st = s & 1;
        const int t0 = s * KB;
        wait_vm0();
        if (!DEBUG) store_scales<WTYPE>(L, st, dv, sv, tid);
        __syncthreads();                       // activations, raw weights, dx of step s ready
        unpack_step<WTYPE>(L, tid);
        __syncthreads();                       // unpacked weights ready; raw buffer free
        if (s + 1 < steps) {
            issue_step<WTYPE>(L, st ^ 1, g, m0, n0, t0 + KB, nb, wave, lane);
            if (!DEBUG) load_scales<WTYPE>(dv, sv, g, m0, t0 + KB, nb, tid);
        }

#pragma unroll
        for (int kp = 0; kp < KB / 2; kp++) {
            i32x4 af[2], bf[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int j = (2 * kp + h) * 2 + hl;
                const int ra = wm0 + l32;
                af[h] = (i32x4)L.a[st][ra * 16 + (j ^ (ra & 7))];
                bf[h] = (i32x4)L.b[swz_slot(j, wn0 + l32, BN)];
            }
            if (DEBUG) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const i32x16 z = {};
                    const i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[h], bf[h], z, 0, 0, 0);
                    const int n = n0 + wn0 + l32;
                    const int t = t0 + 2 * kp + h;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = m0 + wm0 + 8 * (r >> 2) + 4 * hl + (r & 3);
                        if (m < g.M && n < g.N) g.dots[((size_t)m * g.N + n) * nb + t] = I[r];
                    }
                }
                continue;
            }
            const int kbl = 2 * kp + hl;       // lane half hl carries block 2kp + hl
            const float sa = L.sa[st][kbl * BM + wm0 + l32];
            const float sb = L.sb[kbl * BN + wn0 + l32];
            const f32x32 z32 = {};
            const i32x16 z16 = {};
            const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sa, sb, z32, 0, 0, 0);
            const i32x16 I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0], bf[0], z16, 0, 0, 0);
            const i32x16 I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[1], bf[1], z16, 0, 0, 0);
            if (S::Q4K) {
                const float ua = L.ua[st][kbl * BM + wm0 + l32];
                const float mb = -L.mb[kbl * BN + wn0 + l32];
                accm = __builtin_amdgcn_mfma_f32_32x32x2f32(ua, mb, accm, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                acc[r] = __builtin_fmaf(sc[r], (float)I0[r], acc[r]);
                acc[r] = __builtin_fmaf(sc[16 + r], (float)I1[r], acc[r]);
            }
        }
    }
    if (DEBUG) return;

    // fused epilogue: +bias -> act -> +resid (mg-opencl.cpp:485-491)
    const int n = n0 + wn0 + l32;
    if (n >= g.N) return;
    const float bv = g.bias ? g.bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = m0 + wm0 + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (m >= g.M) continue;
        float v = acc[r];
        if (S::Q4K) v += accm[r];
        v = act_s<ACT>(v + bv);
        const size_t idx = (size_t)m * g.N + n;
        if (g.resid) v += g.resid[idx];
        g.y[idx] = v;
    }
}

hipError_t launch_gemm_q_i8_s256(int wtype, const GemmArgs& a, bool dbg, hipStream_t s) {
    const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const dim3 grid(tiles), block(NT);
#define MGH_LAUNCH(WT)                                                                           \
    do {                                                                                         \
        if (dbg) hipLaunchKernelGGL((k_gemm_q_i8_s256<WT, 0, true>), grid, block, 0, s, a);      \
        else if (a.act == 1) hipLaunchKernelGGL((k_gemm_q_i8_s256<WT, 1, false>), grid, block, 0, s, a); \
        else if (a.act == 2) hipLaunchKernelGGL((k_gemm_q_i8_s256<WT, 2, false>), grid, block, 0, s, a); \
        else hipLaunchKernelGGL((k_gemm_q_i8_s256<WT, 0, false>), grid, block, 0, s, a);         \
    } while (0)
    if (wtype == 8) MGH_LAUNCH(8);
    else if (wtype == 12) MGH_LAUNCH(12);
    else return hipErrorInvalidValue;
#undef MGH_LAUNCH
    return hipGetLastError();
}

}  // namespace mgh
