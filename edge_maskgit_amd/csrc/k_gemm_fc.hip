// k_gemm_fc.hip — the dequantize-fused FC path: y = act(x . w^T + bias) + resid with fp16
// operands on MFMA and fp32 accumulation, the weights in one of three forms (template WQ):
//   WQ 8 / 12: the Q8_0 / Q4_K bytes themselves, read on every call and decoded to fp16 in
//              registers as the MFMA fragments are read (the layout of launch_pack_weights_dq:
//              the GGUF blocks regrouped once into 16-row groups of 64-deep K stages, in MFMA
//              fragment order, at the GGUF byte count);
//   WQ 0:      an fp16 copy [N][K] made once at upload (launch_pack_weights_f16), 2 bytes per
//              weight, no decoding in the K loop.
// Both decode each weight to the same fp16 value, so the two forms give identical outputs for
// the same tile plan.
//
// Semantics: the reference's fp16-slab dequant GEMMs k_mul_mat_q8_0_t2_h / k_mul_mat_q4k_t2_h
// (src/mg-opencl/mg-opencl.cpp:320-411), which decode every weight inside the K loop (DEQ_Q8
// :386-387, deq_q4k_elem :252-262):
//   Q8_0: w = d * q            Q4_K: w = (d * sc) * q - dmin * m      (fp32, then to fp16)
// and the activations are rounded to fp16 (vstore_half_rte); the products accumulate in fp32,
// then y = act(acc + bias) + resid (mg-opencl.cpp:485-491). The outputs stay within 1e-3 of
// max|y| of the dequantize-then-F32 product (mg-cpu.cpp:48-72); the only rounding is the
// fp16 storage of the two operands and the fp32 summation.
//
// gfx950 mapping
//  * y tile BN (128 or 64) weight rows x BM (128, 64 or 32) activation rows per 256-thread
//    workgroup (2 x 2 waves, each BN/2 x BM/2 outputs as v_mfma_f32_16x16x32_f16 tiles); K
//    stage 64. gemm_h16_plan picks the tile, the ring depth and the K split per shape.
//  * Operands move with buffer loads into LDS (16 bytes per lane; 4 for the Q8_0 scales and
//    the Q4_K headers) straight into a 2- or 3-deep LDS ring: one instruction moves whole
//    128-byte row segments (fp16 weights, activations: XOR-swizzled so the MFMA fragment reads
//    are bank-conflict free) or whole 16-row groups of quantized weights (already in fragment
//    order). Resource and stage offset are scalar, the lane offset loop-invariant, and the
//    ring slot of each unrolled stage a constant: the K loop's vector instructions are the
//    MFMAs, the decoding and the fp32 -> fp16 rounding, nothing for addresses (every vector
//    instruction per stage and wave adds to the kernel time: the decoding leaves the VALU
//    busier than the matrix pipe). The stage hand-over is an explicit vmcnt/lgkmcnt wait and
//    s_barrier (stage_sync), which keeps the prefetched stages in flight.
//  * Software pipeline: the fragments of the next K half are read from LDS (and decoded) while
//    the current half's MFMAs issue; the stage boundary (vmcnt wait, barrier, next DMA, first
//    fragment reads of the new stage) sits between two halves of the second K half's MFMAs, so
//    the MFMA pipe keeps work while the wave waits.
//  * K rotation: output tiles that share operand rows start their K loop at different stages,
//    so the first touch of each K slice (an L2 miss) is spread over the kernel instead of
//    being paid by every tile in the same step.
//  * Epilogue through LDS: the accumulator tile is transposed in two halves and leaves as whole
//    rows (512 bytes per 32 lanes) with streaming (non-temporal) stores; bias, activation and
//    residual are applied on the way out. With y16 the result is stored rounded to fp16 (the
//    operand form of a following dequantize-fused FC, which would round it to fp16 anyway).
//  * Split-K for shapes with too few tiles: each split writes its partial tile row-major into a
//    workspace (same transposed path) and k_gemm_fc_reduce sums the splits in split order
//    (deterministic) and applies the epilogue.
#include <algorithm>

#include <atomic>
#include <cstdio>
#include <cstdlib>

#include "mgh_common.h"
#include "mgh_kernels.h"
#include "k_ln_row.h"

namespace mgh {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
// 8-byte LDS / global reads go through this vector type: reading the ring through HIP's uint2
// struct made the compiler wait for every outstanding LDS DMA before the read (vmcnt(0)).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// fp32 pairs -> fp16, round to nearest even: gfx950's v_cvt_pk_f16_f32, one instruction per
// pair (a scalar cast per value costs a conversion plus a pack)
__device__ __forceinline__ h16x2 cvt2_f16(float a, float b) { return __builtin_convertvector(f32x2{a, b}, h16x2); }
__device__ __forceinline__ f16x4 cvt4_f16(f32x4 a) {
    const h16x2 p0 = cvt2_f16(a[0], a[1]), p1 = cvt2_f16(a[2], a[3]);
    return f16x4{p0[0], p0[1], p1[0], p1[1]};
}
__device__ __forceinline__ f16x8 cvt8_f16(f32x4 a, f32x4 b) {
    const h16x2 p0 = cvt2_f16(a[0], a[1]), p1 = cvt2_f16(a[2], a[3]);
    const h16x2 p2 = cvt2_f16(b[0], b[1]), p3 = cvt2_f16(b[2], b[3]);
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Stage geometry: a stage is 64 K values; one row's stage segment is CPR 16-byte chunks (fp16
// rows: 8, fp32 rows: 16), whole 128-byte lines. Chunk j of row r sits in slot j ^ swz(r): a
// fragment read (16 consecutive rows, one chunk) then touches 16 distinct 16-byte bank groups
// of the 256-byte bank row, and one DMA instruction (64 lanes x 16 bytes) fills 64 / CPR whole
// row segments. (32-deep stages with a deeper ring measured slower on every FC shape: their
// fp16 row segments are half lines, and the stage boundaries double.)
template <bool F32>
constexpr int kCpr = F32 ? 16 : 8;
template <int CPR>
__device__ __forceinline__ int swz(int r) { return (r / (16 / CPR)) & (CPR - 1); }

// Weight bytes per K stage (64 values) for BN rows, and the per-stage side data the K-loop
// dequantization needs (Q8_0: fp16 block scales; Q4_K: the super-block headers).
template <int WQ, int BN>
constexpr int kWStage = WQ == 0 ? BN * 128 : (WQ == 8 ? BN * 64 : BN * 32);
template <int WQ, int BN>
constexpr int kWAux = WQ == 0 ? 0 : (WQ == 8 ? 1024 : BN * 16);

// NS-deep ring of K stages. Weights: fp16 [stage][row][swizzled 16-byte chunks] (WQ 0), or the
// stage's 16-row groups of the K-loop-dequant layout as stored (1 KB of Q8_0 codes, 512 bytes
// of Q4_K nibbles per group) plus their scales / headers in `aux` (Q8_0: 256 bytes per wave,
// of which its groups' 64-byte scale rows fill the first GPW * 64; Q4_K: the 256-byte headers
// of the tile's groups in order).
template <int BM, int BN, bool XF32, int NS, int WQ>
struct HLds {
    u32x4 w[NS][kWStage<WQ, BN> / 16];
    u32x4 aux[NS][WQ ? kWAux<WQ, BN> / 16 : 1];
    u32x4 x[NS][BM * kCpr<XF32>];
};

// Raw buffer resource over [base, base + bytes) (extent capped at 4 GB): loads past the extent
// return zeros instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
    const int n = bytes >= 0xFFFFFFFFull ? -1 : (int)(uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
// DMA of 16 (4) bytes per lane from resource offset voff + soff into LDS at lds + 16 (4) * lane.
// The resource and soff live in SGPRs and voff is loop-invariant, so a DMA in the K loop costs
// no vector instruction (a global_load_lds takes a 64-bit per-lane address, one 64-bit add per
// DMA and stage).
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ void bdma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 4, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int ACT>
__device__ __forceinline__ float act_h(float v) {
    if (ACT == 1) return gelu_erf(v);
    if (ACT == 2) return v / (1.0f + expf(-v));
    return v;
}

// Logical tile lt -> origin: panels of PH activation-row tiles spanning all weight-row tiles,
// activation rows fastest inside a panel.
__device__ __forceinline__ void tile_origin(int lt, int tiles_m, int tiles_n, int bm, int bn, int ph,
                                            int& m0, int& n0) {
    const int panel = lt / (ph * tiles_n);
    const int pm = min(ph, tiles_m - panel * ph);
    const int rem = lt - panel * ph * tiles_n;
    m0 = (panel * ph + rem % pm) * bm;
    n0 = (rem / pm) * bn;
}

__device__ __forceinline__ uint32_t f16_bits(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

// Q8_0 fragment: eight codes stored as q + 128 (bytes of c.x, c.y in K order) and the block's
// fp16 scale d -> d * q rounded to fp16. Each code byte b becomes the fp16 1024 + b (exponent
// byte 0x64 placed above it by v_perm), minus 1152 gives q exactly, and the fp16 product
// rounds d * q (exact in fp32) once to nearest even: the value k_pack_w16 stores.
__device__ __forceinline__ f16x8 deq_q8(u32x2 c, uint32_t dbits) {
    const uint32_t E = 0x64646464u;
    const h16x2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)dbits);
    const h16x2 dd = {d, d};
    auto pair = [&](uint32_t w, uint32_t sel) {
        return (__builtin_bit_cast(h16x2, __builtin_amdgcn_perm(E, w, sel)) + off) * dd;
    };
    const h16x2 p0 = pair(c.x, 0x04010400u), p1 = pair(c.x, 0x04030402u);
    const h16x2 p2 = pair(c.y, 0x04010400u), p3 = pair(c.y, 0x04030402u);
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Q4_K fragment: eight 4-bit values (byte e of c: element e in the low nibble, element e + 4
// in the high one) of a sub-block with scale s = d * sc and offset m = dmin * mn -> s * q - m
// rounded to fp16. s and s * q are exact in fp32, so the fma rounds once, as the
// multiply-then-subtract of k_pack_w16; then one rounding to fp16.
__device__ __forceinline__ f16x8 deq_q4v(uint32_t c, float s, float m) {
    uint32_t lo = c & 0x0F0F0F0Fu, hn = (c >> 4) & 0x0F0F0F0Fu;
    // (the empty asm keeps the masks apart from the byte conversions below: folded into them,
    // every byte became a 4-bit extract plus a convert instead of one v_cvt_f32_ubyteN)
    asm volatile("" : "+v"(lo), "+v"(hn));
    f32x4 a, b;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        a[e] = __builtin_fmaf(s, (float)((lo >> (8 * e)) & 0xFFu), -m);
        b[e] = __builtin_fmaf(s, (float)((hn >> (8 * e)) & 0xFFu), -m);
    }
    return cvt8_f16(a, b);
}

// (d * sc, dmin * mn) of the sub-blocks j0 = 2 (t % 4) and j0 + 1 of the super-block with header
// h (fp16 d | fp16 dmin, then the 12 bytes of packed 6-bit scales / mins) that 64-value K stage
// t covers (get_scale_min_k4: j < 4 takes the 6 low bits of scales[j] / scales[j + 4]; j >= 4
// the low / high nibble of scales[j + 4] plus the top 2 bits of scales[j - 4] / scales[j]).
// The two sub-blocks lie on the same side of 4, so one set of masks (uniform) decodes both,
// four bytes at a time.
__device__ __forceinline__ void q4_scales(u32x4 h, int t, float& s0, float& m0, float& s1, float& m1) {
    const bool first = (t & 2) == 0;
    const int sh = 16 * (t & 1);                // byte of sub-block j0 in its dword
    const uint32_t lo6 = first ? 0x3F3F3F3Fu : 0u, lo4 = first ? 0u : 0x0F0F0F0Fu, hi2 = first ? 0u : 0x30303030u;
    const uint32_t sc = (h.y & lo6) | (h.w & lo4) | ((h.y >> 2) & hi2);
    const uint32_t mn = (h.z & lo6) | ((h.w >> 4) & lo4) | ((h.z >> 2) & hi2);
    const float d = h2f(h.x & 0xFFFFu), dm = h2f(h.x >> 16);
    s0 = d * (float)((sc >> sh) & 0xFFu);
    s1 = d * (float)((sc >> (sh + 8)) & 0xFFu);
    m0 = dm * (float)((mn >> sh) & 0xFFu);
    m1 = dm * (float)((mn >> (sh + 8)) & 0xFFu);
}

// One sub-block j of a Q4_K super-block (the skinny-M kernel's form)
__device__ __forceinline__ f16x8 deq_q4(uint32_t c, u32x4 h, int j) {
    float s0, m0, s1, m1;
    q4_scales(h, j >> 1, s0, m0, s1, m1);
    return (j & 1) ? deq_q4v(c, s1, m1) : deq_q4v(c, s0, m0);
}

// K-loop-dequant layout (packed_weight_bytes_dq): one thread per 32-value block (row n, block t
// = 2 * stage + half) writes its codes / nibbles to their fragment slots and its scale / header.
template <int WTYPE>
__global__ __launch_bounds__(256) void k_pack_wdq(const uint8_t* __restrict__ w, uint8_t* __restrict__ out,
                                                  int N, int K) {
    const int T = K / 32, S = K / 64;
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (int64_t)N * T) return;
    const int64_t n = blk / T;
    const int t = (int)(blk - n * T);
    const int64_t G = ((int64_t)N + 15) / 16, g = n / 16;
    const int r = (int)(n % 16), st = t / 2, h = t % 2;
    if (WTYPE == 8) {
        const uint8_t* b = w + blk * 34;
        uint8_t* cb = out + (g * S + st) * 1024 + 512 * h + 8 * r;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t v0 = 0, v1 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v0 |= (uint32_t)(uint8_t)(b[2 + 8 * q + e] ^ 0x80u) << (8 * e);
                v1 |= (uint32_t)(uint8_t)(b[2 + 8 * q + 4 + e] ^ 0x80u) << (8 * e);
            }
            *(uint2*)(cb + 128 * q) = uint2{v0, v1};
        }
        uint16_t* sc = (uint16_t*)(out + G * S * 1024);
        sc[(g * S + st) * 32 + 16 * h + r] = (uint16_t)(b[0] | (b[1] << 8));
    } else {
        const int sbi = t / 8, j = t % 8;
        const uint8_t* sb = w + (n * (T / 8) + sbi) * 144;
        const uint8_t* qs = sb + 16 + 32 * (j >> 1);
        const int sh = 4 * (j & 1);
        uint8_t* cb = out + (g * S + st) * 512 + 256 * h + 4 * r;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t lo = (qs[8 * q + e] >> sh) & 15u, hi = (qs[8 * q + 4 + e] >> sh) & 15u;
                v |= (lo | (hi << 4)) << (8 * e);
            }
            *(uint32_t*)(cb + 64 * q) = v;
        }
        if (j == 0) {
            const uint32_t* src = (const uint32_t*)sb;
            u32x4* hd = (u32x4*)(out + G * S * 512);
            hd[(g * (K / 256) + sbi) * 16 + r] = u32x4{src[0], src[1], src[2], src[3]};
        }
    }
}

// The 32 values of block t of weight row n as the reference decodes them (fp32): Q8_0
// d * q (DEQ_Q8, mg-opencl.cpp:386-387), Q4_K (d * sc) * q - dmin * m (deq_q4k_elem, :252-262;
// the 6-bit scale / min unpacking of get_scale_min_k4, :178-184). Bytes are read one at a
// time: Q8_0 rows need not be aligned at all.
template <int WTYPE>
__device__ __forceinline__ void decode_block(const uint8_t* __restrict__ w, int64_t n, int t, int T, float (&v)[32]) {
#pragma clang fp contract(off)
    const int64_t blk = n * T + t;
    if (WTYPE == 8) {
        const uint8_t* b = w + blk * 34;
        const float d = h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = d * (float)(int8_t)b[2 + i];
    } else {
        const uint8_t* sb = w + (n * (T / 8) + t / 8) * 144;
        const int j = t & 7;
        const uint8_t* sc12 = sb + 4;
        uint32_t sc, mn;
        if (j < 4) {
            sc = sc12[j] & 63u;
            mn = sc12[j + 4] & 63u;
        } else {
            sc = (sc12[j + 4] & 0xFu) | ((uint32_t)(sc12[j - 4] >> 6) << 4);
            mn = (uint32_t)(sc12[j + 4] >> 4) | ((uint32_t)(sc12[j] >> 6) << 4);
        }
        const float d = h2f((uint32_t)sb[0] | ((uint32_t)sb[1] << 8));
        const float dmin = h2f((uint32_t)sb[2] | ((uint32_t)sb[3] << 8));
        const float s = d * (float)sc, m = dmin * (float)mn;
        const uint8_t* qs = sb + 16 + 32 * (j >> 1);
        const int sh = 4 * (j & 1);
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = s * (float)((qs[i] >> sh) & 15) - m;
    }
}

// One thread per 32-value block: the block's 32 dequantized values as fp16 (4 x 16 bytes).
template <int WTYPE>
__global__ __launch_bounds__(256) void k_pack_w16(const uint8_t* __restrict__ w, u32x4* __restrict__ out,
                                                  int N, int K) {
    const int T = K / 32;
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (int64_t)N * T) return;
    const int64_t n = blk / T;
    const int t = (int)(blk - n * T);
    float v[32];
    decode_block<WTYPE>(w, n, t, T, v);
    u32x4* dst = out + blk * 4;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        u32x4 c;
#pragma unroll
        for (int e = 0; e < 4; e++) c[e] = f16_bits(v[8 * q + 2 * e]) | (f16_bits(v[8 * q + 2 * e + 1]) << 16);
        dst[q] = c;
    }
}

// One thread per 32-value block: the block's dequantized values as fp32, row-major [N][K] (any
// N; the weight of a MulMat whose shape the tiled kernels do not take)
template <int WTYPE>
__global__ __launch_bounds__(256) void k_dequant_w32(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                     int N, int K) {
    const int T = K / 32;
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (int64_t)N * T) return;
    const int64_t n = blk / T;
    const int t = (int)(blk - n * T);
    float v[32];
    decode_block<WTYPE>(w, n, t, T, v);
    float* dst = out + n * K + t * 32;
#pragma unroll
    for (int i = 0; i < 32; i++) dst[i] = v[i];
}

// fp32 -> fp16 (round to nearest even), 8 values per thread
__global__ __launch_bounds__(256) void k_f32_to_f16(const f32x4* __restrict__ x, u32x4* __restrict__ h,
                                                    int64_t n8) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    h[i] = __builtin_bit_cast(u32x4, cvt8_f16(x[2 * i], x[2 * i + 1]));
}

}  // namespace

// y[M][N] = act(x16[M][K] . w16[N][K]^T + bias) + resid, or (PART) the raw partial tile of
// split ks over its K range into ws. XF32: the activations arrive as fp32 (g.xf) and are
// rounded to fp16 (nearest even, as k_f32_to_f16) when the MFMA fragments are read from LDS.
// Tile BN weight rows x BM activation rows on 2 x WMR waves, each BN/2 weight rows x BM/WMR
// activation rows; K stages of 64 values in an NS-deep ring.
template <int WMR, int BN>
constexpr int kH16MinBlocks = (WMR == 2 && BN == 128) ? 2 : 1;

template <int ACT, int BM, bool PART, bool XF32, int NS, int WMR, int BN, int WQ>
__global__ __launch_bounds__(128 * WMR, (kH16MinBlocks<WMR, BN>)) void k_gemm_fc(GemmH16Args g) {
    constexpr int NW = 2 * WMR;                 // waves
    constexpr int NTH = 64 * NW;                // threads
    constexpr int RW = BM / WMR;                // activation rows per wave
    constexpr int J = RW / 16;                  // 16-row activation subtiles per wave
    constexpr int WN = BN / 2;                  // weight rows per wave
    constexpr int I = WN / 16;                  // 16-row weight subtiles per wave
    constexpr int CPW = kCpr<false>, CPX = kCpr<XF32>;  // chunks per stage row
    constexpr int GPW = BN / 16 / NW;           // 16-row weight groups per wave (dequant layout)
    // weight DMA instructions per wave and stage (every lane of every DMA moves bytes: an
    // exec-masked DMA would make the compiler wait for all of them before any LDS read):
    // fp16 rows; one 16-byte-per-lane DMA per 1 KB Q8_0 group; Q4_K: two 512-byte groups per
    // 16-byte DMA, or a single group as two 4-byte-per-lane DMAs
    constexpr int CW = WQ == 0 ? BN * CPW / 64 / NW : (WQ == 8 ? GPW : (GPW >= 2 ? GPW / 2 : 2));
    // scale / header DMAs (4 bytes per lane): Q8_0 one (the wave's scale rows, then padding),
    // Q4_K one per 256-byte header group
    constexpr int CA = WQ == 0 ? 0 : (WQ == 8 ? 1 : GPW);
    static_assert(WQ == 0 || (BN % (16 * NW) == 0 && GPW <= 4 && (WQ == 8 || GPW == 1 || GPW % 2 == 0)),
                  "dequant layout: whole groups per wave");
    constexpr int CX = BM * CPX / 64 / NW;      // activation DMA instructions per wave and stage
    static_assert(CW >= 1 && CX >= 1 && RW % 16 == 0, "tile shape");
    constexpr int MID = I * J / 2;              // MFMAs issued before a stage boundary
    constexpr int NR = (WQ ? 2 : 1) * I + (XF32 ? 2 : 1) * J;  // LDS reads per K half
    // dequantizing forms: MFMAs that carry the LDS reads (two each), VALU per later MFMA
    constexpr int NRD = (NR + 1) / 2 < I * J ? (NR + 1) / 2 : I * J - 1;
    constexpr int VK = (WQ == 8 ? 14 : 24) * I + (XF32 ? 5 : 0) * J;   // decoding VALU per K half
    constexpr int VPM = (VK + (I * J - NRD) - 1) / (I * J - NRD);
    constexpr int NI = NR < I * J ? NR : I * J;  // MFMA : LDS-read pairs in the interleave
    static_assert(NS >= 2 && (NS - 1) * (CW + CX + CA) < 64, "ring depth");
    __shared__ HLds<BM, BN, XF32, NS, WQ> L;

    const int K = g.K, M = g.M, N = g.N;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const int splits = PART ? g.splits : 1;
    const int lfull = xcd_remap(blockIdx.x, tiles_m * tiles_n * splits);
    const int lt = lfull / splits, ks = lfull - lt * splits;
    int m0, n0;
    tile_origin(lt, tiles_m, tiles_n, BM, BN, g.ph, m0, n0);

    // the wave index is uniform: held in an SGPR, everything derived from it (LDS DMA
    // destinations, group offsets) is scalar work
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = (tid >> 6) & 1, wm = tid >> 7;
    const int l16 = lane & 15, lq = lane >> 4;

    // Operand DMA: per-tile buffer resources, a loop-invariant per-lane offset per DMA
    // instruction and a per-stage scalar offset. DMA instruction c of a row-major operand moves
    // rows (64/CPR)*c + lane/CPR, slot lane % CPR, which holds that row's chunk slot ^ swz(row);
    // rows past the operand's end re-read its last row (their outputs are discarded).
    const int S = K / 64;
    // dequant layout: the tile's first 16-row group g0 and this wave's groups of the tile (past
    // the last group: the last one, whose values only reach discarded rows)
    const int G = (N + 15) / 16, g0 = n0 / 16;
    uint32_t offw[CW], offx[CX], offa[CA > 0 ? CA : 1];
    __amdgpu_buffer_rsrc_t rw, ra, rx;
    if (WQ == 0) {
        rw = make_rsrc((const uint8_t*)g.w + (size_t)n0 * K * 2, (uint64_t)(N - n0) * K * 2);
        ra = rw;
#pragma unroll
        for (int q = 0; q < CW; q++) {
            const int r = (64 / CPW) * (wave + NW * q) + lane / CPW;
            const int n = min(n0 + r, N - 1);
            offw[q] = (uint32_t)(n - n0) * K * 2 + ((lane % CPW) ^ swz<CPW>(r)) * 16;
        }
    } else if (WQ == 8) {
        // codes: 1 KB per group and stage; then the scale rows, 64 bytes per group and stage
        const uint64_t wb = (uint64_t)G * S * 1024;
        rw = make_rsrc((const uint8_t*)g.w + (size_t)g0 * S * 1024, wb - (uint64_t)g0 * S * 1024);
        ra = make_rsrc((const uint8_t*)g.w + wb + (size_t)g0 * S * 64, (uint64_t)(G - g0) * S * 64);
#pragma unroll
        for (int q = 0; q < CW; q++)
            offw[q] = (uint32_t)(min(g0 + wave * GPW + q, G - 1) - g0) * S * 1024 + lane * 16;
        // lanes 16 * GPW.. repeat the wave's last scale row into the padding
        offa[0] = (uint32_t)(min(g0 + wave * GPW + min(lane / 16, GPW - 1), G - 1) - g0) * S * 64 + (lane % 16) * 4;
    } else {
        // nibbles: 512 bytes per group and stage; then the headers, 256 bytes per group and
        // super-block
        const uint64_t wb = (uint64_t)G * S * 512;
        rw = make_rsrc((const uint8_t*)g.w + (size_t)g0 * S * 512, wb - (uint64_t)g0 * S * 512);
        ra = make_rsrc((const uint8_t*)g.w + wb + (size_t)g0 * (K / 256) * 256, (uint64_t)(G - g0) * (K / 256) * 256);
        if (GPW >= 2) {
#pragma unroll
            for (int q = 0; q < CW; q++)
                offw[q] = (uint32_t)(min(g0 + wave * GPW + 2 * q + lane / 32, G - 1) - g0) * S * 512 + (lane % 32) * 16;
        } else {
            const uint32_t gw = (uint32_t)(min(g0 + wave, G - 1) - g0) * S * 512;
#pragma unroll
            for (int q = 0; q < CW; q++) offw[q] = gw + q * 256 + lane * 4;
        }
#pragma unroll
        for (int q = 0; q < CA; q++)
            offa[q] = (uint32_t)(min(g0 + wave * GPW + q, G - 1) - g0) * (K / 256) * 256 + lane * 4;
    }
    {
        constexpr int XB = XF32 ? 4 : 2;        // bytes per activation value
        const uint8_t* xb = XF32 ? (const uint8_t*)g.xf : (const uint8_t*)g.x;
        rx = make_rsrc(xb + (size_t)m0 * K * XB, (uint64_t)(M - m0) * K * XB);
#pragma unroll
        for (int q = 0; q < CX; q++) {
            const int r = (64 / CPX) * (wave + NW * q) + lane / CPX;
            const int m = min(m0 + r, M - 1);
            offx[q] = (uint32_t)(m - m0) * K * XB + ((lane % CPX) ^ swz<CPX>(r)) * 16;
        }
    }
    const int s_beg = (int)((int64_t)ks * S / splits), s_end = (int)((int64_t)(ks + 1) * S / splits);
    const int SL = s_end - s_beg;
    const int s0 = ((m0 / BM) + 4 * (n0 / BN)) % SL;          // K rotation
    auto kst = [&](int s) { int v = s + s0; return s_beg + (v >= SL ? v - SL : v); };
    auto dma_stage = [&](int st, int s) {
        const uint32_t k_ = (uint32_t)kst(s);
        if (WQ == 0) {
#pragma unroll
            for (int d = 0; d < CW; d++) bdma16(rw, offw[d], k_ * 128, &L.w[st][(wave + NW * d) * 64]);
        } else if (WQ == 8) {
#pragma unroll
            for (int d = 0; d < CW; d++) bdma16(rw, offw[d], k_ * 1024, &L.w[st][(wave * GPW + d) * 64]);
            bdma4(ra, offa[0], k_ * 64, &L.aux[st][wave * 16]);
        } else {
            if (GPW >= 2) {
#pragma unroll
                for (int d = 0; d < CW; d++) bdma16(rw, offw[d], k_ * 512, &L.w[st][(wave * GPW + 2 * d) * 32]);
            } else {
#pragma unroll
                for (int d = 0; d < CW; d++) bdma4(rw, offw[d], k_ * 512, &L.w[st][wave * 32 + d * 16]);
            }
#pragma unroll
            for (int d = 0; d < CA; d++) bdma4(ra, offa[d], (k_ >> 2) * 256, &L.aux[st][(wave * GPW + d) * 16]);
        }
#pragma unroll
        for (int d = 0; d < CX; d++) bdma16(rx, offx[d], k_ * (XF32 ? 256 : 128), &L.x[st][(wave + NW * d) * 64]);
    };
    // fragment of 16 rows from r0 (r0 % 16 == 0), K half kb: lane (l16, lq) takes 8 values
    auto frag = [&](const u32x4* B, int r0, int kb) {
        return __builtin_bit_cast(f16x8, B[(r0 + l16) * CPW + ((4 * kb + lq) ^ swz<CPW>(l16))]);
    };
    float q4s[WQ == 12 ? I : 1], q4m[WQ == 12 ? I : 1];   // Q4_K: second-half sub-block scales
    // weight fragment of subtile i (rows r0 = WN*wn + 16i ..) of the tile, K half kb of ring stage st
    // (global K stage ksg): fp16 as stored, or dequantized from the group's codes / nibbles
    auto wfrag = [&](int st, int i, int kb, int ksg) -> f16x8 {
        const int r0 = WN * wn + 16 * i;
        if constexpr (WQ == 0) {
            return frag(L.w[st], r0, kb);
        } else if constexpr (WQ == 8) {
            const int gi = r0 >> 4;
            const u32x2 c = ((const u32x2*)&L.w[st][gi * 64])[kb * 64 + lane];
            const uint32_t d = ((const uint16_t*)&L.aux[st][(gi / GPW) * 16 + (gi % GPW) * 4])[kb * 16 + l16];
            return deq_q8(c, d);
        } else {
            // the stage's two sub-block scales come from its header at the first half's read
            // and serve the second half's
            const int gi = r0 >> 4;
            const uint32_t c = ((const uint32_t*)&L.w[st][gi * 32])[kb * 64 + lane];
            if (kb == 0) {
                float s0, m0;
                q4_scales(L.aux[st][gi * 16 + l16], ksg, s0, m0, q4s[i], q4m[i]);
                return deq_q4v(c, s0, m0);
            }
            return deq_q4v(c, q4s[i], q4m[i]);
        }
    };
    // activation fragment: fp16 rows as stored, or fp32 rows rounded to fp16 on the way in
    auto xfrag = [&](const u32x4* B, int r0, int kb) {
        if (!XF32) return frag(B, r0, kb);
        const int r = r0 + l16, c = 8 * kb + 2 * lq;
        const f32x4 v0 = __builtin_bit_cast(f32x4, B[r * CPX + (c ^ swz<CPX>(l16))]);
        const f32x4 v1 = __builtin_bit_cast(f32x4, B[r * CPX + ((c + 1) ^ swz<CPX>(l16))]);
        return cvt8_f16(v0, v1);
    };

    f32x4 acc[I][J];
#pragma unroll
    for (int i = 0; i < I; i++)
#pragma unroll
        for (int j = 0; j < J; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    f16x8 a[2][I], b[2][J];

    // Ring: stages 0..NS-1 requested up front; at the boundary of stage s, stage s+1 is
    // awaited and stage s+NS goes into stage s's buffer (its fragments are in registers by
    // then). Requests past the last stage re-load it into buffers that are never read, so
    // every boundary issues the same DMA count and the vmcnt waits stay exact.
    constexpr int NDMA = CW + CA + CX;
#pragma unroll
    for (int k = 0; k < NS; k++) dma_stage(k, min(k, SL - 1));
    stage_sync<(NS - 1) * NDMA>();              // stage 0 has landed (mine, then everyone's)
#pragma unroll
    for (int i = 0; i < I; i++) a[0][i] = wfrag(0, i, 0, kst(0));
#pragma unroll
    for (int j = 0; j < J; j++) b[0][j] = xfrag(L.x[0], RW * wm + 16 * j, 0);

    // MFMAs of one K half on (ca, cb) while the next half's fragments go into (na, nb): read
    // from half 1 of the same stage (no boundary), or, at the stage boundary (half 1 of stage
    // s), from half 0 of stage s+1 after MID of the MFMAs
    auto mfma_all = [&](const f16x8 (&ca)[I], const f16x8 (&cb)[J], int q0, int q1) {
#pragma unroll
        for (int q = q0; q < q1; q++)
            acc[q % I][q / I] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ca[q % I], cb[q / I], acc[q % I][q / I], 0, 0, 0);
    };
    auto half_inner = [&](const f16x8 (&ca)[I], const f16x8 (&cb)[J], f16x8 (&na)[I], f16x8 (&nb)[J], int st,
                          int ksg) {
#pragma unroll
        for (int i = 0; i < I; i++) na[i] = wfrag(st, i, 1, ksg);
#pragma unroll
        for (int j = 0; j < J; j++) nb[j] = xfrag(L.x[st], RW * wm + 16 * j, 1);
        mfma_all(ca, cb, 0, I * J);
        if constexpr (WQ == 0) {
#pragma unroll
            for (int t = 0; t < NI; t++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
            }
            if (I * J > NI) __builtin_amdgcn_sched_group_barrier(0x008, I * J - NI, 0);
        } else {
            // the next half's LDS reads ride on the first MFMAs (two per MFMA), its decoding
            // (VALU) on the remaining ones, so the matrix pipe keeps issuing while it runs
#pragma unroll
            for (int t = 0; t < I * J; t++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (t < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                else __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
            }
        }
    };
    auto half_boundary = [&](const f16x8 (&ca)[I], const f16x8 (&cb)[J], f16x8 (&na)[I], f16x8 (&nb)[J],
                             int s, int st, int stn) {
        mfma_all(ca, cb, 0, MID);
        // The boundary runs on the last stage too (its fragment reads fetch an unused buffer):
        // with no branch around the LDS reads, the compiler's wait before the remaining MFMAs
        // covers only the reads those MFMAs consume, not the ones just issued.
        stage_sync<(NS - 2) * NDMA>();          // stage s+1 has landed (mine, then everyone's);
                                                // stage s is no longer read
        // (a 2-deep ring waits for everything, so it skips the re-loads past the end)
        if (NS > 2 ? s + 1 < SL : s + NS < SL) dma_stage(st, min(s + NS, SL - 1));
#pragma unroll
        for (int i = 0; i < I; i++) na[i] = wfrag(stn, i, 0, kst(s + 1 < SL ? s + 1 : s));
#pragma unroll
        for (int j = 0; j < J; j++) nb[j] = xfrag(L.x[stn], RW * wm + 16 * j, 0);
        mfma_all(ca, cb, MID, I * J);
    };

    // Stage s uses ring slot s % NS. The loop runs NS stages per iteration with the slots as
    // constants, so every LDS fragment read is a loop-invariant lane address plus an immediate
    // offset (with the slot a loop variable, each read costs one or two address instructions).
    // 128 x 128 tiles on quantized bytes keep the slot a variable: unrolled, their fragments,
    // accumulators and decoding no longer fit the registers of three workgroups per CU. (The
    // stage body is written out at each call site: called through a lambda capturing the
    // fragment arrays, the 128 x 128 kernels kept ~80 more registers live and spilled.)
    if constexpr (I * J <= 8 || WQ == 0) {
        int s = 0;
        for (; s + NS <= SL; s += NS) {
#pragma unroll
            for (int u = 0; u < NS; u++) {
                half_inner(a[0], b[0], a[1], b[1], u, kst(s + u));
                half_boundary(a[1], b[1], a[0], b[0], s + u, u, u + 1 == NS ? 0 : u + 1);
            }
        }
#pragma unroll
        for (int u = 0; u < NS - 1; u++) {
            if (s + u < SL) {
                half_inner(a[0], b[0], a[1], b[1], u, kst(s + u));
                half_boundary(a[1], b[1], a[0], b[0], s + u, u, u + 1);
            }
        }
    } else {
        int st = 0;
        for (int s = 0; s < SL; s++) {
            const int stn = st + 1 == NS ? 0 : st + 1;
            half_inner(a[0], b[0], a[1], b[1], st, kst(s));
            half_boundary(a[1], b[1], a[0], b[0], s, st, stn);
            st = stn;
        }
    }
    wait_vm0();

    // bias and activation on the accumulators (lane column n0 + WN*wn + 16i + 4lq + e), where
    // every value is independent of the others, before the transpose
    if (!PART) {
        // columns past N (and a null bias: an empty range) read zeros in the range check
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(g.bias, g.bias ? (uint64_t)N * 4 : 0);
#pragma unroll
        for (int i = 0; i < I; i++) {
            const int nb = n0 + WN * wn + 16 * i + 4 * lq;
            const f32x4 bi = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, nb * 4, 0, 0));
#pragma unroll
            for (int j = 0; j < J; j++) {
                acc[i][j] += bi;
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][j][e] = act_h<ACT>(acc[i][j][e]);
            }
        }
    }

    // epilogue: the tile leaves through LDS as whole rows, HR rows (of one wave row) at a time
    constexpr int P = BN + 4;                   // padded row pitch (floats)
    constexpr int HR = RW < 64 ? RW : 64;
    constexpr int HPW = RW / HR;                // passes per wave row
    constexpr int JH = HR / 16;                 // activation subtiles per pass
    static_assert(HR * P * 4 <= (int)sizeof(HLds<BM, BN, XF32, NS, WQ>), "transpose buffer fits the ring");
    constexpr int TR = BN / 4;                  // threads per output row
    float* T = (float*)&L;
    const int c = 4 * (tid % TR);               // this thread's 4 columns
    const int n = n0 + c;
    float* part = PART ? g.ws + ((size_t)lt * splits + ks) * (size_t)BM * BN : nullptr;
    constexpr int NP = HR / (NTH / TR);         // output rows per thread and pass
    // Residual loads and output stores are buffer accesses from the tile origin, over a range
    // that ends with the tile's last row inside M: rows past M fall outside it, and a column
    // past N takes an offset beyond any range (N <= 2^21 keeps every offset below 2^31), so the
    // hardware range check drops those stores and zero-fills those loads — no per-row branch
    // or 64-bit address arithmetic in the store loop.
    const size_t org = (size_t)m0 * N + n0;
    const uint32_t span = (uint32_t)min(BM, M - m0) * (uint32_t)N - (uint32_t)n0;   // elements
    // this thread's byte offset in its first row of the tile, fp32 / fp16 elements (a row
    // offset (HR h + (NTH / TR) p) N elements is added per store)
    const uint32_t el0 = (uint32_t)(tid / TR) * N + c;
    const uint32_t ob4 = n < N ? el0 * 4 : 0x80000000u, ob2 = n < N ? el0 * 2 : 0x80000000u;
    const bool rs = !PART && g.resid, o16 = g.y16 != nullptr, o32 = !PART && !o16 && g.y;
    const __amdgpu_buffer_rsrc_t rres = make_rsrc(rs ? g.resid + org : nullptr, rs ? (uint64_t)span * 4 : 0);
    const __amdgpu_buffer_rsrc_t rout =
        o16 ? make_rsrc(g.y16 + org, (uint64_t)span * 2) : make_rsrc(o32 ? g.y + org : nullptr, o32 ? (uint64_t)span * 4 : 0);
#pragma unroll
    for (int h = 0; h < WMR * HPW; h++) {
        // the pass's residual loads go out before the transpose, all at once (one HBM
        // round trip per pass, overlapped with the LDS work)
        // without a residual -0.0, which leaves every value as it is when added
        f32x4 rv[NP];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            rv[p] = f32x4{-0.f, -0.f, -0.f, -0.f};
            if (rs) {
                const uint32_t ro = ob4 + (uint32_t)(HR * h + (NTH / TR) * p) * N * 4;
                rv[p] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rres, (int)ro, 0, 0));
            }
        }
        __syncthreads();                        // ring / previous rows no longer read
        if (wm == h / HPW) {
#pragma unroll
            for (int i = 0; i < I; i++)
#pragma unroll
                for (int j = 0; j < JH; j++)
                    *(f32x4*)&T[(16 * j + l16) * P + WN * wn + 16 * i + 4 * lq] = acc[i][(h % HPW) * JH + j];
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int r = (NTH / TR) * p + tid / TR;
            const f32x4 v = *(const f32x4*)&T[r * P + c];
            if (PART) {
                __builtin_nontemporal_store(v, (f32x4*)(part + (size_t)(HR * h + r) * BN + c));
                continue;
            }
            const f32x4 o = v + rv[p];
            const uint32_t rb = (uint32_t)(HR * h + (NTH / TR) * p) * N;  // row offset, elements
            // aux 2: non-temporal (the output is not re-read by this launch)
            if (g.y16)
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, cvt4_f16(o)), rout, (int)(ob2 + rb * 2), 0, 2);
            else
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), rout, (int)(ob4 + rb * 4), 0, 2);
        }
    }
}

// One float4 of a split-K output: the splits' partials in split order, then +bias -> act ->
// +resid (part: the float4 in split 0's partial tile; the next split's is q_stride further)
template <int ACT>
__device__ __forceinline__ f32x4 split_sum4(const f32x4* part, size_t q_stride, int splits, const float* bias,
                                            int n, const float* resid, size_t o) {
    // the first KB partials, the bias and the residual are all requested before any is summed
    // (one memory round trip, not one per split); the sum keeps split order
    constexpr int KB = 4;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 p[KB];
#pragma unroll
    for (int k = 0; k < KB; k++) p[k] = k < splits ? __builtin_nontemporal_load(part + (size_t)k * q_stride) : z;
    const f32x4 bv = bias ? *(const f32x4*)(bias + n) : z;
    const f32x4 rv = resid ? *(const f32x4*)(resid + o) : z;
    f32x4 v = p[0];
#pragma unroll
    for (int k = 1; k < KB; k++)
        if (k < splits) v += p[k];
    for (int k = KB; k < splits; k++) v += __builtin_nontemporal_load(part + (size_t)k * q_stride);
    if (bias) v += bv;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = act_h<ACT>(v[e]);
    if (resid) v += rv;
    return v;
}

// Split-K epilogue: one thread per output float4; sums the splits' row-major partial tiles in
// split order, then +bias -> act -> +resid.
template <int ACT, int BM, int BN>
__global__ __launch_bounds__(256) void k_gemm_fc_reduce(GemmH16Args g) {
    const int M = g.M, N = g.N, splits = g.splits;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const size_t idx4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    constexpr int Q = BM * BN / 4;              // float4s per tile
    const int lt = (int)(idx4 / Q);
    if (lt >= tiles_m * tiles_n) return;
    const int q = (int)(idx4 - (size_t)lt * Q);
    const int r = q / (BN / 4), c = 4 * (q % (BN / 4));
    int m0, n0;
    tile_origin(lt, tiles_m, tiles_n, BM, BN, g.ph, m0, n0);
    const int m = m0 + r, n = n0 + c;
    if (m >= M || n >= N) return;
    const size_t o = (size_t)m * N + n;
    const f32x4 v = split_sum4<ACT>((const f32x4*)(g.ws + (size_t)lt * splits * BM * BN) + q, Q, splits, g.bias, n,
                                    g.resid, o);
    if (g.y16)
        __builtin_nontemporal_store(cvt4_f16(v),
                                    (f16x4*)(g.y16 + o));
    else
        __builtin_nontemporal_store(v, (f32x4*)(g.y + o));
}

// Split-K epilogue followed by the LayerNorm-affine of each output row (N = 256 C, no
// activation): one wave per row sums the row's float4s with k_gemm_fc_reduce's arithmetic,
// stores them to y and normalizes the row from registers with the LayerNorm kernel's own
// code (ln_affine_row), so y and every LayerNorm output equal those of k_gemm_fc_reduce
// followed by k_layernorm_affine on y, in one launch.
template <int C, int EMIT>
__global__ __launch_bounds__(256) void k_gemm_fc_reduce_ln(GemmH16Args g, int bm, int bn, LnArgs ln) {
    const int M = g.M, N = g.N, splits = g.splits;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;                       // whole wave exits together
    const int tiles_m = (M + bm - 1) / bm, tiles_n = (N + bn - 1) / bn;
    const int tm = row / bm, r = row - tm * bm;
    // the logical tile of (tm, tn): the inverse of tile_origin's panel order
    const int panel = tm / g.ph, pm = min(g.ph, tiles_m - panel * g.ph);
    const size_t tile = (size_t)bm * bn, q_stride = tile / 4;
    // every partial of a round (up to KB splits x C float4s), the bias and the residual are
    // requested before any is summed: a few round trips per row, not one per split and chunk
    constexpr int KB = 4;
    const f32x4* pc[C];
    f32x4 v[C], bb[C], rb[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int n = 4 * (lane + 64 * c);
        const int tn = n / bn;
        const int lt = panel * g.ph * tiles_n + (tm - panel * g.ph) + pm * tn;
        pc[c] = (const f32x4*)(g.ws + (size_t)lt * splits * tile + (size_t)r * bn + (n - tn * bn));
        v[c] = bb[c] = rb[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (g.bias) bb[c] = *(const f32x4*)(g.bias + n);
        if (g.resid) rb[c] = *(const f32x4*)(g.resid + (size_t)row * N + n);
    }
    for (int k0 = 0; k0 < splits; k0 += KB) {
        f32x4 pv[KB][C];
#pragma unroll
        for (int kk = 0; kk < KB; kk++)
            if (k0 + kk < splits)
#pragma unroll
                for (int c = 0; c < C; c++) pv[kk][c] = __builtin_nontemporal_load(pc[c] + (size_t)(k0 + kk) * q_stride);
        // split order per element, as split_sum4: v = p0, then v + p1, v + p2, ...
#pragma unroll
        for (int kk = 0; kk < KB; kk++)
            if (k0 + kk < splits)
#pragma unroll
                for (int c = 0; c < C; c++) v[c] = k0 + kk == 0 ? pv[kk][c] : v[c] + pv[kk][c];
    }
    // then +bias -> +resid (no activation), each rounded, as split_sum4<0>; y stored unless
    // the caller needs only the LayerNorm's outputs (g.y null)
#pragma unroll
    for (int c = 0; c < C; c++) {
        if (g.bias) v[c] += bb[c];
        if (g.resid) v[c] += rb[c];
        if (g.y) __builtin_nontemporal_store(v[c], (f32x4*)(g.y + (size_t)row * N + 4 * (lane + 64 * c)));
    }
    ln_affine_row<C, EMIT>(v, lane, row, ln.gamma, ln.beta, ln.y, ln.eps, ln.codes, ln.dx, ln.s4);
}

template <int EMIT>
hipError_t launch_reduce_ln_e(const GemmH16Args& a, int bm, int bn, const LnArgs& ln, hipStream_t s) {
    const dim3 grid((unsigned)((a.M + 3) / 4)), block(256);
    switch (a.N / 256) {
#define MGH_RLN(CV)                                                                                       \
    case CV: hipLaunchKernelGGL((k_gemm_fc_reduce_ln<CV, EMIT>), grid, block, 0, s, a, bm, bn, ln); break;
        MGH_RLN(1) MGH_RLN(2) MGH_RLN(3) MGH_RLN(4) MGH_RLN(5) MGH_RLN(6) MGH_RLN(7) MGH_RLN(8)
#undef MGH_RLN
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_reduce_ln(const GemmH16Args& a, int bm, int bn, const LnArgs& ln, hipStream_t s) {
    if (ln.emit == 1) return launch_reduce_ln_e<1>(a, bm, bn, ln, s);
    if (ln.emit == 2) return launch_reduce_ln_e<2>(a, bm, bn, ln, s);
    return launch_reduce_ln_e<0>(a, bm, bn, ln, s);
}

// Skinny-M FC (M <= 16 * MT, decode- and GEMV-shaped calls): one workgroup per 16 weight rows,
// its KS waves split K (wave w takes the 32-deep K steps w, w + KS, ...), each lane streams 16
// bytes of its weight row per step straight into registers (no LDS staging: every weight is
// read once) and multiplies on v_mfma_f32_16x16x32_f16 against the activation rows, taken as MT
// 16-row MFMA tiles (rows past M are zero). The KS partial tiles are summed in LDS in wave order
// (deterministic) and the epilogue is the one of k_gemm_fc: +bias -> act -> +resid, fp32 or
// fp16 out. Same operand rounding as k_gemm_fc (fp32 activations rounded to fp16, nearest
// even), so the two differ only in the fp32 summation order.
template <int ACT, bool XF32, int MT, int KS, int WQ>
__global__ __launch_bounds__(64 * KS) void k_gemv_fc(GemmH16Args g) {
    constexpr int U = 4;                        // K steps in flight per wave
    __shared__ f32x4 part[KS][MT][64];
    const int K = g.K, M = g.M, N = g.N;
    const int T = K / 32;
    const int n0 = blockIdx.x * 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, g4 = lane >> 4;
    const _Float16* wrow = (const _Float16*)g.w + (size_t)min(n0 + r16, N - 1) * K + 8 * g4;
    // K-loop-dequant layout: this workgroup's 16-row group (n0 / 16)
    const int S = K / 64, grp = n0 / 16;
    const uint8_t* wq = (const uint8_t*)g.w;
    const size_t gsz = WQ == 8 ? 1024 : 512;
    const uint8_t* wgrp = wq + (size_t)grp * S * gsz;
    const uint8_t* wside = wq + (size_t)((N + 15) / 16) * S * gsz;
    // weight fragment of 32-deep K step t (stage t / 2, half t % 2)
    auto wld = [&](int t) -> f16x8 {
        if constexpr (WQ == 0) {
            return *(const f16x8*)(wrow + 32 * t);
        } else if constexpr (WQ == 8) {
            const u32x2 c = *(const u32x2*)(wgrp + (size_t)(t >> 1) * 1024 + 512 * (t & 1) + 8 * lane);
            const uint32_t d = ((const uint16_t*)wside)[((size_t)grp * S + (t >> 1)) * 32 + 16 * (t & 1) + r16];
            return deq_q8(c, d);
        } else {
            const uint32_t c = *(const uint32_t*)(wgrp + (size_t)(t >> 1) * 512 + 256 * (t & 1) + 4 * lane);
            const u32x4 h = ((const u32x4*)wside)[((size_t)grp * (K / 256) + (t >> 3)) * 16 + r16];
            return deq_q4(c, h, t & 7);
        }
    };
    size_t xofs[MT];
    bool xin[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = 16 * mt + r16;
        xin[mt] = m < M;
        xofs[mt] = (size_t)min(m, M - 1) * K + 8 * g4;
    }
    auto xfrag = [&](int mt, int t) {
        if (!xin[mt]) return f16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (!XF32) return *(const f16x8*)(g.x + xofs[mt] + 32 * t);
        const f32x4* p = (const f32x4*)(g.xf + xofs[mt] + 32 * t);
        return cvt8_f16(p[0], p[1]);
    };
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    int t = wave;
    for (; t + (U - 1) * KS < T; t += U * KS) {
        f16x8 a[U], b[U][MT];
#pragma unroll
        for (int u = 0; u < U; u++) {
            a[u] = wld(t + u * KS);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) b[u][mt] = xfrag(mt, t + u * KS);
        }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], b[u][mt], acc[mt], 0, 0, 0);
    }
    for (; t < T; t += KS) {
        const f16x8 a = wld(t);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xfrag(mt, t), acc[mt], 0, 0, 0);
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) part[wave][mt][lane] = acc[mt];
    __syncthreads();
    if (tid >= MT * 64) return;
    // thread (mt, l) owns the outputs lane l of every wave holds for tile mt:
    // rows m = 16 mt + l % 16, columns n .. n + 3 with n = n0 + 4 (l / 16)
    const int mt = tid >> 6, l = tid & 63;
    f32x4 v = part[0][mt][l];
#pragma unroll
    for (int w = 1; w < KS; w++) v += part[w][mt][l];
    const int m = 16 * mt + (l & 15), n = n0 + 4 * (l >> 4);
    if (m >= M || n >= N) return;
    if (g.bias) v += *(const f32x4*)(g.bias + n);
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = act_h<ACT>(v[e]);
    const size_t o = (size_t)m * N + n;
    if (g.resid) v += *(const f32x4*)(g.resid + o);
    if (g.y16)
        *(f16x4*)(g.y16 + o) = cvt4_f16(v);
    else
        *(f32x4*)(g.y + o) = v;
}

template <bool XF32, int MT, int WQ>
static hipError_t launch_gemv_w(const GemmH16Args& a, hipStream_t s) {
    constexpr int KS = 8;
    const dim3 grid((unsigned)((a.N + 15) / 16)), block(64 * KS);
    if (a.act == 1) hipLaunchKernelGGL((k_gemv_fc<1, XF32, MT, KS, WQ>), grid, block, 0, s, a);
    else if (a.act == 2) hipLaunchKernelGGL((k_gemv_fc<2, XF32, MT, KS, WQ>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_gemv_fc<0, XF32, MT, KS, WQ>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <bool XF32, int MT>
static hipError_t launch_gemv_t(const GemmH16Args& a, hipStream_t s) {
    if (a.wq == 8) return launch_gemv_w<XF32, MT, 8>(a, s);
    if (a.wq == 12) return launch_gemv_w<XF32, MT, 12>(a, s);
    if (a.wq == 0) return launch_gemv_w<XF32, MT, 0>(a, s);
    return hipErrorInvalidValue;
}

// Skinny-M kernel or tiled plan: measured on the four FC shapes with cold operands (fp32
// activations, buffers rotated over 24 sets): the skinny kernel is faster up to 16 rows on
// every shape (M = 1: 3.5-3.9 against 5.8-6.4 us for K = 768, 6.8 against 11.0 us for the
// K = 3072 down-proj; M = 16: 4.5-4.7 against 6.0-6.3 us, 10.4 against 11.4 us) and up to 32
// rows for K <= 1024 (M = 32: 5.9-6.1 against 6.2-6.5 us); above, the tiled plan wins.
bool use_gemv_h16(int M, int K) { return M >= 1 && (M <= 16 || (M <= 32 && K <= 1024)); }

hipError_t launch_gemv_h16(const GemmH16Args& a, hipStream_t s) {
    const bool xf = a.xf != nullptr;
    if (a.M < 1 || a.M > kGemvMaxRows) return hipErrorInvalidValue;
    if (a.M <= 16) return xf ? launch_gemv_t<true, 1>(a, s) : launch_gemv_t<false, 1>(a, s);
    return xf ? launch_gemv_t<true, 2>(a, s) : launch_gemv_t<false, 2>(a, s);
}

static H16Plan gemm_h16_plan_rules(int M, int N, int K, bool xf32, int wq);

namespace {
// Tile-plan override for measurements, so that the plan comparisons quoted above can be rerun
// with the committed library: MGH_FC_PLAN="bm,bn,ns,splits" (or "bm,bn,ns,splits,K,N" for the
// launches of one K x N shape) replaces the plan of every tiled FC launch. The kernel set holds
// the plans the rules pick and a few more; a plan outside it makes the launch fail with
// hipErrorInvalidValue. Read once per process.
struct PlanOverride {
    bool on = false;
    int bm = 0, bn = 0, ns = 0, splits = 1, k = 0, n = 0;
};
const PlanOverride& plan_override() {
    static const PlanOverride o = [] {
        PlanOverride r;
        const char* e = std::getenv("MGH_FC_PLAN");
        int v[6] = {0, 0, 0, 1, 0, 0};
        if (e && std::sscanf(e, "%d,%d,%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5]) >= 4 && v[0] > 0 &&
            v[1] > 0 && v[2] >= 2 && v[3] >= 1) {
            r.on = true;
            r.bm = v[0], r.bn = v[1], r.ns = v[2], r.splits = v[3], r.k = v[4], r.n = v[5];
        }
        return r;
    }();
    return o;
}
}  // namespace

H16Plan gemm_h16_plan(int M, int N, int K, bool xf32, int wq) {
    H16Plan p = gemm_h16_plan_rules(M, N, K, xf32, wq);
    const PlanOverride& o = plan_override();
    if (o.on && (!o.k || o.k == K) && (!o.n || o.n == N)) {
        p.bm = o.bm;
        p.bn = o.bn;
        p.ns = o.ns;
        p.splits = o.splits;
        const int tiles = ((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
        p.ws_bytes = p.splits > 1 ? (size_t)tiles * p.splits * p.bm * p.bn * 4 : 0;
    }
    return p;
}

static H16Plan gemm_h16_plan_rules(int M, int N, int K, bool xf32, int wq) {
    H16Plan p{};
    p.ns = 2;
    p.bn = 128;
    p.wmr = 2;
    const int t128 = ((M + 127) / 128) * ((N + 127) / 128);
    const int t6464 = ((M + 63) / 64) * ((N + 63) / 64);
    if (wq) {
        // Quantized weight bytes (decoded in the K loop): the decoding is VALU work per weight
        // fragment and wave, so the plans favour more workgroups per CU (a wave's decoding
        // overlaps another's MFMAs) and more activation rows per wave. Measured against the
        // fp16-weight plans on the four FC shapes, Q8_0, buffers rotated over 1 GB:
        //  * fp32 activations, K <= 1024, M > 128: 64 x 64 tiles on a 2-deep ring when they fit
        //    one round of workgroups (three per CU), 32 x 64 when there are fewer than one per
        //    CU (M = 1025: QKV 15.8 against 18.9 us, out-proj 11.8 against 12.7 us; M = 257, all
        //    32 x 64: QKV 10.6 against 11.2 us, out-proj 10.6 against 10.9 us, the 3072-wide
        //    up-proj 11.5 against 12.3 us on the few-tile plan's 3-deep 64 x 64 ring);
        //  * fp16 activations, 128 x 128 tiles from one tile per CU, the long-K narrow
        //    down-proj split in two (M = 4097: QKV 35.6 against 40.2 us including the rounding
        //    pass, down-proj 58.7 against 64.0 us).
        if (xf32 && K <= 1024 && M > 128 && t6464 <= 768) {
            p.ns = 2;
            p.bn = 64;
            p.bm = t6464 < 256 ? 32 : 64;
            p.splits = 1;
            p.ws_bytes = 0;
            p.ph = 8;
            return p;
        }
        if (!xf32 && t128 >= 256) {
            p.bm = 128;
            p.splits = 1;
            p.ws_bytes = 0;
            p.ph = 8;
            return p;
        }
        if (!xf32 && K >= 2048 && N <= 1024 && t128 >= 128) {
            p.bm = 128;
            p.splits = 2;
            p.ws_bytes = (size_t)t128 * 2 * 128 * 128 * 4;
            p.ph = 8;
            return p;
        }
    }
    // Tile choice, from timings of the four FC shapes at M = 1025, 4112 and 16448 on fp16
    // operands with cold weights and activations (buffers rotated over 1 GB): 64-row tiles
    // (three workgroups per CU) up to about four 128-row tiles per CU, 128-row tiles beyond;
    // for narrow outputs (N <= 1024, where the activations are the larger operand) 128-row
    // tiles from about one tile per CU (M = 4112 down-proj: 40.5 against 43.7 us). Larger
    // tiles (128 x 256 on 4 waves, 256 x 256 on 8) measured slower on every shape. With fp32
    // activations, 64-row tiles: their stage is already as large as a 128-row fp16 stage.
    // 3072-wide outputs (the MLP up-proj) take 128-row tiles from about 1.5 tiles per CU
    // (M = 4112: 43.6 against 46.2 us; M = 2056: 23.8 against 27.2 us; at M = 1025 the 64-row
    // tiles win, 15.2 against 17.2 us). Narrow outputs with short K (the out-proj) keep 64-row
    // tiles below 256 128-row tiles (M = 4112 out-proj on fp16 activations: 14.9 against
    // 16.4 us on fp16 copies, 17.5 against 19.0 on Q8_0 bytes; at M = 8193 the 128-row tiles
    // win, 24.4 against 27.0 us)
    const bool wide128 = t128 >= 1024 || (N <= 1024 && t128 >= 192 && (K >= 2048 || t128 >= 256)) ||
                         (N >= 3072 && t128 >= 384);
    p.bm = wide128 && !xf32 ? 128 : 64;
    const int tiles = ((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
    const int S = K / 64;
    p.splits = 1;
    // Few tiles: 64 x 64 tiles on a 3-deep ring (72 KB per workgroup with fp32 activation
    // rows, 48 KB with fp16: two resp. three workgroups per CU) when every tile is resident at
    // once, for short K or at most half a tile per CU; 32-row tiles below half a tile per CU
    // for short K; split K while every split keeps >= 12 stages and stays resident. Measured on
    // the four FC shapes at M = 257 and 1025 against the 64 x 128 2-deep plan (split-K and
    // reduce included), fp32 / fp16 activations: M = 257 QKV 8.7 / 7.0 against 11.0 / 10.4 us,
    // up 9.4 / 7.8 against 12.1 / 10.9, out 6.7 / 6.5 against 9.7 / 9.2, down 13.8 / 12.3
    // against 17.3 / 16.3; M = 1025 out 9.8 / 8.2 against 12.8 / 11.9, QKV (fp16) 11.9 against
    // 12.8. Long-K shapes with more tiles (M = 1025 down-proj on fp32 rows: 23.8 against 22.1)
    // keep the 64 x 128 split-K plan.
    const int slots = xf32 ? 512 : 768;
    if ((K <= 1024 || t6464 <= 128) && t6464 <= slots) {
        p.ns = 3;
        p.bn = 64;
        p.bm = K <= 1024 && t6464 < 128 ? 32 : 64;
        const int ts = ((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
        while (ts * p.splits * 2 <= slots && S / (p.splits * 2) >= 12) p.splits *= 2;
        p.ws_bytes = p.splits > 1 ? (size_t)ts * p.splits * p.bm * p.bn * 4 : 0;
        const int tm = (M + p.bm - 1) / p.bm;
        p.ph = tm <= 32 && (int64_t)M * (xf32 ? 4 : 2) * 2 >= (int64_t)N * 2 ? 1 : 8;
        return p;
    }
    // long-K narrow outputs on fp16 operands with 0.75 to three 64-row tiles per CU: 64-row
    // tiles on a 3-deep ring (72 KB, two workgroups per CU) and no split (M = 4112 down-proj:
    // 38.5 against 42.8 us for 128-row tiles in 2 splits; M = 2056: 26.4 against 28.9 us for
    // 2 splits; at M = 16448 the 128-row tiles win)
    const int t64 = ((M + 63) / 64) * ((N + 127) / 128);
    if (!xf32 && N <= 1024 && K >= 2048 && t64 >= 192 && t64 <= 768) {
        p.bm = 64;
        p.ns = 3;
        p.ws_bytes = 0;
        p.ph = 8;
        return p;
    }
    // split K while there are at most two workgroups per CU and each split keeps >= 12
    // stages (>= 6 with at most half a tile per CU); measured at M = 1025: the down-proj (102
    // tiles, 48 stages) fastest at 4 splits, the out-proj (102 tiles, 12 stages) at 2
    const int min_stages = tiles <= 128 ? 6 : 12;
    while (tiles * p.splits * 2 <= 512 && S / (p.splits * 2) >= min_stages) p.splits *= 2;
    p.ws_bytes = p.splits > 1 ? (size_t)tiles * p.splits * p.bm * p.bn * 4 : 0;
    // tile order: with few activation-row tiles and activations at least half the weight bytes
    // (M ~ 1000, fp32 rows) consecutive tiles walk the weight rows of one activation tile; else
    // panels of 8 activation tiles, which keep an XCD's weight tiles in its L2 (measured: the
    // former wins 3-9% on the four FCs at M = 1025, the latter 6% on one FC at M = 257)
    const int tm = (M + p.bm - 1) / p.bm;
    p.ph = tm <= 32 && (int64_t)M * (xf32 ? 4 : 2) * 2 >= (int64_t)N * 2 ? 1 : 8;
    return p;
}

size_t packed_weight_bytes_f16(int64_t N, int64_t K) { return (size_t)(2 * N * K); }

hipError_t launch_pack_weights_f16(int wtype, const void* w, void* out, int N, int K, hipStream_t s) {
    const int64_t blocks = (int64_t)N * (K / 32);
    if (blocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
    if (wtype == 8)
        hipLaunchKernelGGL(k_pack_w16<8>, grid, block, 0, s, (const uint8_t*)w, (u32x4*)out, N, K);
    else if (wtype == 12)
        hipLaunchKernelGGL(k_pack_w16<12>, grid, block, 0, s, (const uint8_t*)w, (u32x4*)out, N, K);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

size_t packed_weight_bytes_dq(int wtype, int64_t N, int64_t K) {
    const int64_t G = (N + 15) / 16;
    if (wtype == 8) return (size_t)(G * (K / 64) * (1024 + 64));
    if (wtype == 12) return (size_t)(G * ((K / 64) * 512 + (K / 256) * 256));
    return 0;
}

hipError_t launch_pack_weights_dq(int wtype, const void* w, void* out, int N, int K, hipStream_t s) {
    const int64_t blocks = (int64_t)N * (K / 32);
    if (blocks == 0) return hipSuccess;
    // rows past N in the last 16-row group: zero codes and scales
    const size_t bytes = packed_weight_bytes_dq(wtype, N, K);
    if (N % 16) {
        if (hipError_t e = launch_fill_u32((uint32_t*)out, 0u, bytes / 4, s)) return e;
    }
    const dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
    if (wtype == 8)
        hipLaunchKernelGGL(k_pack_wdq<8>, grid, block, 0, s, (const uint8_t*)w, (uint8_t*)out, N, K);
    else if (wtype == 12)
        hipLaunchKernelGGL(k_pack_wdq<12>, grid, block, 0, s, (const uint8_t*)w, (uint8_t*)out, N, K);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_dequant_weights_f32(int wtype, const void* w, float* out, int N, int K, hipStream_t s) {
    const int64_t blocks = (int64_t)N * (K / 32);
    if (blocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
    if (wtype == 8)
        hipLaunchKernelGGL(k_dequant_w32<8>, grid, block, 0, s, (const uint8_t*)w, out, N, K);
    else if (wtype == 12)
        hipLaunchKernelGGL(k_dequant_w32<12>, grid, block, 0, s, (const uint8_t*)w, out, N, K);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_f32_to_f16(const float* x, _Float16* h, int64_t n, hipStream_t s) {
    const int64_t n8 = n / 8;
    if (n8 == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f32_to_f16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s,
                       (const f32x4*)x, (u32x4*)h, n8);
    return hipGetLastError();
}

template <int BM, bool XF32, int NS, int WMR, int BN, int WQ>
static hipError_t launch_h16_w(const GemmH16Args& a, hipStream_t s, const LnArgs* ln) {
    const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const int splits = std::max(a.splits, 1);
    const dim3 block(128 * WMR);
    if (splits > 1) {
        hipLaunchKernelGGL((k_gemm_fc<0, BM, true, XF32, NS, WMR, BN, WQ>), dim3(tiles * splits), block, 0, s, a);
        if (ln) return launch_reduce_ln(a, BM, BN, *ln, s);
        const size_t n4 = (size_t)tiles * BM * BN / 4;
        const dim3 rg((unsigned)((n4 + 255) / 256)), rb(256);
        if (a.act == 1) hipLaunchKernelGGL((k_gemm_fc_reduce<1, BM, BN>), rg, rb, 0, s, a);
        else if (a.act == 2) hipLaunchKernelGGL((k_gemm_fc_reduce<2, BM, BN>), rg, rb, 0, s, a);
        else hipLaunchKernelGGL((k_gemm_fc_reduce<0, BM, BN>), rg, rb, 0, s, a);
    } else {
        if (a.act == 1) hipLaunchKernelGGL((k_gemm_fc<1, BM, false, XF32, NS, WMR, BN, WQ>), dim3(tiles), block, 0, s, a);
        else if (a.act == 2) hipLaunchKernelGGL((k_gemm_fc<2, BM, false, XF32, NS, WMR, BN, WQ>), dim3(tiles), block, 0, s, a);
        else hipLaunchKernelGGL((k_gemm_fc<0, BM, false, XF32, NS, WMR, BN, WQ>), dim3(tiles), block, 0, s, a);
    }
    return hipGetLastError();
}

template <int BM, bool XF32, int NS, int WMR, int BN>
static hipError_t launch_h16_t(const GemmH16Args& a, hipStream_t s, const LnArgs* ln) {
    if (a.wq == 8) return launch_h16_w<BM, XF32, NS, WMR, BN, 8>(a, s, ln);
    if (a.wq == 12) return launch_h16_w<BM, XF32, NS, WMR, BN, 12>(a, s, ln);
    if (a.wq == 0) return launch_h16_w<BM, XF32, NS, WMR, BN, 0>(a, s, ln);
    return hipErrorInvalidValue;
}

// The plan's kernel
static hipError_t dispatch_h16(const H16Plan& p, const GemmH16Args& a, hipStream_t s, const LnArgs* ln) {
    const bool xf = a.xf != nullptr;
    if (p.bn == 128 && p.ns == 2) {
        if (p.bm == 128 && !xf) return launch_h16_t<128, false, 2, 2, 128>(a, s, ln);
        if (p.bm == 64)
            return xf ? launch_h16_t<64, true, 2, 2, 128>(a, s, ln) : launch_h16_t<64, false, 2, 2, 128>(a, s, ln);
    }
    if (p.bn == 128 && p.ns == 3 && p.bm == 64 && !xf) return launch_h16_t<64, false, 3, 2, 128>(a, s, ln);
    if (p.bn == 64 && p.ns == 3) {
        if (p.bm == 64)
            return xf ? launch_h16_t<64, true, 3, 2, 64>(a, s, ln) : launch_h16_t<64, false, 3, 2, 64>(a, s, ln);
        if (p.bm == 32)
            return xf ? launch_h16_t<32, true, 3, 2, 64>(a, s, ln) : launch_h16_t<32, false, 3, 2, 64>(a, s, ln);
    }
    // plans of the quantized-byte forms only
    if (a.wq && p.bn == 64 && p.ns == 2 && xf) {
        if (p.bm == 64)
            return a.wq == 8 ? launch_h16_w<64, true, 2, 2, 64, 8>(a, s, ln) : launch_h16_w<64, true, 2, 2, 64, 12>(a, s, ln);
        if (p.bm == 32)
            return a.wq == 8 ? launch_h16_w<32, true, 2, 2, 64, 8>(a, s, ln) : launch_h16_w<32, true, 2, 2, 64, 12>(a, s, ln);
    }
    return hipErrorInvalidValue;
}

// CUs of the current device (asked once per device)
static int device_cus() {
    static std::atomic<int> n[64];
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 0;
    int v = n[d].load(std::memory_order_relaxed);
    if (v <= 0 && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, d) == hipSuccess) n[d].store(v);
    return v > 0 ? v : 0;
}

hipError_t launch_gemm_h16(const H16Plan& p, const GemmH16Args& a0, hipStream_t s, const LnArgs* ln) {
    GemmH16Args a = a0;
    a.ph = p.ph;
    if (p.wmr != 2) return hipErrorInvalidValue;
    if (a.N > kFcMaxN) return hipErrorInvalidValue;     // the epilogue's 32-bit tile offsets
    // the reduce takes the LayerNorm only when K is split, without activation or fp16 output
    if (ln && (p.splits < 2 || a.act != 0 || a.y16 || a.N % 256 || a.N > 2048)) return hipErrorInvalidValue;
    // A last, partial row of tiles that raises the most tiles any CU runs (ceil(tiles / CUs))
    // goes to the skinny-M kernel instead, after the tiled kernel has taken the whole tile
    // rows: a launch takes about as long as its most loaded CU. At M = 4097 the up-proj's 33rd row of 128-row tiles
    // (24 tiles past 768 = three per CU) costs ~9 us on the Q8_0 bytes (M = 4096: 43.1 us,
    // 4097: 52.5 us, 4224: 51.7 us) and ~6.5 us on fp16 copies, the skinny kernel ~4.5 us at
    // K <= 1024. Rows past the split are summed in the skinny kernel's fp32 order.
    if (!ln && p.splits <= 1 && a.K <= 1024) {
        const int mfull = a.M / p.bm * p.bm, rem = a.M - mfull, cus = device_cus();
        const int tn = (a.N + p.bn - 1) / p.bn, full = (mfull / p.bm) * tn, total = full + tn;
        if (mfull > 0 && rem > 0 && use_gemv_h16(rem, a.K) && cus > 0 &&
            (total + cus - 1) / cus > (full + cus - 1) / cus) {
            GemmH16Args m = a, t = a0;
            m.M = mfull;
            t.M = rem;
            const size_t xo = (size_t)mfull * a.K, yo = (size_t)mfull * a.N;
            if (t.x) t.x += xo;
            if (t.xf) t.xf += xo;
            if (t.resid) t.resid += yo;
            if (t.y) t.y += yo;
            if (t.y16) t.y16 += yo;
            const hipError_t e = dispatch_h16(p, m, s, nullptr);
            return e != hipSuccess ? e : launch_gemv_h16(t, s);
        }
    }
    return dispatch_h16(p, a, s, ln);
}

}  // namespace mgh
