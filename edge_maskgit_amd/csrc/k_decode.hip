// k_decode.hip — one step of MaskGIT iterative decoding on the device (gfx950), so the
// per-step logits never leave HBM.
//
// Semantics: the loop body of the reference's generate(), src/mg-generate.cpp:82-121, for B
// images at once, with each image's random stream being the reference's: std::mt19937_64
// seeded with that image's seed, read through std::uniform_real_distribution<double>, in the
// reference's call order (S categorical draws, then S Gumbel draws per step, :89-114).
//  * the engine is mt19937_64 as the C++ standard defines it ([rand.predef]: w=64, n=312,
//    m=156, r=31, a=0xB5026F5AA96619E9, tempering (u,d)=(29,0x5555555555555555),
//    (s,b)=(17,0x71D67FFFEDA60000), (t,c)=(37,0xFFF7EEE000000000), l=43, seeding multiplier
//    6364136223846793005). One workgroup per image holds the state in LDS; the twist runs in
//    three parallel phases (words [0,156) read only old words, words [156,311) read the new
//    word 156 places back, word 311 reads the new word 0) and the tempering of a whole
//    batch of outputs is one parallel pass.
//  * engine outputs become doubles as libstdc++'s generate_canonical<double,53> does for a
//    64-bit engine: x / 2^64 (x rounded to double, the division exact), with a result >= 1
//    replaced by the largest double below 1; U(a, b) = u * (b - a) + a.
//  * k_decode_sample: one wave per (image, position): softmax over the first CB logits in
//    the reference's fp32 order (max; e_v = exp(l_v - max); sum += e_v for v = 0, 1, ...;
//    p_v = e_v * (1 / sum)) and the categorical search as a sequential double cumsum. The
//    sequential parts walk lane values read with v_readlane, so every lane holds the same
//    running sums.
//  * k_decode_select: one workgroup per image: cosine schedule, confidence
//    log(p) + temp * (1 - ratio) * gumbel, the mask_len-th smallest confidence (the value
//    std::nth_element leaves there: a bitonic sort in LDS gives the same order statistic) and
//    the re-mask.
// exp/log/cos of fp32 values are evaluated in double and rounded once, i.e. correctly
// rounded fp32 results like the host libm's (which is correctly rounded except in rare
// last-bit cases). Floating-point contraction is off so a*b+c rounds twice as in the
// reference.
#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

constexpr int MT_N = 312, MT_M = 156;
constexpr uint64_t MT_A = 0xB5026F5AA96619E9ull;
constexpr uint64_t MT_UPPER = 0xFFFFFFFF80000000ull, MT_LOWER = 0x7FFFFFFFull;
constexpr int STATE_WORDS = MT_N + 1;   // state words + output index
constexpr int DEC_MAXC = 16;            // codebook <= 64 * 16
constexpr int SEL_T = 512;              // positions per image <= 512

__device__ __forceinline__ uint64_t mt_twist(uint64_t hi, uint64_t lo) {
    const uint64_t y = (hi & MT_UPPER) | (lo & MT_LOWER);
    return (y >> 1) ^ ((y & 1) ? MT_A : 0ull);
}

__device__ __forceinline__ uint64_t mt_temper(uint64_t y) {
    y ^= (y >> 29) & 0x5555555555555555ull;
    y ^= (y << 17) & 0x71D67FFFEDA60000ull;
    y ^= (y << 37) & 0xFFF7EEE000000000ull;
    return y ^ (y >> 43);
}

// std::mt19937_64::seed(s): x_0 = s, x_i = f * (x_{i-1} ^ (x_{i-1} >> 62)) + i. Serial
// recurrence, one thread per image; runs once per generation.
__global__ __launch_bounds__(64) void k_mt64_seed(int B, uint64_t* __restrict__ state) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    if (b >= B) return;
    uint64_t* mt = state + (size_t)b * STATE_WORDS;
    uint64_t x = mt[0];
    for (int i = 1; i < MT_N; i++) {
        x = 6364136223846793005ull * (x ^ (x >> 62)) + (uint64_t)i;
        mt[i] = x;
    }
    mt[MT_N] = MT_N;                     // first output twists
}

// n engine outputs per image into out[b][n]; one 256-thread workgroup per image.
__global__ __launch_bounds__(256) void k_mt64_draw(uint64_t* __restrict__ state, int n,
                                                   uint64_t* __restrict__ out) {
    __shared__ uint64_t mt[MT_N];
    const int b = blockIdx.x, t = threadIdx.x;
    uint64_t* g = state + (size_t)b * STATE_WORDS;
    for (int i = t; i < MT_N; i += 256) mt[i] = g[i];
    int idx = (int)g[MT_N];
    __syncthreads();
    uint64_t* o = out + (size_t)b * n;
    for (int done = 0; done < n;) {
        if (idx >= MT_N) {
            uint64_t a0 = 0, a1 = 0, a2 = 0, b1 = 0, n0 = 0;
            if (t < MT_M) {
                a0 = mt[t];
                a1 = mt[t + 1];
                a2 = mt[t + MT_M];
                if (t + MT_M + 1 < MT_N) b1 = mt[t + MT_M + 1];
            }
            __syncthreads();
            if (t < MT_M) {
                n0 = a2 ^ mt_twist(a0, a1);          // i = t, reads words i+1, i+156 (old)
                mt[t] = n0;
            }
            __syncthreads();
            if (t < MT_M) {                          // i = t + 156, reads new word i-156 = n0
                if (t + MT_M + 1 >= MT_N) b1 = mt[0];  // i = 311 pairs with the new word 0
                mt[t + MT_M] = n0 ^ mt_twist(a2, b1);
            }
            __syncthreads();
            idx = 0;
        }
        const int cnt = min(MT_N - idx, n - done);
        for (int j = t; j < cnt; j += 256) o[done + j] = mt_temper(mt[idx + j]);
        idx += cnt;
        done += cnt;
    }
    __syncthreads();
    for (int i = t; i < MT_N; i += 256) g[i] = mt[i];
    if (t == 0) g[MT_N] = (uint64_t)idx;
}

__device__ __forceinline__ double canonical(uint64_t x) {
    const double u = (double)x * 0x1p-64;
    return u >= 1.0 ? 0x1.fffffffffffffp-1 : u;
}

__device__ __forceinline__ float exp_f(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float log_f(float x) { return (float)log((double)x); }

__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// one wave per row (b, s) of logits [B*S][V]; the first CB = 64 * C entries are sampled
__global__ __launch_bounds__(256) void k_decode_sample(DecodeArgs a) {
#pragma clang fp contract(off)
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= a.B * a.S) return;                         // whole wave
    const int b = row / a.S, s = row - b * a.S;
    const float* L = a.logits + (size_t)row * a.V;
    const int C = a.CB >> 6;
    float e[DEC_MAXC];
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < DEC_MAXC; c++) {
        e[c] = c < C ? L[64 * c + lane] : -INFINITY;
        mx = fmaxf(mx, e[c]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < DEC_MAXC; c++) {
        if (c < C) {
            e[c] = exp_f(e[c] - mx);
#pragma unroll
            for (int l = 0; l < 64; l++) sum += lane_f(e[c], l);
        }
    }
    const float inv = (float)(1.0 / (double)sum);         // correctly rounded 1.f / sum
#pragma unroll
    for (int c = 0; c < DEC_MAXC; c++) e[c] = e[c] * inv;
    // first v with r <= p_0 + ... + p_v (double sums); v = CB-1 when none
    const double r = canonical(a.draws[(size_t)b * 2 * a.S + s]);
    double acc = 0.0;
    int sid = -1;
    float psid = 0.f;
#pragma unroll
    for (int c = 0; c < DEC_MAXC; c++) {
        if (c < C && sid < 0) {
            for (int l = 0; l < 64; l++) {
                const float p = lane_f(e[c], l);
                acc += (double)p;
                psid = p;
                if (r <= acc) {
                    sid = 64 * c + l;
                    break;
                }
            }
        }
    }
    if (sid < 0) sid = a.CB - 1;                          // psid already holds p_{CB-1}
    if (lane == 0) {
        const int32_t tk = a.tokens[row];
        const bool unknown = tk == a.mask_id;
        a.sampled[row] = unknown ? sid : tk;
        a.selp[row] = unknown ? psid : INFINITY;
    }
}

// one 512-thread workgroup per image (S <= 512)
__global__ __launch_bounds__(SEL_T) void k_decode_select(DecodeArgs a) {
#pragma clang fp contract(off)
    __shared__ float keys[SEL_T];
    __shared__ int n_unknown;
    const int b = blockIdx.x, t = threadIdx.x, S = a.S;
    const size_t base = (size_t)b * S;
    if (t == 0) n_unknown = 0;
    __syncthreads();
    const float ratio = (float)(a.step + 1) / (float)a.n_steps;
    const float temp = a.choice_temp * (1.f - ratio);
    int32_t smp = 0;
    float conf = INFINITY;
    if (t < S) {
        if (a.tokens[base + t] == a.mask_id) atomicAdd(&n_unknown, 1);
        smp = a.sampled[base + t];
        const double u = canonical(a.draws[(size_t)b * 2 * S + S + t]) * (1.0 - 1e-12) + 1e-12;
        const float gmb = (float)(-log(-log(u)));
        conf = log_f(a.selp[base + t]) + temp * gmb;
    }
    keys[t] = conf;                                       // padding (+inf) sorts last
    __syncthreads();
    for (int k = 2; k <= SEL_T; k <<= 1)                  // bitonic sort, ascending
        for (int j = k >> 1; j > 0; j >>= 1) {
            const int p = t ^ j;
            if (p > t) {
                const float x = keys[t], y = keys[p];
                if ((x > y) == ((t & k) == 0)) {
                    keys[t] = y;
                    keys[p] = x;
                }
            }
            __syncthreads();
        }
    const float half_pi = 3.14159265358979323846f / 2.f;
    const float mask_ratio = (float)cos((double)(half_pi * ratio));
    int mask_len = (int)floorf((float)a.n_tokens * mask_ratio);
    mask_len = max(1, min(mask_len, n_unknown - 1));
    const float cutoff = keys[mask_len];
    if (t < S) {
        a.result[base + t] = smp;
        a.tokens[base + t] = conf < cutoff ? a.mask_id : smp;
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

size_t decode_state_bytes(int B) { return (size_t)B * STATE_WORDS * 8; }

size_t decode_work_bytes(int B, int S) {
    // draws [B][2S] u64 | sampled [B][S] i32 | selp [B][S] f32
    return align256((size_t)B * 2 * S * 8) + 2 * align256((size_t)B * S * 4);
}

hipError_t launch_decode_seed(int B, void* state, hipStream_t s) {
    hipLaunchKernelGGL(k_mt64_seed, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, s, B,
                       (uint64_t*)state);
    return hipGetLastError();
}

hipError_t launch_decode_step(DecodeArgs a, void* state, void* work, hipStream_t s) {
    char* w = (char*)work;
    const size_t o1 = align256((size_t)a.B * 2 * a.S * 8);
    a.draws = (uint64_t*)w;
    a.sampled = (int32_t*)(w + o1);
    a.selp = (float*)(w + o1 + align256((size_t)a.B * a.S * 4));
    hipLaunchKernelGGL(k_mt64_draw, dim3((unsigned)a.B), dim3(256), 0, s, (uint64_t*)state,
                       2 * a.S, a.draws);
    hipLaunchKernelGGL(k_decode_sample, dim3((unsigned)((a.B * a.S + 3) / 4)), dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_decode_select, dim3((unsigned)a.B), dim3(SEL_T), 0, s, a);
    return hipGetLastError();
}

}  // namespace mgh
