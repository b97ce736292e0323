/* mg_oracle.c — CPU restatement of the reference hot path (TEST INFRASTRUCTURE ONLY).
 *
 * The checker for the HIP path; see mg_oracle.h for the usage rule. Compiled with
 * -O2 -ffp-contract=off (no FMA contraction), so every fp32 operation rounds exactly
 * where it is written. OpenMP only splits independent output rows; each output is
 * computed by one thread in a fixed order, so results do not depend on thread count.
 */
#include "mg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int mgo_version(void) { return 1; }

/* ------------------------------------------------------------------------------
 * binary16 conversion. Round-to-nearest-even on the 13 dropped mantissa bits, with
 * gradual underflow into subnormals and overflow to infinity at >= 65520.
 * ------------------------------------------------------------------------------ */
uint16_t mgo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                       /* normal half: |f| >= 2^-14 */
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t mant = ax & 0x7fffffu;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* carry may bump exponent */
        return (uint16_t)(sign | h);
    }
    if (ax <= 0x33000000u) return (uint16_t)sign;  /* |f| <= 2^-25 rounds to (signed) zero */
    /* subnormal half: value / 2^-24 = mant24 * 2^(e-126), shift = 126-e in [14, 24] */
    uint32_t e = ax >> 23;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float mgo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    float f;
    if (e == 0) {
        f = (float)m * 5.9604644775390625e-8f;       /* m * 2^-24, exact */
        memcpy(&x, &f, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &x, 4);
    return f;
}

void mgo_f32_to_f16_array(const float* x, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = mgo_f32_to_f16(x[i]);
}
void mgo_f16_to_f32_array(const uint16_t* h, float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = mgo_f16_to_f32(h[i]);
}
void mgo_round_f16_array(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = mgo_f16_to_f32(mgo_f32_to_f16(x[i]));
}

static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)(v & 0xff); p[1] = (uint8_t)(v >> 8); }

size_t mgo_q8_0_row_bytes(int64_t K) { return (size_t)(K / 32) * 34; }
size_t mgo_q4_k_row_bytes(int64_t K) { return (size_t)(K / 256) * 144; }

/* ------------------------------------------------------------------------------
 * Q8_0 encoder — tools/convert_to_gguf.py:109-124.
 *   amax = max|w| over the 32-block            (float32)
 *   d    = amax / 127                          (float32 division, :118)
 *   q    = clip(rint(w / (d>0 ? d : 1)), ±127) (half-to-even, :120)
 *   block = fp16(d) | 32 x int8                 (:122-123)
 * ------------------------------------------------------------------------------ */
void mgo_quantize_q8_0(const float* w, int64_t N, int64_t K, uint8_t* out) {
    const int64_t nb = K / 32;
    for (int64_t n = 0; n < N; n++) {
        for (int64_t b = 0; b < nb; b++) {
            const float* x = w + n * K + b * 32;
            uint8_t* blk = out + (n * nb + b) * 34;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) {
                float a = fabsf(x[i]);
                if (a > amax) amax = a;
            }
            float d = amax / 127.0f;
            float dsafe = d > 0.0f ? d : 1.0f;
            wr_u16(blk, mgo_f32_to_f16(d));
            for (int i = 0; i < 32; i++) {
                float q = rintf(x[i] / dsafe);
                if (q > 127.0f) q = 127.0f;
                if (q < -127.0f) q = -127.0f;
                blk[2 + i] = (uint8_t)(int8_t)q;
            }
        }
    }
}

/* ------------------------------------------------------------------------------
 * Q4_K encoder — tools/convert_to_gguf.py:68-106 (min/max quantizer, not ggml's search).
 * Per 256-super-block, 8 sub-blocks j of 32 (all float32):
 *   minv_j = max(0, -min_j); sc_j = (max_j+minv_j > 0) ? (max_j+minv_j)/15 : 0   (:77-79)
 *   d = max_j sc_j / 63 (or 0); dmin = max_j minv_j / 63 (or 0)                   (:80-81)
 *   scq_j = clip(round(sc_j/d), 0, 63); mq_j = clip(round(minv_j/dmin), 0, 63)    (:82-83)
 *   q = clip(round((w + dmin*mq_j) / (d*scq_j or 1)), 0, 15)                      (:84-87)
 * then the 6-bit packing (:89-94) and nibble packing (:96-98).
 * ------------------------------------------------------------------------------ */
void mgo_quantize_q4_k(const float* w, int64_t N, int64_t K, uint8_t* out) {
    const int64_t nsb = K / 256;
    for (int64_t n = 0; n < N; n++) {
        for (int64_t s = 0; s < nsb; s++) {
            const float* x = w + n * K + s * 256;
            uint8_t* blk = out + (n * nsb + s) * 144;
            float minv[8], sc[8];
            for (int j = 0; j < 8; j++) {
                float mn = x[j * 32], mx = x[j * 32];
                for (int l = 1; l < 32; l++) {
                    float v = x[j * 32 + l];
                    if (v < mn) mn = v;
                    if (v > mx) mx = v;
                }
                float nm = -mn;
                minv[j] = nm > 0.0f ? nm : 0.0f;
                float r = mx + minv[j];
                sc[j] = r > 0.0f ? r / 15.0f : 0.0f;
            }
            float scmax = sc[0], mnmax = minv[0];
            for (int j = 1; j < 8; j++) {
                if (sc[j] > scmax) scmax = sc[j];
                if (minv[j] > mnmax) mnmax = minv[j];
            }
            float d = scmax > 0.0f ? scmax / 63.0f : 0.0f;
            float dmn = mnmax > 0.0f ? mnmax / 63.0f : 0.0f;
            uint8_t scq[8], mq[8];
            float asc[8], amin[8];
            for (int j = 0; j < 8; j++) {
                float a = d > 0.0f ? rintf(sc[j] / d) : 0.0f;
                float b = dmn > 0.0f ? rintf(minv[j] / dmn) : 0.0f;
                a = a < 0.0f ? 0.0f : (a > 63.0f ? 63.0f : a);
                b = b < 0.0f ? 0.0f : (b > 63.0f ? 63.0f : b);
                scq[j] = (uint8_t)a;
                mq[j] = (uint8_t)b;
                asc[j] = d * (float)scq[j];
                amin[j] = dmn * (float)mq[j];
            }
            uint8_t q[8][32];
            for (int j = 0; j < 8; j++) {
                float safe = asc[j] > 0.0f ? asc[j] : 1.0f;
                for (int l = 0; l < 32; l++) {
                    float v = rintf((x[j * 32 + l] + amin[j]) / safe);
                    v = v < 0.0f ? 0.0f : (v > 15.0f ? 15.0f : v);
                    q[j][l] = (uint8_t)v;
                }
            }
            wr_u16(blk + 0, mgo_f32_to_f16(d));
            wr_u16(blk + 2, mgo_f32_to_f16(dmn));
            uint8_t* scales = blk + 4;
            for (int j = 0; j < 4; j++) {
                scales[j] = (uint8_t)((scq[j] & 63) | (((scq[j + 4] >> 4) & 3) << 6));
                scales[j + 4] = (uint8_t)((mq[j] & 63) | (((mq[j + 4] >> 4) & 3) << 6));
                scales[j + 8] = (uint8_t)((scq[j + 4] & 0xF) | ((mq[j + 4] & 0xF) << 4));
            }
            uint8_t* qs = blk + 16;
            for (int g = 0; g < 4; g++)
                for (int l = 0; l < 32; l++)
                    qs[g * 32 + l] = (uint8_t)((q[2 * g][l] & 0xF) | ((q[2 * g + 1][l] & 0xF) << 4));
        }
    }
}

/* ggml get_scale_min_k4 — mg-opencl.cpp:178-184 */
void mgo_q4k_scale_min(const uint8_t* s, int j, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* nibble value of sub-block j, element l (mg-opencl.cpp:259-260, :529-532) */
static inline int q4k_nib(const uint8_t* blk, int j, int l) {
    uint8_t b = blk[16 + (j >> 1) * 32 + l];
    return (j & 1) ? (b >> 4) : (b & 0xF);
}

/* DEQ_Q8 (mg-opencl.cpp:386-387): fp16(d) * q;  deq_q4k_elem (:252-262): d*sc*q - dmin*m */
void mgo_dequant(int wtype, const uint8_t* w, int64_t N, int64_t K, float* out) {
    if (wtype == MGO_WTYPE_Q8_0) {
        const int64_t nb = K / 32;
        for (int64_t n = 0; n < N; n++)
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t* blk = w + (n * nb + b) * 34;
                float d = mgo_f16_to_f32(rd_u16(blk));
                for (int i = 0; i < 32; i++) out[n * K + b * 32 + i] = d * (float)(int8_t)blk[2 + i];
            }
    } else if (wtype == MGO_WTYPE_Q4_K) {
        const int64_t nsb = K / 256;
        for (int64_t n = 0; n < N; n++)
            for (int64_t s = 0; s < nsb; s++) {
                const uint8_t* blk = w + (n * nsb + s) * 144;
                float d = mgo_f16_to_f32(rd_u16(blk));
                float dmin = mgo_f16_to_f32(rd_u16(blk + 2));
                for (int j = 0; j < 8; j++) {
                    uint8_t sc, m;
                    mgo_q4k_scale_min(blk + 4, j, &sc, &m);
                    for (int l = 0; l < 32; l++) {
                        float q = (float)q4k_nib(blk, j, l);
                        out[n * K + s * 256 + j * 32 + l] = d * (float)sc * q - dmin * (float)m;
                    }
                }
            }
    } else if (wtype == MGO_WTYPE_F32) {
        memcpy(out, w, (size_t)(N * K) * sizeof(float));
    }
}

/* ------------------------------------------------------------------------------
 * k_quantize_q8 — mg-opencl.cpp:424-434. Per (m, 32-block):
 *   amax = max|x|; d = amax/127; id = d>0 ? 1/d : 0; dx = d; q = round(x*id)
 * OpenCL round() is half-away-from-zero, i.e. C roundf().
 * ------------------------------------------------------------------------------ */
void mgo_quantize_act_q8(const float* x, int64_t M, int64_t K, int8_t* qx, float* dx, int32_t* sx) {
    const int64_t nb = K / 32;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++) {
        for (int64_t b = 0; b < nb; b++) {
            const float* r = x + m * K + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(r[i]));
            float d = amax / 127.0f;
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            dx[m * nb + b] = d;
            int32_t s = 0;
            for (int i = 0; i < 32; i++) {
                int8_t q = (int8_t)roundf(r[i] * id);
                qx[m * K + b * 32 + i] = q;
                s += q;
            }
            if (sx) sx[m * nb + b] = s;
        }
    }
}

/* int32 dot of one weight block with one activation block */
static inline int32_t dot_q8_block(const uint8_t* blk, const int8_t* a) {
    int32_t s = 0;
    for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)blk[2 + i] * (int32_t)a[i];
    return s;
}
static inline int32_t dot_q4k_sub(const uint8_t* sblk, int j, const int8_t* a) {
    int32_t s = 0;
    for (int l = 0; l < 32; l++) s += q4k_nib(sblk, j, l) * (int32_t)a[l];
    return s;
}

void mgo_block_dots(int wtype, const uint8_t* w, int64_t N, int64_t K,
                    const int8_t* qx, int64_t M, int32_t* out) {
    const int64_t nb = K / 32;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++)
            for (int64_t t = 0; t < nb; t++) {
                const int8_t* a = qx + m * K + t * 32;
                int32_t v;
                if (wtype == MGO_WTYPE_Q8_0) v = dot_q8_block(w + (n * nb + t) * 34, a);
                else v = dot_q4k_sub(w + (n * (K / 256) + t / 8) * 144, (int)(t & 7), a);
                out[(m * N + n) * nb + t] = v;
            }
}

/* mg_act — mg-opencl.cpp:36-40 / mg-cpu.cpp:64-66 */
float mgo_act(float v, int act) {
    if (act == 1) return 0.5f * v * (1.0f + erff(v * 0.70710678f));
    if (act == 2) return v / (1.0f + expf(-v));
    return v;
}

/* epilogue order, mg-opencl.cpp:485-491: +bias -> act -> +resid */
static inline float epilogue(float v, const float* bias, int act, const float* resid,
                             int64_t m, int64_t n, int64_t N) {
    if (bias) v += bias[n];
    v = mgo_act(v, act);
    if (resid) v += resid[m * N + n];
    return v;
}

/* ------------------------------------------------------------------------------
 * int8-dot GEMMs. Blocks t are visited in order 0..K/32-1 per output (the K loop of
 * mg-opencl.cpp:449 / :513), each contributing
 *   Q8_0 (:480):  acc += (dw * dx) * idot
 *   Q4_K (:577):  acc += (d*sc * dx) * idot - (dmin*m * dx) * sum(qx)
 * with dw = fp16(d) of the weight block and dx the activation block scale.
 * ------------------------------------------------------------------------------ */
void mgo_gemm_q_i8(int wtype, const uint8_t* w, int64_t N, int64_t K,
                   const int8_t* qx, const float* dx, int64_t M,
                   const float* bias, int act, const float* resid, float* y) {
    const int64_t nb = K / 32;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++) {
        int32_t* sumx = (int32_t*)malloc((size_t)nb * sizeof(int32_t));
        for (int64_t t = 0; t < nb; t++) {
            int32_t s = 0;
            for (int i = 0; i < 32; i++) s += qx[m * K + t * 32 + i];
            sumx[t] = s;
        }
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int64_t t = 0; t < nb; t++) {
                const int8_t* a = qx + m * K + t * 32;
                float dxm = dx[m * nb + t];
                if (wtype == MGO_WTYPE_Q8_0) {
                    const uint8_t* blk = w + (n * nb + t) * 34;
                    float dw = mgo_f16_to_f32(rd_u16(blk));
                    int32_t idot = dot_q8_block(blk, a);
                    float s = dw * dxm;
                    float p = s * (float)idot;
                    acc = acc + p;
                } else {
                    const uint8_t* sblk = w + (n * (K / 256) + t / 8) * 144;
                    int j = (int)(t & 7);
                    float d = mgo_f16_to_f32(rd_u16(sblk));
                    float dmin = mgo_f16_to_f32(rd_u16(sblk + 2));
                    uint8_t sc, mm;
                    mgo_q4k_scale_min(sblk + 4, j, &sc, &mm);
                    float scl = d * (float)sc;
                    float mnl = dmin * (float)mm;
                    int32_t idot = dot_q4k_sub(sblk, j, a);
                    float p1 = (scl * dxm) * (float)idot;
                    float p2 = (mnl * dxm) * (float)sumx[t];
                    acc = acc + (p1 - p2);
                }
            }
            y[m * N + n] = epilogue(acc, bias, act, resid, m, n, N);
        }
        free(sumx);
    }
}

/* k_mul_mat — mg-cpu.cpp:48-72: acc += w[k,n]*x[k,m] for k = 0..K-1, then epilogue */
void mgo_gemm_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M,
                  const float* bias, int act, const float* resid, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            const float* wr = w + n * K;
            const float* xr = x + m * K;
            for (int64_t k = 0; k < K; k++) acc = acc + wr[k] * xr[k];
            y[m * N + n] = epilogue(acc, bias, act, resid, m, n, N);
        }
}

void mgo_gemm_q_deq_f32(int wtype, const uint8_t* w, int64_t N, int64_t K, const float* x,
                        int64_t M, const float* bias, int act, const float* resid, float* y) {
    float* wf = (float*)malloc((size_t)(N * K) * sizeof(float));
    mgo_dequant(wtype, w, N, K, wf);
    mgo_gemm_f32(wf, N, K, x, M, bias, act, resid, y);
    free(wf);
}

/* ------------------------------------------------------------------------------
 * LayerNorm + affine — mg-cpu.cpp:105-121 (k_norm) then :249-261 (affine):
 *   mean, var in double; inv = 1/sqrtf((float)var + eps);
 *   y = ((float)(x - mean)) * inv;  y = y*gamma + beta
 * ------------------------------------------------------------------------------ */
void mgo_layernorm_affine(const float* x, const float* gamma, const float* beta,
                          int64_t rows, int64_t D, float eps, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* a = x + r * D;
        double mean = 0.0;
        for (int64_t k = 0; k < D; k++) mean += a[k];
        mean /= (double)D;
        double var = 0.0;
        for (int64_t k = 0; k < D; k++) {
            double d = a[k] - mean;
            var += d * d;
        }
        var /= (double)D;
        float inv = 1.0f / sqrtf((float)var + eps);
        for (int64_t k = 0; k < D; k++) {
            float v = ((float)(a[k] - mean)) * inv;
            if (gamma && beta) v = v * gamma[k] + beta[k];
            y[r * D + k] = v;
        }
    }
}

/* ------------------------------------------------------------------------------
 * Attention — mg-cpu.cpp:211-239. Per (b, h, query s):
 *   score_t = (sum_d q[d]*k[d,t]) * scale; mx = max; p_t = exp(score_t - mx); sum = sum p;
 *   o[d] = sum_t (p_t * (1/sum)) * v[d,t]
 * With f16kv the inputs are first rounded to fp16 (k_flash_attention_h keeps Q row and
 * K/V tiles in half, mg-opencl.cpp:877, :893-894; all math stays fp32).
 * ------------------------------------------------------------------------------ */
void mgo_attention(const float* q, const float* k, const float* v, const int64_t st[4],
                   int64_t D, int64_t S, int64_t H, int64_t B, float scale, int f16kv, float* o) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < H; h++) {
            float* sc = (float*)malloc((size_t)S * sizeof(float));
            float* qr = (float*)malloc((size_t)D * sizeof(float));
            const int64_t base = b * st[3] + h * st[2];
#define LD(p, d, t) (f16kv ? mgo_f16_to_f32(mgo_f32_to_f16((p)[base + (t) * st[1] + (d) * st[0]])) \
                           : (p)[base + (t) * st[1] + (d) * st[0]])
            for (int64_t s = 0; s < S; s++) {
                for (int64_t d = 0; d < D; d++) qr[d] = LD(q, d, s);
                float mx = -INFINITY;
                for (int64_t t = 0; t < S; t++) {
                    float a = 0.0f;
                    for (int64_t d = 0; d < D; d++) a = a + qr[d] * LD(k, d, t);
                    a = a * scale;
                    sc[t] = a;
                    if (a > mx) mx = a;
                }
                float sum = 0.0f;
                for (int64_t t = 0; t < S; t++) {
                    sc[t] = expf(sc[t] - mx);
                    sum = sum + sc[t];
                }
                float inv = 1.0f / sum;
                for (int64_t d = 0; d < D; d++) {
                    float acc = 0.0f;
                    for (int64_t t = 0; t < S; t++) acc = acc + (sc[t] * inv) * LD(v, d, t);
                    o[((b * H + h) * S + s) * D + d] = acc;
                }
            }
#undef LD
            free(sc);
            free(qr);
        }
}

/* k_get_rows — mg-cpu.cpp:74-86: negative ids wrap (r += R) */
void mgo_get_rows(const float* a, int64_t E, int64_t R, const int32_t* ids, int64_t n, float* o) {
    for (int64_t i = 0; i < n; i++) {
        int64_t r = ids[i];
        if (r < 0) r += R;
        memcpy(o + i * E, a + r * E, (size_t)E * sizeof(float));
    }
}

/* {D,S,H,B} contiguous -> {D,H,S,B} contiguous */
void mgo_merge_heads(const float* a, int64_t D, int64_t S, int64_t H, int64_t B, float* o) {
    for (int64_t b = 0; b < B; b++)
        for (int64_t s = 0; s < S; s++)
            for (int64_t h = 0; h < H; h++)
                memcpy(o + ((b * S + s) * H + h) * D, a + ((b * H + h) * S + s) * D,
                       (size_t)D * sizeof(float));
}

/* ------------------------------------------------------------------------------
 * VQGAN int8 conv — k_quantize_conv_w and k_conv2d_i8, mg-opencl.cpp:598-664.
 * Weights: per (oc, 32-block b of k), k = (ic*KH + kh)*KW + kw the kernel's own order,
 *   amax over the block's min(32, K - 32b) values; d = amax/127; id = d>0 ? 1/d : 0;
 *   q = round(w*id) (half away from zero); codes past K are 0. (The reference writes 32 codes
 *   per block from oc*K + 32b, so for K % 32 != 0 its last block overruns into the next
 *   channel's codes; here each channel's row is padded to nb*32 — the two agree for
 *   K % 32 == 0, every convolution of the decoder.)
 * Conv: for each image n, output pixel p and block b: the 32 im2col values
 *   v[i] = in[n][ic][oh*stride - pad + kh][ow*stride - pad + kw] of k = 32b + i (0 outside the
 *   image or past K) are quantized like k_quantize_q8 (dx, qx); idot = sum qx*qw (int32);
 *   acc = acc + (dx*dw)*(float)idot, blocks in order, each operation rounded to fp32 (the
 *   expression `dcm*dwl[nL]*(float)idot` evaluated as written, :651).
 * ------------------------------------------------------------------------------ */
void mgo_conv_quant_w(const float* ker, int64_t OC, int64_t K, int8_t* qw, float* dw) {
    const int64_t nb = (K + 31) / 32;
    for (int64_t oc = 0; oc < OC; oc++)
        for (int64_t b = 0; b < nb; b++) {
            const int64_t k0 = 32 * b, n = K - k0 < 32 ? K - k0 : 32;
            const float* w = ker + oc * K + k0;
            float amax = 0.0f;
            for (int64_t i = 0; i < n; i++) amax = fmaxf(amax, fabsf(w[i]));
            const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
            dw[oc * nb + b] = d;
            for (int64_t i = 0; i < 32; i++) qw[oc * nb * 32 + k0 + i] = i < n ? (int8_t)roundf(w[i] * id) : 0;
        }
}

void mgo_conv2d_i8(const float* in, int64_t IW, int64_t IH, int64_t IC, int64_t N, const int8_t* qw,
                   const float* dw, int64_t KW, int64_t KH, int64_t OC, int stride, int pad, float* out) {
    const int64_t OW = (IW + 2 * pad - KW) / stride + 1, OH = (IH + 2 * pad - KH) / stride + 1;
    const int64_t K = IC * KH * KW, nb = (K + 31) / 32, M = OW * OH;
#pragma omp parallel for schedule(static)
    for (int64_t np = 0; np < N * M; np++) {
        const int64_t n = np / M, p = np % M, ow = p % OW, oh = p / OW;
        float v[32];
        int8_t qx[32];
        float* o = out + n * OC * M + p;
        for (int64_t oc = 0; oc < OC; oc++) o[oc * M] = 0.0f;
        for (int64_t b = 0; b < nb; b++) {
            float amax = 0.0f;
            for (int64_t i = 0; i < 32; i++) {
                const int64_t k = 32 * b + i;
                float x = 0.0f;
                if (k < K) {
                    const int64_t kw = k % KW, t = k / KW, kh = t % KH, ic = t / KH;
                    const int64_t ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                    if (ih >= 0 && ih < IH && iw >= 0 && iw < IW) x = in[((n * IC + ic) * IH + ih) * IW + iw];
                }
                v[i] = x;
                amax = fmaxf(amax, fabsf(x));
            }
            const float d = amax / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
            for (int64_t i = 0; i < 32; i++) qx[i] = (int8_t)roundf(v[i] * id);
            for (int64_t oc = 0; oc < OC; oc++) {
                const int8_t* w = qw + oc * nb * 32 + 32 * b;
                int32_t idot = 0;
                for (int64_t i = 0; i < 32; i++) idot += (int32_t)qx[i] * (int32_t)w[i];
                const float s = d * dw[oc * nb + b];
                o[oc * M] = o[oc * M] + s * (float)idot;
            }
        }
    }
}
