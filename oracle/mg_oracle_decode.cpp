// mg_oracle_decode.cpp — CPU restatement of one iterative-decoding step (TEST INFRASTRUCTURE
// ONLY; only tests/ load it through oracle/__init__.py).
//
// Follows the reference's generate() loop body, src/mg-generate.cpp:82-121, per image:
//   for every position s: softmax over the first CB logits (fp32, sequential sum), one
//     categorical draw u ~ U(0,1) searched by a sequential double cumsum (:31-36, :90-97);
//     unknown (mask) positions take the sample and its probability, known ones keep their
//     token with confidence +inf (:98-100);
//   cosine schedule: mask_ratio = cos(pi/2 * (step+1)/steps), mask_len =
//     clamp(floor(n_tokens * mask_ratio), 1, n_unknown - 1) (:104-110);
//   conf_s = log(p_s) + temp * (1 - ratio) * gumbel_s with gumbel = -log(-log(U(1e-12, 1)))
//     (:26-29, :112-114); positions whose conf is below the mask_len-th smallest value are
//     re-masked (:115-119).
// The random numbers are drawn from std::mt19937_64 through std::uniform_real_distribution
// <double> exactly as the reference does (same library, same call order: S categorical draws,
// then S Gumbel draws per step), so this oracle reproduces the reference's stream; image b
// uses seeds[b] and starts after `draws_before` draws (2*S per completed step).
#include <cmath>
#include <cstdint>
#include <random>
#include <vector>
#include <algorithm>

namespace {

float gumbel(std::mt19937_64& rng) {
    std::uniform_real_distribution<double> u(1e-12, 1.0);
    return (float)(-std::log(-std::log(u(rng))));
}

int sample_categorical(const float* probs, int n, std::mt19937_64& rng) {
    std::uniform_real_distribution<double> u(0.0, 1.0);
    const double r = u(rng);
    double acc = 0.0;
    for (int i = 0; i < n; i++) {
        acc += probs[i];
        if (r <= acc) return i;
    }
    return n - 1;
}

}  // namespace

extern "C" {

// n outputs of std::mt19937_64(seed) (engine known-answer checks)
void mgo_mt64_draws(uint64_t seed, int64_t n, uint64_t* out) {
    std::mt19937_64 g(seed);
    for (int64_t i = 0; i < n; i++) out[i] = g();
}

// n draws of std::uniform_real_distribution<double>(a, b) over std::mt19937_64(seed)
void mgo_uniform_draws(uint64_t seed, double a, double b, int64_t n, double* out) {
    std::mt19937_64 g(seed);
    std::uniform_real_distribution<double> u(a, b);
    for (int64_t i = 0; i < n; i++) out[i] = u(g);
}

// One decoding step for B images. logits [B][S][V]; tokens [B][S] in/out; result [B][S]
// receives the step's samples before re-masking (the reference's `result`).
void mgo_decode_step(const float* logits, int B, int S, int V, int CB, int mask_id, int n_tokens,
                     int step, int n_steps, float choice_temp, const uint64_t* seeds,
                     int64_t draws_before, int32_t* tokens, int32_t* result) {
    std::vector<float> probs((size_t)CB), selp((size_t)S), conf((size_t)S);
    std::vector<int32_t> sampled((size_t)S);
    for (int b = 0; b < B; b++) {
        std::mt19937_64 rng(seeds[b]);
        rng.discard((unsigned long long)draws_before);
        int32_t* tok = tokens + (size_t)b * S;
        for (int s = 0; s < S; s++) {
            const float* row = logits + ((size_t)b * S + s) * V;
            float mx = -INFINITY;
            for (int v = 0; v < CB; v++) mx = std::fmax(mx, row[v]);
            float sum = 0.f;
            for (int v = 0; v < CB; v++) {
                const float e = std::exp(row[v] - mx);
                probs[v] = e;
                sum += e;
            }
            const float inv = 1.f / sum;
            for (int v = 0; v < CB; v++) probs[v] *= inv;
            const int sid = sample_categorical(probs.data(), CB, rng);
            const bool unknown = tok[s] == mask_id;
            sampled[s] = unknown ? sid : tok[s];
            selp[s] = unknown ? probs[sid] : INFINITY;
        }
        for (int s = 0; s < S; s++) result[(size_t)b * S + s] = sampled[s];
        const float ratio = (float)(step + 1) / n_steps;
        const float mask_ratio = std::cos((float)M_PI / 2.f * ratio);
        int n_unknown = 0;
        for (int s = 0; s < S; s++) n_unknown += tok[s] == mask_id;
        int mask_len = (int)std::floor(n_tokens * mask_ratio);
        mask_len = std::max(1, std::min(mask_len, n_unknown - 1));
        const float temp = choice_temp * (1.f - ratio);
        for (int s = 0; s < S; s++) conf[s] = std::log(selp[s]) + temp * gumbel(rng);
        std::vector<float> sorted(conf);
        std::nth_element(sorted.begin(), sorted.begin() + mask_len, sorted.end());
        const float cutoff = sorted[mask_len];
        for (int s = 0; s < S; s++) tok[s] = conf[s] < cutoff ? mask_id : sampled[s];
    }
}

}  // extern "C"
