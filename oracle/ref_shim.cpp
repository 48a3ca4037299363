// oracle/ref_shim.cpp -- C entry points over the reference's own header-only sampling, RNG
// and delay-pattern code, compiled straight from the reference sources (no copy): the
// headers src/mg/sampling.h, src/rng.h and src/mg/pattern.h need only the C++ standard
// library. TEST INFRASTRUCTURE: built into oracle/_ref/ to pin the C oracle against the
// real thing; nothing in the product loads it.
#include "mg/pattern.h"
#include "mg/sampling.h"
#include "rng.h"

#include <cstring>
#include <vector>

extern "C" {

int refx_argmax(const float* logits, int n) { return ac::argmax_token(logits, n); }

void refx_softmax_into(const float* logits, int n, float temperature, float* probs) {
    std::vector<float> p;
    ac::softmax_into(logits, n, temperature, p);
    std::memcpy(probs, p.data(), sizeof(float) * (size_t)n);
}

void refx_top_k_filter(float* probs, int n, int k) {
    std::vector<float> p(probs, probs + n);
    ac::top_k_filter(p, k);
    std::memcpy(probs, p.data(), sizeof(float) * (size_t)n);
}

// Draws `draws` tokens from one logits row with a fresh Rng(seed), as sample_top_k does.
void refx_sample_top_k_seq(const float* logits, int n, int k, float temperature, unsigned long long seed,
                           int draws, int* out) {
    ac::Rng rng(seed);
    std::vector<float> scratch;
    for (int i = 0; i < draws; ++i) out[i] = ac::sample_top_k(logits, n, k, temperature, rng, scratch);
}

// One sample per row over `rows` rows sharing one Rng(seed) (the generation loop's order).
void refx_sample_rows(const float* logits, int rows, int n, int k, float temperature, unsigned long long seed,
                      int* out) {
    ac::Rng rng(seed);
    std::vector<float> scratch;
    for (int r = 0; r < rows; ++r)
        out[r] = ac::sample_top_k(logits + (size_t)r * n, n, k, temperature, rng, scratch);
}

void refx_rng_uniforms(unsigned long long seed, int n, float* out) {
    ac::Rng rng(seed);
    for (int i = 0; i < n; ++i) out[i] = rng.uniform();
}

void refx_rng_raw(unsigned long long seed, int n, unsigned int* out) {
    ac::Rng rng(seed);
    for (int i = 0; i < n; ++i) out[i] = (unsigned int)rng.g();
}

int refx_pattern_steps(int n_q, int timesteps) {
    std::vector<int> d((size_t)n_q);
    for (int i = 0; i < n_q; ++i) d[(size_t)i] = i;
    return ac::DelayPattern(d, timesteps).steps();
}

void refx_build_pattern(int n_q, int timesteps, const int* codes, int special, int* seq) {
    std::vector<int> d((size_t)n_q);
    for (int i = 0; i < n_q; ++i) d[(size_t)i] = i;
    ac::DelayPattern p(d, timesteps);
    std::vector<int32_t> s = ac::build_pattern_sequence(p, codes, special);
    std::memcpy(seq, s.data(), s.size() * sizeof(int32_t));
}

void refx_revert_pattern(int n_q, int timesteps, const int* seq, int special, int* codes) {
    std::vector<int> d((size_t)n_q);
    for (int i = 0; i < n_q; ++i) d[(size_t)i] = i;
    ac::DelayPattern p(d, timesteps);
    std::vector<int32_t> c = ac::revert_pattern_sequence(p, seq, special);
    std::memcpy(codes, c.data(), c.size() * sizeof(int32_t));
}

void refx_pattern_mask(int n_q, int timesteps, unsigned char* mask) {
    std::vector<int> d((size_t)n_q);
    for (int i = 0; i < n_q; ++i) d[(size_t)i] = i;
    ac::DelayPattern p(d, timesteps);
    std::vector<uint8_t> m = ac::pattern_mask(p);
    std::memcpy(mask, m.data(), m.size());
}

int refx_first_step_with_timestep(int n_q, int timesteps, int t) {
    std::vector<int> d((size_t)n_q);
    for (int i = 0; i < n_q; ++i) d[(size_t)i] = i;
    try { return ac::DelayPattern(d, timesteps).first_step_with_timestep(t); } catch (...) { return -1; }
}

}  // extern "C"
