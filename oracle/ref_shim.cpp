// C-ABI wrappers around the reference's own sampling code, so the oracle's restatement can be
// checked against the real thing. TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile (target
// `ref`) together with src/sampling.cpp from the reference checkout, into oracle/_ref/.
// Nothing from the reference is copied here: this file only includes its public header.
#include "gturbo/sampling.hpp"

#include <cstring>
#include <exception>
#include <vector>

namespace {
gturbo::SamplingParams make(float t, float top_p, int top_k, float pen, int has_seed,
                            unsigned long long seed) {
    gturbo::SamplingParams p;
    p.temperature = t;
    p.top_p = top_p;
    p.top_k = top_k;
    p.repetition_penalty = pen;
    p.has_seed = has_seed != 0;
    p.seed = seed;
    return p;
}
}  // namespace

extern "C" {

// src/sampling.cpp:32-54. Returns 1 when accepted, 0 when it throws.
int ref_validate_sampling(float t, float top_p, int top_k, float pen) {
    try {
        gturbo::validate_sampling(make(t, top_p, top_k, pen, 0, 0));
        return 1;
    } catch (const std::exception&) {
        return 0;
    }
}

unsigned long long ref_splitmix64(unsigned long long x) { return gturbo::splitmix64(x); }

unsigned long long ref_seed_for(int has_seed, unsigned long long seed, int position) {
    return gturbo::seed_for(make(0.7f, 1.0f, 0, 1.0f, has_seed, seed), position);
}

void ref_apply_repetition_penalty(float* logits, unsigned vocab, const unsigned* history,
                                  unsigned long long n, float penalty, float softcap) {
    std::vector<uint32_t> h(history, history + n);
    gturbo::apply_repetition_penalty(logits, vocab, h, penalty, softcap);
}

// src/sampling.cpp:92-169. Returns the token, or 0xFFFFFFFF when it throws.
unsigned ref_sample_token(const float* logits, unsigned vocab, float t, float top_p, int top_k,
                          float pen, unsigned long long seed) {
    try {
        return gturbo::sample_token(logits, vocab, make(t, top_p, top_k, pen, 1, 0), seed);
    } catch (const std::exception&) {
        return 0xFFFFFFFFu;
    }
}

}  // extern "C"
