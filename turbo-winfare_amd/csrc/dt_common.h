// Shared host/device helpers for the decode-tail kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tdt {

constexpr uint32_t kGroup = 64;          // quantisation group (src/cpu_reference.cpp:32)
constexpr uint32_t kTileRows = 64;       // vocabulary rows per tile = one wave64 of the GEMV
constexpr uint32_t kDigits = 6;          // signed 4-bit digit planes of the block-fp activations
constexpr uint32_t kDigitWordsPerChunk = kDigits * 4;  // 4 words (32 nibbles) per digit per chunk
constexpr uint32_t kMaxTopK = 256;       // src/sampling.cpp:15
constexpr uint32_t kFlagFullVocab = 1u;

// Per-64-id block summary written by every head-kernel epilogue.
struct BlockPartial {
    float max;       // block maximum after modifiers (-inf when every id is banned)
    uint32_t arg;    // lowest id holding the maximum
    float sumexp;    // sum exp(l - max) over the block (0 when max is -inf)
    float minf;      // smallest finite logit of the block (+inf when none)
};

// One sorted modifier entry (per row, unique id).
struct ModEntry {
    uint32_t id;
    uint32_t count;   // history occurrences
    float bias;       // summed bias (0 when none)
    uint32_t has_bias;
};

// Per-row parameters as the kernels see them.
struct DevRow {
    float temperature;
    float top_p;
    int32_t top_k;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    float u;            // uniform for the draw (ignored when injected uniforms are given)
    uint32_t flags;     // kFlagFullVocab
    uint32_t want;      // shortlist size: top_k, else 256, else vocab (full-vocab mode)
    uint32_t has_mods;  // bit 0: history counts (repetition / presence / frequency); bit 1: bias table
    uint32_t pad[2];
};

__host__ __device__ inline float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Order-preserving map from float to uint32 (larger float -> larger key). -0.0 is mapped to
// +0.0 first, because the reference compares logits with != / > (src/sampling.cpp:126-129),
// under which the two zeros are equal and ordered by index.
__host__ __device__ inline uint32_t float_key(float f) {
    if (f == 0.0f) f = 0.0f;
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__host__ __device__ inline float key_float(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}

// Philox4x32-10 (Salmon et al., SC'11). Returns the first output word.
__host__ __device__ inline uint32_t philox4x32_10_x(uint64_t counter, uint64_t seed) {
    uint32_t c0 = (uint32_t)counter, c1 = (uint32_t)(counter >> 32), c2 = 0u, c3 = 0u;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// ---- wave64 reductions (DPP/permute via __shfl_xor) ---------------------------------------
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ inline float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline uint32_t wave_min_u(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
}
// (value, index) argmax with ties to the lower index.
__device__ inline void wave_argmax(float& v, uint32_t& i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)i, o, 64);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
}

}  // namespace tdt
