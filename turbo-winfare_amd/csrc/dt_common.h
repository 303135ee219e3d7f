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
    float smax;      // second-largest logit of the block, counting repeats (-inf when none)
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

// ---- wave64 cross-lane primitives ---------------------------------------------------------
// Reductions run on the VALU through DPP: quad_perm [1,0,3,2] and [2,3,0,1], then row_ror:4 and
// row_ror:8, leave every lane of a 16-lane row holding the row's result; v_readlane of lanes
// 0, 16, 32 and 48 combines the four rows into a wave-uniform value. Scans use row_shr:1/2/4/8
// (zero fill at the row start) and add the totals of the lower rows read from lanes 15, 31, 47.
// No LDS permute is involved, so a reduction costs a few dozen cycles rather than six
// dependent LDS round trips. Every lane of the wave must be active.
namespace dpp {
constexpr int kXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kRor4 = 0x124;        // row_ror:4
constexpr int kRor8 = 0x128;        // row_ror:8 (= xor 8 within a row)
constexpr int kHalfMirror = 0x141;  // row_half_mirror: lane i <-> 7 - i within each 8 lanes
constexpr int kShr1 = 0x111, kShr2 = 0x112, kShr4 = 0x114, kShr8 = 0x118;  // row_shr:n
}  // namespace dpp

template <int C>
__device__ inline uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, C, 0xF, 0xF, true);
}
template <int C>
__device__ inline float dpp_mov(float v) { return __uint_as_float(dpp_mov<C>(__float_as_uint(v))); }
template <int C>
__device__ inline int dpp_mov(int v) { return (int)dpp_mov<C>((uint32_t)v); }
template <int C>
__device__ inline unsigned long long dpp_mov(unsigned long long v) {
    const uint32_t lo = dpp_mov<C>((uint32_t)v), hi = dpp_mov<C>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
template <int C>
__device__ inline double dpp_mov(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = dpp_mov<C>((uint32_t)u), hi = dpp_mov<C>((uint32_t)(u >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ inline uint32_t lane_read(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ inline int lane_read(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ inline float lane_read(float v, int l) { return __uint_as_float(lane_read(__float_as_uint(v), l)); }
__device__ inline unsigned long long lane_read(unsigned long long v, int l) {
    return ((unsigned long long)lane_read((uint32_t)(v >> 32), l) << 32) | lane_read((uint32_t)v, l);
}
__device__ inline double lane_read(double v, int l) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = lane_read((uint32_t)u, l), hi = lane_read((uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// op over the wave; the result is the same in every lane.
template <class T, class Op>
__device__ inline T wave_reduce(T v, Op op) {
    v = op(v, dpp_mov<dpp::kXor1>(v));
    v = op(v, dpp_mov<dpp::kXor2>(v));
    v = op(v, dpp_mov<dpp::kRor4>(v));
    v = op(v, dpp_mov<dpp::kRor8>(v));
    return op(op(lane_read(v, 0), lane_read(v, 16)), op(lane_read(v, 32), lane_read(v, 48)));
}

__device__ inline float wave_max(float v) { return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); }); }
__device__ inline float wave_min(float v) { return wave_reduce(v, [](float a, float b) { return fminf(a, b); }); }
__device__ inline float wave_sum(float v) { return wave_reduce(v, [](float a, float b) { return a + b; }); }
__device__ inline double wave_sum_d(double v) { return wave_reduce(v, [](double a, double b) { return a + b; }); }
__device__ inline int wave_sum_i(int v) { return wave_reduce(v, [](int a, int b) { return a + b; }); }
__device__ inline uint32_t wave_min_u(uint32_t v) { return wave_reduce(v, [](uint32_t a, uint32_t b) { return min(a, b); }); }
__device__ inline uint32_t wave_max_u(uint32_t v) { return wave_reduce(v, [](uint32_t a, uint32_t b) { return max(a, b); }); }

// (value, index) argmax with ties to the lower index; the result is the same in every lane.
// Branch-free: one 64-bit key per lane, the order-preserving value key above ~index, so a plain
// maximum keeps the larger value and, among equal values, the lower index. -0.0 and +0.0 compare
// equal (both map to the key of +0.0, which is what the reduction returns); inputs are NaN-free.
__device__ inline void wave_argmax(float& v, uint32_t& i) {
    unsigned long long k = ((unsigned long long)float_key(v) << 32) | (uint32_t)~i;
    k = wave_reduce(k, [](unsigned long long a, unsigned long long b) { return a > b ? a : b; });
    v = key_float((uint32_t)(k >> 32));
    i = ~(uint32_t)k;
}

// Inclusive prefix sum over the wave in lane order.
template <typename T>
__device__ inline T wave_incl_scan(T v, uint32_t lane) {
    v += dpp_mov<dpp::kShr1>(v);
    v += dpp_mov<dpp::kShr2>(v);
    v += dpp_mov<dpp::kShr4>(v);
    v += dpp_mov<dpp::kShr8>(v);
    const T r0 = lane_read(v, 15), r1 = lane_read(v, 31), r2 = lane_read(v, 47);
    const uint32_t row = lane >> 4;
    T lower = T(0);
    if (row >= 1u) lower = r0;
    if (row >= 2u) lower += r1;
    if (row >= 3u) lower += r2;
    return v + lower;
}

// The value of lane ^ 32 (gfx950 v_permlane32_swap: the halves of the wave trade places).
__device__ inline uint32_t xor32(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32u) ? r[0] : r[1];
}
__device__ inline float xor32(float v) { return __uint_as_float(xor32(__float_as_uint(v))); }

}  // namespace tdt
