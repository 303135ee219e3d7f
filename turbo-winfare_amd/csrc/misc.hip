// Standalone kernels for the reference's separate stages:
//   k_softcap      shaders/Softcap.hlsl:18-30 (z = cap * tanh(z / cap), in place)
//   k_repetition   src/sampling.cpp:74-90 (per-occurrence penalty with the softcap clamp)
#include <stdexcept>

#include "dt_internal.h"

namespace tdt {

__global__ __launch_bounds__(256) void k_softcap(float* __restrict__ z, size_t n, float cap) {
#pragma clang fp contract(off)
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    z[i] = cap * tanhf(z[i] / cap);
}

void launch_softcap(float* z, size_t n, float cap, hipStream_t st) {
    if (n == 0 || !(cap > 0.0f)) return;
    const size_t blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFFull) throw std::runtime_error("softcap: n too large");
    hipLaunchKernelGGL(k_softcap, dim3((unsigned)blocks), dim3(256), 0, st, z, n, cap);
    check_hip(hipGetLastError(), "softcap");
}

// One workgroup: the history is sorted in LDS, then each run of equal ids applies the
// penalty `count` times to its logit, which equals the reference's sequential loop because
// distinct ids touch distinct logits.
constexpr uint32_t kRepThreads = 1024;
constexpr uint32_t kRepCap = 16384;

__global__ __launch_bounds__(kRepThreads) void k_repetition(float* __restrict__ logits, uint32_t vocab,
                                                            const uint32_t* __restrict__ history,
                                                            uint32_t n, uint32_t P, float penalty,
                                                            float limit) {
#pragma clang fp contract(off)
    extern __shared__ uint32_t ids[];  // [P]
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < P; i += kRepThreads) ids[i] = (i < n) ? history[i] : 0xFFFFFFFFu;
    __syncthreads();
    for (uint32_t size = 2; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = tid; i < P / 2; i += kRepThreads) {
                const uint32_t lo = 2 * i - (i & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool up = ((lo & size) == 0);
                const uint32_t a = ids[lo], c = ids[hi];
                if ((a > c) == up) { ids[lo] = c; ids[hi] = a; }
            }
            __syncthreads();
        }
    }
    for (uint32_t i = tid; i < P; i += kRepThreads) {
        const uint32_t id = ids[i];
        if (id >= vocab || (i > 0 && ids[i - 1] == id)) continue;
        uint32_t count = 0;
        for (uint32_t j = i; j < P && ids[j] == id; ++j) ++count;
        float v = logits[id];
        for (uint32_t c = 0; c < count; ++c) {
            v = (v > 0.0f) ? v / penalty : v * penalty;
            if (limit > 0.0f) v = fminf(fmaxf(v, -limit), limit);
        }
        logits[id] = v;
    }
}

void launch_repetition(float* logits, uint32_t vocab, const uint32_t* history, uint32_t n,
                       float penalty, float softcap, hipStream_t st) {
    if (penalty == 1.0f || n == 0) return;  // src/sampling.cpp:78
    if (n > kRepCap) throw std::runtime_error("repetition penalty: history longer than 16384");
    uint32_t P = 2;
    while (P < n) P <<= 1;
    const float limit = (softcap > 0.0f) ? softcap * 0.9999f : 0.0f;
    hipLaunchKernelGGL(k_repetition, dim3(1), dim3(kRepThreads), (size_t)P * sizeof(uint32_t), st,
                       logits, vocab, history, n, P, penalty, limit);
    check_hip(hipGetLastError(), "repetition penalty");
}

// ---- embedding lookup ------------------------------------------------------------------------
// Row `id` of the tied table from the head's tiled copy, dequantised as (float)q * s + b and
// scaled by sqrtf(D) (src/cpu_reference.cpp:108-124, :323-329; shaders/EmbedLookup.hlsl:32-44).
// One workgroup per token; a thread handles one packed word (8 nibbles) at a time: chunk c of
// row r in tile t is the uint4 Wt[(t NC + c) 64 + r], its word j holds elements 32c + 8j ...
// low nibble first. Ids past the vocabulary give a row of NaN.
__global__ __launch_bounds__(256) void k_embed(const uint32_t* __restrict__ Wt, const uint32_t* __restrict__ SBt,
                                               uint32_t V, uint32_t D, uint32_t NC, uint32_t G, float scale,
                                               const uint32_t* __restrict__ tokens, float* __restrict__ out) {
#pragma clang fp contract(off)
    const uint32_t id = tokens[blockIdx.x];
    float* dst = out + (size_t)blockIdx.x * D;
    const uint32_t tile = id >> 6, r = id & 63u;
    for (uint32_t w = threadIdx.x; w < D / 8u; w += blockDim.x) {
        float v[8];
        if (id < V) {
            const uint32_t word = Wt[(((size_t)tile * NC + (w >> 2)) * kTileRows + r) * 4u + (w & 3u)];
            const uint32_t sb = SBt[((size_t)tile * G + (w >> 3)) * kTileRows + r];
            const float s = bf16_to_f32(sb & 0xFFFFu), b = bf16_to_f32(sb >> 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float x = (float)((word >> (4 * e)) & 15u) * s;
                x = x + b;
                v[e] = x * scale;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __builtin_nanf("");
        }
        reinterpret_cast<float4*>(dst + 8u * w)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(dst + 8u * w)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

void launch_embed(const Head& h, const uint32_t* tokens, int n, float* out, float scale, hipStream_t st) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_embed, dim3((unsigned)n), dim3(256), 0, st, reinterpret_cast<const uint32_t*>(h.Wt),
                       h.SBt, h.V, h.D, h.NC, h.G, scale, tokens, out);
    check_hip(hipGetLastError(), "embedding lookup");
}

}  // namespace tdt
