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

}  // namespace tdt
