// Create-time repack and per-step preparation kernels.
//
//  k_repack_w / k_repack_sb : reference layout -> tiled layout (once, at create)
//  k_prep                   : final RMSNorm (src/cpu_reference.cpp:43-52) and the activation
//                             formats the head kernels read
//  k_modtable               : per-row sorted modifier list (history counts + summed bias)
#include <stdexcept>

#include "dt_internal.h"

namespace tdt {

// ---- repack -------------------------------------------------------------------------------
// Wt[tile][c][r] = W[tile*64 + r][16c .. 16c+15]; rows past V are zero.
__global__ void k_repack_w(const uint8_t* __restrict__ W, uint4* __restrict__ Wt, uint32_t V,
                           uint32_t NC, uint64_t items) {
    const uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (it >= items) return;
    const uint32_t r = (uint32_t)(it % kTileRows);
    const uint64_t tc = it / kTileRows;
    const uint32_t c = (uint32_t)(tc % NC);
    const uint64_t tile = tc / NC;
    const uint64_t row = tile * kTileRows + r;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < V) v = *reinterpret_cast<const uint4*>(W + row * (uint64_t)NC * 16u + (uint64_t)c * 16u);
    Wt[it] = v;
}

// SBt[tile][g][r] = S[row][g] | B[row][g] << 16
__global__ void k_repack_sb(const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
                            uint32_t* __restrict__ SBt, uint32_t V, uint32_t G, uint64_t items) {
    const uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (it >= items) return;
    const uint32_t r = (uint32_t)(it % kTileRows);
    const uint64_t tg = it / kTileRows;
    const uint32_t g = (uint32_t)(tg % G);
    const uint64_t tile = tg / G;
    const uint64_t row = tile * kTileRows + r;
    uint32_t v = 0u;
    if (row < V) v = (uint32_t)S[row * G + g] | ((uint32_t)B[row * G + g] << 16);
    SBt[it] = v;
}

void launch_repack(const Head& h, const uint8_t* W, const uint16_t* S, const uint16_t* B,
                   hipStream_t st) {
    const uint64_t items_w = (uint64_t)h.ntile * h.NC * kTileRows;
    const uint64_t items_sb = (uint64_t)h.ntile * h.G * kTileRows;
    const uint32_t tpb = 256;
    hipLaunchKernelGGL(k_repack_w, dim3((unsigned)((items_w + tpb - 1) / tpb)), dim3(tpb), 0, st,
                       W, h.Wt, h.V, h.NC, items_w);
    check_hip(hipGetLastError(), "repack weights");
    hipLaunchKernelGGL(k_repack_sb, dim3((unsigned)((items_sb + tpb - 1) / tpb)), dim3(tpb), 0,
                       st, S, B, h.SBt, h.V, h.G, items_sb);
    check_hip(hipGetLastError(), "repack scales");
}

// ---- per-step activation preparation ---------------------------------------------------------
// One 256-thread workgroup per batch row.
//
// Digit planes (small-batch GEMV): each 64-element group g is rescaled by 2^(21-e), where
// max|x| = f * 2^e with f in [0.5, 1), and rounded to integers X with |X| <= 2^21. X is written
// as six balanced base-16 digits d_k in [-8, 7] (X = sum d_k 16^k), packed eight per word in
// element order, so v_dot8_i32_i4 can consume them against the weight nibbles directly. The
// group's scale-back factor 2^(e-21) and sum(X) * 2^(e-21) are stored beside them.
//
// fp16 (MFMA path): x rounded to fp16 and stored k-permuted within each octet as
// (x0, x4, x1, x5, x2, x6, x3, x7), the order in which the weight dequant produces halves.
constexpr uint32_t kPrepThreads = 256;

__global__ __launch_bounds__(kPrepThreads) void k_prep(
    const void* __restrict__ hidden, int dtype, int normed, const uint16_t* __restrict__ gamma,
    float eps, uint32_t D, float* __restrict__ xn, uint32_t* __restrict__ xdig,
    float* __restrict__ xws, float* __restrict__ xsum, uint16_t* __restrict__ x16, int path) {
    extern __shared__ float sx[];  // [D]
    __shared__ double red[kPrepThreads / 64];
    const uint32_t b = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;

    for (uint32_t i = tid; i < D; i += kPrepThreads) {
        float v;
        if (dtype == 1) v = bf16_to_f32(reinterpret_cast<const uint16_t*>(hidden)[(size_t)b * D + i]);
        else v = reinterpret_cast<const float*>(hidden)[(size_t)b * D + i];
        sx[i] = v;
    }
    __syncthreads();

    if (!normed) {
        // src/cpu_reference.cpp:44-46: double sum of squares, float mean + eps, 1/sqrt.
        double acc = 0.0;
        for (uint32_t i = tid; i < D; i += kPrepThreads) acc += (double)sx[i] * (double)sx[i];
        acc = wave_sum_d(acc);
        if (lane == 0) red[wave] = acc;
        __syncthreads();
        double tot = 0.0;
        for (uint32_t w = 0; w < kPrepThreads / 64; ++w) tot += red[w];
        const float ms = (float)(tot / (double)D);
        // sqrtf and 1.0f / s, each correctly rounded: computed in double and rounded once to
        // float, which is exact for sqrt and division (53 >= 2 * 24 + 2 bits).
        const float sq = (float)sqrt((double)__fadd_rn(ms, eps));
        const float inv = (float)(1.0 / (double)sq);
        __syncthreads();
        for (uint32_t i = tid; i < D; i += kPrepThreads) {
            float v = __fmul_rn(sx[i], inv);
            if (gamma) v = __fmul_rn(v, bf16_to_f32(gamma[i]));
            sx[i] = v;
        }
        __syncthreads();
    }
    if (xn)
        for (uint32_t i = tid; i < D; i += kPrepThreads) xn[(size_t)b * D + i] = sx[i];

    if (path == 0) {
        const uint32_t G = D / kGroup, NC = D / 32u;
        for (uint32_t g = wave; g < G; g += kPrepThreads / 64) {
            const float x = sx[g * kGroup + lane];
            const float m = wave_max(fabsf(x));
            int e = 0;
            (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1); e = 0 for m = 0
            const int X = (int)rintf(ldexpf(x, 21 - e));
            const int sX = wave_sum_i(X);
            if (lane == 0) {
                xws[(size_t)b * G + g] = ldexpf(1.0f, e - 21);
                xsum[(size_t)b * G + g] = (float)sX * ldexpf(1.0f, e - 21);
            }
            int r = X;
            const uint32_t c = 2u * g + (lane >> 5);     // chunk
            const uint32_t wi = (lane & 31u) >> 3;       // word within chunk
            const uint32_t sh = 4u * (lane & 7u);        // nibble position
#pragma unroll
            for (uint32_t k = 0; k < kDigits; ++k) {
                const int d = ((r + 8) & 15) - 8;
                r = (r - d) >> 4;
                uint32_t v = ((uint32_t)d & 15u) << sh;
                v |= (uint32_t)__shfl_xor((int)v, 1, 64);
                v |= (uint32_t)__shfl_xor((int)v, 2, 64);
                v |= (uint32_t)__shfl_xor((int)v, 4, 64);
                if ((lane & 7u) == 0u)
                    xdig[(((size_t)b * NC + c) * kDigits + k) * 4u + wi] = v;
            }
        }
    } else {
        for (uint32_t i = tid; i < D; i += kPrepThreads) {
            const uint32_t e = i & 7u;
            const uint32_t slot = (e < 4u) ? 2u * e : 2u * (e - 4u) + 1u;
            const _Float16 hv = (_Float16)sx[i];
            x16[(size_t)b * D + (i & ~7u) + slot] = __builtin_bit_cast(uint16_t, hv);
        }
    }
}

void launch_prep(const Head& h, const void* hidden, int dtype, int batch, bool normed,
                 float* xn_out, HeadPath path, hipStream_t st) {
    const size_t lds = (size_t)h.D * sizeof(float);
    hipLaunchKernelGGL(k_prep, dim3((unsigned)batch), dim3(kPrepThreads), lds, st, hidden, dtype,
                       normed ? 1 : 0, h.gamma, h.eps, h.D, xn_out, h.xdig, h.xws, h.xsum, h.x16,
                       path == HeadPath::Digits ? 0 : 1);
    check_hip(hipGetLastError(), "prep");
}

// ---- modifier table ---------------------------------------------------------------------------
// One workgroup per row. History ids (when the row uses them) and bias entries are sorted
// together by (id, source, position) with a bitonic sort in LDS. Each run of equal ids becomes
// one entry: the history count, and the bias values summed in list order from 0.0f. Entries
// are written sorted by id, then block_start[t] = number of entries with id < 64 t.
constexpr uint32_t kModThreads = 1024;

__global__ __launch_bounds__(kModThreads) void k_modtable(
    const DevRow* __restrict__ rows, uint32_t V, uint32_t ntile, const uint32_t* __restrict__ history,
    uint32_t hist_stride, const uint32_t* __restrict__ hist_len, const uint32_t* __restrict__ bias_ids,
    const float* __restrict__ bias_vals, uint32_t bias_stride, const uint32_t* __restrict__ bias_count,
    ModEntry* __restrict__ mods, uint32_t mod_cap, uint32_t* __restrict__ mod_count,
    uint32_t* __restrict__ block_start, uint32_t P) {
    extern __shared__ unsigned long long keys[];  // [P]
    __shared__ uint32_t s_nruns;
    __shared__ uint32_t s_scan[kModThreads / 64];
    const uint32_t b = blockIdx.x, tid = threadIdx.x;
    const uint32_t use = rows[b].has_mods;
    if (use == 0u) return;
    const uint32_t nh = ((use & 1u) && history) ? min(hist_len[b], hist_stride) : 0u;
    const uint32_t nb = ((use & 2u) && bias_ids) ? min(bias_count[b], bias_stride) : 0u;
    const unsigned long long kPad = ~0ull;
    for (uint32_t i = tid; i < P; i += kModThreads) {
        unsigned long long k = kPad;
        if (i < nh) {
            const uint32_t id = history[(size_t)b * hist_stride + i];
            if (id < V) k = ((unsigned long long)id << 32) | i;
        } else if (i < nh + nb) {
            const uint32_t j = i - nh;
            const uint32_t id = bias_ids[(size_t)b * bias_stride + j];
            if (id < V) k = ((unsigned long long)id << 32) | 0x80000000ull | j;
        }
        keys[i] = k;
    }
    __syncthreads();
    // bitonic sort, ascending
    for (uint32_t size = 2; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = tid; i < P / 2; i += kModThreads) {
                const uint32_t lo = 2 * i - (i & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool up = ((lo & size) == 0);
                const unsigned long long a = keys[lo], c = keys[hi];
                if ((a > c) == up) { keys[lo] = c; keys[hi] = a; }
            }
            __syncthreads();
        }
    }
    // run starts -> compacted entry index via a block scan
    const uint32_t per = (P + kModThreads - 1) / kModThreads;
    const uint32_t i0 = tid * per;
    uint32_t cnt = 0;
    for (uint32_t i = i0; i < i0 + per && i < P; ++i) {
        const unsigned long long k = keys[i];
        if (k != kPad && (i == 0 || (keys[i - 1] >> 32) != (k >> 32))) ++cnt;
    }
    // exclusive scan of cnt over threads
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    uint32_t incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = (uint32_t)__shfl_up((int)incl, o, 64);
        if ((int)lane >= o) incl += v;
    }
    if (lane == 63) s_scan[wave] = incl;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (uint32_t w = 0; w < kModThreads / 64; ++w) { const uint32_t t = s_scan[w]; s_scan[w] = run; run += t; }
        s_nruns = run;
    }
    __syncthreads();
    uint32_t e = s_scan[wave] + incl - cnt;
    for (uint32_t i = i0; i < i0 + per && i < P; ++i) {
        const unsigned long long k = keys[i];
        if (k == kPad || (i != 0 && (keys[i - 1] >> 32) == (k >> 32))) continue;
        const uint32_t id = (uint32_t)(k >> 32);
        uint32_t count = 0, has_bias = 0;
        float total = 0.0f;
        for (uint32_t j = i; j < P && keys[j] != kPad && (uint32_t)(keys[j] >> 32) == id; ++j) {
            const uint32_t lo = (uint32_t)keys[j];
            if (lo & 0x80000000u) {
                total = __fadd_rn(total, bias_vals[(size_t)b * bias_stride + (lo & 0x7FFFFFFFu)]);
                has_bias = 1;
            } else {
                ++count;
            }
        }
        mods[(size_t)b * mod_cap + e] = ModEntry{id, count, total, has_bias};
        ++e;
    }
    __syncthreads();
    const uint32_t nruns = s_nruns;
    if (tid == 0) mod_count[b] = nruns;
    // block_start[t] = #entries with id < 64 t (binary search over the run ids in LDS order)
    // Reuse keys[] compacted: after this barrier write run ids into the front of keys.
    // (Run ids are read back from the global entries to keep LDS ownership simple.)
    const ModEntry* me = mods + (size_t)b * mod_cap;
    for (uint32_t t = tid; t <= ntile; t += kModThreads) {
        const uint32_t bound = t * kTileRows;
        uint32_t lo = 0, hi = nruns;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (me[mid].id < bound) lo = mid + 1; else hi = mid;
        }
        block_start[(size_t)b * (ntile + 1) + t] = lo;
    }
}

void launch_modtable(const Head& h, int batch, const uint32_t* history, uint32_t hist_stride,
                     const uint32_t* hist_len, const uint32_t* bias_ids, const float* bias_vals,
                     uint32_t bias_stride, const uint32_t* bias_count, hipStream_t st) {
    uint32_t n = (history ? hist_stride : 0u) + (bias_ids ? bias_stride : 0u);
    uint32_t P = 2;
    while (P < n) P <<= 1;
    if (P > h.mod_cap) throw std::runtime_error("modifier table: history + bias capacity exceeds the per-row limit");
    hipLaunchKernelGGL(k_modtable, dim3((unsigned)batch), dim3(kModThreads),
                       (size_t)P * sizeof(unsigned long long), st, h.rows, h.V, h.ntile, history,
                       hist_stride, hist_len, bias_ids, bias_vals, bias_stride, bias_count, h.mods,
                       h.mod_cap, h.mod_count, h.block_start, P);
    check_hip(hipGetLastError(), "modifier table");
}

}  // namespace tdt
