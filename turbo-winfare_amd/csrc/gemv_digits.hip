// Small-batch (B <= 2) affine-int4 LM head: a bandwidth-bound streaming GEMV.
//
// Reference semantics: out[row] = sum_g s_g * sum_j q_j x_j + b_g * sum_j x_j
// (src/cpu_reference.cpp:55-84; shaders/GemvInt4.hlsl + Common.hlsli:98-141).
//
// Design (gfx950):
//  * One wave64 per 64-row tile, lane = row. The tiled layout makes each wave's load of one
//    16-byte chunk a contiguous 1 KiB (64 lanes x global_load_dwordx4); a tile is one 88 KiB
//    contiguous stream at D = 2816.
//  * Activations are block floating point with 21-bit mantissas per 64-element group, split
//    into six signed 4-bit digit planes. With q' = q - 8 (one XOR of the word with 0x88888888)
//    every weight word needs six v_dot8_i32_i4 against wave-uniform digit words that live in
//    SGPRs (scalar loads). Products are exact integers, so only the per-group scale-back and
//    the fp32 group combination round:
//        row += s * (D_g * 2^(e-21)) + (8 s + b) * S_g,   D_g = sum q'_j X_j,  S_g = sum X_j 2^(e-21)
//  * Per-group scale/bias come from the tiled (s | b << 16) words, one coalesced dword per lane.
//  * Loads are nontemporal and software-pipelined kPF groups ahead.
#include <hip/hip_ext.h>

#include <algorithm>

#include "dt_epilogue.h"

namespace tdt {

constexpr int kDigitWaves = 4;
// Groups in flight per wave. With nontemporal loads a shallow pipeline streams fastest: on
// MI355X depth 1-2 reaches 6.6 TB/s where depth 4 (more VGPRs, fewer resident waves) gave
// 6.1 TB/s and plain loads 5.3 TB/s.
constexpr int kPF = 2;

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// The table is streamed once per step: nontemporal loads keep it from displacing the
// activations and partials in the caches.
__device__ inline uint4 load_stream(const uint4* p) {
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ inline uint32_t load_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }

template <int NB>
__global__ __launch_bounds__(kDigitWaves * 64) void k_head_digits(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SBt, const uint32_t* __restrict__ xdig,
    const float* __restrict__ xws, const float* __restrict__ xsum, uint32_t NC, uint32_t G, EpiArgs ep) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t tile = blockIdx.x * kDigitWaves + wave;
    if (tile >= ep.ntile) return;  // wave-uniform
    const uint4* wp = Wt + (size_t)tile * NC * kTileRows + lane;
    const uint32_t* sbp = SBt + (size_t)tile * G * kTileRows + lane;

    float acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = 0.0f;

    uint4 wa[kPF], wb[kPF];
    uint32_t sb[kPF];
#pragma unroll
    for (int p = 0; p < kPF; ++p) {
        if ((uint32_t)p < G) {
            wa[p] = load_stream(wp + (size_t)(2 * p) * kTileRows);
            wb[p] = load_stream(wp + (size_t)(2 * p + 1) * kTileRows);
            sb[p] = load_stream(sbp + (size_t)p * kTileRows);
        }
    }

    for (uint32_t g0 = 0; g0 < G; g0 += kPF) {
#pragma unroll
        for (int p = 0; p < kPF; ++p) {
            const uint32_t g = g0 + p;
            if (g < G) {
                const uint4 A = wa[p], Bw = wb[p];
                const uint32_t s = sb[p];
                const uint32_t gn = g + kPF;
                if (gn < G) {
                    wa[p] = load_stream(wp + (size_t)(2 * gn) * kTileRows);
                    wb[p] = load_stream(wp + (size_t)(2 * gn + 1) * kTileRows);
                    sb[p] = load_stream(sbp + (size_t)gn * kTileRows);
                }
                const uint32_t wq[8] = {A.x ^ 0x88888888u, A.y ^ 0x88888888u, A.z ^ 0x88888888u,
                                        A.w ^ 0x88888888u, Bw.x ^ 0x88888888u, Bw.y ^ 0x88888888u,
                                        Bw.z ^ 0x88888888u, Bw.w ^ 0x88888888u};
                const float sf = bf16_to_f32(s & 0xFFFFu);
                const float bf = bf16_to_f32(s >> 16);
                const float c8 = fmaf(8.0f, sf, bf);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const uint32_t* xd = xdig + ((size_t)nb * NC + 2u * g) * kDigitWordsPerChunk;
                    int a[kDigits];
#pragma unroll
                    for (uint32_t k = 0; k < kDigits; ++k) a[k] = 0;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
#pragma unroll
                            for (uint32_t k = 0; k < kDigits; ++k)
                                a[k] = __builtin_amdgcn_sdot8((int)wq[4 * h + i],
                                                              (int)xd[h * kDigitWordsPerChunk + k * 4 + i],
                                                              a[k], false);
                        }
                    }
                    uint32_t Dg = (uint32_t)a[0];
#pragma unroll
                    for (uint32_t k = 1; k < kDigits; ++k) Dg += (uint32_t)a[k] << (4u * k);
                    const float t = sf * xws[(size_t)nb * G + g];
                    acc[nb] = fmaf((float)(int)Dg, t, acc[nb]);
                    acc[nb] = fmaf(c8, xsum[(size_t)nb * G + g], acc[nb]);
                }
            }
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) epilogue_wave(acc[nb], (uint32_t)nb, tile, lane, ep);
}

// Matrices with few 64-row tiles (the projection shapes) give one wave per tile too little
// parallelism: here a workgroup of KS waves shares one tile, wave w taking groups
// [w G / KS, (w + 1) G / KS), and the partial sums are added in wave order through LDS before
// wave 0 runs the epilogue.
constexpr uint32_t kMaxSplit = 16;
template <int NB>
__global__ __launch_bounds__(kMaxSplit * 64) void k_head_digits_split(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SBt, const uint32_t* __restrict__ xdig,
    const float* __restrict__ xws, const float* __restrict__ xsum, uint32_t NC, uint32_t G, EpiArgs ep) {
    __shared__ float part[kMaxSplit][NB][64];
    // wave-uniform by construction; read through the scalar unit so the group range, and with it
    // the digit-word addresses, stay scalar (s_load) instead of per-lane loads
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t KS = blockDim.x >> 6;
    const uint32_t tile = blockIdx.x;
    const uint4* wp = Wt + (size_t)tile * NC * kTileRows + lane;
    const uint32_t* sbp = SBt + (size_t)tile * G * kTileRows + lane;
    float acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = 0.0f;
    const uint32_t g0 = wave * G / KS, g1 = (wave + 1u) * G / KS;
    // a wave holds few groups: all of a batch of kBatchG are loaded before any is used, so
    // the wave waits for memory once per batch rather than once per group
    constexpr uint32_t kBatchG = 4;
    for (uint32_t gb = g0; gb < g1; gb += kBatchG) {
        uint4 Ab[kBatchG], Bb[kBatchG];
        uint32_t Sb[kBatchG];
#pragma unroll
        for (uint32_t q = 0; q < kBatchG; ++q) {
            const uint32_t g = min(gb + q, g1 - 1u);  // past the range: a repeated, unused load
            Ab[q] = load_stream(wp + (size_t)(2 * g) * kTileRows);
            Bb[q] = load_stream(wp + (size_t)(2 * g + 1) * kTileRows);
            Sb[q] = load_stream(sbp + (size_t)g * kTileRows);
        }
#pragma unroll
        for (uint32_t q = 0; q < kBatchG; ++q) {
            // branch-free: a group past the range is computed on its clamped copy and dropped,
            // so no branch separates the batch's loads from each other
            const bool in = gb + q < g1;
            const uint32_t g = min(gb + q, g1 - 1u);
            const uint4 A = Ab[q], Bw = Bb[q];
            const uint32_t sbw = Sb[q];
            const uint32_t wq[8] = {A.x ^ 0x88888888u, A.y ^ 0x88888888u, A.z ^ 0x88888888u,
                                    A.w ^ 0x88888888u, Bw.x ^ 0x88888888u, Bw.y ^ 0x88888888u,
                                    Bw.z ^ 0x88888888u, Bw.w ^ 0x88888888u};
            const float sf = bf16_to_f32(sbw & 0xFFFFu);
            const float bf = bf16_to_f32(sbw >> 16);
            const float c8 = fmaf(8.0f, sf, bf);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const uint32_t* xd = xdig + ((size_t)nb * NC + 2u * g) * kDigitWordsPerChunk;
                int a[kDigits];
#pragma unroll
                for (uint32_t k = 0; k < kDigits; ++k) a[k] = 0;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (uint32_t k = 0; k < kDigits; ++k)
                            a[k] = __builtin_amdgcn_sdot8((int)wq[4 * hh + i],
                                                          (int)xd[hh * kDigitWordsPerChunk + k * 4 + i], a[k], false);
                uint32_t Dg = (uint32_t)a[0];
#pragma unroll
                for (uint32_t k = 1; k < kDigits; ++k) Dg += (uint32_t)a[k] << (4u * k);
                float t = fmaf((float)(int)Dg, sf * xws[(size_t)nb * G + g], acc[nb]);
                t = fmaf(c8, xsum[(size_t)nb * G + g], t);
                acc[nb] = in ? t : acc[nb];
            }
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) part[wave][nb][lane] = acc[nb];
    __syncthreads();
    if (wave != 0u) return;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        float v = part[0][nb][lane];
        for (uint32_t w = 1; w < KS; ++w) v += part[w][nb][lane];
        epilogue_wave(v, (uint32_t)nb, tile, lane, ep);
    }
}

void launch_head_digits(const Head& h, int batch, const EpiArgs& ep, hipStream_t st,
                        hipEvent_t ev0, hipEvent_t ev1) {
    // enough waves to fill the chip (~2048) from few tiles: split each tile's groups
    const uint32_t ks = std::min<uint32_t>({kMaxSplit, h.G, (2048u + h.ntile - 1u) / h.ntile});
    if (ks >= 2u && (batch == 1 || batch == 2)) {
        const dim3 grid(h.ntile), block(64u * ks);
        if (batch == 1)
            hipExtLaunchKernelGGL(k_head_digits_split<1>, grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt, h.xdig,
                                  h.xws, h.xsum, h.NC, h.G, ep);
        else
            hipExtLaunchKernelGGL(k_head_digits_split<2>, grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt, h.xdig,
                                  h.xws, h.xsum, h.NC, h.G, ep);
        check_hip(hipGetLastError(), "head (digit GEMV, split groups)");
        return;
    }
    const unsigned grid = (h.ntile + kDigitWaves - 1) / kDigitWaves;
    if (batch == 1)
        hipExtLaunchKernelGGL(k_head_digits<1>, dim3(grid), dim3(kDigitWaves * 64), 0, st, ev0, ev1,
                              0, h.Wt, h.SBt, h.xdig, h.xws, h.xsum, h.NC, h.G, ep);
    else if (batch == 2)
        hipExtLaunchKernelGGL(k_head_digits<2>, dim3(grid), dim3(kDigitWaves * 64), 0, st, ev0, ev1,
                              0, h.Wt, h.SBt, h.xdig, h.xws, h.xsum, h.NC, h.G, ep);
    else
        throw std::runtime_error("digit GEMV supports batch 1 or 2");
    check_hip(hipGetLastError(), "head (digit GEMV)");
}

// Modifier epilogue over caller-provided logits (no softcap, no GEMV): one wave per 64 ids.
__global__ __launch_bounds__(256) void k_logits_epilogue(EpiArgs ep, const float* __restrict__ in) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t tile = blockIdx.x * 4 + wave;
    const uint32_t b = blockIdx.y;
    if (tile >= ep.ntile) return;
    const uint32_t id = tile * kTileRows + lane;
    const float v = (id < ep.V) ? in[(size_t)b * ep.V + id] : -INFINITY;
    epilogue_wave(v, b, tile, lane, ep);
}

void launch_logits_epilogue(const Head& h, int batch, const EpiArgs& ep, hipStream_t st) {
    const unsigned gx = (h.ntile + 3) / 4;
    hipLaunchKernelGGL(k_logits_epilogue, dim3(gx, (unsigned)batch), dim3(256), 0, st, ep,
                       (const float*)ep.logits);
    check_hip(hipGetLastError(), "logits epilogue");
}

}  // namespace tdt
