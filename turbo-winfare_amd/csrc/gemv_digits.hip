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
#include <stdexcept>
#include <type_traits>

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

// ---- the small-batch step with the preparation folded in ------------------------------------
// One workgroup of 16 waves (one per CU) covers 16 consecutive tiles. Before streaming, each
// workgroup recomputes what the step-prep kernel would have written, keeping it in LDS:
//   * final RMSNorm (src/cpu_reference.cpp:43-52): double sum of squares, float mean + eps,
//     1 / sqrt, each correctly rounded;
//   * the block floating-point form of every 64-element group and its six digit planes: thread
//     t owns octet t (elements 8t .. 8t + 7), so a group is 8 lanes (three DPP steps for its
//     maximum and sum) and a lane writes its own digit words, the balanced base-16 digits of
//     X read off Y = X + 0x888888 (its nibbles minus 8);
//   * the occurrence count of each of its own 1024 ids in the row's history
//     (src/sampling.cpp:81-89 visits every occurrence; ids past the vocabulary are ignored).
// The loads of the row, its norm weight and its history are issued first, then the weight
// prefetch, so this work runs while the first groups are in flight; it replaces a kernel launch
// and its dependent-launch gap. Workgroup 0 also copies the row parameters to device memory for
// the select kernel, after its stream.
// The sum of squares adds in a different order from the step-prep kernel; the mean is rounded
// to float from double either way, so the two agree except at a rounding tie of that float.
constexpr uint32_t kFusedWaves = 16;
constexpr uint32_t kFusedThreads = kFusedWaves * 64;
constexpr uint32_t kFusedHistPer = kFusedHistMax / kFusedThreads;
static_assert(kFusedMaxD == 8u * kFusedThreads, "one octet per thread");

template <int NB>
struct FusedLds {
    uint32_t dig[NB][kFusedMaxD / 32 * kDigitWordsPerChunk];
    float ws[NB][kFusedMaxD / 64];
    float sum[NB][kFusedMaxD / 64];
    uint32_t cnt[NB][kFusedThreads];  // history occurrences of the workgroup's ids
    double red[NB][kFusedWaves];
};

// What the preparation reads, loaded before the weight stream is issued (loads complete in
// order, so waiting for these does not wait for the stream).
template <int NB>
struct FusedIn {
    uint4 x[NB][2];  // the thread's octet: fp32 in both, or bf16 pairs in the first
    uint4 gw;        // the octet's bf16 norm weights
    uint32_t hlen[NB];
    uint32_t hid[NB][kFusedHistPer];
};

// Whether row nb's history is counted.
__device__ inline bool fused_hist_on(const FusedPrep& fp, int nb) {
    return fp.history != nullptr && (fp.inl[nb].has_mods & 1u) != 0u;
}

template <int NB>
__device__ inline void fused_load(const FusedPrep& fp, uint32_t D, FusedIn<NB>& in) {
    // Every load is unconditional, from an address that is always valid (the octet clamped to the
    // row; an absent input reads the hidden row instead and is ignored), and nothing is done with
    // the loaded bits here: a select or branch on a loaded value would make the wave wait for it.
    const uint32_t tid = threadIdx.x;
    const uint32_t o = min(tid, D / 8u - 1u);
    const uint32_t esz = (fp.dtype == 1) ? 2u : 4u;
    const char* xb = reinterpret_cast<const char*>(fp.hidden);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const size_t off = (size_t)esz * ((size_t)nb * D + 8u * o);
        in.x[nb][0] = *reinterpret_cast<const uint4*>(xb + off);
        in.x[nb][1] = *reinterpret_cast<const uint4*>(xb + off + (esz == 4u ? 16u : 0u));
    }
    in.gw = fp.gamma ? reinterpret_cast<const uint4*>(fp.gamma)[o] : *reinterpret_cast<const uint4*>(xb);
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(fp.hidden);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const bool on = fused_hist_on(fp, nb);
        const uint32_t* h = on ? fp.history + (size_t)nb * fp.hist_stride : xw;
        const uint32_t lim = on ? fp.hist_stride - 1u : 0u;
        in.hlen[nb] = *(on ? fp.hist_len + nb : xw);
#pragma unroll
        for (uint32_t q = 0; q < kFusedHistPer; ++q) in.hid[nb][q] = h[min(tid + q * kFusedThreads, lim)];
    }
}

__device__ inline uint32_t word_at(const uint4& v, int i) {
    return (i == 0) ? v.x : (i == 1) ? v.y : (i == 2) ? v.z : v.w;
}

// value of 8-lane group reduction (lanes 8k .. 8k + 7)
template <class T, class Op>
__device__ inline T octet_group_reduce(T v, Op op) {
    v = op(v, dpp_mov<dpp::kXor1>(v));
    v = op(v, dpp_mov<dpp::kXor2>(v));
    v = op(v, dpp_mov<dpp::kHalfMirror>(v));
    return v;
}

template <int NB>
__device__ __attribute__((always_inline)) inline void fused_prep(const FusedPrep& fp, uint32_t D, uint32_t V, const FusedIn<NB>& in, FusedLds<NB>& s) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t idbase = blockIdx.x * kFusedThreads;
    const bool ov = 8u * tid < D;  // this thread's octet lies in the row
    // the octet's elements (0 past the row)
    auto elems = [&](int nb, float (&v)[8]) {
        if (fp.dtype == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w = word_at(in.x[nb][0], i);
                v[2 * i] = bf16_to_f32(w & 0xFFFFu);
                v[2 * i + 1] = bf16_to_f32(w >> 16);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(word_at(in.x[nb][i >> 2], i & 3));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ov ? v[i] : 0.0f;
    };
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        s.cnt[nb][tid] = 0u;
        if (!fp.normed) {
            float v[8];
            elems(nb, v);
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc += (double)v[i] * (double)v[i];
            acc = wave_sum_d(acc);
            if (lane == 0) s.red[nb][wave] = acc;
        }
    }
    __syncthreads();  // partial sums written; counts zeroed
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const uint32_t nh = fused_hist_on(fp, nb) ? min(in.hlen[nb], fp.hist_stride) : 0u;
#pragma unroll
        for (uint32_t q = 0; q < kFusedHistPer; ++q) {
            const uint32_t i = tid + q * kFusedThreads, id = in.hid[nb][q];
            if (i < nh && id < V && id - idbase < kFusedThreads) atomicAdd(&s.cnt[nb][id - idbase], 1u);
        }
    }
    const uint32_t g = tid >> 3, j8 = tid & 7u;  // group and octet within it
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (8u * 64u * wave >= D) break;  // wave-uniform: no octet of this wave lies in the row
        float v[8];
        elems(nb, v);
        if (!fp.normed) {
            const double tot = wave_sum_d(lane < kFusedWaves ? s.red[nb][lane] : 0.0);
            const float ms = (float)(tot / (double)D);
            // sqrtf and 1.0f / s, each correctly rounded: computed in double and rounded once
            const float sq = (float)sqrt((double)(ms + fp.eps));
            const float inv = (float)(1.0 / (double)sq);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = v[i] * inv;
                if (fp.gamma) {
                    const uint32_t w = word_at(in.gw, i >> 1);
                    v[i] = v[i] * bf16_to_f32((i & 1) ? (w >> 16) : (w & 0xFFFFu));
                }
            }
        }
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
        m = octet_group_reduce(m, [](float a, float b) { return fmaxf(a, b); });
        int e = 0;
        (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1); e = 0 for m = 0
        int X[8], sX = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            X[i] = (int)rintf(ldexpf(v[i], 21 - e));
            sX += X[i];
        }
        sX = octet_group_reduce(sX, [](int a, int b) { return a + b; });
        if (ov && j8 == 0u) {
            s.ws[nb][g] = ldexpf(1.0f, e - 21);
            s.sum[nb][g] = (float)sX * ldexpf(1.0f, e - 21);
        }
        uint32_t Z[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) Z[i] = ((uint32_t)X[i] + 0x888888u) ^ 0x888888u;
        uint32_t* dst = &s.dig[nb][(2u * g + (j8 >> 2)) * kDigitWordsPerChunk + (j8 & 3u)];
#pragma unroll
        for (uint32_t k = 0; k < kDigits; ++k) {
            uint32_t w = 0u;
#pragma unroll
            for (int i = 0; i < 8; ++i) w |= ((Z[i] >> (4u * k)) & 15u) << (4u * i);
            if (ov) dst[k * 4u] = w;
        }
    }
    __syncthreads();  // digits, scales and counts complete
}

template <int NB>
__global__ __launch_bounds__(kFusedThreads) void k_head_digits_fused(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SBt, uint32_t D, uint32_t NC, uint32_t G,
    FusedPrep fp, EpiArgs ep) {
    __shared__ __attribute__((aligned(16))) FusedLds<NB> s;
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tile_raw = blockIdx.x * kFusedWaves + wave;
    const bool tile_ok = tile_raw < ep.ntile;
    const uint32_t tile = tile_ok ? tile_raw : ep.ntile - 1u;  // loads clamped; no epilogue
    const uint4* wp = Wt + (size_t)tile * NC * kTileRows + lane;
    const uint32_t* sbp = SBt + (size_t)tile * G * kTileRows + lane;

    FusedIn<NB> in;
    fused_load<NB>(fp, D, in);
    __builtin_amdgcn_sched_barrier(0);  // keep the row's loads ahead of the weight stream
    // branch-free (a group past the end is a repeated, unused load): with a branch here the
    // compiler's wait for the row's loads would have to assume the shorter path and also wait
    // for part of the stream
    uint4 wa[kPF], wb[kPF];
    uint32_t sb[kPF];
#pragma unroll
    for (int p = 0; p < kPF; ++p) {
        const uint32_t gp = min((uint32_t)p, G - 1u);
        wa[p] = load_stream(wp + (size_t)(2 * gp) * kTileRows);
        wb[p] = load_stream(wp + (size_t)(2 * gp + 1) * kTileRows);
        sb[p] = load_stream(sbp + (size_t)gp * kTileRows);
    }
    __builtin_amdgcn_sched_barrier(0);
    fused_prep<NB>(fp, D, ep.V, in, s);

    float acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = 0.0f;
    for (uint32_t g0 = 0; g0 < G; g0 += kPF) {
#pragma unroll
        for (int p = 0; p < kPF; ++p) {
            const uint32_t g = g0 + p;
            if (g < G) {
                const uint4 A = wa[p], Bw = wb[p];
                const uint32_t sbw = sb[p];
                const uint32_t gn = g + kPF;
                if (gn < G) {
                    wa[p] = load_stream(wp + (size_t)(2 * gn) * kTileRows);
                    wb[p] = load_stream(wp + (size_t)(2 * gn + 1) * kTileRows);
                    sb[p] = load_stream(sbp + (size_t)gn * kTileRows);
                }
                const uint32_t wq[8] = {A.x ^ 0x88888888u, A.y ^ 0x88888888u, A.z ^ 0x88888888u,
                                        A.w ^ 0x88888888u, Bw.x ^ 0x88888888u, Bw.y ^ 0x88888888u,
                                        Bw.z ^ 0x88888888u, Bw.w ^ 0x88888888u};
                const float sf = bf16_to_f32(sbw & 0xFFFFu);
                const float bf = bf16_to_f32(sbw >> 16);
                const float c8 = fmaf(8.0f, sf, bf);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const uint32_t* xd = &s.dig[nb][(2u * g) * kDigitWordsPerChunk];
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
                    const float t = sf * s.ws[nb][g];
                    acc[nb] = fmaf((float)(int)Dg, t, acc[nb]);
                    acc[nb] = fmaf(c8, s.sum[nb][g], acc[nb]);
                }
            }
        }
    }
    // the row parameters for the select kernel (after the stream: this wait is free here)
    if (blockIdx.x == 0u && threadIdx.x < NB * (sizeof(DevRow) / 4))
        reinterpret_cast<uint32_t*>(fp.rows_dst)[threadIdx.x] = reinterpret_cast<const uint32_t*>(&fp.inl[0])[threadIdx.x];
    if (!tile_ok) return;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const uint32_t cnt = (fp.inl[nb].has_mods & 1u) ? s.cnt[nb][wave * 64u + lane] : 0u;
        epilogue_wave_counted(acc[nb], (uint32_t)nb, tile, lane, ep, fp.inl[nb], cnt);
    }
}

void launch_split_folded(const Head& h, int batch, const FusedPrep& fp, const EpiArgs& ep, hipStream_t st,
                         hipEvent_t ev0, hipEvent_t ev1);

void launch_head_digits_fused(const Head& h, int batch, const FusedPrep& fp, const EpiArgs& ep,
                              hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (h.D > kFusedMaxD || h.D % kGroup != 0u) throw std::runtime_error("folded step needs D <= 8192");
    if (h.ntile < kFusedMinTiles) {
        // few tiles: the split kernel with the digit planes folded in (normalised rows, no history)
        const uint32_t nt = split_threads(h);
        if (!nt || h.D > 8u * nt || !fp.normed || fp.history)
            throw std::runtime_error("folded split head needs normalised rows, no history and D <= 8 x threads");
        launch_split_folded(h, batch, fp, ep, st, ev0, ev1);
        return;
    }
    const dim3 grid((h.ntile + kFusedWaves - 1u) / kFusedWaves), block(kFusedThreads);
    if (batch == 1)
        hipExtLaunchKernelGGL(k_head_digits_fused<1>, grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt, h.D, h.NC,
                              h.G, fp, ep);
    else if (batch == 2)
        hipExtLaunchKernelGGL(k_head_digits_fused<2>, grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt, h.D, h.NC,
                              h.G, fp, ep);
    else
        throw std::runtime_error("folded step supports batch 1 or 2");
    check_hip(hipGetLastError(), "head (digit GEMV, folded preparation)");
}

// Matrices with few 64-row tiles (the projection shapes) give one wave per tile too little
// parallelism: here a workgroup of KS waves shares one tile, wave w taking groups
// [w G / KS, (w + 1) G / KS), and the partial sums are added in wave order through LDS before
// wave 0 runs the epilogue.
// FUSED: the digit planes of the (already normalised) rows are computed by every workgroup into
// LDS from fp.hidden while its first weight groups are in flight, as in k_head_digits_fused,
// instead of being read from a preparation kernel's output; the row parameters come from fp.inl.
// Needs one thread per 8 elements of the row (D <= 8 KS 64).
constexpr uint32_t kMaxSplit = 16;
template <int NB, bool FUSED>
__global__ __launch_bounds__(kMaxSplit * 64) void k_head_digits_split(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SBt, const uint32_t* __restrict__ xdig,
    const float* __restrict__ xws, const float* __restrict__ xsum, uint32_t NC, uint32_t G, EpiArgs ep,
    FusedPrep fp, uint32_t D) {
    __shared__ float part[kMaxSplit][NB][64];
    __shared__ __attribute__((aligned(16))) std::conditional_t<FUSED, FusedLds<NB>, uint32_t> fs;
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
    uint4 Ab[kBatchG], Bb[kBatchG];
    uint32_t Sb[kBatchG];
    auto load_batch = [&](uint32_t gb) {
#pragma unroll
        for (uint32_t q = 0; q < kBatchG; ++q) {
            const uint32_t g = min(gb + q, g1 - 1u);  // past the range: a repeated, unused load
            Ab[q] = load_stream(wp + (size_t)(2 * g) * kTileRows);
            Bb[q] = load_stream(wp + (size_t)(2 * g + 1) * kTileRows);
            Sb[q] = load_stream(sbp + (size_t)g * kTileRows);
        }
    };
    // every wave holds at least one group (KS <= G)
    [[maybe_unused]] FusedIn<NB> in;
    if constexpr (FUSED) {
        fused_load<NB>(fp, D, in);
        __builtin_amdgcn_sched_barrier(0);  // the row's loads ahead of the weight batch
    }
    load_batch(g0);
    if constexpr (FUSED) {
        __builtin_amdgcn_sched_barrier(0);
        fused_prep<NB>(fp, D, ep.V, in, fs);
    }
    for (uint32_t gb = g0; gb < g1; gb += kBatchG) {
        if (gb != g0) load_batch(gb);
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
                const uint32_t* xd;
                float ws, sm;
                if constexpr (FUSED) {
                    xd = &fs.dig[nb][(2u * g) * kDigitWordsPerChunk];
                    ws = fs.ws[nb][g];
                    sm = fs.sum[nb][g];
                } else {
                    xd = xdig + ((size_t)nb * NC + 2u * g) * kDigitWordsPerChunk;
                    ws = xws[(size_t)nb * G + g];
                    sm = xsum[(size_t)nb * G + g];
                }
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
                float t = fmaf((float)(int)Dg, sf * ws, acc[nb]);
                t = fmaf(c8, sm, t);
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
        if constexpr (FUSED) epilogue_wave_counted(v, (uint32_t)nb, tile, lane, ep, fp.inl[nb], 0u);
        else epilogue_wave(v, (uint32_t)nb, tile, lane, ep);
    }
    // the row parameters for a select kernel that may follow (workgroup 0, after its stream)
    if constexpr (FUSED) {
        if (blockIdx.x == 0u && fp.rows_dst && lane < NB * (sizeof(DevRow) / 4))
            reinterpret_cast<uint32_t*>(fp.rows_dst)[lane] = reinterpret_cast<const uint32_t*>(&fp.inl[0])[lane];
    }
}

// Workgroup size of the split kernel for this head: 64 * KS threads, or 0 when the head takes
// one wave per tile instead. Enough waves to fill the chip (~2048) from few tiles.
uint32_t split_threads(const Head& h) {
    const uint32_t ks = split_waves(h.G, h.ntile);
    return ks >= 2u ? 64u * ks : 0u;
}

void launch_split_folded(const Head& h, int batch, const FusedPrep& fp, const EpiArgs& ep, hipStream_t st,
                         hipEvent_t ev0, hipEvent_t ev1) {
    const dim3 grid(h.ntile), block(split_threads(h));
    const uint32_t* no_dig = nullptr;
    const float* no_f = nullptr;
    if (batch == 1)
        hipExtLaunchKernelGGL((k_head_digits_split<1, true>), grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt, no_dig,
                              no_f, no_f, h.NC, h.G, ep, fp, h.D);
    else if (batch == 2)
        hipExtLaunchKernelGGL((k_head_digits_split<2, true>), grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt, no_dig,
                              no_f, no_f, h.NC, h.G, ep, fp, h.D);
    else
        throw std::runtime_error("folded step supports batch 1 or 2");
    check_hip(hipGetLastError(), "head (digit GEMV, split groups, folded digits)");
}

void launch_head_digits(const Head& h, int batch, const EpiArgs& ep, hipStream_t st,
                        hipEvent_t ev0, hipEvent_t ev1) {
    const uint32_t nt = split_threads(h);
    if (nt && (batch == 1 || batch == 2)) {
        const dim3 grid(h.ntile), block(nt);
        const FusedPrep none{};
        if (batch == 1)
            hipExtLaunchKernelGGL((k_head_digits_split<1, false>), grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt,
                                  h.xdig, h.xws, h.xsum, h.NC, h.G, ep, none, h.D);
        else
            hipExtLaunchKernelGGL((k_head_digits_split<2, false>), grid, block, 0, st, ev0, ev1, 0, h.Wt, h.SBt,
                                  h.xdig, h.xws, h.xsum, h.NC, h.G, ep, none, h.D);
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

// ---- grouped matrix-vector products ---------------------------------------------------------
// Several independent matrices, each with its own input row and output, in one launch: the
// projections a token makes in one layer (the routed experts' gate and up matrices, or their down
// matrices), each of which alone is a few microseconds of launch and round-trip latency at 1 - 6 MB.
// Workgroup i serves tile i - tile_begin[m] of the matrix m whose range holds i; within it the work
// is the folded split kernel's (digit planes of that matrix's row computed into LDS, KS waves
// splitting the groups with the same split as one matrix alone, partial sums added in wave order),
// so each output is bit-identical to the matrix's own call. The output is the raw product (no
// softcap, no partials).
__global__ __launch_bounds__(kMaxSplit * 64) void k_matvec_grouped(GroupArgs a) {
    __shared__ float part[kMaxSplit][64];
    __shared__ __attribute__((aligned(16))) FusedLds<1> fs;
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t mi = 0;
    for (uint32_t i = 1; i < a.count; ++i)
        if (blockIdx.x >= a.m[i].tile_begin) mi = i;
    const GroupMat M = a.m[mi];
    const uint32_t tile = blockIdx.x - M.tile_begin;
    const uint32_t D = M.D, G = D / kGroup, NC = D / 32u, KS = M.ks;
    const bool active = wave < KS;
    const uint32_t wv = active ? wave : 0u;  // idle waves load wave 0's range and drop it
    const uint4* wp = M.Wt + (size_t)tile * NC * kTileRows + lane;
    const uint32_t* sbp = M.SBt + (size_t)tile * G * kTileRows + lane;
    const uint32_t g0 = wv * G / KS, g1 = (wv + 1u) * G / KS;
    FusedPrep fp{};
    fp.hidden = M.x;
    fp.dtype = 0;
    fp.normed = 1;
    constexpr uint32_t kBatchG = 4;
    uint4 Ab[kBatchG], Bb[kBatchG];
    uint32_t Sb[kBatchG];
    auto load_batch = [&](uint32_t gb) {
#pragma unroll
        for (uint32_t q = 0; q < kBatchG; ++q) {
            const uint32_t g = min(gb + q, g1 - 1u);
            Ab[q] = load_stream(wp + (size_t)(2 * g) * kTileRows);
            Bb[q] = load_stream(wp + (size_t)(2 * g + 1) * kTileRows);
            Sb[q] = load_stream(sbp + (size_t)g * kTileRows);
        }
    };
    FusedIn<1> in;
    fused_load<1>(fp, D, in);
    __builtin_amdgcn_sched_barrier(0);
    load_batch(g0);
    __builtin_amdgcn_sched_barrier(0);
    fused_prep<1>(fp, D, M.rows, in, fs);
    float acc = 0.0f;
    for (uint32_t gb = g0; gb < g1; gb += kBatchG) {
        if (gb != g0) load_batch(gb);
#pragma unroll
        for (uint32_t q = 0; q < kBatchG; ++q) {
            const bool inr = gb + q < g1;
            const uint32_t g = min(gb + q, g1 - 1u);
            const uint4 A = Ab[q], Bw = Bb[q];
            const uint32_t sbw = Sb[q];
            const uint32_t wq[8] = {A.x ^ 0x88888888u, A.y ^ 0x88888888u, A.z ^ 0x88888888u,
                                    A.w ^ 0x88888888u, Bw.x ^ 0x88888888u, Bw.y ^ 0x88888888u,
                                    Bw.z ^ 0x88888888u, Bw.w ^ 0x88888888u};
            const float sf = bf16_to_f32(sbw & 0xFFFFu);
            const float bf = bf16_to_f32(sbw >> 16);
            const float c8 = fmaf(8.0f, sf, bf);
            const uint32_t* xd = &fs.dig[0][(2u * g) * kDigitWordsPerChunk];
            int d[kDigits];
#pragma unroll
            for (uint32_t k = 0; k < kDigits; ++k) d[k] = 0;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (uint32_t k = 0; k < kDigits; ++k)
                        d[k] = __builtin_amdgcn_sdot8((int)wq[4 * hh + i], (int)xd[hh * kDigitWordsPerChunk + k * 4 + i], d[k],
                                                      false);
            uint32_t Dg = (uint32_t)d[0];
#pragma unroll
            for (uint32_t k = 1; k < kDigits; ++k) Dg += (uint32_t)d[k] << (4u * k);
            float t = fmaf((float)(int)Dg, sf * fs.ws[0][g], acc);
            t = fmaf(c8, fs.sum[0][g], t);
            acc = inr ? t : acc;
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave != 0u) return;
    float v = part[0][lane];
    for (uint32_t w = 1; w < KS; ++w) v += part[w][lane];
    const uint32_t row = tile * kTileRows + lane;
    if (row < M.rows) M.out[row] = v;
}

void launch_matvec_grouped(const GroupArgs& a, uint32_t total_tiles, hipStream_t st) {
    if (a.count == 0u) return;
    hipLaunchKernelGGL(k_matvec_grouped, dim3(total_tiles), dim3(kMaxSplit * 64), 0, st, a);
    check_hip(hipGetLastError(), "grouped int4 matvec");
}

uint32_t split_waves(uint32_t G, uint32_t ntile) {
    return std::min<uint32_t>({kMaxSplit, G, (2048u + ntile - 1u) / ntile});
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
