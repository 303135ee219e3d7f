// Create-time repack and the per-step preparation kernel.
//
//  k_repack_w / k_repack_sb : reference layout -> tiled layout (once, at create)
//  k_step_prep              : one block copies the staged per-row parameters to device memory;
//                             ceil(D / 1024) blocks per row run the final RMSNorm
//                             (src/cpu_reference.cpp:43-52) and write the activation format the
//                             head kernel reads (digit planes for B <= 2, k-permuted fp16 for
//                             B > 2); one block per row with modifiers counts the row's history
//                             occurrences per id and builds its bias table sorted by id (summed
//                             bias) with its first entry per 64-id block.
#include <algorithm>
#include <stdexcept>
#include <string>

#include "dt_internal.h"
#include "dt_sort.h"

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

// SB16t[tile][g][r] = fp16(S[row][g]) * 2^mul_log2 | fp16(B[row][g]) << 16 (zero past V). The
// bf16 -> fp16 conversions round to nearest; the power-of-two scaling is exact unless it leaves
// the fp16 range, which sets *bad.
__global__ void k_repack_sb16(const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
                              uint32_t* __restrict__ SB16t, uint32_t V, uint32_t G, uint64_t items, float mul,
                              uint32_t* bad) {
    const uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (it >= items) return;
    const uint32_t r = (uint32_t)(it % kTileRows);
    const uint64_t tg = it / kTileRows;
    const uint32_t g = (uint32_t)(tg % G);
    const uint64_t row = (tg / G) * kTileRows + r;
    uint32_t v = 0u;
    if (row < V) {
        const _Float16 hs = (_Float16)bf16_to_f32(S[row * G + g]);
        const _Float16 hm = (_Float16)((float)hs * mul);
        const _Float16 hb = (_Float16)bf16_to_f32(B[row * G + g]);
        if (!__builtin_isfinite((float)hm) || !__builtin_isfinite((float)hb)) atomicOr(bad, 1u);
        v = (uint32_t)__builtin_bit_cast(uint16_t, hm) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
    }
    SB16t[it] = v;
}

void launch_repack_table(uint4* Wt, uint32_t* SBt, uint32_t V, uint32_t NC, uint32_t G, uint32_t ntile,
                         const uint8_t* W, const uint16_t* S, const uint16_t* B, hipStream_t st) {
    const uint64_t items_w = (uint64_t)ntile * NC * kTileRows;
    const uint64_t items_sb = (uint64_t)ntile * G * kTileRows;
    const uint32_t tpb = 256;
    hipLaunchKernelGGL(k_repack_w, dim3((unsigned)((items_w + tpb - 1) / tpb)), dim3(tpb), 0, st, W, Wt, V, NC,
                       items_w);
    check_hip(hipGetLastError(), "repack weights");
    hipLaunchKernelGGL(k_repack_sb, dim3((unsigned)((items_sb + tpb - 1) / tpb)), dim3(tpb), 0, st, S, B, SBt, V, G,
                       items_sb);
    check_hip(hipGetLastError(), "repack scales");
}

int launch_repack(const Head& h, const uint8_t* W, const uint16_t* S, const uint16_t* B,
                  hipStream_t st) {
    launch_repack_table(h.Wt, h.SBt, h.V, h.NC, h.G, h.ntile, W, S, B, st);
    const uint64_t items_sb = (uint64_t)h.ntile * h.G * kTileRows;
    const uint32_t tpb = 256;
    // the denormal dequant's s * 2^20 where every scale allows it, else plain s
    uint32_t* bad = nullptr;
    check_hip(hipMalloc(&bad, sizeof(uint32_t)), "alloc repack flag");
    auto fill = [&](float mul, uint32_t* flag) -> hipError_t {
        hipError_t e = hipMemsetAsync(bad, 0, sizeof(uint32_t), st);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_repack_sb16, dim3((unsigned)((items_sb + tpb - 1) / tpb)), dim3(tpb), 0, st, S, B,
                           h.SB16t, h.V, h.G, items_sb, mul, bad);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(flag, bad, sizeof(uint32_t), hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return e;
    };
    uint32_t flag = 0u;
    hipError_t e = fill(1048576.0f, &flag);
    const bool denorm = e == hipSuccess && flag == 0u;
    if (e == hipSuccess && !denorm) e = fill(1.0f, &flag);
    (void)hipFree(bad);
    check_hip(e, "repack fp16 scales");
    if (denorm) return 1;
    return flag == 0u ? 0 : -1;
}

// ---- per-step preparation (one launch) -------------------------------------------------------
// Row copy block: the per-row parameters from the host staging slot (pinned, mapped) into
//   device memory for the later kernels.
// RMSNorm blocks, ceil(D / 1024) per batch row: final RMSNorm (src/cpu_reference.cpp:43-52)
//   and the activation format the head kernel reads, 1024 elements per block.
// Modifier blocks, one per batch row (only when some row uses modifiers): history counts and
//   the bias table.
//
// Digit planes (small-batch GEMV): each 64-element group g is rescaled by 2^(21-e), where
// max|x| = f * 2^e with f in [0.5, 1), and rounded to integers X with |X| <= 2^21. X is written
// as six balanced base-16 digits d_k in [-8, 7] (X = sum d_k 16^k), packed eight per word in
// element order, so v_dot8_i32_i4 consumes them against the weight nibbles directly. The
// group's scale-back factor 2^(e-21) and sum(X) * 2^(e-21) are stored beside them. Eight lanes
// A wave holds one group (lane = element); the eight lanes of an octet OR their nibbles into
// one packed word per digit.
//
// fp16 (MFMA path): x rounded to fp16 and stored k-permuted within each octet as
// (x0, x4, x1, x5, x2, x6, x3, x7), the order in which the weight dequant produces halves, with
// the even elements times 16 (denormal dequant, whose even weight halves carry 1/16) or the odd
// elements divided by 16 (the other dequant, whose odd weight halves carry 16). A row whose
// largest |x| exceeds 2^11 (where 16 x would approach the fp16 maximum, 65504) is stored as
// x * 2^-k, k the smallest shift that brings it to 2^11 or below, and xscale[b] = 2^k tells the
// head epilogue to multiply the row's fp32 accumulators back. A power of two commutes with fp16
// and fp32 rounding in their normal ranges, so the logits are those of an fp16 format without
// an exponent limit; rows within range (k = 0, every normalised hidden state) are unchanged.
//
// History counts: the occurrences of each id < V (merged per id in LDS first) are added to
// hcount[b][id] and the id's bit is set in hbits[b] (global atomics); the head epilogue zeroes
// both as it reads them, so they are zero between steps.
// Bias table: the bias entries in (id, list position) order, each run of equal ids becoming one
// entry whose value is the run's biases summed in list order from 0.0f; entries are written
// sorted by id, and block_start[t] = number of entries with id < 64 t. The order comes from
// 64-id tile buckets (counts, their prefix, a small sort per tile) when the per-tile counters fit
// the LDS and no tile holds more than kBucketMaxRun entries, else from a bitonic sort of the
// whole list and a binary search over the run ids.
constexpr uint32_t kPrepThreads = 1024;
constexpr uint32_t kPrepWaves = kPrepThreads / 64;
// LDS table merging a row's history occurrences per id: 2^kHistSlotBits slots of (id, count).
constexpr uint32_t kHistSlotBits = 11;
constexpr uint32_t kHistSlots = 1u << kHistSlotBits;
static_assert(kHistSlots <= kPrepPoolU64, "the history table lives in the prep kernel's LDS pool");

// RMSNorm block k of row b: every block sums the squares of the whole row (the row is small and
// L2-resident; all blocks of a row compute the same sum in the same order), then normalises and
// converts its own kPrepThreads elements, one per thread. A wave then holds exactly one 64-element
// group, so the group's scale and digit words come from wave reductions.
__device__ void prep_row(const PrepArgs& a, uint32_t b, uint32_t k) {
#pragma clang fp contract(off)
    __shared__ double red[kPrepWaves];
    __shared__ float redm[kPrepWaves];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t D = a.D;
    const uint32_t i = k * kPrepThreads + tid;  // this thread's element
    auto load = [&](uint32_t j) -> float {
        if (a.dtype == 1) return bf16_to_f32(reinterpret_cast<const uint16_t*>(a.hidden)[(size_t)b * D + j]);
        return reinterpret_cast<const float*>(a.hidden)[(size_t)b * D + j];
    };
    // the whole row for the sum (one round trip), this element's norm weight alongside
    constexpr uint32_t kPer = 8;  // D <= 8192 = kPer * kPrepThreads
    float xv[kPer];
#pragma unroll
    for (uint32_t q = 0; q < kPer; ++q) {
        const uint32_t j = tid + q * kPrepThreads;
        xv[q] = (j < D) ? load(j) : 0.0f;
    }
    const float gw = (a.gamma && i < D) ? bf16_to_f32(a.gamma[i]) : 1.0f;
    float v = (k < kPer) ? xv[0] : 0.0f;
#pragma unroll
    for (uint32_t q = 1; q < kPer; ++q)
        if (q == k) v = xv[q];
    // fp16 path: the largest |normalised x| of the row, every block of the row computing it the
    // same way from the same values
    float rmax = 0.0f;
    if (!a.normed) {
        // src/cpu_reference.cpp:44-46: double sum of squares, float mean + eps, 1/sqrt.
        double acc = 0.0;
#pragma unroll
        for (uint32_t q = 0; q < kPer; ++q) acc += (double)xv[q] * (double)xv[q];
        acc = wave_sum_d(acc);
        if (lane == 0) red[wave] = acc;
        __syncthreads();
        const double tot = wave_sum_d(lane < kPrepWaves ? red[lane] : 0.0);
        const float ms = (float)(tot / (double)D);
        // sqrtf and 1.0f / s, each correctly rounded: computed in double and rounded once to
        // float, which is exact for sqrt and division (53 >= 2 * 24 + 2 bits).
        const float sq = (float)sqrt((double)(ms + a.eps));
        const float inv = (float)(1.0 / (double)sq);
        v = v * inv;
        if (a.gamma) v = v * gw;
        if (a.path == 1) {
#pragma unroll
            for (uint32_t q = 0; q < kPer; ++q) {
                const uint32_t j = tid + q * kPrepThreads;
                float t = xv[q] * inv;
                if (a.gamma && j < D) t = t * bf16_to_f32(a.gamma[j]);
                rmax = fmaxf(rmax, fabsf(t));
            }
        }
    } else if (a.path == 1) {
#pragma unroll
        for (uint32_t q = 0; q < kPer; ++q) rmax = fmaxf(rmax, fabsf(xv[q]));
    }
    int shift = 0;  // the row is stored in fp16 as x * 2^-shift
    if (a.path == 1) {
        rmax = wave_max(rmax);
        if (lane == 0) redm[wave] = rmax;
        __syncthreads();
        rmax = wave_max(lane < kPrepWaves ? redm[lane] : 0.0f);
        int e = 0;
        (void)frexpf(rmax, &e);  // rmax = f * 2^e, f in [0.5, 1)
        if (__builtin_isfinite(rmax) && e > 11) shift = e - 11;
        if (k == 0u && tid == 0u && a.xscale) a.xscale[b] = ldexpf(1.0f, shift);
    }
    if (i >= D) return;  // whole waves: D is a multiple of the 64-element group
    if (a.xn) a.xn[(size_t)b * D + i] = v;
    if (a.path == 0) {
        const uint32_t G = D / kGroup, NC = D / 32u;
        const uint32_t g = i / kGroup;  // this wave's group
        const float m = wave_max(fabsf(v));
        int e = 0;
        (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1); e = 0 for m = 0
        int X = (int)rintf(ldexpf(v, 21 - e));
        const int sX = wave_sum_i(X);
        if (lane == 0u) {
            a.xws[(size_t)b * G + g] = ldexpf(1.0f, e - 21);
            a.xsum[(size_t)b * G + g] = (float)sX * ldexpf(1.0f, e - 21);
        }
        // six balanced base-16 digits; the eight lanes of an octet OR their nibbles into one word
        const uint32_t j8 = lane >> 3, c = 2u * g + (j8 >> 2), wi = j8 & 3u;
        uint32_t* dst = a.xdig + (((size_t)b * NC + c) * kDigits) * 4u + wi;
#pragma unroll
        for (uint32_t q = 0; q < kDigits; ++q) {
            const int d = ((X + 8) & 15) - 8;
            X = (X - d) >> 4;
            uint32_t w = ((uint32_t)d & 15u) << (4u * (lane & 7u));
            w |= dpp_mov<dpp::kXor1>(w);
            w |= dpp_mov<dpp::kXor2>(w);
            w |= dpp_mov<dpp::kHalfMirror>(w);
            if ((lane & 7u) == 0u) dst[q * 4u] = w;
        }
    } else {
        const uint32_t e = i & 7u;
        const uint32_t slot = (e < 4u) ? 2u * e : 2u * (e - 4u) + 1u;
        if (shift) v = ldexpf(v, -shift);
        const _Float16 hv = (_Float16)(a.x16_denorm ? ((e & 1u) ? v : v * 16.0f) : ((e & 1u) ? v * 0.0625f : v));
        a.x16[(size_t)b * D + (i & ~7u) + slot] = __builtin_bit_cast(uint16_t, hv);
    }
}

// Row b's history occurrence counts into the dense hcount / hbits arrays.
__device__ void history_counts(const PrepArgs& a, uint32_t b, unsigned long long* keys) {
    const uint32_t tid = threadIdx.x;
    const uint32_t V = a.V;
    // One count per occurrence (src/sampling.cpp:81-89 visits every occurrence); ids past
    // the vocabulary are ignored (:82). Occurrences are first merged per id in an LDS table
    // (one slot per hash of the id; an occurrence whose slot holds another id goes straight
    // to the global counters), so a frequent id costs one global atomic instead of one per
    // occurrence: same-address global atomics serialise in L2.
    uint32_t* hk = reinterpret_cast<uint32_t*>(keys);  // [kHistSlots] ids, ~0 when empty
    uint32_t* hc = hk + kHistSlots;                     // [kHistSlots] occurrence counts
    for (uint32_t i = tid; i < kHistSlots; i += kPrepThreads) {
        hk[i] = ~0u;
        hc[i] = 0u;
    }
    __syncthreads();
    const uint32_t nh = min(a.hist_len[b], a.hist_stride);
    const uint32_t* hist = a.history + (size_t)b * a.hist_stride;
    for (uint32_t i = tid; i < nh; i += kPrepThreads) {
        const uint32_t id = hist[i];
        if (id < V) {
            const uint32_t slot = (id * 2654435761u) >> (32u - kHistSlotBits);
            const uint32_t prev = atomicCAS(&hk[slot], ~0u, id);
            if (prev == ~0u || prev == id) {
                atomicAdd(&hc[slot], 1u);
            } else {
                atomicAdd(a.hcount + (size_t)b * V + id, 1u);
                atomicOr(a.hbits + (size_t)b * a.hbw + (id >> 5), 1u << (id & 31u));
            }
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < kHistSlots; i += kPrepThreads) {
        const uint32_t id = hk[i];
        if (id != ~0u) {
            atomicAdd(a.hcount + (size_t)b * V + id, hc[i]);
            atomicOr(a.hbits + (size_t)b * a.hbw + (id >> 5), 1u << (id & 31u));
        }
    }
}

// Exclusive prefix sums of v[0, n) in place (LDS, every thread of the block calls it): each thread
// adds a contiguous chunk, a wave scan and one pass over the wave totals place the chunks. Returns
// the total; ends with a barrier.
__device__ uint32_t block_excl_scan_lds(uint32_t* v, uint32_t n, uint32_t* s_scan, uint32_t* s_tot) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t per = (n + kPrepThreads - 1u) / kPrepThreads, i0 = tid * per;
    uint32_t sum = 0u;
    for (uint32_t i = i0; i < i0 + per && i < n; ++i) sum += v[i];
    const uint32_t incl = wave_incl_scan(sum, lane);
    if (lane == 63u) s_scan[wave] = incl;
    __syncthreads();
    if (tid == 0u) {
        uint32_t run = 0u;
        for (uint32_t w = 0; w < kPrepWaves; ++w) { const uint32_t t = s_scan[w]; s_scan[w] = run; run += t; }
        *s_tot = run;
    }
    __syncthreads();
    uint32_t run = s_scan[wave] + incl - sum;
    for (uint32_t i = i0; i < i0 + per && i < n; ++i) {
        const uint32_t c = v[i];
        v[i] = run;
        run += c;
    }
    const uint32_t tot = *s_tot;
    __syncthreads();
    return tot;
}

// LDS words of the tile-bucket bias table of a row (two counters per tile and one past the last,
// then the keys and values of the list), or 0 when the counters alone would take more than 64 KB
// (the sort path then builds the table).
__host__ __device__ inline uint32_t bias_bucket_lds(uint32_t ntile, uint32_t P) {
    const uint32_t counters = 2u * (ntile + 1u);
    if (counters * 4u > 65536u) return 0u;
    return ((counters + 1u) & ~1u) * 4u + P * 12u;
}
// A tile holding more list entries than this sorts the whole row instead.
constexpr uint32_t kBucketMaxRun = 32;

// part 0: row b's history counts; part 1: row b's bias table (independent outputs, so the two
// run in separate blocks at the same time).
__device__ void modtable_row(const PrepArgs& a, uint32_t b, unsigned long long* keys, uint32_t part) {
#pragma clang fp contract(off)
    __shared__ uint32_t s_scan[kPrepWaves];
    __shared__ uint32_t s_nruns;
    const uint32_t tid = threadIdx.x;
    const uint32_t use = (a.mod_bits[b >> 4] >> (2u * (b & 15u))) & 3u;
    const uint32_t V = a.V;
    if (part == 0u) {
        if ((use & 1u) && a.history) history_counts(a, b, keys);
        return;
    }
    if (!(use & 2u) || !a.bias_ids) return;
    const uint32_t P = a.P;
    const uint32_t nb = min(a.bias_count[b], a.bias_stride);
    const uint32_t ntile = a.ntile;
    if (bias_bucket_lds(ntile, P) != 0u) {
        // Tile buckets instead of a sort of the whole list: count the entries per 64-id tile,
        // place them by the prefix of the counts, sort each tile's few entries by (id, list
        // position) in one thread, then count the distinct ids per tile and place those. The
        // table comes out the same as from the sort below; a tile with more than kBucketMaxRun
        // entries sends the row there instead.
        __shared__ uint32_t s_tot, s_long;
        uint32_t* cstart = reinterpret_cast<uint32_t*>(keys);   // [ntile + 1] counts, then starts
        uint32_t* fill = cstart + (ntile + 1u);                 // [ntile + 1] fill pointers, then distinct counts
        unsigned long long* slot = keys + ((2u * (ntile + 1u) + 1u) >> 1);  // [P] keys by tile
        float* vals = reinterpret_cast<float*>(slot + P);                    // [P] values by list position
        const uint32_t* ids = a.bias_ids + (size_t)b * a.bias_stride;
        for (uint32_t t = tid; t <= ntile; t += kPrepThreads) cstart[t] = 0u;
        if (tid == 0u) s_long = 0u;
        __syncthreads();
        for (uint32_t i = tid; i < nb; i += kPrepThreads) {
            const uint32_t id = ids[i];
            vals[i] = a.bias_vals[(size_t)b * a.bias_stride + i];
            if (id < V) atomicAdd(&cstart[id / kTileRows], 1u);
        }
        __syncthreads();
        for (uint32_t t = tid; t < ntile; t += kPrepThreads)
            if (cstart[t] > kBucketMaxRun) s_long = 1u;
        __syncthreads();
        if (s_long == 0u) {
            (void)block_excl_scan_lds(cstart, ntile + 1u, s_scan, &s_tot);
            for (uint32_t t = tid; t <= ntile; t += kPrepThreads) fill[t] = cstart[t];
            __syncthreads();
            for (uint32_t i = tid; i < nb; i += kPrepThreads) {
                const uint32_t id = ids[i];
                if (id < V) slot[atomicAdd(&fill[id / kTileRows], 1u)] = ((unsigned long long)id << 32) | i;
            }
            __syncthreads();
            // each tile's entries ascending by (id, position), then its distinct ids counted
            for (uint32_t t = tid; t < ntile; t += kPrepThreads) {
                const uint32_t s0 = cstart[t], s1 = cstart[t + 1u];
                for (uint32_t i = s0 + 1u; i < s1; ++i) {
                    const unsigned long long k = slot[i];
                    uint32_t j = i;
                    while (j > s0 && slot[j - 1u] > k) { slot[j] = slot[j - 1u]; --j; }
                    slot[j] = k;
                }
                uint32_t u = 0u;
                for (uint32_t i = s0; i < s1; ++i) u += (i == s0 || (slot[i - 1u] >> 32) != (slot[i] >> 32)) ? 1u : 0u;
                fill[t] = u;
            }
            if (tid == 0u) fill[ntile] = 0u;
            __syncthreads();
            const uint32_t nruns = block_excl_scan_lds(fill, ntile + 1u, s_scan, &s_tot);
            // block_start[t] = entries with id < 64 t; one entry per id, its values summed in
            // list order from 0.0f
            uint32_t* bs = a.block_start + (size_t)b * (ntile + 1u);
            ModEntry* mods = a.mods + (size_t)b * a.mod_cap;
            for (uint32_t t = tid; t <= ntile; t += kPrepThreads) {
                bs[t] = fill[t];
                if (t == ntile) continue;
                uint32_t e = fill[t];
                const uint32_t s0 = cstart[t], s1 = cstart[t + 1u];
                for (uint32_t i = s0; i < s1;) {
                    const uint32_t id = (uint32_t)(slot[i] >> 32);
                    float total = 0.0f;
                    for (; i < s1 && (uint32_t)(slot[i] >> 32) == id; ++i) total = total + vals[(uint32_t)slot[i]];
                    mods[e++] = ModEntry{id, 0u, total, 1u};
                }
            }
            if (tid == 0u) a.mod_count[b] = nruns;
            return;
        }
        // a long tile: the sort path below (its table layout differs; nothing of the above is kept)
        __syncthreads();
    }
    uint32_t* rs = reinterpret_cast<uint32_t*>(keys + P);  // run starts, [nruns + 1] <= P + 1
    float* vals = reinterpret_cast<float*>(rs + P + 2u);    // the list's values, by position
    const unsigned long long kPad = ~0ull;
    for (uint32_t i = tid; i < P; i += kPrepThreads) {
        unsigned long long k = kPad;
        if (i < nb) {
            const uint32_t id = a.bias_ids[(size_t)b * a.bias_stride + i];
            vals[i] = a.bias_vals[(size_t)b * a.bias_stride + i];  // loaded beside the id
            if (id < V) k = ((unsigned long long)id << 32) | i;
        }
        keys[i] = k;
    }
    __syncthreads();
    block_sort_u64<kPrepThreads>(keys, P);
    // Run starts (first key of each id; pads sort last) -> entry index by a block scan over
    // per-thread counts of consecutive keys.
    const uint32_t per = (P + kPrepThreads - 1u) / kPrepThreads;
    const uint32_t i0 = tid * per;
    auto starts_run = [&](uint32_t i) {
        const unsigned long long k = keys[i];
        return k != kPad && (i == 0u || (keys[i - 1u] >> 32) != (k >> 32));
    };
    uint32_t cnt = 0;
    for (uint32_t i = i0; i < i0 + per && i < P; ++i) cnt += starts_run(i) ? 1u : 0u;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t incl = wave_incl_scan(cnt, lane);
    if (lane == 63u) s_scan[wave] = incl;
    __syncthreads();
    if (tid == 0u) {
        uint32_t run = 0;
        for (uint32_t w = 0; w < kPrepWaves; ++w) { const uint32_t t = s_scan[w]; s_scan[w] = run; run += t; }
        s_nruns = run;
    }
    __syncthreads();
    const uint32_t nruns = s_nruns;
    uint32_t e = s_scan[wave] + incl - cnt;
    for (uint32_t i = i0; i < i0 + per && i < P; ++i) {
        if (starts_run(i)) rs[e++] = i;
        // the last valid key closes the final run
        if (keys[i] != kPad && (i + 1u == P || keys[i + 1u] == kPad)) rs[nruns] = i + 1u;
    }
    __syncthreads();
    // One entry per id: its bias values summed in list order from 0.0f.
    ModEntry* mods = a.mods + (size_t)b * a.mod_cap;
    for (uint32_t r = tid; r < nruns; r += kPrepThreads) {
        const uint32_t s0 = rs[r], s1 = rs[r + 1u];
        float total = 0.0f;
        for (uint32_t t = s0; t < s1; ++t) total = total + vals[(uint32_t)keys[t]];
        mods[r] = ModEntry{(uint32_t)(keys[s0] >> 32), 0u, total, 1u};
    }
    // block_start[t] = number of entries with id < 64 t. Each thread covers a contiguous range of
    // tiles: one binary search over the run ids for its first tile, then a walk upwards (the ids
    // are sorted).
    uint32_t* bs = a.block_start + (size_t)b * (ntile + 1u);
    const uint32_t tper = (ntile + 1u + kPrepThreads - 1u) / kPrepThreads;
    const uint32_t t0 = tid * tper;
    if (t0 <= ntile) {
        uint32_t lo = 0, hi = nruns;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if ((uint32_t)(keys[rs[mid]] >> 32) < t0 * kTileRows) lo = mid + 1u;
            else hi = mid;
        }
        for (uint32_t t = t0; t < t0 + tper && t <= ntile; ++t) {
            while (lo < nruns && (uint32_t)(keys[rs[lo]] >> 32) < t * kTileRows) ++lo;
            bs[t] = lo;
        }
    }
    if (tid == 0u) a.mod_count[b] = nruns;
}

// Grid: [row copy block if rows_dst] [B x ceil(D / 1024) RMSNorm blocks if hidden]
// [B history blocks, then B bias-table blocks, if mods].
__global__ __launch_bounds__(kPrepThreads) void k_step_prep(PrepArgs a) {
    // The modifier blocks' table (history merge, then bias keys and run starts), sized per launch:
    // dynamic, so that launches without modifiers, or with small bias lists, fit several blocks
    // per CU.
    extern __shared__ unsigned long long pool[];
    uint32_t blk = blockIdx.x;
    if (a.rows_dst) {
        if (blk == 0u) {
            // From the kernel arguments, or a PCIe round trip to the pinned staging slot: on a
            // block of its own, so no other block waits for it.
            const uint32_t* src = a.rows_src ? reinterpret_cast<const uint32_t*>(a.rows_src)
                                             : reinterpret_cast<const uint32_t*>(&a.inl[0]);
            uint32_t* dst = reinterpret_cast<uint32_t*>(a.rows_dst);
            for (uint32_t i = threadIdx.x; i < (uint32_t)a.B * (sizeof(DevRow) / 4); i += kPrepThreads)
                dst[i] = src[i];
            return;
        }
        --blk;
    }
    if (a.hidden) {
        const uint32_t per = (a.D + kPrepThreads - 1u) / kPrepThreads;  // RMSNorm blocks per row
        if (blk < (uint32_t)a.B * per) {
            prep_row(a, blk / per, blk % per);
            return;
        }
        blk -= (uint32_t)a.B * per;
    }
    modtable_row(a, blk % (uint32_t)a.B, pool, blk / (uint32_t)a.B);
}

void launch_step_prep(const Head& h, const PrepArgs& a, bool with_mods, hipStream_t st) {
    const unsigned per = (a.D + kPrepThreads - 1u) / kPrepThreads;
    const unsigned grid = (a.rows_dst ? 1u : 0u) + (a.hidden ? (unsigned)a.B * per : 0u) +
                          (with_mods ? 2u * (unsigned)a.B : 0u);
    if (grid == 0u) return;
    // LDS for the modifier blocks: the history table (kHistSlots ids + counts) or P bias keys,
    // P + 1 run starts and P values (P <= mod_cap), whichever is larger; none without modifiers.
    size_t lds = 0;
    if (with_mods) {
        const size_t hist = 2u * kHistSlots * sizeof(uint32_t);
        const size_t bias = (size_t)a.P * sizeof(unsigned long long) + ((size_t)a.P + 2u) * sizeof(uint32_t) +
                            (size_t)a.P * sizeof(float);
        const size_t bucket = bias_bucket_lds(a.ntile, a.P);
        lds = (std::max(std::max(hist, bias), bucket) + 15u) & ~(size_t)15u;
    }
    if (lds > 65536u) {
        static_assert(kModCap * 16u + 16u <= 160u * 1024u, "the largest table must fit one CU's LDS");
        check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(k_step_prep),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                  "step prep LDS size");
    }
    hipLaunchKernelGGL(k_step_prep, dim3(grid), dim3(kPrepThreads), lds, st, a);
    check_hip(hipGetLastError(), "step prep");
}

uint32_t modtable_sort_size(const Head& h, uint32_t n) {
    uint32_t P = 2;
    while (P < n) P <<= 1;
    if (P > h.mod_cap)
        throw std::runtime_error("bias_stride exceeds the per-row bias-entry limit of " +
                                 std::to_string(h.mod_cap));
    return P;
}

}  // namespace tdt
