// Token selection: greedy argmax or the sampled draw of sample_token (src/sampling.cpp:92-169).
//
// One 1024-thread workgroup per batch row, reading the row's final logits and the per-64-id
// block partials the head epilogue wrote (max, lowest argmax, sum exp(l - max), finite min,
// second-largest value).
//
//  greedy     argmax of the block partials, ties to the lowest id (:97-104).
//  shortlist  (want = top_k, or 256 without the full-vocabulary flag; :122-137)
//             tau, a lower bound of the want-th largest block maximum and so of the want-th
//             largest logit: from a 256-bin window of width 1/32 below the row maximum, else a
//             2048-bin histogram of the block maxima, else the exact 22-bit key bound. Every
//             shortlist member lies in a block whose maximum is >= tau. A block whose
//             second-largest value is below tau contributes only its maximum, taken from the
//             partial; the other qualifying blocks are gathered (elements >= tau). The
//             candidates are ranked by (logit desc, id asc) (counting ranks up to 256, a bitonic
//             sort beyond), and the first `want` form the shortlist. Nucleus over
//             full-distribution probabilities (:139-151) and the temperature draw (:153-168) run
//             as double-precision scans (one wave up to 64 entries).
//  full vocabulary (top_k = 0 with the full-vocabulary flag; the full-sort sampler of
//             tests/test_sampling.cpp:36-84): one pass builds 2048-bin histograms of both the
//             T = 1 and the temperature weights over equal-width logit-value bins spanning
//             [lo, max] (bin order is rank order); one wave plans the nucleus bin and the bins
//             the draw can land in (bounded before the cut is known), whose elements a second
//             pass gathers. The crossings inside a bin are narrowed by 2048 sub-bins and resolved
//             exactly over a sorted sub-bin. Steps with at most 64 such rows split each one's
//             passes over 4 - 32 workgroups (k_fv_hist, k_fv_gather, k_fv_finish).
//  fallback   shortlist overflow or a bin too large to gather (massive ties): weighted radix
//             select over the order-preserving keys, with ties among equal keys (equal
//             weights) resolved by count and a radix select over ids.
//
// Weight histograms accumulate in LDS as u64 fixed point (w * 2^40, weights relative to the
// row maximum are <= 1): integer LDS atomics run an order of magnitude faster than float ones
// on gfx950. Truncation changes a row total by at most V * 2^-40 relative. Scans of those
// histograms add exact integer sums.
#include <algorithm>
#include <stdexcept>

#include "dt_internal.h"
#include "dt_sort.h"

namespace tdt {

// Workgroups run 1024 threads. Device code reads the size at run time; a 512-thread form measured
// slower on the B = 1 row, and the full-vocabulary passes want every wave for their loads.
constexpr uint32_t kMaxSelThreads = 1024;
constexpr uint32_t kMaxSelWaves = kMaxSelThreads / 64;
__device__ inline uint32_t sel_nt() { return (uint32_t)__builtin_amdgcn_workgroup_size_x(); }
__device__ inline uint32_t sel_nw() { return sel_nt() >> 6; }
constexpr uint32_t kCandCap = 8192;
constexpr uint32_t kTileCap = 2048;
constexpr uint32_t kBins = 2048;
constexpr uint32_t kVBins = 2048;
constexpr uint32_t kKeyCache = 8192;  // block-maximum keys kept in LDS (ntile <= 8192)
constexpr uint32_t kRegTiles = 4096;    // block partials held in registers (kRegTiles / threads each)
constexpr uint32_t kGatherChunk = 8192;   // shortlist gather: elements loaded per workgroup round
constexpr int kInflight = 4;          // float4 loads in flight per thread in row passes
constexpr double kFx = 1099511627776.0;  // 2^40: fixed-point scale of histogram weights

// Must match TurboRowReport in include/turbo_decode_tail.h.
struct RowReport {
    float max_logit;
    float u;
    uint32_t shortlist;
    uint32_t cut;
    uint32_t rank;
    uint32_t path;
    double total;
    double denom;
    double r;
    uint32_t status;
    uint32_t reserved;
};

struct SelShared {
    union {
        unsigned long long hd[kBins];  // key-bin weights, fixed point
        uint32_t hu[kBins];
        struct {
            unsigned long long vm[kVBins];  // value-bin weights, T = 1, fixed point
            unsigned long long vq[kVBins];  // value-bin weights, temperature T, fixed point
        };
    };
    __attribute__((aligned(16))) unsigned long long cand[kCandCap];
    uint32_t tiles[kTileCap];
    uint32_t pkey[kKeyCache];
    double wsum_d[kMaxSelWaves];
    uint32_t wsum_u[kMaxSelWaves];
    float wmax[kMaxSelWaves];
    uint32_t warg[kMaxSelWaves];
    float wmin[kMaxSelWaves];
    float wzm[kMaxSelWaves];
    double wzs[kMaxSelWaves];
    double bd[4];
    uint32_t bu[8];
    uint32_t ntile_q;   // shortlist: qualifying tiles appended (zeroed at kernel start)
    uint32_t ncand_q;   // shortlist: gathered candidates appended (zeroed at kernel start)
};

// ---- block primitives ------------------------------------------------------------------------

template <typename T>
__device__ inline T* wslot(SelShared& s);
template <>
__device__ inline double* wslot<double>(SelShared& s) { return s.wsum_d; }
template <>
__device__ inline uint32_t* wslot<uint32_t>(SelShared& s) { return s.wsum_u; }

// Exclusive scan over the block in thread order; returns the exclusive prefix, total in *tot.
template <typename T>
__device__ __attribute__((always_inline)) inline T block_excl_scan(T v, SelShared& s, T* tot) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const T incl = wave_incl_scan(v, lane);
    T* ws = wslot<T>(s);
    __syncthreads();
    if (lane == 63u) ws[wave] = incl;
    __syncthreads();
    T off = T(0), all = T(0);
    for (uint32_t w = 0; w < sel_nw(); ++w) {
        const T x = ws[w];
        if (w < wave) off += x;
        all += x;
    }
    if (tot) *tot = all;
    __syncthreads();
    return off + incl - v;
}

template <typename T>
__device__ inline T block_sum(T v, SelShared& s) {
    T tot;
    (void)block_excl_scan(v, s, &tot);
    return tot;
}

__device__ inline uint32_t block_min_u(uint32_t v, SelShared& s) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    v = wave_min_u(v);
    __syncthreads();
    if (lane == 0) s.wsum_u[wave] = v;
    __syncthreads();
    uint32_t r = 0xFFFFFFFFu;
    for (uint32_t w = 0; w < sel_nw(); ++w) r = min(r, s.wsum_u[w]);
    __syncthreads();
    return r;
}

// Key histogram scan from the highest bin down: the bin where the running total first reaches
// `target` (before < target <= before + h). Returns 1 with bin/above when target <= total;
// otherwise 0, or with `clamp` target = total (the last non-empty bin). nb is 2048 or 1024.
template <typename T>
__device__ inline T hist_at(SelShared& s, uint32_t i);
template <>
__device__ inline double hist_at<double>(SelShared& s, uint32_t i) { return (double)s.hd[i] / kFx; }
template <>
__device__ inline uint32_t hist_at<uint32_t>(SelShared& s, uint32_t i) { return s.hu[i]; }

template <typename T>
__device__ inline int hist_cross(SelShared& s, uint32_t nb, T target, uint32_t* bin, T* above,
                                 bool clamp = false) {
    const uint32_t tid = threadIdx.x;
    const uint32_t per = nb / sel_nt();
    T loc = T(0);
    for (uint32_t j = 0; j < per; ++j) loc += hist_at<T>(s, nb - 1u - (tid * per + j));
    T tot;
    T before = block_excl_scan(loc, s, &tot);
    if (target > tot) {
        if (!clamp) return 0;  // uniform: tot is the same in every thread
        target = tot;
    }
    if (tid == 0) s.bu[0] = 0xFFFFFFFFu;
    __syncthreads();
    for (uint32_t j = 0; j < per; ++j) {
        const uint32_t bi = nb - 1u - (tid * per + j);
        const T hv = hist_at<T>(s, bi);
        if (before < target && target <= before + hv) {
            s.bu[0] = bi;
            if (sizeof(T) == 8) s.bd[0] = (double)before;
            else s.bu[1] = (uint32_t)before;
        }
        before += hv;
    }
    __syncthreads();
    const uint32_t r = s.bu[0];
    T ab;
    if (sizeof(T) == 8) ab = (T)s.bd[0];
    else ab = (T)s.bu[1];
    __syncthreads();
    if (r == 0xFFFFFFFFu) return 0;
    *bin = r;
    *above = ab;
    return 1;
}

// Sorts s.cand[0, n) ascending with the bitonic network (n padded to a power of two).
__device__ __attribute__((always_inline)) inline void sort_cand(SelShared& s, uint32_t n) {
    const uint32_t tid = threadIdx.x;
    uint32_t P = 2;
    while (P < n) P <<= 1;
    for (uint32_t i = n + tid; i < P; i += sel_nt()) s.cand[i] = ~0ull;
    __syncthreads();
    if (sel_nt() == kMaxSelThreads) block_sort_u64<kMaxSelThreads>(s.cand, P);
    else block_sort_u64<256>(s.cand, P);
}

// Stream compaction with one LDS atomic per wave: the active lanes with pred get consecutive
// slots (in lane order) of dst through *counter; slots past cap are counted but not stored.
template <typename T>
__device__ __attribute__((always_inline)) inline void wave_append(uint32_t* counter, bool pred, T key, T* dst,
                                                                  uint32_t cap) {
    const unsigned long long mask = __ballot(pred);
    if (mask == 0ull) return;
    const uint32_t lane = threadIdx.x & 63u;
    const int leader = __ffsll((long long)mask) - 1;
    uint32_t base = 0u;
    if ((int)lane == leader) base = atomicAdd(counter, (uint32_t)__popcll(mask));
    base = lane_read(base, leader);
    if (pred) {
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
        if (base + rank < cap) dst[base + rank] = key;
    }
}

// Sum of v over aligned groups of P consecutive lanes (P a power of two <= 64, wave-uniform);
// every lane of a group receives the group's sum. All 64 lanes must be active.
__device__ inline uint32_t group_sum(uint32_t v, uint32_t P) {
    if (P >= 2u) v += dpp_mov<dpp::kXor1>(v);
    if (P >= 4u) v += dpp_mov<dpp::kXor2>(v);
    if (P >= 8u) v += dpp_mov<dpp::kHalfMirror>(v);
    if (P >= 16u) v += dpp_mov<dpp::kRor8>(v);
    if (P >= 32u) v += (uint32_t)__shfl_xor((int)v, 16, 64);
    if (P >= 64u) v += xor32(v);
    return v;
}

// Places the W smallest of the n (at most one per thread) distinct keys s.cand[0, n) in ascending order
// at s.cand[0, W). Each key's rank is counted by a group of P threads (P as large as the block
// allows), each over every P-th key, and summed across the group.
__device__ __attribute__((always_inline)) inline void rank_top(SelShared& s, uint32_t n, uint32_t W) {
    const uint32_t tid = threadIdx.x;
    uint32_t lg = 0;
    while (lg < 6u && (n << (lg + 1u)) <= sel_nt()) ++lg;
    const uint32_t P = 1u << lg;
    const uint32_t i = tid >> lg, part = tid & (P - 1u);
    unsigned long long k = 0ull;
    uint32_t r = 0u;
    if (i < n) {
        k = s.cand[i];
        for (uint32_t j = part; j < n; j += P) r += (s.cand[j] < k) ? 1u : 0u;
    }
    r = group_sum(r, P);
    __syncthreads();
    if (i < n && part == 0u && r < W) s.cand[r] = k;
    __syncthreads();
}

// A row pass reads float4s when the row allows it (length a multiple of 4, 16-byte aligned).
__device__ inline bool row_vec(const float* l, uint32_t V) { return (V & 3u) == 0u && ((uintptr_t)l & 15u) == 0u; }

// The first round of a row pass's loads, issued ahead of work the pass does not depend on (the
// row parameters) so that their latency overlaps it. Holds nothing for a row that takes the
// scalar pass.
struct RowPre {
    float4 q[kInflight];
};
__device__ inline void row_preload(const float* l, uint32_t V, RowPre& p) {
    if (!row_vec(l, V)) return;
    const float4* l4 = reinterpret_cast<const float4*>(l);
    const uint32_t V4 = V >> 2;
#pragma unroll
    for (int j = 0; j < kInflight; ++j) {
        const uint32_t idx = (uint32_t)j * sel_nt() + threadIdx.x;
        p.q[j] = (idx < V4) ? l4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Visits every (value, index) of a row with kInflight independent loads per thread in flight;
// the first round comes from pre when given (row_preload of the same l and V).
template <class F>
__device__ inline void row_pass(const float* l, uint32_t V, F&& f, const RowPre* pre = nullptr) {
    const uint32_t tid = threadIdx.x;
    if (row_vec(l, V)) {
        const float4* l4 = reinterpret_cast<const float4*>(l);
        const uint32_t V4 = V >> 2;
        for (uint32_t base = 0; base < V4; base += kInflight * sel_nt()) {
            float4 q[kInflight];
            if (pre && base == 0u) {
#pragma unroll
                for (int j = 0; j < kInflight; ++j) q[j] = pre->q[j];
            } else {
#pragma unroll
                for (int j = 0; j < kInflight; ++j) {
                    const uint32_t idx = base + (uint32_t)j * sel_nt() + tid;
                    q[j] = (idx < V4) ? l4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int j = 0; j < kInflight; ++j) {
                const uint32_t idx = base + (uint32_t)j * sel_nt() + tid;
                if (idx < V4) {
                    f(q[j].x, 4u * idx);
                    f(q[j].y, 4u * idx + 1u);
                    f(q[j].z, 4u * idx + 2u);
                    f(q[j].w, 4u * idx + 3u);
                }
            }
        }
    } else {
        for (uint32_t base = 0; base < V; base += 4u * kInflight * sel_nt()) {
            float q[4 * kInflight];
#pragma unroll
            for (int j = 0; j < 4 * kInflight; ++j) {
                const uint32_t idx = base + (uint32_t)j * sel_nt() + tid;
                q[j] = (idx < V) ? l[idx] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 4 * kInflight; ++j) {
                const uint32_t idx = base + (uint32_t)j * sel_nt() + tid;
                if (idx < V) f(q[j], idx);
            }
        }
    }
}

// ---- per-row context ---------------------------------------------------------------------------

struct RowCtx {
    uint32_t V;
    const float* l;      // row logits
    float m;             // row max
    float T;             // temperature
    uint2* list;         // compaction scratch [V] (radix fallback)
    float inv_w;         // value bins: bin(l) = (m - l) * inv_w, clamped to the last bin
};

// Equal-width value bins over [lo, m], bin 0 holding the largest logits. Monotone in the logit,
// so bin order is rank order. -inf and values below lo land in the last bin.
__device__ inline uint32_t vbin(const RowCtx& c, float l) {
    const float d = (c.m - l) * c.inv_w;
    return (d < (float)(kVBins - 1)) ? (uint32_t)d : kVBins - 1u;
}
// The same bin from dl = l - m, which a weight needs anyway: m - l = -(l - m) and the product
// with -inv_w round identically, so this equals vbin(c, l).
__device__ inline uint32_t vbin_d(const RowCtx& c, float dl) {
    const float d = dl * -c.inv_w;
    return (d < (float)(kVBins - 1)) ? (uint32_t)d : kVBins - 1u;
}

constexpr float kLog2e = 1.4426950408889634f;

// floor(w 2^40) for a weight w in [0, 1]: the integer part of a = w 2^8 is the high word and
// that of frac(a) 2^32 the low word (both products are exact scalings), five instructions where
// the float-to-u64 conversion takes seven, once per element of a row pass.
__device__ inline unsigned long long to_fx(float w) {
    const float a = w * 256.0f;
    const uint32_t hi = (uint32_t)a;
    const uint32_t lo = (uint32_t)(__builtin_amdgcn_fractf(a) * 4294967296.0f);
    return ((unsigned long long)hi << 32) | lo;
}

// Weight of logit v: mode 0 count, 1 exp(v - m), 2 exp((v - m) / T); hardware exp2.
__device__ inline float weight_f(const RowCtx& c, float v, int mode) {
    if (mode == 0) return 1.0f;
    if (v == -INFINITY) return 0.0f;
    const float k = (mode == 1) ? kLog2e : kLog2e / c.T;
    return __builtin_amdgcn_exp2f((v - c.m) * k);
}

// Prefix set in (key desc, id asc) order: bounded by element (kb, ib) inclusive, or everything.
struct PSet {
    int bounded;
    uint32_t kb, ib;
    __device__ bool has(uint32_t k, uint32_t id) const {
        return !bounded || k > kb || (k == kb && id <= ib);
    }
};

// ---- radix fallback ------------------------------------------------------------------------------

// Radix select over ids: the j-th smallest id (0-based) among list entries with key == kx.
__device__ inline uint32_t select_tied_id(SelShared& s, const uint2* list, uint32_t n, uint32_t kx,
                                          uint32_t j) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0, rem = j + 1;  // rank from the bottom, 1-based
    for (int lv = 0; lv < 3; ++lv) {
        const uint32_t nb = (lv < 2) ? 2048u : 1024u;
        const uint32_t sh = (lv == 0) ? 21u : (lv == 1) ? 10u : 0u;
        for (uint32_t i = tid; i < kBins; i += sel_nt()) s.hu[i] = 0u;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += sel_nt()) {
            const uint2 e = list[i];
            if (e.x == kx && (e.y & mask) == prefix) atomicAdd(&s.hu[(e.y >> sh) & (nb - 1u)], 1u);
        }
        __syncthreads();
        // smallest ids first: mirror the bins for hist_cross, which scans from the top
        for (uint32_t i = tid; i < nb / 2; i += sel_nt()) {
            const uint32_t t = s.hu[i];
            s.hu[i] = s.hu[nb - 1u - i];
            s.hu[nb - 1u - i] = t;
        }
        __syncthreads();
        uint32_t bin = 0, above = 0;
        if (!hist_cross<uint32_t>(s, nb, rem, &bin, &above, true)) return 0xFFFFFFFFu;
        const uint32_t d = nb - 1u - bin;
        rem -= above;
        prefix |= d << sh;
        mask |= (nb - 1u) << sh;
    }
    return prefix;
}

// First element of set `ps`, in (key desc, id asc) order, whose cumulative weight reaches
// `target`. Returns 1 with (*kx, *ix); 0 when the set's total weight is below target.
__device__ __attribute__((always_inline)) inline int find_cross(SelShared& s, const RowCtx& c, const PSet& ps, int mode, double target,
                          uint32_t* kx, uint32_t* ix) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < kBins; i += sel_nt()) s.hd[i] = 0ull;
    __syncthreads();
    row_pass(c.l, c.V, [&](float v, uint32_t i) {
        const uint32_t k = float_key(v);
        if (!ps.has(k, i)) return;
        const float w = weight_f(c, v, mode);
        if (w != 0.0f) atomicAdd(&s.hd[k >> 21], to_fx(w));
    });
    __syncthreads();
    uint32_t d1;
    double above;
    if (!hist_cross<double>(s, kBins, target, &d1, &above)) return 0;
    double rem = target - above;
    if (tid == 0) s.bu[2] = 0u;
    __syncthreads();
    row_pass(c.l, c.V, [&](float v, uint32_t i) {
        const uint32_t k = float_key(v);
        if ((k >> 21) != d1 || !ps.has(k, i)) return;
        const uint32_t slot = atomicAdd(&s.bu[2], 1u);
        c.list[slot] = make_uint2(k, i);
    });
    __syncthreads();
    const uint32_t n = s.bu[2];
    __syncthreads();
    uint32_t prefix = d1 << 21, mask = 0xFFE00000u;
    for (int lv = 0; lv < 2; ++lv) {
        const uint32_t nb = (lv == 0) ? 2048u : 1024u;
        const uint32_t sh = (lv == 0) ? 10u : 0u;
        for (uint32_t i = tid; i < kBins; i += sel_nt()) s.hd[i] = 0ull;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += sel_nt()) {
            const uint2 e = c.list[i];
            if ((e.x & mask) != prefix) continue;
            const float w = weight_f(c, key_float(e.x), mode);
            if (w != 0.0f) atomicAdd(&s.hd[(e.x >> sh) & (nb - 1u)], to_fx(w));
        }
        __syncthreads();
        uint32_t d;
        double ab;
        // the bucket's weight was summed in another order at the previous level: clamp
        if (!hist_cross<double>(s, nb, rem, &d, &ab, true)) return 0;
        rem -= ab;
        prefix |= d << sh;
        mask |= (nb - 1u) << sh;
    }
    const uint32_t kk = prefix;
    // ties: equal keys have equal weight w; the crossing is the j-th smallest tied id with
    // (j + 1) * w >= rem
    uint32_t nt = 0;
    for (uint32_t i = tid; i < n; i += sel_nt()) nt += (c.list[i].x == kk) ? 1u : 0u;
    nt = block_sum<uint32_t>(nt, s);
    const double w = (double)weight_f(c, key_float(kk), mode);
    uint32_t j = 0;
    if (w > 0.0 && nt > 0u) {
        const double q = ceil(rem / w) - 1.0;
        j = (q <= 0.0) ? 0u : (q >= (double)(nt - 1u) ? nt - 1u : (uint32_t)q);
    }
    const uint32_t id = select_tied_id(s, c.list, n, kk, j);
    if (id == 0xFFFFFFFFu) return 0;
    *kx = kk;
    *ix = id;
    return 1;
}

// ---- full-vocabulary path on value bins ------------------------------------------------------------

// One wave's lane sums of a kVBins histogram (lane l: bins 32 l .. 32 l + 31, exact integers)
// and their inclusive and exclusive prefixes, for several crossing searches over one histogram.
// Lane l adds its 32 bins starting at bin (l mod 32) of its range: read in bin order, the lanes'
// 256-byte-apart addresses would all fall in one LDS bank on every read. Integer sums do not
// depend on the order.
struct WaveHist {
    unsigned long long loc, incl, run;
};
__device__ __attribute__((always_inline)) inline WaveHist wave_hist(const unsigned long long* h) {
    constexpr uint32_t kPer = kVBins / 64u;
    static_assert((kPer & (kPer - 1u)) == 0u, "the rotated read needs a power-of-two range per lane");
    const uint32_t lane = threadIdx.x & 63u, b0 = lane * kPer;
    WaveHist w;
    w.loc = 0ull;
#pragma unroll 8
    for (uint32_t j = 0; j < kPer; ++j) w.loc += h[b0 + ((j + lane) & (kPer - 1u))];
    w.incl = wave_incl_scan(w.loc, lane);
    w.run = w.incl - w.loc;
    return w;
}

// A crossing search's answer, returned by value (out-parameters chosen per path kept these
// values in scratch memory): found with the bin and the weight before it, or not found with
// the weight of the whole range searched.
struct Cross {
    int found;
    uint32_t bin;
    double w;
};

__device__ inline double fx_of(unsigned long long v) { return (double)v / kFx; }

// The bins of lane L (bin 32 L + j on lane j, bins at or past limit counted as 0) from base, the
// weight below them: the first bin where the running total reaches target.
__device__ __attribute__((always_inline)) inline Cross lane_cross(const unsigned long long* h, uint32_t L,
                                                                  unsigned long long base, uint32_t limit,
                                                                  double target) {
    constexpr uint32_t kPer = kVBins / 64u;
    static_assert(kPer <= 64u, "a lane's bins are resolved one per lane");
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t bj = L * kPer + (lane & (kPer - 1u));
    const unsigned long long hv = (lane < kPer && bj < limit) ? h[bj] : 0ull;
    const unsigned long long ci = base + wave_incl_scan(hv, lane), ce = ci - hv;
    const unsigned long long at = __ballot(hv != 0ull && fx_of(ce) < target && target <= fx_of(ci));
    if (at == 0ull) return Cross{0, 0u, fx_of(lane_read(ci, 63))};
    const uint32_t F = (uint32_t)__ffsll((long long)at) - 1u;
    return Cross{1, L * kPer + F, fx_of(lane_read(ce, (int)F))};
}

// Weight-histogram scan from bin 0 up over bins [0, limit) of h (kVBins u64 fixed-point
// weights), by the 64 lanes of one wave: the bin where the running total first reaches target
// (before < target <= before + h[bin]), or not found with the total of the range; every lane
// gets the same answer. Each lane adds 32 bins as exact integers, a wave scan finds the lane
// whose range holds the crossing, and that lane's 32 bins, one per lane, find the bin.
__device__ __attribute__((always_inline)) inline Cross wave_cross(const unsigned long long* h, uint32_t limit,
                                                                  double target) {
    constexpr uint32_t kPer = kVBins / 64u;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t b0 = lane * kPer;
    unsigned long long loc = 0ull;
#pragma unroll 8
    for (uint32_t j = 0; j < kPer; ++j) {
        const uint32_t bj = b0 + ((j + lane) & (kPer - 1u));  // rotated, as in wave_hist
        loc += (bj < limit) ? h[bj] : 0ull;
    }
    const unsigned long long incl = wave_incl_scan(loc, lane), run = incl - loc;
    const unsigned long long hit = __ballot(loc != 0ull && fx_of(run) < target && target <= fx_of(incl));
    if (hit == 0ull) return Cross{0, 0u, fx_of(lane_read(incl, 63))};
    const uint32_t L = (uint32_t)__ffsll((long long)hit) - 1u;
    const unsigned long long base = lane_read(run, (int)L);
    const Cross r = lane_cross(h, L, base, limit, target);
    if (r.found) return r;
    // unreachable: the sums are monotone and lane L's range holds target
    return Cross{1, min(L * kPer + kPer - 1u, limit - 1u), fx_of(base)};
}

// wave_cross over bins [0, limit) of h from its lane sums H (the same answers): lanes whose bins
// all lie below limit are searched on H, and the lane holding limit, if any, bin by bin.
__device__ __attribute__((always_inline)) inline Cross wave_cross_pre(const unsigned long long* h, const WaveHist& H,
                                                                      uint32_t limit, double target) {
    constexpr uint32_t kPer = kVBins / 64u;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t Lfull = limit / kPer;  // lanes 0 .. Lfull - 1 lie wholly below limit
    const unsigned long long hit =
        __ballot(lane < Lfull && H.loc != 0ull && fx_of(H.run) < target && target <= fx_of(H.incl));
    if (hit != 0ull) {
        const uint32_t L = (uint32_t)__ffsll((long long)hit) - 1u;
        const unsigned long long base = lane_read(H.run, (int)L);
        const Cross r = lane_cross(h, L, base, limit, target);
        if (r.found) return r;
        // unreachable: the sums are monotone and lane L's range holds target
        return Cross{1, L * kPer + kPer - 1u, fx_of(base)};
    }
    const unsigned long long base = (Lfull > 0u) ? lane_read(H.incl, (int)Lfull - 1) : 0ull;
    if (Lfull < 64u && Lfull * kPer < limit) return lane_cross(h, Lfull, base, limit, target);
    return Cross{0, 0u, fx_of(base)};
}

// wave_cross for the whole block: wave 0 scans while the other waves wait at one barrier (a
// block-wide scan costs several barriers, and each phase between them issues on four waves
// per SIMD). Returns 1 with bin/above, or 0 with *above = the range's total.
__device__ __attribute__((always_inline)) inline int scan_cross(SelShared& s, const unsigned long long* h,
                                                                uint32_t limit, double target, uint32_t* bin,
                                                                double* above) {
    const uint32_t tid = threadIdx.x;
    if (tid < 64u) {
        const Cross r = wave_cross(h, limit, target);
        if (tid == 0u) {
            s.bu[0] = r.found ? r.bin : 0xFFFFFFFFu;
            s.bd[0] = r.w;
        }
    }
    __syncthreads();
    const uint32_t r = s.bu[0];
    const double ab = s.bd[0];
    __syncthreads();
    *above = ab;
    if (r == 0xFFFFFFFFu) return 0;
    *bin = r;
    return 1;
}

// ---- full-vocabulary nucleus over value bins ------------------------------------------------
// Pieces shared by the one-workgroup path (full_vocab_value_path) and the multi-workgroup path
// of small batches (k_fv_hist, k_select, k_fv_gather, k_fv_finish): histogram, plan, gather, finish.

// Bins the finish needs: the nucleus bin cb and the range [dlo, dhi] the draw can land in.
struct FvPlan {
    uint32_t cb, dlo, dhi, u_zero;  // u_zero: u = 0 picks the first element in sorted order
    double A;                       // survivor weight (temperature) of the bins above cb
    double target_w, wabove;        // T = 1 nucleus target, and the T = 1 weight above cb
    double total;                   // sum exp(l - m) over the row, from the T = 1 histogram
    unsigned long long dlo_before;  // temperature weight of the bins above dlo (fixed point)
    uint32_t dlo_found;             // dlo is the crossing bin of u A (not a clamped fallback)
};

__device__ inline bool same_weights(const RowCtx& c) { return kLog2e / c.T == kLog2e; }

// Value-bin weight histograms (T = 1 in vm, temperature T in vq) of elements [beg, end).
__device__ __attribute__((always_inline)) inline void fv_hist(SelShared& s, const RowCtx& c, uint32_t beg, uint32_t end,
                                                              const RowPre* pre = nullptr) {
    const float kq = kLog2e / c.T;
    const bool same = same_weights(c);  // T = 1: one weighting serves nucleus and draw
    for (uint32_t i = threadIdx.x; i < kVBins; i += sel_nt()) { s.vm[i] = 0ull; s.vq[i] = 0ull; }
    __syncthreads();
    row_pass(c.l + beg, end - beg, [&](float v, uint32_t) {
        if (v == -INFINITY) return;
        const float d = v - c.m;
        const uint32_t b = vbin_d(c, d);
        atomicAdd(&s.vm[b], to_fx(__builtin_amdgcn_exp2f(d * kLog2e)));
        if (!same) atomicAdd(&s.vq[b], to_fx(__builtin_amdgcn_exp2f(d * kq)));
    }, pre);
    __syncthreads();
}

// From complete histograms in s.vm / s.vq: the nucleus bin and the draw range.
__device__ __attribute__((always_inline)) inline void fv_plan(SelShared& s, const RowCtx& c, float top_p, float u, FvPlan* P) {
    // wave 0 runs the five scans back to back on lane sums taken once per histogram, and hands
    // the plan over through LDS
    FvPlan* sp = reinterpret_cast<FvPlan*>(s.cand);
    if (threadIdx.x < 64u) {
        const bool same = same_weights(c);
        const unsigned long long* hq = same ? s.vm : s.vq;
        const WaveHist Hm = wave_hist(s.vm);
        const WaveHist Hq = same ? Hm : wave_hist(s.vq);
        // nucleus bin: where the T = 1 weight reaches top_p of the row total
        uint32_t cb = kVBins;
        double target_w = 0.0, wabove = 0.0;
        const double total = wave_cross_pre(s.vm, Hm, kVBins, INFINITY).w;
        if (top_p < 1.0f) {
            target_w = (double)top_p * total;
            const Cross r = wave_cross_pre(s.vm, Hm, kVBins, target_w);
            if (r.found) {
                cb = r.bin;
                wabove = r.w;
            }
        }
        // survivor weight bounds: A = bins above the nucleus bin, plus up to all of that bin
        const double A = wave_cross_pre(hq, Hq, cb, INFINITY).w;
        const double Bq = (cb < kVBins) ? (double)hq[cb] / kFx : 0.0;
        FvPlan q;
        q.total = total;
        q.cb = cb;
        q.A = A;
        q.target_w = target_w;
        q.wabove = wabove;
        q.u_zero = (u > 0.0f) ? 0u : 1u;
        q.dlo = q.dhi = cb;
        q.dlo_before = 0ull;
        q.dlo_found = 0u;
        if (!q.u_zero) {
            const uint32_t lim = (cb < kVBins) ? cb + 1u : kVBins;
            const Cross lo = wave_cross_pre(hq, Hq, lim, (double)u * A);
            const Cross hi = wave_cross_pre(hq, Hq, lim, (double)u * (A + Bq));
            q.dlo = lo.found ? lo.bin : lim - 1u;
            q.dhi = hi.found ? hi.bin : lim - 1u;
            q.dlo_found = lo.found ? 1u : 0u;
            // exact fixed-point weight of the bins above dlo: the lane sums before its lane, then
            // that lane's bins up to dlo
            constexpr uint32_t kPer = kVBins / 64u;
            const uint32_t lane = threadIdx.x & 63u, L = q.dlo / kPer, r = q.dlo % kPer;
            const unsigned long long part = (lane < r) ? hq[L * kPer + lane] : 0ull;
            q.dlo_before = lane_read(Hq.run, (int)L) + lane_read(wave_incl_scan(part, lane), 63);
        }
        if (threadIdx.x == 0u) *sp = q;
    }
    __syncthreads();
    *P = *sp;
    __syncthreads();
}

__device__ inline bool fv_wanted(const RowCtx& c, const FvPlan& P, float v) {
    const uint32_t b = vbin(c, v);
    return b == P.cb || (b >= P.dlo && b <= P.dhi);
}

// Appends the elements of [beg, end) in the planned bins to s.cand, counting in s.bu[2]
// (the count may exceed kCandCap; only the first kCandCap are stored).
__device__ __attribute__((always_inline)) inline void fv_gather(SelShared& s, const RowCtx& c, const FvPlan& P, uint32_t beg, uint32_t end,
                                                                const RowPre* pre = nullptr) {
    if (threadIdx.x == 0) s.bu[2] = 0u;
    __syncthreads();
    row_pass(c.l + beg, end - beg, [&](float v, uint32_t i) {
        wave_append(&s.bu[2], fv_wanted(c, P, v), ((unsigned long long)(~float_key(v)) << 32) | (beg + i),
                    s.cand, kCandCap);
    }, pre);
    __syncthreads();
}

// Weighted crossing inside one value bin of the candidate list s.cand[0, n) (unsorted): among
// the elements of `bin` with key <= key_limit, in ascending key order (logit descending, id
// ascending), the first whose cumulative weight exp2((v - m) * kw) reaches `target`. A second
// level of 2048 sub-bins over the bin's value range (u64 fixed-point weights) locates the
// crossing; only that sub-bin's elements are then sorted and summed exactly. Returns 1 with the
// element's key and the weight before it; 0 when the sub-bin holds more than 1024 elements.
__device__ __attribute__((always_inline)) inline int fine_cross(SelShared& s, const RowCtx& c, uint32_t n, uint32_t bin, unsigned long long key_limit,
                          float kw, double target, unsigned long long* key_out, double* before_out) {
    const uint32_t tid = threadIdx.x;
    unsigned long long* hf = reinterpret_cast<unsigned long long*>(s.pkey);   // 2048 sub-bins
    unsigned long long* sub = reinterpret_cast<unsigned long long*>(s.tiles); // <= 1024 elements
    constexpr uint32_t kSubCap = kTileCap / 2u;
    auto sub_of = [&](float v) {
        const float f = ((c.m - v) * c.inv_w - (float)bin) * (float)kVBins;
        return (f <= 0.0f) ? 0u : (f < (float)(kVBins - 1)) ? (uint32_t)f : kVBins - 1u;
    };
    auto in_set = [&](unsigned long long k, float v) { return k <= key_limit && vbin(c, v) == bin; };
    for (uint32_t i = tid; i < kVBins; i += sel_nt()) hf[i] = 0ull;
    __syncthreads();
    for (uint32_t e = tid; e < n; e += sel_nt()) {
        const unsigned long long k = s.cand[e];
        const float v = key_float(~(uint32_t)(k >> 32));
        if (v == -INFINITY || !in_set(k, v)) continue;
        atomicAdd(&hf[sub_of(v)], to_fx(__builtin_amdgcn_exp2f((v - c.m) * kw)));
    }
    __syncthreads();
    uint32_t sb;
    double above;
    if (!scan_cross(s, hf, kVBins, target, &sb, &above)) {
        // target beyond the set's total (rounding): the last non-empty sub-bin
        uint32_t last = 0u;
        for (uint32_t i = tid; i < kVBins; i += sel_nt()) if (hf[i]) last = max(last, i + 1u);
        last = kVBins - block_min_u(kVBins - last, s);  // block max via min
        if (last == 0u) return 0;
        sb = last - 1u;
        (void)scan_cross(s, hf, sb, INFINITY, &last, &above);
    }
    if (tid == 0) s.bu[5] = 0u;
    __syncthreads();
    for (uint32_t e0 = 0; e0 < n; e0 += sel_nt()) {
        const uint32_t e = e0 + tid;
        bool take = false;
        unsigned long long k = 0ull;
        if (e < n) {
            k = s.cand[e];
            const float v = key_float(~(uint32_t)(k >> 32));
            take = v != -INFINITY && in_set(k, v) && sub_of(v) == sb;
        }
        wave_append(&s.bu[5], take, k, sub, kSubCap);
    }
    __syncthreads();
    const uint32_t ns = s.bu[5];
    __syncthreads();
    if (ns == 0u || ns > kSubCap) return 0;
    if (ns <= 64u) {
        // the usual case, in wave 0 alone: the same rank sort, scan and first crossing as the
        // block-wide code below (one lane per element), with one barrier instead of eight. A
        // wave's LDS accesses complete in order, so the in-place placement and the read-back
        // need no barrier.
        if (tid < 64u) {
            const bool act = tid < ns;
            const unsigned long long mine = act ? sub[tid] : 0ull;
            uint32_t rank = 0u;
            for (uint32_t j = 0; j < ns; ++j) rank += (sub[j] < mine) ? 1u : 0u;
            if (act) sub[rank] = mine;
            const unsigned long long ks = act ? sub[tid] : 0ull;
            const double w = act ? (double)__builtin_amdgcn_exp2f((key_float(~(uint32_t)(ks >> 32)) - c.m) * kw) : 0.0;
            const double run = wave_incl_scan(w, tid) - w;
            const unsigned long long hit = __ballot(act && above + run + w >= target);
            const uint32_t pick = hit ? (uint32_t)__ffsll((long long)hit) - 1u : ns - 1u;
            if (tid == pick) {
                s.bd[3] = above + run;
                s.bu[6] = (uint32_t)ks;
                s.bu[7] = (uint32_t)(ks >> 32);
            }
        }
        __syncthreads();
        *key_out = ((unsigned long long)s.bu[7] << 32) | s.bu[6];
        *before_out = s.bd[3];
        __syncthreads();
        return 1;
    }
    // rank sort of the sub-bin (distinct keys)
    unsigned long long mine = 0ull;
    uint32_t rank = 0u;
    if (tid < ns) {
        mine = sub[tid];
        for (uint32_t j = 0; j < ns; ++j) rank += (sub[j] < mine) ? 1u : 0u;
    }
    __syncthreads();
    if (tid < ns) sub[rank] = mine;
    __syncthreads();
    // exact crossing inside the sorted sub-bin
    double w = 0.0;
    if (tid < ns) w = (double)__builtin_amdgcn_exp2f((key_float(~(uint32_t)(sub[tid] >> 32)) - c.m) * kw);
    const double run = block_excl_scan<double>(w, s, nullptr);
    const uint32_t first = block_min_u((tid < ns && above + run + w >= target) ? tid : 0xFFFFFFFFu, s);
    const uint32_t pick = (first == 0xFFFFFFFFu) ? ns - 1u : first;
    if (tid == pick) {
        s.bd[3] = above + run;
        s.bu[6] = (uint32_t)sub[tid];
        s.bu[7] = (uint32_t)(sub[tid] >> 32);
    }
    __syncthreads();
    *key_out = ((unsigned long long)s.bu[7] << 32) | s.bu[6];
    *before_out = s.bd[3];
    __syncthreads();
    return 1;
}

// Sum of exp2((v - m) * kw) over the candidates of `bin` with key <= key_limit.
__device__ __attribute__((always_inline)) inline double bin_weight(SelShared& s, const RowCtx& c, uint32_t n, uint32_t bin, unsigned long long key_limit, float kw) {
    double acc = 0.0;
    for (uint32_t e = threadIdx.x; e < n; e += sel_nt()) {
        const unsigned long long k = s.cand[e];
        const float v = key_float(~(uint32_t)(k >> 32));
        if (v != -INFINITY && k <= key_limit && vbin(c, v) == bin)
            acc += (double)__builtin_amdgcn_exp2f((v - c.m) * kw);
    }
    return block_sum<double>(acc, s);
}

// From the n gathered candidates in s.cand (unsorted) and the histograms in s.vm / s.vq: the
// nucleus cut inside bin cb and the temperature draw. Returns 1 with *token, 0 when rounding
// put the draw outside the gathered bins or a sub-bin is a massive tie (radix fallback).
__device__ __attribute__((always_inline)) inline int fv_finish(SelShared& s, const RowCtx& c, const FvPlan& P, uint32_t n, float u,
                         uint32_t* token, double* denom_out, double* r_out) {
    const float kq = kLog2e / c.T;
    const unsigned long long* hq = same_weights(c) ? s.vm : s.vq;
    if (n > kCandCap || n == 0u) return 0;
    const uint32_t cb = P.cb;
    // nucleus cut inside bin cb: the element where the T = 1 weight reaches the target
    double denom = P.A;
    unsigned long long ecut = ~0ull;
    if (cb < kVBins) {
        double bef;
        if (!fine_cross(s, c, n, cb, ~0ull, kLog2e, P.target_w - P.wabove, &ecut, &bef)) return 0;
        denom = P.A + bin_weight(s, c, n, cb, ecut, kq);
    }
    const double r = (double)u * denom;
    *denom_out = denom;
    *r_out = r;
    unsigned long long kt = 0ull;
    double bef;
    if (cb < kVBins && r > P.A) {
        if (!fine_cross(s, c, n, cb, ecut, kq, r - P.A, &kt, &bef)) return 0;
    } else {
        uint32_t db;
        double dab;
        // The draw's bin lies in [dlo, dhi] unless rounding moved r. When the plan found one bin
        // there, test r against that bin's exact running sums: the scan over [0, cb) would stop
        // at the same bin, since every nonempty bin above it ends at or below its start.
        bool one = false;
        if (P.dlo == P.dhi && P.dlo_found && P.dlo < cb) {
            const unsigned long long ce = P.dlo_before, ci = ce + hq[P.dlo];
            if (hq[P.dlo] != 0ull && fx_of(ce) < r && r <= fx_of(ci)) {
                db = P.dlo;
                dab = fx_of(ce);
                one = true;
            }
        }
        if (!one && !scan_cross(s, hq, cb, r, &db, &dab)) return 0;
        if (db < P.dlo || db > P.dhi) return 0;  // outside the gathered range (rounding)
        if (!fine_cross(s, c, n, db, ~0ull, kq, r - dab, &kt, &bef)) return 0;
    }
    *token = (uint32_t)kt;
    return 1;
}

// Nucleus over the full distribution, then the temperature draw over the survivors, in one
// workgroup. Returns 1 with *token, 0 when a bin is too large to gather (radix fallback).
__device__ __attribute__((always_inline)) inline int full_vocab_value_path(SelShared& s, const RowCtx& c, float top_p, float u,
                                     uint32_t first_id, uint32_t* token, double* denom_out,
                                     double* r_out, double* total_out) {
    fv_hist(s, c, 0u, c.V);
    FvPlan P;
    fv_plan(s, c, top_p, u, &P);
    *total_out = P.total;
    if (P.u_zero) {
        *token = first_id;
        *denom_out = P.A;
        *r_out = 0.0;
        return 1;
    }
    fv_gather(s, c, P, 0u, c.V);
    const uint32_t n = s.bu[2];
    __syncthreads();
    return fv_finish(s, c, P, n, u, token, denom_out, r_out);
}

// Radix fallback over the whole row: shortlist bound, nucleus, then the draw.
__device__ __attribute__((always_inline)) inline void radix_select(SelShared& s, const RowCtx& c, const DevRow& row, float u, uint32_t want,
                             double Z, uint32_t arg, uint32_t* token, RowReport* rep) {
    uint32_t kx, ix;
    PSet s0 = {0, 0u, 0u};
    if (want < c.V && find_cross(s, c, s0, 0, (double)want, &kx, &ix)) s0 = PSet{1, kx, ix};
    PSet s1 = s0;
    if (row.top_p < 1.0f && find_cross(s, c, s0, 1, (double)row.top_p * Z, &kx, &ix))
        s1 = PSet{1, kx, ix};
    double dl = 0.0;
    row_pass(c.l, c.V, [&](float v, uint32_t i) {
        if (s1.has(float_key(v), i)) dl += (double)weight_f(c, v, 2);
    });
    const double tot = block_sum<double>(dl, s);
    const double r = (double)u * tot;
    if (!(r > 0.0)) *token = arg;
    else if (find_cross(s, c, s1, 2, r, &kx, &ix)) *token = ix;
    else *token = s1.bounded ? s1.ib : arg;
    rep->denom = tot;
    rep->r = r;
    rep->path = 4;
}

// Value-bin context of a row from its maximum and finite minimum.
__device__ inline RowCtx make_ctx(uint32_t V, const float* l, float m, float fmin, float T, uint2* list) {
    RowCtx c;
    c.V = V;
    c.l = l;
    c.m = m;
    c.T = T;
    c.list = list;
    const float span = 48.0f * fmaxf(1.0f, T);
    const float lo = fmaxf(fmin, m - span);
    c.inv_w = (m > lo) ? (float)kVBins / (m - lo) : 0.0f;
    return c;
}

// Row report and token, and the history append (src/runner.cpp:878), by thread 0. len: the
// row's history length (read by the caller ahead of time), or ~0 to read it here.
// A full history (len == stride) keeps its contents: the token is not appended, the report's
// status carries kStatusHistoryFull and the host-visible overflow word (when given) is set, so
// the caller's next synchronisation fails instead of the penalties silently drifting from a
// history that grows without bound (src/runner.cpp:878).
__device__ inline void write_row(const SelectArgs& a, uint32_t b, uint32_t token, const RowReport& rep,
                                 uint32_t len = 0xFFFFFFFFu) {
    if (threadIdx.x != 0) return;
    a.tokens[b] = token;
    uint32_t status = 0u;
    if (a.history && a.hist_len && token != 0xFFFFFFFFu) {
        if (len == 0xFFFFFFFFu) len = a.hist_len[b];
        if (len < a.hist_stride) {
            a.history[(size_t)b * a.hist_stride + len] = token;
            a.hist_len[b] = len + 1u;
        } else {
            status |= kStatusHistoryFull;
            if (a.hist_overflow) __hip_atomic_store(a.hist_overflow, b + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (a.report) {
        RowReport r = rep;
        r.status = status;
        reinterpret_cast<RowReport*>(a.report)[b] = r;
    }
}

// Rows that take the full-vocabulary value path: sampled, with the shortlist lifted.
__device__ inline bool is_fv_row(const DevRow& row, uint32_t V) { return row.temperature > 0.0f && row.want >= V; }

// Block-wide maximum and finite minimum of a row's block partials.
__device__ void partial_max_min(SelShared& s, const BlockPartial* parts, uint32_t ntile, float* m_out, float* fmin_out) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    float bm = -INFINITY, bmin = INFINITY;
    for (uint32_t t = tid; t < ntile; t += sel_nt()) {
        const BlockPartial p = parts[t];
        bm = fmaxf(bm, p.max);
        bmin = fminf(bmin, p.minf);
    }
    bm = wave_max(bm);
    bmin = wave_min(bmin);
    if (lane == 0) { s.wmax[wave] = bm; s.wmin[wave] = bmin; }
    __syncthreads();
    float m = s.wmax[0], fmin = s.wmin[0];
    for (uint32_t w = 1; w < sel_nw(); ++w) { m = fmaxf(m, s.wmax[w]); fmin = fminf(fmin, s.wmin[w]); }
    __syncthreads();
    *m_out = m;
    *fmin_out = fmin;
}

// Slice [beg, end) of a row for workgroup k of S; slices are multiples of 4 elements.
__device__ inline void fv_slice(uint32_t V, uint32_t S, uint32_t k, uint32_t* beg, uint32_t* end) {
    const uint32_t len = ((V + S - 1u) / S + 3u) & ~3u;
    *beg = min(k * len, V);
    *end = min(*beg + len, V);
}

// Per-row state of the multi-workgroup path, written by k_select, read by k_fv_gather / k_fv_finish.
struct FvRowState {
    FvPlan plan;
    float m, fmin, T, u, top_p;
    uint32_t arg, want, active, ncand, overflow;
    double Z;
};
static_assert(sizeof(FvRowState) <= kFvStateBytes, "per-row state must fit its slot");
static_assert(kFvBins == kVBins && kFvCandCap == kCandCap, "host sizes must match the kernels'");

__device__ inline FvRowState* fv_state_of(const SelectArgs& a, uint32_t b) {
    return reinterpret_cast<FvRowState*>(reinterpret_cast<char*>(a.fv_state) + (size_t)b * kFvStateBytes);
}

// Slice histograms of the full-vocabulary rows: workgroup (k, b) bins slice k of row b.
__global__ __launch_bounds__(kMaxSelThreads) void k_fv_hist(SelectArgs a, FvList fv) {
    __shared__ SelShared s;
    // the row and its temperature come with the launch: the first loads are the row's own
    const uint32_t k = blockIdx.x, b = fv.row[blockIdx.y];
    const float T = fv.temp[blockIdx.y];
    uint32_t beg, end;
    fv_slice(a.V, gridDim.x, k, &beg, &end);  // the grid's x extent is the slice count
    const float* lrow = a.logits + (size_t)b * a.V;
    RowPre pre;
    row_preload(lrow + beg, end - beg, pre);  // in flight while the row maximum is found
    float m, fmin;
    partial_max_min(s, a.partials + (size_t)b * a.ntile, a.ntile, &m, &fmin);
    if (m == -INFINITY) return;  // degenerate row: k_select reports it
    const RowCtx c = make_ctx(a.V, lrow, m, fmin, T, nullptr);
    fv_hist(s, c, beg, end, &pre);
    // fixed-point bin weights are integers: summing the slices with atomics is exact and
    // order-independent, and k_select reads one 32 KB histogram per row instead of 16
    unsigned long long* acc = a.fv_acc + (size_t)b * 2u * kVBins;
    for (uint32_t i = threadIdx.x; i < kVBins; i += sel_nt()) {
        if (s.vm[i]) atomicAdd(&acc[i], s.vm[i]);
        if (s.vq[i]) atomicAdd(&acc[kVBins + i], s.vq[i]);
    }
}

// Gather of the planned bins, slice k of row b, into the row's global candidate list.
__global__ __launch_bounds__(kMaxSelThreads) void k_fv_gather(SelectArgs a, FvList fv, uint2* __restrict__ scratch) {
    __shared__ SelShared s;
    const uint32_t k = blockIdx.x, b = fv.row[blockIdx.y], tid = threadIdx.x;
    uint32_t beg, end;
    fv_slice(a.V, gridDim.x, k, &beg, &end);
    RowPre pre;
    row_preload(a.logits + (size_t)b * a.V + beg, end - beg, pre);
    // the plan in the same round trip as the slice's first loads (read before the branch)
    FvRowState* st = fv_state_of(a, b);
    const uint32_t active = st->active;
    const FvPlan P = st->plan;
    const float m = st->m, fmin = st->fmin, T = st->T;
    if (active == 0u) return;  // k_select finished the row
    const RowCtx c = make_ctx(a.V, a.logits + (size_t)b * a.V, m, fmin, T, scratch + (size_t)b * a.V);
    fv_gather(s, c, P, beg, end, &pre);
    const uint32_t nl = s.bu[2];
    __syncthreads();
    if (tid == 0) {
        if (nl > kCandCap) {
            atomicOr(&st->overflow, 1u);
            s.bu[3] = 0xFFFFFFFFu;
        } else {
            s.bu[3] = atomicAdd(&st->ncand, nl);
        }
    }
    __syncthreads();
    const uint32_t off = s.bu[3];
    if (off != 0xFFFFFFFFu)
        for (uint32_t i = tid; i < nl; i += sel_nt())
            if (off + i < kCandCap) a.fv_cand[(size_t)b * kCandCap + off + i] = s.cand[i];
}

// Sort of the gathered candidates and the draw, one workgroup per deferred row (the kernel
// boundary orders it after every slice's stores).
__global__ __launch_bounds__(kMaxSelThreads) void k_fv_finish(SelectArgs a, FvList fv, uint2* __restrict__ scratch) {
    constexpr uint32_t kCandPer = kCandCap / kMaxSelThreads, kHistPer = 2u * kVBins / kMaxSelThreads;
    static_assert(kCandCap % kMaxSelThreads == 0u && kVBins % kMaxSelThreads == 0u,
                  "the finish loads whole rounds of candidates and bins");
    __shared__ SelShared s;
    const uint32_t b = fv.row[blockIdx.x], tid = threadIdx.x;
    // Everything the finish reads, in one round trip: the row's state, its merged histograms and
    // every candidate slot (slots past the gathered count hold an earlier step's and are dropped).
    const FvRowState sv = *fv_state_of(a, b);
    const unsigned long long* cg = a.fv_cand + (size_t)b * kCandCap;
    const unsigned long long* mg = a.fv_merged + (size_t)b * 2u * kVBins;
    unsigned long long cv[kCandPer], hv[kHistPer];
#pragma unroll
    for (uint32_t j = 0; j < kCandPer; ++j) cv[j] = cg[tid + j * kMaxSelThreads];
#pragma unroll
    for (uint32_t j = 0; j < kHistPer; ++j) hv[j] = mg[tid + j * kMaxSelThreads];
    if (sv.active == 0u) return;  // k_select finished the row
    const RowCtx c = make_ctx(a.V, a.logits + (size_t)b * a.V, sv.m, sv.fmin, sv.T, scratch + (size_t)b * a.V);
    const uint32_t n = sv.ncand;
    RowReport rep = {};
    rep.max_logit = sv.m;
    rep.u = sv.u;
    rep.shortlist = sv.want;
    rep.total = sv.Z;
    uint32_t token = sv.arg;
    int ok = 0;
    if (sv.overflow == 0u && n > 0u && n <= kCandCap) {
#pragma unroll
        for (uint32_t j = 0; j < kCandPer; ++j)
            if (tid + j * kMaxSelThreads < n) s.cand[tid + j * kMaxSelThreads] = cv[j];
#pragma unroll
        for (uint32_t j = 0; j < kHistPer; ++j) {
            const uint32_t i = tid + j * kMaxSelThreads;
            if (i < kVBins) s.vm[i] = hv[j];
            else s.vq[i - kVBins] = hv[j];
        }
        __syncthreads();
        double dn = 0.0, rr = 0.0;
        uint32_t tk = 0;
        ok = fv_finish(s, c, sv.plan, n, sv.u, &tk, &dn, &rr);
        if (ok) {
            token = tk;
            rep.denom = dn;
            rep.r = rr;
            rep.path = 2;
        }
    }
    if (!ok) {
        // too many candidates, or rounding outside the gathered bins: the one-workgroup paths
        double dn = 0.0, rr = 0.0, zt = 0.0;
        uint32_t tk = 0;
        if (full_vocab_value_path(s, c, sv.top_p, sv.u, sv.arg, &tk, &dn, &rr, &zt)) {
            token = tk;
            rep.denom = dn;
            rep.r = rr;
            rep.path = 2;
        } else {
            const DevRow row = a.rows[b];
            RowReport rr = rep;
            uint32_t tk = token;
            radix_select(s, c, row, sv.u, sv.want, sv.Z, sv.arg, &tk, &rr);
            rep = rr;
            token = tk;
        }
    }
    write_row(a, b, token, rep);
}

// Shortlist threshold from the block-maximum keys held in registers (key[j]: tile tid + j NT,
// 0 past ntile): a histogram of the block maxima over kWinBins value bins of width 1/32 below
// the row maximum m (window_add, during the row-summary pass). With the want-th largest block
// maximum in bin j (counted from m down), every block counted up to bin j lies at or above
// m - (j + 1) w up to rounding far below one bin, so m - (j + 2) w bounds the want-th largest
// block maximum, and with it the want-th largest logit, from below (window_scan, one wave).
// Needs |m| <= 1024 (value rounding << w) and the want-th maximum inside the window; the scan
// returns 0 (not found) otherwise. Every wave runs the scan on the same counts and so finds the
// same bound, with no barrier between the scan and its use.
constexpr uint32_t kWinBins = 256;
constexpr float kWinWidth = 1.0f / 32.0f;
template <uint32_t KP>
__device__ __attribute__((always_inline)) inline void window_add(SelShared& s, const uint32_t* key, float m) {
#pragma unroll
    for (uint32_t j = 0; j < KP; ++j) {
        const float v = key_float(key[j]);
        if (key[j] != 0u && v >= m - (float)kWinBins * kWinWidth)
            atomicAdd(&s.hu[min(kWinBins - 1u, (uint32_t)((m - v) * (1.0f / kWinWidth)))], 1u);
    }
}
__device__ inline uint32_t window_scan(SelShared& s, float m, uint32_t want) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint4 c = *reinterpret_cast<const uint4*>(&s.hu[4u * lane]);  // bins 4 lane .. 4 lane + 3
    const uint32_t sum = c.x + c.y + c.z + c.w;
    const uint32_t incl = wave_incl_scan(sum, lane);
    const unsigned long long mk = __ballot(incl >= want);
    uint32_t res = 0u;
    if (mk != 0ull) {
        const uint32_t L = (uint32_t)__ffsll((long long)mk) - 1u;
        const uint32_t before = lane_read(incl - sum, (int)L);
        const uint4 cl = *reinterpret_cast<const uint4*>(&s.hu[4u * L]);
        uint32_t q = 3u;
        if (before + cl.x >= want) q = 0u;
        else if (before + cl.x + cl.y >= want) q = 1u;
        else if (before + cl.x + cl.y + cl.z >= want) q = 2u;
        res = float_key(m - (float)(4u * L + q + 2u) * kWinWidth);
    }
    return __builtin_amdgcn_readfirstlane(res);
}

// ---- the kernel ----------------------------------------------------------------------------------

template <uint32_t NT>
__global__ __launch_bounds__(NT) void k_select(SelectArgs a, uint2* __restrict__ scratch) {
    constexpr uint32_t KP = kRegTiles / NT;  // block partials per thread on the register path
    __shared__ SelShared s;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t b = blockIdx.x;
    // Every global load that does not depend on the row parameters is issued before anything
    // branches on them, so the row load and these share one memory round trip.
    const DevRow row = a.rows[b];
    const float u = a.uniforms ? a.uniforms[b] : row.u;
    const BlockPartial* parts = a.partials + (size_t)b * a.ntile;
    const bool keys_cached = a.ntile <= kKeyCache;
    const bool reg = a.ntile <= kRegTiles;
    // register path: the partials of tiles tid + j NT, loaded without branches (indices past
    // the last tile are clamped to it and replaced by neutral values once they arrive)
    BlockPartial p[KP];
#pragma unroll
    for (uint32_t j = 0; j < KP; ++j) p[j] = parts[min(tid + j * NT, a.ntile - 1u)];
#pragma unroll
    for (uint32_t j = 0; j < KP; ++j)
        if (tid + j * NT >= a.ntile) p[j] = BlockPartial{-INFINITY, 0xFFFFFFFFu, 0.0f, INFINITY, -INFINITY};
    // history length for the append in write_row (thread 0), fetched now
    const uint32_t hlen = (tid == 0 && a.history && a.hist_len) ? a.hist_len[b] : 0u;
    for (uint32_t i = tid; i < kWinBins; i += NT) s.hu[i] = 0u;  // window histogram, below
    if (tid == 0) { s.ntile_q = 0u; s.ncand_q = 0u; }

    // the multi-workgroup hand-over is re-armed below only for rows this step defers
    if (a.fv_acc && tid == 0 && is_fv_row(row, a.V)) fv_state_of(a, b)->active = 0u;

    const bool sampled = row.temperature > 0.0f;
    // 1. row max, lowest argmax, finite minimum and, for sampled rows,
    //    Z = sum_t sumexp_t * exp(max_t - m) over the block partials
    // shortlist rows with the keys in registers histogram them in the row-summary pass
    const bool win = reg && sampled && row.want <= kMaxTopK && a.ntile > row.want;
    uint32_t key[KP];  // register path: block-maximum keys of tiles tid + j NT (0 past ntile)
    float m, fmin;
    uint32_t arg;
    double Z = 0.0;
    // Shortlist rows with the window bound need Z only for the nucleus: their per-thread shares
    // (zt) are summed while the gather's loads are in flight instead of before the bound.
    double zt = 0.0;
    bool late_z = false;
    if (reg) {
#pragma unroll
        for (uint32_t j = 0; j < KP; ++j) key[j] = (tid + j * NT < a.ntile) ? float_key(p[j].max) : 0u;
        float bm = -INFINITY, bmin = INFINITY;
        uint32_t ba = 0xFFFFFFFFu;
#pragma unroll
        for (uint32_t j = 0; j < KP; ++j) {
            if (p[j].max > bm || (p[j].max == bm && p[j].arg < ba)) { bm = p[j].max; ba = p[j].arg; }
            bmin = fminf(bmin, p[j].minf);
        }
        wave_argmax(bm, ba);
        bmin = wave_min(bmin);
        if (lane == 0) { s.wmax[wave] = bm; s.warg[wave] = ba; s.wmin[wave] = bmin; }
        __syncthreads();
        // every wave combines the wave results, one per lane
        m = -INFINITY;
        arg = 0xFFFFFFFFu;
        fmin = INFINITY;
        if (lane < sel_nw()) { m = s.wmax[lane]; arg = s.warg[lane]; fmin = s.wmin[lane]; }
        wave_argmax(m, arg);
        fmin = wave_min(fmin);
        late_z = win && fabsf(m) <= 1024.0f;
        if (late_z) window_add<KP>(s, key, m);
        if (sampled && m != -INFINITY) {
#pragma unroll
            for (uint32_t j = 0; j < KP; ++j)
                if (p[j].max != -INFINITY)
                    zt += (double)(__builtin_amdgcn_exp2f((p[j].max - m) * kLog2e) * p[j].sumexp);
            if (!late_z) {
                const double z = wave_sum_d(zt);
                if (lane == 0) s.wzs[wave] = z;
            }
        }
        __syncthreads();
        if (!late_z && sampled && m != -INFINITY) Z = wave_sum_d(lane < sel_nw() ? s.wzs[lane] : 0.0);
    } else {
        // any number of tiles: a loop over the partials with a running maximum for Z; the
        // block-maximum keys are kept in LDS when they fit
        float bm = -INFINITY, bmin = INFINITY, zm = -INFINITY;
        uint32_t ba = 0xFFFFFFFFu;
        double zs = 0.0;
        for (uint32_t t = tid; t < a.ntile; t += sel_nt()) {
            const BlockPartial p = parts[t];
            if (p.max > bm || (p.max == bm && p.arg < ba)) { bm = p.max; ba = p.arg; }
            bmin = fminf(bmin, p.minf);
            if (keys_cached) s.pkey[t] = float_key(p.max);
            if (sampled && p.max != -INFINITY) {
                if (p.max > zm) {
                    if (zm != -INFINITY) zs *= (double)__builtin_amdgcn_exp2f((zm - p.max) * kLog2e);
                    zm = p.max;
                }
                zs += (double)(__builtin_amdgcn_exp2f((p.max - zm) * kLog2e) * p.sumexp);
            }
        }
        wave_argmax(bm, ba);
        bmin = wave_min(bmin);
        if (sampled) {
            const float wm = wave_max(zm);
            zs = (zm == -INFINITY) ? 0.0 : zs * (double)__builtin_amdgcn_exp2f((zm - wm) * kLog2e);
            zs = wave_sum_d(zs);
            zm = wm;
        }
        if (lane == 0) {
            s.wmax[wave] = bm; s.warg[wave] = ba; s.wmin[wave] = bmin;
            s.wzm[wave] = zm; s.wzs[wave] = zs;
        }
        __syncthreads();
        m = -INFINITY;
        arg = 0xFFFFFFFFu;
        fmin = INFINITY;
        float wzm = -INFINITY;
        double wzs = 0.0;
        if (lane < sel_nw()) { m = s.wmax[lane]; arg = s.warg[lane]; fmin = s.wmin[lane]; wzm = s.wzm[lane]; wzs = s.wzs[lane]; }
        wave_argmax(m, arg);
        fmin = wave_min(fmin);
        if (sampled && m != -INFINITY)
            Z = wave_sum_d(wzm != -INFINITY ? wzs * (double)__builtin_amdgcn_exp2f((wzm - m) * kLog2e) : 0.0);
        __syncthreads();
    }

    RowReport rep = {};
    rep.max_logit = m;
    rep.u = u;
    uint32_t token = arg;
    bool deferred = false;  // finished by k_fv_finish

    if (row.temperature <= 0.0f) {
        rep.path = 0;
        rep.shortlist = 1;
        rep.cut = 1;
    } else {
        // 2. Z = sum over the row of exp(l - m), from the block partials (pass 1)
        rep.total = Z;
        const float* lrow = a.logits + (size_t)b * a.V;
        const uint32_t want = row.want;
        rep.shortlist = want;
        bool general = (want > kMaxTopK);
        auto pkey = [&](uint32_t t) { return (keys_cached && !reg) ? s.pkey[t] : float_key(parts[t].max); };
        // Full-vocabulary rows take Z from their value histogram (the head may skip the block
        // sums of exp when no row needs them): a finite maximum is the only condition.
        const bool fvrow = want >= a.V;
        // the deferred Z: wave shares (stage 1, before a barrier), then every wave adds them
        auto z_stage1 = [&]() {
            const double z = wave_sum_d(zt);
            if (lane == 0) s.wzs[wave] = z;
        };
        auto z_stage2 = [&]() {
            Z = wave_sum_d(lane < sel_nw() ? s.wzs[lane] : 0.0);
            rep.total = Z;
            late_z = false;
        };
        // with m finite, the tile holding m contributes at least exp(0) to Z (its block sum
        // is computed whenever a row samples from a shortlist): the deferred check below only
        // catches non-finite sums
        if (m == -INFINITY || (!fvrow && !late_z && !(Z > 0.0))) {
            token = 0xFFFFFFFFu;
            rep.path = 3;
            general = false;
        } else if (!general) {
            // ---- shortlist path ----
            // tau: a lower bound of the want-th largest block maximum, hence of the want-th
            // largest logit. With the keys in registers, a 256-bin window of width 1/32 below m
            // (window_add / window_scan); else, or when the want-th maximum lies outside it, one
            // histogram of the block maxima over 2048 bins of width 1/64 (the same bound over a
            // 32-unit span), and failing that the exact 22-bit key bound (two 11-bit levels).
            uint32_t tau = 0u;
            if (win && fabsf(m) <= 1024.0f) tau = window_scan(s, m, want);
            if (a.ntile > want && tau == 0u) {
                // the window's counts may still be read by a slower wave's scan
                __syncthreads();
                constexpr float kTauSpan = 32.0f;
                constexpr float kTauInv = (float)kBins / kTauSpan;
                bool found = false;
                if (fabsf(m) <= 1024.0f) {
                    for (uint32_t i = tid; i < kBins; i += sel_nt()) s.hu[i] = 0u;
                    __syncthreads();
                    for (uint32_t t = tid; t < a.ntile; t += sel_nt()) {
                        const float v = key_float(pkey(t));
                        if (v >= m - kTauSpan) {
                            const uint32_t j = min(kBins - 1u, (uint32_t)((m - v) * kTauInv));
                            atomicAdd(&s.hu[kBins - 1u - j], 1u);  // hist_cross scans from the top bin
                        }
                    }
                    __syncthreads();
                    uint32_t bin = 0, above = 0;
                    if (hist_cross<uint32_t>(s, kBins, want, &bin, &above)) {
                        const uint32_t j = kBins - 1u - bin;
                        tau = float_key(m - (float)(j + 2u) * (kTauSpan / (float)kBins));
                        found = true;
                    }
                }
                if (!found) {
                    uint32_t prefix = 0, mask = 0, rem = want;
                    for (int lv = 0; lv < 2; ++lv) {
                        const uint32_t sh = (lv == 0) ? 21u : 10u;
                        for (uint32_t i = tid; i < kBins; i += sel_nt()) s.hu[i] = 0u;
                        __syncthreads();
                        for (uint32_t t = tid; t < a.ntile; t += sel_nt()) {
                            const uint32_t k = pkey(t);
                            if ((k & mask) == prefix) atomicAdd(&s.hu[(k >> sh) & (kBins - 1u)], 1u);
                        }
                        __syncthreads();
                        uint32_t bin = 0, above = 0;
                        hist_cross<uint32_t>(s, kBins, rem, &bin, &above);
                        rem -= above;
                        prefix |= bin << sh;
                        mask |= (kBins - 1u) << sh;
                    }
                    tau = prefix;
                }
            }
            // tiles whose maximum reaches tau, compacted into s.tiles
            uint32_t nq = 0u;
            if (reg) {
                // A qualifying tile whose second-largest value lies below tau holds exactly one
                // element >= tau, its maximum, known from the partial: it is appended as a
                // candidate directly. Only the other qualifying tiles are gathered. One LDS atomic
                // per wave and key slot; the order does not matter (candidates are ranked by value
                // and id).
#pragma unroll
                for (uint32_t j = 0; j < KP; ++j) {
                    const bool qual = key[j] >= tau && key[j] != 0u;
                    const bool one = qual && float_key(p[j].smax) < tau;
                    wave_append(&s.ncand_q, one, ((unsigned long long)(~key[j]) << 32) | p[j].arg, s.cand, kCandCap);
                    wave_append(&s.ntile_q, qual && !one, tid + j * NT, s.tiles, kTileCap);
                }
                if (late_z) z_stage1();
                __syncthreads();
                nq = s.ntile_q;
            } else {
                if (tid == 0) s.bu[3] = 0u;
                __syncthreads();
                for (uint32_t t = tid; t < a.ntile; t += NT) {
                    if (pkey(t) >= tau) {
                        const uint32_t slot = atomicAdd(&s.bu[3], 1u);
                        if (slot < kTileCap) s.tiles[slot] = t;
                    }
                }
                __syncthreads();
                nq = s.bu[3];
            }
            if (nq > kTileCap) {
                general = true;
                if (late_z) z_stage2();  // its wave shares were written before the last barrier
            } else {
                // gather the elements >= tau of those tiles: GB loads in flight per thread (issued
                // unconditionally from clamped ids, so no branch separates them), appended with one
                // LDS atomic per wave and slot
                constexpr uint32_t GB = kGatherChunk / NT;
                const uint32_t items = nq * kTileRows;
                uint32_t n = 0u;
                for (uint32_t c0 = 0; c0 < items; c0 += kGatherChunk) {
                    float v[GB];
                    uint32_t id[GB];
#pragma unroll
                    for (uint32_t q = 0; q < GB; ++q) {
                        const uint32_t it = c0 + q * NT + tid;
                        id[q] = (it < items) ? s.tiles[min(it, items - 1u) >> 6] * kTileRows + (it & 63u) : 0xFFFFFFFFu;
                        v[q] = lrow[min(id[q], a.V - 1u)];
                    }
#pragma unroll
                    for (uint32_t q = 0; q < GB; ++q)
                        wave_append(&s.ncand_q, id[q] < a.V && float_key(v[q]) >= tau,
                                    ((unsigned long long)(~float_key(v[q])) << 32) | id[q], s.cand, kCandCap);
                }
                if (items > 0u) __syncthreads();  // else every append happened before the last barrier
                n = s.ncand_q;
                if (late_z) z_stage2();
                if (n > kCandCap) general = true;
                if (!general && !(Z > 0.0)) {
                    token = 0xFFFFFFFFu;  // a non-finite Z: the degenerate report, as above
                    rep.path = 3;
                } else if (!general) {
                    // counting ranks costs n^2 / threads compares per thread: the network beyond 256
                    if (n <= 256u) rank_top(s, n, min(want, n));
                    else sort_cand(s, n);
                    // Nucleus over full-distribution probabilities p = exp(l - m) / Z (:139-151),
                    // then the draw over q = exp((l - m) / T) (:153-168). Both are computed for
                    // every shortlist entry; inclusive prefix sums up to the cut are unaffected by
                    // the entries past it.
                    const uint32_t W = min(want, n);
                    uint32_t cut = 0, rank = 0;
                    double denom = 0.0, r = 0.0;
                    if (W <= 64u) {
                        // one wave: shuffle scans and ballots, no barriers
                        if (wave == 0u) {
                            float li = -INFINITY;
                            uint32_t idi = 0;
                            double pv = 0.0, qv = 0.0;
                            if (lane < W) {
                                const unsigned long long cv = s.cand[lane];
                                li = key_float(~(uint32_t)(cv >> 32));
                                idi = (uint32_t)cv;
                                const double dl = (double)li - (double)m;
                                pv = exp(dl) / Z;
                                qv = exp(dl / (double)row.temperature);
                            }
                            const double runp = wave_incl_scan(pv, lane);
                            const double runq = wave_incl_scan(qv, lane);
                            uint32_t ct = W;
                            if (row.top_p < 1.0f) {
                                const unsigned long long mk = __ballot(lane < W && runp >= (double)row.top_p);
                                if (mk) ct = (uint32_t)__ffsll((long long)mk);
                            }
                            if (row.top_k > 0 && ct > (uint32_t)row.top_k) ct = (uint32_t)row.top_k;
                            if (ct < 1u) ct = 1u;
                            const double dn = lane_read(runq, (int)ct - 1);
                            const double rr = (double)u * dn;
                            const unsigned long long mk2 = __ballot(lane < ct && runq >= rr);
                            const uint32_t rk = mk2 ? (uint32_t)(__ffsll((long long)mk2) - 1) : ct - 1u;
                            const uint32_t tk = lane_read(idi, (int)rk);
                            if (lane == 0u) {
                                s.bu[5] = tk; s.bu[6] = ct; s.bu[7] = rk;
                                s.bd[1] = dn; s.bd[2] = rr;
                            }
                        }
                        __syncthreads();
                        token = s.bu[5];
                        cut = s.bu[6];
                        rank = s.bu[7];
                        denom = s.bd[1];
                        r = s.bd[2];
                    } else {
                        // 64 < W <= kMaxTopK: the threads below W compute their entries' two
                        // exponentials side by side, then wave 0 scans them four to a lane
                        // (consecutive entries, so each lane's running sums plus a wave scan of
                        // the lane totals are the running sums in rank order) and picks the cut
                        // and the draw as above: two barriers instead of the block scans' eight
                        constexpr uint32_t kPer = kMaxTopK / 64u;
                        static_assert(2u * kMaxTopK * sizeof(double) <= sizeof(s.vm), "entries fit the bins");
                        double* pd = reinterpret_cast<double*>(s.vm);  // the window counts are spent
                        double* qd = pd + kMaxTopK;
                        if (tid < W) {
                            const unsigned long long cv = s.cand[tid];
                            const double dl = (double)key_float(~(uint32_t)(cv >> 32)) - (double)m;
                            pd[tid] = exp(dl) / Z;
                            qd[tid] = exp(dl / (double)row.temperature);
                        }
                        __syncthreads();
                        if (wave == 0u) {
                            double rp[kPer], rq[kPer];
                            double ap = 0.0, aq = 0.0;
#pragma unroll
                            for (uint32_t j = 0; j < kPer; ++j) {
                                const uint32_t i = lane * kPer + j;
                                ap += (i < W) ? pd[i] : 0.0;
                                aq += (i < W) ? qd[i] : 0.0;
                                rp[j] = ap;
                                rq[j] = aq;
                            }
                            const double bp = wave_incl_scan(ap, lane) - ap, bq = wave_incl_scan(aq, lane) - aq;
#pragma unroll
                            for (uint32_t j = 0; j < kPer; ++j) {
                                rp[j] += bp;
                                rq[j] += bq;
                            }
                            uint32_t ct = W;
                            if (row.top_p < 1.0f) {
                                uint32_t fj = kPer;  // the lane's first entry whose running p reaches top_p
#pragma unroll
                                for (int j = (int)kPer - 1; j >= 0; --j)
                                    if (lane * kPer + (uint32_t)j < W && rp[j] >= (double)row.top_p) fj = (uint32_t)j;
                                const unsigned long long mk = __ballot(fj < kPer);
                                if (mk) {
                                    const uint32_t L = (uint32_t)__ffsll((long long)mk) - 1u;
                                    ct = L * kPer + lane_read(fj, (int)L) + 1u;
                                }
                            }
                            if (row.top_k > 0 && ct > (uint32_t)row.top_k) ct = (uint32_t)row.top_k;
                            if (ct < 1u) ct = 1u;
                            const uint32_t jc = (ct - 1u) % kPer;
                            double qc = rq[0];
#pragma unroll
                            for (uint32_t j = 1; j < kPer; ++j) qc = (j == jc) ? rq[j] : qc;
                            const double dn = lane_read(qc, (int)((ct - 1u) / kPer));
                            const double rr = (double)u * dn;
                            uint32_t fk = kPer;  // the lane's first entry below the cut reaching r
#pragma unroll
                            for (int j = (int)kPer - 1; j >= 0; --j)
                                if (lane * kPer + (uint32_t)j < ct && rq[j] >= rr) fk = (uint32_t)j;
                            const unsigned long long mk2 = __ballot(fk < kPer);
                            uint32_t rk = ct - 1u;
                            if (mk2) {
                                const uint32_t L = (uint32_t)__ffsll((long long)mk2) - 1u;
                                rk = L * kPer + lane_read(fk, (int)L);
                            }
                            if (lane == 0u) {
                                s.bu[5] = (uint32_t)s.cand[rk]; s.bu[6] = ct; s.bu[7] = rk;
                                s.bd[1] = dn; s.bd[2] = rr;
                            }
                        }
                        __syncthreads();
                        token = s.bu[5];
                        cut = s.bu[6];
                        rank = s.bu[7];
                        denom = s.bd[1];
                        r = s.bd[2];
                    }
                    rep.cut = cut;
                    rep.rank = rank;
                    rep.denom = denom;
                    rep.r = r;
                    rep.path = 1;
                    __syncthreads();
                }
            }
        }
        if (general) {
            const RowCtx c = make_ctx(a.V, lrow, m, fmin, row.temperature, scratch + (size_t)b * a.V);
            bool done = false;
            if (want >= a.V && a.fv_acc) {
                // multi-workgroup rows: take the summed slice histograms (and clear them for
                // the next step), plan, and leave the gather and the draw to k_fv_gather and
                // k_fv_finish
                unsigned long long* acc = a.fv_acc + (size_t)b * 2u * kVBins;
                unsigned long long* mg = a.fv_merged + (size_t)b * 2u * kVBins;
                for (uint32_t i = tid; i < kVBins; i += sel_nt()) {
                    const unsigned long long hm = acc[i], hq = acc[kVBins + i];
                    acc[i] = 0ull;
                    acc[kVBins + i] = 0ull;
                    s.vm[i] = hm;
                    s.vq[i] = hq;
                    mg[i] = hm;
                    mg[kVBins + i] = hq;
                }
                __syncthreads();
                FvPlan P;
                fv_plan(s, c, row.top_p, u, &P);
                FvRowState* st = fv_state_of(a, b);
                rep.total = P.total;
                if (P.u_zero) {
                    token = arg;
                    rep.denom = P.A;
                    rep.r = 0.0;
                    rep.path = 2;
                } else {
                    deferred = true;
                }
                if (tid == 0) {
                    st->plan = P;
                    st->m = m;
                    st->fmin = fmin;
                    st->T = row.temperature;
                    st->u = u;
                    st->top_p = row.top_p;
                    st->arg = arg;
                    st->want = want;
                    st->Z = P.total;
                    st->ncand = 0u;
                    st->overflow = 0u;
                    st->active = deferred ? 1u : 0u;
                }
                done = true;
            } else if (want >= a.V) {
                double dn = 0.0, rr = 0.0;
                uint32_t tk = 0;
                const int ok = full_vocab_value_path(s, c, row.top_p, u, arg, &tk, &dn, &rr, &Z);
                rep.total = Z;
                if (ok) {
                    token = tk;
                    rep.denom = dn;
                    rep.r = rr;
                    rep.path = 2;
                    done = true;
                }
            }
            if (!done) {
                // the fallback writes through pointers: copies keep the kernel's own report and
                // token out of addressable (scratch) memory on every other path
                RowReport rr = rep;
                uint32_t tk = token;
                radix_select(s, c, row, u, want, Z, arg, &tk, &rr);
                rep = rr;
                token = tk;
            }
        }
    }

    if (!deferred) write_row(a, b, token, rep, hlen);
}

void launch_select(const Head& h, int batch, const SelectArgs& args, const FvList& fv, hipStream_t st) {
    SelectArgs a = args;
    if (fv.n > kFvMaxRows || fv.n > (uint32_t)batch || (fv.n && batch > 256))
        throw std::runtime_error("full-vocabulary row list too long");
    const bool multi = fv.n > 0u && h.fv_acc;
    const uint32_t slices = multi ? std::min(kFvMaxSlices, std::max(kFvMinSlices, kFvSliceBudget / fv.n)) : 0u;
    a.fv_acc = multi ? h.fv_acc : nullptr;
    a.fv_merged = h.fv_merged;
    a.fv_cand = h.fv_cand;
    a.fv_state = h.fv_state;
    uint2* scratch = reinterpret_cast<uint2*>(h.list_scratch);
    if (multi) {
        hipLaunchKernelGGL(k_fv_hist, dim3(slices, fv.n), dim3(kMaxSelThreads), 0, st, a, fv);
        check_hip(hipGetLastError(), "select (slice histograms)");
    }
    hipLaunchKernelGGL(k_select<kMaxSelThreads>, dim3((unsigned)batch), dim3(kMaxSelThreads), 0, st, a, scratch);
    check_hip(hipGetLastError(), "select");
    if (multi) {
        hipLaunchKernelGGL(k_fv_gather, dim3(slices, fv.n), dim3(kMaxSelThreads), 0, st, a, fv, scratch);
        check_hip(hipGetLastError(), "select (slice gather)");
        hipLaunchKernelGGL(k_fv_finish, dim3(fv.n), dim3(kMaxSelThreads), 0, st, a, fv, scratch);
        check_hip(hipGetLastError(), "select (finish)");
    }
}

}  // namespace tdt
