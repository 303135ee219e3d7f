// Token selection: greedy argmax or the sampled draw of sample_token (src/sampling.cpp:92-169).
//
// One 1024-thread workgroup per batch row, reading the row's final logits and the per-64-id
// block partials the head epilogue wrote (max, lowest argmax, sum exp(l - max)).
//
//  greedy     argmax of the block partials, ties to the lowest id (:97-104).
//  shortlist  (want = top_k, or 256 without the full-vocabulary flag; :122-137)
//             tau = want-th largest block maximum (count radix select over the partials) is a
//             lower bound of the want-th largest logit, so every shortlist member lies in a
//             block whose maximum is >= tau. Those blocks are gathered (elements >= tau),
//             bitonic-sorted by (logit desc, id asc), and the first `want` form the shortlist.
//             Nucleus over full-distribution probabilities (:139-151) and the temperature draw
//             (:153-168) run as double-precision block scans over <= 256 candidates.
//  general    full-vocabulary nucleus (want = V) and shortlist overflow (more than kCandCap
//             elements >= tau, e.g. massive ties): weighted radix select over the whole row.
//             Each "find" locates the first element, in (logit desc, id asc) order within a
//             prefix set, at which a cumulative weight reaches a target: an 11-bit histogram
//             pass over the row, compaction of the crossing bucket, two more radix levels on
//             the compacted list, then the tie among equal keys (equal weights) is resolved
//             by count and a radix select over ids.
#include <stdexcept>

#include "dt_internal.h"

namespace tdt {

constexpr uint32_t kSelThreads = 1024;
constexpr uint32_t kSelWaves = kSelThreads / 64;
constexpr uint32_t kCandCap = 4096;
constexpr uint32_t kTileCap = 2048;
constexpr uint32_t kBins = 2048;

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
};

struct SelShared {
    union {
        double hd[kBins];
        uint32_t hu[kBins];
    };
    unsigned long long cand[kCandCap];
    uint32_t tiles[kTileCap];
    double wsum_d[kSelWaves];
    uint32_t wsum_u[kSelWaves];
    float wmax[kSelWaves];
    uint32_t warg[kSelWaves];
    // broadcast slots
    double bd[4];
    uint32_t bu[8];
    float bf[4];
};

// ---- block primitives ------------------------------------------------------------------------

template <typename T>
__device__ inline T wave_incl_scan(T v, uint32_t lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T n = __shfl_up(v, o, 64);
        if ((int)lane >= o) v += n;
    }
    return v;
}

template <typename T>
__device__ inline T* wslot(SelShared& s);
template <>
__device__ inline double* wslot<double>(SelShared& s) { return s.wsum_d; }
template <>
__device__ inline uint32_t* wslot<uint32_t>(SelShared& s) { return s.wsum_u; }

// Exclusive scan over the block in thread order; returns the exclusive prefix, total in *tot.
template <typename T>
__device__ inline T block_excl_scan(T v, SelShared& s, T* tot) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const T incl = wave_incl_scan(v, lane);
    T* ws = wslot<T>(s);
    __syncthreads();
    if (lane == 63u) ws[wave] = incl;
    __syncthreads();
    T off = T(0), all = T(0);
    for (uint32_t w = 0; w < kSelWaves; ++w) {
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
    for (uint32_t w = 0; w < kSelWaves; ++w) r = min(r, s.wsum_u[w]);
    __syncthreads();
    return r;
}

// Finds, scanning the histogram from the highest bin down, the bin where the running total
// first reaches `target` (before < target <= before + h). Returns 1 and sets bin/above when
// target <= total. Otherwise returns 0, or with `clamp` uses target = total (the last
// non-empty bin). nb is 2048 or 1024.
template <typename T>
__device__ inline int hist_cross(SelShared& s, uint32_t nb, T target, uint32_t* bin, T* above,
                                 bool clamp = false) {
    const uint32_t tid = threadIdx.x;
    const uint32_t per = nb / kSelThreads;  // 1 or 2
    T* h = (T*)(sizeof(T) == 8 ? (void*)s.hd : (void*)s.hu);
    T loc = T(0);
    for (uint32_t j = 0; j < per; ++j) loc += h[nb - 1u - (tid * per + j)];
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
        const T hv = h[bi];
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

// ---- per-row context ---------------------------------------------------------------------------

struct RowCtx {
    uint32_t b, V;
    const float* l;      // row logits
    float m;             // row max
    float T;             // temperature
    uint2* list;         // compaction scratch [V]
};

// Weight of logit v in mode 0 (count), 1 (exp(v - m)), 2 (exp((v - m) / T)).
__device__ inline double weight(const RowCtx& c, float v, int mode) {
    if (mode == 0) return 1.0;
    if (v == -INFINITY) return 0.0;
    const double d = (double)v - (double)c.m;
    if (mode == 1) return (double)expf((float)d);
    return (double)expf((float)(d / (double)c.T));
}

// Prefix set in (key desc, id asc) order: bounded by element (kb, ib) inclusive, or everything.
struct PSet {
    int bounded;
    uint32_t kb, ib;
    __device__ bool has(uint32_t k, uint32_t id) const {
        return !bounded || k > kb || (k == kb && id <= ib);
    }
};

// Radix select over ids: the j-th smallest id (0-based) among list entries with key == kx.
__device__ inline uint32_t select_tied_id(SelShared& s, const uint2* list, uint32_t n, uint32_t kx,
                                          uint32_t j) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0, rem = j + 1;  // rank from the bottom, 1-based
    const int shifts[3] = {21, 10, 0};
    const uint32_t nbs[3] = {2048u, 2048u, 1024u};
    for (int lv = 0; lv < 3; ++lv) {
        const uint32_t nb = nbs[lv], sh = (uint32_t)shifts[lv];
        for (uint32_t i = tid; i < kBins; i += kSelThreads) s.hu[i] = 0u;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kSelThreads) {
            const uint2 e = list[i];
            if (e.x == kx && (e.y & mask) == prefix) atomicAdd(&s.hu[(e.y >> sh) & (nb - 1u)], 1u);
        }
        __syncthreads();
        // ascending scan: smallest ids first. Reverse the bin order for hist_cross (which scans
        // from the top) by reading bins mirrored.
        for (uint32_t i = tid; i < nb / 2; i += kSelThreads) {
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
__device__ int find_cross(SelShared& s, const RowCtx& c, const PSet& ps, int mode, double target,
                          uint32_t* kx, uint32_t* ix) {
    const uint32_t tid = threadIdx.x;
    // level 1: 11-bit histogram over the row
    for (uint32_t i = tid; i < kBins; i += kSelThreads) s.hd[i] = 0.0;
    __syncthreads();
    for (uint32_t i = tid; i < c.V; i += kSelThreads) {
        const float v = c.l[i];
        const uint32_t k = float_key(v);
        if (!ps.has(k, i)) continue;
        const double w = weight(c, v, mode);
        if (w != 0.0) atomicAdd(&s.hd[k >> 21], w);
    }
    __syncthreads();
    uint32_t d1;
    double above;
    if (!hist_cross<double>(s, kBins, target, &d1, &above)) return 0;
    double rem = target - above;
    // compact bucket d1 (set members) into the list
    if (tid == 0) s.bu[2] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < c.V; i += kSelThreads) {
        const float v = c.l[i];
        const uint32_t k = float_key(v);
        if ((k >> 21) != d1 || !ps.has(k, i)) continue;
        const uint32_t slot = atomicAdd(&s.bu[2], 1u);
        c.list[slot] = make_uint2(k, i);
    }
    __syncthreads();
    const uint32_t n = s.bu[2];
    __syncthreads();
    // levels 2 and 3 on the list
    uint32_t prefix = d1 << 21, mask = 0xFFE00000u;
    const int shifts[2] = {10, 0};
    const uint32_t nbs[2] = {2048u, 1024u};
    for (int lv = 0; lv < 2; ++lv) {
        const uint32_t nb = nbs[lv], sh = (uint32_t)shifts[lv];
        for (uint32_t i = tid; i < kBins; i += kSelThreads) s.hd[i] = 0.0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kSelThreads) {
            const uint2 e = c.list[i];
            if ((e.x & mask) != prefix) continue;
            const double w = weight(c, key_float(e.x), mode);
            if (w != 0.0) atomicAdd(&s.hd[(e.x >> sh) & (nb - 1u)], w);
        }
        __syncthreads();
        uint32_t d;
        double ab;
        // The bucket's weight was summed in another order at the previous level, so a target
        // within rounding of the bucket total may exceed this level's total: clamp it.
        if (!hist_cross<double>(s, nb, rem, &d, &ab, true)) return 0;
        rem -= ab;
        prefix |= d << sh;
        mask |= (nb - 1u) << sh;
    }
    const uint32_t kk = prefix;
    // ties: equal keys have equal weight w; the crossing is the j-th smallest tied id with
    // (j + 1) * w >= rem.
    uint32_t nt = 0;
    for (uint32_t i = tid; i < n; i += kSelThreads) nt += (c.list[i].x == kk) ? 1u : 0u;
    nt = block_sum<uint32_t>(nt, s);
    const double w = weight(c, key_float(kk), mode);
    uint32_t j = 0;
    if (w > 0.0) {
        const double q = ceil(rem / w) - 1.0;
        j = (q <= 0.0) ? 0u : (q >= (double)(nt - 1u) ? nt - 1u : (uint32_t)q);
    }
    const uint32_t id = select_tied_id(s, c.list, n, kk, j);
    if (id == 0xFFFFFFFFu) return 0;
    *kx = kk;
    *ix = id;
    return 1;
}

// ---- the kernel ----------------------------------------------------------------------------------

__global__ __launch_bounds__(kSelThreads) void k_select(SelectArgs a, uint2* __restrict__ scratch) {
    __shared__ SelShared s;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t b = blockIdx.x;
    const DevRow row = a.rows[b];
    const float u = a.uniforms ? a.uniforms[b] : row.u;
    const BlockPartial* parts = a.partials + (size_t)b * a.ntile;

    // 1. row max, lowest argmax, total mass from the block partials.
    float bm = -INFINITY;
    uint32_t ba = 0xFFFFFFFFu;
    for (uint32_t t = tid; t < a.ntile; t += kSelThreads) {
        const BlockPartial p = parts[t];
        if (p.max > bm || (p.max == bm && p.arg < ba)) { bm = p.max; ba = p.arg; }
    }
    wave_argmax(bm, ba);
    if (lane == 0) { s.wmax[wave] = bm; s.warg[wave] = ba; }
    __syncthreads();
    float m = s.wmax[0];
    uint32_t arg = s.warg[0];
    for (uint32_t w = 1; w < kSelWaves; ++w) {
        const float v = s.wmax[w];
        const uint32_t i = s.warg[w];
        if (v > m || (v == m && i < arg)) { m = v; arg = i; }
    }
    __syncthreads();

    RowReport rep = {};
    rep.max_logit = m;
    rep.u = u;
    uint32_t token = arg;

    if (row.temperature <= 0.0f) {
        rep.path = 0;
        rep.shortlist = 1;
        rep.cut = 1;
    } else {
        double zl = 0.0;
        if (m != -INFINITY)
            for (uint32_t t = tid; t < a.ntile; t += kSelThreads) {
                const BlockPartial p = parts[t];
                if (p.max != -INFINITY) zl += exp((double)p.max - (double)m) * (double)p.sumexp;
            }
        const double Z = block_sum<double>(zl, s);
        rep.total = Z;
        const float* lrow = a.logits + (size_t)b * a.V;
        const uint32_t want = row.want;
        rep.shortlist = want;
        bool general = (want > kMaxTopK);
        if (!(Z > 0.0) || m == -INFINITY) {
            token = 0xFFFFFFFFu;
            rep.path = 3;
            general = false;
        } else if (!general) {
            // ---- shortlist path ----
            uint32_t tau = 0u;
            if (a.ntile > want) {
                uint32_t prefix = 0, mask = 0, rem = want;
                const int shifts[3] = {21, 10, 0};
                const uint32_t nbs[3] = {2048u, 2048u, 1024u};
                for (int lv = 0; lv < 3; ++lv) {
                    const uint32_t nb = nbs[lv], sh = (uint32_t)shifts[lv];
                    for (uint32_t i = tid; i < kBins; i += kSelThreads) s.hu[i] = 0u;
                    __syncthreads();
                    for (uint32_t t = tid; t < a.ntile; t += kSelThreads) {
                        const uint32_t k = float_key(parts[t].max);
                        if ((k & mask) == prefix) atomicAdd(&s.hu[(k >> sh) & (nb - 1u)], 1u);
                    }
                    __syncthreads();
                    uint32_t bin = 0, above = 0;
                    hist_cross<uint32_t>(s, nb, rem, &bin, &above);
                    rem -= above;
                    prefix |= bin << sh;
                    mask |= (nb - 1u) << sh;
                }
                tau = prefix;
            }
            // qualifying blocks
            if (tid == 0) { s.bu[3] = 0u; s.bu[4] = 0u; }
            __syncthreads();
            for (uint32_t t = tid; t < a.ntile; t += kSelThreads) {
                if (float_key(parts[t].max) >= tau) {
                    const uint32_t slot = atomicAdd(&s.bu[3], 1u);
                    if (slot < kTileCap) s.tiles[slot] = t;
                }
            }
            __syncthreads();
            const uint32_t nq = s.bu[3];
            if (nq > kTileCap) {
                general = true;
            } else {
                for (uint32_t j = wave; j < nq; j += kSelWaves) {
                    const uint32_t id = s.tiles[j] * kTileRows + lane;
                    if (id < a.V) {
                        const uint32_t k = float_key(lrow[id]);
                        if (k >= tau) {
                            const uint32_t slot = atomicAdd(&s.bu[4], 1u);
                            if (slot < kCandCap)
                                s.cand[slot] = ((unsigned long long)(~k) << 32) | id;
                        }
                    }
                }
                __syncthreads();
                const uint32_t n = s.bu[4];
                if (n > kCandCap) general = true;
                __syncthreads();
                if (!general) {
                    uint32_t P = 2;
                    while (P < n) P <<= 1;
                    for (uint32_t i = n + tid; i < P; i += kSelThreads) s.cand[i] = ~0ull;
                    __syncthreads();
                    for (uint32_t size = 2; size <= P; size <<= 1) {
                        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                            for (uint32_t i = tid; i < P / 2; i += kSelThreads) {
                                const uint32_t lo = 2 * i - (i & (stride - 1));
                                const uint32_t hi = lo + stride;
                                const bool up = ((lo & size) == 0);
                                const unsigned long long x = s.cand[lo], y = s.cand[hi];
                                if ((x > y) == up) { s.cand[lo] = y; s.cand[hi] = x; }
                            }
                            __syncthreads();
                        }
                    }
                    const uint32_t W = min(want, n);
                    float li = -INFINITY;
                    uint32_t idi = 0;
                    if (tid < W) {
                        const unsigned long long cv = s.cand[tid];
                        li = key_float(~(uint32_t)(cv >> 32));
                        idi = (uint32_t)cv;
                    }
                    uint32_t cut = W;
                    if (row.top_p < 1.0f) {
                        const double p = (tid < W) ? exp((double)li - (double)m) / Z : 0.0;
                        const double run = block_excl_scan<double>(p, s, nullptr) + p;
                        const uint32_t first =
                            block_min_u((tid < W && run >= (double)row.top_p) ? tid : 0xFFFFFFFFu, s);
                        if (first != 0xFFFFFFFFu) cut = first + 1u;
                    }
                    if (row.top_k > 0 && cut > (uint32_t)row.top_k) cut = (uint32_t)row.top_k;
                    if (cut < 1u) cut = 1u;
                    const double q = (tid < cut) ? exp(((double)li - (double)m) / (double)row.temperature) : 0.0;
                    double denom;
                    const double acc = block_excl_scan<double>(q, s, &denom) + q;
                    const double r = (double)u * denom;
                    const uint32_t pick = block_min_u((tid < cut && acc >= r) ? tid : 0xFFFFFFFFu, s);
                    const uint32_t rank = (pick == 0xFFFFFFFFu) ? cut - 1u : pick;
                    if (tid == rank) s.bu[5] = idi;
                    __syncthreads();
                    token = s.bu[5];
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
            // ---- general path: weighted radix select over the whole row ----
            RowCtx c;
            c.b = b;
            c.V = a.V;
            c.l = lrow;
            c.m = m;
            c.T = row.temperature;
            c.list = scratch + (size_t)b * a.V;
            PSet s0 = {0, 0u, 0u};
            if (want < a.V) {
                uint32_t kx, ix;
                if (find_cross(s, c, s0, 0, (double)want, &kx, &ix)) s0 = PSet{1, kx, ix};
            }
            PSet s1 = s0;
            if (row.top_p < 1.0f) {
                uint32_t kx, ix;
                if (find_cross(s, c, s0, 1, (double)row.top_p * Z, &kx, &ix)) s1 = PSet{1, kx, ix};
            }
            // survivor weight, survivor count, and the last survivor (smallest element)
            double dl = 0.0;
            uint32_t cl = 0;
            uint32_t lk = 0xFFFFFFFFu, li = 0u;  // smallest key, then largest id
            for (uint32_t i = tid; i < a.V; i += kSelThreads) {
                const float v = lrow[i];
                const uint32_t k = float_key(v);
                if (!s1.has(k, i)) continue;
                dl += weight(c, v, 2);
                ++cl;
                if (k < lk || (k == lk && i > li)) { lk = k; li = i; }
            }
            const double denom = block_sum<double>(dl, s);
            const uint32_t cut = block_sum<uint32_t>(cl, s);
            // smallest key then largest id: reduce (lk, ~li) with min
            const unsigned long long lkey = ((unsigned long long)lk << 32) | (uint32_t)(~li);
            {
                unsigned long long v = lkey;
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    const unsigned long long ov = __shfl_xor(v, o, 64);
                    v = ov < v ? ov : v;
                }
                __syncthreads();
                if (lane == 0) s.cand[wave] = v;
                __syncthreads();
                if (tid == 0) {
                    unsigned long long best = s.cand[0];
                    for (uint32_t w = 1; w < kSelWaves; ++w) best = s.cand[w] < best ? s.cand[w] : best;
                    s.bu[6] = ~(uint32_t)best;
                }
                __syncthreads();
            }
            const uint32_t last_id = s1.bounded ? s1.ib : s.bu[6];
            const double r = (double)u * denom;
            uint32_t kx, ix;
            if (r <= 0.0) {
                token = arg;  // first element in sorted order
            } else if (find_cross(s, c, s1, 2, r, &kx, &ix)) {
                token = ix;
            } else {
                token = last_id;
            }
            rep.cut = cut;
            rep.denom = denom;
            rep.r = r;
            rep.path = 2;
        }
    }

    if (tid == 0) {
        a.tokens[b] = token;
        if (a.report) reinterpret_cast<RowReport*>(a.report)[b] = rep;
        if (a.history && a.hist_len && token != 0xFFFFFFFFu) {
            const uint32_t len = a.hist_len[b];
            if (len < a.hist_stride) {
                a.history[(size_t)b * a.hist_stride + len] = token;
                a.hist_len[b] = len + 1u;
            }
        }
    }
}

void launch_select(const Head& h, int batch, const SelectArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(k_select, dim3((unsigned)batch), dim3(kSelThreads), 0, st, a,
                       reinterpret_cast<uint2*>(h.list_scratch));
    check_hip(hipGetLastError(), "select");
}

}  // namespace tdt
