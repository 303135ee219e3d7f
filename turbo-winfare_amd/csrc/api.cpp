// C ABI of the decode tail (include/turbo_decode_tail.h).
//
// Mirrors the conventions of the reference C API (src/c_api.cpp): a thread-local last error,
// NULL / 0 on failure, every entry point catching all exceptions. The host-side numerics that
// the reference keeps on the CPU (validate_sampling, splitmix64, seed_for, the per-token
// uniform; src/sampling.cpp:18-72) are restated here; everything else is enqueued on the GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>

#include "turbo_decode_tail.h"
#include "dt_bundle.h"
#include "dt_internal.h"

namespace tdt {

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    }
}

}  // namespace tdt

using tdt::Head;
using tdt::check_hip;

namespace {

thread_local std::string g_last_error;

void set_error(const std::string& m) { g_last_error = m; }
void clear_error() { g_last_error.clear(); }

constexpr int kMaxBatch = 256;


struct HandleBox {
    uint32_t magic = 0x54445448u;  // "TDTH"
    Head h;
    double t_accum_ms = 0.0;
    int t_accum_n = 0;
};

HandleBox* box(void* p) {
    if (!p) throw std::runtime_error("null handle");
    auto* b = static_cast<HandleBox*>(p);
    if (b->magic != 0x54445448u) throw std::runtime_error("invalid handle");
    return b;
}

template <typename T>
T* dalloc(size_t count, const char* what) {
    void* p = nullptr;
    check_hip(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)), what);
    return static_cast<T*>(p);
}

void dfree(void* p) {
    if (p) (void)hipFree(p);
}

// The private stream of turbo_lmhead_create: drained and destroyed on every way out.
struct CreateStream {
    hipStream_t s = nullptr;
    void drain() {
        if (s) {
            (void)hipStreamSynchronize(s);
            (void)hipStreamDestroy(s);
            s = nullptr;
        }
    }
    ~CreateStream() { drain(); }
};

// ---- host restatement of the reference's scalar sampling helpers ---------------------------

uint64_t splitmix64_h(uint64_t x) {  // src/sampling.cpp:56-61
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

uint64_t seed_for_h(int has_seed, uint64_t seed, int position) {  // src/sampling.cpp:63-72
    const uint64_t base = has_seed ? seed + static_cast<uint64_t>(static_cast<int64_t>(position))
                                   : (0x9E3779B97F4A7C15ULL ^
                                      (static_cast<uint64_t>(static_cast<int64_t>(position)) *
                                       0xD1B54A32D192ED03ULL));
    const uint64_t s = splitmix64_h(base);
    return s ? s : 0x9E3779B97F4A7C15ULL;
}

float xorshift_uniform(uint64_t state) {  // src/sampling.cpp:18-28
    state ^= state >> 12;
    state ^= state << 25;
    state ^= state >> 27;
    const uint64_t r = state * 0x2545F4914F6CDD1DULL;
    return static_cast<float>((r >> 40) & 0xFFFFFF) / 16777216.0f;
}

float row_uniform(const TurboSamplingRow& r) {
    if (r.rng == TURBO_RNG_REFERENCE)
        return xorshift_uniform(seed_for_h(r.has_seed, r.seed, static_cast<int>(r.counter)));
    const uint32_t x = tdt::philox4x32_10_x(r.counter, r.seed);
    return static_cast<float>(x >> 8) / 16777216.0f;
}

// validate_sampling (src/sampling.cpp:32-54) plus the extension fields.
bool validate_row(const TurboSamplingRow& p, std::string* why) {
    if (!std::isfinite(p.temperature) || p.temperature < 0.0f) {
        *why = "temperature must be finite and >= 0 (0 = greedy)";
        return false;
    }
    if (!std::isfinite(p.top_p) || p.top_p <= 0.0f || p.top_p > 1.0f) {
        *why = "top_p must be in (0, 1]";
        return false;
    }
    if (p.top_k < 0 || p.top_k > static_cast<int>(tdt::kMaxTopK)) {
        *why = "top_k must be in 0..256 (0 disables it)";
        return false;
    }
    if (!std::isfinite(p.repetition_penalty) || p.repetition_penalty <= 0.0f) {
        *why = "repetition_penalty must be finite and > 0 (1 = disabled)";
        return false;
    }
    if (!std::isfinite(p.presence_penalty) || !std::isfinite(p.frequency_penalty)) {
        *why = "presence_penalty and frequency_penalty must be finite";
        return false;
    }
    if (p.rng != TURBO_RNG_PHILOX && p.rng != TURBO_RNG_REFERENCE) {
        *why = "rng must be TURBO_RNG_PHILOX or TURBO_RNG_REFERENCE";
        return false;
    }
    // the reference's position is an int (src/sampling.cpp:63): counter holds it as a 64-bit
    // two's-complement value, which must fit
    if (p.rng == TURBO_RNG_REFERENCE) {
        const int64_t pos = static_cast<int64_t>(p.counter);
        if (pos < INT32_MIN || pos > INT32_MAX) {
            *why = "counter must hold an int position (-2^31 .. 2^31-1) for TURBO_RNG_REFERENCE";
            return false;
        }
    }
    if ((p.flags & ~static_cast<uint32_t>(TURBO_ROW_FULL_VOCAB)) != 0u) {
        *why = "unknown row flags";
        return false;
    }
    if (!(p.flags & TURBO_ROW_FULL_VOCAB) && p.temperature > 0.0f && p.top_p < 1.0f &&
        p.top_k == 0) {
        *why = "top_p < 1 with temperature > 0 requires top_k in 1..256; full-vocabulary nucleus "
               "sampling needs TURBO_ROW_FULL_VOCAB";
        return false;
    }
    return true;
}

// Waits for the handle's own stream only (other streams of the process keep running), then frees.
void free_head(Head& h) {
    (void)hipStreamSynchronize(h.stream);
    dfree(h.Wt);
    dfree(h.SBt);
    dfree(h.gamma);
    dfree(h.xn);
    dfree(h.xdig);
    dfree(h.xws);
    dfree(h.xsum);
    dfree(h.x16);
    dfree(h.xscale);
    dfree(h.SB16t);
    dfree(h.logits);
    dfree(h.partials);
    dfree(h.rows);
    dfree(h.mods);
    dfree(h.mod_count);
    dfree(h.block_start);
    dfree(h.hcount);
    dfree(h.hbits);
    dfree(h.list_scratch);
    dfree(h.fv_acc);
    dfree(h.fv_merged);
    dfree(h.fv_cand);
    dfree(h.fv_state);
    if (h.ring_host) (void)hipHostFree(h.ring_host);
    if (h.overflow_host) (void)hipHostFree(h.overflow_host);
    for (int i = 0; i < Head::kRing / Head::kRingGroup; ++i)
        if (h.ring_ev[i]) (void)hipEventDestroy(h.ring_ev[i]);
    for (int i = 0; i < Head::kTimerSlots; ++i) {
        if (h.t_start[i]) (void)hipEventDestroy(h.t_start[i]);
        if (h.t_stop[i]) (void)hipEventDestroy(h.t_stop[i]);
    }
}

// Hands B DevRows to the step-prep kernel, which copies them into device memory (no separate
// copy is enqueued). Up to kInlineRows ride in the kernel arguments. Larger batches use the next
// slot of the pinned ring; a group of slots is refilled only after the event recorded behind the
// prep kernel that read the group's last slot has passed. An event record costs the stream a
// few microseconds (the queue drains and caches are written back for the host), so it is taken
// once per group, not per step. Returns the ring slot used, -1 for none.
int stage_rows(Head& h, const tdt::DevRow* rows, int B, tdt::PrepArgs* a) {
    if (B <= tdt::kInlineRows) {
        std::memcpy(a->inl, rows, sizeof(tdt::DevRow) * B);
        a->rows_src = nullptr;
        return -1;
    }
    const int pos = h.ring_pos;
    h.ring_pos = (h.ring_pos + 1) % Head::kRing;
    if (pos % Head::kRingGroup == 0)
        check_hip(hipEventSynchronize(h.ring_ev[pos / Head::kRingGroup]), "row staging wait");
    tdt::DevRow* slot = h.ring_host + static_cast<size_t>(pos) * h.max_batch;
    std::memcpy(slot, rows, sizeof(tdt::DevRow) * B);
    a->rows_src = h.ring_dev + static_cast<size_t>(pos) * h.max_batch;
    return pos;
}

void release_slot(Head& h, int pos) {
    if (pos >= 0 && pos % Head::kRingGroup == Head::kRingGroup - 1)
        check_hip(hipEventRecord(h.ring_ev[pos / Head::kRingGroup], h.stream), "row staging record");
}

tdt::PrepArgs prep_args(const Head& h, int B) {
    tdt::PrepArgs a{};
    a.B = B;
    a.rows_dst = h.rows;
    a.gamma = h.gamma;
    a.eps = h.eps;
    a.D = h.D;
    a.xdig = h.xdig;
    a.xws = h.xws;
    a.xsum = h.xsum;
    a.x16 = h.x16;
    a.x16_denorm = h.mfma_denorm ? 1 : 0;
    a.xscale = h.xscale;
    a.V = h.V;
    a.ntile = h.ntile;
    a.P = 2;
    a.mods = h.mods;
    a.mod_cap = h.mod_cap;
    a.hcount = h.hcount;
    a.hbits = h.hbits;
    a.hbw = h.hbw;
    a.mod_count = h.mod_count;
    a.block_start = h.block_start;
    return a;
}

// Row parameters + (optionally) activations, no modifiers: one step-prep launch.
void simple_prep(Head& h, const tdt::DevRow* rows, int B, const void* x, int dtype, bool normed,
                 float* xn, tdt::HeadPath path) {
    tdt::PrepArgs a = prep_args(h, B);
    const int pos = stage_rows(h, rows, B, &a);
    a.hidden = x;
    a.dtype = dtype;
    a.normed = normed ? 1 : 0;
    a.xn = xn;
    a.path = path == tdt::HeadPath::Digits ? 0 : 1;
    tdt::launch_step_prep(h, a, false, h.stream);
    release_slot(h, pos);
}

tdt::DevRow make_devrow(const Head& h, const TurboSamplingRow& r, uint32_t has_mods) {
    tdt::DevRow d{};
    d.temperature = r.temperature;
    d.top_p = r.top_p;
    d.top_k = r.top_k;
    d.repetition_penalty = r.repetition_penalty;
    d.presence_penalty = r.presence_penalty;
    d.frequency_penalty = r.frequency_penalty;
    d.u = row_uniform(r);
    d.flags = r.flags;
    if (r.top_k > 0) d.want = std::min<uint32_t>(static_cast<uint32_t>(r.top_k), h.V);
    else if (r.flags & TURBO_ROW_FULL_VOCAB) d.want = h.V;
    else d.want = std::min<uint32_t>(tdt::kMaxTopK, h.V);
    d.has_mods = has_mods;
    return d;
}

tdt::DevRow greedy_devrow(const Head& h) {
    TurboSamplingRow r;
    turbo_sampling_row_default(&r);
    return make_devrow(h, r, 0u);
}

tdt::EpiArgs epi_args(const Head& h, float* logits, bool softcap) {
    tdt::EpiArgs ep{};
    ep.V = h.V;
    ep.ntile = h.ntile;
    ep.cap = softcap ? h.cap : 0.0f;
    ep.logits = logits;
    ep.partials = h.partials;
    ep.rows = h.rows;
    ep.mods = h.mods;
    ep.mod_cap = h.mod_cap;
    ep.block_start = h.block_start;
    ep.hcount = h.hcount;
    ep.hbits = h.hbits;
    ep.hbw = h.hbw;
    ep.ban = nullptr;
    ep.ban_stride = 0;
    ep.rep_limit = (h.cap > 0.0f) ? h.cap * 0.9999f : 0.0f;
    ep.no_sumexp = 1u;  // the sampling step sets 0 when a row samples from a shortlist
    ep.xscale = h.xscale;
    return ep;
}

// fused: the small-batch step with the preparation folded into the head kernel (or null).
void launch_head(HandleBox& bx, int B, const tdt::EpiArgs& ep, const tdt::FusedPrep* fused = nullptr) {
    Head& h = bx.h;
    const bool timed = h.timing && (h.t_launch++ % h.t_stride) == 0u;
    if (timed && h.t_count >= Head::kTimerSlots) {
        check_hip(hipStreamSynchronize(h.stream), "timer fold");
        for (int i = 0; i < h.t_count; ++i) {
            float ms = 0.f;
            check_hip(hipEventElapsedTime(&ms, h.t_start[i], h.t_stop[i]), "timer read");
            bx.t_accum_ms += ms;
        }
        bx.t_accum_n += h.t_count;
        h.t_count = 0;
    }
    hipEvent_t ev0 = timed ? h.t_start[h.t_count] : nullptr;
    hipEvent_t ev1 = timed ? h.t_stop[h.t_count] : nullptr;
    if (fused) tdt::launch_head_digits_fused(h, B, *fused, ep, h.stream, ev0, ev1);
    else if (B <= 2) tdt::launch_head_digits(h, B, ep, h.stream, ev0, ev1);
    else tdt::launch_head_mfma(h, B, ep, h.stream, ev0, ev1);
    if (timed) ++h.t_count;
}

tdt::HeadPath path_for(int B) { return B <= 2 ? tdt::HeadPath::Digits : tdt::HeadPath::Mfma; }

// Batches above two rows run on the matrix cores, whose fp16 table cannot hold scales or biases
// beyond the fp16 range; such a head serves one- and two-row calls only.
void check_head_path(const Head& h, int B) {
    if (B > 2 && !h.mfma_ok)
        throw std::runtime_error("this head's scales or biases exceed the fp16 range (|x| > 65504), which the "
                                 "matrix-core path for batches above 2 rows cannot represent; call with batch <= 2");
    if (B > 2 && !tdt::mfma_table_fits(h))
        throw std::runtime_error("this head's table exceeds the 4 GiB the matrix-core path for batches above 2 "
                                 "rows addresses; call with batch <= 2");
}

// The head over normalised rows x with greedy row parameters (turbo_lmhead_logits,
// turbo_int4_matvec, turbo_lmhead_greedy). One or two 16-byte-aligned rows: the head kernel
// computes the digit planes itself (no preparation kernel), with one workgroup per 16 tiles or,
// for few tiles, per tile; it also stores the rows for a select kernel that follows.
void launch_greedy_head(HandleBox& bx, const tdt::DevRow* rows, int batch, const void* x, int x_dtype,
                        const tdt::EpiArgs& ep) {
    Head& h = bx.h;
    check_head_path(h, batch);
    const uint32_t nt = tdt::split_threads(h);
    const bool fold = batch <= tdt::kFusedRows && h.D <= tdt::kFusedMaxD &&
                      (reinterpret_cast<uintptr_t>(x) & 15u) == 0u &&
                      (h.ntile >= tdt::kFusedMinTiles || (nt && h.D <= 8u * nt));
    if (fold) {
        tdt::FusedPrep fp{};
        fp.hidden = x;
        fp.dtype = x_dtype == TURBO_HIDDEN_BF16 ? 1 : 0;
        fp.normed = 1;
        fp.eps = h.eps;
        fp.rows_dst = h.rows;
        for (int b = 0; b < batch; ++b) fp.inl[b] = rows[b];
        launch_head(bx, batch, ep, &fp);
        return;
    }
    simple_prep(h, rows, batch, x, x_dtype == TURBO_HIDDEN_BF16 ? 1 : 0, true, nullptr, path_for(batch));
    launch_head(bx, batch, ep);
}

void check_batch(const Head& h, int B) {
    if (B < 1 || B > h.max_batch)
        throw std::runtime_error("batch must be in 1.." + std::to_string(h.max_batch));
}

}  // namespace

namespace tdt {

// Shared by turbo_lmhead_step, turbo_sample_logits and turbo_sample_logits_noalloc. bx (the
// handle, for head-kernel timing) may be null when hidden is null: no head kernel runs then.
int run_rows(Head& h, HandleBox* bx, const TurboStepInputs* in, const TurboStepOutputs* out,
             const void* hidden, float* given_logits) {
    if (!in || !out) throw std::runtime_error("null inputs or outputs");
    if (hidden && !bx) throw std::runtime_error("a head step needs a handle");
    const int B = in->batch;
    check_batch(h, B);
    if (hidden) check_head_path(h, B);
    if (!in->rows) throw std::runtime_error("rows is NULL");
    if (!out->tokens) throw std::runtime_error("out->tokens is NULL");
    if (hidden && in->hidden_dtype != TURBO_HIDDEN_F32 && in->hidden_dtype != TURBO_HIDDEN_BF16)
        throw std::runtime_error("hidden_dtype must be TURBO_HIDDEN_F32 or TURBO_HIDDEN_BF16");
    const bool has_hist = in->history && in->history_len && in->history_stride > 0;
    const bool has_bias = in->bias_ids && in->bias_values && in->bias_count && in->bias_stride > 0;
    if ((in->flags & TURBO_STEP_APPEND_HISTORY) && !has_hist)
        throw std::runtime_error("TURBO_STEP_APPEND_HISTORY needs history, history_len and history_stride");
    if (in->ban_bits && in->ban_stride < (h.V + 31u) / 32u)
        throw std::runtime_error("ban_stride must be at least ceil(vocab / 32) words");

    tdt::DevRow rows[kMaxBatch];
    bool all_greedy = true, any_mods = false, any_short = false;
    tdt::FvList fv;
    uint32_t n_fv = 0;
    for (int b = 0; b < B; ++b) {
        const TurboSamplingRow& r = in->rows[b];
        std::string why;
        if (!validate_row(r, &why)) throw std::runtime_error("row " + std::to_string(b) + ": " + why);
        const bool uses_hist = has_hist && (r.repetition_penalty != 1.0f ||
                                            r.presence_penalty != 0.0f || r.frequency_penalty != 0.0f);
        const uint32_t mods = (uses_hist ? 1u : 0u) | (has_bias ? 2u : 0u);
        any_mods = any_mods || mods != 0u;
        all_greedy = all_greedy && r.temperature <= 0.0f;
        rows[b] = make_devrow(h, r, mods);
        if (rows[b].temperature > 0.0f && rows[b].want >= h.V) {  // full-vocabulary rows
            if (n_fv < tdt::kFvMaxRows) {
                fv.temp[n_fv] = rows[b].temperature;
                fv.row[n_fv] = static_cast<uint8_t>(b);
            }
            ++n_fv;
        }
        any_short = any_short || (rows[b].temperature > 0.0f && rows[b].want < h.V);
    }
    fv.n = (n_fv <= tdt::kFvMaxRows) ? n_fv : 0u;  // many such rows: one workgroup per row
    uint32_t P = 2;
    if (has_bias) P = tdt::modtable_sort_size(h, in->bias_stride);
    float* logits = given_logits ? given_logits : (out->logits ? out->logits : (all_greedy ? nullptr : h.logits));

    // Batches of one or two rows over the LM head's shape fold the preparation into the head
    // kernel, unless a bias table is needed (it is sorted by the preparation kernel), the
    // history is long enough that every workgroup scanning it would cost more than one kernel,
    // or the hidden rows are not 16-byte aligned (the fold reads them in 16-byte pieces).
    const bool fold = hidden && B <= tdt::kFusedRows && !has_bias && h.D <= tdt::kFusedMaxD &&
                      h.ntile >= tdt::kFusedMinTiles && (reinterpret_cast<uintptr_t>(hidden) & 15u) == 0u &&
                      (!has_hist || in->history_stride <= tdt::kFusedHistMax);
    if (fold) {
        tdt::FusedPrep fp{};
        fp.hidden = hidden;
        fp.dtype = in->hidden_dtype == TURBO_HIDDEN_BF16 ? 1 : 0;
        fp.normed = (in->flags & TURBO_STEP_NORMED) ? 1 : 0;
        fp.gamma = h.gamma;
        fp.eps = h.eps;
        if (any_mods) {
            fp.history = in->history;
            fp.hist_len = in->history_len;
            fp.hist_stride = in->history_stride;
        }
        fp.rows_dst = h.rows;
        for (int b = 0; b < B; ++b) fp.inl[b] = rows[b];
        tdt::EpiArgs ep = epi_args(h, logits, true);
        ep.no_sumexp = any_short ? 0u : 1u;
        ep.no_smax = any_short ? 0u : 1u;
        ep.ban = in->ban_bits;
        ep.ban_stride = in->ban_stride;
        ep.meta = (any_mods || in->ban_bits) ? 1u : 0u;
        launch_head(*bx, B, ep, &fp);
    }

    tdt::PrepArgs pa = prep_args(h, B);
    const int pos = fold ? -1 : stage_rows(h, rows, B, &pa);
    pa.hidden = hidden;
    pa.dtype = in->hidden_dtype == TURBO_HIDDEN_BF16 ? 1 : 0;
    pa.normed = (in->flags & TURBO_STEP_NORMED) ? 1 : 0;
    pa.path = path_for(B) == tdt::HeadPath::Digits ? 0 : 1;
    pa.P = P;
    for (int b = 0; b < B; ++b) pa.mod_bits[b >> 4] |= (rows[b].has_mods & 3u) << (2 * (b & 15));
    if (has_hist) {
        pa.history = in->history;
        pa.hist_stride = in->history_stride;
        pa.hist_len = in->history_len;
    }
    if (has_bias) {
        pa.bias_ids = in->bias_ids;
        pa.bias_vals = in->bias_values;
        pa.bias_stride = in->bias_stride;
        pa.bias_count = in->bias_count;
    }
    if (!fold) {
        tdt::launch_step_prep(h, pa, any_mods, h.stream);
        release_slot(h, pos);
        tdt::EpiArgs ep = epi_args(h, logits, hidden != nullptr);
        ep.no_sumexp = any_short ? 0u : 1u;  // greedy and full-vocabulary rows do not read them
        ep.no_smax = any_short ? 0u : 1u;
        ep.ban = in->ban_bits;
        ep.ban_stride = in->ban_stride;
        ep.meta = (any_mods || in->ban_bits) ? 1u : 0u;
        if (hidden) launch_head(*bx, B, ep);
        else tdt::launch_logits_epilogue(h, B, ep, h.stream);
    }

    tdt::SelectArgs sa{};
    sa.V = h.V;
    sa.ntile = h.ntile;
    sa.logits = logits;
    sa.partials = h.partials;
    sa.rows = h.rows;
    sa.uniforms = in->uniforms;
    sa.tokens = out->tokens;
    sa.report = out->report;
    if (in->flags & TURBO_STEP_APPEND_HISTORY) {
        sa.history = in->history;
        sa.hist_stride = in->history_stride;
        sa.hist_len = in->history_len;
        sa.hist_overflow = h.overflow_dev;
    }
    tdt::launch_select(h, B, sa, fv, h.stream);
    return 1;
}

void set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }

int sample_on_head(Head& h, const TurboStepInputs* in, const TurboStepOutputs* out, float* logits) {
    if (!logits) throw std::runtime_error("logits is NULL");
    return run_rows(h, nullptr, in, out, nullptr, logits);
}

}  // namespace tdt

using tdt::run_rows;

#define API_TRY try {
#define API_CATCH(ret)                                   \
    }                                                    \
    catch (const std::exception& ex) {                   \
        set_error(ex.what());                            \
        return ret;                                      \
    }                                                    \
    catch (...) {                                        \
        set_error("unknown error");                      \
        return ret;                                      \
    }

namespace {
TurboBundleTensor describe_tensor(const tdt::ResidentEntry& e) {
    TurboBundleTensor t{};
    t.dtype = e.dtype;
    for (int d = 0; d < 4; ++d) t.shape[d] = e.shape[d];
    t.file_offset = e.file_offset;
    t.size_bytes = e.size_bytes;
    t.scale_offset = e.scale_offset;
    t.scale_size = e.scale_size;
    t.bias_offset = e.bias_offset;
    t.bias_size = e.bias_size;
    // src/cpu_reference.cpp:229-247 (an all-zero shape reads as rows = shape[0] = 0 there too)
    t.rows = e.shape[0];
    t.quantized = e.scale_size > 0 ? 1u : 0u;
    if (t.quantized) {
        if (t.rows == 0) throw std::runtime_error(e.name + ": quantised tensor with zero rows");
        const uint64_t groups = e.scale_size / 2u / t.rows;
        t.in_dim = static_cast<uint32_t>(groups * 64u);
        t.bits = (static_cast<uint64_t>(e.shape[1]) * 8u == t.in_dim) ? 4u : 8u;
    } else {
        t.in_dim = t.rows;
        t.bits = 16u;
    }
    return t;
}
}  // namespace

extern "C" {

TURBO_DT_API const char* turbo_lmhead_last_error(void) { return g_last_error.c_str(); }

TURBO_DT_API uint32_t turbo_abi_version(void) { return TURBO_DT_ABI_VERSION; }

TURBO_DT_API size_t turbo_abi_struct_size(int which) {
    switch (which) {
        case TURBO_ABI_LMHEAD_DESC: return sizeof(TurboLMHeadDesc);
        case TURBO_ABI_BUNDLE_TENSOR: return sizeof(TurboBundleTensor);
        case TURBO_ABI_SAMPLING_ROW: return sizeof(TurboSamplingRow);
        case TURBO_ABI_STEP_INPUTS: return sizeof(TurboStepInputs);
        case TURBO_ABI_ROW_REPORT: return sizeof(TurboRowReport);
        case TURBO_ABI_STEP_OUTPUTS: return sizeof(TurboStepOutputs);
        default: return 0;
    }
}

TURBO_DT_API void turbo_lmhead_desc_default(TurboLMHeadDesc* out) {
    if (!out) return;
    std::memset(out, 0, sizeof(*out));
    out->vocab_size = 262144;
    out->hidden_size = 2816;
    out->group_size = 64;
    out->final_logit_softcap = 30.0f;
    out->rms_norm_eps = 1e-6f;
    out->weights_on_device = 0;
    out->device = 0;
}

TURBO_DT_API void* turbo_lmhead_create(const TurboLMHeadDesc* d) {
    clear_error();
    API_TRY
    if (!d) throw std::runtime_error("null descriptor");
    if (d->group_size != 64) throw std::runtime_error("group_size must be 64");
    if (d->hidden_size == 0 || d->hidden_size % 64 != 0 || d->hidden_size > 8192)
        throw std::runtime_error("hidden_size must be a positive multiple of 64, at most 8192");
    if (d->vocab_size == 0 || d->vocab_size > (1u << 24))
        throw std::runtime_error("vocab_size must be in 1..16777216");
    if (!d->weight || !d->scales || !d->biases) throw std::runtime_error("weight/scales/biases are NULL");
    if (!std::isfinite(d->final_logit_softcap) || !std::isfinite(d->rms_norm_eps) || d->rms_norm_eps < 0.f)
        throw std::runtime_error("softcap and eps must be finite, eps >= 0");

    auto bx = std::make_unique<HandleBox>();
    Head& h = bx->h;
    CreateStream cs;
    try {
        int ndev = 0;
        check_hip(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
        if (d->device < 0 || d->device >= ndev) throw std::runtime_error("no such HIP device");
        tdt::DeviceGuard dg(d->device);
        h.device = d->device;
        h.V = d->vocab_size;
        h.D = d->hidden_size;
        h.G = h.D / 64u;
        h.NC = h.D / 32u;
        h.ntile = (h.V + tdt::kTileRows - 1u) / tdt::kTileRows;
        h.cap = d->final_logit_softcap > 0.f ? d->final_logit_softcap : 0.f;
        h.eps = d->rms_norm_eps;
        h.stream = nullptr;
        h.max_batch = kMaxBatch;
        h.mod_cap = tdt::kModCap;
        // create-time uploads, clears and repacks run on a stream of their own, awaited at the end
        check_hip(hipStreamCreateWithFlags(&cs.s, hipStreamNonBlocking), "create stream");

        const size_t wbytes = static_cast<size_t>(h.V) * (h.D / 2u);
        const size_t gcount = static_cast<size_t>(h.V) * h.G;
        h.Wt = dalloc<uint4>(static_cast<size_t>(h.ntile) * h.NC * tdt::kTileRows, "alloc Wt");
        h.SBt = dalloc<uint32_t>(static_cast<size_t>(h.ntile) * h.G * tdt::kTileRows, "alloc SBt");
        h.SB16t = dalloc<uint32_t>(static_cast<size_t>(h.ntile) * h.G * tdt::kTileRows, "alloc SB16t");

        const uint8_t* W = d->weight;
        const uint16_t* S = d->scales;
        const uint16_t* Bi = d->biases;
        uint8_t* tW = nullptr;
        uint16_t* tS = nullptr;
        uint16_t* tB = nullptr;
        if (!d->weights_on_device) {
            tW = dalloc<uint8_t>(wbytes, "alloc staging W");
            tS = dalloc<uint16_t>(gcount, "alloc staging S");
            tB = dalloc<uint16_t>(gcount, "alloc staging B");
            check_hip(hipMemcpyAsync(tW, d->weight, wbytes, hipMemcpyHostToDevice, cs.s), "upload W");
            check_hip(hipMemcpyAsync(tS, d->scales, gcount * 2, hipMemcpyHostToDevice, cs.s), "upload S");
            check_hip(hipMemcpyAsync(tB, d->biases, gcount * 2, hipMemcpyHostToDevice, cs.s), "upload B");
            W = tW;
            S = tS;
            Bi = tB;
        }
        const int repack = tdt::launch_repack(h, W, S, Bi, cs.s);  // waits for cs.s
        h.mfma_denorm = repack == 1;
        h.mfma_ok = repack >= 0;
        dfree(tW);
        dfree(tS);
        dfree(tB);

        if (d->norm_weight) {
            h.gamma = dalloc<uint16_t>(h.D, "alloc gamma");
            check_hip(hipMemcpyAsync(h.gamma, d->norm_weight, h.D * 2u,
                                     d->weights_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, cs.s),
                      "upload gamma");
        }
        const size_t MB = static_cast<size_t>(h.max_batch);
        h.xn = dalloc<float>(MB * h.D, "alloc xn");
        h.xdig = dalloc<uint32_t>(MB * h.NC * tdt::kDigitWordsPerChunk, "alloc xdig");
        h.xws = dalloc<float>(MB * h.G, "alloc xws");
        h.xsum = dalloc<float>(MB * h.G, "alloc xsum");
        h.x16 = dalloc<uint16_t>(MB * h.D, "alloc x16");
        h.xscale = dalloc<float>(MB, "alloc xscale");
        check_hip(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(h.xscale), 0x3f800000, MB, cs.s),
                  "clear xscale");  // 1.0f
        h.logits = dalloc<float>(MB * h.V, "alloc logits");
        h.partials = dalloc<tdt::BlockPartial>(MB * h.ntile, "alloc partials");
        h.rows = dalloc<tdt::DevRow>(MB, "alloc rows");
        h.mods = dalloc<tdt::ModEntry>(MB * h.mod_cap, "alloc mods");
        h.mod_count = dalloc<uint32_t>(MB, "alloc mod_count");
        h.block_start = dalloc<uint32_t>(MB * (h.ntile + 1u), "alloc block_start");
        h.hbw = (h.V + 31u) / 32u;
        h.hcount = dalloc<uint32_t>(MB * h.V, "alloc history counts");
        h.hbits = dalloc<uint32_t>(MB * h.hbw, "alloc history bitmap");
        check_hip(hipMemsetAsync(h.hcount, 0, MB * h.V * sizeof(uint32_t), cs.s), "clear history counts");
        check_hip(hipMemsetAsync(h.hbits, 0, MB * h.hbw * sizeof(uint32_t), cs.s), "clear history bitmap");
        h.list_scratch = dalloc<uint2>(MB * h.V, "alloc list scratch");
        h.fv_acc = dalloc<unsigned long long>(MB * 2u * tdt::kFvBins, "alloc select slice-histogram sums");
        check_hip(hipMemsetAsync(h.fv_acc, 0, MB * 2u * tdt::kFvBins * 8u, cs.s), "clear select slice-histogram sums");
        h.fv_merged = dalloc<unsigned long long>(MB * 2u * tdt::kFvBins, "alloc select histograms");
        h.fv_cand = dalloc<unsigned long long>(MB * tdt::kFvCandCap, "alloc select candidates");
        h.fv_state = dalloc<unsigned char>(MB * tdt::kFvStateBytes, "alloc select state");
        check_hip(hipMemsetAsync(h.fv_state, 0, MB * tdt::kFvStateBytes, cs.s),
                  "clear select state");
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&h.ring_host),
                                sizeof(tdt::DevRow) * MB * Head::kRing,
                                hipHostMallocMapped | hipHostMallocCoherent),
                  "alloc pinned ring");
        check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&h.ring_dev), h.ring_host, 0),
                  "map pinned ring");
        for (int i = 0; i < Head::kRing / Head::kRingGroup; ++i)
            check_hip(hipEventCreateWithFlags(&h.ring_ev[i], hipEventDisableTiming), "ring events");
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&h.overflow_host), sizeof(uint32_t),
                                hipHostMallocMapped | hipHostMallocCoherent),
                  "alloc history overflow word");
        *h.overflow_host = 0u;
        check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&h.overflow_dev), h.overflow_host, 0),
                  "map history overflow word");
        check_hip(hipStreamSynchronize(cs.s), "create");
    } catch (...) {
        cs.drain();
        free_head(h);
        throw;
    }
    return bx.release();
    API_CATCH(nullptr)
}

TURBO_DT_API void turbo_lmhead_destroy(void* handle) {
    if (!handle) return;
    try {
        HandleBox* b = box(handle);
        tdt::DeviceGuard dg(b->h.device);
        free_head(b->h);
        b->magic = 0;
        delete b;
    } catch (...) {
    }
}

TURBO_DT_API int turbo_lmhead_set_stream(void* handle, void* stream) {
    clear_error();
    API_TRY
    Head& h = box(handle)->h;
    const hipStream_t next = static_cast<hipStream_t>(stream);
    if (next != h.stream) {
        // the handle's scratch and timer events belong to work already on the old stream: let it
        // finish before the next step can reuse them from another stream
        tdt::DeviceGuard dg(h.device);
        check_hip(hipStreamSynchronize(h.stream), "set_stream: wait for the previous stream");
        h.stream = next;
    }
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_synchronize(void* handle) {
    clear_error();
    API_TRY
    Head& h = box(handle)->h;
    tdt::DeviceGuard dg(h.device);
    check_hip(hipStreamSynchronize(h.stream), "synchronize");
    if (h.overflow_host && *h.overflow_host) {
        const uint32_t row = *h.overflow_host - 1u;
        *h.overflow_host = 0u;
        throw std::runtime_error("history full: row " + std::to_string(row) +
                                 "'s token was not appended (history_len reached history_stride); "
                                 "later repetition/presence/frequency penalties would miss it");
    }
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_limits(void* handle, int* max_batch, int* max_row_modifiers) {
    clear_error();
    API_TRY
    Head& h = box(handle)->h;
    if (max_batch) *max_batch = h.max_batch;
    if (max_row_modifiers) *max_row_modifiers = static_cast<int>(h.mod_cap);
    return 1;
    API_CATCH(0)
}

TURBO_DT_API void turbo_sampling_row_default(TurboSamplingRow* out) {
    if (!out) return;
    std::memset(out, 0, sizeof(*out));
    out->temperature = 0.0f;
    out->top_p = 1.0f;
    out->top_k = 0;
    out->repetition_penalty = 1.0f;
    out->presence_penalty = 0.0f;
    out->frequency_penalty = 0.0f;
    out->rng = TURBO_RNG_PHILOX;
    out->has_seed = 0;
    out->seed = 0;
    out->counter = 0;
    out->flags = 0;
}

TURBO_DT_API int turbo_validate_sampling(const TurboSamplingRow* row) {
    clear_error();
    API_TRY
    if (!row) throw std::runtime_error("null row");
    std::string why;
    if (!validate_row(*row, &why)) throw std::runtime_error(why);
    return 1;
    API_CATCH(0)
}

TURBO_DT_API uint64_t turbo_splitmix64(uint64_t x) { return splitmix64_h(x); }

TURBO_DT_API uint64_t turbo_seed_for(int has_seed, uint64_t seed, int position) {
    return seed_for_h(has_seed, seed, position);
}

TURBO_DT_API float turbo_row_uniform(const TurboSamplingRow* row) {
    if (!row) return 0.0f;
    return row_uniform(*row);
}

TURBO_DT_API int turbo_lmhead_step(void* handle, const TurboStepInputs* in,
                                   const TurboStepOutputs* out) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    tdt::DeviceGuard dg(bx->h.device);
    if (!in || !in->hidden) throw std::runtime_error("hidden is NULL");
    return run_rows(bx->h, bx, in, out, in->hidden, nullptr);
    API_CATCH(0)
}

TURBO_DT_API int turbo_sample_logits(void* handle, float* logits, const TurboStepInputs* in,
                                     const TurboStepOutputs* out) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    tdt::DeviceGuard dg(bx->h.device);
    if (!logits) throw std::runtime_error("logits is NULL");
    return run_rows(bx->h, bx, in, out, nullptr, logits);
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_rms_norm(void* handle, const float* x, int batch, float* out) {
    clear_error();
    API_TRY
    Head& h = box(handle)->h;
    tdt::DeviceGuard dg(h.device);
    check_batch(h, batch);
    if (!x || !out) throw std::runtime_error("x or out is NULL");
    tdt::DevRow rows[kMaxBatch];
    for (int b = 0; b < batch; ++b) rows[b] = greedy_devrow(h);
    simple_prep(h, rows, batch, x, 0, false, out, tdt::HeadPath::Digits);
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_logits(void* handle, const void* x, int x_dtype, int batch,
                                     int apply_softcap, float* logits) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    Head& h = bx->h;
    tdt::DeviceGuard dg(h.device);
    check_batch(h, batch);
    if (!x || !logits) throw std::runtime_error("x or logits is NULL");
    if (x_dtype != TURBO_HIDDEN_F32 && x_dtype != TURBO_HIDDEN_BF16)
        throw std::runtime_error("x_dtype must be TURBO_HIDDEN_F32 or TURBO_HIDDEN_BF16");
    tdt::DevRow rows[kMaxBatch];
    for (int b = 0; b < batch; ++b) rows[b] = greedy_devrow(h);
    tdt::EpiArgs ep = epi_args(h, logits, apply_softcap != 0);
    ep.partials = nullptr;  // no select follows
    launch_greedy_head(*bx, rows, batch, x, x_dtype, ep);
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_greedy(void* handle, const void* x, int x_dtype, int batch,
                                     uint32_t* tokens) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    Head& h = bx->h;
    tdt::DeviceGuard dg(h.device);
    check_batch(h, batch);
    if (!x || !tokens) throw std::runtime_error("x or tokens is NULL");
    if (x_dtype != TURBO_HIDDEN_F32 && x_dtype != TURBO_HIDDEN_BF16)
        throw std::runtime_error("x_dtype must be TURBO_HIDDEN_F32 or TURBO_HIDDEN_BF16");
    tdt::DevRow rows[kMaxBatch];
    for (int b = 0; b < batch; ++b) rows[b] = greedy_devrow(h);
    launch_greedy_head(*bx, rows, batch, x, x_dtype, epi_args(h, nullptr, true));
    tdt::SelectArgs sa{};
    sa.V = h.V;
    sa.ntile = h.ntile;
    sa.partials = h.partials;
    sa.rows = h.rows;
    sa.tokens = tokens;
    tdt::launch_select(h, batch, sa, tdt::FvList{}, h.stream);
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_softcap(void* stream, float* z, size_t n, float cap) {
    clear_error();
    API_TRY
    if (!z && n) throw std::runtime_error("z is NULL");
    tdt::launch_softcap(z, n, cap, static_cast<hipStream_t>(stream));
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_apply_repetition_penalty(void* stream, float* logits, uint32_t vocab,
                                                const uint32_t* history, uint32_t n,
                                                float penalty, float softcap) {
    clear_error();
    API_TRY
    if (!logits || (n && !history)) throw std::runtime_error("logits or history is NULL");
    tdt::launch_repetition(logits, vocab, history, n, penalty, softcap,
                           static_cast<hipStream_t>(stream));
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_enable_head_timing(void* handle, int enable) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    Head& h = bx->h;
    if (enable < 0) throw std::runtime_error("enable must be >= 0");
    tdt::DeviceGuard dg(h.device);
    if (enable && !h.t_start[0]) {
        for (int i = 0; i < Head::kTimerSlots; ++i) {
            check_hip(hipEventCreate(&h.t_start[i]), "timer events");
            check_hip(hipEventCreate(&h.t_stop[i]), "timer events");
        }
    }
    h.timing = enable != 0;
    h.t_stride = enable > 1 ? static_cast<uint32_t>(enable) : 1u;
    h.t_launch = 0;
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_lmhead_head_kernel_time(void* handle, double* total_ms, int* launches,
                                               int reset) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    Head& h = bx->h;
    tdt::DeviceGuard dg(h.device);
    check_hip(hipStreamSynchronize(h.stream), "timer sync");
    double ms = bx->t_accum_ms;
    int n = bx->t_accum_n;
    for (int i = 0; i < h.t_count; ++i) {
        float e = 0.f;
        check_hip(hipEventElapsedTime(&e, h.t_start[i], h.t_stop[i]), "timer read");
        ms += e;
    }
    n += h.t_count;
    if (total_ms) *total_ms = ms;
    if (launches) *launches = n;
    if (reset) {
        bx->t_accum_ms = 0.0;
        bx->t_accum_n = 0;
        h.t_count = 0;
    }
    return 1;
    API_CATCH(0)
}


TURBO_DT_API int turbo_int4_matvec(void* handle, const void* x, int x_dtype, int batch, float* out) {
    return turbo_lmhead_logits(handle, x, x_dtype, batch, 0, out);
}

TURBO_DT_API int turbo_lmhead_embed(void* handle, const uint32_t* tokens, int n, float* out) {
    clear_error();
    API_TRY
    HandleBox* bx = box(handle);
    Head& h = bx->h;
    tdt::DeviceGuard dg(h.device);
    if (n < 0) throw std::runtime_error("n must be >= 0");
    if (n > 0 && (!tokens || !out)) throw std::runtime_error("tokens or out is NULL");
    if (n > 65535 * 16) throw std::runtime_error("at most 1048560 tokens per call");
    // src/cpu_reference.cpp:328: the scale is sqrt of the hidden size in float
    tdt::launch_embed(h, tokens, n, out, std::sqrt(static_cast<float>(h.D)), h.stream);
    return 1;
    API_CATCH(0)
}

TURBO_DT_API int turbo_bundle_decode_header(const uint8_t* bytes, size_t count, uint64_t out[3]) {
    clear_error();
    API_TRY
    if (!bytes || !out) throw std::runtime_error("bytes or out is NULL");
    const tdt::ResidentHeader h = tdt::decode_resident_header(bytes, count);
    out[0] = h.index_size;
    out[1] = h.resident_size;
    out[2] = h.entry_count;
    return 1;
    API_CATCH(0)
}


TURBO_DT_API int turbo_bundle_find_tensor(const char* resident_path, const char* name, TurboBundleTensor* out) {
    clear_error();
    API_TRY
    if (!resident_path || !name || !out) throw std::runtime_error("path, name or out is NULL");
    *out = describe_tensor(tdt::find_resident_tensor(resident_path, name, nullptr));
    return 1;
    API_CATCH(0)
}

TURBO_DT_API void* turbo_lmhead_create_from_bundle(const char* resident_path, float final_logit_softcap,
                                                   float rms_norm_eps, int device) {
    clear_error();
    API_TRY
    if (!resident_path) throw std::runtime_error("resident_path is NULL");
    const std::string path(resident_path);
    const tdt::ResidentEntry ee = tdt::find_resident_tensor(path, "model.embed_tokens.weight", nullptr);
    const tdt::ResidentEntry ne = tdt::find_resident_tensor(path, "model.norm.weight", nullptr);
    const TurboBundleTensor et = describe_tensor(ee);
    if (!et.quantized || et.bits != 4u)
        throw std::runtime_error("model.embed_tokens.weight: expected a 4-bit quantised tensor");
    const uint64_t V = et.rows, D = et.in_dim, G = D / 64u;
    if (V == 0 || D == 0) throw std::runtime_error("model.embed_tokens.weight: empty shape");
    if (ee.size_bytes < V * (D / 2u) || ee.scale_size != V * G * 2u || ee.bias_size != V * G * 2u)
        throw std::runtime_error("model.embed_tokens.weight: region sizes do not match its shape");
    if (ne.dtype != 1u || ne.size_bytes < D * 2u)
        throw std::runtime_error("model.norm.weight: expected " + std::to_string(D) + " BF16 values");
    std::vector<uint8_t> W(static_cast<size_t>(V * (D / 2u)));
    std::vector<uint16_t> S(static_cast<size_t>(V * G)), B(static_cast<size_t>(V * G)), g(static_cast<size_t>(D));
    tdt::read_file_region(path, ee.file_offset, W.size(), W.data());
    tdt::read_file_region(path, ee.scale_offset, S.size() * 2u, S.data());
    tdt::read_file_region(path, ee.bias_offset, B.size() * 2u, B.data());
    tdt::read_file_region(path, ne.file_offset, g.size() * 2u, g.data());
    TurboLMHeadDesc d;
    turbo_lmhead_desc_default(&d);
    d.vocab_size = static_cast<uint32_t>(V);
    d.hidden_size = static_cast<uint32_t>(D);
    d.final_logit_softcap = final_logit_softcap;
    d.rms_norm_eps = rms_norm_eps;
    d.weights_on_device = 0;
    d.weight = W.data();
    d.scales = S.data();
    d.biases = B.data();
    d.norm_weight = g.data();
    d.device = device;
    void* h = turbo_lmhead_create(&d);
    if (!h) throw std::runtime_error(g_last_error);
    return h;
    API_CATCH(nullptr)
}
}  // extern "C"
