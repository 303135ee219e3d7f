/*
 * Oracle restatement of the reference decode tail. TEST INFRASTRUCTURE ONLY: the product
 * library never links this. Compiled with -O2 -ffp-contract=off and no fast-math so float
 * expressions round exactly as written (the reference's loops are plain scalar FP32).
 * See orc.h for the per-function reference citations and pinning status.
 */
#define _GNU_SOURCE
#include "orc.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---- numeric primitives ---------------------------------------------------------------- */

float orc_bf16_to_f32(uint16_t bits) {
    uint32_t w = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &w, sizeof f);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t w;
    memcpy(&w, &f, sizeof w);
    uint32_t rounding = 0x7FFFu + ((w >> 16) & 1u);
    return (uint16_t)((w + rounding) >> 16);
}

void orc_rms_norm(const float* x, const uint16_t* w, size_t n, float eps, float* out) {
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) acc += (double)x[i] * x[i];
    const float inv = 1.0f / sqrtf((float)(acc / (double)n) + eps);
    if (w) {
        for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv * orc_bf16_to_f32(w[i]);
    } else {
        for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv;
    }
}

#define ORC_GROUP 64u

void orc_matvec_int4(const uint8_t* W, const uint16_t* S, const uint16_t* B, uint32_t in_dim,
                     const float* x, float* out, uint32_t row_begin, uint32_t row_end) {
    const uint32_t groups = in_dim / ORC_GROUP;
    const size_t row_bytes = in_dim / 2;
    for (uint32_t r = row_begin; r < row_end; ++r) {
        const uint8_t* wrow = W + (size_t)r * row_bytes;
        const uint16_t* srow = S + (size_t)r * groups;
        const uint16_t* brow = B + (size_t)r * groups;
        float acc = 0.0f;
        for (uint32_t g = 0; g < groups; ++g) {
            const float s = orc_bf16_to_f32(srow[g]);
            const float b = orc_bf16_to_f32(brow[g]);
            const uint32_t base = g * ORC_GROUP;
            float dot = 0.0f, sum = 0.0f;
            for (uint32_t j = 0; j < ORC_GROUP; j += 2) {
                const uint8_t byte = wrow[(base + j) / 2];
                const float x0 = x[base + j];
                const float x1 = x[base + j + 1];
                dot += (float)(byte & 0x0F) * x0;
                dot += (float)(byte >> 4) * x1;
                sum += x0 + x1;
            }
            acc += s * dot + b * sum;
        }
        out[r] = acc;
    }
}

void orc_embed_row(const uint8_t* W, const uint16_t* S, const uint16_t* B, uint32_t in_dim,
                   uint32_t row, float* out) {
    const uint32_t groups = in_dim / ORC_GROUP;
    const uint8_t* wrow = W + (size_t)row * (in_dim / 2);
    const uint16_t* srow = S + (size_t)row * groups;
    const uint16_t* brow = B + (size_t)row * groups;
    for (uint32_t g = 0; g < groups; ++g) {
        const float s = orc_bf16_to_f32(srow[g]);
        const float b = orc_bf16_to_f32(brow[g]);
        for (uint32_t j = 0; j < ORC_GROUP; ++j) {
            const uint32_t c = g * ORC_GROUP + j;
            const uint8_t byte = wrow[c / 2];
            const uint32_t q = (c % 2 == 0) ? (byte & 0x0Fu) : (byte >> 4u);
            out[c] = (float)q * s + b;
        }
    }
    const float scale = sqrtf((float)in_dim);
    for (uint32_t i = 0; i < in_dim; ++i) out[i] *= scale;
}

typedef struct {
    const uint8_t* W;
    const uint16_t* S;
    const uint16_t* B;
    uint32_t in_dim;
    const float* x;
    float* out;
    uint32_t begin, end;
} mv_job;

static void* mv_worker(void* arg) {
    mv_job* j = (mv_job*)arg;
    orc_matvec_int4(j->W, j->S, j->B, j->in_dim, j->x, j->out, j->begin, j->end);
    return NULL;
}

void orc_matvec_int4_mt(const uint8_t* W, const uint16_t* S, const uint16_t* B, uint32_t rows,
                        uint32_t in_dim, const float* x, float* out, int threads) {
    if (threads <= 1 || rows < 2) {
        orc_matvec_int4(W, S, B, in_dim, x, out, 0, rows);
        return;
    }
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    mv_job jobs[256];
    const uint32_t per = (rows + (uint32_t)threads - 1) / (uint32_t)threads;
    int launched = 0;
    for (int t = 0; t < threads; ++t) {
        uint32_t b = (uint32_t)t * per;
        if (b >= rows) break;
        uint32_t e = b + per < rows ? b + per : rows;
        jobs[t] = (mv_job){W, S, B, in_dim, x, out, b, e};
        if (pthread_create(&tid[t], NULL, mv_worker, &jobs[t]) != 0) {
            mv_worker(&jobs[t]);
            tid[t] = 0;
        }
        launched = t + 1;
    }
    for (int t = 0; t < launched; ++t)
        if (tid[t]) pthread_join(tid[t], NULL);
}

void orc_softcap(float* z, size_t n, float cap) {
    if (!(cap > 0.0f)) return;
    for (size_t i = 0; i < n; ++i) z[i] = cap * tanhf(z[i] / cap);
}

/* ---- sampling ---------------------------------------------------------------------------- */

static void set_err(char* err, size_t errlen, const char* msg) {
    if (err && errlen) snprintf(err, errlen, "%s", msg);
}

int orc_validate_sampling(const orc_params* p, char* err, size_t errlen) {
    if (!isfinite(p->temperature) || p->temperature < 0.0f) {
        set_err(err, errlen, "temperature must be finite and >= 0 (0 = greedy)");
        return 0;
    }
    if (!isfinite(p->top_p) || p->top_p <= 0.0f || p->top_p > 1.0f) {
        set_err(err, errlen, "top_p must be in (0, 1]");
        return 0;
    }
    if (p->top_k < 0 || p->top_k > ORC_MAX_TOP_K) {
        set_err(err, errlen, "top_k must be in 0..256 (0 disables it)");
        return 0;
    }
    if (!isfinite(p->repetition_penalty) || p->repetition_penalty <= 0.0f) {
        set_err(err, errlen, "repetition_penalty must be finite and > 0 (1 = disabled)");
        return 0;
    }
    if (!isfinite(p->presence_penalty) || !isfinite(p->frequency_penalty)) {
        set_err(err, errlen, "presence_penalty and frequency_penalty must be finite");
        return 0;
    }
    if (!(p->flags & ORC_FLAG_FULL_VOCAB) && p->temperature > 0.0f && p->top_p < 1.0f &&
        p->top_k == 0) {
        set_err(err, errlen,
                "top_p < 1 with temperature > 0 requires top_k in 1..256; full-vocabulary "
                "nucleus sampling is not implemented");
        return 0;
    }
    set_err(err, errlen, "");
    return 1;
}

uint64_t orc_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

uint64_t orc_seed_for(int has_seed, uint64_t seed, int position) {
    uint64_t base = has_seed ? seed + (uint64_t)(int64_t)position
                             : (0x9E3779B97F4A7C15ULL ^
                                ((uint64_t)(int64_t)position * 0xD1B54A32D192ED03ULL));
    uint64_t s = orc_splitmix64(base);
    return s ? s : 0x9E3779B97F4A7C15ULL;
}

float orc_next_uniform(uint64_t* state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    const uint64_t r = s * 0x2545F4914F6CDD1DULL;
    return (float)((r >> 40) & 0xFFFFFFu) / 16777216.0f;
}

void orc_apply_repetition_penalty(float* logits, uint32_t vocab, const uint32_t* history,
                                  size_t n, float penalty, float softcap) {
    if (penalty == 1.0f || n == 0) return;
    const float limit = (softcap > 0.0f) ? softcap * 0.9999f : 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const uint32_t id = history[i];
        if (id >= vocab) continue;
        float v = logits[id];
        v = (v > 0.0f) ? (v / penalty) : (v * penalty);
        if (limit > 0.0f) {
            /* std::clamp(v, -limit, limit) */
            if (v < -limit) v = -limit;
            else if (limit < v) v = limit;
        }
        logits[id] = v;
    }
}

/* Strict total order of src/sampling.cpp:126-129: larger logit first, then lower index. */
static inline int before(const float* l, uint32_t a, uint32_t b) {
    if (l[a] != l[b]) return l[a] > l[b];
    return a < b;
}

static int cmp_idx(const void* pa, const void* pb, void* ctx) {
    const float* l = (const float*)ctx;
    const uint32_t a = *(const uint32_t*)pa, b = *(const uint32_t*)pb;
    if (a == b) return 0;
    return before(l, a, b) ? -1 : 1;
}

/* Reorders idx[0..n) so that idx[0..k) holds the k first elements under `before` (any order).
 * The order is total, so the selected set is the one std::nth_element selects. */
static void select_first_k(uint32_t* idx, size_t n, size_t k, const float* l) {
    if (k >= n) return;
    size_t lo = 0, hi = n;
    while (hi - lo > 16) {
        const size_t mid = lo + (hi - lo) / 2;
        /* median of three moved to mid */
        uint32_t a = idx[lo], b = idx[mid], c = idx[hi - 1];
        if (before(l, b, a)) { uint32_t t = a; a = b; b = t; }
        if (before(l, c, b)) { uint32_t t = b; b = c; c = t; }
        if (before(l, b, a)) { uint32_t t = a; a = b; b = t; }
        idx[lo] = a; idx[mid] = b; idx[hi - 1] = c;
        const uint32_t piv = b;
        size_t i = lo - 1, j = hi;
        for (;;) {
            do { ++i; } while (before(l, idx[i], piv));
            do { --j; } while (before(l, piv, idx[j]));
            if (i >= j) break;
            uint32_t t = idx[i]; idx[i] = idx[j]; idx[j] = t;
        }
        if (k <= j + 1) hi = j + 1;
        else lo = j + 1;
    }
    for (size_t i = lo + 1; i < hi; ++i) {
        uint32_t v = idx[i];
        size_t j = i;
        while (j > lo && before(l, v, idx[j - 1])) { idx[j] = idx[j - 1]; --j; }
        idx[j] = v;
    }
}

uint32_t orc_sample_token_u(const float* logits, uint32_t vocab, const orc_params* p, float u,
                            orc_sample_info* info) {
    orc_sample_info tmp;
    if (!info) info = &tmp;
    memset(info, 0, sizeof *info);
    info->u = u;
    if (vocab == 0) return UINT32_MAX;

    /* max and second under the total order, for diagnostics */
    {
        uint32_t best = 0, second = UINT32_MAX;
        for (uint32_t i = 1; i < vocab; ++i) {
            if (logits[i] > logits[best]) { second = best; best = i; }
            else if (second == UINT32_MAX || before(logits, i, second)) second = i;
        }
        info->max_logit = logits[best];
        info->second_logit = (second == UINT32_MAX) ? -INFINITY : logits[second];
    }

    if (p->temperature <= 0.0f) {
        uint32_t best = 0;
        float best_v = logits[0];
        for (uint32_t i = 1; i < vocab; ++i) {
            if (logits[i] > best_v) { best_v = logits[i]; best = i; }
        }
        info->token = best;
        info->shortlist = 1;
        info->cut = 1;
        return best;
    }

    float max_logit = logits[0];
    for (uint32_t i = 1; i < vocab; ++i) max_logit = (max_logit < logits[i]) ? logits[i] : max_logit;

    double total = 0.0;
    for (uint32_t i = 0; i < vocab; ++i) total += exp((double)logits[i] - max_logit);
    info->total = total;
    if (!(total > 0.0)) return UINT32_MAX;

    size_t want;
    if (p->top_k > 0) want = (size_t)p->top_k < vocab ? (size_t)p->top_k : vocab;
    else if (p->flags & ORC_FLAG_FULL_VOCAB) want = vocab;
    else want = ORC_MAX_TOP_K < vocab ? ORC_MAX_TOP_K : vocab;

    uint32_t* idx = (uint32_t*)malloc((size_t)vocab * sizeof(uint32_t));
    if (!idx) return UINT32_MAX;
    for (uint32_t i = 0; i < vocab; ++i) idx[i] = i;
    select_first_k(idx, vocab, want, logits);
    qsort_r(idx, want, sizeof(uint32_t), cmp_idx, (void*)logits);
    info->shortlist = (uint32_t)want;

    size_t cut = want;
    if (p->top_p < 1.0f) {
        double run = 0.0, prev = 0.0;
        for (size_t i = 0; i < want; ++i) {
            prev = run;
            run += exp((double)logits[idx[i]] - max_logit) / total;
            if (run >= (double)p->top_p) { cut = i + 1; break; }
        }
        info->nucleus_run = run;
        info->nucleus_prev = prev;
    }
    if (p->top_k > 0 && cut > (size_t)p->top_k) cut = (size_t)p->top_k;
    if (cut < 1) cut = 1;
    info->cut = (uint32_t)cut;

    double* q = (double*)malloc(cut * sizeof(double));
    if (!q) { free(idx); return UINT32_MAX; }
    double denom = 0.0;
    for (size_t i = 0; i < cut; ++i) {
        q[i] = exp(((double)logits[idx[i]] - max_logit) / p->temperature);
        denom += q[i];
    }
    info->denom = denom;
    const double r = (double)u * denom;
    info->r = r;
    double acc = 0.0;
    uint32_t tok = idx[cut - 1];
    size_t rank = cut - 1;
    info->acc_prev = 0.0;
    for (size_t i = 0; i < cut; ++i) {
        const double before_acc = acc;
        acc += q[i];
        if (acc >= r) { tok = idx[i]; rank = i; info->acc_prev = before_acc; break; }
        info->acc_prev = before_acc;
    }
    info->acc_at = acc;
    info->token = tok;
    info->rank = (uint32_t)rank;
    free(q);
    free(idx);
    return tok;
}

uint32_t orc_sample_token(const float* logits, uint32_t vocab, const orc_params* p,
                          uint64_t seed, orc_sample_info* info) {
    uint64_t state = seed;
    /* Greedy never consumes the uniform (src/sampling.cpp:97-104), which is harmless here. */
    const float u = orc_next_uniform(&state);
    return orc_sample_token_u(logits, vocab, p, u, info);
}

/* ---- EXTENSIONS -------------------------------------------------------------------------- */

static inline void mulhilo32(uint32_t a, uint32_t b, uint32_t* hi, uint32_t* lo) {
    const uint64_t prod = (uint64_t)a * (uint64_t)b;
    *hi = (uint32_t)(prod >> 32);
    *lo = (uint32_t)prod;
}

void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int round = 0; round < 10; ++round) {
        uint32_t hi0, lo0, hi1, lo1;
        mulhilo32(0xD2511F53u, c0, &hi0, &lo0);
        mulhilo32(0xCD9E8D57u, c2, &hi1, &lo1);
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n1 = lo1;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        const uint32_t n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float orc_philox_uniform(uint64_t seed, uint64_t counter) {
    const uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    orc_philox4x32_10(ctr, key, out);
    return (float)(out[0] >> 8) / 16777216.0f;
}

typedef struct {
    uint32_t id;
    uint32_t pos;
} id_pos;

static int cmp_id_pos(const void* a, const void* b) {
    const id_pos* x = (const id_pos*)a;
    const id_pos* y = (const id_pos*)b;
    if (x->id != y->id) return x->id < y->id ? -1 : 1;
    if (x->pos != y->pos) return x->pos < y->pos ? -1 : 1;
    return 0;
}

void orc_apply_logit_bias(float* logits, uint32_t vocab, const uint32_t* ids, const float* values,
                          size_t n) {
    if (!n) return;
    id_pos* e = (id_pos*)malloc(n * sizeof(id_pos));
    if (!e) return;
    for (size_t i = 0; i < n; ++i) e[i] = (id_pos){ids[i], (uint32_t)i};
    qsort(e, n, sizeof(id_pos), cmp_id_pos);
    size_t i = 0;
    while (i < n) {
        size_t j = i;
        float total = 0.0f;
        while (j < n && e[j].id == e[i].id) { total += values[e[j].pos]; ++j; }
        if (e[i].id < vocab) logits[e[i].id] += total;
        i = j;
    }
    free(e);
}

void orc_apply_presence_frequency(float* logits, uint32_t vocab, const uint32_t* history,
                                  size_t n, float presence, float frequency) {
    if (n == 0 || (presence == 0.0f && frequency == 0.0f)) return;
    id_pos* e = (id_pos*)malloc(n * sizeof(id_pos));
    if (!e) return;
    for (size_t i = 0; i < n; ++i) e[i] = (id_pos){history[i], (uint32_t)i};
    qsort(e, n, sizeof(id_pos), cmp_id_pos);
    size_t i = 0;
    while (i < n) {
        size_t j = i;
        while (j < n && e[j].id == e[i].id) ++j;
        const uint32_t id = e[i].id;
        if (id < vocab) {
            float v = logits[id];
            v = v - presence;
            v = v - frequency * (float)(j - i);
            logits[id] = v;
        }
        i = j;
    }
    free(e);
}

void orc_apply_ban(float* logits, uint32_t vocab, const uint32_t* words) {
    if (!words) return;
    for (uint32_t i = 0; i < vocab; ++i)
        if ((words[i >> 5] >> (i & 31u)) & 1u) logits[i] = -INFINITY;
}

void orc_apply_modifiers(float* logits, uint32_t vocab, const orc_params* p, float softcap,
                         const uint32_t* history, size_t history_len,
                         const uint32_t* bias_ids, const float* bias_values, size_t bias_count,
                         const uint32_t* ban_words) {
    if (bias_ids && bias_values && bias_count)
        orc_apply_logit_bias(logits, vocab, bias_ids, bias_values, bias_count);
    if (history && history_len) {
        orc_apply_repetition_penalty(logits, vocab, history, history_len, p->repetition_penalty,
                                     softcap);
        orc_apply_presence_frequency(logits, vocab, history, history_len, p->presence_penalty,
                                     p->frequency_penalty);
    }
    if (ban_words) orc_apply_ban(logits, vocab, ban_words);
}

/* ---- timed decode loop (CPU baseline of the benchmark) ---------------------------------- */

static double now_seconds(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

int orc_time_decode_steps(const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* gamma,
                          uint32_t vocab, uint32_t in_dim, float eps, float softcap, const float* hidden,
                          uint32_t nsteps, uint64_t first_counter, int threads, const orc_params* p,
                          uint64_t seed, uint32_t* history, size_t history_len, size_t history_cap,
                          uint32_t* tokens, double* seconds) {
    float* xn = (float*)malloc(sizeof(float) * in_dim);
    float* l = (float*)malloc(sizeof(float) * vocab);
    if (!xn || !l) {
        free(xn);
        free(l);
        return 0;
    }
    for (uint32_t s = 0; s < nsteps; ++s) {
        const double t0 = now_seconds();
        orc_rms_norm(hidden + (size_t)s * in_dim, gamma, in_dim, eps, xn);
        orc_matvec_int4_mt(W, S, B, vocab, in_dim, xn, l, threads);
        orc_softcap(l, vocab, softcap);
        orc_apply_modifiers(l, vocab, p, softcap, history, history_len, NULL, NULL, 0, NULL);
        const uint32_t tok = orc_sample_token_u(l, vocab, p, orc_philox_uniform(seed, first_counter + s), NULL);
        if (history_len < history_cap) history[history_len++] = tok;
        seconds[s] = now_seconds() - t0;
        tokens[s] = tok;
    }
    free(xn);
    free(l);
    return 1;
}
