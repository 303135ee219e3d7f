/*
 * Oracle: a CPU restatement of Turbo-WinFare's decode tail, used ONLY as test infrastructure.
 *
 *   final RMSNorm -> affine-int4 tied LM head -> softcap -> penalties -> greedy / sampled draw
 *
 * This library is the checker for the HIP implementation. Only tests/, __graft_entry__.smoke()
 * and bench.py's CPU-baseline leg may load it. The product library never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference
 * checkout). Functions marked EXTENSION implement behaviour the reference does not have
 * (Philox uniforms, presence/frequency penalties, logit bias, banned tokens, full-vocabulary
 * nucleus, batching); their semantics are defined here and pinned by closed forms only.
 *
 * Pinning status (which independent checks hold each function; see tests/test_oracle.py):
 *   orc_bf16_to_f32 / orc_f32_to_bf16   bit patterns of known values, RNE tie cases
 *   orc_rms_norm                        closed forms (constant vector, scaled vector), long double
 *   orc_matvec_int4                     closed forms (q const, q=8 with b=-8s, one-hot x),
 *                                       long-double brute force, reference test formula
 *                                       (tests/test_gpu_kernels.cpp:155-172) within its tolerance
 *   orc_softcap                         closed form via libm tanhf, odd symmetry, saturation
 *   orc_validate_sampling               reference accept/reject matrix (tests/test_sampling.cpp:92-112)
 *                                       and the compiled reference (oracle/_ref) on a sweep
 *   orc_splitmix64 / orc_seed_for       reference KATs (tests/test_sampling.cpp:118-121) and _ref
 *   orc_next_uniform                    pinned through orc_sample_token == _ref sample_token
 *   orc_apply_repetition_penalty        reference test values (tests/test_sampling.cpp:199-228), _ref
 *   orc_sample_token                    reference tests (greedy tie, mlx order) and _ref on sweeps
 *                                       at V = 262144 including the reference's 5-config sweep
 *   orc_philox4x32_10                   Random123 known-answer vectors (Salmon et al., SC'11)
 *   EXTENSION penalties/bias/ban        closed forms; "parity unpinned" against the reference
 *   full-vocabulary nucleus             equals the reference's full-sort sampler
 *                                       (tests/test_sampling.cpp:36-84) restated; brute force
 */
#ifndef TURBO_ORACLE_ORC_H
#define TURBO_ORACLE_ORC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numeric primitives ---------------------------------------------------------------- */

/* src/cpu_reference.cpp:21-26 */
float orc_bf16_to_f32(uint16_t bits);
/* tests/test_gpu_kernels.cpp:36-42 (round to nearest even on the truncated mantissa) */
uint16_t orc_f32_to_bf16(float f);

/* src/cpu_reference.cpp:43-52: y = x * (1/sqrt(float(sum x^2 / n) + eps)) * bf16(w); sum in double.
 * w may be NULL (no weight). */
void orc_rms_norm(const float* x, const uint16_t* w, size_t n, float eps, float* out);

/* src/cpu_reference.cpp:55-84, 4-bit branch, exact loop order:
 *   per row, per group: dot += q_lo*x0; dot += q_hi*x1; sum += x0 + x1; acc += s*dot + b*sum.
 * Rows [row_begin, row_end) of out are written. W is [rows][in_dim/2], S and B are [rows][in_dim/64]. */
void orc_matvec_int4(const uint8_t* W, const uint16_t* S, const uint16_t* B, uint32_t in_dim,
                     const float* x, float* out, uint32_t row_begin, uint32_t row_end);

/* Same as orc_matvec_int4 over all rows, split row-parallel over `threads` POSIX threads.
 * Per-row arithmetic is unchanged, so the result is bit-identical to the 1-thread call. */
void orc_matvec_int4_mt(const uint8_t* W, const uint16_t* S, const uint16_t* B, uint32_t rows,
                        uint32_t in_dim, const float* x, float* out, int threads);

/* Embedding lookup: row `row` of the tied table dequantised as (float)q * s + b, element by
 * element in group order (src/cpu_reference.cpp:108-124, dequant_row), then every element
 * multiplied by sqrtf((float)in_dim) (src/cpu_reference.cpp:323-329). Pinned by: a constant
 * nibble k giving (k s + b) sqrt(D) per group, and the one-hot identity
 * orc_matvec_int4(W, e_c)[row] == the unscaled element c (tests/test_oracle.py). */
void orc_embed_row(const uint8_t* W, const uint16_t* S, const uint16_t* B, uint32_t in_dim,
                   uint32_t row, float* out);

/* src/cpu_reference.cpp:535-538: z = cap * tanhf(z / cap) when cap > 0. */
void orc_softcap(float* z, size_t n, float cap);

/* ---- sampling (src/sampling.cpp) -------------------------------------------------------- */

#define ORC_MAX_TOP_K 256            /* src/sampling.cpp:15 */
#define ORC_FLAG_FULL_VOCAB 1u       /* EXTENSION: full-vocabulary nucleus, no 256 shortlist cap */

typedef struct {
    float temperature;        /* include/gturbo/sampling.hpp:22 */
    float top_p;              /* :23 */
    int top_k;                /* :24 */
    float repetition_penalty; /* :25 */
    float presence_penalty;   /* EXTENSION */
    float frequency_penalty;  /* EXTENSION */
    uint32_t flags;           /* EXTENSION: ORC_FLAG_FULL_VOCAB */
} orc_params;

/* src/sampling.cpp:32-54. Returns 1 if valid, else 0 with a message in err. With
 * ORC_FLAG_FULL_VOCAB the rule "T>0 and top_p<1 requires top_k>0" is lifted (EXTENSION).
 * Presence/frequency must be finite (EXTENSION). */
int orc_validate_sampling(const orc_params* p, char* err, size_t errlen);

/* src/sampling.cpp:56-61 */
uint64_t orc_splitmix64(uint64_t x);
/* src/sampling.cpp:63-72 */
uint64_t orc_seed_for(int has_seed, uint64_t seed, int position);
/* src/sampling.cpp:18-28: xorshift64* then the top 24 bits of the product / 2^24. */
float orc_next_uniform(uint64_t* state);

/* src/sampling.cpp:74-90: every history occurrence divides (v>0) or multiplies (v<=0) by the
 * penalty, then clamps to +-0.9999*softcap when softcap > 0. Ids >= vocab are ignored. */
void orc_apply_repetition_penalty(float* logits, uint32_t vocab, const uint32_t* history,
                                  size_t n, float penalty, float softcap);

/* Diagnostics returned by the sampler, used by parity tests to find near-tie rows. */
typedef struct {
    uint32_t token;
    uint32_t shortlist;   /* size of the sorted candidate list (want) */
    uint32_t cut;         /* survivors after top-p and top-k */
    uint32_t rank;        /* position of token in the sorted candidate list */
    float max_logit;      /* row maximum */
    float second_logit;   /* second largest value under the (logit desc, index asc) order */
    double total;         /* sum exp(l - max) over the whole row, double */
    double nucleus_run;   /* run value at the cut (top_p < 1 only) */
    double nucleus_prev;  /* run value one before the cut */
    double denom;         /* sum of survivor weights exp((l - max)/T) */
    double r;             /* u * denom */
    double acc_prev;      /* cumulative survivor weight before the chosen token */
    double acc_at;        /* cumulative survivor weight including the chosen token */
    float u;
} orc_sample_info;

/* src/sampling.cpp:92-169 with the uniform injected (the reference draws it from
 * next_uniform(seed_for(...)) at :161-162). Greedy when temperature <= 0 (:97-104).
 * Shortlist size want = top_k>0 ? min(top_k,V) : min(256,V) (:122-124), or V when
 * ORC_FLAG_FULL_VOCAB is set and top_k == 0 (EXTENSION; then the selection equals the
 * full-sort sampler of tests/test_sampling.cpp:36-84). Returns the token; fills info if given.
 * Returns UINT32_MAX if vocab == 0 or the distribution is degenerate (the reference throws). */
uint32_t orc_sample_token_u(const float* logits, uint32_t vocab, const orc_params* p, float u,
                            orc_sample_info* info);

/* src/sampling.cpp:92-169 exactly: the uniform is next_uniform(state = seed). */
uint32_t orc_sample_token(const float* logits, uint32_t vocab, const orc_params* p,
                          uint64_t seed, orc_sample_info* info);

/* ---- EXTENSIONS (not in the reference; parity unpinned against it) ----------------------- */

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as 1, 2, 3",
 * SC'11). */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* One 24-bit uniform per (seed, counter): key = {seed lo, seed hi}, ctr = {counter lo,
 * counter hi, 0, 0}; u = (out[0] >> 8) / 2^24, the same 24-bit quantisation as
 * src/sampling.cpp:25-28. */
float orc_philox_uniform(uint64_t seed, uint64_t counter);

/* Logit bias: per id, the entries' values are summed in list order starting from 0.0f, then
 * added once to the logit. Ids >= vocab are ignored. */
void orc_apply_logit_bias(float* logits, uint32_t vocab, const uint32_t* ids, const float* values,
                          size_t n);
/* Presence / frequency (OpenAI convention): for each distinct id with count c > 0 in history,
 * l = l - presence; l = l - frequency * (float)c. No-op when both are 0. */
void orc_apply_presence_frequency(float* logits, uint32_t vocab, const uint32_t* history,
                                  size_t n, float presence, float frequency);
/* Banned tokens: bit (id % 32) of words[id / 32] set -> logit = -inf. */
void orc_apply_ban(float* logits, uint32_t vocab, const uint32_t* words);

/* The whole per-row modifier chain in the order the library applies it:
 *   bias -> repetition penalty (reference rule, after softcap) -> presence/frequency -> ban.
 * Any pointer may be NULL / count 0 to skip that stage. */
void orc_apply_modifiers(float* logits, uint32_t vocab, const orc_params* p, float softcap,
                         const uint32_t* history, size_t history_len,
                         const uint32_t* bias_ids, const float* bias_values, size_t bias_count,
                         const uint32_t* ban_words);


/* ---- timed decode loop (the benchmark's CPU baseline; not a restatement) ----------------- */

/* Runs nsteps decode-tail steps of one row exactly as the reference CPU path chains them
 * (src/cpu_reference.cpp:527-539 then :578-586): orc_rms_norm -> orc_matvec_int4_mt (`threads`
 * POSIX threads, row-parallel) -> orc_softcap -> orc_apply_modifiers (history only) ->
 * orc_sample_token_u with the Philox uniform (seed, first_counter + s), appending each token to
 * history while history_len < history_cap. hidden is [nsteps][in_dim]. seconds[s] is the
 * CLOCK_MONOTONIC duration of step s (hidden state in, token out). Returns 1, or 0 when a
 * buffer cannot be allocated. */
int orc_time_decode_steps(const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* gamma,
                          uint32_t vocab, uint32_t in_dim, float eps, float softcap, const float* hidden,
                          uint32_t nsteps, uint64_t first_counter, int threads, const orc_params* p,
                          uint64_t seed, uint32_t* history, size_t history_len, size_t history_cap,
                          uint32_t* tokens, double* seconds);

#ifdef __cplusplus
}
#endif

#endif
