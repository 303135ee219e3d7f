/*
 * turbo_decode_tail.h -- C ABI of the MI355X (gfx950) decode tail.
 *
 * Replaces the decode tail of ForwardRunner::produce_token (src/runner.cpp:719-807):
 *
 *   final RMSNorm -> affine-int4 tied LM head (group 64, BF16 scale + bias) over the whole
 *   vocabulary -> final-logit softcap -> logit modifiers -> greedy argmax or sampled draw
 *
 * Conventions follow include/gturbo/c_api.h:
 *   - plain C types and pointers only; every entry point catches all C++ exceptions;
 *   - handle-returning calls return NULL on failure, int-returning calls return 1 on success
 *     and 0 on failure; the reason is in turbo_lmhead_last_error() (thread-local, "" after a
 *     successful call, valid until the next failing call on the same thread; c_api.h:74-78);
 *   - option structs must be initialised by their *_default() function before use, because
 *     zero-initialisation is not valid (c_api.h:30-47).
 *
 * Memory: unless a comment says "host", every buffer pointer is a HIP device pointer. All
 * work is enqueued on the handle's stream (turbo_lmhead_set_stream; default: the null stream)
 * and is asynchronous to the host. One step in flight per handle; calls on one handle must be
 * serialised by the caller, as the reference serialises generation (README.md:202-206).
 */
#ifndef TURBO_DECODE_TAIL_H
#define TURBO_DECODE_TAIL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TURBO_DT_API __attribute__((visibility("default")))

/* ---- ABI version ------------------------------------------------------------------------- */

/*
 * No counterpart in the reference (its C API has one struct, checked by turbo_options_default).
 * TURBO_DT_ABI_VERSION changes whenever a struct layout or an entry point's meaning changes.
 * A caller compiled against this header checks, once at load time, that
 * turbo_abi_version() == TURBO_DT_ABI_VERSION and that turbo_abi_struct_size() agrees with its
 * sizeof for every struct it passes; a library of another layout would otherwise read or write
 * past the caller's arrays (TurboRowReport per row, for example) without any error.
 */
#define TURBO_DT_ABI_VERSION 1u
enum {
    TURBO_ABI_LMHEAD_DESC = 0,    /* TurboLMHeadDesc */
    TURBO_ABI_BUNDLE_TENSOR = 1,  /* TurboBundleTensor */
    TURBO_ABI_SAMPLING_ROW = 2,   /* TurboSamplingRow */
    TURBO_ABI_STEP_INPUTS = 3,    /* TurboStepInputs */
    TURBO_ABI_ROW_REPORT = 4,     /* TurboRowReport */
    TURBO_ABI_STEP_OUTPUTS = 5    /* TurboStepOutputs */
};
TURBO_DT_API uint32_t turbo_abi_version(void);
/* sizeof of the struct TURBO_ABI_* names, as the library was built; 0 for an unknown id. */
TURBO_DT_API size_t turbo_abi_struct_size(int which);

/* ---- errors ------------------------------------------------------------------------------ */

/* Replaces turbo_engine_last_error (include/gturbo/c_api.h:74-78; src/c_api.cpp:29-40). */
TURBO_DT_API const char* turbo_lmhead_last_error(void);

/* ---- head creation ----------------------------------------------------------------------- */

/*
 * Describes the tied LM head and final norm. Field meanings follow the manifest constants
 * (include/gturbo/manifest.hpp:23-50) and the resident-table layout the reference uploads at
 * ForwardRunner::initialize (src/runner.cpp:260-292, :324-357):
 *   weight       [vocab][hidden/2] bytes, element c in byte c/2, low nibble when c is even
 *                (docs/GTURBO_FORMAT.md:40; shaders/Common.hlsli:27-29)
 *   scales       [vocab][hidden/64] BF16, row-major
 *   biases       [vocab][hidden/64] BF16, row-major; dequantised w = q * scale + bias
 *   norm_weight  [hidden] BF16 model.norm.weight, applied as plain w (not 1 + w,
 *                src/cpu_reference.cpp:40-42); NULL means no weight
 */
typedef struct {
    uint32_t vocab_size;        /* 262144 for Gemma 4 (manifest.hpp:32) */
    uint32_t hidden_size;       /* 2816 (manifest.hpp:24); must be a multiple of 64 */
    uint32_t group_size;        /* must be 64 (src/cpu_reference.cpp:32) */
    float final_logit_softcap;  /* 30 (manifest.hpp:34); <= 0 disables the softcap */
    float rms_norm_eps;         /* 1e-6 (manifest.hpp:39) */
    int weights_on_device;      /* 0: the four pointers are host memory; 1: device memory */
    const uint8_t* weight;
    const uint16_t* scales;
    const uint16_t* biases;
    const uint16_t* norm_weight;
    int device;                 /* HIP device ordinal */
} TurboLMHeadDesc;

/*
 * ---- .gturbo bundle: resident.bin ---------------------------------------------------------
 * One tensor of the resident index (include/gturbo/resident_index.hpp:17-27), with the
 * quantisation geometry the reference derives from it (src/cpu_reference.cpp:229-247).
 */
typedef struct {
    uint32_t dtype;             /* 0 U32 (packed quantised words), 1 BF16, 2 FP16, 3 FP32 */
    uint32_t shape[4];
    uint64_t file_offset, size_bytes;
    uint64_t scale_offset, scale_size;  /* scale_size 0: not quantised */
    uint64_t bias_offset, bias_size;
    uint32_t quantized;
    uint32_t rows;              /* shape[0]; 1 for an empty shape */
    uint32_t in_dim;            /* quantised: scale_size / 2 / rows * 64; otherwise rows */
    uint32_t bits;              /* quantised: 4 when shape[1] * 8 == in_dim, else 8; otherwise 16 */
} TurboBundleTensor;

/* Decodes the 24-byte resident header (ResidentIndexCodec::decode_header,
 * src/resident_index.cpp:42-52): out = {index_size, resident_size, entry_count}. 1/0. */
TURBO_DT_API int turbo_bundle_decode_header(const uint8_t* bytes, size_t count, uint64_t out[3]);
/* Reads and validates the index region of the resident.bin at path
 * (ResidentIndexCodec::decode_region, src/resident_index.cpp:54-104) and describes tensor
 * `name` (ForwardRunner::resident_ref, src/runner.cpp:324-347). 1/0. */
TURBO_DT_API int turbo_bundle_find_tensor(const char* resident_path, const char* name,
                                          TurboBundleTensor* out);
/*
 * Creates the head from a bundle's resident.bin: model.embed_tokens.weight (the tied table,
 * 4-bit, one index entry with its scale and bias regions) and model.norm.weight (BF16), read
 * from their 16 KB-aligned regions (docs/GTURBO_FORMAT.md:26-58). The softcap and eps are the
 * manifest's arch.final_logit_softcap and arch.rms_norm_eps (include/gturbo/manifest.hpp:34,
 * :39), passed by the caller that parsed manifest.json. Replaces the runner's resident lookups
 * for this path (src/runner.cpp:324-357, :722-723, :773). NULL on failure.
 */
TURBO_DT_API void* turbo_lmhead_create_from_bundle(const char* resident_path, float final_logit_softcap,
                                                   float rms_norm_eps, int device);

/* Fills the Gemma 4 26B-A4B constants; the four pointers are NULL. */
TURBO_DT_API void turbo_lmhead_desc_default(TurboLMHeadDesc* out);

/*
 * Copies the table into HBM in the kernels' tiled layout (the caller's buffers may be freed
 * afterwards) and allocates per-step scratch. Replaces the resident upload and buffer set-up
 * of ForwardRunner::initialize for this path (src/runner.cpp:211-215, :260-292).
 * Returns NULL on failure. Batches above two rows compute on the matrix cores in fp16: a table
 * with a scale or bias of magnitude above 65504 is accepted, but such calls on it then fail with
 * an error (one- and two-row calls are unaffected). Hidden states have no such limit.
 */
TURBO_DT_API void* turbo_lmhead_create(const TurboLMHeadDesc* desc);
/* Waits for the handle's stream (the one set by turbo_lmhead_set_stream, which must still exist;
 * other streams are not waited for) and frees everything (src/runner.cpp:25-42). NULL is a
 * no-op. */
TURBO_DT_API void turbo_lmhead_destroy(void* handle);
/* hip_stream is a hipStream_t (NULL = the null stream). Must be created at default priority.
 * Switching to another stream first waits for the current one, whose steps may still be using
 * the handle's scratch buffers. */
TURBO_DT_API int turbo_lmhead_set_stream(void* handle, void* hip_stream);
/* Waits for the handle's stream. Returns 0 (once) when a step since the last call found a full
 * history under TURBO_STEP_APPEND_HISTORY (TURBO_STATUS_HISTORY_FULL). */
TURBO_DT_API int turbo_lmhead_synchronize(void* handle);
/* Largest batch one step accepts, and the largest bias_stride (logit-bias entries per row).
 * History length is not limited. */
TURBO_DT_API int turbo_lmhead_limits(void* handle, int* max_batch, int* max_row_modifiers);

/* ---- sampling parameters ----------------------------------------------------------------- */

enum {
    TURBO_RNG_PHILOX = 0,    /* u = Philox4x32-10(key = seed, counter = counter), 24-bit */
    TURBO_RNG_REFERENCE = 1  /* u = next_uniform(seed_for(has_seed, seed, position = counter)),
                                the reference's map (src/sampling.cpp:18-28, :63-72) */
};

enum {
    /* Lifts the reference's 256-candidate shortlist and accepts top_k == 0 with top_p < 1:
     * nucleus over the full vocabulary, as the full-sort sampler of
     * tests/test_sampling.cpp:36-84. Without it the semantics are exactly sample_token's. */
    TURBO_ROW_FULL_VOCAB = 1u
};

/*
 * Per-row sampling parameters. The first four fields are SamplingParams
 * (include/gturbo/sampling.hpp:21-30); the rest are extensions.
 */
typedef struct {
    float temperature;          /* 0 = greedy */
    float top_p;                /* (0, 1]; 1 = no nucleus */
    int top_k;                  /* 0..256; 0 = off */
    float repetition_penalty;   /* > 0; 1 = off; applied per history occurrence */
    float presence_penalty;     /* extension: l -= presence for ids seen at least once */
    float frequency_penalty;    /* extension: l -= frequency * count */
    int rng;                    /* TURBO_RNG_* */
    int has_seed;               /* TURBO_RNG_REFERENCE only */
    uint64_t seed;
    uint64_t counter;           /* Philox counter (decode step), or the reference's int position
                                   (two's complement; must fit in int for TURBO_RNG_REFERENCE) */
    uint32_t flags;             /* TURBO_ROW_* */
} TurboSamplingRow;

/* Greedy, no penalties, Philox with seed 0 counter 0 (sampling.hpp:21-30 defaults). */
TURBO_DT_API void turbo_sampling_row_default(TurboSamplingRow* out);
/* validate_sampling (src/sampling.cpp:32-54). Returns 1 if valid; else 0 and the reason. */
TURBO_DT_API int turbo_validate_sampling(const TurboSamplingRow* row);
/* splitmix64 and seed_for (src/sampling.cpp:56-72). */
TURBO_DT_API uint64_t turbo_splitmix64(uint64_t x);
TURBO_DT_API uint64_t turbo_seed_for(int has_seed, uint64_t seed, int position);
/* The uniform a step draws for this row (host computation of the device's value). */
TURBO_DT_API float turbo_row_uniform(const TurboSamplingRow* row);

/* ---- the decode-tail step ---------------------------------------------------------------- */

enum { TURBO_HIDDEN_F32 = 0, TURBO_HIDDEN_BF16 = 1 };

enum {
    TURBO_STEP_NORMED = 1u,          /* hidden is already normalised: skip the final RMSNorm */
    TURBO_STEP_APPEND_HISTORY = 2u   /* append each row's token to its history on the device
                                        (src/runner.cpp:878), incrementing history_len. The
                                        reference's history grows without bound; here it holds
                                        history_stride ids per row, so the caller sizes the
                                        stride for the initial length plus every step it will
                                        run. A row whose history is full keeps its token but
                                        does not append it: its report has
                                        TURBO_STATUS_HISTORY_FULL and the next
                                        turbo_lmhead_synchronize returns 0 with the reason. */
};

/* Row-strided side inputs. Any group may be NULL / zero to disable it. */
typedef struct {
    int batch;                  /* 1 .. max_batch */
    const void* hidden;         /* [batch][hidden_size], TURBO_HIDDEN_* (buf_hidden_ at :722) */
    int hidden_dtype;
    uint32_t flags;             /* TURBO_STEP_* */
    const TurboSamplingRow* rows; /* HOST array [batch], copied by the call */
    /* history ids (src/runner.cpp:801-803): row b has history_len[b] ids at
     * history + b * history_stride; ids >= vocab are ignored (src/sampling.cpp:82). */
    uint32_t* history;
    uint32_t history_stride;
    uint32_t* history_len;
    /* banned-token bitmask (extension): bit (id % 32) of word ban_bits[b * ban_stride + id/32] */
    const uint32_t* ban_bits;
    uint32_t ban_stride;
    /* sparse logit bias (extension): bias_count[b] pairs at b * bias_stride */
    const uint32_t* bias_ids;
    const float* bias_values;
    uint32_t bias_stride;
    const uint32_t* bias_count;
    /* injected uniforms [batch] in [0, 1); NULL = derive from each row's rng */
    const float* uniforms;
} TurboStepInputs;

/* Diagnostics per row (optional). */
typedef struct {
    float max_logit;        /* row maximum after modifiers */
    float u;                /* uniform used */
    uint32_t shortlist;     /* candidate list size (want) */
    uint32_t cut;           /* survivors after top-p / top-k */
    uint32_t rank;          /* token's position among the survivors */
    uint32_t path;          /* 0 greedy, 1 shortlist, 2 full-vocabulary value bins,
                               3 degenerate, 4 radix fallback (massive ties) */
    double total;           /* sum exp(l - max) over the row */
    double denom;           /* survivor weight sum */
    double r;               /* u * denom */
    uint32_t status;        /* TURBO_STATUS_* bits */
    uint32_t reserved;
} TurboRowReport;

enum {
    /* TURBO_STEP_APPEND_HISTORY found history_len == history_stride: the token was returned but
     * not appended. turbo_lmhead_synchronize then fails (once) with the row in the message. */
    TURBO_STATUS_HISTORY_FULL = 1u
};

typedef struct {
    uint32_t* tokens;        /* [batch]; 0xFFFFFFFF marks a degenerate distribution */
    float* logits;           /* optional [batch][vocab]: final logits after all modifiers */
    TurboRowReport* report;  /* optional [batch] */
} TurboStepOutputs;

/*
 * One decode-tail step for a batch of independent rows: (RMSNorm) -> int4 head -> softcap ->
 * bias -> repetition -> presence/frequency -> ban -> greedy or sampled token per row.
 * Replaces src/runner.cpp:719-807 (RMSNormK, LMHeadGreedy + ArgmaxReduce or GemvInt4 x5 +
 * Softcap + readback + apply_repetition_penalty + sample_token). Every row is validated
 * first (turbo_validate_sampling); an invalid row fails the call before anything is enqueued.
 */
TURBO_DT_API int turbo_lmhead_step(void* handle, const TurboStepInputs* in,
                                   const TurboStepOutputs* out);

/*
 * Affine-int4 matrix-vector product, out[b][r] = sum_c (q[r][c] * scale + bias) * x[b][c], at
 * any shape a head accepts (rows up to 2^24, in_dim a multiple of 64 up to 8192): the
 * reference's GemvInt4 (shaders/GemvInt4.hlsl:1-38) as dispatched for the q/k/v/o projections,
 * the shared expert and the routed experts (src/runner.cpp:431-442, :621-646, :671-678). A
 * matrix is a handle created with vocab_size = rows, hidden_size = in_dim, final_logit_softcap
 * 0 and no norm weight. x: [batch][in_dim] (TURBO_HIDDEN_*), out: [batch][rows] FP32, device.
 */
TURBO_DT_API int turbo_int4_matvec(void* handle, const void* x, int x_dtype, int batch, float* out);

/*
 * ---- int4 matrices of the layer loop ------------------------------------------------------
 * A matrix handle holds one affine-int4 weight matrix (rows x in_dim, group 64, BF16 scale +
 * bias; the reference layout of turbo_lmhead_create) in the kernels' tiled layout and nothing
 * else, so its device footprint is the table's size (rows * in_dim / 2 + rows * in_dim / 16
 * bytes). These replace the GemvInt4 dispatches of the layer loop (shaders/GemvInt4.hlsl:1-38;
 * src/runner.cpp:431-442, :612-646, :671-678) for the expert slots and projections.
 */
/* rows 1..16777216, in_dim a multiple of 64 up to 8192. Allocates the table only; the contents
 * are undefined until turbo_int4_matrix_load. NULL on failure. */
TURBO_DT_API void* turbo_int4_matrix_create(uint32_t rows, uint32_t in_dim, int device);
/* Repacks one matrix into the handle (the expert streamer's slot refill, src/streamer.cpp:171-214).
 * weights_on_device = 1: the three pointers are device memory (for example the slot's buffer at
 * the tensor's offsets); the repack is one kernel pair enqueued on hip_stream, allocating nothing.
 * 0: host memory, staged through temporary device buffers and finished before the call returns. */
TURBO_DT_API int turbo_int4_matrix_load(void* matrix, const uint8_t* weight, const uint16_t* scales,
                                        const uint16_t* biases, int weights_on_device, void* hip_stream);
/* Waits for the streams the matrix's loads and products were enqueued on (the whole device when
 * more than four distinct streams were used) and frees it. Calls that use one matrix handle are
 * serialised by the caller. */
TURBO_DT_API void turbo_int4_matrix_destroy(void* matrix);
/* out[i][r] = sum_c (q[r][c] * scale + bias) * x[i][c] for each of `count` (0..32) matrices of one
 * device, in one kernel launch on hip_stream: for example the 8 routed experts' gate and up
 * matrices of a token (16 products of 704 x 2816), then their down matrices. x[i]: [in_dim] FP32,
 * 16-byte aligned; out[i]: [rows] FP32; all device memory. Each out[i] is bit-identical to
 * turbo_int4_matvec on a head of the same matrix. */
TURBO_DT_API int turbo_int4_matvec_grouped(void* const* matrices, int count, const float* const* x,
                                           float* const* out, void* hip_stream);

/*
 * Embedding lookup on the same tied table (shaders/EmbedLookup.hlsl:1-45; CPU
 * src/cpu_reference.cpp:108-124 and :323-329): out[i] = row tokens[i] dequantised as
 * (float)q * scale + bias, times sqrtf(hidden). tokens: [n] device ids, out: [n][hidden] FP32
 * device, stream-ordered on the handle's stream. The reference throws for an id past the
 * vocabulary (:325-327); here, where ids stay on the device, such a row is written as NaN.
 */
TURBO_DT_API int turbo_lmhead_embed(void* handle, const uint32_t* tokens, int n, float* out);

/* ---- kernel-level entry points (one per reference kernel on the path) -------------------- */

/* RMSNormK with model.norm.weight (shaders/RMSNormK.hlsl:25-61; src/cpu_reference.cpp:43-52).
 * x, out: [batch][hidden] FP32. */
TURBO_DT_API int turbo_lmhead_rms_norm(void* handle, const float* x, int batch, float* out);

/* GemvInt4 over the tied table (shaders/GemvInt4.hlsl:18-38, src/runner.cpp:429-442, :773),
 * followed by Softcap when apply_softcap (shaders/Softcap.hlsl:18-30, src/runner.cpp:774-779).
 * x: [batch][hidden] (TURBO_HIDDEN_*, already normalised), logits: [batch][vocab] FP32. */
TURBO_DT_API int turbo_lmhead_logits(void* handle, const void* x, int x_dtype, int batch,
                                     int apply_softcap, float* logits);

/* LMHeadGreedy + ArgmaxReduce (shaders/LMHeadGreedy.hlsl:28-73, ArgmaxReduce.hlsl:21-62):
 * argmax of the softcapped logits, ties to the lowest row. tokens: [batch]. */
TURBO_DT_API int turbo_lmhead_greedy(void* handle, const void* x, int x_dtype, int batch,
                                     uint32_t* tokens);

/* Softcap in place on n floats (shaders/Softcap.hlsl:18-30). stream may be NULL. */
TURBO_DT_API int turbo_softcap(void* hip_stream, float* z, size_t n, float cap);

/* apply_repetition_penalty in place on one row (src/sampling.cpp:74-90). stream may be NULL. */
TURBO_DT_API int turbo_apply_repetition_penalty(void* hip_stream, float* logits, uint32_t vocab,
                                                const uint32_t* history, uint32_t n,
                                                float penalty, float softcap);

/*
 * Sampling on caller-provided logits (sample_token, src/sampling.cpp:92-169, plus the
 * modifiers of turbo_lmhead_step). logits: [batch][vocab], modified in place by the
 * modifiers. in->hidden and in->hidden_dtype are ignored. out->logits is ignored.
 */
TURBO_DT_API int turbo_sample_logits(void* handle, float* logits, const TurboStepInputs* in,
                                     const TurboStepOutputs* out);

/* ---- sampling without a handle or an allocation ---------------------------------------- */

#define TURBO_NOALLOC_MAX_BATCH 4
#define TURBO_NOALLOC_MAX_VOCAB 262144

/*
 * turbo_sample_logits without a handle and without allocating: the modifiers of
 * TurboStepInputs and the sampler (sample_token semantics, src/sampling.cpp:92-169) over
 * caller logits [batch][vocab], modified in place, tokens (and reports) into `out`. No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It calls no hipMalloc,
 * hipFree or allocating routine; its working memory is one static device array of about 14 MiB
 * per GPU (held until the process ends), sized for batch <= TURBO_NOALLOC_MAX_BATCH and
 * vocab <= TURBO_NOALLOC_MAX_VOCAB, with at most 8192 logit-bias entries per row. Larger inputs
 * fail with a clear error. The work is enqueued on hip_stream (NULL = the null stream) of the
 * current device; the first call on a device clears the array on that stream. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU race, so the caller serialises them.
 * in->hidden and out->logits are ignored; TURBO_STATUS_HISTORY_FULL is reported per row only.
 */
TURBO_DT_API int turbo_sample_logits_noalloc(void* hip_stream, uint32_t vocab, float final_logit_softcap,
                                             float* logits, const TurboStepInputs* in,
                                             const TurboStepOutputs* out);

/* ---- measurement ------------------------------------------------------------------------- */

/* When enabled, the head kernel (the int4 GEMV / MFMA kernel) is launched with HIP start and
 * stop events on the handle's stream. enable = 1 times every launch; enable = N > 1 times every
 * N-th launch (the events add a few microseconds of gap around the timed launch, so sampling
 * keeps a loop's throughput representative). turbo_lmhead_head_kernel_time synchronises and
 * returns the summed milliseconds and the number of timed launches since the last reset. */
TURBO_DT_API int turbo_lmhead_enable_head_timing(void* handle, int enable);
TURBO_DT_API int turbo_lmhead_head_kernel_time(void* handle, double* total_ms, int* launches,
                                               int reset);

#ifdef __cplusplus
}
#endif

#endif /* TURBO_DECODE_TAIL_H */
