// Internal interfaces between the C-ABI layer (api.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "dt_common.h"
#include "turbo_decode_tail.h"

namespace tdt {

// Logit-bias entries one row's bias table can hold (the sort runs in LDS). History length is
// not limited: occurrences are counted in a dense per-row array.
constexpr uint32_t kModCap = 8192;
// Static LDS of the step-prep kernel, in u64 words: kModCap sort keys plus kModCap + 1 run
// starts (u32).
constexpr uint32_t kPrepPoolU64 = kModCap + (kModCap + 2u) / 2u;

// Device-resident head plus per-step scratch. All sizes are fixed at create time.
struct Head {
    int device = 0;
    uint32_t V = 0;        // vocabulary rows
    uint32_t D = 0;        // hidden size
    uint32_t G = 0;        // groups per row (D / 64)
    uint32_t NC = 0;       // 16-byte chunks per row (D / 32)
    uint32_t ntile = 0;    // 64-row tiles (ceil(V / 64)); rows >= V are zero padding
    float cap = 0.f;       // final-logit softcap (0 = off)
    float eps = 0.f;
    hipStream_t stream = nullptr;

    // Tiled table: Wt[tile][chunk][64 rows] of 16 bytes, SBt[tile][group][64 rows] of
    // (scale bf16 | bias bf16 << 16).
    uint4* Wt = nullptr;
    uint32_t* SBt = nullptr;
    // Matrix-core form of the scales and biases: SB16t[tile][group][64 rows] u32 = fp16(s) * 2^20 |
    // fp16(b) << 16 when mfma_denorm (every |s| < 1/16: the dequant multiplies nibbles held as fp16
    // denormals), else fp16(s) | fp16(b) << 16 (the dequant through the mantissa of 1024.0).
    uint32_t* SB16t = nullptr;
    bool mfma_denorm = true;
    // false when some scale or bias lies outside the fp16 range even unscaled: the matrix-core
    // path cannot represent the table, and batches above two rows fail with an error
    bool mfma_ok = true;
    uint16_t* gamma = nullptr;   // [D] bf16 or null

    int max_batch = 0;
    uint32_t mod_cap = 0;        // max bias entries per row

    // Per-step scratch.
    float* xn = nullptr;         // [max_batch][D] normalised activations
    uint32_t* xdig = nullptr;    // [max_batch][NC][6][4] digit planes (small-batch GEMV)
    float* xws = nullptr;        // [max_batch][G] block-fp scale 2^(e-21)
    float* xsum = nullptr;       // [max_batch][G] sum of the block-fp activations
    uint16_t* x16 = nullptr;     // [max_batch][D] fp16, k-permuted within octets (MFMA path)
    float* xscale = nullptr;     // [max_batch] 2^k: x16 holds row b times 2^-k (MFMA path)
    float* logits = nullptr;     // [max_batch][V] scratch logits
    BlockPartial* partials = nullptr;  // [max_batch][ntile]
    DevRow* rows = nullptr;      // [max_batch]
    ModEntry* mods = nullptr;    // [max_batch][mod_cap] bias table sorted by id
    // History occurrence counts, zero between steps: the step prep adds, the head epilogue
    // reads them and zeroes each entry it read.
    uint32_t* hcount = nullptr;  // [max_batch][V]
    uint32_t* hbits = nullptr;   // [max_batch][hbw] bit per id with a nonzero count
    uint32_t hbw = 0;            // ceil(V / 32)
    uint32_t* mod_count = nullptr;     // [max_batch]
    uint32_t* block_start = nullptr;   // [max_batch][ntile + 1]
    void* list_scratch = nullptr;      // [max_batch][V] uint2 compaction lists (select)
    unsigned long long* fv_acc = nullptr;     // [max_batch][2][kFvBins], zero between steps
    unsigned long long* fv_merged = nullptr;  // [max_batch][2][kFvBins]
    unsigned long long* fv_cand = nullptr;    // [max_batch][kFvCandCap]
    void* fv_state = nullptr;                 // [max_batch] x kFvStateBytes

    // Host staging ring for DevRow uploads (pinned).
    // Rows of batches above kInlineRows are staged in a ring of pinned slots, reused group by
    // group: one event per kRingGroup steps marks the group's slots as read.
    static constexpr int kRing = 16;
    static constexpr int kRingGroup = 8;
    // Set by the select kernel (row + 1) when TURBO_STEP_APPEND_HISTORY meets a full history;
    // turbo_lmhead_synchronize reports and clears it. Pinned, mapped, coherent.
    uint32_t* overflow_host = nullptr;
    uint32_t* overflow_dev = nullptr;
    DevRow* ring_host = nullptr;       // [kRing][max_batch], pinned, mapped, coherent
    DevRow* ring_dev = nullptr;        // device-visible address of ring_host
    hipEvent_t ring_ev[kRing / kRingGroup] = {};
    int ring_pos = 0;

    // Head-kernel timing.
    bool timing = false;
    uint32_t t_stride = 1;       // time every t_stride-th head launch
    uint64_t t_launch = 0;       // head launches since timing was enabled
    static constexpr int kTimerSlots = 1024;
    hipEvent_t t_start[kTimerSlots] = {};
    hipEvent_t t_stop[kTimerSlots] = {};
    int t_count = 0;
};

// Arguments shared by the head-kernel epilogues and the logits-only epilogue.
struct EpiArgs {
    uint32_t V;
    uint32_t ntile;
    float cap;                 // softcap applied to the raw accumulator (0 = skip)
    float* logits;             // [B][V] or null (not written)
    BlockPartial* partials;    // [B][ntile], or null for a logits-only call (not written)
    const DevRow* rows;        // [B]
    const ModEntry* mods;      // [B][mod_cap] bias tables (rows with has_mods & 2)
    uint32_t mod_cap;
    const uint32_t* block_start;  // [B][ntile + 1] first bias entry per tile
    uint32_t* hcount;          // [B][V] history counts (rows with has_mods & 1); zeroed once read
    uint32_t* hbits;           // [B][hbw] bit per id with a nonzero count; zeroed once read
    uint32_t hbw;
    const uint32_t* ban;       // [B][ban_stride] or null
    uint32_t ban_stride;
    float rep_limit;           // 0.9999 * softcap used by the repetition clamp (0 = none)
    uint32_t no_sumexp;        // 1: no row samples from a shortlist, so the block sums of
                               // exp(l - max) are not needed and stay 0
    uint32_t no_smax;          // 1: no row samples from a shortlist, so the blocks' second
                               // largest values are not needed (left -inf by the MFMA head)
    uint32_t meta;             // 1: some row has modifiers or a ban mask (the MFMA head stages
                               // their words in LDS); 0: the MFMA head skips modifiers and ban
    const float* xscale;       // [B] the MFMA head multiplies row b's accumulators by xscale[b]
                               // (the power of two its fp16 activations were scaled down by)
};

enum class HeadPath { Digits, Mfma };

// prep.hip
// Batches of at most this many rows pass their parameters in the step-prep kernel arguments.
constexpr int kInlineRows = 8;
struct PrepArgs {
    int B;
    const DevRow* rows_src;      // host-mapped staging slot (null: the rows are in inl)
    DevRow inl[kInlineRows];     // the rows of a small batch
    DevRow* rows_dst;            // device row buffer, filled by block 0 (null: no copy block)
    // activations (null hidden: no activation work)
    const void* hidden;
    int dtype;                   // 0 fp32, 1 bf16
    int normed;
    const uint16_t* gamma;
    float eps;
    uint32_t D;
    float* xn;                   // optional normalised copy [B][D]
    int path;                    // 0 digit planes, 1 fp16
    uint32_t* xdig;
    float* xws;
    float* xsum;
    uint16_t* x16;
    int x16_denorm;              // fp16 layout: (16 x, x) per (even, odd) element, else (x, x / 16)
    float* xscale;               // [B] 2^k when row b is stored in x16 as x * 2^-k (fp16 path)
    // history counts and the bias table
    uint32_t V, ntile, P;        // P: bias sort size (power of two >= bias_stride)
    uint32_t* hcount;
    uint32_t* hbits;
    uint32_t hbw;
    const uint32_t* history;
    uint32_t hist_stride;
    const uint32_t* hist_len;
    const uint32_t* bias_ids;
    const float* bias_vals;
    uint32_t bias_stride;
    const uint32_t* bias_count;
    ModEntry* mods;
    uint32_t mod_cap;
    uint32_t* mod_count;
    uint32_t* block_start;
    uint32_t mod_bits[16];       // 2 bits per row (DevRow::has_mods), so no block reads the
                                 // host-mapped staging slot except the row copy
};
// Fills Wt, SBt and SB16t on st and waits for it. Returns 1 when every scale fits the denormal
// dequant (|s| < 1/16; SB16t holds s * 2^20), 0 when SB16t holds s, and -1 when some scale or
// bias is outside the fp16 range either way (the matrix-core path cannot use the table).
int launch_repack(const Head& h, const uint8_t* W, const uint16_t* S, const uint16_t* B,
                  hipStream_t st);
void launch_step_prep(const Head& h, const PrepArgs& a, bool with_mods, hipStream_t st);
uint32_t modtable_sort_size(const Head& h, uint32_t n);

// gemv_digits.hip: the small-batch step with the preparation folded into the head kernel.
// Every workgroup recomputes the final RMSNorm and the digit planes of the whole row in LDS and
// counts the history occurrences of its own ids there, so the step needs no preparation kernel
// (and no hcount / hbits traffic). Bias tables still go through the preparation kernel.
constexpr int kFusedRows = 2;
constexpr uint32_t kFusedMaxD = 8192;       // digit planes of a row in LDS: D / 32 * 24 words
constexpr uint32_t kFusedHistMax = 4096;    // history stride scanned by every workgroup
// Heads with fewer tiles fold the digit planes into the split kernel instead (normalised rows
// without history only: the int4 matvec and logits entry points).
constexpr uint32_t kFusedMinTiles = 2048;
struct FusedPrep {
    const void* hidden;
    int dtype;                   // 0 fp32, 1 bf16
    int normed;
    const uint16_t* gamma;
    float eps;
    const uint32_t* history;     // [B][hist_stride] or null
    const uint32_t* hist_len;
    uint32_t hist_stride;
    DevRow* rows_dst;            // device row buffer for the select kernel (block 0 writes it)
    DevRow inl[kFusedRows];
};
void launch_head_digits_fused(const Head& h, int batch, const FusedPrep& fp, const EpiArgs& ep,
                              hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
// Threads per workgroup of the split digit kernel for this head (0: one wave per tile instead).
uint32_t split_threads(const Head& h);
// Waves the split digit kernel gives one 64-row tile of a G-group matrix with ntile tiles.
uint32_t split_waves(uint32_t G, uint32_t ntile);

// Grouped matrix-vector products (one input row per matrix, raw fp32 outputs), one launch.
constexpr uint32_t kMaxGroupMats = 32;
struct GroupMat {
    const uint4* Wt;
    const uint32_t* SBt;
    const float* x;      // [D] fp32 device
    float* out;          // [rows] fp32 device
    uint32_t rows, D;
    uint32_t tile_begin; // first workgroup of this matrix
    uint32_t ks;         // waves per tile (split_waves), at least 1
};
struct GroupArgs {
    GroupMat m[kMaxGroupMats];
    uint32_t count;
};
void launch_matvec_grouped(const GroupArgs& a, uint32_t total_tiles, hipStream_t st);
// prep.hip: the tiled table of any matrix (Wt [ntile][NC][64] x 16 B, SBt [ntile][G][64] u32).
void launch_repack_table(uint4* Wt, uint32_t* SBt, uint32_t V, uint32_t NC, uint32_t G, uint32_t ntile,
                         const uint8_t* W, const uint16_t* S, const uint16_t* B, hipStream_t st);

// gemv_digits.hip / gemm_mfma.hip
// ev0 / ev1 (may be null): timing events stamped by the head kernel's own dispatch
// (hipExtLaunchKernelGGL), so timing adds no packets between kernels.
void launch_head_digits(const Head& h, int batch, const EpiArgs& ep, hipStream_t st,
                        hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
void launch_head_mfma(const Head& h, int batch, const EpiArgs& ep, hipStream_t st,
                      hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
// The matrix-core head addresses the tiled table through buffer resources, whose sizes and
// offsets are 32-bit: it serves tables of at most 4 GiB.
inline bool mfma_table_fits(const Head& h) {
    return (uint64_t)h.ntile * h.NC * kTileRows * 16u <= 0xFFFFFFFFull &&
           (uint64_t)h.ntile * h.G * kTileRows * 4u <= 0xFFFFFFFFull;
}
// epilogue over caller logits (no GEMV): logits are read, modified and summarised in place.
void launch_logits_epilogue(const Head& h, int batch, const EpiArgs& ep, hipStream_t st);

// select.hip
struct SelectArgs {
    uint32_t V;
    uint32_t ntile;
    const float* logits;          // [B][V] final logits (may be null for all-greedy)
    const BlockPartial* partials; // [B][ntile]
    const DevRow* rows;
    const float* uniforms;        // [B] or null
    uint32_t* tokens;
    void* report;                 // TurboRowReport* or null
    uint32_t* history;            // append target or null
    uint32_t hist_stride;
    uint32_t* hist_len;
    uint32_t* hist_overflow;      // host-mapped word set to (row + 1) when a full history drops a token, or null
    // multi-workgroup full-vocabulary path (null fv_acc: one workgroup per row)
    unsigned long long* fv_acc;     // [B][2][kFvBins] slice histograms summed by atomics
    unsigned long long* fv_merged;  // [B][2][kFvBins] merged histograms
    unsigned long long* fv_cand;    // [B][kFvCandCap] gathered candidates
    void* fv_state;                 // [B] x kFvStateBytes per-row plan and counters
};
// Steps with at most kFvMaxRows full-vocabulary rows split each such row's two passes over
// several workgroups (slices): about kFvSliceBudget workgroups in all, from kFvMinSlices to
// kFvMaxSlices per row. More slices shorten each workgroup's pass, but every slice adds its
// histogram into the row's sums with global atomics, which contend once thousands of workgroups
// do it. More such rows than kFvMaxRows take one workgroup per row.
constexpr uint32_t kFvMaxRows = 64;
constexpr uint32_t kFvSliceBudget = 256;
constexpr uint32_t kFvMinSlices = 4;
constexpr uint32_t kFvMaxSlices = 32;
constexpr uint32_t kFvBins = 2048;
constexpr uint32_t kFvCandCap = 8192;
constexpr size_t kFvStateBytes = 128;
// TurboRowReport.status bit: the row's history was full, so its token was not appended.
constexpr uint32_t kStatusHistoryFull = 1u;
// The rows that take the full-vocabulary value path (sampled, shortlist lifted), with their
// temperatures, in ascending row order, when there are at most kFvMaxRows of them (else n = 0).
// The multi-workgroup kernels take their row from this list in the kernel arguments.
struct FvList {
    uint32_t n = 0;
    float temp[kFvMaxRows];
    uint8_t row[kFvMaxRows];  // row indices below 256, the largest batch
};
void launch_select(const Head& h, int batch, const SelectArgs& a, const FvList& fv, hipStream_t st);

// misc.hip
void launch_softcap(float* z, size_t n, float cap, hipStream_t st);
void launch_repetition(float* logits, uint32_t vocab, const uint32_t* history, uint32_t n,
                       float penalty, float softcap, hipStream_t st);
// out[i][D] = row tokens[i] of the tied table dequantised and scaled by `scale` (NaN past V).
void launch_embed(const Head& h, const uint32_t* tokens, int n, float* out, float scale, hipStream_t st);

// Throws std::runtime_error with the HIP error string on failure.
void check_hip(hipError_t e, const char* what);

// Makes `dev` the current device for the guard's lifetime and then restores the caller's, so an
// entry point leaves the calling thread's current device as it found it.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) check_hip(hipSetDevice(dev), "hipSetDevice");
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;
};

// api.cpp: turbo_sample_logits on a head whose scratch the caller provides (h.Wt may be null: no
// head kernel runs). Validates the rows and enqueues the modifier epilogue and the select on
// h.stream; allocates nothing for batches of at most kInlineRows rows.
int sample_on_head(Head& h, const TurboStepInputs* in, const TurboStepOutputs* out, float* logits);
// api.cpp: sets the thread-local string turbo_lmhead_last_error returns.
void set_last_error(const char* msg);

}  // namespace tdt
