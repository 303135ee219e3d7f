// The in-engine caller of the decode tail, in the shape of Turbo-WinFare's ForwardRunner:
//   initialize()      the head from the bundle's resident.bin (src/runner.cpp:83-293, :324-357)
//   produce_token()   embedding -> [layers] -> the decode tail (src/runner.cpp:372-807)
//   generate_tokens() prefill, then the decode loop with a growing history (src/runner.cpp:818-898)
// compiled against include/turbo_decode_tail.h and linked to libturbo_decode_tail.so, so the C++
// path a maintainer adds to runner.cpp is built and run, not only described.
//
// The model between the embedding and the final norm is a stand-in: the 30 layers are replaced by
// one fixed residual per step, hidden = alpha * embedding + z[position] (z: a caller-provided
// [positions][hidden] array), so that every position's next-token distribution depends on the
// token and stays far from one-hot. Everything after it is the tail as the engine would call it.
//
// Exposed to the test through one C entry point, tail_generate; failures come back as 0 with the
// message of turbo_lmhead_last_error (or of the runner) in `err`.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "turbo_decode_tail.h"

namespace {

// include/gturbo/format.hpp:33-37: the engine's error type for bad data and bad requests.
struct GTurboFormatError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// The sampling fields of GenerationOptions that the tail reads (include/gturbo/runner.hpp:26-43,
// include/gturbo/sampling.hpp:21-30).
struct SamplingParams {
    float temperature = 0.0f;
    float top_p = 1.0f;
    int top_k = 0;
    float repetition_penalty = 1.0f;
    bool has_seed = false;
    uint64_t seed = 0;
};

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw GTurboFormatError(std::string(what) + ": " + hipGetErrorString(e));
}

// hidden = alpha * hidden + z, rounded per operation like the oracle's float32 replay.
__global__ void k_stand_in_layers(float* hidden, const float* z, float alpha, uint32_t n) {
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) hidden[i] = alpha * hidden[i] + z[i];
}

class DecodeTailRunner {
  public:
    ~DecodeTailRunner() {
        if (lmhead_) turbo_lmhead_destroy(lmhead_);
        for (void* p : {(void*)d_hidden_, (void*)d_z_, (void*)d_history_, (void*)d_history_len_, (void*)d_tokens_,
                        (void*)d_report_})
            if (p) (void)hipFree(p);
        if (stream_) (void)hipStreamDestroy(stream_);
    }

    // ForwardRunner::initialize (src/runner.cpp:324-357): the tied table and the final norm from
    // the bundle's resident index; per-request buffers sized for the longest generation.
    void initialize(const std::string& resident_path, float final_logit_softcap, float rms_norm_eps,
                    const float* z_host, uint32_t positions, uint32_t history_cap) {
        // the library must have the layout this file was compiled against
        if (turbo_abi_version() != TURBO_DT_ABI_VERSION ||
            turbo_abi_struct_size(TURBO_ABI_SAMPLING_ROW) != sizeof(TurboSamplingRow) ||
            turbo_abi_struct_size(TURBO_ABI_STEP_INPUTS) != sizeof(TurboStepInputs) ||
            turbo_abi_struct_size(TURBO_ABI_STEP_OUTPUTS) != sizeof(TurboStepOutputs) ||
            turbo_abi_struct_size(TURBO_ABI_ROW_REPORT) != sizeof(TurboRowReport) ||
            turbo_abi_struct_size(TURBO_ABI_BUNDLE_TENSOR) != sizeof(TurboBundleTensor))
            throw GTurboFormatError("libturbo_decode_tail.so has another ABI than turbo_decode_tail.h");
        hip_check(hipStreamCreate(&stream_), "hipStreamCreate");  // default priority
        lmhead_ = turbo_lmhead_create_from_bundle(resident_path.c_str(), final_logit_softcap, rms_norm_eps,
                                                  /*device=*/0);
        if (!lmhead_) throw GTurboFormatError(turbo_lmhead_last_error());
        if (!turbo_lmhead_set_stream(lmhead_, stream_)) throw GTurboFormatError(turbo_lmhead_last_error());
        TurboBundleTensor t;
        if (!turbo_bundle_find_tensor(resident_path.c_str(), "model.embed_tokens.weight", &t))
            throw GTurboFormatError(turbo_lmhead_last_error());
        vocab_ = t.rows;
        hidden_size_ = t.in_dim;
        history_cap_ = history_cap;
        positions_ = positions;
        hip_check(hipMalloc(&d_hidden_, sizeof(float) * hidden_size_), "hipMalloc hidden");
        hip_check(hipMalloc(&d_z_, sizeof(float) * hidden_size_ * positions), "hipMalloc z");
        hip_check(hipMemcpy(d_z_, z_host, sizeof(float) * hidden_size_ * positions, hipMemcpyHostToDevice), "upload z");
        hip_check(hipMalloc(&d_history_, sizeof(uint32_t) * history_cap), "hipMalloc history");
        hip_check(hipMalloc(&d_history_len_, sizeof(uint32_t)), "hipMalloc history_len");
        hip_check(hipMalloc(&d_tokens_, sizeof(uint32_t) * (positions + 1u)), "hipMalloc tokens");
    }

    // ForwardRunner::produce_token for the token in d_tokens_[slot_in] at `position`; the next
    // token lands in d_tokens_[slot_out] and is returned (the 4-byte readback the reference does
    // with the Map of buf_out_token_). append: the history grows by the sampled token on the
    // device (the push_back of src/runner.cpp:878).
    uint32_t produce_token(uint32_t slot_in, uint32_t slot_out, int position, const SamplingParams& s, bool append,
                           float alpha) {
        if (position < 0 || static_cast<uint32_t>(position) >= positions_)
            throw GTurboFormatError("position outside the stand-in layers' table");
        // Embedding (src/cpu_reference.cpp:323-329): the same tied table, dequantised and scaled
        // by sqrt(hidden).
        if (!turbo_lmhead_embed(lmhead_, d_tokens_ + slot_in, 1, d_hidden_))
            throw GTurboFormatError(turbo_lmhead_last_error());
        // ... the layers (src/runner.cpp:469-717), here the stand-in residual ...
        hipLaunchKernelGGL(k_stand_in_layers, dim3((hidden_size_ + 255u) / 256u), dim3(256), 0, stream_, d_hidden_,
                           d_z_ + static_cast<size_t>(position) * hidden_size_, alpha, hidden_size_);
        hip_check(hipGetLastError(), "stand-in layers");

        // The decode tail, replacing src/runner.cpp:719-807.
        TurboSamplingRow row;
        turbo_sampling_row_default(&row);
        row.temperature = s.temperature;
        row.top_p = s.top_p;
        row.top_k = s.top_k;
        row.repetition_penalty = s.repetition_penalty;
        row.rng = TURBO_RNG_REFERENCE;                       // the reference's seed_for(position) map
        row.has_seed = s.has_seed ? 1 : 0;
        row.seed = s.seed;
        row.counter = static_cast<uint64_t>(position);

        TurboStepInputs in;
        std::memset(&in, 0, sizeof in);                      // zero = every side input disabled
        in.batch = 1;
        in.hidden = d_hidden_;                               // fp32 [D] on the device (buf_hidden_)
        in.hidden_dtype = TURBO_HIDDEN_F32;
        in.rows = &row;
        in.history = d_history_;                             // device copy of `history`
        in.history_stride = history_cap_;
        in.history_len = d_history_len_;
        in.flags = append ? TURBO_STEP_APPEND_HISTORY : 0u;  // the push_back of src/runner.cpp:878

        TurboRowReport report;
        TurboStepOutputs out;
        std::memset(&out, 0, sizeof out);
        out.tokens = d_tokens_ + slot_out;                   // uint32 on the device
        out.report = report_dev();
        if (!turbo_lmhead_step(lmhead_, &in, &out)) throw GTurboFormatError(turbo_lmhead_last_error());

        uint32_t token = 0;
        hip_check(hipMemcpyAsync(&token, d_tokens_ + slot_out, sizeof token, hipMemcpyDeviceToHost, stream_),
                  "token readback");
        hip_check(hipMemcpyAsync(&report, report_dev(), sizeof report, hipMemcpyDeviceToHost, stream_),
                  "report readback");
        if (!turbo_lmhead_synchronize(lmhead_)) throw GTurboFormatError(turbo_lmhead_last_error());
        // sample_token throws on a degenerate distribution (src/sampling.cpp:116-118); the tail
        // reports it as path 3 with token 0xFFFFFFFF, which must not reach the next embedding.
        if (report.path == 3u || token >= vocab_) throw GTurboFormatError("logit distribution is degenerate");
        return token;
    }

    // ForwardRunner::generate_tokens (src/runner.cpp:818-898) without the detokeniser and stop
    // strings: prefill over the prompt (history = the prompt), then max_tokens decode steps, the
    // history growing by each emitted token. Returns the emitted tokens.
    std::vector<uint32_t> generate_tokens(const std::vector<uint32_t>& prompt, const SamplingParams& s,
                                          int max_tokens, float alpha) {
        if (prompt.empty()) throw GTurboFormatError("empty prompt");
        if (prompt.size() + static_cast<size_t>(max_tokens) > history_cap_)
            throw GTurboFormatError("history capacity below prompt + max_tokens");
        if (prompt.size() + static_cast<size_t>(max_tokens) > positions_)
            throw GTurboFormatError("more positions than the stand-in layers' table");
        // the device history starts as the prompt (src/runner.cpp:858)
        const uint32_t n = static_cast<uint32_t>(prompt.size());
        hip_check(hipMemcpyAsync(d_history_, prompt.data(), sizeof(uint32_t) * n, hipMemcpyHostToDevice, stream_),
                  "upload history");
        hip_check(hipMemcpyAsync(d_history_len_, &n, sizeof n, hipMemcpyHostToDevice, stream_), "upload history_len");
        std::vector<uint32_t> out;
        uint32_t current = 0;
        for (uint32_t i = 0; i < n; ++i) {
            // the prompt token goes in slot 0; the last prefill step's token is the first emitted
            hip_check(hipMemcpyAsync(d_tokens_, &prompt[i], sizeof(uint32_t), hipMemcpyHostToDevice, stream_),
                      "upload prompt token");
            current = produce_token(0u, 1u, static_cast<int>(i), s, /*append=*/i + 1u == n, alpha);
        }
        // decode: token t sits in slot t + 1 and produces slot t + 2, on the device
        for (int t = 0; t < max_tokens; ++t) {
            out.push_back(current);
            if (t + 1 >= max_tokens) break;
            current = produce_token(static_cast<uint32_t>(t) + 1u, static_cast<uint32_t>(t) + 2u,
                                    static_cast<int>(n) + t, s, /*append=*/true, alpha);
        }
        return out;
    }

    uint32_t history_len() {
        uint32_t v = 0;
        hip_check(hipMemcpy(&v, d_history_len_, sizeof v, hipMemcpyDeviceToHost), "history_len readback");
        return v;
    }
    void history(uint32_t* out, uint32_t n) {
        hip_check(hipMemcpy(out, d_history_, sizeof(uint32_t) * n, hipMemcpyDeviceToHost), "history readback");
    }

  private:
    TurboRowReport* report_dev() {
        if (!d_report_) hip_check(hipMalloc(&d_report_, sizeof(TurboRowReport)), "hipMalloc report");
        return d_report_;
    }

    void* lmhead_ = nullptr;
    hipStream_t stream_ = nullptr;
    uint32_t vocab_ = 0, hidden_size_ = 0, history_cap_ = 0, positions_ = 0;
    float* d_hidden_ = nullptr;
    float* d_z_ = nullptr;
    uint32_t* d_history_ = nullptr;
    uint32_t* d_history_len_ = nullptr;
    uint32_t* d_tokens_ = nullptr;
    TurboRowReport* d_report_ = nullptr;
};

}  // namespace

// Runs generate_tokens on a runner created from `resident_path`. z: [positions][hidden] host
// floats of the stand-in layers. Writes the max_tokens emitted tokens and the final device
// history (the prompt, then every emitted token: prompt_len + max_tokens ids). 1/0.
extern "C" __attribute__((visibility("default"))) int tail_generate(
    const char* resident_path, float softcap, float eps, const float* z, uint32_t positions, float alpha,
    const uint32_t* prompt, uint32_t prompt_len, float temperature, float top_p, int top_k,
    float repetition_penalty, int has_seed, uint64_t seed, int max_tokens, uint32_t* tokens_out,
    uint32_t* history_out, uint32_t* history_len_out, char* err, size_t errlen) {
    try {
        DecodeTailRunner r;
        r.initialize(resident_path, softcap, eps, z, positions, prompt_len + static_cast<uint32_t>(max_tokens));
        SamplingParams s;
        s.temperature = temperature;
        s.top_p = top_p;
        s.top_k = top_k;
        s.repetition_penalty = repetition_penalty;
        s.has_seed = has_seed != 0;
        s.seed = seed;
        const std::vector<uint32_t> toks =
            r.generate_tokens(std::vector<uint32_t>(prompt, prompt + prompt_len), s, max_tokens, alpha);
        std::memcpy(tokens_out, toks.data(), sizeof(uint32_t) * toks.size());
        *history_len_out = r.history_len();
        r.history(history_out, *history_len_out);
        return 1;
    } catch (const std::exception& ex) {
        if (err && errlen) {
            std::strncpy(err, ex.what(), errlen - 1);
            err[errlen - 1] = '\0';
        }
        return 0;
    }
}
