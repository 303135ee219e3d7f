// turbo_sample_logits_noalloc: the sampler over caller logits without a handle and without any
// allocation, for callers that cannot call hipMalloc (code under HIP graph capture, tight serving
// loops, harnesses that forbid it).
//
// Every per-call buffer the modifier epilogue and the select kernels need (block partials, row
// parameters, the bias table, history counts, compaction lists, full-vocabulary histograms) lives
// in one file-scope device array, `scratch`, sized for kNaBatch rows of up to kNaVocab ids. Each
// GPU holds its own copy until the process ends. Its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is handed to kernels.
//
// The kernels leave the history counts, their bitmap and the full-vocabulary histogram sums at
// zero after every call (each is cleared by the kernel that consumes it), so one clear on first
// use keeps the invariant. All calls on a GPU share that GPU's array: calls that overlap on one
// GPU (two streams, two threads) race and must be serialised by the caller.
#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <mutex>
#include <stdexcept>
#include <string>

#include "dt_internal.h"

namespace tdt {
namespace {

constexpr uint32_t kNaBatch = TURBO_NOALLOC_MAX_BATCH;
constexpr uint32_t kNaVocab = TURBO_NOALLOC_MAX_VOCAB;
constexpr uint32_t kNaTiles = kNaVocab / kTileRows;
constexpr uint32_t kNaWords = kNaVocab / 32;
static_assert(kNaVocab % kTileRows == 0 && kNaBatch <= (uint32_t)kInlineRows && kNaBatch <= kFvMaxRows,
              "rows ride in the kernel arguments; the full-vocabulary state covers every row");

constexpr size_t align256(size_t n) { return (n + 255u) & ~size_t(255); }

// Region offsets (bytes) inside `scratch`. The first group must be zero between calls.
constexpr size_t kOffHcount = 0;
constexpr size_t kOffHbits = kOffHcount + align256(sizeof(uint32_t) * kNaBatch * kNaVocab);
constexpr size_t kOffFvAcc = kOffHbits + align256(sizeof(uint32_t) * kNaBatch * kNaWords);
constexpr size_t kOffFvState = kOffFvAcc + align256(sizeof(unsigned long long) * kNaBatch * 2u * kFvBins);
constexpr size_t kZeroBytes = kOffFvState + align256(kFvStateBytes * kNaBatch);
constexpr size_t kOffPartials = kZeroBytes;
constexpr size_t kOffRows = kOffPartials + align256(sizeof(BlockPartial) * kNaBatch * kNaTiles);
constexpr size_t kOffMods = kOffRows + align256(sizeof(DevRow) * kNaBatch);
constexpr size_t kOffModCount = kOffMods + align256(sizeof(ModEntry) * kNaBatch * kModCap);
constexpr size_t kOffBlockStart = kOffModCount + align256(sizeof(uint32_t) * kNaBatch);
constexpr size_t kOffList = kOffBlockStart + align256(sizeof(uint32_t) * kNaBatch * (kNaTiles + 1u));
constexpr size_t kOffFvMerged = kOffList + align256(sizeof(uint2) * kNaBatch * kNaVocab);
constexpr size_t kOffFvCand = kOffFvMerged + align256(sizeof(unsigned long long) * kNaBatch * 2u * kFvBins);
constexpr size_t kScratchBytes = kOffFvCand + align256(sizeof(unsigned long long) * kNaBatch * kFvCandCap);
static_assert(kScratchBytes <= (size_t)15 << 20, "the static scratch stays below 15 MiB");

// In host code this name is a stand-in, not a device address: only the address returned by
// hipGetSymbolAddress below is passed to kernels.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void k_zero_words(uint4* p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

struct DeviceScratch {
    unsigned char* ptr = nullptr;  // this device's copy of `scratch`
    bool ready = false;            // zero regions cleared
};
std::mutex g_mu;
std::array<DeviceScratch, 64> g_dev;

// The current device's scratch address: looked up (and its zero regions cleared on `st`) on the
// first call on that device.
unsigned char* device_scratch(int dev, hipStream_t st) {
    if (dev < 0 || dev >= (int)g_dev.size()) throw std::runtime_error("device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceScratch& d = g_dev[(size_t)dev];
    if (!d.ptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        d.ptr = static_cast<unsigned char*>(p);
    }
    if (!d.ready) {
        // A fill kernel, not hipMemsetAsync, so that a captured first call records a kernel
        // node. Under capture the clear runs only when the graph does, so the next call outside
        // a capture clears again.
        static_assert(kZeroBytes % 16u == 0u, "whole 16-byte words");
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        check_hip(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
        hipLaunchKernelGGL(k_zero_words, dim3(1024), dim3(256), 0, st, reinterpret_cast<uint4*>(d.ptr + kOffHcount),
                           kZeroBytes / 16u);
        check_hip(hipGetLastError(), "clear static scratch");
        d.ready = cs == hipStreamCaptureStatusNone;
    }
    return d.ptr;
}

}  // namespace
}  // namespace tdt

// Errors go through the library's one last-error channel (turbo_lmhead_last_error).
extern "C" TURBO_DT_API int turbo_sample_logits_noalloc(void* hip_stream, uint32_t vocab, float final_logit_softcap,
                                                        float* logits, const TurboStepInputs* in,
                                                        const TurboStepOutputs* out) {
    using namespace tdt;
    set_last_error("");
    try {
        if (vocab == 0u || vocab > kNaVocab)
            throw std::runtime_error("vocab must be in 1.." + std::to_string(kNaVocab) + " (the static scratch's size)");
        if (!in) throw std::runtime_error("null inputs");
        if (in->batch < 1 || (uint32_t)in->batch > kNaBatch)
            throw std::runtime_error("batch must be in 1.." + std::to_string(kNaBatch) + " (the static scratch's size)");
        if (in->bias_stride > kModCap)
            throw std::runtime_error("bias_stride exceeds the per-row bias-entry limit of " + std::to_string(kModCap));
        if (!std::isfinite(final_logit_softcap)) throw std::runtime_error("softcap must be finite");
        int dev = 0;
        check_hip(hipGetDevice(&dev), "hipGetDevice");
        hipStream_t st = static_cast<hipStream_t>(hip_stream);
        unsigned char* base = device_scratch(dev, st);

        Head h;
        h.device = dev;
        h.V = vocab;
        h.ntile = (vocab + kTileRows - 1u) / kTileRows;
        h.cap = final_logit_softcap > 0.f ? final_logit_softcap : 0.f;
        h.stream = st;
        h.max_batch = (int)kNaBatch;
        h.mod_cap = kModCap;
        h.hbw = (vocab + 31u) / 32u;
        h.hcount = reinterpret_cast<uint32_t*>(base + kOffHcount);
        h.hbits = reinterpret_cast<uint32_t*>(base + kOffHbits);
        h.fv_acc = reinterpret_cast<unsigned long long*>(base + kOffFvAcc);
        h.fv_state = base + kOffFvState;
        h.partials = reinterpret_cast<BlockPartial*>(base + kOffPartials);
        h.rows = reinterpret_cast<DevRow*>(base + kOffRows);
        h.mods = reinterpret_cast<ModEntry*>(base + kOffMods);
        h.mod_count = reinterpret_cast<uint32_t*>(base + kOffModCount);
        h.block_start = reinterpret_cast<uint32_t*>(base + kOffBlockStart);
        h.list_scratch = base + kOffList;
        h.fv_merged = reinterpret_cast<unsigned long long*>(base + kOffFvMerged);
        h.fv_cand = reinterpret_cast<unsigned long long*>(base + kOffFvCand);
        return sample_on_head(h, in, out, logits);
    } catch (const std::exception& ex) {
        set_last_error(ex.what());
        return 0;
    } catch (...) {
        set_last_error("unknown error");
        return 0;
    }
}
