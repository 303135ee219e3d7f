// Int4 matrix handles and the grouped matrix-vector product (include/turbo_decode_tail.h).
//
// A matrix handle holds one affine-int4 weight matrix in the kernels' tiled layout and nothing
// else: no logits, history counts, bias table, select state, staging ring or events, so its
// device footprint is the table itself (rows x in_dim / 2 bytes + rows x in_dim / 64 x 4 bytes).
// This is the layer-loop use of GemvInt4 (src/runner.cpp:431-442, :612-646, :671-678): many small
// matrices (the routed experts' slots) that the reference dispatches one at a time.
#include <hip/hip_runtime.h>

#include <cstring>
#include <stdexcept>
#include <string>

#include "dt_internal.h"

namespace {

constexpr uint32_t kMatrixMagic = 0x4D544454u;  // "TDTM"

struct MatrixBox {
    uint32_t magic = kMatrixMagic;
    int device = 0;
    uint32_t rows = 0, D = 0, G = 0, NC = 0, ntile = 0;
    uint4* Wt = nullptr;
    uint32_t* SBt = nullptr;
    // the streams this matrix's loads and products were enqueued on, waited for by destroy (more
    // than kStreams distinct streams: destroy waits for the whole device)
    static constexpr int kStreams = 4;
    hipStream_t used[kStreams] = {};
    int nused = 0;
    bool many = false;
    void note(hipStream_t st) {
        for (int i = 0; i < nused; ++i)
            if (used[i] == st) return;
        if (nused < kStreams) used[nused++] = st;
        else many = true;
    }
};

MatrixBox* mbox(void* p) {
    if (!p) throw std::runtime_error("null matrix handle");
    auto* m = static_cast<MatrixBox*>(p);
    if (m->magic != kMatrixMagic) throw std::runtime_error("invalid matrix handle");
    return m;
}

void free_matrix(MatrixBox& m) {
    if (m.Wt) (void)hipFree(m.Wt);
    if (m.SBt) (void)hipFree(m.SBt);
    m.Wt = nullptr;
    m.SBt = nullptr;
}

}  // namespace

#define MAT_TRY try {
#define MAT_CATCH(ret)                       \
    }                                        \
    catch (const std::exception& ex) {       \
        tdt::set_last_error(ex.what());      \
        return ret;                          \
    }                                        \
    catch (...) {                            \
        tdt::set_last_error("unknown error"); \
        return ret;                          \
    }

extern "C" {

TURBO_DT_API void* turbo_int4_matrix_create(uint32_t rows, uint32_t in_dim, int device) {
    tdt::set_last_error("");
    MAT_TRY
    if (rows == 0 || rows > (1u << 24)) throw std::runtime_error("rows must be in 1..16777216");
    if (in_dim == 0 || in_dim % 64u != 0 || in_dim > tdt::kFusedMaxD)
        throw std::runtime_error("in_dim must be a positive multiple of 64, at most 8192");
    int ndev = 0;
    tdt::check_hip(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    if (device < 0 || device >= ndev) throw std::runtime_error("no such HIP device");
    tdt::DeviceGuard dg(device);
    auto* m = new MatrixBox;
    m->device = device;
    m->rows = rows;
    m->D = in_dim;
    m->G = in_dim / 64u;
    m->NC = in_dim / 32u;
    m->ntile = (rows + tdt::kTileRows - 1u) / tdt::kTileRows;
    try {
        tdt::check_hip(hipMalloc(&m->Wt, sizeof(uint4) * (size_t)m->ntile * m->NC * tdt::kTileRows), "alloc matrix");
        tdt::check_hip(hipMalloc(&m->SBt, sizeof(uint32_t) * (size_t)m->ntile * m->G * tdt::kTileRows),
                       "alloc matrix scales");
    } catch (...) {
        free_matrix(*m);
        delete m;
        throw;
    }
    return m;
    MAT_CATCH(nullptr)
}

TURBO_DT_API int turbo_int4_matrix_load(void* handle, const uint8_t* weight, const uint16_t* scales,
                                        const uint16_t* biases, int weights_on_device, void* hip_stream) {
    tdt::set_last_error("");
    MAT_TRY
    MatrixBox* m = mbox(handle);
    if (!weight || !scales || !biases) throw std::runtime_error("weight/scales/biases are NULL");
    tdt::DeviceGuard dg(m->device);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    m->note(st);
    const size_t wbytes = (size_t)m->rows * (m->D / 2u), gcount = (size_t)m->rows * m->G;
    if (weights_on_device) {
        // the slot's bytes are repacked in place of the previous contents, stream-ordered
        tdt::launch_repack_table(m->Wt, m->SBt, m->rows, m->NC, m->G, m->ntile, weight, scales, biases, st);
        return 1;
    }
    // host arrays: staged through temporary device buffers, synchronously
    uint8_t* tW = nullptr;
    uint16_t *tS = nullptr, *tB = nullptr;
    hipError_t e = hipMalloc(&tW, wbytes);
    if (e == hipSuccess) e = hipMalloc(&tS, gcount * 2u);
    if (e == hipSuccess) e = hipMalloc(&tB, gcount * 2u);
    if (e == hipSuccess) e = hipMemcpyAsync(tW, weight, wbytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(tS, scales, gcount * 2u, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(tB, biases, gcount * 2u, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        try {
            tdt::launch_repack_table(m->Wt, m->SBt, m->rows, m->NC, m->G, m->ntile, tW, tS, tB, st);
        } catch (...) {
            e = hipErrorLaunchFailure;
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (tW) (void)hipFree(tW);
    if (tS) (void)hipFree(tS);
    if (tB) (void)hipFree(tB);
    tdt::check_hip(e, "load matrix");
    return 1;
    MAT_CATCH(0)
}

TURBO_DT_API void turbo_int4_matrix_destroy(void* handle) {
    if (!handle) return;
    try {
        MatrixBox* m = mbox(handle);
        tdt::DeviceGuard dg(m->device);
        if (m->many) {
            (void)hipDeviceSynchronize();
        } else {
            for (int i = 0; i < m->nused; ++i) (void)hipStreamSynchronize(m->used[i]);
        }
        free_matrix(*m);
        m->magic = 0;
        delete m;
    } catch (...) {
    }
}

TURBO_DT_API int turbo_int4_matvec_grouped(void* const* matrices, int count, const float* const* x,
                                           float* const* out, void* hip_stream) {
    tdt::set_last_error("");
    MAT_TRY
    if (count < 0 || count > static_cast<int>(tdt::kMaxGroupMats))
        throw std::runtime_error("count must be in 0.." + std::to_string(tdt::kMaxGroupMats));
    if (count == 0) return 1;
    if (!matrices || !x || !out) throw std::runtime_error("matrices, x or out is NULL");
    tdt::GroupArgs a;
    std::memset(&a, 0, sizeof a);
    uint32_t tiles = 0;
    int device = -1;
    for (int i = 0; i < count; ++i) {
        MatrixBox* m = mbox(matrices[i]);
        if (device < 0) device = m->device;
        if (m->device != device) throw std::runtime_error("the matrices of one call must be on one device");
        if (!x[i] || !out[i]) throw std::runtime_error("x[" + std::to_string(i) + "] or out[" + std::to_string(i) + "] is NULL");
        if ((reinterpret_cast<uintptr_t>(x[i]) & 15u) != 0u)
            throw std::runtime_error("x[" + std::to_string(i) + "] must be 16-byte aligned");
        m->note(static_cast<hipStream_t>(hip_stream));
        tdt::GroupMat& g = a.m[i];
        g.Wt = m->Wt;
        g.SBt = m->SBt;
        g.x = x[i];
        g.out = out[i];
        g.rows = m->rows;
        g.D = m->D;
        g.tile_begin = tiles;
        g.ks = tdt::split_waves(m->G, m->ntile);
        if (g.ks == 0u) g.ks = 1u;
        tiles += m->ntile;
    }
    a.count = static_cast<uint32_t>(count);
    tdt::DeviceGuard dg(device);
    tdt::launch_matvec_grouped(a, tiles, static_cast<hipStream_t>(hip_stream));
    return 1;
    MAT_CATCH(0)
}

}  // extern "C"
