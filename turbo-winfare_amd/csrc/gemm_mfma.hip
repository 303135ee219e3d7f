// Batched (B > 2) affine-int4 LM head on the matrix cores.
//
// logits[b][v] = sum_c w[v][c] x[b][c],  w = q * s + b  (src/cpu_reference.cpp:55-84)
//
// Design (gfx950):
//  * v_mfma_f32_32x32x16_f16 with A = dequantised weights (32 vocabulary rows), B = activations
//    (32 batch rows), fp32 accumulation. Each weight is dequantised once per workgroup in
//    registers: the nibble becomes an exact fp16 through the 0x6400 exponent trick and one
//    v_pk_add_f16, then w = fma(q, s, b) rounds once to fp16 (relative error <= 2^-11; bf16
//    would be 2^-8 at the same MFMA rate).
//  * A lane loads 8 bytes (two words = 16 k) of one row per 32-k stage; lanes 0-31 take words
//    0-1 and lanes 32-63 words 2-3 of the same 16-byte chunk, so one 32-row fragment is one
//    contiguous 512-byte read of the tiled layout. MFMA step j in a stage consumes word j:
//    lanes 0-31 supply k-octet j, lanes 32-63 octet 2+j. The activation fragment is read from
//    LDS with the same octet mapping, and the activations are stored k-permuted within each
//    octet to match the (e0,e4,e1,e5,e2,e6,e3,e7) order the dequant produces.
//  * Workgroup = 4 M-waves (4 x 64 rows) x NWN N-waves; a wave owns 64 rows x 32*NB columns.
//    Activations for the next 32-k stage are loaded into registers while the current stage
//    computes, then stored to the other half of a double-buffered LDS tile.
//  * Epilogue in the accumulator layout: per (column, 64-row tile) the lane-local values and
//    one cross-lane exchange give the block partial; logits are stored as float4.
#include <stdexcept>

#include "dt_epilogue.h"

namespace tdt {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr uint32_t kLdsColHalves = 40;  // 32 halves of a stage + 8 padding (bank spread)

__device__ inline h2v as_h2(uint32_t u) { return __builtin_bit_cast(h2v, u); }

// Dequantises one weight word (8 nibbles, element order e0..e7) to 8 halves ordered
// (e0,e4,e1,e5,e2,e6,e3,e7): w = q * s + b, one fp16 rounding.
__device__ inline h8v dequant_word(uint32_t w, h2v s2, h2v b2) {
    const uint32_t magic = 0x64006400u;   // fp16 1024.0 in both halves
    const h2v off = as_h2(magic);
    const uint32_t w4 = w >> 4, w8 = w >> 8, w12 = w >> 12;
    const h2v q0 = as_h2((w & 0x000F000Fu) | magic) - off;    // (e0, e4)
    const h2v q1 = as_h2((w4 & 0x000F000Fu) | magic) - off;   // (e1, e5)
    const h2v q2 = as_h2((w8 & 0x000F000Fu) | magic) - off;   // (e2, e6)
    const h2v q3 = as_h2((w12 & 0x000F000Fu) | magic) - off;  // (e3, e7)
    const h2v r0 = __builtin_elementwise_fma(q0, s2, b2);
    const h2v r1 = __builtin_elementwise_fma(q1, s2, b2);
    const h2v r2 = __builtin_elementwise_fma(q2, s2, b2);
    const h2v r3 = __builtin_elementwise_fma(q3, s2, b2);
    h8v o;
    o[0] = r0[0]; o[1] = r0[1]; o[2] = r1[0]; o[3] = r1[1];
    o[4] = r2[0]; o[5] = r2[1]; o[6] = r3[0]; o[7] = r3[1];
    return o;
}

__device__ inline void sb_pair(uint32_t sb, h2v* s2, h2v* b2) {
    const _Float16 s = (_Float16)bf16_to_f32(sb & 0xFFFFu);
    const _Float16 b = (_Float16)bf16_to_f32(sb >> 16);
    *s2 = h2v{s, s};
    *b2 = h2v{b, b};
}

// Softcap for the batched path. For |z/cap| < 9 it uses tanh(x) = sign(x)(1 - 2/(exp(2|x|)+1))
// with the hardware exp2/rcp (relative error ~1e-6, far below the fp16-dequant error of this
// path); beyond, tanh rounds to +-1 in fp32, as libm's tanhf does.
__device__ inline float softcap_fast(float z, float cap) {
    const float x = z / cap;
    const float ax = fabsf(x);
    float t;
    if (ax >= 9.0f) t = 1.0f;
    else {
        const float e = __expf(2.0f * ax);
        t = 1.0f - 2.0f / (e + 1.0f);
    }
    return cap * copysignf(t, x);
}

template <int NB, int NWN>
__global__ __launch_bounds__(256 * NWN) void k_head_mfma(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SBt, const uint16_t* __restrict__ x16,
    uint32_t B, uint32_t D, uint32_t NC, uint32_t G, EpiArgs ep) {
    constexpr uint32_t NT = 256 * NWN;           // threads
    constexpr uint32_t NCOL = 32 * NB * NWN;     // columns held by the workgroup
    constexpr uint32_t PIECES = NCOL * 4;        // 16-byte activation pieces per stage
    constexpr uint32_t PPT = (PIECES + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) _Float16 lx[2][NCOL * kLdsColHalves];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave & 3u, wn = wave >> 2;
    const uint32_t tile_raw = blockIdx.x * 4u + wm;
    const bool tile_ok = tile_raw < ep.ntile;
    const uint32_t tile = tile_ok ? tile_raw : ep.ntile - 1u;  // clamp loads; skip the epilogue
    const uint32_t hl = lane >> 5, l32 = lane & 31u;

    // weight fragment pointers: row 32mb + l32 of the tile, 8 bytes at offset 8*hl of the chunk
    const uint2* wbase = reinterpret_cast<const uint2*>(Wt + (size_t)tile * NC * kTileRows) + hl;
    const uint32_t* sbbase = SBt + (size_t)tile * G * kTileRows + l32;

    auto load_w = [&](uint32_t c, uint32_t mb) -> uint2 {
        return wbase[((size_t)c * kTileRows + 32u * mb + l32) * 2u];
    };
    auto load_x = [&](uint32_t c, uint4* xr) {
#pragma unroll
        for (uint32_t p = 0; p < PPT; ++p) {
            const uint32_t pc = tid + p * NT;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (pc < PIECES) {
                const uint32_t n = pc >> 2, o = pc & 3u;
                if (n < B) v = *reinterpret_cast<const uint4*>(x16 + (size_t)n * D + 32u * c + 8u * o);
            }
            xr[p] = v;
        }
    };
    auto store_x = [&](uint32_t buf, const uint4* xr) {
#pragma unroll
        for (uint32_t p = 0; p < PPT; ++p) {
            const uint32_t pc = tid + p * NT;
            if (pc < PIECES) {
                const uint32_t n = pc >> 2, o = pc & 3u;
                *reinterpret_cast<uint4*>(&lx[buf][n * kLdsColHalves + 8u * o]) = xr[p];
            }
        }
    };

    f16v acc[2][NB];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

    uint4 xr[PPT];
    load_x(0, xr);
    store_x(0, xr);
    uint2 wc[2] = {load_w(0, 0), load_w(0, 1)};
    uint32_t sbc[2] = {sbbase[0], sbbase[32]};
    __syncthreads();

    for (uint32_t c = 0; c < NC; ++c) {
        const uint32_t buf = c & 1u;
        const bool more = (c + 1u) < NC;
        uint2 wn2[2] = {wc[0], wc[1]};
        uint32_t sbn[2] = {sbc[0], sbc[1]};
        if (more) {
            wn2[0] = load_w(c + 1u, 0);
            wn2[1] = load_w(c + 1u, 1);
            if (((c + 1u) & 1u) == 0u) {
                const uint32_t g = (c + 1u) >> 1;
                sbn[0] = sbbase[(size_t)g * kTileRows];
                sbn[1] = sbbase[(size_t)g * kTileRows + 32u];
            }
            load_x(c + 1u, xr);
        }
        h8v a[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            h2v s2, b2;
            sb_pair(sbc[mb], &s2, &b2);
            a[mb][0] = dequant_word(wc[mb].x, s2, b2);
            a[mb][1] = dequant_word(wc[mb].y, s2, b2);
        }
        const _Float16* lb = &lx[buf][0];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const uint32_t n = wn * (32u * NB) + 32u * nb + l32;
                const h8v bv = *reinterpret_cast<const h8v*>(lb + n * kLdsColHalves + 8u * (j + 2u * hl));
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mb][j], bv, acc[mb][nb], 0, 0, 0);
            }
        }
        if (more) store_x(buf ^ 1u, xr);
        __syncthreads();
        wc[0] = wn2[0];
        wc[1] = wn2[1];
        sbc[0] = sbn[0];
        sbc[1] = sbn[1];
    }
    if (!tile_ok) return;

    // ---- epilogue in the accumulator layout ----
    // acc[mb][nb][r] holds row 32mb + 8(r/4) + 4hl + (r%4) of the tile, column 32nb + l32 of
    // this wave's column range.
    const uint32_t base = tile * kTileRows;
    const bool vec_ok = (ep.V & 3u) == 0u;  // float4 stores need 16-byte aligned rows
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const uint32_t bcol = wn * (32u * NB) + 32u * nb + l32;
        const bool col_ok = bcol < B;
        const uint32_t bq = col_ok ? bcol : 0u;
        const DevRow& row = ep.rows[bq];
        float v[32];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float z = acc[mb][nb][r];
                if (ep.cap > 0.0f) z = softcap_fast(z, ep.cap);
                v[mb * 16 + r] = z;
            }
        if (col_ok && row.has_mods && ep.block_start) {
            const uint32_t* bs = ep.block_start + (size_t)bq * (ep.ntile + 1) + tile;
            const uint32_t s = bs[0], e = bs[1];
            const ModEntry* me = ep.mods + (size_t)bq * ep.mod_cap;
            for (uint32_t k = s; k < e; ++k) {
                const ModEntry m = me[k];
                const uint32_t ro = m.id - base;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t rr = 32u * mb + 8u * (r >> 2) + 4u * hl + (r & 3);
                        if (rr == ro) v[mb * 16 + r] = apply_entry(v[mb * 16 + r], m, row, ep.rep_limit);
                    }
            }
        }
        uint32_t ban0 = 0u, ban1 = 0u;
        if (col_ok && ep.ban) {
            const uint32_t* bw = ep.ban + (size_t)bq * ep.ban_stride + (base >> 5);
            ban0 = bw[0];
            if (base + 32u < ep.V) ban1 = bw[1];
        }
        float bmax = -INFINITY;
        uint32_t barg = 0xFFFFFFFFu;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t rr = 32u * mb + 8u * (r >> 2) + 4u * hl + (r & 3);
                const uint32_t id = base + rr;
                float z = v[mb * 16 + r];
                if (((rr < 32u ? ban0 : ban1) >> (rr & 31u)) & 1u) z = -INFINITY;
                if (id >= ep.V) z = -INFINITY;
                v[mb * 16 + r] = z;
                if (z > bmax || (z == bmax && id < barg)) { bmax = z; barg = id; }
            }
        if (col_ok && ep.logits) {
            float* lrow = ep.logits + (size_t)bq * ep.V + base;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t rr = 32u * mb + 8u * q + 4u * hl;
                    if (vec_ok && base + rr + 3u < ep.V) {
                        *reinterpret_cast<float4*>(lrow + rr) =
                            make_float4(v[mb * 16 + 4 * q], v[mb * 16 + 4 * q + 1],
                                        v[mb * 16 + 4 * q + 2], v[mb * 16 + 4 * q + 3]);
                    } else {
                        for (int t = 0; t < 4; ++t)
                            if (base + rr + t < ep.V) lrow[rr + t] = v[mb * 16 + 4 * q + t];
                    }
                }
        }
        // combine with the partner lane holding the other half of the 64 rows
        const float om = __shfl_xor(bmax, 32, 64);
        const uint32_t oa = (uint32_t)__shfl_xor((int)barg, 32, 64);
        if (om > bmax || (om == bmax && oa < barg)) { bmax = om; barg = oa; }
        float se = 0.0f;
        if (bmax != -INFINITY) {
#pragma unroll
            for (int i = 0; i < 32; ++i) se += __expf(v[i] - bmax);
        }
        se += __shfl_xor(se, 32, 64);
        if (col_ok && hl == 0u) {
            BlockPartial bp;
            bp.max = bmax;
            bp.arg = barg;
            bp.sumexp = se;
            bp.pad = 0u;
            ep.partials[(size_t)bq * ep.ntile + tile] = bp;
        }
    }
}

void launch_head_mfma(const Head& h, int batch, const EpiArgs& ep, hipStream_t st) {
    const unsigned grid = (h.ntile + 3u) / 4u;
    const uint32_t B = (uint32_t)batch;
#define TDT_LAUNCH(NB, NWN)                                                                   \
    hipLaunchKernelGGL((k_head_mfma<NB, NWN>), dim3(grid), dim3(256 * NWN), 0, st, h.Wt, h.SBt, \
                       h.x16, B, h.D, h.NC, h.G, ep)
    if (B <= 32) TDT_LAUNCH(1, 1);
    else if (B <= 64) TDT_LAUNCH(2, 1);
    else if (B <= 128) TDT_LAUNCH(4, 1);
    else if (B <= 256) TDT_LAUNCH(4, 2);
    else throw std::runtime_error("MFMA head supports batch <= 256");
#undef TDT_LAUNCH
    check_hip(hipGetLastError(), "head (MFMA)");
}

}  // namespace tdt
