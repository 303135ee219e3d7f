// Batched (B > 2) affine-int4 LM head on the matrix cores.
//
// logits[b][v] = sum_c w[v][c] x[b][c],  w = q * s + b  (src/cpu_reference.cpp:55-84)
//
// Design (gfx950):
//  * v_mfma_f32_32x32x16_f16: A = dequantised weights (32 vocabulary rows), B = activations
//    (32 batch rows), fp32 accumulation. Weights are dequantised once per wave in registers:
//    a nibble becomes an exact fp16 through the 0x6400 exponent trick and one v_pk_add_f16,
//    then one v_pk_fma_f16 applies scale and bias, rounding once to fp16 (relative error
//    <= 2^-11; bf16 would be 2^-8 at the same MFMA rate).
//  * High nibbles are extracted in place (w & 0x00F000F0 gives 16 q), so their halves hold
//    16 * round16(q s + b) (bias pre-multiplied by 16) and the matching activation slots hold
//    x / 16. Power-of-two scaling commutes with rounding, so every product is exactly the
//    intended w * x while the dequant costs 13 VALU ops per 8 weights.
//  * Per 64-k group a lane loads one 16-byte chunk per 32-row fragment: lanes 0-31 the chunk
//    2g of rows 0-31, lanes 32-63 the chunk 2g+1 of the same rows (two contiguous 512-byte
//    runs of the tiled layout). MFMA step j consumes word j of the lane's chunk; the
//    activation fragment is read from LDS with the same (chunk, word) mapping, and the
//    activations are stored k-permuted within each octet as (x0, x4, x1, x5, x2, x6, x3, x7)
//    to match the order the dequant produces halves in.
//  * Workgroup = 4 M-waves (4 x 64 rows) x NWN N-waves; a wave owns 64 rows x 32*NB columns.
//    For 64 < B <= 128 one wave per SIMD owns all 128 columns (every weight dequantised once);
//    above, two N-waves of 128 columns share each 64-row tile.
//    Weights are prefetched PF groups ahead into registers; activations for group g+1 are
//    staged through registers into the other half of a double-buffered LDS tile while group g
//    computes, one barrier per group.
//  * Epilogue in place on the accumulators: per (column, 64-row tile), lane-local reductions
//    and one cross-lane exchange give the block partial; logits leave as float4 stores.
#include <hip/hip_ext.h>

#include <stdexcept>
#include <utility>

#include "dt_epilogue.h"

namespace tdt {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr uint32_t kColHalves = 72;  // 64 halves of a group + 8 padding (LDS bank spread)

__device__ inline h2v as_h2(uint32_t u) { return __builtin_bit_cast(h2v, u); }

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// The table is streamed once per step (nontemporal: it does not displace the activations).
__device__ inline uint4 load_stream(const uint4* p) {
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ inline uint32_t load_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }

// 8 nibbles -> 8 halves (e0, e4, 16e1', 16e5', e2, e6, 16e3', 16e7') where e' = q s + b and the
// primed slots carry the factor 16 (bias b16 = 16 b).
__device__ inline h8v dequant_word(uint32_t w, h2v s2, h2v b2, h2v b16) {
    const uint32_t magic = 0x64006400u;  // fp16 1024.0 in both halves
    const h2v off = as_h2(magic);
    const uint32_t w8 = w >> 8;
    const h2v q0 = as_h2((w & 0x000F000Fu) | magic) - off;   // (e0, e4)
    const h2v q1 = as_h2((w & 0x00F000F0u) | magic) - off;   // (16 e1, 16 e5)
    const h2v q2 = as_h2((w8 & 0x000F000Fu) | magic) - off;  // (e2, e6)
    const h2v q3 = as_h2((w8 & 0x00F000F0u) | magic) - off;  // (16 e3, 16 e7)
    const h2v r0 = __builtin_elementwise_fma(q0, s2, b2);
    const h2v r1 = __builtin_elementwise_fma(q1, s2, b16);
    const h2v r2 = __builtin_elementwise_fma(q2, s2, b2);
    const h2v r3 = __builtin_elementwise_fma(q3, s2, b16);
    h8v o;
    o[0] = r0[0]; o[1] = r0[1]; o[2] = r1[0]; o[3] = r1[1];
    o[4] = r2[0]; o[5] = r2[1]; o[6] = r3[0]; o[7] = r3[1];
    return o;
}

// Softcap for the batched path. For |z/cap| < 9 it uses tanh(x) = sign(x)(1 - 2/(exp(2|x|)+1))
// with the hardware exp2/rcp (relative error ~1e-6, far below the fp16-dequant error of this
// path); beyond, tanh rounds to +-1 in fp32, as libm's tanhf does.
__device__ inline float softcap_fast(float z, float cap) {
    const float x = z / cap;
    const float ax = fabsf(x);
    float t = 1.0f;
    if (ax < 9.0f) t = 1.0f - 2.0f / (__expf(2.0f * ax) + 1.0f);
    return cap * copysignf(t, x);
}

// Row held in register r of a 32x32 accumulator by a lane with half hl (0/1): 8(r/4) + 4hl + r%4.
__device__ inline uint32_t acc_row(int r, uint32_t hl) { return 8u * (uint32_t)(r >> 2) + 4u * hl + (uint32_t)(r & 3); }

// OCC = minimum waves per SIMD the register allocation must allow.
template <int NB, int NWN, int PF, int OCC>
__global__ __launch_bounds__(256 * NWN, OCC) void k_head_mfma(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SBt, const uint16_t* __restrict__ x16,
    uint32_t B, uint32_t D, uint32_t NC, uint32_t G, EpiArgs ep) {
    constexpr uint32_t NT = 256 * NWN;
    constexpr uint32_t NCOL = 32 * NB * NWN;
    constexpr uint32_t XP = NCOL * 8;                 // 16-byte activation pieces per group
    constexpr uint32_t XPT = (XP + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) _Float16 lx[2][NCOL * kColHalves];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave & 3u, wn = wave >> 2;
    const uint32_t tile_raw = blockIdx.x * 4u + wm;
    const bool tile_ok = tile_raw < ep.ntile;
    const uint32_t tile = tile_ok ? tile_raw : ep.ntile - 1u;  // clamp loads; skip the epilogue
    const uint32_t hl = lane >> 5, l32 = lane & 31u;

    const uint4* wbase = Wt + (size_t)tile * NC * kTileRows + (size_t)hl * kTileRows + l32;
    const uint32_t* sbbase = SBt + (size_t)tile * G * kTileRows + l32;
    auto wptr = [&](uint32_t g, int mb) { return wbase + (size_t)(2u * g) * kTileRows + 32u * mb; };

    auto load_x = [&](uint32_t g, uint4* xr) {
#pragma unroll
        for (uint32_t p = 0; p < XPT; ++p) {
            const uint32_t pc = tid + p * NT;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (pc < XP) {
                const uint32_t n = pc >> 3, o = pc & 7u;
                if (n < B) v = *reinterpret_cast<const uint4*>(x16 + (size_t)n * D + 64u * g + 8u * o);
            }
            xr[p] = v;
        }
    };
    auto store_x = [&](uint32_t buf, const uint4* xr) {
#pragma unroll
        for (uint32_t p = 0; p < XPT; ++p) {
            const uint32_t pc = tid + p * NT;
            if (pc < XP) {
                const uint32_t n = pc >> 3, o = pc & 7u;
                *reinterpret_cast<uint4*>(&lx[buf][n * kColHalves + 8u * o]) = xr[p];
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

    uint4 wr[PF][2];
    uint32_t sbr[PF][2];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        if ((uint32_t)p < G) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                wr[p][mb] = load_stream(wptr(p, mb));
                sbr[p][mb] = load_stream(sbbase + (size_t)p * kTileRows + 32u * mb);
            }
        }
    }
    uint4 xr[XPT];
    load_x(0, xr);
    store_x(0, xr);
    __syncthreads();

    uint32_t buf = 0;
    for (uint32_t g0 = 0; g0 < G; g0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const uint32_t g = g0 + p;
            if (g < G) {
                uint4 wc[2];
                uint32_t sc[2];
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) { wc[mb] = wr[p][mb]; sc[mb] = sbr[p][mb]; }
                const uint32_t gn = g + PF;
                if (gn < G) {
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) {
                        wr[p][mb] = load_stream(wptr(gn, mb));
                        sbr[p][mb] = load_stream(sbbase + (size_t)gn * kTileRows + 32u * mb);
                    }
                }
                const bool more = g + 1u < G;
                if (more) load_x(g + 1u, xr);
                const _Float16* lb = &lx[buf][0];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    h8v a[2];
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) {
                        const _Float16 s = (_Float16)bf16_to_f32(sc[mb] & 0xFFFFu);
                        const float bfv = bf16_to_f32(sc[mb] >> 16);
                        const _Float16 b = (_Float16)bfv;
                        const _Float16 b16 = (_Float16)(16.0f * bfv);
                        const uint32_t wj = (j == 0) ? wc[mb].x : (j == 1) ? wc[mb].y : (j == 2) ? wc[mb].z : wc[mb].w;
                        a[mb] = dequant_word(wj, h2v{s, s}, h2v{b, b}, h2v{b16, b16});
                    }
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        const uint32_t n = wn * (32u * NB) + 32u * nb + l32;
                        const h8v bv = *reinterpret_cast<const h8v*>(lb + n * kColHalves + 32u * hl + 8u * j);
#pragma unroll
                        for (int mb = 0; mb < 2; ++mb)
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mb], bv, acc[mb][nb], 0, 0, 0);
                    }
                }
                if (more) store_x(buf ^ 1u, xr);
                __syncthreads();
                buf ^= 1u;
            }
        }
    }
    if (!tile_ok) return;

    // ---- epilogue, in place on the accumulators ----
    const uint32_t base = tile * kTileRows;
    const bool vec_ok = (ep.V & 3u) == 0u;  // float4 stores need 16-byte aligned rows
    // One column block at a time, indexed at compile time so the accumulators stay in registers.
    auto column = [&]<int nb>() {
        const uint32_t bcol = wn * (32u * NB) + 32u * nb + l32;
        const bool col_ok = bcol < B;
        const uint32_t bq = col_ok ? bcol : 0u;
        if (ep.cap > 0.0f) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mb][nb][r] = softcap_fast(acc[mb][nb][r], ep.cap);
        }
        if (col_ok && ep.rows[bq].has_mods) {
            const DevRow row = ep.rows[bq];
            // history counts: the two bitmap words of this tile decide which ids to look up
            uint32_t hb[2] = {0u, 0u};
            if ((row.has_mods & 1u) && ep.hcount) {
                const uint32_t* hw = ep.hbits + (size_t)bq * ep.hbw + (base >> 5);
                hb[0] = hw[0];
                if (base + 32u < ep.V) hb[1] = hw[1];
            }
            uint32_t s = 0, e = 0;
            const ModEntry* me = ep.mods + (size_t)bq * ep.mod_cap;
            if ((row.has_mods & 2u) && ep.block_start) {
                const uint32_t* bs = ep.block_start + (size_t)bq * (ep.ntile + 1) + tile;
                s = bs[0];
                e = bs[1];
            }
            if ((hb[0] | hb[1]) != 0u || s < e) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t rr = 32u * mb + acc_row(r, hl);
                        const uint32_t id = base + rr;
                        ModEntry m{id, 0u, 0.0f, 0u};
                        if ((hb[mb] >> (rr & 31u)) & 1u) m.count = ep.hcount[(size_t)bq * ep.V + id];
                        for (uint32_t k = s; k < e; ++k) {
                            const ModEntry t = me[k];
                            if (t.id == id) { m.bias = t.bias; m.has_bias = 1u; }
                        }
                        if (m.count || m.has_bias)
                            acc[mb][nb][r] = apply_entry(acc[mb][nb][r], m, row, ep.rep_limit);
                    }
            }
        }
        uint32_t ban0 = 0u, ban1 = 0u;
        if (col_ok && ep.ban) {
            const uint32_t* bw = ep.ban + (size_t)bq * ep.ban_stride + (base >> 5);
            ban0 = bw[0];
            if (base + 32u < ep.V) ban1 = bw[1];
        }
        float bmax = -INFINITY, bmin = INFINITY;
        uint32_t barg = 0xFFFFFFFFu;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t rr = 32u * mb + acc_row(r, hl);
                float z = acc[mb][nb][r];
                if ((((mb == 0) ? ban0 : ban1) >> (rr & 31u)) & 1u) z = -INFINITY;
                if (base + rr >= ep.V) z = -INFINITY;
                acc[mb][nb][r] = z;
                if (z > bmax) { bmax = z; barg = base + rr; }  // rows visited in increasing order
                if (z != -INFINITY) bmin = fminf(bmin, z);
            }
        bmin = fminf(bmin, __shfl_xor(bmin, 32, 64));
        if (col_ok && ep.logits) {
            float* lrow = ep.logits + (size_t)bq * ep.V + base;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t rr = 32u * mb + 8u * q + 4u * hl;
                    if (vec_ok && base + rr + 3u < ep.V) {
                        *reinterpret_cast<float4*>(lrow + rr) =
                            make_float4(acc[mb][nb][4 * q], acc[mb][nb][4 * q + 1],
                                        acc[mb][nb][4 * q + 2], acc[mb][nb][4 * q + 3]);
                    } else {
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            if (base + rr + t < ep.V) lrow[rr + t] = acc[mb][nb][4 * q + t];
                    }
                }
        }
        const float om = __shfl_xor(bmax, 32, 64);
        const uint32_t oa = (uint32_t)__shfl_xor((int)barg, 32, 64);
        if (om > bmax || (om == bmax && oa < barg)) { bmax = om; barg = oa; }
        float se = 0.0f;
        if (bmax != -INFINITY) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) se += __expf(acc[mb][nb][r] - bmax);
        }
        se += __shfl_xor(se, 32, 64);
        if (col_ok && hl == 0u) {
            BlockPartial bp;
            bp.max = bmax;
            bp.arg = (bmax == -INFINITY) ? base : barg;
            bp.sumexp = se;
            bp.minf = bmin;
            ep.partials[(size_t)bq * ep.ntile + tile] = bp;
        }
    };
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (column.template operator()<I>(), ...);
    }(std::make_integer_sequence<int, NB>{});
}

void launch_head_mfma(const Head& h, int batch, const EpiArgs& ep, hipStream_t st, hipEvent_t ev0,
                      hipEvent_t ev1) {
    const unsigned grid = (h.ntile + 3u) / 4u;
    const uint32_t B = (uint32_t)batch;
#define TDT_LAUNCH(NB, NWN, PF, OCC)                                                           \
    hipExtLaunchKernelGGL((k_head_mfma<NB, NWN, PF, OCC>), dim3(grid), dim3(256 * NWN), 0, st, ev0, \
                          ev1, 0, h.Wt, h.SBt, h.x16, B, h.D, h.NC, h.G, ep)
    if (B <= 32) TDT_LAUNCH(1, 1, 4, 4);
    else if (B <= 64) TDT_LAUNCH(2, 1, 4, 3);
    else if (B <= 128) TDT_LAUNCH(4, 1, 2, 1);
    else if (B <= 256) TDT_LAUNCH(4, 2, 2, 2);
    else throw std::runtime_error("MFMA head supports batch <= 256");
#undef TDT_LAUNCH
    check_hip(hipGetLastError(), "head (MFMA)");
}

}  // namespace tdt
