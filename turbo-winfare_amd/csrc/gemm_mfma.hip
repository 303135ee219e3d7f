// Batched (B > 2) affine-int4 LM head on the matrix cores.
//
// logits[b][v] = sum_c w[v][c] x[b][c],  w = q * s + b  (src/cpu_reference.cpp:55-84)
//
// Design (gfx950):
//  * v_mfma_f32_32x32x16_f16: A = dequantised weights (32 vocabulary rows), B = activations
//    (32 batch rows), fp32 accumulation. Weights are dequantised once per wave in registers
//    (dequant_word, dt_mfma.h): q s + b rounded once to fp16 (relative error <= 2^-11; bf16
//    would be 2^-8 at the same MFMA rate), from nibbles masked into fp16 denormals when every
//    scale is below 1/16 (9 VALU ops per 8 weights), else through the mantissa of 1024.0 (13).
//  * Per 64-k group a lane loads one 16-byte chunk per 32-row fragment: lanes 0-31 the chunk
//    2g of rows 0-31, lanes 32-63 the chunk 2g+1 of the same rows (two contiguous 512-byte
//    runs of the tiled layout). MFMA step j consumes word j of the lane's chunk; the
//    activation fragment is read from LDS with the same (chunk, word) mapping, and the
//    activations are stored k-permuted within each octet as (x0, x4, x1, x5, x2, x6, x3, x7)
//    to match the order the dequant produces halves in.
//  * Workgroup = 4 waves, one 64-row tile each, over a block of 32*NB batch columns
//    (B = 256 runs two column blocks, on the same XCD back to back so the second reads the
//    weights from L2). Weights and activations are prefetched PF
//    groups ahead into registers; the activations of group g+1 are written into the other half
//    of a double-buffered LDS tile at the end of group g, one barrier per group.
//  * Epilogue in place on the accumulators: per (column, 64-row tile), lane-local reductions
//    and one cross-lane exchange give the block partial; logits leave as float4 stores.
#include <hip/hip_ext.h>

#include <stdexcept>
#include <utility>

#include "dt_mfma.h"

namespace tdt {

// Workgroup = 4 waves, one 64-row tile each, over a block of NCOL = 32 NB batch columns
// (the column block). Two or more independent workgroups share a CU, so one's epilogue overlaps
// another's main loop and their barriers do not line up.
// FULL: every column of the block exists (B % NCOL == 0): activation loads need no guard.
// The main loop runs in rounds of PF groups (G % PF == 0) without branches: loads past the
// last group are clamped to it and never used, so the compiler's load counters stay exact and
// the weight prefetch is never drained early. The next k-step's weights are dequantised in
// the shadow of the current step's MFMAs.
template <int NB, int PF, int OCC, bool FULL, bool DENORM>
__global__ __launch_bounds__(256, OCC) void k_head_mfma(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SB16t,
    const uint16_t* __restrict__ x16, uint32_t B, uint32_t D, uint32_t NC, uint32_t G, uint32_t ncb, uint32_t ntg, EpiArgs ep) {
    constexpr uint32_t NT = 256;
    constexpr uint32_t NCOL = 32 * NB;
    constexpr uint32_t XP = NCOL * 8;                 // 16-byte activation pieces per group
    constexpr uint32_t XPT = XP / NT;
    static_assert(XP % NT == 0, "activation pieces must split evenly over the threads");
    __shared__ __attribute__((aligned(16))) _Float16 lx[2][NCOL * kColHalves];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // Workgroup i is dispatched to XCD i % 8. The ncb column blocks of one group of four tiles go
    // to workgroups i, i + 8, ... of the same XCD, dispatched back to back, so every block after
    // the first finds the tiles' weights in that XCD's L2 instead of reading HBM again.
    const uint32_t wg = blockIdx.x, xcd = wg & 7u, slot = wg >> 3;
    const uint32_t tg = (slot / ncb) * 8u + xcd;
    if (tg >= ntg) return;                            // padding: ntg rounded up to 8
    const uint32_t cbase = (slot % ncb) * NCOL;       // first batch column of this workgroup
    const uint32_t tile_raw = tg * 4u + wave;
    const bool tile_ok = tile_raw < ep.ntile;
    const uint32_t tile = tile_ok ? tile_raw : ep.ntile - 1u;  // clamp loads; skip the epilogue
    const uint32_t hl = lane >> 5, l32 = lane & 31u;

    const uint4* wbase = Wt + (size_t)tile * NC * kTileRows + (size_t)hl * kTileRows + l32;
    const uint32_t* sbbase = SB16t + (size_t)tile * G * kTileRows + l32;
    auto wload = [&](uint32_t g, int mb) { return mfma_load_stream(wbase + (size_t)(2u * g) * kTileRows + 32u * mb); };
    auto sload = [&](uint32_t g, int mb) { return mfma_load_stream(sbbase + (size_t)g * kTileRows + 32u * mb); };
    const uint32_t magic = DENORM ? 0u : magic_vgpr();

    auto load_x = [&](uint32_t g, v4u* xr) {
#pragma unroll
        for (uint32_t p = 0; p < XPT; ++p) {
            const uint32_t pc = tid + p * NT;
            const uint32_t n = cbase + (pc >> 3), o = pc & 7u;
            if constexpr (FULL) {
                xr[p] = *reinterpret_cast<const v4u*>(x16 + (size_t)n * D + 64u * g + 8u * o);
            } else {
                v4u v = {0u, 0u, 0u, 0u};
                if (n < B) v = *reinterpret_cast<const v4u*>(x16 + (size_t)n * D + 64u * g + 8u * o);
                xr[p] = v;
            }
        }
    };
    auto store_x = [&](uint32_t buf, const v4u* xr) {
#pragma unroll
        for (uint32_t p = 0; p < XPT; ++p) {
            const uint32_t pc = tid + p * NT;
            *reinterpret_cast<v4u*>(&lx[buf][(pc >> 3) * kColHalves + 8u * (pc & 7u)]) = xr[p];
        }
    };

    f16v acc[2][NB];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

    // Weights and activations are prefetched PF groups ahead in the same slots, in the same
    // order: the load counter is in-order, so waiting for a group's activations (at the LDS
    // store) only waits for loads that the next group needs anyway.
    uint4 wr[PF][2];
    uint32_t sbr[PF][2];
    v4u xr[PF][XPT];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        const uint32_t gp = min((uint32_t)p, G - 1u);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) { wr[p][mb] = wload(gp, mb); sbr[p][mb] = sload(gp, mb); }
        load_x(gp, xr[p]);
    }
    store_x(0, xr[0]);
    __syncthreads();

    h8v acur[2], anext[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const SbHalves h = unpack_sb16<DENORM>(sbr[0][mb]);
        acur[mb] = dequant_word<DENORM>(wr[0][mb].x, h.s2, h.b2, h.bx, magic);
    }
    uint32_t buf = 0;
    for (uint32_t g0 = 0; g0 < G; g0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const uint32_t g = g0 + p;
            uint4 wc[2];
            SbHalves hc[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) { wc[mb] = wr[p][mb]; hc[mb] = unpack_sb16<DENORM>(sbr[p][mb]); }
            // slot p held group g, whose activations are already in LDS: refill it with g + PF
            const uint32_t gn = min(g + (uint32_t)PF, G - 1u);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) { wr[p][mb] = wload(gn, mb); sbr[p][mb] = sload(gn, mb); }
            load_x(gn, xr[p]);
            constexpr int kNext = (PF > 1) ? 1 : 0;
            const int pn = (p + kNext) % PF;         // prefetch slot holding group g + 1
            const _Float16* lb = &lx[buf][0];
            // with four column blocks the activation fragments are read one (j, nb) ahead of their
            // MFMAs, so no MFMA pair waits for the LDS read just issued (measured 1.7 % faster
            // there; not at one column block)
            auto bfrag = [&](int j, int nb) {
                return *reinterpret_cast<const h8v*>(lb + (32u * (uint32_t)nb + l32) * kColHalves + 32u * hl + 8u * (uint32_t)j);
            };
            constexpr bool kAhead = NB == 4 && FULL;  // (the partial-column variant would spill)
            h8v bcur = bfrag(0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    if (j < 3) {
                        anext[mb] = dequant_word<DENORM>(word_of(wc[mb], j + 1), hc[mb].s2, hc[mb].b2, hc[mb].bx, magic);
                    } else {
                        const SbHalves h = unpack_sb16<DENORM>(sbr[pn][mb]);
                        anext[mb] = dequant_word<DENORM>(wr[pn][mb].x, h.s2, h.b2, h.bx, magic);
                    }
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    h8v bv, bnext = bcur;
                    if constexpr (kAhead) {
                        bv = bcur;
                        if (nb + 1 < NB) bnext = bfrag(j, nb + 1);
                        else if (j < 3) bnext = bfrag(j + 1, 0);
                    } else {
                        bv = bfrag(j, nb);
                    }
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(acur[mb], bv, acc[mb][nb], 0, 0, 0);
                    bcur = bnext;
                }
                // one LDS read, one MFMA, then dequant VALU work in the MFMA's shadow
#pragma unroll
                for (int i = 0; i < 2 * NB; ++i) {
                    if (i < NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, (NB >= 4) ? 5 : (NB == 2 ? 9 : 17), 0);
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) acur[mb] = anext[mb];
            }
            store_x(buf ^ 1u, xr[(p + 1) % PF]);  // group g + 1 (clamped), loaded PF - 1 groups ago
            __syncthreads();
            buf ^= 1u;
        }
    }
    if (!tile_ok) return;

    // ---- epilogue, in place on the accumulators ----
    // The transposed logit stores (four column blocks) reuse the activation buffer: one
    // 32 x kTrRow float tile per wave, after every wave's last read of it (the main loop ends
    // with a barrier).
    constexpr bool kTransposeStores = NB == 4;
    static_assert(!kTransposeStores || sizeof(lx) >= 4u * 32u * kTrRow * sizeof(float),
                  "four wave tiles must fit the activation buffer");
    float* epi_tl = reinterpret_cast<float*>(&lx[0][0]) + wave * (32u * kTrRow);
    const uint32_t base = tile * kTileRows;
    const bool vec_ok = (ep.V & 3u) == 0u;  // float4 stores need 16-byte aligned rows
    const bool full_tile = base + kTileRows <= ep.V;
    const float inv_cap = (ep.cap > 0.0f) ? 1.0f / ep.cap : 0.0f;
    // One column block at a time, indexed at compile time so the accumulators stay in registers.
    auto column = [&]<int nb>() {
        const uint32_t bcol = cbase + 32u * nb + l32;
        const bool col_ok = bcol < B;
        const uint32_t bq = col_ok ? bcol : 0u;
        if (ep.cap > 0.0f) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mb][nb][r] = softcap_fast(acc[mb][nb][r], ep.cap, inv_cap);
        }
        if (col_ok && ep.rows[bq].has_mods) {
            const DevRow row = ep.rows[bq];
            // history counts: the two bitmap words of this tile decide which ids to look up
            // (both halves of the column read them; the low half zeroes them for the next step)
            uint32_t hb[2] = {0u, 0u};
            if ((row.has_mods & 1u) && ep.hcount) {
                uint32_t* hw = ep.hbits + (size_t)bq * ep.hbw + (base >> 5);
                hb[0] = hw[0];
                if (base + 32u < ep.V) hb[1] = hw[1];
                if (hl == 0u && hb[0] != 0u) hw[0] = 0u;
                if (hl == 0u && hb[1] != 0u) hw[1] = 0u;
            }
            uint32_t s = 0, e = 0;
            const ModEntry* me = ep.mods + (size_t)bq * ep.mod_cap;
            if ((row.has_mods & 2u) && ep.block_start) {
                const uint32_t* bs = ep.block_start + (size_t)bq * (ep.ntile + 1) + tile;
                s = bs[0];
                e = bs[1];
            }
            // bias first (the order of apply_entry): entries are unique per id, so each is read
            // once and added to the one register that holds its id, if this lane holds it
            for (uint32_t k = s; k < e; ++k) {
                const ModEntry t = me[k];
                const uint32_t rr = t.id - base;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (rr == 32u * mb + acc_row(r, hl)) {
#pragma clang fp contract(off)
                            acc[mb][nb][r] = acc[mb][nb][r] + t.bias;
                        }
            }
            // history counts: all loads of a 32-row half are issued before any is consumed, then
            // each read count is zeroed for the next step and applied
            if ((hb[0] | hb[1]) != 0u) {
                uint32_t* hrow = ep.hcount + (size_t)bq * ep.V + base;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    if (hb[mb] == 0u) continue;
                    uint32_t cnt[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t rr = 32u * mb + acc_row(r, hl);
                        cnt[r] = ((hb[mb] >> (rr & 31u)) & 1u) ? hrow[rr] : 0u;
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (cnt[r]) {
                            const uint32_t rr = 32u * mb + acc_row(r, hl);
                            hrow[rr] = 0u;
                            acc[mb][nb][r] = apply_entry(acc[mb][nb][r], ModEntry{base + rr, cnt[r], 0.0f, 0u}, row,
                                                         ep.rep_limit);
                        }
                }
            }
        }
        if (col_ok && ep.ban) {
            const uint32_t* bw = ep.ban + (size_t)bq * ep.ban_stride + (base >> 5);
            const uint32_t ban0 = bw[0];
            const uint32_t ban1 = (base + 32u < ep.V) ? bw[1] : 0u;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t rr = 32u * mb + acc_row(r, hl);
                    if ((((mb == 0) ? ban0 : ban1) >> (rr & 31u)) & 1u) acc[mb][nb][r] = -INFINITY;
                }
        }
        if (!full_tile) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (base + 32u * mb + acc_row(r, hl) >= ep.V) acc[mb][nb][r] = -INFINITY;
        }
        float bmax = -INFINITY, bmin = INFINITY, bsec = -INFINITY;  // bsec: second largest, with repeats
        uint32_t barg = 0xFFFFFFFFu;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float z = acc[mb][nb][r];
                if (z > bmax) {  // rows in increasing order
                    bsec = bmax;
                    bmax = z;
                    barg = base + 32u * mb + acc_row(r, hl);
                } else {
                    bsec = fmaxf(bsec, z);
                }
                if (z != -INFINITY) bmin = fminf(bmin, z);
            }
        bmin = fminf(bmin, xor32(bmin));
        // Logits: with four column blocks (B = 256) the activation buffer is free after the main
        // loop, and each wave transposes its 64 x 32 tile through its own 8.5 KiB of it, so that
        // one float4 store covers four whole 256-byte row segments instead of 16 bytes of 32
        // rows. Otherwise (and for partial tiles or columns) the values leave as they lie.
        if (kTransposeStores && ep.logits && full_tile && vec_ok && cbase + 32u * nb + 32u <= B) {
            float* tl = epi_tl;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<float4*>(tl + l32 * kTrRow + 32u * mb + 8u * q + 4u * hl) =
                        make_float4(acc[mb][nb][4 * q], acc[mb][nb][4 * q + 1], acc[mb][nb][4 * q + 2],
                                    acc[mb][nb][4 * q + 3]);
            const uint32_t c0 = lane >> 4, r4 = 4u * (lane & 15u);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = 4u * (uint32_t)i + c0;  // column of the tile
                const float4 v = *reinterpret_cast<const float4*>(tl + c * kTrRow + r4);
                *reinterpret_cast<float4*>(ep.logits + (size_t)(cbase + 32u * nb + c) * ep.V + base + r4) = v;
            }
        } else if (col_ok && ep.logits) {
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
        const float om = xor32(bmax);
        const uint32_t oa = xor32(barg);
        // second largest of the two halves together: the smaller maximum or the larger second
        bsec = fmaxf(fmaxf(bsec, xor32(bsec)), fminf(bmax, om));
        if (om > bmax || (om == bmax && oa < barg)) { bmax = om; barg = oa; }
        float se = 0.0f;
        if (bmax != -INFINITY && !ep.no_sumexp) {
            const float mb2 = bmax * 1.4426950408889634f;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    se += __builtin_amdgcn_exp2f(fmaf(acc[mb][nb][r], 1.4426950408889634f, -mb2));
        }
        se += xor32(se);
        if (col_ok && hl == 0u) {
            BlockPartial bp;
            bp.max = bmax;
            bp.arg = (bmax == -INFINITY) ? base : barg;
            bp.sumexp = se;
            bp.minf = bmin;
            bp.smax = bsec;
            ep.partials[(size_t)bq * ep.ntile + tile] = bp;
        }
    };
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (column.template operator()<I>(), ...);
    }(std::make_integer_sequence<int, NB>{});
}

void launch_head_mfma(const Head& h, int batch, const EpiArgs& ep, hipStream_t st, hipEvent_t ev0,
                      hipEvent_t ev1) {
    const uint32_t B = (uint32_t)batch;
    if (B > 256u) throw std::runtime_error("MFMA head supports batch <= 256");
    const int nb = (B <= 32u) ? 1 : (B <= 64u) ? 2 : 4;
    const uint32_t ncol = 32u * (uint32_t)nb;
    const uint32_t ntg = (h.ntile + 3u) / 4u, ncb = (B + ncol - 1u) / ncol;
    const dim3 grid(ncb * ((ntg + 7u) / 8u) * 8u);
    const bool full = (B % ncol) == 0u;
    const bool pf2 = (h.G % 2u) == 0u;
#define TDT_LAUNCH(NB, PF, OCC, FULL, DN)                                                           \
    hipExtLaunchKernelGGL((k_head_mfma<NB, PF, OCC, FULL, DN>), grid, dim3(256), 0, st, ev0, ev1, 0, h.Wt, \
                          h.SB16t, h.x16, B, h.D, h.NC, h.G, ncb, ntg, ep)
#define TDT_PICK2(NB, OCC, DN)                                                                     \
    do {                                                                                           \
        if (pf2) { if (full) TDT_LAUNCH(NB, 2, OCC, true, DN); else TDT_LAUNCH(NB, 2, OCC, false, DN); } \
        else { if (full) TDT_LAUNCH(NB, 1, OCC, true, DN); else TDT_LAUNCH(NB, 1, OCC, false, DN); }     \
    } while (0)
#define TDT_PICK(NB, OCC)                                   \
    do {                                                    \
        if (h.mfma_denorm) TDT_PICK2(NB, OCC, true);        \
        else TDT_PICK2(NB, OCC, false);                     \
    } while (0)
    if (nb == 1) TDT_PICK(1, 4);
    else if (nb == 2) TDT_PICK(2, 3);
    else TDT_PICK(4, 2);
#undef TDT_PICK
#undef TDT_PICK2
#undef TDT_LAUNCH
    check_hip(hipGetLastError(), "head (MFMA)");
}

}  // namespace tdt
