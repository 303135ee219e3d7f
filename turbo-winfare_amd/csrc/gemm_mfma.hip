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
//  * Workgroup = WV waves, one 64-row tile each, over a block of 32*NB batch columns
//    (B = 256 runs two column blocks, on the same XCD back to back so the second reads the
//    weights from L2). At 64 columns one 16-wave workgroup per CU shares each activation stage
//    among all 16 tiles; otherwise 4-wave workgroups run several to a CU. Weights and scales are prefetched PF groups ahead into registers by
//    buffer loads; the activations reach a ring in LDS by buffer-to-LDS DMA, PF - 1 groups
//    ahead, a group's DMA instructions spread over its k-steps, with one wait and one barrier
//    per group.
//  * Epilogue in place on the accumulators: a row whose activations were stored scaled by 2^-k
//    (its largest |x| above 2^11, step prep) has its accumulators multiplied by 2^k first; then
//    per (column, 64-row tile), lane-local reductions and one cross-lane exchange give the block
//    partial; logits leave as float4 stores.
#include <hip/hip_ext.h>

#include <stdexcept>
#include <type_traits>
#include <utility>

#include "dt_mfma.h"

namespace tdt {

// Workgroup = WV waves, one 64-row tile each, over a block of NCOL = 32 NB batch columns
// (the column block). With WV = 4, two or more independent workgroups share a CU, so one's
// epilogue overlaps another's main loop and their barriers do not line up. With WV = 16 (64
// columns) the CU's one workgroup stages each group's activations once for its 16 tiles, a
// quarter of the LDS fill and L2 reads of four 4-wave workgroups (B = 64 head 136 -> 125 us;
// at 32 columns the same change measured 6 us slower, and 8 waves 2 - 5 us slower).
// Columns past the batch read zeros (their DMA source lies past the buffer's end).
// The main loop runs in rounds of PF groups (G % PF == 0) without branches: loads past the
// last group are clamped to it and never used, so the compiler's load counters stay exact and
// the weight prefetch is never drained early. The next k-step's weights are dequantised in
// the shadow of the current step's MFMAs.
// META: some row has modifiers or a ban mask; the workgroup's per-(tile, column) modifier words
// are then staged in LDS before the main loop (their loads issue ahead of the weight stream), so
// the epilogue reads them from LDS instead of waiting on global loads.
template <int NB, int WV, int PF, int OCC, bool DENORM, bool META>
__global__ __launch_bounds__(64 * WV, OCC) void k_head_mfma(
    const uint4* __restrict__ Wt, const uint32_t* __restrict__ SB16t,
    const uint16_t* __restrict__ x16, uint32_t B, uint32_t D, uint32_t NC, uint32_t G, uint32_t ncb, uint32_t ntg, EpiArgs ep) {
    constexpr uint32_t NT = 64u * WV;
    constexpr uint32_t NCOL = 32 * NB;
    // Activations: group g (NCOL columns x 64 halves) lives in stage g % NST of a ring in LDS,
    // written by buffer-to-LDS DMA PF - 1 groups ahead (no registers, no LDS store instructions).
    // Column c holds its eight 16-byte pieces p at slot c * 8 + (p ^ ((c >> 1) & 7)): the MFMA's
    // fragment reads (16 lanes = 16 consecutive columns, one piece) then hit 64 distinct banks.
    constexpr uint32_t kStage = NCOL * 128u;
    constexpr uint32_t NST = PF > 1 ? PF : 2;
    // A stage is kRows 1 KiB rows, one DMA instruction each; row r is issued by wave r % WV
    // (with fewer rows than waves, the first kRows waves issue one each and the rest none).
    constexpr uint32_t kRows = kStage / 1024u;
    constexpr uint32_t XDMA = (kRows + WV - 1u) / WV;  // DMA instructions per wave per group
    static_assert(kStage % 1024u == 0u && (kRows % WV == 0u || kRows < WV), "a stage splits into whole DMA rows per wave");
    constexpr uint32_t kXBytes = NST * kStage;
    constexpr uint32_t kTrBytes = (uint32_t)WV * kTrHalfFloats * 4u;  // the epilogue's transposed half tiles, one per wave
    constexpr uint32_t kPoolBytes = kXBytes > kTrBytes ? kXBytes : kTrBytes;
    constexpr uint32_t kLdsBytes = kPoolBytes + (META ? (uint32_t)sizeof(EpiMeta<WV, NCOL>) : 0u);
    __shared__ __attribute__((aligned(16))) unsigned char pool[kLdsBytes];
    EpiMeta<WV, NCOL>& meta = *reinterpret_cast<EpiMeta<WV, NCOL>*>(pool + kPoolBytes);  // used only when META

    // the wave index is uniform: in a scalar register, the DMA's LDS addresses (M0) and the tile
    // offsets are scalar arithmetic, with no readfirstlane per DMA and no VGPRs holding them
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroup i is dispatched to XCD i % 8. The ncb column blocks of one group of WV tiles go
    // to workgroups i, i + 8, ... of the same XCD, dispatched back to back, so every block after
    // the first finds the tiles' weights in that XCD's L2 instead of reading HBM again.
    const uint32_t wg = blockIdx.x, xcd = wg & 7u, slot = wg >> 3;
    const uint32_t tg = (slot / ncb) * 8u + xcd;
    if (tg >= ntg) return;                            // padding: ntg rounded up to 8
    const uint32_t cbase = (slot % ncb) * NCOL;       // first batch column of this workgroup
    const uint32_t tile_raw = tg * (uint32_t)WV + wave;
    const bool tile_ok = tile_raw < ep.ntile;
    const uint32_t tile = tile_ok ? tile_raw : ep.ntile - 1u;  // clamp loads; skip the epilogue
    const uint32_t hl = lane >> 5, l32 = lane & 31u;

    // Weights and scales through buffer loads: a per-lane byte offset plus the group's offset in
    // an SGPR, so no address arithmetic runs per load.
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(Wt), 0, ep.ntile * NC * kTileRows * 16u, kBufDword3);
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(SB16t), 0, ep.ntile * G * kTileRows * 4u, kBufDword3);
    const uint32_t woff = ((tile * NC + hl) * kTileRows + l32) * 16u;
    const uint32_t soff = (tile * G * kTileRows + l32) * 4u;
    auto wload = [&](uint32_t g, int mb) { return buf_load_b128(wrs, woff + 512u * (uint32_t)mb, g * 2048u); };
    auto sload = [&](uint32_t g, int mb) { return buf_load_b32(srs, soff + 128u * (uint32_t)mb, g * 256u); };
    const uint32_t magic = DENORM ? 0u : magic_vgpr();

    // The DMA sources of this thread's pieces: instruction i of wave w fills row WV i + w, slots
    // (WV i + w) * 64 + lane of a stage. Columns past the batch read past the buffer's end (zeros).
    auto dma_row = [&](uint32_t i) { return (uint32_t)WV * i + wave; };
    auto dma_on = [&](uint32_t i) { return kRows % WV == 0u || dma_row(i) < kRows; };  // uniform
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x16), 0, B * D * 2u, kBufDword3);
    uint32_t xoff[XDMA];
#pragma unroll
    for (uint32_t i = 0; i < XDMA; ++i) {
        const uint32_t sl = dma_row(i) * 64u + lane, c = sl >> 3, pc = (sl & 7u) ^ ((c >> 1) & 7u);
        xoff[i] = (dma_on(i) && cbase + c < B) ? ((cbase + c) * D + 8u * pc) * 2u : B * D * 2u;
    }
    auto dma_x = [&](uint32_t g, uint32_t st) {
#pragma unroll
        for (uint32_t i = 0; i < XDMA; ++i)
            if (dma_on(i)) buf_dma_16(xrs, pool + st * kStage + dma_row(i) * 1024u, xoff[i], g * 128u);
    };
    // In the main loop DMA instruction i of a later group's activations is issued at k-step i
    // (0 at the top, beside the two scale loads), so the instructions do not hold up one k-step's
    // MFMAs back to back; the two weight loads go at k-step 2. The DMA of group g + 1 is issued in
    // iteration g + 2 - PF: when iteration g ends, the ops after its last instruction in that
    // iteration (kAfter) and PF - 2 whole iterations followed it, so waiting until at most that
    // many are outstanding waits for it (with PF = 1 it was issued in iteration g itself). Where
    // the DMA came from the prologue (all of a group's instructions at once, before its loads)
    // more followed it: the wait is stricter than needed there. A wave that issues no DMA waits
    // for the same count over its own loads, which it needs by then anyway.
    static_assert(XDMA == 1u || XDMA == 2u || XDMA == 4u, "a group's DMA instructions map onto its k-steps");
    auto dma_one = [&](uint32_t g, uint32_t st, uint32_t i) {
        if (dma_on(i)) buf_dma_16(xrs, pool + st * kStage + dma_row(i) * 1024u, xoff[i], g * 128u);
    };
    constexpr uint32_t kAfter = (XDMA == 1u) ? 4u : (XDMA == 2u) ? 2u : 0u;
    constexpr uint32_t kXWait = (PF > 1) ? kAfter + (PF - 2u) * (XDMA + 4u) : kAfter;
    static_assert(kXWait < 64u, "vmcnt holds 6 bits");

    f16v acc[2][NB];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

    // The modifier words of the workgroup's (tile, column) pairs, loaded before the weight
    // stream; they are stored to LDS after the prologue's wait, which covers them.
    constexpr uint32_t kMetaPer = ((uint32_t)WV * NCOL + NT - 1u) / NT;
    uint32_t mw[META ? kMetaPer : 1][6];
    uint32_t mr[META ? kMetaPer : 1][4];
    if constexpr (META) {
#pragma unroll
        for (uint32_t q = 0; q < kMetaPer; ++q) {
            const uint32_t idx = tid + q * NT, t = idx / NCOL, c = cbase + idx % NCOL, tl = tg * (uint32_t)WV + t;
#pragma unroll
            for (int k = 0; k < 6; ++k) mw[q][k] = 0u;
#pragma unroll
            for (int k = 0; k < 4; ++k) mr[q][k] = 0u;
            if (idx < (uint32_t)WV * NCOL && c < B && tl < ep.ntile) {
                const uint32_t* rw = reinterpret_cast<const uint32_t*>(ep.rows + c);
                mr[q][0] = rw[9];  // has_mods
                mr[q][1] = rw[3];  // repetition_penalty
                mr[q][2] = rw[4];  // presence_penalty
                mr[q][3] = rw[5];  // frequency_penalty
                const bool two = tl * kTileRows + 32u < ep.V;
                if (ep.hcount) {
                    const uint32_t* hw = ep.hbits + (size_t)c * ep.hbw + 2u * tl;
                    mw[q][0] = hw[0];
                    if (two) mw[q][1] = hw[1];
                }
                if (ep.ban) {
                    const uint32_t* bw = ep.ban + (size_t)c * ep.ban_stride + 2u * tl;
                    mw[q][2] = bw[0];
                    if (two) mw[q][3] = bw[1];
                }
                if (ep.block_start) {
                    const uint32_t* bs = ep.block_start + (size_t)c * (ep.ntile + 1u) + tl;
                    mw[q][4] = bs[0];
                    mw[q][5] = bs[1];
                }
            }
        }
    }

    // Prologue: weights of groups 0 .. PF - 1, activations of groups 0 .. PF - 2 (PF = 1: group 0),
    // each clamped to the last group.
    uint4 wr[PF][2];
    uint32_t sbr[PF][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        const uint32_t gp = min((uint32_t)p, G - 1u);
        if (p < PF - 1 || PF == 1) dma_x(gp, (uint32_t)p);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) sbr[p][mb] = sload(gp, mb);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) wr[p][mb] = wload(gp, mb);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (META) {
        __builtin_amdgcn_s_waitcnt(vm_wait(kXWait));  // the modifier loads came first
#pragma unroll
        for (uint32_t q = 0; q < kMetaPer; ++q) {
            const uint32_t idx = tid + q * NT;
            if (idx < (uint32_t)WV * NCOL) {
                const uint32_t t = idx / NCOL, cl = idx % NCOL;
#pragma unroll
                for (int k = 0; k < 6; ++k) meta.w[t][cl][k] = mw[q][k];
                if (t == 0u) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) meta.r[cl][k] = mr[q][k];
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(kXWait));  // this thread's pieces of group 0
    __builtin_amdgcn_s_barrier();

    // fragment offsets within a stage: column 32 nb + l32, piece 4 hl + j
    const uint32_t sw = (l32 >> 1) & 7u;
    uint32_t foff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) foff[j] = l32 * 128u + (((4u * hl + (uint32_t)j) ^ sw) << 4);
    auto bfrag = [&](uint32_t st, int j, int nb) {
        return *reinterpret_cast<const h8v*>(pool + st * kStage + foff[j] + 4096u * (uint32_t)nb);
    };

    h8v acur[2], anext[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const SbHalves h = unpack_sb16<DENORM>(sbr[0][mb]);
        acur[mb] = dequant_word<DENORM>(wr[0][mb].x, h.s2, h.b2, h.bx, magic);
    }
    for (uint32_t g0 = 0; g0 < G; g0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const uint32_t g = g0 + p;
            // At 32 columns every workgroup is resident from the start (four per CU): even
            // progress keeps all four streaming until the end (B = 32 head 94 -> 89 us). With
            // four column blocks the workgroups come in rounds, and the staggered ends that age
            // order gives overlap one round's epilogues with the next round's loop (there the
            // priorities measured 12 us slower). A 16-wave workgroup is alone on its CU.
            if constexpr (NB <= 2 && WV == 4) prio_by_progress(g, G);
            // stage of group g; group g + PF - 1 goes to the stage group g - 1 used (every wave
            // finished with it before the last barrier)
            const uint32_t st = (PF > 1) ? (uint32_t)p : (g & 1u);
            const uint32_t stn = (PF > 1) ? (uint32_t)((p + PF - 1) % PF) : ((g + 1u) & 1u);
            uint4 wc[2];
            SbHalves hc[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) { wc[mb] = wr[p][mb]; hc[mb] = unpack_sb16<DENORM>(sbr[p][mb]); }
            const uint32_t gx = min(g + (uint32_t)(PF > 1 ? PF - 1 : 1), G - 1u);
            const uint32_t gn = min(g + (uint32_t)PF, G - 1u);
            __builtin_amdgcn_sched_barrier(0);
            dma_one(gx, stn, 0u);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) sbr[p][mb] = sload(gn, mb);
            __builtin_amdgcn_sched_barrier(0);
            constexpr int kNext = (PF > 1) ? 1 : 0;
            const int pn = (p + kNext) % PF;         // prefetch slot holding group g + 1
            // with four column blocks the activation fragments are read one (j, nb) ahead of their
            // MFMAs, so no MFMA pair waits for the LDS read just issued
            constexpr bool kAhead = NB == 4;
            h8v bcur = bfrag(st, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j >= 1 && (uint32_t)j < XDMA) {
                    __builtin_amdgcn_sched_barrier(0);
                    dma_one(gx, stn, (uint32_t)j);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    if (j < 3) {
                        anext[mb] = dequant_word<DENORM>(word_of(wc[mb], j + 1), hc[mb].s2, hc[mb].b2, hc[mb].bx, magic);
                    } else {
                        const SbHalves h = unpack_sb16<DENORM>(sbr[pn][mb]);
                        anext[mb] = dequant_word<DENORM>(wr[pn][mb].x, h.s2, h.b2, h.bx, magic);
                    }
                }
                if (j == 2) {
                    // the last use of this slot's weights is behind: refill it with group g + PF
                    // (its registers are reused in place, with no copy at the loop's end)
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) wr[p][mb] = wload(gn, mb);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    h8v bv, bnext = bcur;
                    if constexpr (kAhead) {
                        bv = bcur;
                        if (nb + 1 < NB) bnext = bfrag(st, j, nb + 1);
                        else if (j < 3) bnext = bfrag(st, j + 1, 0);
                    } else {
                        bv = bfrag(st, j, nb);
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
            // group g + 1's activations: this thread's pieces, then everyone's
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(vm_wait(kXWait));
            __builtin_amdgcn_s_barrier();
        }
    }
    // Per column, the power of two that undoes the row scaling of its fp16 activations (1 for
    // every row within the fp16 range), loaded under the wait that drains the ring.
    float csc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const uint32_t c = cbase + 32u * (uint32_t)nb + l32;
        csc[nb] = (ep.xscale && c < B) ? ep.xscale[c] : 1.0f;
    }
    // The clamped DMAs past the last group may still be writing the ring; the epilogue reuses it.
    __builtin_amdgcn_s_waitcnt(vm_wait(0u));
    __builtin_amdgcn_s_barrier();
    if (!tile_ok) return;

    // ---- epilogue, in place on the accumulators ----
    // Lane (l32, hl) holds batch column cbase + 32 nb + l32 and, per 32-row half mb, the 16 rows
    // 32 mb + acc_row(r, hl) of the wave's tile, in increasing order over (mb, r).
    const uint32_t base = tile * kTileRows;
    const bool full_tile = base + kTileRows <= ep.V;
    const bool vec_ok = (ep.V & 3u) == 0u;  // float4 stores need 16-byte aligned rows
    float* tr = reinterpret_cast<float*>(pool) + wave * kTrHalfFloats;
    SoftcapPoly sc;
    if (ep.cap > 0.0f) sc = softcap_poly(ep.cap);
    auto column = [&]<int nb>() {
        const uint32_t bcol = cbase + 32u * nb + l32;
        const bool col_ok = bcol < B;
        const uint32_t bq = col_ok ? bcol : 0u;
        // acc[mb][nb] for mb = 0, 1 as one array of 32 values in row order
        float zz[32];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) zz[16 * mb + r] = acc[mb][nb][r];
        if (csc[nb] != 1.0f) {
#pragma unroll
            for (int i = 0; i < 32; ++i) zz[i] *= csc[nb];
        }
        if (ep.cap > 0.0f) softcap_values<32>(zz, sc, ep.cap);
        bool may_ninf = !full_tile;  // some value may be -inf (padding, ban, a -inf bias)
        if constexpr (META) {
            const uint32_t* mwv = meta.w[wave][32u * nb + l32];
            const uint32_t has_mods = col_ok ? meta.r[32u * nb + l32][0] : 0u;
            const uint32_t hb0 = mwv[0], hb1 = mwv[1], ban0 = mwv[2], ban1 = mwv[3];
            if (has_mods) {
                DevRow row{};
                row.repetition_penalty = __uint_as_float(meta.r[32u * nb + l32][1]);
                row.presence_penalty = __uint_as_float(meta.r[32u * nb + l32][2]);
                row.frequency_penalty = __uint_as_float(meta.r[32u * nb + l32][3]);
                // bias first (the order of apply_entry): entries are unique per id, each read
                // once and added to the one value that holds its id, if this lane holds it
                if ((has_mods & 2u) && ep.block_start) {
                    const ModEntry* me = ep.mods + (size_t)bq * ep.mod_cap;
                    for (uint32_t k = mwv[4]; k < mwv[5]; ++k) {
                        const ModEntry t = me[k];
                        const uint32_t rr = t.id - base;
#pragma unroll
                        for (int i = 0; i < 32; ++i)
                            if (rr == 32u * (i >> 4) + acc_row(i & 15, hl)) {
#pragma clang fp contract(off)
                                zz[i] = zz[i] + t.bias;
                            }
                    }
                    may_ninf = true;
                }
                // history counts: every count of a 32-row half is loaded before any is used,
                // then zeroed for the next step and applied; the low half of the column zeroes
                // the tile's two bitmap words
                if ((has_mods & 1u) && ep.hcount && (hb0 | hb1) != 0u) {
                    uint32_t* hrow = ep.hcount + (size_t)bq * ep.V + base;
                    if (hl == 0u) {
                        uint32_t* hw = ep.hbits + (size_t)bq * ep.hbw + 2u * tile;
                        if (hb0) hw[0] = 0u;
                        if (hb1) hw[1] = 0u;
                    }
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) {
                        const uint32_t hb = mb ? hb1 : hb0;
                        if (hb == 0u) continue;
                        uint32_t cnt[16];
                        if (full_tile && vec_ok) {
                            // The lane's 16 rows of this half are four runs of four consecutive ids
                            // (acc_row): a run with a bit set is read with one 16-byte load and
                            // zeroed with one 16-byte store. Ids without a bit hold 0 already, and
                            // no other lane touches these ids.
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const uint32_t o = 32u * mb + 8u * (uint32_t)q + 4u * hl;
                                uint4 c4 = make_uint4(0u, 0u, 0u, 0u);
                                if ((hb >> (o & 31u)) & 15u) c4 = *reinterpret_cast<const uint4*>(hrow + o);
                                cnt[4 * q] = c4.x;
                                cnt[4 * q + 1] = c4.y;
                                cnt[4 * q + 2] = c4.z;
                                cnt[4 * q + 3] = c4.w;
                            }
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const uint32_t o = 32u * mb + 8u * (uint32_t)q + 4u * hl;
                                if ((hb >> (o & 31u)) & 15u)
                                    *reinterpret_cast<uint4*>(hrow + o) = make_uint4(0u, 0u, 0u, 0u);
                            }
                        } else {
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const uint32_t rr = 32u * mb + acc_row(r, hl);
                                cnt[r] = ((hb >> (rr & 31u)) & 1u) ? hrow[rr] : 0u;
                            }
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                if (cnt[r]) hrow[32u * mb + acc_row(r, hl)] = 0u;
                        }
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            if (cnt[r])
                                zz[16 * mb + r] = apply_entry(zz[16 * mb + r],
                                                              ModEntry{base + 32u * mb + acc_row(r, hl), cnt[r], 0.0f, 0u}, row,
                                                              ep.rep_limit);
                    }
                }
            }
            if (col_ok && ep.ban && (ban0 | ban1) != 0u) {
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const uint32_t rr = 32u * (i >> 4) + acc_row(i & 15, hl);
                    if ((((i < 16) ? ban0 : ban1) >> (rr & 31u)) & 1u) zz[i] = -INFINITY;
                }
                may_ninf = true;
            }
        }
        if (!full_tile) {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (base + 32u * (i >> 4) + acc_row(i & 15, hl) >= ep.V) zz[i] = -INFINITY;
        }
        // Block statistics over the 64 rows (not for a logits-only call, which no select reads):
        // the lane's 32 values, then the other half of the column (lane ^ 32).
        if (ep.partials) {
            float lmax, lsec = -INFINITY;
            if (!ep.no_smax) {
                // running maximum and second maximum (repeats count), two values at a time
                lmax = -INFINITY;
#pragma unroll
                for (int i = 0; i < 32; i += 2) {
                    const float hi = fmaxf(zz[i], zz[i + 1]), lo = fminf(zz[i], zz[i + 1]);
                    lsec = fmaxf(fmaxf(lsec, lo), fminf(lmax, hi));
                    lmax = fmaxf(lmax, hi);
                }
            } else {
                lmax = zz[0];
#pragma unroll
                for (int i = 1; i < 32; ++i) lmax = fmaxf(lmax, zz[i]);
            }
            const float om = xor32(lmax);
            const float bm = fmaxf(lmax, om);  // the block maximum
            // lowest row of the lane holding it, then the lower of the two halves' ids
            uint32_t ri = 32u;
#pragma unroll
            for (int i = 31; i >= 0; --i) ri = (zz[i] == bm) ? (uint32_t)i : ri;
            uint32_t barg = (ri < 32u) ? base + 32u * (ri >> 4) + acc_row((int)(ri & 15u), hl) : 0xFFFFFFFFu;
            barg = min(barg, xor32(barg));
            float bsec = -INFINITY;
            if (!ep.no_smax) bsec = fmaxf(fmaxf(lsec, xor32(lsec)), fminf(lmax, om));
            float bmin;
            if (may_ninf) {
                bmin = INFINITY;
#pragma unroll
                for (int i = 0; i < 32; ++i) bmin = fminf(bmin, zz[i] == -INFINITY ? INFINITY : zz[i]);
            } else {
                bmin = zz[0];
#pragma unroll
                for (int i = 1; i < 32; ++i) bmin = fminf(bmin, zz[i]);
            }
            bmin = fminf(bmin, xor32(bmin));
            float se = 0.0f;
            if (!ep.no_sumexp) {
                if (bm != -INFINITY) {
                    const float mb2 = bm * 1.4426950408889634f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) se += __builtin_amdgcn_exp2f(fmaf(zz[i], 1.4426950408889634f, -mb2));
                }
                se += xor32(se);
            }
            if (col_ok && hl == 0u) {
                BlockPartial bp;
                bp.max = bm;
                bp.arg = (bm == -INFINITY) ? base : barg;
                bp.sumexp = se;
                bp.minf = bmin;
                bp.smax = bsec;
                ep.partials[(size_t)bq * ep.ntile + tile] = bp;
            }
        }
        // Logits: each 32-row half goes through the wave's own LDS tile (32 columns x 32 rows,
        // 16-byte pieces XOR-swizzled so that neither side conflicts), so one float4 store
        // writes four contiguous rows of one column and 8 lanes cover a 128-byte row segment.
        if (ep.logits) {
            if (full_tile && vec_ok) {
                const uint32_t rc = lane >> 3, k = lane & 7u;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t piece = (2u * q + hl) ^ ((l32 >> 1) & 7u);
                        *reinterpret_cast<float4*>(tr + 32u * l32 + 4u * piece) =
                            make_float4(zz[16 * mb + 4 * q], zz[16 * mb + 4 * q + 1], zz[16 * mb + 4 * q + 2],
                                        zz[16 * mb + 4 * q + 3]);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t c = 8u * (uint32_t)i + rc;  // column of the tile
                        const float4 v = *reinterpret_cast<const float4*>(tr + 32u * c + 4u * (k ^ ((c >> 1) & 7u)));
                        if (cbase + 32u * nb + c < B)
                            *reinterpret_cast<float4*>(ep.logits + (size_t)(cbase + 32u * nb + c) * ep.V + base +
                                                       32u * mb + 4u * k) = v;
                    }
                }
            } else if (col_ok) {
                float* lrow = ep.logits + (size_t)bq * ep.V + base;
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const uint32_t rr = 32u * (i >> 4) + acc_row(i & 15, hl);
                    if (base + rr < ep.V) lrow[rr] = zz[i];
                }
            }
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
    if (!mfma_table_fits(h)) throw std::runtime_error("MFMA head supports tables of at most 4 GiB");
    const int nb = (B <= 32u) ? 1 : (B <= 64u) ? 2 : 4;
    const uint32_t ncol = 32u * (uint32_t)nb;
    const uint32_t wv = (nb == 2) ? 16u : 4u;  // waves (tiles) per workgroup, as instantiated below
    const uint32_t ntg = (h.ntile + wv - 1u) / wv, ncb = (B + ncol - 1u) / ncol;
    const dim3 grid(ncb * ((ntg + 7u) / 8u) * 8u);
    const bool meta = ep.meta != 0u;
    // Prefetch depth: four groups when the group count allows it, else two, else one. Two column
    // blocks run as one 16-wave workgroup per CU (all 256 of a 262,144-row head resident at once)
    // and hold two groups, which fits the 128 registers that sixteen waves per CU allow.
    const int pf = (h.G % 4u == 0u) ? 4 : (h.G % 2u == 0u) ? 2 : 1;
#define TDT_LAUNCH(NB, WV, PF, OCC, DN, MT)                                                                   \
    hipExtLaunchKernelGGL((k_head_mfma<NB, WV, PF, OCC, DN, MT>), grid, dim3(64 * WV), 0, st, ev0, ev1, 0, h.Wt, \
                          h.SB16t, h.x16, B, h.D, h.NC, h.G, ncb, ntg, ep)
#define TDT_PF421(NB, WV, OCC, DN, MT)                             \
    do {                                                           \
        if (pf == 4) TDT_LAUNCH(NB, WV, 4, OCC, DN, MT);            \
        else if (pf == 2) TDT_LAUNCH(NB, WV, 2, OCC, DN, MT);       \
        else TDT_LAUNCH(NB, WV, 1, OCC, DN, MT);                    \
    } while (0)
#define TDT_PF21(NB, WV, OCC, DN, MT)                              \
    do {                                                           \
        if (pf >= 2) TDT_LAUNCH(NB, WV, 2, OCC, DN, MT);            \
        else TDT_LAUNCH(NB, WV, 1, OCC, DN, MT);                    \
    } while (0)
#define TDT_PICK(NB, WV, OCC, PFS)                                                                         \
    do {                                                                                                   \
        if (h.mfma_denorm) { if (meta) PFS(NB, WV, OCC, true, true); else PFS(NB, WV, OCC, true, false); } \
        else { if (meta) PFS(NB, WV, OCC, false, true); else PFS(NB, WV, OCC, false, false); }             \
    } while (0)
    if (nb == 1) {
        TDT_PICK(1, 4, 3, TDT_PF421);
    } else if (nb == 2) {
        TDT_PICK(2, 16, 1, TDT_PF21);
    } else {
        TDT_PICK(4, 4, 2, TDT_PF421);
    }
#undef TDT_PICK
#undef TDT_PF21
#undef TDT_PF421
#undef TDT_LAUNCH
    check_hip(hipGetLastError(), "head (MFMA)");
}

}  // namespace tdt
