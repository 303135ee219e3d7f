// Fused epilogue of the head kernels: one wave64 holds 64 consecutive vocabulary ids of one
// batch row. It applies, per id and in this order:
//   softcap      30 * tanh(z / 30)                      src/cpu_reference.cpp:535-538
//   logit bias   + summed bias                           (extension)
//   repetition   per occurrence, clamp +-0.9999*softcap  src/sampling.cpp:74-90
//   presence / frequency                                 (extension)
//   ban          -> -inf                                 (extension)
// then stores the logit (optional) and the block partial (max, lowest argmax, sum exp(l-max),
// smallest finite value, second-largest value).
// Floating-point contraction is off in these functions (the library is built with
// -ffp-contract=fast-honor-pragmas): a fused multiply-add would round once where the reference
// rounds twice, e.g. in l - frequency * count or in cap * tanh(z / cap) + bias.
#pragma once

#include "dt_internal.h"

namespace tdt {

__device__ inline float apply_entry(float l, const ModEntry& m, const DevRow& row, float limit) {
#pragma clang fp contract(off)
    if (m.has_bias) l = l + m.bias;
    if (m.count) {
        const float p = row.repetition_penalty;
        if (p != 1.0f) {
            for (uint32_t c = 0; c < m.count; ++c) {
                float v = (l > 0.0f) ? l / p : l * p;
                if (limit > 0.0f) v = fminf(fmaxf(v, -limit), limit);
                if (v == l) break;  // a fixed point (0, or the clamp): later occurrences keep it
                l = v;
            }
        }
        if (row.presence_penalty != 0.0f || row.frequency_penalty != 0.0f) {
            l = l - row.presence_penalty;
            l = l - row.frequency_penalty * (float)m.count;
        }
    }
    return l;
}

// The modifiers of one id of batch row b: its history count (dense array, read only where the
// id's bit is set in the bitmap word hw) and its summed bias (the row's bias entries of tile
// `tile`). The count is zeroed once read: exactly one wave reads each (row, id), so the array
// is clean again for the next step without a separate pass.
__device__ inline ModEntry lookup_mods(uint32_t id, uint32_t b, uint32_t tile, uint32_t hw, const DevRow& row,
                                       const EpiArgs& ep) {
    ModEntry m{id, 0u, 0.0f, 0u};
    if ((hw >> (id & 31u)) & 1u) {
        uint32_t* cp = ep.hcount + (size_t)b * ep.V + id;
        m.count = *cp;
        if (m.count) *cp = 0u;  // stored after the load it depends on
    }
    if ((row.has_mods & 2u) && ep.block_start) {
        const uint32_t* bs = ep.block_start + (size_t)b * (ep.ntile + 1) + tile;
        const uint32_t s = bs[0], e = bs[1];
        const ModEntry* me = ep.mods + (size_t)b * ep.mod_cap;
        for (uint32_t k = s; k < e; ++k) {
            const ModEntry t = me[k];
            if (t.id == id) { m.bias = t.bias; m.has_bias = 1u; }
        }
    }
    return m;
}

// After the modifiers: ban, padding ids, the logit store and the block partial.
__device__ inline void finish_wave(float l, uint32_t b, uint32_t tile, uint32_t lane, const EpiArgs& ep) {
#pragma clang fp contract(off)
    const uint32_t id = tile * kTileRows + lane;
    const bool valid = id < ep.V;
    if (ep.ban && valid) {
        const uint32_t w = ep.ban[(size_t)b * ep.ban_stride + (id >> 5)];
        if ((w >> (id & 31u)) & 1u) l = -INFINITY;
    }
    if (!valid) l = -INFINITY;
    if (ep.logits && valid) ep.logits[(size_t)b * ep.V + id] = l;
    if (!ep.partials) return;  // a logits-only call: no select reads the block summaries
    const float m = wave_max(l);
    const uint32_t arg = wave_min_u(l == m ? id : 0xFFFFFFFFu);
    const float sm = wave_max(id == arg ? -INFINITY : l);  // a repeat of the maximum counts
    float se = (m == -INFINITY || ep.no_sumexp) ? 0.0f : __expf(l - m);
    if (!ep.no_sumexp) se = wave_sum(se);
    const float mn = wave_min(l == -INFINITY ? INFINITY : l);
    if (lane == 0) {
        BlockPartial bp;
        bp.max = m;
        bp.arg = arg;
        bp.sumexp = se;
        bp.minf = mn;
        bp.smax = sm;
        ep.partials[(size_t)b * ep.ntile + tile] = bp;
    }
}

// acc: the raw head value of id = tile*64 + lane for batch row b (wave-uniform b and tile).
__device__ inline void epilogue_wave(float acc, uint32_t b, uint32_t tile, uint32_t lane,
                                     const EpiArgs& ep) {
#pragma clang fp contract(off)
    const uint32_t id = tile * kTileRows + lane;
    const bool valid = id < ep.V;
    float l = acc;
    if (ep.cap > 0.0f) l = ep.cap * tanhf(l / ep.cap);
    const DevRow& row = ep.rows[b];
    if (row.has_mods && valid) {
        // history bitmap word of this id; lanes 0 and 32 zero the tile's two words once read
        uint32_t hw = 0u;
        if ((row.has_mods & 1u) && ep.hcount) {
            uint32_t* wp = ep.hbits + (size_t)b * ep.hbw + (id >> 5);
            hw = *wp;
            if ((id & 31u) == 0u && hw != 0u) *wp = 0u;
        }
        const ModEntry m = lookup_mods(id, b, tile, hw, row, ep);
        if (m.count || m.has_bias) l = apply_entry(l, m, row, ep.rep_limit);
    }
    finish_wave(l, b, tile, lane, ep);
}

// The same with the id's history count given (no bias table): the folded small-batch step.
__device__ inline void epilogue_wave_counted(float acc, uint32_t b, uint32_t tile, uint32_t lane,
                                             const EpiArgs& ep, const DevRow& row, uint32_t count) {
#pragma clang fp contract(off)
    const uint32_t id = tile * kTileRows + lane;
    float l = acc;
    if (ep.cap > 0.0f) l = ep.cap * tanhf(l / ep.cap);
    if (count && id < ep.V) l = apply_entry(l, ModEntry{id, count, 0.0f, 0u}, row, ep.rep_limit);
    finish_wave(l, b, tile, lane, ep);
}

}  // namespace tdt
