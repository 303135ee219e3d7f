// Pieces of the matrix-core head (gemm_mfma.hip): the in-register int4 -> fp16 dequant, the
// scale / bias unpacking and the accumulator layout of v_mfma_f32_32x32x16_f16.
//
// Accumulation: logits[b][v] = sum_c w[v][c] x[b][c], w = q * s + b (src/cpu_reference.cpp:55-84),
// with A = dequantised weights (32 vocabulary rows), B = activations (32 batch rows), fp32
// accumulation over the groups in order, four 16-k steps per 64-k group.
#pragma once

#include "dt_epilogue.h"

namespace tdt {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr uint32_t kColHalves = 72;  // 64 halves of a group + 8 padding (LDS bank spread)

__device__ inline h2v as_h2(uint32_t u) { return __builtin_bit_cast(h2v, u); }

// The table is streamed once per step (nontemporal: it does not displace the activations).
__device__ inline uint4 mfma_load_stream(const uint4* p) {
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ inline uint32_t mfma_load_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }

// The constant 0x64006400 (fp16 1024.0 in both halves) in a VGPR. With the mask in an SGPR,
// (w & mask) | magic is then one v_and_or_b32 (a VOP3 instruction reads at most one SGPR or
// literal on this architecture, so with both constants scalar it would take two instructions).
__device__ inline uint32_t magic_vgpr() {
    uint32_t r;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(r));
    return r;
}

// 8 nibbles -> 8 halves in the order (e0, e4, e1, e5, e2, e6, e3, e7), e = round16(q s + b) (one
// rounding: every product below is exact), the even elements divided by 16 and their activation
// slots holding 16 x. Power-of-two scaling commutes with the rounding while the value stays in
// the fp16 normal range, so each product is then exactly round16(q s + b) * x. An even element
// with |q s + b| / 16 below 2^-14 (|q s + b| < 2^-10) rounds on the fp16 subnormal grid instead:
// its product is off by at most 2^-25 * 16 |x| = 2^-21 |x|, the same absolute size as the normal
// range's 2^-11 relative error at that magnitude. Two ways to make the fp16 operand of q:
//   DENORM: the nibbles are used where they lie. Masked in place, an even nibble (bits 0-3 of a
//     half) is the fp16 denormal q * 2^-24 and an odd one (bits 4-7) q * 2^-20; with s2 = s * 2^20,
//     (q 2^-20)(s 2^20) = q s and (q 2^-24)(s 2^20) = q s / 16. 9 VALU instructions per 8
//     weights (1 shift, 4 ands, 4 packed FMAs). Needs fp16 denormals preserved (the kernels' FP
//     mode) and |s| < 1/16 so that s 2^20 stays finite.
//   otherwise (any scale): OR-ing a nibble into the mantissa of 1024.0 gives 1024 + q (an odd
//     nibble, extracted in place, 1024 + 16 q) and one v_pk_add_f16 removes the 1024; with
//     s2 = s, even slots then need the scale / 16, so here the even slots take s and b and the
//     odd ones 16 q with b * 16, and the activations the layout (x, x / 16). 13 instructions.
// bx: the bias for the slots that differ from b (b / 16 for DENORM's even slots, 16 b otherwise).
template <bool DENORM>
__device__ inline h8v dequant_word(uint32_t w, h2v s2, h2v b2, h2v bx, uint32_t magic) {
    const uint32_t w8 = w >> 8;
    h2v r0, r1, r2, r3;
    if constexpr (DENORM) {
        r0 = __builtin_elementwise_fma(as_h2(w & 0x000F000Fu), s2, bx);   // (q0, q4) / 16
        r1 = __builtin_elementwise_fma(as_h2(w & 0x00F000F0u), s2, b2);   // (q1, q5)
        r2 = __builtin_elementwise_fma(as_h2(w8 & 0x000F000Fu), s2, bx);  // (q2, q6) / 16
        r3 = __builtin_elementwise_fma(as_h2(w8 & 0x00F000F0u), s2, b2);  // (q3, q7)
    } else {
        const h2v off = as_h2(0x64006400u);
        r0 = __builtin_elementwise_fma(as_h2((w & 0x000F000Fu) | magic) - off, s2, b2);   // (q0, q4)
        r1 = __builtin_elementwise_fma(as_h2((w & 0x00F000F0u) | magic) - off, s2, bx);   // 16 (q1, q5)
        r2 = __builtin_elementwise_fma(as_h2((w8 & 0x000F000Fu) | magic) - off, s2, b2);  // (q2, q6)
        r3 = __builtin_elementwise_fma(as_h2((w8 & 0x00F000F0u) | magic) - off, s2, bx);  // 16 (q3, q7)
    }
    h8v o;
    o[0] = r0[0]; o[1] = r0[1]; o[2] = r1[0]; o[3] = r1[1];
    o[4] = r2[0]; o[5] = r2[1]; o[6] = r3[0]; o[7] = r3[1];
    return o;
}

// A group's scale (fp16 s * 2^20 for DENORM, else s) and bias, each in both halves, and bx (b / 16
// for DENORM, else 16 b), from its SB16t word.
struct SbHalves {
    h2v s2, b2, bx;
};
template <bool DENORM>
__device__ inline SbHalves unpack_sb16(uint32_t w) {
    SbHalves r;
    r.s2 = as_h2(__builtin_amdgcn_perm(w, w, 0x01000100u));
    r.b2 = as_h2(__builtin_amdgcn_perm(w, w, 0x03020302u));
    r.bx = r.b2 * (DENORM ? h2v{(_Float16)0.0625f, (_Float16)0.0625f} : h2v{(_Float16)16.0f, (_Float16)16.0f});
    return r;
}

// Softcap for the batched path: x = z / cap through the reciprocal, then
// tanh(x) = sign(x) (1 - 2 / (exp(2|x|) + 1)) with the hardware exp2 and rcp. For large |x|
// exp overflows to +inf and rcp(inf) = 0 gives exactly +-1, as libm's tanhf does once
// |x| > 9. Relative error ~1e-6, far below this path's fp16-dequant error.
__device__ inline float softcap_fast(float z, float cap, float inv_cap) {
    const float x = z * inv_cap;
    const float e = __builtin_amdgcn_exp2f(fabsf(x) * 2.8853900817779268f);  // exp(2|x|)
    const float t = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
    return cap * copysignf(t, x);
}

// Softcap cap * tanh(z / cap) as z * P(u), u = z^2, for |z| <= cap / 2: P is a degree-5
// polynomial fitted to tanh(x) / x over x^2 in [0, 1/4] (coefficients c_i of x^(2i), Chebyshev-node
// least squares), pre-scaled by cap^(-2i). In fp32 with fused multiply-adds it stays within
// 1e-7 relative of the exact softcap, closer than fp32 cap * tanhf(z / cap) itself (which rounds
// z / cap first). A wave with any larger |z| takes softcap_fast for all its values.
struct SoftcapPoly {
    float k1, k2, k3, k4, k5;  // c_i / cap^(2i)
    float lim;                 // cap / 2
    float inv;                 // 1 / cap
};
__device__ inline SoftcapPoly softcap_poly(float cap) {
    SoftcapPoly p;
    p.inv = 1.0f / cap;
    const float i2 = p.inv * p.inv, i4 = i2 * i2;
    p.k1 = -0.33333325f * i2;
    p.k2 = 0.13332954f * i4;
    p.k3 = -0.053898074f * (i4 * i2);
    p.k4 = 0.021292942f * (i4 * i4);
    p.k5 = -0.0066395057f * (i4 * i4 * i2);
    p.lim = 0.5f * cap;
    return p;
}
template <int N>
__device__ inline void softcap_values(float (&z)[N], const SoftcapPoly& p, float cap) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) m = fmaxf(m, fabsf(z[i]));
    if (__builtin_amdgcn_ballot_w64(m > p.lim) != 0ull) {
#pragma unroll
        for (int i = 0; i < N; ++i) z[i] = softcap_fast(z[i], cap, p.inv);
        return;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float u = z[i] * z[i];
        float q = fmaf(p.k5, u, p.k4);
        q = fmaf(q, u, p.k3);
        q = fmaf(q, u, p.k2);
        q = fmaf(q, u, p.k1);
        q = fmaf(q, u, 1.0f);
        z[i] = z[i] * q;
    }
}

// Modifier words of a workgroup's (tile, column) pairs, staged in LDS before the main loop:
// w[t][c] = {history bitmap word 0, word 1, ban word 0, word 1, first bias entry, end} for its
// WV tiles; and per column r[c] = {has_mods, repetition, presence, frequency penalty bits}.
template <int WV, uint32_t NCOL>
struct EpiMeta {
    uint32_t w[WV][NCOL][6];
    uint32_t r[NCOL][4];
};

// Word 3 of a raw buffer resource on this architecture (32-bit data format, no swizzle).
constexpr int kBufDword3 = 0x00020000;
// Cache policy of the streamed loads: nontemporal.
constexpr int kNt = 2;
// s_waitcnt operand that waits until at most n vector-memory operations are outstanding and
// leaves the other counters unconstrained (vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vm_wait(uint32_t n) { return (int)((n & 15u) | (7u << 4) | (15u << 8) | ((n >> 4) << 14)); }

// Buffer loads (nontemporal) at a per-lane byte offset plus a wave-uniform one, and the
// buffer-to-LDS form: 16 bytes per lane to lds + 16 * lane, counted by vmcnt like any load.
__device__ inline uint4 buf_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const v4u t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNt);
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ inline uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kNt);
}
__device__ inline void buf_dma_16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// Floats of one wave's transposed half tile (32 columns x 32 rows) in the epilogue.
constexpr uint32_t kTrHalfFloats = 32u * 32u;

// Row held in register r of a 32x32 accumulator by a lane with half hl (0/1): 8(r/4) + 4hl + r%4.
__device__ inline uint32_t acc_row(int r, uint32_t hl) { return 8u * (uint32_t)(r >> 2) + 4u * hl + (uint32_t)(r & 3); }

__device__ inline uint32_t word_of(const uint4& w, int j) { return (j == 0) ? w.x : (j == 1) ? w.y : (j == 2) ? w.z : w.w; }

// Issue priority by progress: 3 in the first quarter of the G groups, down to 0 in the last.
// The SIMD arbiter otherwise favours the oldest waves, so workgroups that share a CU finish one
// after another and the last runs alone with a fraction of the CU's loads in flight; lowering
// the priority of the waves ahead lets the others catch up, and they finish together.
__device__ inline void prio_by_progress(uint32_t g, uint32_t G) {
    const uint32_t q = (4u * g) / G;
    if (q == 0u) __builtin_amdgcn_s_setprio(3);
    else if (q == 1u) __builtin_amdgcn_s_setprio(2);
    else if (q == 2u) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

}  // namespace tdt
