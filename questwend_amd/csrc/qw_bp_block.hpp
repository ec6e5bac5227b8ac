// qw_bp_block.hpp -- one quantized weight block (Q4_K / Q6_K) times one Q8_K
// activation block in LDS, every integer of ggml's AVX2 dot for all eight AVX
// lanes at once (ggml-cpu/arch/x86/quants.c: q4_K 2038-2115, q6_K 2426-2508),
// plus the block's float scales: the per-(row, block) step of the
// block-parallel GEMV (mmid.hip) and of the wide persistent decode kernel
// (decode_xcd_wide.hip).  The float chains over the blocks stay with the caller.
#pragma once

#include "qw_kernels.hpp"
#include "qw_rowdot.hpp"

namespace qw {

template <int TYPE>
struct BpType {
    static constexpr int NPW = TYPE == T_Q4_K ? 14 : 9;   // words per (row, block): S[8] (P[4]) fd (fm)
    static constexpr int NCH = TYPE == T_Q4_K ? 12 : 8;   // float chains per row
};

// Activation blocks staged at 304-byte strides, each starting 12 bytes into its
// slot, so its quants and bsums lie 16-byte aligned.
constexpr uint32_t BP_ABLK = 304;

__device__ __forceinline__ u32x4 lds_x4(const uint32_t* lds, uint32_t byte_off) {
    return *(const u32x4*) (lds + (byte_off >> 2));
}

// The integers of one Q4_K block times one Q8_K block for all eight AVX lanes,
// and the two block scales (row_dot_lds<T_Q4_K>'s sumi, prod, d, dmin).
// rw(o): the weight block's 32-bit word at byte offset o.
template <class RW>
__device__ __forceinline__ void bp_q4k_block(RW rw, const uint32_t* lds, uint32_t yb, uint32_t* part) {
    const uint32_t h0 = rw(0), s0 = rw(4), s1 = rw(8), s2 = rw(12);
    const uint8_t q[12] = {(uint8_t) s0, (uint8_t) (s0 >> 8), (uint8_t) (s0 >> 16), (uint8_t) (s0 >> 24),
                           (uint8_t) s1, (uint8_t) (s1 >> 8), (uint8_t) (s1 >> 16), (uint8_t) (s1 >> 24),
                           (uint8_t) s2, (uint8_t) (s2 >> 8), (uint8_t) (s2 >> 16), (uint8_t) (s2 >> 24)};
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) scale_min_k4(j, q, sc[j], mn[j]);
    int sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const u32x4 l0 = lds_x4(lds, yb + 4 + 64 * j), l1 = lds_x4(lds, yb + 20 + 64 * j);
        const u32x4 h0v = lds_x4(lds, yb + 36 + 64 * j), h1v = lds_x4(lds, yb + 52 + 64 * j);
        const uint32_t alo[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
        const uint32_t ahi[8] = {h0v.x, h0v.y, h0v.z, h0v.w, h1v.x, h1v.y, h1v.z, h1v.w};
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const uint32_t wq = rw(16 + 32 * j + 4 * n);
            const int lo = (int) (wq & 0x0F0F0F0Fu), hi = (int) ((wq >> 4) & 0x0F0F0F0Fu);
            sumi[n] += mul24(sc[2 * j], sdot4(lo, (int) alo[n], 0)) + mul24(sc[2 * j + 1], sdot4(hi, (int) ahi[n], 0));
        }
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) part[n] = (uint32_t) sumi[n];
    const u32x4 b0 = lds_x4(lds, yb + 260), b1 = lds_x4(lds, yb + 276);
    const uint32_t bsw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        const uint32_t bs01 = bsw[2 * n], bs23 = bsw[2 * n + 1];
        const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
        const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
        part[8 + n] = (uint32_t) (mul24(mn[2 * n], q8s0) + mul24(mn[2 * n + 1], q8s1));
    }
    const float yd = bitsf(lds_u32a(lds, yb));
    part[12] = __float_as_uint(yd * h2f((uint16_t) (h0 & 0xffff)));
    part[13] = __float_as_uint(-yd * h2f((uint16_t) (h0 >> 16)));
}

// The same for one Q6_K block (row_dot_lds<T_Q6_K>'s sumi and d); d16: the
// block's f16 scale.  VEC: the activations are read a 32-byte quarter at a time
// (fewer LDS reads, more registers: the form for bins of many rows).
template <bool VEC, class RW>
__device__ __forceinline__ void bp_q6k_block(RW rw, uint16_t d16, const uint32_t* lds, uint32_t yb, uint32_t* part) {
    int sc[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t s = rw(192 + 4 * i);
        sc[4 * i + 0] = (int) (int8_t) (s & 0xff);
        sc[4 * i + 1] = (int) (int8_t) ((s >> 8) & 0xff);
        sc[4 * i + 2] = (int) (int8_t) ((s >> 16) & 0xff);
        sc[4 * i + 3] = (int) (int8_t) (s >> 24);
    }
    const u32x4 b0 = lds_x4(lds, yb + 260), b1 = lds_x4(lds, yb + 276);
    const uint32_t bsw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    if constexpr (!VEC) {
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int g = n >= 4 ? 1 : 0;
            int sumi = 0;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t qa = rw(64 * j + 4 * n);
                const uint32_t qb = rw(64 * j + 32 + 4 * n);
                const uint32_t qh = rw(128 + 32 * j + 4 * n);
                const int q0 = (int) ((qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
                const int q1 = (int) ((qb & 0x0F0F0F0Fu) | ((qh & 0x0C0C0C0Cu) << 2));
                const int q2 = (int) (((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u));
                const int q3 = (int) (((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u));
                const uint32_t y = yb + 4 + 128 * j + 4 * n;
                sumi += mul24(sc[8 * j + 0 + g], sdot4(q0, (int) lds_u32a(lds, y), 0));
                sumi += mul24(sc[8 * j + 2 + g], sdot4(q1, (int) lds_u32a(lds, y + 32), 0));
                sumi += mul24(sc[8 * j + 4 + g], sdot4(q2, (int) lds_u32a(lds, y + 64), 0));
                sumi += mul24(sc[8 * j + 6 + g], sdot4(q3, (int) lds_u32a(lds, y + 96), 0));
            }
            const uint32_t bs = bsw[n];
            part[n] = (uint32_t) (sumi - 32 * (mul24((int) (int16_t) (bs & 0xffff), sc[2 * n]) +
                                               mul24((int) (int16_t) (bs >> 16), sc[2 * n + 1])));
        }
        part[8] = __float_as_uint(bitsf(lds_u32a(lds, yb)) * h2f(d16));
        return;
    }
    int sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        // the 6-bit quants of every lane n for the four 32-value quarters of half j
        int qv[4][8];
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const uint32_t qa = rw(64 * j + 4 * n);
            const uint32_t qb = rw(64 * j + 32 + 4 * n);
            const uint32_t qh = rw(128 + 32 * j + 4 * n);
            qv[0][n] = (int) ((qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
            qv[1][n] = (int) ((qb & 0x0F0F0F0Fu) | ((qh & 0x0C0C0C0Cu) << 2));
            qv[2][n] = (int) (((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u));
            qv[3][n] = (int) (((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // the quarter's 32 activation bytes, lane n's four in word n
            const u32x4 a0 = lds_x4(lds, yb + 4 + 128 * j + 32 * q), a1 = lds_x4(lds, yb + 20 + 128 * j + 32 * q);
            const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int n = 0; n < 8; ++n)
                sumi[n] += mul24(sc[8 * j + 2 * q + (n >= 4 ? 1 : 0)], sdot4(qv[q][n], (int) a[n], 0));
        }
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        const uint32_t bs = bsw[n];
        part[n] = (uint32_t) (sumi[n] - 32 * (mul24((int) (int16_t) (bs & 0xffff), sc[2 * n]) +
                                              mul24((int) (int16_t) (bs >> 16), sc[2 * n + 1])));
    }
    part[8] = __float_as_uint(bitsf(lds_u32a(lds, yb)) * h2f(d16));
}

}  // namespace qw
