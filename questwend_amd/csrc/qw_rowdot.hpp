// qw_rowdot.hpp -- one quantized row times one quantized activation row, from
// LDS, with the exact integer lanes and float order of ggml's AVX2 vec_dot
// (ggml/src/ggml-cpu/arch/x86/quants.c: q8_0 1308-1370, q4_K 2038-2115,
// q6_K 2426-2508).  Eight lanes cooperate on a row: lane n computes the AVX
// lane n partial sums, then an 8-lane shuffle tree reproduces hsum_float_8.
#pragma once

#include "qw_common.hpp"

namespace qw {

__device__ __forceinline__ uint32_t lds_u32(const uint32_t* lds, uint32_t byte_off) {
    const uint32_t lo = lds[byte_off >> 2], hi = lds[(byte_off >> 2) + 1];
    return __builtin_amdgcn_alignbyte(hi, lo, byte_off & 3);
}
__device__ __forceinline__ uint32_t lds_u32a(const uint32_t* lds, uint32_t byte_off) { return lds[byte_off >> 2]; }
__device__ __forceinline__ uint16_t lds_u16(const uint32_t* lds, uint32_t byte_off) {
    return (uint16_t) (lds_u32(lds, byte_off) & 0xffff);
}
__device__ __forceinline__ float lds_f32(const uint32_t* lds, uint32_t byte_off) { return bitsf(lds_u32(lds, byte_off)); }

// Row dot products from LDS for one (row, n) lane.  Returns the lane's
// contribution after the 8-lane reduction (valid in lane n == 0 of the group).
template <int TYPE>
__device__ __forceinline__ float row_dot_lds(const uint32_t* lds, uint32_t wbase, uint32_t abase, int nb, int n);

template <>
__device__ __forceinline__ float row_dot_lds<T_Q4_K>(const uint32_t* lds, uint32_t wbase, uint32_t abase, int nb, int n) {
    float acc = 0.0f, accm = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 144u * b;
        const uint32_t yb = abase + 292u * b;
        const uint32_t h0 = lds_u32(lds, blk);
        const uint32_t s0 = lds_u32(lds, blk + 4), s1 = lds_u32(lds, blk + 8), s2 = lds_u32(lds, blk + 12);
        const uint8_t q[12] = {(uint8_t) s0, (uint8_t) (s0 >> 8), (uint8_t) (s0 >> 16), (uint8_t) (s0 >> 24),
                               (uint8_t) s1, (uint8_t) (s1 >> 8), (uint8_t) (s1 >> 16), (uint8_t) (s1 >> 24),
                               (uint8_t) s2, (uint8_t) (s2 >> 8), (uint8_t) (s2 >> 16), (uint8_t) (s2 >> 24)};
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) scale_min_k4(j, q, sc[j], mn[j]);
        int sumi = 0;
        for (int j = 0; j < 4; ++j) {
            const uint32_t wq = lds_u32(lds, blk + 16 + 32 * j + 4 * n);
            const int lo = (int) (wq & 0x0F0F0F0Fu), hi = (int) ((wq >> 4) & 0x0F0F0F0Fu);
            const int alo = (int) lds_u32(lds, yb + 4 + 64 * j + 4 * n);
            const int ahi = (int) lds_u32(lds, yb + 4 + 64 * j + 32 + 4 * n);
            sumi += mul24(sc[2 * j], sdot4(lo, alo, 0)) + mul24(sc[2 * j + 1], sdot4(hi, ahi, 0));
        }
        const float yd = lds_f32(lds, yb);
        const float d = yd * h2f((uint16_t) (h0 & 0xffff));
        acc = __builtin_fmaf(d, (float) sumi, acc);
        if (n < 4) {
            const uint32_t bs01 = lds_u32(lds, yb + 260 + 8 * n), bs23 = lds_u32(lds, yb + 260 + 8 * n + 4);
            const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
            const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
            const int prod = mul24(mn[2 * n], q8s0) + mul24(mn[2 * n + 1], q8s1);
            const float dmin = -yd * h2f((uint16_t) (h0 >> 16));
            accm = __builtin_fmaf(dmin, (float) prod, accm);
        }
    }
    // hsum_float_8(acc) + ((m0 + m2) + (m1 + m3))
    float a = acc;
    a = a + __shfl_down(a, 4, 8);
    a = a + __shfl_down(a, 2, 8);
    a = a + __shfl_down(a, 1, 8);
    float m = accm;
    m = m + __shfl_down(m, 2, 8);
    m = m + __shfl_down(m, 1, 8);
    return a + m;
}

// Q4_K x Q8_K for 4-byte aligned weight and activation rows, NB super-blocks
// known at compile time (unrolled by 4: the LDS reads of four blocks are issued
// together, within the register budget of a 512-thread persistent kernel).
// Same integer lanes and float order as row_dot_lds<T_Q4_K>.
template <int NB>
__device__ __forceinline__ float row_dot_q4k_a(const uint32_t* lds, uint32_t wbase, uint32_t abase, int n) {
    float acc = 0.0f, accm = 0.0f;
    const uint32_t* w = lds + (wbase >> 2);
    const uint32_t* y = lds + (abase >> 2);
#pragma unroll 4
    for (int b = 0; b < NB; ++b) {
        const uint32_t* blk = w + 36 * b;   // 144 bytes
        const uint32_t* yb = y + 73 * b;    // 292 bytes
        const uint32_t h0 = blk[0], s0 = blk[1], s1 = blk[2], s2 = blk[3];
        // the 8 six-bit scales and mins as bytes (the utmp shuffle of quants.c:2067-2072)
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
        const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        int sumi = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t scw = j < 2 ? sc_lo : sc_hi;
            const int sl = (int) ((scw >> (16 * (j & 1))) & 0xff);
            const int sh = (int) ((scw >> (16 * (j & 1) + 8)) & 0xff);
            const uint32_t wq = blk[4 + 8 * j + n];
            const int lo = (int) (wq & 0x0F0F0F0Fu), hi = (int) ((wq >> 4) & 0x0F0F0F0Fu);
            sumi += mul24(sl, sdot4(lo, (int) yb[1 + 16 * j + n], 0)) + mul24(sh, sdot4(hi, (int) yb[1 + 16 * j + 8 + n], 0));
        }
        const float yd = bitsf(yb[0]);
        acc = __builtin_fmaf(yd * h2f((uint16_t) (h0 & 0xffff)), (float) sumi, acc);
        if (n < 4) {
            const uint32_t bs01 = yb[65 + 2 * n], bs23 = yb[66 + 2 * n];
            const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
            const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
            const uint32_t mw = n < 2 ? mn_lo : mn_hi;
            const int m0 = (int) ((mw >> (16 * (n & 1))) & 0xff), m1 = (int) ((mw >> (16 * (n & 1) + 8)) & 0xff);
            accm = __builtin_fmaf(-yd * h2f((uint16_t) (h0 >> 16)), (float) (mul24(m0, q8s0) + mul24(m1, q8s1)), accm);
        }
    }
    float a = acc;
    a = a + __shfl_down(a, 4, 8);
    a = a + __shfl_down(a, 2, 8);
    a = a + __shfl_down(a, 1, 8);
    float m = accm;
    m = m + __shfl_down(m, 2, 8);
    m = m + __shfl_down(m, 1, 8);
    return a + m;
}

template <>
__device__ __forceinline__ float row_dot_lds<T_Q6_K>(const uint32_t* lds, uint32_t wbase, uint32_t abase, int nb, int n) {
    float acc = 0.0f;
    const int g = n >= 4 ? 1 : 0;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 210u * b;
        const uint32_t yb = abase + 292u * b;
        int sc[16];
        for (int i = 0; i < 4; ++i) {
            const uint32_t s = lds_u32(lds, blk + 192 + 4 * i);
            sc[4 * i + 0] = (int) (int8_t) (s & 0xff);
            sc[4 * i + 1] = (int) (int8_t) ((s >> 8) & 0xff);
            sc[4 * i + 2] = (int) (int8_t) ((s >> 16) & 0xff);
            sc[4 * i + 3] = (int) (int8_t) (s >> 24);
        }
        int sumi = 0;
        for (int j = 0; j < 2; ++j) {
            const uint32_t qa = lds_u32(lds, blk + 64 * j + 4 * n);
            const uint32_t qb = lds_u32(lds, blk + 64 * j + 32 + 4 * n);
            const uint32_t qh = lds_u32(lds, blk + 128 + 32 * j + 4 * n);
            const int q0 = (int) ((qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
            const int q1 = (int) ((qb & 0x0F0F0F0Fu) | ((qh & 0x0C0C0C0Cu) << 2));
            const int q2 = (int) (((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u));
            const int q3 = (int) (((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u));
            const uint32_t y = yb + 4 + 128 * j + 4 * n;
            sumi += mul24(sc[8 * j + 0 + g], sdot4(q0, (int) lds_u32(lds, y), 0));
            sumi += mul24(sc[8 * j + 2 + g], sdot4(q1, (int) lds_u32(lds, y + 32), 0));
            sumi += mul24(sc[8 * j + 4 + g], sdot4(q2, (int) lds_u32(lds, y + 64), 0));
            sumi += mul24(sc[8 * j + 6 + g], sdot4(q3, (int) lds_u32(lds, y + 96), 0));
        }
        const uint32_t bs = lds_u32(lds, yb + 260 + 4 * n);
        sumi -= 32 * (mul24((int) (int16_t) (bs & 0xffff), sc[2 * n]) + mul24((int) (int16_t) (bs >> 16), sc[2 * n + 1]));
        const float d = lds_f32(lds, yb) * h2f(lds_u16(lds, blk + 208));
        acc = __builtin_fmaf(d, (float) sumi, acc);
    }
    float a = acc;
    a = a + __shfl_down(a, 4, 8);
    a = a + __shfl_down(a, 2, 8);
    a = a + __shfl_down(a, 1, 8);
    return a;
}

template <>
__device__ __forceinline__ float row_dot_lds<T_Q8_0>(const uint32_t* lds, uint32_t wbase, uint32_t abase, int nb, int n) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 34u * b;
        const uint32_t yb = abase + 34u * b;
        const int sumi = sdot4((int) lds_u32(lds, blk + 2 + 4 * n), (int) lds_u32(lds, yb + 2 + 4 * n), 0);
        const float d = h2f(lds_u16(lds, blk)) * h2f(lds_u16(lds, yb));
        acc = __builtin_fmaf(d, (float) sumi, acc);
    }
    float a = acc;
    a = a + __shfl_down(a, 4, 8);
    a = a + __shfl_down(a, 2, 8);
    a = a + __shfl_down(a, 1, 8);
    return a;
}

// The same row dots for NT activation rows at once: each block's weight bits
// are unpacked once and applied to every row, and the NT chains are independent.
// Per activation row the integers and the float sequence are those above.
template <int TYPE, int NT>
__device__ __forceinline__ void row_dot_lds_mt(const uint32_t* lds, uint32_t wbase, const uint32_t* abase, int nb, int n,
                                               float* out);

template <int NT>
__device__ __forceinline__ void reduce8_mt(const float* acc, float* out) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float a = acc[t];
        a = a + __shfl_down(a, 4, 8);
        a = a + __shfl_down(a, 2, 8);
        a = a + __shfl_down(a, 1, 8);
        out[t] = a;
    }
}

// AL: the weight row starts 4-byte aligned in LDS (every 144-byte block then
// does too) and is read one word per load; the activation rows (Q8_K, 292-byte
// blocks, 4-byte aligned staging) always are.
template <bool AL, int NT>
__device__ __forceinline__ void row_dot_q4k_mt(const uint32_t* lds, uint32_t wbase, const uint32_t* abase, int nb,
                                               int n, float* out) {
    auto rw = [&](uint32_t off) { return AL ? lds_u32a(lds, off) : lds_u32(lds, off); };
    float acc[NT], accm[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = accm[t] = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 144u * b;
        const uint32_t h0 = rw(blk);
        const uint32_t s0 = rw(blk + 4), s1 = rw(blk + 8), s2 = rw(blk + 12);
        const uint8_t q[12] = {(uint8_t) s0, (uint8_t) (s0 >> 8), (uint8_t) (s0 >> 16), (uint8_t) (s0 >> 24),
                               (uint8_t) s1, (uint8_t) (s1 >> 8), (uint8_t) (s1 >> 16), (uint8_t) (s1 >> 24),
                               (uint8_t) s2, (uint8_t) (s2 >> 8), (uint8_t) (s2 >> 16), (uint8_t) (s2 >> 24)};
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) scale_min_k4(j, q, sc[j], mn[j]);
        int lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t wq = rw(blk + 16 + 32 * j + 4 * n);
            lo[j] = (int) (wq & 0x0F0F0F0Fu);
            hi[j] = (int) ((wq >> 4) & 0x0F0F0F0Fu);
        }
        const float wd = h2f((uint16_t) (h0 & 0xffff)), wdm = h2f((uint16_t) (h0 >> 16));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t yb = abase[t] + 292u * b;
            int sumi = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int alo = (int) lds_u32a(lds, yb + 4 + 64 * j + 4 * n);
                const int ahi = (int) lds_u32a(lds, yb + 4 + 64 * j + 32 + 4 * n);
                sumi += mul24(sc[2 * j], sdot4(lo[j], alo, 0)) + mul24(sc[2 * j + 1], sdot4(hi[j], ahi, 0));
            }
            const float yd = bitsf(lds_u32a(lds, yb));
            acc[t] = __builtin_fmaf(yd * wd, (float) sumi, acc[t]);
            const int nn = n & 3;
            const uint32_t bs01 = lds_u32a(lds, yb + 260 + 8 * nn), bs23 = lds_u32a(lds, yb + 260 + 8 * nn + 4);
            const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
            const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
            const int prod = mul24(mn[2 * nn], q8s0) + mul24(mn[2 * nn + 1], q8s1);
            const float pm = __builtin_fmaf(-yd * wdm, (float) prod, accm[t]);
            accm[t] = n < 4 ? pm : accm[t];
        }
    }
    float a[NT], m[NT];
    reduce8_mt<NT>(acc, a);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float mm = accm[t];
        mm = mm + __shfl_down(mm, 2, 8);
        mm = mm + __shfl_down(mm, 1, 8);
        m[t] = mm;
        out[t] = a[t] + m[t];
    }
}

template <>
__device__ __forceinline__ void row_dot_lds_mt<T_Q4_K, 4>(const uint32_t* lds, uint32_t wbase, const uint32_t* abase,
                                                          int nb, int n, float* out) {
    row_dot_q4k_mt<false, 4>(lds, wbase, abase, nb, n, out);
}

// The six-bit scales and mins of one Q4_K block, unpacked once (get_scale_min_k4)
// into four words: sc[0..3], sc[4..7], mn[0..3], mn[4..7], one per byte.
__device__ __forceinline__ u32x4 q4k_scale_words(const uint32_t* lds, uint32_t blk) {
    const uint32_t s0 = lds_u32(lds, blk + 4), s1 = lds_u32(lds, blk + 8), s2 = lds_u32(lds, blk + 12);
    const uint8_t q[12] = {(uint8_t) s0, (uint8_t) (s0 >> 8), (uint8_t) (s0 >> 16), (uint8_t) (s0 >> 24),
                           (uint8_t) s1, (uint8_t) (s1 >> 8), (uint8_t) (s1 >> 16), (uint8_t) (s1 >> 24),
                           (uint8_t) s2, (uint8_t) (s2 >> 8), (uint8_t) (s2 >> 16), (uint8_t) (s2 >> 24)};
    u32x4 w = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        int d, m;
        scale_min_k4(j, q, d, m);
        w[j >> 2] |= (uint32_t) d << (8 * (j & 3));
        w[2 + (j >> 2)] |= (uint32_t) m << (8 * (j & 3));
    }
    return w;
}

// row_dot_q4k_mt with the block scales read from a table of q4k_scale_words
// (tab: the row's first block entry, 16 bytes per block).  Same integers and
// float order.
template <bool AL, int NT>
__device__ __forceinline__ void row_dot_q4k_mt_tab(const uint32_t* lds, uint32_t wbase, uint32_t tab,
                                                   const uint32_t* abase, int nb, int n, float* out) {
    auto rw = [&](uint32_t off) { return AL ? lds_u32a(lds, off) : lds_u32(lds, off); };
    float acc[NT], accm[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = accm[t] = 0.0f;
    const int nn = n & 3;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 144u * b;
        const uint32_t h0 = rw(blk);
        const u32x4 sw = *(const u32x4*) (lds + ((tab + 16u * b) >> 2));
        int sc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] = (int) ((sw[j >> 2] >> (8 * (j & 3))) & 0xffu);
        const uint32_t mw = nn < 2 ? sw[2] : sw[3];
        const int mn0 = (int) ((mw >> (16 * (nn & 1))) & 0xffu), mn1 = (int) ((mw >> (16 * (nn & 1) + 8)) & 0xffu);
        int lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t wq = rw(blk + 16 + 32 * j + 4 * n);
            lo[j] = (int) (wq & 0x0F0F0F0Fu);
            hi[j] = (int) ((wq >> 4) & 0x0F0F0F0Fu);
        }
        const float wd = h2f((uint16_t) (h0 & 0xffff)), wdm = h2f((uint16_t) (h0 >> 16));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t yb = abase[t] + 292u * b;
            int sumi = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int alo = (int) lds_u32a(lds, yb + 4 + 64 * j + 4 * n);
                const int ahi = (int) lds_u32a(lds, yb + 4 + 64 * j + 32 + 4 * n);
                sumi += mul24(sc[2 * j], sdot4(lo[j], alo, 0)) + mul24(sc[2 * j + 1], sdot4(hi[j], ahi, 0));
            }
            const float yd = bitsf(lds_u32a(lds, yb));
            acc[t] = __builtin_fmaf(yd * wd, (float) sumi, acc[t]);
            const uint32_t bs01 = lds_u32a(lds, yb + 260 + 8 * nn), bs23 = lds_u32a(lds, yb + 260 + 8 * nn + 4);
            const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
            const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
            const int prod = mul24(mn0, q8s0) + mul24(mn1, q8s1);
            const float pm = __builtin_fmaf(-yd * wdm, (float) prod, accm[t]);
            accm[t] = n < 4 ? pm : accm[t];
        }
    }
    float a[NT];
    reduce8_mt<NT>(acc, a);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float mm = accm[t];
        mm = mm + __shfl_down(mm, 2, 8);
        mm = mm + __shfl_down(mm, 1, 8);
        out[t] = a[t] + mm;
    }
}

template <int NT>
__device__ __forceinline__ void row_dot_q6k_mt(const uint32_t* lds, uint32_t wbase, const uint32_t* abase, int nb,
                                               int n, float* out) {
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    const int g = n >= 4 ? 1 : 0;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 210u * b;
        int sc[16];
        for (int i = 0; i < 4; ++i) {
            const uint32_t s = lds_u32(lds, blk + 192 + 4 * i);
            sc[4 * i + 0] = (int) (int8_t) (s & 0xff);
            sc[4 * i + 1] = (int) (int8_t) ((s >> 8) & 0xff);
            sc[4 * i + 2] = (int) (int8_t) ((s >> 16) & 0xff);
            sc[4 * i + 3] = (int) (int8_t) (s >> 24);
        }
        int q6[2][4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t qa = lds_u32(lds, blk + 64 * j + 4 * n);
            const uint32_t qb = lds_u32(lds, blk + 64 * j + 32 + 4 * n);
            const uint32_t qh = lds_u32(lds, blk + 128 + 32 * j + 4 * n);
            q6[j][0] = (int) ((qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
            q6[j][1] = (int) ((qb & 0x0F0F0F0Fu) | ((qh & 0x0C0C0C0Cu) << 2));
            q6[j][2] = (int) (((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u));
            q6[j][3] = (int) (((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u));
        }
        const float wd = h2f(lds_u16(lds, blk + 208));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t yb = abase[t] + 292u * b;
            int sumi = 0;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t y = yb + 4 + 128 * j + 4 * n;
                sumi += mul24(sc[8 * j + 0 + g], sdot4(q6[j][0], (int) lds_u32a(lds, y), 0));
                sumi += mul24(sc[8 * j + 2 + g], sdot4(q6[j][1], (int) lds_u32a(lds, y + 32), 0));
                sumi += mul24(sc[8 * j + 4 + g], sdot4(q6[j][2], (int) lds_u32a(lds, y + 64), 0));
                sumi += mul24(sc[8 * j + 6 + g], sdot4(q6[j][3], (int) lds_u32a(lds, y + 96), 0));
            }
            const uint32_t bs = lds_u32a(lds, yb + 260 + 4 * n);
            sumi -= 32 * (mul24((int) (int16_t) (bs & 0xffff), sc[2 * n]) + mul24((int) (int16_t) (bs >> 16), sc[2 * n + 1]));
            const float d = bitsf(lds_u32a(lds, yb)) * wd;
            acc[t] = __builtin_fmaf(d, (float) sumi, acc[t]);
        }
    }
    reduce8_mt<NT>(acc, out);
}

template <int NT>
__device__ __forceinline__ void row_dot_q80_mt(const uint32_t* lds, uint32_t wbase, const uint32_t* abase, int nb,
                                               int n, float* out) {
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint32_t blk = wbase + 34u * b;
        const int wq = (int) lds_u32(lds, blk + 2 + 4 * n);
        const float wd = h2f(lds_u16(lds, blk));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t yb = abase[t] + 34u * b;
            const int sumi = sdot4(wq, (int) lds_u32(lds, yb + 2 + 4 * n), 0);
            const float d = wd * h2f(lds_u16(lds, yb));
            acc[t] = __builtin_fmaf(d, (float) sumi, acc[t]);
        }
    }
    reduce8_mt<NT>(acc, out);
}

template <>
__device__ __forceinline__ void row_dot_lds_mt<T_Q6_K, 4>(const uint32_t* lds, uint32_t wbase, const uint32_t* abase,
                                                          int nb, int n, float* out) {
    row_dot_q6k_mt<4>(lds, wbase, abase, nb, n, out);
}

template <>
__device__ __forceinline__ void row_dot_lds_mt<T_Q8_0, 4>(const uint32_t* lds, uint32_t wbase, const uint32_t* abase,
                                                          int nb, int n, float* out) {
    row_dot_q80_mt<4>(lds, wbase, abase, nb, n, out);
}

}  // namespace qw
