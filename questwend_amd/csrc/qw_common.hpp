// qw_common.hpp -- device-side building blocks shared by every qwmoe kernel.
//
// Block layouts are byte-identical to ggml's (ggml/src/ggml-common.h:252-255,
// 327-337, 362-367, 371-375 of the reference tree); the arithmetic helpers
// reproduce, lane for lane, the float order of ggml's x86 AVX2+FMA CPU backend,
// which is what makes the GPU results bit-identical to it.  All sources are
// compiled with -ffp-contract=off: every fused multiply-add below is explicit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qw {

// Native 4 x u32 vector (arrays of it stay in registers, unlike arrays of uint4).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int WAVE = 64;

enum Type : int { T_F32 = 0, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_Q8_K = 15, T_I32 = 26 };

struct __attribute__((packed)) BlockQ8_0 { uint16_t d; int8_t qs[QK8_0]; };
struct __attribute__((packed)) BlockQ4_K { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; };
struct __attribute__((packed)) BlockQ6_K { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; };
struct __attribute__((packed)) BlockQ8_K { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; };
static_assert(sizeof(BlockQ8_0) == 34, "q8_0 layout");
static_assert(sizeof(BlockQ4_K) == 144, "q4_K layout");
static_assert(sizeof(BlockQ6_K) == 210, "q6_K layout");
static_assert(sizeof(BlockQ8_K) == 292, "q8_K layout");

__host__ __device__ constexpr int block_elems(int t) { return (t == T_Q8_0) ? QK8_0 : (t == T_F32 ? 1 : QK_K); }
__host__ __device__ constexpr int block_bytes(int t) {
    return t == T_Q8_0 ? 34 : t == T_Q4_K ? 144 : t == T_Q6_K ? 210 : t == T_Q8_K ? 292 : t == T_F32 ? 4 : 0;
}
__host__ __device__ constexpr int vec_dot_type(int t) { return t == T_Q8_0 ? T_Q8_0 : T_Q8_K; }

__device__ __forceinline__ uint32_t fbits(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float bitsf(uint32_t u) { return __uint_as_float(u); }

// binary16 <-> binary32, round to nearest even (F16C _cvtss_sh(x, 0) semantics).
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float) v;
}
__device__ __forceinline__ uint16_t f2h(float f) {
    const _Float16 v = (_Float16) f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// ggml-quants.c:621-626: 1.5*2^23 magic add == round half to even for |x| < 2^22.
__device__ __forceinline__ int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i = (int) fbits(val);
    return (i & 0x007fffff) - 0x00400000;
}

// hsum_float_8 (ggml-cpu/arch/x86/quants.c:42-48): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
__device__ __forceinline__ float hsum8(const float a[8]) {
    const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
    return (r0 + r2) + (r1 + r3);
}

// One lane of ggml_v_expf, AVX2+FMA branch (ggml-cpu/vec.h:1215-1254).  The
// constants and step order are ggml's; every fma here is one the AVX2 code does.
__device__ __forceinline__ float v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = __builtin_fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, __builtin_fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = fbits(z) << 23;
    const float k = bitsf(e + 0x3f800000u);
    const float u = b * b;
    const float j = __builtin_fmaf(__builtin_fmaf(__builtin_fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                                                  __builtin_fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                                   u, 0x1.ffffecp-1f * b);
    const float an = __builtin_fabsf(n);
    if (!(an > 126.0f)) return __builtin_fmaf(k, j, k);
    const uint32_t g = (n <= 0.0f) ? 0x82000000u : 0u;
    const float s1 = bitsf(g + 0x7f000000u);
    const float s2 = bitsf(e - g);
    if (an > 192.0f) return s1 * s1;
    return __builtin_fmaf(s2, j, s2) * s1;
}

// ggml_v_silu (vec.h:1256-1263): x / (1 + exp(0 - x)), IEEE division.
__device__ __forceinline__ float v_silu(float x) {
    const float e = v_expf(0.0f - x);
    return x / (1.0f + e);
}

// get_scale_min_k4 (ggml-quants.c:880-887).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& d, int& m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
// a * b for |a|, |b| < 2^23 (v_mul_i32_i24, full rate; a 32-bit multiply is quarter rate)
__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }

// DPP lane exchanges inside a row of 16 lanes (VALU latency, no LDS round trip).
// xor1 / xor2 are exact lane-xor patterns; half_mirror (i <-> 7-i in each 8) and
// mirror (i <-> 15-i) pair lanes across 4- and 8-lane groups, which is all a
// reduction needs once the smaller groups already agree.
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140 };
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// LDS-only workgroup barrier: orders LDS traffic but, unlike __syncthreads,
// does not wait for outstanding global stores to be acknowledged.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Returns v unchanged, but hides where it came from: per-thread addresses
// derived from the result are recomputed where they are used instead of being
// hoisted out of (and kept live across) an enclosing loop.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Unaligned little-endian reads (compiler splits them to what the alignment allows).
template <typename T>
__device__ __forceinline__ T ld_unaligned(const void* p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

// quantize_row_q8_K_ref of one block held by a wave, 4 values per lane
// (values 4*lane .. 4*lane+3).  With h set (the block's 256 slots of an f16 copy
// in the exact Q4_K matrix-core form's layout: 16-byte chunk 8 g + L holds the
// quants of elements 64 g + 4 L + {0, 2, 1, 3} and 64 g + 32 + 4 L + {0, 2, 1, 3})
// each lane also writes its four quants there as f16 (exact).
__device__ __forceinline__ void q8K_h_store(_Float16* h, int lane, int q0, int q1, int q2, int q3) {
    typedef _Float16 h4v __attribute__((ext_vector_type(4)));
    const int c = 8 * (lane >> 4) + (lane & 7), half = (lane >> 3) & 1;
    *(h4v*) (h + 8 * c + 4 * half) = h4v{(_Float16) q0, (_Float16) q2, (_Float16) q1, (_Float16) q3};
}
__device__ __forceinline__ void quant_q8K_wave(const float* v, int lane, BlockQ8_K* y, _Float16* h = nullptr) {
    // first index of the largest |x|: reduce (|x|, -index) lexicographically
    float am = 0.0f;
    int ai = 0x7fffffff;
    for (int i = 0; i < 4; ++i) {
        const float a = __builtin_fabsf(v[i]);
        if (a > am) { am = a; ai = 4 * lane + i; }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float om = __shfl_xor(am, off);
        const int oi = __shfl_xor(ai, off);
        if (om > am || (om == am && oi < ai)) { am = om; ai = oi; }
    }
    if (!(am > 0.0f)) {  // amax == 0: d = 0, qs = 0 (bsums written as 0)
        *(int*) &y->qs[4 * lane] = 0;
        if (lane < 16) y->bsums[lane] = 0;
        if (lane == 0) y->d = 0.0f;
        if (h) q8K_h_store(h, lane, 0, 0, 0, 0);
        return;
    }
    // the signed value at that index, from the lane that holds it
    const int sel = ai & 3;
    const float mine = sel == 0 ? v[0] : sel == 1 ? v[1] : sel == 2 ? v[2] : v[3];
    const float maxv = __shfl(mine, ai >> 2);   // same value in every lane
    const float iscale = -127.f / maxv;
    int qv[4];
    int s = 0;
    for (int i = 0; i < 4; ++i) {
        const int t = nearest_int(iscale * v[i]);
        qv[i] = t < 127 ? t : 127;
        s += qv[i];
    }
    *(uint32_t*) &y->qs[4 * lane] =
        (uint32_t) (qv[0] & 0xff) | ((uint32_t) (qv[1] & 0xff) << 8) | ((uint32_t) (qv[2] & 0xff) << 16) |
        ((uint32_t) (qv[3] & 0xff) << 24);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) y->bsums[lane >> 2] = (int16_t) s;
    if (lane == 0) y->d = 1.0f / iscale;
    if (h) q8K_h_store(h, lane, qv[0], qv[1], qv[2], qv[3]);
}

}  // namespace qw
