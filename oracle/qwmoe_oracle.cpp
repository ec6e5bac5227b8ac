// qwmoe_oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A plain CPU restatement of the reference's quantized MoE expert-FFN path,
// written from the ggml sources vendored in kishida/questwend (ggml commit
// 8e7f22b67ef4667b4ddd50230771287f328cfb3f, third_party/ggml).  Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
// as the checker.  The product library (questwend_amd/) never links it and has
// no CPU fallback.
//
// Float semantics: the reference CPU backend is ggml's non-native x86 build
// (AVX2 + FMA + F16C branch).  Every SIMD lane of that branch is restated here
// as scalar code, so the float results are bit-identical, not just close:
// integer lane partitions, fma chains and horizontal-sum trees are the same.
// This file is built with -ffp-contract=off; every fused multiply-add the
// reference performs is written as an explicit fmaf().
//
// Citations are relative to /root/reference/third_party/ggml/src unless noted.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

constexpr int QK_K  = 256;   // ggml-common.h:89
constexpr int QK8_0 = 32;    // ggml-common.h:251

// ---------------------------------------------------------------------------
// Block layouts, byte-identical to ggml-common.h:252-255, 327-337, 362-367, 371-375.
#pragma pack(push, 1)
struct BlockQ8_0 { uint16_t d; int8_t qs[QK8_0]; };                              // 34 B
struct BlockQ4_K { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; };  // 144 B
struct BlockQ6_K { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; }; // 210 B
struct BlockQ8_K { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; };         // 292 B
#pragma pack(pop)
static_assert(sizeof(BlockQ8_0) == 34, "q8_0");
static_assert(sizeof(BlockQ4_K) == 144, "q4_K");
static_assert(sizeof(BlockQ6_K) == 210, "q6_K");
static_assert(sizeof(BlockQ8_K) == 292, "q8_K");

enum { T_F32 = 0, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_Q8_K = 15 };  // ggml.h:390-416

inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

// IEEE binary16 conversions, round-to-nearest-even (what F16C's
// _cvtss_sh(x, 0) does and what ggml's software ggml_compute_fp32_to_fp16
// produces for finite inputs).
uint16_t f32_to_f16(float f) {
    uint32_t x = fbits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);  // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {  // subnormal half (or zero)
        // value = ax_float; half subnormal unit = 2^-24
        float a = bitsf(ax);
        // exact scaling by 2^24 then RNE to integer
        float s = a * 16777216.0f;           // exact (power of two)
        float r = std::nearbyint(s);         // default rounding mode is RNE
        return (uint16_t) (sign | (uint32_t) r);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  // carries into exponent correctly
    return (uint16_t) (sign | h);
}

float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        float v = (float) m * (1.0f / 16777216.0f);  // exact
        return sign ? -v : v;
    }
    if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
    return bitsf(sign | ((e - 15 + 127) << 23) | (m << 13));
}

// ggml-quants.c:621-626 (the 1.5*2^23 magic add: round half to even).
inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i; memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

// ---------------------------------------------------------------------------
// Quantizers.

// quantize_row_q8_0_ref, ggml-quants.c:276-297 (used for Q8_0 *weights* via
// quantize_q8_0, ggml-quants.c:2295-2300).
void quantize_row_q8_0_ref(const float * x, BlockQ8_0 * y, int64_t k) {
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = std::max(amax, std::fabs(x[i * QK8_0 + j]));
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = f32_to_f16(d);
        for (int j = 0; j < QK8_0; ++j) {
            const float x0 = x[i * QK8_0 + j] * id;
            y[i].qs[j] = (int8_t) std::roundf(x0);
        }
    }
}

// AVX2 quantize_row_q8_0, ggml-cpu/arch/x86/quants.c:302-404 (the Q8_0
// *activation* quantizer mul_mat_id uses).  Differs from the _ref above:
// id = 127/maxAbs (not 1/d) and round-half-even (_mm256_round_ps NEAREST).
void quantize_row_q8_0_x86(const float * x, BlockQ8_0 * y, int64_t k) {
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float * v = x + i * QK8_0;
        float maxAbs = 0.0f;
        for (int j = 0; j < QK8_0; j++) maxAbs = std::max(maxAbs, std::fabs(v[j]));  // max is order-free
        const float d = maxAbs / 127.f;
        y[i].d = f32_to_f16(d);
        const float id = (maxAbs != 0.0f) ? 127.f / maxAbs : 0.0f;
        for (int j = 0; j < QK8_0; j++) {
            float r = std::nearbyint(v[j] * id);   // RNE; |r| <= 127 so the saturating packs never clip
            y[i].qs[j] = (int8_t) (int) r;
        }
    }
}

// quantize_row_q8_K_ref, ggml-quants.c:2768-2803 (x86 quantize_row_q8_K calls
// it: ggml-cpu/arch/x86/quants.c:505-507).  amax == 0 leaves bsums untouched in
// the reference; here they are zeroed (the dot products multiply them by d=0).
void quantize_row_q8_K(const float * x, BlockQ8_K * y, int64_t k) {
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; ++j) {
            float ax = std::fabs(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        if (!amax) {
            y[i].d = 0;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            x += QK_K;
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; ++j) {
            int v = nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t) std::min(127, v);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t) sum;
        }
        y[i].d = 1 / iscale;
        x += QK_K;
    }
}

// make_qkx2_quants, ggml-quants.c:799-878.
float make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L,
                       float * the_min, uint8_t * Laux, float rmin, float rdelta, int nstep,
                       bool use_mad) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t) std::max(0, std::min(nmax, l));
        float diff = scale * L[i] + min - x[i];
        diff = use_mad ? std::fabs(diff) : diff * diff;
        float w = weights[i];
        best_error += w * diff;
    }
    if (nstep < 1) { *the_min = -min; return scale; }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = std::max(0, std::min(nmax, l));
            Laux[i] = (uint8_t) l;
            float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min   = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) { this_min = 0; this_scale = sum_xl / sum_l2; }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = use_mad ? std::fabs(diff) : diff * diff;
                float w = weights[i];
                cur_error += w * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

// get_scale_min_k4, ggml-quants.c:880-887.
inline void get_scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

// quantize_row_q4_K_ref, ggml-quants.c:1457-1527 (quantize_q4_K with no
// imatrix, 1626-1640).
void quantize_row_q4_K_ref(const float * x, BlockQ4_K * y, int64_t k) {
    const int64_t nb = k / QK_K;
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int64_t i = 0; i < nb; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            float av_x = std::sqrt(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux,
                                         -1.f, 0.1f, 20, false);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        float inv_min   = max_min > 0 ? 63.f / max_min : 0.f;
        memset(y[i].scales, 0, 12);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t) nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t) nearest_int(inv_min * mins[j]);
            ls = std::min<uint8_t>(63, ls);
            lm = std::min<uint8_t>(63, lm);
            if (j < 4) { y[i].scales[j] = ls; y[i].scales[j + 4] = lm; }
            else {
                y[i].scales[j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
                y[i].scales[j - 4] |= (uint8_t) ((ls >> 4) << 6);
                y[i].scales[j - 0] |= (uint8_t) ((lm >> 4) << 6);
            }
        }
        y[i].d = f32_to_f16(max_scale / 63.f);
        y[i].dmin = f32_to_f16(max_min / 63.f);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = f16_to_f32(y[i].d) * sc;
            if (!d) continue;
            const float dm = f16_to_f32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                L[32 * j + ii] = (uint8_t) std::max(0, std::min(15, l));
            }
        }
        uint8_t * q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += QK_K;
    }
}

// make_qx_quants, ggml-quants.c:628-700 (rmse_type 1, no quant weights).
float make_qx_quants(int n, int nmax, const float * x, int8_t * L, int rmse_type) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        float ax = std::fabs(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {  // GROUP_MAX_EPS
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            L[i] = (int8_t) (nmax + std::max(-nmax, std::min(nmax - 1, l)));
        }
        return 1 / iscale;
    }
    bool return_early = false;
    if (rmse_type < 0) { rmse_type = -rmse_type; return_early = true; }
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = std::max(-nmax, std::min(nmax - 1, l));
        L[i] = (int8_t) (l + nmax);
        float w = rmse_type == 1 ? x[i] * x[i] : rmse_type == 2 ? 1 : rmse_type == 3 ? std::fabs(x[i]) : std::sqrt(std::fabs(x[i]));
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    if (return_early) return suml2 > 0 ? 0.5f * (scale + 1 / iscale) : 1 / iscale;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = std::max(-nmax, std::min(nmax - 1, l));
            float w = rmse_type == 1 ? x[i] * x[i] : rmse_type == 2 ? 1 : rmse_type == 3 ? std::fabs(x[i]) : std::sqrt(std::fabs(x[i]));
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t) (nmax + std::max(-nmax, std::min(nmax - 1, l)));
            }
            scale = sumlx / suml2; best = scale * sumlx;
        }
    }
    return scale;
}

// quantize_row_q6_K_ref, ggml-quants.c:1869-1937 (quantize_q6_K, 2054-2068).
void quantize_row_q6_K_ref(const float * x, BlockQ6_K * y, int64_t k) {
    const int64_t nb = k / QK_K;
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < nb; i++) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, 1);
            scales[ib] = scale;
            const float abs_scale = std::fabs(scale);
            if (abs_scale > max_abs_scale) { max_abs_scale = abs_scale; max_scale = scale; }
        }
        if (max_abs_scale < 1e-15f) {
            memset(&y[i], 0, sizeof(BlockQ6_K));
            y[i].d = f32_to_f16(0.f);
            x += QK_K;
            continue;
        }
        float iscale = -128.f / max_scale;
        y[i].d = f32_to_f16(1 / iscale);
        for (int ib = 0; ib < QK_K / 16; ++ib) y[i].scales[ib] = (int8_t) std::min(127, nearest_int(iscale * scales[ib]));
        for (int j = 0; j < QK_K / 16; ++j) {
            float d = f16_to_f32(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = std::max(-32, std::min(31, l));
                L[16 * j + ii] = (int8_t) (l + 32);
            }
        }
        uint8_t * ql = y[i].ql;
        uint8_t * qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0]  = (uint8_t) (q1 | (q3 << 4));
                ql[l + 32] = (uint8_t) (q2 | (q4 << 4));
                qh[l] = (uint8_t) ((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                   ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += QK_K;
    }
}

// ---------------------------------------------------------------------------
// Dequantizers: ggml-quants.c:553-566 (q8_0), 1529-1551 (q4_K), 1939-1968 (q6_K).
void dequantize_row_q8_0(const BlockQ8_0 * x, float * y, int64_t k) {
    for (int64_t i = 0; i < k / QK8_0; i++) {
        const float d = f16_to_f32(x[i].d);
        for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = x[i].qs[j] * d;
    }
}
void dequantize_row_q4_K(const BlockQ4_K * x, float * y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++) {
        const uint8_t * q = x[i].qs;
        const float d = f16_to_f32(x[i].d), min = f16_to_f32(x[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = min * m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32; is += 2;
        }
    }
}
void dequantize_row_q6_K(const BlockQ6_K * x, float * y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d = f16_to_f32(x[i].d);
        const uint8_t * ql = x[i].ql;
        const uint8_t * qh = x[i].qh;
        const int8_t * sc = x[i].scales;
        for (int n = 0; n < QK_K; n += 128) {
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                const int8_t q1 = (int8_t) ((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t) ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t) ((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0]  = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128; ql += 64; qh += 32; sc += 8;
        }
    }
}

// ---------------------------------------------------------------------------
// Dot products, restated lane by lane from the AVX2 branch.

// hsum_float_8, ggml-cpu/arch/x86/quants.c:42-48:
// ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
inline float hsum8(const float a[8]) {
    float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
    float s0 = r0 + r2, s1 = r1 + r3;
    return s0 + s1;
}

// Unpack the 12 scale bytes of a Q4_K block into 8 scales and 8 mins (the
// utmp shuffle in quants.c:2067-2072 computes exactly get_scale_min_k4).
inline void q4k_scales_mins(const uint8_t * s12, int sc[8], int mn[8]) {
    for (int j = 0; j < 8; ++j) {
        uint8_t a, b;
        get_scale_min_k4(j, s12, &a, &b);
        sc[j] = a; mn[j] = b;
    }
}

// Integer lanes of one Q4_K x Q8_K super-block (quants.c:2062-2105):
//   sumi[n] (n=0..7) = sum_j sc[2j]  * sum_{b in [4n,4n+4)} q4lo(32j+b)*q8[64j+b]
//                    + sc[2j+1]      * sum_{b in [4n,4n+4)} q4hi(32j+b)*q8[64j+32+b]
//   prod[i] (i=0..3) = mn[2i]*(bs[4i]+bs[4i+1]) + mn[2i+1]*(bs[4i+2]+bs[4i+3])
void q4k_lanes(const BlockQ4_K & x, const BlockQ8_K & y, int32_t sumi[8], int32_t prod[4]) {
    int sc[8], mn[8];
    q4k_scales_mins(x.scales, sc, mn);
    for (int n = 0; n < 8; ++n) {
        int32_t acc = 0;
        for (int j = 0; j < 4; ++j) {
            int32_t lo = 0, hi = 0;
            for (int b = 4 * n; b < 4 * n + 4; ++b) {
                const uint8_t q = x.qs[32 * j + b];
                lo += (q & 0xF) * y.qs[64 * j + b];
                hi += (q >> 4) * y.qs[64 * j + 32 + b];
            }
            acc += sc[2 * j] * lo + sc[2 * j + 1] * hi;
        }
        sumi[n] = acc;
    }
    for (int i = 0; i < 4; ++i) {
        const int q8s0 = y.bsums[4 * i + 0] + y.bsums[4 * i + 1];
        const int q8s1 = y.bsums[4 * i + 2] + y.bsums[4 * i + 3];
        prod[i] = mn[2 * i] * q8s0 + mn[2 * i + 1] * q8s1;
    }
}

// ggml_vec_dot_q4_K_q8_K, AVX2 branch, ggml-cpu/arch/x86/quants.c:2038-2115.
float vec_dot_q4_K_q8_K(int n, const BlockQ4_K * x, const BlockQ8_K * y) {
    const int nb = n / QK_K;
    float acc[8] = {0}, acc_m[4] = {0};
    for (int i = 0; i < nb; ++i) {
        const float d = y[i].d * f16_to_f32(x[i].d);
        const float dmin = -y[i].d * f16_to_f32(x[i].dmin);
        int32_t sumi[8], prod[4];
        q4k_lanes(x[i], y[i], sumi, prod);
        for (int l = 0; l < 4; ++l) acc_m[l] = std::fmaf(dmin, (float) prod[l], acc_m[l]);
        for (int l = 0; l < 8; ++l) acc[l] = std::fmaf(d, (float) sumi[l], acc[l]);
    }
    const float m01 = acc_m[0] + acc_m[2], m23 = acc_m[1] + acc_m[3];
    return hsum8(acc) + (m01 + m23);
}

// Integer lanes of one Q6_K x Q8_K super-block (quants.c:2449-2504):
//   sumi[n] = sum_{j<2,m<4} sc[8j+2m+(n>=4)] * sum_{b in [4n,4n+4)} q6u(128j+32m+b)*q8[128j+32m+b]
//             - 32*(bs[2n]*sc[2n] + bs[2n+1]*sc[2n+1])
void q6k_lanes(const BlockQ6_K & x, const BlockQ8_K & y, int32_t sumi[8]) {
    for (int n = 0; n < 8; ++n) {
        int32_t acc = 0;
        for (int j = 0; j < 2; ++j) {
            const uint8_t * ql = x.ql + 64 * j;
            const uint8_t * qh = x.qh + 32 * j;
            for (int m = 0; m < 4; ++m) {
                const int scv = x.scales[8 * j + 2 * m + (n >= 4 ? 1 : 0)];
                int32_t s = 0;
                for (int b = 4 * n; b < 4 * n + 4; ++b) {
                    int q;
                    switch (m) {
                        case 0: q = (ql[b] & 0xF) | ((qh[b] & 3) << 4); break;
                        case 1: q = (ql[32 + b] & 0xF) | (((qh[b] >> 2) & 3) << 4); break;
                        case 2: q = (ql[b] >> 4) | (((qh[b] >> 4) & 3) << 4); break;
                        default: q = (ql[32 + b] >> 4) | (((qh[b] >> 6) & 3) << 4); break;
                    }
                    s += q * y.qs[128 * j + 32 * m + b];
                }
                acc += scv * s;
            }
        }
        acc -= 32 * (y.bsums[2 * n] * x.scales[2 * n] + y.bsums[2 * n + 1] * x.scales[2 * n + 1]);
        sumi[n] = acc;
    }
}

// ggml_vec_dot_q6_K_q8_K, AVX2 branch, ggml-cpu/arch/x86/quants.c:2426-2508.
float vec_dot_q6_K_q8_K(int n, const BlockQ6_K * x, const BlockQ8_K * y) {
    const int nb = n / QK_K;
    float acc[8] = {0};
    for (int i = 0; i < nb; ++i) {
        const float d = y[i].d * f16_to_f32(x[i].d);
        int32_t sumi[8];
        q6k_lanes(x[i], y[i], sumi);
        for (int l = 0; l < 8; ++l) acc[l] = std::fmaf(d, (float) sumi[l], acc[l]);
    }
    return hsum8(acc);
}

// Integer lanes of one Q8_0 x Q8_0 block: lane n = sum of bytes [4n, 4n+4)
// (mul_sum_i8_pairs_float, quants.c:121-133).
void q8_0_lanes(const BlockQ8_0 & x, const BlockQ8_0 & y, int32_t sumi[8]) {
    for (int n = 0; n < 8; ++n) {
        int32_t s = 0;
        for (int b = 4 * n; b < 4 * n + 4; ++b) s += x.qs[b] * y.qs[b];
        sumi[n] = s;
    }
}

// ggml_vec_dot_q8_0_q8_0, AVX2 branch, ggml-cpu/arch/x86/quants.c:1308-1370.
float vec_dot_q8_0_q8_0(int n, const BlockQ8_0 * x, const BlockQ8_0 * y) {
    const int nb = n / QK8_0;
    float acc[8] = {0};
    for (int ib = 0; ib < nb; ++ib) {
        const float d = f16_to_f32(x[ib].d) * f16_to_f32(y[ib].d);
        int32_t sumi[8];
        q8_0_lanes(x[ib], y[ib], sumi);
        for (int l = 0; l < 8; ++l) acc[l] = std::fmaf(d, (float) sumi[l], acc[l]);
    }
    return hsum8(acc);
}

// ggml_vec_dot_f32, AVX (8-lane) branch: vec.cpp:11-140 with GGML_F32_STEP=32,
// GGML_F32_EPR=8 and GGML_F32x8_REDUCE (ggml-cpu/simd-mappings.h:579-629).
// The scalar tail `sumf += x[i]*y[i]` (n % 32 leftovers) is compiled by GCC at
// the reference's -O3 -mfma (default -ffp-contract=fast) as a 4-wide vector
// multiply with an in-order add for each full group of 4, and an fma for the
// last n % 4 elements.  tail_mode 2 restates that (pinned against the compiled
// reference for every n % 32 in the tests); 0 = plain mul+add, 1 = all fma.
float vec_dot_f32(int n, const float * x, const float * y, int tail_mode) {
    const int np = n & ~31;
    float sum[4][8] = {{0}};
    for (int i = 0; i < np; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l)
                sum[j][l] = std::fmaf(x[i + 8 * j + l], y[i + 8 * j + l], sum[j][l]);
    for (int l = 0; l < 8; ++l) {
        sum[0][l] = sum[0][l] + sum[2][l];
        sum[1][l] = sum[1][l] + sum[3][l];
    }
    for (int l = 0; l < 8; ++l) sum[0][l] = sum[0][l] + sum[1][l];
    float t0[4];
    for (int l = 0; l < 4; ++l) t0[l] = sum[0][l] + sum[0][l + 4];
    // _mm_hadd_ps twice: (t0+t1) + (t2+t3)
    float sumf = (t0[0] + t0[1]) + (t0[2] + t0[3]);
    const int nv = np + ((n - np) & ~3);
    for (int i = np; i < n; ++i) {
        const bool fused = tail_mode == 1 || (tail_mode == 2 && i >= nv);
        sumf = fused ? std::fmaf(x[i], y[i], sumf) : sumf + x[i] * y[i];
    }
    return sumf;
}

// ggml_v_expf, AVX2+FMA branch, ggml-cpu/vec.h:1215-1254, one lane.  The
// constants and the step order are ggml's (adapted there from Arm's optimized
// routines); keeping them is what makes the router probabilities bit-exact.
float v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = std::fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = std::fmaf(-n, 0x1.7f7d1cp-20f, std::fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = fbits(z) << 23;
    const float k = bitsf(e + fbits(1.0f));
    const bool c = std::fabs(n) > 126.0f;
    const float u = b * b;
    const float j = std::fmaf(std::fmaf(std::fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                                        std::fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                              u, 0x1.ffffecp-1f * b);
    if (!c) return std::fmaf(k, j, k);
    const uint32_t g = (n <= 0.0f) ? 0x82000000u : 0u;
    const float s1 = bitsf(g + 0x7f000000u);
    const float s2 = bitsf(e - g);
    if (std::fabs(n) > 192.0f) return s1 * s1;
    return std::fmaf(s2, j, s2) * s1;
}

// ggml_v_silu, vec.h:1256-1263 (AVX2 branch), one lane.
inline float v_silu(float x) {
    const float neg_x = 0.0f - x;
    const float e = v_expf(neg_x);
    return x / (1.0f + e);
}

// ggml_silu_f32, vec.h:1046-1048 (scalar tail; libm expf).
inline float silu_scalar(float x) { return x / (1.0f + expf(-x)); }

// ggml_vec_swiglu_f32, vec.cpp:417-445 (AVX2 branch + scalar tail).
void vec_swiglu(int n, float * y, const float * x, const float * g) {
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int l = 0; l < 8; ++l) y[i + l] = v_silu(x[i + l]) * g[i + l];
    for (; i < n; ++i) y[i] = silu_scalar(x[i]) * g[i];
}

// ggml_compute_forward_soft_max_f32 (ops.cpp:5455-5566, scale 1, no mask, no
// sinks) with ggml_vec_soft_max_f32 (vec.cpp:531-) for one row.
void soft_max_row(int n, const float * x, float * y) {
    float max = -INFINITY;
    for (int i = 0; i < n; ++i) max = std::max(max, x[i]);   // ggml_vec_max_f32 (MAX macro)
    double sum = 0;
    int i = 0;
    for (; i + 7 < n; i += 8) {
        float v[8];
        for (int l = 0; l < 8; ++l) { v[l] = v_expf(x[i + l] - max); y[i + l] = v[l]; }
        sum += (double) hsum8(v);
    }
    for (; i < n; ++i) {
        float v = expf(x[i] - max);
        sum += (double) v;
        y[i] = v;
    }
    sum = 1.0 / sum;
    const float s = (float) sum;
    for (int l = 0; l < n; ++l) y[l] *= s;
}

// ARGSORT DESC (ops.cpp:8332-8382): std::sort of indices with data[a] > data[b].
void argsort_desc(int n, const float * x, int32_t * idx) {
    for (int j = 0; j < n; ++j) idx[j] = j;
    std::sort(idx, idx + n, [x](int32_t a, int32_t b) { return x[a] > x[b]; });
}

// RMS_NORM (ops.cpp:3795-3860), one row.
void rms_norm_row(int n, const float * x, float * y, float eps) {
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += (double) (x[i] * x[i]);
    const float mean = (float) (sum / n);
    const float scale = 1.0f / std::sqrt(mean + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * scale;
}

size_t row_size(int type, int64_t n) {
    switch (type) {
        case T_F32:  return 4 * (size_t) n;
        case T_Q8_0: return (size_t) (n / QK8_0) * sizeof(BlockQ8_0);
        case T_Q4_K: return (size_t) (n / QK_K) * sizeof(BlockQ4_K);
        case T_Q6_K: return (size_t) (n / QK_K) * sizeof(BlockQ6_K);
        case T_Q8_K: return (size_t) (n / QK_K) * sizeof(BlockQ8_K);
    }
    return 0;
}

// type_traits_cpu (ggml-cpu.c:271-281, 310-319, 326-335): weight type ->
// activation (vec_dot) type.
int vec_dot_type(int type) { return type == T_Q8_0 ? T_Q8_0 : T_Q8_K; }

void from_float(int vdt, const float * x, void * y, int64_t n) {
    if (vdt == T_Q8_0) quantize_row_q8_0_x86(x, (BlockQ8_0 *) y, n);
    else quantize_row_q8_K(x, (BlockQ8_K *) y, n);
}

float vec_dot(int type, int n, const void * x, const void * y) {
    switch (type) {
        case T_Q4_K: return vec_dot_q4_K_q8_K(n, (const BlockQ4_K *) x, (const BlockQ8_K *) y);
        case T_Q6_K: return vec_dot_q6_K_q8_K(n, (const BlockQ6_K *) x, (const BlockQ8_K *) y);
        case T_Q8_0: return vec_dot_q8_0_q8_0(n, (const BlockQ8_0 *) x, (const BlockQ8_0 *) y);
    }
    return NAN;
}

}  // namespace

extern "C" {

uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
size_t orc_row_size(int type, int64_t n) { return row_size(type, n); }

// ggml_quantize_chunk(type, src, dst, 0, nrows, n_per_row, NULL), ggml.c:7919-8000.
int orc_quantize(int type, const float * src, void * dst, int64_t nrows, int64_t n_per_row) {
    const int64_t n = nrows * n_per_row;
    switch (type) {
        case T_Q8_0: quantize_row_q8_0_ref(src, (BlockQ8_0 *) dst, n); return 0;
        case T_Q4_K: quantize_row_q4_K_ref(src, (BlockQ4_K *) dst, n); return 0;
        case T_Q6_K: quantize_row_q6_K_ref(src, (BlockQ6_K *) dst, n); return 0;
        case T_Q8_K: quantize_row_q8_K(src, (BlockQ8_K *) dst, n); return 0;
    }
    return -1;
}

// type_traits_cpu[type].from_float on x86 (activation quantizers).
int orc_from_float(int type, const float * x, void * y, int64_t n) {
    if (type != T_Q8_0 && type != T_Q8_K) return -1;
    from_float(type, x, y, n);
    return 0;
}

int orc_dequantize(int type, const void * x, float * y, int64_t n) {
    switch (type) {
        case T_Q8_0: dequantize_row_q8_0((const BlockQ8_0 *) x, y, n); return 0;
        case T_Q4_K: dequantize_row_q4_K((const BlockQ4_K *) x, y, n); return 0;
        case T_Q6_K: dequantize_row_q6_K((const BlockQ6_K *) x, y, n); return 0;
    }
    return -1;
}

int orc_vec_dot(int type, int n, const void * x, const void * y, float * s) {
    *s = vec_dot(type, n, x, y);
    return 0;
}

// The integer lanes behind one vec_dot, for every super-block of the row:
// out[nb][8] (q4_K: plus prod[nb][4] in out2; q6_K / q8_0: out2 unused).
int orc_dot_lanes(int type, int n, const void * x, const void * y, int32_t * out, int32_t * out2) {
    if (type == T_Q4_K) {
        for (int i = 0; i < n / QK_K; ++i)
            q4k_lanes(((const BlockQ4_K *) x)[i], ((const BlockQ8_K *) y)[i], out + 8 * i, out2 + 4 * i);
    } else if (type == T_Q6_K) {
        for (int i = 0; i < n / QK_K; ++i)
            q6k_lanes(((const BlockQ6_K *) x)[i], ((const BlockQ8_K *) y)[i], out + 8 * i);
    } else if (type == T_Q8_0) {
        for (int i = 0; i < n / QK8_0; ++i)
            q8_0_lanes(((const BlockQ8_0 *) x)[i], ((const BlockQ8_0 *) y)[i], out + 8 * i);
    } else {
        return -1;
    }
    return 0;
}

float orc_vec_dot_f32(int n, const float * x, const float * y, int tail_mode) {
    return vec_dot_f32(n, x, y, tail_mode);
}
float orc_v_expf(float x) { return v_expf(x); }
// Number of steps down the float line where v_expf increases: x runs over the
// bit patterns first..last (negative floats, so x decreases as the pattern
// grows) and a step counts when v_expf(next) > v_expf(previous).  A property
// of the restatement (bit-identical to ggml_v_expf), used by the tests that
// support the GPU router's shortcut: a larger logit never gets a smaller exp.
int64_t orc_v_expf_increases(uint32_t first, uint32_t last) {
    int64_t bad = 0;
    float x;
    std::memcpy(&x, &first, 4);
    float prev = v_expf(x);
    for (uint32_t b = first; b != last;) {
        ++b;
        std::memcpy(&x, &b, 4);
        const float y = v_expf(x);
        if (y > prev) ++bad;
        prev = y;
    }
    return bad;
}
void orc_swiglu(int64_t n, const float * gate, const float * up, float * out) { vec_swiglu((int) n, out, gate, up); }
void orc_soft_max(int64_t ne0, int64_t ne1, const float * x, float * y) {
    for (int64_t r = 0; r < ne1; ++r) soft_max_row((int) ne0, x + r * ne0, y + r * ne0);
}
void orc_argsort_desc(int64_t ne0, int64_t ne1, const float * x, int32_t * idx) {
    for (int64_t r = 0; r < ne1; ++r) argsort_desc((int) ne0, x + r * ne0, idx + r * ne0);
}
void orc_rms_norm(int64_t ne0, int64_t ne1, const float * x, float * y, float eps) {
    for (int64_t r = 0; r < ne1; ++r) rms_norm_row((int) ne0, x + r * ne0, y + r * ne0, eps);
}

// The router input of a decoder layer: ggml_mul(ggml_rms_norm(x, eps), w)
// (core/runtime.cpp:2028-2030; ops.cpp:3795-3860, then the element-wise
// binary op, one rounding per op).
void orc_rms_norm_mul(int64_t ne0, int64_t ne1, const float * x, const float * w, float * y, float eps) {
    for (int64_t r = 0; r < ne1; ++r) {
        rms_norm_row((int) ne0, x + r * ne0, y + r * ne0, eps);
        for (int64_t i = 0; i < ne0; ++i) y[r * ne0 + i] = y[r * ne0 + i] * w[i];
    }
}

// The shared-expert branch of build_moe (core/runtime.cpp:963-972), token by
// token: g = mul_mat(gate, x), u = mul_mat(up, x) (ggml_mul_mat of a quantized
// weight: x to the weight's vec_dot type, then one vec_dot per row),
// a = mul(silu(g), u) (ggml_vec_silu_f32 takes ggml_v_silu for every block of 8,
// then one multiply: vec_swiglu's rounding), sh = mul_mat(down, a),
// sg = sigmoid(mul_mat(gate_inp, x)) with the f32 dot in vec_dot_f32's order and
// op_sigmoid's 1 / (1 + expf(-v)) (unary-ops.cpp:31-33, libm expf), then
// out = (moe_out + sh * sg) (+ resid): ggml_mul, ggml_add, the residual add.
// Weights dense: gate / up [F][row(H)], down [H][row(F)]; x, moe_out, resid,
// out [T][H].  Needs F % 8 == 0.
int orc_shared_expert_add(int64_t H, int64_t F, int type_gate, int type_up, int type_down, const void * gate,
                          const void * up, const void * down, const float * gate_inp, const float * x, int64_t T,
                          const float * moe_out, const float * resid, float * out) {
    if (F % 8) return -1;
    const size_t rg = row_size(type_gate, H), ru = row_size(type_up, H), rd = row_size(type_down, F);
    const int vg = vec_dot_type(type_gate), vu = vec_dot_type(type_up), vd = vec_dot_type(type_down);
    std::vector<uint8_t> xg(row_size(vg, H)), xu(row_size(vu, H)), aq(row_size(vd, F));
    std::vector<float> g((size_t) F), u((size_t) F), a((size_t) F);
    for (int64_t t = 0; t < T; ++t) {
        const float * xt = x + t * H;
        from_float(vg, xt, xg.data(), H);
        from_float(vu, xt, xu.data(), H);
        for (int64_t f = 0; f < F; ++f) {
            g[(size_t) f] = vec_dot(type_gate, (int) H, (const uint8_t *) gate + (size_t) f * rg, xg.data());
            u[(size_t) f] = vec_dot(type_up, (int) H, (const uint8_t *) up + (size_t) f * ru, xu.data());
        }
        vec_swiglu((int) F, a.data(), g.data(), u.data());
        from_float(vd, a.data(), aq.data(), F);
        const float v = vec_dot_f32((int) H, gate_inp, xt, 2);
        const float sg = 1.f / (1.f + expf(-v));
        for (int64_t h = 0; h < H; ++h) {
            const float sh = vec_dot(type_down, (int) F, (const uint8_t *) down + (size_t) h * rd, aq.data());
            const float o = moe_out[t * H + h] + sh * sg;
            out[t * H + h] = resid ? o + resid[t * H + h] : o;
        }
    }
    return 0;
}

// Per-expert row grouping of ggml_compute_forward_mul_mat_id
// (ggml-cpu.c:1622-1637): t outer, slot e inner.  counts[n_as]; rows holds,
// for each expert a in 0..n_as-1 in order, its (e, t) pairs as 2 x int32,
// concatenated; offsets[n_as+1] is the exclusive prefix sum of counts.
int orc_group_by_expert(const int32_t * ids, int64_t n_ids, int64_t T, int64_t ids_stride,
                        int64_t n_as, int32_t * counts, int32_t * offsets, int32_t * rows) {
    std::vector<std::vector<std::pair<int32_t, int32_t>>> g((size_t) n_as);
    for (int64_t t = 0; t < T; ++t)
        for (int64_t e = 0; e < n_ids; ++e) {
            const int32_t a = ids[t * ids_stride + e];
            if (a < 0 || a >= n_as) return -1;
            g[(size_t) a].push_back({(int32_t) e, (int32_t) t});
        }
    int32_t off = 0;
    for (int64_t a = 0; a < n_as; ++a) {
        counts[a] = (int32_t) g[(size_t) a].size();
        offsets[a] = off;
        for (auto & p : g[(size_t) a]) { rows[2 * off] = p.first; rows[2 * off + 1] = p.second; ++off; }
    }
    offsets[n_as] = off;
    return 0;
}

// ggml_compute_forward_mul_mat_id (ggml-cpu.c:1534-1707) with the contract of
// ggml.c:3315-3328: dst[:, e, t] = as[:, :, ids[e, t]] . b[:, e % b_ne1, t].
// as: [K, N, n_as] of `type` with row stride nb1 and matrix stride nb2 (bytes);
// b: f32 [K, b_ne1, T] dense; ids [T][ids_stride] i32; dst f32 [N, n_ids, T] dense.
// slot_of (nullable): logical id -> slot, applied before indexing `as`
// (the in-graph remap of core/runtime.cpp:913-919).
int orc_mul_mat_id(int type, int64_t K, int64_t N, int64_t n_as, const void * as, size_t nb1,
                   size_t nb2, int64_t b_ne1, int64_t T, const float * b, int64_t n_ids,
                   const int32_t * ids, int64_t ids_stride, const int32_t * slot_of,
                   int64_t n_logical, float * dst) {
    const int vdt = vec_dot_type(type);
    const size_t rs = row_size(vdt, K);
    std::vector<uint8_t> bq((size_t) (b_ne1 * T) * rs);
    for (int64_t t = 0; t < T; ++t)
        for (int64_t r = 0; r < b_ne1; ++r)
            from_float(vdt, b + (t * b_ne1 + r) * K, bq.data() + (size_t) (t * b_ne1 + r) * rs, K);
    for (int64_t t = 0; t < T; ++t)
        for (int64_t e = 0; e < n_ids; ++e) {
            int32_t a = ids[t * ids_stride + e];
            if (slot_of) {
                if (a < 0 || a >= n_logical) return -1;
                a = slot_of[a];
            }
            if (a < 0 || a >= n_as) return -1;
            const uint8_t * mat = (const uint8_t *) as + (size_t) a * nb2;
            const uint8_t * col = bq.data() + (size_t) ((e % b_ne1) + t * b_ne1) * rs;
            float * d = dst + (t * n_ids + e) * N;
            for (int64_t r = 0; r < N; ++r) d[r] = vec_dot(type, (int) K, mat + r * nb1, col);
        }
    return 0;
}

// Router of core/runtime.cpp:869-897: logits = W x (mul_mat, vec_dot_f32),
// soft_max, argsort_top_k, get_rows, sum_rows, clamp(6.103515625e-5, inf), div,
// optional scale.  W: [E][H]; x: [T][H]; ids/weights: [T][k].  With resident-
// only routing (870-881): want = argsort_top_k of the raw logits ([T][k]; NULL:
// not recorded), then logits + mask ([E], ggml_add broadcast over the tokens;
// NULL: none) before the softmax.  logits_out holds the raw logits.
void orc_router_resident(int64_t H, int64_t E, int64_t k, int64_t T, const float * W, const float * x,
                         float scale, const float * mask, int32_t * want, int32_t * ids, float * weights,
                         float * logits_out, float * probs_out) {
    std::vector<float> logits((size_t) E), masked((size_t) E), probs((size_t) E);
    std::vector<int32_t> order((size_t) E);
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t e = 0; e < E; ++e) logits[(size_t) e] = vec_dot_f32((int) H, W + e * H, x + t * H, 2);
        if (want) {
            argsort_desc((int) E, logits.data(), order.data());
            for (int64_t i = 0; i < k; ++i) want[t * k + i] = order[(size_t) i];
        }
        for (int64_t e = 0; e < E; ++e) masked[(size_t) e] = mask ? logits[(size_t) e] + mask[e] : logits[(size_t) e];
        soft_max_row((int) E, masked.data(), probs.data());
        argsort_desc((int) E, probs.data(), order.data());
        double s = 0.0;  // ggml_vec_sum_f32: double accumulation
        for (int64_t i = 0; i < k; ++i) {
            ids[t * k + i] = order[(size_t) i];
            weights[t * k + i] = probs[(size_t) order[(size_t) i]];
            s += (double) weights[t * k + i];
        }
        float wsum = (float) s;
        wsum = std::max(std::min(wsum, INFINITY), 6.103515625e-5f);   // ggml_clamp
        for (int64_t i = 0; i < k; ++i) {
            weights[t * k + i] = weights[t * k + i] / wsum;
            if (scale != 0.0f && scale != 1.0f) weights[t * k + i] *= scale;
        }
        if (logits_out) memcpy(logits_out + t * E, logits.data(), sizeof(float) * E);
        if (probs_out) memcpy(probs_out + t * E, probs.data(), sizeof(float) * E);
    }
}

void orc_router(int64_t H, int64_t E, int64_t k, int64_t T, const float * W, const float * x,
                float scale, int32_t * ids, float * weights, float * logits_out, float * probs_out) {
    orc_router_resident(H, E, k, T, W, x, scale, nullptr, nullptr, ids, weights, logits_out, probs_out);
}

// One MoE FFN layer, core/runtime.cpp:861-974 (resident path), optionally
// followed by RMS_NORM (rms_eps >= 0); resmask / want_out: resident-only routing
// as in orc_router_resident (both nullable).  Weight tensors are [E] matrices of
// [N][row] bytes: gate/up [F rows of H], down [H rows of F]; slot tables
// (nullable) remap logical expert -> slot for each role.  Any output may be NULL.
int orc_moe_layer(int64_t H, int64_t E, int64_t k, int64_t F, int64_t T, int type_gate,
                  int type_up, int type_down, const float * w_router, const void * w_gate,
                  const void * w_up, const void * w_down, int64_t n_slots,
                  const int32_t * slot_gate, const int32_t * slot_up, const int32_t * slot_down,
                  float scale, float rms_eps, const float * x, float * out, float * xnext,
                  int32_t * ids_out, float * weights_out, float * gate_out, float * up_out,
                  float * act_out, float * experts_out, const float * resmask, int32_t * want_out) {
    std::vector<int32_t> ids((size_t) (T * k));
    std::vector<float> w((size_t) (T * k));
    orc_router_resident(H, E, k, T, w_router, x, scale, resmask, want_out, ids.data(), w.data(), nullptr, nullptr);
    std::vector<float> up((size_t) (T * k * F)), gate((size_t) (T * k * F)), act((size_t) (T * k * F)),
        ex((size_t) (T * k * H));
    const size_t rs_gu = row_size(type_gate, H), rs_u = row_size(type_up, H), rs_d = row_size(type_down, F);
    int rc = 0;
    rc |= orc_mul_mat_id(type_up, H, F, n_slots, w_up, rs_u, rs_u * F, 1, T, x, k, ids.data(), k,
                         slot_up, E, up.data());
    rc |= orc_mul_mat_id(type_gate, H, F, n_slots, w_gate, rs_gu, rs_gu * F, 1, T, x, k, ids.data(), k,
                         slot_gate, E, gate.data());
    if (rc) return rc;
    for (int64_t r = 0; r < T * k; ++r) vec_swiglu((int) F, act.data() + r * F, gate.data() + r * F, up.data() + r * F);
    rc = orc_mul_mat_id(type_down, F, H, n_slots, w_down, rs_d, rs_d * H, k, T, act.data(), k, ids.data(), k,
                        slot_down, E, ex.data());
    if (rc) return rc;
    std::vector<float> o((size_t) (T * H));
    if (T == 1) {
        // et = cont(transpose(experts [H, k])); moe_out = mul_mat(et [k, H], w [k, 1])
        std::vector<float> row((size_t) k);
        for (int64_t h = 0; h < H; ++h) {
            for (int64_t i = 0; i < k; ++i) row[(size_t) i] = ex[(size_t) (i * H + h)];
            o[(size_t) h] = vec_dot_f32((int) k, row.data(), w.data(), 2);
        }
    } else {
        // experts *= weights (broadcast), then ((e0 + e1) + e2) + ... in index order
        for (int64_t t = 0; t < T; ++t)
            for (int64_t h = 0; h < H; ++h) {
                float acc = ex[(size_t) ((t * k + 0) * H + h)] * w[(size_t) (t * k + 0)];
                for (int64_t i = 1; i < k; ++i) acc = acc + ex[(size_t) ((t * k + i) * H + h)] * w[(size_t) (t * k + i)];
                o[(size_t) (t * H + h)] = acc;
            }
    }
    if (out) memcpy(out, o.data(), sizeof(float) * T * H);
    if (xnext && rms_eps >= 0.0f) orc_rms_norm(H, T, o.data(), xnext, rms_eps);
    if (ids_out) memcpy(ids_out, ids.data(), sizeof(int32_t) * T * k);
    if (weights_out) memcpy(weights_out, w.data(), sizeof(float) * T * k);
    if (gate_out) memcpy(gate_out, gate.data(), sizeof(float) * T * k * F);
    if (up_out) memcpy(up_out, up.data(), sizeof(float) * T * k * F);
    if (act_out) memcpy(act_out, act.data(), sizeof(float) * T * k * F);
    if (experts_out) memcpy(experts_out, ex.data(), sizeof(float) * T * k * H);
    return 0;
}

}  // extern "C"
