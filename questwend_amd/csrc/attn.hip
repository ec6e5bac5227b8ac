// attn.hip -- the attention half of a Qwen3 decoder layer's Seg A
// (core/runtime.cpp:1976-2030, build_attn 681-734 on its manual path, RoPE by
// apply_rope 290-300): per-head RMSNorm and NEOX RoPE of Q and K, the f16 KV
// cache write, causal GQA scores, ggml's soft_max_ext and the P.V product,
// then the residual and the FFN input norm.  The four projections run on the
// quantized mul_mat kernels (a one-expert mul_mat_id; api.cpp).
//
// Layout in HBM: Q [T][n_head][128] f32 after RoPE; the caller's caches
// [n_ctx][n_head_kv * 128] f16 (ggml's k_cache / v_cache rows); scores and
// probabilities [T][n_head][n_kv]; the P.V partial sums [split][T][n_head][128].
//
// ggml converts the second operand of a mul_mat with an f16 first operand to
// f16 (vec_dot_type), so Q is rounded to f16 before the scores and the
// probabilities before P.V, as here; sums run in fp32.  The softmax follows
// ggml_compute_forward_soft_max_f32 (ops.cpp:5455-5566): scale, + mask,
// max, ggml_v_expf in groups of eight (hsum of eight, sums in double), expf on
// the tail, times (float) (1 / sum).  Outputs agree with the CPU backend to
// float rounding of the fp32 sums (the 1e-3 bar); they are not bit-identical.
#include <hip/hip_fp16.h>

#include "qw_kernels.hpp"

namespace qw {

namespace {

constexpr int AD = 128;   // head dimension (Qwen3: n_embd_head_k = n_embd_head_v = 128)

__device__ __forceinline__ float to_f16_and_back(float x) { return __half2float(__float2half_rn(x)); }

// One head row of one token per 64-lane block: Q and K heads get ggml_rms_norm
// (sum of squares in double) * norm weight and NEOX RoPE; K and V heads go to
// the caches at row n_past + t.  Lane i holds elements i and i + 64: NEOX's pair.
__global__ void __launch_bounds__(64) k_attn_qk_rope(AttnArgs a) {
    const int t = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const int nq = a.n_head, nk = a.n_head_kv, gqa = nk * AD;
    const int64_t pos = a.n_past + t;
    if (r >= nq + nk) {
        const int g = r - nq - nk;
        const float* src = a.v + (int64_t) t * gqa + g * AD;
        __half* dst = (__half*) a.vc + pos * gqa + g * AD;
        dst[lane] = __float2half_rn(src[lane]);
        dst[lane + 64] = __float2half_rn(src[lane + 64]);
        return;
    }
    const bool is_q = r < nq;
    const float* src = is_q ? a.q + ((int64_t) t * nq + r) * AD : a.k + (int64_t) t * gqa + (r - nq) * AD;
    const float* w = is_q ? a.q_norm : a.k_norm;
    const float x0 = src[lane], x1 = src[lane + 64];
    double s = (double) (x0 * x0) + (double) (x1 * x1);
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    const float mean = (float) (s / (double) AD);
    const float scale = 1.0f / sqrtf(mean + a.eps);
    const float y0 = (x0 * scale) * w[lane], y1 = (x1 * scale) * w[lane + 64];
    // ggml_rope_cache_init: theta_0 = pos, theta_{i+1} = theta_i * theta_scale (fp32, in order)
    float th = (float) pos;
    for (int i = 0; i < lane; ++i) th = th * a.theta_scale;
    const float c = cosf(th), sn = sinf(th);
    const float o0 = y0 * c - y1 * sn, o1 = y0 * sn + y1 * c;
    if (is_q) {
        float* dst = a.qr + ((int64_t) t * nq + r) * AD;
        dst[lane] = o0;
        dst[lane + 64] = o1;
    } else {
        __half* dst = (__half*) a.kc + pos * gqa + (r - nq) * AD;
        dst[lane] = __float2half_rn(o0);
        dst[lane + 64] = __float2half_rn(o1);
    }
}

// ---- decode and small batches (fewer than 64 query rows): split softmax ----
//
// k_attn_split_scores: one workgroup per (kv head g, token t, key split): the
// scores of its keys, 64 at a time with four lanes per key (each loads a quarter
// of the f16 key row and forms its part of each head's dot; the quad's parts
// added by DPP), written to the score rows, and per head the split's max m_s and
// sum l_s = sum_j v_expf(s_j - m_s) (double; chunks rescaled by exp(m_old - m)).
// k_attn_split_pv: per split, M = max_s m_s and S = sum_s exp(m_s - M) l_s (a
// fixed order), then ggml's probabilities p_j = v_expf(s_j - M) * (float) (1 / S)
// rounded to f16 (the f16 vec_dot_type of the V product) and the split's P.V
// partial sums.  The e_j are ggml's (the same M and ggml_v_expf); S differs from
// ggml's double sum only in the order of its terms, so p can move by one f16
// step at a rounding boundary.  k_attn_combine(_q8K) adds the splits.
constexpr int SQS = AD + AD / 32;   // padded query row in LDS (a key's four lanes read four banks)

__global__ void __launch_bounds__(256) k_attn_split_scores(AttnArgs a) {
    __shared__ __align__(16) float sq[ATT_RMAX][SQS];
    __shared__ float ss[ATT_RMAX][64];
    __shared__ float sm[ATT_RMAX];
    __shared__ double sl[ATT_RMAX];
    const int g = blockIdx.x, t = blockIdx.y, sp_i = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, grp = tid >> 6;
    const int nq = a.n_head, R = nq / a.n_head_kv, gqa = a.n_head_kv * AD;
    const int64_t k0 = (int64_t) sp_i * a.split, k1 = min((int64_t) a.n_kv, k0 + a.split);
    const int64_t vis = a.n_past + t;   // last key this token sees
    for (int i = tid; i < R * AD; i += 256) {
        const int h = i / AD, d = i % AD;
        sq[h][d + d / 32] = to_f16_and_back(a.qr[((int64_t) t * nq + g * R + h) * AD + d]);
    }
    if (tid < ATT_RMAX) {
        sm[tid] = -INFINITY;
        sl[tid] = 0.0;
    }
    const int p = tid & 3, kq = tid >> 2;
    for (int64_t c0 = k0; c0 < k1; c0 += 64) {
        const int nc = (int) min((int64_t) 64, k1 - c0);
        const int64_t j = c0 + kq;
        const bool kok = kq < nc;
        const uint4* krow = (const uint4*) ((const __half*) a.kc + (kok ? j : c0) * gqa + g * AD + 32 * p);
        uint4 kv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) kv[i] = krow[i];
        __syncthreads();   // sq staged (first chunk); the previous chunk's ss reads are done
        float kf[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w4[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const __half2 hv = *(const __half2*) &w4[m];
                kf[8 * i + 2 * m] = __low2float(hv);
                kf[8 * i + 2 * m + 1] = __high2float(hv);
            }
        }
        const float* qb = &sq[0][33 * p];
        for (int h = 0; h < R; ++h) {
            float sd = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const float4 q4 = *(const float4*) (qb + h * SQS + i);
                sd = __builtin_fmaf(q4.x, kf[i], sd);
                sd = __builtin_fmaf(q4.y, kf[i + 1], sd);
                sd = __builtin_fmaf(q4.z, kf[i + 2], sd);
                sd = __builtin_fmaf(q4.w, kf[i + 3], sd);
            }
            sd = sd + dpp_f<DPP_XOR1>(sd);
            sd = sd + dpp_f<DPP_XOR2>(sd);
            if (p == 0) {
                const float sv = j <= vis ? sd * a.kq_scale : -INFINITY;
                if (kok) a.s[((int64_t) t * nq + g * R + h) * a.n_kv + j] = sv;
                ss[h][kq] = kok ? sv : -INFINITY;
            }
        }
        __syncthreads();
        for (int h = grp; h < R; h += 4) {   // wave grp: heads grp, grp + 4, ...
            const float sv = ss[h][lane];
            float mc = sv;
            for (int off = 32; off >= 1; off >>= 1) mc = fmaxf(mc, __shfl_xor(mc, off));
            const float mo = sm[h], mn = fmaxf(mo, mc);
            double es = sv == -INFINITY ? 0.0 : (double) v_expf(sv - mn);
            for (int off = 32; off >= 1; off >>= 1) es += __shfl_xor(es, off);
            if (lane == 0) {
                const double al = mo == -INFINITY ? 0.0 : exp((double) mo - (double) mn);
                sm[h] = mn;
                sl[h] = sl[h] * al + es;
            }
        }
    }
    __syncthreads();
    if (tid < R) {
        const int64_t row = ((int64_t) sp_i * a.T + t) * nq + g * R + tid;
        a.stat[2 * row] = sm[tid];
        a.stat[2 * row + 1] = (float) sl[tid];
    }
}

// P.V partial sums over the split's keys for kv head g and token t: four 64-lane
// groups take every fourth key; lane l of a group holds output elements 2 l,
// 2 l + 1 of each of the R query heads (one 4-byte V load per key); the groups'
// sums are added in group order through LDS.
__global__ void __launch_bounds__(256) k_attn_split_pv(AttnArgs a, int n_split) {
    __shared__ float sp[ATT_RMAX][256];
    __shared__ float2 sred[3][ATT_RMAX][64];
    __shared__ float sM[ATT_RMAX], sI[ATT_RMAX];
    const int g = blockIdx.x, t = blockIdx.y, sp_i = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, grp = tid >> 6;
    const int nq = a.n_head, R = nq / a.n_head_kv, gqa = a.n_head_kv * AD;
    const int64_t k0 = (int64_t) sp_i * a.split, k1 = min((int64_t) a.n_kv, k0 + a.split);
    // the first keys' V before the statistics and the staging (their latency overlaps them)
    const __half2* vb0 = (const __half2*) ((const __half*) a.vc + k0 * gqa + g * AD) + lane;
    const int nc0 = (int) min((int64_t) 256, k1 - k0);
    __half2 v16[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int jj = grp + 4 * u;
        v16[u] = jj < nc0 ? vb0[(int64_t) jj * (gqa / 2)] : __half2{};
    }
    // M and S of each head over all splits (wave grp: heads grp, grp + 4, ...; lane s0
    // takes splits s0, s0 + 64, ...; the lanes' sums added in a fixed tree order)
    for (int h = grp; h < R; h += 4) {
        float mx = -INFINITY;
        for (int s0 = lane; s0 < n_split; s0 += 64)
            mx = fmaxf(mx, a.stat[2 * (((int64_t) s0 * a.T + t) * nq + g * R + h)]);
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        double S = 0.0;
        for (int s0 = lane; s0 < n_split; s0 += 64) {
            const int64_t r = ((int64_t) s0 * a.T + t) * nq + g * R + h;
            const float ms = a.stat[2 * r];
            if (ms != -INFINITY) S += exp((double) ms - (double) mx) * (double) a.stat[2 * r + 1];
        }
        for (int off = 32; off >= 1; off >>= 1) S += __shfl_xor(S, off);
        if (lane == 0) {
            sM[h] = mx;
            sI[h] = (float) (1.0 / S);
        }
    }
    float2 acc[ATT_RMAX];
#pragma unroll
    for (int h = 0; h < ATT_RMAX; ++h) acc[h] = float2{0.0f, 0.0f};
    for (int64_t c0 = k0; c0 < k1; c0 += 256) {
        const int nc = (int) min((int64_t) 256, k1 - c0);
        __syncthreads();   // sM / sI written; the previous chunk's sp reads are done
        for (int i = tid; i < R * 256; i += 256) {
            const int h = i / 256, jj = i % 256;
            float pv = 0.0f;
            if (jj < nc) {
                const float sv = a.s[((int64_t) t * nq + g * R + h) * a.n_kv + c0 + jj];
                pv = sv == -INFINITY ? 0.0f : to_f16_and_back(v_expf(sv - sM[h]) * sI[h]);
            }
            sp[h][jj] = pv;
        }
        __syncthreads();
        const __half2* vb = (const __half2*) ((const __half*) a.vc + c0 * gqa + g * AD) + lane;
        if (c0 == k0) {
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int jj = grp + 4 * u;
                if (jj >= nc) break;
                const float2 v = __half22float2(v16[u]);
#pragma unroll
                for (int h = 0; h < ATT_RMAX; ++h)
                    if (h < R) {
                        const float pe = sp[h][jj];
                        acc[h].x = __builtin_fmaf(pe, v.x, acc[h].x);
                        acc[h].y = __builtin_fmaf(pe, v.y, acc[h].y);
                    }
            }
        }
#pragma unroll 4
        for (int jj = grp + (c0 == k0 ? 64 : 0); jj < nc; jj += 4) {
            const float2 v = __half22float2(vb[(int64_t) jj * (gqa / 2)]);
#pragma unroll
            for (int h = 0; h < ATT_RMAX; ++h)
                if (h < R) {
                    const float pe = sp[h][jj];
                    acc[h].x = __builtin_fmaf(pe, v.x, acc[h].x);
                    acc[h].y = __builtin_fmaf(pe, v.y, acc[h].y);
                }
        }
    }
    if (grp > 0) {
#pragma unroll
        for (int h = 0; h < ATT_RMAX; ++h)
            if (h < R) sred[grp - 1][h][lane] = acc[h];
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
        for (int h = 0; h < ATT_RMAX; ++h)
            if (h < R) {
                float2 s2 = acc[h];
#pragma unroll
                for (int q = 0; q < 3; ++q) {
                    const float2 o = sred[q][h][lane];
                    s2.x = s2.x + o.x;
                    s2.y = s2.y + o.y;
                }
                *(float2*) &a.part[(((int64_t) sp_i * a.T + t) * nq + g * R + h) * AD + 2 * lane] = s2;
            }
    }
}

// att[t][h][d] = the sum of the splits' partials, in split order.
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a, int n_split) {
    const int64_t n = (int64_t) a.T * a.n_head * AD;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = a.part[i];
#pragma unroll 8
    for (int k = 1; k < n_split; ++k) s = s + a.part[(int64_t) k * n + i];
    a.att[i] = s;
}

// The P.V split sums (k_attn_combine's order) and the Q8_K quantisation of the
// result (the attn_output projection's input) in one launch: one wave per
// 256-value block of a token's row.
__global__ void __launch_bounds__(256) k_attn_combine_q8K(AttnArgs a, int n_split, BlockQ8_K* __restrict__ dst) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t) a.T * a.n_head * AD, nblk = n / QK_K;
    const int64_t blk = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;
    const int64_t i0 = blk * QK_K + 4 * lane;
    float4 s4 = *(const float4*) (a.part + i0);
#pragma unroll 4
    for (int k = 1; k < n_split; ++k) {
        const float4 o = *(const float4*) (a.part + (int64_t) k * n + i0);
        s4.x = s4.x + o.x;
        s4.y = s4.y + o.y;
        s4.z = s4.z + o.z;
        s4.w = s4.w + o.w;
    }
    const float v[4] = {s4.x, s4.y, s4.z, s4.w};
    quant_q8K_wave(v, lane, dst + blk);
}

// ---- batches of at least 64 query rows: the two products on the matrix cores ----
//
// Rows r = t R + h (token-major) of kv head g.  v_mfma_f32_16x16x16_f16: lane l
// of A holds row l % 16, k = 4 (l / 16) .. +3; lane l of B holds column l % 16,
// the same k; lane l, register i of D is row 4 (l / 16) + i, column l % 16.
// The f16 operands are the values ggml rounds to f16 (Q, and the normalized
// probabilities), so every product is exact in fp32; only the order of the
// fp32 sums differs from the CPU backend's.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h4 f4_to_h4(float x0, float x1, float x2, float x3) {
    return h4{(_Float16) x0, (_Float16) x1, (_Float16) x2, (_Float16) x3};
}

// Softmax statistics of the scores: a workgroup takes 64 rows (a wave per 16,
// their Q in registers) and MF_SK keys, 16 at a time: eight MFMAs over the 128
// dims per 16-key tile, the next tile's key rows loaded while the current one is
// multiplied (B straight from the cache rows, 8 bytes per lane and dim step).
// Only each row's maximum and sum of exp(s - max) over its MF_SK keys are
// written; k_attn_pv_mf forms the scores again beside P.V, so the score rows
// (4 n_head T n_kv bytes) never reach memory.
constexpr int MF_SK = ATT_MF_SK;   // keys per workgroup of k_attn_scores_mf
__global__ void __launch_bounds__(256) k_attn_scores_mf(AttnArgs a) {
    const int g = blockIdx.y, tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, q = l >> 4;
    const int nq = a.n_head, R = nq / a.n_head_kv, gqa = a.n_head_kv * AD;
    const int64_t rows = (int64_t) a.T * R, key0 = (int64_t) blockIdx.x * MF_SK;
    const int64_t ra = (int64_t) blockIdx.z * 64 + 16 * w + li;   // this lane's A row
    h4 qa[8];
    if (ra < rows) {
        const int t = (int) (ra / R), h = (int) (ra % R);
        const float* qrow = a.qr + ((int64_t) t * nq + g * R + h) * AD + 4 * q;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const float4 v = *(const float4*) (qrow + 16 * st);
            qa[st] = f4_to_h4(v.x, v.y, v.z, v.w);
        }
    } else {
#pragma unroll
        for (int st = 0; st < 8; ++st) qa[st] = h4{0, 0, 0, 0};
    }
    // rows of this wave: the last token they hold bounds the keys that are not masked for all of them
    const int64_t rw0 = (int64_t) blockIdx.z * 64 + 16 * w;
    const int64_t kend = min(min((int64_t) a.n_kv, key0 + MF_SK), a.n_kv);
    auto load_b = [&](int64_t j0, h4 (&kb)[8]) __attribute__((always_inline)) {
        const int64_t jb = j0 + li;
        const bool ok = jb < kend;
        const _Float16* krow = (const _Float16*) a.kc + (ok ? jb : 0) * gqa + g * AD + 4 * q;
#pragma unroll
        for (int st = 0; st < 8; ++st) kb[st] = ok ? *(const h4*) (krow + 16 * st) : h4{0, 0, 0, 0};
    };
    if (rw0 >= rows) return;
    // this lane's running max and sum of exp(s - max) for its four D rows over its keys.
    // The sums only normalize (P.V forms each probability with ggml_v_expf): the
    // hardware exp here moves S by ~1e-7 of itself, far below the f16 step of p.
    float mrow[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float lrow[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    h4 kc[8], kn[8];
    load_b(key0, kc);
    for (int64_t j0 = key0; j0 < kend; j0 += 16) {
        if (j0 + 16 < kend) load_b(j0 + 16, kn);
        f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 8; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x16f16(qa[st], kc[st], acc, 0, 0, 0);
        const int64_t jb = j0 + li;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t r = rw0 + 4 * q + i;
            if (r < rows && jb < kend) {
                const int t = (int) (r / R), h = (int) (r % R);
                const float sv = jb > a.n_past + t ? -INFINITY : acc[i] * a.kq_scale;
                if (sv > mrow[i]) {
                    lrow[i] = (mrow[i] == -INFINITY ? 0.0f : lrow[i] * __expf(mrow[i] - sv)) + 1.0f;
                    mrow[i] = sv;
                } else if (sv != -INFINITY) {
                    lrow[i] += __expf(sv - mrow[i]);
                }
            }
        }
#pragma unroll
        for (int st = 0; st < 8; ++st) kc[st] = kn[st];
    }
    // the 16 lanes of a row group hold different keys of the same rows: combine them
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const float mo = __shfl_xor(mrow[i], off);
            const float lo = __shfl_xor(lrow[i], off);
            const float mn = fmaxf(mrow[i], mo);
            const float a0 = mrow[i] == -INFINITY ? 0.0f : lrow[i] * __expf(mrow[i] - mn);
            const float a1 = mo == -INFINITY ? 0.0f : lo * __expf(mo - mn);
            mrow[i] = mn;
            lrow[i] = a0 + a1;
        }
        const int64_t r = rw0 + 4 * q + i;
        if (li == 0 && r < rows) {
            const int t = (int) (r / R), h = (int) (r % R);
            const int64_t sr = (int64_t) blockIdx.x * a.T * nq + (int64_t) t * nq + g * R + h;
            a.stat[2 * sr] = mrow[i];
            a.stat[2 * sr + 1] = lrow[i];
        }
    }
}

// P.V: a workgroup takes 64 rows (a wave per 16) and all 128 dims (eight 16-dim
// tiles), over the keys its rows may see (<= n_past + their last token), 64 keys
// at a time: the V chunk is staged in LDS transposed ([dim][key], f16) so that
// a B operand is one 8-byte read; A (the probabilities, rounded to f16) is read
// straight from the score rows.  Writes att, no partial sums.
constexpr int SVS = 64 + 4;   // padded key stride of the staged V chunk (halves)
__global__ void __launch_bounds__(256) k_attn_pv_mf(AttnArgs a) {
    __shared__ __align__(16) _Float16 sv[AD][SVS];
    __shared__ __align__(16) _Float16 skc[64][AD + 8];   // the chunk's key rows (16 bytes of pad per row)
    const int g = blockIdx.x, tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, q = l >> 4;
    const int nq = a.n_head, R = nq / a.n_head_kv, gqa = a.n_head_kv * AD;
    const int64_t rows = (int64_t) a.T * R, row0 = (int64_t) blockIdx.y * 64;
    const int t_last = (int) (min(rows, row0 + 64) - 1) / R;
    const int64_t klim = min((int64_t) a.n_kv, a.n_past + t_last + 1);   // keys past it are masked for every row
    const int64_t ra = row0 + 16 * w + li;                                // this lane's A row
    const bool row_ok = ra < rows;
    const int64_t rid = row_ok ? (int64_t) (ra / R) * nq + g * R + ra % R : 0;
    const int64_t key_max = row_ok ? a.n_past + ra / R : -1;             // the row's last unmasked key
    // the row's Q (f16, as ggml rounds it) as the B operand of S^T = K Q^T: lane
    // (li, q) holds dims 4 q + 16 st .. +3 of row li, the layout of an A operand
    h4 qb[8];
    if (row_ok) {
        const float* qrow = a.qr + rid * AD + 4 * q;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const float4 v = *(const float4*) (qrow + 16 * st);
            qb[st] = f4_to_h4(v.x, v.y, v.z, v.w);
        }
    } else {
#pragma unroll
        for (int st = 0; st < 8; ++st) qb[st] = h4{0, 0, 0, 0};
    }
    // the row's max M and sum S = sum_b exp(m_b - M) l_b over the 512-key blocks, then
    // p = f16(v_expf(s - M) * (float) (1 / S)): ggml's normalized probabilities
    const int nkb = (int) ((a.n_kv + MF_SK - 1) / MF_SK);
    float M = -INFINITY;
    for (int b = 0; b < nkb; ++b) M = fmaxf(M, row_ok ? a.stat[2 * ((int64_t) b * a.T * nq + rid)] : -INFINITY);
    double S = 0.0;
    for (int b = 0; b < nkb && row_ok; ++b) {
        const float mb = a.stat[2 * ((int64_t) b * a.T * nq + rid)];
        if (mb != -INFINITY) S += exp((double) mb - (double) M) * (double) a.stat[2 * ((int64_t) b * a.T * nq + rid) + 1];
    }
    const float inv = row_ok ? (float) (1.0 / S) : 0.0f;
    f4 acc[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[nt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const int sk = tid & 63, sdq = tid >> 6;   // staging: key sk of the chunk, dims 32 sdq .. +32
    auto load_kv = [&](int64_t c0, uint4 (&vv)[4], uint4 (&kk)[4]) __attribute__((always_inline)) {
        const int64_t kj = c0 + sk;
        const int64_t off = (kj < klim ? kj : 0) * gqa + g * AD + 32 * sdq;
        const uint4* vrow = (const uint4*) ((const _Float16*) a.vc + off);
        const uint4* krow = (const uint4*) ((const _Float16*) a.kc + off);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vv[i] = kj < klim ? vrow[i] : uint4{0u, 0u, 0u, 0u};
            kk[i] = kj < klim ? krow[i] : uint4{0u, 0u, 0u, 0u};
        }
    };
    uint4 vv[4], vn[4], kv4[4], kn4[4];
    load_kv(0, vv, kv4);
    for (int64_t c0 = 0; c0 < klim; c0 += 64) {
        if (c0 + 64 < klim) load_kv(c0 + 64, vn, kn4);   // the next chunk's rows, in flight during this one
        __syncthreads();   // the previous chunk's reads are done
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w4[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int d = 32 * sdq + 8 * i + 2 * m;
                sv[d][sk] = __builtin_bit_cast(_Float16, (uint16_t) (w4[m] & 0xffffu));
                sv[d + 1][sk] = __builtin_bit_cast(_Float16, (uint16_t) (w4[m] >> 16));
            }
            *(uint4*) &skc[sk][32 * sdq + 8 * i] = kv4[i];
        }
        __syncthreads();
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const int64_t k4 = c0 + 16 * kt + 4 * q;   // this lane's four keys of the A operand
            // S^T for keys c0 + 16 kt .. +15 and the wave's 16 rows: A = the key rows
            // (lane (li, q): key li, dims 4 q + 16 st), B = Q; D lane (li, q) register m
            // is the score of row li and key k4 + m, P.V's A layout
            f4 sc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 8; ++st) {
                const h4 kb = *(const h4*) &skc[16 * kt + li][16 * st + 4 * q];   // zero rows past klim
                sc = __builtin_amdgcn_mfma_f32_16x16x16f16(kb, qb[st], sc, 0, 0, 0);
            }
            float p4[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float sv = k4 + m <= key_max && k4 + m < klim ? sc[m] * a.kq_scale : -INFINITY;
                p4[m] = sv == -INFINITY ? 0.0f : v_expf(sv - M) * inv;
            }
            const h4 pa = f4_to_h4(p4[0], p4[1], p4[2], p4[3]);
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                const h4 vb = *(const h4*) &sv[16 * nt + li][16 * kt + 4 * q];
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vb, acc[nt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vv[i] = vn[i];
            kv4[i] = kn4[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r = row0 + 16 * w + 4 * q + i;
        if (r < rows) {
            float* dst = a.att + ((int64_t) (r / R) * nq + g * R + r % R) * AD + li;
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) dst[16 * nt] = acc[nt][i];
        }
    }
}

// resid = x + y (ggml_add), out = rms_norm(resid) * w (k_rms_norm's order); one
// 256-thread block per row of n.
__global__ void __launch_bounds__(256) k_add_rms_norm_mul(const float* __restrict__ x, const float* __restrict__ y,
                                                          float* __restrict__ resid, float* __restrict__ out,
                                                          int64_t n, float eps, const float* __restrict__ w) {
    __shared__ double part[4];
    const int64_t o = (int64_t) blockIdx.x * n;
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = x[o + i] + y[o + i];
        resid[o + i] = v;
        s += (double) (v * v);
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (!out) return;
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float mean = (float) (tot / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) out[o + i] = (resid[o + i] * scale) * w[i];
}

// attn_norm and the Q8_K quantisation of its output in one launch, one
// 256-thread block per row of n (a multiple of 256): the sum of squares and
// scale exactly as k_rms_norm, each value (x * scale) * w as it writes them, and
// each 256-value block quantized by one wave as k_quant_q8K does.
__global__ void __launch_bounds__(256) k_rms_norm_q8K(const float* __restrict__ x, int64_t n, float eps,
                                                      const float* __restrict__ w, BlockQ8_K* __restrict__ dst) {
    __shared__ double part[4];
    const float* xr = x + (int64_t) blockIdx.x * n;
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        s += (double) (v * v);
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float mean = (float) (tot / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t nb = n / QK_K;
    for (int64_t ib = wv; ib < nb; ib += 4) {
        const float4 q = *(const float4*) (xr + ib * QK_K + 4 * lane);
        const float4 ww = *(const float4*) (w + ib * QK_K + 4 * lane);
        const float v[4] = {(q.x * scale) * ww.x, (q.y * scale) * ww.y, (q.z * scale) * ww.z, (q.w * scale) * ww.w};
        quant_q8K_wave(v, lane, dst + (int64_t) blockIdx.x * nb + ib);
    }
}

__global__ void k_fill_i32(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

int launch_attn_core(const AttnArgs& a, hipStream_t st) {
    if (a.T <= 0) return 0;
    const int nq = a.n_head, nk = a.n_head_kv;
    hipLaunchKernelGGL(k_attn_qk_rope, dim3((unsigned) a.T, (unsigned) (nq + 2 * nk)), dim3(64), 0, st, a);
    const int64_t rows = (int64_t) a.T * (nq / nk);
    const bool mf = rows >= 64;   // the matrix-core products (prefill chunks, large batches)
    if (!mf) {   // decode and small batches: split softmax, three launches
        if (a.split <= 0 || !a.stat) return -2;
        const int n_split = (int) ((a.n_kv + a.split - 1) / a.split);
        const dim3 grid((unsigned) nk, (unsigned) a.T, (unsigned) n_split);
        hipLaunchKernelGGL(k_attn_split_scores, grid, dim3(256), 0, st, a);
        hipLaunchKernelGGL(k_attn_split_pv, grid, dim3(256), 0, st, a, n_split);
        const int64_t n = (int64_t) a.T * nq * AD;
        if (a.att_q8K)   // the split sums straight into the attn_output projection's Q8_K rows
            hipLaunchKernelGGL(k_attn_combine_q8K, dim3((unsigned) ((n / QK_K + 3) / 4)), dim3(256), 0, st, a, n_split,
                               (BlockQ8_K*) a.att_q8K);
        else
            hipLaunchKernelGGL(k_attn_combine, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, a, n_split);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    hipLaunchKernelGGL(k_attn_scores_mf, dim3((unsigned) ((a.n_kv + MF_SK - 1) / MF_SK), (unsigned) nk,
                                              (unsigned) ((rows + 63) / 64)), dim3(256), 0, st, a);
    // the softmax is formed inside the P.V kernel from the scores' block statistics;
    // it writes att (a.att_q8K is left to the caller)
    hipLaunchKernelGGL(k_attn_pv_mf, dim3((unsigned) nk, (unsigned) ((rows + 63) / 64)), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_rms_norm_q8K(const float* x, int64_t n, int64_t rows, float eps, const float* w, void* dst,
                        hipStream_t st) {
    if (n % QK_K || !w || (((uintptr_t) x | (uintptr_t) w) & 15)) return -2;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(k_rms_norm_q8K, dim3((unsigned) rows), dim3(256), 0, st, x, n, eps, w, (BlockQ8_K*) dst);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_add_rms_norm_mul(const float* x, const float* y, float* resid, float* out, int64_t n, int64_t rows,
                            float eps, const float* w, hipStream_t st) {
    if (rows == 0) return 0;
    hipLaunchKernelGGL(k_add_rms_norm_mul, dim3((unsigned) rows), dim3(256), 0, st, x, y, resid, out, n, eps, w);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t st) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, p, n, v);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
