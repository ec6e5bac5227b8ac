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

// Scores of 256 keys per block, one key per thread, for the R = n_head /
// n_head_kv query heads of kv head g and token t: s = (f16(q) . k) * kq_scale
// + mask, mask = 0 for key j <= n_past + t, -inf after (the causal mask
// set_attn_inputs fills, core/runtime.cpp:2108-2116).  The key row is held in
// registers; the query rows are read from LDS by every thread (broadcast).
__global__ void __launch_bounds__(256) k_attn_scores(AttnArgs a) {
    __shared__ __align__(16) float sq[ATT_RMAX][AD];
    const int g = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int nq = a.n_head, R = nq / a.n_head_kv, gqa = a.n_head_kv * AD;
    for (int i = tid; i < R * AD; i += 256) {
        const int h = i / AD, d = i % AD;
        sq[h][d] = to_f16_and_back(a.qr[((int64_t) t * nq + g * R + h) * AD + d]);
    }
    __syncthreads();
    const int64_t j = (int64_t) blockIdx.x * 256 + tid;
    if (j >= a.n_kv) return;
    const uint4* krow = (const uint4*) ((const __half*) a.kc + j * gqa + g * AD);
    uint4 kv[AD / 8];
#pragma unroll
    for (int i = 0; i < AD / 8; ++i) kv[i] = krow[i];
    const bool masked = j > a.n_past + t;
    for (int h = 0; h < R; ++h) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < AD / 8; ++i) {
            const float4 qa = *(const float4*) &sq[h][8 * i], qb = *(const float4*) &sq[h][8 * i + 4];
            const uint32_t w4[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
            float kf[8];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const __half2 hv = *(const __half2*) &w4[m];
                kf[2 * m] = __low2float(hv);
                kf[2 * m + 1] = __high2float(hv);
            }
            acc = __builtin_fmaf(qa.x, kf[0], acc);
            acc = __builtin_fmaf(qa.y, kf[1], acc);
            acc = __builtin_fmaf(qa.z, kf[2], acc);
            acc = __builtin_fmaf(qa.w, kf[3], acc);
            acc = __builtin_fmaf(qb.x, kf[4], acc);
            acc = __builtin_fmaf(qb.y, kf[5], acc);
            acc = __builtin_fmaf(qb.z, kf[6], acc);
            acc = __builtin_fmaf(qb.w, kf[7], acc);
        }
        a.s[((int64_t) t * nq + g * R + h) * a.n_kv + j] = masked ? -INFINITY : acc * a.kq_scale;
    }
}

// ggml_compute_forward_soft_max_f32 on one (token, head) row of n_kv scores,
// in place: max; v_expf(x - max) in groups of eight with each group's
// hsum_float_8 added in double, expf on the tail; times (float) (1 / sum).
__global__ void __launch_bounds__(256) k_attn_softmax(AttnArgs a) {
    __shared__ float red[4];
    __shared__ double dred[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float* row = a.s + ((int64_t) blockIdx.y * a.n_head + blockIdx.x) * a.n_kv;
    const int64_t n = a.n_kv, ng = n / 8;
    float mx = -INFINITY;
    for (int64_t i = tid; i < n; i += 256) mx = fmaxf(mx, row[i]);
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    double sum = 0.0;
    for (int64_t q = tid; q < ng; q += 256) {
        float e[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) e[m] = v_expf(row[8 * q + m] - mx);
#pragma unroll
        for (int m = 0; m < 8; ++m) row[8 * q + m] = e[m];
        sum += (double) hsum8(e);
    }
    for (int64_t i = 8 * ng + tid; i < n; i += 256) {
        const float e = (float) exp((double) (row[i] - mx));
        row[i] = e;
        sum += (double) e;
    }
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane == 0) dred[wv] = sum;
    __syncthreads();
    const double tot = (dred[0] + dred[1]) + (dred[2] + dred[3]);
    const float inv = (float) (1.0 / tot);
    for (int64_t i = tid; i < n; i += 256) row[i] = row[i] * inv;
}

// P.V partial sums over the keys [split * ATT_SPLIT, ...) for kv head g and
// token t: thread (d = tid % 128, half = tid / 128) accumulates output element
// d of query heads g R + half, g R + half + 2, ...; the probabilities of a
// 256-key chunk are staged in LDS, rounded to f16.
__global__ void __launch_bounds__(256) k_attn_pv(AttnArgs a) {
    __shared__ float sp[ATT_RMAX][256];
    const int g = blockIdx.x, t = blockIdx.y, sp_i = blockIdx.z, tid = threadIdx.x;
    const int nq = a.n_head, R = nq / a.n_head_kv, gqa = a.n_head_kv * AD;
    const int d = tid & (AD - 1), half = tid >> 7;
    const int64_t k0 = (int64_t) sp_i * ATT_SPLIT, k1 = min((int64_t) a.n_kv, k0 + ATT_SPLIT);
    float acc[ATT_RMAX / 2];
#pragma unroll
    for (int u = 0; u < ATT_RMAX / 2; ++u) acc[u] = 0.0f;
    for (int64_t c0 = k0; c0 < k1; c0 += 256) {
        const int nc = (int) min((int64_t) 256, k1 - c0);
        __syncthreads();
        for (int i = tid; i < R * 256; i += 256) {
            const int h = i / 256, jj = i % 256;
            sp[h][jj] = jj < nc ? to_f16_and_back(a.s[((int64_t) t * nq + g * R + h) * a.n_kv + c0 + jj]) : 0.0f;
        }
        __syncthreads();
        const __half* vcol = (const __half*) a.vc + c0 * gqa + g * AD + d;
        for (int jj = 0; jj < nc; ++jj) {
            const float v = __half2float(vcol[(int64_t) jj * gqa]);
#pragma unroll
            for (int u = 0; u < ATT_RMAX / 2; ++u) {
                const int h = half + 2 * u;
                if (h < R) acc[u] = __builtin_fmaf(sp[h][jj], v, acc[u]);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < ATT_RMAX / 2; ++u) {
        const int h = half + 2 * u;
        if (h < R) a.part[(((int64_t) sp_i * a.T + t) * nq + g * R + h) * AD + d] = acc[u];
    }
}

// att[t][h][d] = the sum of the splits' partials, in split order.
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a, int n_split) {
    const int64_t n = (int64_t) a.T * a.n_head * AD;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = a.part[i];
    for (int k = 1; k < n_split; ++k) s = s + a.part[(int64_t) k * n + i];
    a.att[i] = s;
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

__global__ void k_fill_i32(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

int launch_attn_core(const AttnArgs& a, hipStream_t st) {
    if (a.T <= 0) return 0;
    const int nq = a.n_head, nk = a.n_head_kv;
    hipLaunchKernelGGL(k_attn_qk_rope, dim3((unsigned) a.T, (unsigned) (nq + 2 * nk)), dim3(64), 0, st, a);
    hipLaunchKernelGGL(k_attn_scores, dim3((unsigned) ((a.n_kv + 255) / 256), (unsigned) nk, (unsigned) a.T),
                       dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_attn_softmax, dim3((unsigned) nq, (unsigned) a.T), dim3(256), 0, st, a);
    const int n_split = (int) ((a.n_kv + ATT_SPLIT - 1) / ATT_SPLIT);
    hipLaunchKernelGGL(k_attn_pv, dim3((unsigned) nk, (unsigned) a.T, (unsigned) n_split), dim3(256), 0, st, a);
    const int64_t n = (int64_t) a.T * nq * AD;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, a, n_split);
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
