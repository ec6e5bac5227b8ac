// router.hip -- MoE router on the GPU, bit-identical to the reference CPU path.
//
// Reference op sequence (core/runtime.cpp:869-897, Runtime::Impl::build_moe):
//   logits = mul_mat(W_gate_inp, x)     ggml_vec_dot_f32, vec.cpp:11-140 (AVX: 4 x 8-lane
//                                       fma accumulators, GGML_F32x8_REDUCE simd-mappings.h:579-629)
//   probs  = soft_max(logits)           ops.cpp:5455-5566, vec.cpp:531- (ggml_v_expf, double sum)
//   ids    = argsort_top_k(probs, k)    ggml.c:5344-5361 -> ARGSORT DESC ops.cpp:8332-8382 (std::sort)
//   w      = get_rows / sum_rows / clamp(6.103515625e-5, inf) / div (/ scale)
#include "qw_kernels.hpp"
#include "qw_sort.hpp"
#include "qw_topk.hpp"

namespace qw {


// logits[t][e] = vec_dot_f32(H, W[e], x[t]).  A group of 32 lanes owns one
// expert: lane c is the fma chain c of the AVX reduction (elements i == c mod
// 32, in order), for ROUTER_TT tokens at once; a workgroup holds EPW experts.
// The loads of ROUTER_STEPS 32-element steps are issued together and the next
// batch is in flight while the current one is accumulated, so a chain waits for
// memory once per batch, not once per step.  Small batches take one token per
// group, two experts per workgroup (for more workgroups) and 32-step batches.
// xq (small batches, EPW == 2): workgroups past the router's also quantize x to
// Q8_K, one wave per 256-value block (the k_quant_q8K quantizer), so the
// projections' activation costs no launch of its own.
template <int ROUTER_TT, int EPW, int ROUTER_STEPS>
__global__ void __launch_bounds__(32 * EPW) k_router_logits(const float* __restrict__ W, const float* __restrict__ x,
                                                            int64_t x_stride, int64_t H, int64_t E, int64_t T,
                                                            float* __restrict__ logits, BlockQ8_K* __restrict__ xq) {
    if (EPW == 2 && blockIdx.x >= (E + 1) / 2) {
        const int64_t ib = blockIdx.x - (E + 1) / 2, t = blockIdx.y;
        if (ib >= H / QK_K) return;
        const float4 q = *(const float4*) (x + t * x_stride + ib * QK_K + 4 * threadIdx.x);
        const float v[4] = {q.x, q.y, q.z, q.w};
        quant_q8K_wave(v, threadIdx.x, xq + t * (H / QK_K) + ib);
        return;
    }
    const int c = threadIdx.x & 31;
    const int64_t e = (int64_t) blockIdx.x * EPW + (threadIdx.x >> 5);
    const int64_t t0 = (int64_t) blockIdx.y * ROUTER_TT;
    const int64_t np = H & ~(int64_t) 31;
    const int64_t ns = np / 32;                       // steps
    const bool ev = e < E;
    const float* w = W + (ev ? e : 0) * H + c;
    const float* xt[ROUTER_TT];
#pragma unroll
    for (int tt = 0; tt < ROUTER_TT; ++tt) xt[tt] = x + (t0 + tt < T ? t0 + tt : T - 1) * x_stride + c;
    float acc[ROUTER_TT];
#pragma unroll
    for (int tt = 0; tt < ROUTER_TT; ++tt) acc[tt] = 0.0f;
    float wv[ROUTER_STEPS], xv[ROUTER_TT][ROUTER_STEPS];
    auto load = [&](int64_t s0, float* wd, float (*xd)[ROUTER_STEPS]) {
#pragma unroll
        for (int u = 0; u < ROUTER_STEPS; ++u) {
            const int64_t s = (s0 + u < ns ? s0 + u : ns - 1) * 32;   // (past the end: never accumulated)
            wd[u] = w[s];
#pragma unroll
            for (int tt = 0; tt < ROUTER_TT; ++tt) xd[tt][u] = xt[tt][s];
        }
    };
    if (ns > 0) load(0, wv, xv);
    for (int64_t s0 = 0; s0 < ns; s0 += ROUTER_STEPS) {
        float wn[ROUTER_STEPS], xn[ROUTER_TT][ROUTER_STEPS];
        const bool more = s0 + ROUTER_STEPS < ns;
        if (more) load(s0 + ROUTER_STEPS, wn, xn);
#pragma unroll
        for (int u = 0; u < ROUTER_STEPS; ++u)
#pragma unroll
            for (int tt = 0; tt < ROUTER_TT; ++tt)
                if (s0 + u < ns) acc[tt] = __builtin_fmaf(wv[u], xv[tt][u], acc[tt]);
        if (more) {
#pragma unroll
            for (int u = 0; u < ROUTER_STEPS; ++u) {
                wv[u] = wn[u];
#pragma unroll
                for (int tt = 0; tt < ROUTER_TT; ++tt) xv[tt][u] = xn[tt][u];
            }
        }
    }
    const float* wr = W + (ev ? e : 0) * H;
#pragma unroll
    for (int tt = 0; tt < ROUTER_TT; ++tt) {
        // GGML_F32x8_REDUCE of the four 8-lane accumulators: s_l = (c_l + c_{16+l}) +
        // (c_{8+l} + c_{24+l}), t0_l = s_l + s_{l+4}, then two _mm_hadd_ps
        float v = acc[tt] + __shfl_down(acc[tt], 16, 32);
        v = v + __shfl_down(v, 8, 32);
        v = v + __shfl_down(v, 4, 32);
        const float u = v + __shfl_down(v, 1, 32);
        float sumf = u + __shfl_down(u, 2, 32);
        const int64_t t = t0 + tt;
        if (c == 0 && ev && t < T) {
            // scalar tail (n % 32): 4-wide multiply + in-order add per full group of 4, fma for the rest
            const float* xr = x + t * x_stride;
            const int64_t nv = np + ((H - np) & ~(int64_t) 3);
            for (int64_t i = np; i < H; ++i)
                sumf = (i < nv) ? sumf + wr[i] * xr[i] : __builtin_fmaf(wr[i], xr[i], sumf);
            logits[t * E + e] = sumf;
        }
    }
}

// The same logits for large batches (prefill): lane c of a 32-lane group runs
// chain c for EL experts x TL tokens at once, so one step's EL + TL loads feed
// EL * TL fmas (k_router_logits loads x once per expert and W once per ROUTER_TT
// tokens).  Eight groups per workgroup: two expert subtiles x four token
// subtiles, a tile of 2 EL experts x 4 TL tokens.  Each chain's fmas run in
// step order as before, so the logits are the same bits.
template <int EL, int TL, int STEPS>
__global__ void __launch_bounds__(256) k_router_logits_tile(const float* __restrict__ W, const float* __restrict__ x,
                                                            int64_t x_stride, int64_t H, int64_t E, int64_t T,
                                                            float* __restrict__ logits) {
    const int c = threadIdx.x & 31, gi = threadIdx.x >> 5;
    const int64_t e0 = (int64_t) blockIdx.x * (2 * EL) + (gi & 1) * EL;
    const int64_t t0 = (int64_t) blockIdx.y * (4 * TL) + (gi >> 1) * TL;
    const int64_t np = H & ~(int64_t) 31;
    const int64_t ns = np / 32;
    const float* wr[EL];
    const float* xr[TL];
#pragma unroll
    for (int i = 0; i < EL; ++i) wr[i] = W + (e0 + i < E ? e0 + i : 0) * H + c;
#pragma unroll
    for (int j = 0; j < TL; ++j) xr[j] = x + (t0 + j < T ? t0 + j : T - 1) * x_stride + c;
    float acc[EL][TL];
#pragma unroll
    for (int i = 0; i < EL; ++i)
#pragma unroll
        for (int j = 0; j < TL; ++j) acc[i][j] = 0.0f;
    float wv[STEPS][EL], xv[STEPS][TL];
    auto load = [&](int64_t s0, float (*wd)[EL], float (*xd)[TL]) {
#pragma unroll
        for (int u = 0; u < STEPS; ++u) {
            const int64_t s = (s0 + u < ns ? s0 + u : ns - 1) * 32;   // (past the end: never accumulated)
#pragma unroll
            for (int i = 0; i < EL; ++i) wd[u][i] = wr[i][s];
#pragma unroll
            for (int j = 0; j < TL; ++j) xd[u][j] = xr[j][s];
        }
    };
    if (ns > 0) load(0, wv, xv);
    for (int64_t s0 = 0; s0 < ns; s0 += STEPS) {
        float wn[STEPS][EL], xn[STEPS][TL];
        const bool more = s0 + STEPS < ns;
        if (more) load(s0 + STEPS, wn, xn);
#pragma unroll
        for (int u = 0; u < STEPS; ++u)
            if (s0 + u < ns) {
#pragma unroll
                for (int i = 0; i < EL; ++i)
#pragma unroll
                    for (int j = 0; j < TL; ++j) acc[i][j] = __builtin_fmaf(wv[u][i], xv[u][j], acc[i][j]);
            }
        if (more) {
#pragma unroll
            for (int u = 0; u < STEPS; ++u) {
#pragma unroll
                for (int i = 0; i < EL; ++i) wv[u][i] = wn[u][i];
#pragma unroll
                for (int j = 0; j < TL; ++j) xv[u][j] = xn[u][j];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < EL; ++i)
#pragma unroll
        for (int j = 0; j < TL; ++j) {
            // GGML_F32x8_REDUCE and the scalar tail, as in k_router_logits
            float v = acc[i][j] + __shfl_down(acc[i][j], 16, 32);
            v = v + __shfl_down(v, 8, 32);
            v = v + __shfl_down(v, 4, 32);
            const float u = v + __shfl_down(v, 1, 32);
            float sumf = u + __shfl_down(u, 2, 32);
            const int64_t e = e0 + i, t = t0 + j;
            if (c == 0 && e < E && t < T) {
                const float* we = W + e * H;
                const float* xt = x + t * x_stride;
                const int64_t nv = np + ((H - np) & ~(int64_t) 3);
                for (int64_t h = np; h < H; ++h)
                    sumf = (h < nv) ? sumf + we[h] * xt[h] : __builtin_fmaf(we[h], xt[h], sumf);
                logits[t * E + e] = sumf;
            }
        }
}

// Softmax, exact top-k and weight normalisation for one token per 64-thread
// workgroup.  Supports E % 8 == 0 and E <= 64 * ROUTER_EPL.
constexpr int ROUTER_EPL = 8;
__global__ void __launch_bounds__(64) k_router_topk(const float* __restrict__ logits, int64_t E, int64_t k,
                                                    int64_t T, float clamp_min, float scale, int32_t* __restrict__ ids,
                                                    float* __restrict__ weights, float* __restrict__ probs_out,
                                                    int32_t* __restrict__ status, const float* __restrict__ mask,
                                                    int32_t* __restrict__ want) {
    __shared__ __align__(16) float p[64 * ROUTER_EPL];
    __shared__ float gsum[64 * ROUTER_EPL / 8];
    __shared__ int32_t order[64 * ROUTER_EPL];
    __shared__ SortRange sort_stack[SORT_STACK];
    __shared__ int need_sort;
    topk_token<false>(logits, E, k, blockIdx.x, clamp_min, scale, ids, weights, probs_out, status, p, gsum, order,
                      sort_stack, &need_sort, threadIdx.x, mask, want);
}

int launch_router(const RouterArgs& a, float* logits_ws, hipStream_t stream) {
    if (a.E % 8 != 0 || a.E > 64 * ROUTER_EPL || a.k < 1 || a.k > a.E || a.H < 1) return -2;
    if (a.T == 0) return 0;
    float* logits = a.logits ? a.logits : logits_ws;
    if (a.xq && (a.T > 16 || a.H % QK_K)) return -2;
    if (a.T <= 16) {
        const int64_t nq = a.xq ? a.H / QK_K : 0;
        dim3 g1((unsigned) ((a.E + 1) / 2 + nq), (unsigned) a.T);
        hipLaunchKernelGGL((k_router_logits<1, 2, 32>), g1, dim3(64), 0, stream, a.W, a.x, a.x_stride, a.H, a.E, a.T,
                           logits, (BlockQ8_K*) a.xq);
    } else {
        constexpr int EL = 4, TL = 4;
        dim3 g1((unsigned) ((a.E + 2 * EL - 1) / (2 * EL)), (unsigned) ((a.T + 4 * TL - 1) / (4 * TL)));
        hipLaunchKernelGGL((k_router_logits_tile<EL, TL, 8>), g1, dim3(256), 0, stream, a.W, a.x, a.x_stride, a.H, a.E,
                           a.T, logits);
    }
    if (!a.ids) return hipGetLastError() == hipSuccess ? 0 : -3;   // logits only (top-k fused elsewhere)
    hipLaunchKernelGGL(k_router_topk, dim3((unsigned) a.T), dim3(64), 0, stream, logits, a.E, a.k, a.T, a.clamp_min,
                       a.scale, a.ids, a.weights, a.probs, a.status, a.mask, a.want);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
