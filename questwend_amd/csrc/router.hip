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

// The same logits for large batches through LDS (H % 512 == 0, E % 16 == 0):
// a workgroup computes 16 experts x 16 tokens.  256-element chunks of the 16
// router rows and 16 token rows are copied with 16-byte loads (loaded into
// registers two chunks ahead of their use) into LDS, where lane c of a
// 32-lane group reads element 32 u + c of its 4 experts and 8 tokens for step u
// (consecutive words: no bank conflicts) and runs chain c of those 32 logits in
// step order.  The chains then go to LDS, and thread l forms logit l with the
// GGML_F32x8_REDUCE tree of k_router_logits: ((c + c16) + (c8 + c24)) ... as
// (v3_0 + v3_1) + (v3_2 + v3_3).  Same bits as k_router_logits_tile.
constexpr int RL_CH = 256;
__global__ void __launch_bounds__(256) k_router_logits_lds(const float* __restrict__ W, const float* __restrict__ x,
                                                           int64_t x_stride, int64_t H, int64_t E, int64_t T,
                                                           float* __restrict__ logits) {
    __shared__ __align__(16) float s_buf[2][2][16][RL_CH];   // [stage][W, x][row][element]: 64 KB
    const int tid = threadIdx.x, c = tid & 31, g = tid >> 5;
    const int64_t e0 = (int64_t) blockIdx.x * 16, t0 = (int64_t) blockIdx.y * 16;
    const int eg = 4 * (g & 3), tg = 8 * (g >> 2);
    // copy slots: float4 f = tid + 256 k of each 16 x 256 tile, row f / 64, column 4 (f % 64)
    const int crow = tid >> 6, ccol = 4 * (tid & 63);
    const float* wsrc = W + (e0 + crow) * H + ccol;   // rows crow + 4 k: + 4 k H
    int64_t xoff[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t t = t0 + crow + 4 * k;
        xoff[k] = (t < T ? t : T - 1) * x_stride + ccol;
    }
    const int64_t nch = H / RL_CH;   // (even)
    // chunk n's copies into registers: set A holds the next chunk to store, set B
    // is loaded two chunks ahead of its use (the loop is unrolled by two so the
    // sets swap roles without a register copy of a load in flight)
    // (named registers, not arrays: an array here is moved to LDS by the compiler)
    float4 aw0, aw1, aw2, aw3, ax0, ax1, ax2, ax3, bw0, bw1, bw2, bw3, bx0, bx1, bx2, bx3;
#define RL_FETCH1(rw, rx, k, nn)                                                       \
    rw = *(const float4*) (wsrc + 4 * (k) * H + (nn) * RL_CH);                          \
    rx = *(const float4*) (x + xoff[k] + (nn) * RL_CH);
#define RL_FETCH(p, n)                                                                 \
    {                                                                                  \
        const int64_t nn = (n) < nch ? (n) : nch - 1;                                  \
        RL_FETCH1(p##w0, p##x0, 0, nn) RL_FETCH1(p##w1, p##x1, 1, nn)                  \
        RL_FETCH1(p##w2, p##x2, 2, nn) RL_FETCH1(p##w3, p##x3, 3, nn)                  \
    }
#define RL_PUT1(rw, rx, k, sb)                                                         \
    *(float4*) &s_buf[sb][0][crow + 4 * (k)][ccol] = rw;                                \
    *(float4*) &s_buf[sb][1][crow + 4 * (k)][ccol] = rx;
#define RL_PUT(p, sb)                                                                  \
    {                                                                                  \
        RL_PUT1(p##w0, p##x0, 0, sb) RL_PUT1(p##w1, p##x1, 1, sb)                      \
        RL_PUT1(p##w2, p##x2, 2, sb) RL_PUT1(p##w3, p##x3, 3, sb)                      \
    }
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
    // one chunk: step u + 1's operands are read before step u's fmas (kept there by
    // the scheduling barrier), so the LDS latency hides under the fmas
    auto chunk = [&](int sb) __attribute__((always_inline)) {
        float wv[2][4], xv[2][8];
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[0][i] = s_buf[sb][0][eg + i][c];
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[0][j] = s_buf[sb][1][tg + j][c];
#pragma unroll
        for (int u = 0; u < RL_CH / 32; ++u) {
            const int cu = u & 1, nu = cu ^ 1;
            if (u + 1 < RL_CH / 32) {
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[nu][i] = s_buf[sb][0][eg + i][32 * (u + 1) + c];
#pragma unroll
                for (int j = 0; j < 8; ++j) xv[nu][j] = s_buf[sb][1][tg + j][32 * (u + 1) + c];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_fmaf(wv[cu][i], xv[cu][j], acc[i][j]);
        }
    };
    RL_FETCH(a, 0)
    RL_PUT(a, 0)
    RL_FETCH(a, 1)
    __syncthreads();
    // (past the last chunk the copies repeat it into a stage nobody reads)
    for (int64_t ch = 0; ch < nch; ch += 2) {
        RL_FETCH(b, ch + 2)
        chunk(0);
        RL_PUT(a, 1)   // chunk ch + 1; stage 1 was last read before the previous barrier
        __syncthreads();
        RL_FETCH(a, ch + 3)
        chunk(1);
        RL_PUT(b, 0)   // chunk ch + 2
        __syncthreads();
    }
#undef RL_FETCH1
#undef RL_FETCH
#undef RL_PUT1
#undef RL_PUT
    // chains to LDS: logit l = 16 (token) + expert, 33 words per logit
    float* red = &s_buf[0][0][0][0];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) red[((tg + j) * 16 + eg + i) * 33 + c] = acc[i][j];
    __syncthreads();
    const float* a = red + tid * 33;
    float v2[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v2[q] = (a[q] + a[q + 16]) + (a[q + 8] + a[q + 24]);
    const float v3_0 = v2[0] + v2[4], v3_1 = v2[1] + v2[5], v3_2 = v2[2] + v2[6], v3_3 = v2[3] + v2[7];
    const float sumf = (v3_0 + v3_1) + (v3_2 + v3_3);
    const int64_t t = t0 + (tid >> 4), e = e0 + (tid & 15);
    if (t < T) logits[t * E + e] = sumf;
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
    } else if (a.H % (2 * RL_CH) == 0 && a.E % 16 == 0 && a.x_stride % 4 == 0 && ((uintptr_t) a.x & 15) == 0 &&
               ((uintptr_t) a.W & 15) == 0) {
        dim3 g1((unsigned) (a.E / 16), (unsigned) ((a.T + 15) / 16));
        hipLaunchKernelGGL(k_router_logits_lds, g1, dim3(256), 0, stream, a.W, a.x, a.x_stride, a.H, a.E, a.T, logits);
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
