// qw_topk.hpp -- softmax, exact top-k and weight normalisation of one token's
// router logits, for one wave (ggml_soft_max, ARGSORT + top-k, sum/clamp/div of
// core/runtime.cpp:869-897; bit-identical to the reference CPU path), with the
// resident-decode routing of core/runtime.cpp:870-881: want = the top k of the
// raw logits (ggml_argsort_top_k), then logits + mask (ggml_add of the layer's
// 0 / -inf row) before the softmax.
#pragma once

#include "qw_kernels.hpp"
#include "qw_sort.hpp"

namespace qw {

// A barrier for LDS traffic between the lanes of one wave.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ARGSORT (descending) of the E values in p, first k into order[0..k): ranks by
// count of strictly larger values; a tie group (or NaN) reaching into the first
// k places leaves the order to std::sort, which is then replayed exactly (and
// reported as status bit 0).  Ends synchronised.
template <bool WAVE>
__device__ __forceinline__ void topk_order(const float* p, int64_t E, int64_t k, int32_t* order,
                                           SortRange* sort_stack, int* need_sort, int32_t* __restrict__ status,
                                           int lane) {
    auto sync = [] {
        if constexpr (WAVE) wave_sync();
        else __syncthreads();
    };
    // (p is 16-byte aligned and E % 8 == 0: four values per LDS read)
    for (int64_t i = lane; i < E; i += 64) {
        const float pi = p[i];
        int gt = 0, eq = 0;
#pragma unroll 8
        for (int64_t j = 0; j < E; j += 4) {
            const float4 q = *(const float4*) (p + j);
            gt += (q.x > pi) + (q.y > pi) + (q.z > pi) + (q.w > pi);
            eq += (q.x == pi) + (q.y == pi) + (q.z == pi) + (q.w == pi);
        }
        if (gt < k) {
            if (eq != 1) *need_sort = 1;
            else order[gt] = (int32_t) i;
        }
    }
    sync();
    if (*need_sort) {
        if (lane == 0) {
            for (int64_t i = 0; i < E; ++i) order[i] = (int32_t) i;
            libstdcxx_sort_desc(order, (int) E, p, sort_stack);
            if (status) atomicOr(status, 1);
        }
        sync();
    }
}

// One wave (lane 0..63) handles token t.  p (16-byte aligned), order: E entries; gsum: E / 8;
// sort_stack: SORT_STACK; need_sort: one word (all in LDS, private to the wave
// when WAVE is set, else to a 64-thread workgroup).  mask: [E] added to the
// logits before the softmax, or null; want: [T][k] top k of the raw logits, or null.
template <bool WAVE>
__device__ __forceinline__ void topk_token(const float* __restrict__ logits, int64_t E, int64_t k, int64_t t,
                                           float clamp_min, float scale, int32_t* __restrict__ ids,
                                           float* __restrict__ weights, float* __restrict__ probs_out,
                                           int32_t* __restrict__ status, float* p, float* gsum, int32_t* order,
                                           SortRange* sort_stack, int* need_sort, int lane,
                                           const float* __restrict__ mask = nullptr, int32_t* __restrict__ want = nullptr) {
    auto sync = [] {
        if constexpr (WAVE) wave_sync();
        else __syncthreads();
    };
    const float* l = logits + t * E;
    if (want) {
        for (int64_t i = lane; i < E; i += 64) p[i] = l[i];
        if (lane == 0) *need_sort = 0;
        sync();
        topk_order<WAVE>(p, E, k, order, sort_stack, need_sort, status, lane);
        for (int64_t i = lane; i < k; i += 64) want[t * k + i] = order[i];
        sync();
    }
    auto lm = [&](int64_t i) { return mask ? l[i] + mask[i] : l[i]; };
    float mx = -INFINITY;
    for (int64_t i = lane; i < E; i += 64) mx = fmaxf(mx, lm(i));
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    for (int64_t i = lane; i < E; i += 64) p[i] = v_expf(lm(i) - mx);
    if (lane == 0) *need_sort = 0;
    sync();
    const int64_t ng = E / 8;
    for (int64_t gi = lane; gi < ng; gi += 64) gsum[gi] = hsum8(&p[8 * gi]);
    sync();
    double sum = 0.0;
    if (lane == 0)
        for (int64_t gi = 0; gi < ng; ++gi) sum += (double) gsum[gi];
    sum = __shfl(sum, 0);
    const float inv = (float) (1.0 / sum);
    for (int64_t i = lane; i < E; i += 64) p[i] = p[i] * inv;
    sync();
    if (probs_out)
        for (int64_t i = lane; i < E; i += 64) probs_out[t * E + i] = p[i];
    // the order of the probabilities.  A NaN (eq == 0) goes to the sort replay:
    // softmax makes every probability NaN then, which std::sort treats as all
    // equivalent.
    topk_order<WAVE>(p, E, k, order, sort_stack, need_sort, status, lane);
    if (lane == 0) {
        double s = 0.0;
        for (int64_t i = 0; i < k; ++i) s += (double) p[order[i]];
        float wsum = (float) s;
        wsum = fmaxf(fminf(wsum, INFINITY), clamp_min);
        for (int64_t i = 0; i < k; ++i) {
            float wi = p[order[i]] / wsum;
            if (scale != 0.0f && scale != 1.0f) wi = wi * scale;
            ids[t * k + i] = order[i];
            weights[t * k + i] = wi;
        }
    }
}

}  // namespace qw
