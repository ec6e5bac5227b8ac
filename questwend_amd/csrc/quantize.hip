// quantize.hip -- block quantizers on the GPU, bit-identical to ggml's CPU code.
//
// Activation quantizers (what ggml_compute_forward_mul_mat_id runs on src1,
// ggml/src/ggml-cpu/ggml-cpu.c:1585-1620, through type_traits_cpu.from_float):
//   Q8_K: quantize_row_q8_K_ref      ggml/src/ggml-quants.c:2768-2803
//   Q8_0: x86 quantize_row_q8_0      ggml/src/ggml-cpu/arch/x86/quants.c:302-404
// Weight quantizers (ggml_quantize_chunk with no imatrix, ggml/src/ggml.c:7919-8000):
//   Q4_K: quantize_row_q4_K_ref      ggml-quants.c:1457-1527 (+ make_qkx2_quants 799-878)
//   Q6_K: quantize_row_q6_K_ref      ggml-quants.c:1869-1937 (+ make_qx_quants 628-700)
//   Q8_0: quantize_row_q8_0_ref      ggml-quants.c:276-297
// Division and sqrt are IEEE correctly rounded (HIP default), no contraction.
#include "qw_kernels.hpp"

namespace qw {

// ---------------------------------------------------------------------------
// Activation Q8_K: one wave per 256-value block, 4 values per lane.
// src rows may be strided (ggml nb1/nb2 in bytes); dst rows are dense.
__global__ void __launch_bounds__(256) k_quant_q8K(const float* __restrict__ src, int64_t K, int64_t ne1,
                                                   int64_t nrows, size_t nb1, size_t nb2,
                                                   BlockQ8_K* __restrict__ dst, _Float16* __restrict__ hout) {
    const int lane = threadIdx.x & 63;
    const int64_t nb = K / QK_K;
    const int64_t blk = (int64_t) blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (blk >= nb * nrows) return;
    const int64_t row = blk / nb, ib = blk % nb;
    const int64_t i1 = row % ne1, i2 = row / ne1;
    const float* x = (const float*) ((const char*) src + i1 * nb1 + i2 * nb2) + ib * QK_K;
    const float4 q = *(const float4*) (x + 4 * lane);
    const float v[4] = {q.x, q.y, q.z, q.w};
    quant_q8K_wave(v, lane, dst + blk, hout ? hout + (size_t) blk * QK_K : nullptr);
}

// SwiGLU (ggml_swiglu_split: silu(gate) * up, ops.cpp:3182-3238) of n_rows dense
// rows of F values, quantized straight to Q8_K as the down projection reads it:
// one wave per 256-value block, the same values and quantizer as k_swiglu then
// k_quant_q8K, without the fp32 round trip.
__global__ void __launch_bounds__(256) k_swiglu_q8K(const float* __restrict__ gate, const float* __restrict__ up,
                                                    int64_t F, int64_t n_rows, BlockQ8_K* __restrict__ dst,
                                                    _Float16* __restrict__ hout) {
    const int lane = threadIdx.x & 63;
    const int64_t nb = F / QK_K;
    const int64_t blk = (int64_t) blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (blk >= nb * n_rows) return;
    const int64_t off = (blk / nb) * F + (blk % nb) * QK_K + 4 * lane;
    const float4 g = *(const float4*) (gate + off);
    const float4 u = *(const float4*) (up + off);
    const float v[4] = {v_silu(g.x) * u.x, v_silu(g.y) * u.y, v_silu(g.z) * u.z, v_silu(g.w) * u.w};
    quant_q8K_wave(v, lane, dst + blk, hout ? hout + (size_t) blk * QK_K : nullptr);
}

int launch_swiglu_q8K(const float* gate, const float* up, int64_t F, int64_t n_rows, void* dst, hipStream_t stream,
                      uint16_t* h_out) {
    if (F % QK_K) return -2;
    const int64_t nblk = (F / QK_K) * n_rows;
    if (nblk == 0) return 0;
    hipLaunchKernelGGL(k_swiglu_q8K, dim3((unsigned) ((nblk + 3) / 4)), dim3(256), 0, stream, gate, up, F, n_rows,
                       (BlockQ8_K*) dst, (_Float16*) h_out);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Activation Q8_0 (x86 AVX2 branch): one 32-value block per 8 lanes, 4 per lane.
__global__ void __launch_bounds__(256) k_quant_q8_0_act(const float* __restrict__ src, int64_t K, int64_t ne1,
                                                        int64_t nrows, size_t nb1, size_t nb2,
                                                        BlockQ8_0* __restrict__ dst) {
    const int64_t nb = K / QK8_0;
    const int64_t gid = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int sub = threadIdx.x & 7;
    const bool valid = blk < nb * nrows;
    const int64_t b = valid ? blk : 0;
    const int64_t row = b / nb, ib = b % nb;
    const int64_t i1 = row % ne1, i2 = row / ne1;
    const float* x = (const float*) ((const char*) src + i1 * nb1 + i2 * nb2) + ib * QK8_0;
    float4 q = *(const float4*) (x + 4 * sub);
    float m = fmaxf(fmaxf(__builtin_fabsf(q.x), __builtin_fabsf(q.y)), fmaxf(__builtin_fabsf(q.z), __builtin_fabsf(q.w)));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 4));
    if (!valid) return;
    const float d = m / 127.f;
    const float id = (m != 0.0f) ? 127.f / m : 0.0f;
    BlockQ8_0* y = dst + blk;
    const int q0 = (int) __builtin_rintf(q.x * id), q1 = (int) __builtin_rintf(q.y * id);
    const int q2 = (int) __builtin_rintf(q.z * id), q3 = (int) __builtin_rintf(q.w * id);
    const uint32_t packed = (uint32_t) (q0 & 0xff) | ((uint32_t) (q1 & 0xff) << 8) | ((uint32_t) (q2 & 0xff) << 16) |
                            ((uint32_t) (q3 & 0xff) << 24);
    // qs starts at byte 2 of the 34-byte block: write as two 16-bit halves
    uint16_t* qs16 = (uint16_t*) ((char*) y + 2 + 4 * sub);
    qs16[0] = (uint16_t) (packed & 0xffff);
    qs16[1] = (uint16_t) (packed >> 16);
    if (sub == 0) y->d = f2h(d);
}

int launch_quantize_act(int vdt, const float* src, int64_t K, int64_t ne1, int64_t nrows, size_t nb1, size_t nb2,
                        void* dst, hipStream_t stream, uint16_t* h_out) {
    if (h_out && vdt != T_Q8_K) return -2;
    if (vdt == T_Q8_K) {
        const int64_t nblk = (K / QK_K) * nrows;
        if (nblk == 0) return 0;
        hipLaunchKernelGGL(k_quant_q8K, dim3((unsigned) ((nblk + 3) / 4)), dim3(256), 0, stream, src, K, ne1, nrows,
                           nb1, nb2, (BlockQ8_K*) dst, (_Float16*) h_out);
    } else if (vdt == T_Q8_0) {
        const int64_t nthr = (K / QK8_0) * nrows * 8;
        if (nthr == 0) return 0;
        hipLaunchKernelGGL(k_quant_q8_0_act, dim3((unsigned) ((nthr + 255) / 256)), dim3(256), 0, stream, src, K, ne1,
                           nrows, nb1, nb2, (BlockQ8_0*) dst);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ---------------------------------------------------------------------------
// Weight quantizers.  One thread per 32-value sub-block (Q4_K) or 16-value
// sub-block (Q6_K); the super-block finalisation is done by the first thread of
// each group after exchanging the sub-block results through shuffles.

// make_qkx2_quants(32, 15, x, weights, L, &min, Laux, -1, 0.1, 20, false)
__device__ float qkx2_32(const float* x, const float* w, uint8_t* L, float* the_min) {
    const int n = 32, nmax = 15;
    const float rmin = -1.f, rdelta = 0.1f;
    const int nstep = 20;
    float min = x[0], max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float wi = w[i];
        sum_w += wi;
        sum_x += wi * x[i];
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
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t) l;
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        best_error += w[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        uint8_t Laux[32];
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t) l;
            const float wi = w[i];
            sum_l += wi * l;
            sum_l2 += wi * l * l;
            sum_xl += wi * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += w[i] * diff;
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

// 8 threads per Q4_K super-block; thread j owns sub-block j (32 values).
__global__ void __launch_bounds__(256) k_quant_w_q4K(const float* __restrict__ src, int64_t nblocks,
                                                     BlockQ4_K* __restrict__ dst) {
    const int64_t gid = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int j = (int) (gid & 7);
    const bool valid = blk < nblocks;
    const float* x = src + (valid ? blk : 0) * QK_K + 32 * j;
    float xv[32], wv[32];
    uint8_t L[32];
    float sum_x2 = 0;
    for (int l = 0; l < 32; ++l) {
        xv[l] = x[l];
        sum_x2 += xv[l] * xv[l];
    }
    const float av_x = sqrtf(sum_x2 / 32);
    for (int l = 0; l < 32; ++l) wv[l] = av_x + __builtin_fabsf(xv[l]);
    float mn;
    const float sc = qkx2_32(xv, wv, L, &mn);
    // super-block maxima over the 8 sub-blocks, in sub-block order (strict >)
    float max_scale = 0, max_min = 0;
    float scales[8], mins[8];
    for (int t = 0; t < 8; ++t) {
        scales[t] = __shfl(sc, (threadIdx.x & ~7) + t);
        mins[t] = __shfl(mn, (threadIdx.x & ~7) + t);
        if (scales[t] > max_scale) max_scale = scales[t];
        if (mins[t] > max_min) max_min = mins[t];
    }
    if (!valid) return;
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t sbytes[12];
    for (int t = 0; t < 12; ++t) sbytes[t] = 0;
    for (int t = 0; t < 8; ++t) {
        uint8_t ls = (uint8_t) nearest_int(inv_scale * scales[t]);
        uint8_t lm = (uint8_t) nearest_int(inv_min * mins[t]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        if (t < 4) {
            sbytes[t] = ls;
            sbytes[t + 4] = lm;
        } else {
            sbytes[t + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
            sbytes[t - 4] |= (uint8_t) ((ls >> 4) << 6);
            sbytes[t - 0] |= (uint8_t) ((lm >> 4) << 6);
        }
    }
    const uint16_t dh = f2h(max_scale / 63.f), mh = f2h(max_min / 63.f);
    int scj, mj;
    scale_min_k4(j, sbytes, scj, mj);
    const float d = h2f(dh) * scj;
    if (d != 0.0f) {
        const float dm = h2f(mh) * mj;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((xv[ii] + dm) / d);
            L[ii] = (uint8_t) (l < 0 ? 0 : (l > 15 ? 15 : l));
        }
    }
    // sub-block j = 2*c + h  ->  qs[32c + l] nibble h.  Gather the partner's L.
    BlockQ4_K* y = dst + blk;
    const int c = j >> 1, h = j & 1;
    // thread with h==0 writes the byte pair for chunk c using partner (j+1)'s L values
    for (int l = 0; l < 32; ++l) {
        const int other = __shfl_xor((int) L[l], 1);
        if (h == 0) y->qs[32 * c + l] = (uint8_t) (L[l] | (other << 4));
    }
    if (j == 0) {
        y->d = dh;
        y->dmin = mh;
        for (int t = 0; t < 12; ++t) y->scales[t] = sbytes[t];
    }
}

// make_qx_quants(16, 32, x, L, rmse_type = 1, NULL)
__device__ float qx_16(const float* x, int8_t* L) {
    const int n = 16, nmax = 32;
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = __builtin_fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t) (l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t) (nmax + (l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// 16 threads per Q6_K super-block; thread ib owns sub-block ib (16 values).
__global__ void __launch_bounds__(256) k_quant_w_q6K(const float* __restrict__ src, int64_t nblocks,
                                                     BlockQ6_K* __restrict__ dst) {
    const int64_t gid = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 4;
    const int ib = (int) (gid & 15);
    const bool valid = blk < nblocks;
    const float* x = src + (valid ? blk : 0) * QK_K + 16 * ib;
    float xv[16];
    int8_t L[16];
    for (int l = 0; l < 16; ++l) xv[l] = x[l];
    const float sc = qx_16(xv, L);
    float max_scale = 0, max_abs_scale = 0;
    const int base = threadIdx.x & ~15;
    for (int t = 0; t < 16; ++t) {
        const float s = __shfl(sc, base + t);
        const float as = __builtin_fabsf(s);
        if (as > max_abs_scale) { max_abs_scale = as; max_scale = s; }
    }
    if (!valid) return;
    BlockQ6_K* y = dst + blk;
    uint8_t Lu[16];
    int8_t my_scale = 0;
    uint16_t dh = 0;
    if (max_abs_scale < 1e-15f) {
        for (int l = 0; l < 16; ++l) Lu[l] = 0;  // block is all zeros (memset in the reference)
        dh = f2h(0.f);
    } else {
        const float iscale = -128.f / max_scale;
        dh = f2h(1 / iscale);
        const int q = nearest_int(iscale * sc);
        my_scale = (int8_t) (q < 127 ? q : 127);
        const float d = h2f(dh) * my_scale;
        for (int l = 0; l < 16; ++l) Lu[l] = (uint8_t) L[l];
        if (d != 0.0f) {
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(xv[ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                Lu[ii] = (uint8_t) (l + 32);
            }
        }
    }
    // Packing (quantize_row_q6_K_ref): element e = 128*jj + 32*m + l (l < 32) ->
    // ql[64*jj + 32*(m&1) + l] nibble (m>>1), qh[32*jj + l] bits 2m..2m+1.
    // Thread ib holds elements 16*ib .. 16*ib+15: jj = ib/8, m = (ib%8)/2, l0 = 16*(ib&1).
    const int jj = ib >> 3, m = (ib & 7) >> 1, l0 = 16 * (ib & 1);
    // Assemble per byte from the 4 m-threads sharing (jj, l0): thread with m == 0 writes.
    for (int l = 0; l < 16; ++l) {
        const int v = Lu[l];
        const int v_m1 = __shfl(v, base + (jj * 8 + 2 * 1 + (ib & 1)));
        const int v_m2 = __shfl(v, base + (jj * 8 + 2 * 2 + (ib & 1)));
        const int v_m3 = __shfl(v, base + (jj * 8 + 2 * 3 + (ib & 1)));
        if (m == 0) {
            y->ql[64 * jj + l0 + l] = (uint8_t) ((v & 0xF) | ((v_m2 & 0xF) << 4));
            y->ql[64 * jj + 32 + l0 + l] = (uint8_t) ((v_m1 & 0xF) | ((v_m3 & 0xF) << 4));
            y->qh[32 * jj + l0 + l] = (uint8_t) ((v >> 4) | ((v_m1 >> 4) << 2) | ((v_m2 >> 4) << 4) | ((v_m3 >> 4) << 6));
        }
    }
    y->scales[ib] = my_scale;
    if (ib == 0) y->d = dh;
}

// Q8_0 weights (quantize_row_q8_0_ref): one thread per 32-value block.
__global__ void __launch_bounds__(256) k_quant_w_q8_0(const float* __restrict__ src, int64_t nblocks,
                                                      BlockQ8_0* __restrict__ dst) {
    const int64_t blk = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblocks) return;
    const float* x = src + blk * QK8_0;
    float amax = 0.0f;
    for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, __builtin_fabsf(x[j]));
    const float d = amax / ((1 << 7) - 1);
    const float id = d ? 1.0f / d : 0.0f;
    BlockQ8_0* y = dst + blk;
    y->d = f2h(d);
    for (int j = 0; j < QK8_0; ++j) y->qs[j] = (int8_t) roundf(x[j] * id);
}

int launch_quantize_weights(int type, const float* src, int64_t n, void* dst, hipStream_t stream) {
    if (type == T_Q4_K) {
        const int64_t nb = n / QK_K;
        hipLaunchKernelGGL(k_quant_w_q4K, dim3((unsigned) ((nb * 8 + 255) / 256)), dim3(256), 0, stream, src, nb,
                           (BlockQ4_K*) dst);
    } else if (type == T_Q6_K) {
        const int64_t nb = n / QK_K;
        hipLaunchKernelGGL(k_quant_w_q6K, dim3((unsigned) ((nb * 16 + 255) / 256)), dim3(256), 0, stream, src, nb,
                           (BlockQ6_K*) dst);
    } else if (type == T_Q8_0) {
        const int64_t nb = n / QK8_0;
        hipLaunchKernelGGL(k_quant_w_q8_0, dim3((unsigned) ((nb + 255) / 256)), dim3(256), 0, stream, src, nb,
                           (BlockQ8_0*) dst);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ---------------------------------------------------------------------------
// Dequantizers (dequantize_row_q8_0 / _q4_K / _q6_K, ggml-quants.c:553-566,
// 1529-1551, 1939-1968): one thread per output value.
__global__ void k_dequant(int type, const uint8_t* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (type == T_Q8_0) {
        const BlockQ8_0* b = (const BlockQ8_0*) x + i / QK8_0;
        y[i] = b->qs[i % QK8_0] * h2f(b->d);
    } else if (type == T_Q4_K) {
        const BlockQ4_K* b = (const BlockQ4_K*) x + i / QK_K;
        const int e = (int) (i % QK_K);
        const int c = e / 64, within = e % 64, hi = within >= 32, l = within & 31;
        int sc, m;
        scale_min_k4(2 * c + hi, b->scales, sc, m);
        const float d = h2f(b->d) * sc, mn = h2f(b->dmin) * m;
        const int q = hi ? (b->qs[32 * c + l] >> 4) : (b->qs[32 * c + l] & 0xF);
        y[i] = d * q - mn;
    } else if (type == T_Q6_K) {
        const BlockQ6_K* b = (const BlockQ6_K*) x + i / QK_K;
        const int e = (int) (i % QK_K);
        const int half = e / 128, r = e % 128, m = r / 32, l = r % 32;
        const uint8_t* ql = b->ql + 64 * half;
        const uint8_t* qh = b->qh + 32 * half;
        int q;
        switch (m) {
            case 0: q = (ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4); break;
            case 1: q = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4); break;
            case 2: q = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4); break;
            default: q = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4); break;
        }
        const int is = l / 16;
        y[i] = h2f(b->d) * b->scales[8 * half + is + 2 * m] * (float) (q - 32);
    }
}

int launch_dequantize(int type, const void* x, float* y, int64_t n, hipStream_t stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream, type, (const uint8_t*) x,
                       y, n);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ---------------------------------------------------------------------------
// Seeded N(mean, std) fp32 generator for synthetic weights and inputs:
// splitmix64 over (seed, index) and a Box-Muller pair.  Deterministic on the
// GPU for a given seed; not meant to match any CPU generator bit for bit.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ void k_randn(float* __restrict__ y, int64_t n, uint64_t seed, float mean, float stddev) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t pair = i >> 1;
    if (2 * pair >= n) return;
    const uint64_t r = splitmix64(seed * 0x9e3779b97f4a7c15ull ^ splitmix64((uint64_t) pair));
    const float u1 = ((float) (r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float) ((r >> 16) & 0xffffff) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1));
    const float ang = 6.283185307179586f * u2;
    const float z = (i & 1) ? rad * sinf(ang) : rad * cosf(ang);
    if (i < n) y[i] = mean + stddev * z;
}

int launch_randn(float* y, int64_t n, uint64_t seed, float mean, float stddev, hipStream_t stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_randn, dim3((unsigned) ((n + 1 + 255) / 256)), dim3(256), 0, stream, y, n, seed, mean, stddev);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
