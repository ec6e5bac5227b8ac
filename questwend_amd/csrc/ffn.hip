// ffn.hip -- the element-wise tail of the MoE FFN, bit-identical to the
// reference CPU path.
//   swiglu_split(gate, up)   ggml/src/ggml-cpu/ops.cpp:3182-3238, vec.cpp:417-445 (AVX2 ggml_v_silu)
//   weighted expert sum      core/runtime.cpp:940-959: T == 1 -> mul_mat of the
//                            transposed experts by the weights (ggml_vec_dot_f32 of
//                            length k); T > 1 -> mul by the weights, then an add
//                            chain in slot order
//   rms_norm                 ggml/src/ggml-cpu/ops.cpp:3795-3860, then optionally
//                            ggml_mul by a norm weight (the router input of a
//                            decoder layer, core/runtime.cpp:2028-2030)
//   shared-expert gate       core/runtime.cpp:963-972: sigmoid(mul_mat(gate_inp, x))
//                            times the shared expert's output, added to the MoE output
#include "qw_kernels.hpp"

namespace qw {

// Rows of n values; n % 8 == 0 so every value takes the 8-lane SIMD path.
__global__ void k_swiglu(const float* __restrict__ gate, const float* __restrict__ up, float* __restrict__ out,
                         int64_t n_rows, int64_t n, size_t gs, size_t us, size_t os) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * n) return;
    const int64_t r = i / n, c = i % n;
    const float g = ((const float*) ((const char*) gate + r * gs))[c];
    const float u = ((const float*) ((const char*) up + r * us))[c];
    ((float*) ((char*) out + r * os))[c] = v_silu(g) * u;
}

int launch_swiglu(const float* gate, const float* up, float* out, int64_t n_rows, int64_t n, size_t g_stride,
                  size_t u_stride, size_t o_stride, hipStream_t stream) {
    if (n % 8 != 0) return -2;
    const int64_t tot = n_rows * n;
    if (tot == 0) return 0;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned) ((tot + 255) / 256)), dim3(256), 0, stream, gate, up, out, n_rows, n,
                       g_stride, u_stride, o_stride);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ggml_vec_dot_f32 (AVX, vec.cpp:11-140) of x (stride xs) and y, one thread.
__device__ __forceinline__ float vec_dot_f32_avx(int64_t n, const float* x, int64_t xs, const float* y) {
    const int64_t np = n & ~(int64_t) 31;
    float sumf;
    if (np > 0) {
        float c[32];
        for (int i = 0; i < 32; ++i) c[i] = 0.0f;
        for (int64_t s = 0; s < np; s += 32)
            for (int i = 0; i < 32; ++i) c[i] = __builtin_fmaf(x[(s + i) * xs], y[s + i], c[i]);
        float s8[8];
        for (int l = 0; l < 8; ++l) s8[l] = (c[l] + c[16 + l]) + (c[8 + l] + c[24 + l]);
        float t0[4];
        for (int l = 0; l < 4; ++l) t0[l] = s8[l] + s8[l + 4];
        sumf = (t0[0] + t0[1]) + (t0[2] + t0[3]);
    } else {
        sumf = 0.0f;
    }
    const int64_t nv = np + ((n - np) & ~(int64_t) 3);
    for (int64_t i = np; i < n; ++i)
        sumf = (i < nv) ? sumf + x[i * xs] * y[i] : __builtin_fmaf(x[i * xs], y[i], sumf);
    return sumf;
}

// experts: [T][k][H]; weights: [T][k]; out: [T][H]
__global__ void k_weighted_sum(const float* __restrict__ ex, const float* __restrict__ w, float* __restrict__ out,
                               int64_t H, int64_t k, int64_t T) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H * T) return;
    const int64_t t = i / H, h = i % H;
    const float* e = ex + t * k * H + h;
    const float* wt = w + t * k;
    if (T == 1) {
        out[i] = vec_dot_f32_avx(k, e, H, wt);
    } else {
        float acc = e[0] * wt[0];
        for (int64_t s = 1; s < k; ++s) acc = acc + e[s * H] * wt[s];
        out[i] = acc;
    }
}

int launch_weighted_sum(const float* experts, const float* weights, float* out, int64_t H, int64_t k, int64_t T,
                        hipStream_t stream) {
    const int64_t tot = H * T;
    if (tot == 0) return 0;
    hipLaunchKernelGGL(k_weighted_sum, dim3((unsigned) ((tot + 255) / 256)), dim3(256), 0, stream, experts, weights,
                       out, H, k, T);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// One row per 256-thread block.  The reference sums x*x in double, in order;
// the tree order used here can only differ after the final rounding to float
// when the sum lies within ~1e-13 (relative) of a float rounding boundary.
// w (optional, [n]): ggml_mul of the normed row by the norm weight, rounded
// after the scale as the two ops round.
__global__ void __launch_bounds__(256) k_rms_norm(const float* __restrict__ x, float* __restrict__ y, int64_t n,
                                                  float eps, const float* __restrict__ w) {
    __shared__ double part[4];
    const float* xr = x + (int64_t) blockIdx.x * n;
    float* yr = y + (int64_t) blockIdx.x * n;
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
    if (w)
        for (int64_t i = threadIdx.x; i < n; i += 256) yr[i] = (xr[i] * scale) * w[i];
    else
        for (int64_t i = threadIdx.x; i < n; i += 256) yr[i] = xr[i] * scale;
}

int launch_rms_norm(const float* x, float* y, int64_t n, int64_t rows, float eps, hipStream_t stream,
                    const float* weight) {
    if (rows == 0) return 0;
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned) rows), dim3(256), 0, stream, x, y, n, eps, weight);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ggml_vec_dot_f32 of H values (H % 32 == 0) in its AVX2 order: lane c < 32 of
// the calling wave runs chain c (c, c + 32, ... fused), lane 0 returns the sum
// tree (vec.cpp:11-140 with GGML_F32_STEP 32, GGML_F32_EPR 8).
__device__ __forceinline__ float vec_dot_f32_wave(int64_t H, const float* x, const float* y, int lane) {
    float c = 0.0f;
    if (lane < 32)
        for (int64_t s = lane; s < H; s += 32) c = __builtin_fmaf(x[s], y[s], c);
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __shfl(c, i);
    float s8[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) s8[l] = (v[l] + v[16 + l]) + (v[8 + l] + v[24 + l]);
    float t0[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) t0[l] = s8[l] + s8[l + 4];
    return (t0[0] + t0[1]) + (t0[2] + t0[3]);
}

// The shared expert's gate and its share of the layer output, one token per
// 256-thread block: g = ggml_sigmoid(gate_inp . x) = 1 / (1 + expf(-dot)),
// then out = moe_out + sh * g (and + resid when given), each op rounded as
// ggml's mul and add round.  expf is taken in double and rounded once, which
// gives the correctly rounded float the reference's libm expf returns (that
// one is correctly rounded except in rare cases within 1 ulp).
__global__ void __launch_bounds__(256) k_shared_gate_add(const float* __restrict__ x, size_t x_stride,
                                                         const float* __restrict__ gate_inp,
                                                         const float* __restrict__ sh, const float* moe_out,
                                                         const float* __restrict__ resid, float* out,
                                                         size_t o_stride, int64_t H) {
    __shared__ float s_g;
    const int64_t t = blockIdx.x;
    const float* xt = x + (size_t) t * x_stride;
    if (threadIdx.x < 64) {
        const float d = vec_dot_f32_wave(H, gate_inp, xt, (int) threadIdx.x);
        if (threadIdx.x == 0) {
            const float e = (float) exp((double) (-d));
            s_g = 1.0f / (1.0f + e);
        }
    }
    __syncthreads();
    const float g = s_g;
    const float* mo = moe_out + (size_t) t * o_stride;
    float* o = out + (size_t) t * o_stride;
    const float* sht = sh + (size_t) t * H;
    const float* rt = resid ? resid + (size_t) t * o_stride : nullptr;
    for (int64_t h = threadIdx.x; h < H; h += 256) {
        const float v = mo[h] + sht[h] * g;
        o[h] = rt ? v + rt[h] : v;
    }
}

int launch_shared_gate_add(const float* x, size_t x_stride, const float* gate_inp, const float* sh,
                           const float* moe_out, const float* resid, float* out, size_t o_stride, int64_t H, int64_t T,
                           hipStream_t stream) {
    if (H % 32 != 0) return -2;
    if (T == 0) return 0;
    hipLaunchKernelGGL(k_shared_gate_add, dim3((unsigned) T), dim3(256), 0, stream, x, x_stride, gate_inp, sh, moe_out,
                       resid, out, o_stride, H);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// The weighted expert sum of one token (as k_weighted_sum) and its RMSNorm (as
// k_rms_norm), one 1024-thread block per token: the sums go to LDS in
// parallel, then the first 256 threads form the double sum of squares in
// k_rms_norm's per-thread order and reduce it as it does.
__global__ void __launch_bounds__(1024) k_weighted_sum_rms(const float* __restrict__ ex, const float* __restrict__ w,
                                                           float* __restrict__ out, float* __restrict__ xn, int64_t H,
                                                           int64_t k, int64_t T, float eps) {
    extern __shared__ float ys[];
    __shared__ double part[4];
    const int64_t t = blockIdx.x;
    const float* e0 = ex + t * k * H;
    const float* wt = w + t * k;
    if (T == 1 && k >= 32) {
        for (int64_t h = threadIdx.x; h < H; h += 1024) {
            const float v = vec_dot_f32_avx(k, e0 + h, H, wt);
            out[t * H + h] = v;
            ys[h] = v;
        }
    } else {
        // four outputs per thread, eight experts' values loaded together; each
        // output's sequence is the one above: T == 1 -> vec_dot_f32's scalar tail
        // (groups of four as mul + add, the rest fused), T > 1 -> mul, then adds
        const int64_t nv = k & ~(int64_t) 3;
        for (int64_t h0 = threadIdx.x; h0 < H; h0 += 4 * 1024) {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int64_t j0 = 0; j0 < k; j0 += 8) {
                float ev[8][4];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int64_t h = h0 + 1024 * u, j = j0 + jj;
                        ev[jj][u] = e0[(j < k ? j : k - 1) * H + (h < H ? h : H - 1)];
                    }
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int64_t j = j0 + jj;
                    if (j >= k) break;
                    const float wj = wt[j];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        if (T == 1) acc[u] = (j < nv) ? acc[u] + ev[jj][u] * wj : __builtin_fmaf(ev[jj][u], wj, acc[u]);
                        else acc[u] = j == 0 ? ev[jj][u] * wj : acc[u] + ev[jj][u] * wj;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t h = h0 + 1024 * u;
                if (h < H) {
                    out[t * H + h] = acc[u];
                    ys[h] = acc[u];
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < 256) {
        double s = 0.0;
        for (int64_t h = threadIdx.x; h < H; h += 256) {
            const float v = ys[h];
            s += (double) (v * v);
        }
        for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    }
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float mean = (float) (tot / (double) H);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t h = threadIdx.x; h < H; h += 1024) xn[t * H + h] = ys[h] * scale;
}

// The same for T > 1 with H % 1024 == 0, one 256-thread block per token: thread i
// forms outputs 4 i + 1024 m .. + 3 (16-byte loads, every expert's loads of a
// group of eight issued together), each as k_weighted_sum_rms does for T > 1
// (a multiply, then adds of the products in expert order).  The sum of squares
// reads the outputs back from LDS in k_rms_norm's per-thread order.
__global__ void __launch_bounds__(256) k_weighted_sum_rms4(const float* __restrict__ ex, const float* __restrict__ w,
                                                           float* __restrict__ out, float* __restrict__ xn, int64_t H,
                                                           int64_t k, float eps) {
    extern __shared__ float ys[];
    __shared__ double part[4];
    const int64_t t = blockIdx.x;
    const float* e0 = ex + t * k * H;
    const float* wt = w + t * k;
    const int tid = threadIdx.x;
    for (int64_t h = 4 * tid; h < H; h += 1024) {
        float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t j0 = 0; j0 < k; j0 += 8) {
            float4 ev[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) ev[jj] = *(const float4*) (e0 + (j0 + jj < k ? j0 + jj : k - 1) * H + h);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int64_t j = j0 + jj;
                if (j >= k) break;
                const float wj = wt[j];
                if (j == 0) acc = float4{ev[jj].x * wj, ev[jj].y * wj, ev[jj].z * wj, ev[jj].w * wj};
                else
                    acc = float4{acc.x + ev[jj].x * wj, acc.y + ev[jj].y * wj, acc.z + ev[jj].z * wj,
                                 acc.w + ev[jj].w * wj};
            }
        }
        *(float4*) (out + t * H + h) = acc;
        *(float4*) (ys + h) = acc;
    }
    __syncthreads();
    double s = 0.0;
    for (int64_t h = tid; h < H; h += 256) {
        const float v = ys[h];
        s += (double) (v * v);
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float mean = (float) (tot / (double) H);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t h = 4 * tid; h < H; h += 1024) {
        const float4 v = *(const float4*) (ys + h);
        *(float4*) (xn + t * H + h) = float4{v.x * scale, v.y * scale, v.z * scale, v.w * scale};
    }
}

int launch_weighted_sum_rms(const float* experts, const float* weights, float* out, float* x_next, int64_t H,
                            int64_t k, int64_t T, float eps, hipStream_t stream) {
    if (T == 0) return 0;
    if ((size_t) H * 4 > 64 * 1024) return -2;
    if (T > 1 && H % 1024 == 0 && k >= 1 && ((uintptr_t) experts & 15) == 0 && ((uintptr_t) out & 15) == 0 &&
        ((uintptr_t) x_next & 15) == 0) {
        hipLaunchKernelGGL(k_weighted_sum_rms4, dim3((unsigned) T), dim3(256), (size_t) H * 4, stream, experts, weights,
                           out, x_next, H, k, eps);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    hipLaunchKernelGGL(k_weighted_sum_rms, dim3((unsigned) T), dim3(1024), (size_t) H * 4, stream, experts, weights,
                       out, x_next, H, k, T, eps);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
