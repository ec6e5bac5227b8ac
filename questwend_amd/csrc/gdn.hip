// gdn.hip -- the recurrent half of Seg A for the gated-delta-net layers of
// qwen3next / qwen35moe (core/runtime.cpp:1976-1995 with build_gdn, 737-859):
// the causal depthwise conv over [conv_state | qkv] with its state update,
// SiLU, the per-head L2 norms of q and k, beta = sigmoid, g = softplus(alpha +
// dt_bias) * ssm_a, ggml_gated_delta_net's recurrence over the tokens with the
// state update, and the gated RMSNorm.  The five projections (attn_qkv,
// attn_gate, ssm_beta, ssm_alpha, ssm_out) run on the quantized mul_mat kernels
// as one-expert mul_mat_ids (api.cpp).
//
// Layout in HBM: qkv, conv [T][conv_ch] f32 (conv_ch = H_v S + 2 H_k S: q heads,
// then k heads, then v heads); conv_state [conv_ch][d_conv - 1] and the state
// [H_v][S][S] f32 in ggml's layouts (state[h][j][i] = S_h[i][j], ops.cpp:
// 10840-10842); qn, kn [T][H_k][S]; bg [T][H_v][2] (beta, g); o [T][H_v][S];
// y [T][H_v S].
//
// The float steps follow ggml's CPU ops: ggml_compute_forward_ssm_conv_f32
// (ops.cpp:9557-9610: a float sum over the d_conv taps in order), silu as
// ggml_v_silu, l2_norm with a double sum of squares (ops.cpp:4174-4219),
// sigmoid and softplus (threshold 20) as unary-ops.cpp:31-33 and 80-82, the
// recurrence as ggml_compute_forward_gated_delta_net_one_chunk (ops.cpp:
// 10734-10887; scalar gate), rms_norm with a double sum.  The recurrence's dots
// are summed in another order than ggml's vec_dot_f32, so results agree with
// the CPU backend to float rounding (the 1e-3 bar), not bit for bit.
#include "qw_kernels.hpp"

namespace qw {

namespace {

constexpr int GS = 128;        // state size S (ssm.state_size of the Qwen3-Next family)
constexpr int GJB = 8;         // state rows j per workgroup of the recurrence (32 lanes per row)

// One thread per channel: the d_conv-tap window over [conv_state | qkv rows]
// for every token, SiLU, and the state's new contents (the last d_conv - 1
// inputs).
__global__ void __launch_bounds__(256) k_gdn_conv(GdnArgs a) {
    const int64_t c = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (c >= a.conv_ch) return;
    const int dc = a.d_conv;
    float w[GDN_MAX_CONV], win[GDN_MAX_CONV];
#pragma unroll
    for (int j = 0; j < GDN_MAX_CONV; ++j) {
        w[j] = j < dc ? a.conv1d[c * dc + j] : 0.0f;
        win[j] = j < dc - 1 ? a.conv_state[c * (dc - 1) + j] : 0.0f;
    }
    for (int t = 0; t < a.T; ++t) {
        const float x = a.qkv[(int64_t) t * a.conv_ch + c];
#pragma unroll
        for (int j = 0; j < GDN_MAX_CONV; ++j)
            if (j == dc - 1) win[j] = x;   // (no dynamic index: the window stays in registers)
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < GDN_MAX_CONV; ++j)
            if (j < dc) s = __builtin_fmaf(win[j], w[j], s);
        a.conv[(int64_t) t * a.conv_ch + c] = v_silu(s);
#pragma unroll
        for (int j = 0; j + 1 < GDN_MAX_CONV; ++j)
            if (j < dc - 1) win[j] = win[j + 1];
    }
#pragma unroll
    for (int j = 0; j + 1 < GDN_MAX_CONV; ++j)
        if (j < dc - 1) a.conv_state[c * (dc - 1) + j] = win[j];
}

// Block (t, key head): q and k of that head divided by max(||.||, eps) (the
// sum of squares in double, as ggml_l2_norm); block (t, H_k) instead forms
// beta and g of every value head.
__global__ void __launch_bounds__(GS) k_gdn_prep(GdnArgs a) {
    const int t = blockIdx.x, hk = blockIdx.y, i = threadIdx.x;
    __shared__ double s_red[2][GS / 64];
    if (hk == a.H_k) {
        for (int hv = i; hv < a.H_v; hv += GS) {
            const float b = a.braw[(int64_t) t * a.H_v + hv];
            const float al = a.araw[(int64_t) t * a.H_v + hv] + a.dt_bias[hv];
            const float sp = al > 20.0f ? al : logf(1.0f + expf(al));
            a.bg[((int64_t) t * a.H_v + hv) * 2] = 1.0f / (1.0f + expf(-b));
            a.bg[((int64_t) t * a.H_v + hv) * 2 + 1] = sp * a.ssm_a[hv];
        }
        return;
    }
    const int64_t key_dim = (int64_t) a.H_k * GS;
    const float q = a.conv[(int64_t) t * a.conv_ch + hk * GS + i];
    const float k = a.conv[(int64_t) t * a.conv_ch + key_dim + hk * GS + i];
    double sq = (double) (q * q), sk = (double) (k * k);
    for (int off = 32; off >= 1; off >>= 1) {
        sq += __shfl_xor(sq, off);
        sk += __shfl_xor(sk, off);
    }
    if ((i & 63) == 0) {
        s_red[0][i >> 6] = sq;
        s_red[1][i >> 6] = sk;
    }
    __syncthreads();
    double tq = 0.0, tk = 0.0;
#pragma unroll
    for (int w = 0; w < GS / 64; ++w) {
        tq += s_red[0][w];
        tk += s_red[1][w];
    }
    const float scq = 1.0f / fmaxf(sqrtf((float) tq), a.eps), sck = 1.0f / fmaxf(sqrtf((float) tk), a.eps);
    a.qn[((int64_t) t * a.H_k + hk) * GS + i] = q * scq;
    a.kn[((int64_t) t * a.H_k + hk) * GS + i] = k * sck;
}

// The recurrence.  Workgroup (value head hv, rows j0 .. j0 + 7 of its state
// M = S^T): 32 lanes per row, each holding 4 of its 128 columns in registers
// for all tokens.  Per token, as ggml: M *= exp(g); delta_j = (v_j - M_j . k) beta;
// M_j += delta_j k; o_j = (M_j . q) / sqrt(S).  Rows are independent, so the
// 16 row blocks of a head run in parallel; the next token's q, k, v, beta, g
// are loaded while the current one is applied.
__global__ void __launch_bounds__(256) k_gdn_delta(GdnArgs a) {
    const int hv = blockIdx.x, tid = threadIdx.x, r = tid >> 5, l = tid & 31;
    const int j = blockIdx.y * GJB + r, hk = hv % a.H_k;
    const int64_t vbase = 2 * (int64_t) a.H_k * GS + (int64_t) hv * GS + j;
    float* st = a.state + ((int64_t) hv * GS + j) * GS + 4 * l;
    float4 m = *(const float4*) st;
    const float scale = 1.0f / sqrtf((float) GS);
    auto ld = [&](int t, float4& q, float4& k, float& v, float& beta, float& g) __attribute__((always_inline)) {
        q = *(const float4*) (a.qn + ((int64_t) t * a.H_k + hk) * GS + 4 * l);
        k = *(const float4*) (a.kn + ((int64_t) t * a.H_k + hk) * GS + 4 * l);
        v = a.conv[(int64_t) t * a.conv_ch + vbase];
        beta = a.bg[((int64_t) t * a.H_v + hv) * 2];
        g = a.bg[((int64_t) t * a.H_v + hv) * 2 + 1];
    };
    float4 q, k, qn, kn;
    float v, beta, g, vn = 0.0f, bn = 0.0f, gn = 0.0f;
    ld(0, q, k, v, beta, g);
    for (int t = 0; t < a.T; ++t) {
        if (t + 1 < a.T) ld(t + 1, qn, kn, vn, bn, gn);
        const float e = expf(g);
        m.x *= e;
        m.y *= e;
        m.z *= e;
        m.w *= e;
        float dk = m.x * k.x + m.y * k.y + m.z * k.z + m.w * k.w;
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) dk += __shfl_xor(dk, off, 32);
        const float delta = (v - dk) * beta;
        m.x = __builtin_fmaf(k.x, delta, m.x);
        m.y = __builtin_fmaf(k.y, delta, m.y);
        m.z = __builtin_fmaf(k.z, delta, m.z);
        m.w = __builtin_fmaf(k.w, delta, m.w);
        float o = m.x * q.x + m.y * q.y + m.z * q.z + m.w * q.w;
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) o += __shfl_xor(o, off, 32);
        if (l == 0) a.o[((int64_t) t * a.H_v + hv) * GS + j] = o * scale;
        q = qn;
        k = kn;
        v = vn;
        beta = bn;
        g = gn;
    }
    *(float4*) st = m;
}

// Block (t, value head): rms_norm of the head's 128 outputs (double sum) times
// ssm_norm, times silu(z) of the same elements: ggml_mul(ggml_mul(rms_norm(o),
// ssm_norm), ggml_silu(z)), each product rounded as there.
__global__ void __launch_bounds__(GS) k_gdn_gate_norm(GdnArgs a) {
    const int t = blockIdx.x, hv = blockIdx.y, i = threadIdx.x;
    __shared__ double s_red[GS / 64];
    const int64_t e = ((int64_t) t * a.H_v + hv) * GS + i;
    const float x = a.o[e];
    double s = (double) (x * x);
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((i & 63) == 0) s_red[i >> 6] = s;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < GS / 64; ++w) tot += s_red[w];
    const float mean = (float) (tot / (double) GS);
    const float sc = 1.0f / sqrtf(mean + a.eps);
    const float zn = (x * sc) * a.ssm_norm[i];
    a.y[e] = zn * v_silu(a.z[e]);
}

}  // namespace

bool gdn_shape_ok(int64_t S, int64_t H_k, int64_t H_v, int64_t d_conv) {
    return S == GS && H_k > 0 && H_v > 0 && H_v % H_k == 0 && H_v <= 4096 && d_conv >= 2 && d_conv <= GDN_MAX_CONV;
}

int launch_gdn_core(const GdnArgs& a, hipStream_t stream) {
    if (!gdn_shape_ok(GS, a.H_k, a.H_v, a.d_conv) || a.T <= 0) return -2;
    hipLaunchKernelGGL(k_gdn_conv, dim3((unsigned) ((a.conv_ch + 255) / 256)), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_prep, dim3((unsigned) a.T, (unsigned) (a.H_k + 1)), dim3(GS), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_delta, dim3((unsigned) a.H_v, (unsigned) (GS / GJB)), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_gate_norm, dim3((unsigned) a.T, (unsigned) a.H_v), dim3(GS), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
