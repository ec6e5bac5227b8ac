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
constexpr int GJB = 32;        // state rows j per workgroup of the recurrence (8 lanes per row)

// Thread (channel c, token t): the d_conv-tap window over [conv_state | qkv
// rows] ending at token t, then SiLU.  The inputs x_0 .. x_{d_conv-2} are the
// state, x_{d_conv-1+t} = qkv[t][c].
__global__ void __launch_bounds__(256) k_gdn_conv(GdnArgs a) {
    const int64_t c = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y, dc = a.d_conv;
    if (c >= a.conv_ch) return;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < GDN_MAX_CONV; ++j)
        if (j < dc) {
            const int xi = t + j;   // window element j is x_{t + j}
            const float x = xi < dc - 1 ? a.conv_state[c * (dc - 1) + xi]
                                        : a.qkv[(int64_t) (xi - (dc - 1)) * a.conv_ch + c];
            s = __builtin_fmaf(x, a.conv1d[c * dc + j], s);
        }
    a.conv[(int64_t) t * a.conv_ch + c] = v_silu(s);
}

// The conv state after the call: x_T .. x_{T+d_conv-2}, one thread per channel
// (after k_gdn_conv, which reads the old state).
__global__ void __launch_bounds__(256) k_gdn_conv_state(GdnArgs a) {
    const int64_t c = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (c >= a.conv_ch) return;
    const int dc = a.d_conv, T = a.T;
    float nw[GDN_MAX_CONV];
#pragma unroll
    for (int j = 0; j + 1 < GDN_MAX_CONV; ++j)
        if (j < dc - 1) {
            const int xi = T + j;
            nw[j] = xi < dc - 1 ? a.conv_state[c * (dc - 1) + xi] : a.qkv[(int64_t) (xi - (dc - 1)) * a.conv_ch + c];
        }
#pragma unroll
    for (int j = 0; j + 1 < GDN_MAX_CONV; ++j)
        if (j < dc - 1) a.conv_state[c * (dc - 1) + j] = nw[j];
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

// The recurrence.  Workgroup (value head hv, rows j0 .. j0 + 31 of its state
// M = S^T): 8 lanes per row, each holding 16 of its 128 columns in registers
// for all tokens.  Per token, as ggml: M *= exp(g); delta_j = (v_j - M_j . k) beta;
// M_j += delta_j k; o_j = (M_j . q) / sqrt(S).  A row's dots are reduced over
// its 8 lanes by DPP (quad xor 1, xor 2, half-row mirror).  Rows are
// independent, so the 4 row blocks of a head run in parallel.  Tokens go in
// blocks of GTB: the block's q, k (its key head), v (the workgroup's rows), beta
// and g sit in LDS, and the next block's are loaded into registers while the
// current block is applied, so the chain over the tokens waits on LDS, not on
// a memory round trip per token.
constexpr int GTB = 32;   // tokens per staged block
__global__ void __launch_bounds__(256) k_gdn_delta(GdnArgs a) {
    const int hv = blockIdx.x, tid = threadIdx.x, r = tid >> 3, l = tid & 7;
    const int j0 = blockIdx.y * GJB, j = j0 + r, hk = hv % a.H_k;
    __shared__ __align__(16) float s_q[GTB][GS];
    __shared__ __align__(16) float s_k[GTB][GS];
    __shared__ float s_v[GTB][GJB];
    __shared__ float s_b[GTB], s_g[GTB];
    float* st = a.state + ((int64_t) hv * GS + j) * GS + 16 * l;
    float4 m0 = *(const float4*) st, m1 = *(const float4*) (st + 4), m2 = *(const float4*) (st + 8),
           m3 = *(const float4*) (st + 12);
    const float scale = 1.0f / sqrtf((float) GS);
    const int64_t vbase = 2 * (int64_t) a.H_k * GS + (int64_t) hv * GS + j0;
    // this thread's share of a block: float4 f = tid + 256 u of q and of k
    // (token f / 32, columns 4 (f % 32) ..), v of (token f / 32, row f % 32) for
    // f = tid + 256 u, and beta or g (tid < 2 GTB); named registers, not
    // arrays, so that nothing lands in scratch
    static_assert(GTB * GS / 4 == 4 * 256 && GTB * GJB == 4 * 256, "four float4 of q, k and four v per thread");
    float4 rq0, rq1, rq2, rq3, rk0, rk1, rk2, rk3;
    float rv0, rv1, rv2, rv3, rbg = 0.0f;
    const int64_t qcol = 4 * (tid % (GS / 4));
    auto tok = [&](int t) { return (int64_t) (t < a.T ? t : a.T - 1); };
#define GDN_LOAD(tb_)                                                                                          \
    do {                                                                                                     \
        const int t0_ = (tb_) + tid / (GS / 4);                                                              \
        rq0 = *(const float4*) (a.qn + (tok(t0_) * a.H_k + hk) * GS + qcol);                                 \
        rq1 = *(const float4*) (a.qn + (tok(t0_ + 8) * a.H_k + hk) * GS + qcol);                             \
        rq2 = *(const float4*) (a.qn + (tok(t0_ + 16) * a.H_k + hk) * GS + qcol);                            \
        rq3 = *(const float4*) (a.qn + (tok(t0_ + 24) * a.H_k + hk) * GS + qcol);                            \
        rk0 = *(const float4*) (a.kn + (tok(t0_) * a.H_k + hk) * GS + qcol);                                 \
        rk1 = *(const float4*) (a.kn + (tok(t0_ + 8) * a.H_k + hk) * GS + qcol);                             \
        rk2 = *(const float4*) (a.kn + (tok(t0_ + 16) * a.H_k + hk) * GS + qcol);                            \
        rk3 = *(const float4*) (a.kn + (tok(t0_ + 24) * a.H_k + hk) * GS + qcol);                            \
        const int tv_ = (tb_) + tid / GJB;                                                                   \
        rv0 = a.conv[tok(tv_) * a.conv_ch + vbase + tid % GJB];                                              \
        rv1 = a.conv[tok(tv_ + 8) * a.conv_ch + vbase + tid % GJB];                                          \
        rv2 = a.conv[tok(tv_ + 16) * a.conv_ch + vbase + tid % GJB];                                         \
        rv3 = a.conv[tok(tv_ + 24) * a.conv_ch + vbase + tid % GJB];                                         \
        if (tid < 2 * GTB) rbg = a.bg[(tok((tb_) + (tid >> 1)) * a.H_v + hv) * 2 + (tid & 1)];               \
    } while (0)
    auto red8 = [](float x) __attribute__((always_inline)) {
        x = x + dpp_f<DPP_XOR1>(x);
        x = x + dpp_f<DPP_XOR2>(x);
        return x + dpp_f<DPP_HALF_MIRROR>(x);
    };
    GDN_LOAD(0);
    for (int tb = 0; tb < a.T; tb += GTB) {
        __syncthreads();   // the previous block is consumed
        {
            const int tq = tid / (GS / 4), tv = tid / GJB;
            *(float4*) &s_q[tq][qcol] = rq0;
            *(float4*) &s_q[tq + 8][qcol] = rq1;
            *(float4*) &s_q[tq + 16][qcol] = rq2;
            *(float4*) &s_q[tq + 24][qcol] = rq3;
            *(float4*) &s_k[tq][qcol] = rk0;
            *(float4*) &s_k[tq + 8][qcol] = rk1;
            *(float4*) &s_k[tq + 16][qcol] = rk2;
            *(float4*) &s_k[tq + 24][qcol] = rk3;
            s_v[tv][tid % GJB] = rv0;
            s_v[tv + 8][tid % GJB] = rv1;
            s_v[tv + 16][tid % GJB] = rv2;
            s_v[tv + 24][tid % GJB] = rv3;
            if (tid < 2 * GTB) {
                if (tid & 1) s_g[tid >> 1] = rbg;
                else s_b[tid >> 1] = rbg;
            }
        }
        __syncthreads();
        if (tb + GTB < a.T) GDN_LOAD(tb + GTB);
        const int nt = a.T - tb < GTB ? a.T - tb : GTB;
        for (int tt = 0; tt < nt; ++tt) {
            const float e = expf(s_g[tt]);
            const float* qp = &s_q[tt][16 * l];
            const float* kp = &s_k[tt][16 * l];
            const float4 q0 = *(const float4*) qp, q1 = *(const float4*) (qp + 4), q2 = *(const float4*) (qp + 8),
                         q3 = *(const float4*) (qp + 12);
            const float4 k0 = *(const float4*) kp, k1 = *(const float4*) (kp + 4), k2 = *(const float4*) (kp + 8),
                         k3 = *(const float4*) (kp + 12);
            auto decay_dot = [&](float4& mm, const float4& kk, float& d0, float& d1) __attribute__((always_inline)) {
                mm.x *= e;
                mm.y *= e;
                mm.z *= e;
                mm.w *= e;
                d0 = __builtin_fmaf(mm.x, kk.x, d0);
                d1 = __builtin_fmaf(mm.y, kk.y, d1);
                d0 = __builtin_fmaf(mm.z, kk.z, d0);
                d1 = __builtin_fmaf(mm.w, kk.w, d1);
            };
            float d0 = 0.0f, d1 = 0.0f;
            decay_dot(m0, k0, d0, d1);
            decay_dot(m1, k1, d0, d1);
            decay_dot(m2, k2, d0, d1);
            decay_dot(m3, k3, d0, d1);
            const float delta = (s_v[tt][r] - red8(d0 + d1)) * s_b[tt];
            auto upd_dot = [&](float4& mm, const float4& kk, const float4& qq, float& o0, float& o1)
                __attribute__((always_inline)) {
                mm.x = __builtin_fmaf(kk.x, delta, mm.x);
                mm.y = __builtin_fmaf(kk.y, delta, mm.y);
                mm.z = __builtin_fmaf(kk.z, delta, mm.z);
                mm.w = __builtin_fmaf(kk.w, delta, mm.w);
                o0 = __builtin_fmaf(mm.x, qq.x, o0);
                o1 = __builtin_fmaf(mm.y, qq.y, o1);
                o0 = __builtin_fmaf(mm.z, qq.z, o0);
                o1 = __builtin_fmaf(mm.w, qq.w, o1);
            };
            float o0 = 0.0f, o1 = 0.0f;
            upd_dot(m0, k0, q0, o0, o1);
            upd_dot(m1, k1, q1, o0, o1);
            upd_dot(m2, k2, q2, o0, o1);
            upd_dot(m3, k3, q3, o0, o1);
            const float o = red8(o0 + o1);
            if (l == 0) a.o[((int64_t) (tb + tt) * a.H_v + hv) * GS + j] = o * scale;
        }
    }
#undef GDN_LOAD
    *(float4*) st = m0;
    *(float4*) (st + 4) = m1;
    *(float4*) (st + 8) = m2;
    *(float4*) (st + 12) = m3;
}

// Grouping that gives every token its own bin (all bins the one matrix, through
// the slot rows): the small projections (ssm_beta, ssm_alpha: H_v rows) then
// spread over T workgroups of the GEMV instead of one.
__global__ void k_gdn_group_tokens(int32_t* rows, int32_t* active, int32_t* active_off, int32_t* n_active,
                                   int32_t* slot, int64_t T) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < T) {
        rows[2 * i] = (int32_t) i;
        rows[2 * i + 1] = (int32_t) i;
        active[i] = (int32_t) i;
        active_off[i] = (int32_t) i;
        slot[i] = 0;
    }
    if (i == 0) {
        active_off[T] = (int32_t) T;
        *n_active = (int32_t) T;
    }
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
    hipLaunchKernelGGL(k_gdn_conv, dim3((unsigned) ((a.conv_ch + 255) / 256), (unsigned) a.T), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_conv_state, dim3((unsigned) ((a.conv_ch + 255) / 256)), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_prep, dim3((unsigned) a.T, (unsigned) (a.H_k + 1)), dim3(GS), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_delta, dim3((unsigned) a.H_v, (unsigned) (GS / GJB)), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(k_gdn_gate_norm, dim3((unsigned) a.T, (unsigned) a.H_v), dim3(GS), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_gdn_group_tokens(int32_t* rows, int32_t* active, int32_t* active_off, int32_t* n_active, int32_t* slot,
                            int64_t T, hipStream_t stream) {
    if (T <= 0) return -2;
    hipLaunchKernelGGL(k_gdn_group_tokens, dim3((unsigned) ((T + 255) / 256)), dim3(256), 0, stream, rows, active,
                       active_off, n_active, slot, T);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
