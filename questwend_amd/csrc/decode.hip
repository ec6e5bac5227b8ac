// decode.hip -- persistent whole-stack MoE FFN decode: one launch runs one
// token through every layer of a stack (the work core/runtime.cpp schedules as
// build_moe per layer inside one graph, decode() -> build_graph, 976-1100).
//
// One workgroup per CU, all co-resident (cooperative launch).  Per layer:
//   A  every WG: top-k from the layer's logits; Q8_K(x); stream its slice of the
//      selected experts' gate/up rows into LDS (and, already, its down rows);
//      gate, up, SwiGLU for its row pairs -> act
//   B  every WG: all act -> Q8_K per expert; its H/G output rows of all k experts'
//      down projections; weighted expert sum -> y rows
//   C  every WG: all y -> RMSNorm -> x of the next layer; WG e computes router
//      logit e of the next layer from its LDS copy of that router row
// Cross-WG data (act, y, logits) moves through device memory as 64-bit words
// {value, epoch}; consumers poll the words themselves, so one memory round
// trip both carries the data and signals it.  All such accesses are
// device-scope relaxed atomics; producers order their writes with a wait for
// store completion before anything that depends on them.
//
// Every float operation reproduces ggml's AVX2 CPU order (qw_rowdot.hpp,
// router/ffn semantics), so ids and outputs are bit-identical to the reference.
#include "qw_kernels.hpp"
#include "qw_rowdot.hpp"
#include "qw_sort.hpp"
#include "qw_decode.hpp"

namespace qw {

constexpr int DEC_THREADS = 512;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr long DEC_SPIN_LIMIT = 1L << 22;   // ~seconds: a stuck wait aborts the launch

struct DecodeArgs {
    const DecodeLayer* layers;
    int n_layer;
    int H, E, k, F;
    int type_down;            // Q4_K or Q6_K (gate/up are Q4_K)
    float scale, rms_eps;
    const float* x_in;        // [H]
    float* out;               // [H]   MoE output of the last layer
    float* x_out;             // [H]   RMSNorm of it (may be null)
    int32_t* ids_out;         // [n_layer][k] (may be null)
    float* w_out;             // [n_layer][k] (may be null)
    uint64_t* xa;             // [k * F]   act exchange
    uint64_t* xy;             // [H]       y exchange
    uint64_t* xl;             // [E]       logit exchange
    uint32_t epoch0;
    int32_t* status;          // bit 3: a wait timed out; bit 4: bad slot
    int32_t* abort_flag;
    // partition / LDS layout (host computed)
    int pa_per;               // row pairs per WG (ceil(k*F / G))
    int hb_per;               // down rows per WG (multiple of 4)
    uint32_t lds_rw, lds_a, lds_b, lds_xq, lds_aq, lds_x, lds_act, lds_res, lds_total;
    uint32_t rs_a;            // LDS stride of a gate/up row
    uint32_t rs_b;            // LDS stride of a down row (16-aligned)
};

__device__ __forceinline__ uint64_t ld_dev64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tagged(float v, uint32_t epoch) {
    return ((uint64_t) epoch << 32) | (uint64_t) fbits(v);
}
// The abort word holds the first epoch of a launch that gave up waiting; a
// value from an older launch is ignored, so it never needs clearing.
__device__ __forceinline__ bool aborted(const DecodeArgs& a) {
    return (uint32_t) __hip_atomic_load(a.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= a.epoch0;
}
__device__ __forceinline__ void raise_abort(const DecodeArgs& a, int bit) {
    atomicOr(a.status, bit);
    __hip_atomic_store(a.abort_flag, (int32_t) a.epoch0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls n tagged words (this thread's share: idx = tid + j * DEC_THREADS) until
// all carry `epoch`, storing the float payloads to dst[idx].  Loads of one
// round are independent, so a round costs one memory round trip.  Returns
// false on abort.
template <int MAXJ>
__device__ bool gather_tagged(const DecodeArgs& a, const uint64_t* src, int n, uint32_t epoch, float* dst) {
    const int tid = threadIdx.x;
    bool ok = true;
    for (int base = 0; base < n && ok; base += MAXJ * DEC_THREADS) {
        uint64_t v[MAXJ];
        long spins = 0;
        do {
            ok = true;
            for (int j = 0; j < MAXJ; ++j) {
                const int idx = base + tid + j * DEC_THREADS;
                v[j] = idx < n ? ld_dev64(src + idx) : ((uint64_t) epoch << 32);
            }
            for (int j = 0; j < MAXJ; ++j) ok = ok && ((uint32_t) (v[j] >> 32) == epoch);
            if (!ok) {
                if (++spins > DEC_SPIN_LIMIT) { raise_abort(a, 8); break; }
                if ((spins & 255) == 0 && aborted(a)) break;
            }
        } while (!ok);
        for (int j = 0; j < MAXJ; ++j) {
            const int idx = base + tid + j * DEC_THREADS;
            if (idx < n) dst[idx] = bitsf((uint32_t) v[j]);
        }
    }
    return __syncthreads_or(!ok) == 0;
}

// 16-byte chunks from global to LDS (each thread a strided subset).
__device__ __forceinline__ void copy_chunks(uint32_t* lds, uint32_t lds_off, const uint8_t* g, int nchunks) {
    uint4* d = (uint4*) ((uint8_t*) lds + lds_off);
    const uint4* s = (const uint4*) g;
    for (int c = threadIdx.x; c < nchunks; c += DEC_THREADS) d[c] = s[c];
}

// Q8_K of n fp32 values in LDS (n % 256 == 0) into blocks at lds byte offset q.
// One wave per block; the reduction follows quantize_row_q8_K_ref exactly.
__device__ void quant_q8K_lds(uint32_t* lds, const float* src, int nblocks, uint32_t q) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int b = wave; b < nblocks; b += DEC_WAVES) {
        const float* x = src + b * QK_K;
        float v[4];
        for (int i = 0; i < 4; ++i) v[i] = x[4 * lane + i];
        float am = 0.0f;
        int ai = 0x7fffffff;
        for (int i = 0; i < 4; ++i) {
            const float t = __builtin_fabsf(v[i]);
            if (t > am) { am = t; ai = 4 * lane + i; }
        }
        for (int off = 32; off >= 1; off >>= 1) {
            const float om = __shfl_xor(am, off);
            const int oi = __shfl_xor(ai, off);
            if (om > am || (om == am && oi < ai)) { am = om; ai = oi; }
        }
        uint8_t* blk = (uint8_t*) lds + q + (uint32_t) b * 292u;
        if (!(am > 0.0f)) {
            *(uint32_t*) (blk + 4 + 4 * lane) = 0;
            if (lane < 16) *(int16_t*) (blk + 260 + 2 * lane) = 0;
            if (lane == 0) *(float*) blk = 0.0f;
            continue;
        }
        const float iscale = -127.f / x[ai];
        int qv[4], s = 0;
        for (int i = 0; i < 4; ++i) {
            const int t = nearest_int(iscale * v[i]);
            qv[i] = t < 127 ? t : 127;
            s += qv[i];
        }
        *(uint32_t*) (blk + 4 + 4 * lane) = (uint32_t) (qv[0] & 0xff) | ((uint32_t) (qv[1] & 0xff) << 8) |
                                            ((uint32_t) (qv[2] & 0xff) << 16) | ((uint32_t) (qv[3] & 0xff) << 24);
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if ((lane & 3) == 0) *(int16_t*) (blk + 260 + 2 * (lane >> 2)) = (int16_t) s;
        if (lane == 0) *(float*) blk = 1.0f / iscale;
    }
}

// global_load_lds_dwordx4: lane i of the wave lands at lds + off + 16 * i.
__device__ __forceinline__ void dma16(uint32_t* lds, uint32_t lds_off, const void* src) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*) ((uint8_t*) lds + lds_off), 16, 0, 0);
}
// One wave copies nch 16-byte chunks starting at the 16-byte aligned src to
// LDS at lds_off (no VGPRs held; completion via vmcnt).
__device__ __forceinline__ void dma_row(uint32_t* lds, uint32_t lds_off, const uint8_t* src, int nch, int lane) {
    for (int it = 0; it * 64 < nch; ++it)
        if (it * 64 + lane < nch) dma16(lds, lds_off + (uint32_t) it * 1024u, src + (size_t) (it * 64 + lane) * 16);
}
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int NBH, int NBF, int TYPE_DOWN>
__global__ void __launch_bounds__(DEC_THREADS) k_decode_stack(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    __shared__ int32_t s_ids[32];
    __shared__ float s_w[32];
    __shared__ int32_t s_order[512];
    __shared__ float s_p[512];
    __shared__ float s_e[512];
    __shared__ float s_gsum[64];
    __shared__ double s_red[DEC_WAVES];
    __shared__ SortRange s_stack[SORT_STACK];
    __shared__ int s_need_sort;

    const int b = blockIdx.x, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int H = a.H, E = a.E, k = a.k, F = a.F;
    const int nbH = NBH > 0 ? NBH : H / QK_K, nbF = NBF > 0 ? NBF : F / QK_K;
    const uint32_t rowA = (uint32_t) nbH * 144u;                                   // gate/up row bytes (Q4_K)
    const uint32_t rowB = (uint32_t) nbF * (TYPE_DOWN == T_Q4_K ? 144u : 210u);   // down row bytes
    float* xs = (float*) ((uint8_t*) lds + a.lds_x);       // x (fp32) of the current layer
    float* res = (float*) ((uint8_t*) lds + a.lds_res);    // per-row results, then y
    const int P = k * F;
    const int pa0 = b * a.pa_per < P ? b * a.pa_per : P;
    const int pa1 = pa0 + a.pa_per < P ? pa0 + a.pa_per : P;
    const int np = pa1 - pa0;
    const int h0 = b * a.hb_per < H ? b * a.hb_per : H;
    const int h1 = h0 + a.hb_per < H ? h0 + a.hb_per : H;
    const int nh = h1 - h0;
    const int chA = (int) (rowA / 16);

    // ---- layer 0 input and router row ----------------------------------------
    for (int i = tid; i < H; i += DEC_THREADS) xs[i] = a.x_in[i];
    if (b < E && wave == 0) dma_row(lds, a.lds_rw, (const uint8_t*) (a.layers[0].router + (size_t) b * H), H / 4, lane);
    wait_dma();
    __syncthreads();

    for (int l = 0; l < a.n_layer; ++l) {
        const DecodeLayer& L = a.layers[l];
        const uint32_t ep = a.epoch0 + (uint32_t) l;
        const uint32_t rw_cur = a.lds_rw + (uint32_t) (l & 1) * (uint32_t) H * 4u;
        // ---- router(l): logit e = b from the LDS router row ---------------------
        if (b < E && wave == 0) {
            // lanes 0..31 = the 32 fma chains of the AVX2 ggml_vec_dot_f32 (H % 32 == 0)
            const float* w = (const float*) ((uint8_t*) lds + rw_cur);
            float acc = 0.0f;
            if (lane < 32)
                for (int s = 0; s < H; s += 32) acc = __builtin_fmaf(w[s + lane], xs[s + lane], acc);
            float t = acc + __shfl_down(acc, 16, 32);   // c_l + c_{16+l}
            t = t + __shfl_down(t, 8, 32);               // s_l = (c_l + c_{16+l}) + (c_{8+l} + c_{24+l})
            t = t + __shfl_down(t, 4, 32);               // t0_l = s_l + s_{l+4}
            const float u = t + __shfl_down(t, 1, 32);
            const float logit = u + __shfl_down(u, 2, 32);   // (t0_0 + t0_1) + (t0_2 + t0_3)
            if (lane == 0) st_dev64(a.xl + b, tagged(logit, ep));
        }
        // the next layer's router row streams in behind everything else
        if (b < E && wave == 1 && l + 1 < a.n_layer)
            dma_row(lds, a.lds_rw + (uint32_t) ((l + 1) & 1) * (uint32_t) H * 4u,
                    (const uint8_t*) (a.layers[l + 1].router + (size_t) b * H), H / 4, lane);
        quant_q8K_lds(lds, xs, nbH, a.lds_xq);
        // ---- softmax and exact top-k (every WG) ----------------------------------
        if (!gather_tagged<1>(a, a.xl, E, ep, s_p)) { wait_dma(); return; }
        {
            float mx = -INFINITY;
            for (int i = lane; i < E; i += 64) mx = fmaxf(mx, s_p[i]);
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            for (int i = tid; i < E; i += DEC_THREADS) s_e[i] = v_expf(s_p[i] - mx);
            __syncthreads();
            for (int g = tid; g < E / 8; g += DEC_THREADS) s_gsum[g] = hsum8(&s_e[8 * g]);
            __syncthreads();
            double sum = 0.0;
            for (int g = 0; g < E / 8; ++g) sum += (double) s_gsum[g];
            const float inv = (float) (1.0 / sum);
            for (int i = tid; i < E; i += DEC_THREADS) s_p[i] = s_e[i] * inv;
            __syncthreads();
            if (wave == 0) {
                // k rounds of wave arg-max; a second element equal to a selected
                // value means std::sort's tie order decides -> exact replay below
                float v[8];
                for (int j = 0; j < 8; ++j) v[j] = (lane + 64 * j < E) ? s_p[lane + 64 * j] : -1.0f;
                bool tie = false;
                for (int r = 0; r < k; ++r) {
                    float m = v[0];
                    for (int j = 1; j < 8; ++j) m = fmaxf(m, v[j]);
                    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
                    int cnt = 0, sel = -1;
                    for (int j = 0; j < 8; ++j) {
                        const uint64_t msk = __ballot(v[j] == m);
                        cnt += __popcll(msk);
                        if (sel < 0 && msk) sel = 64 * j + __ffsll((unsigned long long) msk) - 1;
                    }
                    tie = tie || cnt > 1;
                    if (lane == 0) s_order[r] = sel;
                    if (lane == (sel & 63)) v[sel >> 6] = -1.0f;
                }
                if (lane == 0) s_need_sort = tie;
            }
            __syncthreads();
            if (s_need_sort) {
                if (tid == 0) {
                    for (int i = 0; i < E; ++i) s_order[i] = i;
                    libstdcxx_sort_desc(s_order, E, s_p, s_stack);
                    if (b == 0) atomicOr(a.status, 1);
                }
                __syncthreads();
            }
            if (tid == 0) {
                double s = 0.0;
                for (int i = 0; i < k; ++i) s += (double) s_p[s_order[i]];
                float wsum = (float) s;
                wsum = fmaxf(fminf(wsum, INFINITY), 6.103515625e-5f);
                for (int i = 0; i < k; ++i) {
                    float wi = s_p[s_order[i]] / wsum;
                    if (a.scale != 0.0f && a.scale != 1.0f) wi = wi * a.scale;
                    s_ids[i] = s_order[i];
                    s_w[i] = wi;
                    if (b == 0 && a.ids_out) {
                        a.ids_out[l * k + i] = s_order[i];
                        a.w_out[l * k + i] = wi;
                    }
                }
            }
            __syncthreads();
        }
        // ---- stream this WG's gate/up rows (pair p: slot p / F, row p % F) -------
        for (int r = wave; r < 2 * np; r += DEC_WAVES) {
            const int p = pa0 + (r >> 1);
            const int i = p / F, f = p % F;
            const int e = s_ids[i];
            const bool up = r & 1;
            const int32_t* so = up ? L.slot_up : L.slot_gate;
            int64_t mat = so ? so[e] : e;
            if (mat < 0 || mat >= (up ? L.n_slots_up : L.n_slots_gate)) {
                if (lane == 0) atomicOr(a.status, 16);
                mat = 0;
            }
            const uint8_t* src = (up ? L.up : L.gate) + (size_t) mat * (up ? L.up_nb2 : L.gate_nb2) +
                                 (size_t) f * (up ? L.up_nb1 : L.gate_nb1);
            dma_row(lds, a.lds_a + (uint32_t) r * a.rs_a, src, chA, lane);
        }
        wait_dma();
        __syncthreads();
        // ---- and the down rows, which land while A computes and act is exchanged -
        for (int r = wave; r < k * nh; r += DEC_WAVES) {
            const int i = r / nh, hh = r % nh;
            const int e = s_ids[i];
            int64_t mat = L.slot_down ? L.slot_down[e] : e;
            if (mat < 0 || mat >= L.n_slots_down) {
                if (lane == 0) atomicOr(a.status, 16);
                mat = 0;
            }
            const uint8_t* rowp = L.down + (size_t) mat * L.down_nb2 + (size_t) (h0 + hh) * L.down_nb1;
            const uint8_t* base = (const uint8_t*) ((uintptr_t) rowp & ~(uintptr_t) 15);
            dma_row(lds, a.lds_b + (uint32_t) r * a.rs_b, base, (int) ((rowp + rowB - base + 15) / 16), lane);
        }
        // ---- A: gate / up rows, SwiGLU ---------------------------------------------
        for (int r0 = 0; r0 < np * 2; r0 += DEC_WAVES * 8) {
            const int r = r0 + wave * 8 + (lane >> 3);
            const int rr = r < np * 2 ? r : 0;
            float v;
            if constexpr (NBH > 0) v = row_dot_q4k_a<NBH>(lds, a.lds_a + (uint32_t) rr * a.rs_a, a.lds_xq, lane & 7);
            else v = row_dot_lds<T_Q4_K>(lds, a.lds_a + (uint32_t) rr * a.rs_a, a.lds_xq, nbH, lane & 7);
            if (r < np * 2 && (lane & 7) == 0) res[r] = v;
        }
        __syncthreads();
        for (int j = tid; j < np; j += DEC_THREADS) {
            const float act = v_silu(res[2 * j]) * res[2 * j + 1];
            st_dev64(a.xa + pa0 + j, tagged(act, ep));
        }
        // ---- B: all act -> Q8_K per slot; down rows; weighted sum ------------------
        float* actf = (float*) ((uint8_t*) lds + a.lds_act);
        if (!gather_tagged<12>(a, a.xa, P, ep, actf)) { wait_dma(); return; }
        quant_q8K_lds(lds, actf, k * nbF, a.lds_aq);
        wait_dma();
        __syncthreads();
        for (int r0 = 0; r0 < k * nh; r0 += DEC_WAVES * 8) {
            const int r = r0 + wave * 8 + (lane >> 3);
            const int rr = r < k * nh ? r : 0;
            const int i = rr / nh, hh = rr % nh;
            const int e = s_ids[i];
            int64_t mat = L.slot_down ? L.slot_down[e] : e;
            if (mat < 0 || mat >= L.n_slots_down) mat = 0;
            const uint8_t* rowp = L.down + (size_t) mat * L.down_nb2 + (size_t) (h0 + hh) * L.down_nb1;
            const uint32_t wb = a.lds_b + (uint32_t) rr * a.rs_b + (uint32_t) ((uintptr_t) rowp & 15);
            const uint32_t ab = a.lds_aq + (uint32_t) (i * nbF) * 292u;
            float v;
            if constexpr (TYPE_DOWN == T_Q4_K && NBF > 0) {
                v = (wb & 3) == 0 ? row_dot_q4k_a<NBF>(lds, wb, ab, lane & 7)
                                  : row_dot_lds<TYPE_DOWN>(lds, wb, ab, nbF, lane & 7);
            } else {
                v = row_dot_lds<TYPE_DOWN>(lds, wb, ab, nbF, lane & 7);
            }
            if (r < k * nh && (lane & 7) == 0) res[r] = v;
        }
        __syncthreads();
        for (int hh = tid; hh < nh; hh += DEC_THREADS) {
            // ggml_vec_dot_f32(k, experts^T row, w): k < 32 -> scalar tail: groups of
            // four as mul + add, the remainder fused
            float sumf = 0.0f;
            const int nv = k & ~3;
            for (int i = 0; i < k; ++i) {
                const float d = res[i * nh + hh];
                sumf = (i < nv) ? sumf + d * s_w[i] : __builtin_fmaf(d, s_w[i], sumf);
            }
            st_dev64(a.xy + h0 + hh, tagged(sumf, ep));
        }
        // ---- C: all y -> RMSNorm -> x of the next layer ----------------------------
        float* ys = res;   // reused: every thread must be done with the down results
        __syncthreads();
        if (!gather_tagged<4>(a, a.xy, H, ep, ys)) { wait_dma(); return; }
        {
            double s = 0.0;
            for (int i = tid; i < H; i += DEC_THREADS) {
                const float v = ys[i];
                s += (double) (v * v);
            }
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) s_red[wave] = s;
            __syncthreads();
            double tot = 0.0;
            for (int w = 0; w < DEC_WAVES; ++w) tot += s_red[w];
            const float mean = (float) (tot / (double) H);
            const float sc = 1.0f / sqrtf(mean + a.rms_eps);
            for (int i = tid; i < H; i += DEC_THREADS) xs[i] = ys[i] * sc;
            if (l + 1 == a.n_layer && b == 0) {
                for (int i = tid; i < H; i += DEC_THREADS) {
                    a.out[i] = ys[i];
                    if (a.x_out) a.x_out[i] = xs[i];
                }
            }
            __syncthreads();
        }
    }
}

int launch_decode_stack(const DecodeStackDesc& d, const float* x_in, float* out, float* x_out, int32_t* ids_out,
                        float* w_out, uint32_t epoch0, hipStream_t stream) {
    DecodeArgs a{};
    a.layers = d.layers_dev;
    a.n_layer = d.n_layer;
    a.H = (int) d.H;
    a.E = (int) d.E;
    a.k = (int) d.k;
    a.F = (int) d.F;
    a.type_down = d.type_down;
    a.scale = d.scale;
    a.rms_eps = d.rms_eps;
    a.x_in = x_in;
    a.out = out;
    a.x_out = x_out;
    a.ids_out = ids_out;
    a.w_out = w_out;
    a.xa = d.xa;
    a.xy = d.xy;
    a.xl = d.xl;
    a.epoch0 = epoch0;
    a.status = d.status;
    a.abort_flag = d.abort_flag;
    a.pa_per = d.pa_per;
    a.hb_per = d.hb_per;
    a.lds_rw = d.lds_rw;
    a.lds_a = d.lds_a;
    a.lds_b = d.lds_b;
    a.lds_xq = d.lds_xq;
    a.lds_aq = d.lds_aq;
    a.lds_x = d.lds_x;
    a.lds_act = d.lds_act;
    a.lds_res = d.lds_res;
    a.lds_total = d.lds_total;
    a.rs_a = d.rs_a;
    a.rs_b = d.rs_b;
    void* args[] = {&a};
    const void* fn;
    if (d.type_down == T_Q4_K && d.H == 2048 && d.F == 768) fn = (const void*) k_decode_stack<8, 3, T_Q4_K>;
    else if (d.type_down == T_Q6_K) fn = (const void*) k_decode_stack<0, 0, T_Q6_K>;
    else fn = (const void*) k_decode_stack<0, 0, T_Q4_K>;
    hipError_t e = hipLaunchCooperativeKernel(fn, dim3((unsigned) d.grid), dim3(DEC_THREADS), args, d.lds_total, stream);
    return e == hipSuccess ? 0 : -3;
}

int plan_decode_stack(DecodeStackDesc& d, int grid) {
    if (d.H % 256 || d.F % 256 || d.E % 8 || d.E > 512 || d.k < 1 || d.k > 32 || d.k > d.E) return -2;
    if (d.type_down != T_Q4_K && d.type_down != T_Q6_K) return -2;
    d.grid = grid;
    const int P = (int) (d.k * d.F);
    d.pa_per = (P + grid - 1) / grid;
    d.hb_per = (int) (((d.H + grid - 1) / grid + 3) / 4 * 4);
    if (d.E > grid) return -2;                        // one router row per WG
    const uint32_t rowA = (uint32_t) (d.H / 256) * 144u;
    const uint32_t rowB = (uint32_t) (d.F / 256) * (d.type_down == T_Q4_K ? 144u : 210u);
    d.rs_a = rowA + 32;                               // stride = 8 (mod 32) dwords for 144-byte rows
    d.rs_b = ((rowB + 15) / 16 + 1) * 16;
    uint32_t off = 0;
    auto take = [&](uint32_t bytes) { const uint32_t o = off; off += (bytes + 15) / 16 * 16; return o; };
    d.lds_rw = take((uint32_t) (2 * d.H * 4));
    d.lds_a = take((uint32_t) (2 * d.pa_per) * d.rs_a);
    d.lds_b = take((uint32_t) (d.k * d.hb_per) * d.rs_b);
    d.lds_xq = take((uint32_t) (d.H / 256) * 292u + 16);
    d.lds_aq = take((uint32_t) (d.k * d.F / 256) * 292u + 16);
    d.lds_x = take((uint32_t) d.H * 4u);
    // act (fp32, k*F) is gathered after the gate/up rows are consumed: reuse their space if it fits
    const uint32_t act_bytes = (uint32_t) (d.k * d.F) * 4u;
    d.lds_act = act_bytes <= (uint32_t) (2 * d.pa_per) * d.rs_a ? d.lds_a : take(act_bytes);
    d.lds_res = take((uint32_t) std::max<int64_t>(d.H, std::max<int64_t>(2 * d.pa_per, d.k * d.hb_per)) * 4u);
    d.lds_total = off;
    if (d.lds_total > 160 * 1024 - 8 * 1024) return -2;   // static shared arrays need ~6 KB
    return 0;
}

}  // namespace qw
