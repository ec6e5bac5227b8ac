// decode.hip -- persistent whole-stack MoE FFN decode: one launch runs one
// token through every layer of a stack (the work core/runtime.cpp schedules as
// build_moe per layer inside one graph, decode() -> build_graph, 976-1100).
//
// One workgroup per CU, all co-resident (the LDS footprint admits one per CU).
// Per layer:
//   top-k  every WG: softmax + exact top-k from the layer's E logits
//   A      every WG: Q8_K(x); its slice of the selected experts' gate/up row
//          pairs (loaded to LDS) -> gate, up, SwiGLU -> act words
//   B      every WG: all act -> Q8_K per expert; its H/G output rows of all k
//          experts' down projections (loads issued once A has computed, held
//          in registers while act is exchanged); weighted expert sum -> y words
//   C      every WG: all y -> RMSNorm -> x of the next layer; WG e computes
//          router logit e of the next layer from its LDS copy of that row
// Cross-WG data (act, y, logits) moves through device memory as 64-bit words
// {value, epoch}; consumers poll the words themselves, so one memory round
// trip both carries the data and signals it.  Those accesses are device-scope
// relaxed atomics.  Inside a WG all sharing goes through LDS, so the barriers
// order LDS traffic only and never wait for global stores to be acknowledged.
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
constexpr long DEC_SPIN_LIMIT = 1L << 22;   // ~seconds: a stuck wait abandons the launch
constexpr int MAXJ_A = 8;                    // 16-byte gate/up chunks per thread per round
constexpr int MAXJ_B = 4;                    // 16-byte down chunks held per thread
constexpr int TOPK_TPV = 4;                  // lanes ranking one logit
constexpr int LAYER_WORDS = sizeof(DecodeLayer) / 8;
static_assert(sizeof(DecodeLayer) % 8 == 0, "layer descriptors are copied as 64-bit words");

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
    uint32_t lds_rw, lds_a, lds_b, lds_xq, lds_aq, lds_x, lds_act, lds_res, lds_y, lds_total;
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
// all carry `epoch`, storing the float payloads to dst[idx] (LDS).  Loads of one
// round are independent, so a round costs one memory round trip.  A thread
// that gives up sets *fail (LDS); the caller reads it after its next barrier.
template <int MAXJ>
__device__ void gather_tagged(const DecodeArgs& a, const uint64_t* src, int n, uint32_t epoch, float* dst,
                              int* fail) {
    const int tid = threadIdx.x;
    for (int base = 0; base < n; base += MAXJ * DEC_THREADS) {
        uint64_t v[MAXJ];
        long spins = 0;
        bool ok;
        do {
            ok = true;
#pragma unroll
            for (int j = 0; j < MAXJ; ++j) v[j] = ld_dev64(src + min(base + tid + j * DEC_THREADS, n - 1));
#pragma unroll
            for (int j = 0; j < MAXJ; ++j)
                ok = ok && (base + tid + j * DEC_THREADS >= n || (uint32_t) (v[j] >> 32) == epoch);
            if (!ok) {
                if (++spins > DEC_SPIN_LIMIT) { raise_abort(a, 8); break; }
                if ((spins & 255) == 0 && aborted(a)) break;
            }
        } while (!ok);
        if (!ok) {
            *fail = 1;
            return;
        }
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int idx = base + tid + j * DEC_THREADS;
            if (idx < n) dst[idx] = bitsf((uint32_t) v[j]);
        }
    }
}

// Q8_K (quantize_row_q8_K_ref, ggml-quants.c) of nblocks x 256 fp32 values in
// LDS into blocks at LDS byte offset q.  Sixteen lanes (one DPP row) per block,
// sixteen consecutive values per lane: the first-index max |x| is a four-step
// row reduction and each lane's values form exactly one bsums group.
__device__ void quant_q8K_lds16(uint32_t* lds, const float* src, int nblocks, uint32_t q) {
    const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
    for (int b = grp; b < nblocks; b += DEC_THREADS / 16) {
        const float* x = src + b * QK_K + 16 * l;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 t = *(const float4*) (x + i);
            v[i] = t.x;
            v[i + 1] = t.y;
            v[i + 2] = t.z;
            v[i + 3] = t.w;
        }
        float am = 0.0f;
        int ai = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float t = __builtin_fabsf(v[i]);
            if (t > am) { am = t; ai = 16 * l + i; }
        }
#define QW_AMAX_STEP(C)                                             \
    {                                                               \
        const float om = dpp_f<C>(am);                              \
        const int oi = dpp_i<C>(ai);                                \
        if (om > am || (om == am && oi < ai)) { am = om; ai = oi; } \
    }
        QW_AMAX_STEP(DPP_XOR1)
        QW_AMAX_STEP(DPP_XOR2)
        QW_AMAX_STEP(DPP_HALF_MIRROR)
        QW_AMAX_STEP(DPP_MIRROR)
#undef QW_AMAX_STEP
        uint8_t* blk = (uint8_t*) lds + q + (uint32_t) b * 292u;
        uint32_t* qw = (uint32_t*) (blk + 4 + 16 * l);
        if (!(am > 0.0f)) {
            qw[0] = qw[1] = qw[2] = qw[3] = 0;
            *(int16_t*) (blk + 260 + 2 * l) = 0;
            if (l == 0) *(float*) blk = 0.0f;
            continue;
        }
        const float iscale = -127.f / src[b * QK_K + ai];
        int s = 0;
        uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int t = nearest_int(iscale * v[i]);
            t = t < 127 ? t : 127;
            s += t;
            words[i >> 2] |= (uint32_t) (t & 0xff) << (8 * (i & 3));
        }
        qw[0] = words[0];
        qw[1] = words[1];
        qw[2] = words[2];
        qw[3] = words[3];
        *(int16_t*) (blk + 260 + 2 * l) = (int16_t) s;
        if (l == 0) *(float*) blk = 1.0f / iscale;
    }
}

// 16-byte global loads through the global address space (a generic pointer
// would become a flat load, which also occupies the LDS counter).
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
__device__ __forceinline__ u32x4 ldg16(const void* p) { return *(g_u32x4*) p; }
// After a gather the polls were this thread's newest loads and have returned,
// so every older load has too.  Saying so (at a point every thread reaches)
// keeps the compiler's per-register load tracking from carrying loads whose use
// was conditional into later code, where it would wait for every load since.
__device__ __forceinline__ void loads_returned() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)
__device__ __forceinline__ uint64_t ldg_u64(const uint64_t* p) {
    return *(const __attribute__((address_space(1))) uint64_t*) p;
}
__device__ __forceinline__ int32_t ldg_i32(const int32_t* p) {
    return *(const __attribute__((address_space(1))) int32_t*) p;
}
__device__ __forceinline__ void sts16(uint32_t* lds, uint32_t byte_off, u32x4 v) {
    *(u32x4*) ((uint8_t*) lds + byte_off) = v;
}

// 16-byte chunk ch of a down row starting at rowp (any alignment), counted
// from the row's 16-aligned base.  Past the row's end it returns the row's last
// chunk (the load stays where the row is) and sets ok = false.  Loads in this
// kernel are unconditional with clamped addresses: a load inside a divergent
// branch makes the compiler wait for it at the join, one load at a time.
__device__ __forceinline__ const u32x4* down_chunk(const uint8_t* rowp, uint32_t rowB, int ch, bool& ok) {
    const uint8_t* base = (const uint8_t*) ((uintptr_t) rowp & ~(uintptr_t) 15);
    const int last = (int) ((uint32_t) (rowp + rowB - base - 1) / 16u);
    ok = ch <= last;
    return (const u32x4*) base + (ok ? ch : last);
}

template <int NBH, int NBF, int TYPE_DOWN>
__global__ void __launch_bounds__(DEC_THREADS) k_decode_stack(DecodeArgs a) {
    extern __shared__ uint32_t lds[];
    __shared__ int32_t s_ids[32];
    __shared__ float s_w[32];
    __shared__ int32_t s_order[512];
    __shared__ __align__(16) float s_p[512];
    __shared__ float s_e[512];
    __shared__ float s_gsum[64];
    __shared__ double s_red[DEC_WAVES];
    __shared__ const uint8_t* s_rowA[96];
    __shared__ const uint8_t* s_rowB[256];
    __shared__ SortRange s_stack[SORT_STACK];
    __shared__ int32_t s_spec[32];
    __shared__ uint64_t s_L[2][LAYER_WORDS];   // descriptors of layers l (slot l & 1) and l + 1
    __shared__ int s_need_sort, s_wflag;
    __shared__ int s_bad;
    __shared__ int s_reload;
    __shared__ int s_fail;

    const int b = blockIdx.x, tid0 = threadIdx.x;
    const int H = a.H, E = a.E, k = a.k, F = a.F;
    const int nbH = NBH > 0 ? NBH : H / QK_K, nbF = NBF > 0 ? NBF : F / QK_K;
    const int chA = 9 * nbH;                                                       // 144-byte blocks / 16
    const uint32_t rowB = (uint32_t) nbF * (TYPE_DOWN == T_Q4_K ? 144u : 210u);   // down row bytes
    const int chB = (int) ((rowB + 30) / 16);                                     // incl. misalignment
    float* xs = (float*) ((uint8_t*) lds + a.lds_x);       // x (fp32) of the current layer
    float* res = (float*) ((uint8_t*) lds + a.lds_res);    // per-row dot results
    float* ys = (float*) ((uint8_t*) lds + a.lds_y);       // gathered y
    float* actf = (float*) ((uint8_t*) lds + a.lds_act);   // gathered act
    const int P = k * F;
    const int pa0 = b * a.pa_per < P ? b * a.pa_per : P;
    const int pa1 = pa0 + a.pa_per < P ? pa0 + a.pa_per : P;
    const int np = pa1 - pa0;
    const int h0 = b * a.hb_per < H ? b * a.hb_per : H;
    const int h1 = h0 + a.hb_per < H ? h0 + a.hb_per : H;
    const int nh = h1 - h0;
    const int nA = 2 * np * chA;            // gate/up chunks of this WG
    const int nB = k * nh * chB;            // down chunks (upper bound)
    const bool b_fits = nB <= MAXJ_B * DEC_THREADS;

    // ---- layer 0 input and router row ----------------------------------------
    if (tid0 == 0) s_fail = 0;
    if (tid0 < 32) s_spec[tid0] = 0;
    if (tid0 < 2 * LAYER_WORDS && tid0 / LAYER_WORDS < a.n_layer)
        s_L[tid0 / LAYER_WORDS][tid0 % LAYER_WORDS] = ldg_u64((const uint64_t*) a.layers + tid0);
    for (int i = tid0; i < H; i += DEC_THREADS) xs[i] = a.x_in[i];
    if (b < E)
        for (int c = tid0; c < H / 4; c += DEC_THREADS)
            sts16(lds, a.lds_rw + 16u * c, ldg16(a.layers[0].router + (size_t) b * H + 4 * c));
    lds_barrier();
    loads_returned();   // (each was stored to LDS above)

    for (int l = 0; l < a.n_layer; ++l) {
        const DecodeLayer& L = *(const DecodeLayer*) s_L[l & 1];
        const uint32_t ep = a.epoch0 + (uint32_t) l;
        const int tid = opaque(tid0);   // per-thread addresses are rebuilt every layer
        const int wave = tid >> 6, lane = tid & 63;
        // ---- router(l): logit e = b from the LDS router row ---------------------
        if (b < E && wave == 0) {
            // lanes 0..31 = the 32 fma chains of the AVX2 ggml_vec_dot_f32 (H % 32 == 0)
            const float* w = (const float*) ((uint8_t*) lds + a.lds_rw + (uint32_t) (l & 1) * (uint32_t) H * 4u);
            float acc = 0.0f;
            if (lane < 32) {
                // the chain is serial; its LDS reads are not (unrolled so they are in flight together)
                const int Hc = NBH > 0 ? NBH * QK_K : H;
                for (int s0 = 0; s0 < Hc; s0 += 16 * 32) {
                    float wv[16], xv[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        const int s = min(s0 + 32 * u, Hc - 32);   // (past Hc: never used)
                        wv[u] = w[s + lane];
                        xv[u] = xs[s + lane];
                    }
#pragma unroll
                    for (int u = 0; u < 16; ++u)
                        if (s0 + 32 * u < Hc) acc = __builtin_fmaf(wv[u], xv[u], acc);
                }
            }
            float t = acc + __shfl_down(acc, 16, 32);   // c_l + c_{16+l}
            t = t + __shfl_down(t, 8, 32);               // s_l = (c_l + c_{16+l}) + (c_{8+l} + c_{24+l})
            t = t + __shfl_down(t, 4, 32);               // t0_l = s_l + s_{l+4}
            const float u = t + __shfl_down(t, 1, 32);
            const float logit = u + __shfl_down(u, 2, 32);   // (t0_0 + t0_1) + (t0_2 + t0_3)
            if (lane == 0) st_dev64(a.xl + b, tagged(logit, ep));
        }
        quant_q8K_lds16(lds, xs, nbH, a.lds_xq);
        // the next layer's router row: loaded now, written to LDS after the logit wait
        const bool rw_next = b < E && l + 1 < a.n_layer;
        // (loads are unconditional, from clamped addresses -- a WG without a next
        // row reads x_in, an L2 hit -- so that none of them waits for another)
        const float* rw_src = rw_next ? ((const DecodeLayer*) s_L[(l + 1) & 1])->router + (size_t) b * H : a.x_in;
        const uint32_t rw_dst = a.lds_rw + (uint32_t) ((l + 1) & 1) * (uint32_t) H * 4u;
        const bool rw0 = rw_next && tid < H / 4, rw1 = rw_next && tid + DEC_THREADS < H / 4;
        const u32x4 rwv0 = ldg16(rw_src + 4 * min(tid, H / 4 - 1));
        const u32x4 rwv1 = ldg16(rw_src + 4 * min(tid + DEC_THREADS, H / 4 - 1));
        // ---- top-k (every WG) -----------------------------------------------------
        // The order by logit (ties by index) is the order by probability unless the
        // softmax rounds two of the first k + 1 places together.  The gate/up rows of
        // that order are loaded while the softmax runs; the exact order is then
        // checked against it and, on a difference, the rows are loaded again.
        gather_tagged<1>(a, a.xl, E, ep, s_p, &s_fail);
        if (rw0) sts16(lds, rw_dst + 16u * tid, rwv0);
        if (rw1) sts16(lds, rw_dst + 16u * (tid + DEC_THREADS), rwv1);
        if (tid == 0) {
            s_need_sort = 0;
            s_bad = 0;
            s_reload = 0;
        }
        lds_barrier();
        if (s_fail) return;
        loads_returned();
        // resident-only routing: workgroup 0 records the top k of the raw logits,
        // then every workgroup adds the layer's mask row before ranking them
        if (L.resmask) {
            if (b == 0 && L.want) decode_want(s_p, E, k, L.want, s_order, s_stack, &s_wflag, tid, DEC_THREADS);
            for (int i = tid; i < E; i += DEC_THREADS) s_p[i] = s_p[i] + L.resmask[i];
            lds_barrier();
        }
        // logit ranks: rank = number of strictly larger logits, TOPK_TPV lanes per
        // value, lane sub taking the float4 groups c = sub (mod TOPK_TPV).  Equal
        // logits share a rank, so the losing one fails the check below, as does a
        // NaN; either sends the layer to the exact order.  E % 8 == 0, so the groups
        // of a lane come in whole batches of 8 when E % 128 == 0 (else clamped).
        // (s_order holds rank[i] until the check.)
        for (int i0 = 0; i0 < E; i0 += DEC_THREADS / TOPK_TPV) {
            const int i = i0 + tid / TOPK_TPV, sub = tid % TOPK_TPV;
            const float li = s_p[i < E ? i : 0];
            int rank = 0;
            for (int c0 = sub; c0 < E / 4; c0 += 8 * TOPK_TPV) {
                float4 q[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) q[u] = *(const float4*) (s_p + 4 * min(c0 + u * TOPK_TPV, E / 4 - 1));
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int gt = (q[u].x > li) + (q[u].y > li) + (q[u].z > li) + (q[u].w > li);
                    rank += c0 + u * TOPK_TPV < E / 4 ? gt : 0;   // (a clamped repeat counts 0)
                }
            }
#pragma unroll
            for (int o = 1; o < TOPK_TPV; o <<= 1) rank += __shfl_xor(rank, o);
            if (i < E && sub == 0) {
                s_order[i] = rank;
                if (rank < k) s_spec[rank] = i;
                if (li != li) s_bad = 1;
            }
        }
        lds_barrier();
        // gate/up rows of the speculative experts: one round of loads, in flight
        // through the softmax (a slot that does not map is read as slot 0 here and
        // reported below only if the expert is really selected)
        const bool spec = nA > 0 && nA <= MAXJ_A * DEC_THREADS;
        auto table_a = [&](const int32_t* ids, bool report) {
            for (int r = tid; r < 2 * np; r += DEC_THREADS) {
                const int p = pa0 + (r >> 1);
                const int i = p / F, f = p % F;
                const int e = ids[i];
                const bool up = r & 1;
                const int32_t* so = up ? L.slot_up : L.slot_gate;
                int64_t mat = so ? ldg_i32(so + e) : e;
                if (mat < 0 || mat >= (up ? L.n_slots_up : L.n_slots_gate)) {
                    if (report) atomicOr(a.status, 16);
                    mat = 0;
                }
                s_rowA[r] = (up ? L.up : L.gate) + (size_t) mat * (up ? L.up_nb2 : L.gate_nb2) +
                            (size_t) f * (up ? L.up_nb1 : L.gate_nb1);
            }
        };
        u32x4 t[MAXJ_A];
        if (spec) {
            table_a(s_spec, false);
            lds_barrier();
#pragma unroll
            for (int j = 0; j < MAXJ_A; ++j) {
                const int c = min(tid + j * DEC_THREADS, nA - 1);
                t[j] = ldg16(s_rowA[c / chA] + 16 * (c % chA));
            }
        }
        {
            // ggml_soft_max (ggml-cpu/ops.cpp): max, ggml_vec_soft_max_f32 (exp in
            // AVX2 groups of 8, double sum), scale by 1/sum
            float mx = -INFINITY;
            for (int i = lane; i < E; i += 64) mx = fmaxf(mx, s_p[i]);
            mx = fmaxf(mx, dpp_f<DPP_XOR1>(mx));
            mx = fmaxf(mx, dpp_f<DPP_XOR2>(mx));
            mx = fmaxf(mx, dpp_f<DPP_HALF_MIRROR>(mx));
            mx = fmaxf(mx, dpp_f<DPP_MIRROR>(mx));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            for (int i = tid; i < E; i += DEC_THREADS) s_e[i] = v_expf(s_p[i] - mx);
            lds_barrier();
            for (int g = tid; g < E / 8; g += DEC_THREADS) s_gsum[g] = hsum8(&s_e[8 * g]);
            lds_barrier();
            double sum = 0.0;
            for (int g = 0; g < E / 8; ++g) sum += (double) s_gsum[g];
            const float inv = (float) (1.0 / sum);
            for (int i = tid; i < E; i += DEC_THREADS) s_p[i] = s_e[i] * inv;
            lds_barrier();
            // The speculative order is the exact argsort's first k iff its
            // probabilities strictly decrease and every other one is strictly
            // below the k-th (then no tie or NaN can reorder them).
            {
                const float q = s_p[s_spec[k - 1]];
                for (int i = tid; i < E; i += DEC_THREADS) {
                    const int r = s_order[i];
                    const float pi = s_p[i];
                    const bool ok = r >= k ? (pi < q) : (s_spec[r] == i && (r == 0 || s_p[s_spec[r - 1]] > pi));
                    if (!ok) s_bad = 1;
                }
            }
            lds_barrier();
            if (!s_bad) {
                if (tid < k) s_order[tid] = s_spec[tid];
            } else {
                // argsort (descending) by ranks: with no value tied (or unordered)
                // inside the first k places the order is unique; otherwise std::sort's
                // own tie order decides -> exact replay below
                for (int i = tid; i < E; i += DEC_THREADS) {
                    const float pi = s_p[i];
                    int gt = 0, eq = 0;
#pragma unroll 4
                    for (int j = 0; j < E; j += 4) {
                        const float4 q = *(const float4*) (s_p + j);
                        gt += (q.x > pi) + (q.y > pi) + (q.z > pi) + (q.w > pi);
                        eq += (q.x == pi) + (q.y == pi) + (q.z == pi) + (q.w == pi);
                    }
                    if (gt < k) {
                        if (eq != 1) s_need_sort = 1;
                        else s_order[gt] = i;
                    }
                }
                lds_barrier();
                if (s_need_sort) {
                    if (tid == 0) {
                        for (int i = 0; i < E; ++i) s_order[i] = i;
                        libstdcxx_sort_desc(s_order, E, s_p, s_stack);
                        if (b == 0) atomicOr(a.status, 1);
                    }
                }
            }
            lds_barrier();
            if (tid < k) {
                const int id = s_order[tid];
                s_ids[tid] = id;
                s_e[tid] = s_p[id];
                if (id != s_spec[tid]) s_reload = 1;
            }
            lds_barrier();
            // weights: selected probabilities / clamp(sum) (* scale)
            if (tid < k) {
                double s = 0.0;
                for (int i = 0; i < k; ++i) s += (double) s_e[i];
                float wsum = (float) s;
                wsum = fmaxf(fminf(wsum, INFINITY), 6.103515625e-5f);
                float wi = s_e[tid] / wsum;
                if (a.scale != 0.0f && a.scale != 1.0f) wi = wi * a.scale;
                s_w[tid] = wi;
                if (b == 0 && a.ids_out) {
                    a.ids_out[l * k + tid] = s_ids[tid];
                    a.w_out[l * k + tid] = wi;
                }
            }
        }
        // ---- down row addresses; slot checks of the selected experts ------------
        for (int r = tid; r < k * nh; r += DEC_THREADS) {
            const int i = r / nh, hh = r % nh;
            const int e = s_ids[i];
            int64_t mat = L.slot_down ? ldg_i32(L.slot_down + e) : e;
            if (mat < 0 || mat >= L.n_slots_down) {
                atomicOr(a.status, 16);
                mat = 0;
            }
            s_rowB[r] = L.down + (size_t) mat * L.down_nb2 + (size_t) (h0 + hh) * L.down_nb1;
        }
        const bool reload = !spec || s_reload;
        if (!reload && tid < 2 * k) {   // the gate/up table was built without reporting
            const int e = s_ids[tid >> 1];
            const bool up = tid & 1;
            const int32_t* so = up ? L.slot_up : L.slot_gate;
            const int64_t mat = so ? ldg_i32(so + e) : e;
            if (mat < 0 || mat >= (up ? L.n_slots_up : L.n_slots_gate)) atomicOr(a.status, 16);
        }
        // ---- gate/up rows to LDS --------------------------------------------------
        if (!reload) {
#pragma unroll
            for (int j = 0; j < MAXJ_A; ++j) {
                const int c = tid + j * DEC_THREADS;
                if (c < nA) sts16(lds, a.lds_a + (uint32_t) (c / chA) * a.rs_a + 16u * (c % chA), t[j]);
            }
        } else {
            table_a(s_ids, true);
            lds_barrier();
            // every load of a round in flight at once
            for (int base = 0; base < nA; base += MAXJ_A * DEC_THREADS) {
                u32x4 t2[MAXJ_A];
#pragma unroll
                for (int j = 0; j < MAXJ_A; ++j) {
                    const int c = min(base + tid + j * DEC_THREADS, nA - 1);
                    t2[j] = ldg16(s_rowA[c / chA] + 16 * (c % chA));
                }
#pragma unroll
                for (int j = 0; j < MAXJ_A; ++j) {
                    const int c = base + tid + j * DEC_THREADS;
                    if (c < nA) sts16(lds, a.lds_a + (uint32_t) (c / chA) * a.rs_a + 16u * (c % chA), t2[j]);
                }
            }
        }
        lds_barrier();
        // ---- A: gate / up rows, SwiGLU ---------------------------------------------
        for (int r0 = 0; r0 < np * 2; r0 += DEC_WAVES * 8) {
            const int r = r0 + wave * 8 + (lane >> 3);
            const int rr = r < np * 2 ? r : 0;
            float v;
            if constexpr (NBH > 0) v = row_dot_q4k_a<NBH>(lds, a.lds_a + (uint32_t) rr * a.rs_a, a.lds_xq, lane & 7);
            else v = row_dot_lds<T_Q4_K>(lds, a.lds_a + (uint32_t) rr * a.rs_a, a.lds_xq, nbH, lane & 7);
            if (r < np * 2 && (lane & 7) == 0) res[r] = v;
        }
        lds_barrier();
        if (tid < np) {   // np <= 48 (plan)
            const int j = tid;
            const float act = v_silu(res[2 * j]) * res[2 * j + 1];
            st_dev64(a.xa + pa0 + j, tagged(act, ep));
        }
        // ---- down rows: issued now, held in registers while act is exchanged --------
        // (after the act stores: issued before them, the compiler waits for these
        // loads inside the SwiGLU block)
        u32x4 tb[MAXJ_B];
        if (b_fits && nB > 0) {
#pragma unroll
            for (int j = 0; j < MAXJ_B; ++j) {
                const int c = min(tid + j * DEC_THREADS, nB - 1);
                bool ok;
                tb[j] = ldg16(down_chunk(s_rowB[c / chB], rowB, c % chB, ok));
            }
        }
        // ---- B: all act -> Q8_K per slot; down rows; weighted sum ------------------
        // (act lands where the gate/up rows were: every thread is past the A
        // barrier, so they are consumed)
        gather_tagged<12>(a, a.xa, P, ep, actf, &s_fail);
        if (b_fits) {
#pragma unroll
            for (int j = 0; j < MAXJ_B; ++j) {
                const int c = tid + j * DEC_THREADS;
                bool ok = false;
                if (c < nB) down_chunk(s_rowB[c / chB], rowB, c % chB, ok);
                if (ok) sts16(lds, a.lds_b + (uint32_t) (c / chB) * a.rs_b + 16u * (c % chB), tb[j]);
            }
        } else {
            for (int c = tid; c < nB; c += DEC_THREADS) {
                bool ok;
                const u32x4 v = ldg16(down_chunk(s_rowB[c / chB], rowB, c % chB, ok));
                if (ok) sts16(lds, a.lds_b + (uint32_t) (c / chB) * a.rs_b + 16u * (c % chB), v);
            }
        }
        lds_barrier();
        if (s_fail) return;
        loads_returned();
        quant_q8K_lds16(lds, actf, k * nbF, a.lds_aq);
        lds_barrier();
        for (int r0 = 0; r0 < k * nh; r0 += DEC_WAVES * 8) {
            const int r = r0 + wave * 8 + (lane >> 3);
            const int rr = r < k * nh ? r : 0;
            const int i = rr / nh;
            const uint32_t wb = a.lds_b + (uint32_t) rr * a.rs_b + (uint32_t) ((uintptr_t) s_rowB[rr] & 15);
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
        lds_barrier();
        if (tid < nh) {   // nh <= 256 (plan)
            const int hh = tid;
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
        // the descriptor of layer l + 2 replaces this layer's (its loads return
        // before the y polls that follow them)
        const bool next2 = l + 2 < a.n_layer && tid < LAYER_WORDS;
        const uint64_t lw = ldg_u64((const uint64_t*) (a.layers + (next2 ? l + 2 : l)) + (tid % LAYER_WORDS));
        // ---- C: all y -> RMSNorm -> x of the next layer ----------------------------
        gather_tagged<4>(a, a.xy, H, ep, ys, &s_fail);
        if (next2) s_L[l & 1][tid] = lw;
        lds_barrier();
        if (s_fail) return;
        loads_returned();
        {
            double s = 0.0;
            for (int i = tid; i < H; i += DEC_THREADS) {
                const float v = ys[i];
                s += (double) (v * v);
            }
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) s_red[wave] = s;
            lds_barrier();
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
            lds_barrier();
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
    a.lds_y = d.lds_y;
    a.lds_total = d.lds_total;
    a.rs_a = d.rs_a;
    a.rs_b = d.rs_b;
    void* args[] = {&a};
    // A plain launch: one WG per CU, and the LDS footprint admits only one per
    // CU, so on a device this process is not sharing every WG is resident at
    // once (checked at create time by check_decode_residency).  If some WG is
    // held back, the others' bounded waits end the launch with status bit 3.
    hipError_t e = hipLaunchKernel(decode_kernel(d), dim3((unsigned) d.grid), dim3(DEC_THREADS), args, d.lds_total,
                                   stream);
    return e == hipSuccess ? 0 : -3;
}

const void* decode_kernel(const DecodeStackDesc& d) {
    if (d.type_down == T_Q4_K && d.H == 2048 && d.F == 768) return (const void*) k_decode_stack<8, 3, T_Q4_K>;
    if (d.type_down == T_Q6_K) return (const void*) k_decode_stack<0, 0, T_Q6_K>;
    return (const void*) k_decode_stack<0, 0, T_Q4_K>;
}

int check_decode_residency(const DecodeStackDesc& d) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel(d), DEC_THREADS, d.lds_total) !=
        hipSuccess)
        return -3;
    return per_cu >= 1 ? 0 : -2;
}

int plan_decode_stack(DecodeStackDesc& d, int grid) {
    if (d.H % 256 || d.F % 256 || d.E % 8 || d.E > 512 || d.k < 1 || d.k > 32 || d.k > d.E) return -2;
    if (d.type_down != T_Q4_K && d.type_down != T_Q6_K) return -2;
    if (d.H > 2 * 4 * DEC_THREADS) return -2;          // router row held in two uint4 per thread
    d.grid = grid;
    const int P = (int) (d.k * d.F);
    d.pa_per = (P + grid - 1) / grid;
    d.hb_per = (int) (((d.H + grid - 1) / grid + 3) / 4 * 4);
    if (d.E > grid) return -2;                         // one router row per WG
    if (2 * d.pa_per > 96 || d.k * d.hb_per > 256) return -2;   // row address tables
    const uint32_t rowA = (uint32_t) (d.H / 256) * 144u;
    const uint32_t rowB = (uint32_t) (d.F / 256) * (d.type_down == T_Q4_K ? 144u : 210u);
    d.rs_a = rowA + 32;                                // stride = 8 (mod 32) dwords for 144-byte rows
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
    d.lds_res = take((uint32_t) std::max<int64_t>(2 * d.pa_per, d.k * d.hb_per) * 4u);
    d.lds_y = take((uint32_t) d.H * 4u);
    d.lds_total = off;
    if (d.lds_total > 160 * 1024 - 12 * 1024) return -2;   // static shared arrays take ~11 KB
    return 0;
}

}  // namespace qw
