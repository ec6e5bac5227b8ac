// decode_xcd.hip -- persistent whole-stack MoE FFN decode with one selected
// expert per XCD (the work core/runtime.cpp schedules as build_moe per layer
// inside one graph, decode() -> build_graph, 976-1100).
//
// MI355X runs a 256-workgroup launch as 8 XCDs of 32 CUs, workgroup b on XCD
// b % 8, and each XCD has its own L2.  A decode token selects k <= 8 experts per
// layer, so XCD c takes the expert of top-k rank c: its 32 workgroups split
// that expert's gate/up rows (F/32 (gate, up) pairs each) and down rows (H/32
// each).  Of the four data exchanges of a layer only one crosses XCDs:
//   L  every XCD computes all E router logits (E/32 per workgroup, the AVX2
//      ggml_vec_dot_f32 chain order) and all-gathers them inside the XCD;
//   A  the XCD's expert's F SwiGLU values, all-gathered inside the XCD;
//   D  workgroup j of every XCD gathers d_i[h] (i < k) for its H/32 rows from
//      the k expert XCDs and forms y[h] = sum_i d_i[h] * w_i -- the one hop
//      across XCDs;
//   Y  y all-gathered inside the XCD; every workgroup forms the RMSNorm, the
//      Q8_K of x and its router logits of the next layer.
// Exchanged values are 64-bit words {fp32 value, epoch}; a consumer polls the
// words themselves (agent-scope loads), so one memory round trip carries the
// value and says that it is there.  Inside an XCD the producers store with
// workgroup scope (into the XCD's L2, the coherence point of its CUs); the D
// words cross XCDs and are stored with agent scope.  The host enables the
// XCD-local stores only after checking the workgroup -> XCD mapping on the
// device; without that every store is agent scope (correct anywhere, slower).
//
// Weights are loaded with 16-byte loads straight into registers, eight lanes
// per 144-byte Q4_K super-block (lane t holds the header and quant chunk t), and
// consumed there: each lane forms the integer partial sums of four of the
// eight AVX lanes of ggml's q4_K dot, DPP adds finish the integer lane sums,
// and the float steps run in ggml's order -- per AVX lane an fma chain over the
// super-blocks of the row, then hsum_float_8 and the min lanes
// (ggml-cpu/arch/x86/quants.c:2038-2115).  Ids, weights and outputs are
// bit-identical to the reference CPU path.
#include "qw_kernels.hpp"
#include "qw_sort.hpp"
#include "qw_decode.hpp"

#include <vector>

namespace qw {

namespace {

constexpr int XT = 512;                 // threads per workgroup
constexpr int XW = XT / 64;             // waves
constexpr int NXCD = 8;
constexpr int NJ = 32;                  // workgroups per XCD
constexpr long XSPIN = 1L << 22;        // polls before a wait gives up (~seconds)
constexpr int QB = 304;                 // LDS Q8_K block: qs[256] | d | bsums[16] | pad (16-aligned qs)
constexpr int XLW = sizeof(DecodeLayer) / 8;

struct XcdArgs {
    const DecodeLayer* layers;
    int n_layer, k;
    float scale, rms_eps;
    const float* x_in;
    float* out;
    float* x_out;
    int32_t* ids_out;
    float* w_out;
    uint64_t* xl;      // [NXCD][E]          logits, XCD-local
    uint64_t* xa;      // [NXCD][F]          act, XCD-local
    uint64_t* xd;      // [2][NXCD][NJ][NH]  down outputs, across XCDs (double-buffered by layer parity)
    uint64_t* xy;      // [NXCD][H]          y, XCD-local
    uint32_t epoch0;
    int32_t* status;   // bit 0: top-k tie replayed; 3: a wait timed out; 4: bad slot; 6: XCD mapping differs
    int32_t* abort_flag;
    int local_st;      // 1: XCD-local words stored with workgroup scope
};

typedef __attribute__((address_space(1))) const u32x4 gq4_t;
__device__ __forceinline__ u32x4 ldg16(const void* p) { return *(gq4_t*) p; }
__device__ __forceinline__ uint64_t ldg64(const void* p) {
    return *(const __attribute__((address_space(1))) uint64_t*) p;
}
__device__ __forceinline__ int32_t ldg32(const void* p) {
    return *(const __attribute__((address_space(1))) int32_t*) p;
}
__device__ __forceinline__ uint64_t poll64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_cross(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_local(uint64_t* p, uint64_t v, int local) {
    if (local) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tag(float v, uint32_t ep) { return ((uint64_t) ep << 32) | (uint64_t) fbits(v); }

__device__ __forceinline__ bool x_aborted(const XcdArgs& a) {
    return (uint32_t) __hip_atomic_load(a.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= a.epoch0;
}
__device__ __forceinline__ void x_abort(const XcdArgs& a, int bit) {
    atomicOr(a.status, bit);
    __hip_atomic_store(a.abort_flag, (int32_t) a.epoch0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-local LDS ordering: every LDS access of this wave issued before has
// completed, and the compiler keeps memory accesses on their side.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Polls n tagged words (this thread's: i = tid + XT * m, m < MAXJ) until each
// carries epoch ep, then stores the payloads to dst[i] (LDS).  Only the words
// not yet seen are polled again.  Returns false if the wait gave up.
template <int MAXJ>
__device__ __forceinline__ bool gather(const XcdArgs& a, const uint64_t* src, int n, uint32_t ep, float* dst,
                                       int tid) {
    uint32_t got = 0;
    uint32_t val[MAXJ];
#pragma unroll
    for (int m = 0; m < MAXJ; ++m) {
        val[m] = 0;
        if (tid + m * XT >= n) got |= 1u << m;
    }
    const uint32_t all = (1u << MAXJ) - 1u;
    long spins = 0;
    while (got != all) {
        uint64_t v[MAXJ];
#pragma unroll
        for (int m = 0; m < MAXJ; ++m) v[m] = poll64(src + min(tid + m * XT, n - 1));
#pragma unroll
        for (int m = 0; m < MAXJ; ++m)
            if (!(got & (1u << m)) && (uint32_t) (v[m] >> 32) == ep) {
                val[m] = (uint32_t) v[m];
                got |= 1u << m;
            }
        if (got == all) break;
        if (++spins > XSPIN) {
            x_abort(a, 8);
            return false;
        }
        if ((spins & 255) == 0 && x_aborted(a)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int m = 0; m < MAXJ; ++m)
        if (tid + m * XT < n) dst[tid + m * XT] = bitsf(val[m]);
    return true;
}

// quantize_row_q8_K_ref (ggml-quants.c:2768-2803) of nblocks x 256 fp32 values
// in LDS into QB-strided LDS blocks.  Sixteen lanes (one DPP row) per block,
// sixteen consecutive values per lane: the first-index max |x| is a four-step
// row reduction, and each lane's values form exactly one bsums group.
// Threads [0, 16 * nblocks) take part.
__device__ __forceinline__ void quant_q8K_xb(const float* src, int nblocks, uint8_t* q, int tid) {
    const int tt = tid;
    if (tt < 0 || tt >= 16 * nblocks) return;
    const int b = tt >> 4, l = tt & 15;
    const float* x = src + b * QK_K + 16 * l;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        const float4 t4 = *(const float4*) (x + i);
        v[i] = t4.x;
        v[i + 1] = t4.y;
        v[i + 2] = t4.z;
        v[i + 3] = t4.w;
    }
    float am = 0.0f;
    int ai = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = __builtin_fabsf(v[i]);
        if (ax > am) { am = ax; ai = 16 * l + i; }
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
    uint8_t* blk = q + b * QB;
    if (!(am > 0.0f)) {
        *(u32x4*) (blk + 16 * l) = u32x4{0u, 0u, 0u, 0u};
        *(int16_t*) (blk + 260 + 2 * l) = 0;
        if (l == 0) *(float*) (blk + 256) = 0.0f;
        return;
    }
    const float iscale = -127.f / src[b * QK_K + ai];
    int s = 0;
    u32x4 words = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int t = nearest_int(iscale * v[i]);
        t = t < 127 ? t : 127;
        s += t;
        words[i >> 2] |= (uint32_t) (t & 0xff) << (8 * (i & 3));
    }
    *(u32x4*) (blk + 16 * l) = words;
    *(int16_t*) (blk + 260 + 2 * l) = (int16_t) s;
    if (l == 0) *(float*) (blk + 256) = 1.0f / iscale;
}

// Integer partials of one Q4_K super-block for lane t (0..7) of its 8-lane
// group: hdr = bytes 0..15 (d, dmin, scales), qc = quant bytes 16t..16t+15,
// i.e. 64-element chunk j = t >> 1 and AVX lanes n = 4 (t & 1) + i.  yq: the
// Q8_K block's qs in LDS.  p[i] = sc_{2j} . sum(q4lo . q8) + sc_{2j+1} . sum(q4hi . q8)
// over AVX lane n's four bytes (the maddubs + madd of quants.c:2092-2100).
__device__ __forceinline__ void q4k_partials(const u32x4& hdr, const u32x4& qc, const uint8_t* yq, int t, int p[4]) {
    const int j = t >> 1, hb = t & 1;
    const uint32_t s0 = hdr[1], s2 = hdr[3];
    const uint32_t scw = j < 2 ? (s0 & 0x3f3f3f3fu) : ((s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4));
    const int sh = 16 * (j & 1);
    const int scl = (int) ((scw >> sh) & 0xffu), sch = (int) ((scw >> (sh + 8)) & 0xffu);
    const u32x4 alo = *(const u32x4*) (yq + 64 * j + 16 * hb);
    const u32x4 ahi = *(const u32x4*) (yq + 64 * j + 32 + 16 * hb);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int lo = (int) (qc[i] & 0x0F0F0F0Fu), hi = (int) ((qc[i] >> 4) & 0x0F0F0F0Fu);
        p[i] = mul24(scl, sdot4(lo, (int) alo[i], 0)) + mul24(sch, sdot4(hi, (int) ahi[i], 0));
    }
}

// Min lane n = t (t < 4) of a Q4_K super-block: mins of sub-blocks 2n, 2n+1
// times the Q8_K sums of those sub-blocks (_mm_madd_epi16(mins, hadd(bsums)),
// quants.c:2084-2087).  yb: the Q8_K block in LDS (bsums at 260).
__device__ __forceinline__ int q4k_min_prod(const u32x4& hdr, const uint8_t* yb, int t) {
    const uint32_t s1 = hdr[2], s2 = hdr[3];
    const int n = t & 3;
    const uint32_t mw = n < 2 ? (s1 & 0x3f3f3f3fu) : (((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4));
    const int m0 = (int) ((mw >> (16 * (n & 1))) & 0xffu), m1 = (int) ((mw >> (16 * (n & 1) + 8)) & 0xffu);
    const uint32_t bs01 = *(const uint32_t*) (yb + 260 + 8 * n), bs23 = *(const uint32_t*) (yb + 264 + 8 * n);
    const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
    const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
    return mul24(m0, q8s0) + mul24(m1, q8s1);
}

// Sum over the four 64-element chunks: lanes t and t ^ 2 (quad_perm), then t
// and t + 4 (row_shl:4).  Valid in lanes t = 0 (AVX lanes 0..3) and t = 1 (4..7).
__device__ __forceinline__ void reduce_chunks(int p[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int a = p[i] + dpp_i<DPP_XOR2>(p[i]);
        p[i] = a + __builtin_amdgcn_update_dpp(0, a, 0x104, 0xF, 0xF, false);   // row_shl:4: lane i <- i + 4
    }
}

// std::sort's order of tied probabilities (qw_sort.hpp), kept out of line: the
// replay runs only when ties reach into the top k.
__device__ __attribute__((noinline)) void sort_desc_replay(int32_t* order, int n, const float* p, SortRange* stack) {
    libstdcxx_sort_desc(order, n, p, stack);
}

// Router logits e = NLOG * j + hw of x (LDS) from the LDS router rows; lanes
// c < 32 of half-wave hw are the 32 fma chains of AVX2 ggml_vec_dot_f32
// (GGML_F32_STEP 32), then its reduction tree; lane 0 returns the logit.
template <int H>
__device__ __forceinline__ float router_chain(const float* w, const float* x, int c) {
    float acc = 0.0f;
#pragma unroll 1
    for (int s0 = 0; s0 < H; s0 += 16 * 32) {
        float wv[16], xv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            wv[u] = w[s0 + 32 * u + c];
            xv[u] = x[s0 + 32 * u + c];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = __builtin_fmaf(wv[u], xv[u], acc);
    }
    float t = acc + __shfl_down(acc, 16, 32);   // c_l + c_{16+l}
    t = t + __shfl_down(t, 8, 32);               // (c_l + c_{16+l}) + (c_{8+l} + c_{24+l})
    t = t + __shfl_down(t, 4, 32);               // t0_l = s_l + s_{l+4}
    const float u = t + __shfl_down(t, 1, 32);
    return u + __shfl_down(u, 2, 32);            // (t0_0 + t0_1) + (t0_2 + t0_3)
}

}  // namespace

// NBH = H / 256 (8), NBF = F / 256 (down super-blocks per row, <= 3), NLOG = E / 32.
template <int NBH, int NBF, int NLOG>
__global__ void __launch_bounds__(XT) k_decode_xcd(XcdArgs a) {
    constexpr int H = NBH * QK_K, F = NBF * QK_K, E = NLOG * 32;
    constexpr int NP = F / NJ;            // (gate, up) pairs per workgroup
    constexpr int PPW = NP / XW;          // pairs per wave
    constexpr int NH = H / NJ;            // down rows per workgroup
    constexpr int RW = NH / XW;           // down rows per wave (one per 8-lane group)
    static_assert(NBH == 8, "gate/up rows: one super-block per 8-lane group");
    static_assert(PPW >= 1 && PPW * XW == NP && 2 * PPW * 8 <= 64, "pairs per wave");
    static_assert(RW == 8, "down rows: one row per 8-lane group");
    static_assert(E <= 128, "ranking: four lanes per logit");

    __shared__ __align__(16) float s_rw[NLOG * H];              // router rows of this workgroup
    __shared__ __align__(16) float s_x[H];                      // x of the current layer
    __shared__ __align__(16) float s_y[H];                      // gathered y
    __shared__ __align__(16) uint8_t s_xq[NBH * QB];            // Q8_K(x)
    __shared__ __align__(16) float s_act[F];
    __shared__ __align__(16) uint8_t s_aq[NBF * QB];            // Q8_K(act)
    __shared__ __align__(16) uint32_t s_tr[XW][2 * PPW][NBH][16];   // gate/up block records
    __shared__ __align__(16) float s_d8[NXCD * NH];
    __shared__ __align__(16) float s_p[E];
    __shared__ float s_e[E];
    __shared__ int32_t s_order[E];
    __shared__ float s_gsum[E / 8];
    __shared__ int32_t s_slot[2][3][E];
    __shared__ uint64_t s_L[2][XLW];
    __shared__ SortRange s_stack[SORT_STACK];
    __shared__ double s_red[XW];
    __shared__ int32_t s_spec[8];
    __shared__ int32_t s_ids[8];
    __shared__ float s_w[8];
    __shared__ int s_fail, s_bad, s_need_sort;

    const int b = blockIdx.x, tid0 = threadIdx.x;
    const int xcd = b & (NXCD - 1), j = b >> 3;
    const int k = a.k;
    const bool expert_xcd = xcd < k;
    const int local = a.local_st;

    if ((int) (__builtin_amdgcn_s_getreg((3 << 11) | 20) & 7) != xcd && tid0 == 0) atomicOr(a.status, 64);

    // ---- prologue: descriptors, x of layer 0, router rows and slot rows of layer 0
    if (tid0 == 0) s_fail = 0;
    if (tid0 < 8) s_spec[tid0] = 0;
    if (tid0 < 2 * XLW && tid0 / XLW < a.n_layer) s_L[tid0 / XLW][tid0 % XLW] = ldg64((const uint64_t*) a.layers + tid0);
    for (int i = tid0; i < H; i += XT) s_x[i] = a.x_in[i];
    {
        const DecodeLayer& L0 = a.layers[0];
        const float* rsrc = L0.router + (size_t) NLOG * j * H;
        for (int c = tid0; c < NLOG * H / 4; c += XT) *(u32x4*) (s_rw + 4 * c) = ldg16(rsrc + 4 * c);
        for (int i = tid0; i < 3 * E; i += XT) {
            const int32_t* so = i < E ? L0.slot_gate : i < 2 * E ? L0.slot_up : L0.slot_down;
            s_slot[0][i / E][i % E] = so ? ldg32(so + i % E) : i % E;
        }
    }
    __syncthreads();
    quant_q8K_xb(s_x, NBH, s_xq, tid0);
    {
        const int rw0 = XW - (NLOG + 1) / 2;   // router waves: the last ones
        const int w = tid0 >> 6, hw = 2 * (w - rw0) + ((tid0 >> 5) & 1), c = tid0 & 31;
        if (w >= rw0 && hw < NLOG) {
            const float lg = router_chain<H>(s_rw + hw * H, s_x, c);
            if (c == 0) st_local(a.xl + xcd * E + NLOG * j + hw, tag(lg, a.epoch0), local);
        }
    }

    for (int l = 0; l < a.n_layer; ++l) {
        const DecodeLayer& L = *(const DecodeLayer*) s_L[l & 1];
        const uint32_t ep = a.epoch0 + (uint32_t) l;
        const int tid = opaque(tid0);
        const int wave = tid >> 6, lane = tid & 63, g = lane >> 3, t = lane & 7;

        // ---- L: the layer's logits (all E, from this XCD) ----------------------
        if (!gather<1>(a, a.xl + xcd * E, E, ep, s_p, tid)) s_fail = 1;
        if (tid == 0) {
            s_bad = 0;
            s_need_sort = 0;
        }
        lds_barrier();
        if (s_fail) return;
        // logit ranks (strictly larger count; four lanes per value); the rank-c
        // expert is XCD c's speculative expert, its rows are loaded at once
        {
            const int i = tid >> 2, sub = tid & 3;
            const float li = s_p[i < E ? i : 0];
            int rank = 0;
#pragma unroll
            for (int c0 = 0; c0 < E / 4; c0 += 4) {
                const float4 q = *(const float4*) (s_p + 4 * (c0 + sub));
                rank += (q.x > li) + (q.y > li) + (q.z > li) + (q.w > li);
            }
            rank += __shfl_xor(rank, 1);
            rank += __shfl_xor(rank, 2);
            if (i < E && sub == 0) {
                s_order[i] = rank;
                if (rank < k) s_spec[rank] = i;
                if (li != li) s_bad = 1;
            }
        }
        lds_barrier();

        // ---- weight loads of this XCD's expert ------------------------------------
        u32x4 gh[2 * PPW], gq[2 * PPW];    // gate/up rows: header and chunk t of block g
        u32x4 dh[NBF], dq[NBF];            // down row 8 * wave + g: header and chunk t of each block
        // gate/up rows: issued for the speculative expert (reissued if it was wrong);
        // down rows: issued once the expert is certain (they are used after the act exchange)
        auto issue = [&](int e) {
            const int e_c = e < 0 || e >= E ? 0 : e;
            int sg = s_slot[l & 1][0][e_c], su = s_slot[l & 1][1][e_c];
            sg = (sg < 0 || sg >= L.n_slots_gate) ? 0 : sg;
            su = (su < 0 || su >= L.n_slots_up) ? 0 : su;
#pragma unroll
            for (int p = 0; p < PPW; ++p) {
                const int f = NP * j + PPW * wave + p;
                const uint8_t* rg = L.gate + (size_t) sg * L.gate_nb2 + (size_t) f * L.gate_nb1 + 144 * g;
                const uint8_t* ru = L.up + (size_t) su * L.up_nb2 + (size_t) f * L.up_nb1 + 144 * g;
                gh[2 * p] = ldg16(rg);
                gq[2 * p] = ldg16(rg + 16 + 16 * t);
                gh[2 * p + 1] = ldg16(ru);
                gq[2 * p + 1] = ldg16(ru + 16 + 16 * t);
            }
        };
        auto issue_down = [&](int e) {
            const int e_c = e < 0 || e >= E ? 0 : e;
            int sd = s_slot[l & 1][2][e_c];
            sd = (sd < 0 || sd >= L.n_slots_down) ? 0 : sd;
            const uint8_t* rd = L.down + (size_t) sd * L.down_nb2 + (size_t) (NH * j + RW * wave + g) * L.down_nb1;
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) {
                dh[bb] = ldg16(rd + 144 * bb);
                dq[bb] = ldg16(rd + 144 * bb + 16 + 16 * t);
            }
        };
        const int spec_e = expert_xcd ? s_spec[xcd] : 0;
        if (expert_xcd) issue(spec_e);

        // ---- softmax, exact order, weights (every workgroup, same values) -------
        {
            float mx = -INFINITY;
            for (int i = lane; i < E; i += 64) mx = fmaxf(mx, s_p[i]);
            mx = fmaxf(mx, dpp_f<DPP_XOR1>(mx));
            mx = fmaxf(mx, dpp_f<DPP_XOR2>(mx));
            mx = fmaxf(mx, dpp_f<DPP_HALF_MIRROR>(mx));
            mx = fmaxf(mx, dpp_f<DPP_MIRROR>(mx));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            for (int i = tid; i < E; i += XT) s_e[i] = v_expf(s_p[i] - mx);
            lds_barrier();
            for (int gi = tid; gi < E / 8; gi += XT) s_gsum[gi] = hsum8(&s_e[8 * gi]);
            lds_barrier();
            double sum = 0.0;
            for (int gi = 0; gi < E / 8; ++gi) sum += (double) s_gsum[gi];
            const float inv = (float) (1.0 / sum);
            for (int i = tid; i < E; i += XT) s_p[i] = s_e[i] * inv;
            lds_barrier();
            // the speculative order is the argsort's first k iff its probabilities
            // strictly decrease and every other one is strictly below the k-th
            {
                const float q = s_p[s_spec[k - 1]];
                for (int i = tid; i < E; i += XT) {
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
                for (int i = tid; i < E; i += XT) {
                    const float pi = s_p[i];
                    int gt = 0, eq = 0;
                    for (int jj = 0; jj < E; jj += 4) {
                        const float4 q = *(const float4*) (s_p + jj);
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
                    for (int i = tid; i < E; i += XT) s_order[i] = i;
                    lds_barrier();
                    if (tid == 0) {
                        sort_desc_replay(s_order, E, s_p, s_stack);
                        if (b == 0) atomicOr(a.status, 1);
                    }
                }
            }
            lds_barrier();
            if (tid < k) {
                const int id = s_order[tid];
                s_ids[tid] = id;
                s_e[tid] = s_p[id];
            }
            lds_barrier();
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
        // slot checks of the selected experts (reported once, by workgroup 0)
        if (b == 0 && tid < 3 * k) {
            const int role = tid / k, e = s_ids[tid % k];
            const int32_t s = s_slot[l & 1][role][e];
            const int64_t n = role == 0 ? L.n_slots_gate : role == 1 ? L.n_slots_up : L.n_slots_down;
            if (s < 0 || s >= n) atomicOr(a.status, 16);
        }
        const int my_e = expert_xcd ? s_ids[xcd] : 0;
        if (expert_xcd && my_e != spec_e) issue(my_e);   // misspeculated: load the right rows
        if (expert_xcd) issue_down(my_e);

        // ---- A: gate/up rows of this workgroup's pairs, SwiGLU -----------------
        if (expert_xcd) {
#pragma unroll
            for (int r = 0; r < 2 * PPW; ++r) {
                int p[4];
                const uint8_t* yb = s_xq + QB * g;
                q4k_partials(gh[r], gq[r], yb, t, p);
                reduce_chunks(p);
                uint32_t* rec = s_tr[wave][r][g];
                if (t < 2) *(u32x4*) (rec + 4 * t) = u32x4{(uint32_t) p[0], (uint32_t) p[1], (uint32_t) p[2], (uint32_t) p[3]};
                if (t < 4) rec[8 + t] = (uint32_t) q4k_min_prod(gh[r], yb, t);
                if (t == 0) rec[12] = gh[r][0];
            }
            wave_lds_sync();
            // chain lanes: row r = lane >> 3 (< 2 * PPW), AVX lane n = lane & 7
            float res = 0.0f;
            {
                const int r = g < 2 * PPW ? g : 0, n = t;
                float acc = 0.0f, accm = 0.0f;
#pragma unroll
                for (int bb = 0; bb < NBH; ++bb) {
                    const uint32_t* rec = s_tr[wave][r][bb];
                    const int S = (int) rec[n];
                    const int pm = (int) rec[8 + (n & 3)];
                    const uint32_t h0 = rec[12];
                    const float yd = *(const float*) (s_xq + QB * bb + 256);
                    acc = __builtin_fmaf(yd * h2f((uint16_t) (h0 & 0xffff)), (float) S, acc);
                    const float pmv = __builtin_fmaf(-yd * h2f((uint16_t) (h0 >> 16)), (float) pm, accm);
                    accm = n < 4 ? pmv : accm;
                }
                float s = acc;
                s = s + __shfl_down(s, 4, 8);
                s = s + __shfl_down(s, 2, 8);
                s = s + __shfl_down(s, 1, 8);
                float m = accm;
                m = m + __shfl_down(m, 2, 8);
                m = m + __shfl_down(m, 1, 8);
                res = s + m;
            }
            const float up = __shfl_down(res, 8);   // lane 16p: gate of pair p; lane 16p + 8: its up
            if ((lane & 15) == 0 && (lane >> 4) < PPW) {
                const int f = NP * j + PPW * wave + (lane >> 4);
                st_local(a.xa + xcd * F + f, tag(v_silu(res) * up, ep), local);
            }
        }
        // next layer's router rows, slot rows and the descriptor of layer l + 2:
        // issued once the gate/up rows are consumed, stored to LDS once they are needed
        const bool nxt = l + 1 < a.n_layer;
        const DecodeLayer& L1 = *(const DecodeLayer*) s_L[(l + 1) & 1];
        constexpr int RPT = NLOG * H / 4 / XT;   // router chunks per thread
        u32x4 rp[RPT];
        {
            const float* rsrc = nxt ? L1.router + (size_t) NLOG * j * H : (const float*) a.layers;   // (dummy: 16-aligned)
#pragma unroll
            for (int m = 0; m < RPT; ++m) rp[m] = ldg16(rsrc + 4 * (nxt ? tid + m * XT : 0));
        }
        int32_t sl_next = 0;
        if (tid < 3 * E) {
            const int32_t* so = !nxt ? nullptr : tid < E ? L1.slot_gate : tid < 2 * E ? L1.slot_up : L1.slot_down;
            sl_next = so ? ldg32(so + tid % E) : tid % E;
        }
        const bool next2 = l + 2 < a.n_layer && tid < XLW;
        const uint64_t lw = ldg64((const uint64_t*) (a.layers + (next2 ? l + 2 : l)) + (tid % XLW));

        // ---- act of this XCD's expert -> Q8_K ------------------------------------
        float dres = 0.0f;
        if (expert_xcd) {
            if (!gather<(F + XT - 1) / XT>(a, a.xa + xcd * F, F, ep, s_act, tid)) s_fail = 1;
            lds_barrier();
            if (s_fail) return;
            quant_q8K_xb(s_act, NBF, s_aq, tid);
            lds_barrier();
            // ---- D: down rows 8 * wave + g of this workgroup, in-lane block chain
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            float accm = 0.0f;
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) {
                const uint8_t* yb = s_aq + QB * bb;
                int p[4];
                q4k_partials(dh[bb], dq[bb], yb, t, p);
                reduce_chunks(p);
                const float yd = *(const float*) (yb + 256);
                const float D = yd * h2f((uint16_t) (dh[bb][0] & 0xffff));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(D, (float) p[i], acc[i]);
                const int pm = q4k_min_prod(dh[bb], yb, t);
                accm = __builtin_fmaf(-yd * h2f((uint16_t) (dh[bb][0] >> 16)), (float) pm, accm);
            }
            // hsum_float_8: lane t = 0 holds AVX lanes 0..3, lane t = 1 lanes 4..7
            float r4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) r4[i] = acc[i] + dpp_f<DPP_XOR1>(acc[i]);
            const float hs = (r4[0] + r4[2]) + (r4[1] + r4[3]);
            // min lanes 0..3: (m0 + m2) + (m1 + m3)
            const float m2 = accm + dpp_f<DPP_XOR2>(accm);
            const float mm = m2 + dpp_f<DPP_XOR1>(m2);
            dres = hs + mm;
            if (t == 0) st_cross(a.xd + (((size_t) (l & 1) * NXCD + xcd) * NJ + j) * NH + RW * wave + g, tag(dres, ep));
        }
        // next layer's router rows to LDS (this layer's router ran at the end of the last)
#pragma unroll
        for (int m = 0; m < RPT; ++m)
            if (nxt) *(u32x4*) (s_rw + 4 * (tid + m * XT)) = rp[m];

        // ---- D -> y[h] for this workgroup's rows, in every XCD -------------------
        {
            const uint64_t* src = a.xd + (size_t) (l & 1) * NXCD * NJ * NH;
            // word (c, h) of workgroup (c, j) -> s_d8[c * NH + h]
            const int n = k * NH;
            const int i = tid < n ? tid : n - 1;
            const int c = i / NH, h = i % NH;
            uint32_t v = 0;
            bool ok = tid >= n;
            long spins = 0;
            const uint64_t* wp = src + ((size_t) c * NJ + j) * NH + h;
            while (!ok) {
                const uint64_t x = poll64(wp);
                if ((uint32_t) (x >> 32) == ep) {
                    v = (uint32_t) x;
                    ok = true;
                    break;
                }
                if (++spins > XSPIN) {
                    x_abort(a, 8);
                    break;
                }
                if ((spins & 255) == 0 && x_aborted(a)) break;
                __builtin_amdgcn_s_sleep(1);
            }
            if (!ok) s_fail = 1;
            else if (tid < n) s_d8[tid] = bitsf(v);
        }
        lds_barrier();
        if (s_fail) return;
        // every thread is past its last read of layer l's descriptor: the
        // descriptor of layer l + 2 takes its place
        if (next2) s_L[l & 1][tid] = lw;
        if (tid < 3 * E) s_slot[(l + 1) & 1][tid / E][tid % E] = sl_next;   // (in place of layer l - 1's)
        if (tid < NH) {
            // ggml_vec_dot_f32(k, experts^T row, w): k < 32 -> scalar tail: groups
            // of four as mul + add, the remainder fused
            float sumf = 0.0f;
            const int nv = k & ~3;
            for (int i = 0; i < k; ++i) {
                const float d = s_d8[i * NH + tid];
                sumf = (i < nv) ? sumf + d * s_w[i] : __builtin_fmaf(d, s_w[i], sumf);
            }
            st_local(a.xy + xcd * H + NH * j + tid, tag(sumf, ep), local);
        }

        // ---- Y: all y of this XCD -> RMSNorm -> x of the next layer ----------------
        if (!gather<H / XT>(a, a.xy + xcd * H, H, ep, s_y, tid)) s_fail = 1;
        lds_barrier();
        if (s_fail) return;
        {
            double s = 0.0;
            for (int i = tid; i < H; i += XT) {
                const float v = s_y[i];
                s += (double) (v * v);
            }
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) s_red[wave] = s;
            lds_barrier();
            double tot = 0.0;
            for (int w = 0; w < XW; ++w) tot += s_red[w];
            const float mean = (float) (tot / (double) H);
            const float sc = 1.0f / sqrtf(mean + a.rms_eps);
            for (int i = tid; i < H; i += XT) s_x[i] = s_y[i] * sc;
            if (!nxt && b == 0) {
                for (int i = tid; i < H; i += XT) {
                    a.out[i] = s_y[i];
                    if (a.x_out) a.x_out[i] = s_x[i];
                }
            }
            lds_barrier();
        }
        if (nxt) {
            quant_q8K_xb(s_x, NBH, s_xq, tid);
            const int rw0 = XW - (NLOG + 1) / 2;
            const int hw = 2 * (wave - rw0) + ((lane >> 5) & 1), c = lane & 31;
            if (wave >= rw0 && hw < NLOG) {
                const float lg = router_chain<H>(s_rw + hw * H, s_x, c);
                if (c == 0) st_local(a.xl + xcd * E + NLOG * j + hw, tag(lg, ep + 1), local);
            }
        }
    }
}

namespace {

struct XcdKernel {
    int nbf, nlog;
    const void* fn;
};
const XcdKernel kXcdKernels[] = {
    {3, 4, (const void*) k_decode_xcd<8, 3, 4>},
    {3, 2, (const void*) k_decode_xcd<8, 3, 2>},
    {3, 1, (const void*) k_decode_xcd<8, 3, 1>},
};

}  // namespace

const void* decode_xcd_kernel(const DecodeStackDesc& d) {
    if (d.H != 2048 || d.type_down != T_Q4_K) return nullptr;
    for (const XcdKernel& kk : kXcdKernels)
        if (d.F == 256 * kk.nbf && d.E == 32 * kk.nlog) return kk.fn;
    return nullptr;
}

int launch_decode_xcd(const DecodeStackDesc& d, const float* x_in, float* out, float* x_out, int32_t* ids_out,
                      float* w_out, uint32_t epoch0, hipStream_t stream) {
    XcdArgs a{};
    a.layers = d.layers_dev;
    a.n_layer = d.n_layer;
    a.k = (int) d.k;
    a.scale = d.scale;
    a.rms_eps = d.rms_eps;
    a.x_in = x_in;
    a.out = out;
    a.x_out = x_out;
    a.ids_out = ids_out;
    a.w_out = w_out;
    a.xl = d.xl;
    a.xa = d.xa;
    a.xd = d.xd;
    a.xy = d.xy;
    a.epoch0 = epoch0;
    a.status = d.status;
    a.abort_flag = d.abort_flag;
    a.local_st = d.xcd_local;
    void* args[] = {&a};
    hipError_t e = hipLaunchKernel(decode_xcd_kernel(d), dim3(NXCD * NJ), dim3(XT), args, 0, stream);
    return e == hipSuccess ? 0 : -3;
}

// Records each workgroup's XCD id: used once at create time to check that
// workgroup b of a 256-workgroup launch runs on XCD b % 8.
__global__ void k_xcd_probe(int32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = (int32_t) (__builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xf);
}

int probe_xcd_mapping(int32_t* dev_buf, int n, hipStream_t stream, int* ok) {
    *ok = 0;
    hipLaunchKernelGGL(k_xcd_probe, dim3(n), dim3(64), 0, stream, dev_buf);
    if (hipGetLastError() != hipSuccess) return -3;
    std::vector<int32_t> h((size_t) n);
    if (hipMemcpyAsync(h.data(), dev_buf, sizeof(int32_t) * (size_t) n, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return -3;
    int good = 1;
    for (int i = 0; i < n; ++i)
        if (h[(size_t) i] != i % NXCD) good = 0;
    *ok = good;
    return 0;
}

int check_decode_xcd(const DecodeStackDesc& d, int cus) {
    if (cus != NXCD * NJ || d.k < 1 || d.k > NXCD) return -2;
    const void* fn = decode_xcd_kernel(d);
    if (!fn) return -2;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, XT, 0) != hipSuccess) return -3;
    return per_cu >= 1 ? 0 : -2;
}

}  // namespace qw
