// qw_xcd.hpp -- pieces shared by the persistent decode kernels that give one
// selected expert to each XCD (decode_xcd.hip, decode_xcd_wide.hip): the
// kernel arguments, the tagged exchange words and their polls, wave-wide DPP
// reductions, the Q8_K quantizers into LDS, the Q4_K lane helpers and the
// router chain.
#pragma once

#include "qw_kernels.hpp"
#include "qw_sort.hpp"
#include "qw_decode.hpp"

namespace qw {

namespace {


constexpr int XT = 512;                 // threads per workgroup
constexpr int XW = XT / 64;             // waves
constexpr int NXCD = 8;
constexpr int NJ = 32;                  // workgroups per XCD
constexpr long XSPIN = 1L << 22;        // polls before a wait gives up (~seconds)
// Status bits of a wait that gave up (with 8): which exchange it waited for.
constexpr int XW_LOGITS = 256, XW_ACT = 512, XW_DOWN = 1024, XW_Y = 2048, XW_TOPK = 4096;
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

template <class A>
__device__ __forceinline__ bool x_aborted(const A& a) {
    return (uint32_t) __hip_atomic_load(a.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= a.epoch0;
}
template <class A>
__device__ __forceinline__ void x_abort(const A& a, int bit) {
    atomicOr(a.status, bit);
    __hip_atomic_store(a.abort_flag, (int32_t) a.epoch0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wave-uniform value moved to scalar registers.
__device__ __forceinline__ uint32_t uni32(uint32_t v) { return (uint32_t) __builtin_amdgcn_readfirstlane((int) v); }
__device__ __forceinline__ uint64_t uni64(uint64_t v) {
    return ((uint64_t) uni32((uint32_t) (v >> 32)) << 32) | uni32((uint32_t) v);
}

// Wave-local LDS ordering: every LDS access of this wave issued before has
// completed, and the compiler keeps memory accesses on their side.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Says, at a point where it costs nothing, that every load of this thread has
// returned (vmcnt(0)).  The compiler tracks pending loads per register, and a
// load consumed on one path only (the prefetches of the next layer) stays
// "pending" across the loop back-edge: the next write to its register would
// then wait vmcnt(N), i.e. for the weight loads issued after it.
__device__ __forceinline__ void all_loads_returned() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Polls n tagged words (this thread's: i = tid + XT * m, m < MAXJ) until each
// carries epoch ep, then stores the payloads to dst[i] (LDS).  A sweep reloads
// every word of the thread and keeps the first payload seen with the epoch.
// Returns false if the wait gave up.
template <int MAXJ, class A>
__device__ __forceinline__ bool gather(const A& a, const uint64_t* src, int n, uint32_t ep, float* dst,
                                       int tid, int where) {
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
            x_abort(a, 8 | where);
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

// Wave-wide reductions without the LDS crossbar: an all-reduce inside each
// 16-lane row (DPP xor1, xor2, half-mirror, mirror), then row_bcast:15 and
// row_bcast:31 fold rows 0..3 into lane 63, which readlane makes uniform.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows_f(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_rows_i(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ float wave_max_uniform(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    v = fmaxf(v, dpp_rows_f<0x142, 0xA>(v, v));   // rows 1, 3 <- lane 15 of rows 0, 2
    v = fmaxf(v, dpp_rows_f<0x143, 0xC>(v, v));   // rows 2, 3 <- lane 31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// (|x|, index) of the first largest |x| over the wave, uniform.
__device__ __forceinline__ void wave_argmax_first(float& am, int& ai) {
#define QW_AMAX_STEP(OM, OI)                                        \
    {                                                               \
        const float om = OM;                                        \
        const int oi = OI;                                          \
        if (om > am || (om == am && oi < ai)) { am = om; ai = oi; } \
    }
    QW_AMAX_STEP(dpp_f<DPP_XOR1>(am), dpp_i<DPP_XOR1>(ai))
    QW_AMAX_STEP(dpp_f<DPP_XOR2>(am), dpp_i<DPP_XOR2>(ai))
    QW_AMAX_STEP(dpp_f<DPP_HALF_MIRROR>(am), dpp_i<DPP_HALF_MIRROR>(ai))
    QW_AMAX_STEP(dpp_f<DPP_MIRROR>(am), dpp_i<DPP_MIRROR>(ai))
    QW_AMAX_STEP((dpp_rows_f<0x142, 0xA>(am, am)), (dpp_rows_i<0x142, 0xA>(ai, ai)))
    QW_AMAX_STEP((dpp_rows_f<0x143, 0xC>(am, am)), (dpp_rows_i<0x143, 0xC>(ai, ai)))
#undef QW_AMAX_STEP
    am = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(am), 63));
    ai = __builtin_amdgcn_readlane(ai, 63);
}

// quantize_row_q8_K_ref of nblocks x 256 values x[i] = src[i] * mul (LDS) into
// QB-strided LDS blocks.  Sixteen lanes (one DPP row) per block, sixteen
// consecutive values per lane: the first-index max |x| is a four-step row
// reduction and each lane's values form exactly one bsums group.  Lanes
// [0, 16 * nblocks) of the calling wave(s), numbered by tt, take part.  Block b
// lies at q + QB b + BO with its quants at +QO, d at +DO and bsums at +260
// (defaults: quants first; <12, 4, 0>: ggml's block_q8_K 12 bytes into the slot).
template <int BO = 0, int QO = 0, int DO = 256>
__device__ __forceinline__ void quant_q8K_r16(const float* src, float mul, int nblocks, uint8_t* q, int tt) {
    if (tt < 0 || tt >= 16 * nblocks) return;
    const int b = tt >> 4, l = tt & 15;
    const float* x = src + b * QK_K + 16 * l;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        const float4 t4 = *(const float4*) (x + i);
        v[i] = t4.x * mul;
        v[i + 1] = t4.y * mul;
        v[i + 2] = t4.z * mul;
        v[i + 3] = t4.w * mul;
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
    uint8_t* blk = q + b * QB + BO;
    if (!(am > 0.0f)) {
        *(u32x4*) (blk + QO + 16 * l) = u32x4{0u, 0u, 0u, 0u};
        *(int16_t*) (blk + 260 + 2 * l) = 0;
        if (l == 0) *(float*) (blk + DO) = 0.0f;
        return;
    }
    const float iscale = -127.f / (src[b * QK_K + ai] * mul);
    int s = 0;
    u32x4 words = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int t = nearest_int(iscale * v[i]);
        t = t < 127 ? t : 127;
        s += t;
        words[i >> 2] |= (uint32_t) (t & 0xff) << (8 * (i & 3));
    }
    *(u32x4*) (blk + QO + 16 * l) = words;
    *(int16_t*) (blk + 260 + 2 * l) = (int16_t) s;
    if (l == 0) *(float*) (blk + DO) = 1.0f / iscale;
}

// quantize_row_q8_K_ref (ggml-quants.c:2768-2803) of one 256-value block by one
// wave, four values per lane (v[i] = value 4 * lane + i), into a QB-strided LDS
// block: the first-index max |x| is a wave reduction of (|x|, index), each
// four-lane group's values form one bsums group.  Quants at blk + QO, d at
// blk + DO, bsums at blk + 260.
template <int QO = 0, int DO = 256>
__device__ __forceinline__ void quant_q8K_w64(const float v[4], int lane, uint8_t* blk) {
    float am = 0.0f;
    int ai = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float ax = __builtin_fabsf(v[i]);
        if (ax > am) { am = ax; ai = 4 * lane + i; }
    }
    wave_argmax_first(am, ai);
    if (!(am > 0.0f)) {   // amax == 0: d = 0, qs = 0 (bsums written as 0)
        *(uint32_t*) (blk + QO + 4 * lane) = 0u;
        if ((lane & 3) == 0) *(int16_t*) (blk + 260 + 2 * (lane >> 2)) = 0;
        if (lane == 0) *(float*) (blk + DO) = 0.0f;
        return;
    }
    const int sel = ai & 3;
    const float mine = sel == 0 ? v[0] : sel == 1 ? v[1] : sel == 2 ? v[2] : v[3];
    const float maxv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), ai >> 2));   // the signed value
    const float iscale = -127.f / maxv;
    int s = 0;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int q = nearest_int(iscale * v[i]);
        q = q < 127 ? q : 127;
        s += q;
        w |= (uint32_t) (q & 0xff) << (8 * i);
    }
    *(uint32_t*) (blk + QO + 4 * lane) = w;
    s += dpp_i<DPP_XOR1>(s);
    s += dpp_i<DPP_XOR2>(s);
    if ((lane & 3) == 0) *(int16_t*) (blk + 260 + 2 * (lane >> 2)) = (int16_t) s;
    if (lane == 0) *(float*) (blk + DO) = 1.0f / iscale;
}

// The scale bytes of a Q4_K block (get_scale_min_k4 / the utmp shuffle of
// quants.c:2067-2072): sub-blocks 0..3 from s0, 4..7 from s2 and the top bits
// of s0; mins likewise from s1 / s2.  hi selects the upper four (branch-free).
__device__ __forceinline__ uint32_t q4k_scale_word(uint32_t s0, uint32_t s2, bool hi) {
    const uint32_t lo4 = s0 & 0x3f3f3f3fu;
    const uint32_t hi4 = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
    const uint32_t m = 0u - (uint32_t) hi;
    return lo4 ^ ((lo4 ^ hi4) & m);
}
__device__ __forceinline__ uint32_t q4k_min_word(uint32_t s1, uint32_t s2, bool hi) {
    const uint32_t lo4 = s1 & 0x3f3f3f3fu;
    const uint32_t hi4 = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
    const uint32_t m = 0u - (uint32_t) hi;
    return lo4 ^ ((lo4 ^ hi4) & m);
}

// The weight side of one Q4_K super-block for lane t (0..7) of its 8-lane
// group: hdr = bytes 0..15 (d, dmin, scales), qc = the 16 quant bytes of
// 64-element chunk j = t & 3, half hb = t >> 2 (AVX lanes n = 4 hb + i), at
// block offset q4k_chunk(t).  Lanes t, t ^ 1, t ^ 2, t ^ 3 hold the four
// chunks of one half, so their sum is two quad_perm steps.
__device__ __forceinline__ uint32_t q4k_chunk(int t) { return 16u + 16u * (uint32_t) (2 * (t & 3) + (t >> 2)); }
struct Q4KLane {
    uint32_t lo[4], hi[4];   // the nibbles of qc as bytes (sub-blocks 2j and 2j + 1)
    int scl, sch;            // their scales
    int m0, m1;              // the mins of sub-blocks 2n', 2n' + 1, n' = t & 3 (min lane n')
    float d, dmin;           // fp16 d and dmin as fp32
};
__device__ __forceinline__ Q4KLane q4k_lane(const u32x4& hdr, const u32x4& qc, int t) {
    Q4KLane w;
    const int j = t & 3, n = t & 3;
    const uint32_t scw = q4k_scale_word(hdr[1], hdr[3], j >= 2);
    const int sh = 16 * (j & 1);
    w.scl = (int) __builtin_amdgcn_ubfe(scw, sh, 8);
    w.sch = (int) __builtin_amdgcn_ubfe(scw, sh + 8, 8);
    const uint32_t mw = q4k_min_word(hdr[2], hdr[3], n >= 2);
    w.m0 = (int) __builtin_amdgcn_ubfe(mw, 16 * (n & 1), 8);
    w.m1 = (int) __builtin_amdgcn_ubfe(mw, 16 * (n & 1) + 8, 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w.lo[i] = qc[i] & 0x0F0F0F0Fu;
        w.hi[i] = (qc[i] >> 4) & 0x0F0F0F0Fu;
    }
    w.d = h2f((uint16_t) (hdr[0] & 0xffff));
    w.dmin = h2f((uint16_t) (hdr[0] >> 16));
    return w;
}

// Integer partials of that lane against a Q8_K block (qs at yq in LDS):
// p[i] = sc_{2j} . sum(q4lo . q8) + sc_{2j+1} . sum(q4hi . q8) over AVX lane n's
// four bytes (the maddubs + madd of quants.c:2092-2100).
__device__ __forceinline__ void q4k_dot(const Q4KLane& w, const uint8_t* yq, int t, int p[4]) {
    const int j = t & 3, hb = t >> 2;
    const u32x4 alo = *(const u32x4*) (yq + 64 * j + 16 * hb);
    const u32x4 ahi = *(const u32x4*) (yq + 64 * j + 32 + 16 * hb);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        p[i] = mul24(w.scl, sdot4((int) w.lo[i], (int) alo[i], 0)) + mul24(w.sch, sdot4((int) w.hi[i], (int) ahi[i], 0));
}

// Min lane n = t & 3: mins of sub-blocks 2n, 2n+1 times the Q8_K sums of those
// sub-blocks (_mm_madd_epi16(mins, hadd(bsums)), quants.c:2084-2087).  yb: the
// Q8_K block in LDS (bsums at 260).
__device__ __forceinline__ int q4k_min_dot(const Q4KLane& w, const uint8_t* yb, int t) {
    const int n = t & 3;
    const uint32_t bs01 = *(const uint32_t*) (yb + 260 + 8 * n), bs23 = *(const uint32_t*) (yb + 264 + 8 * n);
    const int q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
    const int q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
    return mul24(w.m0, q8s0) + mul24(w.m1, q8s1);
}

// The activation side of q4k_dot / q4k_min_dot in registers: lane t's 32 quant
// bytes of a Q8_K block and its min lane's two sub-block sums.  Rows that share
// the activation block (every gate/up row of a wave) read LDS once for all.
struct Q8KLane {
    u32x4 alo, ahi;
    int q8s0, q8s1;
};
__device__ __forceinline__ Q8KLane q8k_lane(const uint8_t* yb, int t) {
    Q8KLane y;
    const int j = t & 3, hb = t >> 2, n = t & 3;
    y.alo = *(const u32x4*) (yb + 64 * j + 16 * hb);
    y.ahi = *(const u32x4*) (yb + 64 * j + 32 + 16 * hb);
    const uint32_t bs01 = *(const uint32_t*) (yb + 260 + 8 * n), bs23 = *(const uint32_t*) (yb + 264 + 8 * n);
    y.q8s0 = (int) (int16_t) (bs01 & 0xffff) + (int) (int16_t) (bs01 >> 16);
    y.q8s1 = (int) (int16_t) (bs23 & 0xffff) + (int) (int16_t) (bs23 >> 16);
    return y;
}
__device__ __forceinline__ void q4k_dot(const Q4KLane& w, const Q8KLane& y, int p[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        p[i] = mul24(w.scl, sdot4((int) w.lo[i], (int) y.alo[i], 0)) + mul24(w.sch, sdot4((int) w.hi[i], (int) y.ahi[i], 0));
}
__device__ __forceinline__ int q4k_min_dot(const Q4KLane& w, const Q8KLane& y) {
    return mul24(w.m0, y.q8s0) + mul24(w.m1, y.q8s1);
}

// Sum over the four 64-element chunks: lanes t ^ 1, then t ^ 2 (quad_perm; the
// sums are exact integers).  Every lane of a half ends with the sums of its AVX
// lanes 4 hb .. 4 hb + 3.
__device__ __forceinline__ void reduce_chunks(int p[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int a = p[i] + dpp_i<DPP_XOR1>(p[i]);
        p[i] = a + dpp_i<DPP_XOR2>(a);
        // materialised here: an add sunk into a lane-conditional store would
        // keep its DPP operand as a separate v_mov_dpp
        asm volatile("" : "+v"(p[i]));
    }
}

// Router logit of x = y * sc (the RMSNorm, formed value by value); lane c < 32
// of a half-wave is chain c of AVX2 ggml_vec_dot_f32 (GGML_F32_STEP 32) and
// holds that chain's router weights w[s] = W[e][c + 32 s] in registers; then the
// reduction tree of that function; lane 0 returns the logit.  x is read from
// LDS sixteen steps at a time, the next sixteen in flight during the fmas.
template <int H>
__device__ __forceinline__ float router_chain(const float (&w)[H / 32], const float* y, float sc, int c) {
    float acc = 0.0f;
    float xv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) xv[u] = y[32 * u + c];
#pragma unroll
    for (int s0 = 0; s0 < H / 32; s0 += 16) {
        float xn[16];
        const int s1 = s0 + 16 < H / 32 ? s0 + 16 : s0;   // (the last round reloads its own)
#pragma unroll
        for (int u = 0; u < 16; ++u) xn[u] = y[32 * (s1 + u) + c];
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = __builtin_fmaf(w[s0 + u], xv[u] * sc, acc);
#pragma unroll
        for (int u = 0; u < 16; ++u) xv[u] = xn[u];
    }
    float t = acc + __shfl_down(acc, 16, 32);   // c_l + c_{16+l}
    t = t + __shfl_down(t, 8, 32);               // (c_l + c_{16+l}) + (c_{8+l} + c_{24+l})
    t = t + __shfl_down(t, 4, 32);               // t0_l = s_l + s_{l+4}
    const float u = t + __shfl_down(t, 1, 32);
    return u + __shfl_down(u, 2, 32);            // (t0_0 + t0_1) + (t0_2 + t0_3)
}

// The same chain with the router row in LDS (w[i] = W[e][i]): sixteen steps of
// w and x read together, then their fmas.
template <int H>
__device__ __forceinline__ float router_chain_lds(const float* w, const float* y, float sc, int c) {
    float acc = 0.0f;
#pragma unroll
    for (int s0 = 0; s0 < H / 32; s0 += 16) {
        float xv[16], wv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            xv[u] = y[32 * (s0 + u) + c];
            wv[u] = w[32 * (s0 + u) + c];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = __builtin_fmaf(wv[u], xv[u] * sc, acc);
    }
    float t = acc + __shfl_down(acc, 16, 32);
    t = t + __shfl_down(t, 8, 32);
    t = t + __shfl_down(t, 4, 32);
    const float u = t + __shfl_down(t, 1, 32);
    return u + __shfl_down(u, 2, 32);
}

// std::sort's order of tied probabilities (qw_sort.hpp), kept out of line: the
// replay runs only when ties reach into the top k.
__device__ __attribute__((noinline)) void sort_desc_replay(int32_t* order, int n, const float* p, SortRange* stack) {
    libstdcxx_sort_desc(order, n, p, stack);
}

// A float held by lane id & 63 of register (id >> 6) of a two-register array,
// read by every lane (id uniform).
__device__ __forceinline__ float lane_value(const float v[2], int id) {
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[0]), id & 63));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[1]), id & 63));
    return id < 64 ? a : b;
}

}  // namespace

}  // namespace qw
