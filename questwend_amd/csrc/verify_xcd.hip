// verify_xcd.hip -- persistent MoE FFN stack for a batch of T <= 8 tokens (the
// verify forward of MTP speculative decoding: Runtime::decode_verify runs the
// T = n_draft + 1 tokens of a draft through every layer at once,
// core/runtime.cpp:1495-1562; each build_moe sees a T-token batch, 861-974).
// One launch runs all layers, on a 256-CU device, at H = 2048, F = 768, E <= 128,
// Q4_K gate/up/down (the Qwen3-30B-A3B shape).
//
// Per layer the T tokens select T x k (token, expert) pairs; the distinct experts
// of the batch (its union, in increasing id) are dealt to the XCDs round robin:
// union expert u goes to XCD u % 8 as its slot u / 8.  Each XCD loads the rows of
// each of its experts once and applies them to every token routed there, which
// is what makes a batch cheaper than T decode tokens.  Inside an XCD the work is
// decode_xcd.hip's: 32 workgroups split an expert's gate/up pairs (eight lanes
// per Q4_K super-block, the fp32 chains of ggml's eight AVX lanes) and its down
// rows.  Exchanges (tagged words, qw_xcd.hpp):
//   L  every XCD computes the T x E router logits (E/32 experts per workgroup,
//      its router rows in registers) and all-gathers them inside the XCD;
//   A  act of (slot, token), inside the XCD;
//   D  down outputs of (union expert, token), across XCDs;
//   Y  workgroup j forms y[t][h] for its H/32 rows -- build_moe's T > 1 weighted
//      sum, products then an add chain in slot order (940-959) -- and every XCD
//      all-gathers y; RMSNorm per token.
// Top-k per token is exact: wave t ranks token t's logits, takes the ranked
// order when decode_xcd.hip's check proves it is argsort's, else ranks the
// probabilities and replays std::sort on a tie.  Ids, weights and outputs are
// bit-identical to the reference CPU path.
#include "qw_xcd.hpp"
#include "qw_verify.hpp"

#include <vector>

namespace qw {

namespace {

constexpr int VTM = VERIFY_TMAX;          // tokens per batch, at most
constexpr int VU = VTM * 8;               // union experts, at most (k <= 8)
constexpr int VSL = VU / NXCD;            // slots per XCD, at most

// ggml_soft_max of one token's E logits (ops.cpp:5455-5566) by one wave: lane
// holds logits lane and lane + 64; max, ggml_v_expf, sums of eight
// (hsum_float_8) added in double, scale by 1 / sum.
template <int E>
__device__ __forceinline__ void wave_probs(const float* P, int lane, float (&pv)[2]) {
    float lv[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) lv[m] = lane + 64 * m < E ? P[lane + 64 * m] : -INFINITY;
    const float mx = wave_max_uniform(fmaxf(lv[0], lv[1]));
    float ev[2], gs[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        ev[m] = lane + 64 * m < E ? v_expf(lv[m] - mx) : 0.0f;
        const float r = ev[m] + dpp_f<0x104>(ev[m]);   // row_shl:4
        const float r2 = r + dpp_f<0x102>(r);          // row_shl:2
        gs[m] = r2 + dpp_f<0x101>(r2);                  // row_shl:1
    }
    double sum = 0.0;
#pragma unroll
    for (int gi = 0; gi < E / 8; ++gi)
        sum += (double) __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs[gi >> 3]), 8 * (gi & 7)));
    const float inv = (float) (1.0 / sum);
    pv[0] = ev[0] * inv;
    pv[1] = ev[1] * inv;
}

}  // namespace

// NBH = H / 256 (8), NBF = F / 256 (3), NLOG = E / 32.
template <int NBH, int NBF, int NLOG>
__global__ void __launch_bounds__(XT) k_verify_xcd(VerifyArgs a) {
    constexpr int H = NBH * QK_K, F = NBF * QK_K, E = NLOG * 32;
    constexpr int NP = F / NJ;            // (gate, up) pairs per workgroup
    constexpr int PPW = NP / XW;          // pairs per wave
    constexpr int NH = H / NJ;            // down rows per workgroup
    constexpr int RW = NH / XW;           // down rows per wave (one per 8-lane group)
    constexpr int RW0 = XW - (NLOG + 1) / 2;   // first router wave (two logits per router wave)
    constexpr int TRS = NBH * 16 + 8;               // words per record row (8 past a multiple of the 64 banks)
    constexpr int NTR = XW * 2 * PPW * TRS;         // words of the gate/up block records
    static_assert(NBH == 8, "gate/up rows: one super-block per 8-lane group");
    static_assert(PPW >= 1 && PPW * XW == NP && 2 * PPW * 8 <= 64, "pairs per wave");
    static_assert(RW == 8 && NH == 64, "down rows: one row per 8-lane group; y: one row per lane");
    static_assert(E <= 128 && E % 32 == 0, "logits: two per lane in the per-token softmax");
    static_assert(VTM <= XW, "top-k and y: a wave per token");
    static_assert(NTR + VTM * F + VTM * NBF * QB / 4 <= VTM * H, "records, act and Q8_K(act) fit in the y buffer");

    // y of the last layer [T][H] (from the y exchange to the next layer's router);
    // during a layer the same memory holds the gate/up block records, the act rows
    // of one slot and their Q8_K
    __shared__ __align__(16) float s_big[VTM * H];
    uint32_t* const s_tr = (uint32_t*) s_big;                     // [XW][2 PPW][TRS]: 16 words per block
    float* const s_act = s_big + NTR;                             // [VTM][F] (the slot's tokens in order)
    uint8_t* const s_aq = (uint8_t*) (s_act + VTM * F);           // [VTM][NBF * QB]
    __shared__ __align__(16) uint8_t s_xq[VTM][NBH * QB];         // Q8_K(x) per token
    __shared__ __align__(16) float s_p[VTM][E];                   // logits
    __shared__ __align__(16) float s_pe[VTM][E];                  // the exact path's probabilities
    __shared__ __align__(16) int32_t s_order[VTM][E];
    __shared__ __align__(16) int4 s_slotx[2][E];                  // {gate, up, down} slot of each expert
    __shared__ SortRange s_stack[VTM][SORT_STACK];
    __shared__ int32_t s_sel[VTM][8];                             // selected experts of each token, rank order
    __shared__ float s_selw[VTM][8];                              // their weights
    __shared__ int32_t s_u[VTM][8];                               // their union index
    __shared__ int32_t s_uexp[VU];                                // union expert u
    __shared__ int32_t s_uidx[E];                                 // union index of expert e, or -1
    __shared__ int32_t s_utok[VU];                                // tokens routed to union expert u (bits)
    __shared__ uint64_t s_L[2][XLW];
    __shared__ double s_red[XW][VTM];
    __shared__ float s_sc[VTM];
    __shared__ int s_fail, s_U;

    const int b = blockIdx.x, tid0 = threadIdx.x;
    const int xcd = (int) (__builtin_amdgcn_s_getreg((3 << 11) | 20) & (NXCD - 1)), j = b >> 3;
    const int k = a.k, T = a.T;
    const int local = a.local_st;

    // The end of a layer (and the prologue): the next layer's router logits of
    // every token from x = y * sc (router waves; the chains of one token after
    // another) and Q8_K(x) (waves 0 .. RW0 - 1, sixteen lanes per block).
    float rw[H / 32];
    auto load_router = [&](const float* router, int tid) {
        const int wave = tid >> 6, lane = tid & 63;
        const int hw = 2 * (wave - RW0) + ((lane >> 5) & 1), c = lane & 31;
        if (router && wave >= RW0 && hw < NLOG) {
            const float* src = router + (size_t) (NLOG * j + hw) * H + c;
#pragma unroll
            for (int s2 = 0; s2 < H / 32; ++s2) rw[s2] = *(const __attribute__((address_space(1))) float*) (src + 32 * s2);
        } else {
            // (defined on every path: otherwise the registers are carried around the
            // layer loop and the slot buffers spill)
#pragma unroll
            for (int s2 = 0; s2 < H / 32; ++s2) rw[s2] = 0.0f;
        }
    };
    auto next_x = [&](int tid, uint32_t ep_next) {
        const int wave = tid >> 6, lane = tid & 63;
        if (wave >= RW0) {
            const int hw = 2 * (wave - RW0) + ((lane >> 5) & 1), c = lane & 31;
            if (hw < NLOG)
                for (int t = 0; t < T; ++t) {
                    const float lg = router_chain<H>(rw, s_big + t * H, s_sc[t], c);
                    if (c == 0) st_local(a.xl + ((size_t) xcd * VTM + t) * E + NLOG * j + hw, tag(lg, ep_next), local);
                }
        } else {
            constexpr int LPT = 16 * NBH;                 // lanes per token
            constexpr int TPP = (64 * RW0) / LPT;         // tokens per pass
            for (int t0 = 0; t0 < T; t0 += TPP) {
                const int t = t0 + tid / LPT;
                if (tid / LPT < TPP && t < T) quant_q8K_r16(s_big + t * H, s_sc[t], NBH, s_xq[t], tid % LPT);
            }
        }
    };

    // ---- prologue: descriptors, x of layer 0, router rows and slot rows of layer 0
    if (tid0 == 0) s_fail = 0;
    if (tid0 < 2 * XLW && tid0 / XLW < a.n_layer) s_L[tid0 / XLW][tid0 % XLW] = ldg64((const uint64_t*) a.layers + tid0);
    for (int i = tid0; i < T * H; i += XT) s_big[i] = a.x_in[i];   // layer 0 takes x_in as it is (sc = 1)
    if (tid0 < VTM) s_sc[tid0] = 1.0f;
    {
        const DecodeLayer& L0 = a.layers[0];
        load_router(L0.router, tid0);
        for (int i = tid0; i < 3 * E; i += XT) {
            const int32_t* so = i < E ? L0.slot_gate : i < 2 * E ? L0.slot_up : L0.slot_down;
            ((int32_t*) &s_slotx[0][i % E])[i / E] = so ? ldg32(so + i % E) : i % E;
        }
    }
    __syncthreads();
    next_x(tid0, a.epoch0);

    for (int l = 0; l < a.n_layer; ++l) {
        const DecodeLayer& L = *(const DecodeLayer*) s_L[l & 1];
        const uint32_t ep = a.epoch0 + (uint32_t) l;
        const int tid = opaque(tid0);
        const int wave = tid >> 6, lane = tid & 63, g = lane >> 3, t8 = lane & 7;

        all_loads_returned();
        const uint8_t* const Lgate = (const uint8_t*) uni64((uint64_t) L.gate);
        const uint8_t* const Lup = (const uint8_t*) uni64((uint64_t) L.up);
        const uint8_t* const Ldown = (const uint8_t*) uni64((uint64_t) L.down);
        const uint32_t gnb1 = uni32((uint32_t) L.gate_nb1), unb1 = uni32((uint32_t) L.up_nb1);
        const uint32_t dnb1 = uni32((uint32_t) L.down_nb1);
        const uint64_t gnb2 = uni64(L.gate_nb2), unb2 = uni64(L.up_nb2), dnb2 = uni64(L.down_nb2);
        const uint32_t nsg = uni32((uint32_t) min(L.n_slots_gate, (int64_t) INT32_MAX));
        const uint32_t nsu = uni32((uint32_t) min(L.n_slots_up, (int64_t) INT32_MAX));
        const uint32_t nsd = uni32((uint32_t) min(L.n_slots_down, (int64_t) INT32_MAX));

        // ---- L: the T x E logits (this XCD's router workgroups) --------------------
        if (!gather<(VTM * E + XT - 1) / XT>(a, a.xl + (size_t) xcd * VTM * E, T * E, ep, &s_p[0][0], tid, XW_LOGITS))
            s_fail = 1;
        lds_barrier();
        if (s_fail) return;

        // ---- top-k of token `wave` (waves 0 .. T-1) -----------------------------------
        if (wave < T) {
            const int tk = wave;
            const float* P = s_p[tk];
            // the k + 1 largest logits by repeated wave maxima: lane r ends with the
            // logit of rank r and (r < k) its expert; a value held twice among the
            // first k, or a NaN anywhere, sends the token to the exact path
            float v0 = lane < E ? P[lane] : -INFINITY, v1 = lane + 64 < E ? P[lane + 64] : -INFINITY;
            bool uniq = !__any(v0 != v0 || v1 != v1);
            float lr = 0.0f;
            int spec_i = 0;
            for (int r = 0; r <= k; ++r) {
                const float m = wave_max_uniform(fmaxf(v0, v1));
                const uint64_t b0 = __ballot(v0 == m), b1 = __ballot(v1 == m);
                if (r < k && __popcll(b0) + __popcll(b1) != 1) uniq = false;
                const int i = b0 ? (int) __builtin_ctzll(b0) : 64 + (int) __builtin_ctzll(b1);
                if (lane == r) {
                    lr = m;
                    spec_i = i;
                }
                if (i < 64) v0 = lane == i ? -INFINITY : v0;
                else v1 = lane == i - 64 ? -INFINITY : v1;
            }
            // decode_xcd.hip's proof that the ranked order is argsort's
            bool ok = uniq;
            const float er = v_expf(lr - __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lr), 0)));
            const float en = dpp_f<0x101>(er);   // row_shl:1: lane r <- r + 1 (r <= 8)
            bool bad = lane < k && !(er > en * 0x1.00001p+0f);
            if (lane == k - 1 && !(er >= 0x1p-100f)) bad = true;
            ok = ok && !__any(bad);
            float pv[2];
            wave_probs<E>(P, lane, pv);
            int sel_id;
            if (ok) {
                sel_id = __shfl(spec_i, lane & 7);
            } else {
                // exact order: rank the probabilities; a tie or NaN inside the first k
                // places leaves the order to std::sort, which is replayed exactly
                if (lane < E) s_pe[tk][lane] = pv[0];
                if (lane + 64 < E) s_pe[tk][lane + 64] = pv[1];
                wave_lds_sync();
                bool tie = false;
#pragma unroll 1
                for (int m = 0; m < 2; ++m) {
                    const int i = lane + 64 * m;
                    const float pi = i < E ? (m ? pv[1] : pv[0]) : 0.0f;   // (no dynamic index: it would live in scratch)
                    int gt = 0, eq = 0;
#pragma unroll 2
                    for (int jj = 0; jj < E; jj += 4) {
                        const float4 q = *(const float4*) (s_pe[tk] + jj);
                        gt += (q.x > pi) + (q.y > pi) + (q.z > pi) + (q.w > pi);
                        eq += (q.x == pi) + (q.y == pi) + (q.z == pi) + (q.w == pi);
                    }
                    if (i < E && gt < k) {
                        if (eq != 1) tie = true;
                        else s_order[tk][gt] = i;
                    }
                }
                if (__any(tie)) {
                    wave_lds_sync();
                    for (int i = lane; i < E; i += 64) s_order[tk][i] = i;
                    wave_lds_sync();
                    if (lane == 0) {
                        sort_desc_replay(s_order[tk], E, s_pe[tk], s_stack[tk]);
                        if (b == 0) atomicOr(a.status, 1);
                    }
                }
                wave_lds_sync();
                sel_id = s_order[tk][lane & 7];
            }
            // weights: selected probabilities / clamp(sum) (* scale), core/runtime.cpp:887-897
            const float pa = __shfl(pv[0], sel_id & 63), pb = __shfl(pv[1], sel_id & 63);
            const float pr = sel_id < 64 ? pa : pb;
            double sp = 0.0;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (r < k) sp += (double) __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr), r));
            float wsum = (float) sp;
            wsum = fmaxf(fminf(wsum, INFINITY), 6.103515625e-5f);
            float sel_w = pr / wsum;
            if (a.scale != 0.0f && a.scale != 1.0f) sel_w = sel_w * a.scale;
            if (lane < k) {
                s_sel[tk][lane] = sel_id;
                s_selw[tk][lane] = sel_w;
                if (b == 0) {
                    if (a.ids_out) {
                        a.ids_out[((size_t) l * T + tk) * k + lane] = sel_id;
                        a.w_out[((size_t) l * T + tk) * k + lane] = sel_w;
                    }
                    const int4 sl = s_slotx[l & 1][sel_id];
                    if ((uint32_t) sl.x >= nsg || (uint32_t) sl.y >= nsu || (uint32_t) sl.z >= nsd) atomicOr(a.status, 16);
                }
            }
        }
        lds_barrier();

        // ---- the batch's distinct experts, in increasing id (wave 0) -----------------
        if (wave == 0) {
            if (lane < E) s_uidx[lane] = -1;
            if (lane + 64 < E) s_uidx[lane + 64] = -1;
            wave_lds_sync();
            if (lane < T * k) s_uidx[s_sel[lane / k][lane % k]] = 0;
            wave_lds_sync();
            const bool m0 = lane < E && s_uidx[lane] == 0, m1 = lane + 64 < E && s_uidx[lane + 64] == 0;
            const uint64_t b0 = __ballot(m0), b1 = __ballot(m1);
            const uint64_t below = (1ull << lane) - 1ull;
            const int n0 = __popcll(b0);
            const int u0 = __popcll(b0 & below), u1 = n0 + __popcll(b1 & below);
            wave_lds_sync();
            if (lane < E) s_uidx[lane] = m0 ? u0 : -1;
            if (lane + 64 < E) s_uidx[lane + 64] = m1 ? u1 : -1;
            if (m0) s_uexp[u0] = lane;
            if (m1) s_uexp[u1] = lane + 64;
            const int U = n0 + __popcll(b1);
            if (lane < U) s_utok[lane] = 0;
            if (lane == 0) s_U = U;
            wave_lds_sync();
            if (lane < T * k) {
                const int tk = lane / k, c = lane % k;
                const int u = s_uidx[s_sel[tk][c]];
                s_u[tk][c] = u;
                atomicOr(&s_utok[u], 1 << tk);
            }
        }
        lds_barrier();
        const int U = s_U;

        // Slots of this XCD: union experts u = xcd + 8 s < U, processed in order; the
        // next slot's rows are loaded while the current slot is computed.
        int nslot = 0;
        while (nslot < VSL && xcd + NXCD * nslot < U) ++nslot;

        // ---- A: gate/up of each slot's expert, applied to its tokens -------------------
        // rows: pair PPW wave + p (gate, up), block g of each: header and chunk t8
        auto issue_gu = [&](int s, u32x4 (&gh)[2 * PPW], u32x4 (&gq)[2 * PPW]) {
            const int4 sl = s_slotx[l & 1][s_uexp[xcd + NXCD * s]];
            uint32_t sg = (uint32_t) __builtin_amdgcn_readfirstlane(sl.x), su = (uint32_t) __builtin_amdgcn_readfirstlane(sl.y);
            sg = sg < nsg ? sg : 0u;   // (a slot out of range reads slot 0; reported above)
            su = su < nsu ? su : 0u;
            const uint8_t* bg = Lgate + (uint64_t) sg * gnb2;
            const uint8_t* bu = Lup + (uint64_t) su * unb2;
#pragma unroll
            for (int p = 0; p < PPW; ++p) {
                const uint32_t f = (uint32_t) (NP * j + PPW * wave + p);
                const uint32_t og = f * gnb1 + 144u * (uint32_t) g, ou = f * unb1 + 144u * (uint32_t) g;
                gh[2 * p] = ldg16(bg + og);
                gq[2 * p] = ldg16(bg + og + q4k_chunk(t8));
                gh[2 * p + 1] = ldg16(bu + ou);
                gq[2 * p + 1] = ldg16(bu + ou + q4k_chunk(t8));
            }
        };
        auto compute_gu = [&](int s, const u32x4 (&gh)[2 * PPW], const u32x4 (&gq)[2 * PPW]) {
            const uint32_t tm = (uint32_t) s_utok[xcd + NXCD * s];
            for (uint32_t rem = tm; rem; rem &= rem - 1u) {
                const int tk = __builtin_ctz(rem);
                const uint8_t* xq = s_xq[tk];
                const Q8KLane yv = q8k_lane(xq + QB * g, t8);   // block g of the token's Q8_K(x), for every row
#pragma unroll
                for (int r = 0; r < 2 * PPW; ++r) {
                    int p[4];
                    const Q4KLane w = q4k_lane(gh[r], gq[r], t8);
                    q4k_dot(w, yv, p);
                    reduce_chunks(p);
                    const int pm = q4k_min_dot(w, yv);
                    uint32_t* rec = s_tr + (wave * 2 * PPW + r) * TRS + 16 * g;
                    // every lane stores two words (rec[t8] = AVX lane t8's sum, rec[8 + t8] = min
                    // lane t8's term, d, dmin): no lane-conditional stores
                    const int q = t8 & 3;
                    const int pt = q == 0 ? p[0] : q == 1 ? p[1] : q == 2 ? p[2] : p[3];
                    rec[t8] = (uint32_t) pt;
                    rec[8 + t8] = t8 < 4 ? (uint32_t) pm : t8 == 4 ? fbits(w.d) : fbits(w.dmin);
                }
                wave_lds_sync();
                // chain lanes: row r = lane >> 3 (< 2 PPW), AVX lane n = lane & 7
                float res;
                {
                    const int r = g < 2 * PPW ? g : 0, n = t8;
                    float acc = 0.0f, accm = 0.0f;
#pragma unroll
                    for (int bb = 0; bb < NBH; ++bb) {
                        const uint32_t* rec = s_tr + (wave * 2 * PPW + r) * TRS + 16 * bb;
                        const int S = (int) rec[n];
                        const int pm = (int) rec[8 + (n & 3)];
                        const float wd = bitsf(rec[12]), wdm = bitsf(rec[13]);
                        const float yd = *(const float*) (xq + QB * bb + 256);
                        acc = __builtin_fmaf(yd * wd, (float) S, acc);
                        const float pmv = __builtin_fmaf(-yd * wdm, (float) pm, accm);
                        accm = n < 4 ? pmv : accm;
                    }
                    // hsum_float_8 and the min lanes into lane 8r: row_shl inside the 16-lane
                    // row (DPP), the same pairs as ggml's tree
                    float s2 = acc;
                    s2 = s2 + dpp_f<0x104>(s2);
                    s2 = s2 + dpp_f<0x102>(s2);
                    s2 = s2 + dpp_f<0x101>(s2);
                    float m = accm;
                    m = m + dpp_f<0x102>(m);
                    m = m + dpp_f<0x101>(m);
                    res = s2 + m;
                }
                const float up = dpp_f<0x108>(res);     // lane 16p: gate of pair p; lane 16p + 8: its up
                if ((lane & 15) == 0 && (lane >> 4) < PPW) {
                    const int f = NP * j + PPW * wave + (lane >> 4);
                    st_local(a.xa + (((size_t) xcd * VSL + s) * VTM + tk) * F + f, tag(v_silu(res) * up, ep), local);
                }
                wave_lds_sync();   // the records are read before the next token's are written
            }
        };
        // Two register sets, A for even slots and B for odd ones (the loop unrolled by
        // two): slot s + 2's rows are issued into the set slot s used as soon as slot s
        // is computed, while slot s + 1's are still in flight, so two slots' rows are
        // in flight at a time.  (Copying the next slot's set into the current one after
        // each slot waited for the next slot's loads before the one after could be
        // issued: one slot in flight.)  Each set is defined on both arms of its
        // condition (a set left undefined on one arm is carried around the loops by the
        // compiler, and spills).
        auto zero_gu = [&](u32x4 (&gh)[2 * PPW], u32x4 (&gq)[2 * PPW]) {
#pragma unroll
            for (int r = 0; r < 2 * PPW; ++r) gh[r] = gq[r] = u32x4{0u, 0u, 0u, 0u};
        };
        if (nslot > 0) {
            u32x4 ghA[2 * PPW], gqA[2 * PPW], ghB[2 * PPW], gqB[2 * PPW];
            issue_gu(0, ghA, gqA);
            if (nslot > 1) issue_gu(1, ghB, gqB);
            else zero_gu(ghB, gqB);
            for (int s = 0; s < nslot; s += 2) {
                compute_gu(s, ghA, gqA);
                if (s + 2 < nslot) issue_gu(s + 2, ghA, gqA);
                else zero_gu(ghA, gqA);
                if (s + 1 >= nslot) break;
                compute_gu(s + 1, ghB, gqB);
                if (s + 3 < nslot) issue_gu(s + 3, ghB, gqB);
                else zero_gu(ghB, gqB);
            }
        }

        // ---- D: per slot, its tokens' act -> Q8_K -> down rows -------------------------
        // down row RW wave + g of the slot's expert: header and chunk t8 of each block
        auto issue_dn = [&](int s, u32x4 (&dh)[NBF], u32x4 (&dq)[NBF]) {
            uint32_t sd = (uint32_t) __builtin_amdgcn_readfirstlane(s_slotx[l & 1][s_uexp[xcd + NXCD * s]].z);
            sd = sd < nsd ? sd : 0u;
            const uint8_t* rd = Ldown + (uint64_t) sd * dnb2 + (uint32_t) (NH * j + RW * wave + g) * dnb1;
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) {
                dh[bb] = ldg16(rd + 144 * bb);
                dq[bb] = ldg16(rd + 144 * bb + q4k_chunk(t8));
            }
        };
        // down rows of slot s for its tokens, whose Q8_K(act) rows are s_aq rows i0, i0 + 1, ...
        auto compute_dn = [&](int s, const u32x4 (&dh)[NBF], const u32x4 (&dq)[NBF], int i0) {
            const int u = xcd + NXCD * s;
            const uint32_t tm = (uint32_t) s_utok[u];
            Q4KLane dw[NBF];
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) dw[bb] = q4k_lane(dh[bb], dq[bb], t8);
            int i = i0;
            for (uint32_t rem = tm; rem; rem &= rem - 1u, ++i) {
                const int tk = __builtin_ctz(rem);
                float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                float accm = 0.0f;
#pragma unroll
                for (int bb = 0; bb < NBF; ++bb) {
                    const uint8_t* yb = s_aq + (i * NBF + bb) * QB;
                    int p[4];
                    q4k_dot(dw[bb], yb, t8, p);
                    reduce_chunks(p);
                    const float yd = *(const float*) (yb + 256);
                    const float D = yd * dw[bb].d;
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[c] = __builtin_fmaf(D, (float) p[c], acc[c]);
                    const int pm = q4k_min_dot(dw[bb], yb, t8);
                    accm = __builtin_fmaf(-yd * dw[bb].dmin, (float) pm, accm);
                }
                // hsum_float_8: lane t8 = 0 holds AVX lanes 0..3, lane t8 = 4 lanes 4..7
                float r4[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) r4[c] = acc[c] + dpp_f<0x12C>(acc[c]);   // row_ror:12
                const float hs = (r4[0] + r4[2]) + (r4[1] + r4[3]);
                const float m2 = accm + dpp_f<DPP_XOR2>(accm);
                const float mm = m2 + dpp_f<DPP_XOR1>(m2);
                if (t8 == 0)
                    st_cross(a.xd + (((size_t) (l & 1) * VU + u) * VTM + tk) * H + NH * j + RW * wave + g, tag(hs + mm, ep));
            }
        };
        auto zero_dn = [&](u32x4 (&dh)[NBF], u32x4 (&dq)[NBF]) {
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) dh[bb] = dq[bb] = u32x4{0u, 0u, 0u, 0u};
        };
        if (nslot > 0) {
            u32x4 dhc[NBF], dqc[NBF], dhn[NBF], dqn[NBF];
            issue_dn(0, dhc, dqc);
            if (nslot > 1) issue_dn(1, dhn, dqn);
            else zero_dn(dhn, dqn);
            // batches of slots whose (slot, token) pairs fit the VTM act rows: one act
            // exchange and one quantisation per batch, then the slots' down rows in turn
            for (int sb = 0; sb < nslot;) {
                int se = sb, np = 0;
                while (se < nslot && np + __popc((uint32_t) s_utok[xcd + NXCD * se]) <= VTM)
                    np += __popc((uint32_t) s_utok[xcd + NXCD * se++]);
                int i = 0;
                for (int s = sb; s < se; ++s)
                    for (uint32_t rem = (uint32_t) s_utok[xcd + NXCD * s]; rem; rem &= rem - 1u, ++i) {
                        const int tk = __builtin_ctz(rem);
                        if (!gather<(F + XT - 1) / XT>(a, a.xa + (((size_t) xcd * VSL + s) * VTM + tk) * F, F, ep,
                                                       s_act + i * F, tid, XW_ACT))
                            s_fail = 1;
                    }
                lds_barrier();
                if (s_fail) return;
                for (int q = wave; q < np * NBF; q += XW) {
                    const int r = q / NBF, bb = q - r * NBF;
                    const float4 v4 = *(const float4*) (s_act + r * F + QK_K * bb + 4 * lane);
                    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
                    quant_q8K_w64(v, lane, s_aq + (r * NBF + bb) * QB);
                }
                lds_barrier();
                int i0 = 0;
                for (int s = sb; s < se; ++s) {
                    compute_dn(s, dhc, dqc, i0);
                    i0 += __popc((uint32_t) s_utok[xcd + NXCD * s]);
#pragma unroll
                    for (int bb = 0; bb < NBF; ++bb) {
                        dhc[bb] = dhn[bb];
                        dqc[bb] = dqn[bb];
                    }
                    if (s + 2 < nslot) issue_dn(s + 2, dhn, dqn);
                    else zero_dn(dhn, dqn);
                }
                lds_barrier();   // s_act / s_aq are read before the next batch's are written
                sb = se;
            }
        }

        // next layer's router rows (registers), slot rows and the descriptor of layer l + 2
        const bool nxt = l + 1 < a.n_layer;
        const DecodeLayer& L1 = *(const DecodeLayer*) s_L[(l + 1) & 1];
        int32_t sl_next = 0;
        if (tid < 3 * E) {
            const int32_t* so = !nxt ? nullptr : tid < E ? L1.slot_gate : tid < 2 * E ? L1.slot_up : L1.slot_down;
            sl_next = so ? ldg32(so + tid % E) : tid % E;
        }
        const bool next2 = l + 2 < a.n_layer && tid < XLW;
        const uint64_t lw = ldg64((const uint64_t*) (a.layers + (next2 ? l + 2 : l)) + (tid % XLW));
        load_router(nxt ? L1.router : nullptr, tid);   // (rw defined on both paths: see load_router)

        // ---- D -> y[t][h]: wave t, lane h; build_moe's T > 1 sum: products, then an add
        // chain in slot order ------------------------------------------------------------
        if (wave < T) {
            const int tk = wave;
            const uint64_t* src = a.xd + ((size_t) (l & 1) * VU * VTM + tk) * H + NH * j + lane;
            int uu[8];
            float wc[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                uu[c] = c < k ? s_u[tk][c] : 0;
                wc[c] = c < k ? s_selw[tk][c] : 0.0f;
            }
            float dv[8];
            uint32_t got = 0;
            const uint32_t all = (1u << k) - 1u;
            long spins = 0;
            while (got != all) {
                uint64_t v[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) v[c] = poll64(src + (size_t) uu[c] * VTM * H);
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    if (c < k && !(got & (1u << c)) && (uint32_t) (v[c] >> 32) == ep) {
                        dv[c] = bitsf((uint32_t) v[c]);
                        got |= 1u << c;
                    }
                if (got == all) break;
                if (++spins > XSPIN) {
                    x_abort(a, 8 | XW_DOWN);
                    break;
                }
                if ((spins & 255) == 0 && x_aborted(a)) break;
                __builtin_amdgcn_s_sleep(1);
            }
            if (got != all) s_fail = 1;
            else {
                float y = dv[0] * wc[0];
#pragma unroll
                for (int c = 1; c < 8; ++c)
                    if (c < k) y = y + dv[c] * wc[c];
                st_local(a.xy + ((size_t) xcd * VTM + tk) * H + NH * j + lane, tag(y, ep), local);
            }
        }

        // ---- Y: all y of this XCD, RMSNorm per token (sums of squares in double) -------
        for (int t = 0; t < T; ++t) {
            if (!gather<H / XT>(a, a.xy + ((size_t) xcd * VTM + t) * H, H, ep, s_big + t * H, tid, XW_Y)) {
                s_fail = 1;
                break;
            }
            double s = 0.0;
#pragma unroll
            for (int m = 0; m < H / XT; ++m) {
                const float yv = s_big[t * H + tid + m * XT];
                s += (double) (yv * yv);
            }
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) s_red[wave][t] = s;
        }
        lds_barrier();
        if (s_fail) return;
        if (next2) s_L[l & 1][tid] = lw;
        if (tid < 3 * E) ((int32_t*) &s_slotx[(l + 1) & 1][tid % E])[tid / E] = sl_next;
        if (tid < T) {
            double tot = 0.0;
#pragma unroll
            for (int w = 0; w < XW; ++w) tot += s_red[w][tid];
            const float mean = (float) (tot / (double) H);
            s_sc[tid] = 1.0f / sqrtf(mean + a.rms_eps);
        }
        lds_barrier();
        if (!nxt) {
            if (b == 0)
                for (int i = tid; i < T * H; i += XT) {
                    a.out[i] = s_big[i];
                    if (a.x_out) a.x_out[i] = s_big[i] * s_sc[i / H];
                }
        } else {
            next_x(tid, ep + 1);
        }
    }
}

namespace {

struct VerifyKernel {
    int nlog;
    const void* fn;
};
const VerifyKernel kVerifyKernels[] = {
    {4, (const void*) k_verify_xcd<8, 3, 4>},
    {2, (const void*) k_verify_xcd<8, 3, 2>},
    {1, (const void*) k_verify_xcd<8, 3, 1>},
};

}  // namespace

const void* verify_xcd_kernel(int64_t H, int64_t F, int64_t E) {
    if (H != 2048 || F != 768) return nullptr;
    for (const VerifyKernel& kk : kVerifyKernels)
        if (E == 32 * kk.nlog) return kk.fn;
    return nullptr;
}

int launch_verify_xcd(const void* fn, const VerifyArgs& a, hipStream_t stream) {
    VerifyArgs args = a;
    void* p[] = {&args};
    return hipLaunchKernel(fn, dim3(NXCD * NJ), dim3(XT), p, 0, stream) == hipSuccess ? 0 : -3;
}

int verify_xcd_occupancy(const void* fn) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, XT, 0) != hipSuccess) return -3;
    return per_cu >= 1 ? 0 : -2;
}

}  // namespace qw
