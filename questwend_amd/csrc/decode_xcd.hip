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
#include "qw_xcd.hpp"

#include <vector>

namespace qw {

// NBH = H / 256 (8), NBF = F / 256 (down super-blocks per row, <= 3), NLOG = E / 32.
template <int NBH, int NBF, int NLOG>
__global__ void __launch_bounds__(XT) k_decode_xcd(XcdArgs a) {
    constexpr int H = NBH * QK_K, F = NBF * QK_K, E = NLOG * 32;
    constexpr int NP = F / NJ;            // (gate, up) pairs per workgroup
    constexpr int PPW = NP / XW;          // pairs per wave
    constexpr int NH = H / NJ;            // down rows per workgroup
    constexpr int RW = NH / XW;           // down rows per wave (one per 8-lane group)
    constexpr int RW0 = XW - (NLOG + 1) / 2;   // first router wave (two logits per router wave)
    constexpr int QXW = 4, QXN = NBH / 4; // waves 4, 5 quantize the next layer's x, 16 lanes per block (they share
                                          // SIMDs with waves 0, 1, which poll the logits, not with the router waves)
    static_assert(NBH == 8, "gate/up rows: one super-block per 8-lane group");
    static_assert(PPW >= 1 && PPW * XW == NP && 2 * PPW * 8 <= 64, "pairs per wave");
    static_assert(RW == 8 && NH == 64, "down rows: one row per 8-lane group; y: one row per lane of wave 0");
    static_assert(E <= 128 && E % 32 == 0, "logits: two per lane in the per-wave softmax");
    static_assert(NBF <= XW, "Q8_K of act: one wave per block");
    static_assert(QXW + QXN <= RW0 && QXN * 4 == NBH, "x quantizer and router waves");

    __shared__ __align__(16) float s_y[H];                      // y of the last layer (x = y * sc)
    __shared__ __align__(16) uint8_t s_xq[NBH * QB];            // Q8_K(x)
    __shared__ __align__(16) float s_act[F];
    __shared__ __align__(16) uint8_t s_aq[NBF * QB];            // Q8_K(act)
    __shared__ __align__(16) uint32_t s_tr[XW][2 * PPW][NBH][16];   // gate/up block records
    __shared__ __align__(16) float s_p[E];                      // logits
    __shared__ __align__(16) float s_pe[E];                     // the exact path's probabilities
    __shared__ __align__(16) int32_t s_order[E];
    __shared__ __align__(16) int4 s_slotx[2][E];              // {gate, up, down} slot of each expert
    __shared__ __align__(16) int4 s_specx[8];                 // speculative expert of rank r and its slots
    __shared__ float s_specl[9];                              // logit of rank r <= k
    __shared__ __align__(16) int4 s_my;                       // this XCD's expert and its slots (wave 0)
    __shared__ uint32_t s_topk_ep;                            // epoch of the layer whose s_my is posted
    __shared__ uint64_t s_L[2][XLW];
    __shared__ SortRange s_stack[SORT_STACK];
    __shared__ double s_red[XW];
    __shared__ int s_fail, s_need_sort, s_wflag;

    const int b = blockIdx.x, tid0 = threadIdx.x;
    // Roles: the XCD this workgroup runs on (XCC_ID) and j = b / 8.  The
    // dispatcher deals workgroups to the XCDs round robin, starting where the
    // previous dispatch left off, so XCD (b + r) % 8 for one rotation r per
    // launch: every XCD holds exactly one workgroup of each j.
    const int xcd = (int) (__builtin_amdgcn_s_getreg((3 << 11) | 20) & (NXCD - 1)), j = b >> 3;
    const int k = a.k;
    const bool expert_xcd = xcd < k;
    const int local = a.local_st;


    // The end of a layer (and the prologue): the next layer's router logits from
    // x = y * sc (router waves) and Q8_K(x) (waves QXW..QXW + QXN - 1).
    // Router weights of this lane's chain (router waves): W[NLOG j + hw][c + 32 s].
    float rw[H / 32];
    auto load_router = [&](const float* router, int tid) {
        const int wave = tid >> 6, lane = tid & 63;
        const int hw = 2 * (wave - RW0) + ((lane >> 5) & 1), c = lane & 31;
        if (router && wave >= RW0 && hw < NLOG) {
            const float* src = router + (size_t) (NLOG * j + hw) * H + c;
#pragma unroll
            for (int s2 = 0; s2 < H / 32; ++s2) rw[s2] = *(const __attribute__((address_space(1))) float*) (src + 32 * s2);
        } else {
            // (defined on every path, so the registers are not carried around the layer loop)
#pragma unroll
            for (int s2 = 0; s2 < H / 32; ++s2) rw[s2] = 0.0f;
        }
    };
    auto next_x = [&](int tid, float sc, uint32_t ep_next) {
        const int wave = tid >> 6, lane = tid & 63;
        const int hw = 2 * (wave - RW0) + ((lane >> 5) & 1), c = lane & 31;
        if (wave >= RW0 && hw < NLOG) {
            const float lg = router_chain<H>(rw, s_y, sc, c);
            if (c == 0) st_local(a.xl + xcd * E + NLOG * j + hw, tag(lg, ep_next), local);
        }
        if (wave >= QXW && wave < QXW + QXN) quant_q8K_r16(s_y, sc, NBH, s_xq, tid - 64 * QXW);
    };

    // ---- prologue: descriptors, x of layer 0, router rows and slot rows of layer 0
    if (tid0 == 0) s_fail = 0;
    if (tid0 < 8) s_specx[tid0] = int4{0, 0, 0, 0};
    if (tid0 == 0) s_topk_ep = 0;
    if (tid0 < 2 * XLW && tid0 / XLW < a.n_layer) s_L[tid0 / XLW][tid0 % XLW] = ldg64((const uint64_t*) a.layers + tid0);
    for (int i = tid0; i < H; i += XT) s_y[i] = a.x_in[i];   // layer 0 takes x_in as it is (sc = 1)
    {
        const DecodeLayer& L0 = a.layers[0];
        load_router(L0.router, tid0);
        for (int i = tid0; i < 3 * E; i += XT) {
            const int32_t* so = i < E ? L0.slot_gate : i < 2 * E ? L0.slot_up : L0.slot_down;
            ((int32_t*) &s_slotx[0][i % E])[i / E] = so ? ldg32(so + i % E) : i % E;
        }
    }
    __syncthreads();
    next_x(tid0, 1.0f, a.epoch0);

    for (int l = 0; l < a.n_layer; ++l) {
        const DecodeLayer& L = *(const DecodeLayer*) s_L[l & 1];
        const uint32_t ep = a.epoch0 + (uint32_t) l;
        const int tid = opaque(tid0);
        const int wave = tid >> 6, lane = tid & 63, g = lane >> 3, t = lane & 7;

        all_loads_returned();   // (the last were the y polls and the prefetches they follow)
        // The layer's tensors (uniform) and this lane's row offsets: read once, while
        // the logits are awaited.  Rows: gate/up pairs f = NP j + PPW wave + p (block
        // g of each), down row NH j + RW wave + g.
        const uint8_t* const Lgate = (const uint8_t*) uni64((uint64_t) L.gate);
        const uint8_t* const Lup = (const uint8_t*) uni64((uint64_t) L.up);
        const uint8_t* const Ldown = (const uint8_t*) uni64((uint64_t) L.down);
        const uint32_t gnb1 = uni32((uint32_t) L.gate_nb1), unb1 = uni32((uint32_t) L.up_nb1);
        const uint32_t dnb1 = uni32((uint32_t) L.down_nb1);
        const uint64_t gnb2 = uni64(L.gate_nb2), unb2 = uni64(L.up_nb2), dnb2 = uni64(L.down_nb2);
        const uint32_t nsg = uni32((uint32_t) min(L.n_slots_gate, (int64_t) INT32_MAX));
        const uint32_t nsu = uni32((uint32_t) min(L.n_slots_up, (int64_t) INT32_MAX));
        const uint32_t nsd = uni32((uint32_t) min(L.n_slots_down, (int64_t) INT32_MAX));
        uint32_t og[PPW], ou[PPW];
#pragma unroll
        for (int p = 0; p < PPW; ++p) {
            const uint32_t f = (uint32_t) (NP * j + PPW * wave + p);
            og[p] = f * gnb1 + 144u * (uint32_t) g;
            ou[p] = f * unb1 + 144u * (uint32_t) g;
        }
        const uint32_t od = (uint32_t) (NH * j + RW * wave + g) * dnb1;

        // ---- L: the layer's logits (all E, from this XCD's router workgroups) ------
        if (tid < E && !gather<1>(a, a.xl + xcd * E, E, ep, s_p, tid, XW_LOGITS)) s_fail = 1;
        lds_barrier();
        if (s_fail) return;
        // resident-only routing: workgroup 0 records the top k of the raw logits,
        // then every workgroup adds the layer's mask row before ranking them
        if (const float* const Lmask = (const float*) uni64((uint64_t) L.resmask)) {
            int32_t* const Lwant = (int32_t*) uni64((uint64_t) L.want);
            if (b == 0 && Lwant) decode_want(s_p, E, k, Lwant, s_order, s_stack, &s_wflag, tid, XT);
            for (int i = tid; i < E; i += XT) s_p[i] = s_p[i] + Lmask[i];
            lds_barrier();
        }
        // logit ranks (strictly larger count; four lanes per value); the rank-c
        // expert is XCD c's speculative expert: {id, gate, up, down slots}
        {
            const int i = tid >> 2, sub = tid & 3;
            const float li = s_p[i < E ? i : 0];
            int rank = 0;
#pragma unroll
            for (int c0 = 0; c0 < E / 4; c0 += 4) {
                const float4 q = *(const float4*) (s_p + 4 * (c0 + sub));
                rank += (q.x > li) + (q.y > li) + (q.z > li) + (q.w > li);
            }
            rank += dpp_i<DPP_XOR1>(rank);
            rank += dpp_i<DPP_XOR2>(rank);
            if (i < E && sub == 0) {
                s_order[i] = rank;
                if (rank <= k) s_specl[rank] = li;   // (rank k: any of equal values)
                if (rank < k) {
                    const int4 sl = s_slotx[l & 1][i];
                    s_specx[rank] = int4{i, sl.x, sl.y, sl.z};
                }
            }
        }
        lds_barrier();

        // ---- weight loads of this XCD's expert ------------------------------------
        u32x4 gh[2 * PPW], gq[2 * PPW];    // gate/up rows: header and chunk t of block g
        u32x4 dh[NBF], dq[NBF];            // down row 8 * wave + g: header and chunk t of each block
        // gate/up rows of the speculative expert are issued at once (and again if it
        // was wrong); down rows once the expert is certain (used after the act exchange)
        auto issue = [&](uint32_t sg, uint32_t su) {
            sg = sg < nsg ? sg : 0u;   // (a slot out of range reads slot 0; reported below)
            su = su < nsu ? su : 0u;
            const uint8_t* bg = Lgate + (uint64_t) sg * gnb2;
            const uint8_t* bu = Lup + (uint64_t) su * unb2;
#pragma unroll
            for (int p = 0; p < PPW; ++p) {
                gh[2 * p] = ldg16(bg + og[p]);
                gq[2 * p] = ldg16(bg + og[p] + q4k_chunk(t));
                gh[2 * p + 1] = ldg16(bu + ou[p]);
                gq[2 * p + 1] = ldg16(bu + ou[p] + q4k_chunk(t));
            }
        };
        auto issue_down = [&](uint32_t sd) {
            sd = sd < nsd ? sd : 0u;
            const uint8_t* rd = Ldown + (uint64_t) sd * dnb2 + od;
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) {
                dh[bb] = ldg16(rd + 144 * bb);
                dq[bb] = ldg16(rd + 144 * bb + q4k_chunk(t));
            }
        };
        const int4 spec = s_specx[expert_xcd ? xcd : 0];
        const int spec_e = __builtin_amdgcn_readfirstlane(spec.x);
        if (expert_xcd) issue((uint32_t) __builtin_amdgcn_readfirstlane(spec.y), (uint32_t) __builtin_amdgcn_readfirstlane(spec.z));

        // ---- top-k: wave 0, posted in LDS; the weights follow later ---------------
        // ggml_soft_max (ops.cpp:5455-5566): max, ggml_v_expf, sums of eight
        // (hsum_float_8) added in double, scale by 1 / sum.  Lane holds logits
        // lane and lane + 64.
        auto probs = [&](float (&pv)[2]) {
            float lv[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) lv[m] = lane + 64 * m < E ? s_p[lane + 64 * m] : -INFINITY;
            const float mx = wave_max_uniform(fmaxf(lv[0], lv[1]));
            float ev[2], gs[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                ev[m] = lane + 64 * m < E ? v_expf(lv[m] - mx) : 0.0f;
                // hsum_float_8 of lanes 8q..8q+7 into lane 8q: (a_i + a_{i+4}),
                // then (r0 + r2), (r1 + r3), then their sum (quants.c:42-48 pairing)
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
        };
        // Lane r < k ends with selected expert r (and, after the gate/up rows, its weight).
        int sel_id = 0;
        float sel_w = 0.0f;
        if (wave == 0) {
            // The speculative order (logit ranks) is argsort's first k when
            //  (1) ranks 0..k-1 are held once each (no equal or NaN logit there), and
            //  (2) e_r = v_expf(l_r - l_0) of ranks r = 0..k satisfy e_r > e_{r+1} (1 + 2^-20)
            //      for r < k, and e_{k-1} >= 2^-100.
            // v_expf is non-decreasing on (-inf, 0] (checked over every float), and so
            // is rounding e * inv for the softmax's inv in [1/E, 1]: every other
            // probability is at most p_k, and a ratio above 1 + 2^-21 survives the
            // rounding of e * inv, so p_0 > ... > p_{k-1} > every other p.
            int rk[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) rk[m] = lane + 64 * m < E ? s_order[lane + 64 * m] : E;
            const float lr = s_specl[lane <= k ? lane : 0];
            bool ok = __popcll(__ballot(rk[0] < k)) + __popcll(__ballot(rk[1] < k)) == k;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (r < k) ok = ok && __ballot(rk[0] == r || rk[1] == r) != 0;
            const float er = v_expf(lr - __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lr), 0)));
            const float en = dpp_f<0x101>(er);   // row_shl:1: lane r <- r + 1 (r <= 8)
            bool bad = lane < k && !(er > en * 0x1.00001p+0f);
            if (lane == k - 1 && !(er >= 0x1p-100f)) bad = true;
            ok = ok && !__any(bad);
            if (ok) {
                sel_id = s_specx[lane & 7].x;
            } else {
                // exact order: rank the probabilities; a tie or NaN inside the first
                // k places leaves the order to std::sort, which is replayed exactly
                float pv[2];
                probs(pv);
                if (lane < E) s_pe[lane] = pv[0];
                if (lane + 64 < E) s_pe[lane + 64] = pv[1];
                wave_lds_sync();
                bool tie = false;
#pragma unroll 1
                for (int m = 0; m < 2; ++m) {
                    const int i = lane + 64 * m;
                    const float pi = i < E ? pv[m] : 0.0f;
                    int gt = 0, eq = 0;
#pragma unroll 2
                    for (int jj = 0; jj < E; jj += 4) {
                        const float4 q = *(const float4*) (s_pe + jj);
                        gt += (q.x > pi) + (q.y > pi) + (q.z > pi) + (q.w > pi);
                        eq += (q.x == pi) + (q.y == pi) + (q.z == pi) + (q.w == pi);
                    }
                    if (i < E && gt < k) {
                        if (eq != 1) tie = true;
                        else s_order[gt] = i;
                    }
                }
                if (__any(tie)) {
                    wave_lds_sync();
                    for (int i = lane; i < E; i += 64) s_order[i] = i;
                    wave_lds_sync();
                    if (lane == 0) {
                        sort_desc_replay(s_order, E, s_pe, s_stack);
                        if (b == 0) atomicOr(a.status, 1);
                    }
                }
                wave_lds_sync();
                sel_id = s_order[lane & 7];
            }
            // this XCD's expert and its slots, for the other waves
            const int my_e = __builtin_amdgcn_readlane(sel_id, expert_xcd ? xcd : 0);
            if (lane == 0) {
                const int4 sl = s_slotx[l & 1][my_e];
                s_my = int4{my_e, sl.x, sl.y, sl.z};
            }
            wave_lds_sync();
            if (lane == 0) __hip_atomic_store(&s_topk_ep, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);   // posted after the values above
        }

        // ---- A: gate/up rows of this workgroup's pairs, SwiGLU -----------------
        if (expert_xcd) {
            int e_cur = spec_e;
            int4 my;
            float res, up;
            const Q8KLane yv = q8k_lane(s_xq + QB * g, t);   // block g of Q8_K(x): the same for every row
            for (;;) {
#pragma unroll
                for (int r = 0; r < 2 * PPW; ++r) {
                    int p[4];
                    const Q4KLane w = q4k_lane(gh[r], gq[r], t);
                    q4k_dot(w, yv, p);
                    reduce_chunks(p);
                    const int pm = q4k_min_dot(w, yv);
                    uint32_t* rec = s_tr[wave][r][g];
                    // every lane stores two words, no lane-conditional stores: rec[t] = AVX
                    // lane t's sum, rec[8 + t] = min lane t's term (t < 4), d (t = 4), dmin (t = 5)
                    const int q = t & 3;
                    const int pt = q == 0 ? p[0] : q == 1 ? p[1] : q == 2 ? p[2] : p[3];
                    const uint32_t w2 = t < 4 ? (uint32_t) pm : t == 4 ? fbits(w.d) : fbits(w.dmin);
                    rec[t] = (uint32_t) pt;
                    rec[8 + t] = w2;
                }
                wave_lds_sync();
                // chain lanes: row r = lane >> 3 (< 2 * PPW), AVX lane n = lane & 7
                {
                    const int r = g < 2 * PPW ? g : 0, n = t;
                    float acc = 0.0f, accm = 0.0f;
#pragma unroll
                    for (int bb = 0; bb < NBH; ++bb) {
                        const uint32_t* rec = s_tr[wave][r][bb];
                        const int S = (int) rec[n];
                        const int pm = (int) rec[8 + (n & 3)];
                        const float wd = bitsf(rec[12]), wdm = bitsf(rec[13]);
                        const float yd = *(const float*) (s_xq + QB * bb + 256);
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
                up = dpp_f<0x108>(res);     // lane 16p: gate of pair p; lane 16p + 8: its up
                // the exact expert of this XCD (posted by wave 0)
                long spins = 0;
                while (__hip_atomic_load(&s_topk_ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != ep) {
                    if (++spins > XSPIN) {
                        x_abort(a, 8 | XW_TOPK);
                        return;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                my = s_my;
                if (__builtin_amdgcn_readfirstlane(my.x) == e_cur) break;
                // misspeculated: load the right rows and compute again
                e_cur = __builtin_amdgcn_readfirstlane(my.x);
                issue((uint32_t) __builtin_amdgcn_readfirstlane(my.y), (uint32_t) __builtin_amdgcn_readfirstlane(my.z));
            }
            if ((lane & 15) == 0 && (lane >> 4) < PPW) {
                const int f = NP * j + PPW * wave + (lane >> 4);
                st_local(a.xa + xcd * F + f, tag(v_silu(res) * up, ep), local);
            }
            issue_down((uint32_t) __builtin_amdgcn_readfirstlane(my.w));
        }
        // ---- weights of the selected experts (wave 0; used by the y sum) -----------
        // selected probabilities / clamp(sum) (* scale), core/runtime.cpp:887-897
        if (wave == 0) {
            float pv[2];
            probs(pv);
            const float pa = __shfl(pv[0], sel_id & 63), pb = __shfl(pv[1], sel_id & 63);
            const float pr = sel_id < 64 ? pa : pb;
            double sp = 0.0;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (r < k) sp += (double) __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr), r));
            float wsum = (float) sp;
            wsum = fmaxf(fminf(wsum, INFINITY), 6.103515625e-5f);
            sel_w = pr / wsum;
            if (a.scale != 0.0f && a.scale != 1.0f) sel_w = sel_w * a.scale;
            if (lane < k && b == 0) {
                if (a.ids_out) {
                    a.ids_out[l * k + lane] = sel_id;
                    a.w_out[l * k + lane] = sel_w;
                }
                // slot checks of the selected experts (reported once, by workgroup 0)
                const int4 sl = s_slotx[l & 1][sel_id];
                if ((uint32_t) sl.x >= nsg || (uint32_t) sl.y >= nsu || (uint32_t) sl.z >= nsd) atomicOr(a.status, 16);
            }
        }
        // next layer's slot rows and the descriptor of layer l + 2: issued once the
        // gate/up rows are consumed, stored to LDS after the y exchange
        const bool nxt = l + 1 < a.n_layer;
        const DecodeLayer& L1 = *(const DecodeLayer*) s_L[(l + 1) & 1];
        int32_t sl_next = 0;
        if (tid < 3 * E) {
            const int32_t* so = !nxt ? nullptr : tid < E ? L1.slot_gate : tid < 2 * E ? L1.slot_up : L1.slot_down;
            sl_next = so ? ldg32(so + tid % E) : tid % E;
        }
        const bool next2 = l + 2 < a.n_layer && tid < XLW;
        const uint64_t lw = ldg64((const uint64_t*) (a.layers + (next2 ? l + 2 : l)) + (tid % XLW));

        // ---- act of this XCD's expert -> Q8_K (one wave per block) -----------------
        if (expert_xcd) {
            // the weight side of the down rows, prepared while the act words are awaited
            Q4KLane dw[NBF];
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) dw[bb] = q4k_lane(dh[bb], dq[bb], t);
            if (!gather<(F + XT - 1) / XT>(a, a.xa + xcd * F, F, ep, s_act, tid, XW_ACT)) s_fail = 1;
            lds_barrier();
            if (s_fail) return;
            if (wave < NBF) {
                const float4 v4 = *(const float4*) (s_act + QK_K * wave + 4 * lane);
                const float v[4] = {v4.x, v4.y, v4.z, v4.w};
                quant_q8K_w64(v, lane, s_aq + QB * wave);
            }
            lds_barrier();
            // ---- D: down rows 8 * wave + g of this workgroup, in-lane block chain
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            float accm = 0.0f;
#pragma unroll
            for (int bb = 0; bb < NBF; ++bb) {
                const uint8_t* yb = s_aq + QB * bb;
                int p[4];
                q4k_dot(dw[bb], yb, t, p);
                reduce_chunks(p);
                const float yd = *(const float*) (yb + 256);
                const float D = yd * dw[bb].d;
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(D, (float) p[i], acc[i]);
                const int pm = q4k_min_dot(dw[bb], yb, t);
                accm = __builtin_fmaf(-yd * dw[bb].dmin, (float) pm, accm);
            }
            // hsum_float_8: lane t = 0 holds AVX lanes 0..3, lane t = 4 lanes 4..7
            float r4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) r4[i] = acc[i] + dpp_f<0x12C>(acc[i]);   // row_ror:12: lane i <- (i + 4) mod 16
            const float hs = (r4[0] + r4[2]) + (r4[1] + r4[3]);
            // min lanes 0..3: (m0 + m2) + (m1 + m3)
            const float m2 = accm + dpp_f<DPP_XOR2>(accm);
            const float mm = m2 + dpp_f<DPP_XOR1>(m2);
            if (t == 0)
                st_cross(a.xd + (((size_t) (l & 1) * NXCD + xcd) * NJ + j) * NH + RW * wave + g, tag(hs + mm, ep));
        }
        // next layer's router weights, into the router lanes' registers (the gate/up
        // and down rows are consumed; they arrive while y is exchanged and normed)
        load_router(nxt ? L1.router : nullptr, tid);

        // ---- D -> y[h]: wave 0, lane h; the k expert XCDs' down outputs of row h --------
        if (wave == 0) {
            const uint64_t* src = a.xd + ((size_t) (l & 1) * NXCD * NJ + j) * NH + lane;
            float dv[8];
            uint32_t got = 0;
            const uint32_t all = (1u << k) - 1u;
            long spins = 0;
            while (got != all) {
                uint64_t v[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) v[c] = poll64(src + (size_t) (c < k ? c : 0) * NJ * NH);
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
                // ggml_vec_dot_f32(k, experts^T row, w): k < 32 -> scalar tail: groups
                // of four as mul + add, the remainder fused
                float sumf = 0.0f;
                const int nv = k & ~3;
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    if (c < k) {
                        const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sel_w), c));
                        sumf = (c < nv) ? sumf + dv[c] * wc : __builtin_fmaf(dv[c], wc, sumf);
                    }
                st_local(a.xy + xcd * H + NH * j + lane, tag(sumf, ep), local);
            }
        }

        // ---- Y: all y of this XCD, its RMSNorm (sum of squares in double) ------------
        {
            float yv[H / XT];
            bool ok = true;
            {
                const uint64_t* src = a.xy + xcd * H;
                uint32_t got = 0;
                const uint32_t all = (1u << (H / XT)) - 1u;
                long spins = 0;
                while (got != all) {
                    uint64_t v[H / XT];
#pragma unroll
                    for (int m = 0; m < H / XT; ++m) v[m] = poll64(src + tid + m * XT);
#pragma unroll
                    for (int m = 0; m < H / XT; ++m)
                        if (!(got & (1u << m)) && (uint32_t) (v[m] >> 32) == ep) {
                            yv[m] = bitsf((uint32_t) v[m]);
                            got |= 1u << m;
                        }
                    if (got == all) break;
                    if (++spins > XSPIN) {
                        x_abort(a, 8 | XW_Y);
                        ok = false;
                        break;
                    }
                    if ((spins & 255) == 0 && x_aborted(a)) {
                        ok = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            double s = 0.0;
#pragma unroll
            for (int m = 0; m < H / XT; ++m) {
                s_y[tid + m * XT] = yv[m];
                s += (double) (yv[m] * yv[m]);
            }
            for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
            if (lane == 0) s_red[wave] = s;
            if (!ok) s_fail = 1;
        }
        lds_barrier();
        if (s_fail) return;
        // every thread is past its last read of layer l's descriptor: the
        // descriptor of layer l + 2 takes its place
        if (next2) s_L[l & 1][tid] = lw;
        if (tid < 3 * E) ((int32_t*) &s_slotx[(l + 1) & 1][tid % E])[tid / E] = sl_next;   // (in place of layer l - 1's)
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < XW; ++w) tot += s_red[w];
        const float mean = (float) (tot / (double) H);
        const float sc = 1.0f / sqrtf(mean + a.rms_eps);
        if (!nxt) {
            if (b == 0)
                for (int i = tid; i < H; i += XT) {
                    a.out[i] = s_y[i];
                    if (a.x_out) a.x_out[i] = s_y[i] * sc;
                }
        } else {
            next_x(tid, sc, ep + 1);
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
    if (d.H == 2048 && d.type_down == T_Q4_K)
        for (const XcdKernel& kk : kXcdKernels)
            if (d.F == 256 * kk.nbf && d.E == 32 * kk.nlog) return kk.fn;
    return decode_xcd_wide_kernel(d);
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
// the workgroups of a 256-workgroup launch are dealt to the XCDs round robin
// (XCD (b + r) % 8 for one r).
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
    int good = n > 0;
    for (int i = 0; i < n; ++i)
        if (h[(size_t) i] < 0 || h[(size_t) i] >= NXCD || (h[(size_t) i] - i - h[0]) % NXCD != 0) good = 0;
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
