// decode_xcd_wide.hip -- persistent whole-stack MoE FFN decode for wide layers
// (H = 4096, F = 1536, E = 128, Q4_K gate/up, Q6_K or Q4_K down: the shape of
// Qwen3-235B-A22B), one selected expert per XCD as in decode_xcd.hip: the
// work core/runtime.cpp schedules as build_moe per layer inside one graph
// (decode() -> build_graph, 976-1100; the slot remap 903-931).
//
// Per XCD c (the expert of top-k rank c) the 32 workgroups split 12 MB of
// expert rows per layer, four times the 30B shape's, so the work inside an XCD
// is laid out differently:
//   - a lane holds whole super-blocks (lane = (row, block), the block-parallel
//     GEMV's mapping, qw_bp_block.hpp) instead of eight lanes per block: three
//     Q4_K gate/up blocks per lane, issued as soon as the logits rank the
//     expert, then up to two down blocks per lane once it is certain;
//   - every integer of a block's eight AVX lanes is formed in its lane and
//     written to LDS; lanes (row, AVX lane) then run the fp32 chains over the
//     blocks in order and one lane per row the hsum tree (quants.c: q4_K
//     2038-2115, q6_K 2426-2508);
//   - every XCD computes all E router logits, as decode_xcd.hip does:
//     workgroup j computes logits 4 j .. 4 j + 3 (waves 6 and 7, 32 lanes per
//     logit) from its router rows in LDS, kept in the block-integer buffer,
//     which is idle from the down phase to the next layer's gate/up phase.
//     (Each router row read once per device, its logit exchanged across XCDs,
//     measured slower: the logit gather then waits for the slowest of 128
//     workgroups chip-wide plus a cross-XCD hop.)
// The exchanges are decode_xcd.hip's tagged words: logits and act inside the
// XCD, down outputs across XCDs, y inside the XCD.  Ids,
// weights and outputs are bit-identical to the reference CPU path.
#include "qw_xcd.hpp"
#include "qw_bp_block.hpp"

namespace qw {

namespace {

typedef __attribute__((address_space(1))) const uint32_t gu32_t;

}  // namespace

// NBH = H / 256, NBF = F / 256, NLOG = E / 32, TD = the down type.
template <int NBH, int NBF, int NLOG, int TD>
__global__ void __launch_bounds__(XT) k_decode_xcd_wide(XcdArgs a) {
    constexpr int H = NBH * QK_K, F = NBF * QK_K, E = NLOG * 32;
    constexpr int NP = F / NJ;                    // (gate, up) pairs per workgroup: rows p (gate), NP + p (up)
    constexpr int NR = 2 * NP;                    // gate/up rows per workgroup
    constexpr int UG = NR * NBH;                  // gate/up blocks per workgroup
    constexpr int UGL = UG / XT;                  // per lane
    constexpr int NH = H / NJ;                    // down rows per workgroup
    constexpr int UD = NH * NBF;                  // down blocks per workgroup
    constexpr int UDL = (UD + XT - 1) / XT;       // per lane (the last round partial)
    constexpr int DW = TD == T_Q6_K ? 53 : 36;    // words a lane holds per down block
    constexpr int NPG = BpType<T_Q4_K>::NPW, NCG = BpType<T_Q4_K>::NCH;
    constexpr int NPD = BpType<TD>::NPW, NCD = BpType<TD>::NCH;
    constexpr int PART = UG * NPG > UD * NPD ? UG * NPG : UD * NPD;
    constexpr int CHN = NR * NCG > NH * NCD ? NR * NCG : NH * NCD;
    static_assert(UG % XT == 0 && NP % 4 == 0, "gate/up blocks: whole per lane, gate or up uniform per wave");
    static_assert((UD % XT) % 64 == 0, "down blocks: the last round covers whole waves");
    static_assert(NR <= XT && NH <= 128, "rows per workgroup");
    static_assert(E == 4 * NJ && PART >= 4 * H, "logits: four per workgroup (rows in s_part), two per lane in the softmax");
    static_assert(NBF <= XW, "Q8_K of act: one wave per block");
    static_assert(NBH * 16 <= 4 * 64 && H % (2 * XT) == 0, "Q8_K of x: four waves; router row: two 16-byte loads per lane");
    static_assert(TD == T_Q6_K || TD == T_Q4_K, "down type");

    __shared__ __align__(16) float s_y[H];                  // y of the last layer (x = y * sc)
    __shared__ __align__(16) uint32_t s_xq[NBH * BP_ABLK / 4];   // Q8_K(x): block b at 304 b + 12
    __shared__ __align__(16) float s_act[F];
    __shared__ __align__(16) uint32_t s_aq[NBF * BP_ABLK / 4];   // Q8_K(act), same layout
    __shared__ __align__(16) uint32_t s_part[PART];         // per-block integers and scales; from the y exchange
                                                            // to the router chains, router rows 4 j .. 4 j + 3
    __shared__ __align__(16) float s_ch[CHN];               // per-(row, chain) fp32 sums
    __shared__ __align__(16) float s_g[NR];                 // gate / up outputs
    __shared__ __align__(16) float s_p[E];                  // logits
    __shared__ __align__(16) float s_pe[E];                 // the exact path's probabilities
    __shared__ __align__(16) int32_t s_order[E];
    __shared__ __align__(16) int4 s_slotx[2][E];            // {gate, up, down} slot of each expert
    __shared__ __align__(16) int4 s_specx[8];               // speculative expert of rank r and its slots
    __shared__ float s_specl[9];                            // logit of rank r <= k
    __shared__ float s_selw[8];                             // weights of the selected experts
    __shared__ __align__(16) int4 s_my;                     // this XCD's expert and its slots (wave 0)
    __shared__ int s_exact;                                 // 1: the exact top-k path runs this layer
    __shared__ uint64_t s_L[2][XLW];
    __shared__ SortRange s_stack[SORT_STACK];
    __shared__ double s_red[XW];
    __shared__ int s_fail, s_wflag;

    const int b = blockIdx.x, tid0 = threadIdx.x;
    // roles: the XCD this workgroup runs on (XCC_ID) and j = b / 8 (decode_xcd.hip)
    const int xcd = (int) (__builtin_amdgcn_s_getreg((3 << 11) | 20) & (NXCD - 1)), j = b >> 3;
    const int k = a.k;
    const bool expert_xcd = xcd < k;
    const int local = a.local_st;
    float* const s_rw = (float*) s_part;   // router rows 4 j .. 4 j + 3 of the next layer

    // The end of a layer (and the prologue): this workgroup's four logits of the
    // next layer from x = y * sc (waves 6 and 7: lanes 32 h .. 32 h + 31 = the 32
    // chains of logit 4 j + 2 (wave - 6) + h), stored inside the XCD, and Q8_K(x)
    // (waves 0, 1, 4, 5, sixteen lanes per block).
    auto next_x = [&](int tid, float sc, uint32_t ep_next) {
        const int wave = tid >> 6, lane = tid & 63;
        if (wave >= XW - 2) {
            const int li = 2 * (wave - (XW - 2)) + (lane >> 5);
            const float lg = router_chain_lds<H>(s_rw + H * li, s_y, sc, lane & 31);
            if ((lane & 31) == 0) st_local(a.xl + xcd * E + 4 * j + li, tag(lg, ep_next), local);
        }
        const int tt = wave < 2 ? tid : wave == 4 || wave == 5 ? tid - 128 : -1;
        if (tt >= 0) quant_q8K_r16<12, 4, 0>(s_y, sc, NBH, (uint8_t*) s_xq, tt);
    };

    // ---- prologue: descriptors, x of layer 0, router row and slot rows of layer 0
    if (tid0 == 0) s_fail = 0;
    if (tid0 < 8) s_specx[tid0] = int4{0, 0, 0, 0};
    if (tid0 < 2 * XLW && tid0 / XLW < a.n_layer) s_L[tid0 / XLW][tid0 % XLW] = ldg64((const uint64_t*) a.layers + tid0);
    for (int i = tid0; i < H; i += XT) s_y[i] = a.x_in[i];   // layer 0 takes x_in as it is (sc = 1)
    {
        const DecodeLayer& L0 = a.layers[0];
        for (int i = tid0; i < 4 * H; i += XT) s_rw[i] = L0.router[(size_t) 4 * j * H + i];
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
        const int wave = tid >> 6, lane = tid & 63;

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
        // this lane's gate/up blocks: unit u = tid + XT m -> row r = u / NBH (gate row
        // NP j + r for r < NP, else up row NP j + r - NP), block u % NBH; gate or up is
        // uniform per wave
        uint32_t og[UGL];
        bool gup[UGL];
#pragma unroll
        for (int m = 0; m < UGL; ++m) {
            const int u = tid + XT * m, r = u / NBH, bb = u % NBH;
            gup[m] = r >= NP;
            og[m] = (uint32_t) (NP * j + (gup[m] ? r - NP : r)) * (gup[m] ? unb1 : gnb1) + 144u * (uint32_t) bb;
        }

        // ---- L: the layer's E logits (this XCD's words) ----------------------------
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
                if (rank <= k) s_specl[rank] = li;
                if (rank < k) {
                    const int4 sl = s_slotx[l & 1][i];
                    s_specx[rank] = int4{i, sl.x, sl.y, sl.z};
                }
            }
        }
        lds_barrier();

        // ---- weight loads of this XCD's expert ------------------------------------
        // Each weight array is defined and consumed inside one branch (and both
        // arms of a conditional load define it), so no register set is carried
        // from one layer to the next.
        u32x4 wg[UGL][9];       // gate/up: this lane's Q4_K blocks
        auto issue = [&](uint32_t sg, uint32_t su) {
            sg = sg < nsg ? sg : 0u;   // (a slot out of range reads slot 0; reported below)
            su = su < nsu ? su : 0u;
            const uint8_t* bg = Lgate + (uint64_t) sg * gnb2;
            const uint8_t* bu = Lup + (uint64_t) su * unb2;
#pragma unroll
            for (int m = 0; m < UGL; ++m) {
                const uint8_t* p = (gup[m] ? bu : bg) + og[m];
#pragma unroll
                for (int i = 0; i < 9; ++i) wg[m][i] = ldg16(p + 16 * i);
            }
        };
        auto gate_up_parts = [&]() {
#pragma unroll
            for (int m = 0; m < UGL; ++m) {
                const int u = tid + XT * m;
                uint32_t part[NPG];
                bp_q4k_block([&, m](uint32_t o) { return wg[m][o / 16][(o / 4) % 4]; }, s_xq,
                             BP_ABLK * (uint32_t) (u % NBH) + 12u, part);
#pragma unroll
                for (int i = 0; i < NPG; ++i) s_part[u * NPG + i] = part[i];
            }
        };
        const int4 spec = s_specx[expert_xcd ? xcd : 0];
        const int spec_e = __builtin_amdgcn_readfirstlane(spec.x);

        // ---- top-k: wave 0 (decode_xcd.hip's check) ---------------------------------
        auto probs = [&](float (&pv)[2]) {
            float lv[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) lv[m] = lane + 64 * m < E ? s_p[lane + 64 * m] : -INFINITY;
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
        };
        // The speculative order is taken when decode_xcd.hip's check passes (ranks
        // 0..k-1 held once each, the v_expf ratios of ranks 0..k strictly above
        // 1 + 2^-20, e_{k-1} >= 2^-100).  Otherwise the exact order (ranked
        // probabilities, std::sort replayed on a tie) is formed after the
        // speculative gate/up blocks are consumed, so no weight registers are
        // live across the replay's call, and the blocks are loaded again if the
        // expert changed.
        int sel_id = 0;
        auto post_my = [&]() {   // wave 0: this XCD's expert and its slots
            const int my_e = __builtin_amdgcn_readlane(sel_id, expert_xcd ? xcd : 0);
            if (lane == 0) {
                const int4 sl = s_slotx[l & 1][my_e];
                s_my = int4{my_e, sl.x, sl.y, sl.z};
            }
        };
        auto topk_fast = [&]() {
            if (wave != 0) return;
            int rk[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) rk[m] = lane + 64 * m < E ? s_order[lane + 64 * m] : E;
            const float lr = s_specl[lane <= k ? lane : 0];
            bool ok = __popcll(__ballot(rk[0] < k)) + __popcll(__ballot(rk[1] < k)) == k;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (r < k) ok = ok && __ballot(rk[0] == r || rk[1] == r) != 0;
            const float er = v_expf(lr - __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lr), 0)));
            const float en = dpp_f<0x101>(er);
            bool bad = lane < k && !(er > en * 0x1.00001p+0f);
            if (lane == k - 1 && !(er >= 0x1p-100f)) bad = true;
            ok = ok && !__any(bad);
            if (ok) {
                sel_id = s_specx[lane & 7].x;
                post_my();
            }
            if (lane == 0) s_exact = ok ? 0 : 1;
        };
        auto topk_exact = [&]() {
            if (wave != 0) return;
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
            post_my();
        };
        // weights of the selected experts (wave 0; used by the y sum):
        // selected probabilities / clamp(sum) (* scale), core/runtime.cpp:887-897
        auto weights = [&]() {
            if (wave != 0) return;
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
            float sel_w = pr / wsum;
            if (a.scale != 0.0f && a.scale != 1.0f) sel_w = sel_w * a.scale;
            if (lane < 8) s_selw[lane] = sel_w;
            if (lane < k && b == 0) {
                if (a.ids_out) {
                    a.ids_out[l * k + lane] = sel_id;
                    a.w_out[l * k + lane] = sel_w;
                }
                const int4 sl = s_slotx[l & 1][sel_id];
                if ((uint32_t) sl.x >= nsg || (uint32_t) sl.y >= nsu || (uint32_t) sl.z >= nsd) atomicOr(a.status, 16);
            }
        };

        // next layer's slot rows and the descriptor of layer l + 2 (stored after the y exchange)
        const bool nxt = l + 1 < a.n_layer;
        const DecodeLayer& L1 = *(const DecodeLayer*) s_L[(l + 1) & 1];
        int32_t sl_next = 0;
        if (tid < 3 * E) {
            const int32_t* so = !nxt ? nullptr : tid < E ? L1.slot_gate : tid < 2 * E ? L1.slot_up : L1.slot_down;
            sl_next = so ? ldg32(so + tid % E) : tid % E;
        }
        const bool next2 = l + 2 < a.n_layer && tid < XLW;
        const uint64_t lw = ldg64((const uint64_t*) (a.layers + (next2 ? l + 2 : l)) + (tid % XLW));

        // Down block u (row NH j + u / NBF, block u % NBF) of slot sd into w (Q6_K:
        // the aligned words holding its 210 bytes, sh its byte offset in the first);
        // zeros for u >= UD (uniform per wave).
        uint32_t wd0[DW], wd1[DW], dsh0, dsh1;   // this lane's down blocks u = tid, tid + XT
        auto load_down = [&](uint32_t sd, int u, uint32_t (&w)[DW], uint32_t& sh) {
            sd = sd < nsd ? sd : 0u;
            if (u < UD) {
                const uint8_t* bp = Ldown + (uint64_t) sd * dnb2 + (uint32_t) (NH * j + u / NBF) * dnb1 +
                                    (uint32_t) block_bytes(TD) * (uint32_t) (u % NBF);
                if constexpr (TD == T_Q6_K) {
                    sh = (uint32_t) ((uintptr_t) bp & 3);
                    gu32_t* src = (gu32_t*) ((uintptr_t) bp & ~(uintptr_t) 3);
#pragma unroll
                    for (int i = 0; i < DW; ++i) w[i] = src[i];
                } else {
                    sh = 0;
#pragma unroll
                    for (int i = 0; i < 9; ++i) {
                        const u32x4 v = ldg16(bp + 16 * i);
                        w[4 * i] = v[0];
                        w[4 * i + 1] = v[1];
                        w[4 * i + 2] = v[2];
                        w[4 * i + 3] = v[3];
                    }
                }
            } else {
                sh = 0;
#pragma unroll
                for (int i = 0; i < DW; ++i) w[i] = 0u;
            }
        };
        // the integers of down block u from w (Q6_K: aligned in place first) into s_part
        auto down_parts = [&](int u, uint32_t (&w)[DW], uint32_t sh) {
            if (u >= UD) return;
            uint32_t part[NPD];
            const uint32_t yb = BP_ABLK * (uint32_t) (u % NBF) + 12u;
            if constexpr (TD == T_Q6_K) {
                const uint16_t d16 = (uint16_t) (sh ? w[52] >> 16 : w[52] & 0xffff);
#pragma unroll
                for (int i = 0; i < 52; ++i) w[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
                bp_q6k_block<true>([&](uint32_t o) { return w[o / 4]; }, d16, s_aq, yb, part);
            } else {
                bp_q4k_block([&](uint32_t o) { return w[o / 4]; }, s_aq, yb, part);
            }
#pragma unroll
            for (int i = 0; i < NPD; ++i) s_part[u * NPD + i] = part[i];
        };

        if (expert_xcd) {
            // ---- A: the speculative expert's gate/up blocks and the first down block
            // of each lane, issued together; the gate/up integers
            issue((uint32_t) __builtin_amdgcn_readfirstlane(spec.y), (uint32_t) __builtin_amdgcn_readfirstlane(spec.z));
            load_down((uint32_t) __builtin_amdgcn_readfirstlane(spec.w), tid, wd0, dsh0);
            topk_fast();
            gate_up_parts();
            lds_barrier();
            if (s_exact) {
                topk_exact();
                lds_barrier();
                const int4 my = s_my;
                if (__builtin_amdgcn_readfirstlane(my.x) != spec_e) {
                    // misspeculated: the right rows, one gate/up block at a time (a rare
                    // path; its own registers keep the fast path's blocks out of scratch)
                    uint32_t sg = (uint32_t) __builtin_amdgcn_readfirstlane(my.y);
                    uint32_t su = (uint32_t) __builtin_amdgcn_readfirstlane(my.z);
                    sg = sg < nsg ? sg : 0u;
                    su = su < nsu ? su : 0u;
#pragma unroll
                    for (int m = 0; m < UGL; ++m) {
                        const uint8_t* p = (gup[m] ? Lup + (uint64_t) su * unb2 : Lgate + (uint64_t) sg * gnb2) + og[m];
                        u32x4 w1[9];
#pragma unroll
                        for (int i = 0; i < 9; ++i) w1[i] = ldg16(p + 16 * i);
                        const int u = tid + XT * m;
                        uint32_t part[NPG];
                        bp_q4k_block([&](uint32_t o) { return w1[o / 16][(o / 4) % 4]; }, s_xq,
                                     BP_ABLK * (uint32_t) (u % NBH) + 12u, part);
#pragma unroll
                        for (int i = 0; i < NPG; ++i) s_part[u * NPG + i] = part[i];
                    }
                    load_down((uint32_t) __builtin_amdgcn_readfirstlane(my.w), tid, wd0, dsh0);
                }
                lds_barrier();
            }
            const int4 my = s_my;
            load_down((uint32_t) __builtin_amdgcn_readfirstlane(my.w), tid + XT, wd1, dsh1);
            // ---- chains -> rows -> SwiGLU ---------------------------------------------
            // chain (row, c): c < 8 -> AVX lane c of acc over the blocks in order, c >= 8
            // -> min lane c - 8 of acc_m
            for (int q = tid; q < NR * NCG; q += XT) {
                const int r = q / NCG, c = q - r * NCG;
                const int sw = c < 8 ? NPG - 2 : NPG - 1;
                float acc = 0.0f;
#pragma unroll
                for (int bb = 0; bb < NBH; ++bb) {
                    const int pw = (r * NBH + bb) * NPG;
                    acc = __builtin_fmaf(bitsf(s_part[pw + sw]), (float) (int) s_part[pw + c], acc);
                }
                s_ch[q] = acc;
            }
            lds_barrier();
            if (tid < NR) {   // hsum_float_8(acc) + ((m0 + m2) + (m1 + m3))
                const float* A = s_ch + tid * NCG;
                const float v = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
                s_g[tid] = v + ((A[8] + A[10]) + (A[9] + A[11]));
            }
            lds_barrier();
            if (tid < NP) st_local(a.xa + xcd * F + NP * j + tid, tag(v_silu(s_g[tid]) * s_g[NP + tid], ep), local);

            weights();

            // ---- act of this XCD's expert -> Q8_K -> D: down blocks -> rows ------------
            if (!gather<(F + XT - 1) / XT>(a, a.xa + xcd * F, F, ep, s_act, tid, XW_ACT)) s_fail = 1;
            lds_barrier();
            if (s_fail) return;
            if (wave < NBF) {
                const float4 v4 = *(const float4*) (s_act + QK_K * wave + 4 * lane);
                const float v[4] = {v4.x, v4.y, v4.z, v4.w};
                quant_q8K_w64<4, 0>(v, lane, (uint8_t*) s_aq + BP_ABLK * wave + 12);
            }
            lds_barrier();
            down_parts(tid, wd0, dsh0);
            down_parts(tid + XT, wd1, dsh1);
            lds_barrier();
            for (int q = tid; q < NH * NCD; q += XT) {
                const int r = q / NCD, c = q - r * NCD;
                const int sw = c < 8 ? NPD - (TD == T_Q4_K ? 2 : 1) : NPD - 1;
                float acc = 0.0f;
#pragma unroll
                for (int bb = 0; bb < NBF; ++bb) {
                    const int pw = (r * NBF + bb) * NPD;
                    acc = __builtin_fmaf(bitsf(s_part[pw + sw]), (float) (int) s_part[pw + c], acc);
                }
                s_ch[q] = acc;
            }
            lds_barrier();
            if (tid < NH) {
                const float* A = s_ch + tid * NCD;
                float v = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
                if constexpr (TD == T_Q4_K) v = v + ((A[8] + A[10]) + (A[9] + A[11]));
                st_cross(a.xd + (((size_t) (l & 1) * NXCD + xcd) * NJ + j) * NH + tid, tag(v, ep));
            }
        } else {
            topk_fast();
            lds_barrier();
            if (s_exact) {
                topk_exact();
                lds_barrier();
                lds_barrier();
            }
            weights();
        }
        // the next layer's router rows 4 j .. 4 j + 3, into registers (stored to LDS
        // after the y exchange)
        u32x4 rwv[8];
        if (nxt) {
            const float* src = L1.router + (size_t) 4 * j * H;
#pragma unroll
            for (int i = 0; i < 8; ++i) rwv[i] = ldg16(src + 4 * (tid + XT * i));
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) rwv[i] = u32x4{0u, 0u, 0u, 0u};
        }
        lds_barrier();   // s_selw posted by wave 0

        // ---- D -> y[h]: waves 0, 1, lane h; the k expert XCDs' down outputs of row h --
        if (tid < NH) {
            const uint64_t* src = a.xd + ((size_t) (l & 1) * NXCD * NJ + j) * NH + tid;
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
                // ggml_vec_dot_f32(k, experts^T row, w), k < 32: the scalar tail
                float sumf = 0.0f;
                const int nv = k & ~3;
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    if (c < k) {
                        const float wc = s_selw[c];
                        sumf = (c < nv) ? sumf + dv[c] * wc : __builtin_fmaf(dv[c], wc, sumf);
                    }
                st_local(a.xy + xcd * H + NH * j + tid, tag(sumf, ep), local);
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
            if (nxt) {
#pragma unroll
                for (int i = 0; i < 8; ++i) *(u32x4*) (s_rw + 4 * (tid + XT * i)) = rwv[i];
            }
        }
        lds_barrier();
        if (s_fail) return;
        if (next2) s_L[l & 1][tid] = lw;
        if (tid < 3 * E) ((int32_t*) &s_slotx[(l + 1) & 1][tid % E])[tid / E] = sl_next;
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

struct XcdWideKernel {
    int nbh, nbf, nlog, td;
    const void* fn;
};
const XcdWideKernel kXcdWideKernels[] = {
    {16, 6, 4, T_Q6_K, (const void*) k_decode_xcd_wide<16, 6, 4, T_Q6_K>},
    {16, 6, 4, T_Q4_K, (const void*) k_decode_xcd_wide<16, 6, 4, T_Q4_K>},
};

}  // namespace

const void* decode_xcd_wide_kernel(const DecodeStackDesc& d) {
    for (const XcdWideKernel& kk : kXcdWideKernels)
        if (d.H == 256 * kk.nbh && d.F == 256 * kk.nbf && d.E == 32 * kk.nlog && d.type_down == kk.td) return kk.fn;
    return nullptr;
}

}  // namespace qw
