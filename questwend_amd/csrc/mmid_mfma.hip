// mmid_mfma.hip -- ggml_mul_mat_id for experts with many routed rows (prefill,
// large verify batches): the Q4_K x Q8_K block products as int8 matrix-core
// (MFMA) contractions over staged super-block tiles, bit-identical to ggml.
//
// Reference: ggml_vec_dot_q4_K_q8_K, AVX2 branch (ggml/src/ggml-cpu/arch/x86/
// quants.c:2038-2115).  Per (weight row, activation row, super-block) it keeps
// eight int32 lanes, lane L holding
//     sumi_L = sum_{j=0..7} sc_j * sum_{e=0..3} q4[32 j + 4 L + e] * q8[32 j + 4 L + e]
// (maddubs pairs, madd with the sub-block scale), four min lanes
//     prod_m = mins[2m] * q8s[2m] + mins[2m+1] * q8s[2m+1],  q8s[j] = sum of q8 over sub-block j
// and then, over the super-blocks i in order, acc_L = fma(d_i, sumi_L, acc_L),
// accm_m = fma(dmin_i, prod_m, accm_m) with d = y.d * fp16(x.d),
// dmin = -y.d * fp16(x.dmin); the result is hsum_float_8(acc) + ((m0+m2)+(m1+m3)).
// This kernel computes exactly those integers on the matrix cores and replays
// the float steps lane for lane, so its outputs equal ggml's bit for bit.
//
// Matrix-core mapping.  v_mfma_i32_16x16x32_i8 (D = A x B + C, 16 x 16 x 32):
// A lane l holds weight row l % 16 and k-slots 8 (l/16) .. +8; B lane l holds
// activation row l % 16 and the same k-slots; D lane l, register r is row
// 4 (l/16) + r, activation row l % 16.  For AVX lane L the 32 k-slots are the
// 32 positions of that lane: slot 8 g + 4 h + e is sub-block j = 2 g + h,
// element 4 L + e, i.e. nibble h of qs byte 32 g + 4 L + e -- one qs dword per
// MFMA lane gives both of its sub-blocks.  The scale goes into A: with
// sc = 8 sc_hi + sc_lo (sc_hi, sc_lo <= 7), A_lo = sc_lo * q4 and
// A_hi = sc_hi * q4 fit int8 and the byte-wise products never carry, and
// sumi_L = 8 (A_hi . q8) + (A_lo . q8).  The min lanes use
// v_mfma_i32_16x16x64_i8 over the 64 positions of sub-blocks 2m and 2m+1 with
// every A byte equal to that sub-block's min.  20 MFMAs per 16 x 16 tile and
// super-block.
#include "qw_kernels.hpp"

#include <type_traits>

namespace qw {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4m __attribute__((ext_vector_type(4)));

constexpr int MF_M = 64;          // weight rows per workgroup (4 waves x 16)
constexpr uint32_t MF_WS = 144;   // LDS stride of a staged Q4_K block (9 x 16 B)
constexpr uint32_t MF_AS = 276;   // LDS stride of a staged Q8_K block (69 dwords): d at 0, qs at 16
                                  // (an odd dword stride: 16 or 32 lanes reading one offset of their
                                  // rows hit distinct banks)
constexpr int MF_AD = 69;         // dwords per staged activation row
constexpr int MF_NB_X = 1;        // 16-row activation tiles per pass: exact form (2 measured no faster)
constexpr int MF_NB_B = 4;        // block-sum form

// 16 bytes of LDS at a 4-byte aligned address.
__device__ __forceinline__ v4i lds_v4i(const uint8_t* p) {
    const uint32_t* q = (const uint32_t*) p;
    return v4i{(int) q[0], (int) q[1], (int) q[2], (int) q[3]};
}

// Waits until at most N of this wave's vector memory operations are in flight.
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Buffer resource words over [base, base + bytes) (the layout
// __builtin_amdgcn_make_buffer_rsrc builds; loads past the end return zeros).
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t) base;
    return i32x4{(int) (uint32_t) a, (int) ((uint32_t) (a >> 32) & 0xffffu), (int) bytes, 0x00020000};
}

// Buffer loads straight into LDS: lane l's 16 (4) bytes from voff + soff land at
// LDS byte lds_base + 16 l (4 l).  Written as instructions, not through the
// compiler's builtin: the compiler then inserts no wait of its own before the
// LDS reads (it would wait for every copy in flight, the prefetched stages
// included); the kernel waits with vm_wait and orders waves with a barrier.
// M0 holds the LDS base for the instruction and is restored after it.
__device__ __forceinline__ void dma_b128(i32x4 rsrc, uint32_t lds_base, uint32_t voff, uint32_t soff) {
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
        : "memory");
}
__device__ __forceinline__ void dma_b32(i32x4 rsrc, uint32_t lds_base, uint32_t voff, uint32_t soff) {
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dword %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
        : "memory");
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) { return (long) (((uint64_t) hi << 32) | lo); }

// Byte-wise products of four bytes b (each <= 15) with s (<= 7), as one packed
// 16-bit multiply: each half holds b0 + 256 b1 and b0 s < 256 never carries.
typedef unsigned short u16x2m __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t mul_bytes(uint32_t b, uint32_t s) {
    const u16x2m ss = {(unsigned short) s, (unsigned short) s};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2m, b) * ss);
}

// Raw buffer resource over [base, base + bytes): 32-bit offsets, loads past the
// end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short) 0, (int) bytes, 0x00020000);
}

// Work items: the routed rows of each heavy expert (at least mfma_min_rows)
// cut into chunks of R rows; item i is chunk c of active expert g, items in
// expert order.  Wave 0 scans the active experts' chunk counts 64 at a time and
// leaves (g, c) in s_item, g = -1 past the last item.  Splitting an expert's
// rows over workgroups keeps the longest workgroup at R rows whatever the skew
// of the routing (one expert can hold every token of the batch).
__device__ __forceinline__ void mf_item(const MmidArgs& m, int item, int R, int wave, int lane, int* s_item) {
    if (wave == 0) {
        const int n = *m.n_active;
        int run = 0, fg = -1, fc = 0;
        for (int base = 0; base < n; base += 64) {
            const int j = base + lane;
            int ch = 0;
            if (j < n) {
                const int cnt = m.active_off[j + 1] - m.active_off[j];
                ch = cnt >= m.mfma_min_rows ? (cnt + R - 1) / R : 0;
            }
            int incl = ch;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_up(incl, o);
                if (lane >= o) incl += v;
            }
            const int excl = incl - ch;
            const uint64_t hit = __ballot(item >= run + excl && item < run + incl);
            if (hit) {   // uniform
                const int src = __ffsll((unsigned long long) hit) - 1;
                fg = base + src;
                fc = item - run - __shfl(excl, src);
                break;
            }
            run += __shfl(incl, 63);
        }
        if (lane == 0) {
            s_item[0] = fg;
            s_item[1] = fc;
        }
    }
    __syncthreads();
}

// Upper bound on the items of a launch: at most min(max_active, n_pairs /
// mfma_min_rows) heavy experts, each with at most one partial chunk.
inline int64_t mf_max_items(const MmidArgs& m, int R) {
    const int64_t heavy = std::min<int64_t>(m.max_active, m.n_pairs / std::max(m.mfma_min_rows, 1));
    return heavy + m.n_pairs / R;
}

// One launch runs the matrix-core part of one mul_mat_id, or of two of the same
// type, shape and grouping (gate and up of an FFN): workgroups [0, groups) take
// m[0], [groups, 2 groups) m[1], so the second matrix's workgroups fill the CUs
// the first one's last round leaves idle.
struct MfLaunch {
    MmidArgs m[2];
    uint32_t groups;   // workgroups per matrix
};

// Workgroup b = (work item, row tile): weight rows r0 .. r0 + 63 of the expert's
// matrix against one pass of 16 NB routed activation rows (the item).  Items
// bound the longest workgroup: with one workgroup walking all of a tile's rows,
// the heaviest expert of a skewed batch (266 rows of 512 tokens) set the time of
// the whole launch.
//
// Pipeline.  Super-block i of the tile and of the pass's activation rows is
// copied by buffer loads straight into LDS (no registers in between) into stage
// buffer i % 3, two super-blocks ahead of the one being computed: a stage's
// loads have two super-blocks of matrix-core work to land.  One barrier per
// super-block: after it every wave has finished the previous super-block, whose
// buffer then takes the loads of super-block i + 2.  A wave waits for its own
// loads of super-block i (s_waitcnt vmcnt) before that barrier, so after it
// every wave's copies are in LDS.
//
// Staging layout: weight chunk q (16 B; 9 per row) at byte 16 q, from row q / 9,
// byte 16 (q % 9) of the super-block; activation dword slot u of row n (69 per
// row) at byte 4 (69 n + u), from byte 4 u - 12 (4 <= u < 68: the qs) or 0 (the
// d, and the pads) of the row's Q8_K block.  One DMA instruction covers 64
// consecutive chunks or slots, one per lane; the last activation instruction's
// slots past the rows land in the buffer's slack.
// Occupancy: the exact form (41.7 KB of LDS, ~128 VGPRs) runs three
// workgroups per CU, the block-sum form (81 KB, ~206 VGPRs) two.
template <int NB, bool EXACT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(EXACT ? 3 : 2, EXACT ? 3 : 2)))
k_mmid_mfma_q4k(MfLaunch lp) {
    const uint32_t zm = blockIdx.x >= lp.groups ? 1u : 0u;   // uniform: which matrix
    const MmidArgs& m = lp.m[zm];
    const uint32_t bid = blockIdx.x - zm * lp.groups;
    constexpr int NR = 16 * NB;               // activation rows per pass (and per item)
    constexpr int AW = (NR * MF_AD + 63) / 64;   // activation DMA instructions per stage
    constexpr int AWW = (AW + 3) / 4;         // ... per wave, at most
    constexpr int VM_STAGE = 2 + AW / 4;      // fewest DMA instructions any wave issues per stage
    static_assert(VM_STAGE <= 63, "staging shape");
    __shared__ __align__(16) uint8_t s_w0[MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_w1[MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_w2[MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_a0[AW * 256];   // NR * MF_AS and the last instruction's slack
    __shared__ __align__(16) uint8_t s_a1[AW * 256];
    __shared__ __align__(16) uint8_t s_a2[AW * 256];
    __shared__ int32_t s_arow[NR];
    __shared__ int32_t s_et[NR][2];
    __shared__ int s_item[2];
    const int tiles = (int) (m.N / MF_M);
    const int tile = (int) (bid % (uint32_t) tiles);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    mf_item(m, (int) (bid / (uint32_t) tiles), NR, wave, lane, s_item);
    const int g = s_item[0];
    if (g < 0) return;   // past the last item (light experts have none: the GEMV kernel's)
    const int p0 = m.active_off[g] + NR * s_item[1], p1 = min(m.active_off[g + 1], p0 + NR);
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) tile * MF_M;
    const int lr = lane & 15, gq = lane >> 4;   // A row / B row within a 16 x 16 tile; k-slot group
    const int nb = (int) (m.K / QK_K);
    const uint8_t* wtile = m.w + (size_t) mat * m.nb2 + (size_t) r0 * m.nb1;
    const i32x4 wrsrc = rsrc_words(wtile, (uint32_t) (MF_M * m.nb1));
    const i32x4 arsrc = rsrc_words(m.act_q, 0x7fffffffu);
    const int arow_l = 16 * wave + lr;          // this lane's A row in the staged tile
    const int ntok = p1 - p0;                   // 1 .. NR
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    if (tid < NR) {
        const int pp = p0 + (tid < ntok ? tid : 0);   // rows past ntok are staged from row 0, never written
        const int e = m.rows[2 * pp], t = m.rows[2 * pp + 1];
        s_et[tid][0] = e;
        s_et[tid][1] = t;
        s_arow[tid] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
    }
    lds_barrier();
    // this lane's source offsets (the super-block adds i * 144 / i * 292 as the scalar offset)
    uint32_t woff[3], aoff[AWW];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int q = 64 * (wave + 4 * k) + lane;
        const int qc = q < MF_M * 9 ? q : 0;
        woff[k] = (uint32_t) (qc / 9) * (uint32_t) m.nb1 + 16u * (uint32_t) (qc % 9);
    }
#pragma unroll
    for (int k = 0; k < AWW; ++k) {
        const int sl = 64 * (wave + 4 * k) + lane;
        const int slc = sl < NR * MF_AD ? sl : 0;
        const int n = slc / MF_AD, u = slc - MF_AD * n;
        aoff[k] = (uint32_t) s_arow[n] * (uint32_t) m.act_row_bytes + (u < 4 || u >= 68 ? 0u : 4u * (uint32_t) u - 12u);
    }
    auto issue = [&](uint8_t* sw, uint8_t* sa, int i) __attribute__((always_inline)) {
        // LDS bases recomputed per stage, not kept live across the loop (scalar registers)
        uint32_t lw = (uint32_t) (uintptr_t) sw, la = (uint32_t) (uintptr_t) sa;
        asm volatile("" : "+s"(lw), "+s"(la));
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (wv + 4 * k < 9) dma_b128(wrsrc, lw + 1024u * (uint32_t) (wv + 4 * k), woff[k], 144u * (uint32_t) i);
#pragma unroll
        for (int k = 0; k < AWW; ++k)
            if (wv + 4 * k < AW) dma_b32(arsrc, la + 256u * (uint32_t) (wv + 4 * k), aoff[k], 292u * (uint32_t) i);
    };

    // EXACT: per activation tile and output (D register r) the eight AVX lanes
    // and four min lanes.  Block sums: per output and tile, one chain and one
    // for the mins.
    constexpr int XT = EXACT ? NB : 1, NACC = EXACT ? 8 : NB, NACCM = EXACT ? 4 : NB;
    float acc[XT][4][NACC], accm[XT][4][NACCM];
#pragma unroll
    for (int t = 0; t < XT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int L = 0; L < NACC; ++L) acc[t][r][L] = 0.0f;
#pragma unroll
            for (int q = 0; q < NACCM; ++q) accm[t][r][q] = 0.0f;
        }
    const int nbt = (ntok + 15) / 16;   // activation tiles holding rows (uniform)

    auto compute = [&](const uint8_t* sw, const uint8_t* sa) __attribute__((always_inline)) {
        // this lane's A row: the 6-bit scales and mins of the 8 sub-blocks
        // (the utmp shuffle of quants.c:2067-2072), as bytes
        const u32x4m hdr = *(const u32x4m*) (sw + arow_l * MF_WS);
        const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
        const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        // sub-blocks 2 gq (low nibbles) and 2 gq + 1 (high nibbles) of this lane's k-slots
        const uint32_t scw = gq < 2 ? sc_lo : sc_hi;
        const uint32_t sa_ = (scw >> (16 * (gq & 1))) & 0xffu, sb_ = (scw >> (16 * (gq & 1) + 8)) & 0xffu;
        // fp16 block scales of the D rows 4 gq + r
        float xd[4], xdm[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t h0 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + r) * MF_WS);
            xd[r] = h2f((uint16_t) (h0 & 0xffff));
            xdm[r] = h2f((uint16_t) (h0 >> 16));
        }
        int mbq[4];   // min operands: sub-blocks 2q (k-slots of lane groups 0, 1) and 2q + 1 (groups 2, 3)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int sbk = 2 * q + (gq >> 1);
            const uint32_t mnw = sbk < 4 ? mn_lo : mn_hi;
            mbq[q] = (int) (((mnw >> (8 * (sbk & 3))) & 0xffu) * 0x01010101u);
        }
        if constexpr (EXACT) {
            // A operands formed once per AVX lane for all activation tiles
            float d[NB][4], dmin[NB][4];
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const float dy = *(const float*) (sa + (16 * t + lr) * MF_AS);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    d[t][r] = dy * xd[r];
                    dmin[t][r] = -dy * xdm[r];
                }
            }
#pragma unroll
            for (int L = 0; L < 8; ++L) {
                const uint32_t w = *(const uint32_t*) (sw + arow_l * MF_WS + 16 + 32 * gq + 4 * L);
                const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
                const long a_lo = pack2(mul_bytes(lo, sa_ & 7u), mul_bytes(hi, sb_ & 7u));
                const long a_hi = pack2(mul_bytes(lo, sa_ >> 3), mul_bytes(hi, sb_ >> 3));
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    if (t >= nbt) break;
                    const uint8_t* ab = sa + (16 * t + lr) * MF_AS + 16 + 64 * gq + 4 * L;
                    const long bq = pack2(*(const uint32_t*) ab, *(const uint32_t*) (ab + 32));
                    const v4i z4 = v4i{0, 0, 0, 0};
                    const v4i dlo = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, bq, z4, 0, 0, 0);
                    const v4i dhi = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, bq, z4, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[t][r][L] = __builtin_fmaf(d[t][r], (float) (8 * dhi[r] + dlo[r]), acc[t][r][L]);
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    if (t >= nbt) break;
                    const v4i bq = lds_v4i(sa + (16 * t + lr) * MF_AS + 16 + 64 * q + 16 * gq);
                    const v4i dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i{mbq[q], mbq[q], mbq[q], mbq[q]}, bq,
                                                                         v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) accm[t][r][q] = __builtin_fmaf(dmin[t][r], (float) dm[r], accm[t][r][q]);
                }
        } else {
            // this lane's A operands for the eight AVX lanes (scale digits times the
            // nibbles), formed once for all activation tiles
            long alo[8], ahi[8];
#pragma unroll
            for (int L = 0; L < 8; ++L) {
                const uint32_t w = *(const uint32_t*) (sw + arow_l * MF_WS + 16 + 32 * gq + 4 * L);
                const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
                alo[L] = pack2(mul_bytes(lo, sa_ & 7u), mul_bytes(hi, sb_ & 7u));
                ahi[L] = pack2(mul_bytes(lo, sa_ >> 3), mul_bytes(hi, sb_ >> 3));
            }
            // activation tiles in pairs: two independent MFMA accumulation chains
#pragma unroll
            for (int bp = 0; bp < NB; bp += 2) {
                if (bp >= nbt) break;
                v4i slo[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}}, shi[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
                v4i sm[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
                for (int L = 0; L < 8; ++L)
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const uint8_t* ab = sa + (16 * (bp + u) + lr) * MF_AS + 16 + 64 * gq + 4 * L;
                        const long bq = pack2(*(const uint32_t*) ab, *(const uint32_t*) (ab + 32));
                        slo[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo[L], bq, slo[u], 0, 0, 0);
                        shi[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi[L], bq, shi[u], 0, 0, 0);
                    }
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const v4i bq = lds_v4i(sa + (16 * (bp + u) + lr) * MF_AS + 16 + 64 * q + 16 * gq);
                        sm[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i{mbq[q], mbq[q], mbq[q], mbq[q]}, bq, sm[u],
                                                                      0, 0, 0);
                    }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float dy = *(const float*) (sa + (16 * (bp + u) + lr) * MF_AS);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        acc[0][r][bp + u] =
                            __builtin_fmaf(dy * xd[r], (float) (8 * shi[u][r] + slo[u][r]), acc[0][r][bp + u]);
                        accm[0][r][bp + u] = __builtin_fmaf(-dy * xdm[r], (float) sm[u][r], accm[0][r][bp + u]);
                    }
                }
            }
        }
    };
    auto stage = [&](int i, const uint8_t* cw, const uint8_t* ca, uint8_t* nw, uint8_t* na) __attribute__((always_inline)) {
        if (i + 1 < nb) vm_wait<VM_STAGE>();   // super-block i + 1's loads may stay in flight
        else vm_wait<0>();
        lds_barrier();
        if (i + 2 < nb) issue(nw, na, i + 2);
        compute(cw, ca);
    };
    issue(s_w0, s_a0, 0);
    if (nb > 1) issue(s_w1, s_a1, 1);
    for (int i = 0; i < nb; i += 3) {
        stage(i, s_w0, s_a0, s_w2, s_a2);
        if (i + 1 < nb) stage(i + 1, s_w1, s_a1, s_w0, s_a0);
        if (i + 2 < nb) stage(i + 2, s_w2, s_a2, s_w1, s_a1);
    }
    if constexpr (EXACT) {
        // hsum_float_8(acc) + ((m0 + m2) + (m1 + m3)); rows r0 + 16 wave + 4 gq .. +3 of B row 16 t + lr
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float* a = acc[t][r];
                const float hs = ((a[4] + a[0]) + (a[6] + a[2])) + ((a[5] + a[1]) + (a[7] + a[3]));
                const float* mm = accm[t][r];
                o[r] = hs + ((mm[0] + mm[2]) + (mm[1] + mm[3]));
            }
            const int row = 16 * t + lr;
            if (row < ntok) {
                const int e = s_et[row][0], tt = s_et[row][1];
                float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2) + r0 +
                            16 * wave + 4 * gq;
                *(float4*) dp = float4{o[0], o[1], o[2], o[3]};
            }
        }
    } else {
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) {
            const int row = 16 * bt + lr;
            if (row < ntok) {
                const int e = s_et[row][0], tt = s_et[row][1];
                float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2) + r0 +
                            16 * wave + 4 * gq;
                *(float4*) dp = float4{acc[0][0][bt] + accm[0][0][bt], acc[0][1][bt] + accm[0][1][bt],
                                       acc[0][2][bt] + accm[0][2][bt], acc[0][3][bt] + accm[0][3][bt]};
            }
        }
    }
}

// The block-sum form (mfma_exact == 0) of the same kernel.  Same integers, fewer
// float steps: per (weight row, activation row, super-block) the eight AVX
// lanes' sums add up in the MFMA's own int32 accumulator (sumi = sum_L sumi_L,
// the block's exact integer dot with its scales; |sumi| < 2^25), the mins
// likewise (prod = sum_m prod_m), and the float steps are
// acc = fma(y.d fp16(x.d), sumi, acc) and accm = fma(-y.d fp16(x.dmin), prod,
// accm) over the super-blocks, then acc + accm.  The integers are ggml's
// exactly; the floats round in another order (relative difference ~1e-7 of the
// terms).  Each wave keeps four 16-row activation tiles per pass (64 rows), so a
// weight row's operand is formed once for all of them and the tile is streamed
// a quarter as often.

// ---- exact Q4_K on the f16 matrix cores ------------------------------------
// The integers of the int8 exact form above, from v_mfma_f32_16x16x32_f16.  For
// AVX lane L, A lane (weight row, gq) holds sc * q4 of elements
// 64 gq + 4 L + {0, 2, 1, 3} (sub-block 2 gq, low nibbles of qs dword 8 gq + L)
// and 64 gq + 32 + 4 L + {0, 2, 1, 3} (sub-block 2 gq + 1, its high nibbles) as
// f16 (at most 63 * 15 = 945: exact); B lane (activation row, gq) holds the q8 of
// the same elements, one 16-byte chunk (gq, L) of an f16 copy of the Q8_K rows
// laid out that way (k_q8K_to_h).  Every product and partial sum is an integer
// below 2^24, so the f32 D is sumi_L exactly: one MFMA per AVX lane and tile in
// place of two int8 ones, and the float chain takes D as it is (no shift-add, no
// convert).  Min lane m: two MFMAs over chunks (m, 0..3) and (m, 4..7), A = the
// mins of sub-blocks 2m (slots 0-3) and 2m + 1 (slots 4-7).
//
// A from a qs dword w: (w & 0x000F000F) | 0x64006400 is the f16 pair
// (1024 + q4 of byte 0, 1024 + q4 of byte 2); an fma with (sc, sc) and -1024 sc
// leaves sc * q4 (one rounding of an exact integer below 2048).  High nibbles
// stay in place: 1024 + 16 q4, times sc / 16, minus 64 sc.
//
// Staging as in the int8 form, three super-blocks deep; the activation rows come
// from the f16 copy (512 bytes per row and super-block), chunk c of row n stored
// at chunk c ^ (n & 15) (16 rows read at one offset hit distinct banks), their d
// from the Q8_K rows.  ~52 KB of LDS: three workgroups per CU.
typedef _Float16 h8m __attribute__((ext_vector_type(8)));
typedef _Float16 h2m __attribute__((ext_vector_type(2)));
typedef float f4m __attribute__((ext_vector_type(4)));
constexpr int MH_NB = 1;   // 16-row activation tiles per pass of the f16 form (two measured slower, 78 KB
                           // of LDS and two workgroups per CU, and failed the bit-exact test: not used)

__device__ __forceinline__ h2m h2_bits(uint32_t x) { return __builtin_bit_cast(h2m, x); }
__device__ __forceinline__ uint32_t h2_u32(h2m x) { return __builtin_bit_cast(uint32_t, x); }

template <int NB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) k_mmid_mfma_q4k_h(MfLaunch lp) {
    static_assert(NB == 1, "one 16-row activation tile per pass (the form that is tested)");
    const uint32_t zm = blockIdx.x >= lp.groups ? 1u : 0u;   // uniform: which matrix
    const MmidArgs& m = lp.m[zm];
    const uint32_t bid = blockIdx.x - zm * lp.groups;
    constexpr int NR = 16 * NB;               // activation rows per pass (and per item)
    constexpr int AHI = NR / 2;               // f16 activation DMA instructions per stage (two rows each)
    constexpr int AHW = (AHI + 3) / 4;        // ... per wave, at most
    static_assert(AHI % 4 == 0, "activation copies spread evenly over the waves");
    // fewest DMA instructions any wave issues per stage: 2 or 3 of the 9 weight
    // ones, AHI / 4 activation ones, the d's (wave 3)
    constexpr int VM_STAGE = 2 + AHI / 4;
    __shared__ __align__(16) uint8_t s_w0[MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_w1[MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_w2[MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_h0[NR * 512];
    __shared__ __align__(16) uint8_t s_h1[NR * 512];
    __shared__ __align__(16) uint8_t s_h2[NR * 512];
    __shared__ __align__(16) float s_d0[64], s_d1[64], s_d2[64];   // NR d's (a DMA instruction's 64 slots)
    __shared__ int32_t s_arow[NR];
    __shared__ int32_t s_et[NR][2];
    __shared__ int s_item[2];
    const int tiles = (int) (m.N / MF_M);
    const int tile = (int) (bid % (uint32_t) tiles);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    mf_item(m, (int) (bid / (uint32_t) tiles), NR, wave, lane, s_item);
    const int g = s_item[0];
    if (g < 0) return;   // past the last item
    const int p0 = m.active_off[g] + NR * s_item[1], p1 = min(m.active_off[g + 1], p0 + NR);
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) tile * MF_M;
    const int lr = lane & 15, gq = lane >> 4;
    const int nb = (int) (m.K / QK_K);
    const uint8_t* wtile = m.w + (size_t) mat * m.nb2 + (size_t) r0 * m.nb1;
    const i32x4 wrsrc = rsrc_words(wtile, (uint32_t) (MF_M * m.nb1));
    const i32x4 hrsrc = rsrc_words(m.act_h, 0x7fffffffu);
    const i32x4 arsrc = rsrc_words(m.act_q, 0x7fffffffu);
    const int arow_l = 16 * wave + lr;
    const int ntok = p1 - p0;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    if (tid < NR) {
        const int pp = p0 + (tid < ntok ? tid : 0);   // rows past ntok are staged from row 0, never written
        const int e = m.rows[2 * pp], t = m.rows[2 * pp + 1];
        s_et[tid][0] = e;
        s_et[tid][1] = t;
        s_arow[tid] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
    }
    lds_barrier();
    uint32_t woff[3], hoff[AHW], doff = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int q = 64 * (wave + 4 * k) + lane;
        const int qc = q < MF_M * 9 ? q : 0;
        woff[k] = (uint32_t) (qc / 9) * (uint32_t) m.nb1 + 16u * (uint32_t) (qc % 9);
    }
#pragma unroll
    for (int k = 0; k < AHW; ++k) {
        const int ii = wave + 4 * k;                      // instruction: rows 2 ii, 2 ii + 1
        const int n = ii < AHI ? 2 * ii + (lane >> 5) : 0, c = lane & 31;
        hoff[k] = (uint32_t) s_arow[n] * (uint32_t) (2 * m.K) + 16u * (uint32_t) (c ^ (n & 15));
    }
    if (lane < NR) doff = (uint32_t) s_arow[lane] * (uint32_t) m.act_row_bytes;
    auto issue = [&](uint8_t* sw, uint8_t* sh, float* sd, int i) __attribute__((always_inline)) {
        uint32_t lw = (uint32_t) (uintptr_t) sw, lh = (uint32_t) (uintptr_t) sh, ld = (uint32_t) (uintptr_t) sd;
        asm volatile("" : "+s"(lw), "+s"(lh), "+s"(ld));
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (wv + 4 * k < 9) dma_b128(wrsrc, lw + 1024u * (uint32_t) (wv + 4 * k), woff[k], 144u * (uint32_t) i);
#pragma unroll
        for (int k = 0; k < AHW; ++k)
            if (wv + 4 * k < AHI) dma_b128(hrsrc, lh + 1024u * (uint32_t) (wv + 4 * k), hoff[k], 512u * (uint32_t) i);
        if (wv == 3 && lane < NR) dma_b32(arsrc, ld, doff, 292u * (uint32_t) i);
    };

    float acc[NB][4][8], accm[NB][4][4];
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int L = 0; L < 8; ++L) acc[t][r][L] = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) accm[t][r][q] = 0.0f;
        }
    const int nbt = (ntok + 15) / 16;   // activation tiles holding rows (uniform)

    // 0x64006400 as a register operand, so that (w & mask) | it is one v_and_or_b32
    uint32_t hmag = 0x64006400u;
    asm volatile("" : "+v"(hmag));
    auto compute = [&](const uint8_t* sw, const uint8_t* sh, const float* sd) __attribute__((always_inline)) {
        // this lane's A row: the 6-bit scales and mins of the 8 sub-blocks (quants.c:2067-2072)
        const u32x4m hdr = *(const u32x4m*) (sw + arow_l * MF_WS);
        const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
        const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        // sub-blocks 2 gq (low nibbles) and 2 gq + 1 (high nibbles) of this lane's k-slots
        const uint32_t scw = gq < 2 ? sc_lo : sc_hi;
        const uint32_t sab = (scw >> (16 * (gq & 1))) & 0xffffu;        // sc_a | sc_b << 8
        // (sc_a, sc_a), (sc_b / 16, sc_b / 16) and the offsets as f16 pairs
        const h2m pa = h2_bits(__builtin_amdgcn_perm(0u, sab, 0x0c000c00u) | 0x64006400u) - h2m{1024, 1024};
        const h2m pb = h2_bits(__builtin_amdgcn_perm(0u, sab, 0x0c010c01u) | 0x64006400u) - h2m{1024, 1024};
        const h2m S_lo = pa, C_lo = pa * h2m{-1024, -1024};
        const h2m S_hi = pb * h2m{0.0625, 0.0625}, C_hi = pb * h2m{-64, -64};
        float xd[4], xdm[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t h0 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + r) * MF_WS);
            xd[r] = h2f((uint16_t) (h0 & 0xffff));
            xdm[r] = h2f((uint16_t) (h0 >> 16));
        }
        float d[NB][4], dmin[NB][4];
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const float dy = sd[16 * t + lr];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                d[t][r] = dy * xd[r];
                dmin[t][r] = -dy * xdm[r];
            }
        }
#pragma unroll
        for (int L = 0; L < 8; ++L) {
            const uint32_t w = *(const uint32_t*) (sw + arow_l * MF_WS + 16 + 32 * gq + 4 * L);
            const uint32_t v = w >> 8;
            const h2m a0 = __builtin_elementwise_fma(h2_bits((w & 0x000F000Fu) | hmag), S_lo, C_lo);
            const h2m a1 = __builtin_elementwise_fma(h2_bits((v & 0x000F000Fu) | hmag), S_lo, C_lo);
            const h2m a2 = __builtin_elementwise_fma(h2_bits((w & 0x00F000F0u) | hmag), S_hi, C_hi);
            const h2m a3 = __builtin_elementwise_fma(h2_bits((v & 0x00F000F0u) | hmag), S_hi, C_hi);
            const h8m A = __builtin_bit_cast(h8m, u32x4m{h2_u32(a0), h2_u32(a1), h2_u32(a2), h2_u32(a3)});
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                if (t >= nbt) break;
                const int n = 16 * t + lr;
                const h8m B = *(const h8m*) (sh + n * 512 + 16 * ((8 * gq + L) ^ (n & 15)));
                const f4m D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, f4m{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[t][r][L] = __builtin_fmaf(d[t][r], D[r], acc[t][r][L]);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // (m_2q, m_2q) and (m_2q+1, m_2q+1) as f16 pairs
            const uint32_t mnw = q < 2 ? mn_lo : mn_hi;
            const uint32_t b0 = (uint32_t) (2 * (q & 1)), b1 = b0 + 1;
            const h2m m0 = h2_bits(__builtin_amdgcn_perm(0u, mnw, 0x0c000c00u | b0 | (b0 << 16)) | 0x64006400u) -
                           h2m{1024, 1024};
            const h2m m1 = h2_bits(__builtin_amdgcn_perm(0u, mnw, 0x0c000c00u | b1 | (b1 << 16)) | 0x64006400u) -
                           h2m{1024, 1024};
            const h8m Am = __builtin_bit_cast(h8m, u32x4m{h2_u32(m0), h2_u32(m0), h2_u32(m1), h2_u32(m1)});
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                if (t >= nbt) break;
                const int n = 16 * t + lr;
                const h8m B0 = *(const h8m*) (sh + n * 512 + 16 * ((8 * q + gq) ^ (n & 15)));
                const h8m B1 = *(const h8m*) (sh + n * 512 + 16 * ((8 * q + 4 + gq) ^ (n & 15)));
                f4m Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(Am, B0, f4m{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(Am, B1, Dm, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) accm[t][r][q] = __builtin_fmaf(dmin[t][r], Dm[r], accm[t][r][q]);
            }
        }
    };
    auto stage = [&](int i, const uint8_t* cw, const uint8_t* ch, const float* cd, uint8_t* nw, uint8_t* nh,
                     float* nd) __attribute__((always_inline)) {
        if (i + 1 < nb) vm_wait<VM_STAGE>();   // super-block i + 1's loads may stay in flight
        else vm_wait<0>();
        lds_barrier();
        if (i + 2 < nb) issue(nw, nh, nd, i + 2);
        compute(cw, ch, cd);
    };
    issue(s_w0, s_h0, s_d0, 0);
    if (nb > 1) issue(s_w1, s_h1, s_d1, 1);
    for (int i = 0; i < nb; i += 3) {
        stage(i, s_w0, s_h0, s_d0, s_w2, s_h2, s_d2);
        if (i + 1 < nb) stage(i + 1, s_w1, s_h1, s_d1, s_w0, s_h0, s_d0);
        if (i + 2 < nb) stage(i + 2, s_w2, s_h2, s_d2, s_w1, s_h1, s_d1);
    }
    // hsum_float_8(acc) + ((m0 + m2) + (m1 + m3)); rows r0 + 16 wave + 4 gq .. +3 of B row 16 t + lr
#pragma unroll
    for (int t = 0; t < NB; ++t) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float* a = acc[t][r];
            const float hs = ((a[4] + a[0]) + (a[6] + a[2])) + ((a[5] + a[1]) + (a[7] + a[3]));
            const float* mm = accm[t][r];
            o[r] = hs + ((mm[0] + mm[2]) + (mm[1] + mm[3]));
        }
        const int row = 16 * t + lr;
        if (row < ntok) {
            const int e = s_et[row][0], tt = s_et[row][1];
            float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2) + r0 +
                        16 * wave + 4 * gq;
            *(float4*) dp = float4{o[0], o[1], o[2], o[3]};
        }
    }
}

// The f16 copy k_mmid_mfma_q4k_h reads: per activation row (K values at out + r K)
// and super-block, 32 chunks of 16 bytes; chunk 8 g + L holds the q8 of elements
// 64 g + 4 L + {0, 2, 1, 3} and 64 g + 32 + 4 L + {0, 2, 1, 3} (the A operands'
// order of qs dword 8 g + L's low and high nibbles).  A thread writes one chunk.
__global__ void k_q8K_to_h(const uint8_t* __restrict__ q, size_t row_bytes, int64_t K, int64_t rows,
                           _Float16* __restrict__ out) {
    const int64_t per_row = K / 8;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * per_row) return;
    const int64_t r = i / per_row, ci = i - r * per_row, bb = ci / 32;
    const int c = (int) (ci % 32), g = c >> 3, L = c & 7;
    const uint8_t* src = q + (size_t) r * row_bytes + 292 * (size_t) bb + 4 + 64 * g + 4 * L;
    const uint32_t u0 = *(const uint32_t*) src, u1 = *(const uint32_t*) (src + 32);
    auto b = [](uint32_t u, int k) { return (_Float16) (float) (int8_t) (u >> (8 * k)); };
    *(h8m*) (out + (size_t) r * K + 8 * ci) = h8m{b(u0, 0), b(u0, 2), b(u0, 1), b(u0, 3), b(u1, 0), b(u1, 2), b(u1, 1), b(u1, 3)};
}

int launch_q8K_to_f16(const uint8_t* q, size_t row_bytes, int64_t K, int64_t rows, uint16_t* out, hipStream_t stream) {
    if (K % QK_K != 0 || rows <= 0 || row_bytes % 4 != 0 || ((uintptr_t) q & 3) || ((uintptr_t) out & 15)) return -2;
    const int64_t n = rows * (K / 8);
    hipLaunchKernelGGL(k_q8K_to_h, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, stream, q, row_bytes, K, rows,
                       (_Float16*) out);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ---- exact Q4_K on the f16 matrix cores, persistent -------------------------
// k_mmid_mfma_q4k_hp computes what k_mmid_mfma_q4k_h computes -- the same A and
// B operands, one v_mfma_f32_16x16x32_f16 per AVX lane and tile, the same fp32
// steps in the same order, so the same bits -- with another schedule:
//  - a grid of two workgroups per CU walks the work units u = b, b + grid, ...
//    A unit is (item, 64-row weight tile) of one of the launch's one or two
//    matrices; an item is up to 32 routed rows of one heavy expert.  Each
//    workgroup builds the item table (first item of each active expert) once in
//    LDS; a unit's expert is a count over that table.
//  - the three-stage copy pipeline runs on across units: while the last
//    super-blocks of a unit are computed, the first ones of the next unit are
//    being copied.  The next unit's (e, t) pairs are copied into LDS by the same
//    DMA path one super-block ahead, so they are counted by the same waits.
//  - two 16-row activation tiles per item: each A operand (sc * q4 of 16 weight
//    rows) serves 32 activation rows.  A last item of at most 16 rows computes
//    one tile; those items are numbered after all others, so a workgroup runs
//    its two-tile units, then its one-tile units, each as straight-line code
//    (the tile count a compile-time constant: no branch between a matrix-core
//    instruction and the reads of its result, and no register shuffling of the
//    accumulators between two code paths at every super-block).
//  - activation rows i and i + 16 share one DMA instruction and sit 1040 bytes
//    per pair apart (16 bytes of pad): the 16 rows a tile reads at one chunk
//    offset fall on distinct LDS banks, and every B read is the lane's base plus
//    a constant.
// ~81 KB of LDS: two workgroups per CU.  Needs K >= 768 (three super-blocks: the
// next unit's pairs land one super-block before they are used) and at most
// MP_MAXG active bins.  Measured at configs[2] (T = 512, Zipf-skewed routing):
// gate + up 170 us, down 104 us per launch against 174 / 114 us for
// k_mmid_mfma_q4k_h; counters put it at ~56 % VALU-busy and ~16 % MFMA-busy,
// with waves waiting a third of their cycles (two waves per SIMD).
constexpr int MP_NR = 32;             // activation rows per item (two 16-row tiles)
constexpr uint32_t MP_HS = 1040;      // LDS bytes per activation DMA instruction (rows i, i + 16, pad)
constexpr int MP_MAXG = 128;          // active bins the item table holds
constexpr int MP_VM = 6;              // fewest DMA instructions a wave issues per stage (waves 1, 2: 2 + 4)

struct MpUnit {
    int z, ntok, ok, p0;
    uint32_t r0;
    i32x4 wrsrc;
};

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_mmid_mfma_q4k_hp(MfLaunch lp, uint32_t nz) {
    __shared__ __align__(16) uint8_t s_w[3][MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_h[3][16 * MP_HS];
    __shared__ __align__(16) float s_d[3][MP_NR];
    __shared__ __align__(16) int32_t s_meta[2][2 * MP_NR];   // (e, t) of a unit's 32 rows
    __shared__ int32_t s_if[MP_MAXG + 1], s_if1[MP_MAXG + 1], s_aoff[MP_MAXG + 1], s_mat[2][MP_MAXG];
    const MmidArgs& m0 = lp.m[0];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int lr = lane & 15, gq = lane >> 4;
    const int nb = (int) (m0.K / QK_K), tiles = (int) (m0.N / MF_M);

    // ---- the item table.  An active bin's rows (at least mfma_min_rows) are cut
    // into items of 32 rows; a last item of 17..31 rows counts with the full ones
    // (two-tile items, s_if[g] = the bin's first), one of 1..16 rows is a one-tile
    // item (s_if1[g] = its index among those).  Two-tile items come first.
    int n = __builtin_amdgcn_readfirstlane(*(const volatile int32_t*) m0.n_active);
    n = n < MP_MAXG ? n : MP_MAXG;   // (the host bounds max_active by MP_MAXG)
    if (wave == 0) {
        int run = 0, run1 = 0;
        for (int base = 0; base <= n; base += 64) {
            const int j = base + lane;
            int ch = 0, c1 = 0;
            if (j < n) {
                const int cnt = m0.active_off[j + 1] - m0.active_off[j];
                if (cnt >= m0.mfma_min_rows) {
                    const int rem = cnt % MP_NR;
                    ch = cnt / MP_NR + (rem > 16 ? 1 : 0);
                    c1 = rem > 0 && rem <= 16 ? 1 : 0;
                }
            }
            int incl = ch, incl1 = c1;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_up(incl, o), v1 = __shfl_up(incl1, o);
                if (lane >= o) {
                    incl += v;
                    incl1 += v1;
                }
            }
            if (j <= n) {
                s_if[j] = run + incl - ch;
                s_if1[j] = run1 + incl1 - c1;
                s_aoff[j] = m0.active_off[j];
            }
            run += __shfl(incl, 63);
            run1 += __shfl(incl1, 63);
        }
    } else if (wave <= 2 && (uint32_t) (wave - 1) < nz) {
        const MmidArgs& mz = lp.m[wave - 1];
        for (int j = lane; j < n; j += 64) {
            const int bin = mz.active[j];
            int64_t mat = bin;
            if (mz.slot_of) mat = bin < mz.n_slot_of ? mz.slot_of[bin] : -1;
            s_mat[wave - 1][j] = (mat >= 0 && mat < mz.n_as) ? (int) mat : -1;
        }
    }
    __syncthreads();
    const int n2 = __builtin_amdgcn_readfirstlane(s_if[n]), n1 = __builtin_amdgcn_readfirstlane(s_if1[n]);
    const int U2 = n2 * tiles * (int) nz, total = U2 + n1 * tiles * (int) nz;
    const int P = (int) gridDim.x, b = (int) blockIdx.x;
    const int my_units = total > b ? (total - b + P - 1) / P : 0;
    if (my_units == 0) return;

    const int64_t b_ne1 = m0.b_ne1;
    const i32x4 hrsrc = rsrc_words(m0.act_h, 0x7fffffffu);
    const i32x4 arsrc = rsrc_words(m0.act_q, 0x7fffffffu);
    const i32x4 prsrc = rsrc_words(m0.rows, (uint32_t) (8 * m0.n_pairs));
    // unit u: its matrix, rows and weight tile (uniform).  Units [0, U2) are the
    // two-tile items' (matrix, item, tile), then the one-tile items'.  (Units
    // dealt to the XCDs by item chunks, for L2 reuse, measured slower.)
    auto decode = [&](int u) __attribute__((always_inline)) {
        MpUnit r;
        const bool one = u >= U2;
        const int uc = one ? u - U2 : u, ni = one ? n1 : n2;
        r.z = uc >= ni * tiles ? 1 : 0;
        const int uu = uc - r.z * ni * tiles, item = uu / tiles, tile = uu - item * tiles;
        const int32_t* tab = one ? s_if1 : s_if;
        int g = 0;
        for (int j0 = 1; j0 <= n; j0 += 64) {
            const int j = j0 + lane;
            g += __popcll(__ballot(j <= n && tab[j] <= item));
        }
        g = __builtin_amdgcn_readfirstlane(g);
        const int a0 = s_aoff[g], a1 = s_aoff[g + 1];
        r.p0 = __builtin_amdgcn_readfirstlane(one ? a0 + MP_NR * ((a1 - a0) / MP_NR) : a0 + MP_NR * (item - s_if[g]));
        const int ntok = a1 - r.p0;
        r.ntok = __builtin_amdgcn_readfirstlane(ntok < MP_NR ? ntok : MP_NR);
        const int mat = __builtin_amdgcn_readfirstlane(s_mat[r.z][g]);
        r.ok = mat >= 0;
        r.r0 = (uint32_t) tile * MF_M;
        const MmidArgs& mz = lp.m[r.z];
        const uint8_t* wt = mz.w + (size_t) (mat >= 0 ? mat : 0) * mz.nb2 + (size_t) r.r0 * mz.nb1;
        const i32x4 w4 = rsrc_words(wt, (uint32_t) (MF_M * mz.nb1));
        r.wrsrc = i32x4{__builtin_amdgcn_readfirstlane(w4.x), __builtin_amdgcn_readfirstlane(w4.y),
                        __builtin_amdgcn_readfirstlane(w4.z), __builtin_amdgcn_readfirstlane(w4.w)};
        return r;
    };
    // this lane's copy offsets for a unit whose (e, t) pairs are in s_meta[mb]
    uint32_t woff[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int q = 64 * (wave + 4 * k) + lane;
        const int qc = q < MF_M * 9 ? q : 0;
        woff[k] = (uint32_t) (qc / 9) * (uint32_t) m0.nb1 + 16u * (uint32_t) (qc % 9);
    }
    auto arow = [&](int mb, int nn) __attribute__((always_inline)) {
        // (32-bit: slot e >= 0 and 1 <= b_ne1 <= 65535 -- mp_ok -- give e % b_ne1 without
        // the 64-bit division's ~130 instructions per call)
        const uint32_t e = (uint32_t) s_meta[mb][2 * nn], t = (uint32_t) s_meta[mb][2 * nn + 1];
        const uint32_t bn = (uint32_t) b_ne1;
        const uint32_t er = bn == 1u ? 0u : e < bn ? e : e % bn;
        return er + t * bn;
    };
    auto lane_offs = [&](int mb, int ntok, uint32_t (&ho)[4], uint32_t& dof) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int nrow = wave + 4 * k + 16 * (lane >> 5);
            ho[k] = arow(mb, nrow < ntok ? nrow : 0) * (uint32_t) (2 * m0.K) + 16u * (uint32_t) (lane & 31);
        }
        dof = arow(mb, lane < ntok && lane < MP_NR ? lane : 0) * (uint32_t) m0.act_row_bytes;
    };
    // copies of super-block i of a unit into stage buffer sb
    auto issue = [&](int sb, const MpUnit& U, const uint32_t (&ho)[4], uint32_t dof, int i) __attribute__((always_inline)) {
        uint32_t lw = (uint32_t) (uintptr_t) s_w[sb], lh = (uint32_t) (uintptr_t) s_h[sb];
        uint32_t ld = (uint32_t) (uintptr_t) s_d[sb];
        asm volatile("" : "+s"(lw), "+s"(lh), "+s"(ld));
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (wv + 4 * k < 9) dma_b128(U.wrsrc, lw + 1024u * (uint32_t) (wv + 4 * k), woff[k], 144u * (uint32_t) i);
#pragma unroll
        for (int k = 0; k < 4; ++k) dma_b128(hrsrc, lh + MP_HS * (uint32_t) (wv + 4 * k), ho[k], 512u * (uint32_t) i);
        if (wv == 3 && lane < MP_NR) dma_b32(arsrc, ld, dof, 292u * (uint32_t) i);
    };

    float acc[2][4][8], accm[2][4][4];
    auto zero = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int L = 0; L < 8; ++L) acc[t][r][L] = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) accm[t][r][q] = 0.0f;
            }
    };
    uint32_t hmag = 0x64006400u;
    asm volatile("" : "+v"(hmag));
    const int arow_l = 16 * wave + lr;
    // NBT activation tiles (1 or 2, a compile-time constant): straight-line code
    // from each matrix-core instruction to the reads of its result.  (With the tile
    // count tested inside the unrolled loops, the compiler put its wait states for
    // the matrix-core result only on the path that computes the second tile; the
    // branch around it read the first tile's result too early.)
    auto compute = [&](int sb, auto nbt_c) __attribute__((always_inline)) {
        constexpr int NBT = decltype(nbt_c)::value;
        const uint8_t* sw = s_w[sb];
        const uint8_t* sh = s_h[sb] + MP_HS * (uint32_t) lr;   // this lane's rows: lr (tile 0), lr + 16 (tile 1)
        const float* sd = s_d[sb];
        // this lane's A row: the 6-bit scales and mins of the 8 sub-blocks (quants.c:2067-2072);
        // the fp16 d / dmin of the four rows of its D registers; the activation rows' d.
        // All read before any is used (one LDS wait: the empty asm takes them all).
        uint32_t hx0 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + 0) * MF_WS);
        uint32_t hx1 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + 1) * MF_WS);
        uint32_t hx2 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + 2) * MF_WS);
        uint32_t hx3 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + 3) * MF_WS);
        float dy0 = sd[lr], dy1 = NBT > 1 ? sd[16 + lr] : 0.0f;
        const u32x4m hdr = *(const u32x4m*) (sw + arow_l * MF_WS);
        uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w, sx = hdr.x;
        // and the 8 quant words of its 32-byte group gq (one per AVX lane)
        u32x4m wq0 = *(const u32x4m*) (sw + arow_l * MF_WS + 16 + 32 * gq);
        u32x4m wq1 = *(const u32x4m*) (sw + arow_l * MF_WS + 32 + 32 * gq);
        asm volatile("" : "+v"(sx), "+v"(s0), "+v"(s1), "+v"(s2), "+v"(hx0), "+v"(hx1), "+v"(hx2), "+v"(hx3), "+v"(dy0),
                     "+v"(dy1), "+v"(wq0), "+v"(wq1));
        const uint32_t wl[8] = {wq0.x, wq0.y, wq0.z, wq0.w, wq1.x, wq1.y, wq1.z, wq1.w};
        const uint32_t hxr[4] = {hx0, hx1, hx2, hx3};
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
        const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        const uint32_t scw = gq < 2 ? sc_lo : sc_hi;
        const uint32_t sab = (scw >> (16 * (gq & 1))) & 0xffffu;
        const h2m pa = h2_bits(__builtin_amdgcn_perm(0u, sab, 0x0c000c00u) | 0x64006400u) - h2m{1024, 1024};
        const h2m pb = h2_bits(__builtin_amdgcn_perm(0u, sab, 0x0c010c01u) | 0x64006400u) - h2m{1024, 1024};
        const h2m S_lo = pa, C_lo = pa * h2m{-1024, -1024};
        const h2m S_hi = pb * h2m{0.0625, 0.0625}, C_hi = pb * h2m{-64, -64};
        float xd[4], xdm[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            xd[r] = h2f((uint16_t) (hxr[r] & 0xffff));
            xdm[r] = h2f((uint16_t) (hxr[r] >> 16));
        }
        float d[2][4], dmin[2][4];
#pragma unroll
        for (int t = 0; t < NBT; ++t) {
            const float dy = t == 0 ? dy0 : dy1;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                d[t][r] = dy * xd[r];
                dmin[t][r] = -dy * xdm[r];
            }
        }
        // software-pipelined over the AVX lanes: lane L's matrix-core products are
        // issued before lane L - 1's fp32 steps, so each result is read an
        // iteration after its instruction (the same operations per accumulator)
        // (the B operands are read from LDS one step ahead of their products)
        f4m Dp[NBT];
        h8m Bc[NBT];
#pragma unroll
        for (int t = 0; t < NBT; ++t) Bc[t] = *(const h8m*) (sh + 512 * t + 16 * (8 * gq));
#pragma unroll
        for (int L = 0; L < 8; ++L) {
            const uint32_t w = wl[L];
            h8m Bn[NBT];
#pragma unroll
            for (int t = 0; t < NBT; ++t)
                Bn[t] = *(const h8m*) (sh + 512 * t + 16 * (L < 7 ? 8 * gq + L + 1 : gq));
            __builtin_amdgcn_sched_barrier(0);   // (keeps those reads issued here, a step ahead)
            const uint32_t v = w >> 8;
            const h2m a0 = __builtin_elementwise_fma(h2_bits((w & 0x000F000Fu) | hmag), S_lo, C_lo);
            const h2m a1 = __builtin_elementwise_fma(h2_bits((v & 0x000F000Fu) | hmag), S_lo, C_lo);
            const h2m a2 = __builtin_elementwise_fma(h2_bits((w & 0x00F000F0u) | hmag), S_hi, C_hi);
            const h2m a3 = __builtin_elementwise_fma(h2_bits((v & 0x00F000F0u) | hmag), S_hi, C_hi);
            const h8m A = __builtin_bit_cast(h8m, u32x4m{h2_u32(a0), h2_u32(a1), h2_u32(a2), h2_u32(a3)});
            f4m Dc[NBT];
#pragma unroll
            for (int t = 0; t < NBT; ++t)
                Dc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bc[t], f4m{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            if (L > 0) {
#pragma unroll
                for (int t = 0; t < NBT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][r][L - 1] = __builtin_fmaf(d[t][r], Dp[t][r], acc[t][r][L - 1]);
            }
#pragma unroll
            for (int t = 0; t < NBT; ++t) {
                Dp[t] = Dc[t];
                Bc[t] = Bn[t];   // (after lane 7: min lane 0's first operand, chunk gq)
            }
        }
#pragma unroll
        for (int t = 0; t < NBT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r][7] = __builtin_fmaf(d[t][r], Dp[t][r], acc[t][r][7]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t mnw = q < 2 ? mn_lo : mn_hi;
            const uint32_t b0 = (uint32_t) (2 * (q & 1)), b1 = b0 + 1;
            const h2m mm0 = h2_bits(__builtin_amdgcn_perm(0u, mnw, 0x0c000c00u | b0 | (b0 << 16)) | 0x64006400u) -
                            h2m{1024, 1024};
            const h2m mm1 = h2_bits(__builtin_amdgcn_perm(0u, mnw, 0x0c000c00u | b1 | (b1 << 16)) | 0x64006400u) -
                            h2m{1024, 1024};
            const h8m Am = __builtin_bit_cast(h8m, u32x4m{h2_u32(mm0), h2_u32(mm0), h2_u32(mm1), h2_u32(mm1)});
            // Bc holds chunk 8 q + gq of each tile (read a step ahead); chunk 8 q + 4 + gq
            // is read here, and the next min lane's first chunk for the step after
            h8m B1[NBT], Bn[NBT];
#pragma unroll
            for (int t = 0; t < NBT; ++t) {
                B1[t] = *(const h8m*) (sh + 512 * t + 16 * (8 * q + 4 + gq));
                Bn[t] = *(const h8m*) (sh + 512 * t + 16 * (q < 3 ? 8 * (q + 1) + gq : gq));
            }
            __builtin_amdgcn_sched_barrier(0);
            f4m Dc[NBT];
#pragma unroll
            for (int t = 0; t < NBT; ++t) {
                Dc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Am, Bc[t], f4m{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                Dc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Am, B1[t], Dc[t], 0, 0, 0);
            }
            if (q > 0) {   // (min lane q - 1's fp32 steps, pipelined as above)
#pragma unroll
                for (int t = 0; t < NBT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        accm[t][r][q - 1] = __builtin_fmaf(dmin[t][r], Dp[t][r], accm[t][r][q - 1]);
            }
#pragma unroll
            for (int t = 0; t < NBT; ++t) {
                Dp[t] = Dc[t];
                Bc[t] = Bn[t];
            }
        }
#pragma unroll
        for (int t = 0; t < NBT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) accm[t][r][3] = __builtin_fmaf(dmin[t][r], Dp[t][r], accm[t][r][3]);
    };
    // hsum_float_8(acc) + ((m0 + m2) + (m1 + m3)) of a finished unit; weight rows
    // r0 + 16 wave + 4 gq .. +3, activation rows lr and 16 + lr
    auto finish = [&](const MpUnit& U, int mb, auto nbt_c) __attribute__((always_inline)) {
        constexpr int NBT = decltype(nbt_c)::value;
        const MmidArgs& mz = lp.m[U.z];
        if (!U.ok) {
            if (tid == 0 && mz.status) atomicOr(mz.status, 4);
            return;
        }
#pragma unroll
        for (int t = 0; t < NBT; ++t) {
            const int row = 16 * t + lr;
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float* a = acc[t][r];
                const float hs = ((a[4] + a[0]) + (a[6] + a[2])) + ((a[5] + a[1]) + (a[7] + a[3]));
                const float* mm = accm[t][r];
                o[r] = hs + ((mm[0] + mm[2]) + (mm[1] + mm[3]));
            }
            if (row < U.ntok) {
                const int e = s_meta[mb][2 * row], tt = s_meta[mb][2 * row + 1];
                float* dp = (float*) ((char*) mz.dst + (size_t) e * mz.dst_nb1 + (size_t) tt * mz.dst_nb2) + U.r0 +
                            16 * wave + 4 * gq;
                *(float4*) dp = float4{o[0], o[1], o[2], o[3]};
            }
        }
    };

    // ---- prologue: the first unit's pairs, then its super-blocks 0 and 1
    MpUnit cur = decode(b), nxt = cur;
    if (wv == 0) dma_b32(prsrc, (uint32_t) (uintptr_t) s_meta[0], 4u * (uint32_t) lane, 8u * (uint32_t) cur.p0);
    vm_wait<0>();
    lds_barrier();
    uint32_t ho[4], dof, hn[4], dn = 0;
    lane_offs(0, cur.ntok, ho, dof);
#pragma unroll
    for (int k = 0; k < 4; ++k) hn[k] = ho[k];
    zero();
    issue(0, cur, ho, dof, 0);
    issue(1, cur, ho, dof, 1);
    const int S = my_units * nb;
    int i = 0, j = 0, sb = 0, s = 0;
    // one step: super-block i of unit j.  The unit's tile count is a template
    // argument: a workgroup meets its two-tile units first, then its one-tile ones.
    auto step = [&](auto nbt_c) __attribute__((always_inline)) {
        if (s + 1 < S) vm_wait<MP_VM>();   // super-block s + 1's copies may stay in flight
        else vm_wait<0>();
        lds_barrier();
        const bool more = j + 1 < my_units;
        if (i == 0 && more) {   // the next unit's pairs: copied before this step's super-block copies
            nxt = decode(b + (j + 1) * P);
            if (wv == 0)
                dma_b32(prsrc, (uint32_t) (uintptr_t) s_meta[(j + 1) & 1], 4u * (uint32_t) lane, 8u * (uint32_t) nxt.p0);
        }
        if (i == 1 && more) lane_offs((j + 1) & 1, nxt.ntok, hn, dn);   // (landed: waited for above)
        if (s + 2 < S) {
            const int i2 = i + 2, sb2 = sb == 0 ? 2 : sb - 1;
            if (i2 < nb) issue(sb2, cur, ho, dof, i2);
            else issue(sb2, nxt, hn, dn, i2 - nb);
        }
        compute(sb, nbt_c);
        if (++i == nb) {
            finish(cur, j & 1, nbt_c);
            zero();
            cur = nxt;
#pragma unroll
            for (int k = 0; k < 4; ++k) ho[k] = hn[k];
            dof = dn;
            i = 0;
            ++j;
        }
        sb = sb == 2 ? 0 : sb + 1;
        ++s;
    };
    while (s < S && cur.ntok > 16) step(std::integral_constant<int, 2>{});
    while (s < S) step(std::integral_constant<int, 1>{});
}


// Q6_K x Q8_K on the matrix cores, block-sum form only: the down projections of
// the layer entry points under QWMOE_MFMA_AUTO, every projection under
// QWMOE_MFMA_BLOCK_SUM.  (Replaying ggml's eight float lanes for Q6_K is not
// done on the matrix cores; the exact form keeps Q6_K on the GEMV.)
//
// Reference: ggml_vec_dot_q6_K_q8_K (ggml/src/ggml-cpu/arch/x86/quants.c:
// 2426-2508).  Its integers, per (weight row, activation row, super-block):
//     sumi = sum_{j<16} sc_j * sum_{e<16} (q6[16 j + e] - 32) * q8[16 j + e]
// with q6 = ql nibble | qh 2-bit field << 4 (the dequantize_row_q6_K order:
// element 128 n + 32 c + l of half n is nibble c >> 1 of ql[64 n + 32 (c & 1) +
// l] and bits 2c of qh[32 n + l]); here acc = fma(y.d * fp16(x.d), sumi, acc).
//
// Matrix-core mapping: v_mfma_i32_32x32x16_i8, K = 16 = one sub-block, so D
// holds each sub-block's dot and its scale multiplies after (sc_j * q6 does not
// fit int8).  A = 32 activation rows (lane l: row l % 32, elements 8 (l / 32)
// .. +8 of the sub-block), B = 32 weight rows (the same elements); D lane l,
// register r: weight row l % 32, activation row 8 (r / 4) + 4 (l / 32) + r % 4.
// Each lane thus owns one weight row of D and that row's scale.  The int32 sums
// are exact (|sumi| < 2^28).
//
// Workgroup: 128 weight rows x 32 activation rows (one work item), wave w takes
// weight rows 32 w .. +32 (a tile past N leaves its last waves idle; 32-row
// items keep the padding of partly filled items small).  Two stage buffers:
// super-block i + 1 is copied into LDS while i is computed.  A Q6_K block (210
// B) starts 2 bytes past a dword boundary in every other super-block, so a row's
// block is staged as the 53 dwords from the dword at or below its start (s = 0
// or 2 bytes before it); with s = 0 the 53rd dword would reach past the block
// (and, for the matrix's last block, past the tensor), so it repeats the 52nd
// and the block's fp16 d comes from a separate 16-bit copy per row.
constexpr int M6_M = 128;             // weight rows per workgroup
constexpr int M6_N = 32;              // activation rows per pass (= rows per work item)
constexpr uint32_t M6_WS = 212;       // LDS stride of a staged Q6_K block (53 dwords)

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) k_mmid_mfma_q6k(MfLaunch lp) {
    const uint32_t zm = blockIdx.x >= lp.groups ? 1u : 0u;   // uniform: which matrix
    const MmidArgs& m = lp.m[zm];
    const uint32_t bid = blockIdx.x - zm * lp.groups;
    constexpr int WDMA = M6_M * 53 / 64;            // weight DMA instructions per stage (M6_M rows x 53 dwords)
    constexpr int WDW = (WDMA + 3) / 4;             // ... per wave, at most
    constexpr int ADMA = (M6_N * MF_AD + 63) / 64;  // activation DMA instructions per stage
    constexpr int ADW = (ADMA + 3) / 4;
    __shared__ __align__(16) uint8_t s_w0[M6_M * M6_WS];
    __shared__ __align__(16) uint8_t s_w1[M6_M * M6_WS];
    __shared__ __align__(16) uint8_t s_a0[ADMA * 256];   // M6_N * MF_AS and the last instruction's slack
    __shared__ __align__(16) uint8_t s_a1[ADMA * 256];
    __shared__ __align__(16) uint32_t s_d0[M6_M];   // fp16 d of each staged weight row (zero-extended dword)
    __shared__ __align__(16) uint32_t s_d1[M6_M];
    __shared__ int32_t s_arow[M6_N];
    __shared__ int32_t s_et[M6_N][2];
    __shared__ int s_item[2];
    const int tiles = (int) ((m.N + M6_M - 1) / M6_M);
    const int tile = (int) (bid % (uint32_t) tiles);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    mf_item(m, (int) (bid / (uint32_t) tiles), M6_N, wave, lane, s_item);
    const int g = s_item[0];
    if (g < 0) return;   // past the last item (light experts have none: the GEMV kernel's)
    const int p0 = m.active_off[g] + M6_N * s_item[1], p1 = min(m.active_off[g + 1], p0 + M6_N);
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) tile * M6_M;
    const int trows = (int) min((int64_t) M6_M, m.N - r0);   // 64 or 128 (N % 64 == 0)
    const int nb = (int) (m.K / QK_K);
    const uint32_t nb1 = (uint32_t) m.nb1;
    const uint8_t* wtile = m.w + (size_t) mat * m.nb2 + (size_t) r0 * m.nb1;
    const i32x4 wrsrc = rsrc_words(wtile, (uint32_t) trows * nb1);   // rows past trows read as zeros
    const i32x4 arsrc = rsrc_words(m.act_q, 0x7fffffffu);
    const int ntok = p1 - p0;   // 1 .. M6_N
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    if (tid < M6_N) {
        const int pp = p0 + (tid < ntok ? tid : 0);   // rows past ntok are staged from row 0, never written
        const int e = m.rows[2 * pp], t = m.rows[2 * pp + 1];
        s_et[tid][0] = e;
        s_et[tid][1] = t;
        s_arow[tid] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
    }
    lds_barrier();
    // weight slot q = 64 j + lane: row q / 53, dword u = q % 53.  wbase = row * nb1 + 4 u,
    // bit 0 set for u = 52 (row * nb1 is even); the stage's offset is
    // (wbase + 210 i) & ~3, less 4 for u = 52 when the block starts on a dword
    uint32_t wbase[WDW], aoff[ADW];
#pragma unroll
    for (int k = 0; k < WDW; ++k) {
        const int q = 64 * (wave + 4 * k) + lane;
        const int qc = q < M6_M * 53 ? q : 0;
        const int row = qc / 53, u = qc - 53 * row;
        wbase[k] = (uint32_t) row * nb1 + 4u * (uint32_t) u + (u == 52 ? 1u : 0u);
    }
#pragma unroll
    for (int k = 0; k < ADW; ++k) {
        const int sl = 64 * (wave + 4 * k) + lane;
        const int slc = sl < M6_N * MF_AD ? sl : 0;
        const int n = slc / MF_AD, u = slc - MF_AD * n;
        aoff[k] = (uint32_t) s_arow[n] * (uint32_t) m.act_row_bytes + (u < 4 || u >= 68 ? 0u : 4u * (uint32_t) u - 12u);
    }
    const uint32_t dvoff = (uint32_t) lane * nb1 + 208u;   // the fp16 d of row `lane` (+ 64 for the second copy)
    auto issue = [&](uint8_t* sw, uint8_t* sa, uint32_t* sd, int i) __attribute__((always_inline)) {
        // LDS bases recomputed per stage, not kept live across the loop (scalar registers)
        uint32_t lw = (uint32_t) (uintptr_t) sw, la = (uint32_t) (uintptr_t) sa, ld = (uint32_t) (uintptr_t) sd;
        int w = wv;
        asm volatile("" : "+s"(lw), "+s"(la), "+s"(ld), "+s"(w));
        const uint32_t si = 210u * (uint32_t) i;
#pragma unroll
        for (int k = 0; k < WDW; ++k)
            if (w + 4 * k < WDMA) {
                const uint32_t t = wbase[k] + si;
                const uint32_t vo = (t & ~3u) - (((t & 1u) && !(t & 2u)) ? 4u : 0u);
                dma_b32(wrsrc, lw + 256u * (uint32_t) (w + 4 * k), vo, 0u);
            }
        if (w < M6_M / 64) {   // waves 0, 1: rows 64 w + lane
            uint32_t keep;
            const uint32_t ldw = ld + 256u * (uint32_t) w, sio = si + 64u * nb1 * (uint32_t) w;
            asm volatile(
                "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_ushort %2, %3, %4 offen lds\n\t"
                "s_mov_b32 m0, %0"
                : "=&s"(keep)
                : "s"(ldw), "v"(dvoff), "s"(wrsrc), "s"(sio)
                : "memory");
        }
#pragma unroll
        for (int k = 0; k < ADW; ++k)
            if (w + 4 * k < ADMA) dma_b32(arsrc, la + 256u * (uint32_t) (w + 4 * k), aoff[k], 292u * (uint32_t) i);
    };

    const int lc = lane & 31, h = lane >> 5;
    const int wrow = 32 * wave + lc;               // this lane's weight row in the tile (D column)
    constexpr int arow0 = 0;                       // the wave's activation rows: the whole pass
    const bool active = 32 * wv < trows;           // uniform: the wave's weight rows exist
    const uint32_t par = ((uint32_t) wrow * nb1) & 2u;
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    auto compute = [&](const uint8_t* sw, const uint8_t* sa, const uint32_t* sd, int i) __attribute__((always_inline)) {
        const uint32_t sh = 8u * (par ^ (2u * ((uint32_t) i & 1u)));   // bit shift of the block in its staged dwords
        const uint32_t* wr = (const uint32_t*) (sw + wrow * M6_WS);
        // two dwords of the block at byte offset off (a multiple of 4) of this row
        auto w2 = [&](int off, uint32_t& lo, uint32_t& hi) __attribute__((always_inline)) {
            const uint32_t a = wr[off / 4], b = wr[off / 4 + 1], c = wr[off / 4 + 2];
            lo = __builtin_amdgcn_alignbyte(b, a, sh / 8);
            hi = __builtin_amdgcn_alignbyte(c, b, sh / 8);
        };
        uint32_t sc4[4];
#pragma unroll
        for (int k = 0; k < 4; k += 2) w2(192 + 4 * k, sc4[k], sc4[k + 1]);
        int32_t isum[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) isum[r] = 0;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            uint32_t ql[2][2][2], qh[2][2];   // [c & 1][p][dword], [p][dword]
#pragma unroll
            for (int c1 = 0; c1 < 2; ++c1)
#pragma unroll
                for (int p = 0; p < 2; ++p) w2(64 * n + 32 * c1 + 16 * p + 8 * h, ql[c1][p][0], ql[c1][p][1]);
#pragma unroll
            for (int p = 0; p < 2; ++p) w2(128 + 32 * n + 16 * p + 8 * h, qh[p][0], qh[p][1]);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int j = 8 * n + jj, c = jj >> 1, p = jj & 1;
                uint32_t bw[2];
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const uint32_t v = ((ql[c & 1][p][d] >> (4 * (c >> 1))) & 0x0F0F0F0Fu) |
                                       (((qh[p][d] >> (2 * c)) & 0x03030303u) << 4);
                    const uint32_t x = v ^ 0x20202020u;          // q6 - 32 as a 6-bit two's complement ...
                    const uint32_t sg = x & 0x20202020u;
                    bw[d] = x | (sg << 1) | (sg << 2);           // ... sign-extended to 8 bits
                }
                const uint8_t* ab = sa + (arow0 + lc) * MF_AS + 16 + 16 * j + 8 * h;
                const long aq = pack2(*(const uint32_t*) ab, *(const uint32_t*) (ab + 4));
                typedef int v16i __attribute__((ext_vector_type(16)));
                v16i z16;
#pragma unroll
                for (int r = 0; r < 16; ++r) z16[r] = 0;
                const v16i dd = __builtin_amdgcn_mfma_i32_32x32x16_i8(aq, pack2(bw[0], bw[1]), z16, 0, 0, 0);
                const int scj = (int) (int8_t) ((sc4[j >> 2] >> (8 * (j & 3))) & 0xffu);
                // |dd| <= 16 * 32 * 128 < 2^23: the 24-bit multiply-add (full rate) is exact.
                // The empty asm keeps each sum's adds one per sub-block, so they fuse
                // with the multiplies (v_mad_i32_i24) instead of pairing into add3s.
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    isum[r] += mul24(scj, dd[r]);
                    asm("" : "+v"(isum[r]));
                }
            }
        }
        const float dx = h2f((uint16_t) sd[wrow]);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ar = arow0 + 8 * (r >> 2) + 4 * h + (r & 3);
            const float dy = *(const float*) (sa + ar * MF_AS);
            acc[r] = __builtin_fmaf(dy * dx, (float) isum[r], acc[r]);
        }
    };
    // stage i: wait for its copies, barrier (every wave is done with stage i - 1,
    // whose buffer then takes super-block i + 1), issue i + 1, compute i
    issue(s_w0, s_a0, s_d0, 0);
    for (int i = 0; i < nb; i += 2) {
        vm_wait<0>();
        lds_barrier();
        if (i + 1 < nb) issue(s_w1, s_a1, s_d1, i + 1);
        if (active) compute(s_w0, s_a0, s_d0, i);
        if (i + 1 >= nb) break;
        vm_wait<0>();
        lds_barrier();
        if (i + 2 < nb) issue(s_w0, s_a0, s_d0, i + 2);
        if (active) compute(s_w1, s_a1, s_d1, i + 1);
    }
    if (!active) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int ar = arow0 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (ar < ntok) {
            const int e = s_et[ar][0], tt = s_et[ar][1];
            float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2);
            dp[r0 + wrow] = acc[r];
        }
    }
}

// Q6_K x Q8_K on the matrix cores, bit-identical to ggml: the exact form.
//
// ggml_vec_dot_q6_K_q8_K's AVX2 branch (quants.c:2426-2508) keeps eight int32
// lanes per (weight row, activation row, super-block),
//     sumi_L = sum_{g<8} sc[2 g + (L >= 4)] * sum_{e<4} q6[32 g + 4 L + e] * q8[32 g + 4 L + e]
//              - 32 (sc[2 L] bsum[2 L] + sc[2 L + 1] bsum[2 L + 1])
// with q6 in [0, 63] (maddubs on the unsigned 6-bit values, madd with the
// sub-block scale; q8sclsub), then acc_L = fma(y.d * fp16(x.d), (float) sumi_L,
// acc_L) over the super-blocks and hsum_float_8(acc).  Element 32 g + l of a
// block is the dequantize_row_q6_K element 128 n + 32 c + l with g = 4 n + c.
//
// sc * q6 does not fit int8, so each product v enters A as two base-64 digits:
// v = 64 hi + lo, lo in [-32, 31], hi in [-126, 125].  The bsum term is a
// contraction over the 32 elements of sub-blocks 2 L, 2 L + 1 (storage order)
// with -32 sc = 64 h + l, h = floor(-sc / 2) in [-64, 64], l = 32 (sc & 1).
// Per AVX lane L and 16 x 16 tile, two v_mfma_i32_16x16x64_i8:
//     D_hi = [hi of lane L's 32 products | h] . [q8 of lane L's elements | q8 of 32 L .. 32 L + 31]
//     D_lo = [lo | l] . (same B)
//     sumi_L = 64 D_hi + D_lo
// (Two independent contractions from zero: no matrix-core result feeds another
// of a different shape.)
// A lane l holds weight row l % 16, B lane l activation row l % 16; byte
// positions 0..7 of both are lane L's elements of segments g = 2 gq, 2 gq + 1
// (gq = l / 16: the k-slots of the Q4_K exact form), positions 8..15 the
// elements 32 L + 8 gq .. +8 of the bsum term (sub-block 2 L + gq / 2).  Any
// assignment of elements to (lane group, byte) that A and B share gives the
// same contraction.  The float steps then follow ggml lane for lane.
//
// Workgroup: 64 weight rows (a wave per 16) x one work item of 16 NB routed
// activation rows; super-blocks staged by DMA as in k_mmid_mfma_q6k (53 dwords
// from the dword at or below the block's start; the fp16 d from a 16-bit copy),
// one super-block ahead.
constexpr int MX_NB = 2;   // activation tiles per pass of the exact Q6_K form

// Base-64 digits of v = s * q for the four bytes q of w (each 0..63), s in
// [-128, 127]: v = 64 hi + lo with lo in [-32, 31], hi in [-126, 125]
// (hi = (v + 32) >> 6), returned as four signed bytes each.  Packed 16-bit
// multiply-adds: the low 16 bits of v + 32 are exact (|v| < 2^13).
__device__ __forceinline__ void q6_digits(uint32_t w, int s, uint32_t& hi, uint32_t& lo) {
    typedef short s16x2m __attribute__((ext_vector_type(2)));
    const u16x2m ss = {(unsigned short) s, (unsigned short) s}, c32 = {32, 32}, m63 = {63, 63};
    const u16x2m e = __builtin_bit_cast(u16x2m, w & 0x00FF00FFu) * ss + c32;
    const u16x2m o = __builtin_bit_cast(u16x2m, (w >> 8) & 0x00FF00FFu) * ss + c32;
    const uint32_t he = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2m, e) >> (short) 6);
    const uint32_t ho = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2m, o) >> (short) 6);
    const uint32_t le = __builtin_bit_cast(uint32_t, (u16x2m) ((e & m63) - c32));
    const uint32_t lo_ = __builtin_bit_cast(uint32_t, (u16x2m) ((o & m63) - c32));
    // bytes 0 and 2 of each (v_perm_b32: selector 0-3 picks the second operand's
    // bytes, 4-7 the first's)
    hi = __builtin_amdgcn_perm(ho, he, 0x06020400u);
    lo = __builtin_amdgcn_perm(lo_, le, 0x06020400u);
}

template <int NB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) k_mmid_mfma_q6k_x(MfLaunch lp) {
    const uint32_t zm = blockIdx.x >= lp.groups ? 1u : 0u;   // uniform: which matrix
    const MmidArgs& m = lp.m[zm];
    const uint32_t bid = blockIdx.x - zm * lp.groups;
    constexpr int NR = 16 * NB;                  // activation rows per pass (and per item)
    constexpr int WDMA = MF_M * 53 / 64;         // weight DMA instructions per stage (64 rows x 53 dwords)
    constexpr int WDW = (WDMA + 3) / 4;          // ... per wave, at most
    constexpr int AW = (NR * MF_AD + 63) / 64;   // activation DMA instructions per stage
    constexpr int AWW = (AW + 3) / 4;
    static_assert(MF_M * 53 % 64 == 0 && WDW + 1 + AWW <= 63, "staging shape");
    __shared__ __align__(16) uint8_t s_w0[MF_M * M6_WS];
    __shared__ __align__(16) uint8_t s_w1[MF_M * M6_WS];
    __shared__ __align__(16) uint8_t s_a0[AW * 256];   // NR * MF_AS and the last instruction's slack
    __shared__ __align__(16) uint8_t s_a1[AW * 256];
    __shared__ __align__(16) uint32_t s_d0[MF_M];      // fp16 d of each staged weight row (zero-extended dword)
    __shared__ __align__(16) uint32_t s_d1[MF_M];
    __shared__ int32_t s_arow[NR];
    __shared__ int32_t s_et[NR][2];
    __shared__ int s_item[2];
    const int tiles = (int) (m.N / MF_M);
    const int tile = (int) (bid % (uint32_t) tiles);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    mf_item(m, (int) (bid / (uint32_t) tiles), NR, wave, lane, s_item);
    const int g = s_item[0];
    if (g < 0) return;   // past the last item (light experts have none: the GEMV kernel's)
    const int p0 = m.active_off[g] + NR * s_item[1], p1 = min(m.active_off[g + 1], p0 + NR);
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) tile * MF_M;
    const int nb = (int) (m.K / QK_K);
    const uint32_t nb1 = (uint32_t) m.nb1;
    const uint8_t* wtile = m.w + (size_t) mat * m.nb2 + (size_t) r0 * m.nb1;
    const i32x4 wrsrc = rsrc_words(wtile, (uint32_t) MF_M * nb1);
    const i32x4 arsrc = rsrc_words(m.act_q, 0x7fffffffu);
    const int ntok = p1 - p0;   // 1 .. NR
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    if (tid < NR) {
        const int pp = p0 + (tid < ntok ? tid : 0);   // rows past ntok are staged from row 0, never written
        const int e = m.rows[2 * pp], t = m.rows[2 * pp + 1];
        s_et[tid][0] = e;
        s_et[tid][1] = t;
        s_arow[tid] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
    }
    lds_barrier();
    // weight slot q = 64 j + lane: row q / 53, dword u = q % 53 (as k_mmid_mfma_q6k)
    uint32_t wbase[WDW], aoff[AWW];
#pragma unroll
    for (int k = 0; k < WDW; ++k) {
        const int q = 64 * (wave + 4 * k) + lane;
        const int qc = q < MF_M * 53 ? q : 0;
        const int row = qc / 53, u = qc - 53 * row;
        wbase[k] = (uint32_t) row * nb1 + 4u * (uint32_t) u + (u == 52 ? 1u : 0u);
    }
#pragma unroll
    for (int k = 0; k < AWW; ++k) {
        const int sl = 64 * (wave + 4 * k) + lane;
        const int slc = sl < NR * MF_AD ? sl : 0;
        const int n = slc / MF_AD, u = slc - MF_AD * n;
        aoff[k] = (uint32_t) s_arow[n] * (uint32_t) m.act_row_bytes + (u < 4 || u >= 68 ? 0u : 4u * (uint32_t) u - 12u);
    }
    const uint32_t dvoff = (uint32_t) lane * nb1 + 208u;   // the fp16 d of row `lane`
    auto issue = [&](uint8_t* sw, uint8_t* sa, uint32_t* sd, int i) __attribute__((always_inline)) {
        uint32_t lw = (uint32_t) (uintptr_t) sw, la = (uint32_t) (uintptr_t) sa, ld = (uint32_t) (uintptr_t) sd;
        int w = wv;
        asm volatile("" : "+s"(lw), "+s"(la), "+s"(ld), "+s"(w));
        const uint32_t si = 210u * (uint32_t) i;
#pragma unroll
        for (int k = 0; k < WDW; ++k)
            if (w + 4 * k < WDMA) {
                const uint32_t t = wbase[k] + si;
                const uint32_t vo = (t & ~3u) - (((t & 1u) && !(t & 2u)) ? 4u : 0u);
                dma_b32(wrsrc, lw + 256u * (uint32_t) (w + 4 * k), vo, 0u);
            }
        if (w == 0) {
            uint32_t keep;
            asm volatile(
                "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_ushort %2, %3, %4 offen lds\n\t"
                "s_mov_b32 m0, %0"
                : "=&s"(keep)
                : "s"(ld), "v"(dvoff), "s"(wrsrc), "s"(si)
                : "memory");
        }
#pragma unroll
        for (int k = 0; k < AWW; ++k)
            if (w + 4 * k < AW) dma_b32(arsrc, la + 256u * (uint32_t) (w + 4 * k), aoff[k], 292u * (uint32_t) i);
    };

    const int lr = lane & 15, gq = lane >> 4;   // A row / B row within a 16 x 16 tile; k-slot group
    const int arow_l = 16 * wave + lr;          // this lane's A row in the staged tile
    const int nh = gq >> 1, nib = gq & 1;       // half n of this lane's segments, their ql nibble
    const uint32_t par = ((uint32_t) arow_l * nb1) & 2u;
    const int nbt = (ntok + 15) / 16;           // activation tiles holding rows (uniform)
    float acc[NB][4][8];
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int L = 0; L < 8; ++L) acc[t][r][L] = 0.0f;

    auto compute = [&](const uint8_t* sw, const uint8_t* sa, const uint32_t* sd, int i) __attribute__((always_inline)) {
        const uint32_t sh = par ^ (2u * ((uint32_t) i & 1u));   // byte offset of the block in its staged dwords
        const uint32_t* wr = (const uint32_t*) (sw + arow_l * M6_WS);
        auto wd = [&](int off) __attribute__((always_inline)) {   // the block's dword at byte off (multiple of 4)
            return __builtin_amdgcn_alignbyte(wr[off / 4 + 1], wr[off / 4], sh);
        };
        uint32_t scw[4];   // the 16 sub-block scales
#pragma unroll
        for (int k = 0; k < 4; ++k) scw[k] = wd(192 + 4 * k);
        const uint32_t scm = wd(192 + 4 * gq);   // scales of sub-blocks 4 gq .. 4 gq + 3 (this lane's segments)
        float d[NB][4];
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const float dy = *(const float*) (sa + (16 * t + lr) * MF_AS);
#pragma unroll
            for (int r = 0; r < 4; ++r) d[t][r] = dy * h2f((uint16_t) sd[16 * wave + 4 * gq + r]);
        }
#pragma unroll
        for (int L = 0; L < 8; ++L) {
            const uint32_t qa = wd(64 * nh + 4 * L), qb = wd(64 * nh + 32 + 4 * L), qhw = wd(128 + 32 * nh + 4 * L);
            const uint32_t c0 = 4u * (uint32_t) nib;   // qh shift of segment 2 gq (2 c, c = 2 nib); + 2 for 2 gq + 1
            const uint32_t q0 = ((qa >> (4u * nib)) & 0x0F0F0F0Fu) | (((qhw >> c0) & 0x03030303u) << 4);
            const uint32_t q1 = ((qb >> (4u * nib)) & 0x0F0F0F0Fu) | (((qhw >> (c0 + 2u)) & 0x03030303u) << 4);
            const int hs = L >= 4 ? 8 : 0;
            uint32_t h0, l0, h1, l1;
            q6_digits(q0, (int) (int8_t) (scm >> hs), h0, l0);
            q6_digits(q1, (int) (int8_t) (scm >> (16 + hs)), h1, l1);
            // the bsum term's scale: sub-block 2 L + nh
            const int sm = (int) (int8_t) (scw[L >> 1] >> (8 * (2 * (L & 1)) + 8 * nh));
            const uint32_t hb = __builtin_amdgcn_perm((uint32_t) ((-sm) >> 1), (uint32_t) ((-sm) >> 1), 0u);   // byte 0 x 4
            const uint32_t lb = (sm & 1) ? 0x20202020u : 0u;
            const v4i ahi = v4i{(int) h0, (int) h1, (int) hb, (int) hb};
            const v4i alo = v4i{(int) l0, (int) l1, (int) lb, (int) lb};
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                if (t >= nbt) break;   // (computing empty tiles too measured slower: 5 VGPRs spilled)
                const uint8_t* ab = sa + (16 * t + lr) * MF_AS + 16;
                const uint32_t bm0 = *(const uint32_t*) (ab + 64 * gq + 4 * L);
                const uint32_t bm1 = *(const uint32_t*) (ab + 64 * gq + 32 + 4 * L);
                const uint32_t bn0 = *(const uint32_t*) (ab + 32 * L + 8 * gq);
                const uint32_t bn1 = *(const uint32_t*) (ab + 32 * L + 8 * gq + 4);
                const v4i bq = v4i{(int) bm0, (int) bm1, (int) bn0, (int) bn1};
                const v4i z4 = v4i{0, 0, 0, 0};
                const v4i dhi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, bq, z4, 0, 0, 0);
                const v4i dlo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, bq, z4, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[t][r][L] = __builtin_fmaf(d[t][r], (float) (64 * dhi[r] + dlo[r]), acc[t][r][L]);
            }
        }
    };
    // stage i: wait for its copies, barrier (every wave is done with stage i - 1,
    // whose buffer then takes super-block i + 1), issue i + 1, compute i.  Two
    // stage buffers (45 KB of LDS) let three workgroups share a CU.
    issue(s_w0, s_a0, s_d0, 0);
    for (int i = 0; i < nb; i += 2) {
        vm_wait<0>();
        lds_barrier();
        if (i + 1 < nb) issue(s_w1, s_a1, s_d1, i + 1);
        compute(s_w0, s_a0, s_d0, i);
        if (i + 1 >= nb) break;
        vm_wait<0>();
        lds_barrier();
        if (i + 2 < nb) issue(s_w0, s_a0, s_d0, i + 2);
        compute(s_w1, s_a1, s_d1, i + 1);
    }
    // hsum_float_8(acc); rows r0 + 16 wave + 4 gq .. +3 of B row 16 t + lr
#pragma unroll
    for (int t = 0; t < NB; ++t) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float* a = acc[t][r];
            o[r] = ((a[4] + a[0]) + (a[6] + a[2])) + ((a[5] + a[1]) + (a[7] + a[3]));
        }
        const int row = 16 * t + lr;
        if (row < ntok) {
            const int e = s_et[row][0], tt = s_et[row][1];
            float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2) + r0 +
                        16 * wave + 4 * gq;
            *(float4*) dp = float4{o[0], o[1], o[2], o[3]};
        }
    }
}

// Whether a matrix-core kernel can take (type, form, shape, strides): Q4_K rows
// of 16-byte aligned super-blocks, or Q6_K rows on 4-byte aligned tensors;
// 64-row tiles, 16-byte aligned output rows.
bool mmid_mfma_supported(const MmidArgs& m) {
    const bool q4 = m.type == T_Q4_K && m.nb1 % 16 == 0 && m.nb2 % 16 == 0 && ((uintptr_t) m.w & 15) == 0;
    const bool q6 = m.type == T_Q6_K && m.nb1 % 2 == 0 && m.nb2 % 4 == 0 && ((uintptr_t) m.w & 3) == 0 &&
                    (uint64_t) M6_M * m.nb1 + 64ull * m.nb1 < (1ull << 31);
    return (q4 || q6) && m.N % MF_M == 0 && m.K % QK_K == 0 && m.dst_nb1 % 16 == 0 && m.dst_nb2 % 16 == 0 &&
           ((uintptr_t) m.dst & 15) == 0 && m.act_row_bytes % 4 == 0 && ((uintptr_t) m.act_q & 3) == 0;
}

// Whether the exact Q4_K form can run on the f16 matrix cores (act_h set from
// launch_q8K_to_f16 over all n_rows activation rows).
bool mmid_mfma_h_ok(const MmidArgs& m, int64_t n_rows) {
    return m.type == T_Q4_K && m.mfma_exact && m.mfma_min_rows > 0 && mmid_mfma_supported(m) && n_rows > 0 &&
           (uint64_t) n_rows * (uint64_t) m.K * 2u + 512u < (1ull << 31);
}

// Whether the persistent f16 kernel takes the launch: the exact form with the f16
// copy, at least three super-blocks per row, at most MP_MAXG active bins, and for
// two matrices one grouping and one activation buffer.  QWMOE_MFMA_PERSIST=0 in
// the environment keeps k_mmid_mfma_q4k_h (a test switch).
static bool mp_ok(const MfLaunch& lp, int nz) {
    const MmidArgs& a = lp.m[0];
    if (a.type != T_Q4_K || !a.mfma_exact || !a.act_h || a.K < 3 * QK_K || a.max_active > MP_MAXG ||
        a.n_pairs <= 0 || 8 * a.n_pairs >= (int64_t(1) << 31) || a.b_ne1 < 1 || a.b_ne1 > 65535)
        return false;
    if (nz == 2) {
        const MmidArgs& b = lp.m[1];
        if (b.rows != a.rows || b.active != a.active || b.active_off != a.active_off || b.n_active != a.n_active ||
            b.act_h != a.act_h || b.act_q != a.act_q || b.b_ne1 != a.b_ne1 || b.act_row_bytes != a.act_row_bytes ||
            b.mfma_min_rows != a.mfma_min_rows || b.nb1 != a.nb1 || b.K != a.K || b.N != a.N)
            return false;
    }
    const char* e = getenv("QWMOE_MFMA_PERSIST");
    return !(e && e[0] == '0');
}

// Two workgroups per CU of the current device (cached per device).
static unsigned mp_grid() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
    if (cus[dev] <= 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return 2u * (unsigned) cus[dev];
}

static int launch_mf(const MfLaunch& lp, int nz, hipStream_t stream) {
    const MmidArgs& m = lp.m[0];
    if (lp.groups == 0) return 0;
    if (mp_ok(lp, nz)) {
        // at most (items of 32 rows) x tiles x nz units: no more workgroups than that
        const int64_t units = mf_max_items(m, MP_NR) * (m.N / MF_M) * nz;
        const unsigned grid = (unsigned) std::min<int64_t>(units, (int64_t) mp_grid());
        if (grid == 0) return 0;
        hipLaunchKernelGGL(k_mmid_mfma_q4k_hp, dim3(grid), dim3(256), 0, stream, lp, (uint32_t) nz);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    const unsigned grid = lp.groups * (unsigned) nz;
    const bool q6x = m.type == T_Q6_K && m.mfma_exact, q6b = m.type == T_Q6_K && !m.mfma_exact;
    if (q6b) hipLaunchKernelGGL(k_mmid_mfma_q6k, dim3(grid), dim3(256), 0, stream, lp);
    else if (q6x) hipLaunchKernelGGL((k_mmid_mfma_q6k_x<MX_NB>), dim3(grid), dim3(256), 0, stream, lp);
    else if (m.mfma_exact && m.act_h) hipLaunchKernelGGL((k_mmid_mfma_q4k_h<MH_NB>), dim3(grid), dim3(256), 0, stream, lp);
    else if (m.mfma_exact) hipLaunchKernelGGL((k_mmid_mfma_q4k<MF_NB_X, true>), dim3(grid), dim3(256), 0, stream, lp);
    else hipLaunchKernelGGL((k_mmid_mfma_q4k<MF_NB_B, false>), dim3(grid), dim3(256), 0, stream, lp);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Workgroups of one matrix: (work item, row tile) pairs.
static int64_t mf_groups(const MmidArgs& m) {
    const bool q6b = m.type == T_Q6_K && !m.mfma_exact;
    const int rows = q6b ? M6_N
                         : 16 * (m.type == T_Q6_K ? MX_NB : !m.mfma_exact ? MF_NB_B : m.act_h ? MH_NB : MF_NB_X);
    return mf_max_items(m, rows) * (q6b ? (m.N + M6_M - 1) / M6_M : m.N / MF_M);
}

int launch_mmid_mfma(const MmidArgs& m, hipStream_t stream) {
    if (!mmid_mfma_supported(m)) return -2;
    const int64_t groups = mf_groups(m);
    if (groups > (int64_t(1) << 30)) return -2;
    MfLaunch lp;
    lp.m[0] = lp.m[1] = m;
    lp.groups = (uint32_t) groups;
    return launch_mf(lp, 1, stream);
}

int launch_mmid_mfma2(const MmidArgs& a, const MmidArgs& b, hipStream_t stream) {
    if (!mmid_mfma_supported(a) || !mmid_mfma_supported(b) || a.type != b.type || a.mfma_exact != b.mfma_exact ||
        a.K != b.K || a.N != b.N || !a.act_h != !b.act_h)
        return -2;
    const int64_t groups = mf_groups(a);
    if (groups != mf_groups(b) || groups > (int64_t(1) << 29)) return -2;
    MfLaunch lp;
    lp.m[0] = a;
    lp.m[1] = b;
    lp.groups = (uint32_t) groups;
    return launch_mf(lp, 2, stream);
}

}  // namespace qw
