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

namespace qw {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4m __attribute__((ext_vector_type(4)));

constexpr int MF_M = 64;          // weight rows per workgroup (4 waves x 16)
constexpr int MF_N = 16;          // activation rows per workgroup (one 16-row tile per wave)
constexpr uint32_t MF_WS = 144;   // LDS stride of a staged Q4_K block (9 x 16 B)
constexpr uint32_t MF_AS = 272;   // LDS stride of a staged Q8_K block: d at 0, qs at 16 (16-aligned)
constexpr int MF_WCH = (MF_M * 9 + 255) / 256;    // 16-byte weight chunks per thread and super-block
constexpr int MF_ACH = (MF_N * 65 + 255) / 256;   // activation dwords per thread and super-block
constexpr int MF_RX = 32;         // rows per work item of the exact form (two passes)

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

// Workgroup b = (work item, row tile): weight rows r0 .. r0 + 63 of the expert's
// matrix against the item's MF_RX routed activation rows, 16 per pass.  Super-
// block i + 1 is loaded into registers while super-block i is computed from LDS.
// Items bound the longest workgroup: with one workgroup walking all of a tile's
// rows, the heaviest expert of a skewed batch (266 rows of 512 tokens) set the
// time of the whole launch.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) k_mmid_mfma_q4k(MmidArgs m) {
    __shared__ __align__(16) uint8_t s_w[2][MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_a[2][MF_N * MF_AS];
    __shared__ int32_t s_arow[MF_N];
    __shared__ int32_t s_et[MF_N][2];
    const int tiles = (int) (m.N / MF_M);
    const int tile = (int) (blockIdx.x % (uint32_t) tiles);
    __shared__ int s_item[2];
    mf_item(m, (int) (blockIdx.x / (uint32_t) tiles), MF_RX, threadIdx.x >> 6, threadIdx.x & 63, s_item);
    const int g = s_item[0];
    if (g < 0) return;   // past the last item (light experts have none: the GEMV kernel's)
    const int p0 = m.active_off[g] + MF_RX * s_item[1], p1 = min(m.active_off[g + 1], p0 + MF_RX);
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) tile * MF_M;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, gq = lane >> 4;   // A row / B row within the tile; k-slot group
    const int nb = (int) (m.K / QK_K);
    const uint8_t* wtile = m.w + (size_t) mat * m.nb2 + (size_t) r0 * m.nb1;
    const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(wtile, (uint32_t) (MF_M * m.nb1));
    const __amdgpu_buffer_rsrc_t arsrc = buffer_rsrc(m.act_q, 0x7fffffffu);
    const int arow_l = 16 * wave + lr;          // this lane's A row in the staged tile
    for (int pass = 0;; ++pass) {
    const int pc = p0 + MF_N * pass;
    if (pc >= p1) break;
    const int ntok = (p1 - pc) < MF_N ? (p1 - pc) : MF_N;
    lds_barrier();   // the previous pass is done with the staged tiles
    if (tid < MF_N) {
        const int pp = pc + (tid < ntok ? tid : 0);
        const int e = m.rows[2 * pp], t = m.rows[2 * pp + 1];
        s_et[tid][0] = e;
        s_et[tid][1] = t;
        s_arow[tid] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
    }
    lds_barrier();

    // staging: this thread's weight chunks and activation dwords of super-block i,
    // through buffer loads (32-bit offsets from a uniform base; a load past the
    // buffer's end returns zeros instead of reading out of bounds).  Offsets and
    // LDS destinations are fixed for the pass; a super-block adds i * 144 / i * 292.
    uint32_t woff[MF_WCH], wdst[MF_WCH], aoff[MF_ACH], adst[MF_ACH];
#pragma unroll
    for (int j = 0; j < MF_WCH; ++j) {
        const int z = tid + 256 * j;
        const int zc = min(z, MF_M * 9 - 1);
        const int r = zc / 9, c = zc - r * 9;
        woff[j] = (uint32_t) r * (uint32_t) m.nb1 + 16u * (uint32_t) c;
        wdst[j] = z < MF_M * 9 ? (uint32_t) (r * MF_WS + 16 * c) : 0xffffffffu;
    }
#pragma unroll
    for (int j = 0; j < MF_ACH; ++j) {
        const int z = tid + 256 * j;
        const int zc = min(z, ntok * 65 - 1);
        const int n = zc / 65, c = zc - n * 65;
        aoff[j] = (uint32_t) s_arow[n] * (uint32_t) m.act_row_bytes + 4u * (uint32_t) c;
        adst[j] = z < ntok * 65 ? (uint32_t) (n * MF_AS + (c == 0 ? 0 : 12 + 4 * c)) : 0xffffffffu;
    }
    u32x4m wreg[MF_WCH];
    uint32_t areg[MF_ACH];
    auto load = [&](int i) {
#pragma unroll
        for (int j = 0; j < MF_WCH; ++j)
            wreg[j] = __builtin_bit_cast(u32x4m, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, woff[j] + (uint32_t) i * 144u, 0, 0));
#pragma unroll
        for (int j = 0; j < MF_ACH; ++j) areg[j] = __builtin_amdgcn_raw_buffer_load_b32(arsrc, aoff[j] + (uint32_t) i * 292u, 0, 0);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < MF_WCH; ++j)
            if (wdst[j] != 0xffffffffu) *(u32x4m*) (s_w[buf] + wdst[j]) = wreg[j];
#pragma unroll
        for (int j = 0; j < MF_ACH; ++j)
            if (adst[j] != 0xffffffffu) *(uint32_t*) (s_a[buf] + adst[j]) = areg[j];
    };

    // per output (D register r): the eight AVX lanes and four min lanes
    float acc[4][8], accm[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int L = 0; L < 8; ++L) acc[r][L] = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) accm[r][q] = 0.0f;
    }
    load(0);
    store(0);
    lds_barrier();
    for (int i = 0; i < nb; ++i) {
        const int buf = i & 1;
        if (i + 1 < nb) load(i + 1);
        const uint8_t* sw = s_w[buf];
        const uint8_t* sa = s_a[buf];
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
        // block scales of the D rows 4 gq + r and of this lane's B row
        float d[4], dmin[4];
        const float dy = *(const float*) (sa + lr * MF_AS);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t h0 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + r) * MF_WS);
            d[r] = dy * h2f((uint16_t) (h0 & 0xffff));
            dmin[r] = -dy * h2f((uint16_t) (h0 >> 16));
        }
        // AVX lanes
#pragma unroll
        for (int L = 0; L < 8; ++L) {
            const uint32_t w = *(const uint32_t*) (sw + arow_l * MF_WS + 16 + 32 * gq + 4 * L);
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            const long a_lo = pack2(mul_bytes(lo, sa_ & 7u), mul_bytes(hi, sb_ & 7u));
            const long a_hi = pack2(mul_bytes(lo, sa_ >> 3), mul_bytes(hi, sb_ >> 3));
            const uint8_t* ab = sa + lr * MF_AS + 16 + 64 * gq + 4 * L;
            const long bq = pack2(*(const uint32_t*) ab, *(const uint32_t*) (ab + 32));
            const v4i z4 = v4i{0, 0, 0, 0};
            const v4i dlo = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, bq, z4, 0, 0, 0);
            const v4i dhi = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, bq, z4, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r][L] = __builtin_fmaf(d[r], (float) (8 * dhi[r] + dlo[r]), acc[r][L]);
        }
        // min lanes: sub-blocks 2q (k-slots of lane groups 0, 1) and 2q + 1 (groups 2, 3)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int sbk = 2 * q + (gq >> 1);
            const uint32_t mnw = sbk < 4 ? mn_lo : mn_hi;
            const int mb = (int) (((mnw >> (8 * (sbk & 3))) & 0xffu) * 0x01010101u);
            const v4i a_mn = v4i{mb, mb, mb, mb};
            const v4i bq = *(const v4i*) (sa + lr * MF_AS + 16 + 64 * q + 16 * gq);
            const v4i dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_mn, bq, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) accm[r][q] = __builtin_fmaf(dmin[r], (float) dm[r], accm[r][q]);
        }
        if (i + 1 < nb) store(buf ^ 1);   // the other buffer was last read before the previous barrier
        lds_barrier();
    }
    // hsum_float_8(acc) + ((m0 + m2) + (m1 + m3)); rows r0 + 16 wave + 4 gq .. +3 of B row lr
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float* a = acc[r];
        const float hs = ((a[4] + a[0]) + (a[6] + a[2])) + ((a[5] + a[1]) + (a[7] + a[3]));
        const float* mm = accm[r];
        o[r] = hs + ((mm[0] + mm[2]) + (mm[1] + mm[3]));
    }
    if (lr < ntok) {
        const int e = s_et[lr][0], tt = s_et[lr][1];
        float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2) + r0 + 16 * wave + 4 * gq;
        *(float4*) dp = float4{o[0], o[1], o[2], o[3]};
    }
    }
}

// The block-sum form (mfma_exact == 0).  Same integers, fewer float steps:
// per (weight row, activation row, super-block) the eight AVX lanes' sums add up
// in the MFMA's own int32 accumulator (sumi = sum_L sumi_L, the block's exact
// integer dot with its scales; |sumi| < 2^25), the mins likewise (prod = sum_m
// prod_m), and the float steps are acc = fma(d_i, sumi, acc) and
// accm = fma(dmin_i, prod, accm) over the super-blocks, then acc + accm.  The
// integers are ggml's exactly; the floats round in another order (relative
// difference ~1e-7 of the terms), inside the 1e-3 bar.  Each wave keeps four
// 16-row activation tiles per pass (64 rows), so a weight row's operand is
// formed once for all of them and the tile is streamed a quarter as often.
constexpr int MF_NB = 4;                               // activation tiles per pass
constexpr int MF_N4 = 16 * MF_NB;                      // activation rows per pass
constexpr int MF_RB = MF_N4;                           // rows per work item (one pass)

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) k_mmid_mfma_q4k_bs(MmidArgs m) {
    __shared__ __align__(16) uint8_t s_w[2][MF_M * MF_WS];
    __shared__ __align__(16) uint8_t s_a[2][MF_N4 * MF_AS];
    __shared__ int32_t s_arow[MF_N4];
    __shared__ int32_t s_et[MF_N4][2];
    const int tiles = (int) (m.N / MF_M);
    const int tile = (int) (blockIdx.x % (uint32_t) tiles);
    __shared__ int s_item[2];
    mf_item(m, (int) (blockIdx.x / (uint32_t) tiles), MF_RB, threadIdx.x >> 6, threadIdx.x & 63, s_item);
    const int g = s_item[0];
    if (g < 0) return;   // past the last item (light experts have none: the GEMV kernel's)
    const int p0 = m.active_off[g] + MF_RB * s_item[1], p1 = min(m.active_off[g + 1], p0 + MF_RB);
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) tile * MF_M;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, gq = lane >> 4;
    const int nb = (int) (m.K / QK_K);
    const uint8_t* wtile = m.w + (size_t) mat * m.nb2 + (size_t) r0 * m.nb1;
    const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(wtile, (uint32_t) (MF_M * m.nb1));
    const __amdgpu_buffer_rsrc_t arsrc = buffer_rsrc(m.act_q, 0x7fffffffu);
    const int arow_l = 16 * wave + lr;
    for (int pass = 0;; ++pass) {
    const int pc = p0 + MF_N4 * pass;
    if (pc >= p1) break;
    const int ntok = (p1 - pc) < MF_N4 ? (p1 - pc) : MF_N4;
    lds_barrier();
    if (tid < MF_N4) {
        const int pp = pc + (tid < ntok ? tid : 0);
        const int e = m.rows[2 * pp], t = m.rows[2 * pp + 1];
        s_et[tid][0] = e;
        s_et[tid][1] = t;
        s_arow[tid] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
    }
    lds_barrier();
    // staging: thread (row n = tid / 4, sub = tid % 4) copies dwords c = sub + 4 j of
    // activation row n (65: d, then the 64 of qs) and 16-byte chunks c = sub + 4 j of
    // weight row n (9 per row): one base offset per thread, the rest immediates
    const int sn = tid >> 2, sub = tid & 3;
    const uint32_t abase = (uint32_t) s_arow[sn < ntok ? sn : 0] * (uint32_t) m.act_row_bytes + 4u * (uint32_t) sub;
    const uint32_t adst = (uint32_t) (sn * MF_AS + 12 + 4 * sub);   // dword c >= 1 at adst + 16 j; c = 0 (the d) at sn * MF_AS
    const uint32_t wbase = (uint32_t) sn * (uint32_t) m.nb1 + 16u * (uint32_t) sub;
    const uint32_t wdst = (uint32_t) (sn * MF_WS + 16 * sub);
    constexpr int AJ = 17, WJ = 3;   // c = sub + 4 j <= 64 (activations), <= 8 (weights)
    u32x4m wreg[WJ];
    uint32_t areg[AJ];
    auto load = [&](int i) {
        const uint32_t wi = wbase + (uint32_t) i * 144u, ai = abase + (uint32_t) i * 292u;
#pragma unroll
        for (int jj = 0; jj < WJ; ++jj)
            if (sub + 4 * jj <= 8)
                wreg[jj] = __builtin_bit_cast(u32x4m, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, wi + 64u * jj, 0, 0));
#pragma unroll
        for (int jj = 0; jj < AJ; ++jj)
            if (sub + 4 * jj <= 64) areg[jj] = __builtin_amdgcn_raw_buffer_load_b32(arsrc, ai + 16u * jj, 0, 0);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int jj = 0; jj < WJ; ++jj)
            if (sub + 4 * jj <= 8) *(u32x4m*) (s_w[buf] + wdst + 64 * jj) = wreg[jj];
        *(uint32_t*) (s_a[buf] + (sub == 0 ? (uint32_t) (sn * MF_AS) : adst)) = areg[0];
#pragma unroll
        for (int jj = 1; jj < AJ; ++jj)
            if (sub + 4 * jj <= 64) *(uint32_t*) (s_a[buf] + adst + 16 * jj) = areg[jj];
    };
    // rows of activation tile bt past ntok are staged from row 0 and never written out
    float acc[MF_NB][4], accm[MF_NB][4];
#pragma unroll
    for (int bt = 0; bt < MF_NB; ++bt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[bt][r] = 0.0f;
            accm[bt][r] = 0.0f;
        }
    const int nbt = (ntok + 15) / 16;   // activation tiles holding rows this pass (uniform)
    load(0);
    store(0);
    lds_barrier();
    for (int i = 0; i < nb; ++i) {
        const int buf = i & 1;
        if (i + 1 < nb) load(i + 1);
        const uint8_t* sw = s_w[buf];
        const uint8_t* sa = s_a[buf];
        const u32x4m hdr = *(const u32x4m*) (sw + arow_l * MF_WS);
        const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = s1 & 0x3f3f3f3fu;
        const uint32_t mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        const uint32_t scw = gq < 2 ? sc_lo : sc_hi;
        const uint32_t sa_ = (scw >> (16 * (gq & 1))) & 0xffu, sb_ = (scw >> (16 * (gq & 1) + 8)) & 0xffu;
        float xd[4], xdm[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t h0 = *(const uint32_t*) (sw + (16 * wave + 4 * gq + r) * MF_WS);
            xd[r] = h2f((uint16_t) (h0 & 0xffff));
            xdm[r] = h2f((uint16_t) (h0 >> 16));
        }
        // this lane's A operands for the eight AVX lanes (scale digits times the
        // nibbles), and the four min operands, formed once for all activation tiles
        long alo[8], ahi[8];
#pragma unroll
        for (int L = 0; L < 8; ++L) {
            const uint32_t w = *(const uint32_t*) (sw + arow_l * MF_WS + 16 + 32 * gq + 4 * L);
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            alo[L] = pack2(mul_bytes(lo, sa_ & 7u), mul_bytes(hi, sb_ & 7u));
            ahi[L] = pack2(mul_bytes(lo, sa_ >> 3), mul_bytes(hi, sb_ >> 3));
        }
        int mbq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int sbk = 2 * q + (gq >> 1);
            const uint32_t mnw = sbk < 4 ? mn_lo : mn_hi;
            mbq[q] = (int) (((mnw >> (8 * (sbk & 3))) & 0xffu) * 0x01010101u);
        }
        // activation tiles in pairs: two independent MFMA accumulation chains
#pragma unroll
        for (int bp = 0; bp < MF_NB; bp += 2) {
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
                    const v4i bq = *(const v4i*) (sa + (16 * (bp + u) + lr) * MF_AS + 16 + 64 * q + 16 * gq);
                    sm[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i{mbq[q], mbq[q], mbq[q], mbq[q]}, bq, sm[u], 0, 0, 0);
                }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float dy = *(const float*) (sa + (16 * (bp + u) + lr) * MF_AS);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[bp + u][r] = __builtin_fmaf(dy * xd[r], (float) (8 * shi[u][r] + slo[u][r]), acc[bp + u][r]);
                    accm[bp + u][r] = __builtin_fmaf(-dy * xdm[r], (float) sm[u][r], accm[bp + u][r]);
                }
            }
        }
        if (i + 1 < nb) store(buf ^ 1);
        lds_barrier();
    }
#pragma unroll
    for (int bt = 0; bt < MF_NB; ++bt) {
        const int row = 16 * bt + lr;
        if (bt < nbt && row < ntok) {
            const int e = s_et[row][0], tt = s_et[row][1];
            float* dp = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) tt * m.dst_nb2) + r0 + 16 * wave +
                        4 * gq;
            *(float4*) dp = float4{acc[bt][0] + accm[bt][0], acc[bt][1] + accm[bt][1], acc[bt][2] + accm[bt][2],
                                   acc[bt][3] + accm[bt][3]};
        }
    }
    }
}

// Whether the matrix-core kernel can take (type, shape, strides): Q4_K rows of
// 16-byte aligned super-blocks, 64-row tiles, 16-byte aligned output rows.
bool mmid_mfma_supported(const MmidArgs& m) {
    return m.type == T_Q4_K && m.N % MF_M == 0 && m.K % QK_K == 0 && m.nb1 % 16 == 0 && m.nb2 % 16 == 0 &&
           ((uintptr_t) m.w & 15) == 0 && m.dst_nb1 % 16 == 0 && m.dst_nb2 % 16 == 0 && ((uintptr_t) m.dst & 15) == 0 &&
           m.act_row_bytes % 4 == 0 && ((uintptr_t) m.act_q & 3) == 0;
}

int launch_mmid_mfma(const MmidArgs& m, hipStream_t stream) {
    if (!mmid_mfma_supported(m)) return -2;
    // one workgroup per (work item, row tile)
    const int64_t groups = mf_max_items(m, m.mfma_exact ? MF_RX : MF_RB) * (m.N / MF_M);
    if (groups == 0) return 0;
    if (groups > (int64_t(1) << 30)) return -2;
    const unsigned grid = (unsigned) groups;
    if (m.mfma_exact) hipLaunchKernelGGL(k_mmid_mfma_q4k, dim3(grid), dim3(256), 0, stream, m);
    else hipLaunchKernelGGL(k_mmid_mfma_q4k_bs, dim3(grid), dim3(256), 0, stream, m);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
