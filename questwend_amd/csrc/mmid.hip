// mmid.hip -- ggml_mul_mat_id on the GPU: per-expert grouping and the
// quantized GEMV over grouped rows.
//
// Contract (ggml/src/ggml.c:3315-3328):  dst[:, e, t] = as[:, :, ids[e, t]] . b[:, e % b_ne1, t]
// CPU semantics reproduced (ggml/src/ggml-cpu/ggml-cpu.c:1534-1707):
//   * b is quantized to the weight type's vec_dot_type first (quantize.hip);
//   * rows are grouped per expert with token outer, slot inner (1622-1637);
//   * each output is vec_dot(row, quantized column); here every output equals the
//     AVX2 vec_dot bit for bit (arch/x86/quants.c:1308-1370, 2038-2115, 2426-2508):
//     the same 8 integer lanes per super-block, the same fma chain over blocks and
//     the same horizontal-sum tree.
#include <type_traits>

#include "qw_kernels.hpp"
#include "qw_bp_rows.hpp"
#include "qw_bp_block.hpp"
#include "qw_rowdot.hpp"
#include "qw_topk.hpp"

namespace qw {

// ---------------------------------------------------------------------------
// Grouping: stable counting sort of the (e, t) pairs by bin (= ids value).
// One workgroup of GROUP_WAVES waves; wave w owns a contiguous slice of the
// flattened pair index f = t * n_ids + e, so slice order == ggml row order.

// Per-slice counters: in LDS when GROUP_WAVES * n_bins fits (GROUP_LDS_BINS),
// else in global memory touched only through L2 atomics (so no lane ever reads
// a stale per-CU cached copy).
constexpr int GROUP_LDS_BINS = 1024;
constexpr int GROUP_UNROLL = 4;  // 64-pair chunks whose ids are loaded together

template <bool IN_LDS>
__device__ __forceinline__ int32_t hist_add(int32_t* h, int32_t v) {
    if constexpr (IN_LDS) return atomicAdd(h, v);
    else return __hip_atomic_fetch_add(h, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool IN_LDS>
__device__ __forceinline__ int32_t hist_load(int32_t* h) {
    if constexpr (IN_LDS) return *h;
    else return __hip_atomic_load(h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Replaces a counter that only the calling thread touches in this phase.
template <bool IN_LDS>
__device__ __forceinline__ int32_t hist_exchange(int32_t* h, int32_t v) {
    if constexpr (IN_LDS) {
        const int32_t old = *h;
        *h = v;
        return old;
    } else {
        return __hip_atomic_exchange(h, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Ranks the keys of one 64-pair chunk without serialising over distinct keys:
// the lanes holding a lane's key (its peers) are found bit by bit from one
// ballot per key bit (keys < 2^nbits); rank = earlier peers, cnt = peers, first
// = lowest peer.  Lanes with key < 0 are nobody's peers and are ignored.
struct ChunkRank {
    int rank, cnt, first;
};
__device__ __forceinline__ ChunkRank chunk_rank(int key, int nbits) {
    const int lane = threadIdx.x & 63;
    uint64_t peers = __ballot(key >= 0);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    return ChunkRank{(int) __popcll(peers & lt), (int) __popcll(peers), __ffsll((unsigned long long) peers) - 1};
}

// Key of pair f = t * n_ids + e (-1 past the slice end or out of range).
__device__ __forceinline__ int pair_key(const GroupArgs& g, int f, int f1, int& t, int& e, bool flag) {
    t = 0;
    e = 0;
    if (f >= f1) return -1;
    t = (int) ((uint32_t) f / (uint32_t) g.n_ids);
    e = f - t * (int) g.n_ids;
    int key = g.ids[(int64_t) t * g.ids_stride + e];
    if (key < 0 || key >= g.n_bins) {
        if (flag && g.status) atomicOr(g.status, 2);
        key = -1;
    }
    return key;
}

// The grouping itself, for a GROUP_WAVES * 64-thread workgroup: s_hist holds
// GROUP_WAVES * n_bins counters when IN_LDS, s_wsum 2 * GROUP_WAVES words.
template <bool IN_LDS>
__device__ __forceinline__ void group_body(const GroupArgs& g, int32_t* s_hist, int32_t (*s_wsum)[GROUP_WAVES]) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int P = (int) (g.T * g.n_ids);
    const int S = (P + GROUP_WAVES - 1) / GROUP_WAVES;
    const int f0 = w * S, f1 = (f0 + S < P) ? f0 + S : P;
    int32_t* hist_base = IN_LDS ? s_hist : g.hist_ws;
    int32_t* hist = hist_base + (int64_t) w * g.n_bins;
    const int nbits = g.n_bins > 1 ? 32 - __clz((int) (g.n_bins - 1)) : 0;
    for (int64_t a = lane; a < g.n_bins; a += 64) {
        if constexpr (IN_LDS) hist[a] = 0;
        else __hip_atomic_store(hist + a, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    // phase A: per-slice histogram; the first lane of each key in a chunk adds
    // the chunk's count for it.  A slice of at most GROUP_UNROLL chunks keeps its
    // keys and in-chunk ranks in registers for phase C (one pass of each loop).
    const bool one = f1 - f0 <= GROUP_UNROLL * 64;   // (uniform)
    int t[GROUP_UNROLL], e[GROUP_UNROLL], key[GROUP_UNROLL];
    ChunkRank rk[GROUP_UNROLL];
    for (int c = f0; c < f1; c += GROUP_UNROLL * 64) {
#pragma unroll
        for (int u = 0; u < GROUP_UNROLL; ++u) key[u] = pair_key(g, c + 64 * u + lane, f1, t[u], e[u], true);
#pragma unroll
        for (int u = 0; u < GROUP_UNROLL; ++u) {
            rk[u] = chunk_rank(key[u], nbits);
            if (key[u] >= 0 && rk[u].rank == 0) hist_add<IN_LDS>(hist + key[u], rk[u].cnt);
        }
    }
    __syncthreads();
    // phase B: totals, exclusive scan over bins, per-slice bases, active list.
    // Each thread takes a contiguous run of bins; run sums are scanned across
    // the workgroup (wave prefix sums, then the wave totals).
    const int nthr = GROUP_WAVES * 64;
    const int64_t per = (g.n_bins + nthr - 1) / nthr;
    const int64_t b0 = threadIdx.x * per, b1 = (b0 + per < g.n_bins) ? b0 + per : g.n_bins;
    int32_t csum = 0, asum = 0;
    for (int64_t a = b0; a < b1; ++a) {
        int32_t tot = 0;
        for (int ww = 0; ww < GROUP_WAVES; ++ww) tot += hist_load<IN_LDS>(hist_base + (int64_t) ww * g.n_bins + a);
        csum += tot;
        asum += tot > 0;
    }
    int32_t ic = csum, ia = asum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t uc = __shfl_up(ic, d), ua = __shfl_up(ia, d);
        if (lane >= d) {
            ic += uc;
            ia += ua;
        }
    }
    if (lane == 63) {
        s_wsum[0][w] = ic;
        s_wsum[1][w] = ia;
    }
    __syncthreads();
    int32_t off = ic - csum, aidx = ia - asum, tc = 0, ta = 0;
    for (int ww = 0; ww < GROUP_WAVES; ++ww) {
        const int32_t wc = s_wsum[0][ww], wa = s_wsum[1][ww];
        if (ww < w) {
            off += wc;
            aidx += wa;
        }
        tc += wc;
        ta += wa;
    }
    if (threadIdx.x == 0) {
        if (g.n_active) *g.n_active = ta;
        if (g.offsets) g.offsets[g.n_bins] = tc;
        if (g.active_off) g.active_off[ta] = tc;
    }
    for (int64_t a = b0; a < b1; ++a) {
        int32_t run = off, tot = 0;
        for (int ww = 0; ww < GROUP_WAVES; ++ww) {
            const int32_t c = hist_exchange<IN_LDS>(hist_base + (int64_t) ww * g.n_bins + a, run);  // -> write cursor
            run += c;
            tot += c;
        }
        if (g.counts) g.counts[a] = tot;
        if (g.offsets) g.offsets[a] = off;
        if (tot > 0) {
            g.active[aidx] = (int32_t) a;
            g.active_off[aidx] = off;
            ++aidx;
        }
        off += tot;
    }
    __syncthreads();
    // phase C: stable scatter of (e, t) pairs: the first lane of each key takes
    // the chunk's positions from the slice cursor, the others offset by rank
    for (int c = f0; c < f1; c += GROUP_UNROLL * 64) {
        if (!one) {
#pragma unroll
            for (int u = 0; u < GROUP_UNROLL; ++u) key[u] = pair_key(g, c + 64 * u + lane, f1, t[u], e[u], false);
#pragma unroll
            for (int u = 0; u < GROUP_UNROLL; ++u) rk[u] = chunk_rank(key[u], nbits);
        }
#pragma unroll
        for (int u = 0; u < GROUP_UNROLL; ++u) {
            const ChunkRank r = rk[u];
            int32_t base = 0;
            if (key[u] >= 0 && r.rank == 0) base = hist_add<IN_LDS>(hist + key[u], r.cnt);
            base = __shfl(base, r.first & 63);
            if (key[u] >= 0) {
                const int32_t pos = base + r.rank;
                g.rows[2 * pos] = (int32_t) e[u];
                g.rows[2 * pos + 1] = (int32_t) t[u];
            }
        }
    }
}

// The same grouping by one wave when there are at most 64 pairs and 128 bins:
// lane p holds pair p; in-bin ranks from the ballots of chunk_rank; the bins'
// counts (two bins per lane) are scanned across the wave for the offsets and the
// active list.  cnt: 128 LDS words.
__device__ __forceinline__ void group_wave(const GroupArgs& g, int32_t* cnt) {
    const int lane = threadIdx.x & 63;
    const int P = (int) (g.T * g.n_ids);
    const int nb = (int) g.n_bins;
    int t, e;
    const int key = pair_key(g, lane, P, t, e, true);
    const int nbits = nb > 1 ? 32 - __clz(nb - 1) : 0;
    const ChunkRank r = chunk_rank(key, nbits);
    cnt[lane] = 0;
    cnt[lane + 64] = 0;
    wave_sync();
    if (key >= 0 && r.rank == 0) cnt[key] = r.cnt;
    wave_sync();
    const int b0 = 2 * lane, b1 = 2 * lane + 1;
    const int c0 = b0 < nb ? cnt[b0] : 0, c1 = b1 < nb ? cnt[b1] : 0;
    int ic = c0 + c1, ia = (c0 > 0) + (c1 > 0);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int uc = __shfl_up(ic, d), ua = __shfl_up(ia, d);
        if (lane >= d) {
            ic += uc;
            ia += ua;
        }
    }
    const int tc = __shfl(ic, 63), ta = __shfl(ia, 63);
    const int off0 = ic - (c0 + c1), off1 = off0 + c0;
    int aidx = ia - ((c0 > 0) + (c1 > 0));
    if (b0 < nb) {
        if (g.counts) g.counts[b0] = c0;
        if (g.offsets) g.offsets[b0] = off0;
        if (c0 > 0) {
            g.active[aidx] = b0;
            g.active_off[aidx] = off0;
            ++aidx;
        }
    }
    if (b1 < nb) {
        if (g.counts) g.counts[b1] = c1;
        if (g.offsets) g.offsets[b1] = off1;
        if (c1 > 0) {
            g.active[aidx] = b1;
            g.active_off[aidx] = off1;
        }
    }
    if (lane == 0) {
        if (g.n_active) *g.n_active = ta;
        if (g.offsets) g.offsets[nb] = tc;
        g.active_off[ta] = tc;
    }
    wave_sync();
    cnt[b0] = off0;   // (bins past nb are never a key)
    cnt[b1] = off1;
    wave_sync();
    if (key >= 0) {
        const int pos = cnt[key] + r.rank;
        g.rows[2 * pos] = e;
        g.rows[2 * pos + 1] = t;
    }
}

template <bool IN_LDS>
__global__ void __launch_bounds__(GROUP_WAVES * 64) k_group(GroupArgs g) {
    __shared__ int32_t s_hist[IN_LDS ? GROUP_WAVES * GROUP_LDS_BINS : 1];
    __shared__ int32_t s_wsum[2][GROUP_WAVES];
    group_body<IN_LDS>(g, s_hist, s_wsum);
}

// Small batches (T <= GROUP_WAVES tokens, E <= 128): the router's softmax /
// top-k / weights for token t on wave t (the k_router_topk steps, with wave
// barriers), then the grouping of all tokens' ids by the whole workgroup, in one
// launch.  Dynamic LDS: per wave p[E], order[E], gsum[E / 8], the sort stack and
// a flag; then the GROUP_WAVES * E counters.
__global__ void __launch_bounds__(GROUP_WAVES * 64) k_topk_group(RouterArgs ra, const float* __restrict__ logits,
                                                                 GroupArgs g) {
    extern __shared__ uint32_t dyn[];
    __shared__ int32_t s_wsum[2][GROUP_WAVES];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int E = (int) ra.E;
    const uint32_t per_wave = (uint32_t) (2 * E + E / 8 + 1) * 4u + (uint32_t) sizeof(SortRange) * SORT_STACK;
    uint8_t* mine = (uint8_t*) dyn + (size_t) w * ((per_wave + 15u) & ~15u);
    float* p = (float*) mine;
    int32_t* order = (int32_t*) (p + E);
    float* gsum = (float*) (order + E);
    int* need_sort = (int*) (gsum + E / 8);
    SortRange* stack = (SortRange*) (need_sort + 1);
    // up to 64 pairs: the ids go to LDS, the one-wave grouping reads them there
    // while the next wave copies them out to the caller's buffer
    __shared__ int32_t s_ids[64];
    const bool small = ra.T * ra.k <= 64;
    if (w < ra.T)
        topk_token<true>(logits, ra.E, ra.k, w, ra.clamp_min, ra.scale, small ? s_ids : ra.ids, ra.weights, ra.probs,
                         ra.status, p, gsum, order, stack, need_sort, lane, ra.mask, ra.want);
    __syncthreads();   // every token's ids are written
    int32_t* hist = (int32_t*) ((uint8_t*) dyn + (size_t) GROUP_WAVES * ((per_wave + 15u) & ~15u));
    if (small) {
        if (w == 0) {
            GroupArgs gl = g;
            gl.ids = s_ids;
            group_wave(gl, hist);
        } else if (w == 1 && lane < ra.T * ra.k) {
            ra.ids[lane] = s_ids[lane];
        }
    } else {
        group_body<true>(g, hist, s_wsum);
    }
}

int launch_topk_group(const RouterArgs& ra, const float* logits, const GroupArgs& g, hipStream_t stream) {
    if (ra.T < 1 || ra.T > GROUP_WAVES || ra.E % 8 || ra.E > 128 || ra.k < 1 || ra.k > ra.E || !ra.ids || !ra.weights)
        return -2;
    if (g.n_bins != ra.E || g.ids != ra.ids || g.n_ids != ra.k || g.T != ra.T || g.ids_stride != ra.k) return -2;
    const uint32_t per_wave = (uint32_t) (2 * ra.E + ra.E / 8 + 1) * 4u + (uint32_t) sizeof(SortRange) * SORT_STACK;
    const size_t lds = (size_t) GROUP_WAVES * ((per_wave + 15u) & ~15u) + (size_t) GROUP_WAVES * ra.E * 4;
    hipLaunchKernelGGL(k_topk_group, dim3(1), dim3(GROUP_WAVES * 64), lds, stream, ra, logits, g);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

__global__ void k_group_dense(int32_t* rows, int32_t* active, int32_t* active_off, int32_t* n_active, int64_t T) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t < T) {
        rows[2 * t] = 0;
        rows[2 * t + 1] = (int32_t) t;
    }
    if (t == 0) {
        active[0] = 0;
        active_off[0] = 0;
        active_off[1] = (int32_t) T;
        *n_active = 1;
    }
}

int launch_group_dense(int32_t* rows, int32_t* active, int32_t* active_off, int32_t* n_active, int64_t T,
                       hipStream_t stream) {
    if (T <= 0 || T >= (int64_t(1) << 31)) return -2;
    hipLaunchKernelGGL(k_group_dense, dim3((unsigned) ((T + 255) / 256)), dim3(256), 0, stream, rows, active, active_off,
                       n_active, T);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_group(const GroupArgs& g, hipStream_t stream) {
    if (g.n_bins <= 0 || g.n_bins >= (int64_t(1) << 30) || g.n_ids <= 0 || g.T < 0 || g.T * g.n_ids >= (int64_t(1) << 31))
        return -2;
    if (g.n_bins <= GROUP_LDS_BINS) hipLaunchKernelGGL(k_group<true>, dim3(1), dim3(GROUP_WAVES * 64), 0, stream, g);
    else hipLaunchKernelGGL(k_group<false>, dim3(1), dim3(GROUP_WAVES * 64), 0, stream, g);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

// ---------------------------------------------------------------------------
// GEMV over grouped rows.  Workgroup = 4 waves = MMID_ROWS weight rows of one
// expert matrix, staged once in LDS and applied to every token routed to it.
// Lane (row, n): n is the AVX2 lane index 0..7 of the reference reduction.

constexpr int MMID_ROWS = 32;   // rows per workgroup (8 per wave)
constexpr int MMID_CT = 16;     // activation rows staged per pass
constexpr int MMID_NT = 4;      // activation rows per row-dot call
constexpr int MMID_LD = 8;      // staging loads per thread in flight together

// Activation rows staged per pass: MMID_CT, or fewer when no bin can hold more
// rows (max_rows bounds the rows of one bin), so small batches take less LDS and
// more workgroups fit on a CU.  More rows than this only mean more passes.
__host__ __device__ inline int mmid_stage_rows(int64_t max_rows) {
    return max_rows < 1 ? 1 : max_rows < MMID_CT ? (int) max_rows : MMID_CT;
}

__host__ __device__ inline uint32_t mmid_slot_bytes(size_t row_bytes) {
    return (uint32_t) (((row_bytes + 15 + 15) / 16) * 16 + 16);
}

// One launch computes up to two mul_mat_ids of the same weight type and shape
// over the same grouping (gate and up of an FFN): blockIdx.z picks the matrix.
struct MmidPair {
    MmidArgs m[2];
};

template <int TYPE>
__global__ void __launch_bounds__(256) k_mmid_gemv(MmidPair pr) {
    const MmidArgs m = pr.m[blockIdx.z];
    extern __shared__ uint32_t lds[];
    __shared__ int s_chunk[MMID_CT][3];   // (e, t, activation row) of the staged chunk
    const int g = blockIdx.y;
    if (g >= *m.n_active) return;
    if (m.mfma_min_rows > 0 && m.active_off[g + 1] - m.active_off[g] >= m.mfma_min_rows) return;   // matrix cores take it
    const int bin = m.active[g];
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int64_t r0 = (int64_t) blockIdx.x * MMID_ROWS;
    if (r0 >= m.N) return;
    const int nrows = (int) ((m.N - r0) < MMID_ROWS ? (m.N - r0) : MMID_ROWS);
    const size_t row_bytes = (size_t) (m.K / block_elems(TYPE)) * block_bytes(TYPE);
    const uint32_t RS = mmid_slot_bytes(row_bytes);
    const uint8_t* wmat = m.w + (size_t) mat * m.nb2;
    // stage the weight rows: each row as its 16-byte aligned superset, in rounds
    // of MMID_LD loads per thread issued together (one memory latency per round)
    const int nchmax = (int) ((row_bytes + 15) / 16) + 1;
    for (int base = 0; base < nrows * nchmax; base += MMID_LD * 256) {
        u32x4 v[MMID_LD];
        bool ok[MMID_LD];
#pragma unroll
        for (int j = 0; j < MMID_LD; ++j) {
            const int idx = base + threadIdx.x + j * 256;
            const int r = idx / nchmax, c = idx % nchmax;
            const uint8_t* src = wmat + (size_t) (r0 + (r < nrows ? r : 0)) * m.nb1;
            const uintptr_t s0 = (uintptr_t) src & ~(uintptr_t) 15;
            const uintptr_t s1 = ((uintptr_t) src + row_bytes + 15) & ~(uintptr_t) 15;
            ok[j] = idx < nrows * nchmax && c < (int) ((s1 - s0) / 16);
            v[j] = ((const u32x4*) s0)[ok[j] ? c : 0];   // (a row's first chunk when unused)
        }
#pragma unroll
        for (int j = 0; j < MMID_LD; ++j) {
            const int idx = base + threadIdx.x + j * 256;
            if (ok[j]) ((u32x4*) (lds + ((idx / nchmax) * RS) / 4))[idx % nchmax] = v[j];
        }
    }
    const uint32_t ABASE = RS * MMID_ROWS;  // activation staging follows the weights
    const uint32_t ARS = (uint32_t) (((m.act_row_bytes + 3) / 4) * 4 + 16);
    // Q4_K: the scales of every staged block, unpacked once (table after the
    // activation staging, 16 bytes per (row, block))
    const uint32_t STAB = (ABASE + (uint32_t) mmid_stage_rows(m.max_rows) * ARS + 15u) & ~15u;
    if constexpr (TYPE == T_Q4_K) {
        const int nbk = (int) (m.K / QK_K);
        __syncthreads();   // rows staged
        for (int idx = threadIdx.x; idx < nrows * nbk; idx += 256) {
            const int r = idx / nbk, b = idx - r * nbk;
            const uint32_t blk = (uint32_t) r * RS + (uint32_t) ((uintptr_t) (wmat + (size_t) (r0 + r) * m.nb1) & 15) +
                                 144u * (uint32_t) b;
            *(u32x4*) (lds + ((STAB + 16u * (uint32_t) idx) >> 2)) = q4k_scale_words(lds, blk);
        }
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rl = wave * 8 + (lane >> 3);  // row within the tile
    const int n = lane & 7;
    const bool rvalid = rl < nrows;
    const int rrow = rvalid ? rl : 0;
    const uint32_t wbase = rrow * RS + (uint32_t) ((uintptr_t) (wmat + (size_t) (r0 + rrow) * m.nb1) & 15);
    const int nb = (int) (m.K / block_elems(TYPE));
    // every staged row 4-byte aligned in LDS (uniform per workgroup)
    const bool w_al = (((uintptr_t) wmat | (uintptr_t) m.nb1) & 3) == 0;
    const int p0 = m.active_off[g], p1 = m.active_off[g + 1];
    const int nw = (int) ((m.act_row_bytes + 3) / 4);
    const int CT = mmid_stage_rows(m.max_rows);
    for (int pc = p0; pc < p1; pc += CT) {
        const int cnt = (p1 - pc) < CT ? (p1 - pc) : CT;
        __syncthreads();  // weights staged / previous chunk consumed
        if (threadIdx.x < cnt) {
            const int e = m.rows[2 * (pc + threadIdx.x)], t = m.rows[2 * (pc + threadIdx.x) + 1];
            s_chunk[threadIdx.x][0] = e;
            s_chunk[threadIdx.x][1] = t;
            s_chunk[threadIdx.x][2] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
        }
        __syncthreads();
        // all activation rows of the chunk in one cooperative pass, MMID_LD loads
        // per thread in flight at a time
        for (int base = 0; base < cnt * nw; base += MMID_LD * 256) {
            uint32_t v[MMID_LD];
#pragma unroll
            for (int j = 0; j < MMID_LD; ++j) {
                const int idx = min(base + (int) threadIdx.x + j * 256, cnt * nw - 1);
                const int tk = idx / nw, c = idx - tk * nw;
                v[j] = ((const uint32_t*) (m.act_q + (size_t) s_chunk[tk][2] * m.act_row_bytes))[c];
            }
#pragma unroll
            for (int j = 0; j < MMID_LD; ++j) {
                const int idx = base + (int) threadIdx.x + j * 256;
                if (idx < cnt * nw) {
                    const int tk = idx / nw, c = idx - tk * nw;
                    lds[(ABASE + tk * ARS) / 4 + c] = v[j];
                }
            }
        }
        __syncthreads();
        // up to MMID_NT activation rows per row-dot call (4, 2 or 1, as many as are
        // left): the weight bits are unpacked once per block for all of them
        auto rows_dot = [&](auto nt_tag, int tk0) {
            constexpr int NT = decltype(nt_tag)::value;
            uint32_t ab[NT];
#pragma unroll
            for (int u = 0; u < NT; ++u) ab[u] = ABASE + (uint32_t) (tk0 + u) * ARS;
            float v[NT];
            if constexpr (TYPE == T_Q4_K) {
                const uint32_t tab = STAB + 16u * (uint32_t) (rrow * nb);
                if (w_al) row_dot_q4k_mt_tab<true, NT>(lds, wbase, tab, ab, nb, n, v);
                else row_dot_q4k_mt_tab<false, NT>(lds, wbase, tab, ab, nb, n, v);
            } else if constexpr (TYPE == T_Q6_K) {
                row_dot_q6k_mt<NT>(lds, wbase, ab, nb, n, v);
            } else {
                row_dot_q80_mt<NT>(lds, wbase, ab, nb, n, v);
            }
            if (rvalid && n == 0) {
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    const int e = s_chunk[tk0 + u][0], t = s_chunk[tk0 + u][1];
                    float* d = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) t * m.dst_nb2);
                    d[r0 + rl] = v[u];
                }
            }
        };
        for (int tk0 = 0; tk0 < cnt;) {
            const int rem = cnt - tk0;
            if (rem >= 4) {
                rows_dot(std::integral_constant<int, 4>{}, tk0);
                tk0 += 4;
            } else if (rem >= 2) {
                rows_dot(std::integral_constant<int, 2>{}, tk0);
                tk0 += 2;
            } else {
                rows_dot(std::integral_constant<int, 1>{}, tk0);
                tk0 += 1;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Block-parallel GEMV (Q4_K / Q6_K rows of at most 16 super-blocks).  Lane =
// (row, super-block): each lane forms every integer of its block for all eight
// AVX lanes at once (the sums that dominate the work, independent per block),
// then lanes (row, chain) run the float fma chains over the blocks in order
// from those integers, and one lane per row forms the horizontal-sum tree.
// Integers, chain order and tree are those of row_dot_lds.  With aligned rows
// each lane loads its own block straight into registers; otherwise each wave
// stages its own rows in LDS (16-byte loads over the rows' bytes).  Either way a
// wave needs no workgroup barrier for its weights; the workgroup shares the
// staged activations.  (Measured at K = 4096: staging the Q4_K rows in LDS
// costs 27.6 us per gate/up launch against 19.6 us for the register loads, the
// larger LDS footprint halving the workgroups per CU.)

constexpr int BP_LD = 12;        // staging loads per lane in flight together
constexpr int BP_SWIGLU_MAX_ROWS = 8;   // bins of at most this many rows form SwiGLU's rows in the kernel

// Lanes per row: the next of 4, 8, 16 (3 and 6 lanes per row for K = 768 and
// 1536, with no idle lanes, measured no faster: 20.1 against 19.4 us for the
// configs[4] down projection at T = 1).
__host__ __device__ inline int bp_bpr(int64_t nb) { return nb <= 4 ? 4 : nb <= 8 ? 8 : 16; }

template <int TYPE>
__host__ __device__ inline uint32_t bp_wave_bytes(int bpr, uint32_t RS) {
    return (uint32_t) (64 / bpr) * RS + 64u * BpType<TYPE>::NPW * 4u + (uint32_t) (64 / bpr) * BpType<TYPE>::NCH * 4u;
}

// DIRECT: every lane loads its own block into registers (rows 16-byte aligned
// for Q4_K, 4-byte aligned for Q6_K), no weight staging in LDS.
// SWIGLU: the activation rows are formed from m.swiglu_gate / m.swiglu_up
// (small bins only; the other kernels take Q6_K's many-row form).
template <int TYPE, int BPR, bool DIRECT, bool SWIGLU>
__global__ void __launch_bounds__(256) k_mmid_gemv_bp(MmidPair pr) {
    constexpr int RPW = bp_rows_per_wave(BPR);    // rows per wave
    constexpr int NPW = BpType<TYPE>::NPW, NCH = BpType<TYPE>::NCH;
    const MmidArgs m = pr.m[blockIdx.z];
    extern __shared__ uint32_t lds[];
    __shared__ int s_chunk[MMID_CT][3];
    const int g = blockIdx.y;
    const int64_t r0 = bp_wg_row0(blockIdx.x, BPR);
    if (r0 >= m.N) return;
    // the bin's count, offsets and id in one round (g < max_active keeps every
    // address inside the grouping's arrays; the values count only when g < n_active)
    const int n_act = *m.n_active;
    const int p0 = m.active_off[g], p1 = m.active_off[g + 1];
    const int bin = m.active[g];
    if (g >= n_act) return;
    if (m.mfma_min_rows > 0 && p1 - p0 >= m.mfma_min_rows) return;
    const int CT = mmid_stage_rows(m.max_rows);
    // the slot and the first chunk's pairs in the next round
    int64_t mat = bin;
    if (m.slot_of) mat = (bin < m.n_slot_of) ? m.slot_of[bin] : -1;
    int pe = 0, pt = 0;
    if ((int) threadIdx.x < min(p1 - p0, CT)) {
        pe = m.rows[2 * (p0 + threadIdx.x)];
        pt = m.rows[2 * (p0 + threadIdx.x) + 1];
    }
    if (mat < 0 || mat >= m.n_as) {
        if (threadIdx.x == 0 && m.status) atomicOr(m.status, 4);
        return;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nb = (int) (m.K / QK_K);
    const size_t row_bytes = (size_t) nb * block_bytes(TYPE);
    const uint32_t RS = mmid_slot_bytes(row_bytes);
    const uint32_t ARS = (uint32_t) nb * BP_ABLK;   // one staged activation row
    const uint32_t WB = (uint32_t) CT * ARS;                         // this wave's region
    const uint32_t WBASE = WB + (uint32_t) wave * bp_wave_bytes<TYPE>(BPR, DIRECT ? 0u : RS);
    const uint32_t PBASE = WBASE + (DIRECT ? 0u : (uint32_t) RPW * RS);   // partials [64][NPW]
    const uint32_t CBASE = PBASE + 64u * NPW * 4u;                  // chain values [RPW][NCH]
    const int64_t wr0 = bp_wave_row0(blockIdx.x, wave, BPR);
    const int wrows = bp_wave_rows(m.N, wr0, BPR);
    const uint8_t* wmat = m.w + (size_t) mat * m.nb2;
    const int rl = lane / BPR, b = lane % BPR;
    const bool bvalid = rl < wrows && b < nb;
    const int rrow = rl < wrows ? rl : 0;
    // DIRECT: the lane's block (Q4_K 36 words from a 16-byte aligned address;
    // Q6_K the 53 aligned words holding its 210 bytes, sh = its byte offset in
    // the first, 0 or 2)
    constexpr int NWD = DIRECT ? (TYPE == T_Q4_K ? 36 : 53) : 1;
    uint32_t wd[NWD];
    uint32_t sh = 0;
    if constexpr (DIRECT) {
        // a wave past the matrix end (wrows == 0) loads the workgroup's first row,
        // which exists (r0 < N), and uses nothing it loaded
        const int64_t lrow = bp_direct_row(r0, wr0, wrows, rl);
        const uint8_t* bp = wmat + (size_t) lrow * m.nb1 + block_bytes(TYPE) * (size_t) (b < nb ? b : 0);
        if constexpr (TYPE == T_Q4_K) {
#pragma unroll
            for (int i = 0; i < 9; ++i) {
                const u32x4 v = ((const u32x4*) bp)[i];
                wd[4 * i] = v.x; wd[4 * i + 1] = v.y; wd[4 * i + 2] = v.z; wd[4 * i + 3] = v.w;
            }
        } else {
            sh = (uint32_t) ((uintptr_t) bp & 3);
            const uint32_t* a = (const uint32_t*) ((uintptr_t) bp & ~(uintptr_t) 3);
#pragma unroll
            for (int i = 0; i < 53; ++i) wd[i] = a[i];
        }
    }
    // this wave's rows, each as its 16-byte aligned superset
    const int nchmax = (int) ((row_bytes + 15) / 16) + 1;
    for (int base = 0; base < (DIRECT ? 0 : wrows * nchmax); base += BP_LD * 64) {
        u32x4 v[BP_LD];
        bool ok[BP_LD];
#pragma unroll
        for (int j = 0; j < BP_LD; ++j) {
            const int idx = base + lane + j * 64;
            const int r = idx / nchmax, c = idx % nchmax;
            const uint8_t* src = wmat + (size_t) bp_staged_row(wr0, wrows, r) * m.nb1;
            const uintptr_t s0 = (uintptr_t) src & ~(uintptr_t) 15;
            const uintptr_t s1 = ((uintptr_t) src + row_bytes + 15) & ~(uintptr_t) 15;
            ok[j] = idx < wrows * nchmax && c < (int) ((s1 - s0) / 16);
            v[j] = ((const u32x4*) s0)[ok[j] ? c : 0];
        }
#pragma unroll
        for (int j = 0; j < BP_LD; ++j) {
            const int idx = base + lane + j * 64;
            if (ok[j]) ((u32x4*) (lds + (WBASE + (uint32_t) (idx / nchmax) * RS) / 4))[idx % nchmax] = v[j];
        }
    }
    const uint32_t blk = WBASE + (uint32_t) rrow * RS +
                         (uint32_t) ((uintptr_t) (wmat + (size_t) (wr0 + rrow) * m.nb1) & 15) +
                         (uint32_t) block_bytes(TYPE) * (uint32_t) b;
    const bool w_al = (((uintptr_t) wmat | (uintptr_t) m.nb1) & 3) == 0;
    const int nw = (int) ((m.act_row_bytes + 3) / 4);
    for (int pc = p0; pc < p1; pc += CT) {
        const int cnt = (p1 - pc) < CT ? (p1 - pc) : CT;
        __syncthreads();   // previous chunk consumed
        if (threadIdx.x < cnt) {
            const int e = pc == p0 ? pe : m.rows[2 * (pc + threadIdx.x)];
            const int t = pc == p0 ? pt : m.rows[2 * (pc + threadIdx.x) + 1];
            s_chunk[threadIdx.x][0] = e;
            s_chunk[threadIdx.x][1] = t;
            s_chunk[threadIdx.x][2] = (int) ((int64_t) (e % m.b_ne1) + (int64_t) t * m.b_ne1);
        }
        __syncthreads();
        if constexpr (SWIGLU) {
            // SwiGLU straight into Q8_K, one block per wave (k_swiglu_q8K's values and quantizer)
            for (int q = wave; q < cnt * nb; q += 4) {
                const int tk = q / nb, ib = q - tk * nb;
                const size_t off = (size_t) s_chunk[tk][2] * (size_t) m.K + (size_t) ib * QK_K + 4 * (size_t) lane;
                const float4 gv = *(const float4*) (m.swiglu_gate + off);
                const float4 uv = *(const float4*) (m.swiglu_up + off);
                const float v[4] = {v_silu(gv.x) * uv.x, v_silu(gv.y) * uv.y, v_silu(gv.z) * uv.z, v_silu(gv.w) * uv.w};
                quant_q8K_wave(v, lane, (BlockQ8_K*) ((char*) lds + (uint32_t) tk * ARS + BP_ABLK * (uint32_t) ib + 12u));
            }
        } else {
            for (int base = 0; base < cnt * nw; base += MMID_LD * 256) {
                uint32_t v[MMID_LD];
#pragma unroll
                for (int j = 0; j < MMID_LD; ++j) {
                    const int idx = min(base + (int) threadIdx.x + j * 256, cnt * nw - 1);
                    const int tk = idx / nw, c = idx - tk * nw;
                    v[j] = ((const uint32_t*) (m.act_q + (size_t) s_chunk[tk][2] * m.act_row_bytes))[c];
                }
#pragma unroll
                for (int j = 0; j < MMID_LD; ++j) {
                    const int idx = base + (int) threadIdx.x + j * 256;
                    if (idx < cnt * nw) {
                        const int tk = idx / nw, c = idx - tk * nw;
                        lds[(tk * ARS) / 4 + (uint32_t) (c / 73) * (BP_ABLK / 4) + 3 + (uint32_t) (c % 73)] = v[j];
                    }
                }
            }
        }
        __syncthreads();   // activations (and, on the first pass, every wave's rows) staged
        for (int tk = 0; tk < cnt; ++tk) {
            const uint32_t yb = (uint32_t) tk * ARS + BP_ABLK * (uint32_t) b + 12u;
            if (bvalid) {
                uint32_t part[NPW];
                if constexpr (DIRECT && TYPE == T_Q4_K) {
                    bp_q4k_block([&](uint32_t o) { return wd[o / 4]; }, lds, yb, part);
                } else if constexpr (DIRECT) {
                    const uint16_t d16 = (uint16_t) (sh ? wd[52] >> 16 : wd[52] & 0xffff);
                    bp_q6k_block<!SWIGLU>(
                        [&](uint32_t o) { return __builtin_amdgcn_alignbyte(wd[o / 4 + 1], wd[o / 4], sh); }, d16, lds,
                        yb, part);
                } else if constexpr (TYPE == T_Q4_K) {
                    if (w_al) bp_q4k_block([&](uint32_t o) { return lds_u32a(lds, blk + o); }, lds, yb, part);
                    else bp_q4k_block([&](uint32_t o) { return lds_u32(lds, blk + o); }, lds, yb, part);
                } else {
                    bp_q6k_block<!SWIGLU>([&](uint32_t o) { return lds_u32(lds, blk + o); }, lds_u16(lds, blk + 208),
                                          lds, yb, part);
                }
#pragma unroll
                for (int i = 0; i < NPW; ++i) lds[PBASE / 4 + (uint32_t) lane * NPW + i] = part[i];
            }
            wave_sync();
            // chain (row, c): c < 8 -> AVX lane c of acc over the blocks in order;
            // Q4_K c >= 8 -> lane c - 8 of the mins' accm
            for (int q = lane; q < wrows * NCH; q += 64) {
                const int r = q / NCH, c = q - r * NCH;
                const int sw = c < 8 ? NPW - (TYPE == T_Q4_K ? 2 : 1) : NPW - 1;
                float acc = 0.0f;
#pragma unroll
                for (int bb = 0; bb < BPR; ++bb) {
                    if (bb >= nb) break;
                    const uint32_t pw = PBASE / 4 + (uint32_t) (r * BPR + bb) * NPW;
                    acc = __builtin_fmaf(bitsf(lds[pw + sw]), (float) (int) lds[pw + c], acc);
                }
                lds[CBASE / 4 + (uint32_t) q] = __float_as_uint(acc);
            }
            wave_sync();
            if (lane < wrows) {
                const uint32_t* A = lds + CBASE / 4 + (uint32_t) lane * NCH;
                auto f = [&](int i) { return bitsf(A[i]); };
                float v = ((f(0) + f(4)) + (f(2) + f(6))) + ((f(1) + f(5)) + (f(3) + f(7)));
                if constexpr (TYPE == T_Q4_K) v = v + ((f(8) + f(10)) + (f(9) + f(11)));
                const int e = s_chunk[tk][0], t = s_chunk[tk][1];
                float* d = (float*) ((char*) m.dst + (size_t) e * m.dst_nb1 + (size_t) t * m.dst_nb2);
                d[wr0 + lane] = v;
            }
        }
    }
}

// Rows every lane can load directly: Q4_K 16-byte aligned, Q6_K 4-byte aligned.
static bool gemv_bp_direct(const MmidArgs& m) {
    const uintptr_t a = (uintptr_t) m.w | (uintptr_t) m.nb1 | (uintptr_t) m.nb2;
    return (a & (m.type == T_Q4_K ? 15 : 3)) == 0;
}

// Direct loads for a launch of nz matrices: every matrix's rows must allow them
// (gate and up of one launch may sit at different alignments).
static bool gemv_bp_direct(const MmidPair& pr, int nz) {
    return gemv_bp_direct(pr.m[0]) && (nz < 2 || gemv_bp_direct(pr.m[1]));
}

// The block-parallel kernel's LDS bytes, or 0 when it does not apply.
static size_t gemv_bp_lds(const MmidArgs& m, bool direct) {
    if ((m.type != T_Q4_K && m.type != T_Q6_K) || m.K % QK_K != 0) return 0;
    const int64_t nb = m.K / QK_K;
    if (nb < 1 || nb > 16 || m.act_row_bytes != (size_t) nb * 292) return 0;
    const size_t row_bytes = (size_t) nb * block_bytes(m.type);
    const uint32_t RS = mmid_slot_bytes(row_bytes);
    const int bpr = bp_bpr(nb);
    const uint32_t rs = direct ? 0u : RS;
    const uint32_t wb = m.type == T_Q4_K ? bp_wave_bytes<T_Q4_K>(bpr, rs) : bp_wave_bytes<T_Q6_K>(bpr, rs);
    const size_t lds = (size_t) mmid_stage_rows(m.max_rows) * (size_t) nb * BP_ABLK + 4 * (size_t) wb;
    return lds <= 160 * 1024 ? lds : 0;
}

bool mmid_gemv_swiglu_ok(const MmidArgs& m) {
    // (larger batches: every row tile of a bin would form the same rows again)
    return m.mfma_min_rows == 0 && m.max_rows <= BP_SWIGLU_MAX_ROWS && gemv_bp_lds(m, gemv_bp_direct(m)) != 0 &&
           (((uintptr_t) m.swiglu_gate | (uintptr_t) m.swiglu_up | (uintptr_t) (m.K * 4)) & 15) == 0;
}

static int launch_gemv_bp(const MmidPair& pr, int nz, size_t lds_bytes, hipStream_t stream) {
    const MmidArgs& m = pr.m[0];
    const int bpr = bp_bpr(m.K / QK_K);
    dim3 grid((unsigned) ((m.N + 4 * (64 / bpr) - 1) / (4 * (64 / bpr))), (unsigned) m.max_active, (unsigned) nz);
    if (grid.y == 0) return 0;
    const bool direct = gemv_bp_direct(pr, nz), sw = m.swiglu_gate != nullptr;
#define QW_BP2(T, B, D)                                                                                   \
    do {                                                                                                  \
        if (sw) hipLaunchKernelGGL((k_mmid_gemv_bp<T, B, D, true>), grid, dim3(256), lds_bytes, stream, pr);   \
        else hipLaunchKernelGGL((k_mmid_gemv_bp<T, B, D, false>), grid, dim3(256), lds_bytes, stream, pr);     \
    } while (0)
#define QW_BP(T, B)                  \
    do {                             \
        if (direct) QW_BP2(T, B, true);  \
        else QW_BP2(T, B, false);        \
    } while (0)
    if (m.type == T_Q4_K) {
        if (bpr == 4) QW_BP(T_Q4_K, 4);
        else if (bpr == 8) QW_BP(T_Q4_K, 8);
        else QW_BP(T_Q4_K, 16);
    } else {
        if (bpr == 4) QW_BP(T_Q6_K, 4);
        else if (bpr == 8) QW_BP(T_Q6_K, 8);
        else QW_BP(T_Q6_K, 16);
    }
#undef QW_BP
#undef QW_BP2
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

static int launch_gemv(const MmidPair& pr, int nz, hipStream_t stream) {
    const MmidArgs& m = pr.m[0];
    if (m.swiglu_gate || pr.m[nz - 1].swiglu_gate) {
        if (!mmid_gemv_swiglu_ok(m) || (nz == 2 && !mmid_gemv_swiglu_ok(pr.m[1]))) return -2;
    }
    if (const size_t bp = gemv_bp_lds(m, gemv_bp_direct(pr, nz))) return launch_gemv_bp(pr, nz, bp, stream);
    const size_t row_bytes = (size_t) (m.K / block_elems(m.type)) * block_bytes(m.type);
    size_t lds_bytes = (size_t) mmid_slot_bytes(row_bytes) * MMID_ROWS +
                       (size_t) mmid_stage_rows(m.max_rows) * (((m.act_row_bytes + 3) / 4) * 4 + 16);
    if (m.type == T_Q4_K) lds_bytes = ((lds_bytes + 15) & ~(size_t) 15) + (size_t) MMID_ROWS * (m.K / QK_K) * 16;
    if (lds_bytes > 160 * 1024) return -2;
    dim3 grid((unsigned) ((m.N + MMID_ROWS - 1) / MMID_ROWS), (unsigned) m.max_active, (unsigned) nz);
    if (grid.y == 0) return 0;
    switch (m.type) {
        case T_Q4_K: hipLaunchKernelGGL(k_mmid_gemv<T_Q4_K>, grid, dim3(256), lds_bytes, stream, pr); break;
        case T_Q6_K: hipLaunchKernelGGL(k_mmid_gemv<T_Q6_K>, grid, dim3(256), lds_bytes, stream, pr); break;
        case T_Q8_0: hipLaunchKernelGGL(k_mmid_gemv<T_Q8_0>, grid, dim3(256), lds_bytes, stream, pr); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_mmid_gemv(const MmidArgs& m, hipStream_t stream) {
    MmidPair pr;
    pr.m[0] = m;
    pr.m[1] = m;
    return launch_gemv(pr, 1, stream);
}

int launch_mmid_gemv2(const MmidArgs& a, const MmidArgs& b, hipStream_t stream) {
    // the grid covers a's rows; b may have fewer (its workgroups past b.N return)
    if (a.type != b.type || a.K != b.K || a.N < b.N || a.max_active != b.max_active || a.max_rows != b.max_rows ||
        a.act_row_bytes != b.act_row_bytes)
        return -2;
    MmidPair pr;
    pr.m[0] = a;
    pr.m[1] = b;
    return launch_gemv(pr, 2, stream);
}

}  // namespace qw
