// qw_kernels.hpp -- launch wrappers exported by each kernel translation unit and
// used by the C-ABI layer (api.cpp).  All launches are stream-ordered and
// asynchronous; each returns 0 or a negative status (see include/qwmoe.h).
#pragma once

#include "qw_common.hpp"

namespace qw {

// quantize.hip
// h_out (optional, Q8_K only): the f16 copy the exact Q4_K matrix-core form reads
// (launch_q8K_to_f16's layout), written by the same launch
int launch_quantize_act(int vdt, const float* src, int64_t K, int64_t ne1, int64_t nrows, size_t nb1, size_t nb2,
                        void* dst, hipStream_t stream, uint16_t* h_out = nullptr);
int launch_quantize_weights(int type, const float* src, int64_t n, void* dst, hipStream_t stream);
int launch_dequantize(int type, const void* x, float* y, int64_t n, hipStream_t stream);
int launch_randn(float* y, int64_t n, uint64_t seed, float mean, float stddev, hipStream_t stream);

// router.hip
struct RouterArgs {
    const float* W;       // [E][H] fp32 (ggml [H, E])
    const float* x;       // token t at x + t * x_stride (floats)
    int64_t x_stride;
    int64_t H, E, k, T;
    float clamp_min;      // 6.103515625e-5 in the reference
    float scale;          // expert_weights_scale (applied when != 0 and != 1)
    int32_t* ids;         // [T][k]
    float* weights;       // [T][k]
    float* logits;        // optional [T][E]
    float* probs;         // optional [T][E]
    int32_t* status;      // optional device word: bit 0 set when a top-k tie needed the exact sort
    void* xq;             // optional [T][H/256] Q8_K of x, made in the same launch (T <= 16, dense x rows)
    const float* mask;    // optional [E] added to every token's logits before the softmax
    int32_t* want;        // optional [T][k]: top k of the raw (unmasked) logits
};
int launch_router(const RouterArgs& a, float* logits_ws, hipStream_t stream);

// mmid.hip
struct GroupArgs {
    const int32_t* ids;   // [T][ids_stride]
    int64_t n_ids, T, ids_stride;
    int64_t n_bins;       // number of matrices (or logical experts)
    int32_t* counts;      // [n_bins]        (optional)
    int32_t* offsets;     // [n_bins + 1]    (optional)
    int32_t* rows;        // [T * n_ids][2]  (e, t) pairs grouped by bin, ggml order
    int32_t* active;      // [min(n_bins, T*n_ids)] bins with count > 0, ascending
    int32_t* active_off;  // [n_active + 1]  offsets into rows for each active bin
    int32_t* n_active;    // [1]
    int32_t* status;      // bit 1 set on an out-of-range id
    int32_t* hist_ws;     // workspace: GROUP_WAVES * n_bins ints
};
constexpr int GROUP_WAVES = 16;
int launch_group(const GroupArgs& g, hipStream_t stream);
// The grouping of T tokens that all use matrix 0 once (a dense mul_mat through
// the mul_mat_id kernels): rows (0, t), one active bin.
int launch_group_dense(int32_t* rows, int32_t* active, int32_t* active_off, int32_t* n_active, int64_t T,
                       hipStream_t stream);
// api.cpp: changes whenever the library workspace is (re)allocated or freed (captured graphs
// that baked in workspace addresses are stale then)
uint64_t workspace_generation();
// small batches: top-k (from ready logits) and grouping in one launch; ra.ids must be g.ids
int launch_topk_group(const RouterArgs& ra, const float* logits, const GroupArgs& g, hipStream_t stream);

struct MmidArgs {
    int type;                 // weight type
    const uint8_t* w;         // matrix a at w + a * nb2, row r at + r * nb1
    size_t nb1, nb2;
    int64_t K, N, n_as;
    const uint8_t* act_q;     // quantized activation rows, row (e % b_ne1) + t * b_ne1
    int64_t b_ne1;
    size_t act_row_bytes;
    const int32_t* rows;      // grouped (e, t) pairs
    const int32_t* active;    // active bins
    const int32_t* active_off;
    const int32_t* n_active;
    const int32_t* slot_of;   // optional bin -> matrix index
    int64_t n_slot_of;
    float* dst;               // dst[r] of pair (e, t) at dst + e * dst_nb1 + t * dst_nb2 (bytes)
    size_t dst_nb1, dst_nb2;
    int32_t* status;          // bit 2 set on an out-of-range slot
    int64_t max_active;       // grid bound on active bins
    int mfma_min_rows;        // bins with at least this many rows go to the matrix-core kernel (0: none do)
    int mfma_exact;           // matrix cores: 1 replays ggml's eight fp32 AVX-lane chains (bit-identical);
                              // 0 adds each super-block's exact integer sum in one fp32 chain
    int64_t max_rows;         // bound on the rows of one bin
    int64_t n_pairs;          // bound on the grouped (e, t) pairs of all bins
    // optional (Q8_K activations only): activation row r is the Q8_K of
    // silu(swiglu_gate[r]) * swiglu_up[r] (f32 rows of K values), formed inside
    // the GEMV instead of read from act_q; see mmid_gemv_swiglu_ok
    const float* swiglu_gate;
    const float* swiglu_up;
    // optional (exact Q4_K matrix-core form): the f16 copy of act_q's quants made by
    // launch_q8K_to_f16; with it the exact form runs on the f16 matrix cores (the same bits)
    const uint16_t* act_h;
};
int launch_mmid_gemv(const MmidArgs& m, hipStream_t stream);
// whether launch_mmid_gemv forms the activations itself for these arguments with
// swiglu_gate / swiglu_up set (small bins on the block-parallel kernel)
bool mmid_gemv_swiglu_ok(const MmidArgs& m);
// two GEMVs of the same type, K and grouping in one launch (a.N >= b.N; gate and up, or Q and K)
int launch_mmid_gemv2(const MmidArgs& a, const MmidArgs& b, hipStream_t stream);
// mmid_mfma.hip
bool mmid_mfma_supported(const MmidArgs& m);
int launch_mmid_mfma(const MmidArgs& m, hipStream_t stream);
// the matrix-core parts of two mul_mat_ids of the same type, form, shape and
// grouping (gate and up) in one launch
int launch_mmid_mfma2(const MmidArgs& a, const MmidArgs& b, hipStream_t stream);
// f16 copy of n_rows Q8_K activation rows (row_bytes apart, K values each) for
// the exact Q4_K form on the f16 matrix cores: row r at out + r * K, every group
// of four quants in the order 0, 2, 1, 3
int launch_q8K_to_f16(const uint8_t* q, size_t row_bytes, int64_t K, int64_t n_rows, uint16_t* out, hipStream_t stream);
// whether m (with act_q holding n_rows rows) can take such a copy as act_h
bool mmid_mfma_h_ok(const MmidArgs& m, int64_t n_rows);

// ffn.hip
int launch_swiglu(const float* gate, const float* up, float* out, int64_t n_rows, int64_t n, size_t g_stride,
                  size_t u_stride, size_t o_stride, hipStream_t stream);
int launch_weighted_sum(const float* experts, const float* weights, float* out, int64_t H, int64_t k, int64_t T,
                        hipStream_t stream);
int launch_rms_norm(const float* x, float* y, int64_t n, int64_t rows, float eps, hipStream_t stream,
                    const float* weight = nullptr);
// out[t] = moe_out[t] + sh[t] * sigmoid(gate_inp . x[t]) (+ resid[t]); rows of
// x / moe_out / resid / out at the given float strides, sh dense [T][H].
int launch_shared_gate_add(const float* x, size_t x_stride, const float* gate_inp, const float* sh,
                           const float* moe_out, const float* resid, float* out, size_t o_stride, int64_t H, int64_t T,
                           hipStream_t stream);
// k_weighted_sum then k_rms_norm of its output, in one launch (H <= 16384)
int launch_weighted_sum_rms(const float* experts, const float* weights, float* out, float* x_next, int64_t H,
                            int64_t k, int64_t T, float eps, hipStream_t stream);
// k_swiglu then k_quant_q8K of its output, in one launch (F % 256 == 0; rows dense)
// h_out (optional): the f16 copy of the Q8_K rows the exact Q4_K matrix-core form
// reads (launch_q8K_to_f16's layout), written by the same launch
int launch_swiglu_q8K(const float* gate, const float* up, int64_t F, int64_t n_rows, void* dst, hipStream_t stream,
                      uint16_t* h_out = nullptr);

// Static device scratch of the allocation-free entry point (scratch.hip):
// kScratchBytes per GPU.  scratch_setup(device), with that device current,
// looks up this GPU's copy once; scratch_ptr(device) returns it (null before).
constexpr size_t kScratchBytes = (size_t) 8 << 20;
int scratch_setup(int device);
void* scratch_ptr(int device);

// attn.hip: the attention half of Seg A (per-head norms, NEOX RoPE, f16 KV cache,
// GQA scores, softmax, P.V), head dimension 128
constexpr int ATT_RMAX = 16;      // query heads per kv head, at most
constexpr int ATT_MF_SK = 512;   // keys per block of the matrix-core scores (and of their softmax statistics)
// Keys per split of the split-softmax path (fewer than 64 query rows): a
// multiple of 64 that gives the (kv head, token, split) workgroups about 512 in
// all (64 keys at the 30B decode shape up to 8 k keys of context).
inline int64_t attn_split(int64_t T, int64_t n_head_kv, int64_t n_kv) {
    const int64_t pairs = T * n_head_kv > 0 ? T * n_head_kv : 1;
    const int64_t want = 512 / pairs > 1 ? 512 / pairs : 1;   // splits per (kv head, token)
    const int64_t keys = (n_kv + want - 1) / want;
    return 64 * ((keys + 63) / 64 > 0 ? (keys + 63) / 64 : 1);
}
struct AttnArgs {
    int T, n_head, n_head_kv;
    int64_t n_past, n_kv;         // n_kv = n_past + T keys after this call's rows are written
    float eps, theta_scale, kq_scale;
    const float* q;               // [T][n_head][128] projections
    const float* k;               // [T][n_head_kv][128]
    const float* v;               // [T][n_head_kv][128]
    const float* q_norm;          // [128]
    const float* k_norm;          // [128]
    float* qr;                    // [T][n_head][128] Q after norm and RoPE
    uint16_t* kc;                 // f16 caches [n_ctx][n_head_kv * 128], 16-byte aligned
    uint16_t* vc;
    float* s;                     // [T][n_head][n_kv] scores, then probabilities
    int64_t split;                // keys per split (attn_split; fewer than 64 query rows)
    float* part;                  // [ceil(n_kv / split)][T][n_head][128] partial products
    float* stat;                  // [blocks][T][n_head][2]: each key split's / 512-key block's max and sum
                                  // (attn_stat_blocks blocks)
    float* att;                   // [T][n_head * 128]
    void* att_q8K;                // optional: Q8_K rows of att (the split path writes these instead of att)
};
// blocks of softmax statistics launch_attn_core writes: one per key split (fewer
// than 64 query rows) or per 512-key block of the matrix-core scores
inline int64_t attn_stat_blocks(int64_t T, int64_t n_head_kv, int64_t n_kv) {
    const int64_t sp = attn_split(T, n_head_kv, n_kv), ns = (n_kv + sp - 1) / sp, nb = (n_kv + ATT_MF_SK - 1) / ATT_MF_SK;
    return ns > nb ? ns : nb;
}
int launch_attn_core(const AttnArgs& a, hipStream_t stream);
// whether launch_attn_core writes a.att_q8K (and not att) for these arguments
inline bool attn_writes_q8K(const AttnArgs& a) {
    return a.att_q8K && (int64_t) a.T * (a.n_head / a.n_head_kv) < 64;
}
// attn_norm and its Q8_K quantisation in one launch (n % 256 == 0, x and w 16-byte aligned)
int launch_rms_norm_q8K(const float* x, int64_t n, int64_t rows, float eps, const float* w, void* dst,
                        hipStream_t stream);
// resid = x + y; out = rms_norm(resid) * w (rows of n, dense), out may be null
int launch_add_rms_norm_mul(const float* x, const float* y, float* resid, float* out, int64_t n, int64_t rows,
                            float eps, const float* w, hipStream_t stream);
int launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream);

// gdn.hip -- the gated-delta-net half of Seg A (qwen3next / qwen35moe)
constexpr int GDN_MAX_CONV = 8;   // conv taps (ssm.conv_kernel), at most
struct GdnArgs {
    int T, H_k, H_v, d_conv;
    int64_t conv_ch;              // H_v S + 2 H_k S
    float eps;
    const float* qkv;             // [T][conv_ch] the attn_qkv projection
    const float* z;               // [T][H_v S] the attn_gate projection
    const float* braw;            // [T][H_v] ssm_beta projection
    const float* araw;            // [T][H_v] ssm_alpha projection
    const float* dt_bias;         // [H_v]
    const float* ssm_a;           // [H_v]
    const float* conv1d;          // [conv_ch][d_conv]
    const float* ssm_norm;        // [S]
    float* conv_state;            // [conv_ch][d_conv - 1], updated
    float* state;                 // [H_v][S][S] (ggml's layout, S^T per head), updated
    float* conv;                  // [T][conv_ch] silu(conv)
    float* qn;                    // [T][H_k][S] l2-normed q
    float* kn;                    // [T][H_k][S] l2-normed k
    float* bg;                    // [T][H_v][2] beta, g
    float* o;                     // [T][H_v][S] the recurrence's outputs
    float* y;                     // [T][H_v S] the gated norm's outputs
};
// S = 128, H_v a multiple of H_k, 2 <= d_conv <= GDN_MAX_CONV
bool gdn_shape_ok(int64_t S, int64_t H_k, int64_t H_v, int64_t d_conv);
int launch_gdn_core(const GdnArgs& a, hipStream_t stream);
// one bin per token (bin i = token i, slot rows all 0): rows[2 T], active[T],
// active_off[T + 1], n_active[1], slot[T]
int launch_gdn_group_tokens(int32_t* rows, int32_t* active, int32_t* active_off, int32_t* n_active, int32_t* slot,
                            int64_t T, hipStream_t stream);

}  // namespace qw
