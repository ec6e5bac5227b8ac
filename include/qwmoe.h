/*
 * qwmoe.h -- C ABI of the MI355X (gfx950) quantized MoE expert-FFN library.
 *
 * The library replaces, for QuestWend's MoE FFN path, what the ggml backend
 * executes for the graph that core/runtime.cpp builds per layer
 * (Runtime::Impl::build_moe, core/runtime.cpp:861-974; build_moe_cached
 * 1857-1887; the seg-B lambda of decode_cached_batch 2061-2089).  Paths below
 * are relative to the reference tree; ggml sources are under
 * third_party/ggml/.
 *
 * Conventions
 *   - ggml ne/nb conventions: ne0 is the contiguous dimension, nb* are byte
 *     strides.  Quantized block layouts are ggml's, byte for byte
 *     (ggml/src/ggml-common.h:252-255 Q8_0, 327-337 Q4_K, 362-367 Q6_K,
 *     371-375 Q8_K).  Type ids are ggml's (ggml/include/ggml.h:390-416).
 *   - Every pointer argument named as data (weights, activations, ids,
 *     outputs) is device memory owned by the caller.  The library owns only the
 *     workspace it allocates in qwmoe_init and frees in qwmoe_shutdown; no
 *     entry point allocates device memory.
 *   - `stream` is a hipStream_t (NULL = the default stream).  All compute calls
 *     are asynchronous and stream-ordered; none synchronises with the host.
 *     Calls that use the workspace must not run concurrently on two streams.
 *   - Results are bit-identical to ggml's CPU backend in its x86 AVX2+FMA
 *     build for the same inputs: router ids and weights, token grouping,
 *     quantized activations, integer block sums and fp32 outputs.
 *   - Every function returns QWMOE_OK (0) or a negative status and never
 *     aborts.  Errors a kernel can only see on the device (an expert id out of
 *     range) set bits of a device status word read by qwmoe_device_status().
 */
#ifndef QWMOE_H
#define QWMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWMOE_OK 0
#define QWMOE_ERR_INVALID_ARG (-1)
#define QWMOE_ERR_UNSUPPORTED (-2)
#define QWMOE_ERR_HIP (-3)
#define QWMOE_ERR_WORKSPACE (-4)
#define QWMOE_ERR_NOT_INITIALIZED (-5)
#define QWMOE_ERR_FORMAT (-6)          /* malformed or unsupported GGUF file */
#define QWMOE_ERR_IO (-7)              /* a file could not be opened or read */
#define QWMOE_ERR_SCRATCH (-8)         /* the call needs more than the static scratch of qwmoe_mul_mat_id_noalloc */

/* ggml_type values used on the path (ggml/include/ggml.h:390-416). */
enum qwmoe_type {
    QWMOE_TYPE_F32 = 0,
    QWMOE_TYPE_Q8_0 = 8,
    QWMOE_TYPE_Q4_K = 12,
    QWMOE_TYPE_Q6_K = 14,
    QWMOE_TYPE_Q8_K = 15,
    QWMOE_TYPE_I32 = 26
};

/* Device status bits (qwmoe_device_status). */
#define QWMOE_STATUS_TOPK_TIE_SORT 1   /* a top-k tie was resolved by the exact std::sort replay (informational) */
#define QWMOE_STATUS_BAD_ID 2          /* an ids entry was outside [0, n_as) and was skipped */
#define QWMOE_STATUS_BAD_SLOT 4        /* a slot table entry was outside [0, n_slots) and was skipped */

/* ---- library ------------------------------------------------------------ */

/* Selects `device`, allocates the workspace (workspace_bytes == 0: 256 MiB).
 * Replaces backend initialisation (ggml_backend_reg_i, ggml/src/ggml-backend-impl.h:214-227). */
int qwmoe_init(int device, size_t workspace_bytes);
int qwmoe_shutdown(void);
const char * qwmoe_strerror(int status);
/* Experts that receive at least `rows` rows in one mul_mat_id (prefill and
 * large verify batches) are computed on the matrix cores when the weight type
 * is Q4_K or Q6_K; lighter experts, and every expert when rows == 0, use the
 * LDS-tiled GEMV, which is bit-identical to ggml.  Default 8.  The exact Q4_K
 * form runs on the f16 matrix cores with an f16 copy of the activation quants
 * (2 K bytes per activation row, taken from the workspace; without room for it
 * the int8 matrix cores run, with the same bits).  No reference counterpart: ggml's CPU
 * backend has one dot product per type (ggml-cpu.c:1463-1524); this only
 * selects the GPU kernel. */
int qwmoe_set_mfma_min_rows(int rows);
int qwmoe_get_mfma_min_rows(void);
/* How the matrix-core kernel forms its floats (no reference counterpart).
 * Every form computes ggml's integers exactly: per super-block the eight AVX2
 * lane sums (and, for Q4_K, the four min lanes) of ggml_vec_dot_q4_K_q8_K and
 * ggml_vec_dot_q6_K_q8_K.
 *   QWMOE_MFMA_EXACT: replays ggml's float steps lane for lane (eight fp32 fma
 *       chains and hsum_float_8): bit-identical to the CPU backend, for Q4_K and
 *       Q6_K experts alike;
 *   QWMOE_MFMA_BLOCK_SUM: adds each super-block's exact integer sums in one
 *       fp32 chain (and one for the mins): the same integers, floats rounded in
 *       another order (~1e-6 of the output's magnitude), ~2.5x faster per
 *       projection.  A projection whose output is re-quantized downstream (gate
 *       and up: SwiGLU, then Q8_K for the down projection) can then move a Q8_K
 *       value that sat at a rounding boundary by one step, which moves that
 *       token's layer output by up to ~1.5e-3 of its magnitude;
 *   QWMOE_MFMA_AUTO: the exact form for qwmoe_mul_mat_id and for the gate/up
 *       projections of qwmoe_ffn_layer, qwmoe_shared_expert_add and the layer
 *       stacks; the block-sum form for their down projections.  The layer
 *       output then differs from ggml's in the last bits (~1e-6 of its
 *       magnitude), and since the next layer and its router re-quantize that
 *       output to Q8_K, the difference can move a Q8_K value, and over many
 *       layers a top-k choice, as in QWMOE_MFMA_BLOCK_SUM.
 * The default is QWMOE_MFMA_EXACT: every result is ggml's bits.  The other
 * forms are opt-in speed settings for callers that accept that drift (a T = 8
 * verify batch under them need not give the bits of eight T = 1 decodes).
 * Captured layer-stack graphs are re-captured when the setting changes. */
enum { QWMOE_MFMA_BLOCK_SUM = 0, QWMOE_MFMA_EXACT = 1, QWMOE_MFMA_AUTO = 2 };
int qwmoe_set_mfma_form(int form);
int qwmoe_get_mfma_form(void);
/* Bytes used by the workspace of the most demanding call so far. */
size_t qwmoe_workspace_high_water(void);

/* ggml_row_size (ggml/src/ggml.c) for the supported types; 0 if unsupported. */
size_t qwmoe_row_size(int type, int64_t ne);
/* type_traits_cpu[type].vec_dot_type (ggml/src/ggml-cpu/ggml-cpu.c:271-335): Q8_0 -> Q8_0, Q4_K/Q6_K -> Q8_K. */
int qwmoe_vec_dot_type(int type);

/* Synchronises `stream`, returns the OR of the device status bits raised since
 * the last clear, and clears them when `clear` != 0. */
int qwmoe_device_status(void * stream, int32_t * status_out, int clear);

/* ---- quantization --------------------------------------------------------- */

/* Activation quantizer used by mul_mat_id (type_traits_cpu[vdt].from_float,
 * ggml/src/ggml-cpu/ggml-cpu.c:1585-1620): vdt = Q8_K -> quantize_row_q8_K_ref
 * (ggml/src/ggml-quants.c:2768-2803); vdt = Q8_0 -> the x86 AVX2
 * quantize_row_q8_0 (ggml/src/ggml-cpu/arch/x86/quants.c:302-404).
 * src: f32 [ne0, ne1, ne2] with byte strides nb1, nb2; dst: dense rows,
 * row (i1 + i2 * ne1) at dst + row * qwmoe_row_size(vdt, ne0). */
int qwmoe_quantize_act(void * stream, int vdt, const float * src, int64_t ne0, int64_t ne1, int64_t ne2,
                       size_t nb1, size_t nb2, void * dst);

/* Weight quantizer: ggml_quantize_chunk(type, src, dst, 0, nrows, n_per_row, NULL)
 * (ggml/src/ggml.c:7919-8000) for type Q4_K (quantize_row_q4_K_ref,
 * ggml-quants.c:1457-1527), Q6_K (quantize_row_q6_K_ref, 1869-1937) and Q8_0
 * (quantize_row_q8_0_ref, 276-297).  Bit-identical to the CPU code. */
int qwmoe_quantize_chunk(void * stream, int type, const float * src, void * dst, int64_t nrows, int64_t n_per_row);

/* type_traits[type].to_float: dequantize_row_q8_0 / _q4_K / _q6_K
 * (ggml-quants.c:553-566, 1529-1551, 1939-1968). */
int qwmoe_dequantize(void * stream, int type, const void * x, float * y, int64_t n);

/* Seeded synthetic N(mean, stddev) f32 data (no reference counterpart; the
 * benchmark's weight/input generator). */
int qwmoe_fill_randn(void * stream, float * y, int64_t n, uint64_t seed, float mean, float stddev);

/* ---- the op: ggml_mul_mat_id ------------------------------------------- */

/* dst[:, e, t] = as[:, :, a(ids[e, t])] . b[:, e % ne11, t]
 * Replaces GGML_OP_MUL_MAT_ID as constructed by ggml_mul_mat_id
 * (ggml/include/ggml.h:1445-1449, ggml/src/ggml.c:3315-3356) and computed by
 * ggml_compute_forward_mul_mat_id (ggml/src/ggml-cpu/ggml-cpu.c:1534-1707).
 *   as   : [ne00 = K, ne01 = N, ne02 = n_as] of `type` (Q4_K, Q6_K, Q8_0), strides nb01, nb02
 *   b    : f32 [K, ne11, ne12 = T], strides nb11, nb12
 *   ids  : i32 [n_ids, T], row stride ids_nb1 bytes (the strided view argsort_top_k returns is fine)
 *   slot_of : optional [n_slot_of] table: a(id) = slot_of[id] (the in-graph
 *          remap of core/runtime.cpp:913-919 / ExpertCache::slot_of_row,
 *          core/expert_cache.cpp:694-697); NULL: a(id) = id
 *   dst  : f32 [N, n_ids, T], strides nb1, nb2 (nb0 = 4)
 * Requirements: K a multiple of 256 (Q4_K, Q6_K) or 64 (Q8_0). */
int qwmoe_mul_mat_id(void * stream, int type, const void * as, int64_t ne00, int64_t ne01, int64_t ne02,
                     size_t nb01, size_t nb02, const float * b, int64_t ne11, int64_t ne12, size_t nb11,
                     size_t nb12, const int32_t * ids, int64_t n_ids, size_t ids_nb1, const int32_t * slot_of,
                     int64_t n_slot_of, float * dst, size_t nb1, size_t nb2);

/* qwmoe_mul_mat_id that allocates nothing and uses no library workspace.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory during the call (HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, results bit-identical to
 * qwmoe_mul_mat_id.  The quantized activations and the grouping arrays live in
 * a static device array of 8 MiB per GPU (held until the process ends), whose
 * address qwmoe_init looks up once; the call runs on the library's device.
 * A call needing more (about ne11 * ne12 * row_size(vec_dot_type, ne00) +
 * 8 * n_ids * ne12 + 72 * n_bins bytes, n_bins = n_slot_of or ne02) returns
 * QWMOE_ERR_SCRATCH before anything is enqueued.  Every call on a GPU shares
 * that array: calls that overlap on one GPU (two streams, two threads) race. */
int qwmoe_mul_mat_id_noalloc(void * stream, int type, const void * as, int64_t ne00, int64_t ne01, int64_t ne02,
                             size_t nb01, size_t nb02, const float * b, int64_t ne11, int64_t ne12, size_t nb11,
                             size_t nb12, const int32_t * ids, int64_t n_ids, size_t ids_nb1,
                             const int32_t * slot_of, int64_t n_slot_of, float * dst, size_t nb1, size_t nb2);

/* Per-expert grouping of the (slot e, token t) pairs, in the order of
 * ggml-cpu.c:1622-1637 (token outer, slot inner): counts[n_as],
 * offsets[n_as + 1] (exclusive prefix sum), rows[T * n_ids][2] = (e, t). */
int qwmoe_group_by_expert(void * stream, const int32_t * ids, int64_t n_ids, int64_t T, size_t ids_nb1,
                          int64_t n_as, int32_t * counts, int32_t * offsets, int32_t * rows);

/* ---- router and FFN tail ---------------------------------------------------- */

/* Router of core/runtime.cpp:869-897: logits = mul_mat(W, x) -> soft_max ->
 * argsort_top_k(k) -> get_rows / sum_rows / clamp(clamp_min, inf) / div
 * (/ scale when scale is neither 0 nor 1).
 *   W: f32 [H, E] (row e contiguous); x: f32 [H, T] with row stride x_nb1 bytes
 *   ids, weights: [k, T] dense; probs: optional [E, T] dense.
 * Requirements: E % 8 == 0, E <= 512, H % 4 == 0. */
int qwmoe_router_topk(void * stream, const float * W, const float * x, int64_t H, int64_t E, int64_t k,
                      int64_t T, size_t x_nb1, float clamp_min, float scale, int32_t * ids, float * weights,
                      float * probs);
/* The router of a resident-only decode (core/runtime.cpp:870-881, under
 * cache_fast_build && resident_decode): want = argsort_top_k(logits, k), the
 * experts the unmasked router prefers, recorded for the host's background
 * refill; then logits = logits + mask (the layer's row of resmask_all: 0 for a
 * resident expert, -inf for an absent one) before the softmax, so top-k can
 * never pick an absent expert.  mask: f32 [E] added to every token's logits (NULL:
 * none); want: [k, T] (NULL: not recorded).  Otherwise as qwmoe_router_topk. */
int qwmoe_router_topk_resident(void * stream, const float * W, const float * x, int64_t H, int64_t E, int64_t k,
                               int64_t T, size_t x_nb1, float clamp_min, float scale, const float * mask,
                               int32_t * want, int32_t * ids, float * weights, float * probs);

/* ggml_swiglu_split(gate, up) = silu(gate) * up (ggml/src/ggml.c:3060-3065,
 * ggml/src/ggml-cpu/ops.cpp:3182-3238): `rows` rows of n values, n % 8 == 0. */
int qwmoe_swiglu(void * stream, const float * gate, const float * up, float * out, int64_t n, int64_t rows);

/* Weighted expert sum of core/runtime.cpp:940-959.  experts: [H, k, T];
 * weights: [k, T]; out: [H, T]. */
int qwmoe_weighted_sum(void * stream, const float * experts, const float * weights, float * out, int64_t H,
                       int64_t k, int64_t T);

/* ggml_rms_norm (ggml/src/ggml-cpu/ops.cpp:3795-3860) over `rows` rows of n. */
int qwmoe_rms_norm(void * stream, const float * x, float * y, int64_t n, int64_t rows, float eps);

/* ---- the step either side of the expert FFN (one decoder layer's FFN half) ---- */

/* The router input of a decoder layer: y = ggml_mul(ggml_rms_norm(x, eps), w),
 * w [n] the layer's ffn_norm (or post_attention_norm) weight, as Seg A builds
 * it (core/runtime.cpp:2028-2030); every row rounded as those two ops round. */
int qwmoe_rms_norm_mul(void * stream, const float * x, const float * w, float * y, int64_t n, int64_t rows,
                       float eps);

/* The shared expert of a layer (blk.N.ffn_{gate,up,down}_shexp and
 * ffn_gate_inp_shexp). */
typedef struct qwmoe_shared_expert {
    int64_t n_ff;              /* rows of gate / up, columns of down */
    int type_gate, type_up, type_down;   /* Q4_K, Q6_K or Q8_0 */
    const void * gate;         /* [H, n_ff], row stride gate_nb1 */
    const void * up;           /* [H, n_ff], row stride up_nb1 */
    const void * down;         /* [n_ff, H], row stride down_nb1 */
    size_t gate_nb1, up_nb1, down_nb1;
    const float * gate_inp;    /* f32 [H] (the [H, 1] gate matrix) */
} qwmoe_shared_expert;

/* The shared-expert branch of build_moe (core/runtime.cpp:963-972) for T
 * tokens: out = moe_out + down(silu(gate x) * up x) * sigmoid(gate_inp . x),
 * plus resid when it is non-NULL (the layer's residual add).  x, moe_out, resid,
 * out: f32 [H, T] dense; out may be moe_out.  The projections are ggml_mul_mat
 * of the quantized weights (the mul_mat_id row dots, x quantized to the
 * weight's vec_dot type); silu then mul rounds as swiglu does; the gate's dot
 * follows ggml_vec_dot_f32's AVX2 order and its expf is correctly rounded.
 * Requirements: H a multiple of 32 (and of 256 for K-quant gate/up), n_ff a
 * multiple of 8 (and of 256 for a K-quant down). */
int qwmoe_shared_expert_add(void * stream, const qwmoe_shared_expert * se, int64_t H, const float * x, int64_t T,
                            const float * moe_out, const float * resid, float * out);

/* ---- fused layer ------------------------------------------------------------ */

/* One MoE FFN layer's tensors: the ggml graph inputs of build_moe
 * (core/runtime.cpp:861-974).  Expert tensors are either the full
 * blk.N.ffn_{gate,up,down}_exps.weight [K, N, n_expert] or ExpertCache slot
 * pools [K, N, n_slots] (core/expert_cache.h:53-62) addressed through the
 * logical-expert -> slot rows slot_{gate,up,down} (NULL: identity). */
typedef struct qwmoe_layer {
    int64_t n_embd;            /* H */
    int64_t n_expert;          /* E */
    int64_t n_expert_used;     /* k */
    int64_t n_ff;              /* F (n_ff_exp) */
    float expert_weights_scale;
    const float * router;      /* f32 [H, E]: blk.N.ffn_gate_inp.weight */
    int type_gate, type_up, type_down;
    const void * gate;         /* [H, F, n_slots_gate] */
    const void * up;           /* [H, F, n_slots_up] */
    const void * down;         /* [F, H, n_slots_down] */
    size_t gate_nb1, gate_nb2, up_nb1, up_nb2, down_nb1, down_nb2;
    int64_t n_slots_gate, n_slots_up, n_slots_down;
    const int32_t * slot_gate; /* [E] or NULL */
    const int32_t * slot_up;
    const int32_t * slot_down;
    /* Resident-only routing (core/runtime.cpp:870-881; see
     * qwmoe_router_topk_resident): resmask f32 [E] added to the router logits
     * before the softmax, want_ids [k, T] the top k of the raw logits.  Both
     * NULL for the plain router. */
    const float * resmask;
    int32_t * want_ids;
} qwmoe_layer;

/* The whole layer for T tokens: router -> 3x mul_mat_id + swiglu -> weighted
 * sum, then (rms_eps >= 0) x_next = rms_norm(out, rms_eps).
 * x, out, x_next: f32 [H, T] dense.  ids_out / weights_out: optional [k, T].
 * Requirements (else QWMOE_ERR_INVALID_ARG / QWMOE_ERR_UNSUPPORTED): each
 * expert stride covers its rows (nb1 >= row size, nb2 >= nb1 * rows), every
 * n_slots_* > 0, E a multiple of 8 up to 512, H a multiple of 4, x and the
 * router 16-byte aligned, F a multiple of 8. */
int qwmoe_ffn_layer(void * stream, const qwmoe_layer * layer, const float * x, int64_t T, float * out,
                    float rms_eps, float * x_next, int32_t * ids_out, float * weights_out);

/* ---- the attention half of a decoder layer ------------------------------------ */

/* One non-recurrent, non-gated Qwen3 attention block (Seg A of a MoE layer:
 * build_segA, core/runtime.cpp:1976-2030; build_attn, 681-734; NEOX RoPE,
 * apply_rope 290-300).  Weights as in the GGUF: attn_q [H, n_head * D],
 * attn_k / attn_v [H, n_head_kv * D], attn_output [n_head * D, H] (rows of
 * nb1 bytes, Q4_K / Q6_K / Q8_0), f32 norms.  The caches are ggml's k_cache /
 * v_cache: f16 [n_ctx][n_head_kv * D] rows, 16-byte aligned, owned by the
 * caller. */
typedef struct qwmoe_attn_layer {
    int64_t n_embd;            /* H */
    int64_t n_head, n_head_kv; /* query and key/value heads (n_head % n_head_kv == 0) */
    int64_t n_embd_head;       /* D = 128 */
    int64_t n_rot;             /* RoPE dimensions = D */
    float rope_freq_base;      /* 1e6 for Qwen3 */
    const float * attn_norm;   /* [H]: blk.N.attn_norm.weight */
    int type_q, type_k, type_v, type_o;
    const void * wq; size_t wq_nb1;   /* blk.N.attn_q.weight */
    const void * wk; size_t wk_nb1;   /* blk.N.attn_k.weight */
    const void * wv; size_t wv_nb1;   /* blk.N.attn_v.weight */
    const void * wo; size_t wo_nb1;   /* blk.N.attn_output.weight */
    const float * q_norm;      /* [D]: blk.N.attn_q_norm.weight */
    const float * k_norm;      /* [D]: blk.N.attn_k_norm.weight */
    const float * ffn_norm;    /* [H]: blk.N.ffn_norm.weight (the router input's norm) */
    uint16_t * k_cache;        /* f16 [n_ctx][n_head_kv * D] */
    uint16_t * v_cache;
    int64_t n_ctx;
} qwmoe_attn_layer;

/* T tokens at positions n_past .. n_past + T - 1 (a decode step, a verify batch
 * or a prefill chunk), h f32 [T, H] the layer input (the residual stream):
 *   cur = rms_norm(h) * attn_norm; Q, K, V = projections of cur;
 *   Q = rope(rms_norm(Q) * q_norm), K = rope(rms_norm(K) * k_norm) per head;
 *   K, V (f16) into cache rows n_past ..; causal attention over the n_past + T
 *   cached keys, kq_scale = 1 / sqrt(D), ggml's soft_max_ext;
 *   attn_resid = attn_output(att) + h; ffn_in = rms_norm(attn_resid) * ffn_norm
 *   (ffn_in may be NULL).
 * The projections are the quantized mul_mat row dots (activations quantized to
 * the weight's vec_dot type, as ggml_mul_mat); Q and the probabilities are
 * rounded to f16 before their products as ggml's f16 mul_mat does.  Outputs
 * agree with the reference CPU graph within the fp32 rounding of the sums
 * (1e-3), not bit for bit.  Requires D = n_rot = 128, n_head / n_head_kv <= 16,
 * n_past + T <= n_ctx, h 16-byte aligned.  Workspace: ~40 T n_embd bytes of
 * projections, plus, for batches of fewer than 64 query rows per kv head
 * (T n_head / n_head_kv < 64: decode, verify), the score rows (4 n_head T
 * (n_past + T) bytes); larger chunks keep only per-512-key softmax statistics
 * and recompute the scores beside P.V (QWMOE_ERR_WORKSPACE when it does not
 * fit, nothing enqueued). */
int qwmoe_attn_seg(void * stream, const qwmoe_attn_layer * layer, const float * h, int64_t T, int64_t n_past,
                   float rms_eps, float * attn_resid, float * ffn_in);

/* One gated-delta-net block (Seg A of a recurrent layer of qwen3next /
 * qwen35moe: build_segA with build_gdn, core/runtime.cpp:1976-1995, 737-859).
 * Weight rows are dense quantized rows (Q4_K / Q6_K / Q8_0); the f32 tensors are
 * ggml's: conv1d [conv_ch][d_conv], the states in their ggml layouts.  d_inner =
 * dt_rank * d_state, conv_ch = d_inner + 2 n_group d_state.  Requires d_state =
 * 128, dt_rank a multiple of n_group, 2 <= d_conv <= 8. */
typedef struct qwmoe_gdn_layer {
    int64_t n_embd;            /* H */
    int64_t d_state;           /* S: ssm.state_size (128) */
    int64_t n_group;           /* H_k: ssm.group_count (key heads) */
    int64_t dt_rank;           /* H_v: ssm.time_step_rank (value heads) */
    int64_t d_conv;            /* ssm.conv_kernel (4) */
    const float * attn_norm;   /* [H]: blk.N.attn_norm.weight */
    int type_qkv, type_gate, type_beta, type_alpha, type_out;
    const void * w_qkv; size_t w_qkv_nb1;       /* blk.N.attn_qkv.weight: conv_ch rows of H */
    const void * w_gate; size_t w_gate_nb1;     /* blk.N.attn_gate.weight: d_inner rows (z) */
    const void * w_beta; size_t w_beta_nb1;     /* blk.N.ssm_beta.weight: H_v rows */
    const void * w_alpha; size_t w_alpha_nb1;   /* blk.N.ssm_alpha.weight: H_v rows */
    const void * w_out; size_t w_out_nb1;       /* blk.N.ssm_out.weight: H rows of d_inner */
    const float * dt_bias;     /* [H_v]: blk.N.ssm_dt.bias */
    const float * ssm_a;       /* [H_v]: blk.N.ssm_a */
    const float * conv1d;      /* [conv_ch][d_conv]: blk.N.ssm_conv1d.weight */
    const float * ssm_norm;    /* [S]: blk.N.ssm_norm.weight */
    const float * ffn_norm;    /* [H]: the router input's norm (ffn_norm / post_attention_norm) */
    float * conv_state;        /* [conv_ch][d_conv - 1], read and written */
    float * ssm_state;         /* [H_v][S][S] (S_h transposed per head, as ggml), read and written */
} qwmoe_gdn_layer;

/* T tokens through the block, h f32 [T, H] the layer input:
 *   cur = rms_norm(h) * attn_norm; qkv, z, beta, alpha = projections of cur;
 *   beta = sigmoid(beta); g = softplus(alpha + dt_bias) * ssm_a;
 *   conv = silu(causal conv of [conv_state | qkv] with conv1d), the conv state
 *   advanced by T; q, k (H_k heads), v (H_v heads) from conv, q and k l2-normed;
 *   per value head h (key head h % H_k) and token: S *= exp(g),
 *   S += k (beta (v - S^T k))^T, o = S^T q / sqrt(S) (ggml_gated_delta_net);
 *   y = rms_norm(o) * ssm_norm * silu(z) per head; attn_resid = ssm_out(y) + h;
 *   ffn_in = rms_norm(attn_resid) * ffn_norm (ffn_in may be NULL).
 * The projections are the quantized mul_mat row dots (ggml's bits); the rest
 * agrees with the reference CPU graph within float rounding (1e-3).  Calls
 * carry the layer's states: one call of T tokens equals consecutive calls of
 * its parts.  Workspace ~4 T (3 conv_ch + 5 d_inner + 2 H) bytes plus the
 * quantized activations. */
int qwmoe_gdn_seg(void * stream, const qwmoe_gdn_layer * layer, const float * h, int64_t T, float rms_eps,
                  float * attn_resid, float * ffn_in);

/* One whole decoder layer of a Qwen3-MoE model for T tokens: qwmoe_attn_seg,
 * then qwmoe_ffn_layer on ffn_in (the router reads ffn_in; build_moe's T = 1 or
 * T > 1 weighted sum), then h_out = moe_out + attn_resid (build_segB's residual,
 * core/runtime.cpp:2087).  h, h_out f32 [T, H]; ids_out / weights_out
 * optional [T, k]. */
int qwmoe_decoder_layer(void * stream, const qwmoe_attn_layer * attn, const qwmoe_layer * moe, const float * h,
                        int64_t T, int64_t n_past, float rms_eps, float * h_out, int32_t * ids_out,
                        float * weights_out);

/* ---- persistent multi-layer decode ------------------------------------------ */

/* A stack of MoE FFN layers decoded one token per launch, all layers in a
 * single persistent kernel (one workgroup per CU).  Replaces, for the MoE FFN
 * layers, the per-token graph the reference builds and replays in
 * Runtime::decode -> decode_reuse / build_graph (core/runtime.cpp:1768-1829,
 * 976-1100), with ggml_rms_norm between layers as in the benchmark stack.
 * All layers must share n_embd, n_expert, n_expert_used, n_ff, types
 * (Q4_K gate/up, Q4_K or Q6_K down) and expert_weights_scale; row strides must
 * be multiples of 16 bytes.  Creation allocates (descriptor table and exchange
 * buffers); running does not. */
typedef struct qwmoe_decode_stack qwmoe_decode_stack;
int qwmoe_decode_stack_create(const qwmoe_layer * layers, int n_layer, float rms_eps, qwmoe_decode_stack ** out);
/* One token: x [H] -> out [H] (MoE output of the last layer) and, when
 * non-NULL, x_out [H] = rms_norm(out); ids_out / weights_out [n_layer][k].
 * The kernel is persistent: every workgroup must be resident at once, so the
 * launch must not share the device with other work that holds CUs (a
 * workgroup that waits too long gives up: status bit 8, outputs invalid, the
 * call itself still returns QWMOE_OK -- check qwmoe_decode_stack_status).
 * Each launch takes a fresh exchange epoch from the host, so a launch recorded
 * under stream capture could not be replayed: on a capturing stream the call
 * returns QWMOE_ERR_UNSUPPORTED and enqueues nothing. */
int qwmoe_decode_stack_run(void * stream, qwmoe_decode_stack * s, const float * x, float * out, float * x_out,
                           int32_t * ids_out, float * weights_out);
/* Synchronises `stream`; status bits: 1 top-k tie replayed, 8 a wait timed out
 * (launch abandoned), 16 a slot table entry was out of range.  With 8, the
 * XCD kernels (qwmoe_decode_stack_kernel 2 to 5) name the exchange they waited
 * for: 256 router logits, 512 act, 1024 down outputs, 2048 y, 4096 top-k. */
int qwmoe_decode_stack_status(void * stream, qwmoe_decode_stack * s, int32_t * status_out, int clear);
void qwmoe_decode_stack_free(qwmoe_decode_stack * s);
/* Which kernel a stack runs (no reference counterpart; the kernel choice only):
 * 1 = one workgroup per CU over every selected expert; 2 = one selected expert
 * per XCD (256-CU devices, k <= 8, H = 2048, Q4_K down), exchanges inside an XCD
 * through its L2; 3 = the same with every exchange word stored at device scope
 * (used when creation finds the workgroups not dealt to the XCDs round robin);
 * 4 and 5 = the forms of 2 and 3 for wide layers (H = 4096, F = 1536, E = 128,
 * Q6_K or Q4_K down with 4- / 16-byte aligned rows; router logits exchanged
 * across XCDs).  Creation picks 2 to 5 where the shape allows, else 1;
 * QWMOE_DECODE_XCD=0 in the environment at creation forces 1,
 * QWMOE_DECODE_XCD_LOCAL=0 forces device-scope words.  Results are identical. */
int qwmoe_decode_stack_kernel(const qwmoe_decode_stack * s);

/* ---- T-token batches through a layer stack (speculative-decoding verify) ------ */

/* The FFN half of the verify forward: Runtime::decode_verify runs the model on
 * the T = n_draft + 1 tokens of an MTP draft at once (core/runtime.cpp:1495-1562,
 * driven by generate_mtp, 1628-1762), so every MoE layer sees a T-token batch
 * with build_moe's T > 1 semantics (core/runtime.cpp:861-974).  Each layer is
 * qwmoe_ffn_layer on the batch, RMSNorm between layers as in the decode stack.
 * The chain for one T is captured into a HIP graph at its first run and
 * replayed after that, as the reference keeps a persistent verify graph
 * (1503-1525); mul_mat_id settings (qwmoe_set_mfma_min_rows) are those at
 * capture.  Layers must share n_embd and n_expert_used.  Creation allocates the
 * stack's buffers; the first run at each T captures and instantiates a graph;
 * later runs allocate nothing (a run after qwmoe_init reallocated the workspace
 * captures again). */
#define QWMOE_STACK_NO_GRAPH 1     /* run the chain eagerly every time */
typedef struct qwmoe_layer_stack qwmoe_layer_stack;
int qwmoe_layer_stack_create(const qwmoe_layer * layers, int n_layer, float rms_eps, int max_tokens, int flags,
                             qwmoe_layer_stack ** out);
/* x [T][H] -> out [T][H] (MoE output of the last layer), x_out [T][H] (its
 * RMSNorm, may be NULL), ids_out / weights_out [n_layer][T][k] (both or none).
 * 1 <= T <= max_tokens.  Runs at T = 1 and 2 <= T <= 8 may take persistent
 * kernels (qwmoe_layer_stack_kernel, qwmoe_layer_stack_kernel_t1), with the
 * decode stack's rule: they need every CU, and a wait that gives up leaves the
 * outputs invalid while the call returns QWMOE_OK -- the status bits then
 * appear in qwmoe_layer_stack_status (not in qwmoe_device_status, which the
 * per-layer chain uses for bad slots).  The T = 1 decode stack is created at
 * the first T = 1 run.  On a capturing stream (HIP graph capture) every T runs
 * the per-layer chain, which the caller's graph records; that recording holds
 * the library workspace's addresses, so re-capture after qwmoe_init. */
int qwmoe_layer_stack_run(void * stream, qwmoe_layer_stack * s, const float * x, int64_t T, float * out,
                          float * x_out, int32_t * ids_out, float * weights_out);
void qwmoe_layer_stack_free(qwmoe_layer_stack * s);
/* Graphs the stack has captured so far (no reference counterpart; a
 * diagnostic): a run captures again after qwmoe_init reallocated the workspace
 * or qwmoe_set_mfma_min_rows changed the threshold. */
int64_t qwmoe_layer_stack_captures(const qwmoe_layer_stack * s);
/* Which path a stack's runs at 2 <= T <= 8 take (no reference counterpart; the
 * kernel choice only): 1 = the per-layer chain above (every T); 2 = one
 * persistent launch for all layers (verify_xcd.hip: the batch's distinct experts
 * dealt to the XCDs, each expert's rows loaded once for all its tokens), picked
 * at creation on 256-CU devices when every layer has H = 2048, F = 768, E of 32,
 * 64 or 128, k <= 8, Q4_K gate/up/down with 16-byte aligned rows, no resident
 * mask and one expert_weights_scale; 3 = the same with every exchange word at
 * device scope.  T = 1 runs on the whole-stack decode kernel
 * (qwmoe_decode_stack_*, one launch per token) wherever qwmoe_decode_stack_create
 * takes the stack's layers, else on the per-layer chain.  QWMOE_VERIFY_XCD=0 in
 * the environment at creation forces the per-layer chain for every T (1).
 * Results are identical. */
int qwmoe_layer_stack_kernel(const qwmoe_layer_stack * s);
/* The kernel a T = 1 run takes outside capture (no reference counterpart):
 * qwmoe_decode_stack_kernel's value for the stack's private decode stack
 * (created here if no T = 1 run has created it yet), or 0 for the per-layer
 * chain (shapes the decode stack does not take, or QWMOE_VERIFY_XCD=0). */
int qwmoe_layer_stack_kernel_t1(qwmoe_layer_stack * s);
/* Synchronises `stream`; the persistent launches' status bits (those of the
 * T >= 2 kernel or'ed with the T = 1 decode kernel's, as
 * qwmoe_decode_stack_status: 1 top-k tie replayed, 8 a wait timed out plus the
 * exchange, 16 a slot out of range), 0 for the per-layer chain. */
int qwmoe_layer_stack_status(void * stream, qwmoe_layer_stack * s, int32_t * status_out, int clear);

/* ---- expert slot table (host) ------------------------------------------------ */

/* Resident-only counterpart of ExpertCache's slot bookkeeping
 * (core/expert_cache.h:39-166; key = layer * n_expert + expert,
 * core/expert_cache.cpp:691-721): one (role, layer) row maps logical expert ids
 * to slots of that role's pool.  Tables live in host memory; copy a row to the
 * device for qwmoe_layer.slot_*.  role: 0 gate, 1 up, 2 down (ExpertCache::Role). */
typedef struct qwmoe_slot_table qwmoe_slot_table;
qwmoe_slot_table * qwmoe_slot_table_create(int n_layer, int n_expert);
void qwmoe_slot_table_free(qwmoe_slot_table * t);
/* Places every (layer, expert) of every role: identity (seed == 0) or a seeded
 * random permutation of the n_layer * n_expert slots of each role's pool. */
int qwmoe_slot_table_fill(qwmoe_slot_table * t, uint64_t seed);
int qwmoe_slot_table_set(qwmoe_slot_table * t, int role, int layer, int expert, int32_t slot);
int32_t qwmoe_slot_table_slot_of(const qwmoe_slot_table * t, int role, int layer, int expert);
/* Dense row for (role, layer): n_expert entries (ExpertCache::slot_of_row). */
const int32_t * qwmoe_slot_table_row(const qwmoe_slot_table * t, int role, int layer);

/* ---- GGUF models --------------------------------------------------------------- */

/* GGUF metadata of a model file, or of a "<name>-00001-of-0000N.gguf" shard set
 * (KV from the first shard, tensors from all).  Replaces gguf_init_from_file
 * with no_alloc per shard (ggml/src/gguf.cpp:451-906) and Model::load's unified
 * tensor map with per-tensor (shard file, absolute offset) sources
 * (core/model.cpp:400-502).  Opening reads metadata only (host memory); the
 * same files the reference rejects are rejected with QWMOE_ERR_FORMAT. */
typedef struct qwmoe_gguf qwmoe_gguf;
typedef struct qwmoe_gguf_tensor_info {
    char name[64];
    int32_t type;              /* ggml type id */
    int32_t n_dims;
    int64_t ne[4];
    uint64_t offset;           /* within its shard's data section (gguf_get_tensor_offset) */
    uint64_t file_offset;      /* absolute, in its shard file (Model::src_) */
    uint64_t nbytes;           /* gguf_get_tensor_size */
    int32_t shard;
} qwmoe_gguf_tensor_info;
/* Hyperparameters of the MoE FFN path, read as Model::load_hparams does
 * (core/model.cpp:504-548): "<arch>.block_count", ".embedding_length",
 * ".expert_count", ".expert_used_count", ".expert_feed_forward_length",
 * ".expert_weights_scale" (default 1). */
typedef struct qwmoe_moe_hparams {
    char arch[32];
    int32_t n_layer, n_embd, n_expert, n_expert_used, n_ff_exp;
    float expert_weights_scale;
} qwmoe_moe_hparams;

int qwmoe_gguf_open(const char * path, qwmoe_gguf ** out);
void qwmoe_gguf_close(qwmoe_gguf * g);
int qwmoe_gguf_n_shards(const qwmoe_gguf * g);
int qwmoe_gguf_shard_info(const qwmoe_gguf * g, int shard, uint32_t * version, uint64_t * alignment,
                          uint64_t * data_offset);
/* KV pairs (gguf_get_n_kv, gguf_find_key -> index or -1, gguf_get_kv_type /
 * gguf_get_arr_type / gguf_get_arr_n, gguf_get_arr_data / gguf_get_val_data:
 * `data` is the raw little-endian payload of fixed-size values, NULL for
 * strings, which qwmoe_gguf_kv_str returns element by element). */
/* Path of shard `shard` (the file Model::tensor_file names, core/model.cpp:300-304). */
int qwmoe_gguf_shard_path(const qwmoe_gguf * g, int shard, const char ** out);
int qwmoe_gguf_n_kv(const qwmoe_gguf * g);
int qwmoe_gguf_find_key(const qwmoe_gguf * g, const char * key);
int qwmoe_gguf_kv(const qwmoe_gguf * g, int idx, const char ** key, int32_t * type, int32_t * arr_type, uint64_t * n,
                  const void ** data);
int qwmoe_gguf_kv_str(const qwmoe_gguf * g, int idx, uint64_t i, const char ** out);
/* Typed lookups with a default, with the conversions of core/gguf_util.cpp:21-51
 * (u32 accepts UINT32/INT32/UINT64/INT64, f32 accepts FLOAT32/FLOAT64). */
int qwmoe_gguf_get_u32(const qwmoe_gguf * g, const char * key, uint32_t def, uint32_t * out);
int qwmoe_gguf_get_f32(const qwmoe_gguf * g, const char * key, float def, float * out);
int qwmoe_gguf_get_str(const qwmoe_gguf * g, const char * key, const char * def, const char ** out);
int qwmoe_gguf_n_tensors(const qwmoe_gguf * g);
int qwmoe_gguf_tensor_at(const qwmoe_gguf * g, int idx, qwmoe_gguf_tensor_info * out);
/* index of `name`, or -1 (gguf_find_tensor) */
int qwmoe_gguf_find_tensor(const qwmoe_gguf * g, const char * name, qwmoe_gguf_tensor_info * out);
int qwmoe_gguf_moe_hparams(const qwmoe_gguf * g, qwmoe_moe_hparams * hp);
/* Device bytes layer `il`'s blk.il.ffn_gate_inp / ffn_{gate,up,down}_exps
 * tensors take in qwmoe_gguf_load_moe_layer's layout (each 256-byte aligned). */
int qwmoe_gguf_moe_layer_bytes(const qwmoe_gguf * g, int il, size_t * out);
/* Reads layer `il`'s router and expert tensors into the caller's device buffer
 * `dev` (dev_bytes >= qwmoe_gguf_moe_layer_bytes) through pinned host staging
 * (the handle keeps two 16 MiB pinned buffers from its first load until close),
 * and fills `out` with pointers into it (identity slots).  Returns once the
 * copies on `stream` are complete.  Expert types: Q4_K, Q6_K, Q8_0; router: F32. */
int qwmoe_gguf_load_moe_layer(void * stream, qwmoe_gguf * g, int il, void * dev, size_t dev_bytes, qwmoe_layer * out);

/* ---- expert cache: slot pools fed from a slower tier ------------------------- */

/* ExpertCache (core/expert_cache.h:39-166, core/expert_cache.cpp:90-832): when
 * not every expert fits in HBM, slot pools hold the hot (layer, expert) slabs
 * and the rest are fetched on demand.  One pool per (role, type, ne0, ne1)
 * signature, shared by the layers that have it (cpp:128-152); every pool gets
 * the same residency fraction budget / total expert bytes, at least n_used and
 * at most n_layer_of_pool * n_expert slots (cpp:155-186); LRU victim = the first
 * slot with the smallest access stamp (cpp:374-391); key = layer * n_expert +
 * expert.  Slot rows use 0 as the non-resident sentinel, as slot_of_row does
 * (cpp:694-697): a kernel run on rows with absent experts reads slot 0, so a
 * caller that speculates checks residency of the ids it got back afterwards
 * (core/runtime.cpp:2921-2933) and repairs with ensure_resident.
 *
 * Tiers: host memory (each (role, layer) tensor's n_expert slabs back to back,
 * the RAM tier of cpp:355-364; from pinned memory, runs of consecutive slabs
 * are copied by the copy engine and scattered slabs by one gather kernel per
 * call, both asynchronous) or a file (slabs read with pread by a pool of worker threads into
 * pinned staging, then copied asynchronously: the SSD tier of cpp:297-352 and
 * 412-687, without the opt-in coalescing).  Every copy and row upload is
 * issued on the cache's stream, so work the caller issues on that stream
 * afterwards sees the slabs; calls on one cache must not overlap, and the
 * stream must outlive the cache (freeing it waits for that stream). */
typedef struct qwmoe_expert_cache qwmoe_expert_cache;

typedef struct qwmoe_expert_src {
    int32_t type;              /* ggml type: Q4_K, Q6_K or Q8_0 */
    int64_t ne0, ne1;          /* one expert's slab is [ne0, ne1]; the tensor is [ne0, ne1, n_expert] */
    const void * host;         /* host tier: n_expert slabs back to back, or NULL for the file tier */
    const char * path;         /* file tier: the file holding the same bytes ... */
    uint64_t file_offset;      /* ... from this absolute offset */
} qwmoe_expert_src;

#define QWMOE_CACHE_DRY_RUN 1  /* bookkeeping only: no device pools, no copies, no file reads (planning, tests) */
#define QWMOE_CACHE_COPY_ENGINE 2  /* host tier: every fetch by hipMemcpyAsync (no slab gather kernel) */

typedef struct qwmoe_expert_cache_config {
    size_t vram_budget;        /* bytes the slot pools may take (core/expert_cache.h:43-45) */
    int32_t n_used;            /* experts per token: every pool holds at least this many slots */
    int32_t io_threads;        /* file tier read workers (0: 8, core/expert_cache.cpp:100) */
    int32_t flags;             /* QWMOE_CACHE_DRY_RUN */
} qwmoe_expert_cache_config;

typedef struct qwmoe_expert_cache_stats {  /* ExpertCache::Stats, core/expert_cache.h:86-88 */
    uint64_t hits, misses, evictions;
    double fetch_ms;           /* host time spent reading files and issuing copies */
    uint64_t fetch_bytes;
} qwmoe_expert_cache_stats;

/* srcs: [3][n_layer] (role-major: gate, up, down), copied at creation; host
 * sources must stay valid for the cache's lifetime.  Allocates the pools and
 * a device row table [3][n_layer][n_expert] with one hipMalloc. */
int qwmoe_expert_cache_create(void * stream, int n_layer, int n_expert, const qwmoe_expert_src * srcs,
                              const qwmoe_expert_cache_config * cfg, qwmoe_expert_cache ** out);
/* From a GGUF model's blk.N.ffn_{gate,up,down}_exps.weight tensors (the
 * expert tensors ExpertCache's constructor looks up, cpp:76-89, 110-122).
 * tier 0: host RAM -- every expert tensor is read once into pinned host memory
 * the cache owns (the CPU expert buffer Model keeps for the RAM tier);
 * tier 1: file -- slabs are read from the shard files on each miss.
 * cfg->n_used == 0 takes n_expert_used from the metadata. */
int qwmoe_expert_cache_create_gguf(void * stream, const qwmoe_gguf * g, int tier, const qwmoe_expert_cache_config * cfg,
                                   qwmoe_expert_cache ** out);
void qwmoe_expert_cache_free(qwmoe_expert_cache * c);

int qwmoe_expert_cache_n_pools(const qwmoe_expert_cache * c);
/* One pool: its role, type, slab shape, slots, slab bytes and device base
 * (NULL in a dry run). */
int qwmoe_expert_cache_pool_info(const qwmoe_expert_cache * c, int pool, int32_t * role, int32_t * type, int64_t * ne0,
                                 int64_t * ne1, int64_t * n_slots, uint64_t * slab_bytes, void ** base);
/* Pool serving (role, layer) (ExpertCache::layer_pool_). */
int qwmoe_expert_cache_pool_of(const qwmoe_expert_cache * c, int role, int layer);
int qwmoe_expert_cache_min_slots(const qwmoe_expert_cache * c);          /* cpp:282-286 */
int qwmoe_expert_cache_capacity(const qwmoe_expert_cache * c, int layer); /* cpp:288-293 */

/* ExpertCache::ensure (cpp:790-832): make `layer`'s experts ids[0..n) resident
 * for all three roles, fetching the misses, and write their slot ids (host
 * arrays of n; any may be NULL).  Rejects, before changing anything, a call
 * naming more distinct experts than capacity(layer) (the reference leaves that
 * to its callers, core/runtime.cpp:2131-2146: such a call would evict its own
 * slots). */
int qwmoe_expert_cache_ensure(qwmoe_expert_cache * c, int layer, const int32_t * ids, int n, int32_t * slot_gate,
                              int32_t * slot_up, int32_t * slot_down);
/* ExpertCache::ensure_resident (cpp:779-788): fetch what is absent of
 * (layer, expert) in the three pools, counting misses only. */
int qwmoe_expert_cache_ensure_resident(qwmoe_expert_cache * c, int layer, int expert);
/* ExpertCache::touch (cpp:699-707): a resident access; no-op when absent. */
int qwmoe_expert_cache_touch(qwmoe_expert_cache * c, int role, int layer, int expert);
/* 1 resident, 0 absent, < 0 error (cpp:689-692). */
int qwmoe_expert_cache_resident(const qwmoe_expert_cache * c, int role, int layer, int expert);
/* Host row for (role, layer): n_expert slot ids, 0 when absent (cpp:694-697). */
const int32_t * qwmoe_expert_cache_slot_of_row(const qwmoe_expert_cache * c, int role, int layer);
/* Device copy of that row, kept current on the cache's stream by every call
 * that changes residency (the in-graph remap table g2s_all,
 * core/runtime.cpp:2877-2884).  NULL in a dry run. */
const int32_t * qwmoe_expert_cache_device_row(const qwmoe_expert_cache * c, int role, int layer);
/* The residency check of a speculative run (decode_cached_fast's verify and
 * accept, core/runtime.cpp:2922-2934, 2959-2972): ids [n_layer][k] are the experts a
 * whole-stack decode used (qwmoe_decode_stack_run's ids_out).  Returns how
 * many (layer, id) entries miss in at least one role; when none does and
 * `touch` is set, touches every role of every entry (hits, LRU stamps,
 * counts).  Changes nothing otherwise. */
int qwmoe_expert_cache_verify(qwmoe_expert_cache * c, const int32_t * ids, int n_layer, int k, int touch);
/* The resident-decode mask (decode_cached_fast's fill_resmask, core/runtime.cpp:
 * 2900-2919): mask [n_layer][n_expert] gets 0 for an expert resident in all
 * three roles and -inf otherwise; a layer with fewer than floor_res residents
 * is left unmasked (all 0).  floor_res below n_expert_used counts as n_expert_used
 * (a thinner mask would let top-k pick absent experts).  Returns 1 when every layer is masked ("complete":
 * the masked decode cannot miss), 0 otherwise.  mask_dev (optional, device):
 * the same values copied there on the cache's stream before returning -- the
 * layers' resmask rows point into it. */
int qwmoe_expert_cache_resmask(const qwmoe_expert_cache * c, int floor_res, float * mask, float * mask_dev);
/* The background refill after a masked decode (core/runtime.cpp:2976-3008):
 * touches every selected expert sel [n_layer][k] in all roles, then, walking
 * the layers round robin from *cursor, fetches (ensure_resident) wanted-but-
 * absent experts of want [n_layer][k] (the layers' want_ids) until `budget`
 * fetches are spent; *cursor advances by one layer.  Returns the fetches made.
 * budget <= 0 does nothing, as in the reference. */
int qwmoe_expert_cache_refill(qwmoe_expert_cache * c, const int32_t * sel, const int32_t * want, int n_layer, int k,
                              int budget, int * cursor);
/* Fills L's expert fields (types, pool bases, strides, slot counts, device
 * rows) for `layer`; the caller sets shapes, router and scale. */
int qwmoe_expert_cache_layer(const qwmoe_expert_cache * c, int layer, qwmoe_layer * L);
int qwmoe_expert_cache_get_stats(const qwmoe_expert_cache * c, qwmoe_expert_cache_stats * out);
/* Hot-expert profile in the reference's text format (cpp:723-741):
 * "QWENEXPCACHE 1", "<n_layer> <n_expert>", then "<role> <layer> <expert> <count>"
 * lines; keys are written in ascending order per pool. */
int qwmoe_expert_cache_save_profile(const qwmoe_expert_cache * c, const char * path);
/* ExpertCache::load_prefetch (cpp:743-777): installs the most-accessed keys
 * until each pool is full; equal counts keep file order (the reference's
 * std::sort leaves their order unspecified).  A missing or incompatible file
 * prefetches nothing and is not an error.  *n_prefetched may be NULL. */
int qwmoe_expert_cache_load_prefetch(qwmoe_expert_cache * c, const char * path, uint64_t * n_prefetched);
/* Waits for every copy the cache issued. */
int qwmoe_expert_cache_sync(qwmoe_expert_cache * c);
/* One layer of decode_cached (core/runtime.cpp:2458-2662, ensure_layer 2593-2600)
 * on the cache's stream: the router's ids for x [T][H] are read back (pinned
 * host buffer, one synchronisation), ensure() makes them resident, then
 * qwmoe_ffn_layer runs on the pools.  L gives shapes, router and scale (its
 * expert fields are taken from the cache).  At most 64 * n_expert_used ids per
 * call; outputs as qwmoe_ffn_layer's.  The first call allocates a small id buffer. */
int qwmoe_expert_cache_run_layer(qwmoe_expert_cache * c, int layer, const qwmoe_layer * L, const float * x, int64_t T,
                                 float * out, float rms_eps, float * x_next, int32_t * ids_out, float * weights_out);
/* plan_slices of the chunked prefill (core/runtime.cpp:2144-2170): tokens
 * t = 0..T-1 with selections sel [T][n_used] are cut into slices (t0, len) so
 * that no slice names more than `cap` distinct experts (one ensure() must not
 * evict its own slots) nor runs longer than max_slice tokens (< 1: 1024); a
 * token that would overflow opens the next slice.  slices: [T][2] capacity;
 * union_list (optional, [n_expert]) receives the chunk's distinct experts in
 * first-use order, n_union (optional) their count.  Host only. */
int qwmoe_plan_slices(const int32_t * sel, int T, int n_used, int n_expert, int cap, int max_slice, int32_t * slices,
                      int * n_slices, int32_t * union_list, int * n_union);
/* The same for a cache layer, with the reference's cap = max(n_used,
 * capacity(layer) - 8). */
int qwmoe_expert_cache_plan_slices(const qwmoe_expert_cache * c, int layer, const int32_t * sel, int T, int max_slice,
                                   int32_t * slices, int * n_slices);
/* One layer of the chunked prefill through the cache (segment B of
 * core/runtime.cpp:2100-2300): the router's ids for all T tokens are read back,
 * planned into slices, and each slice's experts made resident (ensure) before
 * qwmoe_ffn_layer runs on its tokens -- lossless, the FFN being per token.
 * Any T; outputs as qwmoe_ffn_layer's; *n_slices_out (optional) the slices run.
 * Grows the cache's id buffers when T needs more. */
int qwmoe_expert_cache_run_batch(qwmoe_expert_cache * c, int layer, const qwmoe_layer * L, const float * x, int64_t T,
                                 float * out, float rms_eps, float * x_next, int32_t * ids_out, float * weights_out,
                                 int max_slice, int * n_slices_out);

/* ---- host-side checks (no GPU needed) ---------------------------------------- */

/* The std::sort replay the router uses when top-k ties occur, run on the host:
 * idx[0..n) = argsort of values, descending, in exactly std::sort's order. */
int qwmoe_host_argsort_desc(const float * values, int n, int32_t * idx);

#ifdef __cplusplus
}
#endif

#endif /* QWMOE_H */
