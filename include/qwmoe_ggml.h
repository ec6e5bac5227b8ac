/* qwmoe_ggml.h -- glue for a ggml backend that hands GGML_OP_MUL_MAT_ID nodes
 * to libqwmoe (the drop-in for the reference's mul_mat_id op; ggml's backend
 * interface: ggml-backend-impl.h:130 graph_compute, :189 supports_op).
 * Header only, C or C++: include after ggml.h.
 *
 *   supports_op:   return qwmoe_ggml_supports_mul_mat_id(op);
 *   graph_compute: for a node t with t->op == GGML_OP_MUL_MAT_ID,
 *                  qwmoe_ggml_mul_mat_id(stream, t, NULL, 0) == QWMOE_OK
 *
 * The node's tensors must live in device memory; their ne / nb fields are
 * passed as they are, so the strided ids view ggml_argsort_top_k returns
 * (nb[1] = n_expert * 4) and [K, N, n_as] expert tensors need no copies. */
#ifndef QWMOE_GGML_H
#define QWMOE_GGML_H

#include "qwmoe.h"

/* Whether the op is a mul_mat_id libqwmoe takes: Q4_K / Q6_K / Q8_0 experts
 * with whole blocks per row, f32 activations and output with contiguous rows,
 * i32 ids, no fourth dimension. */
static inline int qwmoe_ggml_supports_mul_mat_id(const struct ggml_tensor * op) {
    if (op->op != GGML_OP_MUL_MAT_ID) return 0;
    const struct ggml_tensor * as = op->src[0], * b = op->src[1], * ids = op->src[2];
    const int wtype = as->type == GGML_TYPE_Q4_K || as->type == GGML_TYPE_Q6_K || as->type == GGML_TYPE_Q8_0;
    const int64_t blk = as->type == GGML_TYPE_Q8_0 ? 64 : 256;
    return wtype && b->type == GGML_TYPE_F32 && ids->type == GGML_TYPE_I32 && op->type == GGML_TYPE_F32 &&
           as->ne[0] % blk == 0 && as->ne[3] == 1 && b->ne[3] == 1 && b->nb[0] == sizeof(float) &&
           ids->nb[0] == sizeof(int32_t) && op->nb[0] == sizeof(float);
}

/* Runs the node on `stream` (a hipStream_t).  slot_row: optional logical id ->
 * matrix index map of n_slot_row entries (ExpertCache::slot_of_row), instead
 * of the graph's get_rows(g2s, selected) remap.  Returns a QWMOE_* status. */
static inline int qwmoe_ggml_mul_mat_id(void * stream, const struct ggml_tensor * t, const int32_t * slot_row,
                                        int64_t n_slot_row) {
    const struct ggml_tensor * as = t->src[0], * b = t->src[1], * ids = t->src[2];
    return qwmoe_mul_mat_id(stream, (int) as->type, as->data, as->ne[0], as->ne[1], as->ne[2], as->nb[1], as->nb[2],
                            (const float *) b->data, b->ne[1], b->ne[2], b->nb[1], b->nb[2],
                            (const int32_t *) ids->data, ids->ne[0], ids->nb[1], slot_row, n_slot_row,
                            (float *) t->data, t->nb[1], t->nb[2]);
}

#endif /* QWMOE_GGML_H */
