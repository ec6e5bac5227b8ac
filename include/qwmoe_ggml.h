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

#include <stdint.h>

#include "qwmoe.h"

/* Whether the op is a mul_mat_id libqwmoe takes -- exactly the nodes
 * qwmoe_mul_mat_id accepts, so a scheduler that asks first never sees the call
 * fail: Q4_K / Q6_K experts with K a multiple of 256 or Q8_0 with K a multiple
 * of 64, f32 activations whose rows broadcast as ggml's e % ne11 with
 * ne11 = 1 or n_ids, 16-byte aligned activation data and row / matrix strides
 * (the activation quantizer's loads), i32 ids with contiguous rows, an f32
 * output whose strides cover its rows, no fourth dimension. */
static inline int qwmoe_ggml_supports_mul_mat_id(const struct ggml_tensor * op) {
    if (op->op != GGML_OP_MUL_MAT_ID) return 0;
    const struct ggml_tensor * as = op->src[0], * b = op->src[1], * ids = op->src[2];
    if (!as || !b || !ids) return 0;
    const int wtype = as->type == GGML_TYPE_Q4_K || as->type == GGML_TYPE_Q6_K || as->type == GGML_TYPE_Q8_0;
    const int64_t blk = as->type == GGML_TYPE_Q8_0 ? 64 : 256;
    const int64_t n_ids = ids->ne[0];
    if (!wtype || b->type != GGML_TYPE_F32 || ids->type != GGML_TYPE_I32 || op->type != GGML_TYPE_F32) return 0;
    if (as->ne[0] <= 0 || as->ne[0] % blk != 0 || as->ne[3] != 1 || b->ne[3] != 1 || ids->ne[2] != 1) return 0;
    if (as->nb[2] < as->nb[1] * (size_t) as->ne[1]) return 0;
    if (b->ne[1] != 1 && b->ne[1] != n_ids) return 0;
    if (b->nb[0] != sizeof(float) || b->nb[1] % 16 != 0 || b->nb[2] % 16 != 0 || ((uintptr_t) b->data & 15)) return 0;
    if (ids->nb[0] != sizeof(int32_t) || ids->nb[1] < (size_t) n_ids * 4 || ids->nb[1] % 4 != 0) return 0;
    if (op->nb[0] != sizeof(float) || op->nb[1] < (size_t) as->ne[1] * 4 || op->nb[2] < op->nb[1] * (size_t) n_ids)
        return 0;
    return 1;
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
