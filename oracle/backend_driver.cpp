// backend_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Runs build_moe's graph (core/runtime.cpp:861-974: router mul_mat -> soft_max
// -> argsort_top_k -> weight normalisation -> 3x mul_mat_id + swiglu_split ->
// weighted sum, then an RMSNorm) through ggml_backend_sched with two backends:
// the QWMOE backend (questwend_amd/libggml-qwmoe.so, include/ggml-qwmoe.h)
// first and ggml's CPU backend after it.  The expert tensors live in a QWMOE
// buffer, so the scheduler gives the three mul_mat_id nodes to QWMOE and every
// other node to the CPU, copying activations between them.  The router weight
// lives in a CPU buffer.  Both weight buffers are marked as weights, as the
// reference marks its model and ExpertCache buffers.  Built by oracle/Makefile.ref into
// oracle/_ref/libqwbe.so against the reference ggml (libqwref.so); only tests/
// load it.  It calls ggml's public API and the backend's registration only.

#include "ggml.h"
#include "ggml-alloc.h"
#include "ggml-backend.h"
#include "ggml-cpu.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "ggml-qwmoe.h"

extern "C" {

// weights as qwref_layer_create takes them: router f32 [E][H]; gate / up
// [E][F] rows of H, down [E][H] rows of F (ggml [K, N, E]).  x [T][H].
// Outputs: out / xnext [T][H], ids [T][k]; n_splits: the scheduler's graph
// splits; n_mmid_qwmoe: mul_mat_id nodes the scheduler gave to QWMOE.
// Returns 0, or < 0 when a step failed.
int qwbe_sched_moe(int64_t H, int64_t E, int64_t k, int64_t F, int64_t T, int type_gate, int type_up, int type_down,
                   const float* w_router, const void* w_gate, const void* w_up, const void* w_down, float rms_eps,
                   const float* x, float* out, float* xnext, int32_t* ids, int* n_splits, int* n_mmid_qwmoe,
                   int n_threads) {
    ggml_backend_t qw = ggml_backend_qwmoe_init(0);
    if (!qw) return -1;
    ggml_backend_t cpu = ggml_backend_cpu_init();
    if (!cpu) {
        ggml_backend_free(qw);
        return -2;
    }
    ggml_backend_cpu_set_n_threads(cpu, n_threads);
    int rc = 0;

    // weights: experts in a QWMOE buffer, the router in a CPU buffer
    ggml_init_params wp = {ggml_tensor_overhead() * 8, nullptr, true};
    ggml_context* wctx_q = ggml_init(wp);
    ggml_context* wctx_c = ggml_init(wp);
    ggml_tensor* Wg = ggml_new_tensor_3d(wctx_q, (ggml_type) type_gate, H, F, E);
    ggml_tensor* Wu = ggml_new_tensor_3d(wctx_q, (ggml_type) type_up, H, F, E);
    ggml_tensor* Wd = ggml_new_tensor_3d(wctx_q, (ggml_type) type_down, F, H, E);
    ggml_tensor* Wr = ggml_new_tensor_2d(wctx_c, GGML_TYPE_F32, H, E);
    ggml_backend_buffer_t bq = ggml_backend_alloc_ctx_tensors(wctx_q, qw);
    ggml_backend_buffer_t bc = ggml_backend_alloc_ctx_tensors(wctx_c, cpu);
    if (!bq || !bc) rc = -3;
    // model weights, as core/model.cpp:190 and core/expert_cache.cpp:190 mark
    // them: the scheduler runs an op where its weights live
    if (bq) ggml_backend_buffer_set_usage(bq, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    if (bc) ggml_backend_buffer_set_usage(bc, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    ggml_context* ctx = nullptr;
    ggml_backend_sched_t sched = nullptr;
    if (rc == 0) {
        ggml_backend_tensor_set(Wg, w_gate, 0, ggml_nbytes(Wg));
        ggml_backend_tensor_set(Wu, w_up, 0, ggml_nbytes(Wu));
        ggml_backend_tensor_set(Wd, w_down, 0, ggml_nbytes(Wd));
        ggml_backend_tensor_set(Wr, w_router, 0, ggml_nbytes(Wr));

        ggml_init_params ip = {ggml_tensor_overhead() * 512 + ggml_graph_overhead() + (1 << 16), nullptr, true};
        ctx = ggml_init(ip);
        ggml_tensor* X = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, T);
        ggml_set_input(X);
        ggml_tensor* logits = ggml_mul_mat(ctx, Wr, X);
        ggml_tensor* probs = ggml_soft_max(ctx, logits);
        ggml_tensor* selected = ggml_argsort_top_k(ctx, probs, (int) k);
        ggml_tensor* weights = ggml_get_rows(ctx, ggml_reshape_3d(ctx, probs, 1, E, T), selected);
        weights = ggml_reshape_2d(ctx, weights, k, T);
        ggml_tensor* wsum = ggml_clamp(ctx, ggml_sum_rows(ctx, weights), 6.103515625e-5f, INFINITY);
        weights = ggml_reshape_3d(ctx, ggml_div(ctx, weights, wsum), 1, k, T);
        ggml_tensor* x3 = ggml_reshape_3d(ctx, X, H, 1, T);
        ggml_tensor* up = ggml_mul_mat_id(ctx, Wu, x3, selected);
        ggml_tensor* gate = ggml_mul_mat_id(ctx, Wg, x3, selected);
        ggml_tensor* experts = ggml_mul_mat_id(ctx, Wd, ggml_swiglu_split(ctx, gate, up), selected);
        ggml_cgraph* gf = ggml_new_graph(ctx);
        ggml_tensor* moe_out;
        if (T == 1) {
            ggml_tensor* et = ggml_cont(ctx, ggml_transpose(ctx, ggml_reshape_2d(ctx, experts, H, k)));
            moe_out = ggml_mul_mat(ctx, et, ggml_reshape_2d(ctx, weights, k, 1));
        } else {
            ggml_tensor* ew = ggml_mul(ctx, experts, weights);
            moe_out = ggml_view_2d(ctx, ew, H, T, ew->nb[2], 0);
            for (int i = 1; i < k; ++i)
                moe_out = ggml_add(ctx, moe_out, ggml_view_2d(ctx, ew, H, T, ew->nb[2], (size_t) i * ew->nb[1]));
            if (k == 1) moe_out = ggml_cont(ctx, moe_out);
        }
        ggml_tensor* xn = ggml_rms_norm(ctx, moe_out, rms_eps);
        ggml_tensor* ids_c = ggml_cont(ctx, selected);
        ggml_set_output(moe_out);
        ggml_set_output(xn);
        ggml_set_output(ids_c);
        ggml_build_forward_expand(gf, moe_out);
        ggml_build_forward_expand(gf, xn);
        ggml_build_forward_expand(gf, ids_c);

        ggml_backend_t backends[2] = {qw, cpu};
        sched = ggml_backend_sched_new(backends, nullptr, 2, GGML_DEFAULT_GRAPH_SIZE, false, true);
        if (!sched || !ggml_backend_sched_alloc_graph(sched, gf)) rc = -4;
        if (rc == 0) {
            ggml_backend_tensor_set(X, x, 0, ggml_nbytes(X));
            if (ggml_backend_sched_graph_compute(sched, gf) != GGML_STATUS_SUCCESS) rc = -5;
        }
        if (rc == 0) {
            ggml_backend_tensor_get(moe_out, out, 0, ggml_nbytes(moe_out));
            ggml_backend_tensor_get(xn, xnext, 0, ggml_nbytes(xn));
            ggml_backend_tensor_get(ids_c, ids, 0, ggml_nbytes(ids_c));
            *n_splits = ggml_backend_sched_get_n_splits(sched);
            int n = 0;
            for (int i = 0; i < ggml_graph_n_nodes(gf); ++i) {
                ggml_tensor* nd = ggml_graph_node(gf, i);
                if (nd->op == GGML_OP_MUL_MAT_ID && ggml_backend_sched_get_tensor_backend(sched, nd) == qw) ++n;
            }
            *n_mmid_qwmoe = n;
        }
    }
    if (sched) ggml_backend_sched_free(sched);
    if (ctx) ggml_free(ctx);
    if (bq) ggml_backend_buffer_free(bq);
    if (bc) ggml_backend_buffer_free(bc);
    ggml_free(wctx_q);
    ggml_free(wctx_c);
    ggml_backend_free(cpu);
    ggml_backend_free(qw);
    return rc;
}

// The registry as ggml's reg API reports it: device count and the first
// device's name into name (cap bytes).
int qwbe_registry(char* name, int cap) {
    ggml_backend_reg_t reg = ggml_backend_qwmoe_reg();
    const size_t n = ggml_backend_reg_dev_count(reg);
    if (n > 0 && name && cap > 0) {
        strncpy(name, ggml_backend_dev_name(ggml_backend_reg_dev_get(reg, 0)), (size_t) cap - 1);
        name[cap - 1] = 0;
    }
    return (int) n;
}

}  // extern "C"
