// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A small C-ABI shim over the *real* ggml CPU backend, compiled from the sources
// under /root/reference/third_party/ggml by oracle/Makefile.ref into
// oracle/_ref/libqwref.so.  It is this repository's own code and calls only
// ggml's public API.  It exists to (1) pin the CPU restatement in
// oracle/qwmoe_oracle.cpp against the reference bit for bit, (2) write the
// golden fixtures under tests/golden/, and (3) serve as the timed CPU baseline
// ("kind": "reference") in bench.py.  The product library never links it.
//
// The MoE layer graph below is the op sequence of
// core/runtime.cpp:861-974 (Runtime::Impl::build_moe, non-cache path):
//   router mul_mat (869) -> soft_max (883) -> argsort_top_k (885) ->
//   get_rows/sum_rows/clamp/div (887-897) -> 3x mul_mat_id + swiglu_split
//   (935-938) -> weighted sum: transposed mul_mat for T=1 (940-945) or
//   mul + add chain for T>1 (947-959).
// An optional ggml_rms_norm (ggml/src/ggml-cpu/ops.cpp:3795-3860) follows it so
// layers can be stacked the way the 48-layer decode benchmark does.

#include "ggml.h"
#include "ggml-cpu.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

extern "C" {

// ggml_cpu_init fills the CPU backend's lookup tables (fp16 table, type
// traits); it is idempotent and cheap after the first call.
static void ensure_init() {
    static bool done = false;
    if (!done) { ggml_cpu_init(); done = true; }
}

// ggml_quantize_chunk with imatrix = NULL (ggml/src/ggml.c:7919-8000).
size_t qwref_quantize(int type, const float * src, void * dst, int64_t nrows, int64_t n_per_row) {
    ensure_init();
    return ggml_quantize_chunk((enum ggml_type) type, src, dst, 0, nrows, n_per_row, nullptr);
}

// type_traits_cpu[type].from_float: the activation quantizer mul_mat_id uses.
int qwref_from_float(int type, const float * x, void * y, int64_t n) {
    ensure_init();
    const struct ggml_type_traits_cpu * t = ggml_get_type_traits_cpu((enum ggml_type) type);
    if (!t || !t->from_float) return -1;
    t->from_float(x, y, n);
    return 0;
}

// type_traits_cpu[type].vec_dot on one (weight row, quantized activation row).
int qwref_vec_dot(int type, int n, const void * x, const void * y, float * s) {
    ensure_init();
    const struct ggml_type_traits_cpu * t = ggml_get_type_traits_cpu((enum ggml_type) type);
    if (!t || !t->vec_dot) return -1;
    t->vec_dot(n, s, 0, x, 0, y, 0, 1);
    return 0;
}

int qwref_vec_dot_type(int type) {
    ensure_init();
    return (int) ggml_get_type_traits_cpu((enum ggml_type) type)->vec_dot_type;
}

int qwref_dequantize(int type, const void * x, float * y, int64_t n) {
    ensure_init();
    const struct ggml_type_traits * t = ggml_get_type_traits((enum ggml_type) type);
    if (!t || !t->to_float) return -1;
    t->to_float(x, y, n);
    return 0;
}

size_t qwref_row_size(int type, int64_t n) { return ggml_row_size((enum ggml_type) type, n); }

// ---------------------------------------------------------------------------
// One MoE FFN layer on the CPU backend, built once and evaluated many times.

struct qwref_layer {
    ggml_context * wctx = nullptr;   // weights: no_alloc, data owned by the caller
    ggml_context * ctx  = nullptr;   // activations and intermediates
    ggml_cgraph  * gf   = nullptr;
    ggml_tensor * x = nullptr, * logits = nullptr, * probs = nullptr, * selected = nullptr,
                * weights = nullptr, * up = nullptr, * gate = nullptr, * act = nullptr,
                * experts = nullptr, * out = nullptr, * xnext = nullptr;
    std::vector<uint8_t> work;
    int n_threads = 1;
    int64_t H = 0, E = 0, K = 0, F = 0, T = 0;
};

// types: ggml type ids for gate/up/down expert tensors [K=H,N=F,E] / [K=F,N=H,E].
// w_router: f32 [H, E] (ne0 = H).  rms_eps < 0 disables the trailing RMSNorm.
qwref_layer * qwref_layer_create(int64_t H, int64_t E, int64_t k, int64_t F, int64_t T,
                                 int type_gate, int type_up, int type_down,
                                 const float * w_router, const void * w_gate, const void * w_up,
                                 const void * w_down, float expert_weights_scale, float rms_eps,
                                 int n_threads) {
    ensure_init();
    qwref_layer * L = new qwref_layer();
    L->H = H; L->E = E; L->K = k; L->F = F; L->T = T; L->n_threads = n_threads;

    ggml_init_params wp = { ggml_tensor_overhead() * 8, nullptr, true };
    L->wctx = ggml_init(wp);
    ggml_tensor * Wr = ggml_new_tensor_2d(L->wctx, GGML_TYPE_F32, H, E);
    ggml_tensor * Wg = ggml_new_tensor_3d(L->wctx, (ggml_type) type_gate, H, F, E);
    ggml_tensor * Wu = ggml_new_tensor_3d(L->wctx, (ggml_type) type_up, H, F, E);
    ggml_tensor * Wd = ggml_new_tensor_3d(L->wctx, (ggml_type) type_down, F, H, E);
    Wr->data = (void *) w_router; Wg->data = (void *) w_gate;
    Wu->data = (void *) w_up;     Wd->data = (void *) w_down;

    // intermediates: generous bound, all f32 except ids
    size_t act_bytes = sizeof(float) * (size_t) T * (size_t) (
        H * 4 + E * 4 + k * 8 + F * k * 4 + H * k * 4 + H * k * 2);
    ggml_init_params ip = { act_bytes + ggml_tensor_overhead() * 256 + ggml_graph_overhead() + (1 << 20),
                            nullptr, false };
    L->ctx = ggml_init(ip);
    ggml_context * ctx = L->ctx;

    L->x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, T);
    ggml_tensor * logits = ggml_mul_mat(ctx, Wr, L->x);                       // [E, T]
    ggml_tensor * probs  = ggml_soft_max(ctx, logits);
    ggml_tensor * selected = ggml_argsort_top_k(ctx, probs, (int) k);         // [k, T] i32 view
    ggml_tensor * probs3 = ggml_reshape_3d(ctx, probs, 1, E, T);
    ggml_tensor * weights = ggml_get_rows(ctx, probs3, selected);             // [1, k, T]
    weights = ggml_reshape_2d(ctx, weights, k, T);
    ggml_tensor * wsum = ggml_sum_rows(ctx, weights);
    wsum = ggml_clamp(ctx, wsum, 6.103515625e-5f, INFINITY);
    weights = ggml_div(ctx, weights, wsum);
    weights = ggml_reshape_3d(ctx, weights, 1, k, T);
    if (expert_weights_scale != 0.0f && expert_weights_scale != 1.0f)
        weights = ggml_scale(ctx, weights, expert_weights_scale);

    ggml_tensor * x3 = ggml_reshape_3d(ctx, L->x, H, 1, T);
    ggml_tensor * up   = ggml_mul_mat_id(ctx, Wu, x3, selected);
    ggml_tensor * gate = ggml_mul_mat_id(ctx, Wg, x3, selected);
    ggml_tensor * act  = ggml_swiglu_split(ctx, gate, up);
    ggml_tensor * experts = ggml_mul_mat_id(ctx, Wd, act, selected);          // [H, k, T]

    L->gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(L->gf, weights);
    ggml_tensor * moe_out;
    if (T == 1) {
        ggml_tensor * et = ggml_cont(ctx, ggml_transpose(ctx, ggml_reshape_2d(ctx, experts, H, k)));
        ggml_tensor * w  = ggml_reshape_2d(ctx, weights, k, 1);
        moe_out = ggml_mul_mat(ctx, et, w);
    } else {
        ggml_tensor * ew = ggml_mul(ctx, experts, weights);
        ggml_build_forward_expand(L->gf, ew);
        std::vector<ggml_tensor *> cur(k);
        for (int i = 0; i < k; ++i) {
            cur[i] = ggml_view_2d(ctx, ew, H, T, ew->nb[2], (size_t) i * ew->nb[1]);
            ggml_build_forward_expand(L->gf, cur[i]);
        }
        moe_out = cur[0];
        for (int i = 1; i < k; ++i) {
            moe_out = ggml_add(ctx, moe_out, cur[i]);
            ggml_build_forward_expand(L->gf, moe_out);
        }
        if (k == 1) moe_out = ggml_cont(ctx, moe_out);
    }
    ggml_build_forward_expand(L->gf, moe_out);
    ggml_tensor * xnext = nullptr;
    if (rms_eps >= 0.0f) {
        xnext = ggml_rms_norm(ctx, moe_out, rms_eps);
        ggml_build_forward_expand(L->gf, xnext);
    }
    // keep intermediates observable
    ggml_build_forward_expand(L->gf, up);
    ggml_build_forward_expand(L->gf, gate);
    ggml_build_forward_expand(L->gf, act);
    ggml_build_forward_expand(L->gf, experts);

    L->logits = logits; L->probs = probs; L->selected = selected; L->weights = weights;
    L->up = up; L->gate = gate; L->act = act; L->experts = experts; L->out = moe_out; L->xnext = xnext;

    ggml_cplan plan = ggml_graph_plan(L->gf, n_threads, nullptr);
    L->work.resize(plan.work_size + 64);
    return L;
}

void qwref_layer_free(qwref_layer * L) {
    if (!L) return;
    ggml_free(L->ctx);
    ggml_free(L->wctx);
    delete L;
}

static void copy_2d(const ggml_tensor * t, void * dst, size_t elt) {
    // copies a (possibly strided in dim 1) 2-D tensor to a dense buffer
    const int64_t n0 = t->ne[0], n1 = t->ne[1] * t->ne[2] * t->ne[3];
    for (int64_t i1 = 0; i1 < n1; ++i1) {
        memcpy((char *) dst + i1 * n0 * elt, (const char *) t->data + i1 * t->nb[1], n0 * elt);
    }
}

// The router of a resident-only decode, core/runtime.cpp:869-897 with the
// cache_fast_build && resident_decode branch (870-881): want =
// argsort_top_k(logits), logits = add(logits, mask [E] broadcast over the
// tokens), then soft_max / argsort_top_k / get_rows / sum_rows / clamp / div
// (/ scale).  W: f32 [H, E]; x [T, H]; want / ids / weights [T, k]; probs [T, E]
// (nullable).
int qwref_router_resident(int64_t H, int64_t E, int64_t k, int64_t T, const float * w_router, const float * x,
                          const float * mask, float expert_weights_scale, int32_t * want, int32_t * ids,
                          float * weights_out, float * probs_out, int n_threads) {
    ensure_init();
    ggml_init_params ip = { sizeof(float) * (size_t) T * (size_t) (H + 4 * E + 4 * k) + sizeof(float) * (size_t) E
                                + ggml_tensor_overhead() * 64 + ggml_graph_overhead() + (1 << 20),
                            nullptr, false };
    ggml_context * ctx = ggml_init(ip);
    ggml_tensor * Wr = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, E);
    memcpy(Wr->data, w_router, sizeof(float) * H * E);
    ggml_tensor * X = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, T);
    memcpy(X->data, x, sizeof(float) * H * T);
    ggml_tensor * M = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, E, 1);
    memcpy(M->data, mask, sizeof(float) * E);
    ggml_tensor * logits = ggml_mul_mat(ctx, Wr, X);
    ggml_tensor * wnt = ggml_argsort_top_k(ctx, logits, (int) k);
    ggml_tensor * probs = ggml_soft_max(ctx, ggml_add(ctx, logits, M));
    ggml_tensor * selected = ggml_argsort_top_k(ctx, probs, (int) k);
    ggml_tensor * weights = ggml_get_rows(ctx, ggml_reshape_3d(ctx, probs, 1, E, T), selected);
    weights = ggml_reshape_2d(ctx, weights, k, T);
    ggml_tensor * wsum = ggml_clamp(ctx, ggml_sum_rows(ctx, weights), 6.103515625e-5f, INFINITY);
    weights = ggml_div(ctx, weights, wsum);
    if (expert_weights_scale != 0.0f && expert_weights_scale != 1.0f)
        weights = ggml_scale(ctx, weights, expert_weights_scale);
    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, wnt);
    ggml_build_forward_expand(gf, weights);
    ggml_build_forward_expand(gf, selected);
    ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    const int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    if (rc == 0) {
        if (want) copy_2d(wnt, want, 4);
        if (ids) copy_2d(selected, ids, 4);
        if (weights_out) copy_2d(weights, weights_out, 4);
        if (probs_out) copy_2d(probs, probs_out, 4);
    }
    ggml_free(ctx);
    return rc;
}

// Evaluates the layer on x [T, H] (row-major == ggml [H, T]).  Any output
// pointer may be NULL.  ids/weights are [T, k]; logits/probs [T, E];
// gate/up/act [T, k, F]; experts [T, k, H]; out / xnext [T, H].
int qwref_layer_eval(qwref_layer * L, const float * x, float * out, float * xnext,
                     int32_t * ids, float * weights, float * logits, float * probs,
                     float * gate, float * up, float * act, float * experts, int n_threads) {
    memcpy(L->x->data, x, sizeof(float) * L->H * L->T);
    ggml_cplan plan = ggml_graph_plan(L->gf, n_threads > 0 ? n_threads : L->n_threads, nullptr);
    if (plan.work_size + 64 > L->work.size()) L->work.resize(plan.work_size + 64);
    plan.work_data = L->work.data();
    if (ggml_graph_compute(L->gf, &plan) != GGML_STATUS_SUCCESS) return -1;
    if (out)     copy_2d(L->out, out, 4);
    if (xnext && L->xnext) copy_2d(L->xnext, xnext, 4);
    if (ids)     copy_2d(L->selected, ids, 4);
    if (weights) copy_2d(L->weights, weights, 4);
    if (logits)  copy_2d(L->logits, logits, 4);
    if (probs)   copy_2d(L->probs, probs, 4);
    if (gate)    copy_2d(L->gate, gate, 4);
    if (up)      copy_2d(L->up, up, 4);
    if (act)     copy_2d(L->act, act, 4);
    if (experts) copy_2d(L->experts, experts, 4);
    return 0;
}

// A stack of T = 1 layers (each created with rms_eps >= 0) on n_warmup +
// n_steps independent tokens xs[s] (the decode benchmark's inputs): each step
// runs x = xs[s] through every layer in order, x <- xnext.  Per timed step:
// the seconds it took (steady_clock around the whole stack), the last layer's
// output out[s] [H], every layer's ids[s][l] [k], and the top-k margin of every
// layer: the k-th largest probability minus the (k+1)-th, margin[s][l].
int qwref_stack_run(qwref_layer ** Ls, int n_layer, const float * xs, int n_warmup, int n_steps,
                    float * out, int32_t * ids, float * margin, double * step_s, int n_threads) {
    if (n_layer <= 0 || !Ls || !xs) return -2;
    const int64_t H = Ls[0]->H;
    std::vector<float> x((size_t) H), xn((size_t) H);
    for (int s = 0; s < n_warmup + n_steps; ++s) {
        const int ts = s - n_warmup;   // < 0: warm-up
        memcpy(x.data(), xs + (size_t) s * H, sizeof(float) * H);
        const auto t0 = std::chrono::steady_clock::now();
        for (int l = 0; l < n_layer; ++l) {
            qwref_layer * L = Ls[l];
            const bool last = l + 1 == n_layer;
            if (qwref_layer_eval(L, x.data(), last && ts >= 0 && out ? out + (size_t) ts * H : nullptr, xn.data(),
                                 nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                 n_threads) != 0)
                return -1;
            x.swap(xn);
        }
        const auto t1 = std::chrono::steady_clock::now();
        if (ts >= 0 && step_s) step_s[ts] = std::chrono::duration<double>(t1 - t0).count();
    }
    // ids and margins: a second, untimed pass (a layer graph keeps only its
    // last evaluation, and reading them inside the timed steps would add copies)
    if (ids || margin) {
        const int64_t E = Ls[0]->E, k = Ls[0]->K;
        std::vector<float> probs((size_t) E);
        for (int ts = 0; ts < n_steps; ++ts) {
            memcpy(x.data(), xs + (size_t) (n_warmup + ts) * H, sizeof(float) * H);
            for (int l = 0; l < n_layer; ++l) {
                qwref_layer * L = Ls[l];
                int32_t * id = ids ? ids + ((size_t) ts * n_layer + l) * k : nullptr;
                if (qwref_layer_eval(L, x.data(), nullptr, xn.data(), id, nullptr, nullptr, probs.data(), nullptr,
                                     nullptr, nullptr, nullptr, n_threads) != 0)
                    return -1;
                if (margin) {
                    std::vector<float> p(probs);
                    std::nth_element(p.begin(), p.begin() + k, p.end(), [](float a, float b) { return a > b; });
                    const float pk1 = p[(size_t) k];
                    const float pk = *std::min_element(p.begin(), p.begin() + k);
                    margin[(size_t) ts * n_layer + l] = pk - pk1;
                }
                x.swap(xn);
            }
        }
    }
    return 0;
}

// The shared-expert branch of build_moe (core/runtime.cpp:963-972) on the CPU
// backend, for T tokens, as the reference builds it: g = mul_mat(gate, x),
// u = mul_mat(up, x), sh = mul_mat(down, mul(silu(g), u)),
// sg = sigmoid(mul_mat(gate_inp, x)), out = add(moe_out, mul(sh, sg)), then
// add(out, resid) when resid is given.  Weights: gate / up [H, F], down [F, H]
// of their types, gate_inp f32 [H, 1]; x, moe_out, resid, out [H, T] dense.
int qwref_shared_expert_add(int64_t H, int64_t F, int64_t T, int type_gate, int type_up, int type_down,
                            const void * gate, const void * up, const void * down, const float * gate_inp,
                            const float * x, const float * moe_out, const float * resid, float * out,
                            int n_threads) {
    ensure_init();
    ggml_init_params wp = { ggml_tensor_overhead() * 8, nullptr, true };
    ggml_context * wctx = ggml_init(wp);
    ggml_tensor * Wg = ggml_new_tensor_2d(wctx, (ggml_type) type_gate, H, F);
    ggml_tensor * Wu = ggml_new_tensor_2d(wctx, (ggml_type) type_up, H, F);
    ggml_tensor * Wd = ggml_new_tensor_2d(wctx, (ggml_type) type_down, F, H);
    ggml_tensor * Wi = ggml_new_tensor_2d(wctx, GGML_TYPE_F32, H, 1);
    Wg->data = (void *) gate; Wu->data = (void *) up; Wd->data = (void *) down; Wi->data = (void *) gate_inp;
    const size_t bytes = sizeof(float) * (size_t) T * (size_t) (H * 8 + F * 6 + 8);
    ggml_init_params ip = { bytes + ggml_tensor_overhead() * 32 + ggml_graph_overhead() + (1 << 20), nullptr, false };
    ggml_context * ctx = ggml_init(ip);
    ggml_tensor * X = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, T);
    ggml_tensor * M = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, T);
    memcpy(X->data, x, sizeof(float) * H * T);
    memcpy(M->data, moe_out, sizeof(float) * H * T);
    ggml_tensor * g = ggml_mul_mat(ctx, Wg, X);
    ggml_tensor * u = ggml_mul_mat(ctx, Wu, X);
    ggml_tensor * sh = ggml_mul_mat(ctx, Wd, ggml_mul(ctx, ggml_silu(ctx, g), u));
    ggml_tensor * sg = ggml_sigmoid(ctx, ggml_mul_mat(ctx, Wi, X));
    sh = ggml_mul(ctx, sh, sg);
    ggml_tensor * O = ggml_add(ctx, M, sh);
    if (resid) {
        ggml_tensor * R = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, T);
        memcpy(R->data, resid, sizeof(float) * H * T);
        O = ggml_add(ctx, O, R);
    }
    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, O);
    ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    const int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    if (rc == 0) memcpy(out, O->data, sizeof(float) * H * T);
    ggml_free(ctx);
    ggml_free(wctx);
    return rc;
}

// The ISA branch this build of the ggml CPU backend takes (compile-time
// flags): 512 for AVX-512, 256 for AVX2, 0 otherwise.
int qwref_isa(void) {
    ensure_init();
    if (ggml_cpu_has_avx512()) return 512;
    if (ggml_cpu_has_avx2()) return 256;
    return 0;
}

// ggml_mul_mat_id alone on the CPU backend (ggml.c:3329-3356,
// ggml-cpu.c:1534-1707): as [K, N, n_as] of `type`, b f32 [K, b_ne1, T]
// (dense), ids i32 [n_ids, T] (dense) -> dst f32 [N, n_ids, T].
int qwref_mul_mat_id(int type, int64_t K, int64_t N, int64_t n_as, const void * as,
                     int64_t b_ne1, int64_t T, const float * b, int64_t n_ids,
                     const int32_t * ids, float * dst, int n_threads) {
    ensure_init();
    ggml_init_params wp = { ggml_tensor_overhead() * 4, nullptr, true };
    ggml_context * wctx = ggml_init(wp);
    ggml_tensor * A = ggml_new_tensor_3d(wctx, (ggml_type) type, K, N, n_as);
    A->data = (void *) as;
    size_t bytes = sizeof(float) * (size_t) (K * b_ne1 * T + N * n_ids * T) + sizeof(int32_t) * n_ids * T;
    ggml_init_params ip = { bytes + ggml_tensor_overhead() * 16 + ggml_graph_overhead() + (1 << 20), nullptr, false };
    ggml_context * ctx = ggml_init(ip);
    ggml_tensor * B = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, K, b_ne1, T);
    ggml_tensor * I = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, n_ids, T);
    memcpy(B->data, b, sizeof(float) * K * b_ne1 * T);
    memcpy(I->data, ids, sizeof(int32_t) * n_ids * T);
    ggml_tensor * C = ggml_mul_mat_id(ctx, A, B, I);
    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, C);
    ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    if (rc == 0) memcpy(dst, C->data, sizeof(float) * N * n_ids * T);
    ggml_free(ctx);
    ggml_free(wctx);
    return rc;
}

// Single-op helpers on the CPU backend, used to pin the oracle op by op.
// op: 0 soft_max rows [E, T]; 1 argsort DESC rows (i32 out); 2 rms_norm rows
// (param = eps); 3 swiglu_split(a = gate, b = up); 4 vec_dot_f32 via mul_mat
// of a [n, rows] by b [n, 1]; 5 mul(rms_norm(a, param), b [n]).
int qwref_unary(int op, const float * a, const float * b, int64_t ne0, int64_t ne1, float param,
                void * dst, int n_threads) {
    ensure_init();
    size_t bytes = sizeof(float) * (size_t) ne0 * ne1 * 4;
    ggml_init_params ip = { bytes + ggml_tensor_overhead() * 16 + ggml_graph_overhead() + (1 << 20), nullptr, false };
    ggml_context * ctx = ggml_init(ip);
    ggml_tensor * A = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, ne0, ne1);
    memcpy(A->data, a, sizeof(float) * ne0 * ne1);
    ggml_tensor * R = nullptr;
    switch (op) {
        case 0: R = ggml_soft_max(ctx, A); break;
        case 1: R = ggml_argsort(ctx, A, GGML_SORT_ORDER_DESC); break;
        case 2: R = ggml_rms_norm(ctx, A, param); break;
        case 3: {
            ggml_tensor * B = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, ne0, ne1);
            memcpy(B->data, b, sizeof(float) * ne0 * ne1);
            R = ggml_swiglu_split(ctx, A, B);
            break;
        }
        case 4: {
            ggml_tensor * B = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, ne0, 1);
            memcpy(B->data, b, sizeof(float) * ne0);
            R = ggml_mul_mat(ctx, A, B);   // [ne1, 1]
            break;
        }
        case 5: {   // the router input: mul(rms_norm(a, param), b) with b [ne0] broadcast over rows
            ggml_tensor * B = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, ne0);
            memcpy(B->data, b, sizeof(float) * ne0);
            R = ggml_mul(ctx, ggml_rms_norm(ctx, A, param), B);
            break;
        }
        default: ggml_free(ctx); return -2;
    }
    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, R);
    ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    if (rc == 0) memcpy(dst, R->data, ggml_nbytes(R));
    ggml_free(ctx);
    return rc;
}

} // extern "C"

extern "C" {

// ---------------------------------------------------------------------------
// Seg A's attention half for one non-recurrent, non-gated Qwen3 layer on the
// CPU backend, the op sequence of core/runtime.cpp:1976-2030 (build_segA)
// with build_attn's manual (non-flash) path, 681-734, and 1D NEOX RoPE
// (apply_rope, 290-300):
//   cur = rms_norm(h) * attn_norm; Q/K/V = mul_mat(W, cur), reshaped per head;
//   Q = rms_norm(Q) * q_norm, K = rms_norm(K) * k_norm; rope_ext NEOX at
//   positions n_past + i; K, V copied into the f16 caches at row n_past;
//   kq = mul_mat(cont(permute(Kc)), permute(Q)); soft_max_ext(kq, mask, 1/sqrt(D));
//   kqv = mul_mat(cont(transpose(Vc)) as [n_kv, D, n_head_kv], kq);
//   att = cont_2d(permute(kqv)); cur = mul_mat(Wo, att);
//   attn_resid = cur + h; ffn_in = rms_norm(attn_resid) * ffn_norm.
// The causal f16 mask is filled as set_attn_inputs does (2108-2116).
// h, attn_resid, ffn_in: [T, H]; k_cache / v_cache: f16 [n_ctx, n_head_kv * D],
// read and written in place (rows n_past .. n_past + T - 1); q_out / att_out
// ([T, n_head * D], the roped Q and the attention output) may be NULL.
int qwref_attn_seg(int64_t H, int64_t n_head, int64_t n_head_kv, int64_t D, int64_t n_rot, float freq_base,
                   float eps, int64_t T, int64_t n_past, int64_t n_ctx, const float * h, const float * attn_norm,
                   int tq, const void * wq, int tk, const void * wk, int tv, const void * wv, int to,
                   const void * wo, const float * q_norm, const float * k_norm, const float * ffn_norm,
                   uint16_t * k_cache, uint16_t * v_cache, float * attn_resid, float * ffn_in, float * q_out,
                   float * att_out, int n_threads) {
    ensure_init();
    if (n_past + T > n_ctx || n_head % n_head_kv) return -2;
    const int64_t n_kv = n_past + T, gqa = n_head_kv * D;
    const size_t cache_bytes = sizeof(uint16_t) * (size_t) (n_ctx * gqa);
    const size_t act = sizeof(float) * (size_t) T * (size_t) (16 * H + 16 * n_head * D + 8 * gqa)
                       + sizeof(float) * (size_t) (4 * n_head * T * n_kv + 2 * n_kv * gqa)
                       + 2 * cache_bytes + sizeof(uint16_t) * (size_t) (n_kv * T);
    const size_t wbytes = ggml_row_size((ggml_type) tq, H) * (size_t) (n_head * D) +
                          ggml_row_size((ggml_type) tk, H) * (size_t) gqa +
                          ggml_row_size((ggml_type) tv, H) * (size_t) gqa +
                          ggml_row_size((ggml_type) to, n_head * D) * (size_t) H + sizeof(float) * (size_t) (4 * H + 4 * D);
    ggml_init_params ip = { act + wbytes + ggml_tensor_overhead() * 128 + ggml_graph_overhead() + (4 << 20), nullptr,
                            false };
    ggml_context * ctx = ggml_init(ip);
    auto wt = [&](int type, int64_t ne0, int64_t ne1, const void * data) {
        ggml_tensor * t = ggml_new_tensor_2d(ctx, (ggml_type) type, ne0, ne1);
        memcpy(t->data, data, ggml_nbytes(t));
        return t;
    };
    auto vec = [&](const float * v, int64_t n) { return wt(GGML_TYPE_F32, n, 1, v); };
    ggml_tensor * Wq = wt(tq, H, n_head * D, wq), * Wk = wt(tk, H, gqa, wk), * Wv = wt(tv, H, gqa, wv);
    ggml_tensor * Wo = wt(to, n_head * D, H, wo);
    ggml_tensor * An = ggml_reshape_1d(ctx, vec(attn_norm, H), H), * Fn = ggml_reshape_1d(ctx, vec(ffn_norm, H), H);
    ggml_tensor * Qn = ggml_reshape_1d(ctx, vec(q_norm, D), D), * Kn = ggml_reshape_1d(ctx, vec(k_norm, D), D);
    ggml_tensor * KC = wt(GGML_TYPE_F16, gqa, n_ctx, k_cache), * VC = wt(GGML_TYPE_F16, gqa, n_ctx, v_cache);
    ggml_tensor * X = wt(GGML_TYPE_F32, H, T, h);
    ggml_tensor * pos = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, T);
    for (int64_t i = 0; i < T; ++i) ((int32_t *) pos->data)[i] = (int32_t) (n_past + i);
    ggml_tensor * mask = ggml_new_tensor_2d(ctx, GGML_TYPE_F16, n_kv, T);
    const ggml_fp16_t z = ggml_fp32_to_fp16(0.0f), ninf = ggml_fp32_to_fp16(-INFINITY);
    for (int64_t i = 0; i < T; ++i)
        for (int64_t j = 0; j < n_kv; ++j) ((ggml_fp16_t *) mask->data)[i * n_kv + j] = j <= n_past + i ? z : ninf;

    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_tensor * cur = ggml_mul(ctx, ggml_rms_norm(ctx, X, eps), An);
    ggml_tensor * Q = ggml_reshape_3d(ctx, ggml_mul_mat(ctx, Wq, cur), D, n_head, T);
    ggml_tensor * K = ggml_reshape_3d(ctx, ggml_mul_mat(ctx, Wk, cur), D, n_head_kv, T);
    ggml_tensor * V = ggml_reshape_3d(ctx, ggml_mul_mat(ctx, Wv, cur), D, n_head_kv, T);
    Q = ggml_mul(ctx, ggml_rms_norm(ctx, Q, eps), Qn);
    K = ggml_mul(ctx, ggml_rms_norm(ctx, K, eps), Kn);
    Q = ggml_rope_ext(ctx, Q, pos, nullptr, (int) n_rot, GGML_ROPE_TYPE_NEOX, 0, freq_base, 1.0f, 0.0f, 1.0f, 0.0f,
                      0.0f);
    K = ggml_rope_ext(ctx, K, pos, nullptr, (int) n_rot, GGML_ROPE_TYPE_NEOX, 0, freq_base, 1.0f, 0.0f, 1.0f, 0.0f,
                      0.0f);
    ggml_tensor * k_dst = ggml_view_2d(ctx, KC, gqa, T, KC->nb[1], (size_t) n_past * KC->nb[1]);
    ggml_build_forward_expand(gf, ggml_cpy(ctx, ggml_reshape_2d(ctx, K, gqa, T), k_dst));
    ggml_tensor * v_dst = ggml_view_2d(ctx, VC, gqa, T, VC->nb[1], (size_t) n_past * VC->nb[1]);
    ggml_build_forward_expand(gf, ggml_cpy(ctx, ggml_reshape_2d(ctx, V, gqa, T), v_dst));
    ggml_tensor * Kc = ggml_view_2d(ctx, KC, gqa, n_kv, KC->nb[1], 0);
    Kc = ggml_permute(ctx, ggml_reshape_3d(ctx, Kc, D, n_head_kv, n_kv), 0, 2, 1, 3);
    ggml_tensor * Qp = ggml_permute(ctx, Q, 0, 2, 1, 3);
    ggml_tensor * kq = ggml_mul_mat(ctx, ggml_cont(ctx, Kc), Qp);
    kq = ggml_soft_max_ext(ctx, kq, mask, 1.0f / sqrtf((float) D), 0.0f);
    ggml_tensor * Vslice = ggml_view_2d(ctx, VC, gqa, n_kv, VC->nb[1], 0);
    ggml_tensor * Vm = ggml_reshape_3d(ctx, ggml_cont(ctx, ggml_transpose(ctx, Vslice)), n_kv, D, n_head_kv);
    ggml_tensor * kqv = ggml_mul_mat(ctx, Vm, kq);
    ggml_tensor * att = ggml_cont_2d(ctx, ggml_permute(ctx, kqv, 0, 2, 1, 3), n_head * D, T);
    ggml_tensor * resid = ggml_add(ctx, ggml_mul_mat(ctx, Wo, att), X);
    ggml_tensor * fin = ggml_mul(ctx, ggml_rms_norm(ctx, resid, eps), Fn);
    ggml_tensor * qc = ggml_cont(ctx, Q);
    ggml_build_forward_expand(gf, qc);
    ggml_build_forward_expand(gf, fin);

    ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    const int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    if (rc == 0) {
        if (attn_resid) copy_2d(resid, attn_resid, 4);
        if (ffn_in) copy_2d(fin, ffn_in, 4);
        if (q_out) copy_2d(qc, q_out, 4);
        if (att_out) copy_2d(att, att_out, 4);
        memcpy(k_cache, KC->data, cache_bytes);
        memcpy(v_cache, VC->data, cache_bytes);
    }
    ggml_free(ctx);
    return rc;
}

}  // extern "C" (attention)

extern "C" {

// ---------------------------------------------------------------------------
// Seg A's recurrent half (a gated-delta-net layer of qwen3next / qwen35moe) on
// the CPU backend, the op sequence of core/runtime.cpp:1976-1995 (build_segA)
// with build_gdn, 737-859, in its one-pass (non-verify) form:
//   cur = rms_norm(h) * attn_norm;
//   qkv = mul_mat(attn_qkv, cur) [conv_ch]; z = mul_mat(attn_gate, cur) [d_inner];
//   beta = sigmoid(mul_mat(ssm_beta, cur)); g = softplus(mul_mat(ssm_alpha, cur) + dt_bias) * ssm_a;
//   conv_input = concat(conv_state, transpose(qkv)); conv_state <- its last d_conv - 1 steps;
//   conv = silu(ssm_conv(conv_input, conv1d)); q, k, v = views of conv (H_k, H_k, H_v heads of S);
//   q, k = l2_norm(.., eps); (out, state) = gated_delta_net(q, k, v, g, beta, ssm_state, 1);
//   out = rms_norm(out) * ssm_norm * silu(z) per head; cur = mul_mat(ssm_out, out);
//   attn_resid = cur + h; ffn_in = rms_norm(attn_resid) * ffn_norm.
// h, attn_resid, ffn_in: [T, H]; conv_state f32 [conv_ch][d_conv - 1] and ssm_state
// f32 [H_v][S][S] (ggml's layouts) are read and written in place; gdn_out
// ([T, H_v * S], the gated norm's output) may be NULL.
int qwref_gdn_seg(int64_t H, int64_t S, int64_t H_k, int64_t H_v, int64_t d_conv, float eps, int64_t T,
                  const float * h, const float * attn_norm, int t_qkv, const void * w_qkv, int t_gate,
                  const void * w_gate, int t_beta, const void * w_beta, int t_alpha, const void * w_alpha,
                  const float * dt_bias, const float * ssm_a, const float * conv1d, const float * ssm_norm,
                  int t_out, const void * w_out, const float * ffn_norm, float * conv_state, float * ssm_state,
                  float * attn_resid, float * ffn_in, float * gdn_out, int n_threads) {
    ensure_init();
    if (H_v % H_k || d_conv < 2) return -2;
    const int64_t d_inner = H_v * S, key_dim = H_k * S, conv_ch = d_inner + 2 * key_dim;
    const size_t el = sizeof(float);
    const size_t wbytes = ggml_row_size((ggml_type) t_qkv, H) * (size_t) conv_ch +
                          ggml_row_size((ggml_type) t_gate, H) * (size_t) d_inner +
                          ggml_row_size((ggml_type) t_beta, H) * (size_t) H_v +
                          ggml_row_size((ggml_type) t_alpha, H) * (size_t) H_v +
                          ggml_row_size((ggml_type) t_out, d_inner) * (size_t) H;
    const size_t act = el * (size_t) T * (size_t) (12 * H + 8 * conv_ch + 12 * d_inner + 8 * H_v) +
                       el * (size_t) (4 * conv_ch * (d_conv + T) + 3 * S * S * H_v + 4 * H + 2 * S + 4 * H_v) +
                       el * (size_t) (S * H_v * T + S * S * H_v);
    ggml_init_params ip = { act + wbytes + ggml_tensor_overhead() * 160 + ggml_graph_overhead() + (4 << 20), nullptr,
                            false };
    ggml_context * ctx = ggml_init(ip);
    auto wt = [&](int type, int64_t ne0, int64_t ne1, const void * data) {
        ggml_tensor * t = ggml_new_tensor_2d(ctx, (ggml_type) type, ne0, ne1);
        memcpy(t->data, data, ggml_nbytes(t));
        return t;
    };
    auto vec = [&](const float * v, int64_t n) { return ggml_reshape_1d(ctx, wt(GGML_TYPE_F32, n, 1, v), n); };
    ggml_tensor * Wqkv = wt(t_qkv, H, conv_ch, w_qkv), * Wgate = wt(t_gate, H, d_inner, w_gate);
    ggml_tensor * Wbeta = wt(t_beta, H, H_v, w_beta), * Walpha = wt(t_alpha, H, H_v, w_alpha);
    ggml_tensor * Wout = wt(t_out, d_inner, H, w_out);
    ggml_tensor * An = vec(attn_norm, H), * Fn = vec(ffn_norm, H), * Sn = vec(ssm_norm, S);
    ggml_tensor * DTb = vec(dt_bias, H_v), * Aa = vec(ssm_a, H_v);
    ggml_tensor * CK = wt(GGML_TYPE_F32, d_conv, conv_ch, conv1d);
    ggml_tensor * CS = wt(GGML_TYPE_F32, d_conv - 1, conv_ch, conv_state);
    ggml_tensor * SS = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, S, S, H_v);
    memcpy(SS->data, ssm_state, ggml_nbytes(SS));
    ggml_tensor * X = wt(GGML_TYPE_F32, H, T, h);

    ggml_cgraph * gf = ggml_new_graph(ctx);
    ggml_tensor * cur = ggml_mul(ctx, ggml_rms_norm(ctx, X, eps), An);
    ggml_tensor * qkv = ggml_mul_mat(ctx, Wqkv, cur);                                  // [conv_ch, T]
    ggml_tensor * z = ggml_mul_mat(ctx, Wgate, cur);                                   // [d_inner, T]
    ggml_tensor * beta = ggml_sigmoid(ctx, ggml_mul_mat(ctx, Wbeta, cur));
    beta = ggml_reshape_4d(ctx, beta, 1, H_v, T, 1);
    ggml_tensor * alpha = ggml_softplus(ctx, ggml_add(ctx, ggml_mul_mat(ctx, Walpha, cur), DTb));
    ggml_tensor * g = ggml_reshape_4d(ctx, ggml_mul(ctx, alpha, Aa), 1, H_v, T, 1);
    ggml_tensor * cs = ggml_reshape_3d(ctx, CS, d_conv - 1, conv_ch, 1);
    ggml_tensor * conv_input = ggml_concat(ctx, cs, ggml_transpose(ctx, qkv), 0);   // [d_conv - 1 + T, conv_ch, 1]
    ggml_tensor * cs_last = ggml_view_3d(ctx, conv_input, d_conv - 1, conv_ch, 1, conv_input->nb[1],
                                         conv_input->nb[2], ggml_row_size(conv_input->type, T));
    ggml_build_forward_expand(gf, ggml_cpy(ctx, cs_last, CS));
    ggml_tensor * conv = ggml_silu(ctx, ggml_ssm_conv(ctx, conv_input, CK));          // [conv_ch, T, 1]
    const size_t nb1q = ggml_row_size(conv->type, conv_ch);
    ggml_tensor * q = ggml_view_4d(ctx, conv, S, H_k, T, 1, el * S, nb1q, nb1q * T, 0);
    ggml_tensor * k = ggml_view_4d(ctx, conv, S, H_k, T, 1, el * S, nb1q, nb1q * T, el * key_dim);
    ggml_tensor * v = ggml_view_4d(ctx, conv, S, H_v, T, 1, el * S, nb1q, nb1q * T, el * 2 * key_dim);
    q = ggml_cont(ctx, ggml_l2_norm(ctx, q, eps));
    k = ggml_cont(ctx, ggml_l2_norm(ctx, k, eps));
    v = ggml_cont(ctx, v);
    ggml_tensor * s_in = ggml_reshape_4d(ctx, SS, S, S, H_v, 1);
    ggml_tensor * res = ggml_gated_delta_net(ctx, q, k, v, g, beta, s_in, 1);
    ggml_tensor * out = ggml_view_4d(ctx, res, S, H_v, T, 1, el * S, el * S * H_v, el * S * H_v * T, 0);
    ggml_tensor * st = ggml_view_4d(ctx, res, S, S, H_v, 1, el * S, el * S * S, el * S * S * H_v, el * S * H_v * T);
    ggml_build_forward_expand(gf, ggml_cpy(ctx, st, ggml_reshape_3d(ctx, SS, S, S, H_v)));
    out = ggml_mul(ctx, ggml_rms_norm(ctx, ggml_cont(ctx, out), eps), Sn);
    out = ggml_mul(ctx, out, ggml_silu(ctx, ggml_reshape_4d(ctx, z, S, H_v, T, 1)));
    out = ggml_reshape_2d(ctx, out, S * H_v, T);
    ggml_tensor * resid = ggml_add(ctx, ggml_mul_mat(ctx, Wout, out), X);
    ggml_tensor * fin = ggml_mul(ctx, ggml_rms_norm(ctx, resid, eps), Fn);
    ggml_build_forward_expand(gf, out);
    ggml_build_forward_expand(gf, fin);

    ggml_cplan plan = ggml_graph_plan(gf, n_threads, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    const int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -1;
    if (rc == 0) {
        if (attn_resid) copy_2d(resid, attn_resid, 4);
        if (ffn_in) copy_2d(fin, ffn_in, 4);
        if (gdn_out) copy_2d(out, gdn_out, 4);
        memcpy(conv_state, CS->data, ggml_nbytes(CS));
        memcpy(ssm_state, SS->data, ggml_nbytes(SS));
    }
    ggml_free(ctx);
    return rc;
}

}  // extern "C" (gated delta net)
