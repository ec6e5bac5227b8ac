// glue_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Runs one GGML_OP_MUL_MAT_ID node of a real ggml graph both ways: on ggml's
// CPU backend (oracle/_ref/libqwref.so, built from the reference sources), and
// through include/qwmoe_ggml.h -- the glue a ggml backend adds -- with the
// node's own tensors (their ne / nb fields untouched) copied to device memory.
// The graph is build_moe's: logits -> soft_max -> argsort_top_k (a strided
// [k, T] view with nb[1] = n_as * 4) -> mul_mat_id over [K, N, n_as] experts
// (core/runtime.cpp:869-938).  Built by oracle/Makefile.ref into
// oracle/_ref/libqwglue.so; loaded only by tests/.

#include "ggml.h"
#include "ggml-cpu.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <vector>

#include "qwmoe_ggml.h"

namespace {

// A device copy of tensor t (its byte extent from t->data) with the same ne / nb.
struct DevTensor {
    ggml_tensor t{};
    void* mem = nullptr;
    size_t bytes = 0;
    int make(const ggml_tensor* src) {
        t = *src;
        bytes = ggml_nbytes(src);
        if (hipMalloc(&mem, bytes) != hipSuccess) return -1;
        if (hipMemcpy(mem, src->data, bytes, hipMemcpyHostToDevice) != hipSuccess) return -1;
        t.data = mem;
        return 0;
    }
    ~DevTensor() {
        if (mem) (void) hipFree(mem);
    }
};

}  // namespace

extern "C" {

// weights_f32 [n_as][N][K] (quantized here to `type` by ggml_quantize_chunk),
// b [T][ne11][K], scores [T][n_as] (routing logits; the top k per token after a
// softmax pick the experts).  Outputs: ids [T][k] (the graph's selection),
// cpu_out / gpu_out [T][k][N] (dst of ggml's mul_mat_id and of the glue),
// status (the glue's return code).  Returns 0, or < 0 when a step failed.
int qwglue_mul_mat_id(int type, int64_t K, int64_t N, int64_t n_as, int64_t ne11, int64_t T, int64_t k,
                      const float* weights_f32, const float* b, const float* scores, int32_t* ids, float* cpu_out,
                      float* gpu_out, int* status) {
    ggml_cpu_init();
    const size_t wbytes = ggml_row_size((ggml_type) type, K) * (size_t) (N * n_as);
    ggml_init_params ip = {wbytes + sizeof(float) * (size_t) (T * (ne11 * K + 4 * n_as + k * N + k)) +
                               ggml_tensor_overhead() * 32 + ggml_graph_overhead() + (1 << 20),
                           nullptr, false};
    ggml_context* ctx = ggml_init(ip);
    if (!ctx) return -1;
    ggml_tensor* as = ggml_new_tensor_3d(ctx, (ggml_type) type, K, N, n_as);
    ggml_quantize_chunk((ggml_type) type, weights_f32, as->data, 0, N * n_as, K, nullptr);
    ggml_tensor* bt = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, K, ne11, T);
    memcpy(bt->data, b, sizeof(float) * (size_t) (K * ne11 * T));
    ggml_tensor* sc = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, n_as, T);
    memcpy(sc->data, scores, sizeof(float) * (size_t) (n_as * T));
    ggml_tensor* probs = ggml_soft_max(ctx, sc);
    ggml_tensor* sel = ggml_argsort_top_k(ctx, probs, (int) k);   // [k, T], nb[1] = n_as * 4
    ggml_tensor* node = ggml_mul_mat_id(ctx, as, bt, sel);        // [N, k, T]
    ggml_cgraph* gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, node);
    ggml_cplan plan = ggml_graph_plan(gf, 4, nullptr);
    std::vector<uint8_t> work(plan.work_size + 64);
    plan.work_data = work.data();
    int rc = ggml_graph_compute(gf, &plan) == GGML_STATUS_SUCCESS ? 0 : -2;
    if (rc == 0 && !qwmoe_ggml_supports_mul_mat_id(node)) rc = -3;
    if (rc == 0) {
        for (int64_t t = 0; t < T; ++t)
            memcpy(ids + t * k, (const char*) sel->data + t * sel->nb[1], sizeof(int32_t) * (size_t) k);
        for (int64_t t = 0; t < T; ++t)
            for (int64_t i = 0; i < k; ++i)
                memcpy(cpu_out + (t * k + i) * N, (const char*) node->data + t * node->nb[2] + i * node->nb[1],
                       sizeof(float) * (size_t) N);
        // the node with its sources and destination in device memory
        DevTensor das, db, dids, ddst;
        if (das.make(as) || db.make(bt) || dids.make(sel) || ddst.make(node)) {
            rc = -4;
        } else {
            ggml_tensor nd = *node;
            nd.src[0] = &das.t;
            nd.src[1] = &db.t;
            nd.src[2] = &dids.t;
            nd.data = ddst.mem;
            (void) hipMemset(ddst.mem, 0xff, ddst.bytes);   // NaN: every output must be written
            *status = qwmoe_ggml_mul_mat_id(nullptr, &nd, nullptr, 0);
            std::vector<uint8_t> back(ddst.bytes);
            if (hipDeviceSynchronize() != hipSuccess ||
                hipMemcpy(back.data(), ddst.mem, ddst.bytes, hipMemcpyDeviceToHost) != hipSuccess) {
                rc = -5;
            } else {
                for (int64_t t = 0; t < T; ++t)
                    for (int64_t i = 0; i < k; ++i)
                        memcpy(gpu_out + (t * k + i) * N, back.data() + t * node->nb[2] + i * node->nb[1],
                               sizeof(float) * (size_t) N);
            }
        }
    }
    ggml_free(ctx);
    return rc;
}

}  // extern "C"
