// layer_stack.cpp -- a batch of T tokens through a stack of MoE FFN layers:
// the FFN half of the verify forward of speculative decoding, where
// Runtime::decode_verify runs the main model on the T = n_draft + 1 tokens of a
// draft at once (core/runtime.cpp:1495-1562, driven by generate_mtp,
// 1628-1762), and every layer's build_moe sees a T-token batch
// (core/runtime.cpp:861-974: T > 1 takes the mul + add-chain weighted sum).
//
// Each layer is qwmoe_ffn_layer on the batch (router, grouping, gate/up/down
// mul_mat_id, SwiGLU, weighted sum, RMSNorm into the next layer's input).  The
// per-layer kernels are latency-bound at these T, so the whole chain for one T
// is captured once into a HIP graph (on a private stream: capturing launches
// nothing) and replayed on the caller's stream, as the reference keeps a
// persistent verify graph (1503-1525).  The graph reads and writes only buffers
// the stack owns; the caller's input and outputs are copied in and out around it.
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include <cstdlib>

#include "../../include/qwmoe.h"
#include "qw_kernels.hpp"
#include "qw_verify.hpp"

struct qwmoe_layer_stack {
    std::vector<qwmoe_layer> layers;
    float rms_eps = 1e-6f;
    int max_T = 0;
    int64_t H = 0, k = 0;
    bool graphs = true;
    uint8_t* blk = nullptr;
    float* xb[2] = {nullptr, nullptr};   // [max_T][H] ping-pong layer inputs
    float* ob = nullptr;                 // [max_T][H] layer outputs
    int32_t* ids = nullptr;              // [n_layer][max_T][k]
    float* w = nullptr;                  // [n_layer][max_T][k]
    hipStream_t cap = nullptr;           // capture stream
    std::vector<hipGraphExec_t> exec;    // [T]: the captured chain, or null
    std::vector<uint64_t> exec_gen;      // [T]: the library generation it was captured with
    int64_t captures = 0;                // graphs captured so far (a diagnostic)
    // The persistent verify kernel (verify_xcd.hip) for 2 <= T <= VERIFY_TMAX, where
    // the shape and device allow it: one launch for all layers.
    const void* vfn = nullptr;
    qw::VerifyArgs va{};                 // its arguments but the per-run ones
    uint8_t* vblk = nullptr;             // layer table | exchange words | status, abort
    uint32_t vepoch = 1;                 // next launch's first layer epoch
    // T = 1: the whole-stack decode kernel (qwmoe_decode_stack_*), one launch per
    // token, where it takes this stack's layers; the same bits as the chain.
    // Created at the first T = 1 run outside stream capture (ds_tried).
    qwmoe_decode_stack* ds = nullptr;
    bool ds_allowed = true, ds_tried = false;

    ~qwmoe_layer_stack() {
        if (ds) qwmoe_decode_stack_free(ds);
        for (hipGraphExec_t e : exec)
            if (e) (void) hipGraphExecDestroy(e);
        if (cap) (void) hipStreamDestroy(cap);
        if (blk) (void) hipFree(blk);
        if (vblk) (void) hipFree(vblk);
    }

    // Sets up the persistent verify kernel when every layer has the shape it
    // takes (H = 2048, F = 768, E of 32, 64 or 128, k <= 8, Q4_K gate/up/down with
    // 16-byte aligned rows, no resident mask, one expert_weights_scale) and the
    // device has 256 CUs; QWMOE_VERIFY_XCD=0 in the environment turns it off.
    // Leaves vfn null otherwise (the per-layer path serves every T).
    int setup_verify() {
        const char* env = getenv("QWMOE_VERIFY_XCD");
        if (env && env[0] == '0') return QWMOE_OK;
        const qwmoe_layer& L0 = layers[0];
        for (const qwmoe_layer& L : layers) {
            if (L.n_embd != L0.n_embd || L.n_ff != L0.n_ff || L.n_expert != L0.n_expert ||
                L.n_expert_used != L0.n_expert_used || L.expert_weights_scale != L0.expert_weights_scale)
                return QWMOE_OK;
            if (L.type_gate != qw::T_Q4_K || L.type_up != qw::T_Q4_K || L.type_down != qw::T_Q4_K) return QWMOE_OK;
            if (!L.router || !L.gate || !L.up || !L.down || L.resmask) return QWMOE_OK;
            const uintptr_t al = (uintptr_t) L.gate | (uintptr_t) L.up | (uintptr_t) L.down | (uintptr_t) L.router |
                                 (uintptr_t) L.gate_nb1 | (uintptr_t) L.gate_nb2 | (uintptr_t) L.up_nb1 |
                                 (uintptr_t) L.up_nb2 | (uintptr_t) L.down_nb1 | (uintptr_t) L.down_nb2;
            if (al & 15) return QWMOE_OK;
            if (L.n_slots_gate <= 0 || L.n_slots_up <= 0 || L.n_slots_down <= 0) return QWMOE_OK;
        }
        if (L0.n_expert_used > 8 || max_T < 2) return QWMOE_OK;
        const void* fn = qw::verify_xcd_kernel(L0.n_embd, L0.n_ff, L0.n_expert);
        if (!fn) return QWMOE_OK;
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return QWMOE_ERR_HIP;
        if (cus != 256 || qw::verify_xcd_occupancy(fn) != 0) return QWMOE_OK;
        const int n = (int) layers.size();
        auto a256 = [](size_t v) { return (v + 255) & ~(size_t) 255; };
        const size_t o_xl = a256(sizeof(qw::DecodeLayer) * (size_t) n);
        const size_t o_xa = o_xl + a256(8 * qw::verify_words_xl(L0.n_expert));
        const size_t o_xd = o_xa + a256(8 * qw::verify_words_xa(L0.n_ff));
        const size_t o_xy = o_xd + a256(8 * qw::verify_words_xd(L0.n_embd));
        const size_t o_st = o_xy + a256(8 * qw::verify_words_xy(L0.n_embd));
        const size_t total = o_st + 256;
        if (hipMalloc(&vblk, total) != hipSuccess) {
            vblk = nullptr;
            (void) hipGetLastError();
            return QWMOE_ERR_HIP;
        }
        std::vector<qw::DecodeLayer> host((size_t) n);
        for (int l = 0; l < n; ++l) {
            const qwmoe_layer& L = layers[(size_t) l];
            qw::DecodeLayer& D = host[(size_t) l];
            D = qw::DecodeLayer{};
            D.router = L.router;
            D.gate = (const uint8_t*) L.gate;
            D.up = (const uint8_t*) L.up;
            D.down = (const uint8_t*) L.down;
            D.gate_nb1 = L.gate_nb1;
            D.gate_nb2 = L.gate_nb2;
            D.up_nb1 = L.up_nb1;
            D.up_nb2 = L.up_nb2;
            D.down_nb1 = L.down_nb1;
            D.down_nb2 = L.down_nb2;
            D.slot_gate = L.slot_gate;
            D.slot_up = L.slot_up;
            D.slot_down = L.slot_down;
            D.n_slots_gate = L.n_slots_gate;
            D.n_slots_up = L.n_slots_up;
            D.n_slots_down = L.n_slots_down;
        }
        if (hipMemset(vblk, 0, total) != hipSuccess ||
            hipMemcpy(vblk, host.data(), sizeof(qw::DecodeLayer) * (size_t) n, hipMemcpyHostToDevice) != hipSuccess)
            return QWMOE_ERR_HIP;
        // XCD-local words with workgroup scope only where the launch's workgroups
        // are dealt to the XCDs round robin (the probe writes into the down words)
        int ok = 0;
        if (qw::probe_xcd_mapping((int32_t*) (vblk + o_xd), 256, nullptr, &ok) != 0) return QWMOE_ERR_HIP;
        if (hipMemset(vblk + o_xd, 0, 256 * sizeof(int32_t)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
            return QWMOE_ERR_HIP;
        const char* le = getenv("QWMOE_DECODE_XCD_LOCAL");
        va = qw::VerifyArgs{};
        va.layers = (const qw::DecodeLayer*) vblk;
        va.n_layer = n;
        va.k = (int) L0.n_expert_used;
        va.scale = L0.expert_weights_scale;
        va.rms_eps = rms_eps;
        va.xl = (uint64_t*) (vblk + o_xl);
        va.xa = (uint64_t*) (vblk + o_xa);
        va.xd = (uint64_t*) (vblk + o_xd);
        va.xy = (uint64_t*) (vblk + o_xy);
        va.status = (int32_t*) (vblk + o_st);
        va.abort_flag = (int32_t*) (vblk + o_st + 128);
        va.local_st = (ok && !(le && le[0] == '0')) ? 1 : 0;
        vfn = fn;
        return QWMOE_OK;
    }

    // The chain for T tokens on stream st (eager, or recorded while capturing).
    int enqueue(hipStream_t st, int64_t T) {
        const int n = (int) layers.size();
        for (int l = 0; l < n; ++l) {
            const int rc = qwmoe_ffn_layer(st, &layers[(size_t) l], xb[l & 1], T, ob, rms_eps, xb[(l + 1) & 1],
                                           ids + (size_t) l * max_T * k, w + (size_t) l * max_T * k);
            if (rc != QWMOE_OK) return rc;
        }
        return QWMOE_OK;
    }

    int capture(int64_t T) {
        const uint64_t gen = qw::workspace_generation();
        if (!cap && hipStreamCreateWithFlags(&cap, hipStreamNonBlocking) != hipSuccess) return QWMOE_ERR_HIP;
        if (hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal) != hipSuccess) return QWMOE_ERR_HIP;
        const int rc = enqueue(cap, T);
        hipGraph_t g = nullptr;
        const hipError_t ec = hipStreamEndCapture(cap, &g);
        if (rc != QWMOE_OK || ec != hipSuccess || !g) {
            if (g) (void) hipGraphDestroy(g);
            (void) hipGetLastError();
            return rc != QWMOE_OK ? rc : QWMOE_ERR_HIP;
        }
        hipGraphExec_t e = nullptr;
        const hipError_t ei = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
        (void) hipGraphDestroy(g);
        if (ei != hipSuccess) return QWMOE_ERR_HIP;
        exec[(size_t) T] = e;
        exec_gen[(size_t) T] = gen;
        ++captures;
        return QWMOE_OK;
    }
};

extern "C" {

int qwmoe_layer_stack_create(const qwmoe_layer* layers, int n_layer, float rms_eps, int max_tokens, int flags,
                             qwmoe_layer_stack** out) {
    if (!out) return QWMOE_ERR_INVALID_ARG;
    *out = nullptr;
    if (!layers || n_layer <= 0 || max_tokens <= 0 || max_tokens > 64 || !(rms_eps >= 0.0f))
        return QWMOE_ERR_INVALID_ARG;
    const qwmoe_layer& L0 = layers[0];
    for (int l = 1; l < n_layer; ++l)
        if (layers[l].n_embd != L0.n_embd || layers[l].n_expert_used != L0.n_expert_used)
            return QWMOE_ERR_INVALID_ARG;
    if (L0.n_embd <= 0 || L0.n_expert_used <= 0) return QWMOE_ERR_INVALID_ARG;
    auto* s = new (std::nothrow) qwmoe_layer_stack();
    if (!s) return QWMOE_ERR_WORKSPACE;
    s->layers.assign(layers, layers + n_layer);
    s->rms_eps = rms_eps;
    s->max_T = max_tokens;
    s->H = L0.n_embd;
    s->k = L0.n_expert_used;
    s->graphs = (flags & QWMOE_STACK_NO_GRAPH) == 0;
    s->exec.assign((size_t) max_tokens + 1, nullptr);
    s->exec_gen.assign((size_t) max_tokens + 1, 0);
    auto a256 = [](size_t n) { return (n + 255) & ~(size_t) 255; };
    const size_t xs = a256((size_t) max_tokens * (size_t) s->H * 4);
    const size_t is = a256((size_t) n_layer * (size_t) max_tokens * (size_t) s->k * 4);
    if (hipMalloc(&s->blk, 3 * xs + 2 * is) != hipSuccess) {
        s->blk = nullptr;
        (void) hipGetLastError();
        delete s;
        return QWMOE_ERR_HIP;
    }
    s->xb[0] = (float*) s->blk;
    s->xb[1] = (float*) (s->blk + xs);
    s->ob = (float*) (s->blk + 2 * xs);
    s->ids = (int32_t*) (s->blk + 3 * xs);
    s->w = (float*) (s->blk + 3 * xs + is);
    const int rc = s->setup_verify();
    if (rc != QWMOE_OK) {
        delete s;
        return rc;
    }
    // runs at T = 1 go to the decode stack where it takes these layers, created at
    // the first such run; QWMOE_VERIFY_XCD=0 keeps the chain for every T
    const char* env = getenv("QWMOE_VERIFY_XCD");
    s->ds_allowed = !(env && env[0] == '0');
    *out = s;
    return QWMOE_OK;
}

int qwmoe_layer_stack_run(void* stream, qwmoe_layer_stack* s, const float* x, int64_t T, float* out, float* x_out,
                          int32_t* ids_out, float* weights_out) {
    if (!s || !x || !out || T <= 0 || T > s->max_T) return QWMOE_ERR_INVALID_ARG;
    if ((ids_out == nullptr) != (weights_out == nullptr)) return QWMOE_ERR_INVALID_ARG;
    hipStream_t st = (hipStream_t) stream;
    // Under stream capture the persistent kernels cannot run (each launch takes a
    // fresh exchange epoch from the host, which a replayed graph would repeat), and
    // nothing may be allocated: the caller's capture records the per-layer chain.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return QWMOE_ERR_HIP;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (T == 1 && !capturing && s->ds_allowed && !s->ds_tried) {
        s->ds_tried = true;
        if (qwmoe_decode_stack_create(s->layers.data(), (int) s->layers.size(), s->rms_eps, &s->ds) != QWMOE_OK) {
            s->ds = nullptr;
            (void) hipGetLastError();
        }
    }
    if (T == 1 && s->ds && !capturing) return qwmoe_decode_stack_run(stream, s->ds, x, out, x_out, ids_out, weights_out);
    const size_t xbytes = (size_t) T * (size_t) s->H * 4;
    const int n = (int) s->layers.size();
    if (s->vfn && T >= 2 && T <= qw::VERIFY_TMAX && !capturing) {
        // the persistent kernel: the caller's buffers directly, one launch
        if (s->vepoch > 0x7fffffffu - (uint32_t) n) return QWMOE_ERR_UNSUPPORTED;   // epoch space exhausted
        qw::VerifyArgs a = s->va;
        a.T = (int) T;
        a.x_in = x;
        a.out = out;
        a.x_out = x_out;
        a.ids_out = ids_out;
        a.w_out = weights_out;
        a.epoch0 = s->vepoch;
        s->vepoch += (uint32_t) n;
        return qw::launch_verify_xcd(s->vfn, a, st) == 0 ? QWMOE_OK : QWMOE_ERR_HIP;
    }
    if (hipMemcpyAsync(s->xb[0], x, xbytes, hipMemcpyDeviceToDevice, st) != hipSuccess) return QWMOE_ERR_HIP;
    int rc;
    if (capturing) {
        if ((rc = s->enqueue(st, T)) != QWMOE_OK) return rc;
    } else if (s->graphs) {
        // a graph holds the workspace addresses and the kernel choices of its capture: capture again
        // after qwmoe_init reallocated the workspace or qwmoe_set_mfma_min_rows changed the threshold
        if (s->exec[(size_t) T] && s->exec_gen[(size_t) T] != qw::workspace_generation()) {
            if (hipStreamSynchronize(st) != hipSuccess) return QWMOE_ERR_HIP;   // its last replay has finished
            (void) hipGraphExecDestroy(s->exec[(size_t) T]);
            s->exec[(size_t) T] = nullptr;
        }
        if (!s->exec[(size_t) T] && (rc = s->capture(T)) != QWMOE_OK) return rc;
        if (hipGraphLaunch(s->exec[(size_t) T], st) != hipSuccess) return QWMOE_ERR_HIP;
    } else if ((rc = s->enqueue(st, T)) != QWMOE_OK) {
        return rc;
    }
    if (hipMemcpyAsync(out, s->ob, xbytes, hipMemcpyDeviceToDevice, st) != hipSuccess) return QWMOE_ERR_HIP;
    if (x_out && hipMemcpyAsync(x_out, s->xb[n & 1], xbytes, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return QWMOE_ERR_HIP;
    if (ids_out) {
        // [n_layer][T][k] from the stack's [n_layer][max_T][k]
        const size_t row = (size_t) T * (size_t) s->k * 4, pitch = (size_t) s->max_T * (size_t) s->k * 4;
        if (hipMemcpy2DAsync(ids_out, row, s->ids, pitch, row, (size_t) n, hipMemcpyDeviceToDevice, st) != hipSuccess ||
            hipMemcpy2DAsync(weights_out, row, s->w, pitch, row, (size_t) n, hipMemcpyDeviceToDevice, st) != hipSuccess)
            return QWMOE_ERR_HIP;
    }
    return QWMOE_OK;
}

int64_t qwmoe_layer_stack_captures(const qwmoe_layer_stack* s) { return s ? s->captures : -1; }

int qwmoe_layer_stack_kernel(const qwmoe_layer_stack* s) {
    if (!s) return QWMOE_ERR_INVALID_ARG;
    return s->vfn ? (s->va.local_st ? 2 : 3) : 1;
}

int qwmoe_layer_stack_kernel_t1(qwmoe_layer_stack* s) {
    if (!s) return QWMOE_ERR_INVALID_ARG;
    if (s->ds_allowed && !s->ds_tried) {
        s->ds_tried = true;
        if (qwmoe_decode_stack_create(s->layers.data(), (int) s->layers.size(), s->rms_eps, &s->ds) != QWMOE_OK) {
            s->ds = nullptr;
            (void) hipGetLastError();
        }
    }
    return s->ds ? qwmoe_decode_stack_kernel(s->ds) : 0;
}

int qwmoe_layer_stack_status(void* stream, qwmoe_layer_stack* s, int32_t* status_out, int clear) {
    if (!s) return QWMOE_ERR_INVALID_ARG;
    int32_t v = 0;
    if (hipStreamSynchronize((hipStream_t) stream) != hipSuccess) return QWMOE_ERR_HIP;
    if (s->vfn) {
        if (hipMemcpy(&v, s->va.status, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) return QWMOE_ERR_HIP;
        if (clear && hipMemset(s->va.status, 0, sizeof(int32_t)) != hipSuccess) return QWMOE_ERR_HIP;
    }
    if (s->ds) {
        int32_t vd = 0;
        const int rc = qwmoe_decode_stack_status(stream, s->ds, &vd, clear);
        if (rc != QWMOE_OK) return rc;
        v |= vd;
    }
    if (status_out) *status_out = v;
    return QWMOE_OK;
}

void qwmoe_layer_stack_free(qwmoe_layer_stack* s) {
    if (!s) return;
    (void) hipDeviceSynchronize();
    delete s;
}

}  // extern "C"
