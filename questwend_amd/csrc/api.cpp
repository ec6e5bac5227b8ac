// api.cpp -- the extern "C" boundary (include/qwmoe.h): argument validation,
// workspace carving and dispatch to the HIP kernels.  Host code only.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <new>
#include <random>
#include <vector>

#include "../../include/qwmoe.h"
#include "qw_kernels.hpp"
#include "qw_sort.hpp"
#include "qw_decode.hpp"

namespace {

struct Library {
    bool ready = false;
    int device = -1;
    uint8_t* ws = nullptr;       // device workspace arena
    size_t ws_bytes = 0;
    size_t high_water = 0;
    int32_t* status = nullptr;   // device status word (first 256 bytes of the arena)
    int mfma_min_rows = 8;       // experts with this many routed rows use the matrix-core kernel (0: never)
    int mfma_form = QWMOE_MFMA_EXACT;  // matrix cores' float tail (QWMOE_MFMA_*): ggml's bits unless a caller opts out
};

Library g_lib;
std::mutex g_mu;
// Changes whenever something a captured layer-stack graph baked in changes: the
// workspace is (re)allocated or freed, or the matrix-core row threshold is set.
std::atomic<uint64_t> g_ws_generation{1};

// Lowest workspace offset a call's arena may use: raised while an entry point
// that chains others keeps its own temporaries below it (ArenaFloor).
size_t g_arena_floor = 0;

// Bump allocator over the workspace for one call.
struct Arena {
    uint8_t* base;
    size_t cap, off;
    bool track = true;   // record the high-water mark of the library workspace
    explicit Arena(size_t reserved)
        : base(g_lib.ws), cap(g_lib.ws_bytes), off(reserved > g_arena_floor ? reserved : g_arena_floor) {}
    Arena(void* buf, size_t bytes) : base((uint8_t*) buf), cap(bytes), off(0), track(false) {}
    template <typename T>
    T* take(size_t count) {
        off = (off + 255) & ~(size_t) 255;
        if (off + count * sizeof(T) + 64 > cap) return nullptr;
        T* p = (T*) (base + off);
        off += count * sizeof(T) + 64;  // + slack: kernels may read a few bytes past a row end
        return p;
    }
    ~Arena() {
        if (track && off > g_lib.high_water) g_lib.high_water = off;
    }
};

constexpr size_t kReserved = 256;  // status word lives here

// Keeps the workspace below `off` for the enclosing call while it runs others.
struct ArenaFloor {
    size_t prev;
    explicit ArenaFloor(size_t off) : prev(g_arena_floor) { g_arena_floor = off; }
    ~ArenaFloor() { g_arena_floor = prev; }
};

inline hipStream_t S(void* s) { return (hipStream_t) s; }

bool weight_type_ok(int t) { return t == qw::T_Q4_K || t == qw::T_Q6_K || t == qw::T_Q8_0; }

int check_k(int type, int64_t K) {
    if (K <= 0) return QWMOE_ERR_INVALID_ARG;
    if ((type == qw::T_Q4_K || type == qw::T_Q6_K) && K % 256 != 0) return QWMOE_ERR_UNSUPPORTED;
    if (type == qw::T_Q8_0 && K % 64 != 0) return QWMOE_ERR_UNSUPPORTED;
    return QWMOE_OK;
}

// The kernel arguments of mul_mat_id once b is quantized and ids are grouped.
qw::MmidArgs mmid_args(int type, const void* as, int64_t K, int64_t N, int64_t n_as, size_t nb01, size_t nb02,
                       const uint8_t* bq, int64_t ne11, size_t bq_row, const int32_t* rows, const int32_t* active,
                       const int32_t* active_off, const int32_t* n_active, int64_t max_active,
                       const int32_t* slot_of, int64_t n_slot_of, float* dst, size_t nb1, size_t nb2,
                       int64_t max_rows, int64_t n_pairs, bool fp32_out = false) {
    qw::MmidArgs m{};
    m.type = type;
    m.w = (const uint8_t*) as;
    m.nb1 = nb01;
    m.nb2 = nb02;
    m.K = K;
    m.N = N;
    m.n_as = n_as;
    m.act_q = bq;
    m.b_ne1 = ne11;
    m.act_row_bytes = bq_row;
    m.rows = rows;
    m.active = active;
    m.active_off = active_off;
    m.n_active = n_active;
    m.slot_of = slot_of;
    m.n_slot_of = n_slot_of;
    m.dst = dst;
    m.dst_nb1 = nb1;
    m.dst_nb2 = nb2;
    m.status = g_lib.status;
    m.max_active = max_active;
    // experts with at least mfma_min_rows routed rows (possible only when the
    // batch holds that many pairs) go to the int8 matrix-core kernel; the rest
    // stay on the bit-exact GEMV
    m.mfma_min_rows = 0;
    m.max_rows = max_rows;
    m.n_pairs = n_pairs;
    // the matrix cores' float tail: block sums only where the caller opted in --
    // QWMOE_MFMA_BLOCK_SUM everywhere, QWMOE_MFMA_AUTO for fp32_out (the down
    // projection of a layer entry point)
    m.mfma_exact = g_lib.mfma_form == QWMOE_MFMA_EXACT || (g_lib.mfma_form == QWMOE_MFMA_AUTO && !fp32_out);
    const bool mfma = g_lib.mfma_min_rows > 0 && max_rows >= g_lib.mfma_min_rows && qw::mmid_mfma_supported(m);
    if (mfma) m.mfma_min_rows = g_lib.mfma_min_rows;
    return m;
}

// The exact Q4_K matrix-core form on the f16 matrix cores: an f16 copy of the
// n_rows activation rows in act_q, in the call's workspace.  Without room for it
// the int8 form runs (the same bits).
// QWMOE_MFMA_F16=0 in the environment keeps the int8 form (a test switch).
int mfma_f16_prep(Arena& ar, qw::MmidArgs& m, int64_t n_rows, hipStream_t st) {
    if (!qw::mmid_mfma_h_ok(m, n_rows)) return 0;
    const char* env = getenv("QWMOE_MFMA_F16");
    if (env && env[0] == '0') return 0;
    uint16_t* h = ar.take<uint16_t>((size_t) (n_rows * m.K));
    if (!h) return 0;
    if (int rc = qw::launch_q8K_to_f16(m.act_q, m.act_row_bytes, m.K, n_rows, h, st)) return rc == -2 ? 0 : rc;
    m.act_h = h;
    return 0;
}

// The same copy, written by the launch that quantizes the rows (the returned
// buffer goes to launch_quantize_act / launch_swiglu_q8K as h_out): reserved
// and attached to m, nothing launched; null where the f16 form does not apply.
uint16_t* mfma_f16_reserve(Arena& ar, qw::MmidArgs& m, int64_t n_rows) {
    if (!qw::mmid_mfma_h_ok(m, n_rows)) return nullptr;
    const char* env = getenv("QWMOE_MFMA_F16");
    if (env && env[0] == '0') return nullptr;
    uint16_t* h = ar.take<uint16_t>((size_t) (n_rows * m.K));
    m.act_h = h;
    return h;
}

// Gate and up reading one activation buffer share its f16 copy.
int mfma_f16_prep_pair(Arena& ar, qw::MmidArgs& mu, qw::MmidArgs& mg, int64_t n_rows, hipStream_t st) {
    if (int rc = mfma_f16_prep(ar, mu, n_rows, st)) return rc;
    if (mg.act_q == mu.act_q && mg.act_row_bytes == mu.act_row_bytes && mg.K == mu.K &&
        qw::mmid_mfma_h_ok(mg, n_rows)) {
        mg.act_h = mu.act_h;
        return 0;
    }
    return mfma_f16_prep(ar, mg, n_rows, st);
}

int mmid_launch(const qw::MmidArgs& m, hipStream_t st) {
    // with mfma_min_rows == 1 the matrix cores take every bin that holds a row:
    // the GEMV's workgroups would only return
    int rc = m.mfma_min_rows == 1 ? 0 : qw::launch_mmid_gemv(m, st);
    if (rc == 0 && m.mfma_min_rows > 0) rc = qw::launch_mmid_mfma(m, st);
    return rc;
}

// Gate and up of a layer (same type, shape and grouping): one GEMV launch and
// one matrix-core launch for both, else each on its own.
int mmid_launch_pair(const qw::MmidArgs& mu, const qw::MmidArgs& mg, hipStream_t st) {
    const bool same = mu.type == mg.type && mu.K == mg.K && mu.N == mg.N && mu.mfma_min_rows == mg.mfma_min_rows &&
                      mu.mfma_exact == mg.mfma_exact;
    if (same) {
        int rc = mu.mfma_min_rows == 1 ? 0 : qw::launch_mmid_gemv2(mu, mg, st);
        if (rc == 0 && mu.mfma_min_rows > 0) rc = qw::launch_mmid_mfma2(mu, mg, st);
        if (rc != -2) return rc;
    }
    const int rc = mmid_launch(mu, st);
    return rc ? rc : mmid_launch(mg, st);
}

struct Grouping {
    int32_t *rows, *active, *active_off, *n_active, *counts, *offsets;
    int64_t max_active;
};

int group_args(Arena& ar, const int32_t* ids, int64_t n_ids, int64_t T, size_t ids_nb1, int64_t n_bins,
               int32_t* counts, int32_t* offsets, int32_t* rows_out, Grouping& G, qw::GroupArgs& g) {
    const int64_t P = n_ids * T;
    G.max_active = std::min<int64_t>(n_bins, P);
    G.rows = rows_out ? rows_out : ar.take<int32_t>((size_t) (2 * P + 2));
    G.active = ar.take<int32_t>((size_t) G.max_active + 1);
    G.active_off = ar.take<int32_t>((size_t) G.max_active + 2);
    G.n_active = ar.take<int32_t>(1);
    int32_t* hist = ar.take<int32_t>((size_t) qw::GROUP_WAVES * (size_t) n_bins);
    if (!G.rows || !G.active || !G.active_off || !G.n_active || !hist) return QWMOE_ERR_WORKSPACE;
    G.counts = counts;
    G.offsets = offsets;
    g = qw::GroupArgs{};
    g.ids = ids;
    g.n_ids = n_ids;
    g.T = T;
    g.ids_stride = (int64_t) (ids_nb1 / sizeof(int32_t));
    g.n_bins = n_bins;
    g.counts = counts;
    g.offsets = offsets;
    g.rows = G.rows;
    g.active = G.active;
    g.active_off = G.active_off;
    g.n_active = G.n_active;
    g.status = g_lib.status;
    g.hist_ws = hist;
    return QWMOE_OK;
}

int group(hipStream_t st, Arena& ar, const int32_t* ids, int64_t n_ids, int64_t T, size_t ids_nb1, int64_t n_bins,
          int32_t* counts, int32_t* offsets, int32_t* rows_out, Grouping& G) {
    qw::GroupArgs g;
    const int rc = group_args(ar, ids, n_ids, T, ids_nb1, n_bins, counts, offsets, rows_out, G, g);
    return rc != QWMOE_OK ? rc : qw::launch_group(g, st);
}

}  // namespace

namespace qw {
uint64_t workspace_generation() { return g_ws_generation.load(); }
}  // namespace qw

extern "C" {

int qwmoe_init(int device, size_t workspace_bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    const int mfma_min_rows = g_lib.mfma_min_rows, mfma_form = g_lib.mfma_form;   // settings, kept across re-init
    if (g_lib.ready) {
        if (g_lib.device == device && (workspace_bytes == 0 || workspace_bytes <= g_lib.ws_bytes)) return QWMOE_OK;
        (void) hipFree(g_lib.ws);
        g_lib = Library{};
        g_lib.mfma_min_rows = mfma_min_rows;
        g_lib.mfma_form = mfma_form;
    }
    if (hipSetDevice(device) != hipSuccess) return QWMOE_ERR_HIP;
    const size_t bytes = workspace_bytes ? workspace_bytes : ((size_t) 256 << 20);
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return QWMOE_ERR_HIP;
    if (hipMemset(p, 0, kReserved) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        qw::scratch_setup(device) != 0) {
        (void) hipFree(p);
        return QWMOE_ERR_HIP;
    }
    g_lib.ws = (uint8_t*) p;
    g_lib.ws_bytes = bytes;
    g_lib.status = (int32_t*) p;
    g_lib.device = device;
    g_lib.ready = true;
    g_ws_generation.fetch_add(1);
    return QWMOE_OK;
}

int qwmoe_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_lib.ready) return QWMOE_OK;
    (void) hipDeviceSynchronize();
    (void) hipFree(g_lib.ws);
    const int mfma_min_rows = g_lib.mfma_min_rows, mfma_form = g_lib.mfma_form;
    g_lib = Library{};
    g_lib.mfma_min_rows = mfma_min_rows;
    g_lib.mfma_form = mfma_form;
    g_ws_generation.fetch_add(1);
    return QWMOE_OK;
}

const char* qwmoe_strerror(int status) {
    switch (status) {
        case QWMOE_OK: return "ok";
        case QWMOE_ERR_INVALID_ARG: return "invalid argument";
        case QWMOE_ERR_UNSUPPORTED: return "unsupported type or shape";
        case QWMOE_ERR_HIP: return "HIP runtime error";
        case QWMOE_ERR_WORKSPACE: return "workspace too small";
        case QWMOE_ERR_NOT_INITIALIZED: return "qwmoe_init has not been called";
        case QWMOE_ERR_FORMAT: return "malformed or unsupported GGUF file";
        case QWMOE_ERR_IO: return "file could not be opened or read";
        case QWMOE_ERR_SCRATCH:
            return "the call needs more than the 8 MiB static scratch of the allocation-free entry point";
    }
    return "unknown status";
}

int qwmoe_set_mfma_min_rows(int rows) {
    if (rows < 0) return QWMOE_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_lib.mfma_min_rows != rows) {
        g_lib.mfma_min_rows = rows;
        g_ws_generation.fetch_add(1);   // captured graphs chose kernels with the old threshold
    }
    return QWMOE_OK;
}

int qwmoe_get_mfma_min_rows(void) { return g_lib.mfma_min_rows; }

int qwmoe_set_mfma_form(int form) {
    if (form != QWMOE_MFMA_BLOCK_SUM && form != QWMOE_MFMA_EXACT && form != QWMOE_MFMA_AUTO)
        return QWMOE_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_lib.mfma_form != form) {
        g_lib.mfma_form = form;
        g_ws_generation.fetch_add(1);   // captured graphs chose the kernel with the old setting
    }
    return QWMOE_OK;
}

int qwmoe_get_mfma_form(void) { return g_lib.mfma_form; }

size_t qwmoe_workspace_high_water(void) { return g_lib.high_water; }

size_t qwmoe_row_size(int type, int64_t ne) {
    const int be = qw::block_elems(type), bb = qw::block_bytes(type);
    if (bb == 0 || ne < 0 || ne % be != 0) return 0;
    return (size_t) (ne / be) * (size_t) bb;
}

int qwmoe_vec_dot_type(int type) { return weight_type_ok(type) ? qw::vec_dot_type(type) : QWMOE_ERR_UNSUPPORTED; }

int qwmoe_device_status(void* stream, int32_t* status_out, int clear) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    int32_t v = 0;
    if (hipStreamSynchronize(S(stream)) != hipSuccess) return QWMOE_ERR_HIP;
    if (hipMemcpy(&v, g_lib.status, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) return QWMOE_ERR_HIP;
    if (clear && hipMemset(g_lib.status, 0, sizeof(int32_t)) != hipSuccess) return QWMOE_ERR_HIP;
    if (status_out) *status_out = v;
    return QWMOE_OK;
}

int qwmoe_quantize_act(void* stream, int vdt, const float* src, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1,
                       size_t nb2, void* dst) {
    if (!src || !dst || ne0 <= 0 || ne1 < 0 || ne2 < 0) return QWMOE_ERR_INVALID_ARG;
    if (vdt != qw::T_Q8_K && vdt != qw::T_Q8_0) return QWMOE_ERR_UNSUPPORTED;
    if (ne0 % qw::block_elems(vdt) != 0) return QWMOE_ERR_UNSUPPORTED;
    if (nb1 % 16 != 0 || nb2 % 16 != 0 || ((uintptr_t) src & 15)) return QWMOE_ERR_UNSUPPORTED;
    return qw::launch_quantize_act(vdt, src, ne0, ne1 ? ne1 : 1, ne1 * ne2, nb1, nb2, dst, S(stream));
}

int qwmoe_quantize_chunk(void* stream, int type, const float* src, void* dst, int64_t nrows, int64_t n_per_row) {
    if (!src || !dst || nrows < 0 || n_per_row <= 0) return QWMOE_ERR_INVALID_ARG;
    if (!weight_type_ok(type)) return QWMOE_ERR_UNSUPPORTED;
    if (n_per_row % qw::block_elems(type) != 0) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_quantize_weights(type, src, nrows * n_per_row, dst, S(stream));
}

int qwmoe_dequantize(void* stream, int type, const void* x, float* y, int64_t n) {
    if (!x || !y || n < 0) return QWMOE_ERR_INVALID_ARG;
    if (!weight_type_ok(type)) return QWMOE_ERR_UNSUPPORTED;
    if (n % qw::block_elems(type) != 0) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_dequantize(type, x, y, n, S(stream));
}

int qwmoe_fill_randn(void* stream, float* y, int64_t n, uint64_t seed, float mean, float stddev) {
    if (!y || n < 0) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_randn(y, n, seed, mean, stddev, S(stream));
}

int qwmoe_group_by_expert(void* stream, const int32_t* ids, int64_t n_ids, int64_t T, size_t ids_nb1, int64_t n_as,
                          int32_t* counts, int32_t* offsets, int32_t* rows) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!ids || !rows || n_ids <= 0 || T < 0 || n_as <= 0 || ids_nb1 < (size_t) n_ids * 4 || ids_nb1 % 4)
        return QWMOE_ERR_INVALID_ARG;
    Arena ar(kReserved);
    Grouping G{};
    return group(S(stream), ar, ids, n_ids, T, ids_nb1, n_as, counts, offsets, rows, G);
}

}  // extern "C"

namespace {

// qwmoe_mul_mat_id with its quantized activations and grouping arrays taken
// from `ar` (the library workspace, or the static scratch of the
// allocation-free variant); err_space: the status when `ar` is too small.
int mul_mat_id_in(Arena& ar, int err_space, void* stream, int type, const void* as, int64_t ne00, int64_t ne01,
                  int64_t ne02, size_t nb01, size_t nb02, const float* b, int64_t ne11, int64_t ne12, size_t nb11,
                  size_t nb12, const int32_t* ids, int64_t n_ids, size_t ids_nb1, const int32_t* slot_of,
                  int64_t n_slot_of, float* dst, size_t nb1, size_t nb2) {
    if (!as || !b || !ids || !dst || ne01 <= 0 || ne02 <= 0 || ne11 <= 0 || ne12 < 0 || n_ids <= 0)
        return QWMOE_ERR_INVALID_ARG;
    if (!weight_type_ok(type)) return QWMOE_ERR_UNSUPPORTED;
    int rc = check_k(type, ne00);
    if (rc) return rc;
    const size_t rs = qwmoe_row_size(type, ne00);
    if (nb01 < rs || nb02 < nb01 * (size_t) ne01) return QWMOE_ERR_INVALID_ARG;
    if (ids_nb1 < (size_t) n_ids * 4 || ids_nb1 % 4) return QWMOE_ERR_INVALID_ARG;
    if (nb1 < (size_t) ne01 * 4 || nb2 < nb1 * (size_t) n_ids) return QWMOE_ERR_INVALID_ARG;
    if (slot_of && n_slot_of <= 0) return QWMOE_ERR_INVALID_ARG;
    if (ne11 != 1 && ne11 != n_ids) return QWMOE_ERR_UNSUPPORTED;  // the broadcast rule e % ne11 needs ne11 | n_ids
    if (ne12 == 0) return QWMOE_OK;
    const int vdt = qw::vec_dot_type(type);
    const size_t qrow = qwmoe_row_size(vdt, ne00);
    if (qrow % 4) return QWMOE_ERR_UNSUPPORTED;
    hipStream_t st = S(stream);
    uint8_t* bq = ar.take<uint8_t>(qrow * (size_t) (ne11 * ne12) + 64);
    if (!bq) return err_space;
    const int64_t n_bins = slot_of ? n_slot_of : ne02;
    Grouping G{};
    qw::GroupArgs ga;
    rc = group_args(ar, ids, n_ids, ne12, ids_nb1, n_bins, nullptr, nullptr, nullptr, G, ga);
    if (rc) return rc == QWMOE_ERR_WORKSPACE ? err_space : rc;
    rc = qwmoe_quantize_act(stream, vdt, b, ne00, ne11, ne12, nb11, nb12, bq);
    if (rc) return rc;
    if (qw::launch_group(ga, st) != 0) return QWMOE_ERR_HIP;
    qw::MmidArgs m = mmid_args(type, as, ne00, ne01, ne02, nb01, nb02, bq, ne11, qrow, G.rows, G.active, G.active_off,
                               G.n_active, G.max_active, slot_of, n_slot_of, dst, nb1, nb2, n_ids * ne12, n_ids * ne12);
    if ((rc = mfma_f16_prep(ar, m, ne11 * ne12, st))) return rc;
    return mmid_launch(m, st);
}

}  // namespace

extern "C" {

int qwmoe_mul_mat_id(void* stream, int type, const void* as, int64_t ne00, int64_t ne01, int64_t ne02, size_t nb01,
                     size_t nb02, const float* b, int64_t ne11, int64_t ne12, size_t nb11, size_t nb12,
                     const int32_t* ids, int64_t n_ids, size_t ids_nb1, const int32_t* slot_of, int64_t n_slot_of,
                     float* dst, size_t nb1, size_t nb2) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    Arena ar(kReserved);
    return mul_mat_id_in(ar, QWMOE_ERR_WORKSPACE, stream, type, as, ne00, ne01, ne02, nb01, nb02, b, ne11, ne12, nb11,
                         nb12, ids, n_ids, ids_nb1, slot_of, n_slot_of, dst, nb1, nb2);
}

int qwmoe_mul_mat_id_noalloc(void* stream, int type, const void* as, int64_t ne00, int64_t ne01, int64_t ne02,
                             size_t nb01, size_t nb02, const float* b, int64_t ne11, int64_t ne12, size_t nb11,
                             size_t nb12, const int32_t* ids, int64_t n_ids, size_t ids_nb1, const int32_t* slot_of,
                             int64_t n_slot_of, float* dst, size_t nb1, size_t nb2) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return QWMOE_ERR_HIP;
    if (cur != g_lib.device) return QWMOE_ERR_INVALID_ARG;   // the status word lives on the library's device
    void* ptr = qw::scratch_ptr(cur);   // looked up by qwmoe_init
    if (!ptr) return QWMOE_ERR_NOT_INITIALIZED;
    Arena ar(ptr, qw::kScratchBytes);
    return mul_mat_id_in(ar, QWMOE_ERR_SCRATCH, stream, type, as, ne00, ne01, ne02, nb01, nb02, b, ne11, ne12, nb11,
                         nb12, ids, n_ids, ids_nb1, slot_of, n_slot_of, dst, nb1, nb2);
}

int qwmoe_router_topk(void* stream, const float* W, const float* x, int64_t H, int64_t E, int64_t k, int64_t T,
                      size_t x_nb1, float clamp_min, float scale, int32_t* ids, float* weights, float* probs) {
    return qwmoe_router_topk_resident(stream, W, x, H, E, k, T, x_nb1, clamp_min, scale, nullptr, nullptr, ids, weights,
                                      probs);
}

int qwmoe_router_topk_resident(void* stream, const float* W, const float* x, int64_t H, int64_t E, int64_t k,
                               int64_t T, size_t x_nb1, float clamp_min, float scale, const float* mask,
                               int32_t* want, int32_t* ids, float* weights, float* probs) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!W || !x || !ids || !weights || H <= 0 || E <= 0 || k <= 0 || k > E || T < 0) return QWMOE_ERR_INVALID_ARG;
    if (E % 8 || E > 512 || H % 4 || x_nb1 % 16 || ((uintptr_t) x & 15) || ((uintptr_t) W & 15) || x_nb1 < (size_t) H * 4)
        return QWMOE_ERR_UNSUPPORTED;
    Arena ar(kReserved);
    float* logits = ar.take<float>((size_t) (E * T) + 1);
    if (!logits) return QWMOE_ERR_WORKSPACE;
    qw::RouterArgs a{};
    a.W = W;
    a.x = x;
    a.x_stride = (int64_t) (x_nb1 / 4);
    a.H = H;
    a.E = E;
    a.k = k;
    a.T = T;
    a.clamp_min = clamp_min;
    a.scale = scale;
    a.ids = ids;
    a.weights = weights;
    a.probs = probs;
    a.logits = nullptr;
    a.status = g_lib.status;
    a.mask = mask;
    a.want = want;
    return qw::launch_router(a, logits, S(stream));
}

int qwmoe_swiglu(void* stream, const float* gate, const float* up, float* out, int64_t n, int64_t rows) {
    if (!gate || !up || !out || n <= 0 || rows < 0) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_swiglu(gate, up, out, rows, n, (size_t) n * 4, (size_t) n * 4, (size_t) n * 4, S(stream));
}

int qwmoe_weighted_sum(void* stream, const float* experts, const float* weights, float* out, int64_t H, int64_t k,
                       int64_t T) {
    if (!experts || !weights || !out || H <= 0 || k <= 0 || T < 0) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_weighted_sum(experts, weights, out, H, k, T, S(stream));
}

int qwmoe_rms_norm(void* stream, const float* x, float* y, int64_t n, int64_t rows, float eps) {
    if (!x || !y || n <= 0 || rows < 0 || !(eps >= 0.0f)) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_rms_norm(x, y, n, rows, eps, S(stream));
}

int qwmoe_rms_norm_mul(void* stream, const float* x, const float* w, float* y, int64_t n, int64_t rows, float eps) {
    if (!x || !w || !y || n <= 0 || rows < 0 || !(eps >= 0.0f)) return QWMOE_ERR_INVALID_ARG;
    return qw::launch_rms_norm(x, y, n, rows, eps, S(stream), w);
}

int qwmoe_shared_expert_add(void* stream, const qwmoe_shared_expert* se, int64_t H, const float* x, int64_t T,
                            const float* moe_out, const float* resid, float* out) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!se || !x || !moe_out || !out || H <= 0 || T < 0) return QWMOE_ERR_INVALID_ARG;
    const int64_t F = se->n_ff;
    if (F <= 0 || !se->gate || !se->up || !se->down || !se->gate_inp) return QWMOE_ERR_INVALID_ARG;
    if (!weight_type_ok(se->type_gate) || !weight_type_ok(se->type_up) || !weight_type_ok(se->type_down))
        return QWMOE_ERR_UNSUPPORTED;
    int rc;
    if ((rc = check_k(se->type_gate, H)) || (rc = check_k(se->type_up, H)) || (rc = check_k(se->type_down, F)))
        return rc;
    if (F % 8 || H % 32) return QWMOE_ERR_UNSUPPORTED;   // SwiGLU in blocks of 8; the gate's 32 chains
    if (se->gate_nb1 < qwmoe_row_size(se->type_gate, H) || se->up_nb1 < qwmoe_row_size(se->type_up, H) ||
        se->down_nb1 < qwmoe_row_size(se->type_down, F))
        return QWMOE_ERR_INVALID_ARG;
    if (T == 0) return QWMOE_OK;
    hipStream_t st = S(stream);
    Arena ar(kReserved);
    // every token uses "expert" 0 once: the mul_mat_id kernels then compute the
    // dense mul_mat (same row dots as ggml_mul_mat of a quantized weight)
    int32_t* rows = ar.take<int32_t>((size_t) (2 * T + 2));
    int32_t* active = ar.take<int32_t>(2);
    int32_t* active_off = ar.take<int32_t>(3);
    int32_t* n_active = ar.take<int32_t>(1);
    float* upo = ar.take<float>((size_t) (F * T));
    float* gateo = ar.take<float>((size_t) (F * T));
    float* act = ar.take<float>((size_t) (F * T));
    float* sh = ar.take<float>((size_t) (H * T));
    const int vg = qw::vec_dot_type(se->type_gate), vu = qw::vec_dot_type(se->type_up);
    const int vd = qw::vec_dot_type(se->type_down);
    const size_t qg = qwmoe_row_size(vg, H), qu = qwmoe_row_size(vu, H), qd = qwmoe_row_size(vd, F);
    uint8_t* xg = ar.take<uint8_t>(qg * (size_t) T + 64);
    uint8_t* xu = (vu == vg) ? xg : ar.take<uint8_t>(qu * (size_t) T + 64);
    uint8_t* aq = ar.take<uint8_t>(qd * (size_t) T + 64);
    if (!rows || !active || !active_off || !n_active || !upo || !gateo || !act || !sh || !xg || !xu || !aq)
        return QWMOE_ERR_WORKSPACE;
    if ((rc = qw::launch_group_dense(rows, active, active_off, n_active, T, st))) return rc;
    if ((rc = qw::launch_quantize_act(vg, x, H, 1, T, (size_t) H * 4, (size_t) H * 4, xg, st))) return rc;
    if (xu != xg && (rc = qw::launch_quantize_act(vu, x, H, 1, T, (size_t) H * 4, (size_t) H * 4, xu, st))) return rc;
    const size_t fb = (size_t) F * 4;
    qw::MmidArgs mu = mmid_args(se->type_up, se->up, H, F, 1, se->up_nb1, se->up_nb1 * (size_t) F, xu, 1, qu, rows,
                                active, active_off, n_active, 1, nullptr, 0, upo, fb, fb, T, T);
    qw::MmidArgs mg = mmid_args(se->type_gate, se->gate, H, F, 1, se->gate_nb1, se->gate_nb1 * (size_t) F, xg, 1, qg,
                                rows, active, active_off, n_active, 1, nullptr, 0, gateo, fb, fb, T, T);
    if ((rc = mfma_f16_prep_pair(ar, mu, mg, T, st))) return rc;
    if ((rc = mmid_launch_pair(mu, mg, st))) return rc;
    // ggml_mul(ggml_silu(g), u) rounds as swiglu_split does: silu, then one multiply
    qw::MmidArgs md = mmid_args(se->type_down, se->down, F, H, 1, se->down_nb1, se->down_nb1 * (size_t) H, aq, 1, qd,
                                rows, active, active_off, n_active, 1, nullptr, 0, sh, (size_t) H * 4, (size_t) H * 4, T, T, true);
    md.swiglu_gate = gateo;
    md.swiglu_up = upo;
    if (vd == qw::T_Q8_K && qw::mmid_gemv_swiglu_ok(md)) {
        // the down GEMV forms SwiGLU's Q8_K rows itself
    } else if (vd == qw::T_Q8_K) {
        md.swiglu_gate = md.swiglu_up = nullptr;
        if ((rc = qw::launch_swiglu_q8K(gateo, upo, F, T, aq, st))) return rc;
    } else {
        md.swiglu_gate = md.swiglu_up = nullptr;
        if ((rc = qw::launch_swiglu(gateo, upo, act, T, F, fb, fb, fb, st))) return rc;
        if ((rc = qw::launch_quantize_act(vd, act, F, 1, T, fb, fb, aq, st))) return rc;
    }
    if (!md.swiglu_gate && (rc = mfma_f16_prep(ar, md, T, st))) return rc;
    if ((rc = mmid_launch(md, st))) return rc;
    return qw::launch_shared_gate_add(x, (size_t) H, se->gate_inp, sh, moe_out, resid, out, (size_t) H, H, T, st);
}

// The attention half of Seg A (core/runtime.cpp:1976-2030 with build_attn,
// 681-734): projections as ggml_mul_mat of the quantized weights (every token
// "expert" 0 of a one-bin grouping, so the mul_mat_id row dots apply), the
// attention core in attn.hip, the residual and the FFN input norm.
int qwmoe_attn_seg(void* stream, const qwmoe_attn_layer* L, const float* h, int64_t T, int64_t n_past,
                   float rms_eps, float* attn_resid, float* ffn_in) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!L || !h || !attn_resid || T < 0 || n_past < 0 || !(rms_eps >= 0.0f)) return QWMOE_ERR_INVALID_ARG;
    const int64_t H = L->n_embd, nq = L->n_head, nk = L->n_head_kv, D = L->n_embd_head;
    if (H <= 0 || nq <= 0 || nk <= 0 || nq % nk || !L->attn_norm || !L->wq || !L->wk || !L->wv || !L->wo ||
        !L->q_norm || !L->k_norm || !L->k_cache || !L->v_cache || (ffn_in && !L->ffn_norm))
        return QWMOE_ERR_INVALID_ARG;
    if (n_past + T > L->n_ctx) return QWMOE_ERR_INVALID_ARG;
    if (D != 128 || L->n_rot != D || nq / nk > qw::ATT_RMAX || H % 4) return QWMOE_ERR_UNSUPPORTED;
    if (((uintptr_t) L->k_cache & 15) || ((uintptr_t) L->v_cache & 15) || ((uintptr_t) h & 15))
        return QWMOE_ERR_UNSUPPORTED;
    const int types[4] = {L->type_q, L->type_k, L->type_v, L->type_o};
    for (int t : types)
        if (!weight_type_ok(t)) return QWMOE_ERR_UNSUPPORTED;
    const int64_t NQ = nq * D, NK = nk * D;
    int rc;
    if ((rc = check_k(L->type_q, H)) || (rc = check_k(L->type_k, H)) || (rc = check_k(L->type_v, H)) ||
        (rc = check_k(L->type_o, NQ)))
        return rc;
    if (L->wq_nb1 < qwmoe_row_size(L->type_q, H) || L->wk_nb1 < qwmoe_row_size(L->type_k, H) ||
        L->wv_nb1 < qwmoe_row_size(L->type_v, H) || L->wo_nb1 < qwmoe_row_size(L->type_o, NQ))
        return QWMOE_ERR_INVALID_ARG;
    if (T == 0) return QWMOE_OK;
    hipStream_t st = S(stream);
    Arena ar(kReserved);
    const int64_t n_kv = n_past + T, split = qw::attn_split(T, nk, n_kv), n_split = (n_kv + split - 1) / split;
    int32_t* rows = ar.take<int32_t>((size_t) (2 * T + 2));
    int32_t* active = ar.take<int32_t>(2);
    int32_t* active_off = ar.take<int32_t>(3);
    int32_t* n_active = ar.take<int32_t>(1);
    float* cur = ar.take<float>((size_t) (H * T));
    float* q = ar.take<float>((size_t) (NQ * T));
    float* k = ar.take<float>((size_t) (NK * T));
    float* v = ar.take<float>((size_t) (NK * T));
    float* qr = ar.take<float>((size_t) (NQ * T));
    // the score rows and P.V partials exist only on the split path (fewer than 64
    // query rows per kv head); the matrix-core path recomputes scores beside P.V
    const bool mf_path = T * (nq / nk) >= 64;
    float* sc = mf_path ? nullptr : ar.take<float>((size_t) (nq * T * n_kv));
    float* part = mf_path ? nullptr : ar.take<float>((size_t) (n_split * T * NQ));
    float* stat = ar.take<float>((size_t) (qw::attn_stat_blocks(T, nk, n_kv) * T * nq * 2));
    float* att = ar.take<float>((size_t) (NQ * T));
    float* proj = ar.take<float>((size_t) (H * T));
    if (!rows || !active || !active_off || !n_active || !cur || !q || !k || !v || !qr || (!mf_path && (!sc || !part)) ||
        !stat || !att || !proj)
        return QWMOE_ERR_WORKSPACE;
    // quantized activations, one per vec_dot type in use
    const int vqt = qw::vec_dot_type(L->type_q), vkt = qw::vec_dot_type(L->type_k), vvt = qw::vec_dot_type(L->type_v);
    const int vot = qw::vec_dot_type(L->type_o);
    const size_t rq = qwmoe_row_size(vqt, H), rk = qwmoe_row_size(vkt, H), rv = qwmoe_row_size(vvt, H);
    const size_t ro = qwmoe_row_size(vot, NQ);
    uint8_t* xq = ar.take<uint8_t>(rq * (size_t) T + 64);
    uint8_t* xk = vkt == vqt ? xq : ar.take<uint8_t>(rk * (size_t) T + 64);
    uint8_t* xv = vvt == vqt ? xq : vvt == vkt ? xk : ar.take<uint8_t>(rv * (size_t) T + 64);
    uint8_t* aq = ar.take<uint8_t>(ro * (size_t) T + 64);
    if (!xq || !xk || !xv || !aq) return QWMOE_ERR_WORKSPACE;
    if ((rc = qw::launch_group_dense(rows, active, active_off, n_active, T, st))) return rc;
    const size_t hb = (size_t) H * 4;
    // attn_norm, then the projections' input quantized: one launch when every
    // projection reads Q8_K (the K-quants), the same bits as the two steps
    const bool fused_norm = vqt == qw::T_Q8_K && xk == xq && xv == xq &&
                            qw::launch_rms_norm_q8K(h, H, T, rms_eps, L->attn_norm, xq, st) == 0;
    if (!fused_norm) {
        if ((rc = qw::launch_rms_norm(h, cur, H, T, rms_eps, st, L->attn_norm))) return rc;
        if ((rc = qw::launch_quantize_act(vqt, cur, H, 1, T, hb, hb, xq, st))) return rc;
        if (xk != xq && (rc = qw::launch_quantize_act(vkt, cur, H, 1, T, hb, hb, xk, st))) return rc;
        if (xv != xq && xv != xk && (rc = qw::launch_quantize_act(vvt, cur, H, 1, T, hb, hb, xv, st))) return rc;
    }
    auto proj_launch = [&](int type, const void* w, size_t nb1, int64_t K, int64_t N, const uint8_t* xb, size_t xrow,
                           float* dst) {
        const size_t ob = (size_t) N * 4;
        const qw::MmidArgs m = mmid_args(type, w, K, N, 1, nb1, nb1 * (size_t) N, xb, 1, xrow, rows, active,
                                         active_off, n_active, 1, nullptr, 0, dst, ob, ob, T, T);
        return mmid_launch(m, st);
    };
    {   // Q and K in one GEMV launch when they share a type and neither takes the matrix cores
        const qw::MmidArgs mq = mmid_args(L->type_q, L->wq, H, NQ, 1, L->wq_nb1, L->wq_nb1 * (size_t) NQ, xq, 1, rq,
                                          rows, active, active_off, n_active, 1, nullptr, 0, q, (size_t) NQ * 4,
                                          (size_t) NQ * 4, T, T);
        const qw::MmidArgs mk = mmid_args(L->type_k, L->wk, H, NK, 1, L->wk_nb1, L->wk_nb1 * (size_t) NK, xk, 1, rk,
                                          rows, active, active_off, n_active, 1, nullptr, 0, k, (size_t) NK * 4,
                                          (size_t) NK * 4, T, T);
        const bool pair = mq.type == mk.type && mq.mfma_min_rows == 0 && mk.mfma_min_rows == 0 && NQ >= NK &&
                          qw::launch_mmid_gemv2(mq, mk, st) == 0;
        if (!pair) {
            if ((rc = mmid_launch(mq, st))) return rc;
            if ((rc = mmid_launch(mk, st))) return rc;
        }
    }
    if ((rc = proj_launch(L->type_v, L->wv, L->wv_nb1, H, NK, xv, rv, v))) return rc;
    qw::AttnArgs a{};
    a.T = (int) T;
    a.n_head = (int) nq;
    a.n_head_kv = (int) nk;
    a.n_past = n_past;
    a.n_kv = n_kv;
    a.eps = rms_eps;
    a.theta_scale = powf(L->rope_freq_base, -2.0f / (float) L->n_rot);   // ggml_compute_forward_rope_flt
    a.kq_scale = 1.0f / sqrtf((float) D);
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_norm = L->q_norm;
    a.k_norm = L->k_norm;
    a.qr = qr;
    a.kc = L->k_cache;
    a.vc = L->v_cache;
    a.s = sc;
    a.split = split;
    a.part = part;
    a.stat = stat;
    a.att = att;
    a.att_q8K = vot == qw::T_Q8_K ? aq : nullptr;   // the split path quantizes att as it sums it
    if ((rc = qw::launch_attn_core(a, st))) return rc;
    const size_t qb = (size_t) NQ * 4;
    if (!qw::attn_writes_q8K(a) && (rc = qw::launch_quantize_act(vot, att, NQ, 1, T, qb, qb, aq, st))) return rc;
    if ((rc = proj_launch(L->type_o, L->wo, L->wo_nb1, NQ, H, aq, ro, proj))) return rc;
    return qw::launch_add_rms_norm_mul(proj, h, attn_resid, ffn_in, H, T, rms_eps, L->ffn_norm, st);
}

// The recurrent half of Seg A for a gated-delta-net layer (build_segA with
// build_gdn, core/runtime.cpp:1976-1995 and 737-859): the five projections as
// one-expert mul_mat_ids (ggml's row dots), the conv, the recurrence and the
// gated norm in gdn.hip, the residual and the FFN input norm.
int qwmoe_gdn_seg(void* stream, const qwmoe_gdn_layer* L, const float* h, int64_t T, float rms_eps,
                  float* attn_resid, float* ffn_in) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!L || !h || !attn_resid || T < 0 || !(rms_eps >= 0.0f)) return QWMOE_ERR_INVALID_ARG;
    const int64_t H = L->n_embd, Sd = L->d_state, Hk = L->n_group, Hv = L->dt_rank, dc = L->d_conv;
    if (H <= 0 || Sd <= 0 || Hk <= 0 || Hv <= 0 || dc <= 0 || !L->attn_norm || !L->w_qkv || !L->w_gate ||
        !L->w_beta || !L->w_alpha || !L->w_out || !L->dt_bias || !L->ssm_a || !L->conv1d || !L->ssm_norm ||
        !L->conv_state || !L->ssm_state || (ffn_in && !L->ffn_norm))
        return QWMOE_ERR_INVALID_ARG;
    if (!qw::gdn_shape_ok(Sd, Hk, Hv, dc) || H % 4 || ((uintptr_t) h & 15) || ((uintptr_t) L->ssm_state & 15))
        return QWMOE_ERR_UNSUPPORTED;
    const int64_t d_inner = Hv * Sd, key_dim = Hk * Sd, conv_ch = d_inner + 2 * key_dim;
    const int types[5] = {L->type_qkv, L->type_gate, L->type_beta, L->type_alpha, L->type_out};
    for (int t : types)
        if (!weight_type_ok(t)) return QWMOE_ERR_UNSUPPORTED;
    int rc;
    if ((rc = check_k(L->type_qkv, H)) || (rc = check_k(L->type_gate, H)) || (rc = check_k(L->type_beta, H)) ||
        (rc = check_k(L->type_alpha, H)) || (rc = check_k(L->type_out, d_inner)))
        return rc;
    if (L->w_qkv_nb1 < qwmoe_row_size(L->type_qkv, H) || L->w_gate_nb1 < qwmoe_row_size(L->type_gate, H) ||
        L->w_beta_nb1 < qwmoe_row_size(L->type_beta, H) || L->w_alpha_nb1 < qwmoe_row_size(L->type_alpha, H) ||
        L->w_out_nb1 < qwmoe_row_size(L->type_out, d_inner))
        return QWMOE_ERR_INVALID_ARG;
    if (T == 0) return QWMOE_OK;
    if (T > INT32_MAX / 2) return QWMOE_ERR_UNSUPPORTED;
    hipStream_t st = S(stream);
    Arena ar(kReserved);
    int32_t* rows = ar.take<int32_t>((size_t) (2 * T + 2));
    int32_t* active = ar.take<int32_t>(2);
    int32_t* active_off = ar.take<int32_t>(3);
    int32_t* n_active = ar.take<int32_t>(1);
    float* cur = ar.take<float>((size_t) (H * T));
    float* qkv = ar.take<float>((size_t) (conv_ch * T));
    float* z = ar.take<float>((size_t) (d_inner * T));
    float* braw = ar.take<float>((size_t) (Hv * T));
    float* araw = ar.take<float>((size_t) (Hv * T));
    float* conv = ar.take<float>((size_t) (conv_ch * T));
    float* qn = ar.take<float>((size_t) (key_dim * T));
    float* kn = ar.take<float>((size_t) (key_dim * T));
    float* bg = ar.take<float>((size_t) (2 * Hv * T));
    float* o = ar.take<float>((size_t) (d_inner * T));
    float* y = ar.take<float>((size_t) (d_inner * T));
    float* proj = ar.take<float>((size_t) (H * T));
    // one bin per token for the H_v-row projections (beta, alpha)
    int32_t* trows = ar.take<int32_t>((size_t) (2 * T));
    int32_t* tactive = ar.take<int32_t>((size_t) T);
    int32_t* toff = ar.take<int32_t>((size_t) (T + 1));
    int32_t* tn = ar.take<int32_t>(1);
    int32_t* tslot = ar.take<int32_t>((size_t) T);
    if (!rows || !active || !active_off || !n_active || !cur || !qkv || !z || !braw || !araw || !conv || !qn || !kn ||
        !bg || !o || !y || !proj || !trows || !tactive || !toff || !tn || !tslot)
        return QWMOE_ERR_WORKSPACE;
    // the input quantized once per vec_dot type the four input projections use
    int vt[4] = {qw::vec_dot_type(L->type_qkv), qw::vec_dot_type(L->type_gate), qw::vec_dot_type(L->type_beta),
                 qw::vec_dot_type(L->type_alpha)};
    uint8_t* xq[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t xr[4];
    for (int i = 0; i < 4; ++i) {
        xr[i] = qwmoe_row_size(vt[i], H);
        for (int j = 0; j < i; ++j)
            if (vt[j] == vt[i]) xq[i] = xq[j];
        if (!xq[i] && !(xq[i] = ar.take<uint8_t>(xr[i] * (size_t) T + 64))) return QWMOE_ERR_WORKSPACE;
    }
    const int vot = qw::vec_dot_type(L->type_out);
    const size_t ro = qwmoe_row_size(vot, d_inner);
    uint8_t* yq = ar.take<uint8_t>(ro * (size_t) T + 64);
    if (!yq) return QWMOE_ERR_WORKSPACE;
    if ((rc = qw::launch_group_dense(rows, active, active_off, n_active, T, st))) return rc;
    if ((rc = qw::launch_gdn_group_tokens(trows, tactive, toff, tn, tslot, T, st))) return rc;
    const size_t hb = (size_t) H * 4;
    if ((rc = qw::launch_rms_norm(h, cur, H, T, rms_eps, st, L->attn_norm))) return rc;
    for (int i = 0; i < 4; ++i) {
        bool done = false;
        for (int j = 0; j < i; ++j) done = done || xq[j] == xq[i];
        if (!done && (rc = qw::launch_quantize_act(vt[i], cur, H, 1, T, hb, hb, xq[i], st))) return rc;
    }
    auto proj_launch = [&](int type, const void* w, size_t nb1, int64_t K, int64_t N, const uint8_t* xb, size_t xrow,
                           float* dst) {
        const size_t ob = (size_t) N * 4;
        qw::MmidArgs m = mmid_args(type, w, K, N, 1, nb1, nb1 * (size_t) N, xb, 1, xrow, rows, active, active_off,
                                   n_active, 1, nullptr, 0, dst, ob, ob, T, T);
        if (int r = mfma_f16_prep(ar, m, T, st)) return r;
        return mmid_launch(m, st);
    };
    if ((rc = proj_launch(L->type_qkv, L->w_qkv, L->w_qkv_nb1, H, conv_ch, xq[0], xr[0], qkv))) return rc;
    if ((rc = proj_launch(L->type_gate, L->w_gate, L->w_gate_nb1, H, d_inner, xq[1], xr[1], z))) return rc;
    {   // beta and alpha: a workgroup per token (and both in one launch when they share a type)
        auto small = [&](int type, const void* w, size_t nb1, const uint8_t* xb, size_t xrow, float* dst) {
            return mmid_args(type, w, H, Hv, 1, nb1, nb1 * (size_t) Hv, xb, 1, xrow, trows, tactive, toff, tn, T,
                             tslot, T, dst, 0, (size_t) Hv * 4, 1, T);
        };
        const qw::MmidArgs mb = small(L->type_beta, L->w_beta, L->w_beta_nb1, xq[2], xr[2], braw);
        const qw::MmidArgs ma = small(L->type_alpha, L->w_alpha, L->w_alpha_nb1, xq[3], xr[3], araw);
        if (!(mb.type == ma.type && qw::launch_mmid_gemv2(mb, ma, st) == 0)) {
            if ((rc = mmid_launch(mb, st))) return rc;
            if ((rc = mmid_launch(ma, st))) return rc;
        }
    }
    qw::GdnArgs a{};
    a.T = (int) T;
    a.H_k = (int) Hk;
    a.H_v = (int) Hv;
    a.d_conv = (int) dc;
    a.conv_ch = conv_ch;
    a.eps = rms_eps;
    a.qkv = qkv;
    a.z = z;
    a.braw = braw;
    a.araw = araw;
    a.dt_bias = L->dt_bias;
    a.ssm_a = L->ssm_a;
    a.conv1d = L->conv1d;
    a.ssm_norm = L->ssm_norm;
    a.conv_state = L->conv_state;
    a.state = L->ssm_state;
    a.conv = conv;
    a.qn = qn;
    a.kn = kn;
    a.bg = bg;
    a.o = o;
    a.y = y;
    if ((rc = qw::launch_gdn_core(a, st))) return rc == -2 ? QWMOE_ERR_UNSUPPORTED : QWMOE_ERR_HIP;
    const size_t yb = (size_t) d_inner * 4;
    if ((rc = qw::launch_quantize_act(vot, y, d_inner, 1, T, yb, yb, yq, st))) return rc;
    if ((rc = proj_launch(L->type_out, L->w_out, L->w_out_nb1, d_inner, H, yq, ro, proj))) return rc;
    return qw::launch_add_rms_norm_mul(proj, h, attn_resid, ffn_in, H, T, rms_eps, L->ffn_norm, st);
}

int qwmoe_decoder_layer(void* stream, const qwmoe_attn_layer* attn, const qwmoe_layer* moe, const float* h,
                        int64_t T, int64_t n_past, float rms_eps, float* h_out, int32_t* ids_out,
                        float* weights_out) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!attn || !moe || !h || !h_out || T < 0 || !(rms_eps >= 0.0f)) return QWMOE_ERR_INVALID_ARG;
    if (moe->n_embd != attn->n_embd || !attn->ffn_norm) return QWMOE_ERR_INVALID_ARG;
    if (T == 0) return QWMOE_OK;
    const int64_t H = attn->n_embd;
    Arena ar(kReserved);
    float* resid = ar.take<float>((size_t) (H * T));
    float* fin = ar.take<float>((size_t) (H * T));
    float* moe_out = ar.take<float>((size_t) (H * T));
    if (!resid || !fin || !moe_out) return QWMOE_ERR_WORKSPACE;
    const ArenaFloor keep(ar.off);   // the calls below take their temporaries above these
    int rc = qwmoe_attn_seg(stream, attn, h, T, n_past, rms_eps, resid, fin);
    if (rc == QWMOE_OK) rc = qwmoe_ffn_layer(stream, moe, fin, T, moe_out, -1.0f, nullptr, ids_out, weights_out);
    // h_new = moe_out + attn_resid (build_segB, core/runtime.cpp:2087)
    if (rc == QWMOE_OK) rc = qw::launch_add_rms_norm_mul(moe_out, resid, h_out, nullptr, H, T, 0.0f, nullptr, S(stream));
    return rc;
}

int qwmoe_ffn_layer(void* stream, const qwmoe_layer* L, const float* x, int64_t T, float* out, float rms_eps,
                    float* x_next, int32_t* ids_out, float* weights_out) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!L || !x || !out || T < 0) return QWMOE_ERR_INVALID_ARG;
    const int64_t H = L->n_embd, E = L->n_expert, k = L->n_expert_used, F = L->n_ff;
    if (H <= 0 || E <= 0 || k <= 0 || k > E || F <= 0 || !L->router || !L->gate || !L->up || !L->down)
        return QWMOE_ERR_INVALID_ARG;
    if (!weight_type_ok(L->type_gate) || !weight_type_ok(L->type_up) || !weight_type_ok(L->type_down))
        return QWMOE_ERR_UNSUPPORTED;
    int rc;
    if ((rc = check_k(L->type_gate, H)) || (rc = check_k(L->type_up, H)) || (rc = check_k(L->type_down, F))) return rc;
    if (F % 8) return QWMOE_ERR_UNSUPPORTED;
    if (rms_eps >= 0.0f && !x_next) return QWMOE_ERR_INVALID_ARG;
    // the checks of the calls it fuses: expert strides (qwmoe_mul_mat_id) and
    // the router's shape and 16-byte alignment (qwmoe_router_topk)
    const size_t rsg = qwmoe_row_size(L->type_gate, H), rsu = qwmoe_row_size(L->type_up, H);
    const size_t rsd = qwmoe_row_size(L->type_down, F);
    if (L->gate_nb1 < rsg || L->gate_nb2 < L->gate_nb1 * (size_t) F || L->up_nb1 < rsu ||
        L->up_nb2 < L->up_nb1 * (size_t) F || L->down_nb1 < rsd || L->down_nb2 < L->down_nb1 * (size_t) H ||
        L->n_slots_gate <= 0 || L->n_slots_up <= 0 || L->n_slots_down <= 0)
        return QWMOE_ERR_INVALID_ARG;
    if (E % 8 || E > 512 || H % 4 || ((uintptr_t) x & 15) || ((uintptr_t) L->router & 15)) return QWMOE_ERR_UNSUPPORTED;
    if (T == 0) return QWMOE_OK;
    hipStream_t st = S(stream);
    Arena ar(kReserved);
    // the router writes ids and weights straight into the caller's buffers when it gave them
    int32_t* ids = ids_out ? ids_out : ar.take<int32_t>((size_t) (k * T));
    float* w = weights_out ? weights_out : ar.take<float>((size_t) (k * T));
    float* logits = ar.take<float>((size_t) (E * T));
    float* upo = ar.take<float>((size_t) (F * k * T));
    float* gateo = ar.take<float>((size_t) (F * k * T));
    float* act = ar.take<float>((size_t) (F * k * T));
    float* ex = ar.take<float>((size_t) (H * k * T));
    if (!ids || !w || !logits || !upo || !gateo || !act || !ex) return QWMOE_ERR_WORKSPACE;
    // router
    qw::RouterArgs ra{};
    ra.W = L->router;
    ra.x = x;
    ra.x_stride = H;
    ra.H = H;
    ra.E = E;
    ra.k = k;
    ra.T = T;
    ra.clamp_min = 6.103515625e-5f;
    ra.scale = L->expert_weights_scale;
    ra.ids = ids;
    ra.weights = w;
    ra.status = g_lib.status;
    ra.mask = L->resmask;
    ra.want = L->want_ids;
    if (E % 8 || E > 512 || H % 4) return QWMOE_ERR_UNSUPPORTED;
    // x quantized once per distinct activation type of gate / up; a small batch's
    // Q8_K copy is made by the router launch
    const int vg = qw::vec_dot_type(L->type_gate), vu = qw::vec_dot_type(L->type_up);
    const size_t qg = qwmoe_row_size(vg, H), qu = qwmoe_row_size(vu, H);
    uint8_t* xg = ar.take<uint8_t>(qg * (size_t) T + 64);
    uint8_t* xu = (vu == vg) ? xg : ar.take<uint8_t>(qu * (size_t) T + 64);
    if (!xg || !xu) return QWMOE_ERR_WORKSPACE;
    const bool xq_fused = T <= 16 && vg == qw::T_Q8_K && H % 256 == 0;
    ra.xq = xq_fused ? xg : nullptr;
    // grouping by logical expert (slot rows are injective for resident layers)
    Grouping G{};
    if (T <= qw::GROUP_WAVES && E <= 128) {
        // small batch: logits (+ Q8_K of x), then top-k and grouping in one launch
        qw::GroupArgs g;
        if ((rc = group_args(ar, ids, k, T, (size_t) k * 4, E, nullptr, nullptr, nullptr, G, g))) return rc;
        qw::RouterArgs rl = ra;
        rl.ids = nullptr;
        if ((rc = qw::launch_router(rl, logits, st))) return rc;
        if ((rc = qw::launch_topk_group(ra, logits, g, st))) return rc;
    } else {
        if ((rc = qw::launch_router(ra, logits, st))) return rc;
        if ((rc = group(st, ar, ids, k, T, (size_t) k * 4, E, nullptr, nullptr, nullptr, G))) return rc;
    }
    const size_t dnb1 = (size_t) F * 4, dnb2 = (size_t) F * 4 * (size_t) k;
    qw::MmidArgs mu = mmid_args(L->type_up, L->up, H, F, L->n_slots_up, L->up_nb1, L->up_nb2, xu, 1, qu, G.rows,
                                      G.active, G.active_off, G.n_active, G.max_active, L->slot_up,
                                      L->slot_up ? E : 0, upo, dnb1, dnb2, T, k * T);
    qw::MmidArgs mg = mmid_args(L->type_gate, L->gate, H, F, L->n_slots_gate, L->gate_nb1, L->gate_nb2, xg, 1, qg,
                                      G.rows, G.active, G.active_off, G.n_active, G.max_active, L->slot_gate,
                                      L->slot_gate ? E : 0, gateo, dnb1, dnb2, T, k * T);
    // x's f16 copy for the exact matrix-core form, written by the quantizing launch
    // (gate and up share it when they read one buffer)
    uint16_t* hx = nullptr;
    if (!xq_fused && xu == xg && vg == qw::T_Q8_K) {
        hx = mfma_f16_reserve(ar, mu, T);
        if (hx && qw::mmid_mfma_h_ok(mg, T)) mg.act_h = hx;
        else if (hx) {
            mu.act_h = nullptr;
            hx = nullptr;
        }
    }
    if (!xq_fused && (rc = qw::launch_quantize_act(vg, x, H, 1, T, (size_t) H * 4, (size_t) H * 4, xg, st, hx)))
        return rc;
    if (xu != xg && (rc = qw::launch_quantize_act(vu, x, H, 1, T, (size_t) H * 4, (size_t) H * 4, xu, st))) return rc;
    if (!hx && (rc = mfma_f16_prep_pair(ar, mu, mg, T, st))) return rc;
    if ((rc = mmid_launch_pair(mu, mg, st))) return rc;   // gate and up in one launch each
    const int vd = qw::vec_dot_type(L->type_down);
    const size_t qd = qwmoe_row_size(vd, F);
    uint8_t* aq = ar.take<uint8_t>(qd * (size_t) (k * T) + 64);
    if (!aq) return QWMOE_ERR_WORKSPACE;
    qw::MmidArgs md = mmid_args(L->type_down, L->down, F, H, L->n_slots_down, L->down_nb1, L->down_nb2, aq, k, qd,
                                G.rows, G.active, G.active_off, G.n_active, G.max_active, L->slot_down,
                                L->slot_down ? E : 0, ex, (size_t) H * 4, (size_t) H * 4 * (size_t) k, T, k * T, true);
    md.swiglu_gate = gateo;
    md.swiglu_up = upo;
    if (vd == qw::T_Q8_K && qw::mmid_gemv_swiglu_ok(md)) {
        // small bins: the down GEMV forms SwiGLU's Q8_K rows itself
    } else if (vd == qw::T_Q8_K) {   // SwiGLU straight into Q8_K (and the f16 copy the matrix cores read)
        md.swiglu_gate = md.swiglu_up = nullptr;
        uint16_t* ha = mfma_f16_reserve(ar, md, k * T);
        if ((rc = qw::launch_swiglu_q8K(gateo, upo, F, k * T, aq, st, ha))) return rc;
    } else {
        md.swiglu_gate = md.swiglu_up = nullptr;
        if ((rc = qw::launch_swiglu(gateo, upo, act, k * T, F, (size_t) F * 4, (size_t) F * 4, (size_t) F * 4, st)))
            return rc;
        if ((rc = qw::launch_quantize_act(vd, act, F, k, k * T, (size_t) F * 4, (size_t) F * 4 * (size_t) k, aq, st)))
            return rc;
    }
    if (!md.swiglu_gate && !md.act_h && (rc = mfma_f16_prep(ar, md, k * T, st))) return rc;
    if ((rc = mmid_launch(md, st))) return rc;
    if (rms_eps >= 0.0f && H <= 16384) {
        if ((rc = qw::launch_weighted_sum_rms(ex, w, out, x_next, H, k, T, rms_eps, st))) return rc;
    } else {
        if ((rc = qw::launch_weighted_sum(ex, w, out, H, k, T, st))) return rc;
        if (rms_eps >= 0.0f && (rc = qw::launch_rms_norm(out, x_next, H, T, rms_eps, st))) return rc;
    }
    return QWMOE_OK;
}

}  // extern "C"

struct qwmoe_decode_stack {
    qw::DecodeStackDesc d;
};

extern "C" {

int qwmoe_decode_stack_create(const qwmoe_layer* layers, int n_layer, float rms_eps, qwmoe_decode_stack** out) {
    if (!g_lib.ready) return QWMOE_ERR_NOT_INITIALIZED;
    if (!layers || n_layer <= 0 || !out || !(rms_eps >= 0.0f)) return QWMOE_ERR_INVALID_ARG;
    *out = nullptr;
    const qwmoe_layer& L0 = layers[0];
    for (int l = 0; l < n_layer; ++l) {
        const qwmoe_layer& L = layers[l];
        if (L.n_embd != L0.n_embd || L.n_expert != L0.n_expert || L.n_expert_used != L0.n_expert_used ||
            L.n_ff != L0.n_ff || L.type_gate != L0.type_gate || L.type_up != L0.type_up ||
            L.type_down != L0.type_down || L.expert_weights_scale != L0.expert_weights_scale)
            return QWMOE_ERR_INVALID_ARG;
        if (!L.router || !L.gate || !L.up || !L.down) return QWMOE_ERR_INVALID_ARG;
        if (L.type_gate != qw::T_Q4_K || L.type_up != qw::T_Q4_K) return QWMOE_ERR_UNSUPPORTED;
        if (L.gate_nb1 % 16 || L.gate_nb2 % 16 || L.up_nb1 % 16 || L.up_nb2 % 16 || ((uintptr_t) L.gate & 15) ||
            ((uintptr_t) L.up & 15) || ((uintptr_t) L.router & 15))
            return QWMOE_ERR_UNSUPPORTED;
        if (L.n_slots_gate <= 0 || L.n_slots_up <= 0 || L.n_slots_down <= 0) return QWMOE_ERR_INVALID_ARG;
    }
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return QWMOE_ERR_HIP;
    auto* s = new (std::nothrow) qwmoe_decode_stack();
    if (!s) return QWMOE_ERR_INVALID_ARG;
    qw::DecodeStackDesc& d = s->d;
    d.n_layer = n_layer;
    d.H = L0.n_embd;
    d.E = L0.n_expert;
    d.k = L0.n_expert_used;
    d.F = L0.n_ff;
    d.type_down = L0.type_down;
    d.scale = L0.expert_weights_scale;
    d.rms_eps = rms_eps;
    // The kernel with one selected expert per XCD where the shape and device
    // allow it (QWMOE_DECODE_XCD=0 selects the per-CU kernel everywhere).
    const char* xe = getenv("QWMOE_DECODE_XCD");
    const bool allow_xcd = !(xe && xe[0] == '0');
    int rc = 0;
    if (allow_xcd && qw::check_decode_xcd(d, cus) == 0) {
        d.use_xcd = 1;
        d.grid = cus;
        // the wide form loads whole down blocks per lane: Q6_K rows 4-byte, Q4_K
        // rows 16-byte aligned
        d.xcd_wide = qw::decode_xcd_wide_kernel(d) != nullptr;
        const uintptr_t dal = d.type_down == qw::T_Q6_K ? 3 : 15;
        for (int l = 0; d.xcd_wide && l < n_layer; ++l)
            if (((uintptr_t) layers[l].down | (uintptr_t) layers[l].down_nb1 | (uintptr_t) layers[l].down_nb2) & dal)
                d.use_xcd = d.xcd_wide = 0;
    }
    if (!d.use_xcd) {
        rc = qw::plan_decode_stack(d, cus);
        if (rc == 0) rc = qw::check_decode_residency(d);
    }
    if (rc) {
        delete s;
        return rc;
    }
    // one device block: layer table | act | y | logits | down outputs | status, abort
    auto r256 = [](size_t n) { return (n + 255) & ~(size_t) 255; };
    const size_t nx = d.use_xcd ? 8 : 1;   // XCD kernel: one region per XCD
    const size_t n_layers_b = sizeof(qw::DecodeLayer) * (size_t) n_layer;
    const size_t off_xa = r256(n_layers_b);
    const size_t off_xy = off_xa + r256((size_t) (d.use_xcd ? d.F : d.k * d.F) * 8 * nx);
    const size_t off_xl = off_xy + r256((size_t) d.H * 8 * nx);
    const size_t off_xd = off_xl + r256((size_t) d.E * 8 * nx);
    const size_t off_st = off_xd + (d.use_xcd ? r256((size_t) d.H * 8 * 16) : 0);
    const size_t total = off_st + 256;
    void* blk = nullptr;
    if (hipMalloc(&blk, total) != hipSuccess) {
        delete s;
        return QWMOE_ERR_HIP;
    }
    if (d.use_xcd) {
        // XCD-local exchange words may be stored with workgroup scope only when
        // the launch's workgroups are dealt to the XCDs round robin (each XCD
        // then holds one workgroup of every role; QWMOE_DECODE_XCD_LOCAL=0: never)
        const char* le = getenv("QWMOE_DECODE_XCD_LOCAL");
        int ok = 0;
        if (qw::probe_xcd_mapping((int32_t*) ((uint8_t*) blk + off_xd), d.grid, nullptr, &ok) != 0) {
            (void) hipFree(blk);
            delete s;
            return QWMOE_ERR_HIP;
        }
        d.xcd_local = (ok && !(le && le[0] == '0')) ? 1 : 0;
    }
    std::vector<qw::DecodeLayer> host((size_t) n_layer);
    for (int l = 0; l < n_layer; ++l) {
        const qwmoe_layer& L = layers[l];
        qw::DecodeLayer& D = host[(size_t) l];
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
        D.resmask = L.resmask;
        D.want = L.want_ids;
    }
    uint8_t* base = (uint8_t*) blk;
    if (hipMemset(blk, 0, total) != hipSuccess ||
        hipMemcpy(base, host.data(), n_layers_b, hipMemcpyHostToDevice) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        (void) hipFree(blk);
        delete s;
        return QWMOE_ERR_HIP;
    }
    d.dev_block = blk;
    d.layers_dev = (qw::DecodeLayer*) base;
    d.xa = (uint64_t*) (base + off_xa);
    d.xy = (uint64_t*) (base + off_xy);
    d.xl = (uint64_t*) (base + off_xl);
    d.xd = d.use_xcd ? (uint64_t*) (base + off_xd) : nullptr;
    d.status = (int32_t*) (base + off_st);
    d.abort_flag = (int32_t*) (base + off_st + 128);
    d.epoch = 1;
    *out = s;
    return QWMOE_OK;
}

int qwmoe_decode_stack_run(void* stream, qwmoe_decode_stack* s, const float* x, float* out, float* x_out,
                           int32_t* ids_out, float* weights_out) {
    if (!s || !x || !out) return QWMOE_ERR_INVALID_ARG;
    if ((ids_out == nullptr) != (weights_out == nullptr)) return QWMOE_ERR_INVALID_ARG;
    qw::DecodeStackDesc& d = s->d;
    // the launch carries its exchange epoch from the host: a captured launch would
    // replay the same epoch and accept the previous replay's words
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(S(stream), &cs) != hipSuccess) return QWMOE_ERR_HIP;
    if (cs != hipStreamCaptureStatusNone) return QWMOE_ERR_UNSUPPORTED;
    if (d.epoch > 0x7fffffffu - (uint32_t) d.n_layer) return QWMOE_ERR_UNSUPPORTED;  // epoch space exhausted
    const uint32_t e0 = d.epoch;
    d.epoch += (uint32_t) d.n_layer;
    if (d.use_xcd) return qw::launch_decode_xcd(d, x, out, x_out, ids_out, weights_out, e0, S(stream));
    return qw::launch_decode_stack(d, x, out, x_out, ids_out, weights_out, e0, S(stream));
}

int qwmoe_decode_stack_kernel(const qwmoe_decode_stack* s) {
    if (!s) return QWMOE_ERR_INVALID_ARG;
    return s->d.use_xcd ? (s->d.xcd_local ? 2 : 3) + (s->d.xcd_wide ? 2 : 0) : 1;
}

int qwmoe_decode_stack_status(void* stream, qwmoe_decode_stack* s, int32_t* status_out, int clear) {
    if (!s) return QWMOE_ERR_INVALID_ARG;
    int32_t v = 0;
    if (hipStreamSynchronize(S(stream)) != hipSuccess) return QWMOE_ERR_HIP;
    if (hipMemcpy(&v, s->d.status, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) return QWMOE_ERR_HIP;
    if (clear && hipMemset(s->d.status, 0, sizeof(int32_t)) != hipSuccess) return QWMOE_ERR_HIP;
    if (status_out) *status_out = v;
    return QWMOE_OK;
}

void qwmoe_decode_stack_free(qwmoe_decode_stack* s) {
    if (!s) return;
    (void) hipDeviceSynchronize();
    (void) hipFree(s->d.dev_block);
    delete s;
}

int qwmoe_host_argsort_desc(const float* values, int n, int32_t* idx) {
    if (!values || !idx || n < 0) return QWMOE_ERR_INVALID_ARG;
    for (int i = 0; i < n; ++i) idx[i] = i;
    qw::SortRange stack[qw::SORT_STACK];
    qw::libstdcxx_sort_desc(idx, n, values, stack);
    return QWMOE_OK;
}

}  // extern "C"
