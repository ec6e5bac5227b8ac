// expert_cache.cpp -- expert slot pools in HBM fed from host memory or from the
// model file: the counterpart of ExpertCache (core/expert_cache.{h,cpp}).
//
// Policy, kept as the reference has it:
//   * one pool per (role, type, ne0, ne1) signature; each layer's role routes to
//     the pool of its own tensor's signature (core/expert_cache.cpp:128-152);
//   * every pool gets the same residency fraction f = budget / total expert
//     bytes (capped at 1), n_slots = (int) (f * n_layers_of_pool * n_expert)
//     clamped to [n_used, n_layers_of_pool * n_expert] (cpp:155-186);
//   * key = layer * n_expert + expert; an access counts as a use of the key and,
//     on a hit, stamps the slot with the next tick; a miss installs into the
//     slot with the oldest stamp, the lowest such slot (empty slots have stamp
//     0), evicting its key (cpp:374-410, 709-721);
//   * slot_of rows hold 0 for absent experts (cpp:694-697).
//
// Mechanics, MI355X-first:
//   * pools and the device row table [3][n_layer][n_expert] are one hipMalloc;
//   * host tier: misses go to their slots asynchronously on the cache's stream,
//     as the RAM tier's ggml_backend_tensor_set_async (cpp:355-364): runs of
//     consecutive slabs by the copy engine, scattered slabs of pinned sources by
//     one gather kernel launch per call (slab_copy.hip);
//   * file tier: misses of one call are read with pread by a persistent worker
//     pool into one of two pinned 64 MiB stages while the other stage's slabs
//     are being copied (cpp:412-687 reads into a pinned batch and uploads it);
//   * after every call that changed residency, the changed span of the row table
//     is copied to the device through a pinned stage on the same stream, so a
//     kernel launched next on that stream reads rows and slabs that agree.
#include <fcntl.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "../../include/qwmoe.h"
#include "qw_slab_copy.hpp"

namespace {

constexpr int N_ROLE = 3;
constexpr size_t STAGE_BYTES = 64ull << 20;  // one file-tier staging batch (cpp:652)
constexpr int DEFAULT_IO_THREADS = 8;        // cpp:100

size_t align256(size_t n) { return (n + 255) & ~(size_t) 255; }

// Bytes of one row of ne0 elements for the expert types the kernels take.
int64_t row_bytes(int type, int64_t ne0) {
    switch (type) {
        case QWMOE_TYPE_Q4_K: return ne0 % 256 ? -1 : ne0 / 256 * 144;
        case QWMOE_TYPE_Q6_K: return ne0 % 256 ? -1 : ne0 / 256 * 210;
        case QWMOE_TYPE_Q8_0: return ne0 % 32 ? -1 : ne0 / 32 * 34;
        default: return -1;
    }
}

// One slot pool: the experts of every layer whose tensors of one role share a
// type and shape.  Keys are layer * n_expert + expert.  Residency is two
// tables kept in step: what each slot holds, and where each key is.
struct Pool {
    int role = 0, type = 0;
    int64_t ne0 = 0, ne1 = 0;
    size_t slab = 0;
    int n_layers = 0;
    int n_slots = 0;
    uint8_t* dev = nullptr;                   // [n_slots][slab]
    std::vector<int32_t> holder;              // [n_slots]: the key a slot holds, -1 when empty
    std::vector<uint64_t> stamp;              // [n_slots]: tick of its last install or hit, 0 never
    std::vector<int32_t> home;                // [n_layer * n_expert]: the slot holding a key, -1 absent
    int n_held = 0;                           // keys resident
    std::map<int, uint64_t> uses;             // accesses per key (ascending keys: the profile file's order)

    bool holds(int key) const { return home[(size_t) key] >= 0; }
    // The slot a newly admitted key takes: the one used longest ago (never-used
    // slots first), the lowest index among equal stamps.
    int oldest() const { return (int) (std::min_element(stamp.begin(), stamp.end()) - stamp.begin()); }
};

struct Source {
    const uint8_t* host = nullptr;            // host tier
    const uint8_t* mapped = nullptr;          // its device-visible address when it is pinned, else null
    int file = -1;                            // file tier: index into the cache's files
    uint64_t offset = 0;
};

struct Job {
    int pool, role, layer, expert, slot;
};

// A fixed set of threads that run one indexed task at a time: run(n, f) calls
// f(0..n-1) spread over the workers and the caller, and returns when all are done.
class Workers {
  public:
    explicit Workers(int n) {
        for (int i = 1; i < n; ++i) threads_.emplace_back([this] { loop(); });
    }
    ~Workers() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }
    void run(int n, const std::function<void(int)>& f) {
        if (n <= 0) return;
        if (threads_.empty() || n == 1) {
            for (int i = 0; i < n; ++i) f(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            task_ = &f;
            n_ = n;
            next_.store(0);
            active_ = (int) threads_.size();
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return active_ == 0; });
        task_ = nullptr;
    }

  private:
    void work() {
        for (int i; (i = next_.fetch_add(1)) < n_;) (*task_)(i);
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
            std::lock_guard<std::mutex> lk(mu_);
            if (--active_ == 0) done_cv_.notify_one();
        }
    }
    std::vector<std::thread> threads_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int)>* task_ = nullptr;
    int n_ = 0, active_ = 0;
    std::atomic<int> next_{0};
    uint64_t gen_ = 0;
    bool stop_ = false;
};

bool pread_all(int fd, void* dst, size_t n, uint64_t off) {
    uint8_t* p = (uint8_t*) dst;
    while (n > 0) {
        const ssize_t got = pread(fd, p, n, (off_t) off);
        if (got <= 0) return false;
        p += got;
        n -= (size_t) got;
        off += (uint64_t) got;
    }
    return true;
}

}  // namespace

struct qwmoe_expert_cache {
    int n_layer = 0, n_expert = 0, n_used = 0;
    bool dry = false;
    hipStream_t stream = nullptr;
    std::vector<Pool> pools;
    std::vector<int> layer_pool[N_ROLE];
    std::vector<Source> src[N_ROLE];
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::vector<int32_t> rows;                // [3][n_layer][n_expert], 0 = absent
    size_t dirty_lo = SIZE_MAX, dirty_hi = 0; // changed span of rows
    uint64_t tick = 0;                        // use counter behind the slots' stamps
    qwmoe_expert_cache_stats stats{};
    std::vector<Job> jobs;                    // installs whose slab is not fetched yet
    uint8_t* dev_block = nullptr;
    int32_t* dev_rows = nullptr;
    std::vector<void*> owned_host;            // pinned copies of the expert tensors (GGUF host tier)
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
    bool stage_pending[2] = {false, false};
    int stage_next = 0;
    void* row_stage[2] = {nullptr, nullptr};
    hipEvent_t row_ev[2] = {nullptr, nullptr};
    bool row_pending[2] = {false, false};
    int row_next = 0;
    int io_threads = DEFAULT_IO_THREADS;
    bool copy_engine_only = false;            // QWMOE_CACHE_COPY_ENGINE: no slab gather kernel
    int32_t* run_ids_dev = nullptr;           // run_layer: router ids / weights (device) and their read-back
    float* run_w_dev = nullptr;
    int32_t* run_ids_host = nullptr;
    size_t run_cap = 0;
    Workers* workers = nullptr;

    ~qwmoe_expert_cache() {
        if (!dry) (void) hipStreamSynchronize(stream);
        delete workers;
        for (int b = 0; b < 2; ++b) {
            if (stage_ev[b]) (void) hipEventDestroy(stage_ev[b]);
            if (stage[b]) (void) hipHostFree(stage[b]);
            if (row_ev[b]) (void) hipEventDestroy(row_ev[b]);
            if (row_stage[b]) (void) hipHostFree(row_stage[b]);
        }
        for (void* p : owned_host) (void) hipHostFree(p);
        if (run_ids_dev) (void) hipFree(run_ids_dev);
        if (run_ids_host) (void) hipHostFree(run_ids_host);
        for (int fd : fds)
            if (fd >= 0) close(fd);
        if (dev_block) (void) hipFree(dev_block);
    }

    // The run paths' router ids / weights (device) and id read-back (pinned
    // host), grown to hold n ids; the old buffers are freed once the stream has
    // finished with them.
    int grow_run_buffers(size_t n) {
        if (n <= run_cap) return QWMOE_OK;
        if (hipStreamSynchronize(stream) != hipSuccess) return QWMOE_ERR_HIP;
        if (run_ids_dev) (void) hipFree(run_ids_dev);
        if (run_ids_host) (void) hipHostFree(run_ids_host);
        run_ids_dev = nullptr;
        run_ids_host = nullptr;
        run_w_dev = nullptr;
        run_cap = 0;
        if (hipMalloc(&run_ids_dev, n * 8) != hipSuccess ||
            hipHostMalloc(&run_ids_host, n * 4, hipHostMallocDefault) != hipSuccess) {
            (void) hipGetLastError();
            return QWMOE_ERR_HIP;
        }
        run_w_dev = (float*) (run_ids_dev + n);
        run_cap = n;
        return QWMOE_OK;
    }

    size_t row_index(int role, int layer) const { return ((size_t) role * n_layer + layer) * (size_t) n_expert; }
    Pool& pool_of(int role, int layer) { return pools[layer_pool[role][layer]]; }
    const Pool& pool_of(int role, int layer) const { return pools[layer_pool[role][layer]]; }

    void set_row(int role, int key, int32_t slot) {
        const size_t i = (size_t) role * n_layer * n_expert + (size_t) key;
        rows[i] = slot;
        dirty_lo = std::min(dirty_lo, i);
        dirty_hi = std::max(dirty_hi, i + 1);
    }

    // Puts `key` in the oldest slot of pool pi; the key held there before (if
    // any) is evicted and its slot-table row cleared.  The policy of the
    // reference's install / reserve_victim (core/expert_cache.cpp:374-410); the
    // slab itself is fetched later, with the other jobs of the call.
    int admit(int pi, int key) {
        Pool& p = pools[pi];
        const int s = p.oldest();
        if (const int prev = p.holder[(size_t) s]; prev >= 0) {
            p.home[(size_t) prev] = -1;
            --p.n_held;
            set_row(p.role, prev, 0);
            stats.evictions++;
        }
        p.holder[(size_t) s] = key;
        p.home[(size_t) key] = s;
        ++p.n_held;
        p.stamp[(size_t) s] = ++tick;
        set_row(p.role, key, s);
        return s;
    }

    int install(int role, int layer, int expert) {
        const int pi = layer_pool[role][layer];
        const int slot = admit(pi, layer * n_expert + expert);
        jobs.push_back({pi, role, layer, expert, slot});
        return slot;
    }

    // The slot of (role, layer, expert), admitting it on a miss; every lookup
    // counts as a use, a hit renews the slot's stamp (slot_for,
    // core/expert_cache.cpp:709-721).
    int slot_for(int role, int layer, int expert) {
        const int key = layer * n_expert + expert;
        Pool& p = pool_of(role, layer);
        ++p.uses[key];
        const int s = p.home[(size_t) key];
        if (s < 0) {
            stats.misses++;
            return install(role, layer, expert);
        }
        stats.hits++;
        p.stamp[(size_t) s] = ++tick;
        return s;
    }

    // Slot counts: every pool keeps the same share of its experts, the budget
    // over the bytes of all experts of all pools (at most all of them), and at
    // least n_used slots but never more than it has experts
    // (core/expert_cache.cpp:155-186).  Slots start empty.
    void size_pools(size_t budget, int n_used) {
        size_t all_bytes = 0;
        for (const Pool& p : pools) all_bytes += p.slab * (size_t) p.n_layers * (size_t) n_expert;
        const double share = all_bytes == 0 ? 1.0 : std::min(1.0, (double) budget / (double) all_bytes);
        for (Pool& p : pools) {
            const int experts = p.n_layers * n_expert;
            p.n_slots = std::min(experts, std::max(n_used, (int) (share * experts)));
            p.holder.assign((size_t) p.n_slots, -1);
            p.stamp.assign((size_t) p.n_slots, 0);
            p.home.assign((size_t) n_layer * (size_t) n_expert, -1);
            p.n_held = 0;
        }
    }

    // Forgets installs whose fetch failed: their slots are empty again.
    void drop(const Job& j) {
        Pool& p = pools[j.pool];
        const int key = j.layer * n_expert + j.expert;
        if (p.home[(size_t) key] >= 0) --p.n_held;
        p.home[(size_t) key] = -1;
        p.holder[(size_t) j.slot] = -1;
        p.stamp[(size_t) j.slot] = 0;
        set_row(p.role, key, 0);
    }

    // Host tier.  Installs whose source slabs and destination slots are both
    // consecutive go as one copy-engine copy per run (a cold fill of a layer's
    // experts is one copy per role).  The remaining single slabs of a pool go
    // through the slab gather kernel, up to 64 per launch, when their source is
    // pinned (device-mapped) memory; otherwise one copy each.
    int fetch_host(std::vector<Job> js) {
        std::sort(js.begin(), js.end(), [](const Job& a, const Job& b) {
            return a.pool != b.pool ? a.pool < b.pool : a.slot < b.slot;
        });
        qw::SlabCopyArgs g{};
        int g_pool = -1;
        auto flush_gather = [&]() -> int {
            if (g.n == 0) return QWMOE_OK;
            const int rc = qw::launch_slab_copy(g, stream);
            g.n = 0;
            return rc == 0 ? QWMOE_OK : QWMOE_ERR_HIP;
        };
        for (size_t i = 0; i < js.size();) {
            size_t n = 1;
            while (i + n < js.size() && js[i + n].pool == js[i].pool && js[i + n].layer == js[i].layer &&
                   js[i + n].slot == js[i].slot + (int) n && js[i + n].expert == js[i].expert + (int) n)
                ++n;
            const Pool& p = pools[js[i].pool];
            const Source& sr = src[js[i].role][js[i].layer];
            uint8_t* dst = p.dev + (size_t) js[i].slot * p.slab;
            const size_t off = (size_t) js[i].expert * p.slab;
            if (n == 1 && sr.mapped && !copy_engine_only && p.slab % 16 == 0) {
                if (g_pool != js[i].pool || g.n == (uint32_t) qw::SLAB_COPY_MAX) {
                    const int rc = flush_gather();
                    if (rc != QWMOE_OK) return rc;
                    g_pool = js[i].pool;
                    g.bytes = p.slab;
                }
                g.src[g.n] = sr.mapped + off;
                g.dst[g.n] = dst;
                g.n++;
            } else if (hipMemcpyAsync(dst, sr.host + off, n * p.slab, hipMemcpyHostToDevice, stream) != hipSuccess) {
                return QWMOE_ERR_HIP;
            }
            i += n;
        }
        return flush_gather();
    }

    int ensure_stage() {
        if (stage[0]) return QWMOE_OK;
        for (int b = 0; b < 2; ++b)
            if (hipHostMalloc(&stage[b], STAGE_BYTES, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&stage_ev[b], hipEventDisableTiming) != hipSuccess)
                return QWMOE_ERR_HIP;
        return QWMOE_OK;
    }

    // File tier: batches of slabs fill one pinned stage with parallel preads,
    // then go to their slots by async copies; the next batch fills the other
    // stage meanwhile.  A stage is reused only after its copies completed.
    int fetch_file(const std::vector<Job>& js, size_t* n_done) {
        *n_done = 0;
        int rc = ensure_stage();
        if (rc != QWMOE_OK) return rc;
        size_t i0 = 0;
        while (i0 < js.size()) {
            // batch: as many slabs as fit one stage
            size_t bytes = 0, i1 = i0;
            std::vector<size_t> at;
            while (i1 < js.size() && (i1 == i0 || bytes + pools[js[i1].pool].slab <= STAGE_BYTES)) {
                at.push_back(bytes);
                bytes += align256(pools[js[i1].pool].slab);
                ++i1;
            }
            if (bytes > STAGE_BYTES) return QWMOE_ERR_UNSUPPORTED;  // a slab larger than a stage
            const int b = stage_next;
            stage_next ^= 1;
            if (stage_pending[b]) {
                if (hipEventSynchronize(stage_ev[b]) != hipSuccess) return QWMOE_ERR_HIP;
                stage_pending[b] = false;
            }
            uint8_t* base = (uint8_t*) stage[b];
            std::atomic<bool> ok{true};
            workers->run((int) (i1 - i0), [&](int k) {
                const Job& j = js[i0 + k];
                const Source& s = src[j.role][j.layer];
                const size_t slab = pools[j.pool].slab;
                if (!pread_all(fds[s.file], base + at[k], slab, s.offset + (uint64_t) j.expert * slab))
                    ok.store(false);
            });
            if (!ok.load()) return QWMOE_ERR_IO;
            for (size_t k = i0; k < i1; ++k) {
                const Pool& p = pools[js[k].pool];
                if (hipMemcpyAsync(p.dev + (size_t) js[k].slot * p.slab, base + at[k - i0], p.slab,
                                   hipMemcpyHostToDevice, stream) != hipSuccess)
                    return QWMOE_ERR_HIP;
            }
            if (hipEventRecord(stage_ev[b], stream) != hipSuccess) return QWMOE_ERR_HIP;
            stage_pending[b] = true;
            *n_done = i1;
            i0 = i1;
        }
        return QWMOE_OK;
    }

    int upload_rows() {
        if (dirty_lo >= dirty_hi) return QWMOE_OK;
        const size_t lo = dirty_lo, n = dirty_hi - dirty_lo;
        dirty_lo = SIZE_MAX;
        dirty_hi = 0;
        const int b = row_next;
        row_next ^= 1;
        if (row_pending[b]) {
            if (hipEventSynchronize(row_ev[b]) != hipSuccess) return QWMOE_ERR_HIP;
            row_pending[b] = false;
        }
        int32_t* st = (int32_t*) row_stage[b];
        memcpy(st, rows.data() + lo, n * sizeof(int32_t));
        if (hipMemcpyAsync(dev_rows + lo, st, n * sizeof(int32_t), hipMemcpyHostToDevice, stream) != hipSuccess ||
            hipEventRecord(row_ev[b], stream) != hipSuccess)
            return QWMOE_ERR_HIP;
        row_pending[b] = true;
        return QWMOE_OK;
    }

    // Fetches every pending install, then brings the device rows up to date.
    int flush() {
        std::vector<Job> js;
        js.swap(jobs);
        for (const Job& j : js) stats.fetch_bytes += pools[j.pool].slab;
        if (dry) {
            dirty_lo = SIZE_MAX;
            dirty_hi = 0;
            return QWMOE_OK;
        }
        if (js.empty()) return upload_rows();
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<Job> host_jobs, file_jobs;
        for (const Job& j : js) (src[j.role][j.layer].host ? host_jobs : file_jobs).push_back(j);
        int rc = fetch_host(host_jobs);
        size_t done = 0;
        if (rc == QWMOE_OK && !file_jobs.empty()) rc = fetch_file(file_jobs, &done);
        if (rc != QWMOE_OK) {
            // the slabs of unfinished installs never arrived: make them absent
            for (size_t k = done; k < file_jobs.size(); ++k) {
                drop(file_jobs[k]);
                stats.fetch_bytes -= pools[file_jobs[k].pool].slab;
            }
            if (host_jobs.size() && rc == QWMOE_ERR_HIP)
                for (const Job& j : host_jobs) drop(j);
        }
        stats.fetch_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        const int rc2 = upload_rows();
        return rc != QWMOE_OK ? rc : rc2;
    }
};

namespace {

// The device-visible address of host range [p, p + n) when all of it is
// pinned host memory of one allocation, else null (pageable memory is copied by
// the copy engine only).
const uint8_t* device_mapped(const void* p, size_t n) {
    hipPointerAttribute_t a0, a1;
    if (hipPointerGetAttributes(&a0, p) != hipSuccess) {
        (void) hipGetLastError();
        return nullptr;
    }
    const uint8_t* last = (const uint8_t*) p + (n - 1);
    if (hipPointerGetAttributes(&a1, last) != hipSuccess) {
        (void) hipGetLastError();
        return nullptr;
    }
    if (a0.type != hipMemoryTypeHost || a1.type != hipMemoryTypeHost || !a0.devicePointer || !a1.devicePointer)
        return nullptr;
    if ((const uint8_t*) a1.devicePointer != (const uint8_t*) a0.devicePointer + (n - 1)) return nullptr;
    if ((uintptr_t) a0.devicePointer % 16 != 0) return nullptr;
    return (const uint8_t*) a0.devicePointer;
}

bool valid_role_layer(const qwmoe_expert_cache* c, int role, int layer) {
    return c && role >= 0 && role < N_ROLE && layer >= 0 && layer < c->n_layer;
}

int build(qwmoe_expert_cache* c, void* stream, int n_layer, int n_expert, const qwmoe_expert_src* srcs,
          const qwmoe_expert_cache_config* cfg) {
    c->n_layer = n_layer;
    c->n_expert = n_expert;
    c->n_used = cfg->n_used;
    c->dry = (cfg->flags & QWMOE_CACHE_DRY_RUN) != 0;
    c->stream = c->dry ? nullptr : (hipStream_t) stream;
    c->io_threads = cfg->io_threads > 0 ? std::min(cfg->io_threads, 64) : DEFAULT_IO_THREADS;
    c->copy_engine_only = (cfg->flags & QWMOE_CACHE_COPY_ENGINE) != 0;

    // Pools, numbered in order of first appearance (roles outer, layers inner):
    // one per (role, type, ne0, ne1); layer_pool[r][l] names the pool of layer
    // l's tensor of role r.
    std::map<std::tuple<int, int, int64_t, int64_t>, int> pool_by_shape;
    bool any_file = false;
    for (int r = 0; r < N_ROLE; ++r) {
        c->layer_pool[r].assign(n_layer, -1);
        c->src[r].assign(n_layer, Source{});
        for (int il = 0; il < n_layer; ++il) {
            const qwmoe_expert_src& s = srcs[(size_t) r * n_layer + il];
            const int64_t rb = row_bytes(s.type, s.ne0);
            if (rb <= 0 || s.ne1 <= 0) return QWMOE_ERR_UNSUPPORTED;
            const size_t slab = (size_t) rb * (size_t) s.ne1;
            if (s.host) {
                c->src[r][il].host = (const uint8_t*) s.host;
                if (!c->dry) c->src[r][il].mapped = device_mapped(s.host, slab * (size_t) n_expert);
            } else if (s.path) {
                any_file = true;
                int fi = -1;
                for (size_t k = 0; k < c->paths.size(); ++k)
                    if (c->paths[k] == s.path) fi = (int) k;
                if (fi < 0) {
                    fi = (int) c->paths.size();
                    c->paths.emplace_back(s.path);
                    c->fds.push_back(-1);
                }
                c->src[r][il].file = fi;
                c->src[r][il].offset = s.file_offset;
            } else {
                return QWMOE_ERR_INVALID_ARG;
            }
            const auto [at, fresh] = pool_by_shape.try_emplace({r, s.type, s.ne0, s.ne1}, (int) c->pools.size());
            if (fresh) {
                Pool np;
                np.role = r;
                np.type = s.type;
                np.ne0 = s.ne0;
                np.ne1 = s.ne1;
                np.slab = slab;
                c->pools.push_back(std::move(np));
            }
            c->pools[(size_t) at->second].n_layers++;
            c->layer_pool[r][il] = at->second;
        }
    }
    c->size_pools(cfg->vram_budget, cfg->n_used);
    size_t dev_bytes = 0;
    std::vector<size_t> pool_off(c->pools.size());
    for (size_t k = 0; k < c->pools.size(); ++k) {
        pool_off[k] = dev_bytes;
        dev_bytes += align256(c->pools[k].slab * (size_t) c->pools[k].n_slots);
    }
    c->rows.assign((size_t) N_ROLE * n_layer * n_expert, 0);
    if (c->dry) return QWMOE_OK;

    const size_t rows_off = dev_bytes;
    dev_bytes += align256(c->rows.size() * sizeof(int32_t));
    if (hipMalloc(&c->dev_block, dev_bytes) != hipSuccess) {
        c->dev_block = nullptr;
        (void) hipGetLastError();
        return QWMOE_ERR_HIP;
    }
    for (size_t k = 0; k < c->pools.size(); ++k) c->pools[k].dev = c->dev_block + pool_off[k];
    c->dev_rows = (int32_t*) (c->dev_block + rows_off);
    for (int b = 0; b < 2; ++b)
        if (hipHostMalloc(&c->row_stage[b], c->rows.size() * sizeof(int32_t), hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&c->row_ev[b], hipEventDisableTiming) != hipSuccess)
            return QWMOE_ERR_HIP;
    // empty slots read as zeros (a run that speculates on absent experts reads
    // slot 0 of a pool: zeros or a real slab, never stale bytes), and every row
    // starts at the sentinel on the device too
    if (hipMemsetAsync(c->dev_block, 0, rows_off, c->stream) != hipSuccess) return QWMOE_ERR_HIP;
    c->dirty_lo = 0;
    c->dirty_hi = c->rows.size();
    int rc = c->upload_rows();
    if (rc != QWMOE_OK) return rc;
    if (any_file) {
        for (size_t k = 0; k < c->paths.size(); ++k) {
            c->fds[k] = open(c->paths[k].c_str(), O_RDONLY | O_CLOEXEC);
            if (c->fds[k] < 0) return QWMOE_ERR_IO;
        }
        c->workers = new Workers(c->io_threads);
    }
    return QWMOE_OK;
}

const char* role_name(int r) { return r == 0 ? "gate" : r == 1 ? "up" : "down"; }

}  // namespace

extern "C" {

int qwmoe_expert_cache_create(void* stream, int n_layer, int n_expert, const qwmoe_expert_src* srcs,
                              const qwmoe_expert_cache_config* cfg, qwmoe_expert_cache** out) {
    if (!out) return QWMOE_ERR_INVALID_ARG;
    *out = nullptr;
    if (!srcs || !cfg || n_layer <= 0 || n_expert <= 0 || cfg->n_used <= 0 || cfg->n_used > n_expert ||
        (int64_t) n_layer * n_expert > INT32_MAX / 2)
        return QWMOE_ERR_INVALID_ARG;
    auto* c = new (std::nothrow) qwmoe_expert_cache();
    if (!c) return QWMOE_ERR_WORKSPACE;
    int rc;
    try {
        rc = build(c, stream, n_layer, n_expert, srcs, cfg);
    } catch (...) {
        rc = QWMOE_ERR_WORKSPACE;
    }
    if (rc != QWMOE_OK) {
        delete c;
        return rc;
    }
    *out = c;
    return QWMOE_OK;
}

int qwmoe_expert_cache_create_gguf(void* stream, const qwmoe_gguf* g, int tier, const qwmoe_expert_cache_config* cfg,
                                   qwmoe_expert_cache** out) {
    if (!out) return QWMOE_ERR_INVALID_ARG;
    *out = nullptr;
    if (!g || !cfg || (tier != 0 && tier != 1)) return QWMOE_ERR_INVALID_ARG;
    qwmoe_moe_hparams hp;
    int rc = qwmoe_gguf_moe_hparams(g, &hp);
    if (rc != QWMOE_OK) return rc;
    if (hp.n_layer <= 0 || hp.n_expert <= 0) return QWMOE_ERR_FORMAT;
    const bool dry = (cfg->flags & QWMOE_CACHE_DRY_RUN) != 0;
    std::vector<qwmoe_expert_src> srcs((size_t) N_ROLE * hp.n_layer);
    std::vector<std::string> paths(srcs.size());
    std::vector<qwmoe_gguf_tensor_info> infos(srcs.size());
    for (int r = 0; r < N_ROLE; ++r)
        for (int il = 0; il < hp.n_layer; ++il) {
            char name[64];
            snprintf(name, sizeof(name), "blk.%d.ffn_%s_exps.weight", il, role_name(r));
            qwmoe_gguf_tensor_info& ti = infos[(size_t) r * hp.n_layer + il];
            if (qwmoe_gguf_find_tensor(g, name, &ti) < 0) return QWMOE_ERR_FORMAT;  // cpp:136-137 throws
            if (ti.n_dims != 3 || ti.ne[2] != hp.n_expert) return QWMOE_ERR_FORMAT;
            const char* path = nullptr;
            if (qwmoe_gguf_shard_path(g, ti.shard, &path) != QWMOE_OK) return QWMOE_ERR_FORMAT;
            paths[(size_t) r * hp.n_layer + il] = path;
            qwmoe_expert_src& s = srcs[(size_t) r * hp.n_layer + il];
            s.type = ti.type;
            s.ne0 = ti.ne[0];
            s.ne1 = ti.ne[1];
            s.host = nullptr;
            s.path = paths[(size_t) r * hp.n_layer + il].c_str();
            s.file_offset = ti.file_offset;
            const int64_t rb = row_bytes(ti.type, ti.ne[0]);
            if (rb <= 0 || (uint64_t) rb * (uint64_t) ti.ne[1] * (uint64_t) hp.n_expert != ti.nbytes)
                return QWMOE_ERR_UNSUPPORTED;
        }
    qwmoe_expert_cache_config c2 = *cfg;
    if (c2.n_used == 0) c2.n_used = hp.n_expert_used;
    std::vector<void*> owned;
    if (tier == 0 && !dry) {
        // host tier: every expert tensor once into pinned memory (the pinned
        // CPU expert buffers of core/model.cpp:249-255)
        Workers w(cfg->io_threads > 0 ? std::min(cfg->io_threads, 64) : DEFAULT_IO_THREADS);
        auto free_owned = [&] {
            for (void* p : owned) (void) hipHostFree(p);
        };
        struct Piece {
            size_t t;
            uint64_t off, n;
        };
        std::vector<Piece> pieces;
        std::vector<int> fds(srcs.size(), -1);
        for (size_t t = 0; t < srcs.size(); ++t) {
            void* p = nullptr;
            if (hipHostMalloc(&p, infos[t].nbytes, hipHostMallocDefault) != hipSuccess) {
                (void) hipGetLastError();
                free_owned();
                return QWMOE_ERR_HIP;
            }
            owned.push_back(p);
            srcs[t].host = p;
            for (uint64_t o = 0; o < infos[t].nbytes; o += 8ull << 20)
                pieces.push_back({t, o, std::min<uint64_t>(8ull << 20, infos[t].nbytes - o)});
        }
        std::vector<int> shard_fd;
        std::map<std::string, int> fd_of;
        for (size_t t = 0; t < srcs.size(); ++t) {
            auto it = fd_of.find(paths[t]);
            if (it == fd_of.end()) {
                const int fd = open(paths[t].c_str(), O_RDONLY | O_CLOEXEC);
                if (fd < 0) {
                    for (auto& kv : fd_of) close(kv.second);
                    free_owned();
                    return QWMOE_ERR_IO;
                }
                it = fd_of.emplace(paths[t], fd).first;
            }
            fds[t] = it->second;
        }
        std::atomic<bool> ok{true};
        w.run((int) pieces.size(), [&](int i) {
            const Piece& pc = pieces[i];
            if (!pread_all(fds[pc.t], (uint8_t*) owned[pc.t] + pc.off, pc.n, infos[pc.t].file_offset + pc.off))
                ok.store(false);
        });
        for (auto& kv : fd_of) close(kv.second);
        if (!ok.load()) {
            free_owned();
            return QWMOE_ERR_IO;
        }
    } else if (tier == 0) {
        // a dry run reads nothing: any non-null host pointer marks the tier
        static const uint8_t none = 0;
        for (auto& s : srcs) s.host = &none;
    }
    rc = qwmoe_expert_cache_create(stream, hp.n_layer, hp.n_expert, srcs.data(), &c2, out);
    if (rc != QWMOE_OK) {
        for (void* p : owned) (void) hipHostFree(p);
        return rc;
    }
    (*out)->owned_host = std::move(owned);
    return QWMOE_OK;
}

void qwmoe_expert_cache_free(qwmoe_expert_cache* c) { delete c; }

int qwmoe_expert_cache_n_pools(const qwmoe_expert_cache* c) {
    return c ? (int) c->pools.size() : QWMOE_ERR_INVALID_ARG;
}

int qwmoe_expert_cache_pool_info(const qwmoe_expert_cache* c, int pool, int32_t* role, int32_t* type, int64_t* ne0,
                                 int64_t* ne1, int64_t* n_slots, uint64_t* slab_bytes, void** base) {
    if (!c || pool < 0 || pool >= (int) c->pools.size()) return QWMOE_ERR_INVALID_ARG;
    const Pool& p = c->pools[pool];
    if (role) *role = p.role;
    if (type) *type = p.type;
    if (ne0) *ne0 = p.ne0;
    if (ne1) *ne1 = p.ne1;
    if (n_slots) *n_slots = p.n_slots;
    if (slab_bytes) *slab_bytes = p.slab;
    if (base) *base = p.dev;
    return QWMOE_OK;
}

int qwmoe_expert_cache_pool_of(const qwmoe_expert_cache* c, int role, int layer) {
    if (!valid_role_layer(c, role, layer)) return QWMOE_ERR_INVALID_ARG;
    return c->layer_pool[role][layer];
}

int qwmoe_expert_cache_min_slots(const qwmoe_expert_cache* c) {
    if (!c) return QWMOE_ERR_INVALID_ARG;
    int m = c->pools.empty() ? 0 : c->pools[0].n_slots;
    for (const Pool& p : c->pools) m = std::min(m, p.n_slots);
    return m;
}

int qwmoe_expert_cache_capacity(const qwmoe_expert_cache* c, int layer) {
    if (!valid_role_layer(c, 0, layer)) return QWMOE_ERR_INVALID_ARG;
    int m = c->pools[c->layer_pool[0][layer]].n_slots;
    for (int r = 1; r < N_ROLE; ++r) m = std::min(m, c->pools[c->layer_pool[r][layer]].n_slots);
    return m;
}

int qwmoe_expert_cache_ensure(qwmoe_expert_cache* c, int layer, const int32_t* ids, int n, int32_t* slot_gate,
                              int32_t* slot_up, int32_t* slot_down) {
    if (!valid_role_layer(c, 0, layer) || n < 0 || (n > 0 && !ids)) return QWMOE_ERR_INVALID_ARG;
    std::vector<int> distinct;
    for (int i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= c->n_expert) return QWMOE_ERR_INVALID_ARG;
        distinct.push_back(ids[i]);
    }
    std::sort(distinct.begin(), distinct.end());
    distinct.erase(std::unique(distinct.begin(), distinct.end()), distinct.end());
    if ((int) distinct.size() > qwmoe_expert_cache_capacity(c, layer)) return QWMOE_ERR_INVALID_ARG;
    int32_t* outs[N_ROLE] = {slot_gate, slot_up, slot_down};
    // token-major, role-minor, as both of the reference's paths walk (cpp:799-830)
    for (int i = 0; i < n; ++i)
        for (int r = 0; r < N_ROLE; ++r) {
            const int s = c->slot_for(r, layer, ids[i]);
            if (outs[r]) outs[r][i] = s;
        }
    return c->flush();
}

int qwmoe_expert_cache_ensure_resident(qwmoe_expert_cache* c, int layer, int expert) {
    if (!valid_role_layer(c, 0, layer) || expert < 0 || expert >= c->n_expert) return QWMOE_ERR_INVALID_ARG;
    const int key = layer * c->n_expert + expert;
    for (int r = 0; r < N_ROLE; ++r) {
        if (!c->pool_of(r, layer).holds(key)) {
            c->stats.misses++;
            c->install(r, layer, expert);
        }
    }
    return c->flush();
}

int qwmoe_expert_cache_touch(qwmoe_expert_cache* c, int role, int layer, int expert) {
    if (!valid_role_layer(c, role, layer) || expert < 0 || expert >= c->n_expert) return QWMOE_ERR_INVALID_ARG;
    Pool& p = c->pool_of(role, layer);
    const int key = layer * c->n_expert + expert;
    const int s = p.home[(size_t) key];
    if (s < 0) return QWMOE_OK;
    ++p.uses[key];
    p.stamp[(size_t) s] = ++c->tick;
    c->stats.hits++;
    return QWMOE_OK;
}

int qwmoe_expert_cache_verify(qwmoe_expert_cache* c, const int32_t* ids, int n_layer, int k, int touch) {
    if (!c || !ids || n_layer < 0 || n_layer > c->n_layer || k < 0) return QWMOE_ERR_INVALID_ARG;
    int missing = 0;
    for (int l = 0; l < n_layer; ++l)
        for (int i = 0; i < k; ++i) {
            const int e = ids[(size_t) l * k + i];
            if (e < 0 || e >= c->n_expert) return QWMOE_ERR_INVALID_ARG;
            for (int r = 0; r < N_ROLE; ++r)
                if (!c->pool_of(r, l).holds(l * c->n_expert + e)) {
                    ++missing;
                    break;
                }
        }
    if (missing == 0 && touch)
        for (int l = 0; l < n_layer; ++l)
            for (int i = 0; i < k; ++i)
                for (int r = 0; r < N_ROLE; ++r) qwmoe_expert_cache_touch(c, r, l, ids[(size_t) l * k + i]);
    return missing;
}

int qwmoe_expert_cache_resmask(const qwmoe_expert_cache* c, int floor_res, float* mask, float* mask_dev) {
    if (!c || !mask) return QWMOE_ERR_INVALID_ARG;
    // a layer masked to fewer than n_used residents would let top-k pick masked
    // (absent) experts, which read slot 0's weights: the floor is at least n_used,
    // as the reference's (core/runtime.cpp:2896-2898)
    if (floor_res < c->n_used) floor_res = c->n_used;
    if (mask_dev && c->dry) return QWMOE_ERR_UNSUPPORTED;
    bool complete = true;
    for (int l = 0; l < c->n_layer; ++l) {
        float* row = mask + (size_t) l * c->n_expert;
        int n_res = 0;
        for (int e = 0; e < c->n_expert; ++e) {
            const int key = l * c->n_expert + e;
            bool res = true;
            for (int r = 0; r < N_ROLE; ++r) res = res && c->pool_of(r, l).holds(key);
            row[e] = res ? 0.0f : -INFINITY;
            n_res += res ? 1 : 0;
        }
        if (n_res < floor_res) {   // palette too thin: the layer routes unmasked
            for (int e = 0; e < c->n_expert; ++e) row[e] = 0.0f;
            complete = false;
        }
    }
    if (mask_dev) {
        const size_t bytes = sizeof(float) * (size_t) c->n_layer * (size_t) c->n_expert;
        if (hipMemcpyAsync(mask_dev, mask, bytes, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
            hipStreamSynchronize(c->stream) != hipSuccess)
            return QWMOE_ERR_HIP;
    }
    return complete ? 1 : 0;
}

int qwmoe_expert_cache_refill(qwmoe_expert_cache* c, const int32_t* sel, const int32_t* want, int n_layer, int k,
                              int budget, int* cursor) {
    if (!c || !sel || !want || !cursor || n_layer != c->n_layer || k <= 0 || *cursor < 0 || *cursor >= n_layer)
        return QWMOE_ERR_INVALID_ARG;
    for (int i = 0; i < n_layer * k; ++i)
        if (sel[i] < 0 || sel[i] >= c->n_expert || want[i] < 0 || want[i] >= c->n_expert) return QWMOE_ERR_INVALID_ARG;
    if (budget <= 0) return 0;
    // the actually used experts are touched first, so the refill's evictions
    // land on stale entries
    for (int l = 0; l < n_layer; ++l)
        for (int i = 0; i < k; ++i)
            for (int r = 0; r < N_ROLE; ++r) qwmoe_expert_cache_touch(c, r, l, sel[(size_t) l * k + i]);
    int fetched = 0;
    for (int step = 0; step < n_layer && budget > 0; ++step) {
        const int l = (*cursor + step) % n_layer;
        for (int i = 0; i < k && budget > 0; ++i) {
            const int e = want[(size_t) l * k + i];
            const int key = l * c->n_expert + e;
            bool res = true;
            for (int r = 0; r < N_ROLE; ++r) res = res && c->pool_of(r, l).holds(key);
            if (res) continue;
            const int rc = qwmoe_expert_cache_ensure_resident(c, l, e);
            if (rc < 0) return rc;
            --budget;
            ++fetched;
        }
    }
    *cursor = (*cursor + 1) % n_layer;
    return fetched;
}

int qwmoe_expert_cache_resident(const qwmoe_expert_cache* c, int role, int layer, int expert) {
    if (!valid_role_layer(c, role, layer) || expert < 0 || expert >= c->n_expert) return QWMOE_ERR_INVALID_ARG;
    const Pool& p = c->pools[c->layer_pool[role][layer]];
    return p.holds(layer * c->n_expert + expert) ? 1 : 0;
}

const int32_t* qwmoe_expert_cache_slot_of_row(const qwmoe_expert_cache* c, int role, int layer) {
    if (!valid_role_layer(c, role, layer)) return nullptr;
    return c->rows.data() + c->row_index(role, layer);
}

const int32_t* qwmoe_expert_cache_device_row(const qwmoe_expert_cache* c, int role, int layer) {
    if (!valid_role_layer(c, role, layer) || !c->dev_rows) return nullptr;
    return c->dev_rows + c->row_index(role, layer);
}

int qwmoe_expert_cache_layer(const qwmoe_expert_cache* c, int layer, qwmoe_layer* L) {
    if (!valid_role_layer(c, 0, layer) || !L) return QWMOE_ERR_INVALID_ARG;
    if (c->dry) return QWMOE_ERR_UNSUPPORTED;
    const Pool* p[N_ROLE];
    for (int r = 0; r < N_ROLE; ++r) p[r] = &c->pools[c->layer_pool[r][layer]];
    L->type_gate = p[0]->type;
    L->type_up = p[1]->type;
    L->type_down = p[2]->type;
    L->gate = p[0]->dev;
    L->up = p[1]->dev;
    L->down = p[2]->dev;
    L->gate_nb1 = (size_t) row_bytes(p[0]->type, p[0]->ne0);
    L->up_nb1 = (size_t) row_bytes(p[1]->type, p[1]->ne0);
    L->down_nb1 = (size_t) row_bytes(p[2]->type, p[2]->ne0);
    L->gate_nb2 = p[0]->slab;
    L->up_nb2 = p[1]->slab;
    L->down_nb2 = p[2]->slab;
    L->n_slots_gate = p[0]->n_slots;
    L->n_slots_up = p[1]->n_slots;
    L->n_slots_down = p[2]->n_slots;
    L->slot_gate = qwmoe_expert_cache_device_row(c, 0, layer);
    L->slot_up = qwmoe_expert_cache_device_row(c, 1, layer);
    L->slot_down = qwmoe_expert_cache_device_row(c, 2, layer);
    return QWMOE_OK;
}

int qwmoe_expert_cache_get_stats(const qwmoe_expert_cache* c, qwmoe_expert_cache_stats* out) {
    if (!c || !out) return QWMOE_ERR_INVALID_ARG;
    *out = c->stats;
    return QWMOE_OK;
}

int qwmoe_expert_cache_save_profile(const qwmoe_expert_cache* c, const char* path) {
    if (!c || !path) return QWMOE_ERR_INVALID_ARG;
    FILE* f = fopen(path, "wb");
    if (!f) return QWMOE_ERR_IO;
    fprintf(f, "QWENEXPCACHE 1\n%d %d\n", c->n_layer, c->n_expert);
    for (const Pool& p : c->pools)
        for (const auto& kv : p.uses)
            fprintf(f, "%d %d %d %llu\n", p.role, kv.first / c->n_expert, kv.first % c->n_expert,
                    (unsigned long long) kv.second);
    const bool ok = fclose(f) == 0;
    return ok ? QWMOE_OK : QWMOE_ERR_IO;
}

int qwmoe_expert_cache_load_prefetch(qwmoe_expert_cache* c, const char* path, uint64_t* n_prefetched) {
    if (n_prefetched) *n_prefetched = 0;
    if (!c || !path) return QWMOE_ERR_INVALID_ARG;
    FILE* f = fopen(path, "rb");
    if (!f) return QWMOE_OK;  // missing profile: cold start
    int ver = 0, nl = 0, ne = 0;
    if (fscanf(f, "QWENEXPCACHE %d", &ver) != 1 || ver != 1 || fscanf(f, "%d %d", &nl, &ne) != 2 ||
        nl != c->n_layer || ne != c->n_expert) {
        fclose(f);
        return QWMOE_OK;  // incompatible profile: cold start
    }
    struct Ent {
        int role, layer, expert;
        unsigned long long count;
    };
    std::vector<Ent> ents;
    int r, l, e;
    unsigned long long cnt;
    while (fscanf(f, "%d %d %d %llu", &r, &l, &e, &cnt) == 4)
        if (r >= 0 && r < N_ROLE && l >= 0 && l < c->n_layer && e >= 0 && e < c->n_expert) ents.push_back({r, l, e, cnt});
    fclose(f);
    std::stable_sort(ents.begin(), ents.end(), [](const Ent& a, const Ent& b) { return a.count > b.count; });
    uint64_t n = 0;
    for (const Ent& en : ents) {
        Pool& p = c->pool_of(en.role, en.layer);
        if (p.n_held >= p.n_slots) continue;
        const int key = en.layer * c->n_expert + en.expert;
        if (p.holds(key)) continue;
        c->install(en.role, en.layer, en.expert);
        n++;
    }
    const int rc = c->flush();
    if (n_prefetched) *n_prefetched = n;
    return rc;
}

int qwmoe_expert_cache_run_layer(qwmoe_expert_cache* c, int layer, const qwmoe_layer* L, const float* x, int64_t T,
                                 float* out, float rms_eps, float* x_next, int32_t* ids_out, float* weights_out) {
    if (!valid_role_layer(c, 0, layer) || !L || !x || !out || T < 0) return QWMOE_ERR_INVALID_ARG;
    if (c->dry) return QWMOE_ERR_UNSUPPORTED;
    if (L->n_expert != c->n_expert || L->n_expert_used <= 0 || T > 64) return QWMOE_ERR_INVALID_ARG;
    if (T == 0) return QWMOE_OK;
    const size_t n = (size_t) T * (size_t) L->n_expert_used;
    int rc = c->grow_run_buffers(std::max(n, (size_t) 64 * (size_t) L->n_expert_used));
    if (rc != QWMOE_OK) return rc;
    // the router's selection, read back (the reference's ensure_layer)
    rc = qwmoe_router_topk(c->stream, L->router, x, L->n_embd, L->n_expert, L->n_expert_used, T,
                               (size_t) L->n_embd * 4, 6.103515625e-5f, L->expert_weights_scale, c->run_ids_dev,
                               c->run_w_dev, nullptr);
    if (rc != QWMOE_OK) return rc;
    if (hipMemcpyAsync(c->run_ids_host, c->run_ids_dev, n * 4, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return QWMOE_ERR_HIP;
    if ((rc = qwmoe_expert_cache_ensure(c, layer, c->run_ids_host, (int) n, nullptr, nullptr, nullptr)) != QWMOE_OK)
        return rc;
    qwmoe_layer Lc = *L;
    if ((rc = qwmoe_expert_cache_layer(c, layer, &Lc)) != QWMOE_OK) return rc;
    return qwmoe_ffn_layer(c->stream, &Lc, x, T, out, rms_eps, x_next, ids_out, weights_out);
}

int qwmoe_plan_slices(const int32_t* sel, int T, int n_used, int n_expert, int cap, int max_slice, int32_t* slices,
                      int* n_slices, int32_t* union_list, int* n_union) {
    if (!sel || !slices || !n_slices || T < 0 || n_used <= 0 || n_expert <= 0 || cap < n_used)
        return QWMOE_ERR_INVALID_ARG;
    for (int64_t i = 0; i < (int64_t) T * n_used; ++i)
        if (sel[i] < 0 || sel[i] >= n_expert) return QWMOE_ERR_INVALID_ARG;
    if (max_slice < 1) max_slice = 1024;
    std::vector<uint8_t> in_slice((size_t) n_expert, 0), in_union((size_t) n_expert, 0);
    int ns = 0, nu = 0, distinct = 0, t0 = 0;
    for (int t = 0; t < T; ++t) {
        const int32_t* row = sel + (size_t) t * n_used;
        int fresh = 0;
        for (int j = 0; j < n_used; ++j) {
            if (!in_union[(size_t) row[j]]) {
                in_union[(size_t) row[j]] = 1;
                if (union_list) union_list[nu] = row[j];
                ++nu;
            }
            if (!in_slice[(size_t) row[j]]) {
                in_slice[(size_t) row[j]] = 1;
                ++fresh;
            }
        }
        // token t would take the slice past the pool's capacity (or its length
        // past max_slice): the slice ends before t, and t opens the next one
        if ((distinct + fresh > cap || t - t0 >= max_slice) && t > t0) {
            slices[2 * ns] = t0;
            slices[2 * ns + 1] = t - t0;
            ++ns;
            std::fill(in_slice.begin(), in_slice.end(), 0);
            fresh = 0;
            for (int j = 0; j < n_used; ++j)
                if (!in_slice[(size_t) row[j]]) {
                    in_slice[(size_t) row[j]] = 1;
                    ++fresh;
                }
            distinct = 0;
            t0 = t;
        }
        distinct += fresh;
    }
    if (T > 0) {
        slices[2 * ns] = t0;
        slices[2 * ns + 1] = T - t0;
        ++ns;
    }
    *n_slices = ns;
    if (n_union) *n_union = nu;
    return QWMOE_OK;
}

int qwmoe_expert_cache_plan_slices(const qwmoe_expert_cache* c, int layer, const int32_t* sel, int T, int max_slice,
                                   int32_t* slices, int* n_slices) {
    if (!valid_role_layer(c, 0, layer)) return QWMOE_ERR_INVALID_ARG;
    const int cap = std::max(c->n_used, qwmoe_expert_cache_capacity(c, layer) - 8);
    return qwmoe_plan_slices(sel, T, c->n_used, c->n_expert, cap, max_slice, slices, n_slices, nullptr, nullptr);
}

int qwmoe_expert_cache_run_batch(qwmoe_expert_cache* c, int layer, const qwmoe_layer* L, const float* x, int64_t T,
                                 float* out, float rms_eps, float* x_next, int32_t* ids_out, float* weights_out,
                                 int max_slice, int* n_slices_out) {
    if (!valid_role_layer(c, 0, layer) || !L || !x || !out || T < 0 || T > INT32_MAX / 64) return QWMOE_ERR_INVALID_ARG;
    if (c->dry) return QWMOE_ERR_UNSUPPORTED;
    if (L->n_expert != c->n_expert || L->n_expert_used != c->n_used) return QWMOE_ERR_INVALID_ARG;
    if (n_slices_out) *n_slices_out = 0;
    if (T == 0) return QWMOE_OK;
    const int k = (int) L->n_expert_used;
    const int64_t H = L->n_embd;
    int rc = c->grow_run_buffers((size_t) T * (size_t) k);
    if (rc != QWMOE_OK) return rc;
    // the router's selection for the whole batch, read back
    rc = qwmoe_router_topk(c->stream, L->router, x, H, L->n_expert, k, T, (size_t) H * 4, 6.103515625e-5f,
                           L->expert_weights_scale, c->run_ids_dev, c->run_w_dev, nullptr);
    if (rc != QWMOE_OK) return rc;
    const size_t n = (size_t) T * (size_t) k;
    if (hipMemcpyAsync(c->run_ids_host, c->run_ids_dev, n * 4, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return QWMOE_ERR_HIP;
    std::vector<int32_t> slices((size_t) (2 * T));
    int ns = 0;
    if ((rc = qwmoe_expert_cache_plan_slices(c, layer, c->run_ids_host, (int) T, max_slice, slices.data(), &ns)))
        return rc;
    // each slice: its experts made resident (evictions land after the previous
    // slice's kernels on the same stream), then the layer on its tokens
    for (int s = 0; s < ns; ++s) {
        const int t0 = slices[(size_t) (2 * s)], len = slices[(size_t) (2 * s + 1)];
        if ((rc = qwmoe_expert_cache_ensure(c, layer, c->run_ids_host + (size_t) t0 * k, len * k, nullptr, nullptr,
                                            nullptr)) != QWMOE_OK)
            return rc;
        qwmoe_layer Lc = *L;
        if ((rc = qwmoe_expert_cache_layer(c, layer, &Lc)) != QWMOE_OK) return rc;
        const size_t o = (size_t) t0 * (size_t) H, oi = (size_t) t0 * (size_t) k;
        if ((rc = qwmoe_ffn_layer(c->stream, &Lc, x + o, len, out + o, rms_eps, x_next ? x_next + o : nullptr,
                                  ids_out ? ids_out + oi : nullptr, weights_out ? weights_out + oi : nullptr)))
            return rc;
    }
    if (n_slices_out) *n_slices_out = ns;
    return QWMOE_OK;
}

int qwmoe_expert_cache_sync(qwmoe_expert_cache* c) {
    if (!c) return QWMOE_ERR_INVALID_ARG;
    if (c->dry) return QWMOE_OK;
    return hipStreamSynchronize(c->stream) == hipSuccess ? QWMOE_OK : QWMOE_ERR_HIP;
}

}  // extern "C"
