// ggml-qwmoe.cpp -- a ggml backend whose graph_compute runs GGML_OP_MUL_MAT_ID
// nodes on libqwmoe: the drop-in for the op that ggml-hip's
// ggml_cuda_mul_mat_id (ggml-cuda/ggml-cuda.cu:1899-1960) runs in the
// reference, behind ggml's backend interface (ggml-backend-impl.h:105-227):
//
//   registry   ggml_backend_reg_i: one device per visible HIP GPU;
//   device     ggml_backend_device_i: supports_op claims the mul_mat_id nodes
//              qwmoe_ggml_supports_mul_mat_id accepts (and the no-op view
//              nodes), supports_buft only its own buffer type;
//   buffers    device memory (hipMalloc), 256-byte aligned tensors, blocking
//              set / get / memset / copy;
//   backend    graph_compute: every MUL_MAT_ID node through
//              qwmoe_ggml_mul_mat_id on the backend's stream, view nodes
//              skipped; synchronize waits for the stream.
//
// A ggml_backend_sched with this backend first and the CPU backend after it
// runs each mul_mat_id whose experts live in a QWMOE buffer here, and every
// other op (router, softmax, top-k, swiglu, the weighted sum) on the CPU, with
// the copies between them that the scheduler inserts.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-qwmoe.h"
#include "qwmoe.h"
#include "qwmoe_ggml.h"

namespace {

constexpr size_t kAlign = 256;

struct QwDevice {
    int index = 0;
    std::string name, description;
    ggml_backend_buffer_type buft{};
    ggml_backend_device dev{};
};

struct QwBackendCtx {
    int index = 0;
    hipStream_t stream = nullptr;
    std::string name;
};

struct QwBuffer {
    void* base = nullptr;
    int index = 0;
};

// ---- buffers -------------------------------------------------------------

void buf_free(ggml_backend_buffer_t b) {
    auto* c = (QwBuffer*) b->context;
    (void) hipSetDevice(c->index);
    (void) hipFree(c->base);
    delete c;
}
void* buf_base(ggml_backend_buffer_t b) { return ((QwBuffer*) b->context)->base; }
void buf_memset(ggml_backend_buffer_t b, ggml_tensor* t, uint8_t value, size_t offset, size_t size) {
    (void) hipSetDevice(((QwBuffer*) b->context)->index);
    (void) hipMemset((char*) t->data + offset, value, size);
    (void) hipDeviceSynchronize();
}
void buf_set(ggml_backend_buffer_t b, ggml_tensor* t, const void* data, size_t offset, size_t size) {
    (void) hipSetDevice(((QwBuffer*) b->context)->index);
    (void) hipMemcpy((char*) t->data + offset, data, size, hipMemcpyHostToDevice);
}
void buf_get(ggml_backend_buffer_t b, const ggml_tensor* t, void* data, size_t offset, size_t size) {
    (void) hipSetDevice(((QwBuffer*) b->context)->index);
    (void) hipMemcpy(data, (const char*) t->data + offset, size, hipMemcpyDeviceToHost);
}
bool buf_cpy(ggml_backend_buffer_t b, const ggml_tensor* src, ggml_tensor* dst) {
    if (!src->buffer || src->buffer->buft != b->buft) return false;   // the scheduler goes through the host
    (void) hipSetDevice(((QwBuffer*) b->context)->index);
    return hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice) == hipSuccess;
}
void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    auto* c = (QwBuffer*) b->context;
    (void) hipSetDevice(c->index);
    (void) hipMemset(c->base, value, b->size);
    (void) hipDeviceSynchronize();
}

const ggml_backend_buffer_i kBufferIface = {
    /* .free_buffer   = */ buf_free,
    /* .get_base      = */ buf_base,
    /* .init_tensor   = */ nullptr,
    /* .memset_tensor = */ buf_memset,
    /* .set_tensor    = */ buf_set,
    /* .get_tensor    = */ buf_get,
    /* .set_tensor_2d = */ nullptr,
    /* .get_tensor_2d = */ nullptr,
    /* .cpy_tensor    = */ buf_cpy,
    /* .clear         = */ buf_clear,
    /* .reset         = */ nullptr,
};

const char* buft_name(ggml_backend_buffer_type_t buft) { return ((QwDevice*) buft->context)->name.c_str(); }
ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    const int index = ((QwDevice*) buft->context)->index;
    void* p = nullptr;
    if (hipSetDevice(index) != hipSuccess || hipMalloc(&p, size ? size : kAlign) != hipSuccess) {
        (void) hipGetLastError();
        return nullptr;
    }
    auto* c = new QwBuffer{p, index};
    return ggml_backend_buffer_init(buft, kBufferIface, c, size);
}
size_t buft_align(ggml_backend_buffer_type_t) { return kAlign; }
bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

const ggml_backend_buffer_type_i kBuftIface = {
    /* .get_name       = */ buft_name,
    /* .alloc_buffer   = */ buft_alloc,
    /* .get_alignment  = */ buft_align,
    /* .get_max_size   = */ nullptr,
    /* .get_alloc_size = */ nullptr,
    /* .is_host        = */ buft_is_host,
};

// ---- backend (stream) ----------------------------------------------------

const char* be_name(ggml_backend_t be) { return ((QwBackendCtx*) be->context)->name.c_str(); }
void be_free(ggml_backend_t be) {
    auto* c = (QwBackendCtx*) be->context;
    (void) hipSetDevice(c->index);
    (void) hipStreamSynchronize(c->stream);
    (void) hipStreamDestroy(c->stream);
    delete c;
    delete be;
}
void be_sync(ggml_backend_t be) {
    auto* c = (QwBackendCtx*) be->context;
    (void) hipSetDevice(c->index);
    (void) hipStreamSynchronize(c->stream);
}
bool is_view(const ggml_tensor* t) {
    switch (t->op) {
        case GGML_OP_NONE:
        case GGML_OP_RESHAPE:
        case GGML_OP_VIEW:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:
            return true;
        default:
            return false;
    }
}
ggml_status be_compute(ggml_backend_t be, ggml_cgraph* g) {
    auto* c = (QwBackendCtx*) be->context;
    if (hipSetDevice(c->index) != hipSuccess) return GGML_STATUS_FAILED;
    for (int i = 0; i < ggml_graph_n_nodes(g); ++i) {
        ggml_tensor* n = ggml_graph_node(g, i);
        if (is_view(n)) continue;
        if (n->op != GGML_OP_MUL_MAT_ID) {
            fprintf(stderr, "ggml-qwmoe: op %s was scheduled here but is not supported\n", ggml_op_name(n->op));
            return GGML_STATUS_FAILED;
        }
        const int rc = qwmoe_ggml_mul_mat_id(c->stream, n, nullptr, 0);
        if (rc != QWMOE_OK) {
            fprintf(stderr, "ggml-qwmoe: mul_mat_id %s failed: %s\n", n->name, qwmoe_strerror(rc));
            return GGML_STATUS_FAILED;
        }
    }
    return GGML_STATUS_SUCCESS;
}

ggml_guid_t guid() {
    static ggml_guid g = {0x71, 0x77, 0x6d, 0x6f, 0x65, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x2d, 0x6d, 0x6d, 0x69};
    return &g;
}

const ggml_backend_i kBackendIface = {
    /* .get_name            = */ be_name,
    /* .free                = */ be_free,
    /* .set_tensor_async    = */ nullptr,
    /* .get_tensor_async    = */ nullptr,
    /* .set_tensor_2d_async = */ nullptr,
    /* .get_tensor_2d_async = */ nullptr,
    /* .cpy_tensor_async    = */ nullptr,
    /* .synchronize         = */ be_sync,
    /* .graph_plan_create   = */ nullptr,
    /* .graph_plan_free     = */ nullptr,
    /* .graph_plan_update   = */ nullptr,
    /* .graph_plan_compute  = */ nullptr,
    /* .graph_compute       = */ be_compute,
    /* .event_record        = */ nullptr,
    /* .event_wait          = */ nullptr,
    /* .graph_optimize      = */ nullptr,
};

// ---- device ----------------------------------------------------------------

const char* dev_name(ggml_backend_dev_t d) { return ((QwDevice*) d->context)->name.c_str(); }
const char* dev_desc(ggml_backend_dev_t d) { return ((QwDevice*) d->context)->description.c_str(); }
void dev_memory(ggml_backend_dev_t d, size_t* free_b, size_t* total_b) {
    *free_b = *total_b = 0;
    if (hipSetDevice(((QwDevice*) d->context)->index) == hipSuccess) (void) hipMemGetInfo(free_b, total_b);
}
enum ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }
void dev_props(ggml_backend_dev_t d, ggml_backend_dev_props* p) {
    p->name = dev_name(d);
    p->description = dev_desc(d);
    p->type = dev_type(d);
    p->device_id = nullptr;
    dev_memory(d, &p->memory_free, &p->memory_total);
    p->caps.async = false;
    p->caps.host_buffer = false;
    p->caps.buffer_from_host_ptr = false;
    p->caps.events = false;
    p->caps.mmap_support = false;
}
ggml_backend_t dev_init(ggml_backend_dev_t d, const char*) {
    auto* dv = (QwDevice*) d->context;
    if (hipSetDevice(dv->index) != hipSuccess) return nullptr;
    if (qwmoe_init(dv->index, 0) != QWMOE_OK) return nullptr;   // no-op when already initialised on this device
    auto* c = new QwBackendCtx{dv->index, nullptr, dv->name};
    if (hipStreamCreate(&c->stream) != hipSuccess) {   // a blocking stream: ordered with the buffers' copies
        delete c;
        return nullptr;
    }
    return new ggml_backend{guid(), kBackendIface, d, c};
}
ggml_backend_buffer_type_t dev_buft(ggml_backend_dev_t d) { return &((QwDevice*) d->context)->buft; }
bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor* op) {
    if (is_view(op)) return true;
    return qwmoe_ggml_supports_mul_mat_id(op) != 0;
}
bool dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) { return buft == dev_buft(d); }

const ggml_backend_device_i kDeviceIface = {
    /* .get_name             = */ dev_name,
    /* .get_description      = */ dev_desc,
    /* .get_memory           = */ dev_memory,
    /* .get_type             = */ dev_type,
    /* .get_props            = */ dev_props,
    /* .init_backend         = */ dev_init,
    /* .get_buffer_type      = */ dev_buft,
    /* .get_host_buffer_type = */ nullptr,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    /* .offload_op           = */ nullptr,
    /* .event_new            = */ nullptr,
    /* .event_free           = */ nullptr,
    /* .event_synchronize    = */ nullptr,
};

// ---- registry --------------------------------------------------------------

struct QwReg {
    std::vector<QwDevice*> devices;
    ggml_backend_reg reg{};
};

const char* reg_name(ggml_backend_reg_t) { return "QWMOE"; }
size_t reg_count(ggml_backend_reg_t r) { return ((QwReg*) r->context)->devices.size(); }
ggml_backend_dev_t reg_device(ggml_backend_reg_t r, size_t i) {
    auto* q = (QwReg*) r->context;
    return i < q->devices.size() ? &q->devices[i]->dev : nullptr;
}
void* reg_proc(ggml_backend_reg_t, const char*) { return nullptr; }

const ggml_backend_reg_i kRegIface = {
    /* .get_name         = */ reg_name,
    /* .get_device_count = */ reg_count,
    /* .get_device       = */ reg_device,
    /* .get_proc_address = */ reg_proc,
};

}  // namespace

extern "C" {

ggml_backend_reg_t ggml_backend_qwmoe_reg(void) {
    static QwReg* reg = nullptr;
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    if (!reg) {
        reg = new QwReg();
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void) hipGetLastError();
            n = 0;
        }
        for (int i = 0; i < n; ++i) {
            auto* d = new QwDevice();
            d->index = i;
            d->name = "QWMOE" + std::to_string(i);
            hipDeviceProp_t prop{};
            d->description = hipGetDeviceProperties(&prop, i) == hipSuccess ? std::string(prop.name) + " (libqwmoe)"
                                                                             : std::string("HIP GPU (libqwmoe)");
            d->buft = ggml_backend_buffer_type{kBuftIface, &d->dev, d};
            d->dev = ggml_backend_device{kDeviceIface, &reg->reg, d};
            reg->devices.push_back(d);
        }
        reg->reg = ggml_backend_reg{GGML_BACKEND_API_VERSION, kRegIface, reg};
    }
    return &reg->reg;
}

ggml_backend_t ggml_backend_qwmoe_init(int device) {
    ggml_backend_reg_t r = ggml_backend_qwmoe_reg();
    if (device < 0 || (size_t) device >= reg_count(r)) return nullptr;
    return dev_init(reg_device(r, (size_t) device), nullptr);
}

bool ggml_backend_is_qwmoe(ggml_backend_t backend) {
    return backend && memcmp(backend->guid, guid(), sizeof(ggml_guid)) == 0;
}

}  // extern "C"
