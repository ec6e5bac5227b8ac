// gguf.cpp -- GGUF (v2, v3) metadata reader and MoE layer loader.
//
// Replaces, for the MoE FFN path, what the reference does to get expert weights
// from disk: gguf_init_from_file with no_alloc per shard (ggml/src/gguf.cpp:451-906)
// and Model::load's unified tensor map with per-tensor (shard file, absolute
// offset) sources (core/model.cpp:444-502; shard naming 400-423), plus the
// hparam lookups of Model::load_hparams (core/model.cpp:504-548, helper
// semantics core/gguf_util.cpp:21-51).  Only metadata is read at open; a layer's
// router and expert tensors are streamed into caller-owned device memory on
// request, through two pinned staging buffers.
//
// File layout (little endian): "GGUF", u32 version, i64 n_tensors, i64 n_kv;
// n_kv x {string key, i32 type, value}; n_tensors x {string name, u32 n_dims,
// i64 ne[n_dims], i32 ggml type, u64 offset}; padding to the alignment
// ("general.alignment", u32, default 32); the data section, tensor i at
// data + offset_i, each padded to the alignment and stored in info order.
// A string is u64 length + bytes; an array is i32 element type + u64 count +
// elements.  The checks below are the format's own rules as the reference
// enforces them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <new>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qwmoe.h"

namespace {

enum : int {
    GG_U8 = 0, GG_I8 = 1, GG_U16 = 2, GG_I16 = 3, GG_U32 = 4, GG_I32 = 5, GG_F32 = 6, GG_BOOL = 7,
    GG_STRING = 8, GG_ARRAY = 9, GG_U64 = 10, GG_I64 = 11, GG_F64 = 12, GG_COUNT = 13
};
size_t value_size(int t) {
    switch (t) {
        case GG_U8: case GG_I8: case GG_BOOL: return 1;
        case GG_U16: case GG_I16: return 2;
        case GG_U32: case GG_I32: case GG_F32: return 4;
        case GG_U64: case GG_I64: case GG_F64: return 8;
        default: return 0;
    }
}

// ggml tensor types: (elements per block, bytes per block); 0 = removed / unknown.
// The block layouts are ggml's (ggml/include/ggml.h:389-433).
struct TypeTrait { int blck; int bytes; };
constexpr TypeTrait TYPE_TRAITS[] = {
    {1, 4}, {1, 2}, {32, 18}, {32, 20}, {0, 0}, {0, 0}, {32, 22}, {32, 24}, {32, 34}, {32, 36},   // 0..9
    {256, 84}, {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292},                        // 10..15 K-quants
    {256, 66}, {256, 74}, {256, 98}, {256, 50}, {32, 18}, {256, 110}, {256, 82}, {256, 136},      // 16..23 IQ
    {1, 1}, {1, 2}, {1, 4}, {1, 8}, {1, 8}, {256, 56}, {1, 2},                                     // 24..30
    {0, 0}, {0, 0}, {0, 0}, {256, 54}, {256, 66}, {0, 0}, {0, 0}, {0, 0},                          // 31..38
    {32, 17}, {64, 36}, {128, 18}, {64, 18},                                                       // 39..42
};
constexpr int N_GGML_TYPES = (int) (sizeof(TYPE_TRAITS) / sizeof(TYPE_TRAITS[0]));
constexpr size_t MAX_NAME = 64;                    // ggml's tensor name buffer, incl. the terminator
constexpr uint64_t MAX_STRING = 1ull << 30;
constexpr uint64_t MAX_ARRAY = 1ull << 30;

struct KV {
    std::string key;
    int type = -1;           // GG_ARRAY for arrays
    int arr_type = -1;       // element type of an array
    uint64_t n = 1;          // element count (1 for a scalar)
    std::vector<uint8_t> raw;          // fixed-size scalar / array payload
    std::vector<std::string> strs;     // string scalar / array
};

struct Tensor {
    std::string name;
    int type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;     // in the data section
    uint64_t nbytes = 0;
    int shard = 0;
};

struct Shard {
    std::string path;
    uint32_t version = 0;
    size_t alignment = 32;
    uint64_t data_offset = 0;
    uint64_t file_size = 0;
};

// Bounded sequential reader over a file.
struct Reader {
    FILE* f = nullptr;
    uint64_t size = 0, pos = 0;
    bool bytes(void* dst, uint64_t n) {
        if (n > size - pos) return false;
        if (n && fread(dst, 1, (size_t) n, f) != n) return false;
        pos += n;
        return true;
    }
    template <class T> bool get(T& v) { return bytes(&v, sizeof(T)); }
    bool str(std::string& s) {
        uint64_t n = 0;
        if (!get(n) || n > MAX_STRING || n > size - pos) return false;
        s.resize((size_t) n);
        return bytes(&s[0], n);
    }
    bool seek(uint64_t p) {
        if (p > size || fseeko(f, (off_t) p, SEEK_SET) != 0) return false;
        pos = p;
        return true;
    }
};

}  // namespace

struct qwmoe_gguf {
    std::vector<Shard> shards;
    std::vector<KV> kv;                               // first shard's
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;                      // all shards, in file order
    std::unordered_map<std::string, size_t> tensor_index;
    // loader state (created on the first load)
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    size_t stage_bytes = 0;
};

namespace {

constexpr size_t STAGE_BYTES = 16u << 20;

bool read_value(Reader& r, int type, uint64_t n, KV& kv) {
    if (type == GG_STRING) {
        kv.strs.resize((size_t) n);
        for (uint64_t i = 0; i < n; ++i)
            if (!r.str(kv.strs[i])) return false;
        return true;
    }
    const size_t es = value_size(type);
    if (es == 0) return false;                        // an array of arrays, or an unknown type
    if (n > (r.size - r.pos) / es) return false;
    kv.raw.resize((size_t) (n * es));
    return r.bytes(kv.raw.data(), n * es);
}

// Parses one file's metadata into g (kv only when keep_kv).  Returns a status.
int parse_shard(qwmoe_gguf& g, const std::string& path, int shard_idx, bool keep_kv) {
    Reader r;
    r.f = fopen(path.c_str(), "rb");
    if (!r.f) return QWMOE_ERR_IO;
    struct Closer { FILE* f; ~Closer() { fclose(f); } } closer{r.f};
    if (fseeko(r.f, 0, SEEK_END) != 0) return QWMOE_ERR_IO;
    r.size = (uint64_t) ftello(r.f);
    if (fseeko(r.f, 0, SEEK_SET) != 0) return QWMOE_ERR_IO;

    Shard sh;
    sh.path = path;
    char magic[4];
    if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) return QWMOE_ERR_FORMAT;
    if (!r.get(sh.version)) return QWMOE_ERR_FORMAT;
    // version 0 is invalid, 1 is no longer supported, a version with zero low bits
    // is another endianness, and versions above 3 are unknown
    if (sh.version == 0 || sh.version == 1 || (sh.version & 0xFFFFu) == 0 || sh.version > 3) return QWMOE_ERR_FORMAT;
    int64_t n_tensors = 0, n_kv = 0;
    if (!r.get(n_tensors) || !r.get(n_kv)) return QWMOE_ERR_FORMAT;
    // every key needs at least 12 bytes, every tensor info at least 24
    if (n_tensors < 0 || n_kv < 0 || (uint64_t) n_kv > r.size / 12 || (uint64_t) n_tensors > r.size / 24)
        return QWMOE_ERR_FORMAT;

    std::vector<KV> kvs;
    std::unordered_map<std::string, size_t> kidx;
    for (int64_t i = 0; i < n_kv; ++i) {
        KV kv;
        if (!r.str(kv.key) || kv.key.empty() || kidx.count(kv.key)) return QWMOE_ERR_FORMAT;
        int32_t type = -1;
        if (!r.get(type)) return QWMOE_ERR_FORMAT;
        kv.type = type;
        if (type == GG_ARRAY) {
            int32_t at = -1;
            uint64_t n = 0;
            if (!r.get(at) || !r.get(n) || n > MAX_ARRAY) return QWMOE_ERR_FORMAT;
            kv.arr_type = at;
            kv.n = n;
            if (at < 0 || at >= GG_COUNT || at == GG_ARRAY || !read_value(r, at, n, kv)) return QWMOE_ERR_FORMAT;
        } else {
            if (type < 0 || type >= GG_COUNT || !read_value(r, type, 1, kv)) return QWMOE_ERR_FORMAT;
        }
        kidx[kv.key] = kvs.size();
        kvs.push_back(std::move(kv));
    }
    auto al = kidx.find("general.alignment");
    if (al != kidx.end()) {
        const KV& a = kvs[al->second];
        if (a.type != GG_U32) return QWMOE_ERR_FORMAT;
        uint32_t v;
        memcpy(&v, a.raw.data(), 4);
        if (v == 0 || (v & (v - 1)) != 0) return QWMOE_ERR_FORMAT;
        sh.alignment = v;
    }

    std::vector<Tensor> ts;
    for (int64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        t.shard = shard_idx;
        if (!r.str(t.name) || t.name.size() >= MAX_NAME) return QWMOE_ERR_FORMAT;
        uint32_t n_dims = 0;
        if (!r.get(n_dims) || n_dims > 4) return QWMOE_ERR_FORMAT;
        t.n_dims = (int) n_dims;
        for (uint32_t j = 0; j < n_dims; ++j)
            if (!r.get(t.ne[j]) || t.ne[j] < 0) return QWMOE_ERR_FORMAT;
        int32_t type = -1;
        if (!r.get(type) || type < 0 || type >= N_GGML_TYPES) return QWMOE_ERR_FORMAT;
        t.type = type;
        const TypeTrait tt = TYPE_TRAITS[type];
        if (tt.blck == 0 || t.ne[0] % tt.blck != 0) return QWMOE_ERR_FORMAT;
        // element count and byte size representable
        uint64_t nel = 1;
        for (int j = 0; j < 4; ++j) {
            if (t.ne[j] == 0) { nel = 0; break; }
            if (nel > (uint64_t) INT64_MAX / (uint64_t) t.ne[j]) return QWMOE_ERR_FORMAT;
            nel *= (uint64_t) t.ne[j];
        }
        const uint64_t nblk = nel / (uint64_t) tt.blck;
        if (nblk > UINT64_MAX / (uint64_t) tt.bytes) return QWMOE_ERR_FORMAT;
        t.nbytes = nblk * (uint64_t) tt.bytes;
        if (!r.get(t.offset)) return QWMOE_ERR_FORMAT;
        ts.push_back(std::move(t));
    }
    // the data section starts at the next aligned position; tensors follow in info
    // order, each padded to the alignment
    const uint64_t a = sh.alignment;
    sh.data_offset = (r.pos + a - 1) / a * a;
    if (n_tensors > 0 && sh.data_offset > r.size) return QWMOE_ERR_FORMAT;
    uint64_t expect = 0;
    for (const Tensor& t : ts) {
        if (t.offset != expect) return QWMOE_ERR_FORMAT;
        const uint64_t padded = (t.nbytes + a - 1) / a * a;
        if (padded < t.nbytes || UINT64_MAX - expect < padded) return QWMOE_ERR_FORMAT;
        expect += padded;
    }
    sh.file_size = r.size;

    for (Tensor& t : ts) {
        if (g.tensor_index.count(t.name)) return QWMOE_ERR_FORMAT;   // a name in two shards
        g.tensor_index[t.name] = g.tensors.size();
        g.tensors.push_back(std::move(t));
    }
    if (keep_kv) {
        g.kv = std::move(kvs);
        g.kv_index = std::move(kidx);
    }
    g.shards.push_back(sh);
    return QWMOE_OK;
}

// "<prefix>-00001-of-00003.gguf" -> the three shard paths; anything else -> itself.
std::vector<std::string> shard_paths(const std::string& path) {
    auto digits = [&](size_t p, int n) {
        for (int i = 0; i < n; ++i)
            if (p + i >= path.size() || path[p + i] < '0' || path[p + i] > '9') return false;
        return true;
    };
    const size_t op = path.rfind("-of-");
    if (op != std::string::npos && op >= 6 && path[op - 6] == '-' && digits(op - 5, 5) && digits(op + 4, 5) &&
        path.compare(op + 9, std::string::npos, ".gguf") == 0) {
        const int total = std::stoi(path.substr(op + 4, 5));
        if (total >= 1) {
            std::vector<std::string> out;
            const std::string prefix = path.substr(0, op - 5);
            char buf[32];
            for (int i = 1; i <= total; ++i) {
                snprintf(buf, sizeof(buf), "%05d-of-%05d.gguf", i, total);
                out.push_back(prefix + buf);
            }
            return out;
        }
    }
    return {path};
}

const KV* find_kv(const qwmoe_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second];
}

template <class T> T scalar(const KV& kv) {
    T v;
    memcpy(&v, kv.raw.data(), sizeof(T));
    return v;
}

void fill_info(const qwmoe_gguf* g, const Tensor& t, qwmoe_gguf_tensor_info* out) {
    memset(out, 0, sizeof(*out));
    snprintf(out->name, sizeof(out->name), "%s", t.name.c_str());
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int j = 0; j < 4; ++j) out->ne[j] = t.ne[j];
    out->offset = t.offset;
    out->file_offset = g->shards[t.shard].data_offset + t.offset;
    out->nbytes = t.nbytes;
    out->shard = t.shard;
}

uint64_t row_bytes(const Tensor& t) { return (uint64_t) t.ne[0] / TYPE_TRAITS[t.type].blck * TYPE_TRAITS[t.type].bytes; }

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct LayerTensors {
    const Tensor* t[4];   // router, gate, up, down
};

int layer_tensors(const qwmoe_gguf* g, int il, const qwmoe_moe_hparams& hp, LayerTensors& lt) {
    static const char* fmt[4] = {"blk.%d.ffn_gate_inp.weight", "blk.%d.ffn_gate_exps.weight", "blk.%d.ffn_up_exps.weight",
                                 "blk.%d.ffn_down_exps.weight"};
    for (int j = 0; j < 4; ++j) {
        char name[MAX_NAME];
        snprintf(name, sizeof(name), fmt[j], il);
        auto it = g->tensor_index.find(name);
        if (it == g->tensor_index.end()) return QWMOE_ERR_INVALID_ARG;
        lt.t[j] = &g->tensors[it->second];
    }
    const int64_t H = hp.n_embd, E = hp.n_expert, F = hp.n_ff_exp;
    const Tensor& r = *lt.t[0];
    if (r.type != QWMOE_TYPE_F32 || r.ne[0] != H || r.ne[1] != E || r.ne[2] != 1 || r.ne[3] != 1) return QWMOE_ERR_FORMAT;
    for (int j = 1; j < 4; ++j) {
        const Tensor& m = *lt.t[j];
        const int64_t K = j < 3 ? H : F, N = j < 3 ? F : H;
        if (m.ne[0] != K || m.ne[1] != N || m.ne[2] != E || m.ne[3] != 1) return QWMOE_ERR_FORMAT;
        if (m.type != QWMOE_TYPE_Q4_K && m.type != QWMOE_TYPE_Q6_K && m.type != QWMOE_TYPE_Q8_0) return QWMOE_ERR_UNSUPPORTED;
    }
    return QWMOE_OK;
}

}  // namespace

extern "C" {

int qwmoe_gguf_open(const char* path, qwmoe_gguf** out) {
    if (!path || !out) return QWMOE_ERR_INVALID_ARG;
    *out = nullptr;
    qwmoe_gguf* g = new (std::nothrow) qwmoe_gguf();
    if (!g) return QWMOE_ERR_WORKSPACE;
    const std::vector<std::string> paths = shard_paths(path);
    for (size_t i = 0; i < paths.size(); ++i) {
        int rc;
        try {
            rc = parse_shard(*g, paths[i], (int) i, i == 0);
        } catch (...) {
            rc = QWMOE_ERR_WORKSPACE;
        }
        if (rc != QWMOE_OK) {
            delete g;
            return rc;
        }
    }
    *out = g;
    return QWMOE_OK;
}

void qwmoe_gguf_close(qwmoe_gguf* g) {
    if (!g) return;
    for (int i = 0; i < 2; ++i) {
        if (g->ev[i]) (void) hipEventDestroy(g->ev[i]);
        if (g->stage[i]) (void) hipHostFree(g->stage[i]);
    }
    delete g;
}

int qwmoe_gguf_n_shards(const qwmoe_gguf* g) { return g ? (int) g->shards.size() : QWMOE_ERR_INVALID_ARG; }

int qwmoe_gguf_shard_info(const qwmoe_gguf* g, int shard, uint32_t* version, uint64_t* alignment, uint64_t* data_offset) {
    if (!g || shard < 0 || shard >= (int) g->shards.size()) return QWMOE_ERR_INVALID_ARG;
    const Shard& s = g->shards[shard];
    if (version) *version = s.version;
    if (alignment) *alignment = s.alignment;
    if (data_offset) *data_offset = s.data_offset;
    return QWMOE_OK;
}

int qwmoe_gguf_shard_path(const qwmoe_gguf* g, int shard, const char** out) {
    if (!g || !out || shard < 0 || shard >= (int) g->shards.size()) return QWMOE_ERR_INVALID_ARG;
    *out = g->shards[shard].path.c_str();
    return QWMOE_OK;
}

int qwmoe_gguf_n_kv(const qwmoe_gguf* g) { return g ? (int) g->kv.size() : QWMOE_ERR_INVALID_ARG; }

int qwmoe_gguf_find_key(const qwmoe_gguf* g, const char* key) {
    if (!g || !key) return QWMOE_ERR_INVALID_ARG;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? -1 : (int) it->second;
}

int qwmoe_gguf_kv(const qwmoe_gguf* g, int idx, const char** key, int32_t* type, int32_t* arr_type, uint64_t* n,
                  const void** data) {
    if (!g || idx < 0 || idx >= (int) g->kv.size()) return QWMOE_ERR_INVALID_ARG;
    const KV& kv = g->kv[idx];
    if (key) *key = kv.key.c_str();
    if (type) *type = kv.type;
    if (arr_type) *arr_type = kv.arr_type;
    if (n) *n = kv.n;
    if (data) *data = kv.raw.empty() ? nullptr : kv.raw.data();
    return QWMOE_OK;
}

int qwmoe_gguf_kv_str(const qwmoe_gguf* g, int idx, uint64_t i, const char** out) {
    if (!g || !out || idx < 0 || idx >= (int) g->kv.size()) return QWMOE_ERR_INVALID_ARG;
    const KV& kv = g->kv[idx];
    if (i >= kv.strs.size()) return QWMOE_ERR_INVALID_ARG;
    *out = kv.strs[i].c_str();
    return QWMOE_OK;
}

int qwmoe_gguf_get_u32(const qwmoe_gguf* g, const char* key, uint32_t def, uint32_t* out) {
    if (!g || !key || !out) return QWMOE_ERR_INVALID_ARG;
    const KV* kv = find_kv(g, key);
    *out = def;
    if (!kv) return QWMOE_OK;
    switch (kv->type) {
        case GG_U32: *out = scalar<uint32_t>(*kv); break;
        case GG_I32: *out = (uint32_t) scalar<int32_t>(*kv); break;
        case GG_U64: *out = (uint32_t) scalar<uint64_t>(*kv); break;
        case GG_I64: *out = (uint32_t) scalar<int64_t>(*kv); break;
        default: break;
    }
    return QWMOE_OK;
}

int qwmoe_gguf_get_f32(const qwmoe_gguf* g, const char* key, float def, float* out) {
    if (!g || !key || !out) return QWMOE_ERR_INVALID_ARG;
    const KV* kv = find_kv(g, key);
    *out = def;
    if (!kv) return QWMOE_OK;
    if (kv->type == GG_F32) *out = scalar<float>(*kv);
    else if (kv->type == GG_F64) *out = (float) scalar<double>(*kv);
    return QWMOE_OK;
}

int qwmoe_gguf_get_str(const qwmoe_gguf* g, const char* key, const char* def, const char** out) {
    if (!g || !key || !out) return QWMOE_ERR_INVALID_ARG;
    const KV* kv = find_kv(g, key);
    *out = (kv && kv->type == GG_STRING) ? kv->strs[0].c_str() : def;
    return QWMOE_OK;
}

int qwmoe_gguf_n_tensors(const qwmoe_gguf* g) { return g ? (int) g->tensors.size() : QWMOE_ERR_INVALID_ARG; }

int qwmoe_gguf_tensor_at(const qwmoe_gguf* g, int idx, qwmoe_gguf_tensor_info* out) {
    if (!g || !out || idx < 0 || idx >= (int) g->tensors.size()) return QWMOE_ERR_INVALID_ARG;
    fill_info(g, g->tensors[idx], out);
    return QWMOE_OK;
}

int qwmoe_gguf_find_tensor(const qwmoe_gguf* g, const char* name, qwmoe_gguf_tensor_info* out) {
    if (!g || !name || !out) return QWMOE_ERR_INVALID_ARG;
    auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return -1;
    fill_info(g, g->tensors[it->second], out);
    return (int) it->second;
}

int qwmoe_gguf_moe_hparams(const qwmoe_gguf* g, qwmoe_moe_hparams* hp) {
    if (!g || !hp) return QWMOE_ERR_INVALID_ARG;
    memset(hp, 0, sizeof(*hp));
    const char* arch = nullptr;
    qwmoe_gguf_get_str(g, "general.architecture", "unknown", &arch);
    snprintf(hp->arch, sizeof(hp->arch), "%s", arch);
    const std::string a = arch;
    auto u32 = [&](const char* suffix, uint32_t def) {
        uint32_t v = def;
        qwmoe_gguf_get_u32(g, (a + "." + suffix).c_str(), def, &v);
        return (int32_t) v;
    };
    hp->n_layer = u32("block_count", 0);
    hp->n_embd = u32("embedding_length", 0);
    hp->n_expert = u32("expert_count", 0);
    hp->n_expert_used = u32("expert_used_count", 0);
    hp->n_ff_exp = u32("expert_feed_forward_length", 0);
    qwmoe_gguf_get_f32(g, (a + ".expert_weights_scale").c_str(), 1.0f, &hp->expert_weights_scale);
    return QWMOE_OK;
}

int qwmoe_gguf_moe_layer_bytes(const qwmoe_gguf* g, int il, size_t* out) {
    if (!g || !out) return QWMOE_ERR_INVALID_ARG;
    qwmoe_moe_hparams hp;
    qwmoe_gguf_moe_hparams(g, &hp);
    if (il < 0 || il >= hp.n_layer) return QWMOE_ERR_INVALID_ARG;
    LayerTensors lt;
    const int rc = layer_tensors(g, il, hp, lt);
    if (rc != QWMOE_OK) return rc;
    size_t total = 0;
    for (int j = 0; j < 4; ++j) total += align256((size_t) lt.t[j]->nbytes);
    *out = total;
    return QWMOE_OK;
}

int qwmoe_gguf_load_moe_layer(void* stream, qwmoe_gguf* g, int il, void* dev, size_t dev_bytes, qwmoe_layer* out) {
    if (!g || !dev || !out) return QWMOE_ERR_INVALID_ARG;
    qwmoe_moe_hparams hp;
    qwmoe_gguf_moe_hparams(g, &hp);
    if (il < 0 || il >= hp.n_layer) return QWMOE_ERR_INVALID_ARG;
    LayerTensors lt;
    int rc = layer_tensors(g, il, hp, lt);
    if (rc != QWMOE_OK) return rc;
    size_t need = 0, off[4];
    for (int j = 0; j < 4; ++j) {
        off[j] = need;
        need += align256((size_t) lt.t[j]->nbytes);
    }
    if (dev_bytes < need) return QWMOE_ERR_INVALID_ARG;
    hipStream_t st = (hipStream_t) stream;
    if (!g->stage[0]) {
        for (int i = 0; i < 2; ++i) {
            if (hipHostMalloc(&g->stage[i], STAGE_BYTES, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&g->ev[i], hipEventDisableTiming) != hipSuccess)
                return QWMOE_ERR_HIP;
        }
        g->stage_bytes = STAGE_BYTES;
    }
    // stream each tensor's bytes: file -> pinned stage (alternating) -> device
    int k = 0;
    bool pending[2] = {false, false};
    for (int j = 0; j < 4 && rc == QWMOE_OK; ++j) {
        const Tensor& t = *lt.t[j];
        const Shard& sh = g->shards[t.shard];
        const uint64_t src = sh.data_offset + t.offset;
        if (src > sh.file_size || t.nbytes > sh.file_size - src) {
            rc = QWMOE_ERR_IO;
            break;
        }
        FILE* f = fopen(sh.path.c_str(), "rb");
        if (!f || fseeko(f, (off_t) src, SEEK_SET) != 0) {
            if (f) fclose(f);
            rc = QWMOE_ERR_IO;
            break;
        }
        for (uint64_t done = 0; done < t.nbytes; done += g->stage_bytes, ++k) {
            const size_t n = (size_t) std::min<uint64_t>(g->stage_bytes, t.nbytes - done);
            const int b = k & 1;
            if (pending[b] && hipEventSynchronize(g->ev[b]) != hipSuccess) { rc = QWMOE_ERR_HIP; break; }
            if (fread(g->stage[b], 1, n, f) != n) { rc = QWMOE_ERR_IO; break; }
            if (hipMemcpyAsync((uint8_t*) dev + off[j] + done, g->stage[b], n, hipMemcpyHostToDevice, st) != hipSuccess ||
                hipEventRecord(g->ev[b], st) != hipSuccess) {
                rc = QWMOE_ERR_HIP;
                break;
            }
            pending[b] = true;
        }
        fclose(f);
    }
    // the stages are reused by the next call: wait for the copies that read them
    for (int b = 0; b < 2; ++b)
        if (pending[b] && hipEventSynchronize(g->ev[b]) != hipSuccess && rc == QWMOE_OK) rc = QWMOE_ERR_HIP;
    if (rc != QWMOE_OK) return rc;

    qwmoe_layer L;
    memset(&L, 0, sizeof(L));
    L.n_embd = hp.n_embd;
    L.n_expert = hp.n_expert;
    L.n_expert_used = hp.n_expert_used;
    L.n_ff = hp.n_ff_exp;
    L.expert_weights_scale = hp.expert_weights_scale;
    L.router = (const float*) ((uint8_t*) dev + off[0]);
    const void* ptr[3] = {(uint8_t*) dev + off[1], (uint8_t*) dev + off[2], (uint8_t*) dev + off[3]};
    size_t nb1[3], nb2[3];
    int typ[3];
    for (int j = 0; j < 3; ++j) {
        const Tensor& m = *lt.t[j + 1];
        typ[j] = m.type;
        nb1[j] = (size_t) row_bytes(m);
        nb2[j] = nb1[j] * (size_t) m.ne[1];
    }
    L.type_gate = typ[0]; L.gate = ptr[0]; L.gate_nb1 = nb1[0]; L.gate_nb2 = nb2[0]; L.n_slots_gate = hp.n_expert;
    L.type_up = typ[1];   L.up = ptr[1];   L.up_nb1 = nb1[1];   L.up_nb2 = nb2[1];   L.n_slots_up = hp.n_expert;
    L.type_down = typ[2]; L.down = ptr[2]; L.down_nb1 = nb1[2]; L.down_nb2 = nb2[2]; L.n_slots_down = hp.n_expert;
    *out = L;
    return QWMOE_OK;
}

}  // extern "C"
