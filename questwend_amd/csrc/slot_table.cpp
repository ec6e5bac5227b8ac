// slot_table.cpp -- host-side expert slot bookkeeping for an all-resident HBM
// layout (the resident subset of core/expert_cache.{h,cpp}).
//
// ExpertCache keeps one pool per (role, type, shape) and maps the key
// layer * n_expert + expert to a slot (core/expert_cache.cpp:691-721), with 0 as
// its "absent" sentinel in slot_of (core/expert_cache.h:104).  On MI355X every
// expert of every layer is resident (288 GB of HBM), so there are no misses,
// fetches or evictions; what remains is the indirection itself: each role's
// pool holds n_layer * n_expert slabs in an arbitrary (here optionally seeded
// random) order, and a dense per-(role, layer) row gives logical expert -> slot
// (ExpertCache::slot_of_row, core/expert_cache.cpp:694-697).  Unassigned
// entries are -1, not 0, so slot 0 stays unambiguous.
#include <cstdint>
#include <new>
#include <random>
#include <vector>

#include "../../include/qwmoe.h"

struct qwmoe_slot_table {
    int n_layer = 0, n_expert = 0;
    std::vector<int32_t> slot_of[3];  // [role][layer * n_expert + expert]
};

extern "C" {

qwmoe_slot_table* qwmoe_slot_table_create(int n_layer, int n_expert) {
    if (n_layer <= 0 || n_expert <= 0) return nullptr;
    auto* t = new (std::nothrow) qwmoe_slot_table();
    if (!t) return nullptr;
    t->n_layer = n_layer;
    t->n_expert = n_expert;
    for (auto& v : t->slot_of) v.assign((size_t) n_layer * (size_t) n_expert, -1);
    return t;
}

void qwmoe_slot_table_free(qwmoe_slot_table* t) { delete t; }

int qwmoe_slot_table_fill(qwmoe_slot_table* t, uint64_t seed) {
    if (!t) return QWMOE_ERR_INVALID_ARG;
    const size_t n = (size_t) t->n_layer * (size_t) t->n_expert;
    for (int r = 0; r < 3; ++r) {
        std::vector<int32_t> perm(n);
        for (size_t i = 0; i < n; ++i) perm[i] = (int32_t) i;
        if (seed != 0) {
            // Fisher-Yates with a 64-bit LCG/xorshift stream (platform independent)
            uint64_t s = seed * 0x9e3779b97f4a7c15ull + (uint64_t) (r + 1) * 0xbf58476d1ce4e5b9ull;
            for (size_t i = n - 1; i > 0; --i) {
                s ^= s >> 12;
                s ^= s << 25;
                s ^= s >> 27;
                const uint64_t rnd = s * 0x2545f4914f6cdd1dull;
                const size_t j = (size_t) (rnd % (uint64_t) (i + 1));
                const int32_t tmp = perm[i];
                perm[i] = perm[j];
                perm[j] = tmp;
            }
        }
        t->slot_of[r] = perm;
    }
    return QWMOE_OK;
}

int qwmoe_slot_table_set(qwmoe_slot_table* t, int role, int layer, int expert, int32_t slot) {
    if (!t || role < 0 || role > 2 || layer < 0 || layer >= t->n_layer || expert < 0 || expert >= t->n_expert ||
        slot < 0)
        return QWMOE_ERR_INVALID_ARG;
    t->slot_of[role][(size_t) layer * t->n_expert + expert] = slot;
    return QWMOE_OK;
}

int32_t qwmoe_slot_table_slot_of(const qwmoe_slot_table* t, int role, int layer, int expert) {
    if (!t || role < 0 || role > 2 || layer < 0 || layer >= t->n_layer || expert < 0 || expert >= t->n_expert)
        return -1;
    return t->slot_of[role][(size_t) layer * t->n_expert + expert];
}

const int32_t* qwmoe_slot_table_row(const qwmoe_slot_table* t, int role, int layer) {
    if (!t || role < 0 || role > 2 || layer < 0 || layer >= t->n_layer) return nullptr;
    return t->slot_of[role].data() + (size_t) layer * t->n_expert;
}

}  // extern "C"
