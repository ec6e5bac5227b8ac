// qw_decode.hpp -- host/device descriptors of the persistent decode stack.
#pragma once

#include <stdint.h>

#include "qw_common.hpp"
#include "qw_sort.hpp"

namespace qw {

// Per-layer tensors as the kernel sees them (device memory).
struct DecodeLayer {
    const float* router;          // [E][H]
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    uint64_t gate_nb1, gate_nb2, up_nb1, up_nb2, down_nb1, down_nb2;
    const int32_t* slot_gate;     // logical -> slot, or null
    const int32_t* slot_up;
    const int32_t* slot_down;
    int64_t n_slots_gate, n_slots_up, n_slots_down;
    const float* resmask;         // [E] added to the logits before the softmax, or null
    int32_t* want;                // [k] top k of the raw logits (with resmask), or null
};

// Resident-only routing in a decode kernel (core/runtime.cpp:870-881): want[0..k)
// = ggml_argsort_top_k of the raw logits v[0..E) (ranks by strictly larger
// count; std::sort's order on a tie inside the first k), computed by the nt
// threads of one workgroup.  ord: E ints of LDS scratch; flag: an LDS word.
// Ends synchronised.  Runs only for layers with a mask, so it is kept out of line.
__device__ __attribute__((noinline)) inline void decode_want(const float* v, int E, int k, int32_t* want,
                                                             int32_t* ord, SortRange* stack, int* flag, int tid,
                                                             int nt) {
    if (tid == 0) *flag = 0;
    __syncthreads();
    for (int i = tid; i < E; i += nt) {
        const float vi = v[i];
        int gt = 0, eq = 0;
        for (int j = 0; j < E; ++j) {
            gt += v[j] > vi;
            eq += v[j] == vi;
        }
        if (gt < k) {
            if (eq != 1) *flag = 1;
            else ord[gt] = i;
        }
    }
    __syncthreads();
    if (*flag) {
        if (tid == 0) {
            for (int i = 0; i < E; ++i) ord[i] = i;
            libstdcxx_sort_desc(ord, E, v, stack);
        }
        __syncthreads();
    }
    for (int i = tid; i < k; i += nt) want[i] = ord[i];
    __syncthreads();
}

struct DecodeStackDesc {
    DecodeLayer* layers_dev = nullptr;
    int n_layer = 0;
    int64_t H = 0, E = 0, k = 0, F = 0;
    int type_down = 0;
    float scale = 0.0f, rms_eps = 1e-6f;
    uint64_t* xa = nullptr;       // exchange words
    uint64_t* xy = nullptr;
    uint64_t* xl = nullptr;
    uint64_t* xd = nullptr;       // XCD kernel: down outputs crossing XCDs
    int use_xcd = 0;              // 1: k_decode_xcd (one expert per XCD), 0: k_decode_stack
    int xcd_local = 0;            // XCD kernel: XCD-local words stored with workgroup scope
    int xcd_wide = 0;             // XCD kernel: the wide form (decode_xcd_wide.hip)
    int32_t* status = nullptr;
    int32_t* abort_flag = nullptr;
    uint32_t epoch = 1;           // next launch's first layer epoch
    int grid = 0;
    int pa_per = 0, hb_per = 0;
    uint32_t lds_rw = 0, lds_a = 0, lds_b = 0, lds_xq = 0, lds_aq = 0, lds_x = 0, lds_act = 0, lds_res = 0,
             lds_y = 0, lds_total = 0;
    uint32_t rs_a = 0, rs_b = 0;
    void* dev_block = nullptr;    // one allocation holding everything above
};

int plan_decode_stack(DecodeStackDesc& d, int grid);
const void* decode_kernel(const DecodeStackDesc& d);
// 0 if one WG of the planned kernel fits on a CU (grid = CU count => all resident).
int check_decode_residency(const DecodeStackDesc& d);
// decode_xcd.hip: the kernel with one selected expert per XCD (grid = 8 XCDs x 32 CUs);
// decode_xcd_wide.hip: its form for wide layers (H = 4096, F = 1536), or null
const void* decode_xcd_kernel(const DecodeStackDesc& d);
const void* decode_xcd_wide_kernel(const DecodeStackDesc& d);
// 0 if the shape has an XCD kernel and the device has 256 CUs
int check_decode_xcd(const DecodeStackDesc& d, int cus);
// writes each workgroup's XCD id to dev_buf[0..n) and sets *ok when workgroup b runs on XCD b % 8
int probe_xcd_mapping(int32_t* dev_buf, int n, hipStream_t stream, int* ok);
int launch_decode_xcd(const DecodeStackDesc& d, const float* x_in, float* out, float* x_out, int32_t* ids_out,
                      float* w_out, uint32_t epoch0, hipStream_t stream);
int launch_decode_stack(const DecodeStackDesc& d, const float* x_in, float* out, float* x_out, int32_t* ids_out,
                        float* w_out, uint32_t epoch0, hipStream_t stream);

}  // namespace qw
