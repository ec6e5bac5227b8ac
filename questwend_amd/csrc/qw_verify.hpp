// qw_verify.hpp -- host/device interface of the persistent verify-batch kernel
// (verify_xcd.hip): T <= VERIFY_TMAX tokens through a stack of MoE FFN layers in
// one launch, used by qwmoe_layer_stack_run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qw_decode.hpp"

namespace qw {

constexpr int VERIFY_TMAX = 8;

struct VerifyArgs {
    const DecodeLayer* layers;
    int n_layer, k, T;
    float scale, rms_eps;
    const float* x_in;   // [T][H]
    float* out;          // [T][H]
    float* x_out;        // [T][H] or null
    int32_t* ids_out;    // [n_layer][T][k] or null
    float* w_out;
    uint64_t* xl;        // [8][VERIFY_TMAX][E]                 logits, XCD-local
    uint64_t* xa;        // [8][slots][VERIFY_TMAX][F]          act, XCD-local
    uint64_t* xd;        // [2][8 VERIFY_TMAX][VERIFY_TMAX][H]  down outputs, across XCDs
    uint64_t* xy;        // [8][VERIFY_TMAX][H]                 y, XCD-local
    uint32_t epoch0;
    int32_t* status;     // bit 0: top-k tie replayed; 3: a wait timed out; 4: bad slot
    int32_t* abort_flag;
    int local_st;        // 1: XCD-local words stored with workgroup scope
};

// Exchange words the kernel needs (uint64 each) for H, F, E.
inline size_t verify_words_xl(int64_t E) { return (size_t) 8 * VERIFY_TMAX * (size_t) E; }
inline size_t verify_words_xa(int64_t F) { return (size_t) 8 * VERIFY_TMAX * VERIFY_TMAX * (size_t) F; }
inline size_t verify_words_xd(int64_t H) { return (size_t) 2 * 8 * VERIFY_TMAX * VERIFY_TMAX * (size_t) H; }
inline size_t verify_words_xy(int64_t H) { return (size_t) 8 * VERIFY_TMAX * (size_t) H; }

// The kernel for H, F, E (Q4_K gate/up/down), or null.
const void* verify_xcd_kernel(int64_t H, int64_t F, int64_t E);
// 0 if one workgroup fits on a CU.
int verify_xcd_occupancy(const void* fn);
int launch_verify_xcd(const void* fn, const VerifyArgs& a, hipStream_t stream);

}  // namespace qw
