// Static device scratch of the allocation-free entry point
// (qwmoe_mul_mat_id_noalloc): the quantized activations and the grouping
// arrays of one call live in a file-scope device array instead of the
// library's workspace, so the call itself allocates nothing.
//
// Each GPU the library runs on holds its own copy of `scratch` (kScratchBytes)
// until the process ends, at its own address.  In host code the array's name
// is only a stand-in for the symbol: its device address comes from
// hipGetSymbolAddress, once per device with that device current
// (scratch_setup, called by qwmoe_init), and only that address is handed to
// kernels.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

#include "qw_kernels.hpp"

namespace qw {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
}  // namespace

int scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return -2;
    if (g_scratch[device].load()) return 0;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != device) return -2;
    void* ptr = nullptr;
    if (hipGetSymbolAddress((void**) &ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return -3;
    g_scratch[device].store(ptr);
    return 0;
}

void* scratch_ptr(int device) {
    return device >= 0 && device < kMaxDevices ? g_scratch[device].load() : nullptr;
}

}  // namespace qw
