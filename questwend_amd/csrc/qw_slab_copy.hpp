// qw_slab_copy.hpp -- launch interface of the slab gather kernel (slab_copy.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qw {

constexpr int SLAB_COPY_MAX = 64;  // slabs per launch (the table travels in the kernel arguments)

struct SlabCopyArgs {
    const uint8_t* src[SLAB_COPY_MAX];  // device-visible addresses (pinned host memory mapped to the GPU)
    uint8_t* dst[SLAB_COPY_MAX];
    uint64_t bytes;                     // per slab, a multiple of 16; every src/dst 16-byte aligned
    uint32_t n;
};

// Copies a.n slabs of a.bytes each; 0 or a negative qwmoe status.
int launch_slab_copy(const SlabCopyArgs& a, hipStream_t stream);

}  // namespace qw
