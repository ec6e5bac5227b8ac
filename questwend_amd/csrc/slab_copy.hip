// slab_copy.hip -- one launch that copies many expert slabs from pinned host
// memory into slot pools.  The expert cache's scattered misses (one slab per
// (role, layer, expert), 0.9-1.3 MB at the 30B shape) would otherwise be one
// hipMemcpyAsync each; here every workgroup moves one 32 KiB chunk of one slab
// with eight 16-byte loads in flight per thread, so all misses of a call cross
// PCIe together from a single launch.
#include "qw_slab_copy.hpp"

namespace qw {

typedef unsigned int sc_u32x4 __attribute__((ext_vector_type(4)));

constexpr int SC_THREADS = 256;
constexpr int SC_VEC = 8;
constexpr uint64_t SC_CHUNK = (uint64_t) SC_THREADS * SC_VEC * 16;

__global__ void __launch_bounds__(SC_THREADS) k_slab_copy(SlabCopyArgs a, uint32_t chunks) {
    const uint32_t j = blockIdx.x / chunks, c = blockIdx.x - j * chunks;
    if (j >= a.n) return;
    constexpr uint32_t CH16 = (uint32_t) (SC_CHUNK / 16);
    const uint64_t left = a.bytes / 16 - (uint64_t) c * CH16;
    const uint32_t n16 = left < CH16 ? (uint32_t) left : CH16;
    const sc_u32x4* s = (const sc_u32x4*) a.src[j] + (size_t) c * CH16;
    sc_u32x4* d = (sc_u32x4*) a.dst[j] + (size_t) c * CH16;
    const uint32_t t = threadIdx.x;
    if (n16 == CH16) {
        sc_u32x4 v[SC_VEC];
#pragma unroll
        for (int u = 0; u < SC_VEC; ++u) v[u] = __builtin_nontemporal_load(s + t + u * SC_THREADS);
#pragma unroll
        for (int u = 0; u < SC_VEC; ++u) d[t + u * SC_THREADS] = v[u];
    } else {
        for (uint32_t i = t; i < n16; i += SC_THREADS) d[i] = __builtin_nontemporal_load(s + i);
    }
}

int launch_slab_copy(const SlabCopyArgs& a, hipStream_t stream) {
    if (a.n == 0) return 0;
    if (a.n > (uint32_t) SLAB_COPY_MAX || a.bytes == 0 || a.bytes % 16 != 0) return -1;
    for (uint32_t j = 0; j < a.n; ++j)
        if (!a.src[j] || !a.dst[j] || ((uintptr_t) a.src[j] | (uintptr_t) a.dst[j]) % 16 != 0) return -1;
    const uint64_t chunks = (a.bytes + SC_CHUNK - 1) / SC_CHUNK;
    if (chunks * a.n > 0x7fffffffull) return -1;
    hipLaunchKernelGGL(k_slab_copy, dim3((unsigned) (chunks * a.n)), dim3(SC_THREADS), 0, stream, a,
                       (uint32_t) chunks);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace qw
