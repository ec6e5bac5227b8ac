// Weight-row indexing of the block-parallel mul_mat_id GEMV (k_mmid_gemv_bp):
// which rows of an N-row matrix its loads touch.  Shared by the kernel and a
// host-side check that every row index stays inside [0, N).
#pragma once

#include <cstdint>

#ifdef __HIPCC__
#define QW_BP_HD __host__ __device__
#else
#define QW_BP_HD
#endif

namespace qw {

// Rows per wave for BPR lanes per row, and the first row of workgroup g and of
// its wave w (4 waves per workgroup).
QW_BP_HD constexpr int bp_rows_per_wave(int bpr) { return 64 / bpr; }
QW_BP_HD inline int64_t bp_wg_row0(int64_t g, int bpr) { return g * (4 * (int64_t) bp_rows_per_wave(bpr)); }
QW_BP_HD inline int64_t bp_wave_row0(int64_t g, int w, int bpr) {
    return bp_wg_row0(g, bpr) + (int64_t) w * bp_rows_per_wave(bpr);
}
// Rows of the wave that exist (0 for a wave past the matrix end).
QW_BP_HD inline int bp_wave_rows(int64_t N, int64_t wr0, int bpr) {
    const int rpw = bp_rows_per_wave(bpr);
    return (int) (N - wr0 < 0 ? 0 : N - wr0 < rpw ? N - wr0 : rpw);
}
// The row the direct loads of lane row rl (lane / BPR) read: its own row, row 0
// of the wave for lanes past the wave's rows, and the workgroup's first row (it
// exists) for a wave past the matrix end, which uses nothing it loaded.
QW_BP_HD inline int64_t bp_direct_row(int64_t r0, int64_t wr0, int wrows, int rl) {
    return wrows > 0 ? wr0 + (rl < wrows ? rl : 0) : r0;
}
// The row staged chunk r of the wave reads (r < wrows for every chunk taken;
// the others read row 0 of the wave and are dropped).
QW_BP_HD inline int64_t bp_staged_row(int64_t wr0, int wrows, int r) { return wr0 + (r < wrows ? r : 0); }

}  // namespace qw
