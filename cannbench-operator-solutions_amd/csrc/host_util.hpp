// host_util.hpp - host-side helpers shared by the entry points: pointer alignment, group_list
// validation and the by-value group table the grouped kernels receive as a kernel argument.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cannbench_amd.h"

namespace cb {

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// The vector GEMM paths address one group's [K, N] weight block (and a tile's activation rows)
// through buffer resources with 32-bit byte offsets; larger blocks take the generic kernels, which
// index in 64 bits.
inline bool offsets32_ok(int64_t K, int64_t N) { return K * N < (1LL << 31); }

// A dispatch counts its work-items (blocks x threads per dimension) in 32 bits.  The row kernels
// launch one block per row (or per few rows); an operator whose launch would not fit returns
// CB_ERR_SHAPE instead of launching a truncated grid.
inline bool grid_fits(int64_t blocks, int64_t threads) { return blocks * threads < (1LL << 32); }

// Cumsum group boundaries plus the prefix of M-tiles per group, passed by value to the grouped
// kernels (no host->device copy, no device allocation).  row_end[g] is the exclusive end row of
// group g; tile_start[g] is the first M-tile of group g in the launch's tile enumeration.
struct GroupTable {
    int32_t n_groups;
    int32_t total_mtiles;
    int32_t max_rows;
    int32_t pad;
    int32_t row_end[CB_MAX_EXPERTS];
    int32_t tile_start[CB_MAX_EXPERTS + 1];
};

// group_list validation, in the reference's order (gmsq_plugin.cpp:105-117,
// grouped_matmul_plugin.cpp:82-95, 133-136).
inline int validate_group_list(const int64_t* gl, int64_t len, int64_t E, int64_t M)
{
    if (!gl) return CB_ERR_NULL_POINTER;
    if (len != E) return CB_ERR_GROUP_LEN;
    if (len < 1 || len > CB_MAX_EXPERTS) return CB_ERR_GROUP_COUNT;
    int64_t prev = 0;
    for (int64_t g = 0; g < len; ++g) {
        if (gl[g] < prev || gl[g] > M) return CB_ERR_GROUP_ORDER;
        prev = gl[g];
    }
    if (prev != M) return CB_ERR_GROUP_TOTAL;
    return CB_OK;
}

// Fill the table for M-tiles of `bm` rows.  Assumes validate_group_list() passed.
inline void build_group_table(GroupTable& t, const int64_t* gl, int64_t E, int bm)
{
    t.n_groups = (int32_t)E;
    t.pad = 0;
    int32_t prev = 0, tiles = 0, mx = 0;
    for (int64_t g = 0; g < E; ++g) {
        const int32_t end = (int32_t)gl[g];
        const int32_t rows = end - prev;
        t.row_end[g] = end;
        t.tile_start[g] = tiles;
        tiles += (rows + bm - 1) / bm;
        mx = rows > mx ? rows : mx;
        prev = end;
    }
    for (int64_t g = E; g < CB_MAX_EXPERTS; ++g) {
        t.row_end[g] = prev;
        t.tile_start[g] = tiles;
    }
    t.tile_start[CB_MAX_EXPERTS] = tiles;
    t.total_mtiles = tiles;
    t.max_rows = mx;
}

inline int check_launch()
{
    return hipGetLastError() == hipSuccess ? CB_OK : CB_ERR_LAUNCH;
}

// Test hooks (set by cb_set_test_overrides, per thread, until changed): a forced grid for the
// persistent GEMM kernels (0: the CU count; < 0: persistent launch off), a poll limit for the
// GroupedMatmulSwigluQuant exchange wait (0: the default), and the GroupedMatmul tile (128 forces
// the 128 x 128 kernel; 0: automatic).
struct TestOverrides {
    int persistent_grid = 0, exchange_spin_limit = 0, gmm_tile = 0;
};
extern thread_local TestOverrides g_overrides;

// Optional per-thread instrumentation: events recorded around the next main kernel launch of an
// operator (set by cb_set_kernel_timing, consumed and cleared by that launch).
struct KernelTiming {
    hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local KernelTiming g_timing;

struct TimedLaunch {
    hipStream_t st;
    KernelTiming t;
    explicit TimedLaunch(hipStream_t s) : st(s), t(g_timing)
    {
        g_timing = KernelTiming();
        if (t.start) (void)hipEventRecord(t.start, st);
    }
    ~TimedLaunch()
    {
        if (t.stop) (void)hipEventRecord(t.stop, st);
    }
};

}  // namespace cb
