// Tile scheduling and synchronisation helpers shared by the large-M GEMM
// kernels (gemm.hip, gemm_w4.hip).
#pragma once

#include "h3q_common.hpp"

namespace h3q {

// Logical tile of block index bid.  Workgroups are dealt to the 8 XCDs round
// robin (XCD = blockIdx % 8); give each XCD a contiguous run of tiles so the
// tiles resident on one XCD share A and B rows in that XCD's L2.  Within the
// run, tiles go column-major in groups of kGroupM tile-rows.  A persistent
// grid passes bid = blockIdx + j * gridDim with gridDim % 8 == 0, which keeps
// bid % 8 equal to the XCD the workgroup runs on.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kXcds = 8, kGroupM = 8;
    const int total = tiles_m * tiles_n;
    const int q = total / kXcds, rem = total % kXcds;
    const int xcd = bid % kXcds, local = bid / kXcds;
    const int t = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int in_group = t - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Workgroup barrier for the copy ring.  __syncthreads() would add a release
// fence, which waits for every in-flight LDS copy (vmcnt(0)) and so drains the
// ring; here the caller has already waited for exactly the stage it needs, and
// only this wave's LDS reads must be complete before others overwrite a
// buffer.  The asm memory clobber keeps LDS accesses on their side.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Lane index that the compiler cannot hoist out of a loop: recomputing
// lane-derived offsets inside each tile iteration keeps them from staying
// live (in registers) across the epilogue of the persistent kernel.
__device__ __forceinline__ int opaque_lane() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// Workgroups of the persistent GEMM: one per CU of the current device (the
// LDS ring allows one per CU), rounded down to a multiple of the 8 XCDs.
static inline int persistent_grid(int tiles) {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    int cus = dev < 64 ? __atomic_load_n(&cached[dev], __ATOMIC_RELAXED) : 0;
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8) cus = 8;
        if (dev < 64) __atomic_store_n(&cached[dev], cus, __ATOMIC_RELAXED);
    }
    cus -= cus % 8;
    return tiles < cus ? tiles : cus;
}

}  // namespace h3q
