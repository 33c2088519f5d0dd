// Work lists of the query-block kernels (the D = 64 forward and dq).
//
// The unit of work is one 64-query block j of one (b, h) head: it reduces
// key tiles 0 .. j, so its cost is j + 1 tiles plus a fixed part (loading
// Q, the epilogue).  A causal head's blocks therefore range from 1 to nqt
// tiles.  Each workgroup runs a short list of blocks, one after the other,
// from a table built on the host per shape:
//   items[wg_start[w] .. wg_start[w + 1])  the blocks of workgroup w, each
//                                           packed as (bh << kSchedJBits) | j.
// Every (bh, j) of the problem appears exactly once in the table.
//
// Two ways of building it are evaluated and the one with the smaller
// largest per-CU sum of costs is kept:
//   pairs  workgroup = blocks j and nqt-1-j of one head (equal cost nqt+1
//          for every workgroup: ideal when the pairs fill the resident
//          slots exactly, as at B=8, H=12, T=1024);
//   lpt    blocks longest first onto the least-loaded CU, then onto that
//          CU's least-loaded workgroup slot (longest-processing-time
//          first); the heads are dealt to the 8 XCDs in contiguous ranges
//          of equal work, so that the blocks of a head share one XCD's L2
//          (a head at a range boundary is split at block granularity).
// Placement uses the dispatch order measured on the MI355X: workgroup
// blockIdx runs on XCD blockIdx % 8, and the i-th workgroup of an XCD
// (i = blockIdx / 8) on CU i % cus in dispatch round i / cus.
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

namespace gptc {

constexpr int kSchedJBits = 12;  // j < 4096 (T < 262144)
constexpr int kSchedXcds = 8;

// Device view of a table (pointers into device memory).
struct BlockSched {
    const int *wg_start;  // num_wg + 1 offsets into items
    const int *items;     // (bh << kSchedJBits) | j
};

__device__ __forceinline__ int sched_bh(int item) { return item >> kSchedJBits; }
__device__ __forceinline__ int sched_j(int item) { return item & ((1 << kSchedJBits) - 1); }

// Host-side table of one shape.
struct SchedTable {
    int num_wg = 0;
    std::vector<int> wg_start, items;
    double max_cu_load = 0.0;  // largest per-CU sum of block costs (tiles)
    bool pairs = false;        // which construction won
};

// Builds the table for BH heads of nqt blocks, for a kernel that keeps
// per_cu workgroups resident per CU on an XCD of cus CUs.
SchedTable build_block_schedule(int BH, int nqt, int per_cu, int cus);

// The device copy of build_block_schedule(BH, nqt, per_cu of `kernel`) for
// the current device, built and uploaded (stream-ordered on `stream`) on
// first use and cached for the life of the process.
BlockSched device_block_schedule(int BH, int nqt, const void *kernel, hipStream_t stream, int *num_wg);

}  // namespace gptc
