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
// largest per-CU sum of costs is kept (the pairs on ties; the lpt lists
// when the pairs leave resident slots empty and lpt is within 2 %):
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
//
// A table may also hold a pool: the blocks j < pool_j0 of every head are
// then left out of the lists, and a workgroup whose list is done takes them
// one at a time, largest first, from a counter in device memory (pool item
// r = block pool_j0 - 1 - r / BH of head r % BH).  The workgroups of a CU do
// not progress at the same rate (the SIMDs issue from the oldest waves
// first) and neither do the CUs, so static lists of equal cost do not end
// together; the pool lets the first ones to finish take the remainder.
// Every workgroup takes exactly one index at or past the pool's end, after
// which it stops; the last workgroup to finish resets the counters for the
// next launch.  Launches that share a table must not overlap.
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
    int pool_n;           // pool items (0: no pool)
    int pool_j0, pool_bh, pool_bh0;  // pool item r: head pool_bh0 + r % pool_bh, block pool_j0 - 1 - r / pool_bh
    int *counters;        // 128 ints: [0] next pool index, [64] workgroups done, [1..63] unused
                          // (zero between launches; see the forward's pool protocol)
};

__device__ __forceinline__ int sched_bh(int item) { return item >> kSchedJBits; }
__device__ __forceinline__ int sched_j(int item) { return item & ((1 << kSchedJBits) - 1); }

// Host-side table of one shape.
struct SchedTable {
    int num_wg = 0;
    std::vector<int> wg_start, items;
    double max_cu_load = 0.0;  // largest per-CU sum of block costs (tiles)
    bool pairs = false;        // which construction won
    int pool_j0 = 0;           // blocks j < pool_j0 of every head form the pool (0: none)
};

// Builds the table for BH heads of nqt blocks, for a kernel that keeps
// per_cu workgroups resident per CU on an XCD of cus CUs.  pool: leave the
// smallest blocks to a pool (kPoolJ0 of them per head) where every list
// keeps at least one block; otherwise, or with pool false, there is none.
SchedTable build_block_schedule(int BH, int nqt, int per_cu, int cus, bool pool = false);
constexpr int kPoolJ0 = 3;  // pool blocks per head: j = 0, 1, 2 (6 of a head's tiles)

// The device copy of build_block_schedule(BH, nqt, per_cu of `kernel`) for
// the current device, with bh0 added to every head index (the heads
// [bh0, bh0 + BH) of a larger problem), built and uploaded (stream-ordered on
// `stream`) on first use and cached for the life of the process.  The first
// use of a shape must not happen while `stream` is being captured into a
// graph (it allocates and copies from host memory): that is a fatal error.
BlockSched device_block_schedule(int BH, int nqt, const void *kernel, hipStream_t stream, int *num_wg, int bh0 = 0,
                                 bool pool = false);

// ---- Work lists of the D = 64 dk/dv kernel ----
//
// The unit of work is one 128-key block kb of one head: query tiles
// 2kb .. nqt-1 (the first two hold the diagonal).  Key block kb of head bh
// costs nqt - 2kb tiles, less 3/4 for the diagonal's two partly masked tiles,
// plus a fixed part (V rows, epilogue).  The blocks of a head therefore range
// from about 1 to nqt tiles, and a grid of one workgroup per block leaves the
// CUs that hold the longest blocks busy long after the others.  Here each
// workgroup runs a list of items, one after the other:
//   items[4i .. 4i+3] = (bh, kb, qa, qe): query tiles [qa, qe) of key block
//   kb of head bh.
// Key blocks kb < nsplit (the same for every head) are cut in two at a tile
// edge into items of about equal cost, whose dK, dV the kernel adds into rows
// the delta kernel zeroed (two addends: the same sum in either order).
// Every other block is one item.  The items are placed like the query-block
// lists (heads dealt to the XCDs in contiguous ranges of equal work, longest
// first onto the least-loaded CU, then its least-loaded slot), and the CU's
// heavier list goes to the slot dispatched first.  nsplit is 0 when that
// is within 5 % of the best estimated time (a CU's total, or its longest
// list run alone) over 0 .. nkb, else the smallest count within 2 %.
struct KeySched {
    const int *wg_start;  // num_wg + 1 offsets into items (in items, not ints)
    const int *items;     // 4 ints per item
};

struct KeyTable {
    int num_wg = 0;
    int nsplit = 0;
    std::vector<int> wg_start, items;
    double est = 0.0;  // the estimated time the choice of nsplit minimised (tiles)
};

// max_split: the largest nsplit considered (-1: every count up to nkb).
KeyTable build_key_schedule(int BH, int nqt, int per_cu, int cus, int max_split = -1);

// The device copy of build_key_schedule for the current device and the
// residency of `kernel`, with bh0 added to every head index, built,
// uploaded (stream-ordered on `stream`) and cached like device_block_schedule.
KeySched device_key_schedule(int BH, int nqt, const void *kernel, hipStream_t stream, int *num_wg, int *nsplit,
                             int bh0 = 0, int max_split = -1);

}  // namespace gptc
