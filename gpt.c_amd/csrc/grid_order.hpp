// XCD- and CU-aware grid order for the query-block kernels (forward and dq).
//
// Their workgroups all do the same per-tile work, but a query block b of a
// causal head covers b + 1 key blocks: the longest block is nblk times the
// shortest.  When every workgroup of the grid is resident at once, what
// bounds the kernel is the busiest CU, so the order below deals long and
// short blocks to every CU.
//
// MI355X dispatch, measured with per-workgroup clocks and HW_ID: workgroup
// blockIdx runs on XCD blockIdx % 8; within an XCD, its i-th workgroup
// (i = blockIdx / 8) goes to CU i % cus in "round" i / cus, and the rounds
// that fit the occupancy stay resident together.  Position pos enumerates
// the blocks longest first with the head index fastest (so that all blocks
// of a head share one XCD and its L2); round r maps CU u to position
// r * cus + (u + rot[r]) % cus, a permutation of i, with the rotations
// chosen on the host to even out the per-CU sums of block lengths.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <climits>
#include <map>
#include <mutex>
#include <utility>

#include "hip_check.hpp"

namespace gptc {

constexpr int kXcds = 8;          // XCDs of an MI355X
constexpr int kOrderRounds = 4;   // co-resident dispatch rounds an order balances

struct GridOrder {
    int cus;                  // CUs per XCD the order is laid out for (0: plain order)
    int rot[kOrderRounds];    // CU-index rotation of each dispatch round
};

// Block index (0 = longest) and head of this workgroup.  bh_pad is a
// multiple of kXcds; heads at or past B*H are padding.
__device__ __forceinline__ void grid_position(const GridOrder &o, int nblk, int bh_pad, int &blk, int &bh) {
    const int x = blockIdx.x % kXcds, i = blockIdx.x / kXcds;
    const int nbh_x = bh_pad / kXcds;
    int pos = i;
    if (o.cus > 0) {
        const int r = i / o.cus, u = i - r * o.cus;
        if (r < kOrderRounds && (r + 1) * o.cus <= nblk * nbh_x) pos = r * o.cus + (u + o.rot[r]) % o.cus;
    }
    blk = pos / nbh_x;
    bh = x + kXcds * (pos - blk * nbh_x);
}

// The rotations for `kernel` (256-thread workgroups) launched over nblk x
// bh_pad workgroups: minimise the largest per-CU sum of block lengths over
// the co-resident rounds (ties: the largest smallest sum).  Cached per shape.
template <typename Kernel>
GridOrder choose_grid_order(int nblk, int bh_pad, Kernel kernel) {
    // Device properties and the kernel's occupancy, once per device and
    // kernel (this runs on every launch, so no runtime queries after the
    // first).  Keyed on the kernel's address: template variants of a kernel
    // share one function type but not their register counts.  Both caches
    // below are shared by every host thread that launches: one lock guards
    // them.
    struct DeviceInfo {
        int cus_total, per_cu;
    };
    static std::mutex mu;
    static std::map<std::pair<int, const void *>, DeviceInfo> devices;
    int dev = 0;
    hipCheck(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    const std::pair<int, const void *> dkey{dev, reinterpret_cast<const void *>(kernel)};
    auto d = devices.find(dkey);
    if (d == devices.end()) {
        DeviceInfo info{};
        hipCheck(hipDeviceGetAttribute(&info.cus_total, hipDeviceAttributeMultiprocessorCount, dev));
        hipCheck(hipOccupancyMaxActiveBlocksPerMultiprocessor(&info.per_cu, kernel, 256, 0));
        d = devices.emplace(dkey, info).first;
    }
    GridOrder o{};
    const int cus_total = d->second.cus_total, per_cu = d->second.per_cu;
    if (cus_total % kXcds != 0 || per_cu < 2) return o;
    const int cus = cus_total / kXcds, nbh_x = bh_pad / kXcds, M = nblk * nbh_x;
    const int rounds = std::min(per_cu, kOrderRounds);

    static std::map<std::array<int, 4>, std::array<int, kOrderRounds>> cache;
    const std::array<int, 4> key{nblk, nbh_x, cus, rounds};
    auto it = cache.find(key);
    if (it == cache.end()) {
        auto len = [&](int pos) { return pos < M ? nblk - pos / nbh_x : 0; };
        std::array<int, kOrderRounds> rot{}, best{};
        int best_max = INT_MAX, best_min = -1;
        long combos = 1;
        for (int r = 1; r < rounds; ++r) combos *= cus;
        for (long c = 0; c < combos; ++c) {
            long v = c;
            for (int r = 1; r < rounds; ++r, v /= cus) rot[r] = static_cast<int>(v % cus);
            int mx = 0, mn = INT_MAX;
            for (int u = 0; u < cus; ++u) {
                int load = 0;
                for (int r = 0; r < rounds; ++r) {
                    const bool full = (r + 1) * cus <= M;
                    load += len(r * cus + (full ? (u + rot[r]) % cus : u));
                }
                mx = std::max(mx, load);
                mn = std::min(mn, load);
            }
            if (mx < best_max || (mx == best_max && mn > best_min)) {
                best_max = mx;
                best_min = mn;
                best = rot;
            }
        }
        it = cache.emplace(key, best).first;
    }
    o.cus = cus;
    for (int r = 0; r < kOrderRounds; ++r) o.rot[r] = it->second[r];
    return o;
}

}  // namespace gptc
