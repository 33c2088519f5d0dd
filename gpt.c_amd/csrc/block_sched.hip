// Host construction and device upload of the query-block work lists
// (block_sched.hpp).
#include "block_sched.hpp"

#include <algorithm>
#include <array>
#include <map>
#include <mutex>
#include <numeric>
#include <tuple>

#include "gpu_kernels.h"
#include "hip_check.hpp"
#include "utils.h"

namespace gptc {

namespace {

constexpr double kBlockOverhead = 0.5;  // Q load and epilogue of a block, in tiles

double block_cost(int j) { return j + 1 + kBlockOverhead; }

int pack(int bh, int j) { return (bh << kSchedJBits) | j; }

// Largest per-CU sum of block costs of a table under the dispatch order.
double max_cu_load(const SchedTable &t, int cus) {
    std::vector<double> load(static_cast<size_t>(kSchedXcds) * cus, 0.0);
    for (int w = 0; w < t.num_wg; ++w) {
        const int x = w % kSchedXcds, u = (w / kSchedXcds) % cus;
        for (int k = t.wg_start[w]; k < t.wg_start[w + 1]; ++k)
            load[static_cast<size_t>(x) * cus + u] += block_cost(t.items[k] & ((1 << kSchedJBits) - 1));
    }
    return *std::max_element(load.begin(), load.end());
}

// Workgroup = blocks j and nqt-1-j of one head, less the blocks j < j0 (the
// pool's); heads fastest, so the pairs of a head land on one XCD
// (blockIdx % 8 == bh % 8).
SchedTable pairs_schedule(int BH, int nqt, int j0) {
    SchedTable t;
    const int bh_pad = (BH + kSchedXcds - 1) / kSchedXcds * kSchedXcds, nbh_x = bh_pad / kSchedXcds;
    const int npair = (nqt + 1) / 2;
    t.num_wg = npair * bh_pad;
    t.wg_start.push_back(0);
    for (int w = 0; w < t.num_wg; ++w) {
        const int x = w % kSchedXcds, i = w / kSchedXcds;
        const int pair = i / nbh_x, bh = x + kSchedXcds * (i - pair * nbh_x);
        if (bh < BH) {
            if (pair >= j0) t.items.push_back(pack(bh, pair));
            if (nqt - 1 - pair != pair && nqt - 1 - pair >= j0) t.items.push_back(pack(bh, nqt - 1 - pair));
        }
        t.wg_start.push_back(static_cast<int>(t.items.size()));
    }
    t.pairs = true;
    return t;
}

SchedTable lpt_schedule(int BH, int nqt, int per_cu, int cus, int j0) {
    struct Item {
        double cost;
        int bh, j;
    };
    double per_head = 0.0;
    for (int j = j0; j < nqt; ++j) per_head += block_cost(j);
    const double target = per_head * BH / kSchedXcds;
    // Heads dealt to XCDs in contiguous ranges of equal work (block granularity).
    std::vector<std::vector<Item>> xitems(kSchedXcds);
    double acc = 0.0;
    for (int bh = 0; bh < BH; ++bh)
        for (int j = j0; j < nqt; ++j) {
            const double c = block_cost(j);
            const int x = std::min(static_cast<int>((acc + 0.5 * c) / target), kSchedXcds - 1);
            xitems[x].push_back({c, bh, j});
            acc += c;
        }
    // slots[x][u][s]: the block list of slot s of CU u on XCD x.
    std::vector<std::vector<std::vector<std::vector<int>>>> slots(
        kSchedXcds, std::vector<std::vector<std::vector<int>>>(cus, std::vector<std::vector<int>>(per_cu)));
    int rounds = 1;
    for (int x = 0; x < kSchedXcds; ++x) {
        auto &its = xitems[x];
        std::stable_sort(its.begin(), its.end(), [](const Item &a, const Item &b) { return a.cost > b.cost; });
        std::vector<double> cu(cus, 0.0);
        std::vector<std::vector<double>> sl(cus, std::vector<double>(per_cu, 0.0));
        for (const Item &it : its) {
            const int u = static_cast<int>(std::min_element(cu.begin(), cu.end()) - cu.begin());
            const int s = static_cast<int>(std::min_element(sl[u].begin(), sl[u].end()) - sl[u].begin());
            cu[u] += it.cost;
            sl[u][s] += it.cost;
            slots[x][u][s].push_back(pack(it.bh, it.j));
            rounds = std::max(rounds, s + 1);
        }
    }
    SchedTable t;
    t.num_wg = kSchedXcds * cus * rounds;
    t.wg_start.push_back(0);
    for (int w = 0; w < t.num_wg; ++w) {
        const int x = w % kSchedXcds, i = w / kSchedXcds, u = i % cus, s = i / cus;
        for (int item : slots[x][u][s]) t.items.push_back(item);
        t.wg_start.push_back(static_cast<int>(t.items.size()));
    }
    return t;
}

// ---- dk/dv key-block lists ----

constexpr double kKeyItemOverhead = 0.3;  // V rows and epilogue of an item, in tiles
// A workgroup left alone on its CU gets this share of what the CU's full set
// of workgroups gets (measured: one wave per SIMD runs the C2 grid 253 us
// against 206 us with two).
constexpr double kAloneShare = 0.81;
constexpr int kKeyTilesPerBlock = 2;        // 128 keys = 2 query tiles of 64 on the diagonal

double key_cost(int kb, int qa, int qe) {
    const int diag = kKeyTilesPerBlock * kb;
    return (qe - qa) - (qa == diag ? 0.75 : 0.0) + kKeyItemOverhead;
}

KeyTable key_schedule_with(int BH, int nqt, int nsplit, int per_cu, int cus) {
    struct Item {
        double cost;
        int bh, kb, qa, qe;
    };
    const int nkb = (nqt + kKeyTilesPerBlock - 1) / kKeyTilesPerBlock;
    std::vector<Item> all;
    for (int bh = 0; bh < BH; ++bh)
        for (int kb = 0; kb < nkb; ++kb) {
            const int qa = kKeyTilesPerBlock * kb, qe = nqt;
            if (kb < nsplit && qe - qa >= 2) {
                int best = qa + 1;
                for (int m = qa + 1; m < qe; ++m)
                    if (std::abs(key_cost(kb, qa, m) - key_cost(kb, m, qe)) <
                        std::abs(key_cost(kb, qa, best) - key_cost(kb, best, qe)))
                        best = m;
                all.push_back({key_cost(kb, qa, best), bh, kb, qa, best});
                all.push_back({key_cost(kb, best, qe), bh, kb, best, qe});
            } else {
                all.push_back({key_cost(kb, qa, qe), bh, kb, qa, qe});
            }
        }
    // Heads dealt to XCDs in contiguous ranges of equal work (item granularity).
    double total = 0.0;
    for (const Item &it : all) total += it.cost;
    const double target = total / kSchedXcds;
    std::vector<std::vector<Item>> xitems(kSchedXcds);
    double acc = 0.0;
    for (const Item &it : all) {
        const int x = std::min(static_cast<int>((acc + 0.5 * it.cost) / target), kSchedXcds - 1);
        xitems[x].push_back(it);
        acc += it.cost;
    }
    std::vector<std::vector<std::vector<std::vector<Item>>>> slots(
        kSchedXcds, std::vector<std::vector<std::vector<Item>>>(cus, std::vector<std::vector<Item>>(per_cu)));
    double est = 0.0;
    int rounds = 1;
    for (int x = 0; x < kSchedXcds; ++x) {
        auto &its = xitems[x];
        std::stable_sort(its.begin(), its.end(), [](const Item &a, const Item &b) { return a.cost > b.cost; });
        std::vector<double> cu(cus, 0.0);
        std::vector<std::vector<double>> sl(cus, std::vector<double>(per_cu, 0.0));
        for (const Item &it : its) {
            const int u = static_cast<int>(std::min_element(cu.begin(), cu.end()) - cu.begin());
            const int s = static_cast<int>(std::min_element(sl[u].begin(), sl[u].end()) - sl[u].begin());
            cu[u] += it.cost;
            sl[u][s] += it.cost;
            slots[x][u][s].push_back(it);
        }
        for (int u = 0; u < cus; ++u) {
            // The heavier list on the slot dispatched first (older waves issue first).
            std::vector<int> order(per_cu);
            std::iota(order.begin(), order.end(), 0);
            std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return sl[u][a] > sl[u][b]; });
            std::vector<std::vector<Item>> sorted;
            for (int s : order) sorted.push_back(std::move(slots[x][u][s]));
            slots[x][u] = std::move(sorted);
            int used = 0;
            double longest = 0.0;
            for (int s = 0; s < per_cu; ++s) {
                if (!slots[x][u][s].empty()) used = s + 1;
                longest = std::max(longest, sl[u][s]);
            }
            rounds = std::max(rounds, used);
            // Time in tiles of one slot's share of the CU: the CU's total
            // shared by its slots, or the longest list, which runs alone
            // once the others are done.
            const double alone = per_cu > 1 ? longest / (per_cu * kAloneShare) : longest;
            est = std::max(est, std::max(cu[u] / per_cu, alone));
        }
    }
    KeyTable t;
    t.nsplit = nsplit;
    t.est = est;
    t.num_wg = kSchedXcds * cus * rounds;
    t.wg_start.push_back(0);
    int n = 0;
    for (int w = 0; w < t.num_wg; ++w) {
        const int x = w % kSchedXcds, i = w / kSchedXcds, u = i % cus, s = i / cus;
        for (const Item &it : slots[x][u][s]) {
            t.items.insert(t.items.end(), {it.bh, it.kb, it.qa, it.qe});
            ++n;
        }
        t.wg_start.push_back(n);
    }
    return t;
}

struct DeviceTable {
    int num_wg = 0;
    int *wg_start = nullptr;
    int *items = nullptr;
    int *counters = nullptr;  // the pool's two counters (nullptr: no pool)
    SchedTable host;          // kept: the source of the stream-ordered upload
};

struct DeviceKeyTable {
    int num_wg = 0, nsplit = 0;
    int *wg_start = nullptr;
    int *items = nullptr;
    KeyTable host;  // kept: the source of the stream-ordered upload
};

std::mutex g_mu;
// (device, BH, nqt, per_cu * 1024 + cus, bh0[, max_split])
std::map<std::tuple<int, int, int, int, int>, DeviceTable> g_tables;
std::map<std::tuple<int, int, int, int, int, int>, DeviceKeyTable> g_key_tables;

// The uploads below allocate and copy from host memory, which a stream under
// graph capture cannot record: refuse with a clear message instead.
void check_not_capturing(hipStream_t stream, const char *what) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    hipCheck(hipStreamIsCapturing(stream, &st));
    CHECK_ERROR(st != hipStreamCaptureStatusNone,
                "The %s of this attention shape is built on its first call, which must not be captured into a graph: "
                "run one forward and backward of the shape before capturing.",
                what);
}
std::map<std::pair<int, const void *>, std::pair<int, int>> g_occupancy;  // (device, kernel) -> (per_cu, cus)

// (workgroups per CU, CUs per XCD) of `kernel` on device dev; g_mu held.
std::pair<int, int> occupancy_locked(int dev, const void *kernel) {
    auto occ = g_occupancy.find({dev, kernel});
    if (occ == g_occupancy.end()) {
        int per_cu = 0, cus_total = 0;
        hipCheck(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0));
        hipCheck(hipDeviceGetAttribute(&cus_total, hipDeviceAttributeMultiprocessorCount, dev));
        const int cus = std::max(1, cus_total / kSchedXcds);
        occ = g_occupancy.emplace(std::make_pair(dev, kernel), std::make_pair(std::max(1, per_cu), cus)).first;
    }
    return occ->second;
}

}  // namespace

KeyTable build_key_schedule(int BH, int nqt, int per_cu, int cus, int max_split) {
    CHECK_ERROR(BH < 0 || nqt < 1 || per_cu < 1 || cus < 1, "key schedule: unsupported shape (heads %d, tiles %d, per CU %d, CUs %d).",
                BH, nqt, per_cu, cus);
    const int nkb = (nqt + kKeyTilesPerBlock - 1) / kKeyTilesPerBlock;
    const int ns_max = max_split < 0 ? nkb : std::min(max_split, nkb);
    std::vector<KeyTable> cand;
    double best = 0.0;
    for (int ns = 0; ns <= ns_max; ++ns) {
        cand.push_back(key_schedule_with(BH, nqt, ns, per_cu, cus));
        best = ns == 0 ? cand.back().est : std::min(best, cand.back().est);
    }
    // No split unless it gains more than 5 % by the estimate: a split block
    // costs what the estimate leaves out (the zeroing of its rows, the adds,
    // a second item's V rows and epilogue).  At C5 the estimate put one split
    // 1.6 % and the best count 3.4 % ahead of none; one split measured 1 us
    // slower than none.
    if (cand.front().est <= 1.05 * best) return std::move(cand.front());
    for (KeyTable &t : cand)
        if (t.est <= 1.02 * best) return std::move(t);
    return std::move(cand.front());
}

namespace {

SchedTable build_with(int BH, int nqt, int per_cu, int cus, int j0) {
    SchedTable best = pairs_schedule(BH, nqt, j0);
    best.max_cu_load = max_cu_load(best, cus);
    SchedTable lpt = lpt_schedule(BH, nqt, per_cu, cus, j0);
    lpt.max_cu_load = max_cu_load(lpt, cus);
    // Pairs on ties when they fill every resident slot: equal cost per
    // workgroup also balances the workgroups of a CU.  With slots left over
    // (dq16 keeps four workgroups per CU, C2 has pairs for three), lists over
    // all the slots win up to a 2 % larger CU load: the extra workgroup's
    // waves cover the others' waits (dq16 at C2: 55 against 54 tiles per
    // CU, 69.8-70.2 against 70.5-71.1 us).
    const bool pairs_fill = best.num_wg >= per_cu * cus * kSchedXcds;
    if (lpt.max_cu_load < best.max_cu_load - 1e-9 || (!pairs_fill && lpt.max_cu_load <= 1.02 * best.max_cu_load))
        best = std::move(lpt);
    best.pool_j0 = j0;
    return best;
}

}  // namespace

SchedTable build_block_schedule(int BH, int nqt, int per_cu, int cus, bool pool) {
    CHECK_ERROR(BH < 0 || nqt < 1 || nqt > (1 << kSchedJBits) || per_cu < 1 || cus < 1 ||
                    static_cast<long long>(BH) >= (1LL << (31 - kSchedJBits)),
                "block schedule: unsupported shape (heads %d, blocks %d, per CU %d, CUs %d).", BH, nqt, per_cu, cus);
    if (pool && nqt > 2 * kPoolJ0) {
        SchedTable t = build_with(BH, nqt, per_cu, cus, kPoolJ0);
        bool every_list_used = true;
        for (int w = 0; w < t.num_wg; ++w) every_list_used = every_list_used && t.wg_start[w + 1] > t.wg_start[w];
        if (every_list_used) return t;
    }
    return build_with(BH, nqt, per_cu, cus, 0);
}

BlockSched device_block_schedule(int BH, int nqt, const void *kernel, hipStream_t stream, int *num_wg, int bh0,
                                 bool pool) {
    int dev = 0;
    hipCheck(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_mu);
    const auto occ = occupancy_locked(dev, kernel);
    const int per_cu = occ.first, cus = occ.second;
    const auto key = std::make_tuple(dev, BH, nqt, per_cu * 1024 + cus, bh0 * 2 + (pool ? 1 : 0));
    auto it = g_tables.find(key);
    if (it == g_tables.end()) {
        check_not_capturing(stream, "work list");
        CHECK_ERROR(static_cast<long long>(bh0) + BH >= (1LL << (31 - kSchedJBits)),
                    "block schedule: head index %d beyond the work-list format.", bh0 + BH);
        DeviceTable d;
        d.host = build_block_schedule(BH, nqt, per_cu, cus, pool);
        for (int &item : d.host.items) item += bh0 << kSchedJBits;
        if (d.host.pool_j0 > 0) {
            hipCheck(hipMalloc(&d.counters, 128 * sizeof(int)));
            hipCheck(hipMemsetAsync(d.counters, 0, 128 * sizeof(int), stream));
        }
        d.num_wg = d.host.num_wg;
        const size_t nw = d.host.wg_start.size() * sizeof(int), ni = std::max<size_t>(1, d.host.items.size()) * sizeof(int);
        hipCheck(hipMalloc(&d.wg_start, nw));
        hipCheck(hipMalloc(&d.items, ni));
        hipCheck(hipMemcpyAsync(d.wg_start, d.host.wg_start.data(), nw, hipMemcpyHostToDevice, stream));
        if (!d.host.items.empty())
            hipCheck(hipMemcpyAsync(d.items, d.host.items.data(), d.host.items.size() * sizeof(int),
                                    hipMemcpyHostToDevice, stream));
        it = g_tables.emplace(key, std::move(d)).first;
    }
    *num_wg = it->second.num_wg;
    const DeviceTable &t = it->second;
    const int j0 = t.host.pool_j0;
    return BlockSched{t.wg_start, t.items, j0 * BH, j0, BH, bh0, t.counters};
}

KeySched device_key_schedule(int BH, int nqt, const void *kernel, hipStream_t stream, int *num_wg, int *nsplit,
                             int bh0, int max_split) {
    int dev = 0;
    hipCheck(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_mu);
    const auto occ = occupancy_locked(dev, kernel);
    const int per_cu = occ.first, cus = occ.second;
    const auto key = std::make_tuple(dev, BH, nqt, per_cu * 1024 + cus, bh0, max_split);
    auto it = g_key_tables.find(key);
    if (it == g_key_tables.end()) {
        check_not_capturing(stream, "key-block work list");
        DeviceKeyTable d;
        d.host = build_key_schedule(BH, nqt, per_cu, cus, max_split);
        for (size_t i = 0; i < d.host.items.size(); i += 4) d.host.items[i] += bh0;
        d.num_wg = d.host.num_wg;
        d.nsplit = d.host.nsplit;
        const size_t nw = d.host.wg_start.size() * sizeof(int), ni = std::max<size_t>(1, d.host.items.size()) * sizeof(int);
        hipCheck(hipMalloc(&d.wg_start, nw));
        hipCheck(hipMalloc(&d.items, ni));
        hipCheck(hipMemcpyAsync(d.wg_start, d.host.wg_start.data(), nw, hipMemcpyHostToDevice, stream));
        if (!d.host.items.empty())
            hipCheck(hipMemcpyAsync(d.items, d.host.items.data(), d.host.items.size() * sizeof(int),
                                    hipMemcpyHostToDevice, stream));
        it = g_key_tables.emplace(key, std::move(d)).first;
    }
    *num_wg = it->second.num_wg;
    *nsplit = it->second.nsplit;
    return KeySched{it->second.wg_start, it->second.items};
}

}  // namespace gptc

// Host-side view of a table, for tests: fills wg_start (num_wg + 1 ints)
// and items (cap ints) and returns num_wg (-1 if cap is too small).
// per_cu and cus describe the GPU the table is built for.
extern "C" int gptc_attention_block_schedule(int BH, int nqt, int per_cu, int cus, int *wg_start, int *items,
                                             int cap, double *max_cu_load, int *used_pairs) {
    const gptc::SchedTable t = gptc::build_block_schedule(BH, nqt, per_cu, cus);
    if (static_cast<int>(t.items.size()) > cap || t.num_wg + 1 > cap) return -1;
    std::copy(t.wg_start.begin(), t.wg_start.end(), wg_start);
    std::copy(t.items.begin(), t.items.end(), items);
    if (max_cu_load) *max_cu_load = t.max_cu_load;
    if (used_pairs) *used_pairs = t.pairs ? 1 : 0;
    return t.num_wg;
}

// The same with the pool (the table device_block_schedule builds with pool
// true): fills the lists like gptc_attention_block_schedule and returns
// num_wg; *pool_j0 receives the pool's blocks per head (0: no pool).
extern "C" int gptc_attention_block_schedule_pool(int BH, int nqt, int per_cu, int cus, int *wg_start, int *items,
                                                  int cap, int *pool_j0) {
    const gptc::SchedTable t = gptc::build_block_schedule(BH, nqt, per_cu, cus, true);
    if (static_cast<int>(t.items.size()) > cap || t.num_wg + 1 > cap) return -1;
    std::copy(t.wg_start.begin(), t.wg_start.end(), wg_start);
    std::copy(t.items.begin(), t.items.end(), items);
    if (pool_j0) *pool_j0 = t.pool_j0;
    return t.num_wg;
}

// Host-side view of a dk/dv key-block table, for tests: fills wg_start
// (num_wg + 1 ints, in items) and items (4 ints each, cap ints in all) and
// returns num_wg (-1 if cap is too small).
extern "C" int gptc_attention_key_schedule(int BH, int nqt, int per_cu, int cus, int *wg_start, int *items, int cap,
                                           double *est, int *nsplit) {
    const gptc::KeyTable t = gptc::build_key_schedule(BH, nqt, per_cu, cus);
    if (static_cast<int>(t.items.size()) > cap || t.num_wg + 1 > cap) return -1;
    std::copy(t.wg_start.begin(), t.wg_start.end(), wg_start);
    std::copy(t.items.begin(), t.items.end(), items);
    if (est) *est = t.est;
    if (nsplit) *nsplit = t.nsplit;
    return t.num_wg;
}
