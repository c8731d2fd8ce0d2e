// merge_model.cpp — CPU model of the split-SW completion protocol of the SpMM kernel.
//
// TEST INFRASTRUCTURE ONLY (tests/test_merge_protocol.py runs it; the product library never links
// it). It restates, for host threads, what the kernel in tcc_spmm_amd/csrc/kernel/spmm.hip does at
// the end of a split task (runTask, mergeSlice), following the protocol of the reference
// (src/kernel/spmm_kernel.cuh:228-282):
//   - a split task writes its row groups of task.mask as 8-row partial tiles [tile][8][F];
//   - per 128-feature slice it takes a ticket: an atomic wrapping increment of
//     counters[sw * F/128 + slice] with limit chunks - 1 (old >= limit ? 0 : old + 1, the
//     semantics of the GPU's atomic_inc), acquire-release, so the counter returns to zero by itself;
//   - the task whose ticket is chunks - 1 merges the slice: per row group, the tiles of the
//     group's reduction range summed in partialIds order from 0.0f, with the kernel's lane layout
//     (lane L: row L >> 3, columns slice * 128 + (L & 7) * 4 + 32 j + t), its 64-id chunks and
//     its batches of four tiles, then writes Y.
//
// Modes (one JSON line on stdout; exit status 0 when every check holds, 1 when one fails, 2 on a
// usage or input error):
//   merge_model map <plan>
//       lane-map check on every split SW, slice and row group of the plan: every element of the
//       8 x 128 block is summed by exactly one lane, from every tile of the range exactly once, in
//       partialIds order, and written to Y exactly once.
//   merge_model map-lengths <F> <n>...
//       the same for single reduction ranges of n tiles each (synthetic, distinct tile ids).
//   merge_model run <plan> <threads> <launches> <workspaces> <seed>
//       the protocol on host threads: every split task of every workspace, in a shuffled order with
//       random delays between the tile writes and the tickets, repeated for several launches on
//       the same counters. Checks: exactly one merger per (SW, slice) and launch, counters at zero
//       after every launch, and every merged Y element bitwise equal to the serial sum of the tile
//       values in partialIds order (which also shows the merger saw every tile's final contents).
//   merge_model --plant <mistake> <mode> ...
//       the same with a mistake planted in the model, to show that the checks catch it:
//       relaxed       relaxed tickets and no acquire fence: nothing orders the mergers' tile reads
//                     after the other tasks' writes (for the ThreadSanitizer build to report);
//       batch-order   the tiles of a batch added last to first;
//       ticket-limit  the ticket wraps at chunks instead of chunks - 1.
//
// Plan file (little-endian u32): magic 0x50434354, version 1, features, rows, taskCount,
// reductionCount, partialIdCount, partialCount, then tasks [taskCount][7] (sw, begin, end,
// partial, mask, chunks, reduceFirst), reductions [reductionCount][2] (begin, end), partialIds.
#include <algorithm>
#include <atomic>
#include <cinttypes>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr std::uint32_t kNoPartial = 0xFFFFFFFFu;
constexpr unsigned kWave = 64, kSlice = 128, kMergeBatch = 4;

enum Plant { kNoPlant, kRelaxed, kBatchOrder, kTicketLimit };
Plant gPlant = kNoPlant; // a mistake planted on purpose (--plant), to test the checks

struct Task {
    std::uint32_t sw, begin, end, partial, mask, chunks, reduceFirst;
};
struct Range {
    std::uint32_t begin, end;
};
struct Plan {
    std::uint32_t features = 0, rows = 0, partialCount = 0;
    std::vector<Task> tasks;
    std::vector<Range> reductions;
    std::vector<std::uint32_t> partialIds;
};

bool readPlan(const char* path, Plan& p) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    std::uint32_t h[8];
    bool ok = std::fread(h, 4, 8, f) == 8 && h[0] == 0x50434354u && h[1] == 1;
    if (ok) {
        p.features = h[2];
        p.rows = h[3];
        p.partialCount = h[7];
        p.tasks.resize(h[4]);
        p.reductions.resize(h[5]);
        p.partialIds.resize(h[6]);
        ok = std::fread(p.tasks.data(), sizeof(Task), h[4], f) == h[4] &&
             std::fread(p.reductions.data(), sizeof(Range), h[5], f) == h[5] &&
             std::fread(p.partialIds.data(), 4, h[6], f) == h[6];
    }
    std::fclose(f);
    return ok && (p.features == 128 || p.features == 256);
}

// ---- lane map ------------------------------------------------------------------------------

// One row group's merge as the kernel walks it: calls add(lane, tileId, row, col) for every
// addition in the order a lane performs them, then store(lane, row, col) for its Y writes.
template <class Add, class Store>
void walkMerge(const std::uint32_t* ids, std::uint32_t begin, std::uint32_t end, unsigned slice,
               Add add, Store store) {
    for (unsigned lane = 0; lane < kWave; ++lane) {
        const unsigned mrow = lane >> 3, mcol = slice * kSlice + (lane & 7) * 4;
        auto tile = [&](std::uint32_t id) {
            for (unsigned j = 0; j < 4; ++j)
                for (unsigned t = 0; t < 4; ++t) add(lane, id, mrow, mcol + 32 * j + t);
        };
        for (std::uint32_t base = begin; base < end; base += kWave) {
            const unsigned items = std::min<std::uint32_t>(end - base, kWave);
            // Lane l of the wave holds ids[base + min(l, items - 1)]; readlane(i) broadcasts id i.
            auto readlane = [&](unsigned i) { return ids[base + std::min(i, items - 1)]; };
            unsigned i = 0;
            for (; i + kMergeBatch <= items; i += kMergeBatch) {
                // The batch's loads are issued first and added afterwards, in order: per element
                // the additions are those of the batch's tiles in increasing i.
                for (unsigned u = 0; u < kMergeBatch; ++u)
                    tile(readlane(gPlant == kBatchOrder ? i + kMergeBatch - 1 - u : i + u));
            }
            for (; i < items; ++i) tile(readlane(i));
        }
        for (unsigned j = 0; j < 4; ++j)
            for (unsigned t = 0; t < 4; ++t) store(lane, mrow, mcol + 32 * j + t);
    }
}

// Checks one range; returns an empty string or the first failure.
std::string checkRange(const std::uint32_t* ids, std::uint32_t begin, std::uint32_t end,
                       unsigned slice) {
    const std::uint32_t n = end - begin;
    std::vector<std::vector<std::uint32_t>> seq(8 * kSlice);
    std::vector<int> owner(8 * kSlice, -1), stores(8 * kSlice, 0);
    std::string err;
    walkMerge(ids, begin, end, slice,
              [&](unsigned lane, std::uint32_t id, unsigned row, unsigned col) {
                  const unsigned e = row * kSlice + (col - slice * kSlice);
                  if (col < slice * kSlice || col >= (slice + 1) * kSlice || row >= 8) {
                      if (err.empty()) err = "element outside the slice's row group";
                      return;
                  }
                  if (owner[e] < 0) owner[e] = int(lane);
                  else if (owner[e] != int(lane) && err.empty())
                      err = "element summed by two lanes";
                  seq[e].push_back(id);
              },
              [&](unsigned, unsigned row, unsigned col) {
                  ++stores[row * kSlice + (col - slice * kSlice)];
              });
    if (!err.empty()) return err;
    for (unsigned e = 0; e < 8 * kSlice; ++e) {
        if (owner[e] < 0 && n > 0) return "element never summed"; // an empty range writes 0
        if (stores[e] != 1) return "element not written exactly once";
        if (seq[e].size() != n) return "element summed a wrong number of times";
        for (std::uint32_t k = 0; k < n; ++k)
            if (seq[e][k] != ids[begin + k]) return "tiles not added in partialIds order";
    }
    return "";
}

int mapPlan(const Plan& p) {
    const unsigned slices = p.features / kSlice;
    std::uint64_t ranges = 0, maxLen = 0;
    std::vector<bool> seen;
    for (const Task& t : p.tasks) {
        if (t.partial == kNoPartial) continue;
        // Every task of a split SW names the same ranges; check them once per SW.
        if (t.sw >= seen.size()) seen.resize(std::size_t(t.sw) + 1, false);
        if (seen[t.sw]) continue;
        seen[t.sw] = true;
        if (std::uint64_t(t.reduceFirst) + 4 > p.reductions.size()) {
            std::printf("{\"ok\": false, \"error\": \"reduceFirst outside reductions\"}\n");
            return 1;
        }
        for (unsigned g = 0; g < 4; ++g) {
            const Range r = p.reductions[t.reduceFirst + g];
            if (r.end < r.begin || r.end > p.partialIds.size()) {
                std::printf("{\"ok\": false, \"error\": \"reduction range outside partialIds\"}\n");
                return 1;
            }
            for (unsigned k = 0; k < slices; ++k) {
                const std::string err = checkRange(p.partialIds.data(), r.begin, r.end, k);
                if (!err.empty()) {
                    std::printf("{\"ok\": false, \"error\": \"%s\", \"sw\": %u, \"group\": %u}\n",
                                err.c_str(), t.sw, g);
                    return 1;
                }
            }
            ++ranges;
            maxLen = std::max<std::uint64_t>(maxLen, r.end - r.begin);
        }
    }
    std::printf("{\"ok\": true, \"ranges\": %" PRIu64 ", \"max_tiles\": %" PRIu64 "}\n", ranges,
                maxLen);
    return 0;
}

int mapLengths(unsigned features, const std::vector<std::uint32_t>& lengths) {
    std::mt19937 rng(12345);
    for (std::uint32_t n : lengths) {
        std::vector<std::uint32_t> ids(n);
        for (std::uint32_t i = 0; i < n; ++i) ids[i] = 3 * i + 7;
        std::shuffle(ids.begin(), ids.end(), rng); // partialIds need not be increasing
        for (unsigned k = 0; k < features / kSlice; ++k) {
            const std::string err = checkRange(ids.data(), 0, n, k);
            if (!err.empty()) {
                std::printf("{\"ok\": false, \"error\": \"%s\", \"tiles\": %u}\n", err.c_str(), n);
                return 1;
            }
        }
    }
    std::printf("{\"ok\": true, \"lengths\": %zu}\n", lengths.size());
    return 0;
}

// ---- protocol on host threads ----------------------------------------------------------------

std::uint64_t mix(std::uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// The value a task leaves in element (row, col) of partial tile `id` in launch `launch`: spread
// over 40 binades with both signs, so that the FP32 sum depends on the order of the additions.
float tileValue(std::uint32_t id, unsigned launch, unsigned row, unsigned col) {
    const std::uint64_t h = mix((std::uint64_t(id) << 32) ^ (std::uint64_t(launch) << 20) ^
                                (row << 12) ^ col);
    const float m = 1.0f + float(h & 0xFFFFFF) / 16777216.0f;
    const int e = int((h >> 24) % 40) - 20;
    return std::ldexp((h >> 40) & 1 ? -m : m, e);
}

struct Workspace {
    std::unique_ptr<std::atomic<std::uint32_t>[]> counters, mergers;
    std::vector<float> partials, y;
};

// GPU atomic_inc with limit `limit`: returns the old value and stores old >= limit ? 0 : old + 1.
std::uint32_t wrappingTicket(std::atomic<std::uint32_t>& c, std::uint32_t limit, bool relaxed) {
    std::uint32_t old = c.load(std::memory_order_relaxed);
    const auto order = relaxed ? std::memory_order_relaxed : std::memory_order_acq_rel;
    while (!c.compare_exchange_weak(old, old >= limit ? 0u : old + 1u, order,
                                    std::memory_order_relaxed)) {
    }
    return old;
}

void runTask(const Plan& p, Workspace& ws, const Task& task, unsigned launch, std::mt19937& rng) {
    const bool relaxed = gPlant == kRelaxed;
    const unsigned F = p.features, slices = F / kSlice;
    // Partial tiles of the row groups in task.mask.
    for (unsigned rw = 0; rw < 4; ++rw) {
        if (!((task.mask >> rw) & 1u)) continue;
        const std::uint32_t id = task.partial + unsigned(__builtin_popcount(task.mask & ((1u << rw) - 1u)));
        for (unsigned r = 0; r < 8; ++r)
            for (unsigned c = 0; c < F; ++c)
                ws.partials[(std::size_t(id) * 8 + r) * F + c] = tileValue(id, launch, r, c);
    }
    // A random delay between the writes and the tickets varies the arrival order.
    const unsigned spin = rng() % 2000;
    for (volatile unsigned i = 0; i < spin; i = i + 1) {
    }
    if (rng() % 4 == 0) std::this_thread::yield();
    bool last[2] = {false, false};
    for (unsigned k = 0; k < slices; ++k) {
        const std::uint32_t ticket =
            wrappingTicket(ws.counters[std::size_t(task.sw) * slices + k],
                           gPlant == kTicketLimit ? task.chunks : task.chunks - 1, relaxed);
        last[k] = ticket == task.chunks - 1;
    }
    for (unsigned k = 0; k < slices; ++k) {
        if (!last[k]) continue;
        if (!relaxed) std::atomic_thread_fence(std::memory_order_acquire);
        ws.mergers[std::size_t(task.sw) * slices + k].fetch_add(1, std::memory_order_relaxed);
        for (unsigned g = 0; g < 4; ++g) {
            const Range red = p.reductions[task.reduceFirst + g];
            const std::uint32_t row0 = task.sw * 32 + g * 8;
            if (row0 >= p.rows) continue;
            float sum[kWave][16] = {};
            walkMerge(p.partialIds.data(), red.begin, red.end, k,
                      [&](unsigned lane, std::uint32_t id, unsigned row, unsigned col) {
                          const unsigned slot = ((col - k * kSlice - (lane & 7) * 4) / 32) * 4 +
                                                (col - k * kSlice - (lane & 7) * 4) % 32;
                          sum[lane][slot] += ws.partials[(std::size_t(id) * 8 + row) * F + col];
                      },
                      [&](unsigned lane, unsigned row, unsigned col) {
                          const unsigned slot = ((col - k * kSlice - (lane & 7) * 4) / 32) * 4 +
                                                (col - k * kSlice - (lane & 7) * 4) % 32;
                          if (row0 + row < p.rows)
                              ws.y[std::size_t(row0 + row) * F + col] = sum[lane][slot];
                      });
        }
    }
}

int runPlan(const Plan& p, unsigned threads, unsigned launches, unsigned workspaces,
            unsigned seed) {
    const unsigned F = p.features, slices = F / kSlice;
    std::uint32_t nSW = 0;
    std::vector<std::uint32_t> split; // indices of split tasks
    for (std::uint32_t t = 0; t < p.tasks.size(); ++t) {
        nSW = std::max(nSW, p.tasks[t].sw + 1);
        if (p.tasks[t].partial != kNoPartial) split.push_back(t);
    }
    std::vector<Workspace> ws(workspaces);
    for (Workspace& w : ws) {
        w.counters.reset(new std::atomic<std::uint32_t>[std::size_t(nSW) * slices]);
        w.mergers.reset(new std::atomic<std::uint32_t>[std::size_t(nSW) * slices]);
        for (std::size_t i = 0; i < std::size_t(nSW) * slices; ++i) w.counters[i] = 0;
        w.partials.assign(std::size_t(p.partialCount) * 8 * F, 0.0f);
        w.y.assign(std::size_t(p.rows) * F, std::nanf(""));
    }
    // Which tile ids each split SW's ranges name (for the serial expectation).
    std::uint64_t checked = 0, merges = 0;
    for (unsigned launch = 0; launch < launches; ++launch) {
        for (Workspace& w : ws)
            for (std::size_t i = 0; i < std::size_t(nSW) * slices; ++i) w.mergers[i] = 0;
        std::vector<std::pair<unsigned, std::uint32_t>> work;
        for (unsigned w = 0; w < workspaces; ++w)
            for (std::uint32_t t : split) work.push_back({w, t});
        std::mt19937 shuffler(seed * 7919u + launch);
        std::shuffle(work.begin(), work.end(), shuffler);
        std::atomic<std::size_t> next{0};
        std::vector<std::thread> pool;
        for (unsigned th = 0; th < threads; ++th) {
            pool.emplace_back([&, th] {
                std::mt19937 rng(seed * 131u + launch * 977u + th);
                for (std::size_t i; (i = next.fetch_add(1, std::memory_order_relaxed)) < work.size();)
                    runTask(p, ws[work[i].first], p.tasks[work[i].second], launch, rng);
            });
        }
        for (auto& t : pool) t.join();
        // Checks after the launch (the joins order them after every task).
        for (unsigned w = 0; w < workspaces; ++w) {
            for (std::size_t i = 0; i < std::size_t(nSW) * slices; ++i)
                if (ws[w].counters[i].load() != 0) {
                    std::printf("{\"ok\": false, \"error\": \"counter not back at zero\", "
                                "\"launch\": %u, \"workspace\": %u, \"counter\": %zu}\n",
                                launch, w, i);
                    return 1;
                }
            for (std::size_t s = 0; s < split.size(); ++s) {
                const Task& t = p.tasks[split[s]];
                if (s > 0 && p.tasks[split[s - 1]].sw == t.sw) continue; // once per SW
                for (unsigned k = 0; k < slices; ++k) {
                    if (ws[w].mergers[std::size_t(t.sw) * slices + k].load() != 1) {
                        std::printf("{\"ok\": false, \"error\": \"not exactly one merger\", "
                                    "\"launch\": %u, \"sw\": %u, \"slice\": %u}\n", launch, t.sw, k);
                        return 1;
                    }
                    ++merges;
                    for (unsigned g = 0; g < 4; ++g) {
                        const Range red = p.reductions[t.reduceFirst + g];
                        for (unsigned r = 0; r < 8; ++r) {
                            const std::uint32_t row = t.sw * 32 + g * 8 + r;
                            if (row >= p.rows) continue;
                            for (unsigned c = k * kSlice; c < (k + 1) * kSlice; ++c) {
                                float want = 0.0f;
                                for (std::uint32_t q = red.begin; q < red.end; ++q)
                                    want += tileValue(p.partialIds[q], launch, r, c);
                                const float got = ws[w].y[std::size_t(row) * F + c];
                                if (std::memcmp(&got, &want, 4) != 0) {
                                    std::printf("{\"ok\": false, \"error\": \"merged value differs "
                                                "from the serial sum\", \"launch\": %u, \"row\": %u,"
                                                " \"col\": %u}\n", launch, row, c);
                                    return 1;
                                }
                                ++checked;
                            }
                        }
                    }
                }
            }
        }
    }
    std::printf("{\"ok\": true, \"split_tasks\": %zu, \"merges\": %" PRIu64 ", \"elements\": %" PRIu64
                ", \"launches\": %u, \"workspaces\": %u, \"threads\": %u}\n",
                split.size(), merges, checked, launches, workspaces, threads);
    return 0;
}

} // namespace

int main(int argc, char** argv) {
    if (argc >= 3 && std::strcmp(argv[1], "--plant") == 0) {
        if (std::strcmp(argv[2], "relaxed") == 0) gPlant = kRelaxed;
        else if (std::strcmp(argv[2], "batch-order") == 0) gPlant = kBatchOrder;
        else if (std::strcmp(argv[2], "ticket-limit") == 0) gPlant = kTicketLimit;
        else return 2;
        argc -= 2;
        argv += 2;
    }
    if (argc >= 3 && std::strcmp(argv[1], "map") == 0) {
        Plan p;
        if (!readPlan(argv[2], p)) return 2;
        return mapPlan(p);
    }
    if (argc >= 4 && std::strcmp(argv[1], "map-lengths") == 0) {
        std::vector<std::uint32_t> lengths;
        for (int i = 3; i < argc; ++i) lengths.push_back(std::uint32_t(std::strtoul(argv[i], nullptr, 10)));
        const unsigned F = unsigned(std::strtoul(argv[2], nullptr, 10));
        if (F != 128 && F != 256) return 2;
        return mapLengths(F, lengths);
    }
    if (argc >= 7 && std::strcmp(argv[1], "run") == 0) {
        Plan p;
        if (!readPlan(argv[2], p)) return 2;
        return runPlan(p, unsigned(std::atoi(argv[3])), unsigned(std::atoi(argv[4])),
                       unsigned(std::atoi(argv[5])), unsigned(std::atoi(argv[6])));
    }
    std::fprintf(stderr, "usage: merge_model [--plant relaxed|batch-order|ticket-limit] "
                         "map <plan> | map-lengths <F> <n>... | "
                         "run <plan> <threads> <launches> <workspaces> <seed>\n");
    return 2;
}
