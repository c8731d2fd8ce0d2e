// SW32 host format builder and panel-task planner.
//
// Output contract: byte-identical arrays to the reference's convertCsrToSw32 / buildPanelTasks
// (src/format/sw32.cpp:25-167) for the same canonical CSR — the device kernel and every
// descriptor consumer depend on that layout. The construction is our own: instead of a
// single-threaded 32-way heap merge, each SW sorts its (source, row) keys, and SW blocks are built
// in parallel into private buffers that are stitched together with offset fix-ups afterwards.
#include "format/sw32.h"
#include "../parallel.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <limits>
#include <stdexcept>

namespace {

constexpr std::uint32_t kPad = std::numeric_limits<std::uint32_t>::max();

std::uint32_t fit32(std::uint64_t n) {
    if (n > std::numeric_limits<std::uint32_t>::max())
        throw std::overflow_error("source-mask format exceeds uint32 offsets");
    return static_cast<std::uint32_t>(n);
}

// 4-bit mask of the 8-row groups touched by a 32-bit row mask.
inline unsigned groupsOf(std::uint32_t rowMask) {
    unsigned g = 0;
    for (unsigned rw = 0; rw < 4; ++rw)
        g |= unsigned((rowMask >> (8 * rw)) & 0xFFu ? 1u : 0u) << rw;
    return g;
}

// One block of consecutive SWs, with block-local panel and value numbering.
struct WindowBlock {
    std::vector<std::uint32_t> sourceIds, rowGroupMasks, bucketOffsets, windowEnds;
    std::vector<std::uint64_t> metadata; // value base is block-local here
    std::vector<float> values;
};

struct Entry {
    std::uint64_t key; // source << 5 | local row
    std::uint32_t pos; // index into the CSR arrays
};

struct Item {
    std::uint32_t source, mask, first; // first = index of its first Entry in the sorted list
};

// Entry-level defects of one SW, reported as the reference's converter meets them. It visits the
// SW's entries in ascending (source, row) order, one cursor per row (src/format/sw32.cpp:96-120):
// a source at or past `cols` fails when it is first reached, before its entry's value is checked;
// an entry's value is checked when it is visited; and the entry that follows it in its row must
// have a larger source, checked right after the value. So within a row, the checks run in entry
// order and stop at the first defect; across rows, the defect reported is the one with the
// smallest key (source, row, check), check = 0 column range, 1 value, 2 order of the next entry.
class SwDefect {
public:
    void note(std::uint32_t source, std::uint32_t row, unsigned check) {
        const std::uint64_t key = (std::uint64_t(source) << 32) | (std::uint64_t(row) << 2) | check;
        if (key < key_) key_ = key;
    }
    void raise() const {
        if (key_ == kNone) return;
        switch (unsigned(key_ & 3u)) {
        case 0: throw std::invalid_argument("source-mask source outside column range");
        case 1: throw std::invalid_argument("source-mask requires finite nonzero values");
        default: throw std::invalid_argument("source-mask requires increasing row sources");
        }
    }

private:
    static constexpr std::uint64_t kNone = ~std::uint64_t(0);
    std::uint64_t key_ = kNone;
};

void buildBlock(std::uint32_t rows, std::uint32_t cols, const CsrMatrix& csr, bool bucketed,
                std::uint32_t swBegin, std::uint32_t swEnd, WindowBlock& out) {
    std::vector<Entry> entries;
    std::array<std::vector<Item>, 16> buckets;
    for (std::uint32_t sw = swBegin; sw < swEnd; ++sw) {
        const std::uint64_t base = std::uint64_t(sw) * 32;
        const std::uint32_t count = std::uint32_t(std::min<std::uint64_t>(32, rows - base));
        entries.clear();
        SwDefect defect;
        for (std::uint32_t r = 0; r < count; ++r) {
            const std::size_t row = base + r;
            const std::uint32_t e0 = csr.rowOffsets[row], e1 = csr.rowOffsets[row + 1];
            for (std::uint32_t e = e0; e < e1; ++e) {
                const std::uint32_t s = csr.sourceIds[e];
                const float v = csr.values[e];
                const unsigned check = s >= cols                         ? 0u
                                       : (!std::isfinite(v) || v == 0)   ? 1u
                                       : (e + 1 < e1 && csr.sourceIds[e + 1] <= s) ? 2u
                                                                         : 3u;
                if (check < 3) {
                    defect.note(s, r, check);
                    break; // the rest of this row is never reached
                }
                entries.push_back({(std::uint64_t(s) << 5) | r, e});
            }
        }
        defect.raise();
        std::sort(entries.begin(), entries.end(),
                  [](const Entry& a, const Entry& b) { return a.key < b.key; });
        for (auto& b : buckets) b.clear();
        for (std::size_t i = 0; i < entries.size();) {
            const std::uint32_t source = std::uint32_t(entries[i].key >> 5);
            Item item{source, 0, std::uint32_t(i)};
            while (i < entries.size() && std::uint32_t(entries[i].key >> 5) == source)
                item.mask |= 1u << (entries[i++].key & 31);
            buckets[bucketed ? groupsOf(item.mask) : 0].push_back(item);
        }
        for (unsigned slot = 0; slot < 16; ++slot) {
            const auto& bucket = buckets[sw32BucketOrder[slot]];
            if (bucketed) out.bucketOffsets.push_back(std::uint32_t(out.rowGroupMasks.size()));
            unsigned inPanel = 0, panelMask = 0;
            for (const Item& item : bucket) {
                out.sourceIds.push_back(item.source);
                out.metadata.push_back((std::uint64_t(out.values.size()) << 32) | item.mask);
                const unsigned n = unsigned(__builtin_popcount(item.mask));
                for (unsigned k = 0; k < n; ++k)
                    out.values.push_back(csr.values[entries[item.first + k].pos]);
                panelMask |= groupsOf(item.mask);
                if (++inPanel == 8) {
                    out.rowGroupMasks.push_back(panelMask);
                    inPanel = panelMask = 0;
                }
            }
            if (inPanel) {
                for (; inPanel < 8; ++inPanel) {
                    out.sourceIds.push_back(kPad);
                    out.metadata.push_back(0);
                }
                out.rowGroupMasks.push_back(panelMask);
            }
        }
        if (bucketed) out.bucketOffsets.push_back(std::uint32_t(out.rowGroupMasks.size()));
        out.windowEnds.push_back(std::uint32_t(out.rowGroupMasks.size()));
    }
}

} // namespace

void buildPanelTasks(Sw32HostFormat& format) {
    if (format.windowOffsets.empty())
        throw std::invalid_argument("SW32 format has no window offsets");
    const std::uint32_t windows = fit32(format.windowOffsets.size() - 1);
    if (format.bucketOffsets.size() != std::size_t(windows) * 17)
        throw std::invalid_argument("panel tasks need the RW-bucketed SW32 format");
    format.tasks.clear();
    format.reductions.clear();
    format.partialIds.clear();
    format.tasks.reserve(windows);
    std::array<std::vector<std::uint32_t>, 4> groupTiles;
    std::uint64_t tiles = 0;
    for (std::uint32_t sw = 0; sw < windows; ++sw) {
        const std::uint32_t first = format.windowOffsets[sw], last = format.windowOffsets[sw + 1];
        const std::uint32_t panels = last - first;
        if (panels <= sw32TaskPanelLimit) {
            format.tasks.push_back({sw, first, last, kPad, 15, 1, 0});
            continue;
        }
        const std::uint32_t chunks = (panels + sw32TaskPanelLimit - 1) / sw32TaskPanelLimit;
        const std::uint32_t reduceFirst = fit32(format.reductions.size());
        for (auto& g : groupTiles) g.clear();
        const std::uint32_t* slotBounds = format.bucketOffsets.data() + std::size_t(sw) * 17;
        for (std::uint32_t c = 0; c < chunks; ++c) {
            const std::uint32_t begin = first + c * sw32TaskPanelLimit;
            const std::uint32_t end = std::min(last, begin + sw32TaskPanelLimit);
            // Row groups of every bucket (slots 1..15) overlapping this chunk.
            std::uint32_t mask = 0;
            for (unsigned slot = 1; slot < 16; ++slot) {
                const std::uint32_t lo = slotBounds[slot], hi = slotBounds[slot + 1];
                if (std::max(begin, lo) < std::min(end, hi)) mask |= sw32BucketOrder[slot];
            }
            format.tasks.push_back({sw, begin, end, fit32(tiles), mask, chunks, reduceFirst});
            for (unsigned rw = 0; rw < 4; ++rw)
                if (mask >> rw & 1u) groupTiles[rw].push_back(fit32(tiles++));
        }
        for (const auto& g : groupTiles) {
            const std::uint32_t begin = fit32(format.partialIds.size());
            format.partialIds.insert(format.partialIds.end(), g.begin(), g.end());
            format.reductions.push_back({begin, fit32(format.partialIds.size())});
        }
    }
    fit32(format.tasks.size());
    fit32(format.reductions.size());
    format.partialCount = fit32(tiles);
}

namespace {
// The CSR must describe `rows` x `cols`: rows + 1 offsets running from 0 to the entry count without
// decreasing, one value per source id. (The exception messages are the reference's, part of the
// observable behaviour.) Entry-level rules are checked per SW while the stream is built.
void requireCsrLayout(std::uint32_t rows, std::uint32_t cols, const CsrMatrix& csr) {
    const std::vector<std::uint32_t>& off = csr.rowOffsets;
    const std::size_t entries = csr.sourceIds.size();
    const bool sized = rows != 0 && cols != 0 && off.size() == std::size_t(rows) + 1 &&
                       csr.values.size() == entries;
    if (!sized || off.front() != 0 || off.back() != entries)
        throw std::invalid_argument("invalid canonical CSR for source-mask SW32");
    if (!std::is_sorted(off.begin(), off.end()))
        throw std::invalid_argument("decreasing CSR offsets");
}
} // namespace

Sw32HostFormat convertCsrToSw32(std::uint32_t rows, std::uint32_t cols, const CsrMatrix& csr,
                                bool bucketByRwMask) {
    requireCsrLayout(rows, cols, csr);

    const std::uint32_t windows = std::uint32_t((std::uint64_t(rows) + 31) / 32);
    // Blocks of consecutive SWs balanced by entry count, so power-law rows do not serialise.
    const std::size_t target = std::max<std::size_t>(1, std::min<std::size_t>(windows, 4096));
    std::vector<std::uint32_t> cut{0};
    {
        const std::uint64_t total = csr.sourceIds.size();
        std::uint64_t next = total / target;
        for (std::uint32_t w = 1; w < windows; ++w) {
            const std::uint64_t at = csr.rowOffsets[std::size_t(w) * 32];
            if (at >= next || w - cut.back() >= 65536) {
                cut.push_back(w);
                next = at + std::max<std::uint64_t>(1, total / target);
            }
        }
        cut.push_back(windows);
    }
    const std::size_t blocks = cut.size() - 1;
    std::vector<WindowBlock> parts(blocks);
    tcc::parallelChunks(blocks, blocks, [&](std::size_t b, std::size_t, std::size_t) {
        buildBlock(rows, cols, csr, bucketByRwMask, cut[b], cut[b + 1], parts[b]);
    });

    std::vector<std::uint64_t> slotAt(blocks + 1, 0), panelAt(blocks + 1, 0), valueAt(blocks + 1, 0);
    for (std::size_t b = 0; b < blocks; ++b) {
        slotAt[b + 1] = slotAt[b] + parts[b].sourceIds.size();
        panelAt[b + 1] = panelAt[b] + parts[b].rowGroupMasks.size();
        valueAt[b + 1] = valueAt[b] + parts[b].values.size();
    }
    fit32(panelAt[blocks]);
    fit32(valueAt[blocks]);

    Sw32HostFormat out;
    out.rows = rows;
    out.cols = cols;
    out.windowOffsets.assign(std::size_t(windows) + 1, 0);
    out.sourceIds.resize(slotAt[blocks]);
    out.sourceMetadata.resize(slotAt[blocks]);
    out.rowGroupMasks.resize(panelAt[blocks]);
    out.values.resize(valueAt[blocks]);
    if (bucketByRwMask) out.bucketOffsets.resize(std::size_t(windows) * 17);
    tcc::parallelChunks(blocks, blocks, [&](std::size_t b, std::size_t, std::size_t) {
        const WindowBlock& p = parts[b];
        const std::uint32_t panel0 = std::uint32_t(panelAt[b]);
        const std::uint64_t value0 = valueAt[b];
        std::copy_n(p.sourceIds.begin(), p.sourceIds.size(), out.sourceIds.begin() + slotAt[b]);
        for (std::size_t i = 0; i < p.metadata.size(); ++i) {
            const std::uint64_t m = p.metadata[i];
            // Padding slots keep metadata 0; real slots get the global value base.
            out.sourceMetadata[slotAt[b] + i] =
                p.sourceIds[i] == kPad ? m : m + (value0 << 32);
        }
        std::copy_n(p.rowGroupMasks.begin(), p.rowGroupMasks.size(),
                    out.rowGroupMasks.begin() + panelAt[b]);
        std::copy_n(p.values.begin(), p.values.size(), out.values.begin() + value0);
        for (std::size_t i = 0; i < p.windowEnds.size(); ++i)
            out.windowOffsets[cut[b] + 1 + i] = p.windowEnds[i] + panel0;
        for (std::size_t i = 0; i < p.bucketOffsets.size(); ++i)
            out.bucketOffsets[std::size_t(cut[b]) * 17 + i] = p.bucketOffsets[i] + panel0;
    });
    parts.clear();
    if (bucketByRwMask) buildPanelTasks(out);
    return out;
}
