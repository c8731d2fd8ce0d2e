// Canonical CSR construction (host). Mirrors the behaviour of the reference's makeCanonicalCsr
// (src/format/csr.cpp:6-40) — same validation, same stable column order, same FP32 duplicate
// sums in input order, same dropped zero sums — but works on row blocks in parallel: each block
// canonicalises into its own buffers, then the blocks are stitched together in row order.
#include "format/csr.h"
#include "../parallel.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <utility>

namespace {
struct Block {
    std::vector<std::uint32_t> cols, rowCounts;
    std::vector<float> vals;
};
} // namespace

CsrMatrix makeCanonicalCsr(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                           const std::uint32_t* rowOffsets, const std::uint32_t* sourceIds,
                           const float* values) {
    // Shape and offset validation happens before any row is touched (reference csr.cpp:9-13).
    if (!rows || !cols || rowOffsets[0] || rowOffsets[rows] != nnz)
        throw std::invalid_argument("invalid CSR dimensions or offsets");
    for (std::uint32_t row = 0; row < rows; ++row)
        if (rowOffsets[row] > rowOffsets[row + 1] || rowOffsets[row + 1] > nnz)
            throw std::invalid_argument("invalid CSR offsets");

    const std::size_t blocks = std::min<std::size_t>(rows, 1024);
    std::vector<Block> parts(blocks);
    tcc::parallelChunks(rows, blocks, [&](std::size_t b, std::size_t r0, std::size_t r1) {
        Block& out = parts[b];
        out.rowCounts.resize(r1 - r0);
        std::vector<std::pair<std::uint32_t, float>> entries;
        for (std::size_t r = r0; r < r1; ++r) {
            const std::uint32_t e0 = rowOffsets[r], e1 = rowOffsets[r + 1];
            entries.clear();
            bool sorted = true;
            for (std::uint32_t e = e0; e < e1; ++e) {
                if (sourceIds[e] >= cols || !std::isfinite(values[e]))
                    throw std::invalid_argument("invalid CSR column or nonfinite value");
                if (e > e0 && sourceIds[e] < sourceIds[e - 1]) sorted = false;
                entries.emplace_back(sourceIds[e], values[e]);
            }
            if (!sorted)
                std::stable_sort(entries.begin(), entries.end(),
                                 [](const auto& a, const auto& b) { return a.first < b.first; });
            std::uint32_t kept = 0;
            for (std::size_t i = 0; i < entries.size();) {
                const std::uint32_t column = entries[i].first;
                float sum = 0.0f;
                do {
                    sum += entries[i++].second;
                } while (i < entries.size() && entries[i].first == column);
                if (!std::isfinite(sum)) throw std::invalid_argument("nonfinite coalesced weight");
                if (sum != 0.0f) {
                    out.cols.push_back(column);
                    out.vals.push_back(sum);
                    ++kept;
                }
            }
            out.rowCounts[r - r0] = kept;
        }
    });

    CsrMatrix result;
    std::vector<std::size_t> entryStart(blocks + 1, 0);
    for (std::size_t b = 0; b < blocks; ++b) entryStart[b + 1] = entryStart[b] + parts[b].cols.size();
    result.rowOffsets.assign(std::size_t(rows) + 1, 0);
    result.sourceIds.resize(entryStart[blocks]);
    result.values.resize(entryStart[blocks]);
    tcc::parallelChunks(blocks, blocks, [&](std::size_t b, std::size_t, std::size_t) {
        const Block& p = parts[b];
        const std::size_t r0 = std::size_t(rows) * b / blocks;
        std::size_t running = entryStart[b];
        for (std::size_t i = 0; i < p.rowCounts.size(); ++i) {
            running += p.rowCounts[i];
            result.rowOffsets[r0 + i + 1] = std::uint32_t(running);
        }
        if (!p.cols.empty()) {
            std::memcpy(result.sourceIds.data() + entryStart[b], p.cols.data(), p.cols.size() * 4);
            std::memcpy(result.values.data() + entryStart[b], p.vals.data(), p.vals.size() * 4);
        }
    });
    return result;
}
