// Canonical CSR construction (host), with the observable behaviour of the reference's
// makeCanonicalCsr (src/format/csr.cpp:6-40): per row, entries ordered by column with ties kept in
// input order, duplicates summed in FP32 in that order starting from 0.0f, zero sums dropped; the
// same exception classes and messages, raised for the first defect in row order.
//
// Design: canonicalisation never makes a row longer, so every row is canonicalised in place into
// its own input range [rowOffsets[r], rowOffsets[r + 1]) of a staging array, independently and in
// parallel over row blocks. A row whose columns already increase strictly is copied (minus zero
// values); any other row is ordered by sorting 64-bit keys (column << 32 | position in the row),
// whose low half breaks ties by input position, and its runs of equal keys are coalesced in one
// pass. A prefix sum of the kept counts gives the output offsets, and a parallel pass compacts the
// staged rows into place.
#include "format/csr.h"
#include "../parallel.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>

namespace {

// Offsets must start at 0, end at nnz and never decrease (checked before any entry is read).
void checkShape(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                const std::uint32_t* rowOffsets) {
    const bool shapeOk = rows != 0 && cols != 0 && rowOffsets[0] == 0 && rowOffsets[rows] == nnz;
    if (!shapeOk) throw std::invalid_argument("invalid CSR dimensions or offsets");
    const std::uint32_t* end = rowOffsets + rows + 1;
    const bool monotone = std::is_sorted(rowOffsets, end);
    if (!monotone || *std::max_element(rowOffsets, end) > nnz)
        throw std::invalid_argument("invalid CSR offsets");
}

// Canonicalises one row of n entries into (outCols, outVals), which have room for n; returns the
// number kept. `keys` is per-thread scratch.
std::uint32_t canonicalRow(const std::uint32_t* col, const float* val, std::uint32_t n,
                           std::uint32_t cols, std::uint32_t* outCols, float* outVals,
                           std::vector<std::uint64_t>& keys) {
    bool strictlyIncreasing = true;
    for (std::uint32_t i = 0; i < n; ++i) {
        if (!(col[i] < cols && std::isfinite(val[i])))
            throw std::invalid_argument("invalid CSR column or nonfinite value");
        strictlyIncreasing = strictlyIncreasing && (i == 0 || col[i - 1] < col[i]);
    }
    std::uint32_t kept = 0;
    if (strictlyIncreasing) {
        // One entry per column: its sum is 0.0f + v = v, dropped when zero (either sign).
        for (std::uint32_t i = 0; i < n; ++i)
            if (val[i] != 0.0f) {
                outCols[kept] = col[i];
                outVals[kept++] = val[i];
            }
        return kept;
    }
    keys.resize(n);
    for (std::uint32_t i = 0; i < n; ++i) keys[i] = std::uint64_t(col[i]) << 32 | i;
    std::sort(keys.begin(), keys.end());
    std::uint32_t i = 0;
    while (i < n) {
        const std::uint32_t column = std::uint32_t(keys[i] >> 32);
        float sum = 0.0f;
        for (; i < n && std::uint32_t(keys[i] >> 32) == column; ++i)
            sum += val[std::uint32_t(keys[i])];
        if (!std::isfinite(sum)) throw std::invalid_argument("nonfinite coalesced weight");
        if (sum != 0.0f) {
            outCols[kept] = column;
            outVals[kept++] = sum;
        }
    }
    return kept;
}

} // namespace

CsrMatrix makeCanonicalCsr(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                           const std::uint32_t* rowOffsets, const std::uint32_t* sourceIds,
                           const float* values) {
    checkShape(rows, cols, nnz, rowOffsets);

    // Stage: row r's canonical entries start at rowOffsets[r]; keptPerRow[r] of them are valid.
    std::vector<std::uint32_t> stageCols(nnz), keptPerRow(rows);
    std::vector<float> stageVals(nnz);
    const std::size_t blocks = std::min<std::size_t>(rows, 1024);
    tcc::parallelChunks(rows, blocks, [&](std::size_t, std::size_t r0, std::size_t r1) {
        std::vector<std::uint64_t> keys;
        for (std::size_t r = r0; r < r1; ++r) {
            const std::uint32_t at = rowOffsets[r], n = rowOffsets[r + 1] - at;
            keptPerRow[r] = canonicalRow(sourceIds + at, values + at, n, cols, stageCols.data() + at,
                                         stageVals.data() + at, keys);
        }
    });

    CsrMatrix out;
    out.rowOffsets.resize(std::size_t(rows) + 1);
    out.rowOffsets[0] = 0;
    for (std::uint32_t r = 0; r < rows; ++r)
        out.rowOffsets[r + 1] = out.rowOffsets[r] + keptPerRow[r];
    out.sourceIds.resize(out.rowOffsets[rows]);
    out.values.resize(out.rowOffsets[rows]);
    tcc::parallelChunks(rows, blocks, [&](std::size_t, std::size_t r0, std::size_t r1) {
        for (std::size_t r = r0; r < r1; ++r) {
            const std::uint32_t from = rowOffsets[r], to = out.rowOffsets[r], n = keptPerRow[r];
            if (!n) continue;
            std::copy_n(stageCols.begin() + from, n, out.sourceIds.begin() + to);
            std::copy_n(stageVals.begin() + from, n, out.values.begin() + to);
        }
    });
    return out;
}
