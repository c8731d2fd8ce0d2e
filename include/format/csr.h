// Canonical CSR input for the SW32 format (host only).
//
// Drop-in for the reference's include/format/csr.h:1-25: same type names, member names, function
// names, argument order and exception classes.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

// Canonical CSR: per row, strictly increasing source columns and finite non-zero FP32 weights.
// (reference include/format/csr.h:7-10)
struct CsrMatrix {
    std::vector<std::uint32_t> rowOffsets{0}, sourceIds;
    std::vector<float> values;
};

// A Matrix Market file read into canonical CSR. (reference include/format/csr.h:13-16)
struct MtxMatrix {
    std::uint32_t rows, cols;
    CsrMatrix csr;
};

// Read a coordinate real/integer/pattern, general/symmetric Matrix Market file (1-based indices;
// symmetric files are mirrored; duplicates are summed by makeCanonicalCsr).
// Throws std::runtime_error on I/O or syntax errors and std::overflow_error past uint32 sizes.
// (reference include/format/csr.h:18, src/format/matrix_market.cpp:30-103)
MtxMatrix loadMatrixMarket(const std::string& path);

// Validate raw CSR arrays and build a CsrMatrix: stable-sort each row by source column, sum
// duplicate coordinates in their input order (FP32, starting from 0), drop zero sums, reject
// non-finite weights/sums, out-of-range columns and invalid offsets (std::invalid_argument).
// (reference include/format/csr.h:23-25, src/format/csr.cpp:6-40)
CsrMatrix makeCanonicalCsr(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                           const std::uint32_t* rowOffsets, const std::uint32_t* sourceIds,
                           const float* values);
