// Deterministic synthetic workloads for the benchmark configurations (C++ entry points of
// generators.cpp; the C ABI wraps the same functions as tcc_synth_csr / tcc_synth_features).
#pragma once
#include "format/csr.h"

#include <cstdint>
#include <string>

struct SyntheticCsr {
    std::uint32_t rows, cols;
    CsrMatrix csr;
};

// Canonical CSR for "c1".."c5" ("c4" is c3's matrix) or "t<rows>_<deg>_<seed>". Throws
// std::invalid_argument for an unknown name.
SyntheticCsr makeSyntheticCsr(const std::string& config);

// sources x features row-major N(0, stddev^2) values (Box-Muller over per-row SplitMix64 streams);
// a fraction `outlierFraction` of rows is multiplied by `outlierScale`.
void makeSyntheticFeatures(std::uint32_t sources, std::uint32_t features, std::uint64_t seed,
                           float stddev, float outlierFraction, float outlierScale, float* out);
