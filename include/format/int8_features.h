// Per-source INT8 feature preparation on the GPU.
//
// Drop-in for the reference's include/format/int8_features.cuh:1-15 with hipStream_t in place of
// cudaStream_t. Callers provide valid, non-aliasing device buffers and non-zero sizes. Zero sizes
// and launch failures throw std::runtime_error; a null buffer throws std::invalid_argument before
// any launch (the reference launches and faults instead). Execution stays asynchronous on `stream`.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>

// X is row-major [source][feature] FP32. Each source row is quantized independently:
// scale = max|X[source,:]| / 127 (IEEE FP32 divide), all-zero rows use scale = 1, and
// q = clamp(round_half_even(X / scale), -127, 127). (reference int8_features.cuh:5-10)
void quantizeFeaturesInt8(const float* x, std::int8_t* q, float* scale, std::uint32_t sources,
                          std::uint32_t features, hipStream_t stream = nullptr);

// Physical byte layout only: each 16-feature tile becomes [q0,q8,q1,q9,...,q7,q15]. Features must
// be a multiple of 16; the output has sources*features bytes, must not alias q, and must be
// 2-byte aligned. Values are unchanged. Throws std::invalid_argument when features % 16 != 0.
// (reference int8_features.cuh:11-15)
void packFeaturesInt8x16(const std::int8_t* q, std::int8_t* packed, std::uint32_t sources,
                         std::uint32_t features, hipStream_t stream = nullptr);

// quantizeFeaturesInt8 followed by packFeaturesInt8x16 in one pass, with no counterpart in the
// reference: `packed` and `scale` are bit for bit what that pair of calls writes, but the
// quantized bytes go straight to the packed layout, so X is read once and nothing else is written
// (5F + 4 bytes per source instead of 7F + 4). For callers that quantize X for every SpMM.
// Features must be a multiple of 16 (std::invalid_argument); zero sizes throw std::runtime_error and
// null buffers std::invalid_argument, before any launch. `packed` must not alias x.
void quantizePackFeaturesInt8(const float* x, std::int8_t* packed, float* scale,
                              std::uint32_t sources, std::uint32_t features,
                              hipStream_t stream = nullptr);
