// Fused INT8-dequantization SpMM on MI355X (gfx950).
//
// Drop-in for the reference's include/spmm.cuh:1-23 with hipStream_t in place of cudaStream_t.
#pragma once
#include "format/sw32.h"

#include <hip/hip_runtime_api.h>

// Per-invocation storage, reusable by serial launches on the same stream.
//   partials: Sw32HostFormat::partialCount * 8 * features floats, no initialisation needed.
//   counters: ceil(rows/32) * (features/128) uint32 values, zero before the first use; every
//             launch leaves them at zero again.
// Both may be null when partialCount is zero. Use separate workspaces for concurrent launches;
// keep all buffers alive until the stream completes. (reference include/spmm.cuh:5-13)
struct SpmmWorkspace {
    float* partials = nullptr;
    std::uint32_t* counters = nullptr;
};

// Y[rows][features] = A * tf32(dequant(X)) for F = 128 or 256, FP32 accumulation, including the
// in-kernel merge of split SWs. packedX is packed16 INT8 [cols][features], scales are per source,
// output is FP32 row-major. The RW-bucketed SW32 format with its task plan must be uploaded in
// full. Every output element is overwritten. Throws std::invalid_argument for other feature
// counts (before any launch) and std::runtime_error on launch failure; execution stays
// asynchronous. (reference include/spmm.cuh:15-23)
void launchSpmmInt8(Sw32DeviceView matrix, const std::int8_t* packedX, const float* scales,
                    float* output, std::uint32_t rows, std::uint32_t cols, std::uint32_t features,
                    SpmmWorkspace workspace, hipStream_t stream = nullptr);
