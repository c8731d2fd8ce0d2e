// Fused INT8-dequantization SpMM on MI355X (gfx950).
//
// Drop-in for the reference's include/spmm.cuh:1-23 with hipStream_t in place of cudaStream_t.
#pragma once
#include "format/sw32.h"

#include <cstddef>

#include <hip/hip_runtime_api.h>

// Scratch the caller owns for one launch at a time; launches queued one after another on a single
// stream may share it.
//   partials: Sw32HostFormat::partialCount * 8 * features floats; their contents on entry are
//             never read.
//   counters: ceil(rows/32) * (features/128) uint32 values, zeroed once before the first launch;
//             each launch returns them to zero.
// A plan without split SWs (partialCount == 0) needs neither, so both pointers may then be null.
// Launches that can overlap need one workspace each, and every buffer must outlive the work
// queued on the stream. (reference include/spmm.cuh:5-13)
struct SpmmWorkspace {
    float* partials = nullptr;
    std::uint32_t* counters = nullptr;
};

// Y[rows][features] = A * tf32(dequant(X)) for F = 128 or 256, FP32 accumulation, including the
// in-kernel merge of split SWs. packedX is packed16 INT8 [cols][features], scales are per source,
// output is FP32 row-major. The RW-bucketed SW32 format with its task plan must be uploaded in
// full. Every output element is overwritten. packedX needs u16 alignment, as in the reference
// (include/format/int8_features.cuh:11-13); a 16-byte-aligned one (any hipMalloc'd buffer) takes
// the fastest load path. output and workspace.partials need float alignment, as in the reference;
// when both are 16-byte aligned (any hipMalloc'd buffer, and any whole-row offset into one, is)
// they are written 16 bytes per lane, else one float at a time, with the same result. Throws
// std::invalid_argument, before any launch, for other feature counts, an odd packedX, an output or
// partials base that is not float-aligned, a null packedX, scales or output, or a view with null
// tasks or bucketOffsets (the reference launches and faults instead); std::runtime_error on launch
// failure. Execution stays asynchronous.
// Y's bits: the products are the reference's TF32 products exactly; only the FP32 summation order
// differs from it. That order is fixed for a given plan and task form: a plan with few tasks for the
// GPU's wave slots (CU count x 4 SIMDs x 4 waves at F=128, x 2 at F=256; under 3 tasks per slot at
// F=128, under half a task per slot at F=256) runs two waves per task, each summing half the
// panels, which orders the additions differently. So Y can differ in the last bits between GPUs
// with different CU counts (or partition modes), and between the task forms forced by
// setSpmmLaunchOverrides; repeated launches of one plan on one GPU are bitwise identical.
// (reference include/spmm.cuh:15-23)
void launchSpmmInt8(Sw32DeviceView matrix, const std::int8_t* packedX, const float* scales,
                    float* output, std::uint32_t rows, std::uint32_t cols, std::uint32_t features,
                    SpmmWorkspace workspace, hipStream_t stream = nullptr);

// Bytes of the library-owned scratch behind launchSpmmInt8NoAlloc, per GPU: room for the split-SW
// workspace of c3 at F=128 (14,731 partial tiles, 60.6 MB).
constexpr std::size_t kNoAllocScratchBytes = std::size_t(64) << 20;

// launchSpmmInt8 without a caller workspace: no counterpart in the reference. For callers that
// cannot allocate device memory (HIP graph capture, serving loops, harnesses that forbid
// hipMalloc): the completion counters and partial tiles live in a static device array of
// kNoAllocScratchBytes that each GPU holds until the process ends, and the call itself allocates
// nothing. partialCount must be Sw32HostFormat::partialCount of the uploaded plan: the view does
// not carry it, the workspace size derives from it, and a wrong count is undefined behaviour (too
// small, and split tasks write partial tiles past the scratch). A plan whose counters and partial
// tiles exceed the scratch throws
// std::invalid_argument before any launch, as do feature counts other than 128 or 256. Every call
// on one GPU shares that GPU's scratch: calls that can overlap on one GPU (other streams, or
// concurrent host threads) race and must be serialised by the caller. Other behaviour is
// launchSpmmInt8's.
void launchSpmmInt8NoAlloc(Sw32DeviceView matrix, const std::int8_t* packedX, const float* scales,
                           float* output, std::uint32_t rows, std::uint32_t cols,
                           std::uint32_t features, std::uint32_t partialCount,
                           hipStream_t stream = nullptr);

// Forces two launch choices that launchSpmmInt8 otherwise makes by itself, for tests and
// measurements (no counterpart in the reference). taskWaves: 0 picks the task form from the plan
// and the GPU (see above), 1 or 2 forces one or two waves per task (two applies to the
// buffer-addressed instance only). forceWide: the 64-bit-addressing instance for any size.
// Process-wide. The environment variables TCC_SPMM_TASK_WAVES (1 or 2) and TCC_SPMM_FORCE_WIDE
// give the initial values, read once, at the first launch or the first call of this function.
// Throws std::invalid_argument for taskWaves > 2. Not to be called while other host threads launch.
void setSpmmLaunchOverrides(std::uint32_t taskWaves, bool forceWide);
