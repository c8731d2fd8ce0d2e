// SW32 superwindow format and bounded panel-task plan (host only).
//
// Drop-in for the reference's include/format/sw32.h:1-56. The constants, struct layouts and the
// order of every array are part of the contract: the arrays built here are byte-identical to the
// reference's for the same canonical CSR, so device views built by either side are interchangeable.
#pragma once
#include "format/csr.h"
#include <cstdint>
#include <vector>

// Physical bucket order of the 16 RW-mask buckets of one SW: slot 0 (mask 0) stays empty, slots
// 1..4 hold sources touching exactly one 8-row group (RW0..RW3), slots 5..15 hold sources shared
// by two or more row groups. (reference include/format/sw32.h:9-10)
inline constexpr unsigned sw32BucketOrder[16] = {0, 1, 2,  4,  8,  3,  5,  6,
                                                 7, 9, 10, 11, 12, 13, 14, 15};

// Panels per task: an SW with more panels is cut into ceil(n/384) tasks whose results are merged
// in-kernel. (reference include/format/sw32.h:12)
inline constexpr std::uint32_t sw32TaskPanelLimit = 384;

// One workgroup's work: panels [begin, end) of SW `sw`. Unsplit tasks have partial == UINT32_MAX,
// mask == 15, chunks == 1, reduceFirst == 0. Split tasks store the row groups in `mask` as partial
// tiles partial + popcount(mask & ((1 << rw) - 1)); the SW's `chunks` tasks share one completion
// counter and reductions[reduceFirst .. reduceFirst + 4). (reference include/format/sw32.h:13-15)
struct Sw32Task {
    std::uint32_t sw, begin, end, partial, mask, chunks, reduceFirst;
};
// partialIds[begin, end) lists the partial tiles of one row group in task order.
// (reference include/format/sw32.h:16-18)
struct Sw32ReduceRange {
    std::uint32_t begin, end;
};
static_assert(sizeof(Sw32Task) == 28, "Sw32Task is seven packed uint32 fields");
static_assert(sizeof(Sw32ReduceRange) == 8, "Sw32ReduceRange is two packed uint32 fields");

// CPU storage for 32-row superwindows (SW); each RW is an 8-row group.
// Rows follow the input matrix order; X and scales are indexed by the input source id.
// (reference include/format/sw32.h:22-39)
struct Sw32HostFormat {
    std::uint32_t rows = 0, cols = 0;
    // windowOffsets[w] = first panel of SW w (nSW + 1 entries). sourceIds has 8 slots per panel,
    // padded with UINT32_MAX; rowGroupMasks has one 4-bit RW mask per panel.
    std::vector<std::uint32_t> windowOffsets{0}, sourceIds, rowGroupMasks;
    // Per slot: low 32 bits = destination-row mask inside the SW; high 32 bits = index of the
    // slot's first value. Values of a slot follow in increasing row order. Padding slots are 0.
    std::vector<std::uint64_t> sourceMetadata;
    std::vector<float> values;
    // Bucketed format only: 17 absolute panel offsets per SW. Slot s (mask sw32BucketOrder[s])
    // occupies [bucketOffsets[17w+s], bucketOffsets[17w+s+1]).
    std::vector<std::uint32_t> bucketOffsets;
    // Bucketed format only: tasks in natural SW order, 4 reductions per split SW, partial tile ids
    // grouped per reduction, and the number of partial tiles.
    std::vector<Sw32Task> tasks;
    std::vector<Sw32ReduceRange> reductions;
    std::vector<std::uint32_t> partialIds;
    std::uint32_t partialCount = 0;
};

// Build the SW32 stream from canonical CSR (CPU). Throws std::invalid_argument for inputs that are
// not canonical (offsets, column range, zero/non-finite values, non-increasing row columns) and
// std::overflow_error when an offset exceeds uint32. Keep bucketByRwMask = true for
// launchSpmmInt8(); the bucketed result already carries its task plan (buildPanelTasks).
// (reference include/format/sw32.h:41-44, src/format/sw32.cpp:69-167)
Sw32HostFormat convertCsrToSw32(std::uint32_t rows, std::uint32_t cols, const CsrMatrix& csr,
                                bool bucketByRwMask = true);

// (Re)build tasks, reductions, partialIds and partialCount of a bucketed format from its
// windowOffsets and bucketOffsets. The reference keeps this function internal
// (src/format/sw32.cpp:25-65, called at :164-165); it is exported here so callers that edit or
// stream formats can re-plan. Throws std::invalid_argument for a non-bucketed format.
void buildPanelTasks(Sw32HostFormat& format);

// Non-owning device pointers to the arrays above; upload is explicit.
// (reference include/format/sw32.h:46-56)
struct Sw32DeviceView {
    const std::uint32_t *windowOffsets, *sourceIds, *rowGroupMasks;
    const std::uint64_t* sourceMetadata;
    const float* values;
    const std::uint32_t* bucketOffsets = nullptr;
    const Sw32Task* tasks = nullptr;
    const Sw32ReduceRange* reductions = nullptr;
    const std::uint32_t* partialIds = nullptr;
    std::uint32_t taskCount = 0;
};
