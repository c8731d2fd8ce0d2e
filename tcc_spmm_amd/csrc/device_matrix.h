// Device owner of an uploaded SW32 format and its split-task workspace.
//
// Counterpart of the reference's src/device_matrix.cuh:8-37: every array of a bucketed
// Sw32HostFormat is uploaded once; `partials` (partialCount * 8 * features floats) and `counters`
// (nSW * features/128 uint32, zeroed) are allocated only when the plan has split SWs. view() and
// workspace() hand out the non-owning descriptors launchSpmmInt8 takes.
#pragma once
#include "format/sw32.h"
#include "hip_support.h"
#include "spmm.h"

#include <stdexcept>

struct DeviceMatrix {
    DeviceBuffer<std::uint32_t> windowOffsets, sourceIds, rowGroupMasks, bucketOffsets, partialIds;
    DeviceBuffer<std::uint64_t> sourceMetadata;
    DeviceBuffer<float> values;
    DeviceBuffer<Sw32Task> tasks;
    DeviceBuffer<Sw32ReduceRange> reductions;
    DeviceBuffer<float> partials;
    DeviceBuffer<std::uint32_t> counters;
    std::uint32_t taskCount;

    DeviceMatrix(const Sw32HostFormat& f, unsigned features)
        : windowOffsets(f.windowOffsets), sourceIds(f.sourceIds), rowGroupMasks(f.rowGroupMasks),
          bucketOffsets(f.bucketOffsets), partialIds(f.partialIds), sourceMetadata(f.sourceMetadata),
          values(f.values), tasks(f.tasks), reductions(f.reductions),
          partials(std::size_t(f.partialCount) * 8 * features),
          counters(f.partialCount ? (f.windowOffsets.size() - 1) * (features / 128) : 0),
          taskCount(std::uint32_t(f.tasks.size())) {
        if (features != 128 && features != 256)
            throw std::invalid_argument("feature dimension must be 128 or 256");
        if (counters.count)
            checkHip(hipMemset(counters.ptr, 0, counters.count * sizeof(std::uint32_t)));
    }

    Sw32DeviceView view() const {
        return {windowOffsets.ptr, sourceIds.ptr, rowGroupMasks.ptr, sourceMetadata.ptr, values.ptr,
                bucketOffsets.ptr, tasks.ptr, reductions.ptr, partialIds.ptr, taskCount};
    }

    SpmmWorkspace workspace() const { return {partials.ptr, counters.ptr}; }
};
