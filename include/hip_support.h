// HIP error convention and RAII device buffers.
//
// Counterpart of the reference's include/cuda_support.cuh:1-36: failures of the runtime are
// reported by throwing std::runtime_error carrying hipGetErrorString(); device buffers are owned
// by DeviceBuffer<T> and freed on destruction. Zero-sized buffers allocate nothing.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <stdexcept>
#include <vector>

inline void checkHip(hipError_t result) {
    if (result != hipSuccess)
        throw std::runtime_error(hipGetErrorString(result));
}

template <typename T> class DeviceBuffer {
  public:
    T* ptr = nullptr;
    std::size_t count = 0;

    explicit DeviceBuffer(std::size_t n) : count(n) {
        if (n)
            checkHip(hipMalloc(reinterpret_cast<void**>(&ptr), n * sizeof(T)));
    }

    explicit DeviceBuffer(const std::vector<T>& data) : DeviceBuffer(data.size()) {
        if (!data.empty())
            checkHip(hipMemcpy(ptr, data.data(), data.size() * sizeof(T), hipMemcpyHostToDevice));
    }

    ~DeviceBuffer() {
        if (ptr)
            (void)hipFree(ptr);
    }

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};
