// gather_probe: how many random requests per second the memory system serves beyond L2 on this GPU
// (measurement infrastructure for the traffic model; run by `bench.py --probe-gather`).
//
// Each wave issues loads of W bytes per row at hashed row indices of a table of a given size, DEPTH
// loads in flight per lane; rows are 128 bytes apart. Sizes below the 4 MiB per-XCD L2 measure L2
// hits; large tables measure the beyond-L2 request rate, for W = 128 (a whole X row of F = 128, eight
// lanes x 16 bytes), 64 and 32. A last case pairs each 128-byte row with a 4-byte load from a 9.8 MB
// table, the kernel's X row + scale pattern. Every index is reduced modulo the row count, so every
// access is inside the table. Prints one JSON object.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned mix(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// W bytes of each of 64 / (W / 16) rows per instruction; DEPTH instructions in flight per lane.
template <int W, int DEPTH>
__global__ __launch_bounds__(64) void gatherRows(const unsigned char* table, unsigned rows,
                                                 unsigned iters, unsigned* sink) {
    constexpr unsigned lanesPerRow = W / 16;
    const unsigned lane = threadIdx.x;
    unsigned acc = 0, seed = blockIdx.x * 7919u + 1;
    for (unsigned it = 0; it < iters; it += DEPTH) {
        u32x4 v[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const unsigned r = mix(seed + (it + d) * 64 + lane / lanesPerRow) % rows;
            v[d] = *reinterpret_cast<const u32x4*>(table + std::size_t(r) * 128 +
                                                   16 * (lane % lanesPerRow));
        }
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) acc += v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
    }
    if (acc == 0x12345678u) sink[blockIdx.x] = acc; // keeps the loads; practically never stores
}

template <int DEPTH>
__global__ __launch_bounds__(64) void gatherRowsAndScales(const unsigned char* table,
                                                          const float* scales, unsigned rows,
                                                          unsigned iters, unsigned* sink) {
    const unsigned lane = threadIdx.x;
    unsigned acc = 0, seed = blockIdx.x * 7919u + 1;
    for (unsigned it = 0; it < iters; it += DEPTH) {
        u32x4 v[DEPTH];
        float s[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const unsigned r = mix(seed + (it + d) * 64 + lane / 8) % rows;
            v[d] = *reinterpret_cast<const u32x4*>(table + std::size_t(r) * 128 + 16 * (lane % 8));
            s[d] = scales[r];
        }
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) acc += v[d][0] ^ __float_as_uint(s[d]);
    }
    if (acc == 0x12345678u) sink[blockIdx.x] = acc;
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "gather_probe: %s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

} // namespace

int main() {
    const std::size_t maxBytes = std::size_t(2560) << 20;
    const unsigned scaleRows = 2449029;
    unsigned char* table = nullptr;
    unsigned* sink = nullptr;
    float* scales = nullptr;
    check(hipMalloc(&table, maxBytes), "hipMalloc table");
    check(hipMalloc(&sink, 1 << 20), "hipMalloc sink");
    check(hipMalloc(&scales, std::size_t(scaleRows) * 4), "hipMalloc scales");
    check(hipMemset(table, 1, maxBytes), "hipMemset");
    check(hipMemset(scales, 0, std::size_t(scaleRows) * 4), "hipMemset");
    hipEvent_t t0, t1;
    check(hipEventCreate(&t0), "event");
    check(hipEventCreate(&t1), "event");
    const unsigned blocks = 256 * 16, iters = 256;
    auto time = [&](auto launch) {
        launch();
        check(hipDeviceSynchronize(), "warm-up");
        check(hipEventRecord(t0), "record");
        launch();
        launch();
        check(hipEventRecord(t1), "record");
        check(hipEventSynchronize(t1), "sync");
        float ms = 0;
        check(hipEventElapsedTime(&ms, t0, t1), "elapsed");
        return double(ms) / 2;
    };
    std::printf("{\"rows128\": [");
    const double MiB = 1 << 20;
    const double sizes[] = {4, 9.8, 32, 64, 128, 256, 313, 627, 1254, 2500};
    for (int i = 0; i < 10; ++i) {
        const unsigned rows = unsigned(sizes[i] * MiB / 128);
        const double ms = time([&] { gatherRows<128, 4><<<blocks, 64>>>(table, rows, iters, sink); });
        const double req = double(blocks) * iters * 8;
        std::printf("%s{\"table_mib\": %.1f, \"ms\": %.4f, \"g_requests_per_s\": %.2f, \"tb_per_s\": %.3f}",
                    i ? ", " : "", sizes[i], ms, req / ms / 1e6, req * 128 / ms / 1e9);
    }
    std::printf("], \"narrow\": [");
    const double narrow[] = {64, 313, 627};
    for (int i = 0; i < 3; ++i) {
        const unsigned rows = unsigned(narrow[i] * MiB / 128);
        const double ms64 = time([&] { gatherRows<64, 4><<<blocks, 64>>>(table, rows, iters, sink); });
        const double ms32 = time([&] { gatherRows<32, 4><<<blocks, 64>>>(table, rows, iters, sink); });
        const double r64 = double(blocks) * iters * 16, r32 = double(blocks) * iters * 32;
        std::printf("%s{\"table_mib\": %.0f, \"g_requests_per_s_64B\": %.2f, \"g_requests_per_s_32B\": %.2f}",
                    i ? ", " : "", narrow[i], r64 / ms64 / 1e6, r32 / ms32 / 1e6);
    }
    const double msXS =
        time([&] { gatherRowsAndScales<4><<<blocks, 64>>>(table, scales, scaleRows, iters, sink); });
    const double slots = double(blocks) * iters * 8;
    std::printf("], \"row_and_scale\": {\"g_slots_per_s\": %.2f, \"g_requests_per_s\": %.2f}}\n",
                slots / msXS / 1e6, 2 * slots / msXS / 1e6);
    check(hipFree(table), "hipFree");
    check(hipFree(sink), "hipFree");
    check(hipFree(scales), "hipFree");
    return 0;
}
