// Fused INT8-dequantization SpMM for MI355X (gfx950, wave64): Y = A x tf32(dequant(X)).
//
// Work decomposition (one wavefront per workgroup):
//   workgroup (task, slice): task = one Sw32Task (<= 384 panels of one 32-row SW), slice = 128
//   features. Lane l owns the packed16 byte pair l of the slice, i.e. features
//   f0 = 16*(l/8) + l%8 and f1 = f0 + 8, and accumulates those two features for all 32 rows of the
//   SW in 64 FP32 accumulators (2 features x 8 four-row "quads" x 4 rows).
//
// Per panel of 8 slots the wave
//   1. expands the panel's A values into a dense [slot][8 rows] table per touched row group (RW):
//      lane (slot k = l/8, row r = l%8) reads its slot's row mask and value base, picks
//      values[base + popcount(mask below the row)] when the row bit is set, rounds it to TF32
//      (round-to-nearest, ties away: (bits + 0x1000) & ~0x1FFF) and stores it to LDS;
//   2. gathers the 8 source rows of X (one coalesced 128-byte load per slot), dequantizes each byte
//      with the source's scale and rounds it to TF32 — the products of two TF32 operands are exact
//      in FP32, so any FP32 accumulation order reproduces the reference's products;
//   3. accumulates with v_mfma_f32_4x4x1_16b_f32: A operand = the 4 row values of one quad
//      (broadcast from LDS), B operand = the lane's dequantized feature, D = 4 rows x the lane's
//      feature. No per-row dynamic register indexing is needed: the quads are compile-time.
// Buckets 1..4 (one RW) touch one RW; buckets 5..15 (shared sources) touch the RWs of their
// bucket mask; the bucket's RW set is a template parameter so every branch on it is static.
//
// Split SWs (reference src/kernel/spmm_kernel.cuh:228-282): a split task stores its RWs of
// `task.mask` as 8-row partial tiles [tile][8][F]; thread 0 then takes an agent-scope acq_rel
// wrapping ticket on counters[sw * (F/128) + slice] (inc with limit chunks-1, so the counter returns
// to zero by itself); the task whose ticket equals chunks-1 merges all partial tiles of the SW in
// partialIds order starting from 0.0f and writes Y. No float atomics, no spin-waits.
#include "spmm.h"
#include "hip_support.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr unsigned kWave = 64;
constexpr unsigned kSlice = 128;
constexpr unsigned kNoPartial = 0xFFFFFFFFu;

// TF32 rounding from its definition: keep 10 explicit mantissa bits, round to nearest with ties
// away from zero (adding half an ulp to the sign-magnitude encoding), carry into the exponent.
// Operands here are always finite (the format rejects non-finite A values; X is finite INT8 times a
// finite scale).
__device__ __forceinline__ float roundTf32(float v) {
    return __uint_as_float((__float_as_uint(v) + 0x1000u) & 0xFFFFE000u);
}

struct KernelArgs {
    Sw32DeviceView m;
    const std::int8_t* packedX;
    const float* scales;
    float* y;
    float* partials;
    unsigned* counters;
    unsigned rows, cols;
};

// Dense A-value table for one row group of one panel: lane (k = l/8, r = l%8).
__device__ __forceinline__ void expandPanelRows(const KernelArgs& a, unsigned panel, unsigned rw,
                                                unsigned lane, float* table) {
    const unsigned k = lane >> 3, r = lane & 7;
    const std::uint64_t meta = a.m.sourceMetadata[std::size_t(panel) * 8 + k];
    const unsigned mask = unsigned(meta), base = unsigned(meta >> 32);
    const unsigned row = rw * 8 + r;
    const bool present = (mask >> row) & 1u;
    // Padding slots have mask 0 and base 0; every other slot owns >= 1 value at `base`.
    const unsigned idx = present ? base + __popc(mask & ((1u << row) - 1u)) : base;
    const float v = a.m.values[idx];
    table[lane] = present ? roundTf32(v) : 0.0f;
}

template <unsigned RWSET>
__device__ __forceinline__ void accumulatePanels(const KernelArgs& a, unsigned begin, unsigned end,
                                                 unsigned lane, unsigned xOffset, unsigned features,
                                                 float (*table)[64], f32x4 (&acc)[2][8]) {
    for (unsigned panel = begin; panel < end; ++panel) {
#pragma unroll
        for (unsigned rw = 0; rw < 4; ++rw)
            if (RWSET & (1u << rw)) expandPanelRows(a, panel, rw, lane, table[rw]);
        __syncthreads();
        const unsigned* ids = a.m.sourceIds + std::size_t(panel) * 8;
#pragma unroll
        for (unsigned k = 0; k < 8; ++k) {
            const unsigned src = ids[k];
            if (src >= a.cols) continue; // padding slot (always at the end of a bucket)
            const unsigned short pair = *reinterpret_cast<const unsigned short*>(
                a.packedX + std::size_t(src) * features + xOffset);
            const float s = a.scales[src];
            const float x0 = roundTf32(float(std::int8_t(pair & 0xFFu)) * s);
            const float x1 = roundTf32(float(std::int8_t(pair >> 8)) * s);
#pragma unroll
            for (unsigned rw = 0; rw < 4; ++rw) {
                if (!(RWSET & (1u << rw))) continue;
#pragma unroll
                for (unsigned half = 0; half < 2; ++half) {
                    const float av = table[rw][k * 8 + half * 4 + (lane & 3)];
                    const unsigned quad = rw * 2 + half;
                    acc[0][quad] = __builtin_amdgcn_mfma_f32_4x4x1f32(av, x0, acc[0][quad], 0, 0, 0);
                    acc[1][quad] = __builtin_amdgcn_mfma_f32_4x4x1f32(av, x1, acc[1][quad], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }
}

// Map workgroups so that each of the 8 XCDs (dispatched round-robin by workgroup id) walks one
// contiguous range of tasks: neighbouring SWs share source rows of X in that XCD's L2.
__device__ __forceinline__ unsigned xcdTask(unsigned bid, unsigned tasks) {
    const unsigned xcd = bid & 7u, j = bid >> 3;
    const unsigned q = tasks >> 3, r = tasks & 7u;
    return xcd * q + min(xcd, r) + j;
}

template <unsigned Features>
__global__ __launch_bounds__(kWave) void spmmInt8Kernel(KernelArgs a) {
    __shared__ float table[4][64];
    __shared__ unsigned lastFlag;
    const unsigned lane = threadIdx.x;
    const unsigned slice = blockIdx.y;
    const unsigned taskIndex = xcdTask(blockIdx.x, a.m.taskCount);
    const Sw32Task task = a.m.tasks[taskIndex];
    const unsigned sw = task.sw;
    const unsigned f0 = 16 * (lane >> 3) + (lane & 7); // f1 = f0 + 8
    const unsigned xOffset = slice * kSlice + 2 * lane;

    f32x4 acc[2][8];
#pragma unroll
    for (unsigned h = 0; h < 2; ++h)
#pragma unroll
        for (unsigned q = 0; q < 8; ++q) acc[h][q] = f32x4{0.f, 0.f, 0.f, 0.f};

    const unsigned* slots = a.m.bucketOffsets + std::size_t(sw) * 17;
#pragma unroll 1
    for (unsigned s = 1; s < 16; ++s) {
        const unsigned begin = max(slots[s], task.begin), end = min(slots[s + 1], task.end);
        if (begin >= end) continue;
        switch (s) {
        case 1: accumulatePanels<1>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 2: accumulatePanels<2>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 3: accumulatePanels<4>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 4: accumulatePanels<8>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 5: accumulatePanels<3>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 6: accumulatePanels<5>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 7: accumulatePanels<6>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 8: accumulatePanels<7>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 9: accumulatePanels<9>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 10: accumulatePanels<10>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 11: accumulatePanels<11>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 12: accumulatePanels<12>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 13: accumulatePanels<13>(a, begin, end, lane, xOffset, Features, table, acc); break;
        case 14: accumulatePanels<14>(a, begin, end, lane, xOffset, Features, table, acc); break;
        default: accumulatePanels<15>(a, begin, end, lane, xOffset, Features, table, acc); break;
        }
    }

    // Write-back: D of quad q holds rows 4q..4q+3 (vector element i = row 4q+i) for the lane's
    // feature column.
    const unsigned col0 = slice * kSlice + f0;
    if (task.partial == kNoPartial) {
        const unsigned rowbase = sw * 32;
#pragma unroll
        for (unsigned q = 0; q < 8; ++q)
#pragma unroll
            for (unsigned i = 0; i < 4; ++i) {
                const unsigned row = rowbase + q * 4 + i;
                if (row < a.rows) {
                    float* yr = a.y + std::size_t(row) * Features;
                    yr[col0] = acc[0][q][i];
                    yr[col0 + 8] = acc[1][q][i];
                }
            }
        return;
    }
#pragma unroll
    for (unsigned rw = 0; rw < 4; ++rw) {
        if (!(task.mask & (1u << rw))) continue;
        const std::size_t tile = task.partial + __popc(task.mask & ((1u << rw) - 1u));
#pragma unroll
        for (unsigned half = 0; half < 2; ++half)
#pragma unroll
            for (unsigned i = 0; i < 4; ++i) {
                float* pr = a.partials + (tile * 8 + half * 4 + i) * Features;
                pr[col0] = acc[0][rw * 2 + half][i];
                pr[col0 + 8] = acc[1][rw * 2 + half][i];
            }
    }
    // Completion ticket: the acq_rel RMW at agent scope publishes this task's partial tiles and, for
    // the last arriver, makes every other task's tiles visible (the XCD L2s are not coherent with
    // each other, so the release writes back and the acquire invalidates).
    __syncthreads();
    if (lane == 0) {
        unsigned* counter = a.counters + std::size_t(sw) * (Features / kSlice) + slice;
        const unsigned ticket =
            __builtin_amdgcn_atomic_inc32(counter, task.chunks - 1, __ATOMIC_ACQ_REL, "agent");
        lastFlag = ticket == task.chunks - 1;
    }
    __syncthreads();
    if (!lastFlag) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // Merge: each lane sums columns lane and lane + 64 of the slice for every valid row, adding the
    // partial tiles in partialIds (task) order starting from 0.0f.
    const unsigned col = slice * kSlice + lane;
#pragma unroll 1
    for (unsigned rw = 0; rw < 4; ++rw) {
        const Sw32ReduceRange red = a.m.reductions[task.reduceFirst + rw];
        const unsigned row0 = sw * 32 + rw * 8;
        if (row0 >= a.rows) continue;
        const unsigned valid = min(8u, a.rows - row0);
#pragma unroll 1
        for (unsigned r = 0; r < valid; ++r) {
            float lo = 0.0f, hi = 0.0f;
#pragma unroll 1
            for (unsigned item = red.begin; item < red.end; ++item) {
                const float* pr =
                    a.partials + (std::size_t(a.m.partialIds[item]) * 8 + r) * Features + col;
                lo += pr[0];
                hi += pr[kWave];
            }
            float* yr = a.y + std::size_t(row0 + r) * Features + col;
            yr[0] = lo;
            yr[kWave] = hi;
        }
    }
}

template <unsigned Features>
void launch(const KernelArgs& args, hipStream_t stream) {
    const dim3 grid(args.m.taskCount, Features / kSlice);
    hipLaunchKernelGGL(spmmInt8Kernel<Features>, grid, dim3(kWave), 0, stream, args);
}

} // namespace

void launchSpmmInt8(Sw32DeviceView matrix, const std::int8_t* packedX, const float* scales,
                    float* output, std::uint32_t rows, std::uint32_t cols, std::uint32_t features,
                    SpmmWorkspace workspace, hipStream_t stream) {
    if (features != 128 && features != 256)
        throw std::invalid_argument("feature dimension must be 128 or 256");
    if (!matrix.taskCount)
        throw std::runtime_error("launchSpmmInt8: invalid configuration argument (no tasks)");
    const KernelArgs args{matrix, packedX, scales, output, workspace.partials, workspace.counters,
                          rows, cols};
    if (features == 128)
        launch<128>(args, stream);
    else
        launch<256>(args, stream);
    checkHip(hipGetLastError());
}
