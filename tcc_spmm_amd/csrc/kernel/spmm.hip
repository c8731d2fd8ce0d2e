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
// Row-group set of bucket slot s (sw32BucketOrder, include/format/sw32.h).
__constant__ unsigned kBucketRwSet[16] = {0, 1, 2, 4, 8, 3, 5, 6, 7, 9, 10, 11, 12, 13, 14, 15};

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
    unsigned xBytes; // cols * features (< 2^32, checked by the launcher)
};

// ---------------------------------------------------------------------------------------------
// Panel pipeline. Inside one phase (the exclusive buckets 1..4, or the shared buckets 5..15) the
// panels of a task are walked in order with a three-stage software pipeline whose per-iteration
// memory operations are identical on every path, so the compiler's wait counters stay exact:
//   stage 1 (panel p+2): lane (k = l/8, r = l%8) loads slot k's source id and metadata;
//   stage 2 (panel p+1): its scale, its A value(s) for row r of the panel's row groups, and the X
//                        gathers of the 8 slots (one 128-byte slice per slot, SGPR row offset);
//   stage 3 (panel p):   A values -> TF32 -> LDS table, dequantize X, MFMA accumulate.
// Panel indices past the phase end are clamped to its last panel (harmless duplicate loads).

struct Meta {
    unsigned id;
    unsigned mask;
    unsigned base;
};

struct Stage2 {
    unsigned src;    // clamped source id of slot k (row 0 for padding)
    float scale;     // scale of that source
    float v[4];      // raw A values of (slot k, row 8g + r), g = the panel's row groups
    unsigned bits;   // bit g set when slot k touches row 8g + r
    unsigned xr[8];  // X byte pairs of the 8 slots for this lane's features
};

__device__ __forceinline__ Meta loadMeta(const KernelArgs& a, unsigned panel, unsigned lane) {
    const std::size_t slot = std::size_t(panel) * 8 + (lane >> 3);
    const std::uint64_t md = a.m.sourceMetadata[slot];
    return {a.m.sourceIds[slot], unsigned(md), unsigned(md >> 32)};
}

// Value of (slot, row) or the slot's first value when the row is absent (always a valid index:
// padding slots have base 0 and the matrix has at least one value when it has panels).
__device__ __forceinline__ float loadValue(const KernelArgs& a, const Meta& m, unsigned row,
                                           bool& present) {
    present = (m.mask >> row) & 1u;
    const unsigned idx = m.base + __popc(m.mask & ((1u << row) - 1u));
    return a.m.values[present ? idx : m.base];
}

template <unsigned NG>
__device__ __forceinline__ void loadStage2(const KernelArgs& a, const Meta& m, const unsigned* rws,
                                           unsigned lane, __amdgpu_buffer_rsrc_t xr,
                                           unsigned xLane, unsigned features, Stage2& s) {
    const bool live = m.id < a.cols;
    s.src = live ? m.id : 0u;
    s.scale = a.scales[s.src];
    s.bits = 0;
#pragma unroll
    for (unsigned g = 0; g < NG; ++g) {
        bool present;
        s.v[g] = loadValue(a, m, rws[g] * 8 + (lane & 7), present);
        s.bits |= unsigned(present && live) << g;
    }
#pragma unroll
    for (unsigned j = 0; j < 8; ++j) {
        const unsigned src = __builtin_amdgcn_readlane(s.src, j * 8);
        s.xr[j] = __builtin_amdgcn_raw_buffer_load_b16(xr, xLane, src * features, 0);
    }
}

// Accumulate one panel whose row groups are rws[0..NG) (NG = 4 in the shared phase, where only the
// groups in `rwset` are computed).
template <unsigned NG>
__device__ __forceinline__ void computeStage3(const Stage2& s, const unsigned* rws, unsigned rwset,
                                              unsigned lane, float* table, f32x4 (&acc)[2][8]) {
    // A table: table[g][k][r] = tf32(A[8*rws[g] + r][slot k]) (0 when absent).
#pragma unroll
    for (unsigned g = 0; g < NG; ++g)
        table[g * 64 + lane] = ((s.bits >> g) & 1u) ? roundTf32(s.v[g]) : 0.0f;
    __syncthreads();
    float x0[8], x1[8];
#pragma unroll
    for (unsigned j = 0; j < 8; ++j) {
        const float sc =
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s.scale), j * 8));
        x0[j] = roundTf32(float(std::int8_t(s.xr[j] & 0xFFu)) * sc);
        x1[j] = roundTf32(float(std::int8_t(s.xr[j] >> 8)) * sc);
    }
#pragma unroll
    for (unsigned g = 0; g < NG; ++g) {
        if (NG > 1 && !(rwset & (1u << g))) continue;
        const unsigned rw = rws[g];
        float a0[8], a1[8];
#pragma unroll
        for (unsigned j = 0; j < 8; ++j) {
            a0[j] = table[g * 64 + j * 8 + (lane & 3)];
            a1[j] = table[g * 64 + j * 8 + 4 + (lane & 3)];
        }
        // rw is uniform; the accumulator quads are selected by a uniform switch.
#define TCC_MFMA_RW(R)                                                                           \
    for (unsigned j = 0; j < 8; ++j) {                                                           \
        acc[0][2 * R] = __builtin_amdgcn_mfma_f32_4x4x1f32(a0[j], x0[j], acc[0][2 * R], 0, 0, 0);   \
        acc[1][2 * R] = __builtin_amdgcn_mfma_f32_4x4x1f32(a0[j], x1[j], acc[1][2 * R], 0, 0, 0);   \
        acc[0][2 * R + 1] =                                                                      \
            __builtin_amdgcn_mfma_f32_4x4x1f32(a1[j], x0[j], acc[0][2 * R + 1], 0, 0, 0);       \
        acc[1][2 * R + 1] =                                                                      \
            __builtin_amdgcn_mfma_f32_4x4x1f32(a1[j], x1[j], acc[1][2 * R + 1], 0, 0, 0);       \
    }
        if (NG > 1) {
            if (g == 0) { TCC_MFMA_RW(0) }
            else if (g == 1) { TCC_MFMA_RW(1) }
            else if (g == 2) { TCC_MFMA_RW(2) }
            else { TCC_MFMA_RW(3) }
        } else {
            switch (rw) {
            case 0: TCC_MFMA_RW(0) break;
            case 1: TCC_MFMA_RW(1) break;
            case 2: TCC_MFMA_RW(2) break;
            default: TCC_MFMA_RW(3) break;
            }
        }
#undef TCC_MFMA_RW
    }
    __syncthreads();
}

// Row group of a panel in the exclusive phase: bucket slots 1..4 are RW0..RW3.
__device__ __forceinline__ unsigned exclusiveGroup(const unsigned* slots, unsigned panel) {
    return (panel >= slots[2]) + (panel >= slots[3]) + (panel >= slots[4]);
}

// Row-group set of a panel in the shared phase (bucket slots 5..15).
__device__ __forceinline__ unsigned sharedGroups(const unsigned* slots, unsigned panel) {
    unsigned s = 5;
#pragma unroll
    for (unsigned t = 6; t < 16; ++t) s += panel >= slots[t];
    return kBucketRwSet[s];
}

__device__ __forceinline__ void exclusivePhase(const KernelArgs& a, const unsigned* slots,
                                               unsigned begin, unsigned end, unsigned lane,
                                               __amdgpu_buffer_rsrc_t xr, unsigned xLane,
                                               unsigned features, float* table,
                                               f32x4 (&acc)[2][8]) {
    if (begin >= end) return;
    const unsigned last = end - 1;
    Meta m2 = loadMeta(a, begin, lane);
    Meta m1 = loadMeta(a, min(begin + 1, last), lane);
    unsigned g0 = exclusiveGroup(slots, begin);
    Stage2 cur;
    loadStage2<1>(a, m2, &g0, lane, xr, xLane, features, cur);
    m2 = loadMeta(a, min(begin + 2, last), lane);
#pragma unroll 1
    for (unsigned p = begin; p < end; ++p) {
        const unsigned q = min(p + 1, last);
        unsigned gq = exclusiveGroup(slots, q);
        Stage2 next;
        loadStage2<1>(a, m1, &gq, lane, xr, xLane, features, next);
        m1 = m2;
        m2 = loadMeta(a, min(p + 3, last), lane);
        computeStage3<1>(cur, &g0, 1u << g0, lane, table, acc);
        cur = next;
        g0 = gq;
    }
}

__device__ __forceinline__ void sharedPhase(const KernelArgs& a, const unsigned* slots,
                                            unsigned begin, unsigned end, unsigned lane,
                                            __amdgpu_buffer_rsrc_t xr, unsigned xLane,
                                            unsigned features, float* table,
                                            f32x4 (&acc)[2][8]) {
    if (begin >= end) return;
    const unsigned last = end - 1;
    const unsigned all[4] = {0, 1, 2, 3};
    Meta m2 = loadMeta(a, begin, lane);
    Meta m1 = loadMeta(a, min(begin + 1, last), lane);
    Stage2 cur;
    loadStage2<4>(a, m2, all, lane, xr, xLane, features, cur);
    unsigned set0 = sharedGroups(slots, begin);
    m2 = loadMeta(a, min(begin + 2, last), lane);
#pragma unroll 1
    for (unsigned p = begin; p < end; ++p) {
        const unsigned q = min(p + 1, last);
        Stage2 next;
        loadStage2<4>(a, m1, all, lane, xr, xLane, features, next);
        m1 = m2;
        m2 = loadMeta(a, min(p + 3, last), lane);
        computeStage3<4>(cur, all, set0, lane, table, acc);
        cur = next;
        set0 = sharedGroups(slots, q);
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
    __shared__ __align__(16) float table[4 * 64];
    __shared__ unsigned lastFlag;
    const unsigned lane = threadIdx.x;
    const unsigned slice = blockIdx.y;
    const unsigned taskIndex = xcdTask(blockIdx.x, a.m.taskCount);
    const Sw32Task task = a.m.tasks[taskIndex];
    const unsigned sw = task.sw;
    const unsigned f0 = 16 * (lane >> 3) + (lane & 7); // f1 = f0 + 8
    const unsigned xLane = slice * kSlice + 2 * lane;

    f32x4 acc[2][8];
#pragma unroll
    for (unsigned h = 0; h < 2; ++h)
#pragma unroll
        for (unsigned q = 0; q < 8; ++q) acc[h][q] = f32x4{0.f, 0.f, 0.f, 0.f};

    const unsigned* slots = a.m.bucketOffsets + std::size_t(sw) * 17;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<std::int8_t*>(a.packedX), 0, a.xBytes, 0x00020000);
    exclusivePhase(a, slots, max(slots[1], task.begin), min(slots[5], task.end), lane, xr, xLane,
                   Features, table, acc);
    sharedPhase(a, slots, max(slots[5], task.begin), min(slots[16], task.end), lane, xr, xLane,
                Features, table, acc);

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
    if (std::uint64_t(cols) * features > 0xFFFFFFFFull)
        throw std::invalid_argument("launchSpmmInt8: X must be smaller than 4 GiB (cols * features)");
    const KernelArgs args{matrix,   packedX, scales, output, workspace.partials, workspace.counters,
                          rows,     cols,    cols * features};
    if (features == 128)
        launch<128>(args, stream);
    else
        launch<256>(args, stream);
    checkHip(hipGetLastError());
}
