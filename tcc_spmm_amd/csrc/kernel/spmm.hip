// Fused INT8-dequantization SpMM for MI355X (gfx950, wave64): Y = A x tf32(dequant(X)).
//
// Work decomposition
//   One wavefront per workgroup. Workgroup (task, half, slice): task = one Sw32Task (<= 384 panels
//   of one 32-row SW), slice = 128 features (blockIdx.y), half = 64 of those features. Lane l owns
//   feature slice*128 + half*64 + l and accumulates it for all 32 rows of the SW: 8 four-row quads
//   x 4 rows = 32 FP32 accumulators.
//
// Per panel of 8 slots (lane layout for per-slot data: slot k = l & 7, row r = (l >> 3) & 7)
//   * the wave expands the panel's A values into a dense LDS table [row group][8 rows][8 slots]
//     (TF32-rounded, zero where the slot does not touch the row);
//   * gathers the 8 source rows of X (one 64-byte load per slot: one INT8 per lane), converts,
//     multiplies by the source's scale (taken from lane k of the 16-lane row by a DPP row broadcast)
//     and rounds to TF32; TF32 x TF32 products are exact in FP32, so any accumulation order
//     reproduces the reference's products;
//   * accumulates with v_mfma_f32_4x4x1_16b_f32: A = the 4 row values of one quad (LDS broadcast
//     read), B = the lane's dequantized feature, D = 4 rows x the lane's feature.
// The panels of a task are walked with a three-stage software pipeline (metadata two panels ahead,
// A values / scales / X one panel ahead) whose memory operations are identical on every path.
// Exclusive buckets (slots 1..4, one row group each) run with the row group as a compile-time
// constant; shared buckets (slots 5..15) compute the row groups of their bucket mask.
//
// Split SWs (reference src/kernel/spmm_kernel.cuh:228-282): a split task stores its row groups of
// `task.mask` as 8-row partial tiles [tile][8][F]; lane 0 then takes an agent-scope acq_rel
// wrapping ticket on counters[sw * (F/128) + slice]. Both feature halves of every chunk of the SW
// take a ticket, so the limit is 2*chunks - 1 and the counter returns to zero by itself; the wave
// whose ticket is the last merges all partial tiles of the SW's 128-feature slice in partialIds
// order starting from 0.0f and writes Y. No float atomics, no spin-waits.
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
constexpr unsigned kHalves = kSlice / kWave;
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

// ------------------------------------------------------------------------------------------------
// Pipeline stages

struct Meta { // slot k = lane & 7 of one panel
    unsigned id;
    unsigned mask;
    unsigned base;
};

struct Stage2 {      // one panel, ready to compute
    unsigned src;    // lane k: clamped source id of slot k (row 0 for padding)
    float scale;     // lane k: scale of that source
    float v[4];      // raw A values of (slot k, row 8g + r) for the panel's row groups g
    unsigned bits;   // bit g: slot k touches row 8g + r
    unsigned xr[8];  // sign-extended X byte of slot j for this lane's feature
};

__device__ __forceinline__ Meta loadMeta(const KernelArgs& a, unsigned panel, unsigned lane) {
    const std::size_t slot = std::size_t(panel) * 8 + (lane & 7);
    const std::uint64_t md = __builtin_nontemporal_load(a.m.sourceMetadata + slot);
    return {__builtin_nontemporal_load(a.m.sourceIds + slot), unsigned(md), unsigned(md >> 32)};
}

// Stage 2 of one panel. G[g] are the row groups whose A values are fetched (NG of them).
template <unsigned NG>
__device__ __forceinline__ void loadStage2(const KernelArgs& a, const Meta& m, const unsigned* G,
                                           unsigned lane, __amdgpu_buffer_rsrc_t xr,
                                           unsigned xLane, unsigned features, Stage2& s) {
    const bool live = m.id < a.cols;
    s.src = live ? m.id : 0u;
    s.scale = a.scales[s.src];
    const unsigned r = (lane >> 3) & 7;
    s.bits = 0;
#pragma unroll
    for (unsigned g = 0; g < NG; ++g) {
        const unsigned row = G[g] * 8 + r;
        const bool present = live && ((m.mask >> row) & 1u);
        // The k-th set row bit of a slot owns values[base + k]; absent rows read values[base]
        // (a valid index: padding has base 0 and a matrix with panels has values).
        const unsigned idx = present ? m.base + __popc(m.mask & ((1u << row) - 1u)) : m.base;
        s.v[g] = __builtin_nontemporal_load(a.m.values + idx);
        s.bits |= unsigned(present) << g;
    }
#pragma unroll
    for (unsigned j = 0; j < 8; ++j) {
        const unsigned src = __builtin_amdgcn_readlane(s.src, j);
        s.xr[j] = unsigned(int(std::int8_t(
            __builtin_amdgcn_raw_buffer_load_b8(xr, xLane, src * features, 0))));
    }
}

// x[j] = tf32(float(q_j) * scale of slot j); the scale comes from lane j of the lane's 16-lane row
// (DPP row broadcast), which holds slot j's scale in the stage-2 lane layout. The s_nop covers the
// VALU-write -> DPP-read hazard on the scale register.
__device__ __forceinline__ void dequantize(const Stage2& s, float (&x)[8]) {
    float q[8];
#pragma unroll
    for (unsigned j = 0; j < 8; ++j) q[j] = float(int(s.xr[j]));
    asm volatile(
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %8, %0 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %1, %8, %1 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %2, %8, %2 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %3, %8, %3 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %4, %8, %4 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %5, %8, %5 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %6, %8, %6 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %7, %8, %7 row_newbcast:7 row_mask:0xf bank_mask:0xf"
        : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]), "+v"(q[6]),
          "+v"(q[7])
        : "v"(s.scale));
#pragma unroll
    for (unsigned j = 0; j < 8; ++j) x[j] = roundTf32(q[j]);
}

// Stage 3: accumulate one panel. Exclusive phase: NG = 1 and the row group is the compile-time G.
// Shared phase: NG = 4, row groups 0..3 of which those in `rwset` are computed.
template <unsigned NG, unsigned G>
__device__ __forceinline__ void computeStage3(const Stage2& s, unsigned rwset, unsigned lane,
                                              float* table, f32x4 (&acc)[8]) {
    // table[g][r][k] = tf32(A[row 8g' + r][slot k]), 0 when absent (g' = the g-th row group).
#pragma unroll
    for (unsigned g = 0; g < NG; ++g)
        table[g * 64 + lane] = ((s.bits >> g) & 1u) ? roundTf32(s.v[g]) : 0.0f;
    __syncthreads();
    float x[8];
    dequantize(s, x);
    const unsigned quadRow = (lane & 3) * 8; // lane 4b+i reads row 4h+i of quad h
#pragma unroll
    for (unsigned g = 0; g < NG; ++g) {
        if (NG > 1 && !(rwset & (1u << g))) continue;
        const unsigned rw = NG > 1 ? g : G;
        float a0[8], a1[8];
#pragma unroll
        for (unsigned j = 0; j < 8; ++j) {
            a0[j] = table[g * 64 + quadRow + j];
            a1[j] = table[g * 64 + 32 + quadRow + j];
        }
#pragma unroll
        for (unsigned j = 0; j < 8; ++j) {
            acc[2 * rw] = __builtin_amdgcn_mfma_f32_4x4x1f32(a0[j], x[j], acc[2 * rw], 0, 0, 0);
            acc[2 * rw + 1] =
                __builtin_amdgcn_mfma_f32_4x4x1f32(a1[j], x[j], acc[2 * rw + 1], 0, 0, 0);
        }
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

struct Pipe {
    Meta m1, m2;  // metadata of panels p+1 and p+2
    Stage2 cur;   // stage-2 data of panel p
};

// Panels [p, pEnd) of exclusive row group G, continuing the pipeline in `st`. Unrolled by two so
// the stage-2 buffers alternate instead of being copied.
template <unsigned G>
__device__ __forceinline__ void exclusiveRun(const KernelArgs& a, const unsigned* slots, unsigned p,
                                             unsigned pEnd, unsigned last, unsigned lane,
                                             __amdgpu_buffer_rsrc_t xr, unsigned xLane,
                                             unsigned features, float* table, Pipe& st,
                                             f32x4 (&acc)[8]) {
#pragma unroll 1
    while (p < pEnd) {
        Stage2 nb;
        {
            const unsigned gq = exclusiveGroup(slots, min(p + 1, last));
            loadStage2<1>(a, st.m1, &gq, lane, xr, xLane, features, nb);
            st.m1 = st.m2;
            st.m2 = loadMeta(a, min(p + 3, last), lane);
        }
        computeStage3<1, G>(st.cur, 1u << G, lane, table, acc);
        if (++p >= pEnd) {
            st.cur = nb;
            return;
        }
        {
            const unsigned gq = exclusiveGroup(slots, min(p + 1, last));
            loadStage2<1>(a, st.m1, &gq, lane, xr, xLane, features, st.cur);
            st.m1 = st.m2;
            st.m2 = loadMeta(a, min(p + 3, last), lane);
        }
        computeStage3<1, G>(nb, 1u << G, lane, table, acc);
        ++p;
    }
}

__device__ __forceinline__ void exclusivePhase(const KernelArgs& a, const unsigned* slots,
                                               unsigned begin, unsigned end, unsigned lane,
                                               __amdgpu_buffer_rsrc_t xr, unsigned xLane,
                                               unsigned features, float* table, f32x4 (&acc)[8]) {
    if (begin >= end) return;
    const unsigned last = end - 1;
    Pipe st;
    const Meta m0 = loadMeta(a, begin, lane);
    st.m1 = loadMeta(a, min(begin + 1, last), lane);
    const unsigned g0 = exclusiveGroup(slots, begin);
    loadStage2<1>(a, m0, &g0, lane, xr, xLane, features, st.cur);
    st.m2 = loadMeta(a, min(begin + 2, last), lane);
    // Row group g covers panels [slots[g+1], slots[g+2]) of the SW.
    unsigned p = begin;
#pragma unroll 1
    for (unsigned g = g0; g < 4 && p < end; ++g) {
        const unsigned gEnd = min(end, slots[g + 2]);
        switch (g) {
        case 0: exclusiveRun<0>(a, slots, p, gEnd, last, lane, xr, xLane, features, table, st, acc); break;
        case 1: exclusiveRun<1>(a, slots, p, gEnd, last, lane, xr, xLane, features, table, st, acc); break;
        case 2: exclusiveRun<2>(a, slots, p, gEnd, last, lane, xr, xLane, features, table, st, acc); break;
        default: exclusiveRun<3>(a, slots, p, gEnd, last, lane, xr, xLane, features, table, st, acc); break;
        }
        p = max(p, gEnd);
    }
}

__device__ __forceinline__ void sharedPhase(const KernelArgs& a, const unsigned* slots,
                                            unsigned begin, unsigned end, unsigned lane,
                                            __amdgpu_buffer_rsrc_t xr, unsigned xLane,
                                            unsigned features, float* table, f32x4 (&acc)[8]) {
    if (begin >= end) return;
    const unsigned last = end - 1;
    const unsigned all[4] = {0, 1, 2, 3};
    Meta m1 = loadMeta(a, begin, lane);
    Meta m2 = loadMeta(a, min(begin + 1, last), lane);
    Stage2 cur;
    loadStage2<4>(a, m1, all, lane, xr, xLane, features, cur);
    unsigned set0 = sharedGroups(slots, begin);
    m1 = m2;
    m2 = loadMeta(a, min(begin + 2, last), lane);
#pragma unroll 1
    for (unsigned p = begin; p < end; ++p) {
        const unsigned q = min(p + 1, last);
        Stage2 next;
        loadStage2<4>(a, m1, all, lane, xr, xLane, features, next);
        m1 = m2;
        m2 = loadMeta(a, min(p + 3, last), lane);
        computeStage3<4, 0>(cur, set0, lane, table, acc);
        cur = next;
        set0 = sharedGroups(slots, q);
    }
}

// ------------------------------------------------------------------------------------------------

// Workgroup -> (task, half): each of the 8 XCDs (workgroups are dispatched round-robin by id)
// walks one contiguous range of tasks, and the two feature halves of a task are neighbours on
// the same XCD, so neighbouring SWs and both halves share X rows in that XCD's L2.
__device__ __forceinline__ void xcdTask(unsigned bid, unsigned tasks, unsigned& task,
                                        unsigned& half) {
    const unsigned units = tasks * kHalves;
    const unsigned xcd = bid & 7u, j = bid >> 3;
    const unsigned q = units >> 3, r = units & 7u;
    const unsigned unit = xcd * q + min(xcd, r) + j;
    task = unit / kHalves;
    half = unit % kHalves;
}

template <unsigned Features>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(4))) void spmmInt8Kernel(
    KernelArgs a) {
    __shared__ __align__(16) float table[4 * 64];
    __shared__ unsigned lastFlag;
    const unsigned lane = threadIdx.x;
    const unsigned slice = blockIdx.y;
    unsigned taskIndex, half;
    xcdTask(blockIdx.x, a.m.taskCount, taskIndex, half);
    const Sw32Task task = a.m.tasks[taskIndex];
    const unsigned sw = task.sw;
    // Feature of this lane and its byte inside the packed16 row: position j of a 16-feature tile
    // is stored at byte 2j (j < 8) or 2(j - 8) + 1 of the tile.
    const unsigned local = half * kWave + lane;
    const unsigned jt = local & 15u;
    const unsigned xLane =
        slice * kSlice + (local & ~15u) + (jt < 8 ? 2 * jt : 2 * (jt - 8) + 1);
    const unsigned col = slice * kSlice + local;

    f32x4 acc[8];
#pragma unroll
    for (unsigned q = 0; q < 8; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};

    const unsigned* slots = a.m.bucketOffsets + std::size_t(sw) * 17;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<std::int8_t*>(a.packedX), 0, a.xBytes, 0x00020000);
    exclusivePhase(a, slots, max(slots[1], task.begin), min(slots[5], task.end), lane, xr, xLane,
                   Features, table, acc);
    sharedPhase(a, slots, max(slots[5], task.begin), min(slots[16], task.end), lane, xr, xLane,
                Features, table, acc);

    // Write-back: D of quad q holds rows 4q..4q+3 (vector element i = row 4q+i) of this lane's
    // feature column.
    if (task.partial == kNoPartial) {
        const unsigned rowbase = sw * 32;
#pragma unroll
        for (unsigned q = 0; q < 8; ++q)
#pragma unroll
            for (unsigned i = 0; i < 4; ++i) {
                const unsigned row = rowbase + q * 4 + i;
                if (row < a.rows)
                    __builtin_nontemporal_store(acc[q][i], a.y + std::size_t(row) * Features + col);
            }
        return;
    }
#pragma unroll
    for (unsigned rw = 0; rw < 4; ++rw) {
        if (!(task.mask & (1u << rw))) continue;
        const std::size_t tile = task.partial + __popc(task.mask & ((1u << rw) - 1u));
#pragma unroll
        for (unsigned h = 0; h < 2; ++h)
#pragma unroll
            for (unsigned i = 0; i < 4; ++i)
                a.partials[(tile * 8 + h * 4 + i) * Features + col] = acc[rw * 2 + h][i];
    }
    // Completion ticket: the acq_rel RMW at agent scope publishes this wave's partial tiles and,
    // for the last arriver, makes every other wave's tiles visible (the XCD L2s are not coherent
    // with each other, so the release writes back and the acquire invalidates).
    __syncthreads();
    if (lane == 0) {
        unsigned* counter = a.counters + std::size_t(sw) * (Features / kSlice) + slice;
        const unsigned arrivals = task.chunks * kHalves;
        const unsigned ticket =
            __builtin_amdgcn_atomic_inc32(counter, arrivals - 1, __ATOMIC_ACQ_REL, "agent");
        lastFlag = ticket == arrivals - 1;
    }
    __syncthreads();
    if (!lastFlag) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // Merge the whole 128-feature slice: each lane sums columns lane and lane + 64, adding the
    // partial tiles in partialIds (task) order starting from 0.0f.
    const unsigned mcol = slice * kSlice + lane;
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
                    a.partials + (std::size_t(a.m.partialIds[item]) * 8 + r) * Features + mcol;
                lo += pr[0];
                hi += pr[kWave];
            }
            float* yr = a.y + std::size_t(row0 + r) * Features + mcol;
            yr[0] = lo;
            yr[kWave] = hi;
        }
    }
}

template <unsigned Features>
void launch(const KernelArgs& args, hipStream_t stream) {
    const dim3 grid(args.m.taskCount * kHalves, Features / kSlice);
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
    if (std::uint64_t(matrix.taskCount) * kHalves > 0x7FFFFFFFull)
        throw std::invalid_argument("launchSpmmInt8: too many tasks for one launch");
    const KernelArgs args{matrix, packedX, scales, output, workspace.partials, workspace.counters,
                          rows,   cols,    cols * features};
    if (features == 128)
        launch<128>(args, stream);
    else
        launch<256>(args, stream);
    checkHip(hipGetLastError());
}
