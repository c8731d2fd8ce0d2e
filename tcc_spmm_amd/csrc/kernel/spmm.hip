// Fused INT8-dequantization SpMM for MI355X (gfx950, wave64): Y = A x tf32(dequant(X)).
//
// Work decomposition
//   One wavefront per workgroup (task, slice): task = one Sw32Task (<= 384 panels of one 32-row
//   SW), slice = 128 features (blockIdx.y). The wave makes one pass per 8-row group (RW) g of the
//   SW, visiting every panel of the task that touches g: the exclusive bucket of g and the shared
//   buckets whose row-group mask contains g. A pass accumulates 8 rows x 128 features in
//   32 FP32 registers per lane; at its end the rows are final (or a partial tile for split tasks).
//
// Lane layout
//   X gathers: dword loads, two slots per instruction. Lane L (half H = L / 32, w = L % 32) loads
//   bytes 4w..4w+3 of the slice row of slot i + 4H in load i (i = 0..3), i.e. features
//   16t + {2m, 2m + 8, 2m + 1, 2m + 9} of the packed16 layout (t = w / 4, m = w % 4).
//   Per-slot data: lane L holds slot k = (L & 3) | (H << 2) and row r = (L >> 2) & 7, so the DPP
//   row broadcast `row_newbcast:i` hands every lane of 16-lane row R the value of slot i + 4*(R/2),
//   which is exactly the slot its half loads in load i.
//   MFMA v_mfma_f32_4x4x1_16b_f32: block b = lanes 4b..4b+3 (all in one half) computes
//   4 rows x 4 lane features; A = the quad's 4 row values of the half's slot (LDS table),
//   B = the lane's dequantized byte e, D = acc[quad][e]. The two halves hold partial sums of the
//   same features (even/odd slot positions) and are added at the end of the pass.
//
// Per panel: the A values of (slot k, row 8g + r) are TF32-rounded into an LDS table [8][8]
// (zero where the slot does not touch the row); X bytes are sign-extended to FP32 (SDWA),
// multiplied by the slot's scale (DPP broadcast) and TF32-rounded; TF32 x TF32 products are exact
// in FP32, so any accumulation order reproduces the reference's products. The panels of a pass are
// walked by a three-stage software pipeline (metadata two panels ahead; scales, A values and X one
// panel ahead) whose memory operations are identical on every path.
//
// Split SWs (reference src/kernel/spmm_kernel.cuh:228-282): a split task stores its row groups of
// `task.mask` as 8-row partial tiles [tile][8][F]; lane 0 then takes an agent-scope acq_rel
// wrapping ticket on counters[sw * (F/128) + slice] with limit chunks - 1, so the counter returns
// to zero by itself; the task whose ticket is chunks - 1 merges all partial tiles of the SW's
// slice in partialIds order starting from 0.0f and writes Y. No float atomics, no spin-waits.
#include "spmm.h"
#include "hip_support.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr unsigned kWave = 64;
constexpr unsigned kSlice = 128;
constexpr unsigned kNoPartial = 0xFFFFFFFFu;
constexpr unsigned kEnd = 0xFFFFFFFFu;

// Indexed buffer load: address = base + vindex * stride + voffset, range-checked on vindex.
__device__ int bufferLoadIndexed(i32x4 rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.buffer.load.i32");

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

// ------------------------------------------------------------------------------------------------
// Panel sets of one pass: the panels of the task that touch row group G, in increasing order.
// Bucket slot t occupies [lo[t], hi[t]) after clipping to the task; slot G + 1 is G's exclusive
// bucket, slots 5..15 are shared buckets, of which those whose row-group mask holds G belong.

__host__ __device__ constexpr bool slotTouches(unsigned slot, unsigned g) {
    // sw32BucketOrder (include/format/sw32.h): slot -> row-group mask.
    constexpr unsigned order[16] = {0, 1, 2, 4, 8, 3, 5, 6, 7, 9, 10, 11, 12, 13, 14, 15};
    return (order[slot] >> g) & 1u;
}

struct Bounds {
    unsigned lo[16], hi[16]; // clipped bucket ranges (uniform)
};

// First panel > p (or >= p when `inclusive`) of pass G, or kEnd.
template <unsigned G>
__device__ __forceinline__ unsigned nextPanel(const Bounds& b, unsigned p) {
    unsigned best = kEnd;
#pragma unroll
    for (unsigned t = 1; t < 16; ++t) {
        if (!slotTouches(t, G)) continue;
        const unsigned c = max(b.lo[t], p);
        if (c < b.hi[t]) best = min(best, c);
    }
    return best;
}

template <unsigned G>
__device__ __forceinline__ unsigned panelCount(const Bounds& b) {
    unsigned n = 0;
#pragma unroll
    for (unsigned t = 1; t < 16; ++t)
        if (slotTouches(t, G) && b.hi[t] > b.lo[t]) n += b.hi[t] - b.lo[t];
    return n;
}

// ------------------------------------------------------------------------------------------------
// Pipeline stages

struct Meta { // slot k(L) of one panel
    unsigned id;
    unsigned mask;
    unsigned base;
};

struct Stage2 {     // one panel, ready to compute
    unsigned src;   // lane: clamped source id of slot k(L) (row 0 for padding)
    float scale;    // lane: scale of that source
    float v;        // lane: raw A value of (slot k(L), row 8G + r(L))
    unsigned bits;  // 1 when slot k(L) touches that row
    unsigned xr[4]; // X dwords of loads 0..3 for this lane
};

__device__ __forceinline__ unsigned slotOf(unsigned lane) { return (lane & 3) | ((lane >> 5) << 2); }

__device__ __forceinline__ Meta loadMeta(const KernelArgs& a, unsigned panel, unsigned lane) {
    const std::size_t slot = std::size_t(panel) * 8 + slotOf(lane);
    const std::uint64_t md = __builtin_nontemporal_load(a.m.sourceMetadata + slot);
    return {__builtin_nontemporal_load(a.m.sourceIds + slot), unsigned(md), unsigned(md >> 32)};
}

template <unsigned G>
__device__ __forceinline__ void loadStage2(const KernelArgs& a, const Meta& m, unsigned lane,
                                           i32x4 xr, unsigned xLane, Stage2& s) {
    const bool live = m.id < a.cols;
    s.src = live ? m.id : 0u;
    s.scale = a.scales[s.src];
    const unsigned row = G * 8 + ((lane >> 2) & 7);
    const bool present = live && ((m.mask >> row) & 1u);
    // The k-th set row bit of a slot owns values[base + k]; absent rows read values[base] (a valid
    // index: padding has base 0 and a matrix with panels has values).
    const unsigned idx = present ? m.base + __popc(m.mask & ((1u << row) - 1u)) : m.base;
    s.v = __builtin_nontemporal_load(a.m.values + idx);
    s.bits = present;
    // Source row of the slot this lane's half loads in load i (slot i + 4H): DPP row broadcast.
    s.xr[0] = unsigned(bufferLoadIndexed(
        xr, __builtin_amdgcn_mov_dpp(int(s.src), 0x150, 0xF, 0xF, true), int(xLane), 0, 0));
    s.xr[1] = unsigned(bufferLoadIndexed(
        xr, __builtin_amdgcn_mov_dpp(int(s.src), 0x151, 0xF, 0xF, true), int(xLane), 0, 0));
    s.xr[2] = unsigned(bufferLoadIndexed(
        xr, __builtin_amdgcn_mov_dpp(int(s.src), 0x152, 0xF, 0xF, true), int(xLane), 0, 0));
    s.xr[3] = unsigned(bufferLoadIndexed(
        xr, __builtin_amdgcn_mov_dpp(int(s.src), 0x153, 0xF, 0xF, true), int(xLane), 0, 0));
}

// Dequantize load i: bytes 0..3 -> FP32 (sign-extended SDWA converts), times the scale of the
// half's slot (DPP row broadcast of lane i of each 16-lane row), rounded to TF32. The s_nop covers
// the VALU-write -> DPP-read hazard on the scale register.
template <unsigned I>
__device__ __forceinline__ void dequantize(unsigned w, float scale, float (&x)[4]) {
    float q0, q1, q2, q3;
    asm volatile(
        "v_cvt_f32_i32_sdwa %0, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f32_i32_sdwa %2, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f32_i32_sdwa %3, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %5, %0 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %1, %5, %1 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %2, %5, %2 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %3, %5, %3 row_newbcast:%6 row_mask:0xf bank_mask:0xf"
        : "=&v"(q0), "=&v"(q1), "=&v"(q2), "=&v"(q3)
        : "v"(w), "v"(scale), "i"(I));
    x[0] = roundTf32(q0);
    x[1] = roundTf32(q1);
    x[2] = roundTf32(q2);
    x[3] = roundTf32(q3);
}

template <unsigned I>
__device__ __forceinline__ void accumulateLoad(const Stage2& s, const float* table,
                                               unsigned tableLane, f32x4 (&acc)[2][4]) {
    float x[4];
    dequantize<I>(s.xr[I], s.scale, x);
    // A of quad h for lane 4b+i: row 4h + i of the half's slot I + 4H.
    const float a0 = table[tableLane + I];
    const float a1 = table[tableLane + 32 + I];
#pragma unroll
    for (unsigned e = 0; e < 4; ++e) {
        acc[0][e] = __builtin_amdgcn_mfma_f32_4x4x1f32(a0, x[e], acc[0][e], 0, 0, 0);
        acc[1][e] = __builtin_amdgcn_mfma_f32_4x4x1f32(a1, x[e], acc[1][e], 0, 0, 0);
    }
}

__device__ __forceinline__ void computeStage3(const Stage2& s, unsigned lane, float* table,
                                              unsigned tableLane, f32x4 (&acc)[2][4]) {
    // table[r][k] = tf32(A[row 8G + r][slot k]), 0 when absent.
    table[((lane >> 2) & 7) * 8 + slotOf(lane)] = s.bits ? roundTf32(s.v) : 0.0f;
    __syncthreads();
    accumulateLoad<0>(s, table, tableLane, acc);
    accumulateLoad<1>(s, table, tableLane, acc);
    accumulateLoad<2>(s, table, tableLane, acc);
    accumulateLoad<3>(s, table, tableLane, acc);
    __syncthreads();
}

// One pass over the panels of row group G. Unrolled by two so the stage-2 buffers alternate
// instead of being copied; panel indices past the end repeat the last panel (harmless loads).
template <unsigned G>
__device__ __forceinline__ void rowGroupPass(const KernelArgs& a, const Bounds& bounds,
                                             unsigned lane, i32x4 xr, unsigned xLane,
                                             float* table, unsigned tableLane,
                                             f32x4 (&acc)[2][4]) {
    const unsigned n = panelCount<G>(bounds);
    if (!n) return;
    unsigned p0 = nextPanel<G>(bounds, 0);
    unsigned p1 = nextPanel<G>(bounds, p0 + 1);
    p1 = p1 == kEnd ? p0 : p1;
    unsigned p2 = nextPanel<G>(bounds, p1 + 1);
    p2 = p2 == kEnd ? p1 : p2;
    Stage2 sa, sb;
    loadStage2<G>(a, loadMeta(a, p0, lane), lane, xr, xLane, sa);
    Meta m1 = loadMeta(a, p1, lane);
    Meta m2 = loadMeta(a, p2, lane);
#pragma unroll 1
    for (unsigned i = 0; i < n; i += 2) {
        // Iteration i: stage 2 of panel i+1 (metadata m1), stage 1 of panel i+3, compute panel i.
        loadStage2<G>(a, m1, lane, xr, xLane, sb);
        {
            unsigned p3 = nextPanel<G>(bounds, p2 + 1);
            p3 = p3 == kEnd ? p2 : p3;
            m1 = m2;
            m2 = loadMeta(a, p3, lane);
            p2 = p3;
        }
        computeStage3(sa, lane, table, tableLane, acc);
        if (i + 1 >= n) break;
        loadStage2<G>(a, m1, lane, xr, xLane, sa);
        {
            unsigned p3 = nextPanel<G>(bounds, p2 + 1);
            p3 = p3 == kEnd ? p2 : p3;
            m1 = m2;
            m2 = loadMeta(a, p3, lane);
            p2 = p3;
        }
        computeStage3(sb, lane, table, tableLane, acc);
    }
}

// Sum the two halves' partial sums (even / odd slot positions) of one pass and store the 8 rows:
// lanes of half 0 store rows 0..3 (quad 0), half 1 rows 4..7 (quad 1). Each lane holds features
// 16t + {2m, 2m+8, 2m+1, 2m+9} (elements e = 0..3), stored as two float2.
__device__ __forceinline__ void storeRows(f32x4 (&acc)[2][4], unsigned lane, float* base,
                                          unsigned rowStride, unsigned validRows, unsigned colA,
                                          bool nontemporal) {
#pragma unroll
    for (unsigned h = 0; h < 2; ++h)
#pragma unroll
        for (unsigned e = 0; e < 4; ++e)
#pragma unroll
            for (unsigned i = 0; i < 4; ++i) acc[h][e][i] += __shfl_xor(acc[h][e][i], 32);
    const unsigned h = lane >> 5;
#pragma unroll
    for (unsigned i = 0; i < 4; ++i) {
        const unsigned row = h * 4 + i;
        if (row >= validRows) continue;
        float* r = base + std::size_t(row) * rowStride + colA;
        const f32x2 lo = h ? f32x2{acc[1][0][i], acc[1][2][i]} : f32x2{acc[0][0][i], acc[0][2][i]};
        const f32x2 hi = h ? f32x2{acc[1][1][i], acc[1][3][i]} : f32x2{acc[0][1][i], acc[0][3][i]};
        if (nontemporal) {
            __builtin_nontemporal_store(lo, reinterpret_cast<f32x2*>(r));
            __builtin_nontemporal_store(hi, reinterpret_cast<f32x2*>(r + 8));
        } else {
            *reinterpret_cast<f32x2*>(r) = lo;
            *reinterpret_cast<f32x2*>(r + 8) = hi;
        }
    }
}

template <unsigned G, unsigned Features>
__device__ __forceinline__ void runGroup(const KernelArgs& a, const Sw32Task& task,
                                         const Bounds& bounds, unsigned lane, i32x4 xr,
                                         unsigned xLane, float* table, unsigned tableLane,
                                         unsigned colA) {
    const bool split = task.partial != kNoPartial;
    if (split && !((task.mask >> G) & 1u)) return;
    f32x4 acc[2][4];
#pragma unroll
    for (unsigned h = 0; h < 2; ++h)
#pragma unroll
        for (unsigned e = 0; e < 4; ++e) acc[h][e] = f32x4{0.f, 0.f, 0.f, 0.f};
    rowGroupPass<G>(a, bounds, lane, xr, xLane, table, tableLane, acc);
    if (!split) {
        const unsigned row0 = task.sw * 32 + G * 8;
        if (row0 < a.rows)
            storeRows(acc, lane, a.y + std::size_t(row0) * Features, Features,
                      min(8u, a.rows - row0), colA, true);
    } else {
        const std::size_t tile = task.partial + __popc(task.mask & ((1u << G) - 1u));
        storeRows(acc, lane, a.partials + tile * 8 * Features, Features, 8, colA, false);
    }
}

// Workgroup -> task: each of the 8 XCDs (workgroups are dispatched round-robin by id) walks one
// contiguous range of tasks, so neighbouring SWs share source rows of X in that XCD's L2.
__device__ __forceinline__ unsigned xcdTask(unsigned bid, unsigned tasks) {
    const unsigned xcd = bid & 7u, j = bid >> 3;
    const unsigned q = tasks >> 3, r = tasks & 7u;
    return xcd * q + min(xcd, r) + j;
}

template <unsigned Features>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(4))) void spmmInt8Kernel(
    KernelArgs a) {
    __shared__ __align__(16) float table[64];
    __shared__ unsigned lastFlag;
    const unsigned lane = threadIdx.x;
    const unsigned slice = blockIdx.y;
    const Sw32Task task = a.m.tasks[xcdTask(blockIdx.x, a.m.taskCount)];
    const unsigned sw = task.sw;

    Bounds bounds;
    {
        const unsigned* slots = a.m.bucketOffsets + std::size_t(sw) * 17;
#pragma unroll
        for (unsigned t = 1; t < 16; ++t) {
            bounds.lo[t] = max(slots[t], task.begin);
            bounds.hi[t] = min(slots[t + 1], task.end);
        }
        bounds.lo[0] = bounds.hi[0] = 0;
    }
    // X rows of this slice: base + src * Features, dword w of the 128-byte slice per lane.
    i32x4 xr;
    {
        const std::uint64_t base = reinterpret_cast<std::uint64_t>(a.packedX) + slice * kSlice;
        xr.x = int(unsigned(base));
        xr.y = int((unsigned(base >> 32) & 0xFFFFu) | (Features << 16));
        xr.z = int(a.cols);
        xr.w = 0x00020000;
    }
    const unsigned w = lane & 31;
    const unsigned xLane = 4 * w;
    // Store column of element 0 (features 16t + 2m and 16t + 2m + 1; +8 for elements 1 and 3).
    const unsigned colA = slice * kSlice + 16 * (w >> 2) + 2 * (w & 3);
    // LDS table index of row (lane & 3) of the quad for the half's slot (load index added later).
    const unsigned tableLane = (lane & 3) * 8 + 4 * (lane >> 5);

    runGroup<0, Features>(a, task, bounds, lane, xr, xLane, table, tableLane, colA);
    runGroup<1, Features>(a, task, bounds, lane, xr, xLane, table, tableLane, colA);
    runGroup<2, Features>(a, task, bounds, lane, xr, xLane, table, tableLane, colA);
    runGroup<3, Features>(a, task, bounds, lane, xr, xLane, table, tableLane, colA);
    if (task.partial == kNoPartial) return;

    // Completion ticket: the acq_rel RMW at agent scope publishes this task's partial tiles and,
    // for the last arriver, makes every other task's tiles visible (the XCD L2s are not coherent
    // with each other, so the release writes back and the acquire invalidates).
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
    // Merge the slice: each lane sums columns lane and lane + 64, adding the partial tiles in
    // partialIds (task) order starting from 0.0f.
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
    if (matrix.taskCount > 0x7FFFFFFFu)
        throw std::invalid_argument("launchSpmmInt8: too many tasks for one launch");
    const KernelArgs args{matrix, packedX, scales, output, workspace.partials, workspace.counters,
                          rows,   cols};
    if (features == 128)
        launch<128>(args, stream);
    else
        launch<256>(args, stream);
    checkHip(hipGetLastError());
}
