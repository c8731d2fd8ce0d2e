// Fused INT8-dequantization SpMM for MI355X (gfx950, wave64): Y = A x tf32(dequant(X)).
//
// Work decomposition
//   One wavefront per workgroup (task, slice): task = one Sw32Task (<= 384 panels of one 32-row
//   SW), slice = 128 features (blockIdx.y). The wave makes one pass per 8-row group (RW) g of the
//   SW, visiting every panel of the task that touches g: the exclusive bucket of g and the shared
//   buckets whose row-group mask contains g. A pass accumulates 8 rows x 128 features in
//   16 FP32 registers per lane; at its end the rows are final (or a partial tile for split tasks).
//
// Lane layout
//   Per-slot data (metadata, scale, A table entries): lane L holds slot k = L & 7 and row
//   r = (L >> 3) & 7, so the DPP row broadcast `row_newbcast:j` hands every lane slot j's value.
//   X gathers: one dwordx4 load per panel, lane L fetching the 16-byte tile L & 7 of the 128-byte
//   slice row of slot L >> 3 (eight rows per instruction). The tile is written to LDS and read back
//   transposed: lane l then holds byte pair l (features 16(l/8) + l%8 and + 8) of all 8 slots.
//   MFMA v_mfma_f32_4x4x4_16b_f16 (16 blocks of 4 x 4 x 4): lane 4b+i supplies A = row 4h+i of
//   quad h for four slots (LDS table), lane 4b+j supplies B = its feature of the same four slots,
//   and D[i][j] (row 4h+i, the lane's feature) lands in lane 4b+j register i: acc[quad][feature].
//
// Per panel: the A values of (slot k, row 8g + r) are TF32-rounded, scaled by 2^(e_k + kShift)
// (e_k: binary exponent of slot k's scale) and stored as f16 in an LDS table [8][8]; X bytes are
// sign-extended to FP32 (SDWA), multiplied by the mantissa of the slot's scale (DPP broadcast),
// TF32-rounded and converted to f16 (exact: 11 significant bits in f16's normal range). The f16
// products are exact in the FP32 accumulator and equal 2^kShift times the reference's TF32 x TF32
// products, so any accumulation order reproduces them; a pass ends by scaling with 2^-kShift. A
// panel whose scaled A values leave f16's normal range takes an FP32 path with the same products
// (v_mfma_f32_4x4x1_16b_f32 on tf32(a) * 2^kShift and the TF32 features). The panels of a pass
// are walked by a three-stage software pipeline (metadata two panels ahead; scales, A values and X
// one panel ahead) whose memory operations are identical on every path.
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
#include <cstdlib>
#include <stdexcept>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __fp16 f16x2 __attribute__((ext_vector_type(2)));

constexpr unsigned kWave = 64;
constexpr unsigned kSlice = 128;
constexpr unsigned kNoPartial = 0xFFFFFFFFu;
constexpr unsigned kEnd = 0xFFFFFFFFu;

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

struct Meta {        // one panel
    unsigned id;     // lane L: source of slot L & 7
    unsigned mask;   // lane L: row mask of slot L & 7
    unsigned base;   // lane L: value base of slot L & 7
    unsigned gather; // lane L: source of slot L >> 3 (the row this lane gathers)
};

struct Stage2 {   // one panel, ready to compute
    float scale;  // lane L: scale of slot L & 7
    float v;      // lane L: raw A value of (slot L & 7, row 8G + r)
    unsigned bits;// 1 when slot L & 7 touches that row
    u32x4 x;      // 16-byte tile L & 7 of the X row of slot L >> 3
};

// Memory access of one task. Narrow (every packed X slice and the scales addressable with 32-bit
// byte offsets, the usual case): buffer loads. sourceIds and sourceMetadata use a per-task base
// and a scalar panel offset; scales and X use buffers sized from `cols`, so the padding sentinel
// source UINT32_MAX lands out of range and reads 0 without a clamp. Wide: 64-bit global loads
// with clamped indices.
constexpr int kNt = 2; // buffer cache policy: nontemporal (streamed once)

template <bool Wide>
struct Loader;

template <>
struct Loader<false> {
    __amdgpu_buffer_rsrc_t ids, meta, scales, x;
    const float* values;
    unsigned first;     // task.begin: panel offsets are relative to it
    unsigned xShift;    // log2(features)
    unsigned sliceByte; // slice * 128

    __device__ Loader(const KernelArgs& a, unsigned begin, unsigned features, unsigned slice)
        : values(a.m.values), first(begin), xShift(features == 256 ? 8u : 7u),
          sliceByte(slice * kSlice) {
        const std::size_t slot0 = std::size_t(begin) * 8;
        ids = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned*>(a.m.sourceIds + slot0), 0,
                                                0x7FFFFFF0, 0x00020000);
        meta = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<std::uint64_t*>(a.m.sourceMetadata + slot0), 0, 0x7FFFFFF0, 0x00020000);
        scales = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.scales), 0, a.cols * 4u,
                                                   0x00020000);
        x = __builtin_amdgcn_make_buffer_rsrc(const_cast<std::int8_t*>(a.packedX), 0,
                                              a.cols << xShift, 0x00020000);
    }
    __device__ Meta meta8(unsigned panel, unsigned lane) const {
        const int off = int((panel - first) * 32u);
        const auto md = __builtin_amdgcn_raw_buffer_load_b64(meta, (lane & 7) * 8, 2 * off, kNt);
        return {__builtin_amdgcn_raw_buffer_load_b32(ids, (lane & 7) * 4, off, kNt), md[0], md[1],
                __builtin_amdgcn_raw_buffer_load_b32(ids, (lane >> 3) * 4, off, kNt)};
    }
    __device__ float scale(unsigned src) const {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(scales, src * 4u, 0, 0));
    }
    __device__ float value(unsigned idx) const { return __builtin_nontemporal_load(values + idx); }
    __device__ u32x4 tile(unsigned src, unsigned lane) const {
        return __builtin_amdgcn_raw_buffer_load_b128(x, (src << xShift) + 16 * (lane & 7),
                                                     int(sliceByte), 0);
    }
};

template <>
struct Loader<true> {
    const KernelArgs* a;
    const std::int8_t* xSlice;
    unsigned features;

    __device__ Loader(const KernelArgs& args, unsigned, unsigned f, unsigned slice)
        : a(&args), xSlice(args.packedX + slice * kSlice), features(f) {}
    __device__ Meta meta8(unsigned panel, unsigned lane) const {
        const std::size_t first = std::size_t(panel) * 8;
        const std::uint64_t md =
            __builtin_nontemporal_load(a->m.sourceMetadata + first + (lane & 7));
        return {__builtin_nontemporal_load(a->m.sourceIds + first + (lane & 7)), unsigned(md),
                unsigned(md >> 32),
                __builtin_nontemporal_load(a->m.sourceIds + first + (lane >> 3))};
    }
    __device__ float scale(unsigned src) const { return a->scales[min(src, a->cols - 1)]; }
    __device__ float value(unsigned idx) const { return __builtin_nontemporal_load(a->m.values + idx); }
    __device__ u32x4 tile(unsigned src, unsigned lane) const {
        return *reinterpret_cast<const u32x4*>(xSlice + std::size_t(min(src, a->cols - 1)) * features +
                                               16 * (lane & 7));
    }
};

template <unsigned G, class Ld>
__device__ __forceinline__ void loadStage2(const Ld& ld, const Meta& m, unsigned lane, Stage2& s) {
    // Padding slots (source UINT32_MAX, metadata 0) have an empty row mask, so `present` needs no
    // source check; their scale and X tile read 0 (narrow) or a clamped row (wide), both unused.
    s.scale = ld.scale(m.id);
    const unsigned row = G * 8 + ((lane >> 3) & 7);
    const bool present = (m.mask >> row) & 1u;
    // The k-th set row bit of a slot owns values[base + k]; absent rows read values[base] (a valid
    // index: padding has base 0 and a matrix with panels has values).
    const unsigned idx = present ? m.base + __popc(m.mask & ((1u << row) - 1u)) : m.base;
    s.v = ld.value(idx);
    s.bits = present;
    s.x = ld.tile(m.gather, lane);
}

// Dequantization into f16 MFMA operands. With the slot's scale written s = m * 2^e (m in [0.5, 1)),
// x_hat = tf32(fp32(q * s)) = tf32(fp32(q * m)) * 2^e exactly whenever s is normal, and
// x~ = tf32(fp32(q * m)) lies in [0.5, 127]: eleven significant bits in f16's normal range, so f16
// holds it exactly. The factor 2^e moves into the A operand: A' = tf32(a) * 2^(e + kShift), also
// an 11-bit value, exact in f16 when it lies in f16's normal range. The MFMA then sums exact
// products A' * x~ = 2^kShift * tf32(a) * x_hat in FP32, and the pass scales by 2^-kShift at the end.
// TF32 rounding (ties away from zero) of the f32 product is "add half an ulp of the 11-bit
// significand, then truncate": the truncation is the round-toward-zero f16 conversion.
constexpr int kShift = 10;
constexpr float kUnshift = 1.0f / 1024.0f;

// X bytes in LDS: lane L (tile t = L & 7 of slot s = L >> 3) writes the 8 byte pairs of its tile to
// rows p = 8t + i, column s, of a [64 pairs][8 slots] u16 array whose 8-row blocks are padded by
// 16 bytes (row p at byte 144 (p / 8) + 16 (p % 8)), so the 64 lanes of each pair-i write hit 32
// distinct banks. Lane l then reads row l — byte pair l of all 8 slots — with one 16-byte load:
// dword m holds slot 2m (low half) and slot 2m + 1 (high half).
constexpr unsigned kPairRowBlock = 144; // bytes per 8 rows of 16 bytes, plus padding

// Dword M of the pair row: x_lo / x_hi of slots 2M and 2M + 1 = fp32(float(byte) * factor of the
// slot), the factor of slot j coming from lane j of the lane's 16-lane row (DPP row broadcast).
// The four conversions ahead of the first DPP read cover the VALU-write -> DPP-read hazard.
template <unsigned M>
__device__ __forceinline__ void scaleDword(unsigned d, float factor, float (&q)[4]) {
    asm("v_cvt_f32_i32_sdwa %0, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f32_i32_sdwa %2, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f32_i32_sdwa %3, sext(%4) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "v_mul_f32_dpp %0, %5, %0 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %1, %5, %1 row_newbcast:%6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %2, %5, %2 row_newbcast:%7 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %3, %5, %3 row_newbcast:%7 row_mask:0xf bank_mask:0xf"
        : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
        : "v"(d), "v"(factor), "i"(2 * M), "i"(2 * M + 1));
}

// TF32-round two values and pack them as f16: adding 0x1000 to the FP32 pattern and converting
// toward zero keeps eleven significant bits, rounded half away from zero.
__device__ __forceinline__ f16x2 roundPack(float a, float b) {
    return __builtin_amdgcn_cvt_pkrtz(__uint_as_float(__float_as_uint(a) + 0x1000u),
                                      __uint_as_float(__float_as_uint(b) + 0x1000u));
}

// Slots 4T..4T+3 as one K = 4 step of v_mfma_f32_4x4x4_16b_f16: B = the lane's feature of the four
// slots (lo and hi byte of the pair), A = four slots of row 4h + (lane & 3) of the f16 table
// (rows0 / rows1: that row of quad 0 / 1, all 8 slots).
template <unsigned T>
__device__ __forceinline__ void accumulateStepF16(const u32x4& pairs, float mant,
                                                  const f16x8& rows0, const f16x8& rows1,
                                                  f32x4 (&acc)[2][2]) {
    float q0[4], q1[4];
    scaleDword<2 * T>(pairs[2 * T], mant, q0);     // slots 4T, 4T+1: lo, hi, lo, hi
    scaleDword<2 * T + 1>(pairs[2 * T + 1], mant, q1); // slots 4T+2, 4T+3
    const f16x2 l01 = roundPack(q0[0], q0[2]);
    const f16x2 h01 = roundPack(q0[1], q0[3]);
    const f16x2 l23 = roundPack(q1[0], q1[2]);
    const f16x2 h23 = roundPack(q1[1], q1[3]);
    const f16x4 bl = __builtin_bit_cast(f16x4, __builtin_shufflevector(l01, l23, 0, 1, 2, 3));
    const f16x4 bh = __builtin_bit_cast(f16x4, __builtin_shufflevector(h01, h23, 0, 1, 2, 3));
    const f16x4 a0 = __builtin_shufflevector(rows0, rows0, 4 * T, 4 * T + 1, 4 * T + 2, 4 * T + 3);
    const f16x4 a1 = __builtin_shufflevector(rows1, rows1, 4 * T, 4 * T + 1, 4 * T + 2, 4 * T + 3);
    acc[0][0] = __builtin_amdgcn_mfma_f32_4x4x4f16(a0, bl, acc[0][0], 0, 0, 0);
    acc[0][1] = __builtin_amdgcn_mfma_f32_4x4x4f16(a0, bh, acc[0][1], 0, 0, 0);
    acc[1][0] = __builtin_amdgcn_mfma_f32_4x4x4f16(a1, bl, acc[1][0], 0, 0, 0);
    acc[1][1] = __builtin_amdgcn_mfma_f32_4x4x4f16(a1, bh, acc[1][1], 0, 0, 0);
}

// Slots 2M, 2M+1 on the exact FP32 path: x = tf32(float(byte) * scale of the slot), A from the FP32
// table, one v_mfma_f32_4x4x1_16b_f32 per (slot, quad, feature).
template <unsigned M>
__device__ __forceinline__ void accumulateDwordF32(const u32x4& pairs, float scale,
                                                   const float* table, unsigned quadRow,
                                                   f32x4 (&acc)[2][2]) {
    float q[4];
    scaleDword<M>(pairs[M], scale, q);
#pragma unroll
    for (unsigned j = 0; j < 2; ++j) {
        const float lo = roundTf32(q[2 * j]), hi = roundTf32(q[2 * j + 1]);
        const float a0 = table[quadRow + 2 * M + j];      // rows 0..3 of the group (quad 0)
        const float a1 = table[quadRow + 32 + 2 * M + j]; // rows 4..7 (quad 1)
        acc[0][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a0, lo, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a0, hi, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a1, lo, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a1, hi, acc[1][1], 0, 0, 0);
    }
}

struct Lds {
    _Float16* table16;    // [8 rows][8 slots] A' values (f16 path)
    float* table32;       // [8 rows][8 slots] tf32(a) * 2^kShift (FP32 path)
    unsigned char* pairs; // X byte pairs, [64 pairs][8 slots] u16 with padded 8-row blocks
};

__device__ __forceinline__ void computeStage3(const Stage2& s, unsigned lane, const Lds& lds,
                                              f32x4 (&acc)[2][2]) {
    // Lane L: slot k = L & 7, row r = (L >> 3) & 7; table index r * 8 + k = L.
    const float at = s.bits ? roundTf32(s.v) : 0.0f;
    const int e = __builtin_amdgcn_frexp_expf(s.scale);
    const float mant = __builtin_amdgcn_frexp_mantf(s.scale);
    const float ap = __builtin_amdgcn_ldexpf(at, e + kShift);
    // f16 normal range [2^-14, 2^16): biased FP32 exponent 113..142. A subnormal scale (e < -125)
    // breaks the exponent split and takes the FP32 path too.
    const bool exact = at == 0.0f || (((__float_as_uint(ap) >> 23) & 0xFFu) - 113u <= 29u &&
                                      e > -126);
    {
        unsigned short* w = reinterpret_cast<unsigned short*>(
            lds.pairs + kPairRowBlock * (lane & 7) + 2 * (lane >> 3));
#pragma unroll
        for (unsigned i = 0; i < 8; ++i)
            w[8 * i] = static_cast<unsigned short>(s.x[i / 2] >> (16 * (i & 1)));
    }
    if (__builtin_amdgcn_ballot_w64(!exact) == 0) {
        lds.table16[lane] = static_cast<_Float16>(ap);
        __syncthreads();
        const u32x4 pairs = *reinterpret_cast<const u32x4*>(
            lds.pairs + kPairRowBlock * (lane >> 3) + 16 * (lane & 7));
        // A operands: row (lane & 3) of quad 0 and of quad 1, all 8 slots (16 bytes each).
        const f16x8* table = reinterpret_cast<const f16x8*>(lds.table16);
        const f16x8 rows0 = table[lane & 3], rows1 = table[4 + (lane & 3)];
        accumulateStepF16<0>(pairs, mant, rows0, rows1, acc);
        accumulateStepF16<1>(pairs, mant, rows0, rows1, acc);
    } else {
        // Some A' leaves f16's normal range (or a scale is subnormal): exact FP32 operands.
        lds.table32[lane] = __builtin_amdgcn_ldexpf(at, kShift);
        __syncthreads();
        const u32x4 pairs = *reinterpret_cast<const u32x4*>(
            lds.pairs + kPairRowBlock * (lane >> 3) + 16 * (lane & 7));
        const unsigned quadRow = (lane & 3) * 8; // lane 4b+i reads row 4h+i of quad h
        accumulateDwordF32<0>(pairs, s.scale, lds.table32, quadRow, acc);
        accumulateDwordF32<1>(pairs, s.scale, lds.table32, quadRow, acc);
        accumulateDwordF32<2>(pairs, s.scale, lds.table32, quadRow, acc);
        accumulateDwordF32<3>(pairs, s.scale, lds.table32, quadRow, acc);
    }
    __syncthreads();
}

// One pass over the panels of row group G. Unrolled by two so the stage-2 buffers alternate
// instead of being copied; panel indices past the end repeat the last panel (harmless loads).
template <unsigned G, class Ld>
__device__ __forceinline__ void rowGroupPass(const Ld& ld, const Bounds& bounds, unsigned lane,
                                             const Lds& lds, f32x4 (&acc)[2][2]) {
    // The panel count is uniform; keep the loop counter scalar.
    const unsigned n = __builtin_amdgcn_readfirstlane(panelCount<G>(bounds));
    if (!n) return;
    unsigned p0 = nextPanel<G>(bounds, 0);
    unsigned p1 = nextPanel<G>(bounds, p0 + 1);
    p1 = p1 == kEnd ? p0 : p1;
    unsigned p2 = nextPanel<G>(bounds, p1 + 1);
    p2 = p2 == kEnd ? p1 : p2;
    Stage2 sa, sb;
    loadStage2<G>(ld, ld.meta8(p0, lane), lane, sa);
    Meta m1 = ld.meta8(p1, lane);
    Meta m2 = ld.meta8(p2, lane);
#pragma unroll 1
    for (unsigned i = 0; i < n; i += 2) {
        // Iteration i: stage 2 of panel i+1 (metadata m1), stage 1 of panel i+3, compute panel i.
        loadStage2<G>(ld, m1, lane, sb);
        {
            unsigned p3 = nextPanel<G>(bounds, p2 + 1);
            p3 = p3 == kEnd ? p2 : p3;
            m1 = m2;
            m2 = ld.meta8(p3, lane);
            p2 = p3;
        }
        computeStage3(sa, lane, lds, acc);
        if (i + 1 >= n) break;
        loadStage2<G>(ld, m1, lane, sa);
        {
            unsigned p3 = nextPanel<G>(bounds, p2 + 1);
            p3 = p3 == kEnd ? p2 : p3;
            m1 = m2;
            m2 = ld.meta8(p3, lane);
            p2 = p3;
        }
        computeStage3(sb, lane, lds, acc);
    }
}

// Store the 8 rows of a pass: lane l holds features col and col + 8 (byte pair l) of rows
// 4h + i (acc[h][0 / 1][i]).
__device__ __forceinline__ void storeRows(const f32x4 (&acc)[2][2], float* base,
                                          unsigned rowStride, unsigned validRows, unsigned col,
                                          bool nontemporal) {
#pragma unroll
    for (unsigned h = 0; h < 2; ++h)
#pragma unroll
        for (unsigned i = 0; i < 4; ++i) {
            const unsigned row = h * 4 + i;
            if (row >= validRows) continue;
            float* r = base + std::size_t(row) * rowStride + col;
            if (nontemporal) {
                __builtin_nontemporal_store(acc[h][0][i], r);
                __builtin_nontemporal_store(acc[h][1][i], r + 8);
            } else {
                r[0] = acc[h][0][i];
                r[8] = acc[h][1][i];
            }
        }
}

template <unsigned G, unsigned Features, class Ld>
__device__ __forceinline__ void runGroup(const KernelArgs& a, const Ld& ld, const Sw32Task& task,
                                         const Bounds& bounds, unsigned lane, const Lds& lds,
                                         unsigned col) {
    const bool split = task.partial != kNoPartial;
    if (split && !((task.mask >> G) & 1u)) return;
    f32x4 acc[2][2];
#pragma unroll
    for (unsigned h = 0; h < 2; ++h) acc[h][0] = acc[h][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    rowGroupPass<G>(ld, bounds, lane, lds, acc);
#pragma unroll
    for (unsigned h = 0; h < 2; ++h) {
        acc[h][0] *= kUnshift; // exact power-of-two scaling back to Y
        acc[h][1] *= kUnshift;
    }
    if (!split) {
        const unsigned row0 = task.sw * 32 + G * 8;
        if (row0 < a.rows)
            storeRows(acc, a.y + std::size_t(row0) * Features, Features, min(8u, a.rows - row0),
                      col, true);
    } else {
        const std::size_t tile = task.partial + __popc(task.mask & ((1u << G) - 1u));
        storeRows(acc, a.partials + tile * 8 * Features, Features, 8, col, false);
    }
}

// Workgroup -> task: each of the 8 XCDs (workgroups are dispatched round-robin by id) walks one
// contiguous range of tasks, so neighbouring SWs share source rows of X in that XCD's L2.
__device__ __forceinline__ unsigned xcdTask(unsigned bid, unsigned tasks) {
    const unsigned xcd = bid & 7u, j = bid >> 3;
    const unsigned q = tasks >> 3, r = tasks & 7u;
    return xcd * q + min(xcd, r) + j;
}

template <unsigned Features, bool Wide>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(4))) void spmmInt8Kernel(
    KernelArgs a) {
    __shared__ __align__(16) _Float16 table16[64];
    __shared__ __align__(16) float table32[64];
    __shared__ __align__(16) unsigned char pairs[8 * kPairRowBlock];
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
    const Loader<Wide> ld(a, task.begin, Features, slice);
    // Byte pair `lane` of the slice: features 16 * (lane / 8) + lane % 8 and + 8.
    const unsigned col = slice * kSlice + 16 * (lane >> 3) + (lane & 7);

    const Lds lds{table16, table32, pairs};
    runGroup<0, Features>(a, ld, task, bounds, lane, lds, col);
    runGroup<1, Features>(a, ld, task, bounds, lane, lds, col);
    runGroup<2, Features>(a, ld, task, bounds, lane, lds, col);
    runGroup<3, Features>(a, ld, task, bounds, lane, lds, col);
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
    // Buffer addressing needs the packed X and the scales within 32-bit byte offsets, with room for
    // the padding sentinel to land out of range.
    // TCC_SPMM_FORCE_WIDE selects the 64-bit instance for any size (used by the tests).
    const bool wide = std::uint64_t(args.cols) * Features > 0xFFFFFF00ull ||
                      std::getenv("TCC_SPMM_FORCE_WIDE") != nullptr;
    if (wide)
        hipLaunchKernelGGL((spmmInt8Kernel<Features, true>), grid, dim3(kWave), 0, stream, args);
    else
        hipLaunchKernelGGL((spmmInt8Kernel<Features, false>), grid, dim3(kWave), 0, stream, args);
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
    // 16-byte X tiles: the packed rows must start 16-byte aligned.
    if (reinterpret_cast<std::uintptr_t>(packedX) % 16)
        throw std::invalid_argument("launchSpmmInt8: packedX must be 16-byte aligned");
    const KernelArgs args{matrix, packedX, scales, output, workspace.partials, workspace.counters,
                          rows,   cols};
    if (features == 128)
        launch<128>(args, stream);
    else
        launch<256>(args, stream);
    checkHip(hipGetLastError());
}
