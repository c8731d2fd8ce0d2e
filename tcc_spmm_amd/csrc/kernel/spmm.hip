// Fused INT8-dequantization SpMM for MI355X (gfx950, wave64): Y = A x tf32(dequant(X)).
//
// Work decomposition
//   One workgroup per task (one Sw32Task: <= 384 panels of one 32-row SW), normally one wavefront;
//   each XCD walks a contiguous range of the task list (xcdTask), balanced by panels when skewed,
//   the range's last 512 tasks longest size class first (tailTask).
//   The wave walks the task's panels once, in order, and accumulates all 32 rows x F features of
//   the SW: four v_mfma_f32_32x32x8_f16 per panel and 128-feature slice (one per 32-feature block;
//   M = features, N = the 32 rows, K = the panel's 8 slots) into 4 x 16 FP32 accumulators per
//   slice. F256 runs both slices in the same wave, so the A side of a panel is loaded and built
//   once, and takes its panels in pairs: four v_mfma_f32_32x32x16_f16 per pair and slice, K = the
//   pair's 16 slots. Plans with few tasks for the chip take two waves per task instead, each walking half the
//   panels, with the second wave's accumulators added by the first (runTask).
//
// Operands of one panel
//   A (features x slots): the 8 slot rows of the X slice are gathered with one dwordx4 load per
//   lane (lane L: 16-byte tile L & 7 of slot L >> 3) and stored to LDS as [slot][128 bytes].
//   Lane l then reads dword l & 31 of slots 4h..4h+3 (h = l >> 5): byte b of that dword is block
//   b's feature for M index l & 31, so each lane dequantizes 16 bytes (4 slots x 4 blocks), with
//   the four slots' scale mantissas read from LDS as one 16-byte broadcast.
//   B (slots x rows): an LDS table [32 rows][8 slots] of f16 A values; lane l reads row l & 31,
//   slots 4h..4h+3. Rows of row groups the panel's bucket does not touch hold 0.
//   D: lane l holds row l & 31 and, per block, M indices 8i + 4h + j (register 4i + j).
//   F256 pairs: both panels' X rows, mantissas and tables sit in two LDS areas, and each operand
//   takes its four values from the first panel and then four from the second (K = 16).
//
// Exact TF32 products in f16. With the slot's scale written s = m * 2^e (m in [0.5, 1)),
// x_hat = tf32(fp32(q * s)) = tf32(fp32(q * m)) * 2^e exactly whenever s is normal, and
// x~ = tf32(fp32(q * m)) lies in [0.5, 127]: eleven significant bits. The factor 2^e moves into B:
// a' = tf32(a) * 2^(e + kShift), also eleven bits, exact in f16 when in f16's normal range (kShift
// keeps the usual A values there). A takes x~ * 2^-kXShift (kXShift = kShift + 1), which stays in
// [2^-12, 2^-4): still eleven bits in f16's normal range. The MFMA thus sums exact products
// a' * x~ * 2^-kXShift = tf32(a) * x_hat / 2 in FP32, so any accumulation order reproduces the
// reference's products, and the task doubles its accumulators at the end (exact). The accumulators
// hold Y / 2, never a scaled-up Y, so no sum overflows where the reference's stays finite. TF32
// rounding (ties away from zero) is "add 0x1000 to the FP32 pattern, truncate", and the truncation is
// the round-toward-zero f16 conversion. A panel whose a' leaves f16's normal range (or whose scale
// is subnormal) takes an FP32 path with the same products: v_mfma_f32_32x32x2_f32 on tf32(a) / 2 and
// the TF32 features. (Halving a value below 2^-125 rounds it, an error far below the tolerance.)
//
// The panels are walked by a software pipeline (F128: metadata two panels ahead, in pairs of panels,
// A values and X one panel ahead; F256: metadata four panels ahead, A values and X two) whose memory
// operations are identical on every path. F128
// runs four waves per SIMD (128 registers each, accumulators included), F256 two (248 registers).
//
// Split SWs (reference src/kernel/spmm_kernel.cuh:228-282): a split task stores its row groups of
// `task.mask` as 8-row partial tiles [tile][8][F]; lane 0 then takes, per slice, an agent-scope
// acq_rel wrapping ticket on counters[sw * (F/128) + slice] with limit chunks - 1, so the counter
// returns to zero by itself; the task whose ticket is chunks - 1 merges all partial tiles of the SW's
// slice in partialIds order starting from 0.0f and writes Y. No float atomics, no spin-waits.
#include "spmm.h"
#include "hip_support.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

// A 4-byte load from a structured buffer (address = base + index x stride + offsets, range-checked
// by index): the LLVM intrinsic behind the raw-buffer builtins, declared by its name since clang
// has no builtin for the structured form.
__device__ float structLoadF32(__amdgpu_buffer_rsrc_t rsrc, int index, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.f32");

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __fp16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr unsigned kWave = 64;
constexpr unsigned kSlice = 128;
constexpr unsigned kNoPartial = 0xFFFFFFFFu;
constexpr int kShift = 10;
constexpr int kXShift = kShift + 1;
// Buffer cache policy of the A stream (sourceIds, sourceMetadata, values): the default. The
// nontemporal hint (2) was measured to raise L2 misses of the gathered X rows by about 1.5 GB per
// c3 F128 launch.
constexpr int kNt = 0;

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
    unsigned vec4; // y and partials are 16-byte aligned: stores and merge loads of 16 bytes
#ifdef TCC_SPMM_TIMELINE
    unsigned long long* stamps; // measurement build only: [taskCount][4], see TaskClock
#endif
};

// sw32BucketOrder (include/format/sw32.h) packed four bits per bucket slot: slot t's row-group mask
// is nibble t of this constant.
constexpr std::uint64_t kBucketGroups = 0xFEDCBA9765384210ull;

// ------------------------------------------------------------------------------------------------
// Memory access of one task. Narrow (the packed X slice and the scales addressable with 32-bit
// byte offsets, the usual case): buffer loads. sourceIds, sourceMetadata and values use a per-task
// base (offsets stay below 1 MiB); scales and X use buffers sized from `cols`, so the padding
// sentinel source UINT32_MAX lands out of range and reads 0 without a clamp, and an absent A entry
// reads 0 through an out-of-range offset. Wide: 64-bit global loads with clamped indices.
// Wide with 2-byte tiles: the same, for a packed X that is u16- but not 16-byte aligned (the
// reference's own requirement, include/format/int8_features.cuh:11-13): each 16-byte tile is read
// as eight naturally aligned u16 loads, which never touch a byte outside the tile.

struct Meta {        // one panel
    unsigned id;     // lane L: source of slot L & 7
    unsigned mask;   // lane L: row mask of slot L & 7
    unsigned base;   // lane L: value base of slot L & 7
};

// Lane L's value of v from lane srcLane (LDS crossbar, no memory access).
__device__ __forceinline__ unsigned lanePermute(unsigned v, unsigned srcLane) {
    return unsigned(__builtin_amdgcn_ds_bpermute(int(srcLane * 4), int(v)));
}

// Metadata of panels q and q + 1 loaded together (F128 walk): lane L holds slot L & 7 of panel
// q + ((L >> 3) & 1), lanes 16..63 repeating lanes 0..15.
struct MetaPair {
    unsigned id, mask, base;
};

// Panel q + E (E = 0, 1) of a pair, in the per-panel lane layout: within each 16-lane DPP row the
// half holding the other panel takes the wanted half's values (row_shr:8 into lanes 8..15 for
// E = 0, row_shl:8 into lanes 0..7 for E = 1), one VALU move per field and no LDS round trip.
template <unsigned E>
__device__ __forceinline__ unsigned pairHalf(unsigned v) {
    return E == 0 ? unsigned(__builtin_amdgcn_update_dpp(int(v), int(v), 0x118, 0xF, 0xC, false))
                  : unsigned(__builtin_amdgcn_update_dpp(int(v), int(v), 0x108, 0xF, 0x3, false));
}
template <unsigned E>
__device__ __forceinline__ Meta pairPanel(const MetaPair& m) {
    return {pairHalf<E>(m.id), pairHalf<E>(m.mask), pairHalf<E>(m.base)};
}

// Addressing modes of the X and A-stream loads, chosen per launch on the host.
enum : unsigned { kBuffer = 0, kGlobal = 1, kGlobalU16 = 2 };

template <unsigned Addr>
struct Loader;

template <>
struct Loader<kBuffer> {
    static constexpr bool kWide = false;
    __amdgpu_buffer_rsrc_t ids, meta, scales, x, vals;
    unsigned first;     // task.begin: panel offsets are relative to it
    unsigned vbase;     // value base of the task's first slot, the smallest of the task
    unsigned xShift;    // log2(features)

    __device__ Loader(const KernelArgs& a, unsigned begin, unsigned end, unsigned features)
        : first(begin), xShift(features == 256 ? 8u : 7u) {
        const std::size_t slot0 = std::size_t(begin) * 8;
        // Value bases grow in slot order (reference src/format/sw32.cpp:131-138) and every panel
        // starts with a real slot, so the first slot of the task has the smallest base.
        vbase = begin < end ? unsigned(a.m.sourceMetadata[slot0] >> 32) : 0u;
        ids = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned*>(a.m.sourceIds + slot0), 0,
                                                0x7FFFFFF0, 0x00020000);
        meta = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<std::uint64_t*>(a.m.sourceMetadata + slot0), 0, 0x7FFFFFF0, 0x00020000);
        vals = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.m.values + vbase), 4,
                                                 0x7FFFFFF0, 0x00020000);
        scales = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.scales), 4, a.cols, 0x00020000);
        x = __builtin_amdgcn_make_buffer_rsrc(const_cast<std::int8_t*>(a.packedX), 0,
                                              a.cols << xShift, 0x00020000);
    }
    __device__ Meta meta8(unsigned panel, unsigned lane) const {
        const int off = int((panel - first) * 32u);
        const auto md = __builtin_amdgcn_raw_buffer_load_b64(meta, (lane & 7) * 8, 2 * off, kNt);
        return {__builtin_amdgcn_raw_buffer_load_b32(ids, (lane & 7) * 4, off, kNt), md[0], md[1]};
    }
    // Panels q and q + 1, each clamped to `last`: one load per array for both.
    __device__ MetaPair meta2(unsigned q, unsigned last, unsigned lane) const {
        const unsigned off = (min(q + ((lane >> 3) & 1u), last) - first) * 32u + (lane & 7) * 4;
        const auto md = __builtin_amdgcn_raw_buffer_load_b64(meta, 2 * off, 0, kNt);
        return {__builtin_amdgcn_raw_buffer_load_b32(ids, off, 0, kNt), md[0], md[1]};
    }
    // scales and values are structured buffers of 4-byte records, addressed by index (no shift) and
    // range-checked by index: an index past the records reads 0.
    __device__ float scale(unsigned src) const { return structLoadF32(scales, int(src), 0, 0, 0); }
    // values[idx] when `present`, else 0.
    __device__ float value(unsigned idx, bool present) const {
        return structLoadF32(vals, int(present ? idx - vbase : 0xFFFFFFFFu), 0, 0, kNt);
    }
    // 16-byte tile `lane & 7` of slice k of the packed X row of `src`. The slice offset goes in the
    // scalar offset, so both slices of a row share one per-lane offset (one VALU instruction fewer
    // per F256 panel).
    __device__ u32x4 tile(unsigned src, unsigned lane, unsigned k) const {
        return __builtin_amdgcn_raw_buffer_load_b128(x, (src << xShift) + 16 * (lane & 7), kSlice * k, 0);
    }
};

template <unsigned Addr>
struct Loader {
    static_assert(Addr == kGlobal || Addr == kGlobalU16, "64-bit addressing modes");
    static constexpr bool kWide = true;
    const KernelArgs* a;
    unsigned features;

    __device__ Loader(const KernelArgs& args, unsigned, unsigned, unsigned f)
        : a(&args), features(f) {}
    __device__ Meta meta8(unsigned panel, unsigned lane) const {
        const std::size_t first = std::size_t(panel) * 8;
        const std::uint64_t md =
            __builtin_nontemporal_load(a->m.sourceMetadata + first + (lane & 7));
        return {__builtin_nontemporal_load(a->m.sourceIds + first + (lane & 7)), unsigned(md),
                unsigned(md >> 32)};
    }
    __device__ MetaPair meta2(unsigned q, unsigned last, unsigned lane) const {
        const std::size_t s = std::size_t(min(q + ((lane >> 3) & 1u), last)) * 8 + (lane & 7);
        const std::uint64_t md = __builtin_nontemporal_load(a->m.sourceMetadata + s);
        return {__builtin_nontemporal_load(a->m.sourceIds + s), unsigned(md), unsigned(md >> 32)};
    }
    __device__ float scale(unsigned src) const { return a->scales[min(src, a->cols - 1)]; }
    // values[idx] (absent entries are masked by Stage::bits).
    __device__ float value(unsigned idx, bool) const {
        return __builtin_nontemporal_load(a->m.values + idx);
    }
    __device__ u32x4 tile(unsigned src, unsigned lane, unsigned k) const {
        const std::int8_t* p =
            a->packedX + std::size_t(min(src, a->cols - 1)) * features + 16 * (lane & 7) + kSlice * k;
        if constexpr (Addr == kGlobalU16) {
            const unsigned short* h = reinterpret_cast<const unsigned short*>(p);
            u32x4 t;
#pragma unroll
            for (unsigned i = 0; i < 4; ++i) t[i] = unsigned(h[2 * i]) | (unsigned(h[2 * i + 1]) << 16);
            return t;
        } else {
            return *reinterpret_cast<const u32x4*>(p);
        }
    }
};

// Panel kinds: G = 0..3, a bucket exclusive to row group G (known at compile time); kShared, a
// shared bucket whose row groups `groups` are known at run time.
constexpr unsigned kShared = 4;

struct Stage {     // one panel, ready to compute
    float scale;   // lane L: scale of slot L & 7
    float v[4];    // lane L: raw A value of (slot L & 7, row 8g + (L >> 3)); v[0] for kind G < 4
    unsigned bits; // bit g: that entry is present (wide loader only; narrow reads 0 instead)
    u32x4 x[2];    // 16-byte tile L & 7 of the X row of slot L >> 3, per slice of the wave
};

// Stage 2 of one panel of kind G (row groups `groups` when G == kShared), with the X tiles of the
// wave's S slices; the scale too unless the caller loads it (LoadScale false).
template <unsigned G, unsigned S, class Ld, bool LoadScale = true>
__device__ __forceinline__ void loadStage(const Ld& ld, const Meta& m, unsigned groups,
                                          unsigned lane, Stage& s) {
    // Padding slots (source UINT32_MAX, metadata 0) have an empty row mask; their scale and X tile
    // read 0 (narrow) or a clamped row (wide), multiplied by A entries that are all 0.
    if constexpr (LoadScale) s.scale = ld.scale(m.id);
    s.bits = 0;
    constexpr unsigned kCount = G < 4 ? 1 : 4;
#pragma unroll
    for (unsigned j = 0; j < kCount; ++j) {
        const unsigned g = G < 4 ? G : j;
        const unsigned row = g * 8 + (lane >> 3);
        const bool present = ((m.mask >> row) & 1u) && (G < 4 || ((groups >> g) & 1u));
        // The k-th set row bit of a slot owns values[base + k].
        const unsigned idx = m.base + __popc(m.mask & ((1u << row) - 1u));
        if constexpr (Ld::kWide) {
            s.v[j] = ld.value(present ? idx : m.base, true);
            s.bits |= unsigned(present) << j;
        } else {
            s.v[j] = ld.value(idx, present);
        }
    }
    // Lane L gathers slot L >> 3's row, whose source lane L >> 3 holds: a cross-lane permute instead
    // of a second sourceIds load (one vector memory instruction fewer per panel, 2% at c3 F128).
    const unsigned gather = lanePermute(m.id, lane >> 3);
#pragma unroll
    for (unsigned k = 0; k < S; ++k) s.x[k] = ld.tile(gather, lane, k);
}

// ------------------------------------------------------------------------------------------------
// Compute

// Block B of the lane's four slots: byte B of d0..d3 (slots 4h + 0..3) sign-extended to FP32 by
// SDWA conversions, then multiplied by the slots' scale mantissas (plain multiplies: a DPP operand
// would cost about twice the issue time of each multiply).
template <unsigned B>
__device__ __forceinline__ void scaleBlock(unsigned d0, unsigned d1, unsigned d2, unsigned d3,
                                           const f32x4& mant, float (&q)[4]) {
    const unsigned d[4] = {d0, d1, d2, d3};
#pragma unroll
    for (unsigned i = 0; i < 4; ++i)
        q[i] = float(static_cast<signed char>(d[i] >> (8 * B))) * mant[i];
}

// TF32-round two values and pack them as f16 (round toward zero after adding half an ulp). Both
// half-ulp additions are one 64-bit add on the pair's patterns: no carry crosses from the low value
// into the high one, since a finite FP32 pattern plus 0x1000 stays below 2^32 (only patterns at or
// above 0xFFFFF000, negative NaNs, would carry). One v_lshl_add_u64 instead of two v_add_u32.
__device__ __forceinline__ f16x2 roundPack(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const unsigned long long both =
        __builtin_bit_cast(unsigned long long, f32x2{a, b}) + 0x0000100000001000ull;
    const f32x2 r = __builtin_bit_cast(f32x2, both);
    return __builtin_amdgcn_cvt_pkrtz(r[0], r[1]);
}

// LDS handoff between the lanes of the workgroup's single wave: the wave's LDS operations execute
// in order, so only the compiler has to be kept from moving memory accesses across this point.
__device__ __forceinline__ void waveSync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct Lds {
    _Float16* table16; // a' (f16 path): F128 [32 rows][8 slots], F256 two areas (tableEntry)
    float* table32;    // [32 rows][8 slots] tf32(a) / 2 (FP32 path)
    u32x4* xtile;      // [8 slots][blocks][128 bytes] X rows: block S * area + slice (xTile)
    float* mant;       // [2 areas][8 slots] scale mantissas of a panel
    unsigned short* redo; // [384]: offsets (from the task's first panel) of the panels that need
                          // the FP32 path, in the order found (a task has <= 384 panels)
};

// Entry j of a stage as tf32(a) (0 when absent).
template <bool Wide>
__device__ __forceinline__ float stageTf32(const Stage& s, unsigned j) {
    return (Wide && !((s.bits >> j) & 1u)) ? 0.0f : roundTf32(s.v[j]); // tf32(0) = 0
}

// Per lane: slot k = lane & 7, row (lane >> 3) of each row group; its table index in row group g
// is (8g + (lane >> 3)) * 8 + k = 64g + lane. Kind G < 4 writes only row group G (the others hold
// 0 for the whole bucket). Returns whether every entry of the panel has an exact f16 a'
// (wave-uniform); if not, the panel contributes nothing here.
// m * 2^-kXShift for a scale s = m * 2^e (m in [0.5, 1)): the sign and mantissa bits of s under the
// biased exponent 126 - kXShift. One v_and_or_b32 (as cheap as a v_frexp_mant); a VOP3 takes no
// literal and one scalar operand on gfx950, so the caller keeps the mask 0x807FFFFF in a VGPR
// (`keep`) and the exponent bits come from an SGPR.
__device__ __forceinline__ float shiftedMantissa(float s, unsigned keep) {
    unsigned r;
    asm("v_and_or_b32 %0, %1, %2, %3"
        : "=v"(r)
        : "v"(__float_as_uint(s)), "v"(keep), "s"(unsigned(126 - kXShift) << 23));
    return __uint_as_float(r);
}

// The lane's row and half of the MFMA operands, m = lane & 31 and h = lane >> 5, computed once per
// task (opaquely, so that the register allocator keeps them rather than recomputing them per panel).
struct LaneMh {
    unsigned m, h;
};

// Lanes whose value is a normal f16 (class bits 3 and 8: -normal, +normal), as a wave mask. The
// comparison writes the mask straight into an SGPR pair; through the class builtin the compiler
// moved the result through a VGPR and compared it again.
__device__ __forceinline__ std::uint64_t normalF16(_Float16 v) {
    std::uint64_t mask;
    asm("v_cmp_class_f16_e64 %0, %1, %2" : "=s"(mask) : "v"(v), "v"(0x108u));
    return mask;
}

__device__ __forceinline__ f16x8 join(f16x4 lo, f16x4 hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// A panel is computed in two parts. stagePanel writes its operands to LDS area 0 or 1: the f16 A
// table, the X tiles and the scale mantissas. crunch reads them back, dequantizes the X blocks and
// runs the MFMAs, over area 0 alone (one v_mfma_f32_32x32x8_f16 per 32-feature block) or over both
// areas (one v_mfma_f32_32x32x16_f16 per block, K = the 16 slots of two panels: lane half h holds
// k = 8h + j, j < 4 area 0's slot 4h + j and j >= 4 area 1's slot 4h + j - 4, in both operands, so
// each MFMA adds both panels' products). F256 computes its panels in pairs: half the MFMAs, and
// half the matrix-core time, of one MFMA per panel and block.
//
// Table layout: F128 (one area) [32 rows][8 slots]; F256 [32 rows][2 halves][2 areas][4 slots], so
// that the entries of row m and slots 4h .. 4h + 3 are 8 contiguous bytes per area and 16 for both.
// Either way they start at f16 index 4 (2m + h) * kAreas of area 0. Lane L writes slot L & 7 of row
// 8g + (L >> 3) of row group g: F128 index 64g + L.
template <unsigned S>
__device__ __forceinline__ unsigned tableEntry(unsigned g, unsigned lane, unsigned area) {
    if constexpr (S == 1) {
        return 64 * g + lane;
    } else {
        const unsigned row = 8 * g + (lane >> 3), slot = lane & 7;
        return ((row * 2 + (slot >> 2)) * 2 + area) * 4 + (slot & 3);
    }
}

// X tiles in LDS: [8 slots][blocks][128 bytes], block S * area + slice (F128: one block; F256: four,
// two areas of two slices). Returns the 16-byte index of the first tile of (slot, block). A lane
// reads dword m of slots 4h .. 4h + 3 of every block: at F256 its 16 reads of a pair lie within 2 KB
// of its first one, so two base addresses 1 KB apart reach them all through the 8-bit dword offsets
// of two-address LDS reads (with one block per 1 KB, as [block][slot], it took four).
template <unsigned S>
__device__ __forceinline__ unsigned xTile(unsigned slot, unsigned block) {
    constexpr unsigned kBlocks = S == 1 ? 1 : 2 * S;
    return (slot * kBlocks + block) * 8;
}

// Writes panel `s` of kind G to LDS area `area`. Per lane: slot lane & 7, row lane >> 3 of each
// row group; kind G < 4 writes only row group G (the others hold 0 for the whole bucket). Returns
// whether every entry of the panel has an exact f16 a' (wave-uniform); if not, its table is all
// zero, so the panel contributes nothing here.
template <bool Wide, unsigned G, unsigned S>
__device__ __forceinline__ bool stagePanel(const Stage& s, unsigned lane, const Lds& lds, unsigned area,
                                           unsigned keep) {
    // 2^(e + kShift) for the slot's scale s = m * 2^e (m in [0.5, 1)): its exponent bits alone are
    // 2^(e - 1). A zero or subnormal scale gives 0 and an infinite or NaN one inf, so that every
    // nonzero entry of such a slot fails the check below and the panel takes the FP32 path (the
    // mantissa trick needs a normal scale; there q x inf is inf or NaN, as in the reference).
    const float pow2 = __builtin_amdgcn_ldexpf(__uint_as_float(__float_as_uint(s.scale) & 0x7F800000u),
                                               kShift + 1);
    std::uint64_t inexact = 0; // lanes with an entry that has no exact f16 a'
    constexpr unsigned kCount = G < 4 ? 1 : 4;
    _Float16 ap[kCount];
#pragma unroll
    for (unsigned j = 0; j < kCount; ++j) {
        const float at = stageTf32<Wide>(s, j);
        // a' = at x pow2 has at most eleven significant bits, so it is exact in f16 exactly when
        // its conversion is a normal f16: [2^-14, 65504]; larger values (inf included) convert to
        // inf, smaller ones to subnormals or zero. (A product that lands in that range is a normal
        // FP32 value, so the multiply itself was exact.) Masks of comparisons combine as scalar
        // operations.
        ap[j] = static_cast<_Float16>(at * pow2);
        const std::uint64_t nonzero = __builtin_amdgcn_ballot_w64(at != 0.0f);
        inexact |= nonzero & ~normalF16(ap[j]);
    }
    // A panel without exact f16 operands still runs its MFMAs (straight-line accumulators), on an
    // all-zero table; the FP32 pass adds it later.
    const bool useF16 = inexact == 0;
#pragma unroll
    for (unsigned j = 0; j < kCount; ++j)
        lds.table16[tableEntry<S>(G < 4 ? G : j, lane, area)] =
            useF16 ? ap[j] : static_cast<_Float16>(0.0f);
#pragma unroll
    for (unsigned k = 0; k < S; ++k) lds.xtile[xTile<S>(lane >> 3, S * area + k) + (lane & 7)] = s.x[k];
    // Lane L holds slot L & 7's scale; lanes of half h read the mantissas of slots 4h .. 4h + 3,
    // stored as m * 2^-kXShift. For a scale that is not normal the bits are not that, but such a
    // panel's table is all zero (pow2 above) and the FP32 pass computes it.
    lds.mant[8 * area + (lane & 7)] = shiftedMantissa(s.scale, keep);
    return useF16;
}

// Dequantized block B (bytes B of the lane's four X dwords) of one area, as f16 x~ * 2^-kXShift.
template <unsigned B>
__device__ __forceinline__ f16x4 dequantBlock(const unsigned (&d)[4], const f32x4& mant) {
    float q[4];
    scaleBlock<B>(d[0], d[1], d[2], d[3], mant, q);
    return __builtin_bit_cast(
        f16x4, __builtin_shufflevector(roundPack(q[0], q[1]), roundPack(q[2], q[3]), 0, 1, 2, 3));
}

// The MFMAs of area 0 (Pair false) or of areas 0 and 1 (Pair true). The S x 4 blocks are
// dequantized one ahead of their MFMAs: block i + 1's conversions run between block i's last pack
// and its MFMA, so the MFMA's operand was written a dozen VALU instructions before it is read and
// needs no wait states.
template <unsigned S, bool Pair>
__device__ __forceinline__ void crunch(const Lds& lds, f32x16 (&acc)[4 * S], LaneMh mh) {
    constexpr unsigned kAreas = Pair ? 2 : 1;
    waveSync();
    const unsigned m = mh.m, h = mh.h;
    f32x4 mant[kAreas];
    unsigned d[kAreas][S][4];
#pragma unroll
    for (unsigned r = 0; r < kAreas; ++r) {
        mant[r] = reinterpret_cast<const f32x4*>(lds.mant + 8 * r)[h];
#pragma unroll
        for (unsigned k = 0; k < S; ++k) {
            const unsigned* xw = reinterpret_cast<const unsigned*>(lds.xtile) + m;
#pragma unroll
            for (unsigned i = 0; i < 4; ++i) d[r][k][i] = xw[4 * xTile<S>(4 * h + i, S * r + k)];
        }
    }
    using I0 = std::integral_constant<unsigned, 0>;
    using I1 = std::integral_constant<unsigned, 1>;
    using I2 = std::integral_constant<unsigned, 2>;
    using I3 = std::integral_constant<unsigned, 3>;
    if constexpr (Pair) {
        const f16x8 b = reinterpret_cast<const f16x8*>(lds.table16)[m * 2 + h];
        auto op = [&](auto blk, unsigned k) {
            constexpr unsigned B = decltype(blk)::value;
            return join(dequantBlock<B>(d[0][k], mant[0]), dequantBlock<B>(d[1][k], mant[1]));
        };
        auto mfma = [&](unsigned t, f16x8 x) {
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x, b, acc[t], 0, 0, 0);
        };
        f16x8 av = op(I0{}, 0);
#pragma unroll
        for (unsigned k = 0; k < S; ++k) {
            f16x8 nx = op(I1{}, k);
            mfma(4 * k + 0, av);
            av = op(I2{}, k);
            mfma(4 * k + 1, nx);
            nx = op(I3{}, k);
            mfma(4 * k + 2, av);
            if (k + 1 < S) av = op(I0{}, k + 1);
            mfma(4 * k + 3, nx);
        }
    } else {
        const f16x4 b = reinterpret_cast<const f16x4*>(lds.table16)[(m * 2 + h) * (S == 1 ? 1 : 2)];
        auto op = [&](auto blk, unsigned k) {
            constexpr unsigned B = decltype(blk)::value;
            return dequantBlock<B>(d[0][k], mant[0]);
        };
        auto mfma = [&](unsigned t, f16x4 x) {
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(x, b, acc[t], 0, 0, 0);
        };
        f16x4 av = op(I0{}, 0);
#pragma unroll
        for (unsigned k = 0; k < S; ++k) {
            f16x4 nx = op(I1{}, k);
            mfma(4 * k + 0, av);
            av = op(I2{}, k);
            mfma(4 * k + 1, nx);
            nx = op(I3{}, k);
            mfma(4 * k + 2, av);
            if (k + 1 < S) av = op(I0{}, k + 1);
            mfma(4 * k + 3, nx);
        }
    }
    waveSync();
}

// One panel alone: staged in area 0 and computed.
template <bool Wide, unsigned G, unsigned S>
__device__ __forceinline__ bool computePanelF16(const Stage& s, unsigned lane, const Lds& lds,
                                                f32x16 (&acc)[4 * S], unsigned keep, LaneMh mh) {
    const bool useF16 = stagePanel<Wide, G, S>(s, lane, lds, 0, keep);
    crunch<S, false>(lds, acc, mh);
    return useF16;
}

// A shared-kind panel with exact FP32 operands (v_mfma_f32_32x32x2_f32): K = 2 steps over slot
// pairs (2j, 2j + 1), lane half h taking slot 2j + h, whose scale comes from lane 2j + h. The
// products are tf32(a) / 2 * x_hat, on the accumulators' Y / 2 scale.
template <bool Wide, unsigned S>
__device__ __forceinline__ void computePanelF32(const Stage& s, unsigned groups, unsigned lane,
                                                const Lds& lds, f32x16 (&acc)[4 * S]) {
#pragma unroll
    for (unsigned g = 0; g < 4; ++g)
        lds.table32[64 * g + lane] = ((groups >> g) & 1u) ? 0.5f * stageTf32<Wide>(s, g) : 0.0f;
#pragma unroll
    for (unsigned k = 0; k < S; ++k) lds.xtile[xTile<S>(lane >> 3, k) + (lane & 7)] = s.x[k];
    waveSync();
    const unsigned m = lane & 31, h = lane >> 5;
#pragma unroll
    for (unsigned j = 0; j < 4; ++j) {
        const unsigned slot = 2 * j + h;
        const float sc =
            __int_as_float(__builtin_amdgcn_ds_bpermute(int(slot * 4), __float_as_int(s.scale)));
        const float b = lds.table32[m * 8 + slot];
#pragma unroll
        for (unsigned k = 0; k < S; ++k) {
            const unsigned d = (reinterpret_cast<const unsigned*>(lds.xtile) + m)[4 * xTile<S>(slot, k)];
#pragma unroll
            for (unsigned blk = 0; blk < 4; ++blk) {
                const float x = roundTf32(float(int(d << (24 - 8 * blk)) >> 24) * sc);
                acc[4 * k + blk] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, b, acc[4 * k + blk], 0, 0, 0);
            }
        }
    }
    waveSync();
}

// ------------------------------------------------------------------------------------------------
// Panel walk

// Row groups of the shared-bucket panels of one task, walked in increasing panel order (bucket slot
// t covers [bucketOffsets[t], bucketOffsets[t + 1]) of the SW). `groups(p)` must be asked for
// non-decreasing p.
struct BucketCursor {
    const unsigned* offsets; // bucketOffsets of the SW (17 entries)
    unsigned t, end;         // current bucket slot and its end panel

    __device__ unsigned groups(unsigned p) {
        while (p >= end) {
            ++t;
            end = offsets[t + 1];
        }
        return unsigned(kBucketGroups >> (4 * t)) & 15u;
    }
};

// Row groups of panel p found from scratch (the FP32 path visits few panels).
__device__ __forceinline__ unsigned groupsOf(const unsigned* offsets, unsigned p) {
    unsigned t = 1;
    while (p >= offsets[t + 1]) ++t;
    return unsigned(kBucketGroups >> (4 * t)) & 15u;
}

struct TaskWalk {
    const unsigned* offsets; // bucketOffsets of the SW
    unsigned begin, end;     // the task's panels
    unsigned lane;
    Lds lds;
    unsigned redoCount;      // entries in lds.redo
    unsigned keep;           // 0x807FFFFF in a VGPR, for shiftedMantissa
    LaneMh mh;
};

// Queues panel `panel` for the FP32 pass when `redo` (wave-uniform) is set. The branch is taken only
// for panels whose operands do not fit f16, so the common path costs one scalar branch; the queue
// length lives in a scalar register.
__device__ __forceinline__ void flagRedo(TaskWalk& w, unsigned panel, bool redo) {
    if (__builtin_expect(redo, 0)) { // wave-uniform and rare
        if (w.lane == 0) w.lds.redo[w.redoCount] = static_cast<unsigned short>(panel - w.begin);
        ++w.redoCount;
    }
}

// The panels [lo, hi) of kind G, pipelined, two panels per iteration with the odd one after the
// loop (a single exit keeps the accumulators in place). Panel indices past the end repeat the last
// panel (harmless loads, never computed).
//
// F128 (S == 1) loads the metadata, sourceIds and scales of two panels with one instruction each, one
// iteration ahead, and hands each panel its slots by DPP row shifts: per panel that is one and
// a half vector memory instructions fewer (c3: 3.51 -> 3.39 ms). F256, at two waves per SIMD, keeps
// one metadata load per panel (pairs cost it 0.5-2% in every form tried) and keeps two panels of
// gathers in flight: stage data two panels ahead, metadata four (1.2% faster than one panel ahead;
// three ahead gained 0.2% for 16 more registers), and computes its panels in pairs, K = 16 per MFMA
// (c3: 5.92 -> 5.72 ms).
template <unsigned G, unsigned S, class Ld>
__device__ __forceinline__ void walkPanels(const Ld& ld, TaskWalk& w, unsigned lo,
                                           unsigned hi, f32x16 (&acc)[4 * S]) {
    if (lo >= hi) return;
    const unsigned n = hi - lo, lane = w.lane;
    if constexpr (G < 4) {
        // The other row groups' table rows (64 entries each per area) stay 0 for the whole bucket.
#pragma unroll
        for (unsigned g = 0; g < 4; ++g) {
            if (g == G) continue;
            if constexpr (S == 1)
                w.lds.table16[64 * g + lane] = static_cast<_Float16>(0.0f);
            else // both areas: 128 entries, two per lane
                reinterpret_cast<f16x2*>(w.lds.table16)[64 * g + lane] = f16x2{0, 0};
        }
    }
    BucketCursor cur{w.offsets, 5, w.offsets[6]};
    auto groupsAt = [&](unsigned p) { return G < 4 ? (1u << G) : cur.groups(p); };
    const unsigned last = hi - 1;
    const unsigned pairs = n / 2;
    Stage sa, sb;
    unsigned ga = groupsAt(lo), gb = 0;
    loadStage<G, S>(ld, ld.meta8(lo, lane), ga, lane, sa);
    if constexpr (S == 1) {
        MetaPair pair = ld.meta2(min(lo + 1, last), last, lane); // panels lo + 1, lo + 2
        // Each panel's row shifts run half an iteration before its loads need them.
        Meta mFirst = pairPanel<0>(pair);
#pragma unroll 1
        for (unsigned k = 0; k < pairs; ++k) {
            // Computes panels lo + 2k (in sa) and lo + 2k + 1; loads the pair after next.
            const MetaPair next = ld.meta2(min(lo + 2 * k + 3, last), last, lane);
            const float sc = ld.scale(pair.id); // both panels' scales, laid out as `pair`
            gb = groupsAt(min(lo + 2 * k + 1, last));
            loadStage<G, S, Ld, false>(ld, mFirst, gb, lane, sb);
            const Meta mSecond = pairPanel<1>(pair);
            // Issue this half's loads before any use of the previous half's: the vmcnt counter
            // is in order, so computing first would wait for loads issued only half an
            // iteration ago.
            __builtin_amdgcn_sched_barrier(0);
            flagRedo(w, lo + 2 * k, !computePanelF16<Ld::kWide, G, S>(sa, lane, w.lds, acc, w.keep, w.mh));
            ga = groupsAt(min(lo + 2 * k + 2, last));
            loadStage<G, S, Ld, false>(ld, mSecond, ga, lane, sa);
            __builtin_amdgcn_sched_barrier(0);
            sb.scale = __uint_as_float(pairHalf<0>(__float_as_uint(sc)));
            flagRedo(w, lo + 2 * k + 1, !computePanelF16<Ld::kWide, G, S>(sb, lane, w.lds, acc, w.keep, w.mh));
            sa.scale = __uint_as_float(pairHalf<1>(__float_as_uint(sc)));
            pair = next;
            mFirst = pairPanel<0>(pair);
        }
        if (n & 1) flagRedo(w, last, !computePanelF16<Ld::kWide, G, S>(sa, lane, w.lds, acc, w.keep, w.mh));
    } else {
        // F256: stage data two panels ahead, metadata four. Three stage buffers rotate: at the step
        // of panel i they hold panels i, i + 1 and (loaded there) i + 2. Loads past the last panel
        // repeat it (harmless, never computed).
        Stage sc;
        unsigned gc = 0;
        const unsigned p1 = min(lo + 1, last), p2 = min(lo + 2, last), p3 = min(lo + 3, last);
        gb = groupsAt(p1);
        loadStage<G, S>(ld, ld.meta8(p1, lane), gb, lane, sb);
        unsigned g1 = groupsAt(p2), g2 = groupsAt(p3);
        // The steps expect m1's loads to be older than m2's (waits are counted in issue order).
        Meta m1 = ld.meta8(p2, lane);
        __builtin_amdgcn_sched_barrier(0);
        Meta m2 = ld.meta8(p3, lane);
        unsigned p = p3;
        // Step of panel `panel` (in `cur`): the loads of panel + 2 into `ahead`, then the panel staged
        // in area 0 (first of a pair) or staged in area 1 and the pair computed (second).
        auto step = [&](auto second, Stage& cur, Stage& ahead, unsigned& gahead,
                        unsigned panel) __attribute__((always_inline)) {
            gahead = g1;
            loadStage<G, S>(ld, m1, gahead, lane, ahead);
            p = min(p + 1, last);
            m1 = m2;
            g1 = g2;
            g2 = groupsAt(p);
            m2 = ld.meta8(p, lane);
            __builtin_amdgcn_sched_barrier(0);
            constexpr bool kSecond = decltype(second)::value;
            flagRedo(w, panel, !stagePanel<Ld::kWide, G, S>(cur, lane, w.lds, kSecond ? 1u : 0u, w.keep));
            if constexpr (kSecond) crunch<S, true>(w.lds, acc, w.mh);
        };
        using First = std::integral_constant<bool, false>;
        using Second = std::integral_constant<bool, true>;
        // Panels in pairs, in a loop unrolled by six (the period of both the pairs and the stage
        // rotation), then the r < 6 panels left: their pairs by the same steps and a last panel
        // without a partner alone, staged in area 0. (A loop that leaves after any panel, computing
        // the unpaired one on its way out, made the register allocator spill the accumulators.)
        const unsigned sixes = n / 6, r = n - 6 * sixes;
        unsigned i = lo;
#pragma unroll 1
        for (unsigned k = 0; k < sixes; ++k, i += 6) {
            step(First{}, sa, sc, gc, i);
            step(Second{}, sb, sa, ga, i + 1);
            step(First{}, sc, sb, gb, i + 2);
            step(Second{}, sa, sc, gc, i + 3);
            step(First{}, sb, sa, ga, i + 4);
            step(Second{}, sc, sb, gb, i + 5);
        }
        if (r >= 2) {
            step(First{}, sa, sc, gc, i);
            step(Second{}, sb, sa, ga, i + 1);
        }
        if (r >= 4) {
            step(First{}, sc, sb, gb, i + 2);
            step(Second{}, sa, sc, gc, i + 3);
        }
        if (r & 1) {
            const Stage& odd = r == 1 ? sa : r == 3 ? sc : sb;
            flagRedo(w, hi - 1, !computePanelF16<Ld::kWide, G, S>(odd, lane, w.lds, acc, w.keep, w.mh));
        }
    }
}

template <unsigned S, class Ld>
__device__ __forceinline__ void walkTask(const Ld& ld, const unsigned* offsets, unsigned begin,
                                         unsigned end, unsigned lane, const Lds& lds,
                                         f32x16 (&acc)[4 * S]) {
    if (begin >= end) return;
    // An opaque definition keeps the mask in one VGPR for the whole walk instead of a
    // rematerialised literal per use.
    unsigned keep;
    asm("v_mov_b32 %0, 0x807fffff" : "=v"(keep));
    LaneMh mh;
    // %0 is written before %2 is read again: early-clobber, so it never shares the input's register.
    asm("v_and_b32 %0, 31, %2\n\tv_lshrrev_b32 %1, 5, %2" : "=&v"(mh.m), "=v"(mh.h) : "v"(lane));
    TaskWalk w{offsets, begin, end, lane, lds, 0u, keep, mh};
    auto clipLo = [&](unsigned t) { return max(offsets[t], begin); };
    auto clipHi = [&](unsigned t) { return min(offsets[t], end); };
    walkPanels<0, S>(ld, w, clipLo(1), clipHi(2), acc);
    walkPanels<1, S>(ld, w, clipLo(2), clipHi(3), acc);
    walkPanels<2, S>(ld, w, clipLo(3), clipHi(4), acc);
    walkPanels<3, S>(ld, w, clipLo(4), clipHi(5), acc);
    walkPanels<kShared, S>(ld, w, clipLo(5), clipHi(16), acc);
    waveSync();
#pragma unroll 1
    for (unsigned i = 0; i < w.redoCount; ++i) {
        const unsigned panel = begin + __builtin_amdgcn_readfirstlane(lds.redo[i]);
        const unsigned groups = groupsOf(offsets, panel);
        Stage st;
        loadStage<kShared, S>(ld, ld.meta8(panel, lane), groups, lane, st);
        computePanelF32<Ld::kWide, S>(st, groups, lane, lds, acc);
    }
}

// Four consecutive floats of Y or of the partial tiles. Vec4: one 16-byte access (the buffer's
// base is 16-byte aligned, which every row offset keeps); otherwise four dword accesses, for a base
// that is only float-aligned (the reference stores single floats, src/kernel/spmm_kernel.cuh:
// 236-245, so it accepts one).
template <bool Vec4>
__device__ __forceinline__ void store4(float* p, const f32x4& v, bool nontemporal) {
    if constexpr (Vec4) {
        if (nontemporal)
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
        else
            *reinterpret_cast<f32x4*>(p) = v;
    } else {
#pragma unroll
        for (unsigned t = 0; t < 4; ++t) {
            if (nontemporal)
                __builtin_nontemporal_store(v[t], p + t);
            else
                p[t] = v[t];
        }
    }
}
template <bool Vec4>
__device__ __forceinline__ f32x4 load4(const float* p) {
    if constexpr (Vec4) return *reinterpret_cast<const f32x4*>(p);
    else return f32x4{p[0], p[1], p[2], p[3]};
}

// Store row `row` (lane & 31) of the accumulators: per tile i the lane holds the 16 features
// 16 (2i + h) .. + 15 of the slice, block b / register 4i + j holding feature 2j + (b >> 1) +
// 8 (b & 1) of that tile.
template <bool Vec4>
__device__ __forceinline__ void storeRow(const f32x16 (&acc)[4], float* rowBase, unsigned h,
                                         bool nontemporal) {
#pragma unroll
    for (unsigned i = 0; i < 4; ++i) {
        float* dst = rowBase + 16 * (2 * i + h);
#pragma unroll
        for (unsigned q = 0; q < 4; ++q) {
            f32x4 v;
#pragma unroll
            for (unsigned t = 0; t < 4; ++t) {
                const unsigned o = 4 * q + t;
                const unsigned hiHalf = o >= 8 ? 1u : 0u;
                const unsigned rem = o - 8 * hiHalf;
                v[t] = acc[(rem & 1u) * 2 + hiHalf][4 * i + (rem >> 1)];
            }
            store4<Vec4>(dst + 4 * q, v, nontemporal);
        }
    }
}

// Workgroup -> task. Workgroups are dispatched to the 8 XCDs round-robin by id, and XCD x walks
// one contiguous range of the task list, so neighbouring SWs share source rows of X in its L2. The
// ranges hold equal task counts unless that leaves some XCD more than 3% above the mean panel
// count (hub SWs cut into many 384-panel tasks); then the ranges hold equal panel counts, each
// boundary moved at most a quarter of a share (T / 32 tasks) from its equal-count place. The grid
// carries half a share (ceil(T / 16)) of spare workgroups per XCD, enough for the longest range
// this allows; workgroups past their XCD's range exit. Task begins never decrease along the list,
// so the panel-balanced boundaries are searches over them (panelBound), the same for every
// workgroup of an XCD.
constexpr unsigned kSpareDiv = 16; // spare workgroups per XCD: ceil(T / 16), half a share

__host__ __device__ inline unsigned spareWorkgroups(unsigned tasks) {
    return (tasks + kSpareDiv - 1) / kSpareDiv;
}

__device__ __forceinline__ unsigned equalBound(unsigned tasks, unsigned x) {
    const unsigned q = tasks >> 3, r = tasks & 7u;
    return x * q + min(x, r);
}

// The tail window: the last kTailWindow tasks of an XCD's range run longest size class first
// (panels >= 288, >= 192, >= 96, the rest; list order within a class), so that the launch does not
// end on a few long tasks started last. The window spans about the SWs an XCD holds resident at its
// end anyway, so the order inside it leaves the L2 sharing of the in-order walk in place.
constexpr unsigned kTailWindow = 512;

__device__ __forceinline__ unsigned sizeClass(const Sw32Task* tasks, unsigned t) {
    const unsigned p = tasks[t].end - tasks[t].begin;
    return unsigned(p >= 96) + unsigned(p >= 192) + unsigned(p >= 288);
}

// Task at position r (r < n <= kTailWindow) of the window [w0, w0 + n) in size-class order. One
// wave, all lanes active; every wave computes the same permutation of the window. The classes of
// the window's tasks are loaded once (lane L: tasks L, L + 64, ...; all loads in flight together),
// kept two bits per task in registers, and both passes below work on those.
__device__ __forceinline__ unsigned tailTask(const Sw32Task* tasks, unsigned w0, unsigned n,
                                             unsigned r, unsigned lane) {
    constexpr unsigned kChunks = kTailWindow / kWave, kWords = (kChunks + 15) / 16;
    unsigned bits[kWords] = {};
#pragma unroll
    for (unsigned ch = 0; ch < kChunks; ++ch)
        bits[ch / 16] |= sizeClass(tasks, w0 + min(ch * kWave + lane, n - 1)) << (2 * (ch % 16));
    auto member = [&](unsigned ch, unsigned c) {
        return ch * kWave + lane < n && ((bits[ch / 16] >> (2 * (ch % 16))) & 3u) == c;
    };
    unsigned counts[4] = {0, 0, 0, 0};
#pragma unroll
    for (unsigned ch = 0; ch < kChunks; ++ch)
#pragma unroll
        for (unsigned c = 0; c < 4; ++c)
            counts[c] += unsigned(__builtin_popcountll(__builtin_amdgcn_ballot_w64(member(ch, c))));
    unsigned c = 3, k = r;
    while (c > 0 && k >= counts[c]) {
        k -= counts[c];
        --c;
    }
#pragma unroll
    for (unsigned ch = 0; ch < kChunks; ++ch) {
        const bool in = member(ch, c);
        const std::uint64_t mask = __builtin_amdgcn_ballot_w64(in);
        const unsigned count = unsigned(__builtin_popcountll(mask));
        if (k < count) {
            const unsigned below = __builtin_amdgcn_mbcnt_hi(unsigned(mask >> 32),
                                                             __builtin_amdgcn_mbcnt_lo(unsigned(mask), 0u));
            const std::uint64_t hit = __builtin_amdgcn_ballot_w64(in && below == k);
            return w0 + ch * kWave + unsigned(__builtin_ctzll(hit));
        }
        k -= count;
    }
    return w0 + r; // not reached: the window holds n tasks
}

// Boundaries x and x + 1 of the panel-balanced ranges: the first task starting at or past k/8 of
// the panels, measured from the first task's begin (k = x, x + 1; `count` when none does; a view
// over a later part of a plan's task list starts past panel 0). Lanes 32h .. 32h + 31 search boundary x + h
// together: each step probes 32 evenly spaced tasks of the half's interval [l, r] (task r is known
// to qualify; r = count stands for past the end) and keeps the stretch between the last probe
// below the target and the first one at or past it, so a search takes about log32(T) dependent
// loads instead of log2(T). Returns the boundary of each lane's half.
__device__ __forceinline__ unsigned panelBound(const Sw32Task* tasks, unsigned count,
                                               unsigned first, std::uint64_t panels, unsigned x,
                                               unsigned lane) {
    const unsigned h = lane >> 5, j = lane & 31;
    const unsigned target = first + unsigned(panels * (x + h) / 8);
    unsigned l = 0, r = count;
    while (__builtin_amdgcn_ballot_w64(l < r) != 0) {
        const unsigned stride = (r - l + 31) / 32; // 32 probes cover [l, r): r - l <= 32 stride
        const unsigned q = l + j * stride;
        const bool at = q >= r || tasks[min(q, count - 1)].begin >= target;
        const unsigned half = unsigned(__builtin_amdgcn_ballot_w64(at) >> (32 * h));
        const unsigned first = half ? unsigned(__builtin_ctz(half)) : 32u;
        const unsigned nl = first == 0 ? l : l + (first - 1) * stride + 1;
        r = first < 32 ? min(l + first * stride, r) : r;
        l = nl;
    }
    return l;
}

// Returns false when the workgroup has no task.
__device__ __forceinline__ bool xcdTask(const KernelArgs& a, unsigned bid, unsigned& task) {
    const Sw32Task* tasks = a.m.tasks;
    const unsigned count = a.m.taskCount, x = bid & 7u, j = bid >> 3;
    const unsigned lane = threadIdx.x & (kWave - 1);
    auto beginOf = [&](unsigned t) { return t < count ? tasks[t].begin : tasks[count - 1].end; };
    unsigned first[9];
    unsigned maxPanels = 0;
#pragma unroll
    for (unsigned k = 0; k <= 8; ++k) first[k] = beginOf(equalBound(count, k));
#pragma unroll
    for (unsigned k = 0; k < 8; ++k) maxPanels = max(maxPanels, first[k + 1] - first[k]);
    const std::uint64_t panels = first[8] - first[0];
    unsigned lo = equalBound(count, x), hi = equalBound(count, x + 1);
    if (std::uint64_t(maxPanels) * 8 * 100 > panels * 103) {
        const unsigned reach = spareWorkgroups(count) / 2;
        const unsigned searched = panelBound(tasks, count, first[0], panels, x, lane);
        const unsigned k = x + (lane >> 5), eq = equalBound(count, k);
        const unsigned b = (k == 0 || k == 8) ? eq : min(max(searched, eq > reach ? eq - reach : 0u), eq + reach);
        lo = __builtin_amdgcn_readlane(b, 0);
        hi = __builtin_amdgcn_readlane(b, 32);
    }
    task = lo + j;
    if (task >= hi) return false;
    const unsigned n = min(hi - lo, kTailWindow), w0 = hi - n;
    if (task >= w0) task = tailTask(tasks, w0, n, task - w0, lane);
    return true;
}

// Merge of slice k of a split SW by the task that took its last ticket (reference
// src/kernel/spmm_kernel.cuh:250-282): Y = the SW's partial tiles summed in partialIds order,
// starting from 0.0f, one row group (8 rows x 128 columns) at a time. Lane L sums the four 16-byte
// column blocks (L & 7) + 8j, j < 4, of row L >> 3. The group's tile ids are loaded once (one per
// lane, broadcast by readlane), and the loads of kMergeBatch tiles are issued before they are added
// in order, so a merge of many chunks waits for one load latency per batch, not per tile. Per element
// the additions run in partialIds order whatever the batch, so Y is bitwise the same for any batch.
template <unsigned Features, bool Vec4>
__device__ __forceinline__ void mergeSlice(const KernelArgs& a, const Sw32Task& task, unsigned k,
                                           unsigned lane) {
    constexpr unsigned kMergeBatch = 4;
    const unsigned sw = task.sw;
    const unsigned mrow = lane >> 3, mcol = k * kSlice + (lane & 7) * 4;
#pragma unroll 1
    for (unsigned g = 0; g < 4; ++g) {
        const Sw32ReduceRange red = a.m.reductions[task.reduceFirst + g];
        const unsigned row0 = sw * 32 + g * 8;
        if (row0 >= a.rows) continue;
        f32x4 sum[4];
#pragma unroll
        for (unsigned j = 0; j < 4; ++j) sum[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        auto tileRow = [&](unsigned id) {
            return a.partials + (std::size_t(id) * 8 + mrow) * Features + mcol;
        };
#pragma unroll 1
        for (unsigned base = red.begin; base < red.end; base += kWave) {
            const unsigned items = min(red.end - base, kWave);
            const unsigned ids = a.m.partialIds[base + min(lane, items - 1)];
            unsigned i = 0;
#pragma unroll 1
            for (; i + kMergeBatch <= items; i += kMergeBatch) {
                f32x4 v[kMergeBatch][4];
#pragma unroll
                for (unsigned u = 0; u < kMergeBatch; ++u) {
                    const float* src = tileRow(__builtin_amdgcn_readlane(ids, i + u));
#pragma unroll
                    for (unsigned j = 0; j < 4; ++j) v[u][j] = load4<Vec4>(src + 32 * j);
                }
#pragma unroll
                for (unsigned u = 0; u < kMergeBatch; ++u)
#pragma unroll
                    for (unsigned j = 0; j < 4; ++j) sum[j] += v[u][j];
            }
#pragma unroll 1
            for (; i < items; ++i) {
                const float* src = tileRow(__builtin_amdgcn_readlane(ids, i));
#pragma unroll
                for (unsigned j = 0; j < 4; ++j) sum[j] += load4<Vec4>(src + 32 * j);
            }
        }
        if (row0 + mrow < a.rows) {
            float* yr = a.y + std::size_t(row0 + mrow) * Features + mcol;
#pragma unroll
            for (unsigned j = 0; j < 4; ++j) store4<Vec4>(yr + 32 * j, sum[j], false);
        }
    }
}

// One task over all S = Features / 128 slices of its SW, by `Waves` waves of one workgroup. With
// more than one wave, wave w walks the w-th of `Waves` equal shares of the task's panels (its own
// LDS tables, the same walk as a whole task), then hands its accumulators to wave 0, which adds them
// in wave order and finishes the task alone. A task then takes about 1/Waves of the time, which
// shortens launches whose longest tasks set the time (few tasks per wave slot).
template <unsigned Features, unsigned Addr, unsigned Waves = 1>
__device__ __forceinline__ void runTask(const KernelArgs& a, unsigned taskIndex) {
    constexpr unsigned S = Features / kSlice;
    constexpr unsigned kAreas = S == 1 ? 1 : 2; // F256 computes its panels in pairs
    __shared__ __align__(16) _Float16 table16[Waves][256 * kAreas];
    __shared__ __align__(16) float table32[Waves][256];
    __shared__ __align__(16) u32x4 xtile[Waves][kAreas * 64 * S];
    __shared__ __align__(16) float mant[Waves][8 * kAreas];
    __shared__ unsigned short redo[Waves][384];
    __shared__ unsigned lastFlag[S];
    const unsigned wave = Waves == 1 ? 0u : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const unsigned lane = Waves == 1 ? threadIdx.x : threadIdx.x & 63u;
    const Sw32Task task = a.m.tasks[taskIndex];
    const unsigned sw = task.sw;
    const Loader<Addr> ld(a, task.begin, task.end, Features);
    const Lds lds{table16[wave], table32[wave], xtile[wave], mant[wave], redo[wave]};

    f32x16 acc[4 * S];
#pragma unroll
    for (unsigned b = 0; b < 4 * S; ++b) acc[b] = f32x16{};
    unsigned lo = task.begin, hi = task.end;
    if constexpr (Waves > 1) {
        const std::uint64_t n = hi - lo;
        lo = task.begin + unsigned(n * wave / Waves);
        hi = task.begin + unsigned(n * (wave + 1) / Waves);
    }
    walkTask<S>(ld, a.m.bucketOffsets + std::size_t(sw) * 17, lo, hi, lane, lds, acc);
#pragma unroll
    for (unsigned b = 0; b < 4 * S; ++b) acc[b] *= 2.0f; // Y / 2 to Y, exact
    if constexpr (Waves > 1) {
        // One accumulator block (16 floats per lane) per round, as four 16-byte chunks per lane
        // laid out chunk-major so that each chunk's 64 lanes are contiguous.
        __shared__ __align__(16) f32x4 handoff[Waves - 1][4][kWave];
#pragma unroll
        for (unsigned b = 0; b < 4 * S; ++b) {
            if (wave != 0) {
#pragma unroll
                for (unsigned q = 0; q < 4; ++q)
                    handoff[wave - 1][q][lane] =
                        f32x4{acc[b][4 * q], acc[b][4 * q + 1], acc[b][4 * q + 2], acc[b][4 * q + 3]};
            }
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (unsigned v = 0; v + 1 < Waves; ++v)
#pragma unroll
                    for (unsigned q = 0; q < 4; ++q) {
                        const f32x4 o = handoff[v][q][lane];
#pragma unroll
                        for (unsigned e = 0; e < 4; ++e) acc[b][4 * q + e] += o[e];
                    }
            }
            __syncthreads();
        }
        if (wave != 0) return;
    }

    const unsigned row = lane & 31, h = lane >> 5;
    // Write-back. An unsplit task stores its rows of Y (nontemporal: nothing reads them again in this
    // launch); a split task stores the row groups of task.mask as 8-row partial tiles. One store site
    // for both, so that the accumulators are dead once it is passed.
    const bool split = task.partial != kNoPartial;
    const unsigned rw = row >> 3;
    float* dst;
    bool mine;
    if (!split) {
        const unsigned r = sw * 32 + row;
        mine = r < a.rows;
        dst = a.y + std::size_t(r) * Features;
    } else {
        mine = (task.mask >> rw) & 1u;
        const std::size_t tile = task.partial + __popc(task.mask & ((1u << rw) - 1u));
        dst = a.partials + (tile * 8 + (row & 7)) * Features;
    }
    auto sub = [&](unsigned k) -> const f32x16(&)[4] {
        return *reinterpret_cast<const f32x16(*)[4]>(&acc[4 * k]);
    };
    if (mine) {
        if (a.vec4) {
#pragma unroll
            for (unsigned k = 0; k < S; ++k) storeRow<true>(sub(k), dst + k * kSlice, h, !split);
        } else {
#pragma unroll
            for (unsigned k = 0; k < S; ++k) storeRow<false>(sub(k), dst + k * kSlice, h, !split);
        }
    }
    if (!split) return;

    // Completion tickets, one per slice: the acq_rel RMW at agent scope publishes this task's
    // partial tiles and, for the last arriver, makes every other task's tiles visible (the XCD L2s
    // are not coherent with each other, so the release writes back and the acquire invalidates).
    waveSync();
    if (lane == 0) {
#pragma unroll
        for (unsigned k = 0; k < S; ++k) {
            unsigned* counter = a.counters + std::size_t(sw) * S + k;
            const unsigned ticket =
                __builtin_amdgcn_atomic_inc32(counter, task.chunks - 1, __ATOMIC_ACQ_REL, "agent");
            lastFlag[k] = ticket == task.chunks - 1;
        }
    }
    waveSync();
#pragma unroll 1
    for (unsigned k = 0; k < S; ++k) {
        if (!lastFlag[k]) continue;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (a.vec4)
            mergeSlice<Features, true>(a, task, k, lane);
        else
            mergeSlice<Features, false>(a, task, k, lane);
    }
}

// Per-task timeline for the measurement build (compiled with TCC_SPMM_TIMELINE by
// model/timeline.py; the library build leaves this empty and the kernels unchanged). Lane 0 of each
// workgroup stores, for its task: the workgroup's start, the time its task was found, its end
// (s_memrealtime, a 100 MHz counter) and its XCC id << 32 | workgroup id, with vector stores.
struct TaskClock {
#ifdef TCC_SPMM_TIMELINE
    unsigned long long start = __builtin_amdgcn_s_memrealtime(), found = 0;
    __device__ void mapped() { found = __builtin_amdgcn_s_memrealtime(); }
    __device__ void done(const KernelArgs& a, unsigned task) const {
        const unsigned long long end = __builtin_amdgcn_s_memrealtime();
        if (threadIdx.x == 0 && a.stamps) {
            const unsigned long long xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20); // HW_REG_XCC_ID
            unsigned long long* out = a.stamps + 4 * std::size_t(task);
            out[0] = start;
            out[1] = found;
            out[2] = end;
            out[3] = xcc << 32 | blockIdx.x;
        }
    }
#else
    __device__ void mapped() {}
    __device__ void done(const KernelArgs&, unsigned) const {}
#endif
};

// F128: four waves per SIMD; the 64 accumulators live in ordinary VGPRs and the kernel fits 128
// registers.
template <unsigned Addr, unsigned Waves = 1>
__global__ __launch_bounds__(kWave * Waves) __attribute__((amdgpu_waves_per_eu(4, 8))) void
spmmInt8Kernel128(KernelArgs a) {
    TaskClock clock;
    unsigned task;
    if (xcdTask(a, blockIdx.x, task)) {
        clock.mapped();
        runTask<128, Addr, Waves>(a, task);
        clock.done(a, task);
    }
}

// F256: both 128-feature slices of a task in one wave (128 accumulator registers, two waves per
// SIMD). The task's A stream, scales and A table are read and built once for both slices; measured
// on c3 this moves 18% fewer bytes (33.1 GB against 40.5 GB) and runs 8.6% faster than one wave
// per (task, slice).
template <unsigned Addr, unsigned Waves = 1>
__global__ __launch_bounds__(kWave * Waves) __attribute__((amdgpu_waves_per_eu(2, 8))) void
spmmInt8Kernel256(KernelArgs a) {
    TaskClock clock;
    unsigned task;
    if (xcdTask(a, blockIdx.x, task)) {
        clock.mapped();
        runTask<256, Addr, Waves>(a, task);
        clock.done(a, task);
    }
}

constexpr int kMaxDevices = 64;

// Launch choices forced by setSpmmLaunchOverrides or, initially, the environment (read once).
std::once_flag overridesRead;
std::atomic<unsigned> forcedWaves{0}; // 0: chosen per launch
std::atomic<bool> forcedWide{false};

void readOverridesOnce() {
    std::call_once(overridesRead, [] {
        if (const char* w = std::getenv("TCC_SPMM_TASK_WAVES"))
            forcedWaves.store(std::strcmp(w, "2") == 0 ? 2u : 1u);
        if (std::getenv("TCC_SPMM_FORCE_WIDE")) forcedWide.store(true);
    });
}

// Compute units of the current device, queried once per device (0 when unknown).
std::atomic<int> deviceCuCount[kMaxDevices];

int currentDeviceCus() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 0;
    int cus = deviceCuCount[device].load(std::memory_order_relaxed);
    if (cus == 0 &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess)
        deviceCuCount[device].store(cus, std::memory_order_relaxed);
    return cus;
}

// Waves per task: 2 when the plan has few tasks for the chip's wave slots, so that the longest
// tasks, not the bandwidth, set the launch time; else 1. Measured crossovers on MI355X (256 CUs;
// wave slots = CUs x 4 SIMDs x the kernel's waves per SIMD, 4 at F128 and 2 at F256): F128 gains
// below about 3 tasks per slot (-39% at 250 tasks, -6% at 8,790, even at 12,500, +3% at 38,281),
// F256 below about half a task per slot (-26% at 1,000 tasks, +1% at 1,875).
unsigned taskWaves(unsigned taskCount, unsigned features) {
    if (const unsigned forced = forcedWaves.load()) return forced;
    const int cus = currentDeviceCus();
    if (cus <= 0) return 1;
    const std::uint64_t slots = std::uint64_t(cus) * 4 * (features == 128 ? 4 : 2);
    const std::uint64_t limit = features == 128 ? 3 * slots : slots / 2;
    return taskCount < limit ? 2u : 1u;
}

template <unsigned Features>
void launch(const KernelArgs& args, hipStream_t stream) {
    // Buffer addressing needs the packed X and the scales within 32-bit byte offsets, with room for
    // the padding sentinel to land out of range, and 16-byte aligned X tiles. A packed X that is
    // only u16-aligned takes the 64-bit instance with 2-byte tile loads. setSpmmLaunchOverrides
    // can select the 64-bit instance for any size (used by the tests).
    const bool misaligned = reinterpret_cast<std::uintptr_t>(args.packedX) % 16 != 0;
    const bool wide = std::uint64_t(args.cols) * Features > 0xFFFFFF00ull || forcedWide.load();
    const dim3 grid(args.m.taskCount + 8 * spareWorkgroups(args.m.taskCount), 1);
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kWave), 0, stream, args); };
    auto go2 = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(2 * kWave), 0, stream, args);
    };
    const bool split = !misaligned && !wide && taskWaves(args.m.taskCount, Features) == 2;
    if constexpr (Features == 256) {
        if (misaligned)
            go(spmmInt8Kernel256<kGlobalU16>);
        else if (wide)
            go(spmmInt8Kernel256<kGlobal>);
        else if (split)
            go2(spmmInt8Kernel256<kBuffer, 2>);
        else
            go(spmmInt8Kernel256<kBuffer>);
    } else {
        if (misaligned)
            go(spmmInt8Kernel128<kGlobalU16>);
        else if (wide)
            go(spmmInt8Kernel128<kGlobal>);
        else if (split)
            go2(spmmInt8Kernel128<kBuffer, 2>);
        else
            go(spmmInt8Kernel128<kBuffer>);
    }
}

} // namespace

namespace {

// Checks shared by both entry points, before anything is launched. Null buffers would fault the GPU
// and are rejected (the reference does not check). Of the view, only the arrays every plan has are
// required (tasks, and bucketOffsets with 17 entries per SW): a plan without panels has empty
// sourceIds, sourceMetadata and values, which may be null. The workspace may be null (a plan
// without split SWs), and its size is the caller's contract.
void checkLaunchArguments(const Sw32DeviceView& matrix, const std::int8_t* packedX,
                          const float* scales, const float* output) {
    if (!matrix.taskCount)
        throw std::runtime_error("launchSpmmInt8: invalid configuration argument (no tasks)");
    if (matrix.taskCount > 0x7FFFFFFFu)
        throw std::invalid_argument("launchSpmmInt8: too many tasks for one launch");
    if (!packedX || !scales || !output)
        throw std::invalid_argument("launchSpmmInt8: null packedX, scales or output");
    if (!matrix.tasks || !matrix.bucketOffsets)
        throw std::invalid_argument("launchSpmmInt8: device view with null tasks or bucketOffsets");
    // The packed features are read as u16 pairs at least (reference include/format/int8_features.cuh:
    // 11-13 states u16 alignment); an odd address cannot be.
    if (reinterpret_cast<std::uintptr_t>(packedX) % 2)
        throw std::invalid_argument("launchSpmmInt8: packedX must be u16-aligned");
    // Y is written as floats (16 bytes per lane when Y and the partials are 16-byte aligned, one
    // float per store otherwise), so a float-aligned base is accepted, as in the reference.
    if (reinterpret_cast<std::uintptr_t>(output) % alignof(float))
        throw std::invalid_argument("launchSpmmInt8: output must be float-aligned");
}

} // namespace

#ifdef TCC_SPMM_TIMELINE
// Measurement build only: the stamp buffer of the last launch, grown as needed, and its read-back.
namespace {
unsigned long long* gStamps = nullptr;
std::uint32_t gStampTasks = 0, gStampCapacity = 0;

unsigned long long* timelineStamps(std::uint32_t tasks) {
    if (tasks > gStampCapacity) {
        if (gStamps) checkHip(hipFree(gStamps));
        checkHip(hipMalloc(&gStamps, std::size_t(tasks) * 32));
        gStampCapacity = tasks;
    }
    gStampTasks = tasks;
    return gStamps;
}
} // namespace

extern "C" int tcc_timeline_stamps(unsigned long long* host, std::uint32_t tasks) {
    if (!gStamps || tasks != gStampTasks || hipDeviceSynchronize() != hipSuccess) return 1;
    return hipMemcpy(host, gStamps, std::size_t(tasks) * 32, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 2;
}
#endif

void launchSpmmInt8(Sw32DeviceView matrix, const std::int8_t* packedX, const float* scales,
                    float* output, std::uint32_t rows, std::uint32_t cols, std::uint32_t features,
                    SpmmWorkspace workspace, hipStream_t stream) {
    if (features != 128 && features != 256)
        throw std::invalid_argument("feature dimension must be 128 or 256");
    checkLaunchArguments(matrix, packedX, scales, output);
    readOverridesOnce();
    if (reinterpret_cast<std::uintptr_t>(workspace.partials) % alignof(float))
        throw std::invalid_argument("launchSpmmInt8: workspace.partials must be float-aligned");
    // Y and the partial tiles move 16 bytes per lane when both bases allow it (any hipMalloc'd
    // buffer and any whole-row offset into one does), else one float per access; Y is bitwise
    // the same either way.
    const bool vec4 = (reinterpret_cast<std::uintptr_t>(output) |
                       reinterpret_cast<std::uintptr_t>(workspace.partials)) % 16 == 0;
    KernelArgs args{matrix, packedX, scales, output, workspace.partials, workspace.counters,
                    rows,   cols,    unsigned(vec4)};
#ifdef TCC_SPMM_TIMELINE
    args.stamps = timelineStamps(matrix.taskCount);
#endif
    if (features == 128)
        launch<128>(args, stream);
    else
        launch<256>(args, stream);
    checkHip(hipGetLastError());
}

void setSpmmLaunchOverrides(std::uint32_t taskWaves, bool forceWide) {
    if (taskWaves > 2)
        throw std::invalid_argument("setSpmmLaunchOverrides: taskWaves must be 0, 1 or 2");
    readOverridesOnce(); // so that a later first launch keeps these rather than the environment's
    forcedWaves.store(taskWaves);
    forcedWide.store(forceWide);
}

// ------------------------------------------------------------------------------------------------
// Allocation-free entry point (no counterpart in the reference): the split-SW workspace lives in a
// library-owned device array instead of caller buffers. Layout: completion counters
// [ceil(rows/32)][F/128] from offset 0, then the partial tiles [K][8][F] from the next 256-byte
// boundary. Every GPU the library runs on holds its own copy for the life of the process.

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex scratchLock;
void* scratchAddress[kMaxDevices]; // device address of `scratch` per device, found once

// The address of the current device's `scratch`. In host code the array's name is only a stand-in
// for the symbol, never a device pointer, so the address is looked up once per device (with that
// device current) and reused.
void* deviceScratch() {
    int device = 0;
    checkHip(hipGetDevice(&device));
    if (device < 0 || device >= kMaxDevices)
        throw std::runtime_error("launchSpmmInt8NoAlloc: device index out of range");
    std::lock_guard<std::mutex> guard(scratchLock);
    if (!scratchAddress[device]) {
        void* address = nullptr;
        checkHip(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
        scratchAddress[device] = address;
    }
    return scratchAddress[device];
}

// Zero `count` words: a kernel rather than hipMemsetAsync, so the entry point can be captured into
// a HIP graph.
__global__ __launch_bounds__(256) void clearWords(unsigned* words, unsigned count) {
    for (unsigned i = blockIdx.x * 256 + threadIdx.x; i < count; i += gridDim.x * 256) words[i] = 0;
}

} // namespace

void launchSpmmInt8NoAlloc(Sw32DeviceView matrix, const std::int8_t* packedX, const float* scales,
                           float* output, std::uint32_t rows, std::uint32_t cols,
                           std::uint32_t features, std::uint32_t partialCount, hipStream_t stream) {
    if (features != 128 && features != 256)
        throw std::invalid_argument("feature dimension must be 128 or 256");
    checkLaunchArguments(matrix, packedX, scales, output);
    SpmmWorkspace workspace;
    if (partialCount) {
        const std::uint64_t counters = (std::uint64_t(rows) + 31) / 32 * (features / 128);
        const std::uint64_t counterBytes = (counters * 4 + 255) / 256 * 256;
        const std::uint64_t partialBytes = std::uint64_t(partialCount) * 8 * features * 4;
        if (counterBytes + partialBytes > kNoAllocScratchBytes)
            throw std::invalid_argument(
                "launchSpmmInt8NoAlloc: the plan's " + std::to_string(partialCount) +
                " partial tiles at F=" + std::to_string(features) + " need " +
                std::to_string(counterBytes + partialBytes) + " bytes of scratch, more than its " +
                std::to_string(kNoAllocScratchBytes) + "; use launchSpmmInt8 with a workspace");
        unsigned char* base = static_cast<unsigned char*>(deviceScratch());
        workspace.counters = reinterpret_cast<std::uint32_t*>(base);
        workspace.partials = reinterpret_cast<float*>(base + counterBytes);
        // The counters must start at zero; a previous call leaves them at zero unless it failed.
        const unsigned blocks = unsigned(std::min<std::uint64_t>((counters + 255) / 256, 1024));
        hipLaunchKernelGGL(clearWords, dim3(blocks), dim3(256), 0, stream, workspace.counters,
                           unsigned(counters));
        checkHip(hipGetLastError());
    }
    launchSpmmInt8(matrix, packedX, scales, output, rows, cols, features, workspace, stream);
}
