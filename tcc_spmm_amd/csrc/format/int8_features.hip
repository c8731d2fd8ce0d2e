// Per-source INT8 quantization and packed16 byte permutation for gfx950 (wave64).
//
// quantize: rows of features % 4 == 0 (16-byte aligned) use 16-byte loads of 4-feature groups and one
// dword store per 4 quantized bytes: quantizeRowsFit for F <= 256 (one group per lane, several rows
// per thread held in registers, X read once), quantizeRowsLong above; other rows one wave per row
// (quantizeRows). The row's |x| maximum is reduced across its lanes with shuffles, and every element
// is divided by the scale with the IEEE-correct FP32 divide and rounded half-to-even. Results are bit-identical to reference
// src/format/int8_quantize.cu:4-25.
//
// pack: one thread per 16-byte tile; four v_perm_b32 byte shuffles turn q[0..15] into
// [q0,q8,q1,q9,...,q7,q15] (reference src/format/pack_int8.cu:6-15). Unaligned buffers use a
// byte-pair kernel with the same result.
//
// quantize + pack fused (no counterpart in the reference): the quantize kernels with `Packed` set
// write the packed layout directly, so q is never written and read back. In the vector kernels the
// four lanes of a 16-feature tile swap their quantized dwords with two quad-permute DPP moves and
// assemble their output dword with one v_perm_b32; the scalar kernel stores each byte at its packed
// position.
#include "format/int8_features.h"
#include "hip_support.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>

namespace {

constexpr unsigned kWave = 64;
constexpr unsigned kRowsPerBlock = 4;

// Byte offset of feature j of a row in the packed16 layout: within each 16-feature tile, feature k
// goes to byte 2k (k < 8) or 2(k - 8) + 1.
__device__ __forceinline__ unsigned packedOffset(unsigned j) {
    const unsigned k = j & 15u;
    return (j & ~15u) + (k < 8 ? 2 * k : 2 * (k - 8) + 1);
}

template <bool Packed>
__global__ __launch_bounds__(kWave* kRowsPerBlock) void quantizeRows(
    const float* __restrict__ x, std::int8_t* __restrict__ q, float* __restrict__ scale,
    unsigned sources, unsigned features) {
    const unsigned lane = threadIdx.x & (kWave - 1);
    const std::size_t row = std::size_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x / kWave);
    if (row >= sources) return;
    const float* xr = x + std::size_t(row) * features;
    float m = 0.0f;
    for (unsigned j = lane; j < features; j += kWave) m = fmaxf(m, fabsf(xr[j]));
#pragma unroll
    for (unsigned offset = kWave / 2; offset > 0; offset >>= 1) m = fmaxf(m, __shfl_xor(m, offset));
    const float s = m == 0.0f ? 1.0f : m / 127.0f;
    if (lane == 0) scale[row] = s;
    std::int8_t* qr = q + std::size_t(row) * features;
    for (unsigned j = lane; j < features; j += kWave) {
        const int v = __float2int_rn(xr[j] / s);
        qr[Packed ? packedOffset(j) : j] = std::int8_t(v < -127 ? -127 : (v > 127 ? 127 : v));
    }
}

// Vector paths for features % 4 == 0 with 16-byte aligned rows. Same arithmetic as quantizeRows
// (IEEE divide, round half to even, clamp).
__device__ __forceinline__ int quantizeOne(float v, float s) {
    const int r = __float2int_rn(v / s);
    return r < -127 ? -127 : (r > 127 ? 127 : r);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned quantizeGroup(f32x4 v, float s) {
    return (unsigned(quantizeOne(v.x, s)) & 0xFFu) | (unsigned(quantizeOne(v.y, s)) & 0xFFu) << 8 |
           (unsigned(quantizeOne(v.z, s)) & 0xFFu) << 16 | (unsigned(quantizeOne(v.w, s)) & 0xFFu) << 24;
}

// The packed16 dword of lane `lane` from the quantized dwords of its 16-feature tile, held by the
// tile's four lanes (w0..w3 = features 0-3, 4-7, 8-11, 12-15): output dword i is bytes
// [q(2i), q(2i+8), q(2i+1), q(2i+9)], i.e. two bytes of w(i/2) and two of w(i/2 + 2). All four lanes
// of the tile must execute this together.
__device__ __forceinline__ unsigned packDword(unsigned qd, unsigned lane) {
    const unsigned lo = unsigned(__builtin_amdgcn_mov_dpp(int(qd), 0x50, 0xF, 0xF, false)); // quad [0,0,1,1]
    const unsigned hi = unsigned(__builtin_amdgcn_mov_dpp(int(qd), 0xFA, 0xF, 0xF, false)); // quad [2,2,3,3]
    // v_perm_b32 selectors: bytes 0-3 pick from the second operand, 4-7 from the first.
    return __builtin_amdgcn_perm(hi, lo, (lane & 1u) ? 0x07030602u : 0x05010400u);
}

__device__ __forceinline__ float absMax(f32x4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Rows of at most 64 groups of 4 features (F <= 256): `Lanes` (a power of two >= groups) lanes per
// row, each holding one group; a thread handles kQuantRows rows kRowsPerPass apart, issuing all of
// its 16-byte loads before the reductions, so a wave keeps 4 KiB of X in flight and reads X once.
// X is streamed with nontemporal loads and q with nontemporal stores (neither is re-read here).
constexpr unsigned kQuantRows = 4;

template <unsigned Lanes, bool Packed>
__global__ __launch_bounds__(256) void quantizeRowsFit(const f32x4* __restrict__ x,
                                                        unsigned* __restrict__ q,
                                                        float* __restrict__ scale,
                                                        unsigned sources, unsigned groups) {
    constexpr unsigned kRowsPerPass = 256 / Lanes;
    const unsigned lane = threadIdx.x & (Lanes - 1);
    const std::size_t row0 = std::size_t(blockIdx.x) * kRowsPerPass * kQuantRows + threadIdx.x / Lanes;
    f32x4 v[kQuantRows];
    float m[kQuantRows];
#pragma unroll
    for (unsigned r = 0; r < kQuantRows; ++r) {
        const std::size_t row = row0 + r * kRowsPerPass;
        const bool live = row < sources && lane < groups;
        v[r] = __builtin_nontemporal_load(x + (live ? row * groups + lane : 0));
        if (!live) v[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        m[r] = absMax(v[r]);
    }
#pragma unroll
    for (unsigned offset = Lanes / 2; offset > 0; offset >>= 1)
#pragma unroll
        for (unsigned r = 0; r < kQuantRows; ++r) m[r] = fmaxf(m[r], __shfl_xor(m[r], offset));
#pragma unroll
    for (unsigned r = 0; r < kQuantRows; ++r) {
        const std::size_t row = row0 + r * kRowsPerPass;
        if (row >= sources) break;
        const float s = m[r] == 0.0f ? 1.0f : m[r] / 127.0f;
        if (lane == 0) scale[row] = s;
        unsigned qd = quantizeGroup(v[r], s);
        if constexpr (Packed) qd = packDword(qd, lane); // the row's tiles are whole lane quads
        if (lane < groups) __builtin_nontemporal_store(qd, q + row * groups + lane);
    }
}

// Rows of more than 64 groups: one wave per row, looping over the groups twice (maximum, then
// quantize; the second read of the row hits L2).
template <bool Packed>
__global__ __launch_bounds__(256) void quantizeRowsLong(const f32x4* __restrict__ x,
                                                         unsigned* __restrict__ q,
                                                         float* __restrict__ scale,
                                                         unsigned sources, unsigned groups) {
    const unsigned lane = threadIdx.x & (kWave - 1);
    const std::size_t row = (std::size_t(blockIdx.x) * 256 + threadIdx.x) / kWave;
    if (row >= sources) return;
    const f32x4* xr = x + row * groups;
    float m = 0.0f;
    for (unsigned j = lane; j < groups; j += kWave) m = fmaxf(m, absMax(xr[j]));
#pragma unroll
    for (unsigned offset = kWave / 2; offset > 0; offset >>= 1) m = fmaxf(m, __shfl_xor(m, offset));
    const float s = m == 0.0f ? 1.0f : m / 127.0f;
    if (lane == 0) scale[row] = s;
    unsigned* qr = q + row * groups;
    for (unsigned j = lane; j < groups; j += kWave) {
        unsigned qd = quantizeGroup(xr[j], s);
        if constexpr (Packed) qd = packDword(qd, lane); // groups % 4 == 0: whole quads
        qr[j] = qd;
    }
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// One thread per 16-byte tile; q is read once and packed written once, so both use nontemporal
// access (measured on c3: 6.5 TB/s against 6.0 with the default policy).
__global__ __launch_bounds__(256) void packTiles(const u32x4* __restrict__ q,
                                                 u32x4* __restrict__ out, std::size_t tiles) {
    const std::size_t t = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= tiles) return;
    const u32x4 w = __builtin_nontemporal_load(q + t);
    // v_perm_b32 selectors: bytes 0-3 pick from the second operand, 4-7 from the first.
    u32x4 r;
    r.x = __builtin_amdgcn_perm(w.z, w.x, 0x05010400u); // q0  q8  q1  q9
    r.y = __builtin_amdgcn_perm(w.z, w.x, 0x07030602u); // q2  q10 q3  q11
    r.z = __builtin_amdgcn_perm(w.w, w.y, 0x05010400u); // q4  q12 q5  q13
    r.w = __builtin_amdgcn_perm(w.w, w.y, 0x07030602u); // q6  q14 q7  q15
    __builtin_nontemporal_store(r, out + t);
}

__global__ __launch_bounds__(256) void packPairs(const std::uint8_t* __restrict__ q,
                                                 unsigned short* __restrict__ out,
                                                 std::size_t pairs) {
    const std::size_t p = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= pairs) return;
    const std::size_t o = (p >> 3) * 16 + (p & 7);
    out[p] = static_cast<unsigned short>(q[o] | (unsigned(q[o + 8]) << 8));
}

} // namespace

namespace {

// The quantize kernels for one call: the vector kernels for 16-byte aligned rows of features % 4 ==
// 0 with a 4-byte aligned output, the scalar kernel otherwise. `Packed` writes the packed16 layout
// (features % 16 == 0, checked by the caller).
template <bool Packed>
void launchQuantize(const float* x, std::int8_t* out, float* scale, std::uint32_t sources,
                    std::uint32_t features, hipStream_t stream) {
    const bool vector = features % 4 == 0 && reinterpret_cast<std::uintptr_t>(x) % 16 == 0 &&
                        reinterpret_cast<std::uintptr_t>(out) % 4 == 0;
    if (vector) {
        const unsigned groups = features / 4;
        const auto* xv = reinterpret_cast<const f32x4*>(x);
        auto* qv = reinterpret_cast<unsigned*>(out);
        if (groups > kWave) {
            const unsigned blocks = unsigned((std::size_t(sources) * kWave + 255) / 256);
            hipLaunchKernelGGL(quantizeRowsLong<Packed>, dim3(blocks), dim3(256), 0, stream, xv, qv,
                               scale, sources, groups);
        } else {
            unsigned lanes = 1;
            while (lanes < groups) lanes *= 2;
            const std::size_t rowsPerBlock = std::size_t(256 / lanes) * kQuantRows;
            const unsigned blocks = unsigned((sources + rowsPerBlock - 1) / rowsPerBlock);
            switch (lanes) {
#define TCC_QUANT_CASE(L)                                                                          \
    case L:                                                                                        \
        hipLaunchKernelGGL((quantizeRowsFit<L, Packed>), dim3(blocks), dim3(256), 0, stream, xv,   \
                           qv, scale, sources, groups);                                            \
        break;
                TCC_QUANT_CASE(1) TCC_QUANT_CASE(2) TCC_QUANT_CASE(4) TCC_QUANT_CASE(8)
                TCC_QUANT_CASE(16) TCC_QUANT_CASE(32) TCC_QUANT_CASE(64)
#undef TCC_QUANT_CASE
            }
        }
    } else {
        const unsigned blocks = unsigned((std::size_t(sources) + kRowsPerBlock - 1) / kRowsPerBlock);
        hipLaunchKernelGGL(quantizeRows<Packed>, dim3(blocks), dim3(kWave * kRowsPerBlock), 0,
                           stream, x, out, scale, sources, features);
    }
    checkHip(hipGetLastError());
}

} // namespace

void quantizeFeaturesInt8(const float* x, std::int8_t* q, float* scale, std::uint32_t sources,
                          std::uint32_t features, hipStream_t stream) {
    // A zero-sized grid is a launch error, reported like the runtime would (std::runtime_error).
    if (!sources || !features) throw std::runtime_error("quantize: invalid configuration argument");
    // A null buffer would fault the GPU; rejected before any launch (the reference does not check).
    if (!x || !q || !scale) throw std::invalid_argument("quantize: null device buffer");
    launchQuantize<false>(x, q, scale, sources, features, stream);
}

void quantizePackFeaturesInt8(const float* x, std::int8_t* packed, float* scale,
                              std::uint32_t sources, std::uint32_t features, hipStream_t stream) {
    if (!sources || !features) throw std::runtime_error("quantize: invalid configuration argument");
    if (features % 16) throw std::invalid_argument("packed16 needs features % 16 == 0");
    if (!x || !packed || !scale) throw std::invalid_argument("quantize-pack: null device buffer");
    launchQuantize<true>(x, packed, scale, sources, features, stream);
}

void packFeaturesInt8x16(const std::int8_t* q, std::int8_t* packed, std::uint32_t sources,
                         std::uint32_t features, hipStream_t stream) {
    if (!sources || !features) throw std::runtime_error("pack: invalid configuration argument");
    if (features % 16) throw std::invalid_argument("packed16 needs features % 16 == 0");
    if (!q || !packed) throw std::invalid_argument("pack: null device buffer");
    const std::size_t bytes = std::size_t(sources) * features;
    const bool aligned = (reinterpret_cast<std::uintptr_t>(q) % 16 == 0) &&
                         (reinterpret_cast<std::uintptr_t>(packed) % 16 == 0);
    if (aligned) {
        const std::size_t tiles = bytes / 16;
        const std::size_t blocks = (tiles + 255) / 256;
        hipLaunchKernelGGL(packTiles, dim3(unsigned(blocks)), dim3(256), 0, stream,
                           reinterpret_cast<const u32x4*>(q), reinterpret_cast<u32x4*>(packed),
                           tiles);
    } else {
        const std::size_t pairs = bytes / 2;
        const std::size_t blocks = (pairs + 255) / 256;
        hipLaunchKernelGGL(packPairs, dim3(unsigned(blocks)), dim3(256), 0, stream,
                           reinterpret_cast<const std::uint8_t*>(q),
                           reinterpret_cast<unsigned short*>(packed), pairs);
    }
    checkHip(hipGetLastError());
}
