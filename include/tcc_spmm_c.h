/*
 * tcc_spmm_c.h — C ABI of libtcc_spmm.so (plain pointers and sizes, no C++ or torch types).
 *
 * The reference exports a C++ API only (a static libtcc_spmm.a). This header is the flat binding a
 * ctypes / cgo / JNI / N-API caller would use; every entry point wraps the C++ function named in
 * its comment, whose reference declaration is cited. All functions return a status code and never
 * throw: 0 success, 1 std::invalid_argument, 2 std::overflow_error, 3 std::runtime_error (HIP
 * failure or I/O), 4 any other exception. tcc_last_error() returns the message of the last failure
 * on the calling thread. A null handle, output pointer or host input array (one with a nonzero
 * count) returns 1 before any work. Device entry points are asynchronous on `stream` (a hipStream_t;
 * NULL is the null stream), like the C++ functions they wrap.
 */
#ifndef TCC_SPMM_C_H
#define TCC_SPMM_C_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TCC_OK = 0, TCC_INVALID_ARGUMENT = 1, TCC_OVERFLOW = 2, TCC_RUNTIME = 3, TCC_OTHER = 4 };

typedef struct tcc_csr tcc_csr;   /* owns a CsrMatrix (include/format/csr.h) */
typedef struct tcc_sw32 tcc_sw32; /* owns a Sw32HostFormat (include/format/sw32.h) */
typedef struct tcc_device_matrix tcc_device_matrix; /* owns uploaded arrays + workspace */

/* Byte-for-byte the layout of Sw32DeviceView (reference include/format/sw32.h:47-56). */
typedef struct {
    const uint32_t* windowOffsets;
    const uint32_t* sourceIds;
    const uint32_t* rowGroupMasks;
    const uint64_t* sourceMetadata;
    const float* values;
    const uint32_t* bucketOffsets;
    const void* tasks;      /* Sw32Task[taskCount], 28 bytes each */
    const void* reductions; /* Sw32ReduceRange[], 8 bytes each */
    const uint32_t* partialIds;
    uint32_t taskCount;
} tcc_device_view;

/* Element counts of every Sw32HostFormat array (reference include/format/sw32.h:22-39). */
typedef struct {
    uint32_t rows, cols, partialCount, bucketed;
    uint64_t windowOffsets, sourceIds, rowGroupMasks, sourceMetadata, values, bucketOffsets, tasks,
        reductions, partialIds;
} tcc_sw32_sizes;

/* Host pointers into a tcc_sw32 (valid until it is freed or re-planned). */
typedef struct {
    const uint32_t* windowOffsets;
    const uint32_t* sourceIds;
    const uint32_t* rowGroupMasks;
    const uint64_t* sourceMetadata;
    const float* values;
    const uint32_t* bucketOffsets;
    const void* tasks;
    const void* reductions;
    const uint32_t* partialIds;
} tcc_sw32_arrays;

const char* tcc_last_error(void);
/* Library version string, e.g. "tcc_spmm_amd 0.1 gfx950". */
const char* tcc_version(void);

/* ---- host format (CPU) ---- */
/* makeCanonicalCsr — reference include/format/csr.h:23-25 (src/format/csr.cpp:6-40). */
int tcc_make_canonical_csr(uint32_t rows, uint32_t cols, uint32_t nnz, const uint32_t* rowOffsets,
                           const uint32_t* sourceIds, const float* values, tcc_csr** out);
/* loadMatrixMarket — reference include/format/csr.h:18 (src/format/matrix_market.cpp:30-103). */
int tcc_load_matrix_market(const char* path, uint32_t* rows, uint32_t* cols, tcc_csr** out);
/* Wrap raw arrays into a CsrMatrix WITHOUT canonicalisation — in the reference CsrMatrix is a plain
 * struct (include/format/csr.h:7-10) that callers may fill directly; convertCsrToSw32 then
 * validates it. rowOffsets has rowOffsetsCount entries, sourceIds/values have nnz. */
int tcc_csr_from_arrays(uint64_t rowOffsetsCount, const uint32_t* rowOffsets, uint64_t nnz,
                        const uint32_t* sourceIds, const float* values, tcc_csr** out);
/* Sizes and host pointers of a CsrMatrix (rowOffsets has rows + 1 entries). */
int tcc_csr_info(const tcc_csr* csr, uint64_t* rowOffsetsCount, uint64_t* nnz);
int tcc_csr_arrays(const tcc_csr* csr, const uint32_t** rowOffsets, const uint32_t** sourceIds,
                   const float** values);
void tcc_csr_free(tcc_csr* csr);

/* convertCsrToSw32 — reference include/format/sw32.h:43-44 (src/format/sw32.cpp:69-167). */
int tcc_convert_csr_to_sw32(uint32_t rows, uint32_t cols, const tcc_csr* csr, int bucketByRwMask,
                            tcc_sw32** out);
/* buildPanelTasks — reference src/format/sw32.cpp:25-65 (internal there, exported here). */
int tcc_build_panel_tasks(tcc_sw32* format);
int tcc_sw32_get_sizes(const tcc_sw32* format, tcc_sw32_sizes* sizes);
int tcc_sw32_get_arrays(const tcc_sw32* format, tcc_sw32_arrays* arrays);
void tcc_sw32_free(tcc_sw32* format);

/* ---- device (HIP) ---- */
/* launchSpmmInt8 — reference include/spmm.cuh:21-23 (src/kernel/spmm.cu:17-31). `partials` and
 * `counters` are the two members of SpmmWorkspace (reference include/spmm.cuh:10-13). */
int tcc_launch_spmm_int8(const tcc_device_view* matrix, const int8_t* packedX, const float* scales,
                         float* output, uint32_t rows, uint32_t cols, uint32_t features,
                         float* partials, uint32_t* counters, void* stream);
/* launchSpmmInt8NoAlloc (include/spmm.h) — no counterpart in the reference. For callers that cannot
 * allocate (HIP graph capture, serving loops): the split-SW workspace lives in a library-owned
 * static device array of kNoAllocScratchBytes (64 MiB) per GPU, and the call allocates nothing.
 * partialCount is the plan's Sw32HostFormat::partialCount; a plan whose workspace does not fit
 * returns TCC_INVALID_ARGUMENT before any launch. Calls that overlap on one GPU race. */
int tcc_launch_spmm_int8_noalloc(const tcc_device_view* matrix, const int8_t* packedX,
                                 const float* scales, float* output, uint32_t rows, uint32_t cols,
                                 uint32_t features, uint32_t partialCount, void* stream);
/* setSpmmLaunchOverrides (include/spmm.h) — no counterpart in the reference: forces the task form
 * (taskWaves 0 automatic, 1 or 2) and the 64-bit-addressing instance (forceWide) of later launches,
 * for tests and measurements. Process-wide. */
int tcc_set_spmm_launch_overrides(uint32_t taskWaves, int forceWide);
/* quantizeFeaturesInt8 — reference include/format/int8_features.cuh:9-10. */
int tcc_quantize_features_int8(const float* x, int8_t* q, float* scale, uint32_t sources,
                               uint32_t features, void* stream);
/* packFeaturesInt8x16 — reference include/format/int8_features.cuh:14-15. */
int tcc_pack_features_int8x16(const int8_t* q, int8_t* packed, uint32_t sources, uint32_t features,
                              void* stream);
/* quantizePackFeaturesInt8 (include/format/int8_features.h) — no counterpart in the reference: the
 * two calls above in one pass, bit-identical output, for callers that quantize X for every SpMM. */
int tcc_quantize_pack_features_int8(const float* x, int8_t* packed, float* scale, uint32_t sources,
                                    uint32_t features, void* stream);

/* DeviceMatrix — reference src/device_matrix.cuh:8-37: uploads every array of a bucketed format,
 * allocates partials (partialCount*8*features floats) and counters (nSW*(features/128) uint32,
 * zeroed) when partialCount > 0, and hands out the view and the workspace. */
int tcc_device_matrix_create(const tcc_sw32* format, uint32_t features, tcc_device_matrix** out);
int tcc_device_matrix_view(const tcc_device_matrix* m, tcc_device_view* view, float** partials,
                           uint32_t** counters);
void tcc_device_matrix_free(tcc_device_matrix* m);

/* ---- synthetic workloads (no reference counterpart: the reference reads .mtx files) ----
 * Deterministic generators for the benchmark configurations, independent of thread count.
 * tcc_synth_csr writes a canonical CSR for config "c1".."c5" (the shapes are documented in
 * tcc_spmm_amd/csrc/synth/generators.cpp); "t<rows>_<deg>_<seed>" gives a small uniform test
 * matrix. */
int tcc_synth_csr(const char* config, uint32_t* rows, uint32_t* cols, tcc_csr** out);
/* N(0, stddev^2) features (Box-Muller on SplitMix64); rows whose hash falls below outlierFraction
 * are multiplied by outlierScale. */
int tcc_synth_features(uint32_t sources, uint32_t features, uint64_t seed, float stddev,
                       float outlierFraction, float outlierScale, float* out);

#ifdef __cplusplus
}
#endif
#endif
