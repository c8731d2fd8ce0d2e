/*
 * tcc_oracle.h — CPU restatement of the TCC-SpMM hot path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this.
 * It is the checker, never the product: the library under tcc_spmm_amd/ never links it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference checkout of Shixg-cnic/tcc_spmm).
 */
#ifndef TCC_ORACLE_H
#define TCC_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes shared with the product C-ABI: 0 ok, 1 invalid argument, 2 overflow, 4 out of memory. */
#define ORC_OK 0
#define ORC_INVALID 1
#define ORC_OVERFLOW 2
#define ORC_NOMEM 4

typedef struct {
    uint32_t sw, begin, end, partial, mask, chunks, reduceFirst;
} orc_task; /* include/format/sw32.h:13-15 */

typedef struct {
    uint32_t begin, end;
} orc_reduce; /* include/format/sw32.h:16-18 */

typedef struct {
    uint32_t rows, cols;
    uint32_t* windowOffsets; size_t nWindowOffsets;
    uint32_t* sourceIds;     size_t nSlots;          /* sourceIds and sourceMetadata share nSlots */
    uint64_t* sourceMetadata;
    uint32_t* rowGroupMasks; size_t nPanels;
    float* values;           size_t nValues;
    uint32_t* bucketOffsets; size_t nBucketOffsets;
    orc_task* tasks;         size_t nTasks;
    orc_reduce* reductions;  size_t nReductions;
    uint32_t* partialIds;    size_t nPartialIds;
    uint32_t partialCount;
} orc_sw32; /* include/format/sw32.h:22-39 */

/* Canonical CSR (src/format/csr.cpp:6-40). Output arrays are caller-allocated with room for
 * rows+1 offsets and nnz entries; *outNnz receives the canonical entry count. */
int orc_canonical_csr(uint32_t rows, uint32_t cols, uint32_t nnz, const uint32_t* rowOffsets,
                      const uint32_t* sourceIds, const float* values, uint32_t* outOffsets,
                      uint32_t* outSources, float* outValues, uint32_t* outNnz);

/* SW32 conversion + task plan (src/format/sw32.cpp:69-167, :25-65). */
int orc_sw32_convert(uint32_t rows, uint32_t cols, const uint32_t* rowOffsets,
                     const uint32_t* sourceIds, const float* values, int bucketByRwMask,
                     orc_sw32* out);
void orc_sw32_free(orc_sw32* f);

/* Quantize per source row (src/format/int8_quantize.cu:4-25). */
void orc_quantize(const float* x, int8_t* q, float* scale, uint32_t sources, uint32_t features);
/* packed16 byte permutation (src/format/pack_int8.cu:6-15). */
void orc_pack16(const int8_t* q, int8_t* packed, uint32_t sources, uint32_t features);
/* Inverse of orc_pack16, used by the SpMM restatements to read packed X. */
void orc_unpack16(const int8_t* packed, int8_t* q, uint32_t sources, uint32_t features);
/* TF32 round-to-nearest, ties away from zero (PTX cvt.rna.tf32.f32 as used at
 * src/kernel/spmm_kernel.cuh:7-11). */
float orc_tf32(float v);

/* Y[r][f] = sum over nonzeros of tf32(a) * tf32(fp32(q*scale)), accumulated in double, read from the
 * plain canonical CSR (definition of the operator, src/kernel/spmm_kernel.cuh:26-90). */
void orc_spmm_csr_f64(uint32_t rows, const uint32_t* rowOffsets, const uint32_t* sourceIds,
                      const float* values, const int8_t* packedX, const float* scales,
                      uint32_t cols, uint32_t features, double* y);

/* The same sum read through the SW32 slot stream (slots, row masks, value bases), in double. */
void orc_spmm_sw32_f64(const orc_sw32* f, const int8_t* packedX, const float* scales,
                       uint32_t features, double* y);

/* As orc_spmm_sw32_f64 but only for the listed SWs: y has n*32 rows (rows past the matrix end stay
 * 0), with optional sum |terms| (below). */
void orc_spmm_sw32_f64_windows(const orc_sw32* f, const int8_t* packedX, const float* scales,
                               uint32_t features, const uint32_t* windows, uint32_t n, double* y,
                               double* yabs);
/* yabs (optional, same shape as y) receives sum |tf32(a) * xhat| per element: the scale of the FP32
 * summation error of any accumulation order (error <~ u * sum|terms| for a random walk). */

/* Full-size comparison of a computed Y [rows][features] (float) against the double reference of
 * orc_spmm_sw32_f64_windows, SW by SW on `threads` threads, without materialising the reference.
 * An element passes when |y - ref| <= atol + rtol |ref| + cond * 2^-24 * sum|terms| (cond = 0: the
 * plain bound). ref (optional, [rows][features] double) receives the reference itself. */
typedef struct {
    uint64_t checked;  /* elements compared */
    uint64_t bad;      /* elements beyond the bound */
    uint64_t relaxed;  /* elements within the bound only thanks to the cond term */
    double maxErr;     /* max |y - ref| (NaN in y counts as +inf) */
    uint64_t firstBad; /* flat index of the smallest bad element, UINT64_MAX when none */
    double firstGot, firstWant, firstBound;
} orc_check_stats;
int orc_check_sw32_mt(const orc_sw32* f, const int8_t* packedX, const float* scales,
                      uint32_t features, const float* y, double atol, double rtol, double cond,
                      int threads, orc_check_stats* out, double* ref);

/* Restatement of the kernel's task/partial/merge protocol in FP32 (spmm_kernel.cuh:228-282):
 * each task accumulates its panels in FP32 (slot order), unsplit tasks write Y, split tasks write
 * partial tiles [K][8][F], and the merge sums partial tiles in partialIds order starting at 0. */
void orc_spmm_tasks_f32(const orc_sw32* f, const int8_t* packedX, const float* scales,
                        uint32_t features, float* partials, float* y);

/* CPU baseline: FP32 SpMM over the SW32 stream, threads split the SW range. Returns threads used.
 * swBegin/swEnd bound the SW range (a bounded sample of the full workload). */
int orc_spmm_sw32_f32_mt(const orc_sw32* f, const int8_t* packedX, const float* scales,
                         uint32_t features, uint32_t swBegin, uint32_t swEnd, int threads,
                         float* y);
/* The same with vector = 0 (scalar, portable C) or 1 (AVX2 + FMA: bitwise the same Y; returns -1
 * when the CPU lacks them or features % 16 != 0, -2 when a worker ran out of memory). */
int orc_spmm_sw32_f32_mt_path(const orc_sw32* f, const int8_t* packedX, const float* scales,
                              uint32_t features, uint32_t swBegin, uint32_t swEnd, int threads,
                              float* y, int vector);
int orc_cpu_has_avx2(void);

#ifdef __cplusplus
}
#endif
#endif
