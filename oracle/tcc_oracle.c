/*
 * tcc_oracle.c — CPU restatement of the TCC-SpMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg are
 * the only callers. The product library (tcc_spmm_amd/) never links or loads this file.
 *
 * Pinning (what fixes each function independently of this restatement):
 *   orc_canonical_csr  -> byte-identical to the reference's own makeCanonicalCsr compiled from
 *                         /root/reference/src/format/csr.cpp (oracle/_ref, tests/golden fixtures).
 *   orc_sw32_convert   -> byte-identical to the reference's convertCsrToSw32 (+ its internal
 *                         buildPanelTasks) compiled from /root/reference/src/format/sw32.cpp.
 *   orc_quantize       -> numpy float32 division + round-half-even (independent IEEE code path),
 *                         closed-form special cases (zero row -> scale 1, extremes -> +-127).
 *   orc_pack16         -> closed-form byte permutation + unpack(pack(q)) == q.
 *   orc_tf32           -> known-answer bit patterns written from the rounding definition.
 *   orc_spmm_*         -> brute-force dense products on tiny inputs (numpy), CSR vs SW32 agreement,
 *                         split vs unsplit agreement.
 *   orc_check_sw32_mt  -> its reference equals orc_spmm_sw32_f64_windows bitwise and the dense
 *                         brute force; planted errors (beyond the bound, NaN, within the bound,
 *                         within only the conditioning term) are flagged exactly.
 */
#include "tcc_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* sw32BucketOrder, include/format/sw32.h:9-10 (a format constant; identical by necessity). */
static const unsigned kBucketOrder[16] = {0, 1, 2, 4, 8, 3, 5, 6, 7, 9, 10, 11, 12, 13, 14, 15};
/* sw32TaskPanelLimit, include/format/sw32.h:12 */
static const uint32_t kPanelLimit = 384;

/* ---------------------------------------------------------------- growable arrays */
typedef struct {
    void* p;
    size_t n, cap, elem;
} vec_t;

static int vec_push(vec_t* v, const void* item) {
    if (v->n == v->cap) {
        size_t nc = v->cap ? v->cap * 2 : 64;
        void* np = realloc(v->p, nc * v->elem);
        if (!np) return ORC_NOMEM;
        v->p = np;
        v->cap = nc;
    }
    memcpy((char*)v->p + v->n * v->elem, item, v->elem);
    v->n++;
    return ORC_OK;
}

/* ---------------------------------------------------------------- canonical CSR */
typedef struct {
    uint32_t col;
    float val;
} entry_t;

/* Stable merge sort by column (the reference uses std::stable_sort, src/format/csr.cpp:22-23). */
static void merge_sort_entries(entry_t* a, entry_t* tmp, size_t n) {
    if (n < 2) return;
    size_t h = n / 2;
    merge_sort_entries(a, tmp, h);
    merge_sort_entries(a + h, tmp, n - h);
    size_t i = 0, j = h, k = 0;
    while (i < h && j < n) tmp[k++] = (a[j].col < a[i].col) ? a[j++] : a[i++];
    while (i < h) tmp[k++] = a[i++];
    while (j < n) tmp[k++] = a[j++];
    memcpy(a, tmp, n * sizeof(entry_t));
}

/* src/format/csr.cpp:6-40 */
int orc_canonical_csr(uint32_t rows, uint32_t cols, uint32_t nnz, const uint32_t* rowOffsets,
                      const uint32_t* sourceIds, const float* values, uint32_t* outOffsets,
                      uint32_t* outSources, float* outValues, uint32_t* outNnz) {
    if (!rows || !cols || rowOffsets[0] || rowOffsets[rows] != nnz) return ORC_INVALID; /* :9-10 */
    for (uint32_t r = 0; r < rows; ++r)                                                  /* :11-13 */
        if (rowOffsets[r] > rowOffsets[r + 1] || rowOffsets[r + 1] > nnz) return ORC_INVALID;
    entry_t* buf = (entry_t*)malloc((nnz ? nnz : 1) * sizeof(entry_t));
    entry_t* tmp = (entry_t*)malloc((nnz ? nnz : 1) * sizeof(entry_t));
    if (!buf || !tmp) {
        free(buf);
        free(tmp);
        return ORC_NOMEM;
    }
    uint32_t out = 0;
    outOffsets[0] = 0;
    int status = ORC_OK;
    for (uint32_t r = 0; r < rows && status == ORC_OK; ++r) {
        uint32_t b = rowOffsets[r], e = rowOffsets[r + 1], n = e - b;
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t c = sourceIds[b + i];
            float v = values[b + i];
            if (c >= cols || !isfinite(v)) { /* :17-19 */
                status = ORC_INVALID;
                break;
            }
            buf[i].col = c;
            buf[i].val = v;
        }
        if (status != ORC_OK) break;
        merge_sort_entries(buf, tmp, n);
        for (uint32_t i = 0; i < n;) { /* :24-36 coalesce duplicates in stable order */
            uint32_t c = buf[i].col;
            float sum = 0.0f;
            do {
                sum += buf[i++].val;
            } while (i < n && buf[i].col == c);
            if (!isfinite(sum)) {
                status = ORC_INVALID;
                break;
            }
            if (sum != 0.0f) {
                outSources[out] = c;
                outValues[out] = sum;
                ++out;
            }
        }
        outOffsets[r + 1] = out;
    }
    free(buf);
    free(tmp);
    if (status == ORC_OK) *outNnz = out;
    return status;
}

/* ---------------------------------------------------------------- SW32 conversion */
typedef struct {
    uint32_t source, row;
    float value;
} triple_t;

static int triple_cmp(const void* pa, const void* pb) {
    const triple_t* a = (const triple_t*)pa;
    const triple_t* b = (const triple_t*)pb;
    if (a->source != b->source) return a->source < b->source ? -1 : 1;
    if (a->row != b->row) return a->row < b->row ? -1 : 1;
    return 0;
}

typedef struct {
    uint32_t source, mask, offset; /* offset into the SW's value list (source-major) */
} item_t;

static unsigned rw_mask_of(uint32_t mask32) {
    return (unsigned)((mask32 & 0xffu) != 0) | ((unsigned)((mask32 & 0xff00u) != 0) << 1) |
           ((unsigned)((mask32 & 0xff0000u) != 0) << 2) |
           ((unsigned)((mask32 & 0xff000000u) != 0) << 3);
}

void orc_sw32_free(orc_sw32* f) {
    free(f->windowOffsets);
    free(f->sourceIds);
    free(f->sourceMetadata);
    free(f->rowGroupMasks);
    free(f->values);
    free(f->bucketOffsets);
    free(f->tasks);
    free(f->reductions);
    free(f->partialIds);
    memset(f, 0, sizeof(*f));
}

#define CHECK32(n)                                                                               \
    do {                                                                                         \
        if ((uint64_t)(n) > 0xFFFFFFFFull) {                                                     \
            status = ORC_OVERFLOW;                                                               \
            goto done;                                                                           \
        }                                                                                        \
    } while (0)

/* buildPanelTasks, src/format/sw32.cpp:25-65 */
static int build_tasks(orc_sw32* f, vec_t* tasks, vec_t* reds, vec_t* pids) {
    int status = ORC_OK;
    uint32_t windows = (uint32_t)(f->nWindowOffsets - 1);
    uint64_t parts = 0;
    vec_t rw[4];
    for (int i = 0; i < 4; ++i) rw[i] = (vec_t){0, 0, 0, sizeof(uint32_t)};
    for (uint32_t sw = 0; sw < windows; ++sw) {
        uint32_t begin = f->windowOffsets[sw], end = f->windowOffsets[sw + 1];
        uint32_t count = end - begin;
        if (count <= kPanelLimit) { /* :33-35 — includes empty SWs */
            orc_task t = {sw, begin, end, 0xFFFFFFFFu, 15, 1, 0};
            if ((status = vec_push(tasks, &t))) goto done;
            continue;
        }
        for (int i = 0; i < 4; ++i) rw[i].n = 0;
        uint32_t chunks = 1 + (count - 1) / kPanelLimit; /* :39 */
        CHECK32(reds->n);
        uint32_t reduceFirst = (uint32_t)reds->n;
        for (uint32_t panel = begin; panel < end;) { /* :41-55 */
            uint32_t rem = end - panel;
            uint32_t panelEnd = panel + (rem < kPanelLimit ? rem : kPanelLimit);
            uint32_t mask = 0;
            for (unsigned slot = 1; slot < 16; ++slot) {
                size_t first = (size_t)sw * 17 + slot;
                uint32_t lo = f->bucketOffsets[first], hi = f->bucketOffsets[first + 1];
                uint32_t a = panel > lo ? panel : lo;
                uint32_t b = panelEnd < hi ? panelEnd : hi;
                if (a < b) mask |= kBucketOrder[slot];
            }
            CHECK32(parts);
            orc_task t = {sw, panel, panelEnd, (uint32_t)parts, mask, chunks, reduceFirst};
            if ((status = vec_push(tasks, &t))) goto done;
            for (unsigned r = 0; r < 4; ++r)
                if (mask & (1u << r)) {
                    CHECK32(parts);
                    uint32_t id = (uint32_t)parts++;
                    if ((status = vec_push(&rw[r], &id))) goto done;
                }
            panel = panelEnd;
        }
        for (unsigned r = 0; r < 4; ++r) { /* :56-60 — always four ranges per split SW */
            CHECK32(pids->n);
            uint32_t first = (uint32_t)pids->n;
            for (size_t i = 0; i < rw[r].n; ++i)
                if ((status = vec_push(pids, (uint32_t*)rw[r].p + i))) goto done;
            CHECK32(pids->n);
            orc_reduce rr = {first, (uint32_t)pids->n};
            if ((status = vec_push(reds, &rr))) goto done;
        }
    }
    CHECK32(tasks->n);
    CHECK32(reds->n);
    CHECK32(parts);
    f->partialCount = (uint32_t)parts;
done:
    for (int i = 0; i < 4; ++i) free(rw[i].p);
    return status;
}

/* convertCsrToSw32, src/format/sw32.cpp:69-167 */
int orc_sw32_convert(uint32_t rows, uint32_t cols, const uint32_t* rowOffsets,
                     const uint32_t* sourceIds, const float* values, int bucketByRwMask,
                     orc_sw32* out) {
    memset(out, 0, sizeof(*out));
    if (!rows || !cols || rowOffsets[0] != 0) return ORC_INVALID; /* :71-74 */
    for (uint32_t r = 0; r < rows; ++r)                            /* :75-77 */
        if (rowOffsets[r] > rowOffsets[r + 1]) return ORC_INVALID;
    int status = ORC_OK;
    vec_t wo = {0, 0, 0, 4}, sid = {0, 0, 0, 4}, meta = {0, 0, 0, 8}, rgm = {0, 0, 0, 4};
    vec_t vals = {0, 0, 0, 4}, bo = {0, 0, 0, 4};
    vec_t tasks = {0, 0, 0, sizeof(orc_task)}, reds = {0, 0, 0, sizeof(orc_reduce)};
    vec_t pids = {0, 0, 0, 4};
    vec_t buckets[16];
    for (int i = 0; i < 16; ++i) buckets[i] = (vec_t){0, 0, 0, sizeof(item_t)};
    triple_t* trip = NULL;
    float* wvals = NULL;
    size_t tripCap = 0;
    uint32_t zero = 0;
    if ((status = vec_push(&wo, &zero))) goto done;
    for (uint64_t base = 0; base < rows; base += 32) {
        uint32_t count = (uint32_t)((rows - base) < 32 ? (rows - base) : 32);
        size_t total = (size_t)rowOffsets[base + count] - rowOffsets[base];
        if (total > tripCap) {
            free(trip);
            free(wvals);
            tripCap = total;
            trip = (triple_t*)malloc(tripCap * sizeof(triple_t));
            wvals = (float*)malloc(tripCap * sizeof(float));
            if (!trip || !wvals) {
                status = ORC_NOMEM;
                goto done;
            }
        }
        /* Gather the SW's (source, row, value) triples and validate the per-row contract the
         * reference enforces while merging (:104-120). */
        size_t n = 0;
        for (uint32_t r = 0; r < count; ++r) {
            uint32_t row = (uint32_t)base + r;
            for (uint32_t p = rowOffsets[row]; p < rowOffsets[row + 1]; ++p) {
                uint32_t s = sourceIds[p];
                float v = values[p];
                if (s >= cols || !isfinite(v) || v == 0.0f) {
                    status = ORC_INVALID;
                    goto done;
                }
                if (p > rowOffsets[row] && s <= sourceIds[p - 1]) {
                    status = ORC_INVALID;
                    goto done;
                }
                trip[n].source = s;
                trip[n].row = r;
                trip[n].value = v;
                ++n;
            }
        }
        if (n) qsort(trip, n, sizeof(triple_t), triple_cmp); /* ascending (source, row): the merge order */
        for (int i = 0; i < 16; ++i) buckets[i].n = 0;
        size_t nv = 0;
        for (size_t i = 0; i < n;) { /* :102-129 */
            uint32_t s = trip[i].source, mask = 0;
            CHECK32(nv);
            uint32_t offset = (uint32_t)nv;
            do {
                mask |= 1u << trip[i].row;
                wvals[nv++] = trip[i].value;
                ++i;
            } while (i < n && trip[i].source == s);
            unsigned rwm = rw_mask_of(mask);
            item_t it = {s, mask, offset};
            if ((status = vec_push(&buckets[bucketByRwMask ? rwm : 0], &it))) goto done;
        }
        for (int bi = 0; bi < 16; ++bi) { /* :130-158 */
            const vec_t* bucket = &buckets[kBucketOrder[bi]];
            if (bucketByRwMask) {
                CHECK32(rgm.n);
                uint32_t off = (uint32_t)rgm.n;
                if ((status = vec_push(&bo, &off))) goto done;
            }
            unsigned slot = 0, pm = 0;
            for (size_t k = 0; k < bucket->n; ++k) {
                const item_t* it = (const item_t*)bucket->p + k;
                if ((status = vec_push(&sid, &it->source))) goto done;
                CHECK32(vals.n);
                uint64_t md = ((uint64_t)vals.n << 32) | it->mask;
                if ((status = vec_push(&meta, &md))) goto done;
                unsigned cnt = (unsigned)__builtin_popcount(it->mask);
                for (unsigned c = 0; c < cnt; ++c)
                    if ((status = vec_push(&vals, &wvals[it->offset + c]))) goto done;
                pm |= rw_mask_of(it->mask);
                if (++slot == 8) {
                    if ((status = vec_push(&rgm, &pm))) goto done;
                    slot = pm = 0;
                }
            }
            if (slot) {
                uint32_t pad = 0xFFFFFFFFu;
                uint64_t pmd = 0;
                while (slot++ < 8) {
                    if ((status = vec_push(&sid, &pad))) goto done;
                    if ((status = vec_push(&meta, &pmd))) goto done;
                }
                if ((status = vec_push(&rgm, &pm))) goto done;
            }
        }
        CHECK32(rgm.n);
        uint32_t pe = (uint32_t)rgm.n;
        if (bucketByRwMask)
            if ((status = vec_push(&bo, &pe))) goto done;
        if ((status = vec_push(&wo, &pe))) goto done;
    }
    CHECK32(vals.n);
    out->rows = rows;
    out->cols = cols;
    out->windowOffsets = (uint32_t*)wo.p;
    out->nWindowOffsets = wo.n;
    out->sourceIds = (uint32_t*)sid.p;
    out->nSlots = sid.n;
    out->sourceMetadata = (uint64_t*)meta.p;
    out->rowGroupMasks = (uint32_t*)rgm.p;
    out->nPanels = rgm.n;
    out->values = (float*)vals.p;
    out->nValues = vals.n;
    out->bucketOffsets = (uint32_t*)bo.p;
    out->nBucketOffsets = bo.n;
    wo.p = sid.p = meta.p = rgm.p = vals.p = bo.p = NULL;
    if (bucketByRwMask) { /* :164-165 */
        status = build_tasks(out, &tasks, &reds, &pids);
        if (status) goto done;
        out->tasks = (orc_task*)tasks.p;
        out->nTasks = tasks.n;
        out->reductions = (orc_reduce*)reds.p;
        out->nReductions = reds.n;
        out->partialIds = (uint32_t*)pids.p;
        out->nPartialIds = pids.n;
        tasks.p = reds.p = pids.p = NULL;
    }
done:
    free(trip);
    free(wvals);
    for (int i = 0; i < 16; ++i) free(buckets[i].p);
    free(wo.p);
    free(sid.p);
    free(meta.p);
    free(rgm.p);
    free(vals.p);
    free(bo.p);
    free(tasks.p);
    free(reds.p);
    free(pids.p);
    if (status) orc_sw32_free(out);
    return status;
}

/* ---------------------------------------------------------------- features */
/* src/format/int8_quantize.cu:4-25 */
void orc_quantize(const float* x, int8_t* q, float* scale, uint32_t sources, uint32_t features) {
    for (uint32_t r = 0; r < sources; ++r) {
        const float* row = x + (size_t)r * features;
        float m = 0.0f;
        for (uint32_t j = 0; j < features; ++j) m = fmaxf(m, fabsf(row[j]));
        volatile float mv = m; /* keep the IEEE single-precision divide */
        float s = (mv == 0.0f) ? 1.0f : mv / 127.0f;
        scale[r] = s;
        for (uint32_t j = 0; j < features; ++j) {
            volatile float t = row[j] / s;
            long v = lrintf(t);
            q[(size_t)r * features + j] = (int8_t)(v < -127 ? -127 : (v > 127 ? 127 : v));
        }
    }
}

/* src/format/pack_int8.cu:6-15: out16[p] = u8(q[o]) | u8(q[o+8]) << 8, o = (p>>3)*16 + (p&7) */
void orc_pack16(const int8_t* q, int8_t* packed, uint32_t sources, uint32_t features) {
    size_t pairs = (size_t)sources * features / 2;
    for (size_t p = 0; p < pairs; ++p) {
        size_t o = (p >> 3) * 16 + (p & 7);
        packed[2 * p] = q[o];
        packed[2 * p + 1] = q[o + 8];
    }
}

void orc_unpack16(const int8_t* packed, int8_t* q, uint32_t sources, uint32_t features) {
    size_t pairs = (size_t)sources * features / 2;
    for (size_t p = 0; p < pairs; ++p) {
        size_t o = (p >> 3) * 16 + (p & 7);
        q[o] = packed[2 * p];
        q[o + 8] = packed[2 * p + 1];
    }
}

/* cvt.rna.tf32.f32 (spmm_kernel.cuh:7-11): 10 explicit mantissa bits, nearest, ties away. */
float orc_tf32(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu)) return v; /* NaN passes */
    b = (b + 0x1000u) & 0xFFFFE000u;
    float r;
    memcpy(&r, &b, 4);
    return r;
}

/* Dequantized, TF32-rounded feature f of source c read from packed16 X
 * (spmm_kernel.cuh:38-47: byte pair holds features g and g+8 of a 16-feature tile). */
static inline float xhat(const int8_t* packedX, const float* scales, uint32_t c, uint32_t f,
                         uint32_t features) {
    uint32_t tile = f >> 4, j = f & 15;
    size_t byte = (size_t)c * features + tile * 16 + (j < 8 ? 2 * j : 2 * (j - 8) + 1);
    float prod = (float)packedX[byte] * scales[c];
    return orc_tf32(prod);
}

void orc_spmm_csr_f64(uint32_t rows, const uint32_t* rowOffsets, const uint32_t* sourceIds,
                      const float* values, const int8_t* packedX, const float* scales,
                      uint32_t cols, uint32_t features, double* y) {
    for (uint32_t r = 0; r < rows; ++r) {
        double* yr = y + (size_t)r * features;
        for (uint32_t f = 0; f < features; ++f) yr[f] = 0.0;
        for (uint32_t p = rowOffsets[r]; p < rowOffsets[r + 1]; ++p) {
            uint32_t c = sourceIds[p];
            if (c >= cols) continue;
            double a = (double)orc_tf32(values[p]);
            for (uint32_t f = 0; f < features; ++f)
                yr[f] += a * (double)xhat(packedX, scales, c, f, features);
        }
    }
}

void orc_spmm_sw32_f64(const orc_sw32* fm, const int8_t* packedX, const float* scales,
                       uint32_t features, double* y) {
    memset(y, 0, (size_t)fm->rows * features * sizeof(double));
    uint32_t windows = (uint32_t)(fm->nWindowOffsets - 1);
    for (uint32_t sw = 0; sw < windows; ++sw) {
        for (size_t slot = (size_t)fm->windowOffsets[sw] * 8;
             slot < (size_t)fm->windowOffsets[sw + 1] * 8; ++slot) {
            uint32_t c = fm->sourceIds[slot];
            uint64_t md = fm->sourceMetadata[slot];
            uint32_t mask = (uint32_t)md, base = (uint32_t)(md >> 32);
            if (c >= fm->cols) continue; /* padding (spmm_kernel.cuh:38,49) */
            uint32_t k = 0;
            for (uint32_t r = 0; r < 32; ++r) {
                if (!(mask & (1u << r))) continue;
                double a = (double)orc_tf32(fm->values[base + k++]);
                double* yr = y + ((size_t)sw * 32 + r) * features;
                for (uint32_t f = 0; f < features; ++f)
                    yr[f] += a * (double)xhat(packedX, scales, c, f, features);
            }
        }
    }
}

void orc_spmm_sw32_f64_windows(const orc_sw32* fm, const int8_t* packedX, const float* scales,
                               uint32_t features, const uint32_t* windows, uint32_t n, double* y,
                               double* yabs) {
    memset(y, 0, (size_t)n * 32 * features * sizeof(double));
    if (yabs) memset(yabs, 0, (size_t)n * 32 * features * sizeof(double));
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t sw = windows[i];
        for (size_t slot = (size_t)fm->windowOffsets[sw] * 8;
             slot < (size_t)fm->windowOffsets[sw + 1] * 8; ++slot) {
            uint32_t c = fm->sourceIds[slot];
            uint64_t md = fm->sourceMetadata[slot];
            uint32_t mask = (uint32_t)md, base = (uint32_t)(md >> 32);
            if (c >= fm->cols) continue;
            uint32_t k = 0;
            for (uint32_t r = 0; r < 32; ++r) {
                if (!(mask & (1u << r))) continue;
                double a = (double)orc_tf32(fm->values[base + k++]);
                double* yr = y + ((size_t)i * 32 + r) * features;
                double* ya = yabs ? yabs + ((size_t)i * 32 + r) * features : NULL;
                for (uint32_t f = 0; f < features; ++f) {
                    double p = a * (double)xhat(packedX, scales, c, f, features);
                    yr[f] += p;
                    if (ya) ya[f] += fabs(p);
                }
            }
        }
    }
}

/* FP32 accumulation of one panel range into acc[32][features] (slot order). */
static void accumulate_panels_f32(const orc_sw32* fm, uint32_t begin, uint32_t end,
                                  const int8_t* packedX, const float* scales, uint32_t features,
                                  float* acc, float* xh) {
    for (size_t slot = (size_t)begin * 8; slot < (size_t)end * 8; ++slot) {
        uint32_t c = fm->sourceIds[slot];
        if (c >= fm->cols) continue;
        uint64_t md = fm->sourceMetadata[slot];
        uint32_t mask = (uint32_t)md, base = (uint32_t)(md >> 32);
        for (uint32_t f = 0; f < features; ++f) xh[f] = xhat(packedX, scales, c, f, features);
        uint32_t k = 0;
        for (uint32_t r = 0; r < 32; ++r) {
            if (!(mask & (1u << r))) continue;
            float a = orc_tf32(fm->values[base + k++]);
            float* ar = acc + (size_t)r * features;
            for (uint32_t f = 0; f < features; ++f) ar[f] += a * xh[f];
        }
    }
}

/* spmm_kernel.cuh:228-282 (write-back, partial tiles, fixed-order merge) */
void orc_spmm_tasks_f32(const orc_sw32* fm, const int8_t* packedX, const float* scales,
                        uint32_t features, float* partials, float* y) {
    float* acc = (float*)malloc((size_t)32 * features * sizeof(float));
    float* xh = (float*)malloc((size_t)features * sizeof(float));
    uint32_t rows = fm->rows;
    for (size_t t = 0; t < fm->nTasks; ++t) {
        const orc_task* task = &fm->tasks[t];
        memset(acc, 0, (size_t)32 * features * sizeof(float));
        accumulate_panels_f32(fm, task->begin, task->end, packedX, scales, features, acc, xh);
        uint32_t rowbase = task->sw * 32;
        if (task->partial == 0xFFFFFFFFu) {
            for (uint32_t r = 0; r < 32; ++r)
                if (rowbase + r < rows)
                    memcpy(y + (size_t)(rowbase + r) * features, acc + (size_t)r * features,
                           features * sizeof(float));
        } else {
            for (uint32_t rw = 0; rw < 4; ++rw) {
                if (!(task->mask & (1u << rw))) continue;
                size_t tile = task->partial + __builtin_popcount(task->mask & ((1u << rw) - 1));
                for (uint32_t r = 0; r < 8; ++r)
                    memcpy(partials + (tile * 8 + r) * features,
                           acc + (size_t)(rw * 8 + r) * features, features * sizeof(float));
            }
        }
    }
    /* Merge: every split SW, after all its tasks (order independent of arrival by construction). */
    for (size_t t = 0; t < fm->nTasks; ++t) {
        const orc_task* task = &fm->tasks[t];
        if (task->partial == 0xFFFFFFFFu) continue;
        if (t + 1 < fm->nTasks && fm->tasks[t + 1].sw == task->sw) continue; /* last chunk only */
        for (uint32_t rw = 0; rw < 4; ++rw) {
            orc_reduce red = fm->reductions[task->reduceFirst + rw];
            uint32_t row = task->sw * 32 + rw * 8;
            if (row >= rows) continue;
            uint32_t valid = rows - row < 8 ? rows - row : 8;
            for (uint32_t r = 0; r < valid; ++r)
                for (uint32_t f = 0; f < features; ++f) {
                    float sum = 0.0f;
                    for (uint32_t i = red.begin; i < red.end; ++i)
                        sum += partials[((size_t)fm->partialIds[i] * 8 + r) * features + f];
                    y[(size_t)(row + r) * features + f] = sum;
                }
        }
    }
    free(acc);
    free(xh);
}

/* ---------------------------------------------------------------- CPU baseline (threads) */
typedef struct {
    const orc_sw32* fm;
    const int8_t* packedX;
    const float* scales;
    uint32_t features, swBegin, swEnd;
    float* y;
} mt_args;

static void* mt_worker(void* p) {
    mt_args* a = (mt_args*)p;
    const orc_sw32* fm = a->fm;
    uint32_t F = a->features;
    float* xh = (float*)malloc(F * sizeof(float));
    int8_t* qrow = (int8_t*)malloc(F);
    for (uint32_t sw = a->swBegin; sw < a->swEnd; ++sw) {
        uint32_t rowbase = sw * 32;
        uint32_t nrows = fm->rows - rowbase < 32 ? fm->rows - rowbase : 32;
        float* ysw = a->y + (size_t)rowbase * F;
        memset(ysw, 0, (size_t)nrows * F * sizeof(float));
        for (size_t slot = (size_t)fm->windowOffsets[sw] * 8;
             slot < (size_t)fm->windowOffsets[sw + 1] * 8; ++slot) {
            uint32_t c = fm->sourceIds[slot];
            if (c >= fm->cols) continue;
            uint64_t md = fm->sourceMetadata[slot];
            uint32_t mask = (uint32_t)md, base = (uint32_t)(md >> 32);
            const int8_t* pr = a->packedX + (size_t)c * F;
            for (uint32_t p = 0; p < F / 2; ++p) { /* unpack packed16 */
                uint32_t o = (p >> 3) * 16 + (p & 7);
                qrow[o] = pr[2 * p];
                qrow[o + 8] = pr[2 * p + 1];
            }
            float s = a->scales[c];
            for (uint32_t f = 0; f < F; ++f) xh[f] = orc_tf32((float)qrow[f] * s);
            uint32_t k = 0;
            while (mask) {
                uint32_t r = (uint32_t)__builtin_ctz(mask);
                mask &= mask - 1;
                float av = orc_tf32(fm->values[base + k++]);
                float* yr = ysw + (size_t)r * F;
                for (uint32_t f = 0; f < F; ++f) yr[f] += av * xh[f];
            }
        }
    }
    free(xh);
    free(qrow);
    return NULL;
}

/* The same computation with AVX2: per slot, the packed16 row is unpacked by a byte shuffle per
 * 16-feature tile, converted, scaled and TF32-rounded eight values at a time, then every row of the
 * slot accumulates it. Same products, same order: av * xh is exact in FP32 (two eleven-bit
 * significands), so the fused multiply-add rounds exactly as the scalar multiply then add does, and
 * Y is bitwise the scalar path's. */
__attribute__((target("avx2,fma"))) static void* mt_worker_avx2(void* p) {
    mt_args* a = (mt_args*)p;
    const orc_sw32* fm = a->fm;
    const uint32_t F = a->features;
    float* xh = (float*)aligned_alloc(32, F * sizeof(float));
    if (!xh) return p; /* non-null: out of memory */
    const __m128i unpack = _mm_setr_epi8(0, 2, 4, 6, 8, 10, 12, 14, 1, 3, 5, 7, 9, 11, 13, 15);
    const __m256i half = _mm256_set1_epi32(0x1000), keep = _mm256_set1_epi32((int)0xFFFFE000u);
    const size_t slotEnd = (size_t)fm->windowOffsets[a->swEnd] * 8;
    for (uint32_t sw = a->swBegin; sw < a->swEnd; ++sw) {
        uint32_t rowbase = sw * 32;
        uint32_t nrows = fm->rows - rowbase < 32 ? fm->rows - rowbase : 32;
        float* ysw = a->y + (size_t)rowbase * F;
        memset(ysw, 0, (size_t)nrows * F * sizeof(float));
        for (size_t slot = (size_t)fm->windowOffsets[sw] * 8;
             slot < (size_t)fm->windowOffsets[sw + 1] * 8; ++slot) {
            /* The X rows and scales of later slots are random reads from memory: request them
             * kAhead slots early. */
            enum { kAhead = 12 };
            if (slot + kAhead < slotEnd) {
                uint32_t cn = fm->sourceIds[slot + kAhead];
                if (cn < fm->cols) {
                    const char* rn = (const char*)(a->packedX + (size_t)cn * F);
                    for (uint32_t b = 0; b < F; b += 64) _mm_prefetch(rn + b, _MM_HINT_T0);
                    _mm_prefetch((const char*)(a->scales + cn), _MM_HINT_T0);
                }
            }
            uint32_t c = fm->sourceIds[slot];
            if (c >= fm->cols) continue;
            uint64_t md = fm->sourceMetadata[slot];
            uint32_t mask = (uint32_t)md, base = (uint32_t)(md >> 32), k = 0;
            const int8_t* pr = a->packedX + (size_t)c * F;
            const __m256 s = _mm256_set1_ps(a->scales[c]);
            for (uint32_t t = 0; t < F / 16; ++t) {
                __m128i q = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i*)(pr + 16 * t)), unpack);
                __m256 lo = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q)), s);
                __m256 hi = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(q, 8))), s);
                lo = _mm256_castsi256_ps(_mm256_and_si256(_mm256_add_epi32(_mm256_castps_si256(lo), half), keep));
                hi = _mm256_castsi256_ps(_mm256_and_si256(_mm256_add_epi32(_mm256_castps_si256(hi), half), keep));
                _mm256_store_ps(xh + 16 * t, lo);
                _mm256_store_ps(xh + 16 * t + 8, hi);
            }
            while (mask) {
                uint32_t r = (uint32_t)__builtin_ctz(mask);
                mask &= mask - 1;
                const __m256 av = _mm256_set1_ps(orc_tf32(fm->values[base + k++]));
                float* yr = ysw + (size_t)r * F;
                for (uint32_t f = 0; f < F; f += 8)
                    _mm256_storeu_ps(yr + f, _mm256_fmadd_ps(av, _mm256_load_ps(xh + f),
                                                             _mm256_loadu_ps(yr + f)));
            }
        }
    }
    free(xh);
    return NULL;
}

int orc_spmm_sw32_f32_mt(const orc_sw32* fm, const int8_t* packedX, const float* scales,
                         uint32_t features, uint32_t swBegin, uint32_t swEnd, int threads,
                         float* y) {
    return orc_spmm_sw32_f32_mt_path(fm, packedX, scales, features, swBegin, swEnd, threads, y, 0);
}

int orc_cpu_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

int orc_spmm_sw32_f32_mt_path(const orc_sw32* fm, const int8_t* packedX, const float* scales,
                              uint32_t features, uint32_t swBegin, uint32_t swEnd, int threads,
                              float* y, int vector) {
    if (vector && (!orc_cpu_has_avx2() || features % 16)) return -1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t th[256];
    mt_args args[256];
    uint32_t span = swEnd - swBegin;
    for (int t = 0; t < threads; ++t) {
        args[t].fm = fm;
        args[t].packedX = packedX;
        args[t].scales = scales;
        args[t].features = features;
        args[t].swBegin = swBegin + (uint32_t)((uint64_t)span * t / threads);
        args[t].swEnd = swBegin + (uint32_t)((uint64_t)span * (t + 1) / threads);
        args[t].y = y;
        pthread_create(&th[t], NULL, vector ? mt_worker_avx2 : mt_worker, &args[t]);
    }
    int failed = 0;
    for (int t = 0; t < threads; ++t) {
        void* r = NULL;
        pthread_join(th[t], &r);
        failed |= r != NULL;
    }
    return failed ? -2 : threads;
}

/* ---------------------------------------------------------------- full-size checker (threads) */
typedef struct {
    const orc_sw32* fm;
    const int8_t* packedX;
    const float* scales;
    const float* y;
    double* ref;
    uint32_t features, swBegin, swEnd;
    double atol, rtol, cond;
    int nomem;
    orc_check_stats st;
} chk_args;

/* Per SW: the reference rows in double in slot order (the accumulation of
 * orc_spmm_sw32_f64_windows, so the values are bitwise the same), then the comparison. */
static void* chk_worker(void* p) {
    chk_args* a = (chk_args*)p;
    const orc_sw32* fm = a->fm;
    const uint32_t F = a->features;
    double* acc = (double*)malloc((size_t)32 * F * sizeof(double));
    double* mag = (double*)malloc((size_t)32 * F * sizeof(double));
    double* xh = (double*)malloc((size_t)F * sizeof(double));
    a->st.checked = a->st.bad = a->st.relaxed = 0;
    a->st.maxErr = 0.0;
    a->st.firstBad = UINT64_MAX;
    a->nomem = !acc || !mag || !xh;
    for (uint32_t sw = a->swBegin; sw < a->swEnd && !a->nomem; ++sw) {
        memset(acc, 0, (size_t)32 * F * sizeof(double));
        memset(mag, 0, (size_t)32 * F * sizeof(double));
        for (size_t slot = (size_t)fm->windowOffsets[sw] * 8;
             slot < (size_t)fm->windowOffsets[sw + 1] * 8; ++slot) {
            uint32_t c = fm->sourceIds[slot];
            if (c >= fm->cols) continue;
            uint64_t md = fm->sourceMetadata[slot];
            uint32_t mask = (uint32_t)md, base = (uint32_t)(md >> 32), k = 0;
            for (uint32_t f = 0; f < F; ++f) xh[f] = (double)xhat(a->packedX, a->scales, c, f, F);
            while (mask) {
                uint32_t r = (uint32_t)__builtin_ctz(mask);
                mask &= mask - 1;
                double av = (double)orc_tf32(fm->values[base + k++]);
                double* yr = acc + (size_t)r * F;
                double* ya = mag + (size_t)r * F;
                for (uint32_t f = 0; f < F; ++f) {
                    double t = av * xh[f];
                    yr[f] += t;
                    ya[f] += fabs(t);
                }
            }
        }
        uint32_t rows = fm->rows - sw * 32 < 32 ? fm->rows - sw * 32 : 32;
        for (uint32_t r = 0; r < rows; ++r) {
            size_t row = (size_t)sw * 32 + r;
            if (a->ref) memcpy(a->ref + row * F, acc + (size_t)r * F, (size_t)F * sizeof(double));
            for (uint32_t f = 0; f < F; ++f) {
                double want = acc[(size_t)r * F + f], got = (double)a->y[row * F + f];
                double err = fabs(got - want);
                if (err != err) err = INFINITY; /* NaN: never within a bound */
                double plain = a->atol + a->rtol * fabs(want);
                double bound = plain + a->cond * 0x1.0p-24 * mag[(size_t)r * F + f];
                a->st.checked++;
                if (err > a->st.maxErr) a->st.maxErr = err;
                if (!(err <= bound)) {
                    if (a->st.bad++ == 0) {
                        a->st.firstBad = row * F + f;
                        a->st.firstGot = got;
                        a->st.firstWant = want;
                        a->st.firstBound = bound;
                    }
                } else if (err > plain) {
                    a->st.relaxed++;
                }
            }
        }
    }
    free(acc);
    free(mag);
    free(xh);
    return NULL;
}

int orc_check_sw32_mt(const orc_sw32* fm, const int8_t* packedX, const float* scales,
                      uint32_t features, const float* y, double atol, double rtol, double cond,
                      int threads, orc_check_stats* out, double* ref) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    uint32_t windows = (uint32_t)(fm->nWindowOffsets - 1);
    pthread_t th[256];
    chk_args* args = (chk_args*)calloc((size_t)threads, sizeof(chk_args));
    if (!args) return ORC_NOMEM;
    for (int t = 0; t < threads; ++t) {
        chk_args* a = &args[t];
        a->fm = fm;
        a->packedX = packedX;
        a->scales = scales;
        a->y = y;
        a->ref = ref;
        a->features = features;
        a->swBegin = (uint32_t)((uint64_t)windows * t / threads);
        a->swEnd = (uint32_t)((uint64_t)windows * (t + 1) / threads);
        a->atol = atol;
        a->rtol = rtol;
        a->cond = cond;
        pthread_create(&th[t], NULL, chk_worker, a);
    }
    memset(out, 0, sizeof(*out));
    out->firstBad = UINT64_MAX;
    int nomem = 0;
    for (int t = 0; t < threads; ++t) {
        pthread_join(th[t], NULL);
        nomem |= args[t].nomem;
        const orc_check_stats* s = &args[t].st;
        out->checked += s->checked;
        out->bad += s->bad;
        out->relaxed += s->relaxed;
        if (s->maxErr > out->maxErr) out->maxErr = s->maxErr;
        /* Threads cover increasing SW ranges: the first thread with a bad element has the
         * smallest index. */
        if (s->firstBad != UINT64_MAX && out->firstBad == UINT64_MAX) {
            out->firstBad = s->firstBad;
            out->firstGot = s->firstGot;
            out->firstWant = s->firstWant;
            out->firstBound = s->firstBound;
        }
    }
    free(args);
    return nomem ? ORC_NOMEM : ORC_OK;
}
