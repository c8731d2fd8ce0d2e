// C ABI over the C++ library surface (declarations and status codes in include/tcc_spmm_c.h).
// Each entry point forwards to the C++ function of the same name and converts its exception
// class into a status code, keeping the message for tcc_last_error().
#include "tcc_spmm_c.h"

#include "device_matrix.h"
#include "format/csr.h"
#include "format/int8_features.h"
#include "format/sw32.h"
#include "spmm.h"

#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>

struct tcc_csr {
    CsrMatrix csr;
};
struct tcc_sw32 {
    Sw32HostFormat format;
};
struct tcc_device_matrix {
    std::unique_ptr<DeviceMatrix> matrix;
};

static_assert(sizeof(tcc_device_view) == sizeof(Sw32DeviceView), "view layouts must match");
static_assert(offsetof(tcc_device_view, taskCount) == offsetof(Sw32DeviceView, taskCount),
              "view layouts must match");

namespace {
thread_local std::string lastError;

template <typename Body> int guarded(Body body) {
    try {
        body();
        return TCC_OK;
    } catch (const std::invalid_argument& e) {
        lastError = e.what();
        return TCC_INVALID_ARGUMENT;
    } catch (const std::overflow_error& e) {
        lastError = e.what();
        return TCC_OVERFLOW;
    } catch (const std::runtime_error& e) {
        lastError = e.what();
        return TCC_RUNTIME;
    } catch (const std::exception& e) {
        lastError = e.what();
        return TCC_OTHER;
    } catch (...) {
        lastError = "unknown exception";
        return TCC_OTHER;
    }
}

// A required pointer argument (an output, or an input array with a nonzero count) must not be null.
void need(const void* p, const char* what) {
    if (!p) throw std::invalid_argument(std::string("null ") + what);
}

Sw32DeviceView toView(const tcc_device_view* v) {
    Sw32DeviceView out;
    std::memcpy(static_cast<void*>(&out), v, sizeof(out));
    return out;
}
} // namespace

extern "C" {

void tccSetLastError(const char* message) { lastError = message ? message : ""; }

int tccWrapCsr(CsrMatrix&& csr, tcc_csr** out) {
    return guarded([&] {
        need(out, "output handle");
        *out = new tcc_csr{std::move(csr)};
    });
}

const char* tcc_last_error(void) { return lastError.c_str(); }

const char* tcc_version(void) { return "tcc_spmm_amd 0.1 gfx950"; }

int tcc_make_canonical_csr(uint32_t rows, uint32_t cols, uint32_t nnz, const uint32_t* rowOffsets,
                           const uint32_t* sourceIds, const float* values, tcc_csr** out) {
    return guarded([&] {
        need(out, "output handle");
        need(rowOffsets, "rowOffsets");
        if (nnz) {
            need(sourceIds, "sourceIds");
            need(values, "values");
        }
        *out = new tcc_csr{makeCanonicalCsr(rows, cols, nnz, rowOffsets, sourceIds, values)};
    });
}

int tcc_load_matrix_market(const char* path, uint32_t* rows, uint32_t* cols, tcc_csr** out) {
    return guarded([&] {
        need(rows, "rows");
        need(cols, "cols");
        need(out, "output handle");
        MtxMatrix m = loadMatrixMarket(path ? path : "");
        *rows = m.rows;
        *cols = m.cols;
        *out = new tcc_csr{std::move(m.csr)};
    });
}

int tcc_csr_from_arrays(uint64_t rowOffsetsCount, const uint32_t* rowOffsets, uint64_t nnz,
                        const uint32_t* sourceIds, const float* values, tcc_csr** out) {
    return guarded([&] {
        need(out, "output handle");
        if (rowOffsetsCount) need(rowOffsets, "rowOffsets");
        if (nnz) {
            need(sourceIds, "sourceIds");
            need(values, "values");
        }
        auto h = std::make_unique<tcc_csr>();
        h->csr.rowOffsets.assign(rowOffsets, rowOffsets + rowOffsetsCount);
        h->csr.sourceIds.assign(sourceIds, sourceIds + nnz);
        h->csr.values.assign(values, values + nnz);
        *out = h.release();
    });
}

int tcc_csr_info(const tcc_csr* csr, uint64_t* rowOffsetsCount, uint64_t* nnz) {
    return guarded([&] {
        if (!csr) throw std::invalid_argument("null CSR handle");
        need(rowOffsetsCount, "rowOffsetsCount");
        need(nnz, "nnz");
        *rowOffsetsCount = csr->csr.rowOffsets.size();
        *nnz = csr->csr.sourceIds.size();
    });
}

int tcc_csr_arrays(const tcc_csr* csr, const uint32_t** rowOffsets, const uint32_t** sourceIds,
                   const float** values) {
    return guarded([&] {
        if (!csr) throw std::invalid_argument("null CSR handle");
        need(rowOffsets, "rowOffsets");
        need(sourceIds, "sourceIds");
        need(values, "values");
        *rowOffsets = csr->csr.rowOffsets.data();
        *sourceIds = csr->csr.sourceIds.data();
        *values = csr->csr.values.data();
    });
}

void tcc_csr_free(tcc_csr* csr) { delete csr; }

int tcc_convert_csr_to_sw32(uint32_t rows, uint32_t cols, const tcc_csr* csr, int bucketByRwMask,
                            tcc_sw32** out) {
    return guarded([&] {
        if (!csr) throw std::invalid_argument("null CSR handle");
        need(out, "output handle");
        *out = new tcc_sw32{convertCsrToSw32(rows, cols, csr->csr, bucketByRwMask != 0)};
    });
}

int tcc_build_panel_tasks(tcc_sw32* format) {
    return guarded([&] {
        if (!format) throw std::invalid_argument("null SW32 handle");
        buildPanelTasks(format->format);
    });
}

int tcc_sw32_get_sizes(const tcc_sw32* format, tcc_sw32_sizes* s) {
    return guarded([&] {
        if (!format) throw std::invalid_argument("null SW32 handle");
        need(s, "sizes");
        const Sw32HostFormat& f = format->format;
        s->rows = f.rows;
        s->cols = f.cols;
        s->partialCount = f.partialCount;
        s->bucketed = f.bucketOffsets.empty() ? 0u : 1u;
        s->windowOffsets = f.windowOffsets.size();
        s->sourceIds = f.sourceIds.size();
        s->rowGroupMasks = f.rowGroupMasks.size();
        s->sourceMetadata = f.sourceMetadata.size();
        s->values = f.values.size();
        s->bucketOffsets = f.bucketOffsets.size();
        s->tasks = f.tasks.size();
        s->reductions = f.reductions.size();
        s->partialIds = f.partialIds.size();
    });
}

int tcc_sw32_get_arrays(const tcc_sw32* format, tcc_sw32_arrays* a) {
    return guarded([&] {
        if (!format) throw std::invalid_argument("null SW32 handle");
        need(a, "arrays");
        const Sw32HostFormat& f = format->format;
        a->windowOffsets = f.windowOffsets.data();
        a->sourceIds = f.sourceIds.data();
        a->rowGroupMasks = f.rowGroupMasks.data();
        a->sourceMetadata = f.sourceMetadata.data();
        a->values = f.values.data();
        a->bucketOffsets = f.bucketOffsets.data();
        a->tasks = f.tasks.data();
        a->reductions = f.reductions.data();
        a->partialIds = f.partialIds.data();
    });
}

void tcc_sw32_free(tcc_sw32* format) { delete format; }

int tcc_launch_spmm_int8(const tcc_device_view* matrix, const int8_t* packedX, const float* scales,
                         float* output, uint32_t rows, uint32_t cols, uint32_t features,
                         float* partials, uint32_t* counters, void* stream) {
    return guarded([&] {
        if (!matrix) throw std::invalid_argument("null device view");
        launchSpmmInt8(toView(matrix), packedX, scales, output, rows, cols, features,
                       SpmmWorkspace{partials, counters}, static_cast<hipStream_t>(stream));
    });
}

int tcc_launch_spmm_int8_noalloc(const tcc_device_view* matrix, const int8_t* packedX,
                                 const float* scales, float* output, uint32_t rows, uint32_t cols,
                                 uint32_t features, uint32_t partialCount, void* stream) {
    return guarded([&] {
        if (!matrix) throw std::invalid_argument("null device view");
        launchSpmmInt8NoAlloc(toView(matrix), packedX, scales, output, rows, cols, features,
                              partialCount, static_cast<hipStream_t>(stream));
    });
}

int tcc_set_spmm_launch_overrides(uint32_t taskWaves, int forceWide) {
    return guarded([&] { setSpmmLaunchOverrides(taskWaves, forceWide != 0); });
}

int tcc_quantize_features_int8(const float* x, int8_t* q, float* scale, uint32_t sources,
                               uint32_t features, void* stream) {
    return guarded([&] {
        quantizeFeaturesInt8(x, q, scale, sources, features, static_cast<hipStream_t>(stream));
    });
}

int tcc_pack_features_int8x16(const int8_t* q, int8_t* packed, uint32_t sources, uint32_t features,
                              void* stream) {
    return guarded([&] {
        packFeaturesInt8x16(q, packed, sources, features, static_cast<hipStream_t>(stream));
    });
}

int tcc_quantize_pack_features_int8(const float* x, int8_t* packed, float* scale, uint32_t sources,
                                    uint32_t features, void* stream) {
    return guarded([&] {
        quantizePackFeaturesInt8(x, packed, scale, sources, features,
                                 static_cast<hipStream_t>(stream));
    });
}

int tcc_device_matrix_create(const tcc_sw32* format, uint32_t features, tcc_device_matrix** out) {
    return guarded([&] {
        if (!format) throw std::invalid_argument("null SW32 handle");
        if (format->format.bucketOffsets.empty())
            throw std::invalid_argument("device matrices need the RW-bucketed SW32 format");
        need(out, "output handle");
        auto m = std::make_unique<DeviceMatrix>(format->format, features);
        *out = new tcc_device_matrix{std::move(m)};
    });
}

int tcc_device_matrix_view(const tcc_device_matrix* m, tcc_device_view* view, float** partials,
                           uint32_t** counters) {
    return guarded([&] {
        if (!m || !m->matrix) throw std::invalid_argument("null device matrix");
        need(view, "view");
        need(partials, "partials");
        need(counters, "counters");
        const Sw32DeviceView v = m->matrix->view();
        std::memcpy(static_cast<void*>(view), &v, sizeof(v));
        const SpmmWorkspace w = m->matrix->workspace();
        *partials = w.partials;
        *counters = w.counters;
    });
}

void tcc_device_matrix_free(tcc_device_matrix* m) { delete m; }

} // extern "C"
