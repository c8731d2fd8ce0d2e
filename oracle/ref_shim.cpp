// ref_shim.cpp — extern "C" access to the REFERENCE's own CPU format code, for tests only.
//
// Compiled by oracle/Makefile together with the reference sources where they lie
// (/root/reference/src/format/{csr,sw32,matrix_market}.cpp, headers from
// /root/reference/include); the result is oracle/_ref/libref_format.so. Nothing here is
// product code: tests/golden/make_fixtures.py and the CPU tests use it to pin the C oracle
// and the product's host format builder against the reference's exact bytes.
#include "format/csr.h"
#include "format/sw32.h"

#include <cstring>
#include <exception>
#include <new>
#include <stdexcept>
#include <string>

namespace {
thread_local std::string lastError;

int classify(const std::exception& e) {
    lastError = e.what();
    if (dynamic_cast<const std::invalid_argument*>(&e)) return 1;
    if (dynamic_cast<const std::overflow_error*>(&e)) return 2;
    return 3;
}

struct RefCsr {
    std::uint32_t rows = 0, cols = 0;
    CsrMatrix csr;
};
} // namespace

extern "C" {
const char* ref_last_error() { return lastError.c_str(); }

// makeCanonicalCsr (reference include/format/csr.h:23-25).
int ref_canonical_csr(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                      const std::uint32_t* offsets, const std::uint32_t* sources,
                      const float* values, void** out) {
    try {
        auto* h = new RefCsr;
        h->rows = rows;
        h->cols = cols;
        try {
            h->csr = makeCanonicalCsr(rows, cols, nnz, offsets, sources, values);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
        return 0;
    } catch (const std::exception& e) {
        return classify(e);
    }
}

// loadMatrixMarket (reference include/format/csr.h:18).
int ref_load_matrix_market(const char* path, void** out) {
    try {
        auto m = loadMatrixMarket(path);
        auto* h = new RefCsr;
        h->rows = m.rows;
        h->cols = m.cols;
        h->csr = std::move(m.csr);
        *out = h;
        return 0;
    } catch (const std::exception& e) {
        return classify(e);
    }
}

void ref_csr_info(void* h, std::uint32_t* rows, std::uint32_t* cols, std::uint64_t* nnz) {
    auto* c = static_cast<RefCsr*>(h);
    *rows = c->rows;
    *cols = c->cols;
    *nnz = c->csr.sourceIds.size();
}

void ref_csr_copy(void* h, std::uint32_t* offsets, std::uint32_t* sources, float* values) {
    auto* c = static_cast<RefCsr*>(h);
    std::memcpy(offsets, c->csr.rowOffsets.data(), c->csr.rowOffsets.size() * 4);
    std::memcpy(sources, c->csr.sourceIds.data(), c->csr.sourceIds.size() * 4);
    std::memcpy(values, c->csr.values.data(), c->csr.values.size() * 4);
}

void ref_csr_free(void* h) { delete static_cast<RefCsr*>(h); }

// convertCsrToSw32 (reference include/format/sw32.h:43-44) on raw canonical CSR arrays.
int ref_convert(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                const std::uint32_t* offsets, const std::uint32_t* sources, const float* values,
                int bucket, void** out) {
    try {
        CsrMatrix csr;
        csr.rowOffsets.assign(offsets, offsets + std::size_t(rows) + 1);
        csr.sourceIds.assign(sources, sources + nnz);
        csr.values.assign(values, values + nnz);
        auto* f = new Sw32HostFormat(convertCsrToSw32(rows, cols, csr, bucket != 0));
        *out = f;
        return 0;
    } catch (const std::exception& e) {
        return classify(e);
    }
}

// Array accessors: index 0 windowOffsets, 1 sourceIds, 2 rowGroupMasks, 3 sourceMetadata,
// 4 values, 5 bucketOffsets, 6 tasks, 7 reductions, 8 partialIds. Returns the byte size and
// stores the data pointer.
std::uint64_t ref_array(void* h, int which, const void** data) {
    auto* f = static_cast<Sw32HostFormat*>(h);
    switch (which) {
    case 0: *data = f->windowOffsets.data(); return f->windowOffsets.size() * 4;
    case 1: *data = f->sourceIds.data(); return f->sourceIds.size() * 4;
    case 2: *data = f->rowGroupMasks.data(); return f->rowGroupMasks.size() * 4;
    case 3: *data = f->sourceMetadata.data(); return f->sourceMetadata.size() * 8;
    case 4: *data = f->values.data(); return f->values.size() * 4;
    case 5: *data = f->bucketOffsets.data(); return f->bucketOffsets.size() * 4;
    case 6: *data = f->tasks.data(); return f->tasks.size() * sizeof(Sw32Task);
    case 7: *data = f->reductions.data(); return f->reductions.size() * sizeof(Sw32ReduceRange);
    case 8: *data = f->partialIds.data(); return f->partialIds.size() * 4;
    default: *data = nullptr; return 0;
    }
}

std::uint32_t ref_partial_count(void* h) { return static_cast<Sw32HostFormat*>(h)->partialCount; }

void ref_free(void* h) { delete static_cast<Sw32HostFormat*>(h); }
}
