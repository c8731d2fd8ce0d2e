// Small host-side thread helpers for the format builders and generators.
#pragma once
#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <exception>
#include <mutex>
#include <thread>
#include <vector>

namespace tcc {

// Worker count: TCC_THREADS if set, else the hardware concurrency, capped at 64.
inline unsigned hostThreads() {
    if (const char* env = std::getenv("TCC_THREADS")) {
        long v = std::strtol(env, nullptr, 10);
        if (v > 0) return unsigned(std::min<long>(v, 256));
    }
    unsigned n = std::thread::hardware_concurrency();
    return std::max(1u, std::min(n ? n : 1u, 64u));
}

// Run body(chunkIndex, begin, end) over [0, n) split into `chunks` contiguous ranges, on up to
// hostThreads() threads. If chunks throw, the exception of the lowest-indexed failing chunk is
// rethrown after all threads finish, so the error reported is the first in range order whatever the
// timing (a chunk that walks its range in order reports its first defect). Chunks after a failed
// one are skipped once the failure is known.
template <typename Body>
void parallelChunks(std::size_t n, std::size_t chunks, Body body) {
    if (chunks == 0) return;
    const unsigned workers = unsigned(std::min<std::size_t>(hostThreads(), chunks));
    std::exception_ptr error;
    std::size_t errorChunk = chunks; // lowest failing chunk so far
    std::mutex errorLock;
    auto failedBefore = [&](std::size_t c) {
        std::lock_guard<std::mutex> g(errorLock);
        return errorChunk < c;
    };
    auto run = [&](unsigned w) {
        for (std::size_t c = w; c < chunks; c += workers) {
            if (failedBefore(c)) break;
            try {
                body(c, n * c / chunks, n * (c + 1) / chunks);
            } catch (...) {
                std::lock_guard<std::mutex> g(errorLock);
                if (c < errorChunk) {
                    errorChunk = c;
                    error = std::current_exception();
                }
            }
        }
    };
    if (workers == 1) {
        run(0);
    } else {
        std::vector<std::thread> pool;
        pool.reserve(workers);
        for (unsigned w = 0; w < workers; ++w) pool.emplace_back(run, w);
        for (auto& t : pool) t.join();
    }
    if (error) std::rethrow_exception(error);
}

} // namespace tcc
