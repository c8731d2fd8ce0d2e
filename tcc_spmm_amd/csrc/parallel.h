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
// hostThreads() threads. The first exception thrown by any chunk is rethrown after all finish.
template <typename Body>
void parallelChunks(std::size_t n, std::size_t chunks, Body body) {
    if (chunks == 0) return;
    const unsigned workers = unsigned(std::min<std::size_t>(hostThreads(), chunks));
    std::exception_ptr error;
    std::mutex errorLock;
    auto run = [&](unsigned w) {
        for (std::size_t c = w; c < chunks; c += workers) {
            try {
                body(c, n * c / chunks, n * (c + 1) / chunks);
            } catch (...) {
                std::lock_guard<std::mutex> g(errorLock);
                if (!error) error = std::current_exception();
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
