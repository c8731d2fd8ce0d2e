// Deterministic synthetic workloads for the benchmark configurations.
//
// Every random draw comes from SplitMix64 streams keyed by (seed, row), so the bytes produced are
// independent of the thread count and identical on every machine with IEEE doubles. Shapes:
//   c1  4,096 x 4,096, exactly 16 distinct uniform columns per row, values U[-1,1] (no exact 0).
//   c2  262,144 square, ~8.39M nnz: degrees from a discrete Pareto with the tail of Zipf(2.1),
//       clipped to [1, 20000] and scaled (bisection) to 32/row on average; columns 70% from the
//       row's 4,096-row community block, 30% uniform; values 1/sqrt(d_i d_j).
//   c3  2,449,029 square, exactly 126,167,053 nnz, mean degree ~51.5, power-law tail clipped at
//       17,000; 60% of a row's columns at offset +-|D| with |D| log-uniform in [1, 32768], 40%
//       uniform; values 1/sqrt(d_i d_j). The tail exponent is calibrated so that the task plan
//       matches the published Products statistics (~1,940 SWs above 384 panels, ~79K tasks).
//   c5  1,000,003 square: 5% empty rows, 64 hub rows (one per distinct SW) with 150,000 distinct
//       uniform columns, the rest Pareto(1.8)-tailed degrees clipped at C/2 and scaled to mean 20,
//       plus 15 planted columns in SW 0 covering every non-empty 4-bit row-group mask; values
//       U[-1,1].
//   t<rows>_<deg>_<seed>  square test matrix with `deg` distinct uniform columns per row.
// Columns of a row are drawn without replacement; every generated CSR is then passed through
// makeCanonicalCsr.
#include "generators.h"

#include "../parallel.h"
#include "format/csr.h"
#include "tcc_spmm_c.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

struct Rng {
    std::uint64_t s;
    explicit Rng(std::uint64_t seed, std::uint64_t stream)
        : s(seed * 0x9E3779B97F4A7C15ull ^ (stream + 0x632BE59BD9B4E019ull) * 0xD1B54A32D192ED03ull) {
        next();
    }
    std::uint64_t next() {
        std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return double(next() >> 11) * 0x1.0p-53; } // [0, 1)
    std::uint32_t below(std::uint32_t n) { return std::uint32_t((next() >> 32) * n >> 32); }
    float signedUnit() { // U[-1, 1) on a 2^-23 grid, never exactly 0
        for (;;) {
            const float v = float(std::int32_t(next() >> 40) - (1 << 23)) * 0x1.0p-23f;
            if (v != 0.0f) return v;
        }
    }
};

// Discrete Pareto draw with P(Z >= k) ~ k^-(alpha-1): the tail of Zipf(alpha).
inline double paretoTail(Rng& g, double alpha) {
    const double u = 1.0 - g.uniform(); // (0, 1]
    return std::floor(std::pow(u, -1.0 / (alpha - 1.0)));
}

struct Csr {
    std::uint32_t rows = 0, cols = 0;
    std::vector<std::uint32_t> offsets, columns;
    std::vector<float> values;
};

// Fill row `row`'s `deg` distinct sorted columns using `draw` (returns a candidate column); after
// `rounds` attempts the remaining columns come from the uniform distribution.
template <typename Draw>
void distinctColumns(Rng& g, std::uint32_t cols, std::uint32_t deg, Draw draw,
                     std::vector<std::uint32_t>& out) {
    out.clear();
    if (deg >= cols) {
        out.resize(cols);
        for (std::uint32_t c = 0; c < cols; ++c) out[c] = c;
        return;
    }
    for (int round = 0; out.size() < deg; ++round) {
        const std::size_t need = deg - out.size();
        for (std::size_t i = 0; i < need; ++i) out.push_back(round < 4 ? draw(g) : g.below(cols));
        std::sort(out.begin(), out.end());
        out.erase(std::unique(out.begin(), out.end()), out.end());
    }
}

void prefixOffsets(const std::vector<std::uint32_t>& degree, Csr& a) {
    a.offsets.assign(degree.size() + 1, 0);
    std::uint64_t run = 0;
    for (std::size_t i = 0; i < degree.size(); ++i) {
        run += degree[i];
        if (run > 0xFFFFFFFFull) throw std::overflow_error("synthetic matrix exceeds uint32 nnz");
        a.offsets[i + 1] = std::uint32_t(run);
    }
    a.columns.resize(run);
    a.values.resize(run);
}

// Generic row fill: columns for every row in parallel, then values from the final degrees.
template <typename Draw, typename Value>
void fillRows(Csr& a, std::uint64_t seed, const std::vector<std::uint32_t>& degree, Draw draw,
              Value value) {
    prefixOffsets(degree, a);
    tcc::parallelChunks(a.rows, std::min<std::size_t>(a.rows, 2048),
                        [&](std::size_t, std::size_t r0, std::size_t r1) {
                            std::vector<std::uint32_t> cols;
                            for (std::size_t r = r0; r < r1; ++r) {
                                Rng g(seed, r);
                                distinctColumns(g, a.cols, degree[r],
                                                [&](Rng& gg) { return draw(gg, std::uint32_t(r)); },
                                                cols);
                                std::copy(cols.begin(), cols.end(),
                                          a.columns.begin() + a.offsets[r]);
                            }
                        });
    tcc::parallelChunks(a.rows, std::min<std::size_t>(a.rows, 2048),
                        [&](std::size_t, std::size_t r0, std::size_t r1) {
                            for (std::size_t r = r0; r < r1; ++r) {
                                Rng g(seed ^ 0x5EEDull, r);
                                for (std::uint32_t e = a.offsets[r]; e < a.offsets[r + 1]; ++e)
                                    a.values[e] = value(g, std::uint32_t(r), a.columns[e]);
                            }
                        });
}

// Scale Pareto draws z_i to degrees clip(round(k z_i), lo, hi) with the total closest to `target`.
std::vector<std::uint32_t> scaledDegrees(const std::vector<double>& z, double target,
                                         std::uint32_t lo, std::uint32_t hi) {
    auto total = [&](double k) {
        double t = 0;
        for (double v : z) t += std::min<double>(hi, std::max<double>(lo, std::nearbyint(k * v)));
        return t;
    };
    double a = 1e-3, b = 1e6;
    for (int it = 0; it < 200; ++it) {
        const double m = std::sqrt(a * b);
        (total(m) < target ? a : b) = m;
    }
    const double k = std::sqrt(a * b);
    std::vector<std::uint32_t> d(z.size());
    for (std::size_t i = 0; i < z.size(); ++i)
        d[i] = std::uint32_t(std::min<double>(hi, std::max<double>(lo, std::nearbyint(k * z[i]))));
    return d;
}

// Adjust the last rows by +-1 until the degree total equals `target` exactly.
void trimToTotal(std::vector<std::uint32_t>& d, std::uint64_t target, std::uint32_t hi) {
    std::uint64_t sum = 0;
    for (auto v : d) sum += v;
    for (std::size_t i = d.size(); sum != target;) {
        i = (i == 0 ? d.size() : i) - 1;
        if (sum < target && d[i] < hi) {
            ++d[i];
            ++sum;
        } else if (sum > target && d[i] > 1) {
            --d[i];
            --sum;
        }
    }
}

Csr makeUniform(std::uint32_t n, std::uint32_t deg, std::uint64_t seed) {
    Csr a;
    a.rows = a.cols = n;
    std::vector<std::uint32_t> degree(n, std::min(deg, n));
    fillRows(
        a, seed, degree, [&](Rng& g, std::uint32_t) { return g.below(n); },
        [](Rng& g, std::uint32_t, std::uint32_t) { return g.signedUnit(); });
    return a;
}

Csr makeC2() {
    Csr a;
    a.rows = a.cols = 262144;
    const std::uint64_t seed = 2;
    std::vector<double> z(a.rows);
    for (std::uint32_t r = 0; r < a.rows; ++r) {
        Rng g(seed ^ 0xDE6ull, r);
        z[r] = paretoTail(g, 2.1);
    }
    auto degree = scaledDegrees(z, 8388608.0, 1, 20000);
    fillRows(
        a, seed, degree,
        [&](Rng& g, std::uint32_t r) {
            if (g.uniform() < 0.7) return (r & ~4095u) + g.below(4096);
            return g.below(a.cols);
        },
        [&](Rng&, std::uint32_t r, std::uint32_t c) {
            return float(1.0 / std::sqrt(double(degree[r]) * double(std::max(1u, degree[c]))));
        });
    return a;
}

Csr makeC3() {
    Csr a;
    a.rows = a.cols = 2449029;
    const std::uint64_t seed = 3;
    const std::uint64_t nnz = 126167053;
    std::vector<double> z(a.rows);
    for (std::uint32_t r = 0; r < a.rows; ++r) {
        Rng g(seed ^ 0xDE6ull, r);
        // Tail exponent 2.65 reproduces the reference's published plan statistics for Products
        // (1,943 split SWs, 78,801 tasks, ~15.2K partial tiles): here 1,941 / 79,199 / 14,731.
        z[r] = paretoTail(g, 2.65);
    }
    auto degree = scaledDegrees(z, double(nnz), 1, 17000);
    trimToTotal(degree, nnz, 17000);
    const double logSpan = std::log(32768.0);
    fillRows(
        a, seed, degree,
        [&](Rng& g, std::uint32_t r) -> std::uint32_t {
            if (g.uniform() < 0.6) {
                const std::uint32_t delta =
                    std::uint32_t(std::max(1.0, std::floor(std::exp(g.uniform() * logSpan))));
                const bool up = g.next() >> 63;
                const std::int64_t c = up ? std::int64_t(r) + delta : std::int64_t(r) - delta;
                if (c >= 0 && c < std::int64_t(a.cols)) return std::uint32_t(c);
                const std::int64_t m = up ? std::int64_t(r) - delta : std::int64_t(r) + delta;
                if (m >= 0 && m < std::int64_t(a.cols)) return std::uint32_t(m);
            }
            return g.below(a.cols);
        },
        [&](Rng&, std::uint32_t r, std::uint32_t c) {
            return float(1.0 / std::sqrt(double(degree[r]) * double(std::max(1u, degree[c]))));
        });
    return a;
}

Csr makeC5() {
    Csr a;
    a.rows = a.cols = 1000003;
    const std::uint64_t seed = 5;
    const std::uint32_t windows = (a.rows + 31) / 32;
    std::vector<double> z(a.rows);
    std::vector<std::uint8_t> empty(a.rows, 0), hub(a.rows, 0);
    for (std::uint32_t r = 0; r < a.rows; ++r) {
        Rng g(seed ^ 0xDE6ull, r);
        z[r] = std::min(paretoTail(g, 1.8), double(a.cols / 2));
        empty[r] = g.uniform() < 0.05;
    }
    {
        // 64 hub rows in 64 distinct SWs (never SW 0, which carries the planted masks).
        Rng g(seed ^ 0x4B5ull, 0);
        std::vector<std::uint8_t> taken(windows, 0);
        taken[0] = 1;
        for (int h = 0; h < 64;) {
            const std::uint32_t w = g.below(windows);
            if (taken[w]) continue;
            taken[w] = 1;
            const std::uint32_t r = std::min(a.rows - 1, w * 32 + g.below(32));
            hub[r] = 1;
            empty[r] = 0;
            ++h;
        }
    }
    double zsum = 0;
    std::uint64_t ordinary = 0;
    for (std::uint32_t r = 0; r < a.rows; ++r)
        if (!empty[r] && !hub[r]) {
            zsum += z[r];
            ++ordinary;
        }
    const double k = 20.0 * double(ordinary) / zsum;
    std::vector<std::uint32_t> degree(a.rows, 0);
    for (std::uint32_t r = 0; r < a.rows; ++r) {
        if (hub[r])
            degree[r] = 150000;
        else if (!empty[r])
            degree[r] = std::uint32_t(std::min<double>(a.cols / 2, std::max(1.0, std::nearbyint(k * z[r]))));
    }
    // SW 0 (rows 0..31) gets planted columns, so keep its rows non-empty for the plant below.
    Csr base;
    base.rows = base.cols = a.rows;
    fillRows(
        base, seed, degree, [&](Rng& g, std::uint32_t) { return g.below(a.cols); },
        [](Rng& g, std::uint32_t, std::uint32_t) { return g.signedUnit(); });
    // Plant one column per non-empty 4-bit mask m in SW 0: column 999000 + m appears in row
    // 8*g + (m % 8) for every row group g of m, so that source's RW mask is exactly m.
    std::vector<std::vector<std::pair<std::uint32_t, float>>> extra(32);
    for (unsigned m = 1; m < 16; ++m)
        for (unsigned grp = 0; grp < 4; ++grp)
            if (m >> grp & 1u)
                extra[grp * 8 + (m % 8)].push_back({999000u + m, 0.5f + 0.03125f * float(m)});
    a.offsets.assign(std::size_t(a.rows) + 1, 0);
    for (std::uint32_t r = 0; r < a.rows; ++r)
        a.offsets[r + 1] = a.offsets[r] + (base.offsets[r + 1] - base.offsets[r]) +
                           (r < 32 ? std::uint32_t(extra[r].size()) : 0u);
    a.columns.resize(a.offsets[a.rows]);
    a.values.resize(a.offsets[a.rows]);
    for (std::uint32_t r = 0; r < a.rows; ++r) {
        std::uint32_t at = a.offsets[r];
        for (std::uint32_t e = base.offsets[r]; e < base.offsets[r + 1]; ++e, ++at) {
            a.columns[at] = base.columns[e];
            a.values[at] = base.values[e];
        }
        if (r < 32)
            for (const auto& cv : extra[r]) { // duplicates with drawn columns are summed later
                a.columns[at] = cv.first;
                a.values[at++] = cv.second;
            }
    }
    return a;
}

} // namespace

SyntheticCsr makeSyntheticCsr(const std::string& name) {
    Csr a;
    if (name == "c1")
        a = makeUniform(4096, 16, 0);
    else if (name == "c2")
        a = makeC2();
    else if (name == "c3" || name == "c4")
        a = makeC3();
    else if (name == "c5")
        a = makeC5();
    else if (name.size() > 1 && name[0] == 't') {
        unsigned long n = 0, deg = 0, seed = 0;
        if (std::sscanf(name.c_str() + 1, "%lu_%lu_%lu", &n, &deg, &seed) != 3 || !n)
            throw std::invalid_argument("test config is t<rows>_<deg>_<seed>");
        a = makeUniform(std::uint32_t(n), std::uint32_t(deg), seed);
    } else {
        throw std::invalid_argument("unknown synthetic config: " + name);
    }
    CsrMatrix csr = makeCanonicalCsr(a.rows, a.cols, std::uint32_t(a.columns.size()),
                                     a.offsets.data(), a.columns.data(), a.values.data());
    return {a.rows, a.cols, std::move(csr)};
}

void makeSyntheticFeatures(std::uint32_t sources, std::uint32_t features, std::uint64_t seed,
                           float stddev, float outlierFraction, float outlierScale, float* out) {
    tcc::parallelChunks(sources, std::min<std::size_t>(sources, 4096),
                        [&](std::size_t, std::size_t r0, std::size_t r1) {
                            for (std::size_t r = r0; r < r1; ++r) {
                                Rng g(seed, r);
                                const bool outlier = g.uniform() < outlierFraction;
                                const double mul = stddev * (outlier ? outlierScale : 1.0f);
                                float* row = out + r * features;
                                for (std::uint32_t f = 0; f < features; f += 2) {
                                    // Box-Muller on (0,1] x [0,1)
                                    const double u1 = 1.0 - g.uniform(), u2 = g.uniform();
                                    const double rad = std::sqrt(-2.0 * std::log(u1));
                                    row[f] = float(mul * rad * std::cos(6.283185307179586 * u2));
                                    if (f + 1 < features)
                                        row[f + 1] = float(mul * rad * std::sin(6.283185307179586 * u2));
                                }
                            }
                        });
}

// Implemented in capi.cpp: wraps a CsrMatrix into the opaque handle.
extern "C" int tccWrapCsr(CsrMatrix&& csr, tcc_csr** out);
extern "C" void tccSetLastError(const char* message);

extern "C" int tcc_synth_csr(const char* config, std::uint32_t* rows, std::uint32_t* cols,
                             tcc_csr** out) {
    try {
        SyntheticCsr a = makeSyntheticCsr(config ? config : "");
        *rows = a.rows;
        *cols = a.cols;
        return tccWrapCsr(std::move(a.csr), out);
    } catch (const std::invalid_argument& e) {
        tccSetLastError(e.what());
        return TCC_INVALID_ARGUMENT;
    } catch (const std::overflow_error& e) {
        tccSetLastError(e.what());
        return TCC_OVERFLOW;
    } catch (const std::exception& e) {
        tccSetLastError(e.what());
        return TCC_OTHER;
    }
}

extern "C" int tcc_synth_features(std::uint32_t sources, std::uint32_t features, std::uint64_t seed,
                                  float stddev, float outlierFraction, float outlierScale,
                                  float* out) {
    try {
        makeSyntheticFeatures(sources, features, seed, stddev, outlierFraction, outlierScale, out);
        return TCC_OK;
    } catch (const std::exception& e) {
        tccSetLastError(e.what());
        return TCC_OTHER;
    }
}
