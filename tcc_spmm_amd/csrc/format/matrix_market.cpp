// Matrix Market coordinate reader (host). Accepts the same files and reports the same error
// classes as the reference's loadMatrixMarket (src/format/matrix_market.cpp:30-103):
// coordinate real/integer/pattern, general/symmetric, 1-based indices, symmetric off-diagonal
// entries mirrored, uint32 limits. The file is read once into memory and scanned twice (count,
// then fill in file order); the row-bucketed entries then go through makeCanonicalCsr.
#include "format/csr.h"

#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

std::string lower(std::string s) {
    for (char& c : s) c = char(std::tolower(static_cast<unsigned char>(c)));
    return s;
}

// Cursor over the file text, one line at a time.
struct Lines {
    const char* p;
    const char* end;
    // Next line that is neither blank nor a '%' comment (leading spaces, tabs and CR ignored).
    bool nextData(const char*& b, const char*& e) {
        while (p < end) {
            const char* s = p;
            const char* nl = static_cast<const char*>(std::memchr(p, '\n', size_t(end - p)));
            const char* le = nl ? nl : end;
            p = nl ? nl + 1 : end;
            const char* q = s;
            while (q < le && (*q == ' ' || *q == '\t' || *q == '\r')) ++q;
            if (q < le && *q != '%') {
                b = s;
                e = le;
                return true;
            }
        }
        return false;
    }
};

// Parse an unsigned integer token; false if the line has no more tokens or the token is bad.
bool readU64(const char*& s, const char* e, std::uint64_t& v) {
    while (s < e && std::isspace(static_cast<unsigned char>(*s))) ++s;
    if (s >= e) return false;
    char buf[32];
    size_t n = 0;
    while (s < e && !std::isspace(static_cast<unsigned char>(*s)) && n < sizeof(buf) - 1)
        buf[n++] = *s++;
    buf[n] = 0;
    char* stop = nullptr;
    errno = 0;
    const unsigned long long x = std::strtoull(buf, &stop, 10);
    if (stop == buf || *stop || errno) return false;
    v = x;
    return true;
}

bool readFloat(const char*& s, const char* e, float& v) {
    while (s < e && std::isspace(static_cast<unsigned char>(*s))) ++s;
    if (s >= e) return false;
    char buf[64];
    size_t n = 0;
    while (s < e && !std::isspace(static_cast<unsigned char>(*s)) && n < sizeof(buf) - 1)
        buf[n++] = *s++;
    buf[n] = 0;
    char* stop = nullptr;
    const float x = std::strtof(buf, &stop);
    if (stop == buf || *stop) return false;
    v = x;
    return true;
}

} // namespace

MtxMatrix loadMatrixMarket(const std::string& path) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("cannot open Matrix Market file: " + path);
    std::string text;
    {
        char chunk[1 << 16];
        size_t got;
        while ((got = std::fread(chunk, 1, sizeof(chunk), f)) > 0) text.append(chunk, got);
        std::fclose(f);
    }
    const char* p = text.data();
    const char* end = p + text.size();
    const char* nl = static_cast<const char*>(std::memchr(p, '\n', text.size()));
    std::string header(p, nl ? nl : end);
    char tok[5][64] = {};
    const int got = std::sscanf(header.c_str(), "%63s %63s %63s %63s %63s", tok[0], tok[1], tok[2],
                                tok[3], tok[4]);
    const std::string banner = lower(got > 0 ? tok[0] : ""), object = lower(got > 1 ? tok[1] : "");
    const std::string storage = lower(got > 2 ? tok[2] : ""), field = lower(got > 3 ? tok[3] : "");
    const std::string symmetry = lower(got > 4 ? tok[4] : "");
    if (banner != "%%matrixmarket" || object != "matrix" || storage != "coordinate" ||
        (field != "real" && field != "integer" && field != "pattern") ||
        (symmetry != "general" && symmetry != "symmetric"))
        throw std::runtime_error(
            "expected a coordinate real/integer/pattern general/symmetric Matrix Market file");
    const bool pattern = field == "pattern", symmetric = symmetry == "symmetric";

    Lines lines{nl ? nl + 1 : end, end};
    const char *b, *e;
    if (!lines.nextData(b, e)) throw std::runtime_error("missing Matrix Market dimensions");
    constexpr std::uint64_t kMax = std::numeric_limits<std::uint32_t>::max();
    std::uint64_t rows64 = 0, cols64 = 0, entries64 = 0;
    if (!readU64(b, e, rows64) || !readU64(b, e, cols64) || !readU64(b, e, entries64) || !rows64 ||
        !cols64 || rows64 > kMax || cols64 > kMax || entries64 > kMax ||
        (symmetric && rows64 != cols64))
        throw std::runtime_error("invalid or unsupported Matrix Market dimensions");
    const auto rows = std::uint32_t(rows64), cols = std::uint32_t(cols64);
    const Lines body = lines;

    std::vector<std::uint32_t> offsets(std::size_t(rows) + 1, 0);
    auto scan = [&](auto consume) {
        Lines it = body;
        for (std::uint64_t i = 0; i < entries64; ++i) {
            if (!it.nextData(b, e)) throw std::runtime_error("truncated Matrix Market file");
            std::uint64_t row = 0, col = 0;
            float value = 1.0f;
            if (!readU64(b, e, row) || !readU64(b, e, col) || !row || row > rows || !col ||
                col > cols || (!pattern && !readFloat(b, e, value)) || !std::isfinite(value))
                throw std::runtime_error("invalid Matrix Market entry");
            consume(std::uint32_t(row - 1), std::uint32_t(col - 1), value);
            if (symmetric && row != col) consume(std::uint32_t(col - 1), std::uint32_t(row - 1), value);
        }
    };
    std::uint64_t expanded = 0;
    scan([&](std::uint32_t row, std::uint32_t, float) {
        if (++expanded > kMax)
            throw std::overflow_error("Matrix Market matrix exceeds uint32 CSR offsets");
        ++offsets[std::size_t(row) + 1];
    });
    for (std::size_t r = 1; r < offsets.size(); ++r) offsets[r] += offsets[r - 1];
    std::vector<std::uint32_t> columns(expanded), fill(offsets.begin(), offsets.end() - 1);
    std::vector<float> values(expanded);
    if (entries64)
        scan([&](std::uint32_t row, std::uint32_t col, float value) {
            const std::uint32_t at = fill[row]++;
            columns[at] = col;
            values[at] = value;
        });
    CsrMatrix csr = makeCanonicalCsr(rows, cols, std::uint32_t(expanded), offsets.data(),
                                     columns.data(), values.data());
    return {rows, cols, std::move(csr)};
}
