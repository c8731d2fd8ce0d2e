// tcc_spmm_run: command-line harness for the fused INT8-dequantizing SpMM on one GPU.
//
// Counterpart of the reference's src/main.cu:1-114, invoked the same way:
//
//     tcc_spmm_run matrix.mtx 128|256 gpu_id
//
// It keeps the reference's inputs and protocol:
//   - the same feature values: a uniform [-1, 1) stream on a 2^-23 grid from std::mt19937 seeded with
//     20261025, row-major over cols x F (main.cu:11-17);
//   - the same untimed preparation: read, canonicalise, convert to SW32, upload, quantize, pack;
//   - the same timing: 10 warm-up launches, a device synchronize, then HIP events around 10
//     launches, reporting their mean (main.cu:30-51);
//   - the same result lines: "SpMM kernel average: <ms> ms" and "Output Y[0,0:8]: ...", and the same
//     exit status (1 with "Usage:" or "Error: <what>" on stderr).
//
// Options (none in the reference):
//   --config NAME      a synthetic workload (c1..c5, t<rows>_<deg>_<seed>) in place of the .mtx path
//   --warmup N         warm-up launches (default 10)
//   --iterations N     timed launches (default 10)
//   --normal-seed S    N(0,1) features from the synthetic generator with seed S instead
//   --json PATH        write the results as one JSON object
//   --save-y PATH      write Y (rows x F float32, row-major) to a raw file
#include "device_matrix.h"
#include "format/csr.h"
#include "format/int8_features.h"
#include "format/sw32.h"
#include "hip_support.h"
#include "spmm.h"
#include "synth/generators.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

struct Options {
    std::string matrixPath, config, jsonPath, savePath;
    unsigned features = 0;
    int device = 0;
    int warmup = 10, iterations = 10;
    bool normal = false;
    std::uint64_t normalSeed = 0;
};

// Uniform [-1, 1) features of the reference harness: the top 24 bits of each mt19937 output scaled
// by 2^-23, minus one.
std::vector<float> uniformFeatures(std::size_t count) {
    std::vector<float> x(count);
    std::mt19937 engine(20261025u);
    for (std::size_t i = 0; i < count; ++i)
        x[i] = float(engine() >> 8) * 0x1.0p-23f - 1.0f;
    return x;
}

// Algorithmic HBM bytes of one launch: the format read once, each referenced X row and scale once,
// Y written once, split partial tiles written and read once.
double algorithmicBytes(const Sw32HostFormat& f, std::uint64_t distinctSources, unsigned features) {
    const double sw = double(f.windowOffsets.size() - 1);
    const double a = 4.0 * f.values.size() + 12.0 * f.sourceIds.size() + 4.0 * f.rowGroupMasks.size() +
                     68.0 * sw + 28.0 * f.tasks.size() + 8.0 * f.reductions.size() +
                     4.0 * f.partialIds.size();
    const double x = double(features + 4) * double(distinctSources);
    const double y = 4.0 * double(f.rows) * features;
    const double p = 64.0 * features * double(f.partialCount);
    return a + x + y + p;
}

std::uint64_t countDistinctSources(const CsrMatrix& csr, std::uint32_t cols) {
    std::vector<unsigned char> seen(cols, 0);
    std::uint64_t n = 0;
    for (std::uint32_t s : csr.sourceIds)
        if (!seen[s]) {
            seen[s] = 1;
            ++n;
        }
    return n;
}

template <typename Launch> float timeLaunches(Launch launch, int warmup, int iterations) {
    for (int i = 0; i < warmup; ++i) launch();
    checkHip(hipDeviceSynchronize());
    hipEvent_t start, stop;
    checkHip(hipEventCreate(&start));
    checkHip(hipEventCreate(&stop));
    checkHip(hipEventRecord(start, nullptr));
    for (int i = 0; i < iterations; ++i) launch();
    checkHip(hipEventRecord(stop, nullptr));
    checkHip(hipEventSynchronize(stop));
    float ms = 0.0f;
    checkHip(hipEventElapsedTime(&ms, start, stop));
    hipEventDestroy(start);
    hipEventDestroy(stop);
    return iterations ? ms / float(iterations) : 0.0f;
}

std::string jsonString(const std::string& s) {
    std::string out = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') out += '\\';
        if (static_cast<unsigned char>(c) < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            out += buf;
        } else {
            out += c;
        }
    }
    return out + "\"";
}

void run(const Options& o) {
    checkHip(hipSetDevice(o.device));
    hipDeviceProp_t prop{};
    checkHip(hipGetDeviceProperties(&prop, o.device));
    const std::string source = o.config.empty() ? o.matrixPath : "config:" + o.config;
    std::cout << "GPU " << o.device << ": " << prop.name << " (" << prop.gcnArchName << ")\n";

    // 1. Canonical CSR from the file or the generator, then the SW32 format and its task plan.
    std::uint32_t rows, cols;
    CsrMatrix csr;
    if (o.config.empty()) {
        std::cout << "Reading Matrix Market: " << o.matrixPath << std::endl;
        MtxMatrix m = loadMatrixMarket(o.matrixPath);
        rows = m.rows;
        cols = m.cols;
        csr = std::move(m.csr);
    } else {
        std::cout << "Generating synthetic matrix " << o.config << std::endl;
        SyntheticCsr m = makeSyntheticCsr(o.config);
        rows = m.rows;
        cols = m.cols;
        csr = std::move(m.csr);
    }
    const std::uint64_t nnz = csr.sourceIds.size();
    const std::uint64_t distinct = countDistinctSources(csr, cols);
    std::cout << "Converting " << rows << " x " << cols << ", nnz=" << nnz << " to SW32..." << std::endl;
    Sw32HostFormat format = convertCsrToSw32(rows, cols, csr);
    csr = CsrMatrix{};
    const std::uint64_t sw = format.windowOffsets.size() - 1, panels = format.rowGroupMasks.size(),
                        tasks = format.tasks.size(), partials = format.partialCount;
    const double bytes = algorithmicBytes(format, distinct, o.features);

    // 2. Upload A, its plan and the split-task workspace (counters zeroed).
    std::cout << "Uploading SW32 (" << sw << " SWs, " << panels << " panels, " << tasks << " tasks, "
              << partials << " partial tiles) and preparing features..." << std::endl;
    DeviceMatrix matrix(format, o.features);
    format = Sw32HostFormat{};

    // 3. INT8 X, prepared outside the timed region.
    const std::size_t elements = std::size_t(cols) * o.features;
    std::vector<float> hostX;
    if (o.normal) {
        hostX.resize(elements);
        makeSyntheticFeatures(cols, o.features, o.normalSeed, 1.0f, 0.0f, 1.0f, hostX.data());
    } else {
        hostX = uniformFeatures(elements);
    }
    DeviceBuffer<float> scales(cols), output(std::size_t(rows) * o.features);
    DeviceBuffer<std::int8_t> packedX(elements);
    {
        DeviceBuffer<float> x(hostX);
        std::vector<float>().swap(hostX);
        DeviceBuffer<std::int8_t> q(elements);
        quantizeFeaturesInt8(x.ptr, q.ptr, scales.ptr, cols, o.features);
        packFeaturesInt8x16(q.ptr, packedX.ptr, cols, o.features);
        checkHip(hipDeviceSynchronize());
    }

    // 4. The timed launches.
    std::cout << "Running fused INT8 dequantization + SpMM (F=" << o.features << ")..." << std::endl;
    const Sw32DeviceView view = matrix.view();
    const SpmmWorkspace workspace = matrix.workspace();
    const float ms = timeLaunches(
        [&] {
            launchSpmmInt8(view, packedX.ptr, scales.ptr, output.ptr, rows, cols, o.features,
                           workspace);
        },
        o.warmup, o.iterations);

    float first[8] = {};
    const std::size_t shown = std::min<std::size_t>(8, std::size_t(rows) * o.features);
    checkHip(hipMemcpy(first, output.ptr, shown * sizeof(float), hipMemcpyDeviceToHost));
    const double gbps = ms > 0.0f ? bytes / (double(ms) * 1e-3) / 1e9 : 0.0;
    std::cout << std::fixed << std::setprecision(6) << "SpMM kernel average: " << ms << " ms ("
              << o.iterations << " launches; includes dequantization)\n"
              << "Algorithmic HBM traffic: " << std::setprecision(1) << gbps << " GB/s ("
              << std::setprecision(1) << gbps / 80.0 << "% of 8 TB/s)\n"
              << "Not timed: matrix read, format conversion, upload, quantization and packing.\n"
              << std::setprecision(6) << "Output Y[0,0:8]:";
    for (std::size_t i = 0; i < shown; ++i) std::cout << ' ' << first[i];
    std::cout << '\n';

    if (!o.savePath.empty()) {
        std::vector<float> y(std::size_t(rows) * o.features);
        checkHip(hipMemcpy(y.data(), output.ptr, y.size() * sizeof(float), hipMemcpyDeviceToHost));
        std::ofstream f(o.savePath, std::ios::binary);
        f.write(reinterpret_cast<const char*>(y.data()), std::streamsize(y.size() * sizeof(float)));
        if (!f) throw std::runtime_error("cannot write " + o.savePath);
    }
    if (!o.jsonPath.empty()) {
        std::ostringstream j;
        j << std::setprecision(9);
        j << "{\"source\": " << jsonString(source) << ", \"rows\": " << rows << ", \"cols\": " << cols
          << ", \"nnz\": " << nnz << ", \"features\": " << o.features << ", \"gpu\": " << o.device
          << ", \"gpu_name\": " << jsonString(prop.name) << ", \"x\": "
          << (o.normal ? jsonString("normal:" + std::to_string(o.normalSeed))
                       : jsonString("mt19937:20261025"))
          << ", \"warmup\": " << o.warmup << ", \"iterations\": " << o.iterations
          << ", \"ms\": " << ms << ", \"sw\": " << sw << ", \"panels\": " << panels
          << ", \"tasks\": " << tasks << ", \"partial_count\": " << partials
          << ", \"distinct_sources\": " << distinct << ", \"algorithmic_bytes\": " << std::fixed
          << std::setprecision(0) << bytes << std::setprecision(3) << ", \"achieved_gbps\": " << gbps
          << std::defaultfloat << std::setprecision(9) << ", \"y0\": [";
        for (std::size_t i = 0; i < shown; ++i) j << (i ? ", " : "") << first[i];
        j << "]}\n";
        std::ofstream f(o.jsonPath);
        f << j.str();
        if (!f) throw std::runtime_error("cannot write " + o.jsonPath);
    }
}

int usage(const char* argv0) {
    std::cerr << "Usage: " << argv0 << " [options] matrix.mtx 128|256 gpu_id\n"
              << "       " << argv0 << " [options] --config c1|c2|c3|c4|c5|t<rows>_<deg>_<seed> 128|256 gpu_id\n"
              << "options: --warmup N  --iterations N  --normal-seed S  --json PATH  --save-y PATH\n";
    return 1;
}

int parseCount(const std::string& v, const char* what) {
    std::size_t used = 0;
    const long n = std::stol(v, &used);
    if (used != v.size() || n < 0 || n > 1000000)
        throw std::invalid_argument(std::string(what) + " must be an integer in [0, 1000000]");
    return int(n);
}

} // namespace

int main(int argc, char** argv) {
    Options o;
    std::vector<std::string> positional;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        const bool takesValue = a == "--config" || a == "--warmup" || a == "--iterations" ||
                                a == "--normal-seed" || a == "--json" || a == "--save-y";
        if (takesValue) {
            if (i + 1 >= argc) return usage(argv[0]);
            const std::string v = argv[++i];
            try {
                if (a == "--config") o.config = v;
                else if (a == "--warmup") o.warmup = parseCount(v, "--warmup");
                else if (a == "--iterations") o.iterations = parseCount(v, "--iterations");
                else if (a == "--normal-seed") { o.normal = true; o.normalSeed = std::stoull(v); }
                else if (a == "--json") o.jsonPath = v;
                else o.savePath = v;
            } catch (const std::exception& e) {
                std::cerr << "Error: " << e.what() << '\n';
                return 1;
            }
        } else if (a.size() > 2 && a[0] == '-' && a[1] == '-') {
            return usage(argv[0]);
        } else {
            positional.push_back(a);
        }
    }
    const std::size_t expected = o.config.empty() ? 3 : 2;
    if (positional.size() != expected) return usage(argv[0]);
    try {
        if (o.config.empty()) o.matrixPath = positional[0];
        const unsigned long features = std::stoul(positional[expected - 2]);
        if (features != 128 && features != 256)
            throw std::invalid_argument("feature dimension must be 128 or 256");
        o.features = unsigned(features);
        o.device = std::stoi(positional[expected - 1]);
        run(o);
    } catch (const std::exception& e) {
        std::cerr << "Error: " << e.what() << '\n';
        return 1;
    }
    return 0;
}
