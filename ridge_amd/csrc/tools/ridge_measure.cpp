// ridge_measure.cpp -- times every registered shape against every kernel variant
// that divides it and writes the ground-truth CSV the model is validated against.
//
// Counterpart of the reference's bench/measure.cu:154-303, with the same
// discipline: the sweep file is registered before any measurement and a
// malformed row is fatal; every row carries provenance; a fixed comparator
// config (the canary, hipBLASLt at 4096^3) is re-timed every 25 measurements and
// a drift above 5% fails the run; a variant that cannot be measured is a failure,
// not a silent skip.
//
//   ridge-measure [sweep.csv] [out.csv] [--allow-skip] [--allow-partitioned] [--warmup-seconds S]
//                 [--settle-seconds T]
//
// --settle-seconds (default 0.2): every timed measurement -- each variant, each
// hipBLASLt comparator and each canary -- first runs its own workload untimed for
// T seconds. The reference locks the SM clock (setup-box.sh); MI355X clocks
// cannot be locked and follow the power drawn by the current workload, so
// without a settle a short measurement partly runs at the previous workload's
// clock (unsettled 4096^3 canaries spread 6.1% over one sweep, with no trend).
// The settle makes every figure a steady-state figure for its own work.
//
// --allow-skip: variants that do not divide a shape are recorded as skipped
// instead of failing (for shapes such as N = 128 that only some tiles divide).
//
// Columns: M,N,K,tag,BM,BN,BK,WM,WN,stages,groupM,regsPerThread,smemBytes,threads,
// tflops,blas_tflops,fraction_of_blas,canary_tflops,ms,iters,schedule -- the
// reference's columns (measure.cu:227-234, with its cuBLAS pair now hipBLASLt)
// plus the per-launch time, the iteration count and the row's schedule
// (0 uniform, 1 ping-pong, 2 persistent; ridge_gemm_variant_t.schedule).

#include "harness.hpp"

#include <filesystem>
#include <fstream>
#include <sstream>

using namespace ridgeh;

namespace {

constexpr int kCanaryEvery = 25;
constexpr double kCanaryMaxDrift = 0.05;

struct Shape {
    int M, N, K;
    std::string tag;
};

std::vector<Shape> loadRegisteredSweep(const char* path) {
    std::ifstream in(path);
    if (!in) {
        std::fprintf(stderr, "cannot open %s\n", path);
        std::exit(2);
    }
    std::vector<Shape> shapes;
    std::string line;
    int lineNo = 0;
    while (std::getline(in, line)) {
        ++lineNo;
        if (line.empty() || line[0] == '#') continue;
        std::istringstream ss(line);
        std::string m, n, k, tag;
        if (!std::getline(ss, m, ',') || !std::getline(ss, n, ',') || !std::getline(ss, k, ',') ||
            !std::getline(ss, tag, ',')) {
            std::fprintf(stderr, "%s:%d: malformed row: %s\n", path, lineNo, line.c_str());
            std::exit(2);
        }
        char* e1 = nullptr;
        char* e2 = nullptr;
        char* e3 = nullptr;
        const long Mv = std::strtol(m.c_str(), &e1, 10), Nv = std::strtol(n.c_str(), &e2, 10),
                   Kv = std::strtol(k.c_str(), &e3, 10);
        if (*e1 || *e2 || *e3 || Mv <= 0 || Nv <= 0 || Kv <= 0) {
            std::fprintf(stderr, "%s:%d: malformed row: %s\n", path, lineNo, line.c_str());
            std::exit(2);
        }
        shapes.push_back({int(Mv), int(Nv), int(Kv), tag});
    }
    if (shapes.empty()) {
        std::fprintf(stderr, "%s contains no shapes\n", path);
        std::exit(2);
    }
    return shapes;
}

}  // namespace

int main(int argc, char** argv) {
    std::vector<std::string> pos;
    bool allowSkip = false;
    bool allowPartitioned = false;
    double warmSeconds = 5.0;
    double settleSeconds = 0.2;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--allow-skip") allowSkip = true;
        else if (a == "--allow-partitioned") allowPartitioned = true;
        else if (a == "--warmup-seconds" && i + 1 < argc) warmSeconds = std::atof(argv[++i]);
        else if (a == "--settle-seconds" && i + 1 < argc) settleSeconds = std::atof(argv[++i]);
        else pos.push_back(a);
    }
    const std::string sweepPath = pos.size() > 0 ? pos[0] : "data/sweep/mi355x-registered.csv";
    const std::string outPath = pos.size() > 1 ? pos[1] : "data/measured/mi355x.csv";

    hipDeviceProp_t prop{};
    RIDGE_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("GPU: %s (%s), %d CUs, clock %.0f MHz\n", prop.name, prop.gcnArchName, prop.multiProcessorCount,
                prop.clockRate / 1000.0);
    requireWholeDevice(prop, allowPartitioned);

    const std::vector<Shape> shapes = loadRegisteredSweep(sweepPath.c_str());
    const int nv = ridge_gemm_num_variants();
    std::printf("sweep: %s, %zu shapes, %d variants\n", sweepPath.c_str(), shapes.size(), nv);

    // Prove the output is writable before spending GPU time.
    {
        std::error_code ec;
        const std::filesystem::path p(outPath);
        if (p.has_parent_path()) std::filesystem::create_directories(p.parent_path(), ec);
        std::ofstream probe(outPath, std::ios::app);
        if (!probe) {
            std::fprintf(stderr, "cannot write %s\n", outPath.c_str());
            return 2;
        }
    }

    // One allocation for the largest shape, reused, so allocator time and
    // first-touch stay out of the measured region.
    size_t maxA = size_t(4096) * 4096, maxB = maxA, maxC = maxA;
    for (const Shape& s : shapes) {
        maxA = std::max(maxA, size_t(s.M) * s.K);
        maxB = std::max(maxB, size_t(s.K) * s.N);
        maxC = std::max(maxC, size_t(s.M) * s.N);
    }
    void *dA = nullptr, *dB = nullptr, *dC = nullptr;
    RIDGE_HIP_CHECK(hipMalloc(&dA, maxA * 2));
    RIDGE_HIP_CHECK(hipMalloc(&dB, maxB * 2));
    RIDGE_HIP_CHECK(hipMalloc(&dC, maxC * 2));
    RIDGE_ABI_CHECK(ridge_fill_uniform_f16(dA, maxA, 1, nullptr));
    RIDGE_ABI_CHECK(ridge_fill_uniform_f16(dB, maxB, 2, nullptr));
    RIDGE_HIP_CHECK(hipDeviceSynchronize());

    BlasLt blas;
    const double canaryFlops = 2.0 * 4096.0 * 4096.0 * 4096.0;
    blas.prepare(dA, dB, dC, 4096, 4096, 4096);
    std::printf("warmup %.0fs\n", warmSeconds);
    warmUp([&] { blas.gemm(dA, dB, dC, 4096, 4096, 4096); }, warmSeconds);
    auto canaryBody = [&] { blas.gemm(dA, dB, dC, 4096, 4096, 4096); };
    auto measureCanary = [&] {
        warmUp(canaryBody, settleSeconds);
        return timeTflops(canaryBody, canaryFlops).tflops;
    };
    const double canaryFirst = measureCanary();
    double canaryNow = canaryFirst, canaryMin = canaryFirst, canaryMax = canaryFirst;
    std::printf("canary (hipBLASLt 4096^3) %.2f TFLOP/s\n\n", canaryFirst);

    std::ofstream out(outPath);
    if (!out) {
        std::fprintf(stderr, "cannot write %s\n", outPath.c_str());
        return 2;
    }
    out << "# gpu," << prop.name << " " << prop.gcnArchName << "\n"
        << "# cus," << prop.multiProcessorCount << "\n"
        << "# nominal_clock_mhz," << prop.clockRate / 1000.0 << "\n"
        << "# sweep," << sweepPath << "\n"
        << "# kernel_library," << ridge_gemm_build_info() << "\n"
        << "# inputs,U[-1;1) fp16 splitmix64 seeds 1 and 2\n"
        << "# warmup_seconds," << warmSeconds << "\n"
        << "# settle_seconds," << settleSeconds << "\n"
        << "# canary_start_tflops," << canaryFirst << "\n"
        << "M,N,K,tag,BM,BN,BK,WM,WN,stages,groupM,regsPerThread,smemBytes,threads,"
           "tflops,blas_tflops,fraction_of_blas,canary_tflops,ms,iters,schedule\n";
    out.flush();

    int measurements = 0, skipped = 0, failed = 0;
    for (const Shape& s : shapes) {
        const double flops = 2.0 * s.M * s.N * s.K;
        blas.prepare(dA, dB, dC, s.M, s.N, s.K);
        auto blasBody = [&] { blas.gemm(dA, dB, dC, s.M, s.N, s.K); };
        warmUp(blasBody, settleSeconds);
        const double blasTflops = timeTflops(blasBody, flops).tflops;
        std::printf("%5dx%5dx%5d  %-24s  hipBLASLt %8.2f TFLOP/s\n", s.M, s.N, s.K, s.tag.c_str(), blasTflops);
        std::fflush(stdout);
        for (int v = 0; v < nv; ++v) {
            ridge_gemm_variant_t kv;
            RIDGE_ABI_CHECK(ridge_gemm_get_variant(v, &kv));
            if (!ridge_gemm_divides(v, s.M, s.N, s.K)) {
                std::printf("    skip variant %d (%dx%dx%d), does not divide this shape\n", v, kv.BM, kv.BN, kv.BK);
                ++skipped;
                continue;
            }
            const int rc = ridge_gemm_launch(v, dA, dB, dC, s.M, s.N, s.K, nullptr);
            if (rc != 0 || hipDeviceSynchronize() != hipSuccess) {
                std::printf("    variant %d launch failed (%d)\n", v, rc);
                ++failed;
                continue;
            }
            auto body = [&] { ridge_gemm_launch(v, dA, dB, dC, s.M, s.N, s.K, nullptr); };
            warmUp(body, settleSeconds);
            const Timing t = timeTflops(body, flops);
            if (++measurements % kCanaryEvery == 0) {
                canaryNow = measureCanary();
                canaryMin = std::min(canaryMin, canaryNow);
                canaryMax = std::max(canaryMax, canaryNow);
            }
            out << s.M << ',' << s.N << ',' << s.K << ',' << s.tag << ',' << kv.BM << ',' << kv.BN << ',' << kv.BK
                << ',' << kv.WM << ',' << kv.WN << ',' << kv.stages << ',' << kv.groupM << ',' << kv.regsPerThread
                << ',' << kv.ldsBytes << ',' << kv.threads << ',' << t.tflops << ',' << blasTflops << ','
                << (t.tflops / blasTflops) << ',' << canaryNow << ',' << t.ms << ',' << t.iters << ','
                << kv.schedule << '\n';
            out.flush();
            std::printf("    %2d %3dx%3dx%2d w%3dx%3d s%d g%-2d  %8.2f TFLOP/s  %5.1f%% of hipBLASLt\n", v, kv.BM,
                        kv.BN, kv.BK, kv.WM, kv.WN, kv.stages, kv.groupM, t.tflops, 100.0 * t.tflops / blasTflops);
            std::fflush(stdout);
        }
    }

    const double canaryLast = measureCanary();
    canaryMin = std::min(canaryMin, canaryLast);
    canaryMax = std::max(canaryMax, canaryLast);
    const double drift = (canaryMax - canaryMin) / canaryMax;
    out << "# canary_end_tflops," << canaryLast << "\n"
        << "# canary_min_tflops," << canaryMin << "\n"
        << "# canary_max_tflops," << canaryMax << "\n"
        << "# canary_drift_fraction," << drift << "\n";
    out.close();
    std::printf("\nwrote %d measurements to %s, %d skipped, %d failed\n", measurements, outPath.c_str(), skipped,
                failed);
    std::printf("canary: start %.2f, end %.2f, min %.2f, max %.2f, drift %.1f%%\n", canaryFirst, canaryLast,
                canaryMin, canaryMax, drift * 100.0);
    RIDGE_HIP_CHECK(hipFree(dA));
    RIDGE_HIP_CHECK(hipFree(dB));
    RIDGE_HIP_CHECK(hipFree(dC));
    if (failed != 0) return 1;
    if (skipped != 0 && !allowSkip) {
        std::printf("\n%d configs skipped, so the measured set no longer matches the sweep\n", skipped);
        return 1;
    }
    if (drift > kCanaryMaxDrift) {
        std::printf("\ncanary drifted %.1f%%, above the %.0f%% limit\n", drift * 100.0, kCanaryMaxDrift * 100.0);
        return 1;
    }
    return 0;
}
