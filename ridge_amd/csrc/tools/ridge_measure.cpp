// ridge_measure.cpp -- the ground truth the model is judged against: every
// registered shape timed on every kernel-table row that divides it.
//
//   ridge-measure [sweep.csv] [out.csv] [--allow-skip] [--allow-partitioned]
//                 [--warmup-seconds S] [--settle-seconds T]
//   ridge-measure --plans plans.csv out.csv [...]
//
// Counterpart of the reference's bench/measure.cu:154-303. Its discipline is
// kept: the shapes come from a list registered before any measurement (read by
// the shared reader, common/textio.hpp, which refuses a malformed record);
// every row carries the provenance of the run; a fixed comparator workload (the
// canary: hipBLASLt at 4096^3) is re-timed every 25 measurements and a drift
// above 5% fails the run; a row that cannot be measured fails the run instead
// of disappearing from it.
//
// --settle-seconds (default 0.2): every timed workload -- each row, each
// hipBLASLt comparator, each canary -- first runs untimed for T seconds. MI355X
// clocks cannot be locked (the reference locks the SM clock in setup-box.sh)
// and follow the power the current work draws, so an unsettled measurement
// partly runs at the previous workload's clock (unsettled 4096^3 canaries
// spread 6.1% over one sweep, with no trend).
//
// --allow-skip: rows of the table that do not divide a shape are recorded as
// skipped instead of failing the run (for shapes such as N = 128).
//
// Output columns (the consumers key on them): M,N,K,tag,BM,BN,BK,WM,WN,stages,
// groupM,regsPerThread,smemBytes,threads,tflops,blas_tflops,fraction_of_blas,
// canary_tflops,ms,iters,schedule -- the reference's columns (measure.cu:227-234)
// with hipBLASLt as the comparator, plus the per-launch time, the iteration
// count and the row's schedule (0 uniform, 1 ping-pong, 2 persistent). '#'
// header and footer lines hold `key,value` provenance; the footer's canary
// drift is the range of every canary reading over their middle value.
//
// --plans: the registered list is of launch plans instead of shapes, one per
// record: M,N,K,tag, the body row's key (BM,BN,BK,WM,WN,stages,groupM),
// body_rows, and the tail row's key (tail_BM … tail_groupM). body_rows == M with
// a tail key of zeros is one launch of the body row; 0 < body_rows < M is a row
// split (ridge_gemm_launch_split). Every record is checked against the table
// before any GPU time is spent. Each distinct shape gets one hipBLASLt reading;
// the output repeats the plan's columns and adds the timing columns above
// (tflops … iters) and both rows' schedules. No extension of the reference (its
// measure.cu times one kernel per row).

#include "harness.hpp"

#include "../common/textio.hpp"

#include <cstdint>
#include <filesystem>
#include <memory>
#include <sstream>

using namespace ridgeh;

namespace {

constexpr int kCanaryPeriod = 25;
constexpr double kCanaryDriftLimit = 0.05;
constexpr int kCanaryDim = 4096;

struct Settings {
    std::string sweep = "data/sweep/mi355x-registered.csv";
    std::string out = "data/measured/mi355x.csv";
    bool plans = false;
    bool allowSkip = false;
    bool allowPartitioned = false;
    double warmSeconds = 5.0;
    double settleSeconds = 0.2;
};

bool parseSettings(int argc, char** argv, Settings& s) {
    int positional = 0;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        double* seconds = a == "--warmup-seconds" ? &s.warmSeconds : a == "--settle-seconds" ? &s.settleSeconds
                                                                                            : nullptr;
        if (a == "--allow-skip") {
            s.allowSkip = true;
        } else if (a == "--plans") {
            s.plans = true;
        } else if (a == "--allow-partitioned") {
            s.allowPartitioned = true;
        } else if (seconds) {
            if (i + 1 >= argc || !ridgeio::toReal(argv[i + 1], *seconds) || *seconds < 0.0) {
                std::fprintf(stderr, "ridge-measure: %s needs a number of seconds\n", a.c_str());
                return false;
            }
            ++i;
        } else if (!a.empty() && a[0] == '-') {
            std::fprintf(stderr, "ridge-measure: unknown option %s\n", a.c_str());
            return false;
        } else if (positional < 2) {
            (positional++ == 0 ? s.sweep : s.out) = a;
        } else {
            std::fprintf(stderr, "ridge-measure: unexpected argument %s\n", a.c_str());
            return false;
        }
    }
    return true;
}

// Every reading of the canary in this run.
struct CanaryLog {
    std::vector<double> readings;
    double first() const { return readings.front(); }
    double last() const { return readings.back(); }
    double lowest() const { return *std::min_element(readings.begin(), readings.end()); }
    double highest() const { return *std::max_element(readings.begin(), readings.end()); }
    double drift() const { return dispersion(readings); }
};

struct Tally {
    int measured = 0, skipped = 0, failed = 0;
};

// One registered launch plan (--plans).
struct Plan {
    ridgeio::Shape shape;
    int body = -1, tail = -1, bodyRows = 0;
    int bodyKey[7] = {}, tailKey[7] = {};
    bool split() const { return tail >= 0; }
};

const char* const kKeyColumns[7] = {"BM", "BN", "BK", "WM", "WN", "stages", "groupM"};

ridgeio::Status readPlans(const std::string& path, std::vector<Plan>& out) {
    std::vector<ridgeio::TableLine> lines;
    ridgeio::Status st = ridgeio::readTable(path, lines);
    if (!st.ok()) return st;
    std::vector<std::string> want = {"M", "N", "K", "tag", "body_rows"};
    for (const char* c : kKeyColumns) {
        want.push_back(c);
        want.push_back(std::string("tail_") + c);
    }
    std::unique_ptr<ridgeio::ColumnIndex> col;
    std::vector<Plan> plans;
    for (const ridgeio::TableLine& line : lines) {
        if (line.kind == ridgeio::TableLine::Comment) continue;
        if (line.kind == ridgeio::TableLine::Header) {
            col.reset(new ridgeio::ColumnIndex(line.fields));
            for (const std::string& c : want)
                if ((*col)[c] < 0) return ridgeio::Status::failure(path, "the header has no column " + c);
            continue;
        }
        const std::string where = path + ":" + std::to_string(line.number);
        auto field = [&](const std::string& name) { return line.fields.at(size_t((*col)[name])); };
        auto integer = [&](const std::string& name, long long& v) {
            return size_t((*col)[name]) < line.fields.size() && ridgeio::toInteger(field(name), v);
        };
        Plan p;
        long long rows = 0, v = 0;
        if (!integer("M", p.shape.M) || !integer("N", p.shape.N) || !integer("K", p.shape.K) ||
            !integer("body_rows", rows) || p.shape.M <= 0 || p.shape.N <= 0 || p.shape.K <= 0 ||
            p.shape.M > INT32_MAX || p.shape.N > INT32_MAX || p.shape.K > INT32_MAX)
            return ridgeio::Status::failure(where, "M, N, K and body_rows must be integers, M, N, K positive");
        p.shape.tag = field("tag");
        bool tailZero = true;
        for (int i = 0; i < 7; ++i) {
            if (!integer(kKeyColumns[i], v)) return ridgeio::Status::failure(where, "bad body key");
            p.bodyKey[i] = int(v);
            if (!integer(std::string("tail_") + kKeyColumns[i], v)) return ridgeio::Status::failure(where, "bad tail key");
            p.tailKey[i] = int(v);
            tailZero = tailZero && v == 0;
        }
        const int M = int(p.shape.M), N = int(p.shape.N), K = int(p.shape.K);
        const int* b = p.bodyKey;
        p.body = ridge_gemm_find_variant(b[0], b[1], b[2], b[3], b[4], b[5], b[6]);
        if (p.body < 0) return ridgeio::Status::failure(where, "the body key is not a row of the table");
        if (rows == p.shape.M) {
            if (!tailZero) return ridgeio::Status::failure(where, "a one-launch plan (body_rows = M) has a zero tail key");
            if (!ridge_gemm_divides(p.body, M, N, K))
                return ridgeio::Status::failure(where, "the body row does not divide the shape");
        } else {
            const int* t = p.tailKey;
            p.tail = ridge_gemm_find_variant(t[0], t[1], t[2], t[3], t[4], t[5], t[6]);
            if (p.tail < 0) return ridgeio::Status::failure(where, "the tail key is not a row of the table");
            if (rows <= 0 || rows >= p.shape.M || !ridge_gemm_divides(p.body, int(rows), N, K) ||
                !ridge_gemm_divides(p.tail, M - int(rows), N, K))
                return ridgeio::Status::failure(where, "a split needs 0 < body_rows < M, the body row dividing "
                                                       "body_rows x N x K and the tail row the rest");
        }
        p.bodyRows = int(rows);
        plans.push_back(p);
    }
    if (plans.empty()) return ridgeio::Status::failure(path, "registers no plan");
    out.swap(plans);
    return ridgeio::Status();
}

std::string planRow(const Plan& p, const Timing& t, double blasTflops, double canary) {
    ridge_gemm_variant_t b, tv{};
    ridge_gemm_get_variant(p.body, &b);
    if (p.split()) ridge_gemm_get_variant(p.tail, &tv);
    std::ostringstream row;
    row << p.shape.M << ',' << p.shape.N << ',' << p.shape.K << ',' << p.shape.tag;
    for (int i = 0; i < 7; ++i) row << ',' << p.bodyKey[i];
    row << ',' << p.bodyRows;
    for (int i = 0; i < 7; ++i) row << ',' << p.tailKey[i];
    row << ',' << t.tflops << ',' << blasTflops << ',' << t.tflops / blasTflops << ',' << canary << ',' << t.ms
        << ',' << t.iters << ',' << b.schedule << ',' << (p.split() ? tv.schedule : -1) << '\n';
    return row.str();
}

std::string dataRow(const ridgeio::Shape& s, const ridge_gemm_variant_t& kv, const Timing& t, double blasTflops,
                    double canary) {
    std::ostringstream row;
    row << s.M << ',' << s.N << ',' << s.K << ',' << s.tag << ',' << kv.BM << ',' << kv.BN << ',' << kv.BK << ','
        << kv.WM << ',' << kv.WN << ',' << kv.stages << ',' << kv.groupM << ',' << kv.regsPerThread << ','
        << kv.ldsBytes << ',' << kv.threads << ',' << t.tflops << ',' << blasTflops << ',' << t.tflops / blasTflops
        << ',' << canary << ',' << t.ms << ',' << t.iters << ',' << kv.schedule << '\n';
    return row.str();
}

}  // namespace

int main(int argc, char** argv) {
    Settings cfg;
    if (!parseSettings(argc, argv, cfg)) return 2;

    std::vector<ridgeio::Shape> shapes;
    std::vector<Plan> plans;
    const ridgeio::Status st = cfg.plans ? readPlans(cfg.sweep, plans) : ridgeio::readShapes(cfg.sweep, shapes);
    if (!st.ok()) {
        std::fprintf(stderr, "ridge-measure: %s\n", st.message().c_str());
        return 2;
    }
    // The list is read and checked before the device is touched.
    hipDeviceProp_t prop{};
    RIDGE_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("GPU: %s (%s), %d CUs, clock %.0f MHz\n", prop.name, prop.gcnArchName, prop.multiProcessorCount,
                prop.clockRate / 1000.0);
    requireWholeDevice(prop, cfg.allowPartitioned);

    const int rows = ridge_gemm_num_variants();
    if (cfg.plans)
        std::printf("registered plans %s: %zu launch plans\n", cfg.sweep.c_str(), plans.size());
    else
        std::printf("registered sweep %s: %zu shapes x %d table rows\n", cfg.sweep.c_str(), shapes.size(), rows);

    // The output is opened (and its directory made) before any GPU time is spent.
    std::error_code ec;
    const std::filesystem::path outPath(cfg.out);
    if (outPath.has_parent_path()) std::filesystem::create_directories(outPath.parent_path(), ec);
    std::FILE* out = std::fopen(cfg.out.c_str(), "w");
    if (!out) {
        std::fprintf(stderr, "ridge-measure: cannot open %s for writing\n", cfg.out.c_str());
        return 2;
    }
    auto emit = [out](const std::string& text) {
        std::fputs(text.c_str(), out);
        std::fflush(out);
    };

    // One set of operands, sized for the largest shape (and the canary), filled
    // once and reused, so allocation and first touch stay out of every timing.
    size_t elemsA = size_t(kCanaryDim) * kCanaryDim, elemsB = elemsA, elemsC = elemsA;
    std::vector<ridgeio::Shape> sized = shapes;
    for (const Plan& p : plans) sized.push_back(p.shape);
    for (const ridgeio::Shape& s : sized) {
        elemsA = std::max(elemsA, size_t(s.M * s.K));
        elemsB = std::max(elemsB, size_t(s.K * s.N));
        elemsC = std::max(elemsC, size_t(s.M * s.N));
    }
    void *dA = nullptr, *dB = nullptr, *dC = nullptr;
    RIDGE_HIP_CHECK(hipMalloc(&dA, elemsA * 2));
    RIDGE_HIP_CHECK(hipMalloc(&dB, elemsB * 2));
    RIDGE_HIP_CHECK(hipMalloc(&dC, elemsC * 2));
    RIDGE_ABI_CHECK(ridge_fill_uniform_f16(dA, elemsA, 1, nullptr));
    RIDGE_ABI_CHECK(ridge_fill_uniform_f16(dB, elemsB, 2, nullptr));
    RIDGE_HIP_CHECK(hipDeviceSynchronize());

    BlasLt blas;
    CanaryLog canary;
    const double canaryFlops = 2.0 * kCanaryDim * kCanaryDim * double(kCanaryDim);
    auto canaryLaunch = [&] { blas.gemm(dA, dB, dC, kCanaryDim, kCanaryDim, kCanaryDim); };
    // The comparator keeps one plan per shape: the canary's is chosen once, here,
    // and every later reading runs that same plan.
    auto readCanary = [&] {
        warmUp(canaryLaunch, cfg.settleSeconds);
        canary.readings.push_back(timeTflops(canaryLaunch, canaryFlops).tflops);
        return canary.last();
    };
    blas.prepare(dA, dB, dC, kCanaryDim, kCanaryDim, kCanaryDim);
    std::printf("warm-up: %.1f s of the canary workload\n", cfg.warmSeconds);
    warmUp(canaryLaunch, cfg.warmSeconds);
    std::printf("canary (hipBLASLt %d^3): %.2f TFLOP/s\n\n", kCanaryDim, readCanary());

    std::ostringstream head;
    head << "# gpu," << prop.name << " " << prop.gcnArchName << "\n"
         << "# cus," << prop.multiProcessorCount << "\n"
         << "# nominal_clock_mhz," << prop.clockRate / 1000.0 << "\n"
         << "# sweep," << cfg.sweep << "\n"
         << "# kernel_library," << ridge_gemm_build_info() << "\n"
         << "# inputs,U[-1;1) fp16 splitmix64 seeds 1 and 2\n"
         << "# warmup_seconds," << cfg.warmSeconds << "\n"
         << "# settle_seconds," << cfg.settleSeconds << "\n"
         << "# canary_start_tflops," << canary.first() << "\n";
    if (cfg.plans)
        head << "M,N,K,tag,BM,BN,BK,WM,WN,stages,groupM,body_rows,tail_BM,tail_BN,tail_BK,tail_WM,tail_WN,"
                "tail_stages,tail_groupM,tflops,blas_tflops,fraction_of_blas,canary_tflops,ms,iters,schedule,"
                "tail_schedule\n";
    else
        head << "M,N,K,tag,BM,BN,BK,WM,WN,stages,groupM,regsPerThread,smemBytes,threads,"
                "tflops,blas_tflops,fraction_of_blas,canary_tflops,ms,iters,schedule\n";
    emit(head.str());

    Tally tally;
    if (cfg.plans) {
        long long lastM = -1, lastN = -1, lastK = -1;
        double blasTflops = 0.0;
        for (const Plan& p : plans) {
            const int M = int(p.shape.M), N = int(p.shape.N), K = int(p.shape.K);
            const double flops = 2.0 * M * N * double(K);
            if (M != lastM || N != lastN || K != lastK) {
                blas.prepare(dA, dB, dC, M, N, K);
                auto blasLaunch = [&] { blas.gemm(dA, dB, dC, M, N, K); };
                warmUp(blasLaunch, cfg.settleSeconds);
                blasTflops = timeTflops(blasLaunch, flops).tflops;
                lastM = M, lastN = N, lastK = K;
                std::printf("%s  %dx%dx%d  hipBLASLt %.2f TFLOP/s\n", p.shape.tag.c_str(), M, N, K, blasTflops);
            }
            auto launch = [&] {
                return p.split() ? ridge_gemm_launch_split(p.body, p.tail, p.bodyRows, dA, dB, dC, M, N, K, nullptr)
                                 : ridge_gemm_launch(p.body, dA, dB, dC, M, N, K, nullptr);
            };
            const int rc = launch();
            const hipError_t sync = hipDeviceSynchronize();
            if (rc != 0 || sync != hipSuccess) {
                std::printf("    plan (row %d, %d rows, tail %d) could not run (launch %d, %s)\n", p.body, p.bodyRows,
                            p.tail, rc, hipGetErrorString(sync));
                ++tally.failed;
                continue;
            }
            warmUp([&] { launch(); }, cfg.settleSeconds);
            const Timing t = timeTflops([&] { launch(); }, flops);
            if (++tally.measured % kCanaryPeriod == 0) readCanary();
            emit(planRow(p, t, blasTflops, canary.last()));
            if (p.split())
                std::printf("    row %2d on %5d rows + row %2d  %8.2f TFLOP/s  %6.3f x hipBLASLt\n", p.body,
                            p.bodyRows, p.tail, t.tflops, t.tflops / blasTflops);
            else
                std::printf("    row %2d alone               %8.2f TFLOP/s  %6.3f x hipBLASLt\n", p.body, t.tflops,
                            t.tflops / blasTflops);
            std::fflush(stdout);
        }
    }
    for (const ridgeio::Shape& s : shapes) {
        const int M = int(s.M), N = int(s.N), K = int(s.K);
        const double flops = 2.0 * M * N * double(K);
        blas.prepare(dA, dB, dC, M, N, K);
        auto blasLaunch = [&] { blas.gemm(dA, dB, dC, M, N, K); };
        warmUp(blasLaunch, cfg.settleSeconds);
        const double blasTflops = timeTflops(blasLaunch, flops).tflops;
        std::printf("%s  %dx%dx%d  hipBLASLt %.2f TFLOP/s\n", s.tag.c_str(), M, N, K, blasTflops);
        std::fflush(stdout);
        for (int v = 0; v < rows; ++v) {
            ridge_gemm_variant_t kv;
            RIDGE_ABI_CHECK(ridge_gemm_get_variant(v, &kv));
            if (!ridge_gemm_divides(v, M, N, K)) {
                std::printf("    row %d (%dx%dx%d) does not divide the shape: skipped\n", v, kv.BM, kv.BN, kv.BK);
                ++tally.skipped;
                continue;
            }
            auto launch = [&] { return ridge_gemm_launch(v, dA, dB, dC, M, N, K, nullptr); };
            const int rc = launch();
            const hipError_t sync = hipDeviceSynchronize();
            if (rc != 0 || sync != hipSuccess) {
                std::printf("    row %d could not run (launch %d, %s)\n", v, rc, hipGetErrorString(sync));
                ++tally.failed;
                continue;
            }
            warmUp([&] { launch(); }, cfg.settleSeconds);
            const Timing t = timeTflops([&] { launch(); }, flops);
            if (++tally.measured % kCanaryPeriod == 0) readCanary();
            emit(dataRow(s, kv, t, blasTflops, canary.last()));
            std::printf("    %2d %3dx%3dx%2d w%3dx%3d s%d g%-2d  %8.2f TFLOP/s  %6.3f x hipBLASLt\n", v, kv.BM, kv.BN,
                        kv.BK, kv.WM, kv.WN, kv.stages, kv.groupM, t.tflops, t.tflops / blasTflops);
            std::fflush(stdout);
        }
    }

    readCanary();
    std::ostringstream foot;
    foot << "# canary_end_tflops," << canary.last() << "\n"
         << "# canary_min_tflops," << canary.lowest() << "\n"
         << "# canary_max_tflops," << canary.highest() << "\n"
         << "# canary_drift_fraction," << canary.drift() << "\n";
    emit(foot.str());
    std::fclose(out);
    RIDGE_HIP_CHECK(hipFree(dA));
    RIDGE_HIP_CHECK(hipFree(dB));
    RIDGE_HIP_CHECK(hipFree(dC));

    std::printf("\n%s: %d rows measured, %d skipped, %d could not run\n", cfg.out.c_str(), tally.measured,
                tally.skipped, tally.failed);
    std::printf("canary over %zu readings: first %.2f, last %.2f, range %.2f..%.2f = %.1f%% of the middle value\n",
                canary.readings.size(), canary.first(), canary.last(), canary.lowest(), canary.highest(),
                100.0 * canary.drift());
    int status = 0;
    if (tally.failed) status = 1;
    if (tally.skipped && !cfg.allowSkip) {
        std::printf("FAILED: %d table rows were skipped, so the measurement is not the registered cross product "
                    "(--allow-skip accepts that)\n", tally.skipped);
        status = 1;
    }
    if (canary.drift() > kCanaryDriftLimit) {
        std::printf("FAILED: the canary drifted %.1f%%, above the %.0f%% limit\n", 100.0 * canary.drift(),
                    100.0 * kCanaryDriftLimit);
        status = 1;
    }
    return status;
}
