// ridge_predict.cpp -- the cost model's command line.
//
// Process contract (the reference's tools/ridge-predict.cpp:15-168, which the
// autotuner and the validator drive by subprocess):
//
//   ridge-predict [--gpu a100|mi355x | --hw model.json] [--m M --n N --k K]
//                 [--bm BM --bn BN --bk BK --warpm WM --warpn WN --stages S --regs R]
//                 [--groupm G --schedule S]            (this build's additions)
//                 [--batch in.csv --out out.csv]
//
// Batch mode: '#' lines are copied to the output as they are; the first other
// line is the header, copied with the prediction columns
//   pred_tflops,pred_bottleneck,pred_compute_ceiling,pred_hbm_ceiling,
//   pred_smem_eff,pred_occ_factor,pred_arith_intensity,pred_ctas_per_sm
// appended; every record is copied with its predictions appended, reals at 6
// significant digits (printf's %.6g, which is also an ostream's default
// rendering). Downstream ranking compares those strings, ties included, so the
// rendering is part of the contract. Config columns are found by name (M, N, K,
// BM, BN, BK, WM, WN, stages, regsPerThread, and this build's groupM and
// schedule); a column the table lacks keeps the GemmConfig default, other
// columns ride along untouched. One line on stderr names the constants used,
// "calibrated" or "placeholder".
//
// Errors (exit 1 with a message on stderr): an unknown option, an option
// without its value or with a value that is not an integer, an unreadable
// input, an unwritable output, a config field that is not an integer.

#include "ridge/hardware.h"
#include "ridge/model.h"

#include "../common/textio.hpp"

#include <cstdio>
#include <functional>
#include <string>
#include <vector>

using namespace ridge;

namespace {

const char* const kUsage =
    "ridge-predict: closed-form throughput of a matrix-core GEMM tile config, and what bounds it\n"
    "  ridge-predict [--gpu a100|mi355x | --hw model.json]\n"
    "                [--m M --n N --k K] [--bm BM --bn BN --bk BK --warpm WM --warpn WN]\n"
    "                [--stages S --regs R] [--groupm G --schedule -1|0|1|2]\n"
    "                [--batch in.csv --out out.csv]\n"
    "  schedule: -1 from the tile, 0 uniform, 1 ping-pong, 2 persistent\n"
    "  defaults: A100 placeholders, 4096^3, tile 128x128x32, wave tile 64x64, 3 stages\n";

const char* const kPredictionColumns =
    "pred_tflops,pred_bottleneck,pred_compute_ceiling,pred_hbm_ceiling,pred_smem_eff,pred_occ_factor,"
    "pred_arith_intensity,pred_ctas_per_sm";

using Setter = std::function<void(GemmConfig&, long long)>;

struct Field {
    const char* flag;    // command-line option
    const char* column;  // batch CSV column
    Setter set;
};

// The config fields reachable from the command line and from a batch table.
const std::vector<Field>& configFields() {
    static const std::vector<Field> fields = {
        {"--m", "M", [](GemmConfig& c, long long v) { c.M = v; }},
        {"--n", "N", [](GemmConfig& c, long long v) { c.N = v; }},
        {"--k", "K", [](GemmConfig& c, long long v) { c.K = v; }},
        {"--bm", "BM", [](GemmConfig& c, long long v) { c.BM = int(v); }},
        {"--bn", "BN", [](GemmConfig& c, long long v) { c.BN = int(v); }},
        {"--bk", "BK", [](GemmConfig& c, long long v) { c.BK = int(v); }},
        {"--warpm", "WM", [](GemmConfig& c, long long v) { c.warpM = int(v); }},
        {"--warpn", "WN", [](GemmConfig& c, long long v) { c.warpN = int(v); }},
        {"--stages", "stages", [](GemmConfig& c, long long v) { c.stages = int(v); }},
        {"--regs", "regsPerThread", [](GemmConfig& c, long long v) { c.regsPerThread = int(v); }},
        {"--groupm", "groupM", [](GemmConfig& c, long long v) { c.groupM = int(v); }},
        {"--schedule", "schedule", [](GemmConfig& c, long long v) { c.schedule = int(v); }},
    };
    return fields;
}

struct Invocation {
    std::string gpu = "a100";
    std::string hwPath, batchIn, batchOut = "predictions.csv";
    GemmConfig cfg;
    bool help = false;
};

bool parseArgs(int argc, char** argv, Invocation& inv, std::string& err) {
    const std::vector<std::pair<const char*, std::string*>> textOptions = {
        {"--gpu", &inv.gpu}, {"--hw", &inv.hwPath}, {"--batch", &inv.batchIn}, {"--out", &inv.batchOut}};
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        if (arg == "-h" || arg == "--help") {
            inv.help = true;
            continue;
        }
        const char* value = i + 1 < argc ? argv[i + 1] : nullptr;
        bool known = false;
        for (const auto& t : textOptions) {
            if (arg != t.first) continue;
            if (!value) return err = arg + " needs a value", false;
            *t.second = value;
            known = true;
        }
        for (const Field& f : configFields()) {
            if (arg != f.flag) continue;
            long long v = 0;
            if (!value || !ridgeio::toInteger(value, v)) return err = arg + " needs an integer value", false;
            f.set(inv.cfg, v);
            known = true;
        }
        if (!known) return err = "unknown option " + arg, false;
        ++i;
    }
    return true;
}

bool loadHardware(const Invocation& inv, HardwareModel& hw, std::string& err) {
    if (!inv.hwPath.empty()) return HardwareModel::loadFromJson(inv.hwPath, hw, err);
    if (inv.gpu == "a100") {
        hw = HardwareModel::a100();
        return true;
    }
    if (inv.gpu == "mi355x") {
        hw = HardwareModel::mi355x();
        return true;
    }
    err = "no built-in model for --gpu " + inv.gpu + " (a100, mi355x)";
    return false;
}

std::string predictionFields(const Prediction& p) {
    char buf[256];
    std::snprintf(buf, sizeof buf, "%.6g,%s,%.6g,%.6g,%.6g,%.6g,%.6g,%d", p.predictedTFLOPS, toString(p.bottleneck),
                  p.computeTFLOPS, p.hbmTFLOPS, p.smEfficiency, p.occFactor, p.arithmeticIntensity, p.ctasPerSM);
    return buf;
}

int runBatch(const Invocation& inv, const HardwareModel& hw) {
    std::vector<ridgeio::TableLine> lines;
    const ridgeio::Status st = ridgeio::readTable(inv.batchIn, lines);
    if (!st.ok()) {
        std::fprintf(stderr, "ridge-predict: %s\n", st.message().c_str());
        return 1;
    }
    std::string out;
    std::vector<std::pair<int, const Field*>> bound;  // (column position, field)
    int predicted = 0;
    for (const ridgeio::TableLine& line : lines) {
        switch (line.kind) {
            case ridgeio::TableLine::Comment:
                out += line.text + "\n";
                break;
            case ridgeio::TableLine::Header: {
                const ridgeio::ColumnIndex index(line.fields);
                for (const Field& f : configFields())
                    if (index[f.column] >= 0) bound.emplace_back(index[f.column], &f);
                out += line.text + "," + kPredictionColumns + "\n";
                break;
            }
            case ridgeio::TableLine::Record: {
                GemmConfig cfg;
                for (const auto& b : bound) {
                    if (b.first >= int(line.fields.size())) continue;
                    long long v = 0;
                    if (!ridgeio::toInteger(line.fields[b.first], v)) {
                        std::fprintf(stderr, "ridge-predict: %s:%zu: column %s holds \"%s\", not an integer\n",
                                     inv.batchIn.c_str(), line.number, b.second->column,
                                     line.fields[b.first].c_str());
                        return 1;
                    }
                    b.second->set(cfg, v);
                }
                out += line.text + "," + predictionFields(predict(cfg, hw)) + "\n";
                ++predicted;
                break;
            }
        }
    }
    std::FILE* f = std::fopen(inv.batchOut.c_str(), "wb");
    const bool written = f && std::fwrite(out.data(), 1, out.size(), f) == out.size();
    if (f && std::fclose(f) != 0) f = nullptr;
    if (!written || !f) {
        std::fprintf(stderr, "ridge-predict: could not write %s\n", inv.batchOut.c_str());
        return 1;
    }
    std::fprintf(stderr, "ridge-predict: %s constants (%s), %d configs -> %s\n",
                 hw.calibrated ? "calibrated" : "placeholder", hw.name.c_str(), predicted, inv.batchOut.c_str());
    return 0;
}

const char* scheduleName(int s) {
    switch (s) {
        case 0: return "uniform";
        case 1: return "ping-pong";
        case 2: return "persistent";
        default: return "from the tile";
    }
}

void describe(const GemmConfig& c, const HardwareModel& hw, const Prediction& p) {
    std::printf("%s [%s, %s constants]\n", hw.name.c_str(), hw.arch.c_str(),
                hw.calibrated ? "calibrated" : "placeholder");
    std::printf("  problem      %lld x %lld x %lld\n", (long long)c.M, (long long)c.N, (long long)c.K);
    std::printf("  tile         %d x %d x %d, wave tile %d x %d, %d stages, groupM %d, %s schedule, %d regs/lane\n",
                c.BM, c.BN, c.BK, c.warpM, c.warpN, c.stages, c.groupM, scheduleName(c.schedule), c.regsPerThread);
    if (p.bottleneck == Bottleneck::DoesNotFit) {
        std::printf("  result       %s: the workgroup's LDS, wave slots or registers exceed one CU\n",
                    toString(p.bottleneck));
        return;
    }
    std::printf("  result       %.1f TFLOP/s, bound by %s\n", p.predictedTFLOPS, toString(p.bottleneck));
    std::printf("  ceilings     matrix peak %.1f, compute %.1f, memory %.1f TFLOP/s\n", p.peakTensorTFLOPS,
                p.computeTFLOPS, p.hbmTFLOPS);
    std::printf("  K-step       %.0f cycles (matrix %.0f, operand reads %.0f); read efficiency %.3f\n",
                p.tStepCycles, p.tComputeCycles, p.tSmemCycles, p.smEfficiency);
    std::printf("  residency    %d waves per workgroup, %d workgroups per CU, latency factor %.3f\n", p.numWarps,
                p.ctasPerSM, p.occFactor);
    std::printf("  grid         %.0f workgroups over %.0f slots = %.2f waves, quantisation efficiency %.3f\n",
                p.totalCtas, p.ctaSlots, p.wavesExact, p.waveEfficiency);
    std::printf("  envelope     %.3f: %.0f K-steps, fill %.0f cycles, drain %.0f cycles\n", p.envelopeEfficiency,
                p.kSteps, p.tPrologueCycles, p.tEpilogueCycles);
    std::printf("  intensity    %.1f FLOP/B per tile, x%.2f cache reuse -> %.1f FLOP/B", p.baseIntensity,
                p.l2ReuseFactor, p.arithmeticIntensity);
    if (p.reuseTilesM > 0.0)
        std::printf(" (an XCD's resident tiles span %.0f x %.0f; compulsory %.1f)", p.reuseTilesM, p.reuseTilesN,
                    p.compulsoryIntensity);
    std::printf("\n");
}

}  // namespace

int main(int argc, char** argv) {
    Invocation inv;
    std::string err;
    if (!parseArgs(argc, argv, inv, err)) {
        std::fprintf(stderr, "ridge-predict: %s\n%s", err.c_str(), kUsage);
        return 1;
    }
    if (inv.help) {
        std::fputs(kUsage, stdout);
        return 0;
    }
    HardwareModel hw;
    if (!loadHardware(inv, hw, err)) {
        std::fprintf(stderr, "ridge-predict: %s\n", err.c_str());
        return 1;
    }
    if (!inv.batchIn.empty()) return runBatch(inv, hw);
    describe(inv.cfg, hw, predict(inv.cfg, hw));
    return 0;
}
