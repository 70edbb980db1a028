// hardware.cpp -- built-in hardware models and the flat-JSON loader.
// Counterpart of the reference's src/hardware.cpp (a100 :19-34, loader :149-200):
// the same all-or-nothing contract and required keys, read through the build's
// shared text reader (common/textio.hpp) and a declarative key schema.

#include "ridge/hardware.h"

#include "../common/textio.hpp"

#include <cstdint>
#include <string>
#include <vector>

namespace ridge {

HardwareModel HardwareModel::a100() {
    // The reference's placeholders, value for value: they anchor its worked
    // example (test/test-model.cpp:47-101).
    HardwareModel h;
    h.name = "A100-80GB (datasheet placeholders, replace with calibration)";
    h.numSMs = 108;
    h.clockHz = 1.41e9;
    h.mmaCyclesPerInst = 2.0;
    h.smemBytesPerCycle = 128.0;
    h.hbmBytesPerSec = 2.0e12;
    h.regsPerSM = 65536;
    h.smemBytesPerSM = 167936;
    h.maxWarpsPerSM = 64;
    h.maxCtasPerSM = 32;
    h.warpsNeededToHide = 16.0;
    h.calibrated = false;
    return h;
}

HardwareModel HardwareModel::mi355x() {
    // Datasheet-derived placeholders for MI355X (gfx950):
    //   256 CUs (8 XCDs x 32) at a 2.4 GHz peak engine clock;
    //   v_mfma_f32_16x16x32_f16 = 16384 FLOP, one per SIMD per 16 cycles, four
    //     SIMDs per CU -> 4 CU-level cycles per instruction, i.e.
    //     16384 / 4 * 2.4e9 * 256 = 2516.6 TFLOP/s dense FP16;
    //   LDS 160 KiB per CU, 128 bytes per cycle (placeholder until measured);
    //   HBM3E 8.0 TB/s;
    //   4 SIMDs x 512 VGPR+AGPR per lane x 64 lanes = 131072 lane-registers per CU,
    //   allocated in granules of 8; 2048 workitems = 32 wavefronts per CU.
    HardwareModel h;
    h.name = "MI355X (datasheet placeholders, replace with calibration)";
    h.numSMs = 256;
    h.clockHz = 2.4e9;
    h.mmaCyclesPerInst = 4.0;
    h.smemBytesPerCycle = 128.0;
    h.hbmBytesPerSec = 8.0e12;
    h.regsPerSM = 131072;
    h.smemBytesPerSM = 163840;
    h.maxWarpsPerSM = 32;
    h.maxCtasPerSM = 32;
    h.warpsNeededToHide = 8.0;
    h.calibrated = false;
    h.arch = "gfx950";
    h.waveSize = 64;
    h.mmaM = 16;
    h.mmaN = 16;
    h.mmaK = 32;
    h.simdsPerSM = 4;
    h.regsPerSimdLane = 512;
    h.regGranule = 8;
    h.numXcds = 8;
    h.cBytes = 2;
    h.l2ReuseModel = 2;
    h.prologueModel = 1;
    h.pingPongModel = 1;
    h.persistentModel = 1;
    return h;
}

namespace {

// How one JSON key lands in a HardwareModel field. A required key must be
// present; a key marked `positive` must also be > 0 (a zero there would divide
// by zero or silently zero a ceiling). Keys the schema does not name (the
// calibration record: skeleton cycles, curves, the note) are ignored.
struct KeyRule {
    const char* key;
    bool required;
    bool positive;
    double* real;  // exactly one of real / integer is set
    int* integer;
};

std::vector<KeyRule> schemaFor(HardwareModel& h) {
    auto R = [](const char* k, double& f, bool req = false, bool pos = false) { return KeyRule{k, req, pos, &f, nullptr}; };
    auto I = [](const char* k, int& f, bool req = false, bool pos = false) { return KeyRule{k, req, pos, nullptr, &f}; };
    return {
        // The ten constants every hardware description carries (the
        // reference's required set); clock and the [CAL] rates must be positive.
        I("numSMs", h.numSMs, true, true), R("clockHz", h.clockHz, true, true),
        R("mmaCyclesPerInst", h.mmaCyclesPerInst, true, true), R("smemBytesPerCycle", h.smemBytesPerCycle, true, true),
        R("hbmBytesPerSec", h.hbmBytesPerSec, true, true), I("regsPerSM", h.regsPerSM, true),
        I("smemBytesPerSM", h.smemBytesPerSM, true), I("maxWarpsPerSM", h.maxWarpsPerSM, true),
        I("maxCtasPerSM", h.maxCtasPerSM, true), R("warpsNeededToHide", h.warpsNeededToHide, true, true),
        // Target description (defaults: the arch's built-in model).
        I("waveSize", h.waveSize), I("mmaM", h.mmaM), I("mmaN", h.mmaN), I("mmaK", h.mmaK),
        I("simdsPerSM", h.simdsPerSM), I("regsPerSimdLane", h.regsPerSimdLane), I("regGranule", h.regGranule),
        I("numXcds", h.numXcds), I("cBytes", h.cBytes),
        // Model terms and the constants they read.
        I("l2ReuseModel", h.l2ReuseModel), I("prologueModel", h.prologueModel), I("pingPongModel", h.pingPongModel),
        I("persistentModel", h.persistentModel), I("ldsReadModel", h.ldsReadModel),
        R("ldsAReadBytesPerCycle", h.ldsAReadBytesPerCycle), R("ldsBTrReadBytesPerCycle", h.ldsBTrReadBytesPerCycle),
        I("clockModel", h.clockModel), R("clockRatioHalfCus", h.clockRatio[0]),
        R("clockRatioQuarterCus", h.clockRatio[1]), R("clockRatioEighthCus", h.clockRatio[2]),
        R("clockRatioSixteenthCus", h.clockRatio[3]), I("l2StreamModel", h.l2StreamModel),
        R("l2HitBytesPerCycle", h.l2HitBytesPerCycle), I("uniformOverlapModel", h.uniformOverlapModel),
        R("freeRunningOverlap", h.freeRunningOverlap), I("powerModel", h.powerModel),
        R("loadedClockRatio", h.loadedClockRatio), R("warpsNeededToHideIlp8", h.warpsNeededToHideIlp8),
        I("hbmWriteModel", h.hbmWriteModel), R("hbmWriteBytesPerSec", h.hbmWriteBytesPerSec),
        I("writeOverlapModel", h.writeOverlapModel),
        I("fillLatencyModel", h.fillLatencyModel), R("fillLatencySec", h.fillLatencySec),
        I("mallStreamModel", h.mallStreamModel), R("mallRefillBytesPerSec", h.mallRefillBytesPerSec),
        R("mallStretchLoad0", h.mallStretchLoad[0]), R("mallStretchLoad1", h.mallStretchLoad[1]),
        R("mallStretchLoad2", h.mallStretchLoad[2]), R("mallStretchLoad3", h.mallStretchLoad[3]),
        R("mallStretchLoad4", h.mallStretchLoad[4]), R("mallStretch0", h.mallStretch[0]),
        R("mallStretch1", h.mallStretch[1]), R("mallStretch2", h.mallStretch[2]), R("mallStretch3", h.mallStretch[3]),
        R("mallStretch4", h.mallStretch[4]), I("persistentStepModel", h.persistentStepModel),
        R("persistentStepCycles1", h.persistentStepCycles[0]), R("persistentStepCycles2", h.persistentStepCycles[1]),
        I("persistentTileModel", h.persistentTileModel), R("persistentTileCycles1", h.persistentTileCycles[0]),
        R("persistentTileCycles2", h.persistentTileCycles[1]),
        I("fillShareModel", h.fillShareModel), I("mallReuseModel", h.mallReuseModel), R("mallBytes", h.mallBytes),
        I("mallWriteModel", h.mallWriteModel), R("mallWriteBytesPerSec", h.mallWriteBytesPerSec),
        I("pingPongStepModel", h.pingPongStepModel), R("pingPongRowStepCycles1", h.pingPongRowStepCycles[0]),
        R("pingPongRowStepCycles2", h.pingPongRowStepCycles[1]),
        I("launchModel", h.launchModel), R("launchOverheadSeconds", h.launchOverheadSeconds),
        R("launchIsolatedSeconds", h.launchIsolatedSeconds), I("labelModel", h.labelModel),
        R("nominalClockHz", h.nominalClockHz),
    };
}

ridgeio::Status applySchema(const ridgeio::FlatObject& kv, const std::vector<KeyRule>& schema) {
    for (const KeyRule& rule : schema) {
        const auto it = kv.find(rule.key);
        const std::string name = std::string("\"") + rule.key + "\"";
        if (it == kv.end()) {
            if (rule.required) return ridgeio::Status::failure("", "required constant " + name + " is absent");
            continue;
        }
        if (kv.quoted.count(rule.key))
            return ridgeio::Status::failure("", name + " must be a number, found the string \"" + it->second + "\"");
        double value = 0.0;
        if (rule.integer) {
            long long n = 0;
            if (!ridgeio::toInteger(it->second, n) || n < INT32_MIN || n > INT32_MAX)
                return ridgeio::Status::failure("", name + " must be an integer, found " + it->second);
            *rule.integer = static_cast<int>(n);
            value = double(n);
        } else {
            if (!ridgeio::toReal(it->second, value))
                return ridgeio::Status::failure("", name + " must be a number, found " + it->second);
            *rule.real = value;
        }
        if (rule.positive && !(value > 0.0))
            return ridgeio::Status::failure("", name + " must be positive, found " + it->second);
    }
    return ridgeio::Status();
}

// Consistency of a loaded model: target-description values in range and every
// switched-on term given the constants it reads. Empty when consistent.
std::string inconsistency(const HardwareModel& h) {
    if (h.waveSize <= 0 || h.mmaM <= 0 || h.mmaN <= 0 || h.mmaK <= 0 || h.regGranule <= 0 || h.numXcds <= 0 ||
        h.cBytes <= 0 || h.simdsPerSM < 0 || (h.simdsPerSM > 0 && h.regsPerSimdLane <= 0))
        return "the target description (waveSize, mma shape, register files, XCDs, cBytes) is out of range";
    // Every term switch takes only the values the model defines; any other value
    // would silently mean "off".
    const struct {
        const char* name;
        int value, max;
    } switches[] = {
        {"l2ReuseModel", h.l2ReuseModel, 2},     {"prologueModel", h.prologueModel, 1},
        {"pingPongModel", h.pingPongModel, 1},   {"persistentModel", h.persistentModel, 1},
        {"ldsReadModel", h.ldsReadModel, 1},     {"clockModel", h.clockModel, 1},
        {"l2StreamModel", h.l2StreamModel, 1},   {"uniformOverlapModel", h.uniformOverlapModel, 1},
        {"powerModel", h.powerModel, 1},         {"hbmWriteModel", h.hbmWriteModel, 1},
        {"writeOverlapModel", h.writeOverlapModel, 1},
        {"fillLatencyModel", h.fillLatencyModel, 1}, {"mallStreamModel", h.mallStreamModel, 1},
        {"persistentStepModel", h.persistentStepModel, 1}, {"persistentTileModel", h.persistentTileModel, 1},
        {"fillShareModel", h.fillShareModel, 1},
        {"mallReuseModel", h.mallReuseModel, 1}, {"mallWriteModel", h.mallWriteModel, 1},
        {"pingPongStepModel", h.pingPongStepModel, 1},
        {"launchModel", h.launchModel, 1},
        {"labelModel", h.labelModel, 2},
    };
    for (const auto& s : switches)
        if (s.value < 0 || s.value > s.max)
            return std::string(s.name) + " must be an integer from 0 to " + std::to_string(s.max) + ", found " +
                   std::to_string(s.value);
    if (h.ldsReadModel == 1 && !(h.ldsAReadBytesPerCycle > 0.0 && h.ldsBTrReadBytesPerCycle > 0.0))
        return "ldsReadModel 1 reads ldsAReadBytesPerCycle and ldsBTrReadBytesPerCycle, which must be positive";
    if (h.clockModel == 1 &&
        !(h.clockRatio[0] > 0.0 && h.clockRatio[1] > 0.0 && h.clockRatio[2] > 0.0 && h.clockRatio[3] > 0.0))
        return "clockModel 1 reads the four clockRatio* constants, which must be positive";
    if (h.l2StreamModel == 1 && !(h.l2HitBytesPerCycle > 0.0))
        return "l2StreamModel 1 reads l2HitBytesPerCycle, which must be positive";
    if (h.uniformOverlapModel == 1 && !(h.freeRunningOverlap >= 0.0 && h.freeRunningOverlap <= 1.0))
        return "uniformOverlapModel 1 reads freeRunningOverlap, which must lie in [0, 1]";
    if (h.powerModel == 1 && !(h.loadedClockRatio > 0.0 && h.loadedClockRatio <= 1.0))
        return "powerModel 1 reads loadedClockRatio, which must lie in (0, 1]";
    if (h.mallStreamModel == 1) {
        bool rising = h.mallRefillBytesPerSec > 0.0 && h.mallStretchLoad[0] >= 0.0;
        for (int i = 0; i < 4; ++i) rising = rising && h.mallStretchLoad[i + 1] > h.mallStretchLoad[i];
        for (int i = 0; i < 5; ++i) rising = rising && h.mallStretch[i] > 0.0;
        if (!rising)
            return "mallStreamModel 1 reads mallRefillBytesPerSec (positive) and the mallStretchLoad0..4 / "
                   "mallStretch0..4 curve (loads increasing, stretches positive)";
    }
    if (h.hbmWriteModel == 1 && !(h.hbmWriteBytesPerSec > 0.0))
        return "hbmWriteModel 1 reads hbmWriteBytesPerSec, which must be positive";
    if (h.writeOverlapModel == 1 && !(h.hbmWriteModel == 1 && h.l2StreamModel == 1))
        return "writeOverlapModel 1 overlaps hbmWriteModel's writes with l2StreamModel's L2-served loads, and "
               "needs both switched on";
    if (h.fillLatencyModel == 1 && !(h.fillLatencySec > 0.0))
        return "fillLatencyModel 1 reads fillLatencySec, which must be positive";
    if (h.fillShareModel == 1 && !(h.l2HitBytesPerCycle > 0.0))
        return "fillShareModel 1 reads l2HitBytesPerCycle, which must be positive";
    if (h.mallReuseModel == 1 && !(h.mallRefillBytesPerSec > 0.0 && h.mallBytes > 0.0))
        return "mallReuseModel 1 reads mallRefillBytesPerSec and mallBytes, which must be positive";
    if (h.mallWriteModel == 1 && !(h.hbmWriteModel == 1 && h.mallWriteBytesPerSec > 0.0 && h.mallBytes > 0.0))
        return "mallWriteModel 1 refines hbmWriteModel 1 and reads mallWriteBytesPerSec and mallBytes, which must be "
               "positive";
    if (h.pingPongStepModel == 1 &&
        !(h.pingPongModel == 1 && h.pingPongRowStepCycles[0] > 0.0 && h.pingPongRowStepCycles[1] > 0.0))
        return "pingPongStepModel 1 refines pingPongModel 1 and reads pingPongRowStepCycles1 and "
               "pingPongRowStepCycles2, which must be positive";
    if (h.persistentStepModel == 1 && !(h.persistentStepCycles[0] > 0.0 && h.persistentStepCycles[1] > 0.0))
        return "persistentStepModel 1 reads persistentStepCycles1 and persistentStepCycles2, which must be positive";
    if (h.persistentTileModel == 1 && !(h.persistentTileCycles[0] >= 0.0 && h.persistentTileCycles[1] >= 0.0 &&
                                        h.persistentModel == 1 && h.persistentStepModel == 1))
        return "persistentTileModel 1 reads persistentTileCycles1 and persistentTileCycles2 (not negative; cycles "
               "of the persistent skeletons) and needs persistentModel 1 and persistentStepModel 1";
    if (h.launchModel == 1 && !(h.launchOverheadSeconds >= 0.0))
        return "launchModel 1 reads launchOverheadSeconds, which must not be negative";
    if (h.labelModel == 1 && !(h.launchIsolatedSeconds >= 0.0 && h.hbmWriteModel == 1 && h.simdsPerSM > 0))
        return "labelModel 1 reads launchIsolatedSeconds (not negative) and needs hbmWriteModel 1 and per-SIMD "
               "register files (simdsPerSM > 0)";
    if (h.labelModel == 2 && !(h.launchIsolatedSeconds >= 0.0 && h.hbmWriteModel == 1 && h.simdsPerSM > 0 &&
                               h.powerModel == 1 && h.nominalClockHz >= h.clockHz))
        return "labelModel 2 reads launchIsolatedSeconds (not negative) and nominalClockHz (at least clockHz), and "
               "needs hbmWriteModel 1, powerModel 1 and per-SIMD register files (simdsPerSM > 0)";
    return "";
}

}  // namespace

bool HardwareModel::loadFromJson(const std::string& path, HardwareModel& out, std::string& err) {
    std::string text;
    ridgeio::FlatObject kv;
    ridgeio::Status st = ridgeio::readWholeFile(path, text);
    if (st.ok()) st = ridgeio::parseFlatObject(text, path, kv);
    if (!st.ok()) {
        err = st.message();
        return false;
    }
    // "arch": "gfx950" starts from the CDNA4 target description; anything else
    // from the reference's sm_80 defaults. The result is assembled in a local
    // and only copied out once complete, so a failure leaves `out` untouched.
    const auto arch = kv.find("arch");
    HardwareModel h = (arch != kv.end() && arch->second == "gfx950") ? mi355x() : HardwareModel();
    const auto name = kv.find("name");
    h.name = name != kv.end() ? name->second : path;
    if (arch != kv.end()) h.arch = arch->second;
    st = applySchema(kv, schemaFor(h));
    if (!st.ok()) {
        err = path + ": " + st.message();
        return false;
    }
    const std::string bad = inconsistency(h);
    if (!bad.empty()) {
        err = path + ": " + bad;
        return false;
    }
    h.calibrated = true;
    out = h;
    return true;
}

}  // namespace ridge
