// hardware.cpp -- built-in hardware models and the flat-JSON loader.
// Counterpart of the reference's src/hardware.cpp (a100 :19-34, loader :149-200).

#include "ridge/hardware.h"

#include <cctype>
#include <cstdlib>
#include <fstream>
#include <map>
#include <sstream>

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

// Parser for one flat JSON object of string and number values. The "note" field
// holds prose that can mention key names, so values are read by parsing, never by
// searching for substrings.
class FlatJson {
public:
    explicit FlatJson(const std::string& text) : s_(text) {}

    bool parse(std::map<std::string, std::string>& out, std::string& err) {
        ws();
        if (!eat('{', err)) return false;
        ws();
        if (peek() == '}') return true;
        while (true) {
            ws();
            std::string key, value;
            if (!str(key, err)) return false;
            ws();
            if (!eat(':', err)) return false;
            ws();
            if (peek() == '"') {
                if (!str(value, err)) return false;
            } else if (!bare(value, err)) {
                return false;
            }
            out[key] = value;
            ws();
            if (peek() == ',') {
                ++i_;
                continue;
            }
            if (peek() == '}') return true;
            err = "expected ',' or '}' at offset " + std::to_string(i_);
            return false;
        }
    }

private:
    char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
    void ws() {
        while (i_ < s_.size() && std::isspace((unsigned char)s_[i_])) ++i_;
    }
    bool eat(char c, std::string& err) {
        if (peek() != c) {
            err = std::string("expected '") + c + "' at offset " + std::to_string(i_);
            return false;
        }
        ++i_;
        return true;
    }
    bool str(std::string& out, std::string& err) {
        if (!eat('"', err)) return false;
        out.clear();
        while (i_ < s_.size() && s_[i_] != '"') {
            if (s_[i_] == '\\' && i_ + 1 < s_.size()) ++i_;
            out.push_back(s_[i_++]);
        }
        return eat('"', err);
    }
    bool bare(std::string& out, std::string& err) {
        const size_t b = i_;
        while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && !std::isspace((unsigned char)s_[i_])) ++i_;
        if (i_ == b) {
            err = "empty value at offset " + std::to_string(b);
            return false;
        }
        out = s_.substr(b, i_ - b);
        return true;
    }

    const std::string& s_;
    size_t i_ = 0;
};

bool number(const std::map<std::string, std::string>& kv, const char* key, double& out, std::string& err) {
    auto it = kv.find(key);
    if (it == kv.end()) {
        err = std::string("missing required key \"") + key + "\"";
        return false;
    }
    char* end = nullptr;
    const double v = std::strtod(it->second.c_str(), &end);
    if (end == it->second.c_str() || *end != '\0') {
        err = std::string("key \"") + key + "\" is not a number: " + it->second;
        return false;
    }
    out = v;
    return true;
}

bool integer(const std::map<std::string, std::string>& kv, const char* key, int& out, std::string& err) {
    double d = 0.0;
    if (!number(kv, key, d, err)) return false;
    out = static_cast<int>(d);
    return true;
}

bool optionalInteger(const std::map<std::string, std::string>& kv, const char* key, int& out, std::string& err) {
    if (kv.find(key) == kv.end()) return true;
    return integer(kv, key, out, err);
}

bool optionalNumber(const std::map<std::string, std::string>& kv, const char* key, double& out, std::string& err) {
    if (kv.find(key) == kv.end()) return true;
    return number(kv, key, out, err);
}

}  // namespace

bool HardwareModel::loadFromJson(const std::string& path, HardwareModel& out, std::string& err) {
    std::ifstream in(path);
    if (!in) {
        err = "cannot open " + path;
        return false;
    }
    std::ostringstream ss;
    ss << in.rdbuf();
    const std::string text = ss.str();
    std::map<std::string, std::string> kv;
    FlatJson parser(text);
    if (!parser.parse(kv, err)) {
        err = path + ": " + err;
        return false;
    }

    // Built in a temporary so a failure cannot leave a half-calibrated model.
    auto archIt = kv.find("arch");
    HardwareModel h = (archIt != kv.end() && archIt->second == "gfx950") ? mi355x() : HardwareModel();
    auto name = kv.find("name");
    h.name = name != kv.end() ? name->second : path;

    if (!integer(kv, "numSMs", h.numSMs, err) || !number(kv, "clockHz", h.clockHz, err) ||
        !number(kv, "mmaCyclesPerInst", h.mmaCyclesPerInst, err) ||
        !number(kv, "smemBytesPerCycle", h.smemBytesPerCycle, err) ||
        !number(kv, "hbmBytesPerSec", h.hbmBytesPerSec, err) || !integer(kv, "regsPerSM", h.regsPerSM, err) ||
        !integer(kv, "smemBytesPerSM", h.smemBytesPerSM, err) ||
        !integer(kv, "maxWarpsPerSM", h.maxWarpsPerSM, err) ||
        !integer(kv, "maxCtasPerSM", h.maxCtasPerSM, err) ||
        !number(kv, "warpsNeededToHide", h.warpsNeededToHide, err) ||
        !optionalInteger(kv, "waveSize", h.waveSize, err) || !optionalInteger(kv, "mmaM", h.mmaM, err) ||
        !optionalInteger(kv, "mmaN", h.mmaN, err) || !optionalInteger(kv, "mmaK", h.mmaK, err) ||
        !optionalInteger(kv, "simdsPerSM", h.simdsPerSM, err) ||
        !optionalInteger(kv, "regsPerSimdLane", h.regsPerSimdLane, err) ||
        !optionalInteger(kv, "regGranule", h.regGranule, err) ||
        !optionalInteger(kv, "numXcds", h.numXcds, err) || !optionalInteger(kv, "cBytes", h.cBytes, err) ||
        !optionalInteger(kv, "l2ReuseModel", h.l2ReuseModel, err) ||
        !optionalInteger(kv, "prologueModel", h.prologueModel, err) ||
        !optionalInteger(kv, "pingPongModel", h.pingPongModel, err) ||
        !optionalInteger(kv, "persistentModel", h.persistentModel, err) ||
        !optionalInteger(kv, "ldsReadModel", h.ldsReadModel, err) ||
        !optionalNumber(kv, "ldsAReadBytesPerCycle", h.ldsAReadBytesPerCycle, err) ||
        !optionalNumber(kv, "ldsBTrReadBytesPerCycle", h.ldsBTrReadBytesPerCycle, err) ||
        !optionalInteger(kv, "clockModel", h.clockModel, err) ||
        !optionalNumber(kv, "clockRatioHalfCus", h.clockRatio[0], err) ||
        !optionalNumber(kv, "clockRatioQuarterCus", h.clockRatio[1], err) ||
        !optionalNumber(kv, "clockRatioEighthCus", h.clockRatio[2], err) ||
        !optionalNumber(kv, "clockRatioSixteenthCus", h.clockRatio[3], err) ||
        !optionalInteger(kv, "l2StreamModel", h.l2StreamModel, err) ||
        !optionalNumber(kv, "l2HitBytesPerCycle", h.l2HitBytesPerCycle, err) ||
        !optionalInteger(kv, "uniformOverlapModel", h.uniformOverlapModel, err) ||
        !optionalNumber(kv, "freeRunningOverlap", h.freeRunningOverlap, err) ||
        !optionalInteger(kv, "powerModel", h.powerModel, err) ||
        !optionalNumber(kv, "loadedClockRatio", h.loadedClockRatio, err) ||
        !optionalNumber(kv, "warpsNeededToHideIlp8", h.warpsNeededToHideIlp8, err)) {
        err = path + ": " + err;
        return false;
    }
    if (archIt != kv.end()) h.arch = archIt->second;

    // Zeros would divide by zero or silently zero a ceiling (reference :190-195).
    if (h.numSMs <= 0 || h.clockHz <= 0.0 || h.mmaCyclesPerInst <= 0.0 || h.smemBytesPerCycle <= 0.0 ||
        h.hbmBytesPerSec <= 0.0 || h.warpsNeededToHide <= 0.0) {
        err = path + ": a required constant is zero or negative";
        return false;
    }
    if (h.waveSize <= 0 || h.mmaM <= 0 || h.mmaN <= 0 || h.mmaK <= 0 || h.regGranule <= 0 || h.numXcds <= 0 ||
        h.cBytes <= 0 || h.simdsPerSM < 0 || (h.simdsPerSM > 0 && h.regsPerSimdLane <= 0)) {
        err = path + ": a target-description key is out of range";
        return false;
    }
    if (h.ldsReadModel == 1 && (h.ldsAReadBytesPerCycle <= 0.0 || h.ldsBTrReadBytesPerCycle <= 0.0)) {
        err = path + ": ldsReadModel 1 needs positive ldsAReadBytesPerCycle and ldsBTrReadBytesPerCycle";
        return false;
    }
    if (h.clockModel == 1 &&
        (h.clockRatio[0] <= 0.0 || h.clockRatio[1] <= 0.0 || h.clockRatio[2] <= 0.0 || h.clockRatio[3] <= 0.0)) {
        err = path + ": clockModel 1 needs the four positive clockRatio* keys";
        return false;
    }
    if (h.l2StreamModel == 1 && h.l2HitBytesPerCycle <= 0.0) {
        err = path + ": l2StreamModel 1 needs a positive l2HitBytesPerCycle";
        return false;
    }
    if (h.uniformOverlapModel == 1 && (h.freeRunningOverlap < 0.0 || h.freeRunningOverlap > 1.0)) {
        err = path + ": uniformOverlapModel 1 needs freeRunningOverlap in [0, 1]";
        return false;
    }
    if (h.powerModel == 1 && (h.loadedClockRatio <= 0.0 || h.loadedClockRatio > 1.0)) {
        err = path + ": powerModel 1 needs loadedClockRatio in (0, 1]";
        return false;
    }
    h.calibrated = true;
    out = h;
    return true;
}

}  // namespace ridge
