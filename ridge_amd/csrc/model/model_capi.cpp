// model_capi.cpp -- C ABI over the C++ cost model (include/ridge_model.h).

#include "ridge_model.h"

#include "ridge/hardware.h"
#include "ridge/model.h"

#include <cstring>
#include <string>

using namespace ridge;

namespace {

void copyErr(char* err, size_t cap, const std::string& msg) {
    if (err == nullptr || cap == 0) return;
    const size_t n = msg.size() < cap - 1 ? msg.size() : cap - 1;
    std::memcpy(err, msg.data(), n);
    err[n] = '\0';
}

GemmConfig toCpp(const ridge_model_config_t& c) {
    GemmConfig g;
    g.M = c.M;
    g.N = c.N;
    g.K = c.K;
    g.BM = c.BM;
    g.BN = c.BN;
    g.BK = c.BK;
    g.warpM = c.warpM;
    g.warpN = c.warpN;
    g.mmaM = c.mmaM;
    g.mmaN = c.mmaN;
    g.mmaK = c.mmaK;
    g.stages = c.stages;
    g.regsPerThread = c.regsPerThread;
    g.groupM = c.groupM;
    g.schedule = c.schedule;
    return g;
}

}  // namespace

extern "C" {

void ridge_model_default_config(ridge_model_config_t* cfg) {
    if (cfg == nullptr) return;
    const GemmConfig g;
    cfg->M = g.M;
    cfg->N = g.N;
    cfg->K = g.K;
    cfg->BM = g.BM;
    cfg->BN = g.BN;
    cfg->BK = g.BK;
    cfg->warpM = g.warpM;
    cfg->warpN = g.warpN;
    cfg->mmaM = g.mmaM;
    cfg->mmaN = g.mmaN;
    cfg->mmaK = g.mmaK;
    cfg->stages = g.stages;
    cfg->regsPerThread = g.regsPerThread;
    cfg->groupM = g.groupM;
    cfg->schedule = g.schedule;
}

void* ridge_model_hw_load(const char* spec, char* err, size_t errcap) {
    if (spec == nullptr) {
        copyErr(err, errcap, "null hardware spec");
        return nullptr;
    }
    const std::string s(spec);
    HardwareModel* hw = new HardwareModel();
    if (s == "a100") {
        *hw = HardwareModel::a100();
    } else if (s == "mi355x") {
        *hw = HardwareModel::mi355x();
    } else {
        std::string e;
        if (!HardwareModel::loadFromJson(s, *hw, e)) {
            copyErr(err, errcap, e);
            delete hw;
            return nullptr;
        }
    }
    return hw;
}

void ridge_model_hw_free(void* hw) { delete static_cast<HardwareModel*>(hw); }

int ridge_model_hw_calibrated(const void* hw) {
    return hw != nullptr && static_cast<const HardwareModel*>(hw)->calibrated ? 1 : 0;
}

const char* ridge_model_hw_name(const void* hw) {
    return hw != nullptr ? static_cast<const HardwareModel*>(hw)->name.c_str() : "";
}

int ridge_model_predict(const void* hwp, const ridge_model_config_t* cfg, ridge_model_prediction_t* out) {
    if (hwp == nullptr || cfg == nullptr || out == nullptr) return 1;
    const Prediction p = predict(toCpp(*cfg), *static_cast<const HardwareModel*>(hwp));
    std::memset(out, 0, sizeof(*out));
    out->predictedTFLOPS = p.predictedTFLOPS;
    out->bottleneck = int(p.bottleneck);
    out->computeTFLOPS = p.computeTFLOPS;
    out->hbmTFLOPS = p.hbmTFLOPS;
    out->peakTensorTFLOPS = p.peakTensorTFLOPS;
    out->smEfficiency = p.smEfficiency;
    out->occFactor = p.occFactor;
    out->arithmeticIntensity = p.arithmeticIntensity;
    out->baseIntensity = p.baseIntensity;
    out->l2ReuseFactor = p.l2ReuseFactor;
    out->waveEfficiency = p.waveEfficiency;
    out->totalCtas = p.totalCtas;
    out->ctaSlots = p.ctaSlots;
    out->wavesExact = p.wavesExact;
    out->envelopeEfficiency = p.envelopeEfficiency;
    out->tPrologueCycles = p.tPrologueCycles;
    out->tEpilogueCycles = p.tEpilogueCycles;
    out->tBodyCycles = p.tBodyCycles;
    out->kSteps = p.kSteps;
    out->numWarps = p.numWarps;
    out->ctasPerSM = p.ctasPerSM;
    out->tComputeCycles = p.tComputeCycles;
    out->tSmemCycles = p.tSmemCycles;
    out->tStepCycles = p.tStepCycles;
    out->reuseTilesM = p.reuseTilesM;
    out->reuseTilesN = p.reuseTilesN;
    out->compulsoryIntensity = p.compulsoryIntensity;
    out->tailClockFactor = p.tailClockFactor;
    out->l2HitBytes = p.l2HitBytes;
    out->powerClockFactor = p.powerClockFactor;
    out->fillRounds = p.fillRounds;
    out->refillMissShare = p.refillMissShare;
    out->mallLoad = p.mallLoad;
    out->mallStretch = p.mallStretch;
    out->kernelSeconds = p.kernelSeconds;
    out->dramReadBytes = p.dramReadBytes;
    out->dramWriteBytes = p.dramWriteBytes;
    out->dramShare = p.dramShare;
    out->bodyFactor = p.bodyFactor;
    out->bodyShare = p.bodyShare;
    out->cuShare = p.cuShare;
    out->mfmaShare = p.mfmaShare;
    out->ldsShare = p.ldsShare;
    out->matrixLoad = p.matrixLoad;
    out->observedClockHz = p.observedClockHz;
    return 0;
}

size_t ridge_model_config_size(void) { return sizeof(ridge_model_config_t); }

size_t ridge_model_prediction_size(void) { return sizeof(ridge_model_prediction_t); }

const char* ridge_model_bottleneck_name(int code) {
    if (code < 0 || code > int(Bottleneck::DoesNotFit)) return "UNKNOWN";
    return toString(static_cast<Bottleneck>(code));
}

}  // extern "C"
