/*
 * ridge_model.h -- C ABI of the closed-form GEMM cost model (libridge_model.so).
 *
 * Replaces, for callers that cannot link C++, the reference's model interface:
 *   ridge::predict(const GemmConfig&, const HardwareModel&) -> Prediction
 *       -- include/ridge/model.h:10, src/model.cpp:22-146
 *   HardwareModel::a100() / loadFromJson(path, out, err)
 *       -- include/ridge/hardware.h:36-48, src/hardware.cpp:19-34,149-200
 *   toString(Bottleneck) -- src/model.cpp:9-20
 * The C++ API itself is in include/ridge/ and the process-level contract is the
 * ridge-predict CLI (tools/ridge-predict.cpp:26-94 of the reference).
 */
#ifndef RIDGE_MODEL_H
#define RIDGE_MODEL_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ridge_model_config {
    long long M, N, K;
    int BM, BN, BK;
    int warpM, warpN;       /* wavefront (warp) tile */
    int mmaM, mmaN, mmaK;   /* 0 = the hardware model's instruction shape */
    int stages;
    int regsPerThread;      /* 0 = unknown */
    int groupM;             /* launch-order group size along M (read by l2ReuseModel 2 only) */
    int schedule;           /* -1: from the tile, 0 uniform, 1 ping-pong, 2 persistent
                               (2 is read by persistentModel 1 only) */
} ridge_model_config_t;

typedef struct ridge_model_prediction {
    double predictedTFLOPS;
    int bottleneck;         /* 0 TENSOR_CORE, 1 SMEM, 2 HBM, 3 OCC, 4 WAVES, 5 ENVELOPE, 6 DOES_NOT_FIT */
    double computeTFLOPS, hbmTFLOPS, peakTensorTFLOPS;
    double smEfficiency, occFactor, arithmeticIntensity, baseIntensity, l2ReuseFactor;
    double waveEfficiency, totalCtas, ctaSlots, wavesExact;
    double envelopeEfficiency, tPrologueCycles, tEpilogueCycles, tBodyCycles, kSteps;
    int numWarps, ctasPerSM;
    double tComputeCycles, tSmemCycles, tStepCycles;
    double reuseTilesM, reuseTilesN, compulsoryIntensity;
    double tailClockFactor;  /* clock of the last wave over the full-chip clock (clockModel 1) */
    double l2HitBytes;       /* tile-load bytes served by the L2s (l2StreamModel 1) */
    double powerClockFactor; /* clock under this row's load over a pure MFMA stream's (powerModel 1) */
    double fillRounds;       /* rounds that each wait one first-tile latency (fillLatencyModel 1) */
    double refillMissShare;  /* share of the tile refill that misses the L2 (mallStreamModel 1) */
    double mallLoad;         /* load that stream puts on the MALL path (mallStreamModel 1) */
    double mallStretch;      /* K-step stretch from the calibrated curve (mallStreamModel 1) */
    /* What the counters read on one launch from an idle stream (labelModel 1; 0 otherwise). */
    double kernelSeconds, dramReadBytes, dramWriteBytes, dramShare, bodyFactor, bodyShare, cuShare, mfmaShare,
        ldsShare, matrixLoad, observedClockHz;
} ridge_model_prediction_t;

/* Default config (the reference's GemmConfig defaults, config.h:18-39). */
void ridge_model_default_config(ridge_model_config_t* cfg);

/* Hardware model from "a100", "mi355x" or a JSON path. Returns an opaque handle,
 * or NULL with a message in err (all-or-nothing, like loadFromJson). */
void* ridge_model_hw_load(const char* spec, char* err, size_t errcap);
void ridge_model_hw_free(void* hw);
/* 1 when every [CAL] constant came from a calibration file. */
int ridge_model_hw_calibrated(const void* hw);
const char* ridge_model_hw_name(const void* hw);

/* Runs the model. Returns 0, or 1 on a null argument. */
int ridge_model_predict(const void* hw, const ridge_model_config_t* cfg, ridge_model_prediction_t* out);

/* Label string of a bottleneck code ("TENSOR_CORE", ..., "DOES_NOT_FIT"). */
const char* ridge_model_bottleneck_name(int code);

/* sizeof the two structs as this library was built, so a binding that declares
 * them itself (ctypes, cgo, JNA) can refuse a layout that disagrees. No
 * counterpart in the reference (its callers compile against its headers). */
size_t ridge_model_config_size(void);
size_t ridge_model_prediction_size(void);

#ifdef __cplusplus
}
#endif

#endif /* RIDGE_MODEL_H */
