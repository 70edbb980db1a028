// ridge/prediction.h -- the cost model's output.
//
// Same labels and fields as the reference (include/ridge/prediction.h:10-49),
// plus the CDNA4 terms (XCD-aware reuse) that explain the new HBM branch.
#pragma once

namespace ridge {

// TENSOR_CORE: the matrix pipe binds; SMEM: operand reads from LDS/shared memory
// serialise with the math; HBM: the memory roofline binds; OCC: too few resident
// waves to hide latency; WAVES: the grid does not fill the machine; ENVELOPE:
// pipeline fill and drain dominate; DOES_NOT_FIT: the tile exceeds a CU/SM.
enum class Bottleneck { TensorCore, Smem, Hbm, Occupancy, Waves, Envelope, DoesNotFit };

const char* toString(Bottleneck b);

struct Prediction {
    double predictedTFLOPS = 0.0;
    Bottleneck bottleneck = Bottleneck::TensorCore;

    double computeTFLOPS = 0.0;        // matrix peak x read, latency, grid and fill/drain factors
    double hbmTFLOPS = 0.0;            // DRAM bandwidth x arithmetic intensity
    double peakTensorTFLOPS = 0.0;     // MFMA issue rate x CUs x clock, nothing subtracted
    double smEfficiency = 0.0;         // share of a K-step the matrix pipe is issuing
    double occFactor = 0.0;            // resident waves over those needed, capped at 1
    double arithmeticIntensity = 0.0;  // FLOP per DRAM byte, after cache reuse
    double baseIntensity = 0.0;        // FLOP per byte of one tile, before reuse
    double l2ReuseFactor = 0.0;        // arithmeticIntensity / baseIntensity

    double waveEfficiency = 0.0;       // busy fraction from grid quantisation
    double totalCtas = 0.0;
    double ctaSlots = 0.0;             // resident workgroups per CU * CUs
    double wavesExact = 0.0;           // totalCtas / ctaSlots

    double envelopeEfficiency = 0.0;   // steady-state fraction of the kernel
    double tPrologueCycles = 0.0;
    double tEpilogueCycles = 0.0;
    double tBodyCycles = 0.0;
    double kSteps = 0.0;

    int numWarps = 0;                  // waves (warps) per workgroup
    int ctasPerSM = 0;                 // resident workgroups per CU (SM)
    double tComputeCycles = 0.0;
    double tSmemCycles = 0.0;
    double tStepCycles = 0.0;          // cycles of one K-step, both phases counted

    // CDNA4 reuse terms (zero in the reference's square-reuse mode).
    double reuseTilesM = 0.0;          // resident row tiles sharing one XCD's L2
    double reuseTilesN = 0.0;          // resident column tiles sharing it
    double compulsoryIntensity = 0.0;  // 2MNK / (A + B + C bytes)

    // Power-limited clock (clockModel 1; 1.0 otherwise).
    double tailClockFactor = 1.0;      // clock of the last wave over the full-chip clock

    // L2 stream (l2StreamModel 1; 0 otherwise).
    double l2HitBytes = 0.0;           // tile-load bytes served by the L2s, not HBM

    // Power-limited clock (powerModel 1; 1.0 otherwise).
    double powerClockFactor = 1.0;     // clock under this row's load over a pure MFMA stream's

    // First-tile latency (fillLatencyModel 1; 0 otherwise).
    double fillRounds = 0.0;           // rounds of workgroups that each wait one first-tile latency
    double refillMissShare = 0.0;      // share of the tile refill that misses the L2 (mallStreamModel 1)
    double mallLoad = 0.0;             // load that stream puts on the MALL path (mallStreamModel 1)
    double mallStretch = 1.0;          // K-step stretch read off the calibrated curve (mallStreamModel 1)

    // What the counters read on one launch from an idle stream (labelModel 1; 0 otherwise).
    double kernelSeconds = 0.0;        // duration of that launch
    double dramReadBytes = 0.0;        // bytes the L2s miss (MALL hits included), A and B
    double dramWriteBytes = 0.0;       // C
    double dramShare = 0.0;            // read bytes at the read rate + C at the write rate, over the duration
    double bodyFactor = 0.0;           // the second K of the body share, as a multiple of K (1/2 or 2)
    double bodyShare = 0.0;            // share of the duration that scales with K, from the two durations
    double cuShare = 0.0;              // CU-time share the grid keeps occupied
    double mfmaShare = 0.0;            // matrix-pipe busy share of the SIMD cycles
    double ldsShare = 0.0;             // LDS busy share of the CU cycles (fragment reads)
    double matrixLoad = 0.0;           // share of the time the matrix pipes are busy (the power term's u)
    double observedClockHz = 0.0;      // the clock the counters count at under that load
};

}  // namespace ridge
