// ridge/hardware.h -- per-GPU constants of the cost model.
//
// The ten required keys and their meaning follow the reference's HardwareModel
// (include/ridge/hardware.h:9-54): constants marked [CAL] come from the
// calibration microbenchmarks, the rest from the datasheet. "SM" fields mean a
// compute unit (CU) on CDNA, "warp" fields a 64-lane wavefront.
//
// The target-description fields below the required keys capture every place the
// reference hard-codes an sm_80 assumption. Their defaults ARE those assumptions,
// so a model built from a reference JSON (or a100()) predicts exactly what the
// reference predicts; mi355x() and a calibrated gfx950 JSON switch them to CDNA4.
#pragma once
#include <string>

namespace ridge {

struct HardwareModel {
    std::string name;
    int numSMs = 0;                  // SMs (sm_80) or CUs (CDNA)
    double clockHz = 0.0;

    double mmaCyclesPerInst = 0.0;   // [CAL] SM/CU-level cycles per matrix instruction
    double smemBytesPerCycle = 0.0;  // [CAL] operand-read bytes per cycle per SM/CU
    double hbmBytesPerSec = 0.0;     // [CAL] sustained DRAM read bandwidth, whole GPU

    int regsPerSM = 0;               // 32-bit registers per SM; lane-registers per CU on CDNA
    int smemBytesPerSM = 0;          // shared memory / LDS per SM/CU
    int maxWarpsPerSM = 0;           // resident warps / wavefronts per SM/CU
    int maxCtasPerSM = 0;            // resident workgroups per SM/CU

    double warpsNeededToHide = 0.0;  // [CAL] resident warps/waves that hide latency
    double warpsNeededToHideIlp8 = 0.0;  // [CAL] the same with 8 independent chains per
                                         // wave; 0 = not measured (reference: unused)

    bool calibrated = false;         // every [CAL] constant came from a measurement

    // ---- target description (defaults = the reference's sm_80 assumptions) ----
    std::string arch = "sm_80";
    int waveSize = 32;               // threads per warp / lanes per wavefront
    int mmaM = 16, mmaN = 8, mmaK = 16;  // matrix instruction shape (FP16)
    int simdsPerSM = 0;              // 0: pooled register file (sm_80 accounting);
                                     // >0: per-SIMD files, waves spread over SIMDs
    int regsPerSimdLane = 0;         // VGPR+AGPR budget per lane per SIMD (512 on CDNA3/4)
    int regGranule = 1;              // per-lane register allocation granule (8 on gfx950)
    int numXcds = 1;                 // separate L2 domains (8 XCDs on MI355X)
    int cBytes = 4;                  // bytes per output element drained by the epilogue
    int l2ReuseModel = 0;            // 0: sqrt(ctaSlots) square reuse (reference)
                                     // 1: per-XCD resident block, bounded by the grid
                                     // 2: the kernels' exact launch order (XCD remap of
                                     //    the GroupM order): distinct panels per XCD
    int prologueModel = 0;           // 0: the prologue always fills stages-1 tiles (reference)
                                     // 1: only the K tiles that exist, min(stages-1, K/BK)
    int pingPongModel = 0;           // 0: operand reads in series with the MFMAs (reference)
                                     // 1: a workgroup of 2 waves per SIMD with >= 3 stages runs
                                     //    the ping-pong schedule: reads overlap the MFMAs
    int persistentModel = 0;         // 0: every row is a one-tile-per-workgroup kernel (reference)
                                     // 1: schedule-2 rows are persistent: two loader waves and
                                     //    the epilogue staging join the workgroup, which walks
                                     //    ceil(tiles / slots) tiles and pays one fill and one
                                     //    drain for all of them
    int ldsReadModel = 0;            // 0: one blended operand-read rate, smemBytesPerCycle (reference)
                                     // 1: A fragments at ldsAReadBytesPerCycle (ds_read_b128),
                                     //    B fragments at ldsBTrReadBytesPerCycle (transposing reads)
    double ldsAReadBytesPerCycle = 0.0;    // [CAL] per CU, read by ldsReadModel 1
    double ldsBTrReadBytesPerCycle = 0.0;  // [CAL] per CU, read by ldsReadModel 1
    int clockModel = 0;              // 0: every wave of workgroups runs at clockHz (reference)
                                     // 1: the chip is power-limited: a last wave that leaves CUs
                                     //    idle runs at clockHz x clockRatio for its busy share
    double clockRatio[4] = {0.0, 0.0, 0.0, 0.0};  // [CAL] loaded clock with 1/2, 1/4, 1/8, 1/16 of the
                                                  // CUs busy, over the clock with all of them busy
    int l2StreamModel = 0;           // 0: the HBM roofline alone bounds the memory side (reference)
                                     // 1: tile loads that the L2s serve (every workgroup re-reading
                                     //    a shared panel) take their own time at
                                     //    l2HitBytesPerCycle x clockHz, in series with the HBM stream
    double l2HitBytesPerCycle = 0.0; // [CAL] whole GPU, per shader cycle, reads served by the XCDs' L2s
    int uniformOverlapModel = 0;     // 0: a uniform-schedule K-step is reads + MFMAs (reference)
                                     // 1: a workgroup of two waves per SIMD hides freeRunningOverlap
                                     //    of the shorter phase under the longer
    double freeRunningOverlap = 0.0; // [CAL] measured by cal-smem-bw's skeleton without barriers
    int powerModel = 0;              // 0: the loaded clock of a pure MFMA stream, clockHz (reference)
                                     // 1: a row that keeps the matrix pipes busy a share u of the
                                     //    time runs at clockHz x (1 - (1 - loadedClockRatio) u)
    double loadedClockRatio = 0.0;   // [CAL] clock of the ping-pong skeleton with the GEMM's reads
                                     // and refill over that of its MFMAs alone (cal-smem-bw)
    int hbmWriteModel = 0;           // 0: every DRAM byte, C included, moves at hbmBytesPerSec (reference)
                                     // 1: C's bytes are written at hbmWriteBytesPerSec and A and B's
                                     //    read at hbmBytesPerSec; the bus carries one direction at a
                                     //    time, so the two times add (the epilogue drains at the
                                     //    write rate too)
    double hbmWriteBytesPerSec = 0.0;  // [CAL] streaming 16-byte stores, whole GPU (cal-hbm-bw)
    int writeOverlapModel = 0;       // 0: DRAM reads, DRAM writes and (l2StreamModel 1) L2-served
                                     //    loads take the sum of their times
                                     // 1: two resources, each used in series: the DRAM bus (reads,
                                     //    then writes) and the CUs' load path (DRAM-served loads, then
                                     //    L2-served ones); the writes and the L2-served loads overlap,
                                     //    so the time is reads + max(writes, L2-served loads)
    int fillLatencyModel = 0;        // 0: fill costs only its bytes at the DRAM rate (reference)
                                     // 1: each round of one-tile-per-workgroup workgroups (one
                                     //    round in all for a persistent grid) also waits
                                     //    fillLatencySec before its first matrix instruction
    double fillLatencySec = 0.0;     // [CAL] a full grid's first-tile load latency (cal-hbm-bw)
    int mallStreamModel = 0;         // 0: every panel reload is an L2 hit (reference)
                                     // 1: the first load of a panel on each XCD (the kernels' launch
                                     //    order) crosses to the MALL; the K-step stretches with the
                                     //    load that stream puts on the MALL path, read off the
                                     //    skeleton's calibrated curve
    double mallRefillBytesPerSec = 0.0;  // [CAL] rate of the L2-missing refill path (cal-smem-bw)
    double mallStretchLoad[5] = {0.0, 0.0, 0.0, 0.0, 0.0};  // [CAL] path load at miss share 0..1
    double mallStretch[5] = {0.0, 0.0, 0.0, 0.0, 0.0};      // [CAL] the skeleton K-step's stretch there
    int persistentStepModel = 0;     // 0: a persistent row's K-step is the uniform schedule's (reference:
                                     //    no persistent rows)
                                     // 1: its K-step is (reads + MFMAs) scaled by what the persistent
                                     //    skeleton measures for the same class of row: the measured
                                     //    cycles per K tile over the model's reads + MFMAs for the
                                     //    skeleton's row (128x128x64 w64x64 s4 with one compute wave
                                     //    per SIMD, 256x128x32 w64x64 s6 with two)
    double persistentStepCycles[2] = {0.0, 0.0};  // [CAL] cycles per K tile of those two skeletons
    int persistentTileModel = 0;     // 0: a persistent walk's tiles pay no cost between them (each tile's
                                     //    stores drain under the next body)
                                     // 1: every tile a persistent workgroup walks adds, to its body, the
                                     //    epilogue its compute waves run before the next tile (staging
                                     //    through LDS, issuing the stores): the cycles the persistent
                                     //    skeleton of the row's class measures per output tile.
                                     //    The calibration writes the cycles but leaves the term off:
                                     //    with them it predicts worse on the measured sweeps
    double persistentTileCycles[2] = {0.0, 0.0};  // [CAL] those cycles, one and two compute waves per SIMD
    int mallReuseModel = 0;         // 0: every A/B byte an XCD's L2 misses is read from HBM (reference:
                                     //    one cache level)
                                     // 1: when A and B fit in the MALL (mallBytes), HBM supplies each
                                     //    once and the L2s' further misses (other XCDs re-fetching the
                                     //    same panels) are MALL hits at mallRefillBytesPerSec, in series
    double mallBytes = 0.0;          // capacity of the memory-side cache in front of HBM (datasheet)
    int mallWriteModel = 0;          // 0: C drains at hbmWriteBytesPerSec, shared by every CU
                                     //    (hbmWriteModel 1)
                                     // 1: the last drain's cached stores of C (every schedule but the
                                     //    persistent one, whose stores are non-temporal) go to the MALL
                                     //    when A, B and C together fit in it (mallBytes), at
                                     //    mallWriteBytesPerSec, shared by the CUs that hold a
                                     //    workgroup, not by all; a drain to HBM and the DRAM-side write
                                     //    time are unchanged
    double mallWriteBytesPerSec = 0.0;  // [CAL] 16-byte cached stores into a MALL-resident buffer (cal-hbm-bw)
    int pingPongStepModel = 0;       // 0: a ping-pong row's K-step is max(MFMAs, operand reads)
                                     //    (pingPongModel 1)
                                     // 1: that max scaled by what the ping-pong row skeleton of the
                                     //    same class measures: its cycles per K tile over the model's
                                     //    max for the skeleton's own row (256x256x32 w128x64 s3 for
                                     //    BK = 32, 256x128x64 w64x64 s3 for BK = 64 and above)
    double pingPongRowStepCycles[2] = {0.0, 0.0};  // [CAL] cycles per K tile of those two skeletons
    int fillShareModel = 0;          // 0: every workgroup fetches its first tiles from HBM (reference)
                                     // 1: the resident workgroups' first tiles come from HBM once per
                                     //    distinct panel an XCD holds (the kernels' launch order) and
                                     //    from the L2s for the rest, at l2HitBytesPerCycle
    int launchModel = 0;             // 0: a launch costs its work alone (reference)
                                     // 1: a kernel boundary adds launchOverheadSeconds to each launch of a
                                     //    back-to-back sequence (the measurement protocol of the sweeps)
    double launchOverheadSeconds = 0.0;  // [CAL] per launch on top of its work, back to back (cal-latency)
    double launchIsolatedSeconds = 0.0;  // [CAL] the same for one launch from an idle stream (cal-latency)
    double nominalClockHz = 0.0;     // engine clock ceiling (cal-mma reports the device's), read by labelModel 1
    int labelModel = 0;              // 0: the label names the derating furthest from 1 (reference :129-143)
                                     // 1: the label is the counter decision table applied to the model's
                                     //    own prediction of what the counters read on one launch from an
                                     //    idle stream: DRAM share, body share from a second K, CU share,
                                     //    LDS and MFMA busy shares (Prediction's observable fields)
                                     // 2: the same, the busy shares counted at the physical clock: from
                                     //    nominalClockHz (matrix pipes idle) to clockHz x loadedClockRatio
                                     //    (always busy), linear in the row's matrix load

    // Datasheet placeholders of the reference (hardware.cpp:19-34).
    static HardwareModel a100();

    // MI355X (gfx950) datasheet placeholders; calibration replaces the [CAL] ones.
    static HardwareModel mi355x();

    // All-or-nothing load of a flat JSON written by the calibration driver (or the
    // reference's data/hardware/*.json). The ten required keys must be present and
    // the [CAL] ones positive; "arch": "gfx950" selects the CDNA4 target
    // description, and any target-description key present overrides it. On
    // failure returns false, leaves `out` untouched and sets `err`
    // (reference hardware.h:38-48).
    static bool loadFromJson(const std::string& path, HardwareModel& out, std::string& err);
};

}  // namespace ridge
