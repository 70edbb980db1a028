// model.cpp -- the closed-form GEMM cost model.
//
// Counterpart of the reference's src/model.cpp:22-146 and src/mma.cpp:5-12. The
// structure of the reference model is kept term for term (per-step compute and
// operand-read time in series, occupancy, wave quantisation, fill/drain
// envelope, HBM roofline, worst-factor label), and every sm_80 assumption it
// hard-codes is read from the hardware model instead:
//
//   threads per workgroup = waves * hw.waveSize             (reference :31, *32)
//   matrix instruction    = hw.mmaM x mmaN x mmaK           (reference mma.cpp:9)
//   register occupancy    = per-SIMD files when hw.simdsPerSM > 0: a workgroup's
//                           waves spread over the SIMDs, each lane holds its
//                           VGPR+AGPR count rounded to hw.regGranule
//   epilogue drain        = BM * BN * hw.cBytes              (reference :99, * 4)
//   L2 reuse              = hw.l2ReuseModel 1: the workgroups resident on one
//                           XCD form a compact block of output tiles, bounded by
//                           the grid, and fetch their A and B panels once into
//                           that XCD's L2; capped by the compulsory intensity of
//                           the whole problem                 (reference :116-123)
//                         = hw.l2ReuseModel 2: the same from the kernels' exact
//                           launch order (XCD remap of the GroupM order), so
//                           groupM changes the prediction
//   K-step time           = hw.pingPongModel 1: max(compute, operand reads) for a
//                           workgroup of two waves per SIMD with >= 3 stages (the
//                           ping-pong schedule), their sum otherwise (reference :47)
//   prologue              = hw.prologueModel 1: min(stages-1, K/BK) tiles, the
//                           tiles the kernel actually issues     (reference :91-98)
//   latency hiding        = hw.warpsNeededToHideIlp8 when a wave carries >= 8
//                           independent accumulator chains      (reference :72-74)
//   operand reads         = hw.ldsReadModel 1: A fragments (ds_read_b128) and B
//                           fragments (transposing ds_read_b64_tr_b16) each at its
//                           calibrated rate, not one blended rate (reference :45)
//   last-wave clock       = hw.clockModel 1: a last wave that leaves CUs idle runs
//                           at the calibrated power-limited clock for its busy
//                           share of CUs (reference: one clock for every wave)
//   uniform overlap       = hw.uniformOverlapModel 1: an 8-wave uniform workgroup
//                           (two waves per SIMD) hides the measured share of the
//                           shorter phase under the longer (reference: in series)
//   power-limited clock   = hw.powerModel 1: the clock falls with the share of
//                           time the matrix pipes are busy, to loadedClockRatio
//                           when they always are (reference: one clock)
//   MALL stream           = hw.mallStreamModel 1: the K-step stretches with the
//                           load the launch order's L2-missing refill puts on
//                           the MALL path, as a calibrated skeleton's does
//                           (reference: the L2 serves every panel)
//   first-tile latency    = hw.fillLatencyModel 1: each round of workgroups waits
//                           one measured DRAM latency for its first tile
//                           (reference: the fill costs only bandwidth)
//   L2 stream             = hw.l2StreamModel 1: tile loads the L2s serve take
//                           their own time, in series with the HBM stream
//                           (reference: the HBM roofline alone)
//   write stream          = hw.hbmWriteModel 1: C is written at the calibrated
//                           streaming-write rate, A and B read at the read rate,
//                           and the two times add (reference: one DRAM rate)
//   MALL reuse            = hw.mallReuseModel 1: when A and B fit in the MALL,
//                           HBM supplies them once and the per-XCD re-fetches
//                           are MALL hits at the calibrated refill rate
//                           (reference: every L2 miss goes to DRAM)
//   shared fill           = hw.fillShareModel 1: the resident tiles' first K
//                           tiles cross from HBM once per distinct panel of an
//                           XCD (the launch order) and come from the L2s for
//                           the rest (reference: every workgroup from HBM)
//   persistent K-step     = hw.persistentStepModel 1: a persistent row's reads +
//                           MFMAs scaled by the measured/modelled ratio of the
//                           persistent skeleton of its class (one or two compute
//                           waves per SIMD) (reference: no persistent rows)
//   write overlap         = hw.writeOverlapModel 1: C's writes to DRAM overlap
//                           the tile loads the L2s serve; the DRAM reads come
//                           before both (reference: one DRAM stream)
//   ping-pong K-step      = hw.pingPongStepModel 1: a ping-pong row's max(compute,
//                           operand reads) scaled by the measured/modelled ratio
//                           of the ping-pong row skeleton of its class (BK 32 or
//                           64) (reference: no ping-pong schedule)
//   MALL drain            = hw.mallWriteModel 1: the last drain of cached C
//                           stores goes to the MALL when A, B and C fit it, at
//                           the MALL's write rate shared by the CUs holding a
//                           workgroup (reference: the DRAM rate over all SMs)
//   persistent tiles      = hw.persistentTileModel 1: every tile a persistent
//                           workgroup walks adds the epilogue its compute waves
//                           run before the next one, as the same skeleton with
//                           the kernel's epilogue measures it per output tile
//   persistent rows       = hw.persistentModel 1 and cfg.schedule 2: two loader
//                           waves and the epilogue staging join the workgroup,
//                           which walks ceil(tiles / slots) tiles and pays one
//                           fill and one drain for all of them (reference: one
//                           tile per workgroup, :91-99)
//
//   kernel boundary       = hw.launchModel 1: each launch of a back-to-back
//                           sequence pays launchOverheadSeconds on top of its
//                           work (reference: launches cost their work alone)
//   label                 = hw.labelModel 1: the model predicts what the
//                           counters read on one launch from an idle stream
//                           (DRAM share, body share from a second K, CU share,
//                           MFMA and LDS busy shares) and labels that prediction
//                           with the counters' decision table (reference: the
//                           derating furthest from 1, :129-143); labelModel 2
//                           counts the busy shares at the physical clock of the
//                           row's matrix load instead of the loaded clock
//
// With the defaults (a100() or a reference JSON) every term reduces to the
// reference's expression in the same double-precision operation order, so the
// A100 predictions match the reference bit for bit; integer divisions are kept
// where the reference has them.

#include "ridge/mma.h"
#include "ridge/model.h"

#include <algorithm>
#include <cmath>
#include <vector>

namespace ridge {

const char* toString(Bottleneck b) {
    switch (b) {
        case Bottleneck::TensorCore: return "TENSOR_CORE";
        case Bottleneck::Smem: return "SMEM";
        case Bottleneck::Hbm: return "HBM";
        case Bottleneck::Occupancy: return "OCC";
        case Bottleneck::Waves: return "WAVES";
        case Bottleneck::Envelope: return "ENVELOPE";
        case Bottleneck::DoesNotFit: return "DOES_NOT_FIT";
    }
    return "UNKNOWN";
}

MmaShape mmaShapeFor(DType dtype) {
    switch (dtype) {
        case DType::FP16: return MmaShape{16, 8, 16, 2LL * 16 * 8 * 16};
    }
    return MmaShape{16, 8, 16, 2LL * 16 * 8 * 16};
}

MmaShape mmaShapeFor(DType dtype, const HardwareModel& hw) {
    (void)dtype;  // FP16 is the only dtype
    return MmaShape{hw.mmaM, hw.mmaN, hw.mmaK, 2LL * hw.mmaM * hw.mmaN * hw.mmaK};
}

namespace {

// Loader wavefronts of a persistent workgroup (the kernels' PersistentTraits).
constexpr int kPersistentLoaderWaves = 2;

// The counters' decision table (the rocprofv3 label check, registration 3),
// first match wins; labelModel 1 applies it to the model's own prediction of
// those counters.
constexpr double kDramShareMin = 0.70;       // DRAM share >= 0.70                      -> HBM
constexpr double kCuShareMin = 0.55;         // CU share < 0.55                         -> WAVES
constexpr double kBodyShareMin = 0.60;       // body share < 0.60                       -> ENVELOPE
constexpr double kLdsOverMfmaMin = 0.70;     // LDS share >= 0.70 x MFMA share          -> SMEM
constexpr double kMfmaOverBodyMin = 0.60;    // MFMA share / min(1, body share) >= 0.60 -> TENSOR_CORE
                                             // otherwise                               -> OCC

// LDS of a persistent workgroup's epilogue staging: each compute wave stages
// the largest number of 16-row tile-rows that divides its tile-rows and fits
// beside the ring (the kernels' PersistentTraits::epiTiles).
double persistentStagingBytes(const GemmConfig& cfg, const HardwareModel& hw, int computeWaves, double ringBytes,
                              int db) {
    const int tileRows = cfg.warpM / cfg.mmaM;
    int p = tileRows;
    auto bytes = [&](int q) { return double(computeWaves) * cfg.mmaM * q * cfg.warpN * db; };
    while (p > 1 && (tileRows % p != 0 || ringBytes + bytes(p) > double(hw.smemBytesPerSM))) --p;
    return bytes(p);
}

// Workgroups per CU allowed by the register file.
double workgroupsByRegisters(const GemmConfig& cfg, const HardwareModel& hw, int numWarps, int threadsPerCta) {
    if (cfg.regsPerThread <= 0) return 1e9;
    if (hw.simdsPerSM <= 0) {
        // One pooled file per SM (reference :59-62).
        return std::floor(double(hw.regsPerSM) / (double(cfg.regsPerThread) * threadsPerCta));
    }
    // Per-SIMD files: each wave of the workgroup lands on one SIMD, and a SIMD
    // holds floor(budget / rounded-registers) waves.
    const int g = hw.regGranule;
    const int rounded = (cfg.regsPerThread + g - 1) / g * g;
    const double wavesPerSimd = std::floor(double(hw.regsPerSimdLane) / rounded);
    const double wavesPerSimdPerCta = std::ceil(double(numWarps) / hw.simdsPerSM);
    return std::floor(wavesPerSimd / wavesPerSimdPerCta);
}

// Loaded-clock ratio for a wave that keeps `busy` (0, 1] of the CUs busy: 1 at
// a full chip, the calibrated ratios at 1/2, 1/4, 1/8 and 1/16, linear in
// log2(1 / busy) between them and flat beyond 1/16.
double clockRatioAtBusyShare(const HardwareModel& hw, double busy) {
    if (busy >= 1.0) return 1.0;
    const double x = std::min(4.0, std::log2(1.0 / std::max(busy, 1e-9)));
    const double pts[5] = {1.0, hw.clockRatio[0], hw.clockRatio[1], hw.clockRatio[2], hw.clockRatio[3]};
    const int i = std::min(3, int(x));
    const double f = x - i;
    return pts[i] + (pts[i + 1] - pts[i]) * f;
}

// Distinct A row panels and B column panels that the first n workgroups touch,
// summed over XCDs, in the kernels' exact launch order: hardware workgroup p runs
// on XCD p % X; the kernel maps it to logical id xcdRemap(p) = x*q + min(x, r) +
// p / X (q, r = tiles / X, % X), and the logical id to a tile by the GroupM
// order. XCD x holds the first ceil((n - x) / X) ids of its range, and fetches
// every distinct panel of its tiles once into its own L2.
void launchOrderPanels(const GemmConfig& cfg, const HardwareModel& hw, long long n, double& rowPanels,
                       double& colPanels) {
    const long long numPidM = cfg.M / cfg.BM;
    const long long numPidN = cfg.N / cfg.BN;
    const long long total = numPidM * numPidN;
    const long long X = hw.numXcds;
    const long long q = total / X, r = total % X;
    const long long G = std::max(1, cfg.groupM);
    std::vector<long long> rowSeen(numPidM, -1), colSeen(numPidN, -1);
    rowPanels = 0.0;
    colPanels = 0.0;
    for (long long x = 0; x < X && x < n; ++x) {
        const long long base = x * q + std::min(x, r);
        const long long count = (n - x + X - 1) / X;
        for (long long j = 0; j < count; ++j) {
            const long long pid = base + j;
            const long long pidInGroup = pid % (G * numPidN);
            const long long firstPidM = (pid / (G * numPidN)) * G;
            const long long groupRows = std::min(numPidM - firstPidM, G);
            const long long row = firstPidM + pidInGroup % groupRows;
            const long long col = pidInGroup / groupRows;
            if (rowSeen[row] != x) {
                rowSeen[row] = x;
                rowPanels += 1.0;
            }
            if (colSeen[col] != x) {
                colSeen[col] = x;
                colPanels += 1.0;
            }
        }
    }
}

// Per K-step cycles of one workgroup's matrix instructions and of the operand
// reads out of LDS that feed them (for cfg's wave grid and BK).
void stepParts(const GemmConfig& cfg, const HardwareModel& hw, int db, double& tCompute, double& tSmem) {
    const int numWarps = (cfg.BM / cfg.warpM) * (cfg.BN / cfg.warpN);
    const double mmasPerWarpPerStep =
        double(cfg.warpM / cfg.mmaM) * (cfg.warpN / cfg.mmaN) * (cfg.BK / cfg.mmaK);
    tCompute = mmasPerWarpPerStep * numWarps * hw.mmaCyclesPerInst;
    const double smemBytesPerStep = double(numWarps) * (cfg.warpM + cfg.warpN) * cfg.BK * db;
    // ldsReadModel 1: A fragments come from ds_read_b128, B fragments from the
    // transposing ds_read_b64_tr_b16 at half its rate; each at its calibrated rate.
    tSmem = hw.ldsReadModel == 1
                ? double(numWarps) * cfg.BK * db *
                      (cfg.warpM / hw.ldsAReadBytesPerCycle + cfg.warpN / hw.ldsBTrReadBytesPerCycle)
                : smemBytesPerStep / hw.smemBytesPerCycle;
}

// persistentStepModel 1: the measured K-step of the persistent skeleton of a
// row's class over the model's reads + MFMAs for the skeleton's own row. The
// skeletons are cal-smem-bw's: 128x128x64 w64x64 (one compute wave per SIMD)
// and 256x128x32 w64x64 (two).
double persistentStepRatio(const GemmConfig& cfg, const HardwareModel& hw, int db, int computeWavesPerSimd) {
    GemmConfig skel = cfg;
    const bool two = computeWavesPerSimd >= 2;
    skel.BM = two ? 256 : 128;
    skel.BN = 128;
    skel.BK = two ? 32 : 64;
    skel.warpM = 64;
    skel.warpN = 64;
    double tC = 0.0, tS = 0.0;
    stepParts(skel, hw, db, tC, tS);
    return hw.persistentStepCycles[two ? 1 : 0] / (tC + tS);
}

// pingPongStepModel 1: the measured K-step of the ping-pong row skeleton of a
// row's class (BK = 32, or BK of 64 and above) over the model's max(MFMAs,
// reads) for the skeleton's own row. The skeletons are cal-smem-bw's: 256x256x32 w128x64 s3 and
// 256x128x64 w64x64 s3, the kernel's phase loop on an L2-resident source.
double pingPongStepRatio(const GemmConfig& cfg, const HardwareModel& hw, int db) {
    GemmConfig skel = cfg;
    const bool deep = cfg.BK >= 64;
    skel.BM = 256;
    skel.BN = deep ? 128 : 256;
    skel.BK = deep ? 64 : 32;
    skel.warpM = deep ? 64 : 128;
    skel.warpN = 64;
    double tC = 0.0, tS = 0.0;
    stepParts(skel, hw, db, tC, tS);
    return hw.pingPongRowStepCycles[deep ? 1 : 0] / std::max(tC, tS);
}

}  // namespace

Prediction predictCore(const GemmConfig& cfgIn, const HardwareModel& hw) {
    GemmConfig cfg = cfgIn;
    const MmaShape mma = mmaShapeFor(cfg.dtype, hw);
    if (cfg.mmaM == 0) {
        cfg.mmaM = mma.m;
        cfg.mmaN = mma.n;
        cfg.mmaK = mma.k;
    }
    const int db = dtypeBytes(cfg.dtype);

    Prediction p;

    const int numWarps = (cfg.BM / cfg.warpM) * (cfg.BN / cfg.warpN);
    // A persistent row's loader waves take wave slots and registers but issue
    // no matrix instructions and no operand reads.
    const bool persistent = hw.persistentModel == 1 && cfg.schedule == 2;
    const int residentWarps = persistent ? numWarps + kPersistentLoaderWaves : numWarps;
    const int threadsPerCta = residentWarps * hw.waveSize;
    p.numWarps = numWarps;

    // Per K-step times of one workgroup: matrix instructions, and the operand
    // reads out of LDS that feed them (in series: the next instruction consumes
    // the registers the read just wrote). The global->LDS copies are
    // asynchronous and appear only in the envelope.
    double tCompute = 0.0, tSmem = 0.0;
    stepParts(cfg, hw, db, tCompute, tSmem);
    // The ping-pong schedule (two waves per SIMD, a ring of three or more stages)
    // runs one wave's operand reads under the other wave's MFMAs, so a K-step
    // costs the longer of the two instead of their sum.
    const bool derivedPingPong = hw.simdsPerSM > 0 && numWarps == 2 * hw.simdsPerSM && cfg.stages >= 3;
    const bool pingPong = hw.pingPongModel == 1 && (cfg.schedule < 0 ? derivedPingPong : cfg.schedule == 1);
    double tStep = pingPong ? std::max(tCompute, tSmem) : tCompute + tSmem;
    // The row skeleton of the same class (BK) runs the schedule's barriers,
    // waits and refill writes, which the max leaves out.
    if (pingPong && hw.pingPongStepModel == 1) tStep *= pingPongStepRatio(cfg, hw, db);
    // uniformOverlapModel 1: two compute waves per SIMD that run the uniform
    // schedule (the 8-wave uniform rows, and the 8-compute-wave persistent rows,
    // whose compute waves run the same loop with one barrier per K tile) hide
    // part of the shorter phase under the longer with no schedule doing it: the
    // share cal-smem-bw measures for the same waves without barriers.
    if (persistent && hw.persistentStepModel == 1 && hw.simdsPerSM > 0) {
        // The persistent skeleton of the row's class has the row's barriers,
        // loader waves and refill; its measured K-step replaces the overlap
        // share of barrier-free waves.
        tStep = persistentStepRatio(cfg, hw, db, numWarps / hw.simdsPerSM) * (tCompute + tSmem);
    } else if (!pingPong && hw.uniformOverlapModel == 1 && hw.simdsPerSM > 0 && numWarps == 2 * hw.simdsPerSM) {
        tStep -= hw.freeRunningOverlap * std::min(tCompute, tSmem);
    }
    p.tComputeCycles = tCompute;
    p.tSmemCycles = tSmem;
    p.tStepCycles = tStep;
    p.smEfficiency = tCompute / tStep;

    // Occupancy: the tightest of LDS, wave slots, registers and the workgroup cap.
    const double ringBytes = double(cfg.stages) * (cfg.BM * cfg.BK + cfg.BK * cfg.BN) * db;
    const double smemBytesPerCta =
        persistent ? ringBytes + persistentStagingBytes(cfg, hw, numWarps, ringBytes, db) : ringBytes;
    const double ctasBySmem = std::floor(hw.smemBytesPerSM / smemBytesPerCta);
    const double ctasByWarps = std::floor(double(hw.maxWarpsPerSM) / residentWarps);
    const double ctasByRegs = workgroupsByRegisters(cfg, hw, residentWarps, threadsPerCta);
    const double ctasPerSM =
        std::min(std::min(ctasBySmem, ctasByWarps), std::min(ctasByRegs, double(hw.maxCtasPerSM)));
    if (ctasPerSM < 1.0) {
        p.bottleneck = Bottleneck::DoesNotFit;
        p.ctasPerSM = 0;
        return p;
    }
    p.ctasPerSM = int(ctasPerSM);

    // mallStreamModel 1: the refill of the panels an XCD's resident tiles share
    // is served by its L2 after the first load; the first loads (distinct panels
    // per XCD, in the kernels' launch order) cross to the MALL. When that stream
    // loads the MALL path, a K-step stretches as the calibrated skeleton's did
    // at the same load (linear between its points, proportional to the load
    // beyond the last, where the path's bandwidth binds).
    if (hw.mallStreamModel == 1 && hw.simdsPerSM > 0) {
        const double slots = ctasPerSM * double(hw.numSMs);
        const double tiles = double((cfg.M / cfg.BM) * (cfg.N / cfg.BN));
        const long long n = (long long)std::min(slots, tiles);
        double rowPanels = 0.0, colPanels = 0.0;
        launchOrderPanels(cfg, hw, n, rowPanels, colPanels);
        p.refillMissShare = std::min(1.0, (rowPanels * cfg.BM + colPanels * cfg.BN) / (double(n) * (cfg.BM + cfg.BN)));
        // Every resident tile advances one K-step per ctasPerSM x tStep cycles of its CU.
        const double missBytes = (rowPanels * cfg.BM + colPanels * cfg.BN) * double(cfg.BK) * db;
        const double stepSeconds = ctasPerSM * tStep / hw.clockHz;
        const double load = missBytes / hw.mallRefillBytesPerSec / stepSeconds;
        const double* x = hw.mallStretchLoad;
        const double* y = hw.mallStretch;
        double stretch = 1.0;
        if (load >= x[4]) {
            stretch = y[4] * load / x[4];
        } else {
            for (int i = 0; i < 4; ++i)
                if (load >= x[i] && load <= x[i + 1])
                    stretch = y[i] + (y[i + 1] - y[i]) * (load - x[i]) / (x[i + 1] - x[i]);
        }
        p.mallLoad = load;
        p.mallStretch = std::max(1.0, stretch);
        tStep *= p.mallStretch;
        p.tStepCycles = tStep;
        p.smEfficiency = tCompute / tStep;
    }
    const double smEfficiency = p.smEfficiency;

    // Latency hiding: resident waves against the calibrated need. A wave that
    // carries 8 or more independent accumulator chains per K-step hides latency
    // on its own ILP, and needs the ILP-8 column of the calibration surface
    // (when measured) instead of the single-chain-pair default.
    const double activeWarps = ctasPerSM * numWarps;
    const double chains = double(cfg.warpM / cfg.mmaM) * (cfg.warpN / cfg.mmaN);
    const double wavesToHide =
        hw.warpsNeededToHideIlp8 > 0.0 && chains >= 8.0 ? hw.warpsNeededToHideIlp8 : hw.warpsNeededToHide;
    const double occFactor = std::min(1.0, activeWarps / wavesToHide);
    p.occFactor = occFactor;

    // Wave quantisation over all resident workgroup slots.
    const double ctaSlots = ctasPerSM * double(hw.numSMs);
    const double totalCtas = double((cfg.M / cfg.BM) * (cfg.N / cfg.BN));
    const double wavesExact = totalCtas / ctaSlots;
    const double fullWaves = std::ceil(wavesExact);
    const double waveEfficiency = fullWaves > 0.0 ? totalCtas / (fullWaves * ctaSlots) : 1.0;
    // clockModel 1: under a full matrix load the chip is power-limited, so the
    // last wave, which leaves CUs idle when the grid does not fill the slots, runs
    // at a higher clock: the calibrated ratio for the share of CUs it keeps busy.
    // The run then lasts (fullWaves - 1) + 1 / ratio full-chip wave times.
    double clockedWaveEfficiency = waveEfficiency;
    if (hw.clockModel == 1 && fullWaves > 0.0) {
        const double tailCtas = totalCtas - (fullWaves - 1.0) * ctaSlots;
        const double busy = std::min(double(hw.numSMs), tailCtas) / double(hw.numSMs);
        p.tailClockFactor = clockRatioAtBusyShare(hw, busy);
        clockedWaveEfficiency = totalCtas / (((fullWaves - 1.0) + 1.0 / p.tailClockFactor) * ctaSlots);
    }
    p.ctaSlots = ctaSlots;
    p.totalCtas = totalCtas;
    p.wavesExact = wavesExact;
    p.waveEfficiency = waveEfficiency;

    // Fill and drain: STAGES-1 tiles land before the first instruction, the output
    // tile drains after the last; only the first fill and last drain of a CU are
    // exposed, hence the division by resident workgroups.
    const double gmemBytesPerCycle = hw.hbmBytesPerSec / (hw.clockHz * double(hw.numSMs));
    const double tileBytes = double(cfg.BM * cfg.BK + cfg.BK * cfg.BN) * db;
    const double kSteps = double(cfg.K) / cfg.BK;
    // The reference fills stages-1 tiles whatever K is; the kernels here issue
    // only the tiles that exist (prologueModel 1).
    const double prologueTiles =
        hw.prologueModel == 1 ? std::min(double(cfg.stages - 1), kSteps) : double(cfg.stages - 1);
    double tPrologue = prologueTiles * tileBytes / gmemBytesPerCycle / ctasPerSM;
    if (hw.fillShareModel == 1) {
        // The resident workgroups fill together. Each XCD fetches each distinct
        // A row panel and B column panel slice of its tiles from HBM once; the
        // other workgroups sharing that slice read it from the XCD's L2. The
        // fill takes that split's time instead of every tile's bytes from HBM.
        const long long n = (long long)std::min(ctaSlots, totalCtas);
        double rowPanels = 0.0, colPanels = 0.0;
        launchOrderPanels(cfg, hw, n, rowPanels, colPanels);
        const double allBytes = double(n) * tileBytes;
        const double uniqueBytes = std::min(allBytes, (rowPanels * cfg.BM + colPanels * cfg.BN) * double(cfg.BK) * db);
        const double shared =
            uniqueBytes / hw.hbmBytesPerSec + (allBytes - uniqueBytes) / (hw.l2HitBytesPerCycle * hw.clockHz);
        tPrologue *= std::min(1.0, shared / (allBytes / hw.hbmBytesPerSec));
    }
    // hbmWriteModel 1: the drain moves at the streaming-write rate.
    // mallWriteModel 1: the last drain's cached stores of C (all but the
    // persistent rows, which store non-temporally) land in the MALL when A, B and
    // C fit in it, at the MALL's write rate, shared by the CUs that hold a
    // workgroup (a grid of fewer workgroups than CUs leaves some idle). A drain to
    // HBM keeps the streaming-write rate over all CUs. The DRAM-side write time
    // below keeps the streaming-write rate too: a write-bound row's sustained C
    // stream does not reach the MALL's rate (measured 2.6-3.3 TB/s at 8192 x 2048
    // x 128 with C in the MALL).
    const bool cachedC = hw.mallWriteModel == 1 && !persistent &&
                         (double(cfg.M) * cfg.K + double(cfg.K) * cfg.N) * db +
                                 double(cfg.M) * cfg.N * hw.cBytes <= hw.mallBytes;
    const double writeRate = cachedC ? hw.mallWriteBytesPerSec : hw.hbmWriteBytesPerSec;
    // The dispatcher gives each workgroup a CU of its own while CUs are free.
    const double drainers =
        cachedC ? std::max(1.0, std::min(double(hw.numSMs), std::min(totalCtas, ctaSlots))) : double(hw.numSMs);
    const double drainBytesPerCycle =
        hw.hbmWriteModel == 1 ? writeRate / (hw.clockHz * drainers) : gmemBytesPerCycle;
    const double tEpilogue = double(cfg.BM) * cfg.BN * double(hw.cBytes) / drainBytesPerCycle / ctasPerSM;
    const double tBody = kSteps * tStep;
    double envelopeEfficiency;
    if (persistent) {
        // One workgroup per slot walks the busiest slot's ceil(tiles / slots)
        // tiles: one fill, that many bodies (each tile's stores drain under the
        // next body), one drain.
        const double walked = tBody * fullWaves;
        // persistentTileModel 1: before each next tile the compute waves stage
        // the finished tile through LDS and issue its stores, with no MFMA to
        // run; the skeleton of the row's class measures those cycles per tile.
        double between = 0.0;
        if (hw.persistentTileModel == 1 && hw.simdsPerSM > 0)
            between = fullWaves * hw.persistentTileCycles[numWarps / hw.simdsPerSM >= 2 ? 1 : 0];
        envelopeEfficiency = walked / (tPrologue + walked + between + tEpilogue);
    } else {
        envelopeEfficiency = tBody / (tPrologue + tBody + tEpilogue);
    }
    p.kSteps = kSteps;
    p.tPrologueCycles = tPrologue;
    p.tEpilogueCycles = tEpilogue;
    p.tBodyCycles = tBody;
    p.envelopeEfficiency = envelopeEfficiency;

    // Compute ceiling: resident workgroups share the matrix pipes, so occupancy
    // hides latency but never multiplies the peak.
    const double peakTensorTFLOPS = (double(mma.flops) / hw.mmaCyclesPerInst) * hw.clockHz * hw.numSMs / 1e12;
    double computeTFLOPS = peakTensorTFLOPS * smEfficiency * occFactor * clockedWaveEfficiency * envelopeEfficiency;
    if (hw.powerModel == 1) {
        // The chip is power-limited: with the GEMM's operand reads and refill under
        // fully busy matrix pipes the clock falls to loadedClockRatio of a pure
        // MFMA stream's; a row that keeps the pipes busy a share u of the time
        // pays that share of the drop.
        const double u = std::min(1.0, computeTFLOPS / peakTensorTFLOPS);
        p.matrixLoad = u;
        p.powerClockFactor = 1.0 - (1.0 - hw.loadedClockRatio) * u;
        computeTFLOPS *= p.powerClockFactor;
    }
    p.peakTensorTFLOPS = peakTensorTFLOPS;
    p.computeTFLOPS = computeTFLOPS;

    // HBM roofline.
    const double globalBytesPerCta = double(cfg.BM * cfg.K + cfg.K * cfg.BN) * db;
    const double flopsPerCta = 2.0 * double(cfg.BM) * cfg.BN * cfg.K;
    const double baseIntensity = flopsPerCta / globalBytesPerCta;
    double arithmeticIntensity;
    double panelIntensity;  // FLOP per byte of A and B panel traffic, before the compulsory cap
    if (hw.l2ReuseModel == 0) {
        // Square reuse over all resident slots (reference :116-123).
        const double l2ReuseFactor = std::sqrt(ctaSlots);
        arithmeticIntensity = baseIntensity * l2ReuseFactor;
        panelIntensity = arithmeticIntensity;
        p.l2ReuseFactor = l2ReuseFactor;
    } else if (hw.l2ReuseModel == 2) {
        // The kernels' launch order, exactly (launchOrderPanels): each XCD
        // fetches every distinct A row panel and B column panel of its resident
        // tiles once into its own L2; the traffic is summed over XCDs.
        const long long n = (long long)std::min(ctaSlots, totalCtas);
        const long long X = hw.numXcds;
        double rowPanels = 0.0, colPanels = 0.0;
        launchOrderPanels(cfg, hw, n, rowPanels, colPanels);
        const double residentFlops = 2.0 * double(n) * cfg.BM * cfg.BN * double(cfg.K);
        const double residentBytes = (rowPanels * cfg.BM + colPanels * cfg.BN) * double(cfg.K) * db;
        const double l2Intensity = residentFlops / residentBytes;
        const double M = double(cfg.M), N = double(cfg.N), K = double(cfg.K);
        const double compulsory = 2.0 * M * N * K / ((M * K + K * N) * db + M * N * hw.cBytes);
        arithmeticIntensity = std::min(l2Intensity, compulsory);
        panelIntensity = l2Intensity;
        p.l2ReuseFactor = arithmeticIntensity / baseIntensity;
        const double xcdsUsed = double(std::min(X, n));
        p.reuseTilesM = rowPanels / xcdsUsed;
        p.reuseTilesN = colPanels / xcdsUsed;
        p.compulsoryIntensity = compulsory;
    } else {
        // The workgroups resident on one XCD at a time, as compact a block of
        // output tiles as the grid allows: a rows x b columns of tiles. Each XCD
        // fetches a row panels of A and b column panels of B once into its own
        // L2. The block can never exceed the grid, which is what lets a
        // tall-skinny problem (one column of tiles) reach the HBM branch.
        const double numPidM = double(cfg.M / cfg.BM);
        const double numPidN = double(cfg.N / cfg.BN);
        const double perXcd = std::max(1.0, std::min(ctaSlots, totalCtas) / double(hw.numXcds));
        double a = std::max(1.0, std::min(numPidM, std::floor(std::sqrt(perXcd))));
        const double b = std::max(1.0, std::min(numPidN, std::ceil(perXcd / a)));
        a = std::max(1.0, std::min(numPidM, std::ceil(perXcd / b)));
        const double blockFlops = 2.0 * (a * cfg.BM) * (b * cfg.BN) * double(cfg.K);
        const double blockBytes = (a * cfg.BM + b * cfg.BN) * double(cfg.K) * db;
        const double l2Intensity = blockFlops / blockBytes;
        // No schedule beats the compulsory traffic of the whole problem.
        const double M = double(cfg.M), N = double(cfg.N), K = double(cfg.K);
        const double compulsory = 2.0 * M * N * K / ((M * K + K * N) * db + M * N * hw.cBytes);
        arithmeticIntensity = std::min(l2Intensity, compulsory);
        panelIntensity = l2Intensity;
        p.l2ReuseFactor = arithmeticIntensity / baseIntensity;
        p.reuseTilesM = a;
        p.reuseTilesN = b;
        p.compulsoryIntensity = compulsory;
    }
    p.baseIntensity = baseIntensity;
    p.arithmeticIntensity = arithmeticIntensity;
    p.hbmTFLOPS = hw.hbmBytesPerSec * arithmeticIntensity / 1e12;
    if (hw.hbmWriteModel == 1) {
        // DRAM traffic split by direction: A and B panels (at least once each)
        // read at the read rate, C written once at the write rate, one after the
        // other on the bus. With l2StreamModel 1 the panel loads that the L2s
        // serve take their own time on top, as below.
        const double M = double(cfg.M), N = double(cfg.N), K = double(cfg.K);
        const double flops = 2.0 * M * N * K;
        const double readBytes = std::max(flops / panelIntensity, (M * K + K * N) * db);
        const double writeBytes = M * N * hw.cBytes;
        p.dramReadBytes = readBytes;
        p.dramWriteBytes = writeBytes;
        double readSeconds = readBytes / hw.hbmBytesPerSec;
        if (hw.mallReuseModel == 1 && (M * K + K * N) * db <= hw.mallBytes) {
            // A and B stay in the MALL: HBM supplies each byte once, and the
            // L2s' further misses (XCDs re-fetching panels) are MALL hits.
            const double compulsory = (M * K + K * N) * db;
            readSeconds = compulsory / hw.hbmBytesPerSec + (readBytes - compulsory) / hw.mallRefillBytesPerSec;
        }
        const double writeSeconds = writeBytes / hw.hbmWriteBytesPerSec;
        double l2Seconds = 0.0;
        if (hw.l2StreamModel == 1) {
            p.l2HitBytes = std::max(0.0, flops / baseIntensity - readBytes);
            l2Seconds = p.l2HitBytes / (hw.l2HitBytesPerCycle * hw.clockHz);
        }
        // writeOverlapModel 1: two resources, each used in series. The DRAM bus
        // carries the reads, then the writes; the CUs' load path takes the loads
        // DRAM serves, then the ones the L2s serve. C's writes and the L2-served
        // loads use neither in common, so they overlap, and the busier resource
        // bounds the launch. Otherwise the three streams are summed.
        const double seconds = hw.writeOverlapModel == 1 ? readSeconds + std::max(writeSeconds, l2Seconds)
                                                         : readSeconds + writeSeconds + l2Seconds;
        p.arithmeticIntensity = flops / (readBytes + writeBytes);
        p.hbmTFLOPS = flops / seconds / 1e12;
    } else if (hw.l2StreamModel == 1) {
        // Every workgroup loads its (BM + BN) x K panels; the share that HBM does
        // not supply (a panel re-read by the workgroups of one XCD) is served by
        // that XCD's L2, and a load-only kernel with the GEMM's streams takes the
        // sum of the two stream times, not the larger.
        const double flops = 2.0 * double(cfg.M) * double(cfg.N) * double(cfg.K);
        const double hbmBytes = flops / arithmeticIntensity;
        const double tileBytes = flops / baseIntensity;
        const double seconds = hbmBytes / hw.hbmBytesPerSec +
                               std::max(0.0, tileBytes - hbmBytes) / (hw.l2HitBytesPerCycle * hw.clockHz);
        p.l2HitBytes = std::max(0.0, tileBytes - hbmBytes);
        p.hbmTFLOPS = flops / seconds / 1e12;
    }

    // The label names the derating furthest from 1.0 (reference :129-143).
    p.predictedTFLOPS = std::min(computeTFLOPS, p.hbmTFLOPS);
    if (hw.fillLatencyModel == 1) {
        // A workgroup's first K tile cannot be fetched before the workgroup
        // exists, so every round of one-tile-per-workgroup workgroups waits one
        // loaded DRAM latency before its first MFMA; a persistent grid waits
        // once. The wait adds to whichever ceiling binds, so it is added to both.
        const double rounds = persistent ? 1.0 : fullWaves;
        const double flops = 2.0 * double(cfg.M) * double(cfg.N) * double(cfg.K);
        const double wait = rounds * hw.fillLatencySec;
        computeTFLOPS = flops / (flops / (computeTFLOPS * 1e12) + wait) / 1e12;
        p.hbmTFLOPS = flops / (flops / (p.hbmTFLOPS * 1e12) + wait) / 1e12;
        p.computeTFLOPS = computeTFLOPS;
        p.fillRounds = rounds;
        p.predictedTFLOPS = std::min(computeTFLOPS, p.hbmTFLOPS);
    }
    if (hw.launchModel == 1) {
        // A kernel boundary in a back-to-back sequence: the next launch's queue
        // processing overlaps the running kernel, the rest of the boundary adds
        // to whichever ceiling binds.
        const double flops = 2.0 * double(cfg.M) * double(cfg.N) * double(cfg.K);
        computeTFLOPS = flops / (flops / (computeTFLOPS * 1e12) + hw.launchOverheadSeconds) / 1e12;
        p.hbmTFLOPS = flops / (flops / (p.hbmTFLOPS * 1e12) + hw.launchOverheadSeconds) / 1e12;
        p.computeTFLOPS = computeTFLOPS;
        p.predictedTFLOPS = std::min(computeTFLOPS, p.hbmTFLOPS);
    }
    if (p.hbmTFLOPS < computeTFLOPS) {
        p.bottleneck = Bottleneck::Hbm;
    } else {
        const double worst =
            std::min(std::min(smEfficiency, occFactor), std::min(waveEfficiency, envelopeEfficiency));
        if (worst >= 0.95)
            p.bottleneck = Bottleneck::TensorCore;
        else if (worst == waveEfficiency)
            p.bottleneck = Bottleneck::Waves;
        else if (worst == envelopeEfficiency)
            p.bottleneck = Bottleneck::Envelope;
        else if (worst == smEfficiency)
            p.bottleneck = Bottleneck::Smem;
        else
            p.bottleneck = Bottleneck::Occupancy;
    }
    return p;
}

namespace {

// labelModel 1: what the counters read on one launch of cfg from an idle
// stream, and the decision table's label for it.
void observe(const GemmConfig& cfg, const HardwareModel& hw, Prediction& p) {
    const double M = double(cfg.M), N = double(cfg.N);
    const double flops = 2.0 * M * N * double(cfg.K);
    const double backToBack = hw.launchModel == 1 ? hw.launchOverheadSeconds : 0.0;
    // One launch from an idle stream: the predicted work plus that launch's
    // kernel boundary in place of the back-to-back one.
    auto isolated = [&](const Prediction& q, double fl) {
        return fl / (q.predictedTFLOPS * 1e12) - backToBack + hw.launchIsolatedSeconds;
    };
    p.kernelSeconds = isolated(p, flops);
    p.dramShare = (p.dramReadBytes / hw.hbmBytesPerSec + p.dramWriteBytes / hw.hbmWriteBytesPerSec) / p.kernelSeconds;

    // Body share: the share of the duration that scales with K, from the
    // duration at a second K (K / 2 when that is a whole number of K tiles,
    // else 2 K): t(K) = fixed + body, t(f K) = fixed + f body.
    const long long half = cfg.K / 2;
    const bool useHalf = cfg.K % 2 == 0 && cfg.BK > 0 && half % cfg.BK == 0 && half >= cfg.BK;
    GemmConfig other = cfg;
    other.K = useHalf ? half : 2 * cfg.K;
    p.bodyFactor = useHalf ? 0.5 : 2.0;
    const Prediction q = predictCore(other, hw);
    const double t2 = isolated(q, 2.0 * M * N * double(other.K));
    p.bodyShare = (t2 - p.kernelSeconds) / ((p.bodyFactor - 1.0) * p.kernelSeconds);

    // CU share: a persistent grid holds min(tiles, slots) workgroups for the
    // whole launch; a one-tile-per-workgroup grid runs ceil(tiles / slots)
    // rounds, all CUs busy but in the last, which keeps min(1, tail / CUs).
    const double cus = double(hw.numSMs);
    const bool persistent = hw.persistentModel == 1 && cfg.schedule == 2;
    if (persistent) {
        p.cuShare = std::min(1.0, std::min(p.totalCtas, p.ctaSlots) / cus);
    } else {
        const double rounds = std::ceil(p.totalCtas / p.ctaSlots);
        const double tail = p.totalCtas - (rounds - 1.0) * p.ctaSlots;
        p.cuShare = ((rounds - 1.0) + std::min(1.0, tail / cus)) / rounds;
    }

    // Busy shares: every MFMA costs its issue cycles on one SIMD, every K-step
    // its fragment reads on the CU's LDS, over the cycles of the duration.
    // labelModel 1 counts those at the model's loaded clock. labelModel 2 counts
    // them at the clock the counters see: with the matrix pipes idle the engine
    // runs at nominalClockHz, with them always busy (and the GEMM's data
    // movement) at the calibrated skeleton's clockHz x loadedClockRatio, and a
    // row whose pipes are busy a share u of the time between the two. (The
    // throughput terms keep the loaded clock their cycle counts were calibrated
    // at; the counters count physical cycles.)
    const MmaShape mma = mmaShapeFor(cfg.dtype, hw);
    const double clock =
        hw.labelModel == 2
            ? hw.nominalClockHz + (hw.clockHz * hw.loadedClockRatio - hw.nominalClockHz) * p.matrixLoad
            : hw.clockHz * p.powerClockFactor;
    p.observedClockHz = clock;
    const double simds = cus * hw.simdsPerSM;
    const double mfmaCyclesPerSimd = flops / double(mma.flops) * hw.mmaCyclesPerInst * hw.simdsPerSM / simds;
    p.mfmaShare = mfmaCyclesPerSimd / (p.kernelSeconds * clock);
    p.ldsShare = p.totalCtas * p.kSteps * p.tSmemCycles / cus / (p.kernelSeconds * clock);

    if (p.dramShare >= kDramShareMin)
        p.bottleneck = Bottleneck::Hbm;
    else if (p.cuShare < kCuShareMin)
        p.bottleneck = Bottleneck::Waves;
    else if (p.bodyShare < kBodyShareMin)
        p.bottleneck = Bottleneck::Envelope;
    else if (p.ldsShare >= kLdsOverMfmaMin * p.mfmaShare)
        p.bottleneck = Bottleneck::Smem;
    else if (p.mfmaShare / std::min(1.0, p.bodyShare) >= kMfmaOverBodyMin)
        p.bottleneck = Bottleneck::TensorCore;
    else
        p.bottleneck = Bottleneck::Occupancy;
}

}  // namespace

Prediction predict(const GemmConfig& cfg, const HardwareModel& hw) {
    Prediction p = predictCore(cfg, hw);
    if ((hw.labelModel == 1 || hw.labelModel == 2) && p.bottleneck != Bottleneck::DoesNotFit) observe(cfg, hw, p);
    return p;
}

}  // namespace ridge
