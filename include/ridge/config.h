// ridge/config.h -- one GEMM tile configuration, the cost model's input.
//
// Same fields and defaults as the reference's ridge::GemmConfig
// (include/ridge/config.h:18-39). "warp" fields are the SIMT group of the target:
// 32-thread warps on sm_80, 64-lane wavefronts on CDNA4.
#pragma once
#include <cstdint>

namespace ridge {

enum class DType { FP16 };

inline int dtypeBytes(DType d) {
    switch (d) {
        case DType::FP16: return 2;
    }
    return 2;
}

struct GemmConfig {
    int64_t M = 4096, N = 4096, K = 4096;
    DType dtype = DType::FP16;

    // Workgroup (CTA) tile.
    int BM = 128, BN = 128, BK = 32;

    // Wavefront (warp) tile. waves = (BM / warpM) * (BN / warpN).
    int warpM = 64, warpN = 64;

    // Matrix instruction shape; 0 means the hardware model's default.
    int mmaM = 0, mmaN = 0, mmaK = 0;

    // LDS (shared memory) ring depth.
    int stages = 3;

    // Registers per lane of the real kernel (VGPR + AGPR on CDNA, ptxas count on
    // sm_80). 0 = unknown: register occupancy is not applied.
    int regsPerThread = 128;

    // Launch-order group size along M (the kernel's GroupM). Only the exact
    // launch-order reuse model (HardwareModel::l2ReuseModel 2) reads it; the
    // reference model has no such field.
    int groupM = 8;

    // Kernel schedule of the row: -1 derives it from the tile (two waves per
    // SIMD with >= 3 stages is ping-pong, anything else uniform), 0 uniform,
    // 1 ping-pong, 2 persistent store-behind. Only HardwareModel::persistentModel
    // 1 reads the value 2; the reference model has no such field.
    int schedule = -1;
};

}  // namespace ridge
