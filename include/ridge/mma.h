// ridge/mma.h -- the matrix instruction shape for a dtype on a target.
// Counterpart of include/ridge/mma.h:7-13 of the reference, now taken from the
// hardware model (m16n8k16 on sm_80, v_mfma_f32_16x16x32_f16 on gfx950).
#pragma once
#include <cstdint>
#include "ridge/config.h"

namespace ridge {

struct HardwareModel;

struct MmaShape {
    int m, n, k;
    int64_t flops;  // 2 * m * n * k
};

// The reference's fixed sm_80 shape (mma.cpp:5-12).
MmaShape mmaShapeFor(DType dtype);

// The shape the given hardware model declares for the dtype.
MmaShape mmaShapeFor(DType dtype, const HardwareModel& hw);

}  // namespace ridge
