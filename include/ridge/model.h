// ridge/model.h -- closed-form throughput and bottleneck prediction.
// Same entry point as the reference (include/ridge/model.h:10).
#pragma once
#include "ridge/config.h"
#include "ridge/hardware.h"
#include "ridge/prediction.h"

namespace ridge {

Prediction predict(const GemmConfig& cfg, const HardwareModel& hw);

}  // namespace ridge
