// harness.hpp -- host-side timing and checking helpers shared by ridge-measure and
// ridge-check. Counterparts of the reference's warmUpGpu / timeMs / timeTflops /
// errorStats (bench/check-gemm.cu:110-179, bench/measure.cu:111-150), on HIP
// events and the C ABI of libridge_gemm.so.
#pragma once

#include "ridge_gemm.h"

#include "../common/stats.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace ridgeh {

#define RIDGE_HIP_CHECK(call)                                                                       \
    do {                                                                                            \
        hipError_t err_ = (call);                                                                   \
        if (err_ != hipSuccess) {                                                                   \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(err_), __FILE__, __LINE__); \
            std::exit(2);                                                                           \
        }                                                                                           \
    } while (0)

#define RIDGE_ABI_CHECK(call)                                                                       \
    do {                                                                                            \
        int rc_ = (call);                                                                           \
        if (rc_ != 0) {                                                                             \
            std::fprintf(stderr, "%s returned %d at %s:%d\n", #call, rc_, __FILE__, __LINE__);      \
            std::exit(2);                                                                           \
        }                                                                                           \
    } while (0)

// MI355X in its whole-device mode: 256 CUs, gfx950. A compute-partitioned GPU
// (CPX, DPX, ...) exposes a fraction of the CUs and XCDs as a device of its own;
// its throughput, wave quantisation and L2 layout are not the ones the sweep
// and the calibration describe, so the harnesses refuse it the way the
// reference's setup refuses a MIG slice (setup-box.sh:37-41) unless told
// otherwise.
constexpr int kWholeDeviceCus = 256;

inline void requireWholeDevice(const hipDeviceProp_t& prop, bool allowPartitioned) {
    const bool gfx950 = std::string(prop.gcnArchName).rfind("gfx950", 0) == 0;
    if (gfx950 && prop.multiProcessorCount == kWholeDeviceCus) return;
    std::fprintf(stderr, "device %s (%s) with %d CUs is not a whole MI355X (gfx950, %d CUs)%s\n", prop.name,
                 prop.gcnArchName, prop.multiProcessorCount, kWholeDeviceCus,
                 allowPartitioned ? "; continuing (--allow-partitioned)" : "; pass --allow-partitioned to run anyway");
    if (!allowPartitioned) std::exit(3);
}

inline double seconds() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// Runs `body` until `secs` of wall time have passed, synchronising every 10
// calls, so the clocks are at their loaded steady state before anything is timed.
inline void warmUp(const std::function<void()>& body, double secs) {
    const double t0 = seconds();
    while (seconds() - t0 < secs) {
        for (int i = 0; i < 10; ++i) body();
        RIDGE_HIP_CHECK(hipDeviceSynchronize());
    }
}

// Average milliseconds per call over `iters` calls after `warm` untimed calls.
inline double timeMs(const std::function<void()>& body, int warm, int iters) {
    hipEvent_t e0, e1;
    RIDGE_HIP_CHECK(hipEventCreate(&e0));
    RIDGE_HIP_CHECK(hipEventCreate(&e1));
    for (int i = 0; i < warm; ++i) body();
    RIDGE_HIP_CHECK(hipDeviceSynchronize());
    RIDGE_HIP_CHECK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i) body();
    RIDGE_HIP_CHECK(hipEventRecord(e1, nullptr));
    RIDGE_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    RIDGE_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    RIDGE_HIP_CHECK(hipEventDestroy(e0));
    RIDGE_HIP_CHECK(hipEventDestroy(e1));
    return double(ms) / iters;
}

struct Timing {
    double tflops = 0.0;
    double ms = 0.0;
    int iters = 0;
};

// The reference's adaptive measurement (measure.cu:121-150): 10 warm calls, a
// 5-call probe, then as many calls as fill `targetSeconds`, clamped to
// [minIters, maxIters].
inline Timing timeTflops(const std::function<void()>& body, double flops, double targetSeconds = 0.4,
                         int minIters = 20, int maxIters = 400) {
    const double probe = timeMs(body, 10, 5);
    int iters = int(targetSeconds * 1000.0 / std::max(probe, 1e-6));
    iters = std::min(std::max(iters, minIters), maxIters);
    Timing t;
    t.ms = timeMs(body, 0, iters);
    t.iters = iters;
    t.tflops = flops / (t.ms * 1e-3) / 1e12;
    return t;
}

using ridgestat::dispersion;
using ridgestat::middle;

// hipBLASLt comparator over the C ABI, prepared once per shape.
struct BlasLt {
    void* h = nullptr;
    BlasLt() { RIDGE_ABI_CHECK(ridge_blaslt_create(&h)); }
    ~BlasLt() { ridge_blaslt_destroy(h); }
    void prepare(const void* A, const void* B, void* C, int M, int N, int K, bool cF32 = false) {
        RIDGE_ABI_CHECK(ridge_blaslt_prepare(h, A, B, C, M, N, K, cF32 ? 1 : 0, 8, 10, nullptr));
    }
    void gemm(const void* A, const void* B, void* C, int M, int N, int K, bool cF32 = false) {
        RIDGE_ABI_CHECK(ridge_blaslt_gemm(h, A, B, C, M, N, K, cF32 ? 1 : 0, nullptr));
    }
};

// Half -> float for host-side checks (IEEE binary16, subnormals included).
inline float halfToFloat(uint16_t h) {
    const uint32_t sign = (uint32_t(h) & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    float f;
    if (e == 0) {
        f = float(m) * (1.0f / 16777216.0f);
        if (sign) f = -f;
        return f;
    }
    uint32_t x = (e == 31) ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    std::memcpy(&f, &x, 4);
    return f;
}

}  // namespace ridgeh
