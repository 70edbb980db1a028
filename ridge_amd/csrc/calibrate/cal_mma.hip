// cal_mma.hip -- mmaCyclesPerInst: CU-level cycles per v_mfma_f32_32x32x16_f16.
//
// Counterpart of the reference's bench/calibrate/cal-mma.cu:41-163. The trap is
// the same: throughput, not latency. Each wave keeps kIlp independent accumulator
// chains in registers so the matrix pipe always has an independent instruction
// queued; nothing touches memory inside the timed loop. Waves per workgroup are
// swept (one workgroup per CU) because "CU-level" only means something once all
// four SIMDs are busy: one wave drives one SIMD, four waves saturate the CU.
//
//   mmaCyclesPerInst  = median cycles / MFMAs issued on the CU
//   impliedPeakTflops = 32768 / mmaCyclesPerInst * measured clock * CUs
#include "cal_common.hpp"

using namespace ridgecal;

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kIlp = 4;
constexpr int kIters = 4000;
constexpr double kMfmaFlops = 32768.0;

template <int Waves>
__global__ __launch_bounds__(Waves * 64) void mfmaThroughputKernel(int iters, float* sink, Stamp* out) {
    extern __shared__ char lds[];  // requested only to force one workgroup per CU
    const int lane = threadIdx.x % 64;
    half8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // Finite values near 1, perturbed per lane so nothing constant-folds.
        a[i] = (_Float16)(1.0f + 0.001f * float((lane + i) & 15));
        b[i] = (_Float16)(1.0f - 0.001f * float((lane * 3 + i) & 15));
    }
    float16_t acc[kIlp];
#pragma unroll
    for (int j = 0; j < kIlp; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = float(threadIdx.x) * 1e-6f;
    if (threadIdx.x == 0) lds[0] = 0;
    __syncthreads();
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < kIlp; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    __syncthreads();
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kIlp; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[j][e];
    if (s == 1.2345678e30f) sink[0] = s;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

template <int Waves>
void measure(int cus, float* dSink, Stamp* dStamps, double& cyclesPerMfma, double& clockHz) {
    auto k = mfmaThroughputKernel<Waves>;
    CAL_HIP_CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kOneWorkgroupLds));
    hipLaunchKernelGGL(k, dim3(cus), dim3(Waves * 64), kOneWorkgroupLds, nullptr, kIters, dSink, dStamps);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(cus);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, cus * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0;
    medianStamps(st, cyc, clockHz);
    cyclesPerMfma = cyc / (double(Waves) * kIters * kIlp);
}

}  // namespace

int main() {
    const hipDeviceProp_t prop = deviceBanner();
    const int cus = prop.multiProcessorCount;
    float* dSink = nullptr;
    Stamp* dStamps = nullptr;
    CAL_HIP_CHECK(hipMalloc(&dSink, sizeof(float)));
    CAL_HIP_CHECK(hipMalloc(&dStamps, cus * sizeof(Stamp)));
    warmUp();

    std::printf("\nv_mfma_f32_32x32x16_f16 issue rate, %d independent chains per wave, %d iterations\n", kIlp,
                kIters);
    std::printf("  %6s %16s %14s %18s\n", "waves", "cycles/MFMA/CU", "clock MHz", "implied TFLOP/s");
    double best = 1e30, bestClock = 0.0;
    int bestWaves = 0;
    std::vector<double> bestReps;
#define CAL_SWEEP(W)                                                                         \
    do {                                                                                     \
        std::vector<double> reps, clocks;                                                    \
        for (int r = 0; r < kRepeats; ++r) {                                                 \
            double c = 0, hz = 0;                                                            \
            measure<W>(cus, dSink, dStamps, c, hz);                                          \
            reps.push_back(c);                                                               \
            clocks.push_back(hz);                                                            \
        }                                                                                    \
        const double c = median(reps), hz = median(clocks);                                  \
        std::printf("  %6d %16.4f %14.1f %18.1f\n", W, c, hz / 1e6, kMfmaFlops / c * hz * cus / 1e12); \
        std::printf("CAL_CURVE waves %d cyclesPerMfma %.6f clockHz %.6e\n", W, c, hz);       \
        if (c < best * 0.999) {                                                              \
            best = c;                                                                        \
            bestWaves = W;                                                                   \
            bestReps = reps;                                                                 \
            bestClock = hz;                                                                  \
        }                                                                                    \
    } while (0)
    CAL_SWEEP(1);
    CAL_SWEEP(2);
    CAL_SWEEP(4);
    CAL_SWEEP(8);
    CAL_SWEEP(16);
#undef CAL_SWEEP

    const double peak = kMfmaFlops / best * bestClock * cus / 1e12;
    const double peakNominal = kMfmaFlops / best * (prop.clockRate * 1e3) * cus / 1e12;
    std::printf("\nsaturated at %d waves per CU\n", bestWaves);
    const bool stable = reportConstant("mmaCyclesPerInst", best, "cycles", bestReps);
    std::printf("  %-24s %12.1f MHz (loaded, measured)\n", "clock", bestClock / 1e6);
    std::printf("  %-24s %12.1f TFLOP/s at the measured clock\n", "implied peak", peak);
    std::printf("  %-24s %12.1f TFLOP/s at the nominal clock\n", "implied peak (nominal)", peakNominal);
    std::printf("  %-24s %12.1f TFLOP/s (datasheet dense FP16, cross-check only)\n", "MI355X", 2516.6);
    std::printf("\nCAL_RESULT mmaCyclesPerInst %.6f\n", best);
    std::printf("CAL_RESULT impliedPeakTflops %.3f\n", peak);
    std::printf("CAL_RESULT impliedPeakTflopsNominalClock %.3f\n", peakNominal);
    std::printf("CAL_RESULT saturationWaves %d\n", bestWaves);
    std::printf("CAL_RESULT clockHz %.6e\n", bestClock);
    std::printf("CAL_RESULT nominalClockHz %.6e\n", prop.clockRate * 1e3);
    CAL_HIP_CHECK(hipFree(dSink));
    CAL_HIP_CHECK(hipFree(dStamps));
    return stable ? 0 : 1;
}
