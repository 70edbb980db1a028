// cal_hbm_bw.hip -- hbmBytesPerSec: sustained HBM read bandwidth of the GPU.
//
// Counterpart of the reference's bench/calibrate/cal-hbm-bw.cu:22-109: a
// grid-stride 16-byte streaming read over a 4 GiB buffer, far beyond both the
// 4 MiB L2 of each XCD and the 256 MiB shared MALL, so the reads come from HBM;
// 7 timed repeats, median. A 64 MiB buffer (MALL-resident) is also timed and
// reported as information: that is the level that serves cross-XCD panel
// re-reads in the GEMM. l2HitBytesPerCycle times the same kind of read (16 GiB of
// it) with every index wrapped into a 1 MiB buffer, which each XCD's L2 holds, in
// shader cycles: the rate at which the L2s serve tiles that every workgroup
// re-reads (the shared operand of a skinny GEMM).
#include "cal_common.hpp"

using namespace ridgecal;

namespace {

typedef float float4_t __attribute__((ext_vector_type(4)));

__global__ void streamReadKernel(const float4_t* __restrict__ src, size_t n, float* sink) {
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) acc += src[i];
    const float s = acc[0] + acc[1] + acc[2] + acc[3];
    if (s == 1.2345678e30f) sink[0] = s;
}

// The same read over `n` float4 positions, each wrapped into the first `mask + 1`
// (a power of two) of the buffer, on a grid that is resident all at once; thread
// 0 of each workgroup stamps shader cycles and real time around its share.
__global__ __launch_bounds__(256) void wrappedReadKernel(const float4_t* __restrict__ src, size_t n, size_t mask,
                                                         float* sink, Stamp* out) {
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    __syncthreads();
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) acc += src[i & mask];
    __syncthreads();
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    const float s = acc[0] + acc[1] + acc[2] + acc[3];
    if (s == 1.2345678e30f) sink[0] = s;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

// Whole-GPU bytes per shader cycle of the wrapped read (median workgroup), and the
// loaded clock it ran at.
double l2BytesPerCycle(const float4_t* src, size_t bytes, size_t wrapBytes, float* sink, Stamp* dStamps, int blocks,
                       std::vector<double>& reps, double& clockHz) {
    const size_t n = bytes / sizeof(float4_t);
    const size_t mask = wrapBytes / sizeof(float4_t) - 1;
    std::vector<double> clocks;
    reps.clear();
    for (int r = 0; r < kRepeats; ++r) {
        hipLaunchKernelGGL(wrappedReadKernel, dim3(blocks), dim3(256), 0, nullptr, src, n, mask, sink, dStamps);
        CAL_HIP_CHECK(hipGetLastError());
        CAL_HIP_CHECK(hipDeviceSynchronize());
        std::vector<Stamp> st(blocks);
        CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, blocks * sizeof(Stamp), hipMemcpyDeviceToHost));
        double cyc = 0.0, hz = 0.0;
        medianStamps(st, cyc, hz);
        reps.push_back(double(bytes) / cyc);
        clocks.push_back(hz);
    }
    clockHz = median(clocks);
    return median(reps);
}

double timeRead(const float4_t* src, size_t bytes, float* sink, int blocks, std::vector<double>& reps) {
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    const size_t n = bytes / sizeof(float4_t);
    reps.clear();
    auto launch = [&]() { hipLaunchKernelGGL(streamReadKernel, dim3(blocks), dim3(256), 0, nullptr, src, n, sink); };
    for (int r = 0; r < kRepeats; ++r) {
        launch();
        CAL_HIP_CHECK(hipDeviceSynchronize());
        CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
        launch();
        CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
        CAL_HIP_CHECK(hipEventSynchronize(e1));
        CAL_HIP_CHECK(hipGetLastError());
        float ms = 0.0f;
        CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        reps.push_back(double(bytes) / (double(ms) * 1e-3));
    }
    CAL_HIP_CHECK(hipEventDestroy(e0));
    CAL_HIP_CHECK(hipEventDestroy(e1));
    return median(reps);
}

}  // namespace

int main() {
    const hipDeviceProp_t prop = deviceBanner();
    constexpr size_t kBytes = 4ull << 30;
    constexpr size_t kMallBytes = 64ull << 20;
    size_t freeB = 0, totalB = 0;
    CAL_HIP_CHECK(hipMemGetInfo(&freeB, &totalB));
    std::printf("device memory: %.1f GB total, %.1f GB free\n", totalB / 1e9, freeB / 1e9);
    if (freeB < kBytes + (256ull << 20)) {
        std::fprintf(stderr, "not enough free memory for a 4 GiB buffer; a smaller one would measure the MALL\n");
        return 2;
    }
    float4_t* src = nullptr;
    float* sink = nullptr;
    CAL_HIP_CHECK(hipMalloc(&src, kBytes));
    CAL_HIP_CHECK(hipMalloc(&sink, sizeof(float)));
    CAL_HIP_CHECK(hipMemset(src, 1, kBytes));
    warmUp();
    const int blocks = prop.multiProcessorCount * 32;
    std::printf("\nHBM streaming read, %.2f GiB buffer, %d blocks x 256 workitems, 16-byte loads\n",
                kBytes / double(1ull << 30), blocks);
    std::vector<double> reps;
    const double hbm = timeRead(src, kBytes, sink, blocks, reps);
    for (size_t i = 0; i < reps.size(); ++i) std::printf("  repeat %zu %10.1f GB/s\n", i, reps[i] / 1e9);
    const bool stable = reportConstant("hbmBytesPerSec", hbm / 1e9, "GB/s", reps);
    std::printf("  %-24s %12.1f GB/s (datasheet, cross-check only)\n", "MI355X HBM3E", 8000.0);
    std::printf("  %-24s %12.1f %%\n", "achieved vs datasheet", 100.0 * hbm / 8.0e12);
    std::vector<double> mallReps;
    const double mall = timeRead(src, kMallBytes, sink, blocks, mallReps);
    std::printf("  %-24s %12.1f GB/s (64 MiB, MALL-resident, information only)\n", "mallBytesPerSec", mall / 1e9);
    // 16 GiB of reads wrapped into 1 MiB, which each XCD's 4 MiB L2 holds, on 8
    // workgroups of 256 per CU (all resident). A rate in bytes per second follows
    // the power-managed clock from launch to launch; bytes per shader cycle is the
    // stable constant, and the model scales it by its own loaded clock.
    constexpr size_t kL2Bytes = 1ull << 20;
    constexpr size_t kL2ReadBytes = 16ull << 30;
    const int l2Blocks = prop.multiProcessorCount * 8;
    Stamp* dStamps = nullptr;
    CAL_HIP_CHECK(hipMalloc(&dStamps, l2Blocks * sizeof(Stamp)));
    std::vector<double> l2Reps;
    double l2Clock = 0.0;
    const double l2 = l2BytesPerCycle(src, kL2ReadBytes, kL2Bytes, sink, dStamps, l2Blocks, l2Reps, l2Clock);
    for (size_t i = 0; i < l2Reps.size(); ++i) std::printf("  L2 repeat %zu %10.1f B/cycle\n", i, l2Reps[i]);
    const bool l2Stable = reportConstant("l2HitBytesPerCycle", l2, "B/cycle (GPU)", l2Reps);
    std::printf("  (16 GiB of reads wrapped into 1 MiB, served by the XCDs' L2s: %.1f TB/s at %.0f MHz)\n",
                l2 * l2Clock / 1e12, l2Clock / 1e6);
    CAL_HIP_CHECK(hipFree(dStamps));
    std::printf("\nCAL_RESULT hbmBytesPerSec %.6e\n", hbm);
    std::printf("CAL_RESULT mallBytesPerSec %.6e\n", mall);
    std::printf("CAL_RESULT l2HitBytesPerCycle %.6f\n", l2);
    CAL_HIP_CHECK(hipFree(src));
    CAL_HIP_CHECK(hipFree(sink));
    return stable && l2Stable ? 0 : 1;
}
