// cal_hbm_bw.hip -- hbmBytesPerSec: sustained HBM read bandwidth of the GPU.
//
// Counterpart of the reference's bench/calibrate/cal-hbm-bw.cu:22-109: a
// grid-stride 16-byte streaming read over a 4 GiB buffer, far beyond both the
// 4 MiB L2 of each XCD and the 256 MiB shared MALL, so the reads come from HBM;
// 7 timed repeats, median. A 64 MiB buffer (MALL-resident) is also timed and
// reported as information: that is the level that serves cross-XCD panel
// re-reads in the GEMM.
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

double timeRead(const float4_t* src, size_t bytes, float* sink, int blocks, std::vector<double>& reps) {
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    const size_t n = bytes / sizeof(float4_t);
    reps.clear();
    for (int r = 0; r < kRepeats; ++r) {
        hipLaunchKernelGGL(streamReadKernel, dim3(blocks), dim3(256), 0, nullptr, src, n, sink);
        CAL_HIP_CHECK(hipDeviceSynchronize());
        CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
        hipLaunchKernelGGL(streamReadKernel, dim3(blocks), dim3(256), 0, nullptr, src, n, sink);
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
    std::printf("\nCAL_RESULT hbmBytesPerSec %.6e\n", hbm);
    std::printf("CAL_RESULT mallBytesPerSec %.6e\n", mall);
    CAL_HIP_CHECK(hipFree(src));
    CAL_HIP_CHECK(hipFree(sink));
    return stable ? 0 : 1;
}
