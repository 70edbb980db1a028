// cal_latency.hip -- warpsNeededToHide: resident wavefronts per CU at which an
// LDS-read -> MFMA dependency chain stops losing throughput.
//
// Counterpart of the reference's bench/calibrate/cal-latency.cu:56-257. Each
// iteration of each of Ilp independent chains reads an A fragment with
// ds_read_b128 from the kernel's swizzled layout and feeds it straight into
// v_mfma_f32_32x32x16_f16, so the read latency sits in front of the matrix
// instruction. The whole waves x ILP surface is printed; the reported constant
// is the ILP = 2 column's first wave count within 95% of that column's best,
// as in the reference. Waves 16 with ILP 8 is omitted: its accumulators
// (8 x 16 per lane) plus fragments exceed the 128 registers a lane may hold at
// four waves per SIMD.
//
// The bench also times the launch floor: back-to-back launches of a kernel
// whose workgroups each store one word, over grids of 64 to 4096 workgroups of
// 256 and 512 workitems, on one stream with HIP events. That per-launch time is
// what a kernel boundary costs a sequence of launches before any work (queue
// processing, workgroup dispatch, completion signal); launchSeconds is its value
// at 256 workgroups of 256 workitems, launchSecondsPerWorkgroup the slope of a
// least-squares line through the 256-workitem grids. A launch that carries
// work pays less than the floor on top of it: the next launch's queue
// processing overlaps the running kernel. So the bench also times a kernel
// whose 256 workgroups each wait a fixed real time (5, 10, 20 and 40 us on the
// 100 MHz counter), back to back and one launch at a time (each launch between
// events, the stream drained before the next): launchOverheadSeconds and
// launchIsolatedSeconds are the median of (per-launch time - wait) over the
// waits, the time a kernel boundary adds to a launch's own work in each case.
#include "cal_common.hpp"
#include "gemm_mfma.hpp"

using namespace ridgecal;

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kIters = 1000;
constexpr double kSaturation = 0.95;

template <int Waves, int Ilp>
__global__ __launch_bounds__(Waves * 64) void readMfmaKernel(int iters, float* sink, Stamp* out) {
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    _Float16* h = reinterpret_cast<_Float16*>(lds);
    for (int i = threadIdx.x; i < 8192; i += blockDim.x) h[i] = (_Float16)(1.0f + 0.0001f * float(i & 63));
    const int lane = threadIdx.x % 64;
    int addr[Ilp];
#pragma unroll
    for (int j = 0; j < Ilp; ++j) {
        const int row = (j % 4) * 32 + lane % 32;
        addr[j] = ridge::swizzleA<8>(row * 8 + 2 * (j / 4) + lane / 32) * 16;
    }
    half8_t b;
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = (_Float16)(1.0f - 0.001f * float((lane + i) & 7));
    float16_t acc[Ilp];
#pragma unroll
    for (int j = 0; j < Ilp; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
    __syncthreads();
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < Ilp; ++j) {
            const half8_t a = *(const __attribute__((address_space(3))) half8_t*)(lds + addr[j]);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
        }
        asm volatile("" ::: "memory");
    }
    __syncthreads();
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < Ilp; ++j) s += acc[j][0] + acc[j][15];
    if (s == -1.0e38f) sink[0] = s;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

__global__ __launch_bounds__(512) void launchProbeKernel(float* sink) {
    if (threadIdx.x == 0) sink[blockIdx.x] = float(blockIdx.x);
}

// Each workgroup waits `ticks` of the 100 MHz real-time counter from its own
// start (the loop ends for every wave: the counter only advances).
__global__ __launch_bounds__(256) void spinKernel(uint64_t ticks, float* sink) {
    const uint64_t t0 = realtime();
    while (realtime() - t0 < ticks) {
    }
    if (threadIdx.x == 0) sink[blockIdx.x] = 1.0f;
}

// Per-launch seconds of the spin kernel (256 workgroups): back to back over
// `launches` launches, or one launch between two events with the stream
// drained before each (isolated). Middle of kRepeats windows.
double spinSeconds(double waitSeconds, bool isolated, float* dSink, int launches) {
    const uint64_t ticks = uint64_t(waitSeconds * kRealtimeHz + 0.5);
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    std::vector<double> w;
    for (int r = 0; r < kRepeats; ++r) {
        CAL_HIP_CHECK(hipDeviceSynchronize());
        if (isolated) {
            std::vector<double> one;
            for (int i = 0; i < launches; ++i) {
                CAL_HIP_CHECK(hipDeviceSynchronize());
                CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
                hipLaunchKernelGGL(spinKernel, dim3(256), dim3(256), 0, nullptr, ticks, dSink);
                CAL_HIP_CHECK(hipGetLastError());
                CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
                CAL_HIP_CHECK(hipEventSynchronize(e1));
                float ms = 0.0f;
                CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
                one.push_back(ms * 1e-3);
            }
            w.push_back(middle(one));
        } else {
            CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
            for (int i = 0; i < launches; ++i)
                hipLaunchKernelGGL(spinKernel, dim3(256), dim3(256), 0, nullptr, ticks, dSink);
            CAL_HIP_CHECK(hipGetLastError());
            CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
            CAL_HIP_CHECK(hipEventSynchronize(e1));
            float ms = 0.0f;
            CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
            w.push_back(ms * 1e-3 / launches);
        }
    }
    CAL_HIP_CHECK(hipEventDestroy(e0));
    CAL_HIP_CHECK(hipEventDestroy(e1));
    return middle(w);
}

// Per-launch seconds of `launches` back-to-back launches of launchProbeKernel
// (grid x threads), middle of kRepeats windows.
double launchSeconds(int grid, int threads, float* dSink, int launches) {
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    std::vector<double> w;
    for (int r = 0; r < kRepeats; ++r) {
        CAL_HIP_CHECK(hipDeviceSynchronize());
        CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
        for (int i = 0; i < launches; ++i)
            hipLaunchKernelGGL(launchProbeKernel, dim3(grid), dim3(threads), 0, nullptr, dSink);
        CAL_HIP_CHECK(hipGetLastError());
        CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
        CAL_HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        w.push_back(ms * 1e-3 / launches);
    }
    CAL_HIP_CHECK(hipEventDestroy(e0));
    CAL_HIP_CHECK(hipEventDestroy(e1));
    return middle(w);
}

template <int Waves, int Ilp>
double mfmaPerCycle(int cus, float* dSink, Stamp* dStamps) {
    auto k = readMfmaKernel<Waves, Ilp>;
    CAL_HIP_CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kOneWorkgroupLds));
    hipLaunchKernelGGL(k, dim3(cus), dim3(Waves * 64), kOneWorkgroupLds, nullptr, kIters, dSink, dStamps);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(cus);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, cus * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0, hz = 0.0;
    medianStamps(st, cyc, hz);
    return double(Waves) * kIters * Ilp / cyc;
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

    constexpr int kWaves[] = {1, 2, 4, 8, 16};
    constexpr int kIlps[] = {1, 2, 4, 8};
    double surface[4][5] = {};
    std::vector<double> reps[4][5];
#define CAL_CELL(IC, WI, W, ILP)                                                         \
    do {                                                                                 \
        for (int r = 0; r < kRepeats; ++r) reps[IC][WI].push_back(mfmaPerCycle<W, ILP>(cus, dSink, dStamps)); \
        surface[IC][WI] = middle(reps[IC][WI]);                                          \
    } while (0)
#define CAL_COLUMN(IC, ILP) \
    CAL_CELL(IC, 0, 1, ILP); CAL_CELL(IC, 1, 2, ILP); CAL_CELL(IC, 2, 4, ILP); CAL_CELL(IC, 3, 8, ILP)
    CAL_COLUMN(0, 1);
    CAL_CELL(0, 4, 16, 1);
    CAL_COLUMN(1, 2);
    CAL_CELL(1, 4, 16, 2);
    CAL_COLUMN(2, 4);
    CAL_CELL(2, 4, 16, 4);
    CAL_COLUMN(3, 8);
#undef CAL_COLUMN
#undef CAL_CELL

    double best[4] = {};
    for (int c = 0; c < 4; ++c)
        for (int w = 0; w < 5; ++w) best[c] = std::max(best[c], surface[c][w]);
    std::printf("\nds_read_b128 -> v_mfma_f32_32x32x16_f16 chains: MFMA per cycle per CU (%% of column best)\n");
    std::printf("  %5s %20s %20s %20s %20s\n", "waves", "ILP=1", "ILP=2", "ILP=4", "ILP=8");
    for (int w = 0; w < 5; ++w) {
        std::printf("  %5d", kWaves[w]);
        for (int c = 0; c < 4; ++c) {
            if (surface[c][w] > 0)
                std::printf("   %9.4f (%5.1f%%)", surface[c][w], 100.0 * surface[c][w] / best[c]);
            else
                std::printf("   %18s", "-");
        }
        std::printf("\n");
    }
    for (int c = 0; c < 4; ++c)
        for (int w = 0; w < 5; ++w)
            if (surface[c][w] > 0)
                std::printf("CAL_SURFACE ilp %d waves %d mfmaPerCycle %.6f\n", kIlps[c], kWaves[w], surface[c][w]);
    int needed[4];
    for (int c = 0; c < 4; ++c) {
        needed[c] = kWaves[4];
        for (int w = 0; w < 5; ++w)
            if (surface[c][w] >= kSaturation * best[c]) {
                needed[c] = kWaves[w];
                break;
            }
        std::printf("  ILP=%d saturates at %2d waves/CU\n", kIlps[c], needed[c]);
        std::printf("CAL_SATURATION ilp %d waves %d\n", kIlps[c], needed[c]);
    }
    int wBest = 0;
    for (int w = 0; w < 5; ++w)
        if (surface[1][w] == best[1]) wBest = w;
    std::printf("\n");
    reportConstant("warpsNeededToHide", double(needed[1]), "waves/CU", reps[1][wBest]);
    std::printf("  the reported constant is the ILP=2 column, a threshold on a smooth curve\n");
    std::printf("\nCAL_RESULT warpsNeededToHide %d\n", needed[1]);

    // The launch floor.
    constexpr int kGrids[] = {64, 128, 256, 512, 1024, 2048, 4096};
    constexpr int kLaunches = 2000;
    float* dLaunchSink = nullptr;
    CAL_HIP_CHECK(hipMalloc(&dLaunchSink, 4096 * sizeof(float)));
    launchSeconds(256, 256, dLaunchSink, kLaunches);  // first launches load the code object
    std::printf("\nlaunch floor: back-to-back launches of a kernel that stores one word per workgroup\n");
    std::printf("  %9s %14s %14s\n", "workgroups", "256 items (us)", "512 items (us)");
    double sx = 0.0, sy = 0.0, sxx = 0.0, sxy = 0.0, at256 = 0.0;
    int n = 0;
    for (int g : kGrids) {
        const double t256 = launchSeconds(g, 256, dLaunchSink, kLaunches);
        const double t512 = launchSeconds(g, 512, dLaunchSink, kLaunches);
        std::printf("  %9d %14.3f %14.3f\n", g, t256 * 1e6, t512 * 1e6);
        std::printf("CAL_INFO launchSeconds_wg%d_items256 %.6e\n", g, t256);
        std::printf("CAL_INFO launchSeconds_wg%d_items512 %.6e\n", g, t512);
        if (g == 256) at256 = t256;
        if (g >= 256) {
            sx += g;
            sy += t256;
            sxx += double(g) * g;
            sxy += g * t256;
            ++n;
        }
    }
    const double slope = (n * sxy - sx * sy) / (n * sxx - sx * sx);
    std::printf("CAL_RESULT launchSeconds %.6e\n", at256);
    std::printf("CAL_RESULT launchSecondsPerWorkgroup %.6e\n", slope);

    // What a kernel boundary adds to a launch that carries work.
    constexpr double kWaits[] = {5e-6, 10e-6, 20e-6, 40e-6};
    std::vector<double> overB2b, overIso;
    std::printf("\nkernel boundary on top of work: 256 workgroups that each wait a fixed time\n");
    std::printf("  %9s %18s %18s\n", "wait (us)", "back to back (us)", "isolated (us)");
    for (double wsec : kWaits) {
        const double b2b = spinSeconds(wsec, false, dLaunchSink, 200);
        const double iso = spinSeconds(wsec, true, dLaunchSink, 20);
        std::printf("  %9.1f %18.3f %18.3f\n", wsec * 1e6, b2b * 1e6, iso * 1e6);
        std::printf("CAL_INFO spinSeconds_wait%.0fus_b2b %.6e\n", wsec * 1e6, b2b);
        std::printf("CAL_INFO spinSeconds_wait%.0fus_isolated %.6e\n", wsec * 1e6, iso);
        overB2b.push_back(b2b - wsec);
        overIso.push_back(iso - wsec);
    }
    std::printf("CAL_RESULT launchOverheadSeconds %.6e\n", middle(overB2b));
    std::printf("CAL_RESULT launchIsolatedSeconds %.6e\n", middle(overIso));
    CAL_HIP_CHECK(hipFree(dLaunchSink));
    CAL_HIP_CHECK(hipFree(dSink));
    CAL_HIP_CHECK(hipFree(dStamps));
    return 0;
}
