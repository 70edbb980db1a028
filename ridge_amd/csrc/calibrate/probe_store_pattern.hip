// probe_store_pattern.hip -- the C stream of a persistent GEMM row, alone.
//
// A persistent grid (one workgroup per CU) walks the output tiles of an M x N FP16
// C in the kernels' launch order (XCD remap, then GroupM), and every wave writes
// its WM x WN part of each tile through the kernels' own staged epilogue
// (storeStaged, non-temporal stores), with `mfmas` MFMAs per wave between tiles
// standing in for the K loop (64 are a K = 128 tile of a 64x64 wave tile, 128 of
// a 128x64 one). Nothing is loaded. This is the ceiling of a row
// whose time is writing C (K = 128): what the row's store pattern and launch
// order allow, without the operand stream.
//
// Reported per case: TB/s of C, cold (launches rotate over C buffers that
// together exceed twice the 256 MB MALL) and warm (one buffer), each the middle
// of 5 windows of 40 launches after the warm-up. A diagnostic, not a
// calibration constant: the model reads none of it.
#include "cal_common.hpp"
#include "gemm_mfma.hpp"

using namespace ridgecal;

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

template <int BM, int BN, int WM, int WN, int GROUPM>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void storePatternKernel(_Float16* C, int M, int N,
                                                                                   int mfmas) {
    constexpr int kWavesN = BN / WN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int kWaves = (BM / WM) * kWavesN;
    constexpr int kRegion = 16 * WN * 2;  // one 16-row tile-row of the wave tile per pass
    __shared__ __attribute__((aligned(1024))) char lds[kWaves * kRegion];
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int waveM = wave / kWavesN, waveN = wave % kWavesN;
    RIDGE_LDS_AS char* region = (RIDGE_LDS_AS char*)(lds) + wave * kRegion;
    const int grid = gridDim.x;
    const int self = ridge::xcdRemap(blockIdx.x, grid);
    const int numTiles = (M / BM) * (N / BN);
    float4_t acc[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[tm][tn][e] = float((lane * 131 + tm * 17 + tn * 7 + e) % 61) / 64.0f - 0.45f;
    half8_t a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (_Float16)(float((lane * 29 + e * 13) % 37) / 64.0f - 0.25f);
        b[e] = (_Float16)(float((lane * 23 + e * 11) % 41) / 64.0f - 0.3f);
    }
    for (int t = self; t < numTiles; t += grid) {
        // The K loop's stand-in: `mfmas` MFMAs spread over the accumulators.
        for (int i = 0; i < mfmas; i += TM * TN) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a, acc[tm][tn], 0, 0, 0);
        }
        int row, col;
        ridge::tileOf<BM, BN, GROUPM>(t, M, N, row, col);
        _Float16* cWave = C + (size_t)(row + waveM * WM) * N + col + waveN * WN;
        ridge::storeStaged<TM, TN, WN, 1, true>(acc, region, cWave, N, lane);
    }
}

// The middle of `windows` HIP-event windows of `launches` launches, launch i
// writing buffer i % n, in seconds per launch.
template <int BM, int BN, int WM, int WN, int GROUPM>
double timeLaunches(const std::vector<_Float16*>& bufs, int M, int N, int mfmas, int cus) {
    auto k = storePatternKernel<BM, BN, WM, WN, GROUPM>;
    const int threads = (BM / WM) * (BN / WN) * 64;
    const int grid = std::min(cus, (M / BM) * (N / BN));
    const int n = int(bufs.size());
    int j = 0;
    // One workgroup per CU, as the GEMM's ring and staging make it: the launch
    // asks for more than half of the LDS.
    CAL_HIP_CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kOneWorkgroupLds));
    auto launch = [&]() {
        hipLaunchKernelGGL(k, dim3(grid), dim3(threads), kOneWorkgroupLds, nullptr, bufs[j % n], M, N, mfmas);
        ++j;
    };
    for (int i = 0; i < 20 * n; ++i) launch();
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    constexpr int kLaunches = 40, kWindows = 5;
    std::vector<double> sec;
    for (int w = 0; w < kWindows; ++w) {
        CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
        for (int i = 0; i < kLaunches; ++i) launch();
        CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
        CAL_HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        sec.push_back(ms * 1e-3 / kLaunches);
    }
    CAL_HIP_CHECK(hipEventDestroy(e0));
    CAL_HIP_CHECK(hipEventDestroy(e1));
    return middle(sec);
}

template <int BM, int BN, int WM, int WN, int GROUPM>
void runCase(int M, int N, int mfmas, int cus, const std::vector<_Float16*>& cold, _Float16* warm) {
    const double bytes = 2.0 * M * N;
    const double tc = timeLaunches<BM, BN, WM, WN, GROUPM>(cold, M, N, mfmas, cus);
    const double tw = timeLaunches<BM, BN, WM, WN, GROUPM>({warm}, M, N, mfmas, cus);
    std::printf("  %5d x %5d  %3dx%3d w%3dx%2d g%-2d  %4d MFMAs/wave/tile   cold %6.2f TB/s   warm %6.2f TB/s\n",
                M, N, BM, BN, WM, WN, GROUPM, mfmas, bytes / tc / 1e12, bytes / tw / 1e12);
    std::printf("PROBE storePattern M %d N %d BM %d BN %d WM %d WN %d groupM %d mfmas %d coldBytesPerSec %.6e "
                "warmBytesPerSec %.6e\n",
                M, N, BM, BN, WM, WN, GROUPM, mfmas, bytes / tc, bytes / tw);
}

}  // namespace

int main() {
    const hipDeviceProp_t prop = deviceBanner();
    const int cus = prop.multiProcessorCount;
    warmUp();
    std::printf("\nC written in a persistent row's store pattern (no loads); cold: C rotated over > 2x the MALL\n");
    struct Shape { int M, N; };
    const Shape shapes[] = {{8192, 8192}, {16384, 4096}, {16384, 16384}};
    for (const Shape& s : shapes) {
        const size_t bytes = size_t(s.M) * s.N * 2;
        const int sets = int(std::max<size_t>(2, (2 * 256 * (size_t(1) << 20) + bytes - 1) / bytes + 1));
        std::vector<_Float16*> bufs(sets, nullptr);
        for (auto& p : bufs) CAL_HIP_CHECK(hipMalloc(&p, bytes));
        // The persistent rows' own patterns (256x128 g4, 128x128 g8), then the
        // same 256x128 tile in other launch orders, its transpose 128x256, and
        // 256x256.
        runCase<256, 128, 64, 64, 4>(s.M, s.N, 0, cus, bufs, bufs[0]);
        runCase<256, 128, 64, 64, 4>(s.M, s.N, 64, cus, bufs, bufs[0]);
        runCase<128, 128, 64, 64, 8>(s.M, s.N, 0, cus, bufs, bufs[0]);
        runCase<128, 128, 64, 64, 8>(s.M, s.N, 64, cus, bufs, bufs[0]);
        runCase<256, 128, 64, 64, 1>(s.M, s.N, 64, cus, bufs, bufs[0]);
        runCase<256, 128, 64, 64, 8>(s.M, s.N, 64, cus, bufs, bufs[0]);
        runCase<128, 256, 64, 64, 4>(s.M, s.N, 0, cus, bufs, bufs[0]);
        runCase<128, 256, 64, 64, 4>(s.M, s.N, 64, cus, bufs, bufs[0]);
        runCase<128, 256, 64, 64, 8>(s.M, s.N, 64, cus, bufs, bufs[0]);
        runCase<256, 256, 128, 64, 4>(s.M, s.N, 0, cus, bufs, bufs[0]);
        runCase<256, 256, 128, 64, 4>(s.M, s.N, 128, cus, bufs, bufs[0]);
        for (auto p : bufs) CAL_HIP_CHECK(hipFree(p));
    }
    return 0;
}
