// cal_smem_bw.hip -- smemBytesPerCycle: sustained LDS operand-read bandwidth per
// CU on the path the GEMM kernel uses.
//
// Counterpart of the reference's bench/calibrate/cal-smem-bw.cu:47-288. As there,
// the measurement uses the kernel's own instructions on the kernel's own layout,
// because bank behaviour belongs to the (instruction, layout) pair:
//   A  ds_read_b128 of MFMA A fragments from the XOR-swizzled A tile (swizzleA)
//   B  ds_read_b64_tr_b16 of B fragments from the swizzled B tile (swizzleB)
//   mix  the GEMM's own ratio for a 128x64 wavefront tile: per k-step, four A
//        reads and four transposing B reads -- reported as smemBytesPerCycle
//   control  linear, conflict-free ds_read_b128 (lane l reads 16 l): the
//        ceiling the others are checked against
// Loads are kept in the loop by a compiler memory barrier per iteration and their
// results are folded into a value that is stored only under an impossible
// condition.
#include "cal_common.hpp"
#include "gemm_mfma.hpp"

using namespace ridgecal;

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kIters = 2000;
constexpr int kAOffset = 0;            // A tile: 128 x 64 halves = 16 KiB
constexpr int kBOffset = 16 * 1024;    // B tile: 64 x 256 halves = 32 KiB
constexpr int kCprB = 32;              // chunks per B row (BN = 256)

enum Pattern { kPatA = 0, kPatB = 1, kPatMix = 2, kPatLinear = 3 };

__device__ __forceinline__ int addrA(int lane, int j) {
    const int tm = j % 4, ks = j / 4;  // 4 row tiles x 4 k-steps of a BK = 64 tile
    const int row = tm * 32 + lane % 32;
    return kAOffset + ridge::swizzleA(row * 8 + 2 * (ks % 4) + lane / 32) * 16;
}

__device__ __forceinline__ int addrB(int lane, int j) {
    const int tn = j % 8, half = j / 8;  // 8 column tiles of 32, two 4-row halves
    const int g = lane / 16, s = lane % 16;
    const int row = 8 * (g / 2) + 4 * (half % 2) + s / 4;
    const int col = tn * 32 + 16 * (g % 2) + 4 * (s % 4);
    return kBOffset + ridge::swizzleB<kCprB>(row * kCprB + col / 8) * 16 + (col % 8) * 2;
}

template <int Waves, int Pat>
__global__ __launch_bounds__(Waves * 64) void ldsReadKernel(int iters, uint32_t* sink, Stamp* out) {
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    for (int i = threadIdx.x; i < 48 * 1024 / 4; i += blockDim.x) reinterpret_cast<uint32_t*>(lds)[i] = i * 2654435761u;
    const int lane = threadIdx.x % 64;
    int addr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (Pat == kPatA) addr[j] = addrA(lane, j);
        else if (Pat == kPatB) addr[j] = addrB(lane, j);
        else if (Pat == kPatMix) addr[j] = (j < 4) ? addrA(lane, j) : addrB(lane, j);
        else addr[j] = lane * 16 + j * 1024;
    }
    uint32_t acc = 0;
    __syncthreads();
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool tr = (Pat == kPatB) || (Pat == kPatMix && j >= 4);
            if (tr) {
                const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) short4_t*)(lds + addr[j]));
                acc ^= uint32_t(v[0]) ^ (uint32_t(v[3]) << 16);
            } else {
                const u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(lds + addr[j]);
                acc ^= v[0] ^ v[3];
            }
        }
        asm volatile("" ::: "memory");
    }
    __syncthreads();
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    if (acc == 0x9e3779b9u) sink[0] = acc;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

constexpr double bytesPerIteration(int pat) {
    // Per wave: 8 instructions of 1024 B (ds_read_b128) or 512 B (tr_b64).
    return pat == kPatB ? 8 * 512.0 : pat == kPatMix ? 4 * 1024.0 + 4 * 512.0 : 8 * 1024.0;
}

template <int Waves, int Pat>
double measure(int cus, uint32_t* dSink, Stamp* dStamps) {
    auto k = ldsReadKernel<Waves, Pat>;
    CAL_HIP_CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kOneWorkgroupLds));
    hipLaunchKernelGGL(k, dim3(cus), dim3(Waves * 64), kOneWorkgroupLds, nullptr, kIters, dSink, dStamps);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(cus);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, cus * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0, hz = 0.0;
    medianStamps(st, cyc, hz);
    return double(Waves) * kIters * bytesPerIteration(Pat) / cyc;
}

struct Curve {
    double best = 0.0;
    int bestWaves = 0;
    std::vector<double> bestReps;
};

template <int Pat>
Curve sweep(const char* label, int cus, uint32_t* dSink, Stamp* dStamps) {
    Curve c;
    std::printf("\n%s\n  %6s %18s\n", label, "waves", "bytes/cycle/CU");
    auto cell = [&](int w, double v, const std::vector<double>& reps) {
        std::printf("  %6d %18.2f\n", w, v);
        std::printf("CAL_CURVE pattern %d waves %d bytesPerCycle %.4f\n", Pat, w, v);
        if (v > c.best * 1.001) {
            c.best = v;
            c.bestWaves = w;
            c.bestReps = reps;
        }
    };
#define CAL_CELL(W)                                                              \
    do {                                                                         \
        std::vector<double> reps;                                                \
        for (int r = 0; r < kRepeats; ++r) reps.push_back(measure<W, Pat>(cus, dSink, dStamps)); \
        cell(W, median(reps), reps);                                             \
    } while (0)
    CAL_CELL(1);
    CAL_CELL(2);
    CAL_CELL(4);
    CAL_CELL(8);
    CAL_CELL(16);
#undef CAL_CELL
    return c;
}

}  // namespace

int main() {
    const hipDeviceProp_t prop = deviceBanner();
    const int cus = prop.multiProcessorCount;
    uint32_t* dSink = nullptr;
    Stamp* dStamps = nullptr;
    CAL_HIP_CHECK(hipMalloc(&dSink, sizeof(uint32_t)));
    CAL_HIP_CHECK(hipMalloc(&dStamps, cus * sizeof(Stamp)));
    warmUp();
    const Curve ctl = sweep<kPatLinear>("control: linear ds_read_b128 (conflict-free)", cus, dSink, dStamps);
    const Curve a = sweep<kPatA>("A fragments: ds_read_b128 on the swizzled A tile", cus, dSink, dStamps);
    const Curve b = sweep<kPatB>("B fragments: ds_read_b64_tr_b16 on the swizzled B tile", cus, dSink, dStamps);
    const Curve mix = sweep<kPatMix>("GEMM mix: 4 A + 4 transposing B reads per k-step", cus, dSink, dStamps);

    std::printf("\n");
    bool ok = reportConstant("ldsControlBytesPerCycle", ctl.best, "B/cycle/CU", ctl.bestReps);
    ok &= reportConstant("ldsAReadBytesPerCycle", a.best, "B/cycle/CU", a.bestReps);
    ok &= reportConstant("ldsBTrReadBytesPerCycle", b.best, "B/cycle/CU", b.bestReps);
    ok &= reportConstant("smemBytesPerCycle", mix.best, "B/cycle/CU", mix.bestReps);
    // Physics check: no pattern may beat the conflict-free control by more than
    // measurement noise (reference cal-smem-bw.cu:265-281 checks its control).
    const double ceiling = ctl.best * 1.05;
    if (a.best > ceiling || b.best > ceiling || mix.best > ceiling) {
        std::printf("  a pattern exceeds the conflict-free control: the benchmark is wrong\n");
        ok = false;
    }
    std::printf("\nCAL_RESULT smemBytesPerCycle %.6f\n", mix.best);
    std::printf("CAL_RESULT smemSaturationWaves %d\n", mix.bestWaves);
    std::printf("CAL_RESULT ldsControlBytesPerCycle %.6f\n", ctl.best);
    std::printf("CAL_RESULT ldsAReadBytesPerCycle %.6f\n", a.best);
    std::printf("CAL_RESULT ldsBTrReadBytesPerCycle %.6f\n", b.best);
    CAL_HIP_CHECK(hipFree(dSink));
    CAL_HIP_CHECK(hipFree(dStamps));
    return ok ? 0 : 1;
}
