// probe_mfma_shape.hip -- the sustained rate of the two FP16 MFMA shapes on random
// and on constant operands, at the headline kernel's data movement per step.
//
// 256 workgroups of 8 wavefronts (one workgroup per CU: 80 KiB of LDS each), as
// in the ping-pong row. Per step every wavefront reads its 128 x 64 wave tile's
// fragments for a K slice of 32 from LDS (8 A and 4 B fragments of 16 bytes per
// lane, 12 KiB per wavefront, the slots moving every step so the operand bits
// change) and then issues either
//   16x16x32  32 x v_mfma_f32_16x16x32_f16 (the table's instruction, snake order)
//   32x32x16  16 x v_mfma_f32_32x32x16_f16 (two K halves of 16)
// on them: the same bytes and the same FLOPs per step. The 32x32x16 shape reads half
// the operand bytes per multiply-add. LDS holds FP16 drawn from U[-1,1) (the
// benchmark's operand distribution) or the constant 1/64. Reported: TFLOP/s, three
// alternating pairs of 10-launch windows after the warm-up. A diagnostic; the model
// reads none of it.
#include "cal_common.hpp"

using namespace ridgecal;

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kSlots = 5120;  // 16-byte LDS slots: 80 KiB, so one workgroup per CU
constexpr int kThreads = 512;
constexpr int kGrid = 256;
constexpr double kFlopPerStep = 2.0 * 128 * 64 * 32 * 8;  // per workgroup

template <bool BIG>
__global__ __launch_bounds__(kThreads) void mfmaShape(const half8_t* __restrict__ src, float* __restrict__ out,
                                                      int steps) {
    __shared__ half8_t lds[kSlots];
    for (int i = threadIdx.x; i < kSlots; i += kThreads) lds[i] = src[i];
    __syncthreads();
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    float4_t acc16[8][4];
    float16_t acc32[4][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc16[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc32[i][j][e] = 0.0f;
    int base = wave * 640;
    for (int it = 0; it < steps; ++it) {
        half8_t a[8], b[4];
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = lds[(base + j * 64 + lane) % kSlots];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = lds[(base + 512 + j * 64 + lane) % kSlots];
        base = (base + 768) % kSlots;
        if constexpr (!BIG) {
#pragma unroll
            for (int tn = 0; tn < 4; ++tn)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int tm = (tn & 1) ? 7 - i : i;
                    acc16[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[tn], a[tm], acc16[tm][tn], 0, 0, 0);
                }
        } else {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int tn = 0; tn < 2; ++tn)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tm = (tn & 1) ? 3 - i : i;
                        acc32[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[kh * 2 + tn], a[kh * 4 + tm],
                                                                               acc32[tm][tn], 0, 0, 0);
                    }
        }
    }
    float s = 0.0f;
    if constexpr (!BIG) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) s += acc16[i][j][0] + acc16[i][j][1] + acc16[i][j][2] + acc16[i][j][3];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) s += acc32[i][j][e];
    }
    out[blockIdx.x * kThreads + threadIdx.x] = s;
}

}  // namespace

int main() {
    deviceBanner();
    constexpr int kSteps = 20000, kLaunches = 10;
    std::vector<_Float16> random(kSlots * 8), constant(kSlots * 8, (_Float16)(1.0f / 64.0f));
    uint64_t x = 0x9e3779b97f4a7c15ull;
    for (auto& v : random) {
        x = x * 6364136223846793005ull + 1442695040888963407ull;
        v = (_Float16)((double)(x >> 11) / 9007199254740992.0 * 2.0 - 1.0);
    }
    half8_t* src = nullptr;
    float* out = nullptr;
    CAL_HIP_CHECK(hipMalloc(&src, kSlots * 16));
    CAL_HIP_CHECK(hipMalloc(&out, kGrid * kThreads * 4));
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    warmUp();
    const double flop = kFlopPerStep * kGrid * kSteps;
    for (int data = 0; data < 2; ++data) {
        CAL_HIP_CHECK(hipMemcpy(src, data ? constant.data() : random.data(), kSlots * 16, hipMemcpyHostToDevice));
        std::printf("\n%s operands\n", data ? "constant 1/64" : "U[-1,1) FP16");
        std::vector<double> tf[2];
        for (int rep = 0; rep < 3; ++rep) {
            for (int big = 0; big < 2; ++big) {
                CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
                for (int l = 0; l < kLaunches; ++l) {
                    if (big)
                        hipLaunchKernelGGL(mfmaShape<true>, dim3(kGrid), dim3(kThreads), 0, nullptr, src, out, kSteps);
                    else
                        hipLaunchKernelGGL(mfmaShape<false>, dim3(kGrid), dim3(kThreads), 0, nullptr, src, out, kSteps);
                }
                CAL_HIP_CHECK(hipGetLastError());
                CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
                CAL_HIP_CHECK(hipEventSynchronize(e1));
                float ms = 0.0f;
                CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
                tf[big].push_back(flop / (ms * 1e-3 / kLaunches) / 1e12);
                std::printf("  %-9s %8.1f TFLOP/s\n", big ? "32x32x16" : "16x16x32", tf[big].back());
            }
        }
        std::printf("PROBE mfmaShape %s small %.1f big %.1f\n", data ? "constant" : "random", middle(tf[0]),
                    middle(tf[1]));
    }
    CAL_HIP_CHECK(hipEventDestroy(e0));
    CAL_HIP_CHECK(hipEventDestroy(e1));
    CAL_HIP_CHECK(hipFree(src));
    CAL_HIP_CHECK(hipFree(out));
    return 0;
}
