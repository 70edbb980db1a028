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
// condition. The ping-pong and persistent skeletons further down time the two
// schedules' K-steps for the model's overlap, power, MALL and persistent terms.
#include "cal_common.hpp"
#include "gemm_mfma.hpp"

#include <string>

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
    return kAOffset + ridge::swizzleA<8>(row * 8 + 2 * (ks % 4) + lane / 32) * 16;
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

// The ping-pong schedule's skeleton: eight waves, waves w and w + 4 on SIMD w % 4,
// group g = w / 4. A K-step has two phases separated by workgroup barriers; in
// each, one group issues the 32 MFMAs of a 128x64 wavefront tile at BK = 32 (8 A
// x 4 B fragments) while the other group reads the next step's fragments from the
// swizzled tiles (8 ds_read_b128 + 8 ds_read_b64_tr_b16: 12 KiB per wave) and
// waits for them. Modes:
//   0  that schedule
//   1  the reads alone (all eight waves, no barriers): checks the per-operand
//      LDS rates against tS = A bytes / ldsAReadBytesPerCycle + B bytes /
//      ldsBTrReadBytesPerCycle
//   2  the MFMAs alone: tC
//   3  mode 0 plus the GEMM's direct-to-LDS refill, 4 KiB per memory-phase wave
//      (32 KiB per step) from a 1 MiB L2-resident buffer into a separate region
//   4  every wave reads its fragments and then issues its MFMAs, with no barriers:
//      the uniform schedule of an 8-wave workgroup, whose two waves per SIMD
//      overlap their phases only as the hardware interleaves them
//   5  mode 3 with one of each wave's four refill loads (a quarter of the bytes)
//      from a window of its own per CU, 512 KiB each: 16 MiB per XCD misses the
//      4 MiB L2 and 128 MiB in all stays in the 256 MiB MALL
//   6  mode 3 with all four refill loads from those windows
//   7  mode 3 with two of the four from those windows
//   8  mode 3 with three of the four from those windows
// A perfect overlap makes mode 0 and mode 3 run at max(tC, tS) cycles; the
// measured clock of each mode shows what the extra data movement costs in power.
// Modes 3, 5, 7, 8 and 6 (a share m = 0, 1/4, 1/2, 3/4, 1 of the refill missing
// the L2) give the K-step's stretch against the load m puts on the MALL path: a
// wave waits for the refill it issued one K-step earlier, the latency budget of
// the three-stage ping-pong GEMM, whose launch order sets its own share m.
// Operands are U[-1,1) halves.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kRefillLoads = 4;              // 1 KiB direct-to-LDS loads per wave per phase
constexpr int kRefillSourceBytes = 1 << 20;  // L2-resident source
constexpr int kRefillRegion = 48 * 1024;     // refills land in [48 KiB, 64 KiB)
constexpr int kMallWindowKiB = 512;          // per-CU window of the L2-missing refill

template <int Mode>
__global__ __launch_bounds__(512) void pingPongKernel(const uint32_t* operands, const char* refill,
                                                      const char* mall, int iters, float* sink, Stamp* out) {
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    // 48 KiB of tiles from the 16 KiB operand block, repeated.
    for (int i = threadIdx.x; i < 48 * 1024 / 4; i += blockDim.x)
        reinterpret_cast<uint32_t*>(lds)[i] = operands[i % (16 * 1024 / 4)];
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int group = wave / 4;
    const uint32_t ldsBase = ridge::ldsAddress(lds);
    int aAddr[8], bAddr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        aAddr[j] = addrA(lane, j);
        bAddr[j] = addrB(lane, j);
    }
    half8_t a[8], b[4];
    auto readFrags = [&]() {
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = *(const __attribute__((address_space(3))) half8_t*)(lds + aAddr[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4_t*)(lds + bAddr[2 * j]));
            const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4_t*)(lds + bAddr[2 * j + 1]));
            b[j] = __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    // Load i of wave w at step it reads 1 KiB at ((it * 8 + w) * 4 + i) mod 1024
    // KiB of the source and writes LDS [48 KiB + ((w % 4) * 4 + i) KiB, +1 KiB).
    // In modes 5 and 6 the first one (or all four) of those loads instead read
    // 1 KiB at ((it * 8 + w) * 4 + i) mod 512 KiB of this CU's own window of
    // `mall` (the window of workgroup g starts at g * 512 KiB).
    const uint32_t window = blockIdx.x * (kMallWindowKiB << 10);
    auto refillLoads = [&](int it) {
#pragma unroll
        for (int i = 0; i < kRefillLoads; ++i) {
            const uint32_t k = (uint32_t)((it * 8 + wave) * kRefillLoads + i);
            const uint32_t dst = ldsBase + kRefillRegion + ((wave % 4) * kRefillLoads + i) * 1024;
            if (i < (Mode == 5 ? 1 : Mode == 7 ? 2 : Mode == 8 ? 3 : Mode == 6 ? 4 : 0))
                ridge::globalLoadLds16(mall, window + ((k % kMallWindowKiB) << 10) + lane * 16, dst);
            else
                ridge::globalLoadLds16(refill, ((k & 1023) << 10) + lane * 16, dst);
        }
    };
    float4_t acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][e] = 0.0f;
    __syncthreads();
    readFrags();
    constexpr bool kRefill = Mode == 3 || Mode >= 5;
    constexpr bool kPingPong = Mode == 0 || kRefill;
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    if (kPingPong && group == 1) __builtin_amdgcn_s_barrier();
    for (int it = 0; it < iters; ++it) {
        if (Mode != 2) {  // modes 0, 1, 3, 4 read
            if (kRefill) refillLoads(it);
            readFrags();
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (kRefill) ridge::waitVmcnt<kRefillLoads>();  // the previous phase's refill has landed
            if (Mode == 1) {
                // Consume every fragment register, at no instruction cost.
#pragma unroll
                for (int j = 0; j < 8; ++j) asm volatile("" ::"v"(a[j]));
#pragma unroll
                for (int j = 0; j < 4; ++j) asm volatile("" ::"v"(b[j]));
            }
        }
        if (kPingPong) __builtin_amdgcn_s_barrier();
        if (Mode != 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc[i * 4 + j]) : "v"(a[i]), "v"(b[j]));
        }
        if (kPingPong) __builtin_amdgcn_s_barrier();
    }
    if (kRefill) ridge::waitVmcnt<0>();
    if (kPingPong && group == 0) __builtin_amdgcn_s_barrier();  // both groups pass 2 * iters + 1 barriers
    __syncthreads();
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s += acc[i][0] + acc[i][3];
    if (s == -1.0e38f) sink[0] = s;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

// Median cycles per K-step of the skeleton in `Mode` over every CU, and the
// median loaded clock.
template <int Mode>
double pingPongCycles(int cus, const uint32_t* dOperands, const char* dRefill, const char* dMall, float* dSink,
                      Stamp* dStamps, double& clockHz) {
    auto k = pingPongKernel<Mode>;
    CAL_HIP_CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kOneWorkgroupLds));
    hipLaunchKernelGGL(k, dim3(cus), dim3(512), kOneWorkgroupLds, nullptr, dOperands, dRefill, dMall, kIters, dSink,
                       dStamps);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(cus);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, cus * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0;
    medianStamps(st, cyc, clockHz);
    return cyc / kIters;
}

// The persistent schedule's main loop for one table row (gemmMfmaPersistentKernel
// without its tile walk and epilogue): compute waves 0 .. kWaves-1 run the
// kernel's k-steps (fragments double-buffered, MFMAs interleaved with the next
// k-step's reads, one barrier per K tile); the two loader waves refill the ring
// with the kernel's direct-to-LDS loads and swizzled lane offsets, from a
// four-tile L2-resident source. G K tiles per launch. Modes: 0 both halves of a
// k-step, 1 the fragment reads alone, 2 the MFMAs alone (on fragments read once),
// 3 mode 0 with the kernel's epilogue after every tileK K tiles: the compute
// waves stage their tile through their LDS region, store it non-temporally
// (storeStaged, as the kernel does) and clear their accumulators. Workgroup b's
// epilogues rotate over kEpiSlots output tiles of C, rows
// [(b kEpiSlots + slot) BM, +BM), columns [0, BN): C holds
// gridDim.x x kEpiSlots x BM rows of BN halves. Every wave passes G barriers,
// as in the kernel.
constexpr int kEpiSlots = 16;

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int Mode>
__global__ __launch_bounds__(((BM / WM) * (BN / WN) + ridge::kPersistentLoaders) * 64) void persistentSkeletonKernel(
    const _Float16* src, int G, float* sink, Stamp* out, _Float16* C, int tileK) {
    using T = ridge::GemmTraits<BM, BN, BK, WM, WN, STAGES, 8>;
    using P = ridge::PersistentTraits<BM, BN, BK, WM, WN, STAGES, 8>;
    using Blk = ridge::GemmBlock<BM, BN, BK, WM, WN, STAGES, 8>;
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = P::kLoads;
    constexpr int kTileBytes = T::kBytesA + T::kBytesB;
    __shared__ __attribute__((aligned(1024))) char lds[P::kLdsBytes];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64;
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    if (wave >= T::kWaves) {
        // The source holds four K tiles, each an A tile (BM rows of BK halves)
        // followed by a B tile (BK rows of BN halves), rows contiguous.
        const int l = wave - T::kWaves;
        const uint32_t ldsBase = ridge::ldsAddress(lds);
        uint32_t offA[P::kLoadsA], offB[P::kLoadsB];
#pragma unroll
        for (int i = 0; i < P::kLoadsA; ++i) {
            const int q = ridge::swizzleA<T::kChunksPerRowA>((i * P::kLoaders + l) * 64 + lane);
            offA[i] = (uint32_t)(((q / T::kChunksPerRowA) * BK + (q % T::kChunksPerRowA) * 8) * 2);
        }
#pragma unroll
        for (int i = 0; i < P::kLoadsB; ++i) {
            const int q = ridge::swizzleB<T::kChunksPerRowB>((i * P::kLoaders + l) * 64 + lane);
            offB[i] = (uint32_t)(T::kBytesA + ((q / T::kChunksPerRowB) * BN + (q % T::kChunksPerRowB) * 8) * 2);
        }
        auto issue = [&](int g, int stage) {
            uint32_t lb = ldsBase;
            asm volatile("" : "+s"(lb));
            const char* base = reinterpret_cast<const char*>(src) + (g & 3) * kTileBytes;
#pragma unroll
            for (int i = 0; i < P::kLoadsA; ++i)
                ridge::globalLoadLds16(base, offA[i], lb + stage * T::kBytesA + (i * P::kLoaders + l) * 1024);
#pragma unroll
            for (int i = 0; i < P::kLoadsB; ++i)
                ridge::globalLoadLds16(base, offB[i],
                                       lb + T::kRegionA + stage * T::kBytesB + (i * P::kLoaders + l) * 1024);
        };
        ridge::staticFor<STAGES - 1>([&](auto sC) {
            if (sC.value < G) issue(sC.value, sC.value);
        });
        if (G >= STAGES - 1) {
            ridge::waitVmcnt<(STAGES - 2) * L>();
        } else {
            ridge::waitVmcnt<0>();
        }
        ridge::barrierLds();  // B_0
        for (int g0 = 0; g0 < G; g0 += STAGES) {
            ridge::staticFor<STAGES>([&](auto sC) {
                constexpr int s = sC.value;
                const int g = g0 + s;
                if (g + 1 < G) {
                    if (g + STAGES - 1 < G) {
                        issue(g + STAGES - 1, (s + STAGES - 1) % STAGES);
                        ridge::waitVmcnt<(STAGES - 2) * L>();
                    } else {
                        ridge::waitVmcnt<0>();
                    }
                    ridge::barrierLds();  // B_{g+1}
                }
            });
        }
        return;
    }
    // One column of tiles, one per workgroup: the block only forms its LDS
    // fragment offsets here and reads no global memory; mode 3 writes C.
    const int rowsC = BM * (int)gridDim.x * (Mode == 3 ? kEpiSlots : 1);
    Blk blk(lds, src, src, rowsC, BN, BK * G);
    RIDGE_LDS_AS char* region = (RIDGE_LDS_AS char*)(lds) + T::kLdsBytes + wave * P::kRegionBytes;
    (void)region;
    // The kernel's own tile cursor: a K-tile count compared with K / BK, and the
    // tile index, so the loop carries the same per-K-tile work as the kernel's.
    int kt = 0, tile = 0;
    (void)kt;
    (void)tile;
    ridge::barrierLds();  // B_0
    half8_t fa[2][TM];
    half8_t fb[2][TN];
    blk.template readFrags<0>(0, fa[0], fb[0]);
    blk.template readFrags<0>(0, fa[1], fb[1]);
    constexpr int U = (STAGES * KS) % 2 == 0 ? STAGES : 2 * STAGES;
    for (int g0 = 0; g0 < G; g0 += U) {
        ridge::staticFor<U>([&](auto iC) {
            constexpr int i = iC.value;
            constexpr int s = i % STAGES;
            constexpr int sNext = (s + 1) % STAGES;
            const int g = g0 + i;
            if (g < G) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int cur = (i * KS + ks) & 1;
                    if (ks + 1 < KS) {
                        if (Mode != 2) blk.template readFrags<s>(ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
                    } else if (g + 1 < G) {
                        ridge::barrierLds();  // B_{g+1}
                        if (Mode != 2) blk.template readFrags<sNext>(0, fa[cur ^ 1], fb[cur ^ 1]);
                    }
                    if (Mode != 1) {
                        blk.mfmaStep(fa[cur], fb[cur]);
                        ridge::interleaveHint<TM, TN>();
                    } else {
                        // Consume the fragments at no instruction cost.
#pragma unroll
                        for (int tm = 0; tm < TM; ++tm) asm volatile("" ::"v"(fa[cur][tm]));
#pragma unroll
                        for (int tn = 0; tn < TN; ++tn) asm volatile("" ::"v"(fb[cur][tn]));
                    }
                }
                if constexpr (Mode == 3) {
                    if (++kt == tileK) {
                        blk.setTile((int)blockIdx.x * kEpiSlots + (tile % kEpiSlots), rowsC, BN, BK * G);
                        ridge::storeStaged<TM, TN, WN, P::kEpiTiles, true>(blk.acc, region, blk.waveC(C, BN), BN,
                                                                           lane);
#pragma unroll
                        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                                for (int e = 0; e < 4; ++e) blk.acc[tm][tn][e] = 0.0f;
                        kt = 0;
                        ++tile;
                    }
                }
            }
        });
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    float acc = 0.0f;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc += blk.acc[tm][tn][0] + blk.acc[tm][tn][3];
    if (acc == -1.0e38f) sink[0] = acc;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

// The ping-pong schedule's main loop for one 8-wave table row
// (gemmMfmaPingPongKernel without its tile order and epilogue): the same two
// groups of four waves, the same M-phase (refill of the freed stage, fragment
// reads) and C-phase (the K tile's MFMAs) one phase barrier apart, the same
// steady ring turns and the same waits. The refill comes from a four-tile
// L2-resident source laid out as the persistent skeleton's. G K tiles per launch.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void pingPongRowSkeletonKernel(const _Float16* src, int G,
                                                                                          float* sink, Stamp* out) {
    using T = ridge::GemmTraits<BM, BN, BK, WM, WN, STAGES, 8>;
    using Blk = ridge::GemmBlock<BM, BN, BK, WM, WN, STAGES, 8>;
    static_assert(T::kWaves == 8 && STAGES >= 3, "the ping-pong schedule pairs two groups of four waves");
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = T::kLoadsPerTile;
    constexpr int kTileBytes = T::kBytesA + T::kBytesB;
    __shared__ __attribute__((aligned(1024))) char lds[T::kLdsBytes];
    // One column of tiles, one per workgroup: the block forms its LDS fragment
    // offsets; its loads are `issue` below, from the four-tile source.
    Blk blk(lds, src, src, BM * (int)gridDim.x, BN, BK * G);
    const int wave = blk.wave;
    const int lane = blk.lane;
    const int group = wave / 4;
    uint32_t offA[T::kPerWaveA], offB[T::kPerWaveB];
#pragma unroll
    for (int i = 0; i < T::kPerWaveA; ++i) {
        const int q = ridge::swizzleA<T::kChunksPerRowA>((i * T::kWaves + wave) * 64 + lane);
        offA[i] = (uint32_t)(((q / T::kChunksPerRowA) * BK + (q % T::kChunksPerRowA) * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < T::kPerWaveB; ++i) {
        const int q = ridge::swizzleB<T::kChunksPerRowB>((i * T::kWaves + wave) * 64 + lane);
        offB[i] = (uint32_t)(T::kBytesA + ((q / T::kChunksPerRowB) * BN + (q % T::kChunksPerRowB) * 8) * 2);
    }
    auto issue = [&](int g, int stage) {
        const char* base = reinterpret_cast<const char*>(src) + (g & 3) * kTileBytes;
        const uint32_t dstA = blk.ldsBase + stage * T::kBytesA;
        const uint32_t dstB = blk.ldsBase + T::kRegionA + stage * T::kBytesB;
#pragma unroll
        for (int i = 0; i < T::kPerWaveA; ++i) ridge::globalLoadLds16(base, offA[i], dstA + (i * T::kWaves + wave) * 1024);
#pragma unroll
        for (int i = 0; i < T::kPerWaveB; ++i) ridge::globalLoadLds16(base, offB[i], dstB + (i * T::kWaves + wave) * 1024);
    };
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    ridge::staticFor<STAGES - 1>([&](auto sC) {
        if (sC.value < G) issue(sC.value, sC.value);
    });
    if (G >= STAGES - 1) {
        ridge::waitVmcnt<(STAGES - 2) * L>();
    } else {
        ridge::waitVmcnt<0>();
    }
    ridge::barrierLds();
    auto tileBody = [&](auto sC, auto groupC, int kt, bool steady) {
        constexpr int st = sC.value;
        constexpr int sRefill = (st + STAGES - 1) % STAGES;
        constexpr int grp = groupC.value;
        if (steady) issue(kt + STAGES - 1, sRefill);
        half8_t fa[KS][TM];
        half8_t fb[KS][TN];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) blk.template readFrags<st>(ks, fa[ks], fb[ks]);
        if constexpr (grp == 1) {
            if (steady) ridge::waitVmcnt<(STAGES - 2) * L>();
            else ridge::waitVmcnt<0>();
        }
        ridge::phaseBarrier();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) blk.mfmaStep(fa[ks], fb[ks]);
        if constexpr (grp == 0) {
            if (steady) ridge::waitVmcnt<(STAGES - 2) * L>();
            else ridge::waitVmcnt<0>();
        }
        ridge::phaseBarrier();
    };
    auto runGroup = [&](auto groupC) {
        constexpr int grp = groupC.value;
        if constexpr (grp == 1) ridge::barrierLds();
        int kt0 = 0;
        for (; kt0 + 2 * STAGES - 2 < G; kt0 += STAGES)
            ridge::staticFor<STAGES>([&](auto sC) { tileBody(sC, groupC, kt0 + sC.value, true); });
        for (; kt0 < G; kt0 += STAGES)
            ridge::staticFor<STAGES>([&](auto sC) {
                const int kt = kt0 + sC.value;
                if (kt < G) tileBody(sC, groupC, kt, kt + STAGES - 1 < G);
            });
        if constexpr (grp == 0) ridge::barrierLds();
    };
    if (group == 0) {
        runGroup(std::integral_constant<int, 0>{});
    } else {
        runGroup(std::integral_constant<int, 1>{});
    }
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    float acc = 0.0f;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc += blk.acc[tm][tn][0] + blk.acc[tm][tn][3];
    if (acc == -1.0e38f) sink[0] = acc;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

// The uniform schedule's main loop for one table row (gemmMfmaKernel without
// its tile order, K stagger and epilogue): the same prologue, fragment buffers
// alternating per k-step, one wait and one barrier per K tile, the refill of the
// freed stage after the barrier, and the steady passes where the kernel has them
// (rows of at most four waves). The refill comes from a four-tile L2-resident
// source laid out as the persistent skeleton's. G K tiles per launch; the host
// launches one or more workgroups per CU.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void uniformRowSkeletonKernel(const _Float16* src, int G,
                                                                                         float* sink, Stamp* out) {
    using T = ridge::GemmTraits<BM, BN, BK, WM, WN, STAGES, 8>;
    using Blk = ridge::GemmBlock<BM, BN, BK, WM, WN, STAGES, 8>;
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = T::kLoadsPerTile;
    constexpr int kTileBytes = T::kBytesA + T::kBytesB;
    __shared__ __attribute__((aligned(1024))) char lds[T::kLdsBytes];
    Blk blk(lds, src, src, BM * (int)gridDim.x, BN, BK * G);
    const int wave = blk.wave;
    const int lane = blk.lane;
    uint32_t offA[T::kPerWaveA], offB[T::kPerWaveB];
#pragma unroll
    for (int i = 0; i < T::kPerWaveA; ++i) {
        const int q = ridge::swizzleA<T::kChunksPerRowA>((i * T::kWaves + wave) * 64 + lane);
        offA[i] = (uint32_t)(((q / T::kChunksPerRowA) * BK + (q % T::kChunksPerRowA) * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < T::kPerWaveB; ++i) {
        const int q = ridge::swizzleB<T::kChunksPerRowB>((i * T::kWaves + wave) * 64 + lane);
        offB[i] = (uint32_t)(T::kBytesA + ((q / T::kChunksPerRowB) * BN + (q % T::kChunksPerRowB) * 8) * 2);
    }
    auto issue = [&](int g, int stage) {
        const char* base = reinterpret_cast<const char*>(src) + (g & 3) * kTileBytes;
        const uint32_t dstA = blk.ldsBase + stage * T::kBytesA;
        const uint32_t dstB = blk.ldsBase + T::kRegionA + stage * T::kBytesB;
#pragma unroll
        for (int i = 0; i < T::kPerWaveA; ++i) ridge::globalLoadLds16(base, offA[i], dstA + (i * T::kWaves + wave) * 1024);
#pragma unroll
        for (int i = 0; i < T::kPerWaveB; ++i) ridge::globalLoadLds16(base, offB[i], dstB + (i * T::kWaves + wave) * 1024);
    };
    const int numK = G;
    const uint64_t c0 = cycles();
    const uint64_t r0 = realtime();
    ridge::staticFor<STAGES>([&](auto sC) {
        if (sC.value < numK) issue(sC.value, sC.value);
    });
    if (numK >= STAGES) {
        ridge::waitVmcnt<(STAGES - 1) * L>();
    } else {
        ridge::waitVmcnt<0>();
    }
    ridge::barrierLds();
    half8_t fa[2][TM];
    half8_t fb[2][TN];
    blk.template readFrags<0>(0, fa[0], fb[0]);
    constexpr int U = (STAGES * KS) % 2 == 0 ? STAGES : 2 * STAGES;
    auto pass = [&](int kt0, auto steadyC) {
        constexpr bool steady = steadyC.value;
        ridge::staticFor<U>([&](auto iC) {
            constexpr int i = iC.value;
            constexpr int st = i % STAGES;
            constexpr int sNext = (st + 1) % STAGES;
            const int kt = kt0 + i;
            if (steady || kt < numK) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int cur = (i * KS + ks) & 1;
                    if (ks + 1 < KS) {
                        blk.template readFrags<st>(ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
                    } else if (steady || kt + 1 < numK) {
                        if (steady || kt + STAGES - 1 < numK) {
                            ridge::waitVmcnt<(STAGES - 2) * L>();
                        } else {
                            ridge::waitVmcnt<0>();
                        }
                        ridge::barrierLds();
                        if (steady || kt + STAGES < numK) issue(kt + STAGES, st);
                        blk.template readFrags<sNext>(0, fa[cur ^ 1], fb[cur ^ 1]);
                    }
                    blk.mfmaStep(fa[cur], fb[cur]);
                    ridge::interleaveHint<TM, TN>();
                }
            }
        });
    };
    int kt0 = 0;
    if constexpr (T::kWaves <= 4) {
        for (; kt0 + U - 1 + STAGES < numK; kt0 += U) pass(kt0, std::true_type{});
    }
    for (; kt0 < numK; kt0 += U) pass(kt0, std::false_type{});
    ridge::barrierLds();
    const uint64_t c1 = cycles();
    const uint64_t r1 = realtime();
    float acc = 0.0f;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc += blk.acc[tm][tn][0] + blk.acc[tm][tn][3];
    if (acc == -1.0e38f) sink[0] = acc;
    if (threadIdx.x == 0) out[blockIdx.x] = Stamp{c0, c1, r0, r1};
}

constexpr int kPersistentTiles = 1024;  // K tiles per skeleton launch

// Median cycles per K tile of the persistent skeleton over every CU (one
// workgroup each), and the median clock.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int Mode>
double persistentCycles(int cus, const _Float16* dSrc, float* dSink, Stamp* dStamps, double& clockHz,
                        _Float16* dC = nullptr, int tileK = 1) {
    using P = ridge::PersistentTraits<BM, BN, BK, WM, WN, STAGES, 8>;
    auto k = persistentSkeletonKernel<BM, BN, BK, WM, WN, STAGES, Mode>;
    hipLaunchKernelGGL(k, dim3(cus), dim3(P::kThreads), 0, nullptr, dSrc, kPersistentTiles, dSink, dStamps, dC,
                       tileK);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(cus);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, cus * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0;
    medianStamps(st, cyc, clockHz);
    return cyc / kPersistentTiles;
}

// One persistent row's cycles per K tile (the median of kRepeats launches),
// reported as `key`; beside it the reads and the MFMAs alone and the share of
// the shorter of the two that the row's waves hide under the longer,
// (t_reads + t_MFMAs - t_both) / min(t_reads, t_MFMAs), as a record.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
double persistentStep(const char* key, int cus, const _Float16* dSrc, float* dSink, Stamp* dStamps, bool& ok) {
    std::vector<double> both, reads, mfma;
    double hz = 0.0, hzBoth = 0.0;
    for (int r = 0; r < kRepeats; ++r) {
        both.push_back(persistentCycles<BM, BN, BK, WM, WN, STAGES, 0>(cus, dSrc, dSink, dStamps, hzBoth));
        reads.push_back(persistentCycles<BM, BN, BK, WM, WN, STAGES, 1>(cus, dSrc, dSink, dStamps, hz));
        mfma.push_back(persistentCycles<BM, BN, BK, WM, WN, STAGES, 2>(cus, dSrc, dSink, dStamps, hz));
    }
    const double tBoth = middle(both), tReads = middle(reads), tMfma = middle(mfma);
    const double hidden = (tReads + tMfma - tBoth) / std::min(tReads, tMfma);
    std::printf("  %dx%dx%d w%dx%d s%d (%d compute waves): both %.1f, reads %.1f, MFMAs %.1f cycles per K tile "
                "at %.1f MHz; hidden share %.3f\n",
                BM, BN, BK, WM, WN, STAGES, (BM / WM) * (BN / WN), tBoth, tReads, tMfma, hzBoth / 1e6, hidden);
    ok &= reportConstant(key, tBoth, "cycles", both);
    // The reads alone share LDS with the loaders' refill and spread more from
    // launch to launch; they are a record, not a constant, so 10% is the limit.
    ok &= reportConstant("persistentReadCycles", tReads, "cycles", reads, 0.10);
    ok &= reportConstant("persistentMfmaCycles", tMfma, "cycles", mfma);
    std::printf("CAL_INFO %sHiddenShare %.6f\n", key, hidden);
    std::printf("CAL_INFO %sClockHz %.6e\n", key, hzBoth);
    std::printf("CAL_RESULT %s %.6f\n", key, tBoth);
    return tBoth;
}

// The epilogue a persistent row's compute waves run between two output tiles,
// in cycles per tile: the skeleton with the epilogue after every tileK K tiles
// against the same skeleton without it, (t(tileK) - t) x tileK, at tileK = 4, 8,
// 16 and 32 K tiles per output tile, each launch pair alternated within a
// repeat. Reported as `key`, the middle of the four; each tile length beside it
// as a record (a constant cost per tile gives four equal figures).
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
double persistentTileCost(const char* key, int cus, const _Float16* dSrc, float* dSink, Stamp* dStamps, _Float16* dC,
                          bool& ok) {
    constexpr int kTileKs[4] = {4, 8, 16, 32};
    std::vector<double> perLength[4];
    for (int r = 0; r < kRepeats; ++r) {
        for (int i = 0; i < 4; ++i) {
            double hz = 0.0;
            const double base = persistentCycles<BM, BN, BK, WM, WN, STAGES, 0>(cus, dSrc, dSink, dStamps, hz);
            const double epi =
                persistentCycles<BM, BN, BK, WM, WN, STAGES, 3>(cus, dSrc, dSink, dStamps, hz, dC, kTileKs[i]);
            perLength[i].push_back((epi - base) * kTileKs[i]);
        }
    }
    std::vector<double> estimates;
    std::printf("  %dx%dx%d w%dx%d s%d: epilogue cycles per output tile at", BM, BN, BK, WM, WN, STAGES);
    for (int i = 0; i < 4; ++i) {
        estimates.push_back(middle(perLength[i]));
        std::printf(" %d: %.0f%s", kTileKs[i], estimates.back(), i < 3 ? "," : "");
    }
    std::printf(" K tiles per tile\n");
    for (int i = 0; i < 4; ++i) std::printf("CAL_INFO %sTileK%d %.6f\n", key, kTileKs[i], estimates[i]);
    const double cost = middle(estimates);
    // A difference of two timings, about a tenth of a K tile at tileK = 32, so
    // the four tile lengths are held to half the cost of one another.
    ok &= reportConstant(key, cost, "cycles", estimates, 0.50);
    std::printf("CAL_RESULT %s %.6f\n", key, cost);
    return cost;
}

// U[-1,1) halves from splitmix64, packed two per word: 16 KiB.
std::vector<uint32_t> randomHalfWords() {
    std::vector<uint32_t> w(16 * 1024 / 4);
    uint64_t state = 0x5eedULL;
    auto next = [&]() {
        state += 0x9e3779b97f4a7c15ULL;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        z ^= z >> 31;
        const _Float16 h = (_Float16)(float(z >> 40) * (1.0f / 8388608.0f) - 1.0f);
        return uint32_t(__builtin_bit_cast(uint16_t, h));
    };
    for (auto& x : w) x = next() | (next() << 16);
    return w;
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
        cell(W, middle(reps), reps);                                             \
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

// Median cycles per K tile of the ping-pong row skeleton over every CU (one
// workgroup each), and the median clock.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
double pingPongRowCycles(int cus, const _Float16* dSrc, float* dSink, Stamp* dStamps, double& clockHz) {
    auto k = pingPongRowSkeletonKernel<BM, BN, BK, WM, WN, STAGES>;
    hipLaunchKernelGGL(k, dim3(cus), dim3((BM / WM) * (BN / WN) * 64), 0, nullptr, dSrc, kPersistentTiles, dSink,
                       dStamps);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(cus);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, cus * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0;
    medianStamps(st, cyc, clockHz);
    return cyc / kPersistentTiles;
}

// One ping-pong row's cycles per K tile (the median of kRepeats launches),
// reported as `key`.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
double pingPongRowStep(const char* key, int cus, const _Float16* dSrc, float* dSink, Stamp* dStamps, bool& ok) {
    std::vector<double> reps;
    double hz = 0.0;
    for (int r = 0; r < kRepeats; ++r) reps.push_back(pingPongRowCycles<BM, BN, BK, WM, WN, STAGES>(cus, dSrc, dSink,
                                                                                                    dStamps, hz));
    const double t = middle(reps);
    std::printf("  %dx%dx%d w%dx%d s%d: %.1f cycles per K tile at %.1f MHz\n", BM, BN, BK, WM, WN, STAGES, t,
                hz / 1e6);
    ok &= reportConstant(key, t, "cycles", reps);
    std::printf("CAL_INFO %sClockHz %.6e\n", key, hz);
    std::printf("CAL_RESULT %s %.6f\n", key, t);
    return t;
}

// Median cycles per K tile of the uniform row skeleton with perCu workgroups on
// every CU (all resident at once), and the median clock.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
double uniformRowCycles(int cus, int perCu, const _Float16* dSrc, float* dSink, Stamp* dStamps, double& clockHz) {
    auto k = uniformRowSkeletonKernel<BM, BN, BK, WM, WN, STAGES>;
    const int blocks = cus * perCu;
    hipLaunchKernelGGL(k, dim3(blocks), dim3((BM / WM) * (BN / WN) * 64), 0, nullptr, dSrc, kPersistentTiles, dSink,
                       dStamps);
    CAL_HIP_CHECK(hipGetLastError());
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(blocks);
    CAL_HIP_CHECK(hipMemcpy(st.data(), dStamps, blocks * sizeof(Stamp), hipMemcpyDeviceToHost));
    double cyc = 0.0;
    medianStamps(st, cyc, clockHz);
    return cyc / kPersistentTiles;
}

// One uniform row's cycles per K tile of each workgroup (the median of kRepeats
// launches), reported as `key`.
template <int BM, int BN, int BK, int WM, int WN, int STAGES>
void uniformRowStep(const char* key, int cus, int perCu, const _Float16* dSrc, float* dSink, Stamp* dStamps,
                    bool& ok) {
    std::vector<double> reps;
    double hz = 0.0;
    for (int r = 0; r < kRepeats; ++r)
        reps.push_back(uniformRowCycles<BM, BN, BK, WM, WN, STAGES>(cus, perCu, dSrc, dSink, dStamps, hz));
    const double t = middle(reps);
    std::printf("  %dx%dx%d w%dx%d s%d, %d per CU: %.1f cycles per K tile of each workgroup at %.1f MHz\n", BM, BN,
                BK, WM, WN, STAGES, perCu, t, hz / 1e6);
    ok &= reportConstant(key, t, "cycles", reps);
    std::printf("CAL_INFO %sClockHz %.6e\n", key, hz);
    std::printf("CAL_RESULT %s %.6f\n", key, t);
}

// The uniform row skeletons of two classes of the table's uniform rows: eight
// waves in one workgroup per CU (256x256x64 w128x64 s2), and four waves in two
// workgroups per CU (128x128x64 w64x64 s2). A record the model does not read,
// run only by --uniform-rows-only: scaling those rows' K-steps by these figures
// predicted the measured sweeps worse.
bool uniformRows(int cus, float* dSink, const std::vector<uint32_t>& hOperands) {
    constexpr int kMaxPerCu = 2;  // the most workgroups per CU either skeleton launches
    Stamp* dStamps = nullptr;
    CAL_HIP_CHECK(hipMalloc(&dStamps, size_t(cus) * kMaxPerCu * sizeof(Stamp)));
    std::printf("\nuniform row skeletons: the kernel's K loop on a four-tile L2-resident source, %d K tiles\n",
                kPersistentTiles);
    _Float16* dSrc = nullptr;
    constexpr size_t kSrcBytes = 4 * 64 * 1024;
    CAL_HIP_CHECK(hipMalloc(&dSrc, kSrcBytes));
    for (size_t off = 0; off < kSrcBytes; off += 16 * 1024)
        CAL_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(dSrc) + off, hOperands.data(), 16 * 1024,
                                hipMemcpyHostToDevice));
    bool ok = true;
    uniformRowStep<256, 256, 64, 128, 64, 2>("uniformRowStepCycles1", cus, 1, dSrc, dSink, dStamps, ok);
    uniformRowStep<128, 128, 64, 64, 64, 2>("uniformRowStepCycles2", cus, kMaxPerCu, dSrc, dSink, dStamps, ok);
    CAL_HIP_CHECK(hipFree(dSrc));
    CAL_HIP_CHECK(hipFree(dStamps));
    return ok;
}

// The persistent skeleton of the table's BK = 128 rows (one compute wave per
// SIMD, 128x64x128 w64x32 s3), reported as persistentStepCycles3: a record the
// model does not read, run only by --persistent-bk128-only. Its 48 KiB refill per
// K tile from the L2s bounds it: the reads alone and the MFMAs alone both take
// about 827 cycles, and the combined figure spreads 7% from launch to launch.
bool persistentDeep(int cus, float* dSink, Stamp* dStamps, const std::vector<uint32_t>& hOperands) {
    std::printf("\npersistent skeleton of the BK = 128 rows: compute waves + 2 loader waves, %d K tiles\n",
                kPersistentTiles);
    _Float16* dSrc = nullptr;
    constexpr size_t kSrcBytes = 4 * 48 * 1024;
    CAL_HIP_CHECK(hipMalloc(&dSrc, kSrcBytes));
    for (size_t off = 0; off < kSrcBytes; off += 16 * 1024)
        CAL_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(dSrc) + off, hOperands.data(), 16 * 1024,
                                hipMemcpyHostToDevice));
    bool ok = true;
    persistentStep<128, 64, 128, 64, 32, 3>("persistentStepCycles3", cus, dSrc, dSink, dStamps, ok);
    CAL_HIP_CHECK(hipFree(dSrc));
    return ok;
}

// The ping-pong row skeletons of the two classes of the table's ping-pong rows:
// BK = 32 with 128x64 (or 64x128) wave tiles, and BK = 64 with 64x64 ones.
bool pingPongRows(int cus, float* dSink, Stamp* dStamps, const std::vector<uint32_t>& hOperands) {
    std::printf("\nping-pong row skeletons: the kernel's phase loop on a four-tile L2-resident source, %d K tiles\n",
                kPersistentTiles);
    _Float16* dSrc = nullptr;
    constexpr size_t kSrcBytes = 4 * 48 * 1024;
    CAL_HIP_CHECK(hipMalloc(&dSrc, kSrcBytes));
    for (size_t off = 0; off < kSrcBytes; off += 16 * 1024)
        CAL_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(dSrc) + off, hOperands.data(), 16 * 1024,
                                hipMemcpyHostToDevice));
    bool ok = true;
    pingPongRowStep<256, 256, 32, 128, 64, 3>("pingPongRowStepCycles1", cus, dSrc, dSink, dStamps, ok);
    pingPongRowStep<256, 128, 64, 64, 64, 3>("pingPongRowStepCycles2", cus, dSrc, dSink, dStamps, ok);
    CAL_HIP_CHECK(hipFree(dSrc));
    return ok;
}

int main(int argc, char** argv) {
    const bool pingPongOnly = argc > 1 && std::string(argv[1]) == "--ping-pong-rows-only";
    const bool deepOnly = argc > 1 && std::string(argv[1]) == "--persistent-bk128-only";
    const bool uniformOnly = argc > 1 && std::string(argv[1]) == "--uniform-rows-only";
    if (argc > 1 && !pingPongOnly && !deepOnly && !uniformOnly) {
        std::fprintf(stderr,
                     "usage: cal-smem-bw [--ping-pong-rows-only | --persistent-bk128-only | --uniform-rows-only]\n");
        return 2;
    }
    const hipDeviceProp_t prop = deviceBanner();
    const int cus = prop.multiProcessorCount;
    uint32_t* dSink = nullptr;
    Stamp* dStamps = nullptr;
    CAL_HIP_CHECK(hipMalloc(&dSink, sizeof(uint32_t)));
    CAL_HIP_CHECK(hipMalloc(&dStamps, cus * sizeof(Stamp)));
    warmUp();
    if (pingPongOnly || deepOnly || uniformOnly) {
        float* dFSink = nullptr;
        CAL_HIP_CHECK(hipMalloc(&dFSink, sizeof(float)));
        const bool ok = pingPongOnly ? pingPongRows(cus, dFSink, dStamps, randomHalfWords())
                        : deepOnly   ? persistentDeep(cus, dFSink, dStamps, randomHalfWords())
                                     : uniformRows(cus, dFSink, randomHalfWords());
        CAL_HIP_CHECK(hipFree(dFSink));
        CAL_HIP_CHECK(hipFree(dSink));
        CAL_HIP_CHECK(hipFree(dStamps));
        return ok ? 0 : 1;
    }
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

    // The ping-pong skeleton.
    uint32_t* dOperands = nullptr;
    char* dRefill = nullptr;
    float* dFSink = nullptr;
    const std::vector<uint32_t> hOperands = randomHalfWords();
    CAL_HIP_CHECK(hipMalloc(&dOperands, hOperands.size() * sizeof(uint32_t)));
    CAL_HIP_CHECK(hipMalloc(&dRefill, kRefillSourceBytes));
    CAL_HIP_CHECK(hipMalloc(&dFSink, sizeof(float)));
    CAL_HIP_CHECK(hipMemcpy(dOperands, hOperands.data(), hOperands.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
    // The L2-resident refill source holds the same U[-1,1) halves as the
    // fragments (the 16 KiB block, tiled): the GEMM streams random operands, and
    // the bits its loads and LDS writes toggle are part of what the loaded clock
    // (mode 3 against mode 2) pays for. The L2-missing windows below keep a
    // constant fill: they time the refill path's rate and stretch, and with
    // random data their repeats spread by up to 25% on one box.
    for (size_t off = 0; off < size_t(kRefillSourceBytes); off += 16 * 1024)
        CAL_HIP_CHECK(hipMemcpy(dRefill + off, hOperands.data(), 16 * 1024, hipMemcpyHostToDevice));
    // The L2-missing windows: one per CU (workgroup g uses [g * 512 KiB, +512 KiB)).
    char* dMall = nullptr;
    const size_t mallBytes = size_t(cus) * (kMallWindowKiB << 10);
    CAL_HIP_CHECK(hipMalloc(&dMall, mallBytes));
    CAL_HIP_CHECK(hipMemset(dMall, 0x3c, mallBytes));
    constexpr int kModes = 9;
    std::vector<double> st[kModes], hz[kModes];
    for (int r = 0; r < kRepeats; ++r) {
        double h = 0.0;
#define CAL_MODE(M)                                                                             \
    st[M].push_back(pingPongCycles<M>(cus, dOperands, dRefill, dMall, dFSink, dStamps, h));    \
    hz[M].push_back(h)
        CAL_MODE(0);
        CAL_MODE(1);
        CAL_MODE(2);
        CAL_MODE(3);
        CAL_MODE(4);
        CAL_MODE(5);
        CAL_MODE(6);
        CAL_MODE(7);
        CAL_MODE(8);
#undef CAL_MODE
    }
    const char* kModeNames[kModes] = {"ping-pong (reads under MFMAs)", "fragment reads alone", "MFMAs alone",
                                      "ping-pong + 32 KiB direct-to-LDS refill", "free-running (no barriers)",
                                      "the refill, 1/4 missing the L2", "the refill, all missing the L2",
                                      "the refill, 1/2 missing the L2", "the refill, 3/4 missing the L2"};
    const char* kModeKeys[kModes] = {"pingPongStepCycles", "pingPongReadCycles", "pingPongMfmaCycles",
                                     "pingPongRefillStepCycles", "freeRunningStepCycles",
                                     "pingPongMiss25StepCycles", "pingPongMiss100StepCycles",
                                     "pingPongMiss50StepCycles", "pingPongMiss75StepCycles"};
    std::printf("\nping-pong skeleton: 8 waves (2 per SIMD), 128x64 wavefront tiles, BK = 32; per K-step per CU\n");
    double tStep[kModes], clock[kModes];
    for (int m = 0; m < kModes; ++m) {
        tStep[m] = middle(st[m]);
        clock[m] = middle(hz[m]);
        std::printf("  %-44s %8.1f cycles  %7.1f MHz\n", kModeNames[m], tStep[m], clock[m] / 1e6);
        std::printf("CAL_INFO %s %.6f\n", kModeKeys[m], tStep[m]);
        std::printf("CAL_INFO %sClockHz %.6e\n", kModeKeys[m], clock[m]);
    }
    // The L2-missing refill path. With all of the refill missing the L2 the
    // K-step is bound by that path (it stretches to its transfer time), which
    // gives the path's rate; a share m of the refill then loads the path to
    // rho = m x (its all-miss transfer time) / (the all-hits K-step time), and
    // the K-step stretches by t(m) / t(0).
    const double refillBytes = 32.0 * 1024.0 * cus;  // per K-step, whole chip
    const double mallRate = refillBytes / (tStep[6] / clock[6]);
    const double allMissLoad = (tStep[6] / clock[6]) / (tStep[3] / clock[3]);
    std::printf("  L2-missing refill path: %.2f TB/s (the all-miss K-step is bound by it)\n", mallRate / 1e12);
    std::printf("CAL_RESULT mallRefillBytesPerSec %.6e\n", mallRate);
    const int curveModes[5] = {3, 5, 7, 8, 6};
    const double shares[5] = {0.0, 0.25, 0.5, 0.75, 1.0};
    std::printf("  %8s %8s %12s %10s\n", "miss", "load", "stretch", "clock");
    for (int i = 0; i < 5; ++i) {
        const int m = curveModes[i];
        const double load = shares[i] * allMissLoad;
        const double stretch = (tStep[m] / clock[m]) / (tStep[3] / clock[3]);
        std::printf("  %8.2f %8.3f %12.4f %10.4f\n", shares[i], load, stretch, clock[m] / clock[3]);
        std::printf("CAL_RESULT mallStretchLoad%d %.6f\n", i, load);
        std::printf("CAL_RESULT mallStretch%d %.6f\n", i, stretch);
    }
    CAL_HIP_CHECK(hipFree(dMall));
    const double tS = 8 * (8 * 1024.0 / a.best + 8 * 512.0 / b.best);
    std::printf("  reads alone against the per-operand rates: %.1f measured, %.1f from ldsA/ldsBTr\n", tStep[1], tS);
    std::printf("  cost of a phase switch: %.1f cycles ((ping-pong - max(reads, MFMAs)) / 2)\n",
                (tStep[0] - std::max(tStep[1], tStep[2])) / 2.0);
    std::printf("CAL_INFO phaseSwitchCycles %.6f\n", (tStep[0] - std::max(tStep[1], tStep[2])) / 2.0);
    // Share of the shorter phase that two free-running waves per SIMD hide under
    // the longer one: 0 = in series, 1 = a perfect overlap.
    const double hidden =
        (tStep[1] + tStep[2] - tStep[4]) / std::min(tStep[1], tStep[2]);
    std::printf("  free-running waves hide %.3f of the shorter phase under the longer\n", hidden);
    std::printf("CAL_RESULT freeRunningOverlap %.6f\n", hidden);
    // Modes bound by the L2-missing path (3/4 and all of the refill missing)
    // queue on it and spread more from launch to launch; their limit is 20%.
    for (int m = 0; m < kModes; ++m)
        ok &= reportConstant(kModeKeys[m], tStep[m], "cycles", st[m], (m == 6 || m == 8) ? 0.20 : 0.05);

    // The persistent schedule's skeletons: one row with one compute wave per
    // SIMD (128x128x64 w64x64 s4) and one with two (256x128x32 w64x64 s6).
    // Source: four K tiles of U[-1,1) halves (the operand block, repeated).
    std::printf("\npersistent skeleton: compute waves + 2 loader waves, one barrier per K tile, %d K tiles\n",
                kPersistentTiles);
    _Float16* dSrc = nullptr;
    constexpr size_t kSrcBytes = 4 * 48 * 1024;
    CAL_HIP_CHECK(hipMalloc(&dSrc, kSrcBytes));
    for (size_t off = 0; off < kSrcBytes; off += 16 * 1024)
        CAL_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(dSrc) + off, hOperands.data(), 16 * 1024,
                                hipMemcpyHostToDevice));
    persistentStep<128, 128, 64, 64, 64, 4>("persistentStepCycles1", cus, dSrc, dFSink, dStamps, ok);
    persistentStep<256, 128, 32, 64, 64, 6>("persistentStepCycles2", cus, dSrc, dFSink, dStamps, ok);
    // The epilogue between output tiles, for the same two rows. C: cus x
    // kEpiSlots output tiles of the larger row (256 x 128 halves each).
    std::printf("\npersistent skeleton with the kernel's epilogue between output tiles\n");
    _Float16* dC = nullptr;
    const size_t cBytes = size_t(cus) * kEpiSlots * 256 * 128 * sizeof(_Float16);
    CAL_HIP_CHECK(hipMalloc(&dC, cBytes));
    persistentTileCost<128, 128, 64, 64, 64, 4>("persistentTileCycles1", cus, dSrc, dFSink, dStamps, dC, ok);
    persistentTileCost<256, 128, 32, 64, 64, 6>("persistentTileCycles2", cus, dSrc, dFSink, dStamps, dC, ok);
    CAL_HIP_CHECK(hipFree(dC));
    CAL_HIP_CHECK(hipFree(dSrc));
    ok &= pingPongRows(cus, dFSink, dStamps, hOperands);
    CAL_HIP_CHECK(hipFree(dOperands));
    CAL_HIP_CHECK(hipFree(dRefill));
    CAL_HIP_CHECK(hipFree(dFSink));

    std::printf("\nCAL_RESULT smemBytesPerCycle %.6f\n", mix.best);
    std::printf("CAL_RESULT smemSaturationWaves %d\n", mix.bestWaves);
    std::printf("CAL_RESULT ldsControlBytesPerCycle %.6f\n", ctl.best);
    std::printf("CAL_RESULT ldsAReadBytesPerCycle %.6f\n", a.best);
    std::printf("CAL_RESULT ldsBTrReadBytesPerCycle %.6f\n", b.best);
    CAL_HIP_CHECK(hipFree(dSink));
    CAL_HIP_CHECK(hipFree(dStamps));
    return ok ? 0 : 1;
}
