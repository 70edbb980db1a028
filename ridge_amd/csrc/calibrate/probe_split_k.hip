// probe_split_k.hip -- a split-K schedule for the tall-skinny GEMM, priced against
// the table's row. Not a table row: a diagnostic, and the model reads none of it.
//
// The BASELINE tall-skinny shape (M = 16384, N = 128, K = 8192) runs on the
// persistent 64x128x128 row at the speed of its operand loads, and B's L2 stream
// (re-read once per 64 rows of A) costs the A stream 18%. Taller tiles read B once
// per more rows, but 128-row tiles give only 128 workgroups for 256 CUs, so the K
// range is split: workgroup u takes part u % S of output tile u / S's K tiles.
//
// Exchange of the parts (no workgroup waits for another): every part writes its
// FP32 accumulators to `partials`, in the accumulators' own register layout; one
// device-scope atomic add on `counters[tile]` tells each part how many came
// before it; the last one adds the S parts in part order (its own from
// registers), writes C through the kernels' staged epilogue and sets the counter
// back to zero for the next launch. Two orderings of the exchange are built:
//   device-scope accesses  partials are written and read with device-scope
//                     (L2-bypassing) dword atomics; a vmcnt(0) wait before the
//                     counter is the only ordering needed;
//   fences            plain float4 stores and loads ordered by __threadfence()
//                     around an acquire-release counter add. On gfx950 each
//                     agent-scope fence writes back and invalidates its XCD's
//                     whole L2.
// Loads are the persistent row's: two loader wavefronts, direct-to-LDS, each
// part's K tiles in a staggered order (from K tile (row panel) mod G, wrapping).
//
// Checked before timing: small-integer operands (every sum exact in FP32, so the
// order of the parts cannot change a bit) against the table row, with every
// counter back at zero. Reported: microseconds per launch, warm (one operand set)
// and cold (launches rotate over 3 sets, 822 MB, beyond the 256 MB MALL), each the
// middle of 5 windows of 30 launches after the warm-up.
#include "cal_common.hpp"
#include "gemm_mfma.hpp"

#include <cstring>

using namespace ridgecal;

namespace {

using ridge::float4_t;
using ridge::half8_t;

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM, bool FENCES>
__global__ __launch_bounds__(((BM / WM) * (BN / WN) + ridge::kPersistentLoaders) * ridge::kWaveSize)
void splitKKernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B, _Float16* __restrict__ C, int M,
                  int N, int K, int split, float* __restrict__ partials, int* __restrict__ counters) {
    using T = ridge::GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    using P = ridge::PersistentTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    using Blk = ridge::GemmBlock<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = P::kLoads;

    __shared__ __attribute__((aligned(1024))) char lds[P::kLdsBytes];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / ridge::kWaveSize);
    const int lane = threadIdx.x % ridge::kWaveSize;
    const int unit = ridge::xcdRemap(blockIdx.x, gridDim.x);
    const int tile = unit / split;
    const int part = unit % split;
    const int G = (K / BK) / split;  // this part's K tiles
    const int kBase = part * G;

    if (wave >= T::kWaves) {
        // Loader wave l issues wave loads l, l + kLoaders, ... of each K tile.
        const int l = wave - T::kWaves;
        const uint32_t ldsBase = ridge::ldsAddress(lds);
        uint32_t offA[P::kLoadsA], offB[P::kLoadsB];
#pragma unroll
        for (int i = 0; i < P::kLoadsA; ++i) {
            const int q = ridge::swizzleA<T::kChunksPerRowA>((i * P::kLoaders + l) * 64 + lane);
            offA[i] = ridge::tileOffset(q / T::kChunksPerRowA, K, q % T::kChunksPerRowA);
        }
#pragma unroll
        for (int i = 0; i < P::kLoadsB; ++i) {
            const int q = ridge::swizzleB<T::kChunksPerRowB>((i * P::kLoaders + l) * 64 + lane);
            offB[i] = ridge::tileOffset(q / T::kChunksPerRowB, N, q % T::kChunksPerRowB);
        }
        int row, col;
        ridge::tileOf<BM, BN, GROUPM>(tile, M, N, row, col);
        const size_t strideB = (size_t)BK * N * 2;
        const char* srcA = reinterpret_cast<const char*>(A + (size_t)row * K) + (size_t)kBase * BK * 2;
        const char* srcB = reinterpret_cast<const char*>(B + col) + (size_t)kBase * strideB;
        int kIdx = (row / BM) % G;
        auto issueNext = [&](int stage) {
            uint32_t lb = ldsBase;
            asm volatile("" : "+s"(lb));
            const uint32_t dstA = lb + stage * T::kBytesA;
            const uint32_t dstB = lb + T::kRegionA + stage * T::kBytesB;
            const char* tA = srcA + (size_t)kIdx * BK * 2;
            const char* tB = srcB + (size_t)kIdx * strideB;
#pragma unroll
            for (int i = 0; i < P::kLoadsA; ++i)
                ridge::globalLoadLds16(tA, offA[i], dstA + (i * P::kLoaders + l) * 1024);
#pragma unroll
            for (int i = 0; i < P::kLoadsB; ++i)
                ridge::globalLoadLds16(tB, offB[i], dstB + (i * P::kLoaders + l) * 1024);
            if (++kIdx == G) kIdx = 0;
        };
        ridge::staticFor<STAGES - 1>([&](auto sC) {
            if (sC.value < G) issueNext(sC.value);
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
                        issueNext((s + STAGES - 1) % STAGES);
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

    Blk blk(lds, A, B, M, N, K);
    blk.setTile(tile, M, N, K);
    RIDGE_LDS_AS char* region = (RIDGE_LDS_AS char*)(lds) + T::kLdsBytes + wave * P::kRegionBytes;
    ridge::barrierLds();  // B_0
    half8_t fa[2][TM];
    half8_t fb[2][TN];
    blk.template readFrags<0>(0, fa[0], fb[0]);
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
                        blk.template readFrags<s>(ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
                    } else if (g + 1 < G) {
                        ridge::barrierLds();  // B_{g+1}
                        blk.template readFrags<sNext>(0, fa[cur ^ 1], fb[cur ^ 1]);
                    }
                    blk.mfmaStep(fa[cur], fb[cur]);
                    ridge::interleaveHint<TM, TN>();
                }
            }
        });
    }
    if (split > 1) {
        // Wave w of part p owns floats [((tile * split + p) * waves + w) * kWaveFloats, + kWaveFloats).
        constexpr int kWaveFloats = TM * TN * 256;
        float* mine = partials + ((size_t)unit * T::kWaves + wave) * kWaveFloats;
        if constexpr (FENCES) {
            float4_t* dst = reinterpret_cast<float4_t*>(mine);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) dst[(tm * TN + tn) * 64 + lane] = blk.acc[tm][tn];
            __threadfence();
        } else {
            // Element e of accumulator (tm, tn) of lane l at ((tm * TN + tn) * 4 + e) * 64 + l.
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        __hip_atomic_store(mine + ((tm * TN + tn) * 4 + e) * 64 + lane, blk.acc[tm][tn][e],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ridge::waitVmcnt<0>();  // this wave's partials are visible device-wide
        }
        ridge::barrierLds();
        // The flag word is the first of wave 0's staging region, unused until the epilogue.
        int* flag = reinterpret_cast<int*>(lds + T::kLdsBytes);
        if (wave == 0 && lane == 0)
            *flag = FENCES ? __hip_atomic_fetch_add(&counters[tile], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT)
                           : __hip_atomic_fetch_add(&counters[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ridge::barrierLds();
        const int before = *reinterpret_cast<volatile int*>(flag);
        if (before != split - 1) return;
        if constexpr (FENCES) __threadfence();
        ridge::barrierLds();  // every wave has read the flag before wave 0's staging region is reused
        float4_t total[TM][TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) total[tm][tn] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        for (int p = 0; p < split; ++p) {
            if (p == part) {
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) total[tm][tn] += blk.acc[tm][tn];
                continue;
            }
            const float* src = partials + ((size_t)(tile * split + p) * T::kWaves + wave) * kWaveFloats;
            if constexpr (FENCES) {
                const float4_t* s4 = reinterpret_cast<const float4_t*>(src);
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) total[tm][tn] += s4[(tm * TN + tn) * 64 + lane];
            } else {
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            total[tm][tn][e] += __hip_atomic_load(src + ((tm * TN + tn) * 4 + e) * 64 + lane,
                                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        ridge::storeStaged<TM, TN, WN, P::kEpiTiles, true>(total, region, blk.waveC(C, N), N, lane);
        if (wave == 0 && lane == 0) __hip_atomic_store(&counters[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    ridge::storeStaged<TM, TN, WN, P::kEpiTiles, true>(blk.acc, region, blk.waveC(C, N), N, lane);
}

// Element i of a U[-1,1) FP16 fill, or of a small-integer one in {-2, ..., 2}.
__global__ void fillKernel(_Float16* p, size_t n, uint64_t seed, int integers) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint64_t z = seed * 0x9e3779b97f4a7c15ull + i;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        p[i] = integers ? (_Float16)(int(z % 5) - 2) : (_Float16)((double)(z >> 11) * (2.0 / 9007199254740992.0) - 1.0);
    }
}

// One way to launch C = A B: the table's persistent row or a split-K kernel.
struct Schedule {
    const char* name;
    int BM, BN, split;
    bool persistentRow;
    const void* kernel;
    int threads;
    size_t partialFloats(int M, int N) const { return split > 1 ? (size_t)(M / BM) * (N / BN) * split * BM * BN : 0; }
};

template <int BM, int BN, int BK, int WM, int WN, int S, int G, bool F>
Schedule splitK(const char* name, int split) {
    using P = ridge::PersistentTraits<BM, BN, BK, WM, WN, S, G>;
    return Schedule{name, BM, BN, split, false, reinterpret_cast<const void*>(&splitKKernel<BM, BN, BK, WM, WN, S, G, F>),
                    P::kThreads};
}

template <int BM, int BN, int BK, int WM, int WN, int S, int G>
Schedule tableRow(const char* name) {
    using P = ridge::PersistentTraits<BM, BN, BK, WM, WN, S, G>;
    return Schedule{name, BM, BN, 1, true,
                    reinterpret_cast<const void*>(&ridge::gemmMfmaPersistentKernel<BM, BN, BK, WM, WN, S, G>),
                    P::kThreads};
}

struct Workspace {
    float* partials = nullptr;
    int* counters = nullptr;
    size_t floats = 0, tiles = 0;
};

// Enqueues one launch; the host checks every size the kernel assumes first.
void launch(const Schedule& s, const _Float16* A, const _Float16* B, _Float16* C, int M, int N, int K, int BK,
            const Workspace& ws, int resident) {
    const size_t tiles = (size_t)(M / s.BM) * (N / s.BN);
    if (M % s.BM || N % s.BN || K % BK || (K / BK) % s.split || (K / BK) / s.split < 1) {
        std::fprintf(stderr, "%s does not divide %dx%dx%d\n", s.name, M, N, K);
        std::exit(1);
    }
    if (s.split > 1 && (ws.floats < s.partialFloats(M, N) || ws.tiles < tiles)) {
        std::fprintf(stderr, "%s: workspace too small\n", s.name);
        std::exit(1);
    }
    if (s.persistentRow) {
        const unsigned grid = (unsigned)(tiles < (size_t)resident ? tiles : (size_t)resident);
        void* args[] = {&A, &B, &C, &M, &N, &K};
        CAL_HIP_CHECK(hipLaunchKernel(s.kernel, dim3(grid), dim3(s.threads), args, 0, nullptr));
    } else {
        int split = s.split;
        float* partials = ws.partials;
        int* counters = ws.counters;
        void* args[] = {&A, &B, &C, &M, &N, &K, &split, &partials, &counters};
        CAL_HIP_CHECK(hipLaunchKernel(s.kernel, dim3((unsigned)(tiles * s.split)), dim3(s.threads), args, 0, nullptr));
    }
}

template <typename Launch>
double timeLaunches(Launch fn, int n, int launches) {
    for (int i = 0; i < 3 * launches; ++i) fn(i % n);
    CAL_HIP_CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CAL_HIP_CHECK(hipEventCreate(&e0));
    CAL_HIP_CHECK(hipEventCreate(&e1));
    std::vector<double> sec;
    for (int w = 0; w < 5; ++w) {
        CAL_HIP_CHECK(hipEventRecord(e0, nullptr));
        for (int i = 0; i < launches; ++i) fn(i % n);
        CAL_HIP_CHECK(hipEventRecord(e1, nullptr));
        CAL_HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CAL_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        sec.push_back(ms * 1e-3 / launches);
    }
    CAL_HIP_CHECK(hipEventDestroy(e0));
    CAL_HIP_CHECK(hipEventDestroy(e1));
    return middle(sec);
}

}  // namespace

int main() {
    deviceBanner();
    constexpr int M = 16384, N = 128, K = 8192, kSets = 3;
    const int BKs[] = {128, 128, 128, 128, 64, 64, 128};
    const Schedule rows[] = {
        tableRow<64, 128, 128, 32, 64, 3, 8>("table row 64x128x128 w32x64 s3 g8"),
        splitK<128, 128, 128, 64, 64, 2, 8, false>("128x128x128 w64x64 s2, K whole", 1),
        splitK<128, 128, 128, 64, 64, 2, 8, false>("128x128x128 w64x64 s2, K in 2", 2),
        splitK<128, 128, 128, 64, 64, 2, 8, true>("128x128x128 s2, K in 2, fences", 2),
        splitK<128, 128, 64, 64, 64, 4, 8, false>("128x128x64 w64x64 s4, K in 2", 2),
        splitK<128, 128, 64, 64, 64, 4, 8, false>("128x128x64 w64x64 s4, K in 4", 4),
        splitK<64, 128, 128, 32, 64, 3, 8, false>("64x128x128 w32x64 s3, K in 2", 2),
    };
    constexpr int kRows = int(sizeof(rows) / sizeof(rows[0]));
    int dev = 0, cus = 0, perCu = 0;
    CAL_HIP_CHECK(hipGetDevice(&dev));
    CAL_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    CAL_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu, rows[0].kernel, rows[0].threads, 0));
    const int resident = cus * (perCu > 0 ? perCu : 1);

    const size_t nA = (size_t)M * K, nB = (size_t)K * N, nC = (size_t)M * N;
    std::vector<_Float16*> As(kSets), Bs(kSets), Cs(kSets);
    for (int s = 0; s < kSets; ++s) {
        CAL_HIP_CHECK(hipMalloc(&As[s], nA * 2));
        CAL_HIP_CHECK(hipMalloc(&Bs[s], nB * 2));
        CAL_HIP_CHECK(hipMalloc(&Cs[s], nC * 2));
    }
    _Float16* Cref = nullptr;
    CAL_HIP_CHECK(hipMalloc(&Cref, nC * 2));
    Workspace ws;
    for (const Schedule& s : rows) ws.floats = std::max(ws.floats, s.partialFloats(M, N));
    ws.tiles = (size_t)(M / 64) * (N / 128);
    CAL_HIP_CHECK(hipMalloc(&ws.partials, ws.floats * 4));
    CAL_HIP_CHECK(hipMalloc(&ws.counters, ws.tiles * 4));
    CAL_HIP_CHECK(hipMemset(ws.counters, 0, ws.tiles * 4));

    // Exactness: small integers, every schedule against the table row, counters back at zero.
    hipLaunchKernelGGL(fillKernel, dim3(1024), dim3(256), 0, nullptr, As[0], nA, 11, 1);
    hipLaunchKernelGGL(fillKernel, dim3(1024), dim3(256), 0, nullptr, Bs[0], nB, 12, 1);
    launch(rows[0], As[0], Bs[0], Cref, M, N, K, BKs[0], ws, resident);
    std::vector<uint16_t> ref(nC), got(nC);
    std::vector<int> cnt(ws.tiles);
    CAL_HIP_CHECK(hipMemcpy(ref.data(), Cref, nC * 2, hipMemcpyDeviceToHost));
    bool exact = true;
    for (int r = 1; r < kRows; ++r) {
        for (int rep = 0; rep < 2; ++rep) {
            CAL_HIP_CHECK(hipMemset(Cs[0], 0xff, nC * 2));
            launch(rows[r], As[0], Bs[0], Cs[0], M, N, K, BKs[r], ws, resident);
            CAL_HIP_CHECK(hipMemcpy(got.data(), Cs[0], nC * 2, hipMemcpyDeviceToHost));
            CAL_HIP_CHECK(hipMemcpy(cnt.data(), ws.counters, ws.tiles * 4, hipMemcpyDeviceToHost));
            const bool same = std::memcmp(ref.data(), got.data(), nC * 2) == 0;
            bool zero = true;
            for (int c : cnt) zero = zero && c == 0;
            if (!same || !zero) {
                std::printf("  %-34s launch %d: %s%s\n", rows[r].name, rep, same ? "" : "C differs from the table row ",
                            zero ? "" : "counters not reset");
                exact = false;
            }
        }
    }
    std::printf("exactness on small integers, two launches per schedule: %s\n", exact ? "all bit-identical" : "FAILED");
    if (!exact) return 1;

    warmUp();
    for (int s = 0; s < kSets; ++s) {
        hipLaunchKernelGGL(fillKernel, dim3(1024), dim3(256), 0, nullptr, As[s], nA, 1 + 2 * s, 0);
        hipLaunchKernelGGL(fillKernel, dim3(1024), dim3(256), 0, nullptr, Bs[s], nB, 2 + 2 * s, 0);
    }
    CAL_HIP_CHECK(hipDeviceSynchronize());
    std::printf("\n16384 x 128 x 8192, microseconds per launch (middle of 5 windows of 30)\n");
    for (int r = 0; r < kRows; ++r) {
        double t[2];
        for (int cold = 0; cold < 2; ++cold)
            t[cold] = timeLaunches([&](int i) {
                const int set = cold ? i : 0;
                launch(rows[r], As[set], Bs[set], Cs[set], M, N, K, BKs[r], ws, resident);
            }, cold ? kSets : 1, 30);
        std::printf("  %-34s warm %7.1f us   cold %7.1f us\n", rows[r].name, t[0] * 1e6, t[1] * 1e6);
        std::printf("PROBE splitK row%d warmSeconds %.6e coldSeconds %.6e\n", r, t[0], t[1]);
    }
    for (int s = 0; s < kSets; ++s) {
        CAL_HIP_CHECK(hipFree(As[s]));
        CAL_HIP_CHECK(hipFree(Bs[s]));
        CAL_HIP_CHECK(hipFree(Cs[s]));
    }
    CAL_HIP_CHECK(hipFree(Cref));
    CAL_HIP_CHECK(hipFree(ws.partials));
    CAL_HIP_CHECK(hipFree(ws.counters));
    return 0;
}
