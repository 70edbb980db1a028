// gemm_kernels.hip -- instantiates the gfx950 GEMM template over the registered
// variant table and exports the table through the C ABI in include/ridge_gemm.h.
//
// Counterpart of bench/kernels/gemm-mma.cu (launchVariant :19-43, kVariants
// :55-117, numVariants/variant/printVariantTable :121-141).

#include "gemm_mfma.hpp"
#include "gemm_resources.h"
#include "ridge_gemm.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>

namespace {

typedef hipError_t (*LaunchFn)(const void*, const void*, void*, int, int, int, hipStream_t);

// Schedules (ridge_gemm_variant_t.schedule). Rows written RIDGE_VARIANT take
// theirs from the tile config: eight wavefronts (two per SIMD) with a ring of
// three or more stages run the ping-pong schedule, every other row the uniform
// one. Rows written RIDGE_VARIANT_PERSISTENT run the persistent store-behind
// schedule.
enum Schedule { kUniform = 0, kPingPong = 1, kPersistent = 2 };
constexpr bool usesPingPong(int waves, int stages) { return waves == 8 && stages >= 3; }

// Workgroups of `kernel` resident on the current device at once (CUs x
// workgroups per CU), cached per device: the persistent grid. Launches from
// several host threads may fill the cache concurrently; they compute the same
// value, and the atomic makes the store and the loads well defined.
int residentSlots(const void* kernel, int threads, std::atomic<int>& cache) {
    const int cached = cache.load(std::memory_order_relaxed);
    if (cached > 0) return cached;
    int dev = 0, cus = 0, perCu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu, kernel, threads, 0) != hipSuccess) return 0;
    const int slots = cus * (perCu > 0 ? perCu : 1);
    cache.store(slots, std::memory_order_relaxed);
    return slots;
}

constexpr int kMaxDevices = 64;

template <int BM, int BN, int BK, int WM, int WN, int S, int G>
hipError_t launchPersistent(const void* A, const void* B, void* C, int M, int N, int K, hipStream_t stream) {
    using P = ridge::PersistentTraits<BM, BN, BK, WM, WN, S, G>;
    static std::atomic<int> slots[kMaxDevices];
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    const void* kernel = reinterpret_cast<const void*>(&ridge::gemmMfmaPersistentKernel<BM, BN, BK, WM, WN, S, G>);
    const int resident = residentSlots(kernel, P::kThreads, slots[dev]);
    if (resident <= 0) return hipErrorInvalidConfiguration;
    // Every workgroup must own at least one tile (the kernel's tile count per
    // workgroup assumes it).
    const int tiles = (M / BM) * (N / BN);
    const dim3 grid((unsigned)(tiles < resident ? tiles : resident));
    hipLaunchKernelGGL((ridge::gemmMfmaPersistentKernel<BM, BN, BK, WM, WN, S, G>), grid, dim3(P::kThreads), 0,
                       stream, static_cast<const _Float16*>(A), static_cast<const _Float16*>(B),
                       static_cast<_Float16*>(C), M, N, K);
    return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN, int S, int G>
hipError_t launchVariant(const void* A, const void* B, void* C, int M, int N, int K, hipStream_t stream) {
    using T = ridge::GemmTraits<BM, BN, BK, WM, WN, S, G>;
    const dim3 grid((unsigned)((M / BM) * (N / BN)));
    const dim3 block(T::kThreads);
    if constexpr (usesPingPong(T::kWaves, S)) {
        hipLaunchKernelGGL((ridge::gemmMfmaPingPongKernel<BM, BN, BK, WM, WN, S, G>), grid, block, 0, stream,
                           static_cast<const _Float16*>(A), static_cast<const _Float16*>(B),
                           static_cast<_Float16*>(C), M, N, K);
    } else {
        hipLaunchKernelGGL((ridge::gemmMfmaKernel<BM, BN, BK, WM, WN, S, G>), grid, block, 0, stream,
                           static_cast<const _Float16*>(A), static_cast<const _Float16*>(B),
                           static_cast<_Float16*>(C), M, N, K);
    }
    return hipGetLastError();
}

struct Entry {
    int BM, BN, BK, WM, WN, stages, groupM;
    int ldsBytes;
    int threads;
    int waves;
    int schedule;
    LaunchFn launch;
};

#define RIDGE_VARIANT(BM, BN, BK, WM, WN, S, G)                                              \
    Entry{BM, BN, BK, WM, WN, S, G,                                                          \
          ridge::GemmTraits<BM, BN, BK, WM, WN, S, G>::kLdsBytes,                            \
          ridge::GemmTraits<BM, BN, BK, WM, WN, S, G>::kThreads,                             \
          ridge::GemmTraits<BM, BN, BK, WM, WN, S, G>::kWaves,                               \
          usesPingPong(ridge::GemmTraits<BM, BN, BK, WM, WN, S, G>::kWaves, S) ? kPingPong : kUniform, \
          &launchVariant<BM, BN, BK, WM, WN, S, G>},

// ldsBytes includes the epilogue staging; threads and waves include the two
// loader wavefronts.
#define RIDGE_VARIANT_PERSISTENT(BM, BN, BK, WM, WN, S, G)                                   \
    Entry{BM, BN, BK, WM, WN, S, G,                                                          \
          ridge::PersistentTraits<BM, BN, BK, WM, WN, S, G>::kLdsBytes,                      \
          ridge::PersistentTraits<BM, BN, BK, WM, WN, S, G>::kThreads,                       \
          ridge::PersistentTraits<BM, BN, BK, WM, WN, S, G>::kWaves,                         \
          kPersistent,                                                                       \
          &launchPersistent<BM, BN, BK, WM, WN, S, G>},

const Entry kTable[] = {
#include "gemm_variants.def"
};
#undef RIDGE_VARIANT
#undef RIDGE_VARIANT_PERSISTENT

constexpr int kNumVariants = int(sizeof(kTable) / sizeof(kTable[0]));

bool validIndex(int i) { return i >= 0 && i < kNumVariants; }

}  // namespace

extern "C" {

int ridge_gemm_num_variants(void) { return kNumVariants; }

int ridge_gemm_get_variant(int i, ridge_gemm_variant_t* out) {
    if (!validIndex(i) || out == nullptr) return (int)hipErrorInvalidValue;
    const Entry& e = kTable[i];
    ridge_gemm_variant_t v;
    std::memset(&v, 0, sizeof(v));
    v.BM = e.BM; v.BN = e.BN; v.BK = e.BK; v.WM = e.WM; v.WN = e.WN;
    v.stages = e.stages; v.groupM = e.groupM;
    v.ldsBytes = e.ldsBytes; v.threads = e.threads; v.waves = e.waves;
    v.pingPong = e.schedule == kPingPong ? 1 : 0;
    v.schedule = e.schedule;
    if (i < ridge_gemm_resource_count) {
        const ridge_gemm_resources_t& r = ridge_gemm_resource_table[i];
        v.vgprs = r.vgprs; v.agprs = r.agprs; v.sgprs = r.sgprs;
        v.scratchBytes = r.scratchBytes; v.occupancy = r.occupancy;
        v.regsPerThread = r.vgprs + r.agprs;
    } else {
        v.regsPerThread = -1;
        v.vgprs = v.agprs = v.sgprs = v.scratchBytes = v.occupancy = -1;
    }
    *out = v;
    return 0;
}

int ridge_gemm_find_variant(int BM, int BN, int BK, int WM, int WN, int stages, int groupM) {
    for (int i = 0; i < kNumVariants; ++i) {
        const Entry& e = kTable[i];
        if (e.BM == BM && e.BN == BN && e.BK == BK && e.WM == WM && e.WN == WN && e.stages == stages &&
            e.groupM == groupM)
            return i;
    }
    return -1;
}

int ridge_gemm_divides(int i, int M, int N, int K) {
    if (!validIndex(i)) return 0;
    const Entry& e = kTable[i];
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    if (M % e.BM || N % e.BN || K % e.BK) return 0;
    // The grid is one-dimensional and offsets inside the kernel are 32-bit.
    if ((long long)(M / e.BM) * (N / e.BN) > 0x7fffffffLL) return 0;
    if ((long long)e.BM * K > 0x7fffffffLL || (long long)e.BK * N > 0x7fffffffLL) return 0;
    return 1;
}

int ridge_gemm_launch(int i, const void* A, const void* B, void* C, int M, int N, int K, void* stream) {
    if (!ridge_gemm_divides(i, M, N, K)) return (int)hipErrorInvalidValue;
    if (A == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15u) return (int)hipErrorInvalidValue;
    return (int)kTable[i].launch(A, B, C, M, N, K, static_cast<hipStream_t>(stream));
}

int ridge_gemm_split_rows(int body, int M, int N, int K, int numCUs) {
    if (!validIndex(body) || numCUs <= 0 || !ridge_gemm_divides(body, M, N, K)) return -1;
    ridge_gemm_variant_t v;
    ridge_gemm_get_variant(body, &v);
    // Resident workgroups per CU: LDS, wave slots, and the register file (the
    // compiler's waves per SIMD; a workgroup's waves spread over the 4 SIMDs).
    int perCU = 163840 / v.ldsBytes;
    perCU = std::min(perCU, 32 / v.waves);
    if (v.occupancy > 0) perCU = std::min(perCU, v.occupancy / ((v.waves + 3) / 4));
    if (perCU < 1) return -1;
    const long long slots = (long long)perCU * numCUs;
    const long long perPanel = N / v.BN, panels = M / v.BM;
    const long long rounds = panels * perPanel / slots;
    if (rounds == 0) return 0;
    const long long bodyPanels = rounds * slots / perPanel;
    return bodyPanels >= panels ? M : (int)(bodyPanels * v.BM);
}

int ridge_gemm_launch_split(int body, int tail, int bodyRows, const void* A, const void* B, void* C, int M, int N,
                            int K, void* stream) {
    // Every check before the first launch: a refused call enqueues nothing.
    if (bodyRows <= 0 || bodyRows >= M) return (int)hipErrorInvalidValue;
    if (!ridge_gemm_divides(body, bodyRows, N, K) || !ridge_gemm_divides(tail, M - bodyRows, N, K))
        return (int)hipErrorInvalidValue;
    if (A == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 15u) return (int)hipErrorInvalidValue;
    const char* tailA = static_cast<const char*>(A) + (size_t)bodyRows * K * 2;
    char* tailC = static_cast<char*>(C) + (size_t)bodyRows * N * 2;
    const int rc = ridge_gemm_launch(body, A, B, C, bodyRows, N, K, stream);
    if (rc != 0) return rc;
    return ridge_gemm_launch(tail, tailA, B, tailC, M - bodyRows, N, K, stream);
}

size_t ridge_gemm_variant_table_csv(char* buf, size_t cap) {
    std::string s = "idx,BM,BN,BK,WM,WN,stages,groupM,ldsBytes,threads,regsPerThread,waves,vgprs,agprs,sgprs,"
                    "scratchBytes,occupancy,pingPong,schedule\n";
    char line[256];
    for (int i = 0; i < kNumVariants; ++i) {
        ridge_gemm_variant_t v;
        ridge_gemm_get_variant(i, &v);
        std::snprintf(line, sizeof(line), "%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d\n", i, v.BM,
                      v.BN, v.BK, v.WM, v.WN, v.stages, v.groupM, v.ldsBytes, v.threads, v.regsPerThread, v.waves,
                      v.vgprs, v.agprs, v.sgprs, v.scratchBytes, v.occupancy, v.pingPong, v.schedule);
        s += line;
    }
    if (buf != nullptr && cap > 0) {
        const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
        std::memcpy(buf, s.data(), n);
        buf[n] = '\0';
    }
    return s.size();
}

size_t ridge_gemm_variant_struct_size(void) { return sizeof(ridge_gemm_variant_t); }

const char* ridge_gemm_build_info(void) {
    return "ridge_gemm gfx950 mfma_f32_16x16x32_f16, direct-to-LDS ring, tr16 B reads, xcd+groupM order, "
           "ping-pong schedule for 8-wave rings of 3+ stages, persistent store-behind rows with loader waves";
}

}  // extern "C"
