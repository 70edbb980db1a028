// gemm_mfma.hpp -- templated FP16 GEMM for gfx950 (MI355X), MFMA with FP32
// accumulate, FP16 output.
//
//   C (M x N, row-major, fp16) = A (M x K, row-major, fp16) * B (K x N, row-major, fp16)
//
// Counterpart of the reference's gemmMmaKernel<BM,BN,BK,WM,WN,Stages,GroupM>
// (bench/kernels/gemm-mma.cuh:116-343): the same template surface, a new
// implementation for CDNA4.
//
// Structure of one workgroup (BM x BN output tile, (BM/WM)*(BN/WN) wavefronts of
// 64 lanes, each owning a WM x WN sub-tile):
//
//  * Global -> LDS: `global_load_lds_dwordx4` moves 16-byte chunks straight into
//    LDS with no VGPR staging. One wave instruction writes 1 KiB of contiguous
//    LDS (lane t at base + 16 t), so the bank-conflict-avoiding layout is made by
//    choosing, per lane, WHICH global chunk lands in each LDS slot: an XOR swizzle
//    on the 16-byte chunk index (swizzleA / swizzleB below). STAGES buffers form
//    a ring; tile kt+STAGES-1 is in flight while tile kt is consumed, and the
//    hand-counted `s_waitcnt vmcnt(n)` + `s_barrier` replaces __syncthreads(),
//    whose fence would drain every outstanding prefetch.
//  * MFMA: v_mfma_f32_16x16x32_f16. At equal cycles per FLOP it draws less power
//    than the 32x32x16 form: under a full-chip stream of each on random operands
//    the loaded clock measured 1.89 GHz against 1.65 GHz. With the GEMM's LDS
//    reads added (probe_mfma_shape.hip) both run at the chip's power ceiling, the
//    smaller one 0.7% slower on one box and 5.5% faster on another.
//  * LDS -> VGPR: an MFMA operand is 8 consecutive k of one row (A) or one column
//    (B) per lane, lane group g = lane/16 holding k = 8g .. 8g+7 and lane%16 the
//    row or column. A fragments are one `ds_read_b128` per lane. B is stored as
//    it sits in memory (n contiguous); its fragments are read with two
//    `ds_read_b64_tr_b16` per 16x32 tile, the gfx950 transposing LDS read: within
//    a 16-lane group, lane s = 4j + r points at B[k0 + j][n0 + 4r .. n0 + 4r + 3]
//    and lane i receives B[k0 .. k0 + 3][n0 + i].
//  * The operands are swapped (B fragment in the instruction's A slot), which
//    yields the transposed accumulator: lane l holds C[m0 + l%16][n0 + 4(l/16) + r]
//    in acc[r]. The epilogue converts those four columns to 8 bytes of FP16 in an
//    LDS staging region and reads whole rows back, so every global store is 16
//    bytes per lane (storeStaged).
//  * Workgroup order: the hardware deals workgroups round-robin over the 8 XCDs,
//    each with its own L2. xcdRemap makes the workgroups of one XCD a contiguous
//    range of the logical order, and the GroupM mapping of that logical order
//    (reference gemm-mma.cuh:158-178) then gives each XCD a compact block of
//    output tiles that shares A and B panels in its L2.
//
// Preconditions (checked by the host launcher, never by the kernel): M % BM ==
// N % BN == K % BK == 0 and K >= BK; BM * K, BK * N and the tile count below 2^31
// (tile offsets are 32-bit); 16-byte aligned A, B, C.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace ridge {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

#define RIDGE_LDS_AS __attribute__((address_space(3)))

// 1: order each k-step's MFMAs and LDS reads with sched_group_barrier hints.
#ifndef RIDGE_GEMM_SCHED
#define RIDGE_GEMM_SCHED 1
#endif

constexpr int kWaveSize = 64;
constexpr int kXcds = 8;
// MFMA instruction shape (v_mfma_f32_16x16x32_f16): 16384 FLOP per instruction.
constexpr int kMfmaM = 16;
constexpr int kMfmaN = 16;
constexpr int kMfmaK = 32;

// ---------------------------------------------------------------------------
// LDS swizzles. Both map a logical 16-byte chunk index to a physical one and are
// involutions (applying one twice is the identity), because the XOR mask depends
// only on bits the XOR does not touch.
// ---------------------------------------------------------------------------

// A tile, [BM][BK] halves, k contiguous, chunk q = row * CPR_A + c with
// CPR_A = BK/8. A fragment read has 16 lanes read 16 consecutive rows at one
// logical chunk, and LDS serves a ds_read_b128 at most 16 lanes (256 bytes)
// at a time, so those 16 chunks must land in 16 distinct 16-byte slots modulo 256
// bytes. For BK of 32 and 64 the mask is a function of the 128-byte LDS line
// q>>3: 8 consecutive rows hit 8 distinct slots, and the `line >> 3` term keeps
// 16 consecutive rows distinct within a 256-byte window when BK = 64. With 16 or
// more chunks per row (BK >= 128) every row starts at slot 0, and XOR-ing the
// chunk with the row modulo 16 gives 16 consecutive rows 16 distinct slots; the
// XOR stays inside the row's aligned group of 16 chunks.
template <int CPR_A>
__device__ __forceinline__ int swizzleA(int q) {
    if constexpr (CPR_A >= 16) {
        return q ^ ((q / CPR_A) & 15);
    } else {
        const int line = q >> 3;
        return q ^ ((line ^ (line >> 3)) & 7);
    }
}

// B tile, [BK][BN] halves, n contiguous, chunk q = k * (BN/8) + c. One
// transposing read has each 16-lane group cover 4 consecutive k rows x 2 chunks,
// the four groups at rows 8g + {0..3} (+ 4 for the second half of a fragment).
// LDS serves these 8-byte reads 32 lanes (256 bytes) at a time, so the 16 chunks
// of a group pair -- rows {r..r+3} and {r+8..r+11}, two chunks each -- must land
// in 16 distinct 16-byte bank slots. The mask 2 * (k%4 + 4 * ((k/8)%2)) gives the
// eight rows eight distinct even offsets, and the chunk pair fills the odd one.
// With only 8 chunks per row (BN = 64) the row's own parity supplies bit 3 of the
// slot, and the mask 2 * ((k/2)%2 + 2 * ((k/8)%2)) separates the rest; it stays
// below the row length. The mask uses k bits 0, 1 and 3 only, so row offsets of
// 4 (fragment half) and 32 (k-step) leave it unchanged.
template <int CPR_B>
__device__ __forceinline__ int swizzleB(int q) {
    const int k = q / CPR_B;
    if constexpr (CPR_B >= 16) {
        return q ^ (2 * ((k & 3) + 4 * ((k >> 3) & 1)));
    } else {
        return q ^ (2 * (((k >> 1) & 1) + 2 * ((k >> 3) & 1)));
    }
}

// Inverse of the hardware's round-robin workgroup-to-XCD dealing: logical ids
// [x*q + min(x,r), ...) run on XCD x, where q = n/8 and r = n%8.
__device__ __forceinline__ int xcdRemap(int pid, int n) {
    const int x = pid % kXcds;
    const int q = n / kXcds;
    const int r = n % kXcds;
    return x * q + (x < r ? x : r) + pid / kXcds;
}

// GroupM launch order: logical id pid -> (row, column) of the output tile's
// first element. Groups of GROUPM tile rows are walked column by column, so
// consecutive ids share B column panels and a group shares A row panels.
template <int BM, int BN, int GROUPM>
__device__ __forceinline__ void tileOf(int pid, int M, int N, int& row, int& col) {
    const int numPidM = M / BM;
    const int numPidN = N / BN;
    const int pidInGroup = pid % (GROUPM * numPidN);
    const int firstPidM = (pid / (GROUPM * numPidN)) * GROUPM;
    const int groupRows = min(numPidM - firstPidM, GROUPM);
    row = (firstPidM + pidInGroup % groupRows) * BM;
    col = (pidInGroup / groupRows) * BN;
}

// Direct-to-LDS 16-byte load: lane t of the wave writes LDS bytes
// [ldsAddr + 16 t, +16) with the 16 bytes at base + offset. base and ldsAddr are
// wave-uniform (scalar registers; ldsAddr is carried in M0), offset is the lane's
// 32-bit byte offset, so issuing a load costs no vector ALU instruction.
//
// Issued through inline asm on purpose. Seen as the builtin, the compiler's
// wait-count pass treats the DMA as an LDS write that may alias later LDS reads
// and puts an `s_waitcnt vmcnt(0)` in front of the transposing B reads, which
// drains every prefetch in flight and serialises the ring. The kernels count
// vmcnt themselves (waitVmcnt) and order LDS with barriers, so the compiler
// needs no view of the DMA. The s_nop covers the M0-write -> LDS-DMA hazard the
// compiler would otherwise insert.
__device__ __forceinline__ void globalLoadLds16(const void* base, uint32_t offset, uint32_t ldsAddr) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(offset), "s"(base), "{m0}"(ldsAddr)
                 : "memory");
}

// LDS byte address of a __shared__ object, as a wave-uniform scalar.
// Byte offset of 16-byte chunk `chunk` of row `row` in an FP16 tile whose rows are
// `ld` elements apart. Unsigned 32-bit arithmetic: the launcher admits only shapes
// with BM * K and BK * N below 2^31, so every tile offset is below 2^32.
__device__ __forceinline__ uint32_t tileOffset(int row, int ld, int chunk) {
    return ((uint32_t)row * (uint32_t)ld + (uint32_t)chunk * 8u) * 2u;
}

__device__ __forceinline__ uint32_t ldsAddress(const void* p) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const RIDGE_LDS_AS char*)(static_cast<const char*>(p)));
}

// s_waitcnt with only the vector-memory counter constrained. The memory clobber
// keeps the compiler from moving LDS or global accesses across it.
template <int N>
__device__ __forceinline__ void waitVmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter on gfx9");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the acquire/release fence of __syncthreads(): this
// wave's LDS accesses are complete (lgkmcnt(0)) and every wave has arrived.
__device__ __forceinline__ void barrierLds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// barrierLds as a phase boundary: the memory clobber orders memory accesses
// only, so without the scheduling barriers the compiler may move register-only
// work (the MFMAs) across the s_barrier within a basic block.
__device__ __forceinline__ void phaseBarrier() {
    __builtin_amdgcn_sched_barrier(0);
    barrierLds();
    __builtin_amdgcn_sched_barrier(0);
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
struct GemmTraits {
    static constexpr int kWavesM = BM / WM;
    static constexpr int kWavesN = BN / WN;
    static constexpr int kWaves = kWavesM * kWavesN;
    static constexpr int kThreads = kWaves * kWaveSize;
    static constexpr int kTilesM = WM / kMfmaM;   // 16x16 MFMA tiles per wave along M
    static constexpr int kTilesN = WN / kMfmaN;   // ... along N
    static constexpr int kSteps = BK / kMfmaK;    // 32-deep MFMA k-steps per K tile
    static constexpr int kChunksPerRowA = BK / 8;
    static constexpr int kChunksPerRowB = BN / 8;
    static constexpr int kBytesA = BM * BK * 2;
    static constexpr int kBytesB = BK * BN * 2;
    static constexpr int kStageBytes = kBytesA + kBytesB;
    static constexpr int kLdsBytes = STAGES * kStageBytes;
    // LDS layout: the A tiles of all stages, then the B tiles of all stages, so a
    // fragment read's stage offset is a small compile-time immediate.
    static constexpr int kRegionA = STAGES * kBytesA;
    // 64-lane x 16-byte direct-to-LDS instructions per stage, and per wave.
    static constexpr int kInstA = kBytesA / 1024;
    static constexpr int kInstB = kBytesB / 1024;
    static constexpr int kPerWaveA = kInstA / kWaves;
    static constexpr int kPerWaveB = kInstB / kWaves;
    static constexpr int kLoadsPerTile = kPerWaveA + kPerWaveB;
    // Byte distance between the k-steps of a B fragment and between its two
    // 4-row halves (k 8g..8g+3 and 8g+4..8g+7).
    static constexpr int kBStepBytes = kMfmaK * BN * 2;
    static constexpr int kBHalfBytes = 4 * BN * 2;

    static_assert(STAGES >= 2, "the ring needs at least two LDS buffers");
    static_assert(BM % WM == 0 && BN % WN == 0, "workgroup tile must split into wave tiles");
    static_assert(WM % kMfmaM == 0 && WN % kMfmaN == 0, "wave tile must split into 16x16 MFMA tiles");
    static_assert(BK % kMfmaK == 0, "BK must be a whole number of MFMA k-steps");
    static_assert(BK == 32 || BK == 64 || BK % 128 == 0, "the A swizzle is derived for BK of 32, 64 or a multiple of 128");
    static_assert(BN == 64 || BN == 128 || BN == 256, "the B swizzle is derived for BN of 64, 128 or 256");
    static_assert(kBytesA % 1024 == 0 && kBytesB % 1024 == 0, "tiles must be whole 1 KiB wave loads");
    static_assert(kInstA % kWaves == 0 && kInstB % kWaves == 0, "loads must split evenly over waves");
    static_assert((STAGES - 1) * kLoadsPerTile < 64, "in-flight loads exceed the vmcnt counter");
    static_assert(kLdsBytes <= 163840, "LDS is 160 KiB per workgroup on gfx950");
};

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1, so loop bodies see
// their index as a compile-time constant.
template <typename F, int... Is>
__device__ __forceinline__ void staticForImpl(F& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void staticFor(F&& f) {
    staticForImpl(f, std::make_integer_sequence<int, N>{});
}

// Epilogue of one wave through a private LDS region. In the MFMA layout a lane
// holds four consecutive columns of one row, so direct stores are 8 bytes wide
// and one wave instruction touches 16 rows x 32 bytes; at small K, where writing
// C is the whole cost, that pattern runs at 2.9 TB/s against 4.1 TB/s for
// full-row 16-byte stores. So the wave converts its TM x TN tiles to FP16
// (nearest even), writes EPI 16-row tile-rows at a time into `region`
// (16 * EPI * WN * 2 bytes) and reads them back row by row: every lane then
// stores 16 contiguous bytes and one instruction covers 64 / (WN / 8) complete
// rows of the wave tile. Row r of the region keeps its chunks XOR-permuted by
// (r * CPR / 16) % CPR: the 8-byte writes (16 rows at one chunk per 32 lanes)
// and the 16-byte reads (8 lanes along a row) are both conflict-free. Up to 8
// read-backs are in flight before their stores issue. The global stores are
// not waited for; NT marks them non-temporal (streamed past the caches), which
// lifts a C-bound kernel's write rate when C is not re-read soon.
template <int TM, int TN, int WN, int EPI, bool NT>
__device__ __forceinline__ void storeStaged(const float4_t (&acc)[TM][TN], RIDGE_LDS_AS char* region,
                                            _Float16* cWave, int N, int lane) {
    constexpr int CPR = WN / 8;            // 16-byte chunks per wave-tile row
    constexpr int kRowsPerStore = 64 / CPR;
    constexpr int kStores = 16 * EPI / kRowsPerStore;   // store instructions per pass
    constexpr int kBatch = kStores < 8 ? kStores : 8;
    static_assert(TM % EPI == 0, "passes must cover the wave tile");
    static_assert(kStores % kBatch == 0, "read-back batches must cover the pass");
    auto swz = [](int row, int chunk) { return chunk ^ ((row * CPR / 16) % CPR); };
    const int g = lane / 16;
    const int r16 = lane % 16;
    staticFor<TM / EPI>([&](auto passC) {
        constexpr int tm0 = passC.value * EPI;
#pragma unroll
        for (int i = 0; i < EPI; ++i) {
            const int row = 16 * i + r16;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int col = tn * kMfmaN + 4 * g;
                half4_t v;
                v[0] = (_Float16)acc[tm0 + i][tn][0];
                v[1] = (_Float16)acc[tm0 + i][tn][1];
                v[2] = (_Float16)acc[tm0 + i][tn][2];
                v[3] = (_Float16)acc[tm0 + i][tn][3];
                *(RIDGE_LDS_AS half4_t*)(region + (row * CPR + swz(row, col / 8)) * 16 + (col % 8) * 2) = v;
            }
        }
        // The region was written by this wave only; wait for the writes
        // before reading them back.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int j0 = 0; j0 < kStores; j0 += kBatch) {
            half8_t v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int row = (j0 + j) * kRowsPerStore + lane / CPR;
                v[j] = *(const RIDGE_LDS_AS half8_t*)(region + (row * CPR + swz(row, lane % CPR)) * 16);
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int row = (j0 + j) * kRowsPerStore + lane / CPR;
                half8_t* dst = (half8_t*)(cWave + (size_t)(16 * tm0 + row) * N + 8 * (lane % CPR));
                if constexpr (NT) {
                    __builtin_nontemporal_store(v[j], dst);
                } else {
                    *dst = v[j];
                }
            }
        }
        // The next pass rewrites the region: its reads must have returned.
        if (passC.value + 1 < TM / EPI) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    });
}

// Per-workgroup state and the operations both schedules are built from: the
// output tile, the direct-to-LDS refill of a stage, the fragment reads of a
// k-step, the MFMAs of a k-step and the epilogue.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
struct GemmBlock {
    using T = GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    static constexpr int TM = T::kTilesM;
    static constexpr int TN = T::kTilesN;
    static constexpr int KS = T::kSteps;
    static constexpr int CPR_A = T::kChunksPerRowA;
    static constexpr int CPR_B = T::kChunksPerRowB;

    const char* lds;      // the workgroup's LDS array (generic pointer to it)
    uint32_t ldsBase;     // its LDS byte address (scalar)
    int lane, wave, waveM, waveN;
    int blockRow, blockCol;
    const _Float16* baseA;
    const _Float16* baseB;
    const char* gA;       // A + blockRow * K (bytes), scalar
    const char* gB;       // B + blockCol (bytes), scalar
    size_t tileStrideB;   // bytes between K tiles of B: BK * N * 2
    uint32_t offA[T::kPerWaveA];  // lane byte offsets of this wave's loads
    uint32_t offB[T::kPerWaveB];
    int rdA[TM][KS];      // A fragment byte offsets within an A tile
    int rdB[TN];          // B fragment byte offsets within the B region
    float4_t acc[TM][TN];
    int numKTiles;        // K / BK
    int kStart = 0;       // first K tile of the loop of issueTile<true>, which wraps

    __device__ __forceinline__ GemmBlock(const char* ldsArray, const _Float16* A, const _Float16* B, int M,
                                         int N, int K) {
        lds = ldsArray;
        ldsBase = ldsAddress(ldsArray);
        lane = threadIdx.x % kWaveSize;
        // Wave index as a scalar: every lane agrees, and load bases must be uniform.
        wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
        waveM = wave / T::kWavesN;
        waveN = wave % T::kWavesN;

        baseA = A;
        baseB = B;
        setTile(xcdRemap(blockIdx.x, gridDim.x), M, N, K);
        tileStrideB = (size_t)BK * N * 2;
        numKTiles = K / BK;
        // Wave instruction j fills physical chunks [64 j, 64 j + 64) of a tile;
        // lane t's chunk holds logical chunk swizzle(64 j + t).
#pragma unroll
        for (int i = 0; i < T::kPerWaveA; ++i) {
            const int q = swizzleA<CPR_A>((i * T::kWaves + wave) * 64 + lane);
            offA[i] = tileOffset(q / CPR_A, K, q % CPR_A);
        }
#pragma unroll
        for (int i = 0; i < T::kPerWaveB; ++i) {
            const int q = swizzleB<CPR_B>((i * T::kWaves + wave) * 64 + lane);
            offB[i] = tileOffset(q / CPR_B, N, q % CPR_B);
        }
        // A fragment of tile tm, k-step ks: row waveM*WM + 16 tm + lane%16,
        // logical chunk 4 ks + lane/16 (k = 32 ks + 8 (lane/16) .. +7).
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                rdA[tm][ks] = swizzleA<CPR_A>((waveM * WM + tm * kMfmaM + lane % 16) * CPR_A + 4 * ks + lane / 16) * 16;
        // B fragment of tile tn: 16-lane group g = lane/16, s = lane%16 reads row
        // 8 g + s/4 (+32 ks + 4 h), columns waveN*WN + 16 tn + 4 (s%4). The
        // swizzle sees rows only through bits 0, 1 and 3, all set per lane here,
        // so k-step and half offsets stay outside the XOR as compile-time
        // immediates.
        {
            const int g = lane / 16;
            const int s = lane % 16;
            const int rowLane = 8 * g + s / 4;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int col = waveN * WN + tn * kMfmaN + 4 * (s % 4);
                rdB[tn] = T::kRegionA + swizzleB<CPR_B>(rowLane * CPR_B + col / 8) * 16 + (col % 8) * 2;
            }
        }
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[tm][tn][e] = 0.0f;
    }

    // The output tile of logical launch id `pid` (after the XCD remap) in the
    // GroupM launch order (reference gemm-mma.cuh:158-178), and its operand bases.
    __device__ __forceinline__ void setTile(int pid, int M, int N, int K) {
        tileOf<BM, BN, GROUPM>(pid, M, N, blockRow, blockCol);
        gA = reinterpret_cast<const char*>(baseA + (size_t)blockRow * K);
        gB = reinterpret_cast<const char*>(baseB + blockCol);
    }

    // Refills LDS stage `stage` with K tile kTile (this wave's share). No vector
    // ALU work: scalar tile bases, constant lane offsets, M0 from scalars. With
    // STAGGERED the loop's K tile kTile is the matrix's K tile (kStart + kTile)
    // mod K/BK.
    template <bool STAGGERED = false>
    __device__ __forceinline__ void issueTile(int kTile, int stage) const {
        if constexpr (STAGGERED) {
            kTile += kStart;
            if (kTile >= numKTiles) kTile -= numKTiles;
        }
        const char* srcA = gA + (size_t)kTile * BK * 2;
        const char* srcB = gB + (size_t)kTile * tileStrideB;
        const uint32_t dstA = ldsBase + stage * T::kBytesA;
        const uint32_t dstB = ldsBase + T::kRegionA + stage * T::kBytesB;
#pragma unroll
        for (int i = 0; i < T::kPerWaveA; ++i) globalLoadLds16(srcA, offA[i], dstA + (i * T::kWaves + wave) * 1024);
#pragma unroll
        for (int i = 0; i < T::kPerWaveB; ++i) globalLoadLds16(srcB, offB[i], dstB + (i * T::kWaves + wave) * 1024);
    }

    // Fragments of k-step ks of the tile in LDS stage STAGE (compile-time, so the
    // stage offset folds into the DS instruction's immediate).
    template <int STAGE>
    __device__ __forceinline__ void readFrags(int ks, half8_t (&a)[TM], half8_t (&b)[TN]) const {
        const RIDGE_LDS_AS char* l = (const RIDGE_LDS_AS char*)(lds);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
            a[tm] = *(const RIDGE_LDS_AS half8_t*)(l + rdA[tm][ks] + STAGE * T::kBytesA);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const RIDGE_LDS_AS char* p = l + rdB[tn] + STAGE * T::kBytesB + ks * T::kBStepBytes;
            const half4_t l4 = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                               (RIDGE_LDS_AS short4_t*)(p)));
            const half4_t h4 = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                               (RIDGE_LDS_AS short4_t*)(p + T::kBHalfBytes)));
            b[tn] = half8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
        }
    }

    // One k-step of MFMAs, B fragment in the first operand (transposed C tile).
    // B outer, A inner: consecutive MFMAs share their first operand (measured
    // slightly faster than sharing the second). The A order snakes (ascending
    // for even tn, descending for odd), so at each change of B the second
    // operand stays too: one operand switch fewer per B column, measured
    // +0.3-0.6% on the power-limited 256x256 rows. Each accumulator still
    // receives its k contributions in order, so the result does not depend on
    // this order.
    __device__ __forceinline__ void mfmaStep(const half8_t (&a)[TM], const half8_t (&b)[TN]) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int tm = (tn & 1) ? TM - 1 - i : i;
                acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[tn], a[tm], acc[tm][tn], 0, 0, 0);
            }
    }

    // Epilogue through LDS (storeStaged below). Regions are per wave, so the
    // only cross-wave hazard is the ring they overlay: every wave must be past
    // its last ring read (a barrier) before the call. Waves whose whole tile does
    // not fit the ring at once make several passes of kEpiTiles 16-row tile-rows.
    static constexpr int epiTiles() {
        int p = TM;
        while (p > 1 && (TM % p != 0 || T::kWaves * 16 * p * WN * 2 > T::kLdsBytes)) --p;
        return p;
    }
    static constexpr int kEpiTiles = epiTiles();
    static constexpr int kEpiRegionBytes = 16 * kEpiTiles * WN * 2;
    static_assert(T::kWaves * kEpiRegionBytes <= T::kLdsBytes, "epilogue regions must fit the ring");

    // This wave's sub-tile of C (row-major, leading dimension N).
    __device__ __forceinline__ _Float16* waveC(_Float16* C, int N) const {
        return C + (size_t)(blockRow + waveM * WM) * N + blockCol + waveN * WN;
    }

    // Regular (cached) stores: these kernels are timed, like the reference's,
    // on operands re-used across launches, where C stays in the MALL.
    __device__ __forceinline__ void store(_Float16* C, int N) const {
        RIDGE_LDS_AS char* region = (RIDGE_LDS_AS char*)(const_cast<char*>(lds)) + wave * kEpiRegionBytes;
        storeStaged<TM, TN, WN, kEpiTiles, false>(acc, region, waveC(C, N), N, lane);
    }
};

// Scheduling hint for one k-step of the uniform schedule: alternate one MFMA
// with one LDS read so the reads of the next k-step hide under this step.
template <int TM, int TN>
__device__ __forceinline__ void interleaveHint() {
#if RIDGE_GEMM_SCHED
    constexpr int kMfmas = TM * TN;
    constexpr int kReads = TM + 2 * TN;
#pragma unroll
    for (int i = 0; i < kMfmas; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if (kReads > kMfmas) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kMfmas, 0);
#endif
}

// ---------------------------------------------------------------------------
// Uniform schedule: every wavefront runs the same phase at the same time.
// Fragments are double-buffered across k-steps; the tile boundary sits inside
// the last k-step of a tile: once tile kt+1 has landed and every wave is past
// its reads of tile kt, the freed stage is refilled with tile kt+STAGES and
// tile kt+1's first fragments are read while tile kt's last MFMAs run.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * kWaveSize)
void gemmMfmaKernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                    _Float16* __restrict__ C, int M, int N, int K) {
    using T = GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    using Blk = GemmBlock<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = T::kLoadsPerTile;

    __shared__ __attribute__((aligned(1024))) char lds[T::kLdsBytes];
    Blk blk(lds, A, B, M, N, K);
    const int numK = K / BK;
    // K stagger for the short K loops of 4-wave BK >= 64 rows: each workgroup
    // starts its K loop at K tile (tile row + tile column) mod K/BK and wraps.
    // Cold, when the first touch of every K slice comes from HBM, workgroups in
    // lockstep all request the same K slice of their panels at once (A's slice
    // strided by a row); staggered, they request different slices. Measured at
    // 1024^3 and 2048 x 2048 x 1024: 5-16% faster cold, between 1.6% slower and
    // 3% faster warm. Not taken where it measured worse: BK = 32 rows (up to 6%
    // slower warm), 8-wave rows (256 x 256 x 64 s2 2% slower at 4096 x 4096 x
    // 2048, whose panels outgrow the L2 once the workgroups drift apart), and
    // long K loops, which gained nothing. Only the summation order of the K tiles
    // changes.
    constexpr bool kStagger = BK >= 64 && T::kWaves <= 4;
    if constexpr (kStagger) {
        if (numK <= 32) blk.kStart = (blk.blockRow / BM + blk.blockCol / BN) % numK;
    }

    // Prologue: every stage filled; a tile that does not exist is not issued,
    // and the waits count only issued loads (near the end of K they drain fully).
    staticFor<STAGES>([&](auto sC) {
        if (sC.value < numK) blk.template issueTile<kStagger>(sC.value, sC.value);
    });
    if (numK >= STAGES) {
        waitVmcnt<(STAGES - 1) * L>();
    } else {
        waitVmcnt<0>();
    }
    barrierLds();

    half8_t fa[2][TM];
    half8_t fb[2][TN];
    blk.template readFrags<0>(0, fa[0], fb[0]);

    // Fragment buffers alternate per k-step across tile boundaries. One pass of
    // the loop covers U tiles, a whole number of ring turns with an even number
    // of k-steps, so every buffer index and stage number is a compile-time
    // constant. Passes whose every tile has its successor and its refill tile
    // (kt0 + U - 1 + STAGES < numK) run first with those tests compiled out, so
    // the steady passes carry no scalar branch; the last passes take the
    // general form. Both forms issue the same loads, barriers and MFMAs
    // (measured 4-9% faster on most 4-wave rows, within 1% on the others).
    constexpr int U = (STAGES * KS) % 2 == 0 ? STAGES : 2 * STAGES;
    auto pass = [&](int kt0, auto steadyC) {
        constexpr bool steady = steadyC.value;
        staticFor<U>([&](auto iC) {
            constexpr int i = iC.value;
            constexpr int s = i % STAGES;
            constexpr int sNext = (s + 1) % STAGES;
            const int kt = kt0 + i;
            if (steady || kt < numK) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int cur = (i * KS + ks) & 1;
                    if (ks + 1 < KS) {
                        blk.template readFrags<s>(ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
                    } else if (steady || kt + 1 < numK) {
                        // Tile kt+1 has landed once at most tiles kt+2 .. kt+STAGES-1
                        // are outstanding.
                        if (steady || kt + STAGES - 1 < numK) {
                            waitVmcnt<(STAGES - 2) * L>();
                        } else {
                            waitVmcnt<0>();
                        }
                        // This wave's reads of tile kt are complete (lgkmcnt(0)) and
                        // every wave arrived: stage s is free and tile kt+1 visible.
                        barrierLds();
                        if (steady || kt + STAGES < numK) blk.template issueTile<kStagger>(kt + STAGES, s);
                        blk.template readFrags<sNext>(0, fa[cur ^ 1], fb[cur ^ 1]);
                    }
                    blk.mfmaStep(fa[cur], fb[cur]);
                    interleaveHint<TM, TN>();
                }
            }
        });
    };
    // The 8-wave rows (two stages, 256 registers per lane) keep the general form
    // only: the second copy of the loop made them spill.
    int kt0 = 0;
    if constexpr (T::kWaves <= 4) {
        for (; kt0 + U - 1 + STAGES < numK; kt0 += U) pass(kt0, std::true_type{});
    }
    for (; kt0 < numK; kt0 += U) pass(kt0, std::false_type{});
    // Every wave is past its last ring read before the epilogue reuses LDS.
    barrierLds();
    blk.store(C, N);
}

// ---------------------------------------------------------------------------
// Ping-pong schedule for 8-wavefront workgroups (two wavefronts per SIMD).
//
// Waves 0-3 (group 0) and 4-7 (group 1) land one per SIMD each (wave w and
// w + 4 share a SIMD, probed with HW_ID). Both run the same body per K tile
//     M-phase: refill this wave's share of the stage freed by tile kt-1 with
//              tile kt+STAGES-1; read all of tile kt's fragments into VGPRs
//     barrier
//     C-phase: all MFMAs of tile kt
//     barrier
// with group 1 one barrier behind, so on every SIMD one wave is in its matrix
// phase while the other is in its memory phase. Every barrier is executed by all
// eight waves (group 0 adds one at the end to match group 1's extra one at the
// start). No wave priority is raised for the matrix phase: the pipe accepts one
// MFMA every 16 cycles, and round-robin issue lets the memory phase's LDS and
// global instructions go out in between (raising the matrix phase to priority
// 1 or 3 measured 1-1.3% slower).
//
// Hazards, with phases p = 0, 1, ...: group 0 reads tile t at p = 2t, group 1 at
// p = 2t+1.
//  * WAR: tile t+STAGES-1 overwrites the stage of tile t-1 and is issued at
//    p = 2t (group 0) or 2t+1 (group 1), after both groups read tile t-1.
//  * RAW: tile t+1 must be in LDS before barrier (2t+1 | 2t+2). Group 0 reaches
//    it at the end of its C-phase and group 1 at the end of its M-phase; each
//    waits there until at most tiles t+2 .. t+STAGES-1 of its own loads are
//    outstanding.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * kWaveSize)
void gemmMfmaPingPongKernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                            _Float16* __restrict__ C, int M, int N, int K) {
    using T = GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    using Blk = GemmBlock<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    static_assert(T::kWaves == 8, "ping-pong pairs two groups of four wavefronts");
    static_assert(STAGES >= 3, "ping-pong refills one tile ahead of two in flight");
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = T::kLoadsPerTile;

    __shared__ __attribute__((aligned(1024))) char lds[T::kLdsBytes];
    Blk blk(lds, A, B, M, N, K);
    const int group = blk.wave / 4;
    const int numK = K / BK;

    staticFor<STAGES - 1>([&](auto sC) {
        if (sC.value < numK) blk.issueTile(sC.value, sC.value);
    });
    if (numK >= STAGES - 1) {
        waitVmcnt<(STAGES - 2) * L>();
    } else {
        waitVmcnt<0>();
    }
    barrierLds();

    // One K tile of group GROUP in ring stage s. `steady`: the refill tile
    // kt+STAGES-1 exists.
    auto tileBody = [&](auto sC, auto groupC, int kt, bool steady) {
        constexpr int s = sC.value;
        constexpr int sRefill = (s + STAGES - 1) % STAGES;
        constexpr int grp = groupC.value;
        // M-phase.
        if (steady) blk.issueTile(kt + STAGES - 1, sRefill);
        half8_t fa[KS][TM];
        half8_t fb[KS][TN];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) blk.template readFrags<s>(ks, fa[ks], fb[ks]);
        if constexpr (grp == 1) {
            if (steady) waitVmcnt<(STAGES - 2) * L>();
            else waitVmcnt<0>();
        }
        phaseBarrier();
        // C-phase.
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) blk.mfmaStep(fa[ks], fb[ks]);
        if constexpr (grp == 0) {
            if (steady) waitVmcnt<(STAGES - 2) * L>();
            else waitVmcnt<0>();
        }
        phaseBarrier();
    };
    // Each group runs its own copy of the K loop with its group a compile-time
    // constant. Whole ring turns whose every tile is steady (kt0 + 2 STAGES - 2 <
    // numK) run first with no per-tile test; the last turns take the general
    // form. The barrier sequence and the arithmetic are those of one loop with
    // run-time tests; only the scalar branches leave the steady turns, each of
    // which sat between an MFMA phase and its barrier, on the ping-pong's
    // critical path (measured 1.8-2.8% faster at 4096^3 and 8192^3, 5% at
    // 2048^3, bit-identical C). phaseBarrier keeps each phase's MFMAs on their
    // side of its barriers once no branch does.
    auto runGroup = [&](auto groupC) {
        constexpr int grp = groupC.value;
        if constexpr (grp == 1) barrierLds();
        int kt0 = 0;
        for (; kt0 + 2 * STAGES - 2 < numK; kt0 += STAGES)
            staticFor<STAGES>([&](auto sC) { tileBody(sC, groupC, kt0 + sC.value, true); });
        for (; kt0 < numK; kt0 += STAGES)
            staticFor<STAGES>([&](auto sC) {
                const int kt = kt0 + sC.value;
                if (kt < numK) tileBody(sC, groupC, kt, kt + STAGES - 1 < numK);
            });
        // Group 0's extra barrier matches group 1's at the start: after it every
        // wave is past its last ring read, and the epilogue may reuse LDS.
        if constexpr (grp == 0) barrierLds();
    };
    if (group == 0) {
        runGroup(std::integral_constant<int, 0>{});
    } else {
        runGroup(std::integral_constant<int, 1>{});
    }
    blk.store(C, N);
}

// ---------------------------------------------------------------------------
// Persistent store-behind schedule, for shapes whose cost is writing C (small K).
//
// One workgroup per CU slot walks the output tiles r, r + grid, r + 2 grid, ...
// of its logical id r (XCD remap, then GroupM order, as above), so at round j
// each XCD works on a compact block of grid / 8 tiles (32 on a 256-CU grid). The
// workgroup has two kinds of wavefronts:
//  * compute waves 0 .. kWaves-1 (the tile's wave grid) read fragments, run the
//    MFMAs and, after a tile's last K tile, convert and store it through a
//    private LDS staging region (storeStaged). They issue no global loads, so
//    their global stores are never waited for: a tile's C drains to memory
//    while the next tile is loaded and multiplied.
//  * loader waves kWaves .. kWaves+kLoaders-1 only issue direct-to-LDS loads.
//    They stream the workgroup's K tiles, in order across output tiles, into
//    an LDS ring of STAGES buffers, and each waits on its own vmcnt, which
//    holds nothing but its loads.
// (On gfx9 one wave's loads and stores share vmcnt and may complete out of
// order, so a wave that both prefetches and stores cannot wait for a load
// without draining its stores; the split keeps the two streams in different
// waves.)
//
// With g = 0, 1, ... the workgroup's K tiles in order, barrier B_g separates
// the compute waves' last reads of K tile g-1 from their first reads of K tile
// g. The loader arrives at B_g only once K tile g is in LDS, and after B_g
// refills the stage of K tile g-1 with K tile g+STAGES-1. Every wave executes
// B_0 .. B_{G-1}, G barriers in all.
// ---------------------------------------------------------------------------
constexpr int kPersistentLoaders = 2;

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
struct PersistentTraits {
    using T = GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    static constexpr int kLoaders = kPersistentLoaders;
    static constexpr int kWaves = T::kWaves + kLoaders;
    static constexpr int kThreads = kWaves * kWaveSize;
    static constexpr int kLoadsA = T::kInstA / kLoaders;   // per loader wave per K tile
    static constexpr int kLoadsB = T::kInstB / kLoaders;
    static constexpr int kLoads = kLoadsA + kLoadsB;
    // Staging: the largest number of 16-row tile-rows per pass that fits
    // beside the ring.
    static constexpr int epiTiles() {
        int p = T::kTilesM;
        while (p > 1 && (T::kTilesM % p != 0 || T::kLdsBytes + T::kWaves * 16 * p * WN * 2 > 163840)) --p;
        return p;
    }
    static constexpr int kEpiTiles = epiTiles();
    static constexpr int kRegionBytes = 16 * kEpiTiles * WN * 2;
    static constexpr int kLdsBytes = T::kLdsBytes + T::kWaves * kRegionBytes;
    static_assert(T::kInstA % kLoaders == 0 && T::kInstB % kLoaders == 0, "loads must split over the loaders");
    static_assert((STAGES - 1) * kLoads < 64, "a loader's in-flight loads exceed the vmcnt counter");
    static_assert(kLdsBytes <= 163840, "ring and staging exceed the 160 KiB of LDS");
};

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
__global__ __launch_bounds__(((BM / WM) * (BN / WN) + kPersistentLoaders) * kWaveSize)
void gemmMfmaPersistentKernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                              _Float16* __restrict__ C, int M, int N, int K) {
    using T = GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    using P = PersistentTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    using Blk = GemmBlock<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int KS = T::kSteps;
    constexpr int L = P::kLoads;

    __shared__ __attribute__((aligned(1024))) char lds[P::kLdsBytes];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const int lane = threadIdx.x % kWaveSize;
    const int grid = gridDim.x;
    const int self = xcdRemap(blockIdx.x, grid);
    const int numTiles = (M / BM) * (N / BN);
    const int numK = K / BK;
    // The launcher makes grid <= numTiles, so every workgroup has a tile.
    const int G = ((numTiles - self + grid - 1) / grid) * numK;

    if (wave >= T::kWaves) {
        // Loader wave l issues wave instructions l, l + kLoaders, ... of each
        // tile; instruction j fills physical chunks [64 j, 64 j + 64).
        const int l = wave - T::kWaves;
        const uint32_t ldsBase = ldsAddress(lds);
        uint32_t offA[P::kLoadsA], offB[P::kLoadsB];
#pragma unroll
        for (int i = 0; i < P::kLoadsA; ++i) {
            const int q = swizzleA<T::kChunksPerRowA>((i * P::kLoaders + l) * 64 + lane);
            offA[i] = tileOffset(q / T::kChunksPerRowA, K, q % T::kChunksPerRowA);
        }
#pragma unroll
        for (int i = 0; i < P::kLoadsB; ++i) {
            const int q = swizzleB<T::kChunksPerRowB>((i * P::kLoaders + l) * 64 + lane);
            offB[i] = tileOffset(q / T::kChunksPerRowB, N, q % T::kChunksPerRowB);
        }
        // K tiles are issued in a fixed order, so a cursor (output tile, K
        // tile) replaces per-issue index arithmetic. An output tile's K loop
        // starts at K tile (row panel) mod numK and wraps: the workgroups
        // streaming different row panels of A then read different 2 * BK-byte
        // columns of their rows at any moment instead of the same one, which
        // spreads the reads over the HBM channels (measured +16% to +19% at
        // 16384 x 128 x 8192 with A streamed from HBM). The two column tiles of
        // a row panel keep one order and share A in L2. Only the summation order
        // of the K tiles changes.
        int curTile = 0, curK = 0, row, col;
        tileOf<BM, BN, GROUPM>(self, M, N, row, col);
        const size_t strideB = (size_t)BK * N * 2;
        const char* srcA = reinterpret_cast<const char*>(A + (size_t)row * K);
        const char* srcB = reinterpret_cast<const char*>(B + col);
        int kIdx = (row / BM) % numK;
        uint32_t kOffA = (uint32_t)kIdx * BK * 2;
        size_t kOffB = (size_t)kIdx * strideB;
        auto issueNext = [&](int stage) {
            // Opaque per call, so the per-stage M0 values are formed here
            // instead of being hoisted out of the loop into scalar registers
            // (which ran the deeper rings out of SGPRs).
            uint32_t lb = ldsBase;
            asm volatile("" : "+s"(lb));
            const uint32_t dstA = lb + stage * T::kBytesA;
            const uint32_t dstB = lb + T::kRegionA + stage * T::kBytesB;
            const char* tA = srcA + kOffA;
            const char* tB = srcB + kOffB;
#pragma unroll
            for (int i = 0; i < P::kLoadsA; ++i)
                globalLoadLds16(tA, offA[i], dstA + (i * P::kLoaders + l) * 1024);
#pragma unroll
            for (int i = 0; i < P::kLoadsB; ++i)
                globalLoadLds16(tB, offB[i], dstB + (i * P::kLoaders + l) * 1024);
            kOffA += BK * 2;
            kOffB += strideB;
            if (++kIdx == numK) {
                kIdx = 0;
                kOffA = 0;
                kOffB = 0;
            }
            if (++curK == numK && ++curTile * numK < G) {
                curK = 0;
                tileOf<BM, BN, GROUPM>(self + curTile * grid, M, N, row, col);
                srcA = reinterpret_cast<const char*>(A + (size_t)row * K);
                srcB = reinterpret_cast<const char*>(B + col);
                kIdx = (row / BM) % numK;
                kOffA = (uint32_t)kIdx * BK * 2;
                kOffB = (size_t)kIdx * strideB;
            }
        };
        staticFor<STAGES - 1>([&](auto sC) {
            if (sC.value < G) issueNext(sC.value);
        });
        if (G >= STAGES - 1) {
            waitVmcnt<(STAGES - 2) * L>();
        } else {
            waitVmcnt<0>();
        }
        barrierLds();  // B_0
        // Turns whose every K tile has its refill tile run with the tests
        // compiled out (g0 + 2 STAGES - 2 < G); the last turns take the general
        // form.
        auto turn = [&](int g0, auto steadyC) {
            constexpr bool steady = steadyC.value;
            staticFor<STAGES>([&](auto sC) {
                constexpr int s = sC.value;
                const int g = g0 + s;
                if (steady || g + 1 < G) {
                    // Past B_g: the stage of K tile g-1 is free.
                    if (steady || g + STAGES - 1 < G) {
                        issueNext((s + STAGES - 1) % STAGES);  // K tile g+STAGES-1
                        waitVmcnt<(STAGES - 2) * L>();
                    } else {
                        waitVmcnt<0>();
                    }
                    barrierLds();  // B_{g+1}: K tile g+1 is in LDS
                }
            });
        };
        int g0 = 0;
        for (; g0 + 2 * STAGES - 2 < G; g0 += STAGES) turn(g0, std::true_type{});
        for (; g0 < G; g0 += STAGES) turn(g0, std::false_type{});
        return;
    }

    Blk blk(lds, A, B, M, N, K);
    RIDGE_LDS_AS char* region = (RIDGE_LDS_AS char*)(lds) + T::kLdsBytes + wave * P::kRegionBytes;
    barrierLds();  // B_0
    half8_t fa[2][TM];
    half8_t fb[2][TN];
    blk.template readFrags<0>(0, fa[0], fb[0]);
    int kt = 0;
    int tile = 0;
    constexpr int U = (STAGES * KS) % 2 == 0 ? STAGES : 2 * STAGES;
    // Passes whose every K tile has a successor (g0 + U < G) run with that test
    // compiled out; the last passes take the general form (measured 7-8% faster
    // at K = 1024 and 8192 on square grids, within 1% on the reported HBM-bound
    // rows, 4% slower for 128x64x64 s6 at 16384 x 128 x 8192). The 8-compute-wave
    // rows (168 registers per lane at 10 waves) keep the general form only: the
    // second copy of the loop made them spill.
    auto pass = [&](int g0, auto steadyC) {
        constexpr bool steady = steadyC.value;
        staticFor<U>([&](auto iC) {
            constexpr int i = iC.value;
            constexpr int s = i % STAGES;
            constexpr int sNext = (s + 1) % STAGES;
            const int g = g0 + i;
            if (steady || g < G) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int cur = (i * KS + ks) & 1;
                    if (ks + 1 < KS) {
                        blk.template readFrags<s>(ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
                    } else if (steady || g + 1 < G) {
                        barrierLds();  // B_{g+1}
                        blk.template readFrags<sNext>(0, fa[cur ^ 1], fb[cur ^ 1]);
                    }
                    blk.mfmaStep(fa[cur], fb[cur]);
                    interleaveHint<TM, TN>();
                }
                if (++kt == numK) {
                    blk.setTile(self + tile * grid, M, N, K);
                    // Non-temporal: measured +21% cold and +1% warm at 8192^2 x 128.
                    storeStaged<TM, TN, WN, P::kEpiTiles, true>(blk.acc, region, blk.waveC(C, N), N, lane);
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
        });
    };
    int g0 = 0;
    if constexpr (T::kWaves <= 4) {
        for (; g0 + U < G; g0 += U) pass(g0, std::true_type{});
    }
    for (; g0 < G; g0 += U) pass(g0, std::false_type{});
}

}  // namespace ridge
