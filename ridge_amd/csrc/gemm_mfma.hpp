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
//  * LDS -> VGPR: A fragments are one `ds_read_b128` per lane (8 consecutive k of
//    one row). B is stored as it sits in memory (n contiguous); its fragments are
//    read with two `ds_read_b64_tr_b16` per 32x32 tile, the gfx950 transposing
//    LDS read. Within a 16-lane group, lane s = 4j + r points at
//    B[k0 + j][n0 + 4r .. n0 + 4r + 3] and lane i receives B[k0 .. k0 + 3][n0 + i].
//  * MFMA: v_mfma_f32_32x32x16_f16 with the operands swapped (B fragment in the
//    "A" slot), which yields the transposed accumulator: lane l holds
//    C[m0 + l%32][n0 + 8i + 4(l/32) + j] in acc[4i + j]. Four consecutive columns
//    per lane let the epilogue write 8-byte FP16 stores with no LDS round trip.
//  * Workgroup order: the hardware deals workgroups round-robin over the 8 XCDs,
//    each with its own L2. xcdRemap makes the workgroups of one XCD a contiguous
//    range of the logical order, and the GroupM mapping of that logical order
//    (reference gemm-mma.cuh:158-178) then gives each XCD a compact block of
//    output tiles that shares A and B panels in its L2.
//
// Preconditions (checked by the host launcher, never by the kernel): M % BM ==
// N % BN == K % BK == 0 and K >= BK; 16-byte aligned A, B, C.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ridge {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

#define RIDGE_LDS_AS __attribute__((address_space(3)))

// 1: order each k-step's MFMAs and LDS reads with sched_group_barrier hints.
#ifndef RIDGE_GEMM_SCHED
#define RIDGE_GEMM_SCHED 1
#endif

constexpr int kWaveSize = 64;
constexpr int kXcds = 8;
// MFMA instruction shape (v_mfma_f32_32x32x16_f16): 32768 FLOP per instruction.
constexpr int kMfmaM = 32;
constexpr int kMfmaN = 32;
constexpr int kMfmaK = 16;

// ---------------------------------------------------------------------------
// LDS swizzles. Both map a logical 16-byte chunk index to a physical one and are
// involutions (applying one twice is the identity), because the XOR mask depends
// only on bits the XOR does not touch.
// ---------------------------------------------------------------------------

// A tile, [BM][BK] halves, k contiguous, chunk q = row * (BK/8) + c. The mask is
// a function of the 128-byte LDS line q>>3, so a ds_read_b128 in which 8 lanes
// read 8 consecutive rows at one logical chunk hits 8 distinct 16-byte bank
// groups; the `line >> 3` term also keeps 16 consecutive rows distinct within a
// 256-byte window when BK = 64.
__device__ __forceinline__ int swizzleA(int q) {
    const int line = q >> 3;
    return q ^ ((line ^ (line >> 3)) & 7);
}

// B tile, [BK][BN] halves, n contiguous, chunk q = k * (BN/8) + c. A transposing
// read has 16 lanes cover 4 consecutive k rows x 2 chunks (and two groups cover
// 4 rows x 4 chunks). The mask depends on k % 4: {0, 10, 4, 14} makes the 8
// chunks of one group distinct modulo 8 and the 16 chunks of a group pair
// distinct modulo 16; with only 8 chunks per row (BN = 64) it falls back to
// {0, 2, 4, 6}, which must stay below the row length.
template <int CPR_B>
__device__ __forceinline__ int swizzleB(int q) {
    const int k4 = (q / CPR_B) & 3;
    if constexpr (CPR_B >= 16) {
        const int m = (k4 == 0) ? 0 : (k4 == 1) ? 10 : (k4 == 2) ? 4 : 14;
        return q ^ m;
    } else {
        return q ^ (2 * k4);
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

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
struct GemmTraits {
    static constexpr int kWavesM = BM / WM;
    static constexpr int kWavesN = BN / WN;
    static constexpr int kWaves = kWavesM * kWavesN;
    static constexpr int kThreads = kWaves * kWaveSize;
    static constexpr int kTilesM = WM / kMfmaM;   // MFMA tiles per wave along M
    static constexpr int kTilesN = WN / kMfmaN;   // ... along N
    static constexpr int kSteps = BK / kMfmaK;    // MFMA k-steps per K tile
    static constexpr int kChunksPerRowA = BK / 8;
    static constexpr int kChunksPerRowB = BN / 8;
    static constexpr int kBytesA = BM * BK * 2;
    static constexpr int kBytesB = BK * BN * 2;
    static constexpr int kStageBytes = kBytesA + kBytesB;
    static constexpr int kLdsBytes = STAGES * kStageBytes;
    // 64-lane x 16-byte direct-to-LDS instructions per stage, and per wave.
    static constexpr int kInstA = kBytesA / 1024;
    static constexpr int kInstB = kBytesB / 1024;
    static constexpr int kPerWaveA = kInstA / kWaves;
    static constexpr int kPerWaveB = kInstB / kWaves;
    static constexpr int kLoadsPerTile = kPerWaveA + kPerWaveB;

    static_assert(STAGES >= 2, "the ring needs at least two LDS buffers");
    static_assert(BM % WM == 0 && BN % WN == 0, "workgroup tile must split into wave tiles");
    static_assert(WM % kMfmaM == 0 && WN % kMfmaN == 0, "wave tile must split into 32x32 MFMA tiles");
    static_assert(BK % kMfmaK == 0, "BK must be a whole number of MFMA k-steps");
    static_assert(kSteps % 2 == 0, "fragment double-buffering assumes an even number of k-steps");
    static_assert(BK == 32 || BK == 64, "the A swizzle is derived for BK of 32 or 64");
    static_assert(BN == 64 || BN == 128 || BN == 256, "the B swizzle is derived for BN of 64, 128 or 256");
    static_assert(kBytesA % 1024 == 0 && kBytesB % 1024 == 0, "tiles must be whole 1 KiB wave loads");
    static_assert(kInstA % kWaves == 0 && kInstB % kWaves == 0, "loads must split evenly over waves");
    static_assert((STAGES - 1) * kLoadsPerTile < 64, "in-flight loads exceed the vmcnt counter");
    static_assert(kLdsBytes <= 163840, "LDS is 160 KiB per workgroup on gfx950");
};

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int GROUPM>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * kWaveSize)
void gemmMfmaKernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                    _Float16* __restrict__ C, int M, int N, int K) {
    using T = GemmTraits<BM, BN, BK, WM, WN, STAGES, GROUPM>;
    constexpr int TM = T::kTilesM;
    constexpr int TN = T::kTilesN;
    constexpr int CPR_A = T::kChunksPerRowA;
    constexpr int CPR_B = T::kChunksPerRowB;

    __shared__ __attribute__((aligned(1024))) char lds[T::kLdsBytes];

    const int lane = threadIdx.x % kWaveSize;
    // Wave index as a scalar: every lane of a wave agrees, and the LDS base of a
    // direct-to-LDS load must be wave-uniform.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
    const int waveM = wave / T::kWavesN;
    const int waveN = wave % T::kWavesN;

    // Output tile for this workgroup.
    const int numPidM = M / BM;
    const int numPidN = N / BN;
    const int pid = xcdRemap(blockIdx.x, gridDim.x);
    const int pidInGroup = pid % (GROUPM * numPidN);
    const int firstPidM = (pid / (GROUPM * numPidN)) * GROUPM;
    const int groupRows = min(numPidM - firstPidM, GROUPM);
    const int pidM = firstPidM + pidInGroup % groupRows;
    const int pidN = pidInGroup / groupRows;
    const int blockRow = pidM * BM;
    const int blockCol = pidN * BN;

    // Per-lane global element offsets of this wave's direct-to-LDS loads,
    // relative to the tile origin. Wave instruction j fills physical chunks
    // [64 j, 64 j + 64) of a stage; lane t's chunk holds logical chunk
    // swizzle(64 j + t).
    int offA[T::kPerWaveA];
    int offB[T::kPerWaveB];
#pragma unroll
    for (int i = 0; i < T::kPerWaveA; ++i) {
        const int j = i * T::kWaves + wave;
        const int q = swizzleA(j * 64 + lane);
        offA[i] = (q / CPR_A) * K + (q % CPR_A) * 8;
    }
#pragma unroll
    for (int i = 0; i < T::kPerWaveB; ++i) {
        const int j = i * T::kWaves + wave;
        const int q = swizzleB<CPR_B>(j * 64 + lane);
        offB[i] = (q / CPR_B) * N + (q % CPR_B) * 8;
    }
    const _Float16* gA = A + (size_t)blockRow * K;
    const _Float16* gB = B + blockCol;

    auto issueTile = [&](int kTile, int stage) {
        const _Float16* srcA = gA + kTile * BK;
        const _Float16* srcB = gB + (size_t)kTile * BK * N;
        char* dst = lds + stage * T::kStageBytes;
#pragma unroll
        for (int i = 0; i < T::kPerWaveA; ++i) {
            const int j = i * T::kWaves + wave;
            __builtin_amdgcn_global_load_lds((const void*)(srcA + offA[i]),
                                             (RIDGE_LDS_AS void*)(dst + j * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < T::kPerWaveB; ++i) {
            const int j = i * T::kWaves + wave;
            __builtin_amdgcn_global_load_lds((const void*)(srcB + offB[i]),
                                             (RIDGE_LDS_AS void*)(dst + T::kBytesA + j * 1024), 16, 0, 0);
        }
    };

    // Fragment read offsets (bytes, within a stage).
    // A: tile tm, k-step ks: row = waveM*WM + tm*32 + lane%32, chunk = 2 ks + lane/32.
    int rdA[TM][T::kSteps];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int ks = 0; ks < T::kSteps; ++ks) {
            const int row = waveM * WM + tm * kMfmaM + lane % 32;
            rdA[tm][ks] = swizzleA(row * CPR_A + 2 * ks + lane / 32) * 16;
        }
    }
    // B: tile tn, k-step ks, half h: 16-lane group g = lane/16, s = lane%16 reads
    // row 16 ks + 8 (g/2) + 4 h + s/4, columns waveN*WN + 32 tn + 16 (g%2) + 4 (s%4).
    // Rows enter the swizzle only through row % 4 = s/4, so the row term adds
    // outside the XOR as a compile-time offset.
    int rdB[TN];
    {
        const int g = lane / 16;
        const int s = lane % 16;
        const int rowLane = 8 * (g / 2) + s / 4;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const int col = waveN * WN + tn * kMfmaN + 16 * (g % 2) + 4 * (s % 4);
            const int q = swizzleB<CPR_B>(rowLane * CPR_B + col / 8);
            rdB[tn] = T::kBytesA + q * 16 + (col % 8) * 2;
        }
    }

    float16_t acc[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[tm][tn][e] = 0.0f;

    const int numK = K / BK;

    // Operand fragments of one k-step: TM A reads (ds_read_b128) and 2 TN
    // transposing B reads.
    auto readFrags = [&](const char* base, int ks, half8_t (&a)[TM], half8_t (&b)[TN]) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            a[tm] = *(const RIDGE_LDS_AS half8_t*)(base + rdA[tm][ks]);
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const char* p = base + rdB[tn] + ks * 16 * CPR_B * 16;
            const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((RIDGE_LDS_AS short4_t*)(p));
            const short4_t hi =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((RIDGE_LDS_AS short4_t*)(p + 4 * CPR_B * 16));
            const half4_t l4 = __builtin_bit_cast(half4_t, lo);
            const half4_t h4 = __builtin_bit_cast(half4_t, hi);
            b[tn] = half8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
        }
    };
    auto mfmaStep = [&](const half8_t (&a)[TM], const half8_t (&b)[TN]) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[tn], a[tm], acc[tm][tn], 0, 0, 0);
    };
    // Scheduling hint for one k-step: alternate one MFMA with one LDS read so
    // the reads of the next k-step hide under this step's matrix work.
    auto interleave = [&]() {
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
    };

    // Prologue: every stage filled (tiles 0 .. STAGES-1). A tile that does not
    // exist is not issued; the waits count only issued loads, and near the end of
    // K fewer were issued, so those waits drain fully.
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
        if (s < numK) issueTile(s, s);
    }
    if (numK >= STAGES) {
        waitVmcnt<(STAGES - 1) * T::kLoadsPerTile>();
    } else {
        waitVmcnt<0>();
    }
    barrierLds();

    half8_t fa[2][TM];
    half8_t fb[2][TN];
    readFrags(lds, 0, fa[0], fb[0]);

    // Fragments are double-buffered across k-steps (kSteps is even, so the
    // buffer parity is the same in every K tile). The tile boundary sits inside
    // the last k-step: once tile kt+1 has landed and every wave is past its reads
    // of tile kt, the freed stage is refilled with tile kt+STAGES and the first
    // fragments of tile kt+1 are read while the last MFMAs of tile kt run.
    int stage = 0;
    for (int kt = 0; kt < numK; ++kt) {
        const char* base = lds + stage * T::kStageBytes;
        const int nextStage = (stage + 1 == STAGES) ? 0 : stage + 1;
#pragma unroll
        for (int ks = 0; ks < T::kSteps; ++ks) {
            const int cur = ks & 1;
            if (ks + 1 < T::kSteps) {
                readFrags(base, ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
            } else if (kt + 1 < numK) {
                // Tile kt+1 has landed once at most tiles kt+2 .. kt+STAGES-1 are
                // outstanding.
                if (kt + STAGES - 1 < numK) {
                    waitVmcnt<(STAGES - 2) * T::kLoadsPerTile>();
                } else {
                    waitVmcnt<0>();
                }
                // This wave's reads of tile kt completed (lgkmcnt(0)) and every
                // wave arrived, so stage `stage` is free and tile kt+1 is visible.
                barrierLds();
                if (kt + STAGES < numK) issueTile(kt + STAGES, stage);
                readFrags(lds + nextStage * T::kStageBytes, 0, fa[cur ^ 1], fb[cur ^ 1]);
            }
            mfmaStep(fa[cur], fb[cur]);
            interleave();
        }
        stage = nextStage;
    }

    // Epilogue: FP32 -> FP16 (round to nearest even) and 8-byte stores of four
    // consecutive columns. No LDS is touched, so no drain of the ring is needed
    // beyond the final wait inside the loop.
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
        const int m = blockRow + waveM * WM + tm * kMfmaM + lane % 32;
        _Float16* crow = C + (size_t)m * N;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const int n0 = blockCol + waveN * WN + tn * kMfmaN + 4 * (lane / 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                half4_t v;
                v[0] = (_Float16)acc[tm][tn][4 * i + 0];
                v[1] = (_Float16)acc[tm][tn][4 * i + 1];
                v[2] = (_Float16)acc[tm][tn][4 * i + 2];
                v[3] = (_Float16)acc[tm][tn][4 * i + 3];
                *(half4_t*)(crow + n0 + 8 * i) = v;
            }
            // One tile at a time: without this fence the scheduler hoists every
            // accumulator read to the top of the epilogue and runs out of VGPRs.
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

}  // namespace ridge
