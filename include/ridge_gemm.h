/*
 * ridge_gemm.h -- C ABI of the MI355X (gfx950) FP16 GEMM kernel table.
 *
 * This is the drop-in for the reference's kernel table, the operator API the
 * correctness check, the measurement sweep and the autotuner drive:
 *
 *   struct KernelVariant { int BM, BN, BK, WM, WN, stages, groupM, smemBytes,
 *       threads, regsPerThread; cudaError_t (*launch)(A, B, C, M, N, K, stream); };
 *   int numVariants(); const KernelVariant& variant(int i); void printVariantTable();
 *       -- bench/kernels/gemm-mma.cuh:368-387, table bench/kernels/gemm-mma.cu:55-141
 *
 * Conventions, kept from the reference (gemm-mma.cu:19-43, check-gemm.cu:269-306):
 *   - the caller allocates and frees A, B and C on the device; a launch neither
 *     allocates nor synchronises, and is asynchronous on `stream` (NULL = default);
 *   - errors come back as hipError_t values (0 = hipSuccess);
 *   - the table is immutable and safe to read from any thread.
 * Deviations, all deliberate:
 *   - C is FP16 (rounded to nearest even from the FP32 accumulator) where the
 *     reference wrote FP32;
 *   - a shape that the variant does not divide, or K < BK, or a misaligned pointer,
 *     returns hipErrorInvalidValue (1) instead of being undefined behaviour;
 *   - WM/WN are wavefront (64-lane) tiles, `threads` = waves * 64, and
 *     `regsPerThread` is VGPRs + AGPRs per lane of the code built here.
 *
 * No HIP header is needed to use this file: streams are passed as void*.
 */
#ifndef RIDGE_GEMM_H
#define RIDGE_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One row of the kernel table; fields follow KernelVariant (gemm-mma.cuh:368-383)
 * in order, then gfx950 resource facts of the built code object. */
typedef struct ridge_gemm_variant {
    int BM, BN, BK;      /* workgroup tile */
    int WM, WN;          /* wavefront tile */
    int stages;          /* LDS ring depth */
    int groupM;          /* launch-order group size along M (1 = row-major) */
    int ldsBytes;        /* LDS per workgroup; the reference's smemBytes */
    int threads;         /* workitems per workgroup = waves * 64 */
    int regsPerThread;   /* arch VGPRs + AGPRs per lane, from the compiler */
    int waves;           /* wavefronts per workgroup */
    int vgprs;           /* arch VGPRs per lane */
    int agprs;           /* accumulation VGPRs per lane */
    int sgprs;           /* scalar registers per wave */
    int scratchBytes;    /* private segment bytes per lane (0 = no spills) */
    int occupancy;       /* waves per SIMD the compiler reports */
    int pingPong;        /* 1: ping-pong schedule (8 wavefronts, >= 3 stages); 0: otherwise */
    int schedule;        /* 0: uniform, 1: ping-pong, 2: persistent store-behind (one workgroup
                            per CU slot walks output tiles; two loader wavefronts feed the ring,
                            so `waves` and `threads` count them and `ldsBytes` includes the
                            epilogue staging) */
} ridge_gemm_variant_t;

/* Number of rows in the table (the reference's numVariants(), gemm-mma.cu:121). */
int ridge_gemm_num_variants(void);

/* Copies row i into *out. Returns 0, or 1 (hipErrorInvalidValue) for a bad
 * index or null pointer (the reference's variant(i), gemm-mma.cu:125). */
int ridge_gemm_get_variant(int i, ridge_gemm_variant_t* out);

/* Index of the row with exactly these tile parameters, or -1. */
int ridge_gemm_find_variant(int BM, int BN, int BK, int WM, int WN, int stages, int groupM);

/* 1 when variant i can run M x N x K (M%BM == N%BN == K%BK == 0, K >= BK, all
 * positive, and BM*K, BK*N and the tile count below 2^31, which keeps the
 * kernels' 32-bit tile offsets exact), else 0. The reference leaves this check
 * to its callers (check-gemm.cu:303, measure.cu:244). */
int ridge_gemm_divides(int i, int M, int N, int K);

/* C = A * B with variant i. A: M x K, B: K x N, C: M x N, all row-major FP16 in
 * device memory, 16-byte aligned. Returns a hipError_t value: 0 on a successful
 * enqueue, 1 (hipErrorInvalidValue) on a bad index, shape or pointer, otherwise
 * the launch error. The reference's KernelVariant::launch (gemm-mma.cu:19-43). */
int ridge_gemm_launch(int i, const void* A, const void* B, void* C, int M, int N, int K, void* stream);

/* Writes the variant table as CSV (header then one row per variant) into buf.
 * Returns the number of bytes the full text needs (excluding the NUL); writes at
 * most cap-1 bytes plus a NUL. Replaces the reference's printVariantTable()
 * (gemm-mma.cu:129-141) and the regex scrape of its source (validate.py:104-112). */
size_t ridge_gemm_variant_table_csv(char* buf, size_t cap);

/* Seeded synthetic inputs, generated on the device. Element i depends only on
 * (seed, i).
 *   uniform: U[-1, 1) -- 24 bits of splitmix64(seed, i) as top24 * 2^-23 - 1,
 *            rounded to FP16 (nearest even);
 *   lcg:     the reference's fill (check-gemm.cu:139-145): state s_{i+1} =
 *            s_i * 1664525 + 1013904223 from s_0 = seed, value
 *            ((s>>16) & 0x7fff) / 32767 - 0.5 in float, rounded to FP16.
 * Return hipError_t values as above. */
int ridge_fill_uniform_f16(void* dst, size_t n, uint64_t seed, void* stream);
int ridge_fill_lcg_f16(void* dst, size_t n, uint32_t seed, void* stream);

/* Vendor comparator: hipBLASLt FP16 GEMM with FP32 compute, row-major via the
 * operand swap C^T = B^T A^T (the reference's cublasReference,
 * check-gemm.cu:147-154, with D10/H10 of the build plan: a workspace and the best
 * of the heuristic's top candidates). c_is_f32 selects an FP32 C (the reference's
 * output type) instead of FP16.
 *   ridge_blaslt_create: returns 0 and an opaque handle;
 *   ridge_blaslt_prepare: picks the algorithm for (M,N,K,c_is_f32) by timing up to
 *       `candidates` heuristic results `iters` times each on the given buffers;
 *       returns 0, or a nonzero hipblasStatus_t/hipError_t value;
 *   ridge_blaslt_gemm: runs the prepared algorithm (prepares on first use).
 */
int ridge_blaslt_create(void** handle);
int ridge_blaslt_destroy(void* handle);
int ridge_blaslt_prepare(void* handle, const void* A, const void* B, void* C, int M, int N, int K, int c_is_f32,
                         int candidates, int iters, void* stream);
int ridge_blaslt_gemm(void* handle, const void* A, const void* B, void* C, int M, int N, int K, int c_is_f32,
                      void* stream);

/* Row split: a grid whose tiles fill whole rounds of resident workgroups and then
 * a fraction of one more (wave quantisation, e.g. 288 tiles of 256 x 256 on 256
 * CUs) runs the whole rounds with one row on the first rows of C and the rest of
 * the rows with another, usually smaller-tile, row. No counterpart in the
 * reference, whose callers launch one variant per shape; these two calls sit
 * beside that contract and change nothing in it.
 *
 * ridge_gemm_split_rows: rows of C the body row `body` takes, the largest multiple
 *   of its BM whose tiles fill whole rounds of its resident workgroups on numCUs
 *   CUs (workgroups per CU from its LDS bytes, waves and the compiler's waves per
 *   SIMD). Returns M when the grid is already whole rounds, 0 when it is less than
 *   one round, -1 for a bad index, CU count or a shape the row does not divide.
 * ridge_gemm_launch_split: variant `body` on rows [0, bodyRows) of A and C and
 *   variant `tail` on rows [bodyRows, M), back to back on `stream`. Both sub-shapes
 *   must be ones their variants divide and 0 < bodyRows < M; every check is made
 *   before the first launch, so a refused call (1, hipErrorInvalidValue) enqueues
 *   nothing. Returns the first launch error otherwise. */
int ridge_gemm_split_rows(int body, int M, int N, int K, int numCUs);
int ridge_gemm_launch_split(int body, int tail, int bodyRows, const void* A, const void* B, void* C, int M, int N,
                            int K, void* stream);

/* Library identification for logs: "ridge_gemm gfx950 <build info>". */
const char* ridge_gemm_build_info(void);

/* sizeof(ridge_gemm_variant_t) as this library was built, so a binding that
 * declares the struct itself (ctypes, cgo, JNA) can refuse a layout that
 * disagrees. No counterpart in the reference (its callers include its header). */
size_t ridge_gemm_variant_struct_size(void);

#ifdef __cplusplus
}
#endif

#endif /* RIDGE_GEMM_H */
