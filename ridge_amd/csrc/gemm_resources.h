// gemm_resources.h -- per-variant register and scratch facts of the built code
// object. The table is generated at build time from the compiler's
// kernel-resource-usage remarks (ridge_amd/build.py) in the same order as
// gemm_variants.def, the way the reference hand-copies ptxas -v output into its
// table (bench/kernels/gemm-mma.cu:377-381).
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ridge_gemm_resources {
    int vgprs;
    int agprs;
    int sgprs;
    int scratchBytes;
    int occupancy;
} ridge_gemm_resources_t;

extern const ridge_gemm_resources_t ridge_gemm_resource_table[];
extern const int ridge_gemm_resource_count;

#ifdef __cplusplus
}
#endif
