// fill.hip -- seeded synthetic GEMM inputs generated on the device, so a bench or
// a test can create 4096^3-sized operands without a host round trip. Element i is
// a pure function of (seed, i); the CPU oracle computes the same values, which is
// how the tests pin these kernels bit for bit.

#include "ridge_gemm.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// splitmix64 (Steele, Lea and Flood, 2014): output i of the stream seeded with s
// is the finaliser applied to s + (i + 1) * 0x9e3779b97f4a7c15.
__device__ __forceinline__ uint64_t splitmix64At(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1u) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ void fillUniformKernel(_Float16* dst, size_t n, uint64_t seed) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t top24 = (uint32_t)(splitmix64At(seed, i) >> 40);
        // top24 * 2^-23 is exact in float and so is the subtraction of 1, which
        // leaves the conversion to half as the only rounding (nearest even).
        const float v = (float)top24 * (1.0f / 8388608.0f) - 1.0f;
        dst[i] = (_Float16)v;
    }
}

// The reference fill (bench/check-gemm.cu:139-145) advances a 32-bit LCG once per
// element. Element i needs state s_{i+1} = T^{i+1}(seed) with T(s) = a s + c mod
// 2^32; the power of the affine map is taken by squaring, so every element is
// independent.
__global__ void fillLcgKernel(_Float16* dst, size_t n, uint32_t seed) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t steps = i + 1;
        uint32_t mulAcc = 1u, addAcc = 0u;           // accumulated map x -> mulAcc x + addAcc
        uint32_t mulPow = 1664525u, addPow = 1013904223u;  // T^(2^b)
        while (steps) {
            if (steps & 1u) {
                // (T^(2^b) o acc)(x) = mulPow (mulAcc x + addAcc) + addPow
                addAcc = mulPow * addAcc + addPow;
                mulAcc = mulPow * mulAcc;
            }
            addPow = mulPow * addPow + addPow;
            mulPow = mulPow * mulPow;
            steps >>= 1;
        }
        const uint32_t s = mulAcc * seed + addAcc;
        const float v = ((float)((s >> 16) & 0x7fffu) / 32767.0f) - 0.5f;
        dst[i] = (_Float16)v;
    }
}

int gridFor(size_t n) {
    const size_t blocks = (n + 255) / 256;
    return (int)(blocks < 65536 ? (blocks == 0 ? 1 : blocks) : 65536);
}

}  // namespace

extern "C" int ridge_fill_uniform_f16(void* dst, size_t n, uint64_t seed, void* stream) {
    if (n == 0) return 0;
    if (dst == nullptr) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(fillUniformKernel, dim3(gridFor(n)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<_Float16*>(dst), n, seed);
    return (int)hipGetLastError();
}

extern "C" int ridge_fill_lcg_f16(void* dst, size_t n, uint32_t seed, void* stream) {
    if (n == 0) return 0;
    if (dst == nullptr) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(fillLcgKernel, dim3(gridFor(n)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<_Float16*>(dst), n, seed);
    return (int)hipGetLastError();
}
