// Device-side helpers shared by the HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wamx {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
// Four bf16 bit patterns: the operand type of MFMA 16x16x16 bf16 (_1k).
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short bf16x4_t;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t) h << 16); }

// Pairwise combines across lanes l and l ^ 16 (or l ^ 32) with gfx950's VALU
// lane swaps (v_permlane16_swap / v_permlane32_swap of a value with itself
// leave the lower and the upper lane's value in the two results in every
// lane), instead of an LDS-routed shuffle.  max and + are commutative, so
// both lanes of a pair get the same bits.
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Round-to-nearest-even f32 -> bf16 with gfx950's v_cvt_pk_bf16_f32.  Checked
// on the device against the integer RNE rule of the host helper over all 2^32
// inputs: identical for every non-NaN input; NaN inputs give a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16) f); }

// The value a bf16 store of f would read back as.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// GELU, tanh form of Hendrycks & Gimpel (arXiv:1606.08415):
// 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3).
// Evaluated through the identity 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)) with the
// hardware base-2 exponential and reciprocal (1 ulp each): a few ulp of f32
// from the tanh form, far inside one bf16 ulp.  Large |x| saturates to x (the
// exponential underflows) or -0 (it overflows to +inf).
__device__ __forceinline__ float gelu_tanh(float x) {
    const float kNeg2Sqrt2OverPiLog2e = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
    const float kCubic = 0.044715f;
    const float t = kNeg2Sqrt2OverPiLog2e * x * fmaf(kCubic, x * x, 1.0f);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// GELU with the exact Gaussian CDF: 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f)); }

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024).  `red` needs
// blockDim.x/64 floats of shared memory.  Every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float * red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float load_as_f32(const void * p, int32_t type, int64_t i) {
    if (type == 0) return ((const float *) p)[i];
    if (type == 30) return bf16_to_f32(((const uint16_t *) p)[i]);
    if (type == 26) return (float) ((const int32_t *) p)[i];
    return (float) ((const _Float16 *) p)[i];
}
__device__ __forceinline__ void store_from_f32(void * p, int32_t type, int64_t i, float v) {
    if (type == 0) ((float *) p)[i] = v;
    else if (type == 30) ((uint16_t *) p)[i] = f32_to_bf16(v);
    else if (type == 26) ((int32_t *) p)[i] = (int32_t) v;
    else ((_Float16 *) p)[i] = (_Float16) v;
}

}  // namespace wamx
