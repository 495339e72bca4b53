// Device-side helpers shared by the gfx950 attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace qw {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// Input dtypes of the projection outputs (qg, k, v): 0 = fp32, 1 = bf16.
template <int DT>
__device__ __forceinline__ float load_in(const void* p, size_t i) {
    if constexpr (DT == 0) {
        return static_cast<const float*>(p)[i];
    } else {
        const uint32_t u = static_cast<const uint16_t*>(p)[i];
        return __uint_as_float(u << 16);
    }
}

// 16x16x32 fp16 MFMA, fp32 accumulate. Lane l: A row / B column l%16, k = 8*(l/16) + slot;
// C rows 4*(l/16) + i, column l%16.
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 32x32x16 fp16 MFMA. Lane l: A row / B column l%32, k = 8*(l/32) + slot; C column l%32,
// rows 8*(j/4) + 4*(l/32) + j%4 for register j.
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Value of lane (l ^ 8) within each 16-lane row (DPP row_ror:8).
__device__ __forceinline__ float xor8(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, false));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    return x;
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

}  // namespace qw
