// Device-side helpers shared by the gfx950 attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// buffer load/store cache policy: device scope (sc1). Such stores reach the point every XCD reads from
// once acknowledged, and such loads never return a stale line of the local L2: partial results written by
// one workgroup can be read by another in the same launch without a cache-wide write-back or invalidate.
constexpr int kScDevice = 0x10;
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

// N consecutive elements of a projection-output row as fp32 with vector loads: fp32 in 16-byte pieces
// when N % 4 == 0, bf16 in 16-byte pieces when N % 8 == 0 (the caller guarantees the alignment).
template <int DT, int N>
__device__ __forceinline__ void load_vec(const void* p, size_t off, float (&x)[N]) {
    if constexpr (DT == 0) {
        const float* f = static_cast<const float*>(p) + off;
        if constexpr (N % 4 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(f + i);
                x[i] = v[0], x[i + 1] = v[1], x[i + 2] = v[2], x[i + 3] = v[3];
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) x[i] = f[i];
        }
    } else {
        const uint16_t* b = static_cast<const uint16_t*>(p) + off;
        if constexpr (N % 8 == 0) {
#pragma unroll
            for (int i = 0; i < N; i += 8) {
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 v = *reinterpret_cast<const u32x4*>(b + i);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    x[i + 2 * k] = __uint_as_float(v[k] << 16);
                    x[i + 2 * k + 1] = __uint_as_float(v[k] & 0xffff0000u);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) x[i] = __uint_as_float((uint32_t)b[i] << 16);
        }
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

// Sum over each 32-lane half of the wave, in every lane of the half, without LDS: butterfly steps over
// quads (quad_perm [1,0,3,2], then [2,3,0,1]), eight lanes (row_half_mirror), sixteen (row_mirror), then
// the two 16-lane rows of the half (permlane16_swap).
__device__ __forceinline__ float sum32(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Maximum over each 32-lane half of the wave, in every lane of the half (the butterfly of sum32).
// Maximum over the four 16-lane rows of the wave for each lane position (lanes l, l ^ 16, l ^ 32, l ^ 48):
// a row swap (permlane16_swap) then a half swap (permlane32_swap), no LDS round trip.
__device__ __forceinline__ float max_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float max32(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false)));
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 1 / (1 + e^-x) with the hardware exponential and reciprocal (about 1 ulp each); saturates to 0 for
// x below about -88 (e^-x overflows, its reciprocal is 0) and to 1 above
__device__ __forceinline__ float sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E-1, each body a separate
// instantiation, so indices into register arrays stay static whatever the body size (flat expansion).
template <int B, typename F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, B + I>{}), ...);
}
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq<B>(f, std::make_integer_sequence<int, E - B>{});
}

// ---- K/V cache layout ------------------------------------------------------------------------------
// Both caches are [NKV][cap/32][32*D] fp16: per KV head, blocks of 32 positions, one 32*D part per block
// (a head's blocks are contiguous, so a workgroup streaming one head's key range reads one contiguous
// range). Inside a part the elements are ordered so that every MFMA operand fragment of the decode and
// prefill kernels is one contiguous kilobyte (64 lanes x 16 bytes):
//  K: (key kb, dim d) -> (((d/32)*2 + s)*4 + (d/8)%4)*16 + c)*8 + d%8 with c = (kb/8)*4 + kb%4,
//     s = (kb/4)%2. Fragment (kk, s) of v_mfma_f32_16x16x32_f16's A operand — lane (c, g) holding key
//     8*(c/4) + 4*s + c%4, dims 32*kk + 8*g .. +7 — is the kilobyte at (kk*2 + s) KB, and the score
//     tile it produces leaves keys 8*g .. 8*g+7 of every column in lane group g.
//  V: (key kb, dim d) -> (((d/16)*4 + kb/8)*16 + d%16)*8 + kb%8. Fragment dt of the P.V product's A
//     operand (V^T: lane (c, g) holding dim 16*dt + c for keys 8*g .. 8*g+7) is the kilobyte at dt KB.
constexpr int kBlk = 32;  // positions per cache block

__device__ __forceinline__ int k_off(int kb, int d) {
    const int c = ((kb >> 3) << 2) | (kb & 3), s = (kb >> 2) & 1;
    return (((((d >> 5) << 1) | s) * 4 + ((d >> 3) & 3)) * 16 + c) * 8 + (d & 7);
}

__device__ __forceinline__ int v_off(int kb, int d) {
    return (((d >> 4) * 4 + (kb >> 3)) * 16 + (d & 15)) * 8 + (kb & 7);
}

// Element offset of the part holding (position p, KV head h) in a cache of capacity cap (a multiple of 32).
__device__ __forceinline__ size_t kv_part(int p, int h, int cap, int D) {
    return ((size_t)h * (cap >> 5) + (p >> 5)) * (size_t)(kBlk * D);
}

}  // namespace qw
