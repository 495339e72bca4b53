// The projections on either side of the attention layer for gfx950: Y[n][rows] = X[n][cols] W^T with W in
// planar Q8_0 (int8 weights, one f32 scale per 32 consecutive weights of a row) or plain f32 rows.
//
// Replaces Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856) on its matrix-vector pipelines q4_matmul_q8 /
// q4_matmul_f32 (shaders/q4_matmul.comp with the C_Q8 / C_F32 codecs of shaders/q4_codec.glsl; the planar
// repacking of GGUF Q8_0 is src/qwen4_vk.cpp:98-106): every output is the fp32 dot product of a dequantized
// weight row (int8 times its block's scale) with a token's input row, then optionally silu(y * post_scale).
//
// MI355X design: the weights are read once per launch and are the bound (a decode step's projections are
// memory-bound); a wave owns RW rows and a workgroup NTP tokens, lane l covering the 16 consecutive columns
// 16 l + 1,024 k of every row, so a wave reads a kilobyte of each row per step in one 16-byte load a lane
// (plus one scale a lane pair), and its slice of the token rows stays in registers across its RW rows. A
// 16-column group never crosses a 32-weight block, so the lane applies its block scale once per group and
// token. The partial dot products are summed over the wave with DPP row operations and permlane swaps.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

namespace {

constexpr int kMatRW = 4;   // rows a wave
constexpr int kMatNTP = 4;  // tokens a workgroup

// Sum over the 64 lanes, in every lane.
__device__ __forceinline__ float mat_wave_sum(float x) {
    x = sum32(x);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

template <bool Q8>
__global__ __launch_bounds__(256) void k_mat(MatArgs a) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = (blockIdx.x * 4 + wave) * kMatRW;
    const int t0 = blockIdx.y * kMatNTP;
    const int nt = min(kMatNTP, a.n - t0);
    if (r0 >= a.rows) return;  // whole waves
    float acc[kMatRW][kMatNTP];
#pragma unroll
    for (int r = 0; r < kMatRW; r++)
#pragma unroll
        for (int t = 0; t < kMatNTP; t++) acc[r][t] = 0.f;
    for (int c = lane * 16; c < a.cols; c += 1024) {
        float xv[kMatNTP][16];
#pragma unroll
        for (int t = 0; t < kMatNTP; t++) {
            const float* xr = a.x + (size_t)(t0 + (t < nt ? t : 0)) * a.x_stride + c;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xr + i);
                xv[t][i] = v[0], xv[t][i + 1] = v[1], xv[t][i + 2] = v[2], xv[t][i + 3] = v[3];
            }
        }
#pragma unroll
        for (int r = 0; r < kMatRW; r++) {
            const int row = min(r0 + r, a.rows - 1);  // past the last row: a valid row, result not stored
            float wv[16];
            float sc = 1.f;
            if constexpr (Q8) {
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 q = *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(a.w) + (size_t)row * a.cols + c);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int v = (int)q[j];
                    wv[4 * j] = (float)((v << 24) >> 24);
                    wv[4 * j + 1] = (float)((v << 16) >> 24);
                    wv[4 * j + 2] = (float)((v << 8) >> 24);
                    wv[4 * j + 3] = (float)(v >> 24);
                }
                sc = a.s[(size_t)row * (a.cols >> 5) + (c >> 5)];
            } else {
                const float* wr = static_cast<const float*>(a.w) + (size_t)row * a.cols + c;
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(wr + i);
                    wv[i] = v[0], wv[i + 1] = v[1], wv[i + 2] = v[2], wv[i + 3] = v[3];
                }
            }
#pragma unroll
            for (int t = 0; t < kMatNTP; t++) {
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) d = __builtin_fmaf(wv[i], xv[t][i], d);
                acc[r][t] = __builtin_fmaf(d, sc, acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kMatRW; r++)
#pragma unroll
        for (int t = 0; t < kMatNTP; t++) {
            float v = mat_wave_sum(acc[r][t]);
            if (a.post == 1) {
                const float u = v * a.post_scale;
                v = u / (1.0f + __expf(-u));
            }
            if (lane == 0 && r0 + r < a.rows && t < nt) a.y[(size_t)(t0 + t) * a.y_stride + r0 + r] = v;
        }
}

}  // namespace

hipError_t launch_mat(const MatArgs& a, bool q8, hipStream_t s) {
    const dim3 grid((a.rows + 4 * kMatRW - 1) / (4 * kMatRW), (a.n + kMatNTP - 1) / kMatNTP), block(256);
    if (q8) hipLaunchKernelGGL(k_mat<true>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(k_mat<false>, grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace qw
