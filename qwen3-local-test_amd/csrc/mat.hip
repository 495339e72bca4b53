// The projections on either side of the attention layer for gfx950: Y[n][rows] = X[n][cols] W^T with W in
// planar Q8_0 (int8 weights, one f32 scale per 32 consecutive weights of a row) or plain f32 rows.
//
// Replaces Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856) on its matrix-vector pipelines q4_matmul_q8 /
// q4_matmul_f32 (shaders/q4_matmul.comp with the C_Q8 / C_F32 codecs of shaders/q4_codec.glsl; the planar
// repacking of GGUF Q8_0 is src/qwen4_vk.cpp:98-106): every output is the fp32 dot product of a dequantized
// weight row (int8 times its block's scale) with a token's input row, then optionally silu(y * post_scale).
//
// MI355X design: the weights are read once per launch and are the bound (a decode step's projections are
// memory-bound); a wave owns RW rows and a workgroup NTP tokens (one for a single token), lane l covering the
// 16 consecutive columns 16 l + 1,024 k of every row, so a wave reads a kilobyte of each row per chunk in
// one 16-byte load a lane (plus one scale a lane pair), and every weight load of a wave's rows is issued
// before the first is used. A 16-column group never crosses a 32-weight block, so the lane applies its
// block scale once per group and token. The partial dot products are summed over the wave with DPP row
// operations and permlane swaps.
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

// f32 weights: a wave's RW rows a 16-column group at a time (f32 projections are the small ones)
template <int NTP>
__global__ __launch_bounds__(256) void k_mat_f32(MatArgs a) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = (blockIdx.x * 4 + wave) * kMatRW;
    const int t0 = blockIdx.y * NTP;
    const int nt = min(NTP, a.n - t0);
    if (r0 >= a.rows) return;  // whole waves
    float acc[kMatRW][NTP];
#pragma unroll
    for (int r = 0; r < kMatRW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) acc[r][t] = 0.f;
    for (int c = lane * 16; c < a.cols; c += 1024) {
        float xv[NTP][16];
#pragma unroll
        for (int t = 0; t < NTP; t++) {
            const float* xr = a.x + (size_t)(t0 + (t < nt ? t : 0)) * a.x_stride + c;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xr + i);
                xv[t][i] = v[0], xv[t][i + 1] = v[1], xv[t][i + 2] = v[2], xv[t][i + 3] = v[3];
            }
        }
#pragma unroll
        for (int r = 0; r < kMatRW; r++) {
            const float* wr = static_cast<const float*>(a.w) + (size_t)min(r0 + r, a.rows - 1) * a.cols + c;
            float wv[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(wr + i);
                wv[i] = v[0], wv[i + 1] = v[1], wv[i + 2] = v[2], wv[i + 3] = v[3];
            }
#pragma unroll
            for (int t = 0; t < NTP; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[r][t] = __builtin_fmaf(wv[i], xv[t][i], acc[r][t]);
        }
    }
#pragma unroll
    for (int r = 0; r < kMatRW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) {
            float v = mat_wave_sum(acc[r][t]);
            if (a.post == 1) {
                const float u = v * a.post_scale;
                v = u / (1.0f + __expf(-u));
            }
            if (lane == 0 && r0 + r < a.rows && t < nt) a.y[(size_t)(t0 + t) * a.y_stride + r0 + r] = v;
        }
}

// planar Q8: every weight load of a batch of up to kMatK 1,024-column chunks (RW rows x kMatK 16-byte
// loads a lane, with their scales) is issued before any is used, so a wave has its whole share of the
// matrix in flight at once (the stream is the bound: the loads have to overlap); then per chunk the token
// rows' 16 columns (cached: every wave reads them) and the dot products
constexpr int kMatK = 4;
template <int NTP>
__global__ __launch_bounds__(256) void k_mat_q8(MatArgs a) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = (blockIdx.x * 4 + wave) * kMatRW;
    const int t0 = blockIdx.y * NTP;
    const int nt = min(NTP, a.n - t0);
    if (r0 >= a.rows) return;  // whole waves
    const int8_t* w8 = static_cast<const int8_t*>(a.w);
    const int nsb = a.cols >> 5;  // scales a row
    float acc[kMatRW][NTP];
#pragma unroll
    for (int r = 0; r < kMatRW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) acc[r][t] = 0.f;
    for (int cb = 0; cb < a.cols; cb += kMatK * 1024) {
        u32x4 q[kMatRW][kMatK];
        float sc[kMatRW][kMatK];
#pragma unroll
        for (int k = 0; k < kMatK; k++) {
            if (cb + k * 1024 >= a.cols) break;  // the whole chunk lies past the row (wave-uniform)
            const int c = min(cb + k * 1024 + lane * 16, a.cols - 16);  // past the row: a valid group, unused
#pragma unroll
            for (int r = 0; r < kMatRW; r++) {
                const int row = min(r0 + r, a.rows - 1);  // past the last row: a valid row, result not stored
                q[r][k] = *reinterpret_cast<const u32x4*>(w8 + (size_t)row * a.cols + c);
                sc[r][k] = a.s[(size_t)row * nsb + (c >> 5)];
            }
        }
#pragma unroll
        for (int k = 0; k < kMatK; k++) {
            if (cb + k * 1024 >= a.cols) break;
            const int c = cb + k * 1024 + lane * 16;
            if (c >= a.cols) continue;  // this lane's group lies past the row
            float xv[NTP][16];
#pragma unroll
            for (int t = 0; t < NTP; t++) {
                const float* xr = a.x + (size_t)(t0 + (t < nt ? t : 0)) * a.x_stride + c;
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + i);
                    xv[t][i] = v[0], xv[t][i + 1] = v[1], xv[t][i + 2] = v[2], xv[t][i + 3] = v[3];
                }
            }
#pragma unroll
            for (int r = 0; r < kMatRW; r++) {
                float wv[16];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int v = (int)q[r][k][j];
                    wv[4 * j] = (float)((v << 24) >> 24);
                    wv[4 * j + 1] = (float)((v << 16) >> 24);
                    wv[4 * j + 2] = (float)((v << 8) >> 24);
                    wv[4 * j + 3] = (float)(v >> 24);
                }
#pragma unroll
                for (int t = 0; t < NTP; t++) {
                    float d = 0.f;
#pragma unroll
                    for (int i = 0; i < 16; i++) d = __builtin_fmaf(wv[i], xv[t][i], d);
                    acc[r][t] = __builtin_fmaf(d, sc[r][k], acc[r][t]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kMatRW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) {
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
    // one token (a decode step): a workgroup's waves take one token; else four tokens a workgroup
    const int ntp = a.n == 1 ? 1 : kMatNTP;
    const dim3 grid((a.rows + 4 * kMatRW - 1) / (4 * kMatRW), (a.n + ntp - 1) / ntp), block(256);
    if (q8) {
        if (ntp == 1) hipLaunchKernelGGL(k_mat_q8<1>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(k_mat_q8<kMatNTP>, grid, block, 0, s, a);
    } else {
        if (ntp == 1) hipLaunchKernelGGL(k_mat_f32<1>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(k_mat_f32<kMatNTP>, grid, block, 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace qw
