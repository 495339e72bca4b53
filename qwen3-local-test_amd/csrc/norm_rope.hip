// Fused QK-RMSNorm + partial rotate-half RoPE + fp16 K/V append for gfx950.
//
// Replaces shaders/qk_norm_rope.comp (pipeline qk_norm_rope_kv16). Same math per (token t, head):
//   y = x * rsqrt(mean(x^2) + eps) * (1 + w)                     (qk_norm_rope.comp:26-34)
//   d < R/2:      y'[d] = y[d] cos_i - y[d + R/2] sin_i            (qk_norm_rope.comp:36-42,
//   R/2 <= d < R: y'[d] = y[d] cos_i + y[d - R/2] sin_i             src/qwen4_cpu.cpp:281-289)
// with (cos_i, sin_i) from row p = pos + t of the rope table. Query heads write q_out; key heads
// write K cache position p (round-to-nearest-even fp16, as packHalf2x16) and copy V into the V cache.
//
// MI355X layout: one 64-lane wavefront per (token, head) — the reference uses a 256-invocation
// workgroup with an LDS reduction per head — so the mean of squares is a wave reduction with no
// barrier (norm_rope_row in common.hpp). The caches are written in the blocked layout of common.hpp.
// The split-KV decode kernel (decode.hip) does the same work inline for its new tokens; this kernel
// serves prefill chunks and callers of the per-dispatch entry point.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

template <int D, int IN_DT, int Q_DT>
__global__ __launch_bounds__(256) void k_qk_norm_rope(NormRopeArgs a) {
    constexpr int DPL = D / 64;  // dims per lane
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int heads = a.NH + a.NKV;
    if (item >= a.n * heads) return;  // whole wave exits
    const int t = item / heads, hh = item % heads;
    const bool is_q = hh < a.NH;
    const int h = is_q ? hh : hh - a.NH;
    const int p = a.pos + t;
    const int d0 = lane * DPL;

    const size_t src = is_q ? ((size_t)t * a.NH + h) * 2 * D : ((size_t)t * a.NKV + h) * D;
    float y[DPL];
    norm_rope_row<D, IN_DT>(is_q ? a.qg : a.k, src, is_q ? a.qn : a.kn, a.rope + (size_t)p * a.R, a.R, a.eps,
                            lane, y);

    if (is_q) {
        if constexpr (Q_DT == 0) {
            float* qo = static_cast<float*>(a.q_out) + ((size_t)t * a.NH + h) * D + d0;
#pragma unroll
            for (int j = 0; j < DPL; j++) qo[j] = y[j];
        } else {
            f16* qo = static_cast<f16*>(a.q_out) + ((size_t)t * a.NH + h) * D + d0;
#pragma unroll
            for (int j = 0; j < DPL; j++) qo[j] = (f16)(y[j] * a.q_scale);
        }
    } else {
        const size_t part = kv_part(p, h, a.NKV, D);
        f16* kc = reinterpret_cast<f16*>(a.kcache) + part;
        f16* vc = reinterpret_cast<f16*>(a.vcache) + part;
        const int kb = p & (kBlk - 1);
        const size_t vs = ((size_t)t * a.NKV + h) * D + d0;
#pragma unroll
        for (int j = 0; j < DPL; j++) {
            kc[k_off(kb, d0 + j)] = (f16)y[j];
            vc[v_off(kb, d0 + j)] = (f16)load_in<IN_DT>(a.v, vs + j);
        }
    }
}

template <int D>
static hipError_t launch_d(const NormRopeArgs& a, int in_dtype, int q_dtype, hipStream_t s) {
    const int items = a.n * (a.NH + a.NKV);
    const dim3 grid((items + 3) / 4), block(256);
    if (in_dtype == 0 && q_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 0, 0>), grid, block, 0, s, a);
    else if (in_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 0, 1>), grid, block, 0, s, a);
    else if (q_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 1, 0>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_qk_norm_rope<D, 1, 1>), grid, block, 0, s, a);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope(const NormRopeArgs& a, int D, int in_dtype, int q_dtype, hipStream_t s) {
    if (D == 256) return launch_d<256>(a, in_dtype, q_dtype, s);
    if (D == 128) return launch_d<128>(a, in_dtype, q_dtype, s);
    return launch_d<64>(a, in_dtype, q_dtype, s);
}

// rope[p][i] = (cos, sin) of the fp32 angle (float)p * inv_freq[i] (src/qwen4_vk.cpp:494-504); the
// device sincosf reduces the argument in full, so large p keeps the host's accuracy.
__global__ __launch_bounds__(256) void k_rope_table(float* rope, const float* inv_freq, int n_pos, int half) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)n_pos * half) return;
    const int p = (int)(idx / half), i = (int)(idx % half);
    const float ang = (float)p * inv_freq[i];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    rope[2 * idx] = cs;
    rope[2 * idx + 1] = sn;
}

hipError_t launch_rope_table(float* rope, const float* inv_freq, int n_pos, int R, hipStream_t s) {
    const size_t total = (size_t)n_pos * (R / 2);
    hipLaunchKernelGGL(k_rope_table, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, rope, inv_freq, n_pos, R / 2);
    return hipGetLastError();
}

}  // namespace qw
