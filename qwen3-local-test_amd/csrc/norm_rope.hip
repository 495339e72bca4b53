// Fused QK-RMSNorm + partial rotate-half RoPE + fp16 K/V append for gfx950.
//
// Replaces shaders/qk_norm_rope.comp (pipeline qk_norm_rope_kv16). Same math per (token t, head):
//   y = x * rsqrt(mean(x^2) + eps) * (1 + w)                     (qk_norm_rope.comp:26-34)
//   d < R/2:      y'[d] = y[d] cos_i - y[d + R/2] sin_i            (qk_norm_rope.comp:36-42,
//   R/2 <= d < R: y'[d] = y[d] cos_i + y[d - R/2] sin_i             src/qwen4_cpu.cpp:281-289)
// with (cos_i, sin_i) from row p = pos + t of the rope table. Query heads write q_out; key heads
// write K cache position p (round-to-nearest-even fp16, as packHalf2x16) and copy V into the V cache.
//
// MI355X layout: a 32-lane half-wavefront per four (token, head) rows, D/32 consecutive dims per lane
// (the reference uses a 256-invocation workgroup with an LDS reduction per head), so the mean of
// squares is a five-step shuffle reduction with no barrier, the rows move in 16-byte loads and stores,
// every load of the four rows is in flight at once, and the RoPE partner d +- R/2 is (R/2)/(D/32)
// lanes away. The caches are written in the blocked layout of
// common.hpp (a key row's 8 consecutive dims are one 16-byte piece). V is a plain copy whose blocked
// layout runs 8 consecutive keys of one dim, so it has lanes of its own (workgroups after the norm
// ones): a lane loads 8 dims of 8 consecutive positions and writes 8 whole 16-byte pieces; only the
// partly new groups at the ends of the range are written element by element.
// The split-KV decode kernel (decode.hip) does the same work inline for its new tokens; this kernel
// serves prefill chunks and callers of the per-dispatch entry point.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

// rows per half-wave: every load of the rows is issued before any is used. Four when the query rows are
// in the launch (NH + NKV rows per token); one for a K/V-only launch, whose few rows then spread over
// four times the workgroups
constexpr int kNormRows = 4;
constexpr int kNormRowsKv = 1;

// V groups of a call: 8-position groups overlapping [pos, pos + n)
__host__ __device__ inline int v_groups(int pos, int n) { return (pos + n - 1) / 8 - pos / 8 + 1; }

// V lane vi: KV head h, 8-position group g (positions 8g .. 8g+7), dims 8c .. 8c+7 (c fastest, so a
// wave's loads are whole row segments). The 8 x 8 block is transposed in registers: dim d's 8 keys
// are one 16-byte piece of the blocked layout. Positions outside [pos, pos + n) are neither read
// (their loads repeat a valid row) nor written.
template <int D, int IN_DT>
__device__ __forceinline__ void v_copy(const NormRopeArgs& a, int vi) {
    constexpr int NC = D / 8;
    const int ng = v_groups(a.pos, a.n);
    if (vi >= a.NKV * ng * NC) return;
    const int c = vi % NC, g = a.pos / 8 + (vi / NC) % ng, h = vi / NC / ng;
    const int p0 = 8 * g;
    float x[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int t = min(max(p0 + i - a.pos, 0), a.n - 1);
        load_vec<IN_DT, 8>(a.v, ((size_t)t * a.NKV + h) * D + 8 * c, x[i]);
    }
    f16* vc = reinterpret_cast<f16*>(a.vcache) + kv_part(p0, h, a.cap, D);
    const int kb0 = p0 & (kBlk - 1);  // a multiple of 8: v_off(kb0, d) starts dim d's 8-key piece
    const bool whole = p0 >= a.pos && p0 + 8 <= a.pos + a.n;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        f16* dst = vc + v_off(kb0, 8 * c + j);
        if (whole) {
            f16x8 o;
#pragma unroll
            for (int i = 0; i < 8; i++) o[i] = (f16)x[i][j];
            *reinterpret_cast<f16x8*>(dst) = o;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (p0 + i >= a.pos && p0 + i < a.pos + a.n) dst[i] = (f16)x[i][j];
        }
    }
}

template <int D, int IN_DT, int Q_DT, int NR>
__global__ __launch_bounds__(256) void k_qk_norm_rope(NormRopeArgs a) {
    // NR rows per half-wave (32 lanes x DPL consecutive dims each): 16-byte loads of the rows and 16-byte
    // stores of the query rows and of the key rows' blocked-layout pieces
    constexpr int DPL = D / 32;
    const int hl = threadIdx.x & 31;
    const int item0 = (blockIdx.x * 8 + (threadIdx.x >> 5)) * NR;
    // without q_out only the key heads are rows of this launch (head index hh = NH + key head)
    const int q_heads = a.q_out ? a.NH : 0;
    const int heads = q_heads + a.NKV;
    const int n_items = a.n * heads;
    const int norm_blocks = (n_items + 8 * NR - 1) / (8 * NR);
    if ((int)blockIdx.x >= norm_blocks) {
        v_copy<D, IN_DT>(a, ((int)blockIdx.x - norm_blocks) * 256 + (int)threadIdx.x);
        return;
    }
    if (item0 >= n_items) return;  // whole half-wave exits
    const int d0 = hl * DPL;
    const int half_r = a.R >> 1;
    const bool rot = d0 < a.R;  // DPL divides R/2: a lane's dims are all rotated or all not
    const bool lo = d0 < half_r;

    float x[NR][DPL], cs[NR][2 * DPL];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int item = min(item0 + r, n_items - 1);  // past the end: the last row again, not stored
        const int t = item / heads, hh = item % heads + a.NH - q_heads;
        const bool is_q = hh < a.NH;
        const int h = is_q ? hh : hh - a.NH;
        const size_t src = is_q ? ((size_t)t * a.NH + h) * 2 * D : ((size_t)t * a.NKV + h) * D;
        load_vec<IN_DT, DPL>(is_q ? a.qg : a.k, src + d0, x[r]);
        if (rot) load_vec<0, 2 * DPL>(a.rope, (size_t)(a.pos + t) * a.R + 2 * (lo ? d0 : d0 - half_r), cs[r]);
    }
    float wq[DPL], wk[DPL];
    load_vec<0, DPL>(a.qn, d0, wq);
    load_vec<0, DPL>(a.kn, d0, wk);
    const int offl = half_r / DPL;
    // rotate-half: the partner dim d +- R/2 sits (R/2)/DPL lanes away in the same half-wave
    const int src_lane = (threadIdx.x & 63 & ~31) + (rot ? (lo ? hl + offl : hl - offl) : hl);

#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int item = item0 + r;
        if (item >= n_items) break;  // uniform over the half-wave
        const int t = item / heads, hh = item % heads + a.NH - q_heads;
        const bool is_q = hh < a.NH;
        const int h = is_q ? hh : hh - a.NH;
        const int p = a.pos + t;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; j++) ss += x[r][j] * x[r][j];
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 32);
        const float rn = 1.0f / sqrtf(ss / (float)D + a.eps);
        float y[DPL];
#pragma unroll
        for (int j = 0; j < DPL; j++) y[j] = x[r][j] * rn * (1.0f + (is_q ? wq[j] : wk[j]));
#pragma unroll
        for (int j = 0; j < DPL; j++) {
            const float partner = __shfl(y[j], src_lane, 64);
            if (rot) y[j] = lo ? y[j] * cs[r][2 * j] - partner * cs[r][2 * j + 1] : y[j] * cs[r][2 * j] + partner * cs[r][2 * j + 1];
        }
        typedef f16 f16v __attribute__((ext_vector_type(DPL)));
        if (is_q) {
            if constexpr (Q_DT == 0) {
                float* qo = static_cast<float*>(a.q_out) + ((size_t)t * a.NH + h) * D + d0;
                if constexpr (DPL % 4 == 0) {
#pragma unroll
                    for (int j = 0; j < DPL; j += 4) *reinterpret_cast<f32x4*>(qo + j) = f32x4{y[j], y[j + 1], y[j + 2], y[j + 3]};
                } else {
#pragma unroll
                    for (int j = 0; j < DPL; j++) qo[j] = y[j];
                }
            } else {
                f16v o;
#pragma unroll
                for (int j = 0; j < DPL; j++) o[j] = (f16)(y[j] * a.q_scale);
                *reinterpret_cast<f16v*>(static_cast<f16*>(a.q_out) + ((size_t)t * a.NH + h) * D + d0) = o;
            }
        } else {
            f16* kc = reinterpret_cast<f16*>(a.kcache) + kv_part(p, h, a.cap, D);
            // K: the lane's DPL dims are consecutive in the blocked layout (d % 8 runs fastest)
            f16v ko;
#pragma unroll
            for (int j = 0; j < DPL; j++) ko[j] = (f16)y[j];
            *reinterpret_cast<f16v*>(kc + k_off(p & (kBlk - 1), d0)) = ko;
        }
    }
}

template <int D>
static hipError_t launch_d(const NormRopeArgs& a, int in_dtype, int q_dtype, hipStream_t s) {
    const int items = a.n * ((a.q_out ? a.NH : 0) + a.NKV);
    const int v_lanes = a.NKV * v_groups(a.pos, a.n) * (D / 8);
    const int nr = a.q_out ? kNormRows : kNormRowsKv;
    const dim3 grid((items + 8 * nr - 1) / (8 * nr) + (v_lanes + 255) / 256), block(256);
    if (!a.q_out) {  // K/V rows only: the query dtype is unused
        if (in_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 0, 1, kNormRowsKv>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((k_qk_norm_rope<D, 1, 1, kNormRowsKv>), grid, block, 0, s, a);
    } else if (in_dtype == 0 && q_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 0, 0, kNormRows>), grid, block, 0, s, a);
    else if (in_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 0, 1, kNormRows>), grid, block, 0, s, a);
    else if (q_dtype == 0) hipLaunchKernelGGL((k_qk_norm_rope<D, 1, 0, kNormRows>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_qk_norm_rope<D, 1, 1, kNormRows>), grid, block, 0, s, a);
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
