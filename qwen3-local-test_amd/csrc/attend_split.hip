// Split-KV causal GQA attention (decode and MTP verify) plus the log-sum-exp combine, for gfx950.
//
// Replaces shaders/attention.comp (attention_kv16) and shaders/attn_combine.comp. Semantics per query
// row (token t, head h): keys j < len_t = pos + t + 1, score q.k_j / sqrt(D), softmax, times V; the
// key axis [0, pos + n) is cut into chunks, each chunk leaves an unnormalized partial (m, l, o[D])
// (attention.comp:26-75) and the combine merges them, skipping l = 0 splits, then applies
// sigmoid(gate) (attn_combine.comp:13-29).
//
// MI355X design (not the reference's): one workgroup per (chunk, KV head) serves all rows that share
// that KV head — the G = NH/NKV query heads of each of the n tokens, RT <= 32 rows — so each K/V row
// leaves HBM exactly once (the reference runs one workgroup per query head and relies on L2 for the
// G-fold re-read). The products run on the matrix cores with fp32 accumulation:
//   S^T[32 keys x rows] = K[32 x D] . Q^T  — v_mfma_f32_16x16x32_f16, A = K rows loaded straight from
//     the fp16 cache as 16-byte lane fragments, B = the query rows split into an fp16 "hi" part and an
//     fp16 "lo" remainder (hi + lo carries 22 mantissa bits), so the score keeps fp32 accuracy;
//   O^T[D x rows] += V^T[D x 32 keys] . P^T — A = V^T read as 16-byte fragments of 8 consecutive keys
//     from the position-interleaved V cache, B = P in fp16 (plus its lo remainder when the rows fit
//     in half a column tile, i.e. decode at G = 8).
// Each wave streams 32-key tiles with an online softmax (max across lanes, lane-partial sums); the 4
// waves of a workgroup merge through LDS and write one partial per (row, chunk). Scores are kept in
// log2 units (the query is pre-multiplied by log2(e)/sqrt(D)) so the exponentials are v_exp_f32.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

template <int D, int RT>
struct SplitCfg {
    static constexpr int NKS = D / 32;                   // k-steps of the QK^T product
    static constexpr int NDT = D / 16;                   // 16-dim tiles of the PV product
    static constexpr bool PLO = RT == 8;                 // lo columns fit in the spare half tile
    static constexpr int QT = PLO ? 1 : 2 * (RT / 16);   // QK column tiles (hi then lo)
    static constexpr int PT = PLO ? 1 : RT / 16;         // PV column tiles
    static constexpr int OSTRIDE = D + 4;                // LDS row stride (floats) for the merge
};

template <int D, int RT>
__global__ __launch_bounds__(256) void k_attend_split(SplitArgs a) {
    using C = SplitCfg<D, RT>;
    constexpr int NKS = C::NKS, NDT = C::NDT, QT = C::QT, PT = C::PT;
    constexpr bool PLO = C::PLO;

    __shared__ float sO[4][RT][C::OSTRIDE];
    __shared__ float sM[4][RT], sL[4][RT];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, g = lane >> 4;
    const int z = blockIdx.x, kvh = blockIdx.y;
    const int G = a.NH / a.NKV;
    const int rows = a.n * G;
    const int maxlen = a.pos + a.n;
    const int kb = z * a.chunk;
    const int ke = min(maxlen, kb + a.chunk);

    // ---- query operand: column c of tile ct holds one row's hi or lo fp16 part -------------------
    f16x8 qop[QT][NKS];
#pragma unroll
    for (int ct = 0; ct < QT; ct++) {
        const int r = PLO ? (c & 7) : (ct % (QT / 2)) * 16 + c;
        const bool lo = PLO ? (c >= 8) : (ct >= QT / 2);
        const bool valid = r < rows;
        const int t = valid ? r / G : 0, h = kvh * G + (valid ? r % G : 0);
        const float* qrow = a.q + ((size_t)t * a.NH + h) * D;
#pragma unroll
        for (int kk = 0; kk < NKS; kk++) {
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(qrow + kk * 32 + g * 8);
            const f32x4 x1 = *reinterpret_cast<const f32x4*>(qrow + kk * 32 + g * 8 + 4);
            f16x8 v;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float xs = (i < 4 ? x0[i] : x1[i - 4]) * a.q_scale;
                const f16 hi = (f16)xs;
                v[i] = valid ? (lo ? (f16)(xs - (float)hi) : hi) : (f16)0.f;
            }
            qop[ct][kk] = v;
        }
    }

    // ---- per PV column: row, its key limit inside this chunk, softmax state -----------------------
    int lim[PT];
    float m_run[PT], l_run[PT];
    f32x4 acc[NDT][PT];
#pragma unroll
    for (int pt = 0; pt < PT; pt++) {
        const int r = PLO ? (c & 7) : pt * 16 + c;
        const int t = r < rows ? r / G : 0;
        lim[pt] = r < rows ? min(a.pos + t + 1, ke) : 0;
        m_run[pt] = kNegInf;
        l_run[pt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) acc[dt][pt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const f16* kc = reinterpret_cast<const f16*>(a.kc);
    const f16* vc = reinterpret_cast<const f16*>(a.vc);
    const int last_blk = (maxlen - 1) >> 3;

    for (int tb = kb + wave * 32; tb < ke; tb += 128) {
        // K fragments: QK sub-tile s, A row c <-> key tb + 8*(c/4) + 4*s + c%4, so that lane (c, g)
        // ends up holding keys tb + 8g + 0..7 of its column, the order the P operand needs
        f16x8 ka[2][NKS];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int key = min(tb + 8 * (c >> 2) + 4 * s + (c & 3), maxlen - 1);
            const f16* kp = kc + ((size_t)key * a.NKV + kvh) * D + g * 8;
#pragma unroll
            for (int kk = 0; kk < NKS; kk++) ka[s][kk] = *reinterpret_cast<const f16x8*>(kp + kk * 32);
        }
        // V^T fragments: dim 16*dt + c, keys tb + 8g .. tb + 8g + 7 (one 16-byte group)
        f16x8 va[NDT];
        {
            const int blk = min((tb >> 3) + g, last_blk);
            const f16* vp = vc + (((size_t)blk * a.NKV + kvh) * D + c) * 8;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) va[dt] = *reinterpret_cast<const f16x8*>(vp + dt * 16 * 8);
        }

        // S^T = K Q^T
        f32x4 sc[QT][2];
#pragma unroll
        for (int ct = 0; ct < QT; ct++)
#pragma unroll
            for (int s = 0; s < 2; s++) {
                f32x4 accs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < NKS; kk++) accs = mfma16(ka[s][kk], qop[ct][kk], accs);
                sc[ct][s] = accs;
            }

        // the last tile may run past the cache end: clear V slots of keys >= maxlen so that stale or
        // unwritten memory can never reach the sum (p is already 0 there)
        if (tb + 32 > maxlen) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (tb + 8 * g + i >= maxlen) {
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++) va[dt][i] = (f16)0.f;
                }
            }
        }

#pragma unroll
        for (int pt = 0; pt < PT; pt++) {
            float sv[8];
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float v = PLO ? sc[0][s][i] + xor8(sc[0][s][i]) : sc[pt][s][i] + sc[pt + PT][s][i];
                    const int key = tb + 8 * g + 4 * s + i;
                    sv[s * 4 + i] = key < lim[pt] ? v : kNegInf;
                }
            float mx = sv[0];
#pragma unroll
            for (int k = 1; k < 8; k++) mx = fmaxf(mx, sv[k]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run[pt], mx);
            const float m_use = m_new == kNegInf ? 0.f : m_new;
            const float corr = exp2_fast(m_run[pt] - m_use);
            m_run[pt] = m_new;
            float psum = 0.f;
            f16x8 pop;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float p = exp2_fast(sv[k] - m_use);
                psum += p;
                const f16 ph = (f16)p;
                pop[k] = (PLO && c >= 8) ? (f16)(p - (float)ph) : ph;
            }
            l_run[pt] = l_run[pt] * corr + psum;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                acc[dt][pt] *= corr;
                acc[dt][pt] = mfma16(va[dt], pop, acc[dt][pt]);
            }
        }
    }

    // ---- wave results -> LDS ---------------------------------------------------------------------
#pragma unroll
    for (int pt = 0; pt < PT; pt++) {
        float l = l_run[pt];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (PLO) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[dt][pt][i] += xor8(acc[dt][pt][i]);
        }
        const int r = PLO ? c : pt * 16 + c;
        const bool writer = PLO ? c < 8 : true;
        if (writer) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                *reinterpret_cast<f32x4*>(&sO[wave][r][dt * 16 + g * 4]) = acc[dt][pt];
            if (g == 0) {
                sM[wave][r] = m_run[pt];
                sL[wave][r] = l;
            }
        }
    }
    __syncthreads();

    // ---- merge the 4 waves, write this chunk's partial per row -----------------------------------
    for (int idx = tid; idx < rows * D; idx += 256) {
        const int r = idx / D, d = idx % D;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; w++)
            if (sL[w][r] > 0.f) M = fmaxf(M, sM[w][r]);
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            if (sL[w][r] > 0.f) {
                const float f = exp2_fast(sM[w][r] - M);
                L += sL[w][r] * f;
                o += sO[w][r][d] * f;
            }
        }
        const int t = r / G, h = kvh * G + r % G;
        const size_t row = ((size_t)t * a.NH + h) * a.n_split + z;
        a.part_o[row * D + d] = o;
        if (d == 0) {
            a.part_ml[row * 2] = M;
            a.part_ml[row * 2 + 1] = L;
        }
    }
}

template <int D>
static hipError_t launch_split_d(const SplitArgs& a, hipStream_t s) {
    const int rows = a.n * (a.NH / a.NKV);
    const dim3 grid(a.n_split, a.NKV), block(256);
    if (rows <= 8) hipLaunchKernelGGL((k_attend_split<D, 8>), grid, block, 0, s, a);
    else if (rows <= 16) hipLaunchKernelGGL((k_attend_split<D, 16>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_attend_split<D, 32>), grid, block, 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attend_split(const SplitArgs& a, int D, hipStream_t s) {
    if (D == 256) return launch_split_d<256>(a, s);
    if (D == 128) return launch_split_d<128>(a, s);
    return launch_split_d<64>(a, s);
}

// ---- combine ---------------------------------------------------------------------------------------
// One workgroup per (row, 64-dim slice): 16 split groups x 16 lanes x 4 dims. The running max M and
// the denominator L come from a block reduction over all splits; empty splits (l = 0) are skipped.
template <int IN_DT>
__global__ __launch_bounds__(256) void k_combine(CombineArgs a, int D) {
    __shared__ float red[256];
    __shared__ f32x4 racc[16][16];
    const int tid = threadIdx.x;
    const int row = blockIdx.x;  // t * NH + h
    const int S = a.n_split;
    const float* ml = a.part_ml + (size_t)row * S * 2;

    float mx = kNegInf;
    for (int z = tid; z < S; z += 256)
        if (ml[2 * z + 1] > 0.f) mx = fmaxf(mx, ml[2 * z]);
    red[tid] = mx;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();
    float ls = 0.f;
    for (int z = tid; z < S; z += 256)
        if (ml[2 * z + 1] > 0.f) ls += ml[2 * z + 1] * exp2_fast(ml[2 * z] - M);
    red[tid] = ls;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] += red[tid + w];
        __syncthreads();
    }
    const float L = red[0];

    const int zg = tid >> 4, lane = tid & 15;
    const int d0 = blockIdx.y * 64 + lane * 4;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    const float* po = a.part_o + (size_t)row * S * D + d0;
    for (int z = zg; z < S; z += 16) {
        const float l = ml[2 * z + 1];
        if (l > 0.f) {
            const float f = exp2_fast(ml[2 * z] - M);
            o += *reinterpret_cast<const f32x4*>(po + (size_t)z * D) * f;
        }
    }
    racc[zg][lane] = o;
    __syncthreads();
    if (zg == 0) {
        f32x4 s = racc[0][lane];
#pragma unroll
        for (int k = 1; k < 16; k++) s += racc[k][lane];
        const int t = row / a.NH, h = row % a.NH;
        const size_t gb = ((size_t)t * a.NH + h) * 2 * D + D + d0;
        float* out = a.out + (size_t)row * D + d0;
        const float inv = 1.0f / L;
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = s[i] * inv * sigmoid(load_in<IN_DT>(a.qg, gb + i));
    }
}

hipError_t launch_combine(const CombineArgs& a, int D, int in_dtype, hipStream_t s) {
    const dim3 grid(a.n * a.NH, D / 64), block(256);
    if (in_dtype == 0) hipLaunchKernelGGL(k_combine<0>, grid, block, 0, s, a, D);
    else hipLaunchKernelGGL(k_combine<1>, grid, block, 0, s, a, D);
    return hipGetLastError();
}

}  // namespace qw
