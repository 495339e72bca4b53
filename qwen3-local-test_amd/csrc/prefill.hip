// Causal chunked prefill attention on the gfx950 matrix cores.
//
// Same result as the reference's prefill path — the split-K shader run with n <= 1024 tokens
// (src/qwen4_vk.cpp:974-992, shaders/attention.comp + attn_combine.comp) — for n tokens at
// positions pos .. pos+n-1: row (t, h) attends to keys [0, pos + t + 1), softmax(q.k/sqrt(D)) V,
// times sigmoid(gate). The reference has no matrix-core attention (every workgroup streams K/V with
// scalar FMAs); this kernel is new design:
//  - GQA packing: a workgroup owns 128 query rows = 128/G consecutive tokens x the G heads of one KV
//    head, so each K/V tile staged in LDS feeds all of them; 4 waves x 32 rows.
//  - S^T[32 keys x 32 rows] = K Q^T and O^T[D x 32 rows] += V^T P^T on v_mfma_f32_32x32x16_f16 (the
//    shape that reaches ~2 PFLOP/s on gfx950; 16x16x32 reaches half of that) with fp32 accumulators.
//    A 64-key tile is two cache blocks; the QK^T product runs as four independent accumulation chains
//    (block x even/odd k-step) and P.V as D/32 chains, so the matrix pipe never waits on one result.
//  - Tiles are copied verbatim from the blocked cache (common.hpp) into LDS: 16 contiguous bytes per
//    lane from global memory, the same bytes lane-linearly into LDS. In that layout every operand
//    fragment read is 8-lane groups over 128 contiguous bytes, so LDS reads are bank-conflict free, and
//    the P^T operand of P.V is exactly the register order the QK^T product leaves (S rows map to keys
//    with bits 2 and 3 swapped), so no shuffles sit between the two products.
//  - Global -> LDS staging is double buffered with direct-to-LDS buffer loads (no registers; range
//    checked, so blocks past the last written position load zeros) and one barrier per tile; V rows past
//    the last position are zeroed in LDS, so stale or unwritten cache memory never reaches the sum.
//  - Softmax in log2 units with a lazy rescale (the reference max moves only when a row's max grows by
//    more than 2^8); tiles below every row's causal limit skip the mask, tiles past it are skipped.
//  - Workgroups are issued longest-first (last tokens first) to shorten the causal tail.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

namespace {

constexpr int PF_ROWS = 128;  // query rows per workgroup
constexpr int PF_KT = 64;     // keys per LDS tile (two cache blocks)

template <int D>
struct PfCfg {
    static constexpr int NKS = D / 16;                  // QK k-steps (32x32x16)
    static constexpr int NDT = D / 32;                  // P.V dim tiles
    static constexpr int BLKE = kBlk * D;               // elements of one (block, head) part
    static constexpr int TILEE = 2 * BLKE;              // elements of a 64-key tile (K or V)
    static constexpr int LOADS = TILEE * 2 / (4 * 1024);  // 1 KB direct loads per wave per tile (K or V)
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

}  // namespace

template <int D, int Q_DT, int IN_DT>
__global__ __launch_bounds__(256, 1) void k_prefill(PrefillArgs a) {
    using C = PfCfg<D>;
    constexpr int NKS = C::NKS, NDT = C::NDT, BLKE = C::BLKE, TILEE = C::TILEE, LOADS = C::LOADS;
    constexpr float TAU = 8.f;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    auto sK = [&](int b) { return reinterpret_cast<f16*>(smem) + (size_t)b * 2 * TILEE; };
    auto sV = [&](int b) { return reinterpret_cast<f16*>(smem) + (size_t)b * 2 * TILEE + TILEE; };

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 31, half = lane >> 5;
    const int G = a.NH / a.NKV;
    const int tok_per_blk = PF_ROWS / G;
    const int n_qt = (a.n + tok_per_blk - 1) / tok_per_blk;
    // longest first: the last query tiles have the most keys
    const int kvh = blockIdx.x % a.NKV;
    const int qt = n_qt - 1 - (int)(blockIdx.x / a.NKV);
    const int t0 = qt * tok_per_blk;

    // this lane's query row (B-operand column) and its causal limit
    const int r = wave * 32 + col;
    const int t = t0 + r / G, h = kvh * G + r % G;
    const bool row_ok = t < a.n;
    const int len = row_ok ? a.pos + t + 1 : 0;
    // the wave's and the workgroup's key ranges
    const int t_wave_first = t0 + wave * 32 / G;
    const bool wave_live = t_wave_first < a.n;
    const int t_wave_last = min(a.n - 1, t0 + (wave * 32 + 31) / G);
    const int wave_end = wave_live ? a.pos + t_wave_last + 1 : 0;
    const int wave_nomask = a.pos + t_wave_first + 1;  // keys below this are visible to every row of the wave
    const int blk_end = a.pos + min(a.n - 1, t0 + tok_per_blk - 1) + 1;
    const int n_tiles = (blk_end + PF_KT - 1) / PF_KT;
    const int maxlen = a.pos + a.n;

    // ---- Q^T operand in registers: lane holds row `col`, dims 16*ks + 8*half .. +8 ----------------
    f16x8 qop[NKS];
    {
        const size_t qoff = ((size_t)(row_ok ? t : 0) * a.NH + h) * D + 8 * half;
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            f16x8 v;
            if constexpr (Q_DT == 2) {
                v = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(a.q) + qoff + 16 * ks);
            } else {
                const float* qp = static_cast<const float*>(a.q) + qoff + 16 * ks;
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = (f16)(qp[i] * a.q_scale);
            }
            qop[ks] = row_ok ? v : f16x8{};
        }
    }

    f32x16 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;

    // ---- K/V staging: range-checked buffer loads of whole blocks of this KV head --------------------
    const int nblk = (maxlen + kBlk - 1) / kBlk;  // blocks holding written positions
    const int bstride = a.NKV * BLKE * 2;         // bytes between consecutive blocks of one head
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kc) + (size_t)kvh * BLKE, (short)0, nblk * bstride, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.vc) + (size_t)kvh * BLKE, (short)0, nblk * bstride, 0x00020000);
    // direct-to-LDS copy of tile kt into buffer b: 16 bytes per lane, lane-linear, one kilobyte per
    // instruction; each wave copies every fourth kilobyte of the K and the V tile
    auto copy_tile = [&](int b, int kt) {
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int ci = wave + 4 * i;                      // kilobyte of the tile
            const int blk = 2 * kt + ci / (BLKE / 512);
            const int off = blk * bstride + (ci % (BLKE / 512)) * 1024 + lane * 16;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, (__attribute__((address_space(3))) void*)(sK(b) + ci * 512), 16, off, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, (__attribute__((address_space(3))) void*)(sV(b) + ci * 512), 16, off, 0, 0, 0);
        }
    };
    // V rows past the last written position: zeroed in LDS (each 16-byte chunk holds 8 consecutive keys
    // of one dim), so stale or unwritten cache memory never reaches the sum
    auto zero_tail = [&](int b, int kt) {
        f16* Vb = sV(b);
        for (int idx = tid; idx < TILEE / 8; idx += 256) {
            const int q = idx % (BLKE / 8);
            const int key0 = (2 * kt + idx / (BLKE / 8)) * kBlk + 8 * ((q >> 4) & 3);
            if (key0 + 7 >= maxlen) {
                u32x4_t v = *reinterpret_cast<u32x4_t*>(Vb + idx * 8);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    v[k] &= (key0 + 2 * k < maxlen ? 0x0000ffffu : 0u) | (key0 + 2 * k + 1 < maxlen ? 0xffff0000u : 0u);
                *reinterpret_cast<u32x4_t*>(Vb + idx * 8) = v;
            }
        }
    };

    // per-lane constant parts of the fragment addresses (elements within a block part)
    // K: S^T row m = col <-> key sigma(col) = col with bits 2 and 3 swapped; dims 16*ks + 8*half
    const int kq = (col & ~12) | ((col & 4) << 1) | ((col & 8) >> 1);
    const int kc_ = ((kq >> 3) << 2) | (kq & 3), ks_ = (kq >> 2) & 1;
    const int koff_lane = ks_ * 512 + half * 128 + kc_ * 8;
    // V^T: dim 32*dt + col, keys 8*(2u + half) .. +7 of a block
    const int voff_lane = (((col >> 4) * 4 + half) * 16 + (col & 15)) * 8;

    if (n_tiles > 0) copy_tile(0, 0);
    for (int kt = 0; kt < n_tiles; kt++) {
        const int buf = kt & 1;
        // this wave's copies of tile kt are complete; after the barrier every wave's are, and every
        // wave is done reading the other buffer (tile kt-1), which the next copy overwrites
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if ((kt + 1) * PF_KT > maxlen) {
            zero_tail(buf, kt);
            __syncthreads();
        }
        if (kt + 1 < n_tiles) copy_tile(buf ^ 1, kt + 1);

        const int k0 = kt * PF_KT;
        if (k0 < wave_end) {
            const f16* K = sK(buf);
            const f16* V = sV(buf);
            // S^T for the tile's two blocks, each as two chains over even/odd k-steps
            f32x16 s2[2][2];
#pragma unroll
            for (int sb = 0; sb < 2; sb++) s2[sb][0] = s2[sb][1] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < NKS; ks++)
#pragma unroll
                for (int sb = 0; sb < 2; sb++) {
                    const f16x8 kf = *reinterpret_cast<const f16x8*>(
                        K + sb * BLKE + koff_lane + (ks >> 1) * 1024 + (ks & 1) * 256);
                    s2[sb][ks & 1] = mfma32(kf, qop[ks], s2[sb][ks & 1]);
                }
            // register j of lane (col, half) in block sb: key k0 + 32*sb + 16*(j/8) + 8*half + j%8
            float sv[2][16];
            const bool full = k0 + PF_KT <= wave_nomask;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float v = s2[sb][0][j] + s2[sb][1][j];
                    const int kj = k0 + 32 * sb + 16 * (j >> 3) + 8 * half + (j & 7);
                    sv[sb][j] = (full || kj < len) ? v : kNegInf;
                }
            float mx = sv[0][0];
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int j = 0; j < 16; j++) mx = fmaxf(mx, sv[sb][j]);
            {
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            }
            // lazy rescale (see the header)
            if (m_run == kNegInf) m_run = mx;
            if (__builtin_amdgcn_ballot_w64(mx > m_run + TAU) != 0) {
                const float m_new = fmaxf(m_run, mx);
                const float corr = exp2_fast(m_run - m_new);
                m_run = m_new;
                l_run *= corr;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) acc[dt] *= corr;
            }
            const float m_use = m_run == kNegInf ? 0.f : m_run;
            f16x8 pop[2][2];
            float ps = 0.f;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float p = exp2_fast(sv[sb][j] - m_use);
                    ps += p;
                    pop[sb][j >> 3][j & 7] = (f16)p;
                }
            l_run += ps;
            // O^T += V^T P^T: four 16-key steps, D/32 independent accumulators
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++) {
                        const f16x8 vf = *reinterpret_cast<const f16x8*>(
                            V + sb * BLKE + voff_lane + (dt * 8 + 2 * u) * 16 * 8);
                        acc[dt] = mfma32(vf, pop[sb][u], acc[dt]);
                    }
        }
        // no second barrier: the next iteration stores into the other buffer, and its barrier is only
        // passed once every wave has finished reading this one
    }

    // ---- epilogue: l across the two lane halves, normalize, gate, store ---------------------------
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
        l_run = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (row_ok) {
        const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
        const size_t ob = ((size_t)t * a.NH + h) * D;
        const size_t gb = ((size_t)t * a.NH + h) * 2 * D + D;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                // accumulator registers 4*q4 .. 4*q4+3 of lane (col, half): dims 32*dt + 8*q4 + 4*half + 0..3
                const int d = dt * 32 + 8 * q4 + 4 * half;
                float g4[4];
                load_vec<IN_DT, 4>(a.qg, gb + d, g4);
                f32x4 o;
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = acc[dt][4 * q4 + i] * inv * sigmoid(g4[i]);
                *reinterpret_cast<f32x4*>(a.out + ob + d) = o;
            }
    }
}

template <int D>
static hipError_t launch_pf_d(const PrefillArgs& a, int q_dtype, int in_dtype, hipStream_t s) {
    using C = PfCfg<D>;
    const int G = a.NH / a.NKV;
    const int tok = PF_ROWS / G;
    const int n_qt = (a.n + tok - 1) / tok;
    const dim3 grid(n_qt * a.NKV), block(256);
    const size_t shm = 2 * 2 * (size_t)C::TILEE * 2;  // two buffers of a K and a V tile
    auto go = [&](auto kern) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, block, shm, s, a);
        return hipGetLastError();
    };
    if (q_dtype == 2 && in_dtype == 0) return go(k_prefill<D, 2, 0>);
    if (q_dtype == 2) return go(k_prefill<D, 2, 1>);
    if (in_dtype == 0) return go(k_prefill<D, 0, 0>);
    return go(k_prefill<D, 0, 1>);
}

hipError_t launch_prefill(const PrefillArgs& a, int D, int q_dtype, int in_dtype, hipStream_t s) {
    if (D == 256) return launch_pf_d<256>(a, q_dtype, in_dtype, s);
    if (D == 128) return launch_pf_d<128>(a, q_dtype, in_dtype, s);
    return launch_pf_d<64>(a, q_dtype, in_dtype, s);
}

}  // namespace qw
