// Causal chunked prefill attention on the gfx950 matrix cores.
//
// Same result as the reference's prefill path — the split-K shader run with n <= 1024 tokens
// (src/qwen4_vk.cpp:974-992, shaders/attention.comp + attn_combine.comp) — for n tokens at
// positions pos .. pos+n-1: row (t, h) attends to keys [0, pos + t + 1), softmax(q.k/sqrt(D)) V,
// times sigmoid(gate). The reference has no matrix-core attention (every workgroup streams K/V with
// scalar FMAs); this kernel is new design:
//  - GQA packing: a workgroup owns 128 query rows = 128/G consecutive tokens x the G heads of one KV
//    head, so each K/V tile staged in LDS feeds all of them; 4 waves x 32 rows.
//  - S^T[32 keys x 32 rows] = K Q^T and O^T[D x 32 rows] += V^T P^T on v_mfma_f32_32x32x16_f16 with
//    fp32 accumulators (O^T lives in 8 x 16 accumulator registers per lane at D = 256). Q is fp16
//    pre-multiplied by log2(e)/sqrt(D) and stays in registers for the whole key sweep.
//  - K tiles (64 keys) are gathered from the blocked cache (common.hpp) into LDS row-major with the
//    16-byte chunk index XOR-swizzled by the key so the 32 lanes that read one dim chunk of 32 different
//    keys hit distinct banks; V tiles are gathered as 8-position groups per dim, the A-operand shape of
//    the P.V product.
//  - Global->LDS staging is double-buffered with one barrier per tile: tile i+1 is in flight in
//    registers while tile i is consumed, then lands in the other LDS buffer.
//  - Key tiles strictly below every row's causal limit skip the mask; tiles past it are skipped.
//  - Workgroups are issued longest-first (last tokens first) to shorten the causal tail.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

namespace {

constexpr int PF_ROWS = 128;  // query rows per workgroup
constexpr int PF_KT = 64;     // keys per LDS tile

template <int D>
struct PfCfg {
    static constexpr int CH = D / 8;                 // 16-byte chunks per K row
    static constexpr int KBYTES = PF_KT * D * 2;     // one K tile
    static constexpr int VBYTES = PF_KT * D * 2;     // one V tile
    static constexpr int LOADS = KBYTES / (256 * 16);  // 16-byte loads per thread per tile (K or V)
    static constexpr int NKS = D / 16;               // QK k-steps (32x32x16)
    static constexpr int NDT = D / 32;               // PV dim tiles
};

// swizzle of key k's chunk index: bits {0,1,3} of k land in bits {0,1,2}
__device__ __forceinline__ int ksw(int k) { return (k & 3) | ((k >> 1) & 4); }

}  // namespace

template <int D, int Q_DT, int IN_DT>
__global__ __launch_bounds__(256, 1) void k_prefill(PrefillArgs a) {
    using C = PfCfg<D>;
    constexpr int NKS = C::NKS, NDT = C::NDT, CH = C::CH, LOADS = C::LOADS;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    auto sK = [&](int b) { return reinterpret_cast<f16*>(smem + b * C::KBYTES); };
    auto sV = [&](int b) { return reinterpret_cast<f16*>(smem + 2 * C::KBYTES + b * C::VBYTES); };

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
    // the wave's and the block's key ranges
    const int t_wave_last = min(a.n - 1, t0 + (wave * 32 + 31) / G);
    const int wave_end = t0 + wave * 32 / G < a.n ? a.pos + t_wave_last + 1 : 0;
    const int t_blk_last = min(a.n - 1, t0 + tok_per_blk - 1);
    const int blk_end = a.pos + t_blk_last + 1;
    const int t_wave_first = t0 + wave * 32 / G;
    const int wave_nomask = a.pos + t_wave_first + 1;  // keys below this are visible to every row of the wave

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
            if (!row_ok) v = f16x8{};
            qop[ks] = v;
        }
    }

    f32x16 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;

    const f16* kc = reinterpret_cast<const f16*>(a.kc);
    const f16* vc = reinterpret_cast<const f16*>(a.vc);
    const int n_tiles = (blk_end + PF_KT - 1) / PF_KT;
    const int last_row = a.pos + a.n - 1;

    // ---- global -> register staging of one K and one V tile --------------------------------------
    f16x8 stK[LOADS], stV[LOADS];
    auto load_tile = [&](int kt) {
        const int k0 = kt * PF_KT;
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int idx = i * 256 + tid;           // chunk index within the tile
            const int key = idx / CH, ch = idx % CH;
            const int gk = min(k0 + key, last_row);
            stK[i] = *reinterpret_cast<const f16x8*>(kc + kv_part(gk, kvh, a.NKV, D) + k_off(gk & (kBlk - 1), ch * 8));
            // V: 8 groups of 8 positions, each D chunks of 16 bytes (8 consecutive keys of one dim)
            const int vb = idx / D, vd = idx % D;
            const int gp = min(k0 / 8 + vb, last_row >> 3) * 8;
            stV[i] = *reinterpret_cast<const f16x8*>(vc + kv_part(gp, kvh, a.NKV, D) + v_off(gp & (kBlk - 1), vd));
        }
    };
    auto store_tile = [&](int buf, int kt) {
        const int k0 = kt * PF_KT;
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int idx = i * 256 + tid;
            const int key = idx / CH, ch = idx % CH;
            *reinterpret_cast<f16x8*>(sK(buf) + (key * CH + (ch ^ ksw(key))) * 8) = stK[i];
            f16x8 v = stV[i];
            const int vb = idx / D;
            // positions past the last written row may hold stale or unwritten memory: zero them
            if (k0 + vb * 8 + 7 > last_row) {
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (k0 + vb * 8 + j > last_row) v[j] = (f16)0.f;
            }
            *reinterpret_cast<f16x8*>(sV(buf) + idx * 8) = v;
        }
    };

    if (n_tiles > 0) load_tile(0);
    for (int kt = 0; kt < n_tiles; kt++) {
        const int buf = kt & 1;
        store_tile(buf, kt);
        __syncthreads();
        if (kt + 1 < n_tiles) load_tile(kt + 1);

        const int k0 = kt * PF_KT;
        if (k0 < wave_end) {
            const f16* K = sK(buf);
            const f16* V = sV(buf);
#pragma unroll
            for (int sub = 0; sub < PF_KT / 32; sub++) {
                // S^T rows m <-> keys: bits 2 and 3 of m swapped, so register j of this lane holds key
                // 16*(j/8) + 8*half + j%8 of the sub-tile (the B-operand order of the P.V step)
                const int m = col;
                const int key = sub * 32 + ((m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1));
                f32x16 s = f32x16{};
#pragma unroll
                for (int ks = 0; ks < NKS; ks++) {
                    const int ch = 2 * ks + half;
                    const f16x8 kf = *reinterpret_cast<const f16x8*>(K + (key * CH + (ch ^ ksw(key))) * 8);
                    s = mfma32(kf, qop[ks], s);
                }
                // mask and online softmax (one column = one query row per lane)
                const int kbase = k0 + sub * 32 + 8 * half;
                float sv[16];
                const bool full = k0 + sub * 32 + 32 <= wave_nomask;
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int kj = kbase + 16 * (j >> 3) + (j & 7);
                    sv[j] = (full || kj < len) ? s[j] : kNegInf;
                }
                float mx = sv[0];
#pragma unroll
                for (int j = 1; j < 16; j++) mx = fmaxf(mx, sv[j]);
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float m_new = fmaxf(m_run, mx);
                const float m_use = m_new == kNegInf ? 0.f : m_new;
                const float corr = exp2_fast(m_run - m_use);
                m_run = m_new;
                f16x8 pop[2];
                float ps = 0.f;
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const float p = exp2_fast(sv[j] - m_use);
                    ps += p;
                    pop[j >> 3][j & 7] = (f16)p;
                }
                l_run = l_run * corr + ps;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) acc[dt] *= corr;
                // O^T += V^T P^T over the two 16-key steps of this sub-tile
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int vb = sub * 4 + u * 2 + half;  // 8-position group of this lane's keys
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++) {
                        const f16x8 vf = *reinterpret_cast<const f16x8*>(V + ((size_t)vb * D + dt * 32 + col) * 8);
                        acc[dt] = mfma32(vf, pop[u], acc[dt]);
                    }
                }
            }
        }
        // no barrier here: the next iteration stores into the other buffer, and its barrier is only
        // passed once every wave has finished reading this one
    }

    // ---- epilogue: l across the two lane halves, normalize, gate, store ---------------------------
    l_run += __shfl_xor(l_run, 32, 64);
    if (row_ok) {
        const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
        const size_t ob = ((size_t)t * a.NH + h) * D;
        const size_t gb = ((size_t)t * a.NH + h) * 2 * D + D;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                // accumulator register j of lane (col, half): dim 32*dt + 8*(j/4) + 4*half + j%4, row col
                const int d = dt * 32 + 8 * (j >> 2) + 4 * half + (j & 3);
                a.out[ob + d] = acc[dt][j] * inv * sigmoid(load_in<IN_DT>(a.qg, gb + d));
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
    const size_t shm = 2 * (size_t)C::KBYTES + 2 * (size_t)C::VBYTES;
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
