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

// Matrix-instruction order of one pipeline step of N slots: QK^T and P.V steps alternate. Slot i is a
// QK^T step (index slot_qk) or a P.V step (index slot_pv); without P.V only the QK^T slots issue.
// slot_rank counts the issuing slots before i, slot_nth is the slot of the u-th issuing one (-1 past
// the end).
constexpr bool slot_is_qk(int, int i) { return i % 2 == 0; }
constexpr int slot_qk(int i) { return i / 2; }
constexpr int slot_pv(int, int i) { return i / 2; }
constexpr bool slot_issues(int n, bool pv, int i) { return pv || slot_is_qk(n, i); }
constexpr int slot_rank(int n, bool pv, int i) {
    int r = 0;
    for (int k = 0; k < i; k++) r += slot_issues(n, pv, k) ? 1 : 0;
    return r;
}
constexpr int slot_nth(int n, bool pv, int u) {
    for (int k = 0; k < n; k++)
        if (slot_issues(n, pv, k) && u-- == 0) return k;
    return -1;
}

}  // namespace

template <int D, int Q_DT, int IN_DT>
__global__ __launch_bounds__(256, 1) void k_prefill(PrefillArgs a) {
    using C = PfCfg<D>;
    constexpr int NKS = C::NKS, NDT = C::NDT, BLKE = C::BLKE, TILEE = C::TILEE, LOADS = C::LOADS;
    constexpr float TAU = 8.f;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // two K tile buffers, then two V tile buffers
    auto sK = [&](int b) { return reinterpret_cast<f16*>(smem) + (size_t)b * TILEE; };
    auto sV = [&](int b) { return reinterpret_cast<f16*>(smem) + (size_t)(2 + b) * TILEE; };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: copy addresses stay scalar
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
        // every load issued before the first use, so the row's fetches overlap
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            f16x8 v;
            if constexpr (Q_DT == 2) {
                v = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(a.q) + qoff + 16 * ks);
            } else {
                float x[8];
                load_vec<0, 8>(a.q, qoff + 16 * ks, x);
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = (f16)(x[i] * a.q_scale);
            }
            qop[ks] = row_ok ? v : f16x8{};
        }
        // the Q fragments are only ever matrix-instruction operands: keep them in accumulation registers,
        // leaving the vector registers to the softmax and the operand staging
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) asm volatile("" : "+a"(qop[ks]));
    }

    f32x16 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;

    // ---- K/V staging: range-checked buffer loads of whole blocks of this KV head --------------------
    const int nblk = (maxlen + kBlk - 1) / kBlk;  // blocks holding written positions
    const int bstride = BLKE * 2;                 // bytes between consecutive blocks of one head
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kc) + kv_part(0, kvh, a.cap, D), (short)0, nblk * bstride, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.vc) + kv_part(0, kvh, a.cap, D), (short)0, nblk * bstride, 0x00020000);
    // direct-to-LDS copy, piece i of tile kt: 16 bytes per lane, lane-linear, one kilobyte per
    // instruction; each wave copies every fourth kilobyte of the tile
    const int lane16 = lane * 16;
    auto copy_piece = [&](const __amdgpu_buffer_rsrc_t& rs, f16* dst, int kt, int i) {
        const int ci = wave + 4 * i;  // kilobyte of the tile
        const int blk = 2 * kt + ci / (BLKE / 512);
        // the whole offset in the per-lane operand, so the range check covers it
        const int off = blk * bstride + (ci % (BLKE / 512)) * 1024 + lane16;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(dst + ci * 512), 16, off, 0, 0, 0);
    };
    auto copy_tile = [&](const __amdgpu_buffer_rsrc_t& rs, f16* dst, int kt) {
#pragma unroll
        for (int i = 0; i < LOADS; i++) copy_piece(rs, dst, kt, i);
    };
    // V rows past the last written position: zeroed in LDS (each 16-byte chunk holds 8 consecutive keys
    // of one dim), so stale or unwritten cache memory never reaches the sum
    auto zero_tail = [&](f16* Vb, int kt) {
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

    // Operand fragments in the order the matrix instructions consume them. Slot i of a tile iteration:
    // even i -> QK^T step i/2 (k-step (i/2)/2 of cache block (i/2)%2), odd i -> P.V step i/2 (block
    // q/(2*NDT), 16-key half (q/NDT)%2, dim tile q%NDT with q = i/2).
    constexpr int NSLOT = 2 * 2 * NKS;  // QK^T and P.V have D/8 steps each
    constexpr int PF = 5;               // fragment reads run this many slots ahead
    auto kfrag = [&](const f16* Kb, int q) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(Kb + (q & 1) * BLKE + ((q >> 1) >> 1) * 1024 + ((q >> 1) & 1) * 256);
    };
    auto vfrag = [&](const f16* Vb, int q) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(Vb + (q / (2 * NDT)) * BLKE + ((q % NDT) * 8 + 2 * ((q / NDT) & 1)) * 16 * 8);
    };

    f32x16 sc[2], sn[2];
    f16x8 pcur[2][2], pprev[2][2];

    // QK^T alone (the first tile) and P.V alone (the last tile), with the same fragment prefetch
    auto qk_only = [&](const f16* Kb) {
        f16x8 fr[PF + 1];
        static_for<0, PF>([&](auto ic) __attribute__((always_inline)) { fr[ic.value] = kfrag(Kb, ic.value); });
        sn[0] = sn[1] = f32x16{};
        static_for<0, 2 * NKS>([&](auto ic) __attribute__((always_inline)) {
            constexpr int q = decltype(ic)::value;
            if constexpr (q + PF < 2 * NKS) fr[(q + PF) % (PF + 1)] = kfrag(Kb, q + PF);
            sn[q & 1] = mfma32(fr[q % (PF + 1)], qop[q >> 1], sn[q & 1]);
            __builtin_amdgcn_sched_barrier(0);  // keep the reads PF slots ahead
        });
    };
    auto pv_only = [&](const f16* Vb) {
        f16x8 fr[PF + 1];
        static_for<0, PF>([&](auto ic) __attribute__((always_inline)) { fr[ic.value] = vfrag(Vb, ic.value); });
        static_for<0, 4 * NDT>([&](auto ic) __attribute__((always_inline)) {
            constexpr int q = decltype(ic)::value;
            if constexpr (q + PF < 4 * NDT) fr[(q + PF) % (PF + 1)] = vfrag(Vb, q + PF);
            acc[q % NDT] = mfma32(fr[q % (PF + 1)], pprev[q / (2 * NDT)][(q / NDT) & 1], acc[q % NDT]);
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // One pipeline step, written in issue order: the softmax of tile kt (scores sc, weights into pc)
    // spread between the matrix instructions of QK^T(kt+1) (into sn, from K buffer Kb) and, when DO_PV,
    // P.V(kt-1) (weights pp, from V buffer Vb). The three are mutually independent, so the softmax
    // arithmetic issues while the matrix pipe works (two QK^T chains and D/32 P.V chains, alternating).
    // Softmax: row max over the first M1 slots, the rescale decision over the next three (one link of
    // that dependent chain per slot), then the exponentials, half-precision weights and row sums.
    float corr = 1.f;
    bool any_rescale = false;
    auto step = [&](auto do_pv, const f16* Kb, const f16* Vb, int kt) __attribute__((always_inline)) {
        constexpr bool DO_PV = decltype(do_pv)::value;
        constexpr int M1 = NSLOT / 4;                   // max phase: slots [0, M1)
        constexpr int E0 = M1 + 4, NE = NSLOT - E0;  // exponentials: slots [E0, NSLOT)
        auto frag = [&](int i) -> f16x8 {
            return slot_is_qk(NSLOT, i) ? kfrag(Kb, slot_qk(i)) : vfrag(Vb, slot_pv(NSLOT, i));
        };
        f16x8 fr[PF + 1];
        static_for<0, PF>([&](auto ic) __attribute__((always_inline)) {
            fr[ic.value] = frag(slot_nth(NSLOT, DO_PV, ic.value));
        });
        sn[0] = sn[1] = f32x16{};
        float mx = kNegInf, m_use = 0.f, m_new = 0.f, ps[2] = {0.f, 0.f};
        bool grow = false;
        static_for<0, NSLOT>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            // staging copies for the next iteration (K tile kt+2, V tile kt), one every third slot: issued
            // in one burst they would fill the vector-memory queue and stall the wave until it drains.
            // Past the last tile they read zeros (range-checked) or unused blocks into free buffers.
            if constexpr (i % 3 == 0 && i / 3 < 2 * LOADS) {
                constexpr int j = i / 3;
                if constexpr (j < LOADS) copy_piece(rk, sK(kt & 1), kt + 2, j);
                else copy_piece(rv, sV(kt & 1), kt, j - LOADS);
            }
            if constexpr (slot_issues(NSLOT, DO_PV, i)) {
                constexpr int u = slot_rank(NSLOT, DO_PV, i);
                constexpr int nx = slot_nth(NSLOT, DO_PV, u + PF);
                if constexpr (nx >= 0) fr[(u + PF) % (PF + 1)] = frag(nx);
                if constexpr (slot_is_qk(NSLOT, i)) {
                    constexpr int qi = slot_qk(i);
                    sn[qi & 1] = mfma32(fr[u % (PF + 1)], qop[qi >> 1], sn[qi & 1]);
                } else {
                    constexpr int pi = slot_pv(NSLOT, i);
                    acc[pi % NDT] = mfma32(fr[u % (PF + 1)], pprev[pi / (2 * NDT)][(pi / NDT) & 1], acc[pi % NDT]);
                }
            }
            if constexpr (i < M1) {
#pragma unroll
                for (int v = i * 32 / M1; v < (i + 1) * 32 / M1; v++) mx = fmaxf(mx, sc[v >> 4][v & 15]);
            } else if constexpr (i == M1) {
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            } else if constexpr (i == M1 + 1) {
                // lazy rescale: the reference max moves only when a row's max passes it by more than TAU
                // (log2 units), or on the row's first visible keys
                grow = m_run == kNegInf ? mx != kNegInf : mx > m_run + TAU;
                m_new = grow ? mx : m_run;
            } else if constexpr (i == M1 + 2) {
                any_rescale = __builtin_amdgcn_ballot_w64(grow) != 0;
                corr = exp2_fast(m_run - m_new);  // 0 on a row's first keys, 1 when unchanged
                m_use = m_new == kNegInf ? 0.f : m_new;
                m_run = m_new;
            }
            if constexpr (i >= E0) {
#pragma unroll
                for (int e = (i - E0) * 16 / NE; e < (i - E0 + 1) * 16 / NE; e++) {
                    const int sb = e >> 3, j = 2 * (e & 7);
                    const f16x2 pp = {(f16)exp2_fast(sc[sb][j] - m_use), (f16)exp2_fast(sc[sb][j + 1] - m_use)};
                    pcur[sb][j >> 3][j & 7] = pp[0];
                    pcur[sb][j >> 3][(j & 7) + 1] = pp[1];
                    // the row sum adds the same half-precision weights the P.V product uses
                    ps[e & 1] = __builtin_amdgcn_fdot2(pp, f16x2{(f16)1.f, (f16)1.f}, ps[e & 1], false);
                }
            }
            // slot boundary: the scheduler would otherwise sink each fragment read to its use and expose
            // the full LDS latency on every matrix instruction
            __builtin_amdgcn_sched_barrier(0);
        });
        l_run = l_run * corr + (ps[0] + ps[1]);
    };

    // Software pipeline over the workgroup's key tiles (every wave runs every tile; rows past their
    // causal limit see all-masked tiles). Staging: K tiles run two ahead of their use and V tiles one,
    // in two buffers each, with one barrier per iteration.
    if (n_tiles > 0) copy_tile(rk, sK(0), 0);
    if (n_tiles > 1) copy_tile(rk, sK(1), 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (n_tiles > 0) qk_only(sK(0) + koff_lane);

    for (int kt = 0; kt < n_tiles; kt++) {
        sc[0] = sn[0];
        sc[1] = sn[1];
        // this wave's copies are complete; after the barrier every wave's are, and every wave is done
        // with the buffers this iteration's copies overwrite (K tile kt, V tile kt-2)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if (kt >= 1 && kt * PF_KT > maxlen) {
            zero_tail(sV((kt - 1) & 1), kt - 1);
            __syncthreads();
        }
        const int k0 = kt * PF_KT;
        if (k0 + PF_KT > wave_nomask) {
            // causal edge: register j of lane (col, half) in block sb holds key
            // k0 + 32*sb + 16*(j/8) + 8*half + j%8, visible to this lane's row when below len
            const int lim = len - k0 - 8 * half;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int j = 0; j < 16; j++)
                    sc[sb][j] = (32 * sb + 16 * (j >> 3) + (j & 7)) < lim ? sc[sb][j] : kNegInf;
        }
        const f16* Kb = sK((kt + 1) & 1) + koff_lane;  // tile kt+1 (stale past the last tile: unused)
        const f16* Vb = sV((kt + 1) & 1) + voff_lane;  // tile kt-1 (no P.V on the first tile)
        if (kt == 0) step(std::false_type{}, Kb, Vb, kt);
        else step(std::true_type{}, Kb, Vb, kt);
        if (any_rescale) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) acc[dt] *= corr;
        }
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            pprev[sb][0] = pcur[sb][0];
            pprev[sb][1] = pcur[sb][1];
        }
    }
    // ---- P.V of the last tile ----
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (n_tiles > 0) {
        if (n_tiles * PF_KT > maxlen) {
            zero_tail(sV((n_tiles - 1) & 1), n_tiles - 1);
            __syncthreads();
        }
        pv_only(sV((n_tiles - 1) & 1) + voff_lane);
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
        // accumulator registers 4*q4 .. 4*q4+3 of lane (col, half): dims 32*dt + 8*q4 + 4*half + 0..3.
        // All gate loads first (the output stores could alias them as far as the compiler knows).
        float g[NDT][4][4];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) load_vec<IN_DT, 4>(a.qg, gb + dt * 32 + 8 * q4 + 4 * half, g[dt][q4]);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                f32x4 o;
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = acc[dt][4 * q4 + i] * inv * sigmoid(g[dt][q4][i]);
                *reinterpret_cast<f32x4*>(a.out + ob + dt * 32 + 8 * q4 + 4 * half) = o;
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
