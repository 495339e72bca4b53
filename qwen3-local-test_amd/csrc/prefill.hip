// Causal chunked prefill attention on the gfx950 matrix cores.
//
// Same result as the reference's prefill path — the split-K shader run with n <= 1024 tokens
// (src/qwen4_vk.cpp:974-992, shaders/attention.comp + attn_combine.comp) — for n tokens at
// positions pos .. pos+n-1: row (t, h) attends to keys [0, pos + t + 1), softmax(q.k/sqrt(D)) V,
// times sigmoid(gate). The reference has no matrix-core attention (every workgroup streams K/V with
// scalar FMAs); this kernel is new design:
//  - GQA packing: a workgroup owns 128 query rows = 128/G consecutive tokens x the G heads of one KV
//    head, so each K/V tile staged in LDS feeds all of them; 8 waves x 16 rows, two waves a SIMD (a wave
//    holds its rows' Q^T, D/4 registers a lane, and their whole output, D/4 more, so two fit the 256
//    registers a wave has at that occupancy; both waves of a SIMD interleave their matrix instructions,
//    LDS reads and softmax).
//  - S^T[16 keys x 16 rows] = K Q^T and O^T[16 dims x 16 rows] += V^T P^T on v_mfma_f32_16x16x32_f16 with
//    fp32 accumulators (the same FLOP rate as the 32x32x16 shape on gfx950). A 64-key tile is two cache
//    blocks; QK^T runs as four independent accumulation chains (block x key set), P.V as D/16.
//  - Tiles are copied verbatim from the blocked cache (common.hpp) into LDS: 16 contiguous bytes per
//    lane from global memory, the same bytes lane-linearly into LDS. In that layout every operand
//    fragment is one contiguous kilobyte read lane-linearly (bank-conflict free), and the P^T operand of
//    P.V is exactly the register order the QK^T product leaves (a lane's scores are keys 8 g .. 8 g + 7 of
//    each block), so no shuffles sit between the two products.
//  - Global -> LDS staging is double buffered with direct-to-LDS buffer loads (no registers; range
//    checked, so blocks past the last written position load zeros) and one barrier per tile; V rows past
//    the last position are zeroed in LDS, so stale or unwritten cache memory never reaches the sum.
//  - Softmax in log2 units with a lazy rescale (the reference max moves only when a row's max grows by
//    more than 2^8); tiles below every row's causal limit skip the mask, tiles past it are skipped.
//  - Causal balance: query tile qt sees ceil((pos + 16(qt+1)) / 64) key tiles (33 to 64 at 2048 on
//    2048), and with one workgroup per CU the launch lasts as long as the longest one. Tiles are paired
//    instead, short qt with long n_qt-1-qt: one workgroup runs the long tile's keys [x, end), the other
//    its first x tiles and then the whole short tile, with x chosen so both get half the pair's tiles.
//    The two halves of the long tile are merged by whichever wave finishes its half last (per-wave
//    arrival counters, log-sum-exp merge of the stored partial), so no workgroup ever waits on another.
//    The workgroup with two segments loads the short tile's query rows and first two K tiles during
//    the long prefix's last P.V and merge, so its second segment starts without a load round trip.
//    Launches small enough that two workgroups per tile fit the CUs split every tile's keys in two
//    instead (same merge), so chunks of up to ~1,024 tokens still fill the chip.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

namespace {

constexpr int PF_ROWS = 128;  // query rows per workgroup
constexpr int PF_KT = 64;     // keys per LDS tile (two cache blocks)

template <int D>
struct PfCfg {
    static constexpr int NKS = D / 32;                  // QK k-steps (16x16x32)
    static constexpr int NDT = D / 16;                  // P.V dim tiles
    static constexpr int BLKE = kBlk * D;               // elements of one (block, head) part
    static constexpr int TILEE = 2 * BLKE;              // elements of a 64-key tile (K or V)
    static constexpr int LOADS = TILEE * 2 / (kPfWaves * 1024);  // 1 KB direct loads per wave per tile (K or V)
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

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

// The raw query values of lane (c, g) — row c of its wave's 16, dims 32 kk + 8 g + j (j < 8) of every
// 32-dim k-step kk: one 16-byte load of bf16 or two of fp32 a k-step — and, for 64 <= R <= 32 kPfRopeEarly
// * 2, the rope (cos, sin) pairs of its first k-steps, loaded first and used only in pf_query_fused: every
// vector load of the prologue is then issued before the first K tiles' copies, so none of them waits
// behind the copies (vector loads complete in issue order), and the math runs while the copies fly.
constexpr int kPfRopeEarly = 1;  // k-steps of (cos, sin) loaded with the query (R = 64)
template <int D, int IN_DT>
struct PfQRaw {
    typename std::conditional<IN_DT == 0, f32x4, u32x4_t>::type v[D / 32][IN_DT == 0 ? 2 : 1];
    f32x4 cs[kPfRopeEarly][4];
    __device__ __forceinline__ void load(const PrefillArgs& a, int t, int h, int g) {
        if (a.R == 64) {
            const float* cs_row = a.rope + (size_t)(a.pos + t) * a.R + 16 * g;
#pragma unroll
            for (int k = 0; k < 4; k++) cs[0][k] = *reinterpret_cast<const f32x4*>(cs_row + 4 * k);
        }
        const size_t off = ((size_t)t * a.NH + h) * 2 * D + 8 * g;
#pragma unroll
        for (int kk = 0; kk < D / 32; kk++) {
            if constexpr (IN_DT == 0) {
                const float* p = static_cast<const float*>(a.qg) + off + 32 * kk;
                v[kk][0] = *reinterpret_cast<const f32x4*>(p);
                v[kk][1] = *reinterpret_cast<const f32x4*>(p + 4);
            } else {
                v[kk][0] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.qg) + off + 32 * kk);
            }
        }
    }
    __device__ __forceinline__ float at(int kk, int j) const {
        if constexpr (IN_DT == 0) return v[kk][j >> 2][j & 3];
        else return __uint_as_float((j & 1) ? v[kk][0][j >> 1] & 0xffff0000u : v[kk][0][j >> 1] << 16);
    }
};

// The Q^T operand of query row (t, h) from the raw projection output: the query half of qg normalized,
// rotated and scaled in registers — the steps of the norm kernel (norm_rope.hip) for a query row, so a
// layer's prefill needs no query buffer: y = x * rsqrt(mean(x^2) + eps) * (1 + qn), rotate-half RoPE
// on dims [0, R) with the (cos, sin) of position pos + t, then fp16(y * q_scale). The four lanes (c, g) of
// a row hold its dims 32 kk + 8 g + j, so the mean of squares is two lane swaps. The rotate-half partner
// of dim d < R/2 is d + R/2: k-step kk + OFF of the same lane for R >= 64 (OFF = R/64), the lane 32 away
// for R = 32 (OFF = -1: dims 0-15 in lanes g < 2, their partners in lanes g + 2). rs = rsqrt term *
// q_scale folds the score scale into the row factor (0 for a row past the chunk).
template <int D, int IN_DT, int OFF>
__device__ __forceinline__ void pf_query_finish(const PrefillArgs& a, PfQRaw<D, IN_DT> raw, const float* sW,
                                                float rs, int t, int g, int lane, f16x8 (&qop)[D / 32]) {
    constexpr int NKS = D / 32;
    const float* cs_row = a.rope + (size_t)(a.pos + t) * a.R + 16 * g;
    // opaque per rope width: the widened raw values and the products raw * rs would otherwise be
    // hoisted above the caller's branch on R as common expressions, all of them live at once
    asm volatile("" : "+v"(rs));
#pragma unroll
    for (int kk = 0; kk < NKS; kk++)
#pragma unroll
        for (int k = 0; k < (IN_DT == 0 ? 2 : 1); k++) asm volatile("" : "+v"(raw.v[kk][k]));
    auto y = [&](int kk, float (&o)[8]) __attribute__((always_inline)) {  // normalized, weighted
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(sW + 32 * kk + 8 * g);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(sW + 32 * kk + 8 * g + 4);
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = raw.at(kk, j) * rs * (j < 4 ? w0[j] : w1[j - 4]);
    };
    auto put = [&](int kk, const float (&o)[8]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; j++) qop[kk][j] = (f16)o[j];
    };
#pragma unroll
    for (int kk = 0; kk < NKS; kk++) {
        if constexpr (OFF < 0) {  // R = 32: dims 0-15 (lanes g < 2) pair with dims 16-31 (lanes g + 2)
            if (kk == 0) {
                float o[8], p[8], cs[16];
                y(0, o);
                // (cos, sin) of i = 8 (g & 1) + j
                load_vec<0, 16>(a.rope + (size_t)(a.pos + t) * a.R, 16 * (g & 1), cs);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[j]), __float_as_uint(o[j]), false, false);
                    p[j] = __uint_as_float(lane < 32 ? sw[1] : sw[0]);
                }
                float r[8];
#pragma unroll
                for (int j = 0; j < 8; j++)
                    r[j] = g < 2 ? o[j] * cs[2 * j] - p[j] * cs[2 * j + 1] : o[j] * cs[2 * j] + p[j] * cs[2 * j + 1];
                put(0, r);
            } else {
                float o[8];
                y(kk, o);
                put(kk, o);
            }
        } else if (kk < OFF) {  // dims d < R/2 and their partners d + R/2
            float lo[8], hi[8], cs[16];  // (cos, sin) of i = 32 kk + 8 g + j
            y(kk, lo);
            y(kk + OFF, hi);
            if constexpr (OFF <= kPfRopeEarly) {
#pragma unroll
                for (int k = 0; k < 16; k++) cs[k] = raw.cs[0][k >> 2][k & 3];
            } else {
                load_vec<0, 16>(cs_row, 64 * kk, cs);
            }
            float rl[8], rh[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                rl[j] = lo[j] * cs[2 * j] - hi[j] * cs[2 * j + 1];
                rh[j] = hi[j] * cs[2 * j] + lo[j] * cs[2 * j + 1];
            }
            put(kk, rl);
            put(kk + OFF, rh);
        } else if (kk >= 2 * OFF) {
            float o[8];
            y(kk, o);
            put(kk, o);
        }
        // k-step boundary: hoisted, the multiplier and rope reads of every k-step would be live at once
        // beside the raw values and the operand
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int D, int IN_DT>
__device__ __forceinline__ void pf_query_fused(const PrefillArgs& a, const PfQRaw<D, IN_DT>& raw, const float* sW,
                                               int t, int g, int lane, bool row_ok, f16x8 (&qop)[D / 32]) {
    constexpr int NKS = D / 32;
    // eight independent partial sums of squares (a single chain would be NKS * 8 instructions long)
    float s8[8];
#pragma unroll
    for (int j = 0; j < 8; j++) s8[j] = raw.at(0, j) * raw.at(0, j);
#pragma unroll
    for (int kk = 1; kk < NKS; kk++)
#pragma unroll
        for (int j = 0; j < 8; j++) s8[j] = __builtin_fmaf(raw.at(kk, j), raw.at(kk, j), s8[j]);
    float ss = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
    // the row's four lanes (c, g): lanes 16 apart, then 32 apart
    const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
    // the row factor with the score scale folded in (the rotation is linear, so it commutes); the raw
    // values of a row past the chunk are those of row 0 (finite), so a zero factor zeroes the row
    const float rs = row_ok ? 1.0f / sqrtf(ss / (float)D + a.eps) * a.q_scale : 0.f;
    // the multipliers 1 + qn come from LDS (sW, the same for every row: broadcast reads)
    if (a.R == 0) pf_query_finish<D, IN_DT, 0>(a, raw, sW, rs, t, g, lane, qop);
    if (a.R == 32) pf_query_finish<D, IN_DT, -1>(a, raw, sW, rs, t, g, lane, qop);
    if constexpr (NKS >= 2) if (a.R == 64) pf_query_finish<D, IN_DT, 1>(a, raw, sW, rs, t, g, lane, qop);
    if constexpr (NKS >= 4) if (a.R == 128) pf_query_finish<D, IN_DT, 2>(a, raw, sW, rs, t, g, lane, qop);
    if constexpr (NKS >= 8) if (a.R == 256) pf_query_finish<D, IN_DT, 4>(a, raw, sW, rs, t, g, lane, qop);
}

// Whether a workgroup's first segment hands the next one its query rows and first K tiles: for rows
// normalized in the kernel from bf16 (the fp32 rows would need twice the registers through the hand-over).
constexpr bool pf_handover(bool qf, int in_dt) { return qf && in_dt == 1; }

// Key tiles of query tile qt: keys [0, pos + last token of the tile + 1) in 64-key tiles.
__device__ __forceinline__ int pf_tiles(const PrefillArgs& a, int tok_per_blk, int qt) {
    return (a.pos + min(a.n - 1, (qt + 1) * tok_per_blk - 1) + 1 + PF_KT - 1) / PF_KT;
}

// One segment of a workgroup's schedule: query tile qt (128 rows of KV head kvh) against key tiles
// [lo, hi). slot < 0: the tile's whole key range; the normalized, gated rows go to the output.
// slot >= 0: one of the two halves of a split tile. Each wave stores its unnormalized partial
// (accumulator, reference max, sum) in its half's region of the pair's slot and counts its arrival,
// unless the partner wave has already arrived; the wave that arrives second merges the two (in a fixed
// order) and writes the rows, then clears the counter for the next launch.
// Hand-over between a workgroup's two segments (bf16 rows normalized in the kernel): the first segment,
// told the next one's query tile (next_qt >= 0), issues that tile's raw query loads (into `carry`) and
// the copies of its first two K tiles right after its own loop, so they complete during its last P.V,
// merge and stores; the second (PRE) starts from them, and from the norm multipliers already in LDS.
template <int D, int IN_DT, bool QF, bool QSA, bool PRE>
__device__ __forceinline__ void pf_segment(const PrefillArgs& a, int kvh, int qt, int lo, int hi, int slot,
                                           int next_qt, PfQRaw<D, IN_DT>& carry) {
    constexpr bool NEXT = pf_handover(QF, IN_DT) && !PRE;
    static_assert(!PRE || pf_handover(QF, IN_DT), "hand-over only for in-kernel bf16 rows");
    using C = PfCfg<D>;
    constexpr int NKS = C::NKS, NDT = C::NDT, BLKE = C::BLKE, TILEE = C::TILEE, LOADS = C::LOADS;
    constexpr int NQK = 4 * NKS, NPV = 2 * NDT;  // matrix instructions a tile: QK^T, P.V (D/8 each)
    constexpr float TAU = 8.f;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // two K tile buffers, then two V tile buffers
    auto sK = [&](int b) { return reinterpret_cast<f16*>(smem) + (size_t)b * TILEE; };
    auto sV = [&](int b) { return reinterpret_cast<f16*>(smem) + (size_t)(2 + b) * TILEE; };

    // the thread index through an empty asm: lane-derived values are computed per segment instead of
    // being hoisted out of the kernel's segment loop, where they would stay live through the tile loop
    int tid_ = threadIdx.x;
    asm volatile("" : "+v"(tid_));
    const int tid = tid_, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: copy addresses stay scalar
    const int col = lane & 15, g = lane >> 4;
    const int G = a.NH / a.NKV;
    const int tok_per_blk = PF_ROWS / G;
    const int t0 = qt * tok_per_blk;

    // this lane's query row (B-operand column) and its causal limit
    const int r = wave * 16 + col;
    const int t = t0 + r / G, h = kvh * G + r % G;
    const bool row_ok = t < a.n;
    const int len = row_ok ? a.pos + t + 1 : 0;
    // the wave's first token: keys below its limit need no mask
    const int t_wave_first = t0 + wave * 16 / G;
    const int wave_nomask = a.pos + t_wave_first + 1;  // keys below this are visible to every row of the wave
    const int maxlen = a.pos + a.n;
    // QSA: the key bits of this lane's token for the current 64-key tile (two words), the next tile's
    // loaded once these are applied; words past the row's end read as zero
    const unsigned* qrow = QSA ? a.kbits + (size_t)(row_ok ? t : 0) * a.kb_words : nullptr;
    unsigned qw0 = 0xFFFFFFFFu, qw1 = 0xFFFFFFFFu;
    auto qsa_words = [&](int kt) __attribute__((always_inline)) {
        if constexpr (QSA) {
            qw0 = 2 * kt < a.kb_words ? qrow[2 * kt] : 0u;
            qw1 = 2 * kt + 1 < a.kb_words ? qrow[2 * kt + 1] : 0u;
        }
    };

    // ---- Q^T operand in registers: lane (col, g) holds row `col`, dims 32*kk + 8*g .. +8 -------------
    // the loads are issued here, the operand finished once the first K tiles' copies are in flight.
    // In-kernel normalization: the norm multipliers 1 + qn go to LDS (after the four tile buffers), loaded
    // by wave 0 ahead of every other load of the first segment (a second segment finds them there)
    f16x8 qop[NKS];
    PfQRaw<D, IN_DT> qraw;
    float* sW = reinterpret_cast<float*>(smem + (size_t)4 * C::TILEE * 2);
    f32x4 wq{};
    if constexpr (PRE) {
        qraw = carry;  // loaded by the previous segment (lo = 0: tiles 0 and 1 are in the K buffers)
    } else if constexpr (QF) {
        if (wave == 0 && lane < D / 4) wq = *reinterpret_cast<const f32x4*>(a.qn + 4 * lane);
        qraw.load(a, row_ok ? t : 0, h, g);
    } else {
        const size_t qoff = ((size_t)(row_ok ? t : 0) * a.NH + h) * D + 8 * g;
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) qop[ks] = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(a.q) + qoff + 32 * ks);
    }
    asm volatile("" ::: "memory");  // the query loads stay ahead of the copies

    f32x4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x4{};
    float m_run = kNegInf, l_run = 0.f;

    // ---- K/V staging: range-checked buffer loads of whole blocks of this KV head --------------------
    const int nblk = (maxlen + kBlk - 1) / kBlk;  // blocks holding written positions
    const int bstride = BLKE * 2;                 // bytes between consecutive blocks of one head
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kc) + kv_part(0, kvh, a.cap, D), (short)0, nblk * bstride, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.vc) + kv_part(0, kvh, a.cap, D), (short)0, nblk * bstride, 0x00020000);
    // direct-to-LDS copy, piece i of tile kt: 16 bytes per lane, lane-linear, one kilobyte per
    // instruction; each wave copies every eighth kilobyte of the tile
    const int lane16 = lane * 16;
    auto copy_piece = [&](const __amdgpu_buffer_rsrc_t& rs, f16* dst, int kt, int i) {
        const int ci = wave + kPfWaves * i;  // kilobyte of the tile
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
        for (int idx = tid; idx < TILEE / 8; idx += 64 * kPfWaves) {
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

    // Operand fragments: every one is the kilobyte of a block part at lane * 8 elements (the cache
    // layout). QK^T step q (of NQK): chain cq = q % 4 = (block b, key set s) = (cq / 2, cq % 2), k-step q / 4:
    // fragment (kk, s) of block b — lane (col, g) holding key 8*(col/4) + 4*s + col%4, dims 32*kk + 8*g ..
    // +7. P.V step q (of NPV): block q / NDT, dim tile dt = q % NDT: V^T fragment dt — lane (col, g) holding
    // dim 16*dt + col, keys 8*g .. +7 of the block. Slot i of a tile iteration: even i -> QK^T step i/2,
    // odd i -> P.V step i/2.
    constexpr int NSLOT = NQK + NPV;
    constexpr int PF = 5;  // fragment reads run this many slots ahead
    const int foff_lane = lane * 8;
    auto kfrag = [&](const f16* Kb, int q) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(Kb + ((q % 4) >> 1) * BLKE + ((q / 4) * 2 + (q & 1)) * 512);
    };
    auto vfrag = [&](const f16* Vb, int q) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(Vb + (q / NDT) * BLKE + (q % NDT) * 512);
    };

    // S^T of tile kt (sc) and kt+1 (sn): chain cq = 2 b + s, value i -> key 32 b + 8 g + 4 s + i of column col
    f32x4 sc[4], sn[4];
    // P^T operands of a tile: block b holds keys 32 b + 8 g + (0..7): {chain 2b value 0..3, chain 2b+1 value 0..3}
    f16x8 pcur[2], pprev[2];

    // QK^T alone (the first tile) and P.V alone (the last tile), with the same fragment prefetch
    auto qk_only = [&](const f16* Kb) {
        f16x8 fr[PF + 1];
        static_for<0, PF>([&](auto ic) __attribute__((always_inline)) { fr[ic.value] = kfrag(Kb, ic.value); });
#pragma unroll
        for (int cq = 0; cq < 4; cq++) sn[cq] = f32x4{};
        static_for<0, NQK>([&](auto ic) __attribute__((always_inline)) {
            constexpr int q = decltype(ic)::value;
            if constexpr (q + PF < NQK) fr[(q + PF) % (PF + 1)] = kfrag(Kb, q + PF);
            sn[q % 4] = mfma16(fr[q % (PF + 1)], qop[q / 4], sn[q % 4]);
            __builtin_amdgcn_sched_barrier(0);  // keep the reads PF slots ahead
        });
    };
    auto pv_only = [&](const f16* Vb) {
        f16x8 fr[PF + 1];
        static_for<0, PF>([&](auto ic) __attribute__((always_inline)) { fr[ic.value] = vfrag(Vb, ic.value); });
        static_for<0, NPV>([&](auto ic) __attribute__((always_inline)) {
            constexpr int q = decltype(ic)::value;
            if constexpr (q + PF < NPV) fr[(q + PF) % (PF + 1)] = vfrag(Vb, q + PF);
            acc[q % NDT] = mfma16(fr[q % (PF + 1)], pprev[q / NDT], acc[q % NDT]);
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // One pipeline step, written in issue order: the softmax of tile kt (scores sc, weights into pc)
    // spread between the matrix instructions of QK^T(kt+1) (into sn, from K buffer Kb) and, when DO_PV,
    // P.V(kt-1) (weights pp, from V buffer Vb). The three are mutually independent, so the softmax
    // arithmetic issues while the matrix pipe works (four QK^T chains and D/16 P.V chains, alternating).
    // Softmax: row max over the first M1 slots and the row's four lanes, the rescale decision over the next
    // two (one link of that dependent chain per slot), then the exponentials, half-precision weights and
    // the lane's part of the row sums.
    float corr = 1.f;
    bool any_rescale = false;
    auto step = [&](auto do_pv, const f16* Kb, const f16* Vb, int kt) __attribute__((always_inline)) {
        constexpr bool DO_PV = decltype(do_pv)::value;
        constexpr int M1 = NSLOT / 4;                   // max phase: slots [0, M1)
        constexpr int E0 = M1 + 4, NE = NSLOT - E0;  // exponentials: slots [E0, NSLOT)
        static_assert(NE >= 1, "slots for the exponentials");
        auto frag = [&](int i) -> f16x8 {
            return slot_is_qk(NSLOT, i) ? kfrag(Kb, slot_qk(i)) : vfrag(Vb, slot_pv(NSLOT, i));
        };
        f16x8 fr[PF + 1];
        static_for<0, PF>([&](auto ic) __attribute__((always_inline)) {
            fr[ic.value] = frag(slot_nth(NSLOT, DO_PV, ic.value));
        });
#pragma unroll
        for (int cq = 0; cq < 4; cq++) sn[cq] = f32x4{};
        float mx = kNegInf, m_use = 0.f, m_new = 0.f, ps[2] = {0.f, 0.f};
        bool grow = false;
        static_for<0, NSLOT>([&](auto ic) __attribute__((always_inline)) {
            constexpr int i = decltype(ic)::value;
            // staging copies for the next iteration (K tile kt+2, V tile kt), one every sixth slot: issued
            // in one burst they would fill the vector-memory queue and stall the wave until it drains.
            // Past the last tile they read zeros (range-checked) or unused blocks into free buffers.
            if constexpr (i % 6 == 0 && i / 6 < 2 * LOADS) {
                constexpr int j = i / 6;
                if constexpr (j < LOADS) copy_piece(rk, sK(kt & 1), kt + 2, j);
                else copy_piece(rv, sV(kt & 1), kt, j - LOADS);
            }
            if constexpr (slot_issues(NSLOT, DO_PV, i)) {
                constexpr int u = slot_rank(NSLOT, DO_PV, i);
                constexpr int nx = slot_nth(NSLOT, DO_PV, u + PF);
                if constexpr (nx >= 0) fr[(u + PF) % (PF + 1)] = frag(nx);
                if constexpr (slot_is_qk(NSLOT, i)) {
                    constexpr int qi = slot_qk(i);
                    sn[qi % 4] = mfma16(fr[u % (PF + 1)], qop[qi / 4], sn[qi % 4]);
                } else {
                    constexpr int pi = slot_pv(NSLOT, i);
                    acc[pi % NDT] = mfma16(fr[u % (PF + 1)], pprev[pi / NDT], acc[pi % NDT]);
                }
            }
            if constexpr (i < M1) {
#pragma unroll
                for (int v = i * 16 / M1; v < (i + 1) * 16 / M1; v++) mx = fmaxf(mx, sc[v >> 2][v & 3]);
            } else if constexpr (i == M1) {
                // the row's lanes (col, 0..3): 16 apart, then 32 apart
                const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
                const auto sx = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = fmaxf(__uint_as_float(sx[0]), __uint_as_float(sx[1]));
            } else if constexpr (i == M1 + 1) {
                // lazy rescale: the reference max moves only when a row's max passes it by more than TAU
                // (log2 units), or on the row's first visible keys
                grow = m_run == kNegInf ? mx != kNegInf : mx > m_run + TAU;
                m_new = grow ? mx : m_run;
            } else if constexpr (i == M1 + 2) {
                any_rescale = __builtin_amdgcn_ballot_w64(grow) != 0;
                // 0 on a row's first keys, 1 when unchanged, and 1 for a row that has seen no key yet (both
                // maxima -inf: a row a QSA mask hides from this tile while another row of the wave grows)
                corr = m_new == kNegInf ? 1.f : exp2_fast(m_run - m_new);
                m_use = m_new == kNegInf ? 0.f : m_new;
                m_run = m_new;
            }
            if constexpr (i >= E0) {
#pragma unroll
                for (int e = (i - E0) * 8 / NE; e < (i - E0 + 1) * 8 / NE; e++) {
                    const int cq = e >> 1, j = 2 * (e & 1);
                    f16x2 pp = {(f16)exp2_fast(sc[cq][j] - m_use), (f16)exp2_fast(sc[cq][j + 1] - m_use)};
                    // consumed here: otherwise the exponentials are sunk below the rescale branch that
                    // follows the step and issue after the last matrix instruction instead of beside them
                    asm volatile("" : "+v"(pp));
                    pcur[cq >> 1][(cq & 1) * 4 + j] = pp[0];
                    pcur[cq >> 1][(cq & 1) * 4 + j + 1] = pp[1];
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

    // Software pipeline over the segment's key tiles [lo, hi) (every wave runs every tile; rows past
    // their causal limit see all-masked tiles). Staging: K tiles run two ahead of their use and V tiles
    // one, in two buffers each (tile kt in buffer kt & 1), with one barrier per iteration. The buffers
    // are free here: the previous segment's last barrier follows its last K read, and its last V tile
    // is only overwritten after the first barrier of the loop below.
    // (tile lo + 1 even past hi: the buffer is free and the copy reads zeros or unused blocks, and a
    // fixed number of copies lets the query's loads be waited for without waiting for any copy)
    if constexpr (!PRE) {
        copy_tile(rk, sK(lo & 1), lo);
        copy_tile(rk, sK((lo + 1) & 1), lo + 1);
    }
    {
        // the Q^T operand, while the copies fly (the query loads were issued before them). sW is free:
        // every wave finished the previous segment's reads of it many barriers ago
        if constexpr (PRE) {
            pf_query_fused<D, IN_DT>(a, qraw, sW, row_ok ? t : 0, g, lane, row_ok, qop);
        } else if constexpr (QF) {
            if (wave == 0 && lane < D / 4)
                *reinterpret_cast<f32x4*>(sW + 4 * lane) = f32x4{1.0f + wq[0], 1.0f + wq[1], 1.0f + wq[2], 1.0f + wq[3]};
            // a barrier for the LDS write alone (__syncthreads would also wait for the copies in flight)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            pf_query_fused<D, IN_DT>(a, qraw, sW, row_ok ? t : 0, g, lane, row_ok, qop);
        } else {
#pragma unroll
            for (int ks = 0; ks < NKS; ks++) qop[ks] = row_ok ? qop[ks] : f16x8{};
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    qk_only(sK(lo & 1) + foff_lane);

    // one tile iteration; the first (QK^T only, no P.V) is peeled off by hand so that the loop body is
    // the full step alone
    auto iter = [&](auto do_pv, int kt) __attribute__((always_inline)) {
        constexpr bool DO_PV = decltype(do_pv)::value;
#pragma unroll
        for (int cq = 0; cq < 4; cq++) sc[cq] = sn[cq];
        // this wave's copies are complete; after the barrier every wave's are, and every wave is done
        // with the buffers this iteration's copies overwrite (K tile kt, V tile kt-2)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if (DO_PV && kt * PF_KT > maxlen) {
            zero_tail(sV((kt - 1) & 1), kt - 1);
            __syncthreads();
        }
        const int k0 = kt * PF_KT;
        if constexpr (QSA) {
            // value i of chain cq = 2 b + s holds key 32 b + 8 g + 4 s + i of the tile: bit 8 g + 4 s + i of
            // word b
#pragma unroll
            for (int cq = 0; cq < 4; cq++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    sc[cq][j] = ((((cq >> 1) ? qw1 : qw0) >> (8 * g + 4 * (cq & 1) + j)) & 1u) ? sc[cq][j] : kNegInf;
            qsa_words(kt + 1);
        }
        if (k0 + PF_KT > wave_nomask) {
            // causal edge: value i of chain cq = 2 b + s holds key k0 + 32 b + 8 g + 4 s + i, visible to
            // this lane's row when below len
            const int lim = len - k0 - 8 * g;
#pragma unroll
            for (int cq = 0; cq < 4; cq++)
#pragma unroll
                for (int j = 0; j < 4; j++) sc[cq][j] = (32 * (cq >> 1) + 4 * (cq & 1) + j) < lim ? sc[cq][j] : kNegInf;
        }
        const f16* Kb = sK((kt + 1) & 1) + foff_lane;  // tile kt+1 (stale past the last tile: unused)
        const f16* Vb = sV((kt + 1) & 1) + foff_lane;  // tile kt-1 (no P.V on the first tile)
        step(do_pv, Kb, Vb, kt);
        if (any_rescale) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) acc[dt] *= corr;
        }
        pprev[0] = pcur[0];
        pprev[1] = pcur[1];
    };
    qsa_words(lo);
    iter(std::false_type{}, lo);
    for (int kt = lo + 1; kt < hi; kt++) iter(std::true_type{}, kt);
    // ---- P.V of the last tile ----
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (hi * PF_KT > maxlen) {
        zero_tail(sV((hi - 1) & 1), hi - 1);
        __syncthreads();
    }
    if constexpr (NEXT) {
        // the next segment's rows and K tiles 0 and 1 (both K buffers are free past the barrier above;
        // nothing before the next segment's first barrier reads them)
        if (next_qt >= 0) {
            const int tn = next_qt * tok_per_blk + r / G;
            carry.load(a, tn < a.n ? tn : 0, h, g);
            copy_tile(rk, sK(0), 0);
            copy_tile(rk, sK(1), 1);
        }
    }
    // the gates of this wave's rows, kept as loaded (bf16 pairs or fp32). Bf16 gates of a whole tile are
    // in flight during the last P.V (fp32 ones would need twice the registers and are loaded after it);
    // a split tile's merging wave loads them after the merge. Accumulator register i of dim tile dt of
    // lane (col, g) holds dim 16*dt + 4*g + i.
    using graw_t = typename std::conditional<IN_DT == 0, f32x4, u32x2_t>::type;
    graw_t graw[NDT];
    const size_t gb = ((size_t)(row_ok ? t : 0) * a.NH + h) * 2 * D + D + 4 * g;
    auto load_gates = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            if constexpr (IN_DT == 0)
                graw[dt] = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.qg) + gb + dt * 16);
            else
                graw[dt] = *reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(a.qg) + gb + dt * 16);
        }
    };
    auto gate = [&](int dt, int i) __attribute__((always_inline)) -> float {
        if constexpr (IN_DT == 0) return graw[dt][i];
        else return __uint_as_float((i & 1) ? graw[dt][i >> 1] & 0xffff0000u : graw[dt][i >> 1] << 16);
    };
    constexpr bool kGateEarly = IN_DT == 1;
    if (kGateEarly && slot < 0) load_gates();
    pv_only(sV((hi - 1) & 1) + foff_lane);

    // ---- epilogue: l across the row's four lanes, merge of a split tile, normalize, gate, store ----
    {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
        l_run = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        const auto sx = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
        l_run = __uint_as_float(sx[0]) + __uint_as_float(sx[1]);
    }
    if (slot >= 0) {
        // a wave's partial: accumulator dim tile dt of every lane as 1 KB, then (max, sum) per lane;
        // each half of the tile has its own region (half 1: keys from lo > 0) and reads the other's
        constexpr int PSTR = pf_part_floats(D);
        const int own = lo > 0 ? 1 : 0;
        float* pw = a.part + (((size_t)slot * 2 + own) * kPfWaves + wave) * PSTR;
        float* pr = a.part + (((size_t)slot * 2 + (1 - own)) * kPfWaves + wave) * PSTR;
        int* cw = a.cnt + slot * kPfWaves + wave;
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(pw, (short)0, PSTR * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(pr, (short)0, PSTR * 4, 0x00020000);
        const float mu = m_run == kNegInf ? 0.f : m_run;  // the offset the weights were taken against
        int other = __builtin_amdgcn_readfirstlane(__hip_atomic_load(cw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (other == 0) {
            // first (as far as this wave can tell): publish the partial (device-coherent stores,
            // acknowledged before the arrival is counted), then count
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) __builtin_amdgcn_raw_buffer_store_b128(acc[dt], rp, (dt * 64 + lane) * 16, 0, kScDevice);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, f32x2{mu, l_run}), rp,
                                                  NDT * 64 * 16 + lane * 8, 0, kScDevice);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            int old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(cw, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            other = __builtin_amdgcn_readfirstlane(old);
            if (other == 0) return;  // the partner wave merges
        }
        // the partner's loads stay behind the count that says its partial is complete
        asm volatile("" ::: "memory");
        // second: the partner's partial (published before its count) merged into this wave's, one dim
        // tile at a time with two more in flight (the whole partial in registers at once would spill)
        const f32x2 ml2 = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rq, NDT * 64 * 16 + lane * 8, 0, kScDevice));
        constexpr int NB = NDT < 6 ? NDT : 6;
        f32x4 o2[NB];
        auto load_dt = [&](int dt) __attribute__((always_inline)) {
            o2[dt % NB] = __builtin_amdgcn_raw_buffer_load_b128(rq, (dt * 64 + lane) * 16, 0, kScDevice);
        };
        static_for<0, NB - 1>([&](auto ic) __attribute__((always_inline)) { load_dt(ic.value); });
        if (lane == 0) __hip_atomic_store(cw, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // fixed order whichever wave merges: the key-suffix half (lo > 0) is the first term, so the
        // result does not depend on arrival order
        const bool own_first = own == 1;
        const float muf = own_first ? mu : ml2[0], mus = own_first ? ml2[0] : mu;
        const float lf = own_first ? l_run : ml2[1], ls = own_first ? ml2[1] : l_run;
        const bool vf = lf > 0.f, vs = ls > 0.f;
        const float mx = vf ? (vs ? fmaxf(muf, mus) : muf) : mus;
        const float cf = vf ? exp2_fast(muf - mx) : 0.f, cs = vs ? exp2_fast(mus - mx) : 0.f;
        l_run = __builtin_fmaf(ls, cs, lf * cf);
        static_for<0, NDT>([&](auto ic) __attribute__((always_inline)) {
            constexpr int dt = decltype(ic)::value;
            if constexpr (dt + NB - 1 < NDT) load_dt(dt + NB - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float x = acc[dt][i], y = o2[dt % NB][i];
                acc[dt][i] = __builtin_fmaf(own_first ? y : x, cs, (own_first ? x : y) * cf);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    if (!kGateEarly || slot >= 0) load_gates();
    if (row_ok) {
        const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
        const size_t ob = ((size_t)t * a.NH + h) * D;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            f32x4 o;
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = acc[dt][i] * inv * sigmoid(gate(dt, i));
            *reinterpret_cast<f32x4*>(a.out + ob + dt * 16 + 4 * g) = o;
        }
    }
}

// Workgroup j of KV head kvh (blockIdx = j * NKV + kvh). Pair p = j / 2 holds query tiles p (short) and
// n_qt-1-p (long) with T = nl + ns key tiles: j = 2p runs the long tile over [x, nl), j = 2p+1 its
// first x tiles, then the short tile, x = max(0, nl - ceil(T/2)). With n_qt odd the last workgroup
// runs the middle tile alone.
template <int D, int IN_DT, bool QF, bool QSA>
__global__ __launch_bounds__(64 * kPfWaves, 1) void k_prefill(PrefillArgs a) {
    const int G = a.NH / a.NKV;
    const int tok_per_blk = PF_ROWS / G;
    const int n_qt = (a.n + tok_per_blk - 1) / tok_per_blk;
    const int kvh = blockIdx.x % a.NKV, j = blockIdx.x / a.NKV;
    const int np = n_qt / 2;
    // segments (query tile, key tiles [lo, hi), partial slot) of this workgroup, in order
    int q0, lo0, hi0, slot0, q1 = 0, hi1 = 0, nseg = 1;
    if (a.split_all) {  // two workgroups per tile, longest tiles first: keys [x, nt) and [0, x)
        const int qt = n_qt - 1 - (j >> 1);
        const int nt = pf_tiles(a, tok_per_blk, qt), x = nt / 2;
        if (x == 0 && (j & 1)) return;  // a one-tile range is not split: the partner runs it whole
        q0 = qt, lo0 = (j & 1) ? 0 : x, hi0 = (j & 1) ? x : nt, slot0 = x > 0 ? kvh * a.slots + qt : -1;
    } else if (j >= 2 * np) {  // the middle tile
        q0 = np, lo0 = 0, hi0 = pf_tiles(a, tok_per_blk, np), slot0 = -1;
    } else {
        const int p = j >> 1, ql = n_qt - 1 - p;
        const int nl = pf_tiles(a, tok_per_blk, ql), ns = pf_tiles(a, tok_per_blk, p);
        const int x = max(0, nl - (nl + ns + 1) / 2);
        slot0 = x > 0 ? kvh * a.slots + p : -1;
        if ((j & 1) == 0) {
            q0 = ql, lo0 = x, hi0 = nl;
        } else if (x > 0) {  // the long tile's prefix first: its partial is published long before the partner ends
            q0 = ql, lo0 = 0, hi0 = x, q1 = p, hi1 = ns, nseg = 2;
        } else {
            q0 = p, lo0 = 0, hi0 = ns;
        }
    }
    PfQRaw<D, IN_DT> carry;
    if constexpr (pf_handover(QF, IN_DT)) {
        // two call sites: the rows handed over are live only between the first segment's loop and the
        // second's prologue (through one runtime segment loop they would stay live through every tile)
        pf_segment<D, IN_DT, QF, QSA, false>(a, kvh, q0, lo0, hi0, slot0, nseg == 2 ? q1 : -1, carry);
        if (nseg == 2) pf_segment<D, IN_DT, QF, QSA, true>(a, kvh, q1, 0, hi1, -1, -1, carry);
    } else {
        // one call site, so the segment body exists once in the code object
        for (int s = 0; s < nseg; s++)
            pf_segment<D, IN_DT, QF, QSA, false>(a, kvh, s ? q1 : q0, s ? 0 : lo0, s ? hi1 : hi0, s ? -1 : slot0, -1, carry);
    }
}

template <int D>
static hipError_t launch_pf_d(const PrefillArgs& a, int q_dtype, int in_dtype, hipStream_t s) {
    using C = PfCfg<D>;
    const int G = a.NH / a.NKV;
    const int tok = PF_ROWS / G;
    const int n_qt = (a.n + tok - 1) / tok;
    // the split tiles' partial slots and counters are the caller's (sized for `slots` per KV head)
    if (a.n < 1 || a.slots != pf_split_slots(n_qt, a.split_all) || (a.slots > 0 && (!a.part || !a.cnt)))
        return hipErrorInvalidValue;
    const dim3 grid((a.split_all ? 2 : 1) * n_qt * a.NKV), block(64 * kPfWaves);
    // two buffers of a K and a V tile; with in-kernel query normalization, the D norm multipliers after them
    const size_t shm = 2 * 2 * (size_t)C::TILEE * 2 + (a.q ? 0 : D * sizeof(float));
    auto go = [&](auto kern) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, block, shm, s, a);
        return hipGetLastError();
    };
    // fp32 queries reach this kernel converted to the fp16 operand (launch_q_f16); without q the kernel
    // normalizes the query half of qg itself
    if (q_dtype != 2) return hipErrorInvalidValue;
    if (!a.q) {
        if (!a.qn || (a.R && !a.rope) || !pf_fused_rope_ok(a.R, D)) return hipErrorInvalidValue;
        if (a.kbits) return in_dtype == 0 ? go(k_prefill<D, 0, true, true>) : go(k_prefill<D, 1, true, true>);
        return in_dtype == 0 ? go(k_prefill<D, 0, true, false>) : go(k_prefill<D, 1, true, false>);
    }
    if (a.kbits) return in_dtype == 0 ? go(k_prefill<D, 0, false, true>) : go(k_prefill<D, 1, false, true>);
    return in_dtype == 0 ? go(k_prefill<D, 0, false, false>) : go(k_prefill<D, 1, false, false>);
}

// fp16(q * scale): the prefill operand from fp32 queries; n4 groups of 4 values
__global__ __launch_bounds__(256) void k_q_f16(const f32x4* __restrict__ q, f16x4* __restrict__ o, float scale, size_t n4) {
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const f32x4 v = q[i];
        o[i] = f16x4{(f16)(v[0] * scale), (f16)(v[1] * scale), (f16)(v[2] * scale), (f16)(v[3] * scale)};
    }
}

hipError_t launch_q_f16(const float* q, void* out, float scale, size_t n, hipStream_t s) {
    if (n % 4) return hipErrorInvalidValue;
    const size_t n4 = n / 4;
    const unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 4096);
    hipLaunchKernelGGL(k_q_f16, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const f32x4*>(q), static_cast<f16x4*>(out), scale, n4);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int D, int q_dtype, int in_dtype, hipStream_t s) {
    if (D == 256) return launch_pf_d<256>(a, q_dtype, in_dtype, s);
    if (D == 128) return launch_pf_d<128>(a, q_dtype, in_dtype, s);
    return launch_pf_d<64>(a, q_dtype, in_dtype, s);
}

}  // namespace qw
