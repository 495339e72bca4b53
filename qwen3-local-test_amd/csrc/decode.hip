// Split-KV causal GQA attention for decode and MTP verify, plus the log-sum-exp combine, for gfx950.
//
// Replaces shaders/attention.comp (attention_kv16) and shaders/attn_combine.comp, and — in the fused
// form used by the layer entry point — also shaders/qk_norm_rope.comp for the new tokens. Semantics per
// query row (token t, head h): keys j < len_t = pos + t + 1, score q.k_j / sqrt(D), softmax, times V;
// the key axis [0, pos + n) is cut into chunks, each chunk leaves an unnormalized partial (m, l, o[D])
// (attention.comp:26-75), and the combine merges them, skipping l = 0 splits, then applies
// sigmoid(gate) (attn_combine.comp:13-29).
//
// MI355X design (not the reference's):
//  - One workgroup per (chunk, KV head) serves every query row that shares the KV head — the G = NH/NKV
//    heads of each of the n tokens, 8 or 16 rows — so each K/V row leaves HBM once (the reference runs
//    one workgroup per query head and relies on L2 for the G-fold re-read). More than 16 rows (the
//    4-token verify at G = 8) go to 16-row slices on grid.z: the slices of a chunk run side by side, so
//    the second read of the chunk is served by the 256 MB Infinity Cache, and each slice keeps the
//    register budget that lets it double-buffer its tiles.
//  - The cache's blocked layout (common.hpp) makes every MFMA operand fragment one contiguous kilobyte,
//    so a 32-key tile (K and V, 32 KB at D = 256) moves with 32 fully coalesced 16-byte-per-lane loads.
//  - Up to 8 rows (k_decode_ld: single-token decode, n * G <= 8): two loader waves copy tiles straight
//    into LDS (buffer_load ... lds) through a two-slot ring per compute wave and publish each landed tile
//    through an LDS counter; two compute waves take a tile into registers, free its slot at once and
//    compute on it, so each compute wave sees up to two tiles in flight with no register cost. The
//    copies start at launch, right after the compute waves have issued their row loads, so the prologue
//    (norm, RoPE, cache append) runs under the first tiles' latency.
//  - More rows (k_decode, 16-row slices): each wave streams its tiles straight into the operand
//    registers, two tiles in flight (register double buffering): the next-but-one tile's K loads go out
//    as soon as the current tile's scores are done, its V loads as soon as P.V is done.
//  - S^T[32 keys x rows] = K . Q^T and O^T[D x rows] += V^T . P^T on v_mfma_f32_16x16x32_f16 with fp32
//    accumulation. Q and P are carried as an fp16 "hi" part plus an fp16 "lo" remainder (22 mantissa
//    bits together), so scores and weights keep fp32-level accuracy against the fp16 cache; with at most
//    8 rows the lo parts ride in the otherwise unused columns 8-15 of the same MFMA.
//  - Scores are in log2 units (q pre-multiplied by log2(e)/sqrt(D)), so exponentials are v_exp_f32.
//  - Fused form: every workgroup normalizes and rotates its own query rows (RMSNorm (1+w) + partial
//    RoPE, while its first tiles are in flight), and the workgroup whose chunk holds the n new positions
//    normalizes/rotates their K rows, writes K and V to the cache and attends over them (the decode
//    kernel copies their block once the stores are complete, the verify kernel patches them into its
//    loaded tiles) — so one launch does the work of the reference's qk_norm_rope + attention dispatches.
//  - The combine runs one workgroup per (row, 64-dim slice) with every partial load of a batch issued
//    before any is used.
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"

namespace qw {

// k_decode: a slice of 16 query rows, hi and lo parts of Q and P as two MFMAs into one accumulator.
template <int D>
struct DecCfg {
    static constexpr int NKS = D / 32;                     // k-steps of the QK^T product
    static constexpr int NDT = D / 16;                     // 16-dim tiles of the P.V product
    static constexpr int RMAX = 16;                        // query rows of the workgroup
    static constexpr int NQS = 2;                          // Q fragment sets in LDS (hi, lo)
    static constexpr int QBYTES = NQS * NKS * 1024;
    static constexpr int OSTRIDE = D + 4;                  // floats per row of the wave-partial buffer
    static constexpr int MBYTES = 4 * RMAX * OSTRIDE * 4;
    static constexpr int UBYTES = QBYTES > MBYTES ? QBYTES : MBYTES;
    static constexpr int BLKE = kBlk * D;                  // elements of one (block, KV head) part
    static constexpr int NB = 2;                           // blocks the new positions of a pass can span
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x8 as_h8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ u32x4 as_u4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

// s_waitcnt immediate for "at most n vector-memory loads outstanding" (gfx9 encoding: vmcnt split over
// bits 3:0 and 15:14, expcnt and lgkmcnt left at their maxima)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Key range [kb, ke) of split z: whole 32-key blocks, split z holding the blocks
// [z*cq + min(z, cr), (z+1)*cq + min(z+1, cr)) of the ceil(maxlen/32) that hold keys (the host keeps
// cq >= 1, so no split is empty). The first cr splits are one block longer, so the last split, whose
// workgroup also appends the new rows, is never the longest.
__device__ __forceinline__ void split_keys(const DecodeArgs& a, int z, int maxlen, int& kb, int& ke) {
    const int b0 = z * a.cq + min(z, a.cr);
    const int b1 = b0 + a.cq + (z < a.cr ? 1 : 0);
    kb = b0 * kBlk;
    ke = min(maxlen, b1 * kBlk);
}

// Tag of a split record of the one-launch decode: the launch's epoch and the KV head. A head's epoch only
// grows, and the head is part of the tag, so a record left by an earlier launch — whatever its head, split
// count or row layout was — never carries the tag a combiner waits for.
__device__ __forceinline__ unsigned long long rec_tag(unsigned long long epoch, int kvh) {
    return (epoch << 5) | (unsigned)kvh;  // NKV <= 32 (host-checked)
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The launch's tag from the head's counter as a streaming workgroup read it at its start, computed where
// the records are stored. The empty asm marks the value as lane-varying, so the compiler keeps it in the
// vector registers it was loaded into; treated as uniform, it is moved to scalar registers right at the
// load, which waits for that load before anything else of the workgroup is issued.
__device__ __forceinline__ unsigned long long tag_of(u32x2 raw, int kvh) {
    asm volatile("" : "+v"(raw));
    const unsigned long long cnt = __builtin_bit_cast(unsigned long long, raw);
    return rec_tag(cnt / kEpochStep + 1u, kvh);
}

// A bounded wait gave up: the launch's output is not valid. The code goes to the host-visible error word
// (the first code stored wins: a later one does not overwrite it).
__device__ __forceinline__ void report_wait(const DecodeArgs& a, int code) {
    if (a.err != nullptr) {
        int expected = 0;
        __hip_atomic_compare_exchange_strong(a.err, &expected, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_SYSTEM);
    }
}


// Rows of the fused prologues (query rows, new key rows), one row per 32-lane half-wave and D/32
// consecutive dims per lane from d0 = (lane & 31) * D/32: y = x * rsqrt(mean(x^2) + eps) * (1 + w), then
// rotate-half RoPE on d < R with the (cos, sin) pairs cv (as k_qk_norm_rope: the partner dim d +- R/2
// sits (R/2)/(D/32) lanes away in the same half; `rot`: this lane's dims are rotated). NP rows at once,
// every step of every row issued before the next step, so the rows' latencies overlap; the mean of
// squares is a DPP/permlane sum (sum32), the partners one LDS-free-address shuffle each. Rows not `valid`
// come out as zero.
template <int D, int NP>
__device__ __forceinline__ void norm_rope_rows(const DecodeArgs& a, int lane, bool rot, const float (&xr)[NP][D / 32],
                                               const float (&cv)[NP][D / 16], const bool (&valid)[NP],
                                               const float (&w)[D / 32], float (&y)[NP][D / 32]) {
    constexpr int DPL2 = D / 32;
    const int d0 = (lane & 31) * DPL2, half_r = a.R >> 1;
    float ss[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        ss[p] = 0.f;
#pragma unroll
        for (int jj = 0; jj < DPL2; jj++) {
            y[p][jj] = valid[p] ? xr[p][jj] : 0.f;
            ss[p] += y[p][jj] * y[p][jj];
        }
    }
#pragma unroll
    for (int p = 0; p < NP; p++) ss[p] = sum32(ss[p]);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const float r = 1.0f / sqrtf(ss[p] / (float)D + a.eps);
#pragma unroll
        for (int jj = 0; jj < DPL2; jj++) y[p][jj] = y[p][jj] * r * (1.0f + w[jj]);
    }
    const int offl = half_r / DPL2;
    const bool lo_half = d0 < half_r;
    const int src_lane = rot ? (lo_half ? lane + offl : lane - offl) : lane;
    float partner[NP][DPL2];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int jj = 0; jj < DPL2; jj++) partner[p][jj] = __shfl(y[p][jj], src_lane, 64);  // all issued, then used
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int jj = 0; jj < DPL2; jj++) {
            const float cs = rot ? cv[p][2 * jj] : 1.f, sn = rot ? cv[p][2 * jj + 1] : 0.f;
            y[p][jj] = lo_half ? y[p][jj] * cs - partner[p][jj] * sn : y[p][jj] * cs + partner[p][jj] * sn;
        }
}

// Merges a batch of split partials (m, l, o) into the running (M, L, O) (attn_combine.comp:17-26: the
// max over the splits with keys, then each partial weighted by exp2(m - max)), in a fixed order and
// without branches: with a branch per split the compiler sinks that split's loads into it and then waits
// for them one split at a time, a memory round trip per split instead of one per batch. Bit k of `keys`
// marks a split of the batch that exists and has keys (l > 0); the others weigh 0 (their o is finite).
template <int B>
__device__ __forceinline__ void merge_batch(float& M, float& L, f32x4& O, const float (&m)[B], const float (&l)[B],
                                            const f32x4 (&o)[B], unsigned keys) {
    float mx = M;  // -inf (with L = 0) before the first split with keys
#pragma unroll
    for (int k = 0; k < B; k++) mx = (keys >> k) & 1 ? fmaxf(mx, m[k]) : mx;
    const float cf = L > 0.f ? exp2_fast(M - mx) : 0.f;
    L *= cf;
    O *= cf;
#pragma unroll
    for (int k = 0; k < B; k++) {
        const float w = (keys >> k) & 1 ? exp2_fast(m[k] - mx) : 0.f;
        L += l[k] * w;
        O += o[k] * w;
    }
    M = mx;
}

// In-launch log-sum-exp combine of the one-launch decode (attn_combine.comp:13-29): one workgroup per
// (output row (t, h), slice of DW = D / nds dims), one of the last chunks of its KV head or 16-row slice
// once its own partials are out, merges that row's split partials over its dims as they arrive. A
// streaming workgroup stores its rows' unnormalized o[D] (device-coherent stores), waits for them to be
// acknowledged, then stores each row's record (m, l, 64-bit tag): a record carrying this launch's tag
// guarantees the row's o is visible. The combiner takes the splits in windows of kCombSlots: wave w owns
// the kCombGroup splits [wb + 32 w, wb + 32 w + 32) of window wb, lane j < 32 polling split wb + 32 w + j's
// record (one 16-byte device-coherent load per round); each split that has arrived has its DW dims loaded
// straight into the wave's registers, 16 bytes a lane: lane group g (LPP = DW / 4 lanes) holds splits
// g NL .. g NL + NL - 1 of the wave's 32. Once its group is complete the wave takes the group's max and
// weights (wave reductions, the weights broadcast through LDS), its weighted sum per lane and then across
// the lane groups; the window's four group results meet in LDS and merge into the running (M, L, O) in
// group order — a fixed order, so the result does not depend on which split arrives first. Splits with
// l = 0 are skipped. Slicing the dims (nds = 4 at decode: 32 combiners of a KV head's 128 chunks) divides
// what one combiner loads (128 splits x DW x 4 bytes) and sums, the tail of the launch. The epoch: see
// kEpochStep. Every wait is bounded (a.spin_max polling rounds); a combiner that gives up reports
// kWaitCombineFlags and merges whatever its registers hold. The host keeps the combiners at half of each
// KV head's (slice's) chunks or fewer, so every wait ends while more CUs than that are free to the launch.
template <int D, int IN_DT, int DW>
__device__ __forceinline__ void combine_slice(const DecodeArgs& a, unsigned char* smem, int r, int ds) {
    constexpr int NS = kCombSlots, GS = kCombGroup;
    constexpr int LPP = DW / 4, PPL = 64 / LPP, NL = GS / PPL;  // lanes a split, splits a load, loads a wave
    static_assert(NS == 4 * GS && GS == 32, "one group of 32 splits per wave and window");
    static_assert(DW % 16 == 0 && DW <= 256 && DW <= D, "16 to 256 dims a combiner, 4 a lane");
    float* s_go = reinterpret_cast<float*>(smem);  // [4][DW] the window's group sums
    float* s_gm = s_go + 4 * DW;                    // [4] group maxima (log2 units)
    float* s_gl = s_gm + 4;                         // [4] group sums of l
    float* s_w = s_gl + 4;                          // [4][GS] each group's weights
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lg = lane / LPP, d4 = (lane % LPP) * 4;  // lane group, first of the lane's 4 dims in the slice
    const int S = a.n_split, G = a.NH / a.NKV;
    const int t = r / a.NH, h = r % a.NH, kvh = h / G;
    const int d0 = ds * DW;
    const unsigned long long cnt = __hip_atomic_load(a.ep + kvh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // this launch's record tag (see rec_tag), skewed by the test hook
    const unsigned long long want = rec_tag(cnt / kEpochStep + 1u + (unsigned long long)(long long)a.epoch_skew, kvh);
    const float gate = tid < DW ? load_in<IN_DT>(a.q, ((size_t)t * a.NH + h) * 2 * D + D + d0 + tid) : 0.f;
    const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(a.rec + (size_t)r * S * 4, (short)0, S * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(a.part_o + (size_t)r * S * D, (short)0, S * D * 4, 0x00020000);
    int spins = 0;
    bool gave_up = false;
    float M = kNegInf, L = 0.f, O = 0.f;  // thread tid < DW: running state of dim d0 + tid
    for (int wb = 0; wb < S; wb += NS) {
        const int z0 = wb + wave * GS;                 // this wave's first split (wave-uniform)
        const int nz = max(0, min(GS, S - z0));        // its splits in this window
        const int z = z0 + lane;
        bool pend = lane < nz;                         // lane j: split z0 + j not arrived yet
        float mj = kNegInf, lj = 0.f;
        f32x4 ov[NL];  // splits past S stay zero (weight 0 too), so the group sum needs no per-split guard
#pragma unroll
        for (int k = 0; k < NL; k++) ov[k] = f32x4{};
        while (__ballot(pend) != 0) {
            const f32x4 rv = __builtin_amdgcn_raw_buffer_load_b128(rrec, (pend ? z : 0) * 16, 0, kScDevice);
            const bool last = ++spins > a.spin_max;
            const bool match = (__float_as_uint(rv[2]) | ((unsigned long long)__float_as_uint(rv[3]) << 32)) == want;
            const bool got = pend && (match || last);
            gave_up |= got && !match;
            if (got) mj = rv[0], lj = rv[1];
            pend = pend && !got;
            const unsigned long long b = __ballot(got);
            // each arrived split's dims: lane group lg loads split lg NL + k into register slot k (static)
#pragma unroll
            for (int k = 0; k < NL; k++) {
                const int j = lg * NL + k;
                if ((b >> j) & 1) ov[k] = __builtin_amdgcn_raw_buffer_load_b128(ro, ((z0 + j) * D + d0 + d4) * 4, 0, kScDevice);
            }
            if (b == 0) __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        // the group's max and weights: lane j < nz holds split z0 + j's (m, l)
        // (DPP/permlane butterflies over the 32 lanes: no LDS round trips)
        const bool use = lane < nz && lj > 0.f;
        const float mg = max32(use ? mj : kNegInf);
        const float w = use ? exp2_fast(mj - mg) : 0.f;
        const float lsum = sum32(lj * w);
        // the weights to every lane through LDS (broadcast reads): lane j < 32 holds split z0 + j's
        if (lane < GS) s_w[wave * GS + lane] = w;
        float wv[NL];
#pragma unroll
        for (int k = 0; k < NL; k += 4) {
            if constexpr (NL >= 4) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(&s_w[wave * GS + lg * NL + k]);
                wv[k] = x[0], wv[k + 1] = x[1], wv[k + 2] = x[2], wv[k + 3] = x[3];
            } else {
#pragma unroll
                for (int u = 0; u < NL; u++) wv[u] = s_w[wave * GS + lg * NL + u];
            }
        }
        f32x4 og = {};
#pragma unroll
        for (int k = 0; k < NL; k++) og += ov[k] * wv[k];
        // the lane groups' sums (a fixed butterfly: the same order whatever arrived when)
#pragma unroll
        for (int sh = LPP; sh < 64; sh <<= 1)
#pragma unroll
            for (int e = 0; e < 4; e++) og[e] += __shfl_xor(og[e], sh, 64);
        if (lane < LPP) *reinterpret_cast<f32x4*>(&s_go[wave * DW + d4]) = og;
        if (lane == 0) {
            s_gm[wave] = mg;
            s_gl[wave] = lsum;
        }
        __syncthreads();
        if (tid < DW) {
#pragma unroll
            for (int gi = 0; gi < 4; gi++) {  // the window's groups in order
                const float gl = s_gl[gi];
                if (gl > 0.f) {
                    const float gm = s_gm[gi], mn = fmaxf(M, gm);
                    const float cf = L > 0.f ? exp2_fast(M - mn) : 0.f, cg = exp2_fast(gm - mn);
                    L = L * cf + gl * cg;
                    O = O * cf + s_go[gi * DW + tid] * cg;
                    M = mn;
                }
            }
        }
        __syncthreads();  // s_go is rewritten by the next window
    }
    if (tid < DW) a.out[((size_t)t * a.NH + h) * D + d0 + tid] = (L > 0.f ? O / L : 0.f) * sigmoid(gate);
    if (__ballot(gave_up) != 0 && lane == 0) report_wait(a, kWaitCombineFlags);
    if (tid == 0) {  // this combiner is done: its share of the head's epoch step (see kEpochStep)
        const unsigned m = (unsigned)(a.ncomb / a.NKV * a.nds), j = (unsigned)((t * G + h % G) * a.nds + ds);
        __hip_atomic_fetch_add(a.ep + kvh, (unsigned long long)((j + 1) * kEpochStep / m - j * kEpochStep / m),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The combiner of output row r, dims slice ds of a.nds (1, 2, 4 or 8: host-checked)
template <int D, int IN_DT>
__device__ __forceinline__ void combine_row(const DecodeArgs& a, unsigned char* smem, int r, int ds) {
    if constexpr (D / 8 >= 16)
        if (a.nds == 8) return combine_slice<D, IN_DT, D / 8>(a, smem, r, ds);
    if (a.nds == 4) combine_slice<D, IN_DT, D / 4>(a, smem, r, ds);
    else if (a.nds == 2) combine_slice<D, IN_DT, D / 2>(a, smem, r, ds);
    else combine_slice<D, IN_DT, D>(a, smem, r, ds);
}

template <int D, int FUSED, int IN_DT, int QSA>
__global__ __launch_bounds__(256, 1) void k_decode(DecodeArgs a) {
    using C = DecCfg<D>;
    constexpr int NKS = C::NKS, NDT = C::NDT, RMAX = C::RMAX, BLKE = C::BLKE, NB = C::NB;
    constexpr int NPT = 2;                  // P operands (hi, lo) per tile
    constexpr int DPL2 = D / 32;            // dims per lane in the row passes
    constexpr int QPASS = RMAX / 8;         // query-row passes per wave
    constexpr float TAU = 8.f;              // a running max moves only when exceeded by this (log2 units)

    __shared__ __attribute__((aligned(16))) unsigned char s_u[C::UBYTES];  // Q fragments, then wave partials
    // new positions (fused): images of their cache blocks, [K, V][block], in the cache's blocked layout
    __shared__ __attribute__((aligned(16))) f16 s_img[FUSED ? 2 * NB : 1][FUSED ? BLKE : 8];
    __shared__ float sM[4][RMAX], sL[4][RMAX], sF[4][RMAX];
    __shared__ unsigned s_qw[QSA ? RMAX : 1][QSA ? kQsaChunkTiles : 1];  // QSA: [slice token][chunk tile] key bits
    f16* s_q = reinterpret_cast<f16*>(s_u);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, g = lane >> 4;
    const int z = blockIdx.x, kvh = blockIdx.y;
    const int G = a.NH / a.NKV;
    const int r0 = blockIdx.z * RMAX;                  // first query row of this slice
    const int rows = min(RMAX, a.n * G - r0);          // query rows of this workgroup
    const int maxlen = a.pos + a.n;
    // one-launch verify: the partials are combined in this launch by the slice's last `rows` chunks (see
    // tail_combine below); the head's launch counter for the epoch tag is read now, before this
    // workgroup stores its records, so its latency hides behind the whole stream
    const bool one = FUSED && a.out != nullptr;
    u32x2 ep_raw = {0u, 0u};
    if constexpr (FUSED) {
        const __amdgpu_buffer_rsrc_t rep = __builtin_amdgcn_make_buffer_rsrc(one ? a.ep + kvh : a.ep, (short)0, one ? 8 : 0, 0x00020000);
        ep_raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rep, 0, 0, kScDevice));
    }
    int kb, ke;
    split_keys(a, z, maxlen, kb, ke);
    const int ntile_wg = (ke - kb + 31) >> 5;
    const int ntile = ntile_wg > wave ? (ntile_wg - wave + 3) >> 2 : 0;  // tiles wave, wave + 4, ...
    // QSA: the key bits of the slice's tokens over this chunk (one word per 32-key tile) into LDS, first
    // thing, while few registers are live (the host keeps a chunk at kQsaChunkTiles tiles or fewer)
    const int tok0 = r0 / G;
    if constexpr (QSA) {
        for (int i = tid; i < RMAX * kQsaChunkTiles; i += 256) {
            const int u = i / kQsaChunkTiles, t = i % kQsaChunkTiles;
            s_qw[u][t] = tok0 + u < a.n && t < ntile_wg ? a.kbits[(size_t)(tok0 + u) * a.kb_words + (kb >> 5) + t] : 0u;
        }
    }
    const int new_lo = FUSED ? a.pos : maxlen;        // first position not read from the cache

    // Buffer resources over this chunk's blocks of this KV head. Tiles past the blocks that hold cached
    // positions (the chunk end, or — fused — blocks of new positions only) fall outside the range and
    // load zeros without touching memory, so every prefetch is issued unconditionally.
    const int load_end = min(ke, new_lo);
    const int nload = load_end > kb ? ((load_end - 1) >> 5) - (kb >> 5) + 1 : 0;
    const int bstride = BLKE * 2;  // bytes between consecutive blocks of one head
    const size_t part0 = kv_part(kb, kvh, a.cap, D);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kc) + part0, (short)0, nload * bstride, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.vc) + part0, (short)0, nload * bstride, 0x00020000);
    auto load_k = [&](f16x8 (&kt)[NKS][2], int t) {  // t: tile index within the chunk
        const int off = t * bstride + lane * 16;
#pragma unroll
        for (int kk = 0; kk < NKS; kk++)
#pragma unroll
            for (int s = 0; s < 2; s++)
                kt[kk][s] = as_h8(__builtin_amdgcn_raw_buffer_load_b128(rk, off + (kk * 2 + s) * 1024, 0, 0));
    };
    auto load_v = [&](f16x8 (&vt)[NDT], int t) {
        const int off = t * bstride + lane * 16;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) vt[dt] = as_h8(__builtin_amdgcn_raw_buffer_load_b128(rv, off + dt * 1024, 0, 0));
    };

    // ---- row passes: query rows (and, fused, the new K/V rows) normalized and rotated -------------
    // Two rows per wave per pass, 32 lanes per row, DPL2 dims per lane. Their loads are issued before
    // the tile loads: load completion is counted in order, so the passes finish while tiles stream in.
    const int hw = lane >> 5, hl = lane & 31, d0 = hl * DPL2;
    const int t_lo = FUSED ? max(a.pos, kb) - a.pos : 0;
    const int t_hi = FUSED ? max(t_lo, min(maxlen, ke) - a.pos) : 0;
    const int half_r = a.R >> 1;
    float wq[DPL2], wk[DPL2];
    float qx[QPASS][DPL2], qcv[QPASS][2 * DPL2];
    float nx[1][DPL2], ncv[1][2 * DPL2], nv[DPL2];
    bool qvalid[QPASS];
    const bool rot = FUSED && d0 < a.R;  // lanes whose DPL2 dims are rotated (R/2 is a multiple of DPL2)
    // one row's DPL2 values and (cos, sin) pairs: raw loads only (an invalid row reads row 0, lanes
    // outside the rotated dims read the start of the table, padded for this); validity is applied
    // when the row is finished, so nothing here waits for memory
    auto issue_row = [&](float (&x)[DPL2], float (&cv)[2 * DPL2], const void* src, size_t off, int p, bool valid) {
        load_vec<FUSED ? IN_DT : 0, DPL2>(src, (valid ? off : 0) + d0, x);
        if constexpr (FUSED) {
            const int i0 = rot ? (d0 < half_r ? d0 : d0 - half_r) : 0;
            load_vec<0, 2 * DPL2>(a.rope, (size_t)(valid && rot ? p : 0) * a.R + 2 * i0, cv);
        }
    };
#pragma unroll
    for (int ps = 0; ps < QPASS; ps++) {
        const int r = ps * 8 + wave * 2 + hw;  // row within the slice
        const bool valid = r < rows;
        const int t = valid ? (r0 + r) / G : 0, h = kvh * G + (valid ? (r0 + r) % G : 0);
        qvalid[ps] = valid;
        if constexpr (FUSED) issue_row(qx[ps], qcv[ps], a.q, ((size_t)t * a.NH + h) * 2 * D, a.pos + t, valid);
        else issue_row(qx[ps], qcv[ps], a.q, ((size_t)t * a.NH + h) * D, 0, valid);
    }
    const int tn = t_lo + wave * 2 + hw;  // new row of this half-wave (fused)
    const bool has_new = FUSED && tn < t_hi;
    if constexpr (FUSED) {
        load_vec<0, DPL2>(a.qn, d0, wq);
        load_vec<0, DPL2>(a.kn, d0, wk);
        const size_t src = ((size_t)(has_new ? tn : 0) * a.NKV + kvh) * D;
        issue_row(nx[0], ncv[0], a.knew, src, a.pos + (has_new ? tn : 0), has_new);
        load_vec<IN_DT, DPL2>(a.vnew, src + d0, nv);
    }

    // ---- first tile in flight (kept after the row loads and before their use); the second follows the
    // passes. Load completion is counted in order with a 6-bit counter: the passes wait for their own
    // loads by allowing the younger tile loads to stay outstanding, which works while those number at
    // most 63. And with HBM saturated, issuing a load stalls the wave until earlier requests drain, so
    // nothing the passes could do should wait behind a long burst of tile loads.
    f16x8 kA[NKS][2], kB[NKS][2], vA[NDT], vB[NDT];
    static_assert(2 * NKS + NDT <= 63, "row-pass wait must fit the load counter");
    __builtin_amdgcn_sched_barrier(0);
    load_k(kA, wave);
    load_v(vA, wave);
    __builtin_amdgcn_sched_barrier(0);

    // ---- finish the passes: query fp16 hi/lo fragments -> LDS; new rows -> block images and caches --
#pragma unroll
    for (int ps = 0; ps < QPASS; ps++) {
        const int r = ps * 8 + wave * 2 + hw;
        // one row at a time here: the first tile is already held in registers
        float y1[1][DPL2];
        if constexpr (FUSED) {
            const bool v1[1] = {qvalid[ps]};
            norm_rope_rows<D, 1>(a, lane, rot, reinterpret_cast<const float (&)[1][DPL2]>(qx[ps]),
                                 reinterpret_cast<const float (&)[1][2 * DPL2]>(qcv[ps]), v1, wq, y1);
        } else {
#pragma unroll
            for (int jj = 0; jj < DPL2; jj++) y1[0][jj] = qvalid[ps] ? qx[ps][jj] : 0.f;
        }
        const float (&y)[DPL2] = y1[0];
        // the lane's DPL2 dims are consecutive inside one 8-dim group, so its hi and lo parts are one
        // vector store each into the fragment layout
        typedef f16 f16v __attribute__((ext_vector_type(DPL2)));
        f16v hv, lv;
#pragma unroll
        for (int jj = 0; jj < DPL2; jj++) {
            const float ys = y[jj] * a.q_scale;
            const f16 hi = (f16)ys;
            hv[jj] = hi;
            lv[jj] = (f16)(ys - (float)hi);
        }
        const int col = r & 15;
        const int kk = d0 >> 5, L = ((d0 >> 3) & 3) * 16 + col, e = d0 & 7;
        *reinterpret_cast<f16v*>(&s_q[(kk * 64 + L) * 8 + e]) = hv;
        *reinterpret_cast<f16v*>(&s_q[((NKS + kk) * 64 + L) * 8 + e]) = lv;
    }
    if constexpr (FUSED) {
        float yn[1][DPL2];
        const bool hn[1] = {has_new};
        norm_rope_rows<D, 1>(a, lane, rot, nx, ncv, hn, wk, yn);  // computed by every half-wave, stored by the owners
        const float (&y)[DPL2] = yn[0];
        if (has_new) {
            const int p = a.pos + tn;
            const size_t part = kv_part(p, kvh, a.cap, D);
            f16* kw = reinterpret_cast<f16*>(a.kc) + part;
            f16* vw = reinterpret_cast<f16*>(a.vc) + part;
            const int pb = p & (kBlk - 1), bi = (p >> 5) - (a.pos >> 5);
#pragma unroll
            for (int jj = 0; jj < DPL2; jj++) {
                const int d = d0 + jj;
                const f16 kh = (f16)y[jj];
                const f16 vh = (f16)nv[jj];
                s_img[bi][k_off(pb, d)] = kh;
                s_img[NB + bi][v_off(pb, d)] = vh;
                if (blockIdx.z == 0) {  // every slice needs the rows; slice 0 writes them to the cache
                    kw[k_off(pb, d)] = kh;
                    vw[v_off(pb, d)] = vh;
                }
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_k(kB, wave + 4);
    load_v(vB, wave + 4);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // ---- per column: query row, causal key limit inside this chunk, softmax state ----------------
    const int rcol = c;
    const int lim = rcol < rows ? min(a.pos + (r0 + rcol) / G + 1, ke) : 0;
    float m_run = kNegInf, l_run = 0.f;
    f32x4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto qfrag = [&](int set, int kk) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(s_q + ((set * NKS + kk) * 64 + lane) * 8);
    };

    // scores of one tile: sc[s][i] is key tb + 8g + 4s + i of column c
    auto scores = [&](f16x8 (&kt)[NKS][2], int tb, f32x4 (&sc)[2]) {
        if (FUSED && tb + 32 > new_lo) {  // new positions: take the fresh rows from the block image
            const int bi = (tb >> 5) - (a.pos >> 5);
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const int key = tb + ((c >> 2) << 3) + 4 * s + (c & 3);
                const bool fresh = key >= new_lo && key < maxlen;
#pragma unroll
                for (int kk = 0; kk < NKS; kk++) {
                    const f16x8 im = *reinterpret_cast<const f16x8*>(&s_img[bi][((kk * 2 + s) * 64 + lane) * 8]);
                    kt[kk][s] = fresh ? im : kt[kk][s];
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < NKS; kk++) {
                x = mfma16(kt[kk][s], qfrag(0, kk), x);
                x = mfma16(kt[kk][s], qfrag(1, kk), x);
            }
            sc[s] = x;
        }
    };

    auto softmax_pv = [&](f16x8 (&vt)[NDT], int tb, f32x4 (&sc)[2]) {
        if (tb + 32 > new_lo) {
            // positions past the cache end may hold stale or unwritten memory: zeroed; new positions
            // (fused) take the fresh V rows from the block image. Masks per dword = two keys.
            uint32_t keep[4], take[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int k0 = tb + 8 * g + 2 * k;
                keep[k] = (k0 < new_lo ? 0x0000ffffu : 0u) | (k0 + 1 < new_lo ? 0xffff0000u : 0u);
                take[k] = FUSED ? ((k0 >= new_lo && k0 < maxlen ? 0x0000ffffu : 0u) |
                                   (k0 + 1 >= new_lo && k0 + 1 < maxlen ? 0xffff0000u : 0u)) : 0u;
            }
            const int bi = (tb >> 5) - (a.pos >> 5);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                u32x4 v = as_u4(vt[dt]);
                u32x4 im = {0u, 0u, 0u, 0u};
                if constexpr (FUSED) im = *reinterpret_cast<const u32x4*>(&s_img[NB + bi][(dt * 64 + lane) * 8]);
#pragma unroll
                for (int k = 0; k < 4; k++) v[k] = (v[k] & keep[k]) | (im[k] & take[k]);
                vt[dt] = as_h8(v);
            }
        }
        // QSA: the column's token sees key tb + i when bit i of its word is set
        const unsigned vis = QSA ? s_qw[min(max((r0 + rcol) / G - tok0, 0), RMAX - 1)][(tb - kb) >> 5] : 0xFFFFFFFFu;
        float sv[8];
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = sc[s][i];
                const int kq = 8 * g + 4 * s + i;
                sv[s * 4 + i] = tb + kq < lim && ((vis >> kq) & 1u) ? v : kNegInf;
            }
        float mx = sv[0];
#pragma unroll
        for (int k = 1; k < 8; k++) mx = fmaxf(mx, sv[k]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // lazy rescale: the reference max moves (and o, l are rescaled) only when a column's max grows
        // by more than TAU, so the weights below stay <= 2^TAU; a column's first finite max is taken
        // as is (its o and l are still zero)
        if (m_run == kNegInf) m_run = mx;
        const bool grow = mx > m_run + TAU;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = fmaxf(m_run, mx);
            const float corr = m_new == kNegInf ? 1.f : exp2_fast(m_run - m_new);  // a column with no key yet: 1
            m_run = m_new;
            l_run *= corr;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) acc[dt] *= corr;
        }
        const float m_use = m_run == kNegInf ? 0.f : m_run;
        float psum = 0.f;
        f16x8 pop[NPT];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float p = exp2_fast(sv[k] - m_use);
            psum += p;
            const f16 ph = (f16)p;
            const f16 pl = (f16)(p - (float)ph);
            pop[0][k] = ph;
            pop[1][k] = pl;
        }
        l_run += psum;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int u = 0; u < NPT; u++) acc[dt] = mfma16(vt[dt], pop[u], acc[dt]);
    };

    // ---- main loop: two register buffers, tiles wave, wave + 4, ...; a buffer's next loads go out
    // once its whole tile is computed, so a wave stalled on issuing them never holds data it could use
    // (past the last cached block the loads read zeros without traffic) --------------------------------
    for (int i = 0; i < ntile; i += 2) {
        {
            const int t = wave + 4 * i, tb = kb + 32 * t;
            f32x4 sc[2];
            scores(kA, tb, sc);
            softmax_pv(vA, tb, sc);
            if (i + 2 < ntile) {
                load_k(kA, t + 8);
                load_v(vA, t + 8);
            }
        }
        if (i + 1 < ntile) {
            const int t = wave + 4 * (i + 1), tb = kb + 32 * t;
            f32x4 sc[2];
            scores(kB, tb, sc);
            softmax_pv(vB, tb, sc);
            if (i + 3 < ntile) {
                load_k(kB, t + 8);
                load_v(vB, t + 8);
            }
        }
    }

    // ---- wave results -> LDS (the Q fragments are dead once every wave is here) -------------------
    __syncthreads();
    float* sO = reinterpret_cast<float*>(s_u);
    {
        float l = l_run;
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                *reinterpret_cast<f32x4*>(&sO[(wave * RMAX + c) * C::OSTRIDE + dt * 16 + g * 4]) = acc[dt];
            if (g == 0) {
                sM[wave][c] = m_run;
                sL[wave][c] = l;
            }
        }
    }
    __syncthreads();

    // ---- merge the 4 waves: per-row weights first, then every element without branches ----------
    if (tid < rows) {
        const int r = tid;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; w++)
            if (sL[w][r] > 0.f) M = fmaxf(M, sM[w][r]);
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = sL[w][r] > 0.f ? exp2_fast(sM[w][r] - M) : 0.f;
            sF[w][r] = f;
            L += sL[w][r] * f;
        }
        const int t = (r0 + r) / G, h = kvh * G + (r0 + r) % G;
        const size_t row = ((size_t)t * a.NH + h) * a.n_split + z;
        if (one) {
            sM[0][r] = M;  // for the record (wave 0 of every row reads its own row's entry back)
            sL[0][r] = L;
        } else {
            a.part_ml[row * 2] = M;
            a.part_ml[row * 2 + 1] = L;
        }
    }
    __syncthreads();
    // one launch: device-coherent stores (they reach the point every XCD reads from once acknowledged),
    // so the combining workgroups read them without any cache-wide write-back
    const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(a.part_o, (short)0, 0x7fffffff, 0x00020000);
    for (int idx = tid; idx < rows * (D / 4); idx += 256) {
        const int r = idx / (D / 4), d = (idx % (D / 4)) * 4;
        f32x4 o = *reinterpret_cast<const f32x4*>(&sO[r * C::OSTRIDE + d]) * sF[0][r];
#pragma unroll
        for (int w = 1; w < 4; w++) o += *reinterpret_cast<const f32x4*>(&sO[(w * RMAX + r) * C::OSTRIDE + d]) * sF[w][r];
        const int t = (r0 + r) / G, h = kvh * G + (r0 + r) % G;
        const size_t row = ((size_t)t * a.NH + h) * a.n_split + z;
        if (one) __builtin_amdgcn_raw_buffer_store_b128(o, rpo, (int)((row * D + d) * 4), 0, kScDevice);
        else *reinterpret_cast<f32x4*>(&a.part_o[row * D + d]) = o;
    }
    if constexpr (FUSED) {
        if (one) {
            // the records go out once every o store of the workgroup is acknowledged (the wait counts the
            // wave's memory operations, the barrier joins the four waves): a record with this launch's
            // tag is the combiner's guarantee that its row's o is visible device-wide
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            if (tid < rows) {
                const unsigned long long tag = tag_of(ep_raw, kvh);
                const int t = (r0 + tid) / G, h = kvh * G + (r0 + tid) % G;
                const int row = (t * a.NH + h) * a.n_split + z;
                const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(a.rec, (short)0, 0x7fffffff, 0x00020000);
                __builtin_amdgcn_raw_buffer_store_b128(f32x4{sM[0][tid], sL[0][tid], __uint_as_float((unsigned)tag), __uint_as_float((unsigned)(tag >> 32))},
                                                       rr, row * 16, 0, kScDevice);
            }
            // the slice's last `rows` chunks (the shortest: the first cr chunks are one block longer) then
            // combine one output row each. A combiner waits for the other chunks of its slice; at most 16
            // per slice wait, so every wait ends while more CUs than waiting combiners are free to the launch
            const int zc = z - (a.n_split - rows * a.nds);
            if (zc >= 0) {
                const int rl = r0 + zc % rows, t = rl / G, h = kvh * G + rl % G;
                combine_row<D, IN_DT>(a, s_u, t * a.NH + h, zc / rows);
            }
        }
    }
}


// ---- decode with producer waves (at most 8 query rows) -------------------------------------------
// With HBM saturated, issuing a load stalls the issuing wave until earlier requests drain, so a wave that
// both streams and computes spends most of the stream blocked with data it could be using. Here the
// workgroup's waves 0-1 only compute and waves 2-3 only stream: loader wave 2 + p copies compute wave
// p's tiles (tiles p, p + 2, ...) with direct-to-LDS loads into two 32-key slots and publishes each tile
// through an LDS counter; the compute wave copies the slot into registers, frees it at once and
// computes, so two tiles per pair are in flight while one is being computed. The new positions are
// appended to the caches in the prologue and a tile holding them is copied only after those stores are
// acknowledged, so it arrives complete (no patching in LDS: LDS stores crawl while the first copies
// land); V past the last position is zeroed in registers. Spin waits are bounded, so every wave exits
// even if a counter were never reached; a wait that gives up is reported through DecodeArgs::err.
template <int D, int FUSED, int IN_DT, int QSA>
__global__ __launch_bounds__(256, 1) void k_decode_ld(DecodeArgs a) {
    constexpr int NKS = D / 32, NDT = D / 16, RMAX = 8, BLKE = kBlk * D;
    constexpr int DPL2 = D / 32;            // dims per lane in the row passes
    constexpr int NCW = 2;                  // compute waves (the other two load)
    constexpr int QPASS = RMAX / (2 * NCW);  // query-row passes per compute wave, two rows per pass
    constexpr int NPASS = RMAX / (2 * NCW);  // new-row passes (at most 8 new rows per workgroup)
    constexpr float TAU = 8.f;
    constexpr int TILE_E = 2 * BLKE;        // a slot: the K part then the V part of one block
    constexpr int PIECES = BLKE * 2 / 1024;  // 1 KB direct loads per part
    constexpr int SPIN_MAX = 1 << 22;
    static_assert(2 * PIECES <= 63, "one tile's loads must fit the load counter");

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f16* ring = reinterpret_cast<f16*>(smem);                 // [NCW][2][TILE_E]
    f16* s_q = ring + NCW * 2 * TILE_E;                        // Q fragments (hi rows 0-7, lo rows 8-15)
    // QSA: the visible tiles (ordinals into the strided sequence) and, per visible tile, each token's
    // 32 key bits
    unsigned* s_vl = reinterpret_cast<unsigned*>(s_q + NKS * 64 * 8);  // [kQsaTiles]
    unsigned* s_vw = s_vl + kQsaTiles;                                  // [kQsaTiles][8]
    // tile counters in a separate LDS object: an access the compiler cannot tell apart from the
    // direct-to-LDS copies' destination makes it wait for every outstanding copy first
    __shared__ int s_cnt[2 * NCW];
    __shared__ int s_nvis;
    int* ready = s_cnt;        // [NCW] tiles published per pair
    int* freed = s_cnt + NCW;  // [NCW] tiles released per pair

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, g = lane >> 4;
    // one-launch decode: each KV head's last chunks combine one output row each once their own partials
    // are out (the end of this kernel)
    const bool one = FUSED && a.out != nullptr;
    const int kvh = blockIdx.x / a.n_split, z = blockIdx.x - kvh * a.n_split;
    const int G = a.NH / a.NKV;
    const int rows = min(RMAX, a.n * G);
    const int maxlen = a.pos + a.n;
    // one-launch: the head's launch counter for this launch's epoch tag (see kEpochStep), read now
    // (device-coherent, unconditionally: a zero-sized range without the combine reads 0 and touches no
    // memory) so that its latency hides behind the prologue; it must be read before this workgroup stores
    // its records
    u32x2 ep_raw = {0u, 0u};
    if constexpr (FUSED) {
        const __amdgpu_buffer_rsrc_t rep = __builtin_amdgcn_make_buffer_rsrc(one ? a.ep + kvh : a.ep, (short)0, one ? 8 : 0, 0x00020000);
        ep_raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rep, 0, 0, kScDevice));
    }
    // ---- this split's tiles: blocks z, z + S, z + 2S, ... of the nb blocks of the head that hold keys
    // (strided: at every step the splits of a head read neighbouring blocks, so the cache is swept front to
    // back, which streams faster than one contiguous range per workgroup)
    const int S = a.n_split;
    const int nb = (maxlen + 31) >> 5;
    const int ntile = z < nb ? (nb - 1 - z) / S + 1 : 0;
    const bool loader = wave >= NCW;
    const int pr = loader ? wave - NCW : 0;                 // loader p streams the tiles p, p + 2, ... of pair p
    // tiles streamed: all ntile, or (QSA) the nvt that some token sees, known once the list is built
    int nvt = ntile;
    int ntp = ntile > pr ? (ntile - pr + 1) / 2 : 0;        // the loader's tile count
    // first new position: the prologue appends the new rows to the caches, and a tile holding any of them
    // is copied only once those stores are complete (after the prologue), so it arrives whole
    const int new_lo = FUSED ? a.pos : maxlen;
    if (tid < 2 * NCW) s_cnt[tid] = 0;  // ready[] and freed[] (published by the barrier below)

    const int bstride = BLKE * 2;  // bytes between consecutive blocks of one head (nb * bstride < 2^31: host-checked)
    const size_t head0 = kv_part(0, kvh, a.cap, D);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kc) + head0, (short)0, nb * bstride, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.vc) + head0, (short)0, nb * bstride, 0x00020000);
    // block of streamed tile t (QSA: of the t-th visible tile; the list is read with an inline LDS load, as
    // the counters are, so a loader wave does not wait for its copies in flight)
    auto blk_of = [&](int t) -> int {
        if constexpr (QSA) {
            int v;
            const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_vl + t));
            asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
            return z + S * __builtin_amdgcn_readfirstlane(v);
        } else {
            return z + S * t;
        }
    };
    // tile t: loader t & 1, its (t >> 1)-th tile, in that loader's slot (t >> 1) & 1
    auto slot_of = [&](int t) { return ring + ((t & 1) * 2 + ((t >> 1) & 1)) * TILE_E; };
    auto has_new = [&](int t) { return FUSED && kBlk * blk_of(t) + kBlk > new_lo; };  // holds new positions
    auto dma = [&](int t) {  // tile t into its slot
        f16* dst = slot_of(t);
        const int off = blk_of(t) * bstride + lane * 16;
#pragma unroll
        for (int j = 0; j < PIECES; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(dst + j * 512), 16,
                                                     off + j * 1024, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < PIECES; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(dst + BLKE + j * 512),
                                                     16, off + j * 1024, 0, 0, 0);
    };
    // new rows this workgroup appends: those in blocks it owns (the n <= 8 new rows span at most two blocks)
    int t_lo = 0, t_hi = 0;
    if constexpr (FUSED) {
        const int B0 = a.pos >> 5, B1 = (maxlen - 1) >> 5;
        const bool own0 = B0 % S == z, own1 = B1 % S == z;
        t_lo = own0 ? 0 : kBlk * B1 - a.pos;
        t_hi = own1 ? a.n : min(a.n, kBlk * (B0 + 1) - a.pos);
        if (!own0 && !own1) t_lo = t_hi = 0;
    }
    // ---- compute waves: query rows (and, fused, the new K/V rows) normalized and rotated ------------
    // Two rows per compute wave per pass, 32 lanes per row, DPL2 dims per lane.
    const int hw = lane >> 5, hl = lane & 31, d0 = hl * DPL2;
    const int half_r = a.R >> 1;
    const bool rot = FUSED && d0 < a.R;  // lanes whose DPL2 dims are rotated (R/2 is a multiple of DPL2)
    auto issue_row = [&](float (&x)[DPL2], float (&cv)[2 * DPL2], const void* src, size_t off, int p, bool valid) {
        load_vec<FUSED ? IN_DT : 0, DPL2>(src, (valid ? off : 0) + d0, x);
        if constexpr (FUSED) {
            const int i0 = rot ? (d0 < half_r ? d0 : d0 - half_r) : 0;
            load_vec<0, 2 * DPL2>(a.rope, (size_t)(valid && rot ? p : 0) * a.R + 2 * i0, cv);
        }
    };
    if (!loader) {
        float wq[DPL2], wk[DPL2];
        float qx[QPASS][DPL2], qcv[QPASS][2 * DPL2];
        float nx[NPASS][DPL2], ncv[NPASS][2 * DPL2], nv[NPASS][DPL2];
        if constexpr (FUSED) {
            load_vec<0, DPL2>(a.qn, d0, wq);
            load_vec<0, DPL2>(a.kn, d0, wk);
        }
#pragma unroll
        for (int ps = 0; ps < QPASS; ps++) {
            const int r = ps * 2 * NCW + wave * 2 + hw;
            const bool valid = r < rows;
            const int t = valid ? r / G : 0, h = kvh * G + (valid ? r % G : 0);
            if constexpr (FUSED) issue_row(qx[ps], qcv[ps], a.q, ((size_t)t * a.NH + h) * 2 * D, a.pos + t, valid);
            else issue_row(qx[ps], qcv[ps], a.q, ((size_t)t * a.NH + h) * D, 0, valid);
        }
        if constexpr (FUSED) {
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++) {
                const int tn = t_lo + ps * 2 * NCW + wave * 2 + hw;
                const bool has = tn < t_hi;
                const size_t src = ((size_t)(has ? tn : 0) * a.NKV + kvh) * D;
                issue_row(nx[ps], ncv[ps], a.knew, src, a.pos + (has ? tn : 0), has);
                load_vec<IN_DT, DPL2>(a.vnew, src + d0, nv[ps]);
            }
        }
        // the rows' loads are out: let the loaders start (a bare barrier, no wait on these loads)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        float yq[QPASS][DPL2];
        bool qv[QPASS];
#pragma unroll
        for (int ps = 0; ps < QPASS; ps++) qv[ps] = ps * 2 * NCW + wave * 2 + hw < rows;
        if constexpr (FUSED) norm_rope_rows<D, QPASS>(a, lane, rot, qx, qcv, qv, wq, yq);
#pragma unroll
        for (int ps = 0; ps < QPASS; ps++) {
            const int r = ps * 2 * NCW + wave * 2 + hw;
            float y[DPL2];
            if constexpr (FUSED) {
#pragma unroll
                for (int jj = 0; jj < DPL2; jj++) y[jj] = yq[ps][jj];
            } else {
#pragma unroll
                for (int jj = 0; jj < DPL2; jj++) y[jj] = r < rows ? qx[ps][jj] : 0.f;
            }
            // fp16 hi part in column r, lo remainder in column r + 8 of the Q^T fragments
            typedef f16 f16v __attribute__((ext_vector_type(DPL2)));
            f16v hv, lv;
#pragma unroll
            for (int jj = 0; jj < DPL2; jj++) {
                const float ys = y[jj] * a.q_scale;
                const f16 hi = (f16)ys;
                hv[jj] = hi;
                lv[jj] = (f16)(ys - (float)hi);
            }
            const int kk = d0 >> 5, L = ((d0 >> 3) & 3) * 16 + r, e = d0 & 7;
            *reinterpret_cast<f16v*>(&s_q[(kk * 64 + L) * 8 + e]) = hv;
            *reinterpret_cast<f16v*>(&s_q[(kk * 64 + L + 8) * 8 + e]) = lv;
        }
        if constexpr (FUSED) {
            float yn[NPASS][DPL2];
            bool nvl[NPASS];
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++) nvl[ps] = t_lo + ps * 2 * NCW + wave * 2 + hw < t_hi;
            norm_rope_rows<D, NPASS>(a, lane, rot, nx, ncv, nvl, wk, yn);
#pragma unroll
            for (int ps = 0; ps < NPASS; ps++) {
                const int tn = t_lo + ps * 2 * NCW + wave * 2 + hw;
                const float (&y)[DPL2] = yn[ps];
                if (tn < t_hi) {
                    const int p = a.pos + tn;
                    const size_t part = kv_part(p, kvh, a.cap, D);
                    f16* kw = reinterpret_cast<f16*>(a.kc) + part;
                    f16* vw = reinterpret_cast<f16*>(a.vc) + part;
                    const int pb = p & (kBlk - 1);
#pragma unroll
                    for (int jj = 0; jj < DPL2; jj++) {
                        const int d = d0 + jj;
                        kw[k_off(pb, d)] = (f16)y[jj];
                        vw[v_off(pb, d)] = (f16)nv[ps][jj];
                    }
                }
            }
            // the appended rows are complete (in this XCD's L2, which the copies of their tiles read)
            // before the barrier below, after which those tiles are copied. Waiting here beats every
            // alternative measured: stores issued now are acknowledged only behind the copies in flight,
            // and any wave that waits for them later stalls a tile instead.
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): s_q and the counters are in LDS
    } else {
        if constexpr (QSA) {
            // the first loader lists the tiles some token sees (a nonzero word of key bits), before any copy
            // of its own is in flight; the barrier below publishes the list
            if (wave == NCW) {
                int nv = 0;
                for (int base = 0; base < ntile; base += 64) {
                    const int t = base + lane;
                    unsigned w[8];
                    bool any = false;
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        w[u] = 0u;
                        if (u < a.n && t < ntile) w[u] = a.kbits[(size_t)u * a.kb_words + z + S * t];
                        any |= w[u] != 0u;
                    }
                    const unsigned long long bal = __ballot(any);
                    const int ord = nv + __builtin_popcountll(bal & ((1ull << lane) - 1ull));
                    if (any) {
                        s_vl[ord] = (unsigned)t;
#pragma unroll
                        for (int u = 0; u < 8; u++) s_vw[ord * 8 + u] = w[u];
                    }
                    nv += __builtin_popcountll(bal);
                }
                if (lane == 0) s_nvis = nv;
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the list is in LDS before the barrier
            }
        }
        // wait until the compute waves' row loads are issued, then put the first two tiles in flight
        // behind them: issued any earlier, the copies would queue the row loads behind the whole stream
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        if constexpr (QSA) {
            int v;
            const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&s_nvis));
            asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
            nvt = __builtin_amdgcn_readfirstlane(v);
            ntp = nvt > pr ? (nvt - pr + 1) / 2 : 0;
        }
        // a tile holding new positions waits until they are appended (after the prologue); such tiles
        // are the pair's last, so the copies still go out in tile order
        if (ntp > 0 && !has_new(pr)) dma(pr);
        if (ntp > 1 && !has_new(pr + 2)) dma(pr + 2);
    }
    // a bare barrier: the LDS writes and cache-row stores above are complete (the compute waves waited
    // for them), and a fenced one would also wait for the copies in flight
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");

    float m_run = kNegInf, l_run = 0.f;
    f32x4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (loader) {
        // ---- stream this pair's tiles; publish each once landed --------------------------------------
        if (ntp > 0 && has_new(pr)) dma(pr);  // the tiles the prologue held back, in tile order
        if (ntp > 1 && has_new(pr + 2)) dma(pr + 2);
        const uint32_t raddr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&ready[pr]));
        const uint32_t faddr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&freed[pr]));
        for (int i = 0; i < ntp; i++) {
            if (i + 1 < ntp) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PIECES));  // tile i landed, i+1 may not
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            // publish: the waits above already order the tile before the counter; an LDS store the compiler
            // can see would also wait for the next tile's copies (it cannot tell the counter from their
            // destination), halving the pipeline
            asm volatile("ds_write_b32 %0, %1" ::"v"(raddr), "v"(i + 1) : "memory");
            if (i + 2 < ntp) {
                // wait for the compute wave to free the slot (read through inline assembly as well: an LDS
                // read the compiler can see would first wait for every copy of this wave)
                for (int spin = 0;; spin++) {
                    int f;
                    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(f) : "v"(faddr) : "memory");
                    if (__builtin_amdgcn_readfirstlane(f) >= i + 1) break;
                    if (spin >= SPIN_MAX) {
                        if (lane == 0) report_wait(a, kWaitRingLoad);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                dma(pr + 2 * (i + 2));
            }
        }
    } else {
        // ---- compute wave p takes the pair's tiles p, p + 2, ... from the slots ------------------------
        const int rcol = c & 7;
        const int lim = rcol < rows ? a.pos + rcol / G + 1 : 0;
        const int utok = min(rcol / G, 7);  // QSA: the column's token
        f16x8 qreg[NKS];
#pragma unroll
        for (int kk = 0; kk < NKS; kk++) qreg[kk] = *reinterpret_cast<const f16x8*>(s_q + (kk * 64 + lane) * 8);
        if constexpr (QSA) nvt = s_nvis;
        const int ntc = nvt > wave ? (nvt - wave + 1) / 2 : 0;
        // P = exp2(s - m) and P V with the running max m (shared by the tile loop and the rescale path)
        auto finish = [&](const float (&sv)[8], const f16x8 (&vt)[NDT]) {
            const float m_use = m_run == kNegInf ? 0.f : m_run;
            float psum = 0.f;
            f16x8 pop;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float pk = exp2_fast(sv[k] - m_use);
                psum += pk;
                const f16 ph = (f16)pk;
                pop[k] = c >= 8 ? (f16)(pk - (float)ph) : ph;
            }
            l_run += psum;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) acc[dt] = mfma16(vt[dt], pop, acc[dt]);
        };
        // The tiles run in an inner loop that leaves only when a tile's max passes the running max by more
        // than TAU; the rescale (rare) happens outside it and the tile is finished there. With the rescale
        // as a conditional block inside the tile loop, the compiler copies every accumulator register on
        // every iteration.
        int i = 0;
        for (;;) {
            bool resc = false;
            float sv[8], mx = kNegInf;
            f16x8 vt[NDT];
            for (; i < ntc; i++) {
                const int t = wave + 2 * i;
                for (int spin = 0; __hip_atomic_load(&ready[wave], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < i + 1;
                     spin++) {
                    if (spin >= SPIN_MAX) {
                        if (lane == 0) report_wait(a, kWaitRingCompute);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                const f16* sl = slot_of(t);
                // K first: the scores start once it is in registers, and V is read behind them
                f16x8 kt[NKS][2];
#pragma unroll
                for (int kk = 0; kk < NKS; kk++)
#pragma unroll
                    for (int s2 = 0; s2 < 2; s2++) kt[kk][s2] = *reinterpret_cast<const f16x8*>(sl + ((kk * 2 + s2) * 64 + lane) * 8);
                // scores: sc[s][i] is key tb + 8g + 4s + i of column c (fp16 hi in columns 0-7, lo in 8-15)
                f32x4 sc[2];
#pragma unroll
                for (int s2 = 0; s2 < 2; s2++) {
                    f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < NKS; kk++) x = mfma16(kt[kk][s2], qreg[kk], x);
                    sc[s2] = x;
                }
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) vt[dt] = *reinterpret_cast<const f16x8*>(sl + BLKE + (dt * 64 + lane) * 8);
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the tile is in registers, the slot is free
                asm volatile("" ::: "memory");
                __hip_atomic_store(&freed[wave], i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

                const int tb = kBlk * blk_of(t);
                if (tb + 32 > maxlen) {
                    // keys from maxlen on: their scores are masked, but V there is whatever the cache memory
                    // holds (P = 0 there, and 0 * NaN is not 0): zero it. V fragment dt: lane (c, g) holds
                    // keys 8 g .. 8 g + 7 of dim 16 dt + c, two keys per 32-bit word
                    const int nvk = min(max(maxlen - tb - 8 * g, 0), 8);
                    u32x4 keep;
#pragma unroll
                    for (int w = 0; w < 4; w++) keep[w] = (2 * w < nvk ? 0xFFFFu : 0u) | (2 * w + 1 < nvk ? 0xFFFF0000u : 0u);
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++) vt[dt] = as_h8(as_u4(vt[dt]) & keep);
                }
                // QSA: the column's token sees key tb + i when bit i of its word is set
                const unsigned vis = QSA ? s_vw[t * 8 + utok] : 0xFFFFFFFFu;
#pragma unroll
                for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float v = sc[s2][e] + xor8(sc[s2][e]);
                        const int kq = 8 * g + 4 * s2 + e;
                        sv[s2 * 4 + e] = tb + kq < lim && ((vis >> kq) & 1u) ? v : kNegInf;
                    }
                mx = sv[0];
#pragma unroll
                for (int k = 1; k < 8; k++) mx = fmaxf(mx, sv[k]);
                mx = max_rows(mx);  // over the column's four lane groups
                // lazy rescale (see k_decode)
                if (m_run == kNegInf) m_run = mx;
                if (__builtin_amdgcn_ballot_w64(mx > m_run + TAU) != 0) {
                    resc = true;
                    break;
                }
                finish(sv, vt);
            }
            if (!resc) break;
            const float m_new = fmaxf(m_run, mx);
            const float corr = m_new == kNegInf ? 1.f : exp2_fast(m_run - m_new);  // a column with no key yet: 1
            m_run = m_new;
            l_run *= corr;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) acc[dt] *= corr;
            finish(sv, vt);
            i++;
        }
        l_run += __shfl_xor(l_run, 16, 64);  // the column's sum over the lane groups
        l_run += __shfl_xor(l_run, 32, 64);
    }

    // ---- merge: the compute waves put their raw accumulators and running (max, sum) in LDS (the ring is
    // dead once every wave is here); then all four waves merge them, wave q taking fragments q NDQ ..
    // q NDQ + NDQ - 1 of both, add each query row's hi and lo columns and store those dims of the split's
    // partial rows (four waves: each does a quarter of the register arithmetic of the merge, which is the
    // bulk of its time). Device-coherent stores (they reach the point every XCD reads from): the combining
    // workgroups of the one-launch decode read them from other XCDs without any cache-wide write-back
    constexpr int NDQ = NDT / 4;                  // 16-dim fragments merged per wave
    float* sO = reinterpret_cast<float*>(ring);   // [NCW][NDT][64 lanes][4]
    float* sML = sO + NCW * NDT * 256;             // [NCW][16 columns][2]
    __syncthreads();
    if (!loader) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) *reinterpret_cast<f32x4*>(&sO[((wave * NDT + dt) * 64 + lane) * 4]) = acc[dt];
        if (g == 0) sML[(wave * 16 + c) * 2] = m_run, sML[(wave * 16 + c) * 2 + 1] = l_run;
    }
    __syncthreads();
    {
        const float m0 = sML[c * 2], l0 = sML[c * 2 + 1], m1 = sML[(16 + c) * 2], l1 = sML[(16 + c) * 2 + 1];
        const float M = fmaxf(l0 > 0.f ? m0 : kNegInf, l1 > 0.f ? m1 : kNegInf);
        const float f0 = l0 > 0.f ? exp2_fast(m0 - M) : 0.f, f1 = l1 > 0.f ? exp2_fast(m1 - M) : 0.f;
        const float L = l0 * f0 + l1 * f1;
        f32x4 o[NDQ];
#pragma unroll
        for (int j = 0; j < NDQ; j++) {
            const int dt = wave * NDQ + j;
            const f32x4 o0 = *reinterpret_cast<const f32x4*>(&sO[(dt * 64 + lane) * 4]);
            const f32x4 o1 = *reinterpret_cast<const f32x4*>(&sO[((NDT + dt) * 64 + lane) * 4]);
            o[j] = o0 * f0 + o1 * f1;  // columns c and c ^ 8 (one query row) share f0, f1
#pragma unroll
            for (int e = 0; e < 4; e++) o[j][e] += xor8(o[j][e]);
        }
        if (c < rows) {  // lanes of column c < 8 hold query row c: dims 16 dt + 4 g .. + 3 of fragment dt
            const int t = c / G, h = kvh * G + c % G;
            const int row = (t * a.NH + h) * S + z;  // the host keeps the partial buffer below 2 GiB
            const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(a.part_o, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
            for (int j = 0; j < NDQ; j++)
                __builtin_amdgcn_raw_buffer_store_b128(o[j], rpo, (row * D + (wave * NDQ + j) * 16 + g * 4) * 4, 0, kScDevice);
            if (!one && wave == 0 && g == 0) {
                a.part_ml[(size_t)row * 2] = M;
                a.part_ml[(size_t)row * 2 + 1] = L;
            }
        }
        m_run = M, l_run = L;
    }
    if (one) {
        // the records go out once every o store of the workgroup is acknowledged (the wait counts the
        // wave's memory operations, the barrier joins the four waves): a record with this launch's tag
        // is the combiner's guarantee that its row's o is visible device-wide
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        if (wave == 0 && g == 0 && c < rows) {
            const unsigned long long tag = tag_of(ep_raw, kvh);
            const int t = c / G, h = kvh * G + c % G;
            const int row = (t * a.NH + h) * S + z;
            const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(a.rec, (short)0, 0x7fffffff, 0x00020000);
            __builtin_amdgcn_raw_buffer_store_b128(f32x4{m_run, l_run, __uint_as_float((unsigned)tag), __uint_as_float((unsigned)(tag >> 32))},
                                                   rr, row * 16, 0, kScDevice);
        }
        if constexpr (FUSED) {
            // the head's last `rows` chunks then combine one output row each (the ring is dead: the merge
            // above was its last use). A combiner waits for the other chunks of its head; at most 8 per head
            // wait, so every wait ends while more than 8 x NKV CUs are free to the launch
            const int zc = z - (S - rows * a.nds);
            if (zc >= 0) {
                __syncthreads();
                const int rl = zc % rows;
                combine_row<D, IN_DT>(a, smem, (rl / G) * a.NH + kvh * G + rl % G, zc / rows);
            }
        }
    }
}

template <int D, int QSA>
constexpr size_t decode_ld_lds() {
    // ring + Q fragments (+ QSA: the visible-tile list and its key words)
    const size_t stream = (size_t)2 * 2 * 2 * kBlk * D * 2 + (size_t)(D / 32) * 64 * 8 * 2 + (QSA ? kQsaTiles * 9 * 4 : 0);
    const size_t comb = (size_t)4 * (D + 2 + kCombGroup) * 4;  // combiner: a window's group sums, maxima, sums, weights
    return stream > comb ? stream : comb;
}

// Launches a kernel with `shm` bytes of dynamic LDS; the limit is a per-device attribute of the
// function, raised once per device (`raised`: one bit per device).
template <typename K>
static hipError_t launch_lds(K kern, std::atomic<uint64_t>& raised, dim3 grid, size_t shm, const DecodeArgs& a, hipStream_t s) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(raised.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        if (e != hipSuccess) return e;
        raised.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL(kern, grid, dim3(256), shm, s, a);
    return hipGetLastError();
}

template <int D, int FUSED, int IN_DT>
static hipError_t launch_mode(const DecodeArgs& a, hipStream_t s) {
    const int rows = a.n * (a.NH / a.NKV);
    // the in-launch combine: fused (it needs the gate), on the last chunks of each KV head (up to 8 rows)
    // or 16-row slice, one output row each, so a head / slice needs that many chunks
    if (a.out != nullptr && (!FUSED || (a.nds != 1 && a.nds != 2 && a.nds != 4 && a.nds != 8) || D / a.nds < 16 ||
                             a.n_split < (rows < 16 ? rows : 16) * a.nds ||
                             a.ncomb != a.n * a.NH || !a.ep || !a.rec))
        return hipErrorInvalidValue;
    if (rows <= 8) {
        static std::atomic<uint64_t> raised{0};
        const dim3 grid(a.n_split * a.NKV);
        if (a.kbits) {
            static std::atomic<uint64_t> raised_q{0};
            return launch_lds(k_decode_ld<D, FUSED, IN_DT, 1>, raised_q, grid, decode_ld_lds<D, 1>(), a, s);
        }
        return launch_lds(k_decode_ld<D, FUSED, IN_DT, 0>, raised, grid, decode_ld_lds<D, 0>(), a, s);
    }
    const dim3 grid(a.n_split, a.NKV, (rows + 15) / 16);
    if (a.kbits) hipLaunchKernelGGL((k_decode<D, FUSED, IN_DT, 1>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_decode<D, FUSED, IN_DT, 0>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int D>
static hipError_t launch_decode_d(const DecodeArgs& a, bool fused, int in_dtype, hipStream_t s) {
    if (!fused) return launch_mode<D, 0, 0>(a, s);
    return in_dtype == 0 ? launch_mode<D, 1, 0>(a, s) : launch_mode<D, 1, 1>(a, s);
}

hipError_t launch_decode(const DecodeArgs& a, int D, bool fused, int in_dtype, hipStream_t s) {
    if (D == 256) return launch_decode_d<256>(a, fused, in_dtype, s);
    if (D == 128) return launch_decode_d<128>(a, fused, in_dtype, s);
    return launch_decode_d<64>(a, fused, in_dtype, s);
}

// ---- combine ---------------------------------------------------------------------------------------
// One workgroup per (row, 64-dim slice): 16 split lanes x 16 dim lanes of 4 dims. Each thread merges
// the splits z = zg, zg + 16, ... in batches of 8 (all loads of a batch issued before any is used,
// merge_batch); the 16 thread-partials of a dim group then merge through LDS. Splits with l = 0 are
// skipped (attn_combine.comp:17-26).
template <int IN_DT>
__global__ __launch_bounds__(256) void k_combine(CombineArgs a, int D) {
    constexpr int BATCH = 8;
    __shared__ float sMt[16][16], sLt[16][16];
    __shared__ f32x4 sOt[16][16];
    const int tid = threadIdx.x;
    const int zg = tid >> 4, q = tid & 15;
    const int row = blockIdx.x;  // t * NH + h
    const int S = a.n_split;
    const int d0 = blockIdx.y * 64 + q * 4;
    const float* ml = a.part_ml + (size_t)row * S * 2;
    const float* po = a.part_o + (size_t)row * S * D + d0;
    // the output gate, loaded up front: loads next to the output stores (which might alias them, as far
    // as the compiler knows) would each wait for the one before
    float gate[4];
    {
        const int t = row / a.NH, h = row % a.NH;
        const size_t gb = ((size_t)t * a.NH + h) * 2 * D + D + d0;
#pragma unroll
        for (int i = 0; i < 4; i++) gate[i] = zg == 0 ? load_in<IN_DT>(a.qg, gb + i) : 0.f;
    }

    float M = kNegInf, L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    for (int z0 = zg; z0 < S; z0 += 16 * BATCH) {
        float m[BATCH], l[BATCH];
        f32x4 o[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; u++) {  // every load of the batch is issued before any is used
            const int zz = min(z0 + 16 * u, S - 1);
            m[u] = ml[2 * zz];
            l[u] = ml[2 * zz + 1];
            o[u] = *reinterpret_cast<const f32x4*>(po + (size_t)zz * D);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the first wait
        unsigned keys = 0;
#pragma unroll
        for (int u = 0; u < BATCH; u++) keys |= (z0 + 16 * u < S && l[u] > 0.f ? 1u : 0u) << u;
        merge_batch(M, L, O, m, l, o, keys);
    }
    sMt[zg][q] = M;
    sLt[zg][q] = L;
    sOt[zg][q] = O;
    __syncthreads();
    if (zg == 0) {
        float Mx = kNegInf;
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (sLt[k][q] > 0.f) Mx = fmaxf(Mx, sMt[k][q]);
        float Ls = 0.f;
        f32x4 Os = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (sLt[k][q] > 0.f) {
                const float f = exp2_fast(sMt[k][q] - Mx);
                Ls += sLt[k][q] * f;
                Os += sOt[k][q] * f;
            }
        }
        const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;  // a row with no visible key: 0, as the CPU path gives
        f32x4 res;
#pragma unroll
        for (int i = 0; i < 4; i++) res[i] = Os[i] * inv * sigmoid(gate[i]);
        *reinterpret_cast<f32x4*>(a.out + (size_t)row * D + d0) = res;
    }
}

hipError_t launch_combine(const CombineArgs& a, int D, int in_dtype, hipStream_t s) {
    const dim3 grid(a.n * a.NH, D / 64), block(256);
    if (in_dtype == 0) hipLaunchKernelGGL(k_combine<0>, grid, block, 0, s, a, D);
    else hipLaunchKernelGGL(k_combine<1>, grid, block, 0, s, a, D);
    return hipGetLastError();
}

}  // namespace qw
