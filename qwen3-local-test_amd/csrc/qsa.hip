// QSA block-sparse attention, the indexer side, for gfx950: pooled block keys, block selection, and the
// per-key visibility bits the attention kernels consume.
//
// Replaces the reference's CPU indexer (class QsaIndexer, src/qwen4_qsa.h:17-115) and the bitmask the
// Vulkan backend builds from its selection (src/qwen4_vk.cpp:952-960). Semantics:
//  - pooling (QsaIndexer::update, :38-54): block b of CR consecutive positions gets the mean of its raw
//    indexer keys (accumulated key by key, 1/CR times each), RMS-normed with the gamma as stored (not
//    1 + gamma) and rotated (rotate-half over the layer's rope_dim) to the block's first position b*CR;
//  - selection (QsaIndexer::select, :58-91): token t at position p sees nblk = (p + 1) / CR complete
//    blocks; with nblk <= top = budget / CR it selects nothing (attention stays dense: mask row all
//    ones). Otherwise its IH indexer query heads are normed and rotated to p, block b scores
//    sum_h max(0, q_h . pooled_b), and the top blocks by (score, then the lower block id) are selected;
//  - visibility (shaders/attention.comp:35-43): key j of token t is visible when it lies in a selected
//    complete block or in the incomplete tail block, j >= nblk * CR.
//
// MI355X design (not the reference's): the indexer runs on the GPU, so a QSA layer needs no GPU -> CPU
// round trip (the reference waits for the GPU and copies the block input out for every QSA layer past
// the budget). Scoring is spread over (token, 256-block chunk) workgroups, 16 lanes per pooled key
// (coalesced 512-byte rows); the scores go to a workspace with device-coherent stores, and the last
// workgroup of a token to arrive (an arrival counter, no waiting anywhere) runs an exact radix select on
// the scores' bit patterns (scores are >= +0, so their bits order like the values) and writes the mask.
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"

namespace qw {

namespace {

constexpr int kQsaThreads = 1024;
constexpr int kQsaChunk = 64;         // blocks scored per workgroup (one key per 16-lane group)
constexpr int kQsaMaskLds = 4608;     // mask words staged in LDS (>= (262144 / 2 + 1 + 31) / 32)

// Sum over each 16-lane row, in every lane of the row (DPP butterfly: quads, eight lanes, sixteen).
__device__ __forceinline__ float sum16(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));
    return x;
}

// Sum over the wave, in every lane: 32-lane halves (DPP + permlane16), then the halves (permlane32).
__device__ __forceinline__ float wave_sum(float x) {
    x = sum32(x);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Integer sum over the wave, in every lane (DPP within 16-lane rows, then permlane16 and permlane32 swaps).
__device__ __forceinline__ unsigned wave_isum(unsigned x) {
    x += (unsigned)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false);
    x += (unsigned)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false);
    x += (unsigned)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xF, 0xF, false);
    x += (unsigned)__builtin_amdgcn_mov_dpp((int)x, 0x140, 0xF, 0xF, false);
    const auto s16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = s16[0] + s16[1];
    const auto s32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return s32[0] + s32[1];
}

__device__ __forceinline__ unsigned wave_min(unsigned x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = min(x, (unsigned)__shfl_xor((int)x, o, 64));
    return x;
}

__device__ __forceinline__ unsigned wave_max(unsigned x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = max(x, (unsigned)__shfl_xor((int)x, o, 64));
    return x;
}

// Rotate-half RoPE of one row held in LDS (src/qwen4_qsa.h:99-107): pairs (i, i + R/2), i < R/2, with the
// (cos, sin) of position p from the rope table [p][R/2][2]; `x` is the normed row, `y` receives the result
// (dims past R copied). Threads [0, nthr) cooperate.
__device__ __forceinline__ void rope_row(const float* x, float* y, const float* rope, int p, int R, int ID, int tid,
                                         int nthr) {
    const int half = R >> 1;
    for (int d = tid; d < ID; d += nthr) {
        if (d < R) {
            const int i = d < half ? d : d - half;
            const float cs = rope[((size_t)p * half + i) * 2], sn = rope[((size_t)p * half + i) * 2 + 1];
            y[d] = d < half ? x[d] * cs - x[d + half] * sn : x[d] * cs + x[d - half] * sn;
        } else {
            y[d] = x[d];
        }
    }
}

// Key bits [32 w, 32 w + 32) of a token with nblk complete blocks of `cr` keys and block mask m: key j is
// visible when block j / cr has its bit set or lies at or past nblk (the tail). One division per word, the
// block of each following key by counting.
__device__ __forceinline__ unsigned key_word(const unsigned* m, int w, int cr, int nblk) {
    const int nmwc = (nblk + 31) >> 5;
    if ((cr & (cr - 1)) == 0) {
        // a power of two: the word lies in one block (cr >= 32) or holds 32 / cr whole blocks of one mask word
        const int lc = __builtin_ctz((unsigned)cr);
        if (cr >= 32) {
            const int blk = (32 * w) >> lc;
            const unsigned mw = (blk >> 5) < nmwc ? m[blk >> 5] : 0u;
            return blk >= nblk || ((mw >> (blk & 31)) & 1u) ? 0xFFFFFFFFu : 0u;
        }
        const int nb = 32 >> lc, blk0 = w * nb;
        const unsigned mw = (blk0 >> 5) < nmwc ? m[blk0 >> 5] : 0u, ones = (1u << cr) - 1u;
        unsigned bits = 0u;
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i < nb) {
                const int blk = blk0 + i;
                bits |= blk >= nblk || ((mw >> (blk & 31)) & 1u) ? ones << (i * cr) : 0u;
            }
        return bits;
    }
    int blk = (32 * w) / cr, r = 32 * w - blk * cr;
    // the 32 keys lie in at most 32 consecutive blocks: two mask words, read once (only words that hold
    // complete blocks are read)
    const int w0 = blk >> 5, nmw = (nblk + 31) >> 5;
    const unsigned m0 = w0 < nmw ? m[w0] : 0u, m1 = w0 + 1 < nmw ? m[w0 + 1] : 0u;
    unsigned bits = 0u;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const unsigned mw = (blk >> 5) == w0 ? m0 : m1;
        const bool vis = blk >= nblk || ((mw >> (blk & 31)) & 1u);
        bits |= (unsigned)vis << i;
        if (++r == cr) r = 0, blk++;
    }
    return bits;
}

}  // namespace

// ---- pooling ---------------------------------------------------------------------------------------------
// Workgroups [0, nbp): one (64 lanes) per block completed by the call, blocks [pos/CR, (pos+n)/CR). The
// block's rows at positions >= pos come from the call's ik, the earlier ones from the raw cache. Workgroups
// [nbp, nbp + n): one per new row, appended to the raw cache (the pooling workgroups never read those).
template <int IN_DT>
__global__ __launch_bounds__(64) void k_qsa_pool(QsaPoolArgs a) {
    __shared__ float s_x[512], s_y[512];
    const int lane = threadIdx.x, ID = a.ID, KD = ID >> 6;
    const int b0 = a.pos / a.CR, nbp = (a.pos + a.n) / a.CR - b0;
    if ((int)blockIdx.x >= nbp) {
        const int t = blockIdx.x - nbp;
        for (int k = 0; k < KD; k++) {
            const int d = lane + 64 * k;
            a.raw[(size_t)(a.pos + t) * ID + d] = load_in<IN_DT>(a.ik, (size_t)t * ID + d);
        }
        return;
    }
    const int b = b0 + blockIdx.x;
    const float inv_cr = 1.0f / (float)a.CR;
    float pk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) pk[k] = 0.f;
    for (int i = 0; i < a.CR; i++) {
        const int q = b * a.CR + i;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k < KD) {
                const int d = lane + 64 * k;
                const float x = q >= a.pos ? load_in<IN_DT>(a.ik, (size_t)(q - a.pos) * ID + d) : a.raw[(size_t)q * ID + d];
                pk[k] = __builtin_fmaf(inv_cr, x, pk[k]);  // ck::axpy with 1/CR, one key at a time
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++)
        if (k < KD) ss += pk[k] * pk[k];
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)ID + a.eps);
#pragma unroll
    for (int k = 0; k < 8; k++)
        if (k < KD) {
            const int d = lane + 64 * k;
            s_x[d] = pk[k] * r * a.gamma[d];
        }
    __syncthreads();
    rope_row(s_x, s_y, a.rope, b * a.CR, a.R, ID, lane, 64);
    __syncthreads();
    for (int d = lane; d < ID; d += 64) a.pooled[(size_t)b * ID + d] = s_y[d];
}

// ---- selection -------------------------------------------------------------------------------------------
// Inclusive sum over the wave's lanes in lane order: within each 16-lane row (DPP row shifts), then the
// totals of the rows below added (three lane reads).
__device__ __forceinline__ int wave_scan(int x, int lane) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
    const int r2 = __builtin_amdgcn_readlane(x, 47);
    return x + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}

// Exclusive sum over the workgroup's threads in thread order (wave scans, then the earlier waves' totals
// through LDS: one barrier). `s_tot` holds 16 words.
__device__ __forceinline__ int block_excl_scan(int x, int* s_tot) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int inc = wave_scan(x, lane);
    if (lane == 63) s_tot[wave] = inc;
    __syncthreads();
    const int base = (int)wave_isum(lane < wave ? (unsigned)s_tot[lane] : 0u);
    return base + inc - x;
}

// The exact top-`top` of token t's nblk block scores (by score, then the lower block id: the scores are >= +0,
// so their bit patterns order like the values), by the last workgroup to arrive; writes the token's mask
// row and key bits. Thread tid owns the blocks [per tid, per tid + per). KR > 0: per = KR and the thread
// holds their keys in registers (nblk <= KR * 1,024; one load per four keys); KR == 0: per is a multiple of
// 32 and the keys are read from memory at each use (device-coherent loads).
//
// The threshold key is found most significant digit first, 11 bits a pass (at most three passes, fewer when
// the smallest and largest keys share their top bits or the digit's bin holds exactly the keys still
// needed): the keys that match the digits found so far are counted per next digit in an LDS histogram
// (2,048 bins, LDS atomic adds), and a scan over the bins from the top, two bins a thread, finds the digit
// where the count of larger keys reaches the number still needed.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int KR, bool COH>
__device__ __forceinline__ void select_blocks(const QsaSelectArgs& a, __amdgpu_buffer_rsrc_t rs, int t, int nblk,
                                              unsigned* s_mask, int* s_misc, int* s_scan, unsigned* s_hist) {
    constexpr int AUX = COH ? kScDevice : 0;  // device-coherent loads in the scoring launch itself
    constexpr int NB = 2048;  // bins of a pass
    static_assert(NB == 2 * kQsaThreads, "two bins a thread");
    static_assert(KR == 0 || KR == 8 || KR == 16 || KR == 32 || KR == 64, "keys a thread");
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int per = KR > 0 ? KR : ((nblk + kQsaThreads - 1) / kQsaThreads + 31) & ~31;
    const int lo = min(nblk, tid * per), hi = min(nblk, lo + per);
    auto load = [&](int b) -> unsigned { return __builtin_amdgcn_raw_buffer_load_b32(rs, b * 4, 0, AUX); };
    unsigned kr[KR > 0 ? KR : 1];
    unsigned kmin = 0xFFFFFFFFu, kmax = 0u;
    if constexpr (KR > 0) {
        // every load issued before any is used. A block past nblk holds the key ~0u: scores are >= +0, so no
        // real key has bit 31 and that key never matches a prefix, equals the threshold or counts in the
        // maximum (no per-key range test, whose lane masks would stay live through every pass)
#pragma unroll
        for (int i = 0; i < KR; i += 4) {
            const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (tid * KR + i) * 4, 0, AUX));
            kr[i] = v[0], kr[i + 1] = v[1], kr[i + 2] = v[2], kr[i + 3] = v[3];
        }
        const int nv = hi - lo;  // this thread's blocks below nblk
#pragma unroll
        for (int i = 0; i < KR; i++) {
            kr[i] = i < nv ? kr[i] : 0xFFFFFFFFu;
            kmin = min(kmin, kr[i]), kmax = max(kmax, kr[i] >> 31 ? 0u : kr[i]);
        }
    } else {
        for (int b = lo; b < hi; b++) {
            const unsigned k = load(b);
            kmin = min(kmin, k), kmax = max(kmax, k);
        }
    }
    s_hist[2 * tid] = 0u, s_hist[2 * tid + 1] = 0u;  // the first pass's bins
    kmin = wave_min(kmin), kmax = wave_max(kmax);
    if (lane == 0) s_scan[wave] = (int)kmin, s_scan[16 + wave] = (int)kmax;
    __syncthreads();
    {
        const unsigned m0 = lane < 16 ? (unsigned)s_scan[lane] : 0xFFFFFFFFu;
        const unsigned m1 = lane < 16 ? (unsigned)s_scan[16 + lane] : 0u;
        kmin = wave_min(m0), kmax = wave_max(m1);  // every wave, the same reduction
    }
    const int nmw = (nblk + 31) >> 5;  // mask words holding complete blocks

    // the bits above the highest one where the smallest and largest keys differ are every key's
    const int hb = kmin == kmax ? -1 : 31 - __builtin_clz(kmin ^ kmax);
    unsigned prefix = hb < 0 ? kmin : (hb == 31 ? 0u : kmin & ~((2u << hb) - 1u));
    unsigned fmask = 0xFFFFFFFFu;  // the bits of a key the final comparison looks at
    int need = a.top;  // keys still to take among those matching the prefix
    for (int hb_ = hb, pass = 0; hb_ >= 0; pass++) {
        const int shift = max(hb_ - 10, 0), width = hb_ - shift + 1;
        const unsigned pmask = hb_ == 31 ? 0u : ~((2u << hb_) - 1u);  // the digits found so far
        const unsigned dmask = (1u << width) - 1u;
        unsigned* h = s_hist + (pass & 1) * NB;
        auto count = [&](unsigned k) {
            if ((k & pmask) == prefix)
                __hip_atomic_fetch_add(&h[(k >> shift) & dmask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        if constexpr (KR > 0) {
#pragma unroll
            for (int i = 0; i < KR; i++) count(kr[i]);
        } else {
            for (int b = lo; b < hi; b++) count(load(b));
        }
        __syncthreads();
        // the next pass's bins (last read two passes ago, before this pass's first barrier)
        s_hist[((pass + 1) & 1) * NB + 2 * tid] = 0u, s_hist[((pass + 1) & 1) * NB + 2 * tid + 1] = 0u;
        // thread tid: digits d1 = 2^width - 1 - 2 tid and d1 - 1 (from the top); the keys with a larger digit
        // are the exclusive scan of the pair counts
        const int d1 = (int)dmask - 2 * tid, d0 = d1 - 1;
        const int c1 = d1 >= 0 ? (int)h[d1] : 0, c0 = d0 >= 0 ? (int)h[d0] : 0;
        const int larger = block_excl_scan(c1 + c0, s_scan + 32);
        if (larger < need && larger + c1 + c0 >= need) {  // exactly one thread
            const bool in1 = larger + c1 >= need;
            s_misc[0] = in1 ? d1 : d0;
            s_misc[1] = in1 ? larger : larger + c1;
            s_misc[2] = in1 ? c1 : c0;
        }
        __syncthreads();
        prefix |= (unsigned)s_misc[0] << shift;
        need -= s_misc[1];
        hb_ = shift - 1;
        if (s_misc[2] == need && hb_ >= 0) {
            // every key matching the digits so far is taken: the lower bits need not be resolved
            fmask = ~((2u << hb_) - 1u);
            break;
        }
    }
    // prefix (under fmask): the top-th largest key; all keys above it are taken, and the first `need` equal
    // to it (in block order): the equal keys of the earlier threads' blocks are an exclusive scan
    int eq = 0;
    if constexpr (KR > 0) {
#pragma unroll
        for (int i = 0; i < KR; i++) eq += (kr[i] & fmask) == prefix;
    } else {
        for (int b = lo; b < hi; b++) eq += (load(b) & fmask) == prefix;
    }
    int taken = block_excl_scan(eq, s_scan + 32);
    auto selected = [&](unsigned k) {
        k &= fmask;
        bool sel = k > prefix;
        if (k == prefix) sel = taken++ < need;
        return sel;
    };
    if constexpr (KR == 8 || KR == 16) {
        unsigned bits = 0u;
#pragma unroll
        for (int i = 0; i < KR; i++) bits |= (unsigned)selected(kr[i]) << i;
        bits &= hi - lo >= KR ? (1u << KR) - 1u : (1u << (hi - lo)) - 1u;  // no bits past nblk
        // the word of blocks [32 (tid / q), + 32), q = 32 / KR threads: their parts OR-ed across the group
        constexpr int Q = 32 / KR;
        unsigned wv = bits << (KR * (tid & (Q - 1)));
        wv |= (unsigned)__builtin_amdgcn_mov_dpp((int)wv, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
        if constexpr (Q == 4) wv |= (unsigned)__builtin_amdgcn_mov_dpp((int)wv, 0x4E, 0xF, 0xF, false);  // [2,3,0,1]
        if ((tid & (Q - 1)) == 0 && tid / Q < nmw) s_mask[tid / Q] = wv;
    } else if constexpr (KR > 0) {
#pragma unroll
        for (int w = 0; w < KR / 32; w++) {
            unsigned bits = 0u;
#pragma unroll
            for (int i = 0; i < 32; i++) bits |= (unsigned)selected(kr[32 * w + i]) << i;
            const int nvw = hi - lo - 32 * w;  // this word's blocks below nblk
            bits &= nvw >= 32 ? 0xFFFFFFFFu : (nvw > 0 ? (1u << nvw) - 1u : 0u);
            if (tid * (KR / 32) + w < nmw) s_mask[tid * (KR / 32) + w] = bits;
        }
    } else {
        // lo is a multiple of 32 whenever lo < hi, so the words [lo/32, ceil(hi/32)) are this thread's alone
        for (int w = lo >> 5; lo < hi && w < (hi + 31) >> 5; w++) {
            unsigned bits = 0u;
            for (int i = 0; i < 32; i++) {
                const int b = 32 * w + i;
                if (b < hi && selected(load(b))) bits |= 1u << i;
            }
            s_mask[w] = bits;
        }
    }
    __syncthreads();
    const int kb_words = a.kb_words;
    if (a.mask)
        for (int w = tid; w < a.mask_words; w += kQsaThreads) a.mask[(size_t)t * a.mask_words + w] = w < nmw ? s_mask[w] : 0u;
    if (a.kbits)
        for (int w = tid; w < kb_words; w += kQsaThreads)
            a.kbits[(size_t)t * kb_words + w] = key_word(s_mask, w, a.CR, nblk);
}


// Grid (chunks, n), 1,024 threads: workgroup (c, t) scores blocks [64 c, 64 c + 64) of token t; the last of
// the token's workgroups to arrive selects. A token that selects nothing has its rows written by workgroup
// (0, t).
// MODE 0: score, then the last workgroup of each token selects (device-coherent score reads). For many
// blocks (64 keys a thread and more) the two run as two launches instead: MODE 1 scores only, MODE 2 (one
// workgroup a token) selects, reading the scores with plain loads (the launch boundary makes them visible):
// the device-coherent reads of 256 KB of scores from one CU, and the select's registers in every scoring
// workgroup, cost more than the second launch.
// (one workgroup a CU at most in every use: the register budget of 4 waves a SIMD, 128 registers, is the
// kernel's to use)
template <int IN_DT, int KR, int MODE, int CH = kQsaChunk>
__global__ __launch_bounds__(kQsaThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_qsa_select(QsaSelectArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    unsigned* s_mask = reinterpret_cast<unsigned*>(smem);  // [kQsaMaskLds] the token's selection
    int* s_misc = reinterpret_cast<int*>(s_mask + kQsaMaskLds);  // [16]
    int* s_tot = s_misc + 16;                               // [16] spare
    int* s_scan = s_tot + 16;                               // [48]: per-wave minima, maxima, sums
    unsigned char* work = reinterpret_cast<unsigned char*>(s_scan + 48);
    float* s_q = reinterpret_cast<float*>(work);            // scoring: [IH][ID] normed, rotated query heads
    float* s_t = s_q + a.IH * a.ID;                         // scoring: [IH][ID] the normed heads before rotation
    unsigned* s_hist = reinterpret_cast<unsigned*>(work);   // select: [2 passes][2,048] digit counts

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = blockIdx.x, t = blockIdx.y;
    const int p = a.pos + t, nblk = (p + 1) / a.CR, ID = a.ID;
    const int kb_words = a.kb_words;
    if (a.raw != nullptr && c == 0)  // the token's raw key into the cache (no block completes in this call)
        for (int d = tid; d < ID; d += kQsaThreads) a.raw[(size_t)p * ID + d] = load_in<IN_DT>(a.ik, (size_t)t * ID + d);
    if (nblk <= a.top) {  // dense: every key visible
        if (c == 0 && MODE != 1) {
            if (a.mask)
                for (int w = tid; w < a.mask_words; w += kQsaThreads) a.mask[(size_t)t * a.mask_words + w] = 0xFFFFFFFFu;
            if (a.kbits)
                for (int w = tid; w < kb_words; w += kQsaThreads) a.kbits[(size_t)t * kb_words + w] = 0xFFFFFFFFu;
        }
        return;
    }
    const int ct = (nblk + CH - 1) / CH;  // this token's workgroups (CH blocks each)
    if (c >= ct) return;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(a.scores + (size_t)t * a.stride, (short)0,
                                                                        a.stride * 4, 0x00020000);
    if constexpr (MODE == 2) {
        select_blocks<KR, false>(a, rs, t, nblk, s_mask, s_misc, s_scan, s_hist);
        return;
    }

    // this chunk's pooled keys, 16 lanes a key (RB rounds of 64 keys), DL = ID / 16 consecutive dims a lane:
    // loaded first, so that their latency hides behind the query heads' prologue
    constexpr int RB = CH / (kQsaThreads / 16);
    static_assert(RB * (kQsaThreads / 16) == CH, "whole rounds of one key per 16-lane group");
    const int grp = tid >> 4, sub = tid & 15, DL = ID >> 4;
    const int bc0 = c * CH, bc1 = min(nblk, bc0 + CH);
    float kv[RB][16];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const float* pk = a.pooled + (size_t)min(bc0 + rr * (kQsaThreads / 16) + grp, bc1 - 1) * ID + sub * DL;
#pragma unroll
        for (int i = 0; i < 16; i += 4)
            if (i < DL) {  // DL <= 16: the host keeps ID <= 256 (past the chunk: a valid row, score not stored)
                const f32x4 v = *reinterpret_cast<const f32x4*>(pk + i);
                kv[rr][i] = v[0], kv[rr][i + 1] = v[1], kv[rr][i + 2] = v[2], kv[rr][i + 3] = v[3];
            }
    }
    // the query heads: RMS-normed (gamma as stored), rotated to p; wave w takes heads w, w + 16, ...
    for (int h = wave; h < a.IH; h += kQsaThreads / 64) {
        float ss = 0.f;
        for (int d = lane; d < ID; d += 64) {
            const float x = load_in<IN_DT>(a.iq, ((size_t)t * a.IH + h) * ID + d);
            s_t[h * ID + d] = x;
            ss += x * x;
        }
        ss = wave_sum(ss);
        const float r = 1.0f / sqrtf(ss / (float)ID + a.eps);
        for (int d = lane; d < ID; d += 64) s_t[h * ID + d] = s_t[h * ID + d] * r * a.gamma[d];
    }
    __syncthreads();
    for (int i = tid; i < a.IH * ID; i += kQsaThreads) {
        const int h = i / ID;
        rope_row(s_t + h * ID, s_q + h * ID, a.rope, p, a.R, ID, i - h * ID, ID);
    }
    __syncthreads();

    // the chunk's scores: sum over the heads of relu(q_h . key), the dot products summed over each 16-lane row
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const int b = bc0 + rr * (kQsaThreads / 16) + grp;
        float sc = 0.f;
        for (int h = 0; h < a.IH; h++) {
            const float* qh = s_q + h * ID + sub * DL;
            float dp = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (i < DL) dp = __builtin_fmaf(qh[i], kv[rr][i], dp);
            dp = sum16(dp);
            sc += dp > 0.f ? dp : 0.f;  // relu; -0 and NaN contribute +0, so every score is >= +0
        }
        if (sub == 0 && b < bc1) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sc), rs, b * 4, 0, kScDevice);
    }
    if constexpr (MODE == 1) return;
    // arrive: the stores are acknowledged (device-coherent) before the counter moves
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(a.cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_misc[0] = old;
        if (old == ct - 1) __hip_atomic_store(a.cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_misc[0] != ct - 1) return;

    // ---- the last workgroup of token t: exact top-`top` by (score desc, block id asc) ---------------
    select_blocks<KR, true>(a, rs, t, nblk, s_mask, s_misc, s_scan, s_hist);  // the host sizes KR for the call's last token
}

// ---- key bits from a block mask (shaders/attention.comp:35-43) -------------------------------------------
__global__ __launch_bounds__(256) void k_qsa_key_bits(QsaKeyBitsArgs a) {
    const int w = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (w >= a.kb_words) return;
    a.kbits[(size_t)t * a.kb_words + w] = key_word(a.mask + (size_t)t * a.mask_words, w, a.CR, (a.pos + t + 1) / a.CR);
}

size_t qsa_select_lds(int IH, int ID) {
    const size_t work = std::max((size_t)2 * IH * ID * 4, (size_t)2 * 2048 * 4);
    return (size_t)(kQsaMaskLds + 32 + 48) * 4 + work;
}

int qsa_mask_lds_words() { return kQsaMaskLds; }

hipError_t launch_qsa_pool(const QsaPoolArgs& a, int in_dtype, hipStream_t s) {
    const int nbp = (a.pos + a.n) / a.CR - a.pos / a.CR;
    const dim3 grid(nbp + a.n);
    if (in_dtype == 0) hipLaunchKernelGGL(k_qsa_pool<0>, grid, dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_qsa_pool<1>, grid, dim3(64), 0, s, a);
    return hipGetLastError();
}

// Keys a thread holds in the select: the smallest of 8, 16, 32, 64 that covers nmax blocks (0: read from memory).
static int select_kr(int nmax) {
    for (int kr = 8; kr <= 64; kr *= 2)
        if (nmax <= kr * kQsaThreads) return kr;
    return 0;
}

// Largest indexer width the host accepts (heads x dims); the select's dynamic LDS grows with it.
constexpr int kQsaMaxHeadDims = 8192;

template <int IN_DT, int KR, int MODE, int CH = kQsaChunk>
static hipError_t launch_select_kr(const QsaSelectArgs& a, size_t shm, dim3 grid, hipStream_t s) {
    // The dynamic LDS limit is raised once per device to what the widest accepted indexer needs, so a later
    // call with more heads x dims than the first one still fits it.
    static std::atomic<uint64_t> raised{0};  // bit per device
    static const size_t shm_max = qsa_select_lds(1, kQsaMaxHeadDims);
    if (shm > shm_max) return hipErrorInvalidValue;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(raised.load(std::memory_order_acquire) & bit)) {
        const hipError_t e = hipFuncSetAttribute((const void*)k_qsa_select<IN_DT, KR, MODE, CH>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm_max);
        if (e != hipSuccess) return e;
        raised.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL((k_qsa_select<IN_DT, KR, MODE, CH>), grid, dim3(kQsaThreads), shm, s, a);
    return hipGetLastError();
}

template <int IN_DT>
static hipError_t launch_select_dt(const QsaSelectArgs& a, int kr, size_t shm, dim3 grid, hipStream_t s) {
    switch (kr) {
        case 8: return launch_select_kr<IN_DT, 8, 0>(a, shm, grid, s);
        case 16: return launch_select_kr<IN_DT, 16, 0>(a, shm, grid, s);
        case 32: return launch_select_kr<IN_DT, 32, 0>(a, shm, grid, s);
        default: {
            // many blocks: scoring (256 blocks a workgroup), then a select launch of one workgroup a token
            // (which does not append)
            constexpr int CH1 = 4 * kQsaChunk;
            const int nmax = (a.pos + a.n) / a.CR;
            if (hipError_t e = launch_select_kr<IN_DT, 8, 1, CH1>(a, shm, dim3((nmax + CH1 - 1) / CH1, grid.y), s)) return e;
            QsaSelectArgs b = a;
            b.raw = nullptr;
            const dim3 g1(1, grid.y);
            return kr == 64 ? launch_select_kr<IN_DT, 64, 2>(b, shm, g1, s) : launch_select_kr<IN_DT, 0, 2>(b, shm, g1, s);
        }
    }
}

hipError_t launch_qsa_select(const QsaSelectArgs& a, int in_dtype, hipStream_t s) {
    const size_t shm = qsa_select_lds(a.IH, a.ID);
    const int nmax = (a.pos + a.n) / a.CR;
    const dim3 grid((nmax + kQsaChunk - 1) / kQsaChunk > 0 ? (nmax + kQsaChunk - 1) / kQsaChunk : 1, a.n);
    const int kr = select_kr(nmax);
    return in_dtype == 0 ? launch_select_dt<0>(a, kr, shm, grid, s) : launch_select_dt<1>(a, kr, shm, grid, s);
}

hipError_t launch_qsa_key_bits(const QsaKeyBitsArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_qsa_key_bits, dim3((a.kb_words + 255) / 256, a.n), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace qw
