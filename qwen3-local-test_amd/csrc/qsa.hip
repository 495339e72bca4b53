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

// v_writelane_b32: `src` (uniform) into lane `lane` of `old` (the LLVM intrinsic, which this compiler offers
// no builtin for)
__device__ unsigned writelane(unsigned src, unsigned lane, unsigned old) __asm("llvm.amdgcn.writelane.i32");

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
// visible when block j / cr has its bit set or lies at or past nblk (the tail). A power of two below 32: the
// word holds 32 / cr whole blocks of one mask word, whose bits are spread over cr bits each by shift-and-mask
// steps and a multiply; 32 and more: one block; otherwise one division per word, the block of each following
// key by counting.
__device__ __forceinline__ unsigned key_word(const unsigned* m, int w, int cr, int nblk) {
    const int nmwc = (nblk + 31) >> 5;
    if ((cr & (cr - 1)) == 0) {
        const int lc = __builtin_ctz((unsigned)cr);
        if (cr >= 32) {
            const int blk = (32 * w) >> lc;
            const unsigned mw = (blk >> 5) < nmwc ? m[blk >> 5] : 0u;
            return blk >= nblk || ((mw >> (blk & 31)) & 1u) ? 0xFFFFFFFFu : 0u;
        }
        const int nb = 32 >> lc, blk0 = w * nb, tail = nblk * cr - 32 * w;  // keys of the word before the tail
        unsigned x = (blk0 >> 5) < nmwc ? m[blk0 >> 5] : 0u;
        if (nb < 32) x = (x >> (blk0 & 31)) & ((1u << nb) - 1u);
        switch (lc) {  // bit i to bits [cr i, cr i + cr)
            case 1:
                x = (x | (x << 8)) & 0x00FF00FFu;
                x = (x | (x << 4)) & 0x0F0F0F0Fu;
                x = (x | (x << 2)) & 0x33333333u;
                x = ((x | (x << 1)) & 0x55555555u) * 3u;
                break;
            case 2:
                x = (x | (x << 12)) & 0x000F000Fu;
                x = (x | (x << 6)) & 0x03030303u;
                x = ((x | (x << 3)) & 0x11111111u) * 15u;
                break;
            case 3:
                x = (x | (x << 14)) & 0x00030003u;
                x = ((x | (x << 7)) & 0x01010101u) * 255u;
                break;
            case 4: x = ((x & 1u) | ((x & 2u) << 15)) * 65535u; break;
            default: break;  // cr 1: the mask word itself
        }
        return tail <= 0 ? 0xFFFFFFFFu : (tail >= 32 ? x : x | (0xFFFFFFFFu << tail));
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

// Sum over the workgroup's threads, in every thread (one barrier; `s_tot` holds 16 words).
__device__ __forceinline__ int block_sum(int x, int* s_tot) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    x = (int)wave_isum((unsigned)x);
    if (lane == 0) s_tot[wave] = x;
    __syncthreads();
    return (int)wave_isum(lane < kQsaThreads / 64 ? (unsigned)s_tot[lane] : 0u);
}

// ---- the selection proper: exact top-`top` of a token's nblk block scores, by (score desc, block id asc) ---
// The scores are >= +0, so their bit patterns order like the values. The threshold's first radix digit,
// bits [30:20], comes from the token's histogram `gh` (2,048 bins), which the scoring workgroups filled
// with global atomic adds; the keys of that digit's bin (the candidates, a few hundred among 65,536 blocks
// of random scores) are compacted into LDS and resolved there, so that a pass over every key (each VALU op
// of which costs the one CU 1,024 cycles at 65,536 blocks) happens only to load them, to compact the
// candidates and to build the mask. A bin of more than kQsaCand keys (bulk exact ties) takes the fallback:
// radix passes over every key.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kQsaCand = 2048;  // candidates compacted into LDS
constexpr int kQsaHistCopies = 8;  // at most, a token's first-digit histogram copies

// The token's mask row and key bits from the selection in LDS.
__device__ __forceinline__ void write_rows(const QsaSelectArgs& a, int t, int nblk, const unsigned* s_mask) {
    const int tid = threadIdx.x, nmw = (nblk + 31) >> 5, kb_words = a.kb_words;
    if (a.mask)
        for (int w = tid; w < a.mask_words; w += kQsaThreads) a.mask[(size_t)t * a.mask_words + w] = w < nmw ? s_mask[w] : 0u;
    if (a.kbits)
        for (int w = tid; w < kb_words; w += kQsaThreads)
            a.kbits[(size_t)t * kb_words + w] = key_word(s_mask, w, a.CR, nblk);
}

// Of the candidates ck[] (blocks cb[]; places tid and tid + 1,024 filled when v0, v1), which share the bits
// above bit 20 (`prefix`), the `need` largest by (key, then the lower block) are taken: T is the smallest
// taken key, and of the keys equal to T those of blocks <= id_end (every one when id_end is ~0u). Two 10-bit
// digit passes over the keys from the top, then, when T has more ties than places, two 9-bit passes over the
// tied keys' blocks from the smallest (block ids < 2^18). LDS histograms of 1,024 bins (four, zero on entry),
// thread tid scanning one.
__device__ __forceinline__ void resolve_candidates(const unsigned* ck, const unsigned* cb, bool v0, bool v1, int need,
                                                   unsigned prefix, unsigned* s_hist, int* s_misc, int* s_scan,
                                                   unsigned& T, unsigned& id_end) {
    static_assert(kQsaCand == 2 * kQsaThreads, "two places a thread");
    const int tid = threadIdx.x;
    for (int pass = 0; pass < 2; pass++) {
        const int shift = pass == 0 ? 10 : 0;
        const unsigned pmask = pass == 0 ? 0xFFF00000u : 0xFFFFFC00u;  // the bits found so far
        unsigned* h = s_hist + pass * 1024;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const unsigned k = ck[tid + r * kQsaThreads];
            if ((r ? v1 : v0) && (k & pmask) == prefix)
                __hip_atomic_fetch_add(&h[(k >> shift) & 1023u], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __syncthreads();
        const int c = (int)h[1023 - tid];
        const int larger = block_excl_scan(c, s_scan + 32);
        if (larger < need && larger + c >= need) s_misc[3] = 1023 - tid, s_misc[4] = larger, s_misc[5] = c;
        __syncthreads();
        prefix |= (unsigned)s_misc[3] << shift;
        need -= s_misc[4];
    }
    T = prefix;
    id_end = 0xFFFFFFFFu;
    if (s_misc[5] > need) {  // more keys equal T than places
        unsigned idp = 0u;
        for (int pass = 0; pass < 2; pass++) {
            const int shift = pass == 0 ? 9 : 0;
            const unsigned pm = pass == 0 ? 0u : ~511u;
            unsigned* h = s_hist + 2048 + pass * 1024;
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int i = tid + r * kQsaThreads;
                if ((r ? v1 : v0) && ck[i] == T && (cb[i] & pm) == idp)
                    __hip_atomic_fetch_add(&h[(cb[i] >> shift) & 511u], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            __syncthreads();
            const int c = tid < 512 ? (int)h[tid] : 0;
            const int smaller = block_excl_scan(c, s_scan + 32);
            if (smaller < need && smaller + c >= need) s_misc[6] = tid, s_misc[7] = smaller;
            __syncthreads();
            idp |= (unsigned)s_misc[6] << shift;
            need -= s_misc[7];
        }
        id_end = idp;
    }
}

// The fallback: the threshold's remaining digits by passes over every key, 11 bits a pass (bits [19:9], then
// [8:0]; none when the whole bin is taken, fewer when a digit's bin holds exactly the keys still needed),
// the matching keys counted per digit in an LDS histogram (2,048 bins, zero on entry) and the bins scanned
// from the top, two a thread. The blocks are dealt in chunks of 4,096: thread tid takes blocks 4 tid ..
// 4 tid + 3 of each, one 16-byte load a chunk; KR > 0: their keys stay in registers, KR == 0: they are read
// from memory at each use. Ties at the threshold are taken in block order (the need-th smallest tied block
// by two passes over the block ids). Writes the mask into s_mask.
template <int KR, bool COH>
__device__ __forceinline__ void select_fallback(__amdgpu_buffer_rsrc_t rs, int nblk, unsigned prefix, int need,
                                                int cnt, unsigned* s_mask, int* s_misc, int* s_scan,
                                                unsigned* s_hist) {
    constexpr int AUX = COH ? kScDevice : 0;  // device-coherent loads in the scoring launch itself
    constexpr int NB = 2048;                  // bins of a pass
    constexpr int CHK = 4 * kQsaThreads;      // blocks of a chunk
    constexpr int NCK = KR / 4;               // chunks held in registers
    static_assert(NB == 2 * kQsaThreads, "two bins a thread");
    const int tid = threadIdx.x;
    const int nch = KR > 0 ? NCK : (nblk + CHK - 1) / CHK;
    // The row holds ~key, and 0 past nblk (written by the scoring, or outside the buffer's range): the key
    // ~word is then ~0u there, whose bit 31 no real key has, so it never matches a digit prefix or equals the
    // threshold (the host pads each score row to a multiple of four blocks: no load crosses the buffer's end).
    auto ld4 = [&](int j) -> u32x4 {
        return ~__builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (j * CHK + 4 * tid) * 4, 0, AUX));
    };
    u32x4 kr[NCK > 0 ? NCK : 1];
    if constexpr (KR > 0) {
#pragma unroll
        for (int j = 0; j < NCK; j++) kr[j] = ld4(j);
    }
    // f(key, block) over this thread's keys
    auto each = [&](auto&& f) {
        if constexpr (KR > 0) {
#pragma unroll
            for (int j = 0; j < NCK; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) f(kr[j][r], j * CHK + 4 * tid + r);
        } else {
            for (int j = 0; j < nch; j++) {
                const u32x4 v = ld4(j);
#pragma unroll
                for (int r = 0; r < 4; r++) f(v[r], j * CHK + 4 * tid + r);
            }
        }
    };
    unsigned fmask = 0xFFF00000u;  // the bits of a key the final comparison looks at
    if (cnt != need) {  // else the whole bin is taken
        fmask = 0xFFFFFFFFu;
        for (int hb_ = 19, pass = 0; hb_ >= 0; pass++) {
            const int shift = max(hb_ - 10, 0), width = hb_ - shift + 1;
            const unsigned pmask = ~((2u << hb_) - 1u);  // the digits found so far
            const unsigned dmask = (1u << width) - 1u;
            unsigned* h = s_hist + (pass & 1) * NB;
            each([&](unsigned k, int) {
                if ((k & pmask) == prefix)
                    __hip_atomic_fetch_add(&h[(k >> shift) & dmask], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            });
            __syncthreads();
            // the next pass's bins (last read two passes ago, before this pass's first barrier)
            s_hist[((pass + 1) & 1) * NB + 2 * tid] = 0u, s_hist[((pass + 1) & 1) * NB + 2 * tid + 1] = 0u;
            // thread tid: digits d1 = 2^width - 1 - 2 tid and d1 - 1 (from the top); the keys with a larger
            // digit are the exclusive scan of the pair counts
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
    }
    // prefix (under fmask): the top-th largest key; every key above it is taken, and the first `need` keys
    // equal to it in block order. The held keys keep only the compared bits (bit 31, set on the blocks past
    // nblk, among them), and the comparisons below are not carried from the count to the marking: both would
    // hold a second copy of every key.
    if constexpr (KR > 0) {
#pragma unroll
        for (int j = 0; j < NCK; j++) kr[j] &= fmask;
    }
    int eq = 0;
    each([&](unsigned k, int) { eq += (k & fmask) == prefix; });
    unsigned id_end = 0xFFFFFFFFu;  // equal keys of blocks <= id_end are taken
    if (block_sum(eq, s_scan) > need) {
        // the need-th smallest block among the equal keys (every read of the bins ended before the last
        // barrier)
        s_hist[2 * tid] = 0u, s_hist[2 * tid + 1] = 0u, s_hist[NB + 2 * tid] = 0u, s_hist[NB + 2 * tid + 1] = 0u;
        __syncthreads();
        unsigned idp = 0u;
        int need2 = need;
        for (int pass = 0; pass < 2; pass++) {
            const int shift = pass == 0 ? 7 : 0;
            const unsigned pm = pass == 0 ? 0u : ~127u;  // the id bits found so far
            unsigned* h = s_hist + pass * NB;
            each([&](unsigned k, int b) {
                if ((k & fmask) == prefix && ((unsigned)b & pm) == idp)
                    __hip_atomic_fetch_add(&h[((unsigned)b >> shift) & 2047u], 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
            });
            __syncthreads();
            const int c0 = (int)h[2 * tid], c1 = (int)h[2 * tid + 1];  // ascending digits
            const int smaller = block_excl_scan(c0 + c1, s_scan + 32);
            if (smaller < need2 && smaller + c0 + c1 >= need2) {  // exactly one thread
                const bool in0 = smaller + c0 >= need2;
                s_misc[4] = in0 ? 2 * tid : 2 * tid + 1;
                s_misc[5] = in0 ? smaller : smaller + c0;
            }
            __syncthreads();
            idp |= (unsigned)s_misc[4] << shift;
            need2 -= s_misc[5];
        }
        id_end = idp;
    }
    asm volatile("" : "+v"(prefix));
    // the mask: a chunk's four bits of each thread, OR-ed over eight lanes into the word of blocks
    // [32 (tid / 8), + 32) of the chunk
    const int nmw = (nblk + 31) >> 5;
    auto mark = [&](u32x4 v, int j) {
        unsigned bits = 0u;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const unsigned k = v[r] & fmask, b = (unsigned)(j * CHK + 4 * tid + r);
            const bool sel = (v[r] >> 31) == 0u && (k > prefix || (k == prefix && b <= id_end));
            bits |= (unsigned)sel << r;
        }
        unsigned wv = bits << (4 * (tid & 7));
        wv |= (unsigned)__builtin_amdgcn_mov_dpp((int)wv, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
        wv |= (unsigned)__builtin_amdgcn_mov_dpp((int)wv, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
        wv |= (unsigned)__builtin_amdgcn_mov_dpp((int)wv, 0x141, 0xF, 0xF, false);  // row_half_mirror
        const int w = j * (CHK / 32) + (tid >> 3);
        if ((tid & 7) == 0 && w < nmw) s_mask[w] = wv;
    };
    if constexpr (KR > 0) {
#pragma unroll
        for (int j = 0; j < NCK; j++) mark(kr[j], j);
    } else {
        for (int j = 0; j < nch; j++) mark(ld4(j), j);
    }
}

// The token's first-digit histogram (nh copies of 2,048 bins at gh): thread tid's bins 2,047 - 2 tid and the
// one below, summed over the copies (one 8-byte device-coherent load a copy, issued at construction; copies
// past nh lie outside the resource and read 0).
struct FirstDigit {
    __amdgpu_buffer_rsrc_t rh;
    u32x2 gv[kQsaHistCopies];
    __device__ __forceinline__ FirstDigit(unsigned* gh, int nh) {
        rh = __builtin_amdgcn_make_buffer_rsrc(gh, (short)0, nh * 2048 * 4, 0x00020000);
#pragma unroll
        for (int i = 0; i < kQsaHistCopies; i++)
            gv[i] = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(rh, (2048 * i + 2046 - 2 * (int)threadIdx.x) * 4, 0, kScDevice));
    }
    // the bin of the top-th largest key, scanned from the top two bins a thread: s_misc[0] the digit, [1] the
    // keys of larger digits, [2] the bin's keys (every thread reads them after the barrier)
    __device__ __forceinline__ void scan(int top, int* s_misc, int* s_scan) const {
        const int tid = threadIdx.x;
        unsigned g1 = 0u, g0 = 0u;
#pragma unroll
        for (int i = 0; i < kQsaHistCopies; i++) g0 += gv[i][0], g1 += gv[i][1];
        const int larger = block_excl_scan((int)(g1 + g0), s_scan + 32);
        if (larger < top && larger + (int)(g1 + g0) >= top) {  // exactly one thread
            const bool in1 = larger + (int)g1 >= top;
            s_misc[0] = in1 ? 2047 - 2 * tid : 2046 - 2 * tid;
            s_misc[1] = in1 ? larger : larger + (int)g1;
            s_misc[2] = (int)(in1 ? g1 : g0);
        }
        __syncthreads();
    }
    // zero for the next launch (after every reader has its counts)
    __device__ __forceinline__ void clear() const {
#pragma unroll
        for (int i = 0; i < kQsaHistCopies; i++)
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{0u, 0u}, rh, (2048 * i + 2046 - 2 * (int)threadIdx.x) * 4, 0,
                                                  kScDevice);
    }
};

// The selection of token t by one workgroup (the row `rs` holds ~score per block and 0 past nblk; the
// token's first-digit histogram is `nh` copies of 2,048 bins at gh, summed here and cleared for the next
// launch); writes the token's mask row and key bits. Thread tid takes blocks 1,024 j + tid (KR > 0: KR of
// them held in registers, nblk <= KR * 1,024; KR == 0: read from memory at each use), so that each wave's
// ballot over one of them is two mask words. A stored word L orders opposite to its key, and as a signed
// value every L of a block (bit 31 set) lies below the 0 past nblk: key > T is (int) L < (int) ~T.
template <int KR, bool COH>
__device__ __forceinline__ void select_blocks(const QsaSelectArgs& a, __amdgpu_buffer_rsrc_t rs, int t, int nblk,
                                              unsigned* s_mask, int* s_misc, int* s_scan, unsigned* s_hist,
                                              unsigned* s_ck, unsigned* gh, int nh) {
    constexpr int AUX = COH ? kScDevice : 0;  // device-coherent loads in the scoring launch itself
    static_assert(KR == 0 || KR == 8 || KR == 16 || KR == 32 || KR == 64, "keys a thread");
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nch = KR > 0 ? KR : (nblk + kQsaThreads - 1) / kQsaThreads;
    unsigned* s_cb = s_ck + kQsaCand;
    const FirstDigit fd(gh, nh);
    auto ld = [&](int j) -> unsigned { return __builtin_amdgcn_raw_buffer_load_b32(rs, (j * kQsaThreads + tid) * 4, 0, AUX); };
    unsigned kr[KR > 0 ? KR : 1];
    if constexpr (KR > 0) {
#pragma unroll
        for (int j = 0; j < KR; j++) kr[j] = ld(j);  // every load issued before any is used
    }
    // the later passes' LDS bins start at zero
#pragma unroll
    for (int i = 0; i < 4; i++) s_hist[tid + i * kQsaThreads] = 0u;
    fd.scan(a.top, s_misc, s_scan);
    fd.clear();
    const unsigned d1 = (unsigned)s_misc[0];
    const int need = a.top - s_misc[1], cnt = s_misc[2];  // to take from the bin, of cnt
    if (cnt > kQsaCand) {
        select_fallback<KR, COH>(rs, nblk, d1 << 20, need, cnt, s_mask, s_misc, s_scan, s_hist);
    } else {
        auto word = [&](int j) -> unsigned {
            if constexpr (KR > 0) return kr[j];
            else return ld(j);
        };
        // the candidates (key bits [30:20] == d1, i.e. L bits [31:20] == 0xFFF - d1; 0 past nblk never is)
        // into LDS: wave w fills places [w kQsaW, + kQsaW) in order (per chunk a ballot, each candidate's place
        // the count of the lanes below it); a wave with more candidates than places sends the whole selection
        // to the fallback
        constexpr int kQsaW = kQsaCand / (kQsaThreads / 64);
        const unsigned dL = 0xFFFu - d1;
        int nw = 0;  // the wave's candidates so far (uniform)
        auto compact = [&](int j) {
            const unsigned L = word(j);
            const bool c = (L >> 20) == dL;
            const unsigned long long bal = __ballot(c);
            if (bal) {
                const int at = nw + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
                if (c && at < kQsaW) s_ck[wave * kQsaW + at] = ~L, s_cb[wave * kQsaW + at] = (unsigned)(j * kQsaThreads + tid);
                nw += (int)__popcll(bal);
            }
        };
        if constexpr (KR > 0) {
#pragma unroll
            for (int j = 0; j < KR; j++) compact(j);
        } else {
            for (int j = 0; j < nch; j++) compact(j);
        }
        if (lane == 0) s_scan[wave] = nw;
        __syncthreads();
        const int nwl = lane < kQsaThreads / 64 ? s_scan[lane] : 0;
        if (wave_max((unsigned)nwl) > (unsigned)kQsaW) {  // uniform: every wave reads the same counts
            select_fallback<KR, COH>(rs, nblk, d1 << 20, need, cnt, s_mask, s_misc, s_scan, s_hist);
            __syncthreads();
            write_rows(a, t, nblk, s_mask);
            return;
        }
        unsigned T, id_end;
        const int* nwv = s_scan;  // wave w's candidates fill places [w kQsaW, + nwv[w])
        resolve_candidates(s_ck, s_cb, (tid % kQsaW) < nwv[tid / kQsaW],
                           ((tid + kQsaThreads) % kQsaW) < nwv[(tid + kQsaThreads) / kQsaW], need, d1 << 20, s_hist,
                           s_misc, s_scan, T, id_end);
        // the mask: per wave and chunk, the ballot of the taken blocks is mask words 32 j + 2 wave (+1),
        // gathered into the lanes of one register per 32 chunks and stored together. A tied key is taken when
        // its block 1,024 j + tid <= id_end (uniform operands: no block id is held per key).
        const int nT = (int)~__builtin_amdgcn_readfirstlane(T);
        const int ide = (int)__builtin_amdgcn_readfirstlane(id_end);
        // the ballot of chunk j into lanes 2 jj, 2 jj + 1 of acc
        auto take = [&](unsigned long long bal, unsigned acc, int jj) -> unsigned {
            return writelane((unsigned)(bal >> 32), 2 * jj + 1, writelane((unsigned)bal, 2 * jj, acc));
        };
        auto put = [&](int jb, unsigned acc) {
            if (lane < 2 * min(32, nch - jb)) s_mask[32 * (jb + (lane >> 1)) + 2 * wave + (lane & 1)] = acc;
        };
        auto marks = [&](auto&& sel) {
            if constexpr (KR > 0) {
#pragma unroll
                for (int jb = 0; jb < KR; jb += 32) {
                    unsigned acc = 0u;
#pragma unroll
                    for (int jj = 0; jj < (KR < 32 ? KR : 32); jj++) acc = take(__ballot(sel(jb + jj)), acc, jj);
                    put(jb, acc);
                }
            } else {
                for (int jb = 0; jb < nch; jb += 32) {
                    unsigned acc = 0u;
                    for (int jj = 0; jj < 32 && jb + jj < nch; jj++) acc = take(__ballot(sel(jb + jj)), acc, jj);
                    put(jb, acc);
                }
            }
        };
        if (id_end == 0xFFFFFFFFu)  // every key equal to T is taken
            marks([&](int j) { return (int)word(j) <= nT; });
        else
            marks([&](int j) {
                const int L = (int)word(j);
                return L < nT || (L == nT && tid <= ide - j * kQsaThreads);
            });
    }
    __syncthreads();
    write_rows(a, t, nblk, s_mask);
}

// The two-launch form's selection, spread: workgroup (g, t) takes blocks [4,096 g, + 4,096) of token t
// (thread tid: blocks 4,096 g + 1,024 j + tid, j < 4). Every workgroup finds the threshold's first digit from
// the histogram itself, writes its part of the mask row and key bits with the blocks above that digit taken
// (device-coherent stores), and hands the digit's keys (the candidates) to its places in the token's
// candidate area; the last to arrive resolves the candidates and ORs the taken ones' bits in (device-scope
// atomics, after every part is stored). A workgroup with more candidates than its places, or more candidates
// in all than LDS holds, sends the token to the one-workgroup selection over every key.
__device__ __forceinline__ void select_spread(const QsaSelectArgs& a, __amdgpu_buffer_rsrc_t rs, int t, int nblk,
                                              int g, unsigned* s_mask, int* s_misc, int* s_scan, unsigned* s_hist,
                                              unsigned* s_ck, unsigned* gh) {
    constexpr int J = kQsaSelBlocks / kQsaThreads;  // keys a thread
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int gt = (nblk + kQsaSelBlocks - 1) / kQsaSelBlocks;  // the token's workgroups
    const FirstDigit fd(gh, a.hcopies);
    unsigned L[J];
#pragma unroll
    for (int j = 0; j < J; j++)
        L[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, (g * kQsaSelBlocks + j * kQsaThreads + tid) * 4, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) s_hist[tid + i * kQsaThreads] = 0u;  // the last workgroup's bins
    fd.scan(a.top, s_misc, s_scan);
    const unsigned d1 = (unsigned)s_misc[0], dL = 0xFFFu - d1;
    const int need = a.top - s_misc[1], cnt = s_misc[2];
    // taken outright: key digit above d1, i.e. L bits [31:20] below 0xFFF - d1 (as signed values, so that the
    // 0 past nblk is not); per chunk the wave's ballot is mask words 128 g + 32 j + 2 wave (+1). Candidates:
    // L bits [31:20] == 0xFFF - d1, counted per wave
    unsigned long long cbal[J];
    int nw = 0;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const unsigned long long above = __ballot((int)L[j] < (int)(dL << 20));
        if (lane < 2) s_mask[128 * g + 32 * j + 2 * wave + lane] = lane ? (unsigned)(above >> 32) : (unsigned)above;
        cbal[j] = __ballot((L[j] >> 20) == dL);
        nw += (int)__popcll(cbal[j]);
    }
    if (lane == 0) s_scan[wave] = nw;
    __syncthreads();
    int at = 0, tot = 0;  // this wave's first place; the workgroup's candidates
    for (int w = 0; w < kQsaThreads / 64; w++) {
        const int c = s_scan[w];
        at += w < wave ? c : 0;
        tot += c;
    }
    unsigned* ck = a.cand + ((size_t)t * kQsaSelWgMax + g) * 2 * kQsaCandWg;  // [keys][blocks]
#pragma unroll
    for (int j = 0; j < J; j++) {
        const unsigned long long bal = cbal[j];
        const int pos = at + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
        if (((bal >> lane) & 1ull) && pos < kQsaCandWg) {
            __hip_atomic_store(ck + pos, ~L[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ck + kQsaCandWg + pos, (unsigned)(g * kQsaSelBlocks + j * kQsaThreads + tid),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        at += (int)__popcll(bal);
    }
    if (tid == 0) __hip_atomic_store(a.cand_n + (size_t)t * kQsaSelWgMax + g, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // this workgroup's words of the mask row and key bits (the last one's run to the rows' ends); the key words
    // of blocks [4,096 g, + 4,096) read only this workgroup's mask words (4,096 CR keys are whole words)
    const int nmw = (nblk + 31) >> 5, last = g == gt - 1;
    if (a.mask) {
        const int w1 = last ? a.mask_words : min(a.mask_words, 128 * (g + 1));
        for (int w = 128 * g + tid; w < w1; w += kQsaThreads)
            __hip_atomic_store(a.mask + (size_t)t * a.mask_words + w, w < nmw ? s_mask[w] : 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    if (a.kbits) {
        const int k0 = 128 * g * a.CR, k1 = last ? a.kb_words : min(a.kb_words, k0 + 128 * a.CR);
        for (int w = k0 + tid; w < k1; w += kQsaThreads)
            __hip_atomic_store(a.kbits + (size_t)t * a.kb_words + w, key_word(s_mask, w, a.CR, nblk), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // arrive: every store acknowledged before the counter moves
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(a.cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_misc[8] = old;
        if (old == gt - 1) __hip_atomic_store(a.cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_misc[8] != gt - 1) return;

    // ---- the last workgroup: every part is stored; the candidates into LDS, in workgroup order -------------
    int* s_cn = reinterpret_cast<int*>(s_mask);  // [gt + 1] the workgroups' first places
    const int cg = tid < gt ? __hip_atomic_load(a.cand_n + (size_t)t * kQsaSelWgMax + tid, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0;
    const int over = __syncthreads_or(cg > kQsaCandWg);
    const int first = block_excl_scan(cg, s_scan + 32);
    if (tid < gt) s_cn[tid] = first;
    if (tid == gt - 1) s_cn[gt] = first + cg;
    __syncthreads();
    const int total = s_cn[gt];
    if (over || total != cnt || total > kQsaCand) {
        select_blocks<0, false>(a, rs, t, nblk, s_mask, s_misc, s_scan, s_hist, s_ck, gh, a.hcopies);
        return;
    }
    unsigned* s_cb = s_ck + kQsaCand;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = tid + r * kQsaThreads;
        if (i < total) {
            int gg = 0;
            while (s_cn[gg + 1] <= i) gg++;
            const unsigned* src = a.cand + ((size_t)t * kQsaSelWgMax + gg) * 2 * kQsaCandWg + (i - s_cn[gg]);
            s_ck[i] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_cb[i] = __hip_atomic_load(src + kQsaCandWg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    fd.clear();  // every workgroup read its counts before arriving
    __syncthreads();
    unsigned T, id_end;
    resolve_candidates(s_ck, s_cb, tid < total, tid + kQsaThreads < total, need, d1 << 20, s_hist, s_misc, s_scan, T,
                       id_end);
    // the taken candidates' bits into the stored rows
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = tid + r * kQsaThreads;
        if (i >= total) continue;
        const unsigned k = s_ck[i], b = s_cb[i];
        if (!(k > T || (k == T && b <= id_end))) continue;
        if (a.mask)
            __hip_atomic_fetch_or(a.mask + (size_t)t * a.mask_words + (b >> 5), 1u << (b & 31), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        if (a.kbits) {
            const int k0 = (int)b * a.CR, k1 = k0 + a.CR;  // the block's keys
            for (int w = k0 >> 5; w <= (k1 - 1) >> 5 && w < a.kb_words; w++) {
                const int lo = max(k0, 32 * w) - 32 * w, hi = min(k1, 32 * w + 32) - 32 * w;
                const unsigned bits = (hi == 32 ? 0xFFFFFFFFu : (1u << hi) - 1u) & ~((1u << lo) - 1u);
                __hip_atomic_fetch_or(a.kbits + (size_t)t * a.kb_words + w, bits, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// The scores of blocks [bc0, bc1) of token t at position p: sum over the heads of relu(q_h . key), stored
// device-coherently into the token's score row as ~bits, and each score's first radix digit (bits [30:20])
// counted in the LDS histogram `hist`. 16 lanes a pooled key (coalesced rows), DL = ID / 16 consecutive dims a lane,
// RB rounds of 64 keys; the keys are loaded first, so that their latency hides behind the query heads'
// prologue (RMS norm with the gamma as stored, rope to p).
template <int IN_DT, int DL, int RB>
__device__ __forceinline__ void score_chunk(const QsaSelectArgs& a, __amdgpu_buffer_rsrc_t rs, int t, int p, int bc0,
                                            int bc1, float* s_q, float* s_t, unsigned* hist) {
    constexpr int ID = 16 * DL, G = kQsaThreads / 16;  // dims; keys a round
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, grp = tid >> 4, sub = tid & 15;
    float kv[RB][DL];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        // past the chunk: a valid row, its score not stored
        const float* pk = a.pooled + (size_t)min(bc0 + rr * G + grp, bc1 - 1) * ID + sub * DL;
#pragma unroll
        for (int i = 0; i < DL; i += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(pk + i);
            kv[rr][i] = v[0], kv[rr][i + 1] = v[1], kv[rr][i + 2] = v[2], kv[rr][i + 3] = v[3];
        }
    }
    // the query heads: wave w takes heads w, w + 16, ...
    for (int h = wave; h < a.IH; h += kQsaThreads / 64) {
        float x[ID / 64], ss = 0.f;
#pragma unroll
        for (int k = 0; k < ID / 64; k++) {
            x[k] = load_in<IN_DT>(a.iq, ((size_t)t * a.IH + h) * ID + lane + 64 * k);
            ss += x[k] * x[k];
        }
        ss = wave_sum(ss);
        const float r = 1.0f / sqrtf(ss / (float)ID + a.eps);
#pragma unroll
        for (int k = 0; k < ID / 64; k++) s_t[h * ID + lane + 64 * k] = x[k] * r * a.gamma[lane + 64 * k];
    }
    __syncthreads();
    for (int i = tid; i < a.IH * ID; i += kQsaThreads) {
        const int h = i / ID;
        rope_row(s_t + h * ID, s_q + h * ID, a.rope, p, a.R, ID, i - h * ID, ID);
    }
    __syncthreads();
    float sc[RB];
#pragma unroll
    for (int rr = 0; rr < RB; rr++) sc[rr] = 0.f;
    for (int h = 0; h < a.IH; h++) {
        float q[DL];
#pragma unroll
        for (int i = 0; i < DL; i += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(s_q + h * ID + sub * DL + i);
            q[i] = v[0], q[i + 1] = v[1], q[i + 2] = v[2], q[i + 3] = v[3];
        }
#pragma unroll
        for (int rr = 0; rr < RB; rr++) {
            float dp = 0.f;
#pragma unroll
            for (int i = 0; i < DL; i++) dp = __builtin_fmaf(q[i], kv[rr][i], dp);
            dp = sum16(dp);
            sc[rr] += dp > 0.f ? dp : 0.f;  // relu; -0 and NaN contribute +0, so every score is >= +0
        }
    }
#pragma unroll
    for (int rr = 0; rr < RB; rr++) {
        const int b = bc0 + rr * G + grp;
        if (sub == 0 && b < bc1) {
            __builtin_amdgcn_raw_buffer_store_b32(~__float_as_uint(sc[rr]), rs, b * 4, 0, kScDevice);
            // bits [30:20] (a score is >= +0: bit 31 is clear)
            __hip_atomic_fetch_add(&hist[__float_as_uint(sc[rr]) >> 20], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
}

// Grid (chunks, n), 1,024 threads: workgroup (c, t) scores blocks [CH c, CH c + CH) of token t and adds the
// counts of its scores' first radix digit into the token's histogram; the last of the token's workgroups to
// arrive selects. A token that selects nothing has its rows written by workgroup (0, t).
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
    unsigned* s_mask = reinterpret_cast<unsigned*>(smem);  // [kQsaMaskLds] the token's selection; scoring: the
                                                           // first-digit counts [2,048]
    int* s_misc = reinterpret_cast<int*>(s_mask + kQsaMaskLds);  // [16]
    int* s_tot = s_misc + 16;                               // [16] spare
    int* s_scan = s_tot + 16;                               // [48]: per-wave sums
    unsigned char* work = reinterpret_cast<unsigned char*>(s_scan + 48);
    float* s_q = reinterpret_cast<float*>(work);            // scoring: [IH][ID] normed, rotated query heads
    float* s_t = s_q + a.IH * a.ID;                         // scoring: [IH][ID] the normed heads before rotation
    unsigned* s_hist = reinterpret_cast<unsigned*>(work);   // select: [4,096] digit counts
    unsigned* s_ck = s_hist + 4096;                         // select: [2][kQsaCand] candidate keys, blocks

    const int tid = threadIdx.x;
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
    unsigned* gh = a.hist + (size_t)t * a.hcopies * 2048;  // the token's histogram copies
    if constexpr (MODE == 2) {
        select_spread(a, rs, t, nblk, c, s_mask, s_misc, s_scan, s_hist, s_ck, gh);
        return;
    }
    s_mask[tid] = 0u, s_mask[tid + kQsaThreads] = 0u;  // the chunk's first-digit counts
    if (c == ct - 1)  // the row past nblk reads 0 (its words up to the row's end, a multiple of four)
        for (int b = nblk + tid; b < a.stride; b += kQsaThreads)
            __builtin_amdgcn_raw_buffer_store_b32(0u, rs, b * 4, 0, kScDevice);

    constexpr int RB = CH / (kQsaThreads / 16);
    static_assert(RB * (kQsaThreads / 16) == CH, "whole rounds of one key per 16-lane group");
    const int bc0 = c * CH, bc1 = min(nblk, bc0 + CH);
    switch (ID) {  // the host keeps ID a multiple of 64, <= 256
        case 64: score_chunk<IN_DT, 4, RB>(a, rs, t, p, bc0, bc1, s_q, s_t, s_mask); break;
        case 128: score_chunk<IN_DT, 8, RB>(a, rs, t, p, bc0, bc1, s_q, s_t, s_mask); break;
        case 192: score_chunk<IN_DT, 12, RB>(a, rs, t, p, bc0, bc1, s_q, s_t, s_mask); break;
        default: score_chunk<IN_DT, 16, RB>(a, rs, t, p, bc0, bc1, s_q, s_t, s_mask); break;
    }
    // the chunk's counts into one of the token's histogram copies (workgroups in turn: fewer adds meet at
    // one address), which the selecting workgroup sums and clears
    __syncthreads();
    unsigned* gc = gh + (size_t)(c % a.hcopies) * 2048;
    for (int i = tid; i < 2048; i += kQsaThreads)
        if (const unsigned v = s_mask[i]) __hip_atomic_fetch_add(gc + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (MODE == 1) return;
    // arrive: the score stores and histogram adds are acknowledged (device-coherent) before the counter moves
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
    select_blocks<KR, true>(a, rs, t, nblk, s_mask, s_misc, s_scan, s_hist, s_ck, gh, a.hcopies);  // KR: the last token's
}

// ---- key bits from a block mask (shaders/attention.comp:35-43) -------------------------------------------
__global__ __launch_bounds__(256) void k_qsa_key_bits(QsaKeyBitsArgs a) {
    const int w = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (w >= a.kb_words) return;
    a.kbits[(size_t)t * a.kb_words + w] = key_word(a.mask + (size_t)t * a.mask_words, w, a.CR, (a.pos + t + 1) / a.CR);
}

size_t qsa_select_lds(int IH, int ID) {
    const size_t work = std::max((size_t)2 * IH * ID * 4, (size_t)(4096 + 2 * kQsaCand) * 4);
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

int qsa_select_tokens(int nmax) {
    const int kr = select_kr(nmax);
    return kr >= 64 || kr == 0 ? kQsaCandTokens : 1 << 30;  // the two-launch form hands candidates over
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
            // many blocks: scoring (256 blocks a workgroup), then the spread selection launch (4,096 blocks a
            // workgroup; it does not append)
            constexpr int CH1 = 4 * kQsaChunk;
            const int nmax = (a.pos + a.n) / a.CR;
            if (a.n > kQsaCandTokens || a.cand == nullptr || a.cand_n == nullptr) return hipErrorInvalidValue;
            if (hipError_t e = launch_select_kr<IN_DT, 8, 1, CH1>(a, shm, dim3((nmax + CH1 - 1) / CH1, grid.y), s)) return e;
            QsaSelectArgs b = a;
            b.raw = nullptr;
            return launch_select_kr<IN_DT, 0, 2, kQsaSelBlocks>(b, shm, dim3((nmax + kQsaSelBlocks - 1) / kQsaSelBlocks, grid.y), s);
        }
    }
}

hipError_t launch_qsa_select(const QsaSelectArgs& a, int in_dtype, hipStream_t s) {
    if (a.hcopies < 1 || a.hcopies > kQsaHistCopies || a.n * a.hcopies > kQsaHistTokens || a.hist == nullptr ||
        a.stride % 4)
        return hipErrorInvalidValue;
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
