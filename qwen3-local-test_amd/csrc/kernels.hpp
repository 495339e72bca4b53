// Host-side launchers of the gfx950 kernels (internal to libqwattn; the C ABI in qwattn.cpp checks
// every shape and pointer before calling these). K/V caches use the blocked layout of common.hpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qw {

constexpr float kLog2eHost = 1.4426950408889634f;

struct NormRopeArgs {
    const void* qg;      // [n][NH][2D]
    const void* k;       // [n][NKV][D]
    const void* v;       // [n][NKV][D]
    const float* qn;     // [D], w of the (1 + w) multiplier
    const float* kn;     // [D]
    const float* rope;   // [>= pos+n][R/2][2]
    uint16_t* kcache;    // blocked fp16
    uint16_t* vcache;    // blocked fp16
    void* q_out;         // [n][NH][D] fp32, or fp16 pre-scaled by log2(e)/sqrt(D); NULL: K/V rows only
    int pos, n, NH, NKV, R;
    float eps, q_scale;
    int cap;             // capacity (positions) of the caches
};
hipError_t launch_qk_norm_rope(const NormRopeArgs& a, int D, int in_dtype, int q_dtype, hipStream_t s);

// Split-KV decode / verify. With `fused`, q is the projection output qg [n][NH][2D] (in_dtype) and the
// kernel also does the QK-norm, RoPE and the K/V append of the n new tokens (knew/vnew [n][NKV][D]);
// otherwise q is the normalized, rotated query [n][NH][D] fp32 and the new rows are already cached.
struct DecodeArgs {
    const void* q;
    const void* knew;
    const void* vnew;
    const float* qn;      // fused: norm weights w (multiplier 1 + w)
    const float* kn;
    const float* rope;    // fused: rope table
    uint16_t* kc;         // blocked K cache
    uint16_t* vc;         // blocked V cache
    float* part_o;        // [n*NH][n_split][D]
    float* part_ml;       // [n*NH][n_split][2]: running max (log2 units), sum
    int pos, n, NH, NKV, R;
    int cq, cr;           // split z holds the 32-key blocks [z*cq + min(z, cr), (z+1)*cq + min(z+1, cr))
    int n_split;
    float eps, q_scale;   // q_scale = log2(e) / sqrt(D)
    float* out;           // fused decode: the gated output [n][NH][D], combined in the same launch (nullptr:
                          // partials only, for a separate combine)
    unsigned long long* ep;  // with out: per KV head, the launch counter the epochs come from (zero at first)
    float* rec;           // with out: [n*NH][n_split][4] split records (m, l, epoch tag, 0)
    int ncomb;            // with out: output rows (n * NH), each combined by nds of the last chunks of its
                          // KV head (up to 8 rows) or 16-row slice, one slice of D / nds dims each
    int nds;              // with out: 1, 2, 4 or 8 (D / nds >= 16)
    int cap;              // capacity (positions) of the caches kc, vc
    int* err;             // a bounded wait that gives up stores its kWait* code here (nullptr: not reported)
    const unsigned* kbits;  // QSA: per-token key visibility bits [n][kb_words] (nullptr: dense attention)
    int kb_words;
    int spin_max;         // polls of the in-launch combine's flag wait before it gives up
    int epoch_skew;       // added to the epoch the combine waits for: 0, or nonzero to force the give-up path
};

// Codes a kernel stores into DecodeArgs::err when a bounded wait gives up (the launch's output is then
// not valid; the host reports QWATTN_ETIMEOUT)
constexpr int kWaitCombineFlags = 1;  // a combining workgroup: a split's record never came
constexpr int kWaitRingLoad = 3;      // a loader wave: its compute wave never released a slot
constexpr int kWaitRingCompute = 4;   // a compute wave: its loader wave never published a tile
constexpr int kSpinDefault = 1 << 22; // default DecodeArgs::spin_max (seconds of polling)
constexpr int kQsaTiles = 256;        // QSA decode (up to 8 rows): tiles per streaming workgroup at most
constexpr int kQsaChunkTiles = 64;    // QSA verify (16-row slices): tiles per chunk at most
hipError_t launch_decode(const DecodeArgs& a, int D, bool fused, int in_dtype, hipStream_t s);

// One-launch decode: combining workgroup j of a KV head's m adds (j+1)K/m - jK/m (integer division,
// K = kEpochStep) to its head's counter when done. The shares add up to exactly K, so a launch whose
// combiners have all finished advances the counter by K whatever their number (1..32), any part of them by
// less, and floor(counter / K) + 1 is the epoch of the next launch — also for a participant that reads the
// counter after some combiners of its own launch are done.
constexpr unsigned kEpochStep = 840;
constexpr int kCombSlots = 128;       // split partials a combining workgroup stages in LDS at once
constexpr int kCombGroup = 32;        // splits merged together (in a fixed order) once all are staged

struct CombineArgs {
    const float* part_o;
    const float* part_ml;
    const void* qg;       // gate = qg[t][h][D + d]
    float* out;           // [n][NH][D]
    int n, NH, n_split;
};
hipError_t launch_combine(const CombineArgs& a, int D, int in_dtype, hipStream_t s);

struct PrefillArgs {
    const void* q;        // [n][NH][D]: fp16 pre-scaled; NULL: the kernel normalizes the query half of qg
    const uint16_t* kc;
    const uint16_t* vc;
    const void* qg;       // gate source
    float* out;           // [n][NH][D]
    int pos, n, NH, NKV;
    float q_scale;
    int cap;              // capacity (positions) of the caches kc, vc
    float* part;          // [NKV][slots][2 halves][kPfWaves][pf_part_floats(D)]: partials of split query tiles
    int* cnt;             // [NKV][slots][kPfWaves] arrival counters, zero between launches
    int slots;            // split tiles per KV head: pf_split_slots(n_qt, split_all)
    int split_all;        // 0: short and long tiles paired; 1: every tile's keys split over two workgroups
    // queries normalized in the kernel (q == NULL): RMSNorm weights, rope table [>= pos+n][R/2][2], R
    // a multiple of 32 with R/32 in {1, 2, 4, 8} and R <= D (pf_fused_rope_ok), or 0
    const float* qn;
    const float* rope;
    int R;
    float eps;
    const unsigned* kbits;  // QSA: per-token key visibility bits [n][kb_words] (nullptr: dense)
    int kb_words;
};
// Rope widths the prefill kernel's in-kernel query normalization handles: the rotate-half partner of a
// lane's dim is then in the same lane.
__host__ __device__ constexpr bool pf_fused_rope_ok(int R, int D) {
    return R == 0 || ((R == 32 || R == 64 || R == 128 || R == 256) && R <= D);
}
// Split slots per KV head of a launch with n_qt query tiles per KV head.
__host__ __device__ constexpr int pf_split_slots(int n_qt, int split_all) { return split_all ? n_qt : n_qt / 2; }
// Waves of a prefill workgroup (16 query rows each).
constexpr int kPfWaves = 8;
// Floats of one wave's prefill partial: 64 lanes x (D/4 accumulator values + max and sum).
__host__ __device__ constexpr int pf_part_floats(int D) { return 64 * (D / 4 + 2); }
// Query tiles of an n-token prefill with GQA group G (128 query rows per tile).
__host__ __device__ constexpr int pf_query_tiles(int n, int G) { return (n + 128 / G - 1) / (128 / G); }
hipError_t launch_prefill(const PrefillArgs& a, int D, int q_dtype, int in_dtype, hipStream_t s);
// out[i] = fp16(q[i] * scale), i < n (n a multiple of 4): the prefill operand from fp32 queries
hipError_t launch_q_f16(const float* q, void* out, float scale, size_t n, hipStream_t s);

hipError_t launch_rope_table(float* rope, const float* inv_freq, int n_pos, int R, hipStream_t s);

// ---- QSA indexer (qsa.hip) ----
struct QsaPoolArgs {
    const void* ik;       // [n][ID] raw indexer keys of positions pos.. (in_dtype)
    const float* gamma;   // [ID] the indexer key norm's gamma (applied as is)
    const float* rope;    // rope table [>= pos+n][R/2][2]
    float* raw;           // [cap][ID] raw keys of every cached position
    float* pooled;        // [cap / CR + 1][ID] pooled block keys
    int pos, n, ID, CR, R;
    float eps;
};
hipError_t launch_qsa_pool(const QsaPoolArgs& a, int in_dtype, hipStream_t s);

struct QsaSelectArgs {
    const void* iq;       // [n][IH][ID] raw indexer queries (in_dtype)
    const float* gamma;   // [ID] the indexer query norm's gamma (applied as is)
    const float* rope;
    const float* pooled;  // [>= (pos+n)/CR][ID]
    float* scores;        // workspace [n][stride], stride >= (pos+n)/CR and a multiple of 4
    int* cnt;             // [n] arrival counters, zero between launches
    unsigned* hist;       // [n][hcopies][2048] first-digit counts of the scores, zero between launches
    unsigned* cand;       // two-launch form: [n][kQsaSelWgMax][2][kQsaCandWg] candidates handed to the last
    int* cand_n;          //   workgroup, [n][kQsaSelWgMax] their counts
    unsigned* mask;       // [n][mask_words] block bitmask, or NULL
    unsigned* kbits;      // [n][kb_words] key visibility bits, or NULL
    const void* ik;       // with raw: the tokens' raw indexer keys [n][ID] (in_dtype), appended by the launch
    float* raw;           // [>= pos+n][ID] the raw key cache, or NULL (no append)
    int mask_words, kb_words, stride;
    int pos, n, IH, ID, CR, top, R;
    float eps;
    int hcopies;          // histogram copies a token (n * hcopies <= kQsaHistTokens)
};
hipError_t launch_qsa_select(const QsaSelectArgs& a, int in_dtype, hipStream_t s);
// First-digit histograms (2,048 bins) a select launch may use: a token takes 1 to 8 copies
constexpr int kQsaHistTokens = 1024;
// The two-launch form (more than 32,768 complete blocks): selection workgroups of kQsaSelBlocks blocks, each
// handing over at most kQsaCandWg candidates, at most kQsaSelWgMax a token (kQsaMaskLds * 32 blocks), for at
// most kQsaCandTokens tokens a launch
constexpr int kQsaSelBlocks = 4096, kQsaCandWg = 256, kQsaSelWgMax = 36, kQsaCandTokens = 32;
int qsa_select_tokens(int nmax);  // tokens a select launch may hold at nmax complete blocks
size_t qsa_select_lds(int IH, int ID);
int qsa_mask_lds_words();  // complete blocks a select launch can hold: 32 x this

struct QsaKeyBitsArgs {
    const unsigned* mask;  // [n][mask_words]
    unsigned* kbits;       // [n][kb_words]
    int mask_words, kb_words, pos, n, CR;
};
hipError_t launch_qsa_key_bits(const QsaKeyBitsArgs& a, hipStream_t s);

// Projection Y = X W^T (csrc/mat.hip)
struct MatArgs {
    const void* w;     // planar Q8: int8 [rows][cols]; f32: float [rows][cols]
    const float* s;    // planar Q8: [rows][cols / 32] scales; f32: unused
    const float* x;    // [n][x_stride]
    float* y;          // [n][y_stride]
    int rows, cols, n, x_stride, y_stride, post;
    float post_scale;  // post 1: y = silu(y * post_scale)
};
// Token counts from which launch_mat runs the tiled MFMA GEMM (columns a multiple of 32) instead of the
// matrix-vector kernel.
constexpr int kGemmMinN = 16;
hipError_t launch_mat(const MatArgs& a, bool q8, hipStream_t s);

// Up to kMatMulti matrices with the same input (x, cols, n, x_stride) in one launch; wg_end is filled by
// launch_mat_multi.
constexpr int kMatMulti = 4;
struct MatMultiArgs {
    MatArgs m[kMatMulti];
    int wg_end[kMatMulti];
    int count;
};
hipError_t launch_mat_multi(const MatMultiArgs& a, bool q8, hipStream_t s);

}  // namespace qw
