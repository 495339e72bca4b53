/*
 * qwattn — MI355X (gfx950) full-attention hot path of the qwen4exp / Qwen3-Next engine, as a C ABI.
 *
 * The reference engine has no plugin ABI for attention: each backend runs it in a private
 * `attention(l, n[, pos])` method behind `class Backend` (reference: src/backend.h:9-41). The GPU
 * backend's body is three dispatches whose push-constant structs carry raw device addresses plus
 * u32 dims (src/qwen4_vk.cpp:66-69, 937-996). This header exports exactly that work, one entry point
 * per dispatch plus the state a HIP backend owns around them (KV caches, rope table, split
 * partials), so a `HipBackend : Backend` can call it from its per-layer loop in the positions of
 * src/qwen4_vk.cpp:1198/1255, src/vk_backend.cpp:806, src/qwen4_cpu.cpp:108 and
 * src/cpu_backend.cpp:121.
 *
 * Conventions
 *  - Every pointer argument named `*_dev` or documented as "device" is a device address on the
 *    context's GPU; `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *  - Every function returns QWATTN_OK (0) or a negative QWATTN_E* code and never throws; the text
 *    of the last error of a context is returned by qwattn_last_error(ctx).
 *  - No entry point allocates device memory except qwattn_create, qwattn_kv_alloc and
 *    qwattn_kv_grow. Launches are asynchronous on `stream`.
 *  - A context is driven by one host thread at a time (the reference backends are not re-entrant).
 *
 * Data layouts (row-major, innermost last)
 *  - qg   [n][NH][2*D]   projection output, per head the query (first D) then the gate (second D);
 *                        fp32 or bf16 (`in_dtype`). Reference: q_proj emits 2*NH*D rows,
 *                        src/qwen4.cpp:112, shaders/qk_norm_rope.comp:26.
 *  - k, v [n][NKV][D]    projection outputs, same dtype as qg.
 *  - qn, kn [D] fp32     QK-RMSNorm weights stored as (gamma - 1): the kernel multiplies by (1 + w),
 *                        as the reference uploads them (src/qwen4_vk.cpp:444-448, qk_norm_rope.comp:33).
 *  - rope [n_pos][R/2][2] fp32 (cos, sin) of the fp32 angle (float)p * inv_freq[i],
 *                        inv_freq[i] = (float)(1 / theta^(2i/R)) (src/qwen4_vk.cpp:494-504).
 *  - K and V caches [NKV][cap/32][32*D] fp16, cap a multiple of 32: per KV head, blocks of 32
 *                        positions, one 32*D part per block (a head's key range is one contiguous
 *                        byte range). The reference keeps [cap][NKV][D] rows
 *                        (src/qwen4_vk.cpp:565-574); here the elements inside a part are ordered so
 *                        that every matrix-core operand fragment is one contiguous kilobyte:
 *                          K (key kb = p % 32, dim d): (((d/32)*2 + (kb/4)%2)*4 + (d/8)%4)*16
 *                                                      + (kb/8)*4 + kb%4) * 8 + d%8
 *                          V (key kb, dim d):          (((d/16)*4 + kb/8)*16 + d%16) * 8 + kb%8
 *                        Blocks stay in position order within a head, so the reference's
 *                        grow-by-copy (ensure_kv) carries over head by head: each head's old region is
 *                        a byte prefix of its new one.
 *  - q    [n][NH][D] fp32 normalized + rotated query (the reference's q_out).
 *  - out  [n][NH][D] fp32 gated attention output (the reference's att_, input of o_proj).
 */
#ifndef QWATTN_H
#define QWATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWATTN_OK 0
#define QWATTN_EINVAL -1  /* bad argument (shape, pointer, range) */
#define QWATTN_EHIP -2    /* a HIP runtime call failed */
#define QWATTN_ENOMEM -3  /* device allocation failed */
#define QWATTN_ERANGE -4  /* position/context overflow ("context overflow" in the reference) */
#define QWATTN_ESTATE -5  /* call out of order (e.g. no KV cache allocated) */
#define QWATTN_ETIMEOUT -6 /* a bounded wait inside an earlier decode launch gave up: that launch's output
                              is not valid (reported once, by the next call or qwattn_sync_status) */

#define QWATTN_F32 0
#define QWATTN_BF16 1
#define QWATTN_F16 2

typedef struct qwattn_ctx qwattn_ctx;

/* Attention shape of a model (reference: Q4Config attention fields src/qwen4.h:22-25, loaded and
 * checked at src/qwen4.cpp:17-21, 37-39; Config src/model.h:15-20). */
typedef struct qwattn_config {
    int n_heads;      /* NH: query heads (16 for Qwen3-Next) */
    int n_kv_heads;   /* NKV: key/value heads (2); NH % NKV == 0 */
    int head_dim;     /* D: 64, 128 or 256 */
    int rope_dim;     /* R: rotated leading dims per head, even, <= D */
    float rope_theta; /* 1e7 */
    float rms_eps;    /* 1e-6 */
    int max_ctx;      /* context limit: rope table length (262144 by default, src/main.cpp:313) */
    int max_tokens;   /* largest n per call (the reference's NMAX = 1024 chunk, src/qwen4_vk.cpp:41) */
    int max_splits;   /* largest split-KV count (the reference caps at 64, src/qwen4_vk.cpp:976-978) */
} qwattn_config;

/* Creates a context on `device`: checks the shape, allocates the rope table for max_ctx positions,
 * the split-KV partials for max_tokens x NH x max_splits rows, the prefill's split-tile partials and
 * arrival counters for max_tokens tokens, and the query buffers; fills the rope table.
 * Replaces the backend constructor's rope upload (src/qwen4_vk.cpp:494-504) and the partials
 * buffer (src/qwen4_vk.cpp:540). */
int qwattn_create(qwattn_ctx** ctx, int device, const qwattn_config* cfg);
int qwattn_destroy(qwattn_ctx* ctx);
/* Text of the last error on ctx (or of the last failed qwattn_create when ctx is NULL). */
const char* qwattn_last_error(const qwattn_ctx* ctx);
/* Waits for `stream` and returns the status of the decode launches queued on it so far: QWATTN_OK, or
 * QWATTN_ETIMEOUT once when a bounded in-kernel wait gave up. The decode kernels' waits (the in-launch
 * combine waiting for every split's ready flag, the loader/compute hand-offs) are bounded so that every
 * kernel ends; a wait that gives up stores a code into a host-visible word of the context, which this
 * call and every later kernel entry point report (once) instead of returning silently wrong output.
 * No reference counterpart: the Vulkan backend's fence waits either complete or throw
 * (src/vk_common.h:306-350). */
int qwattn_sync_status(qwattn_ctx* ctx, void* stream);
/* Test hook of the bounded waits (no reference counterpart). spin_max: polls before the in-launch
 * combine's flag wait gives up (0 = the default, seconds of polling). epoch_skew: added to the epoch the
 * combine waits for; nonzero makes every flag look stale, so the wait gives up after spin_max polls while
 * every kernel still ends normally. Production code leaves both at 0. */
int qwattn_set_wait_limits(qwattn_ctx* ctx, int spin_max, int epoch_skew);
/* Test hook of the K/V allocation failure path (no reference counterpart). nth > 0: the nth K/V buffer
 * allocation of the next qwattn_kv_alloc or qwattn_kv_grow fails as an out-of-memory hipMalloc would (slot
 * order, K before V; counted within that call), then the hook clears itself. 0 = off. Production code never
 * calls it. */
int qwattn_set_alloc_fault(qwattn_ctx* ctx, int nth);
int qwattn_get_config(const qwattn_ctx* ctx, qwattn_config* cfg);
/* Device address of the context's rope table ([max_ctx][R/2][2] fp32). */
int qwattn_rope_table(const qwattn_ctx* ctx, const float** rope);

/* Fills a caller-owned table rope[n_pos][R/2][2] on the GPU with the same values as the context's
 * (reference: the rope loop of upload_weights, src/qwen4_vk.cpp:494-504). */
int qwattn_fill_rope(qwattn_ctx* ctx, void* stream, float* rope, int n_pos);

/* ---- KV cache owned by the context (reference: alloc_state / ensure_kv, src/qwen4_vk.cpp:565-574,
 * 657-685) ---- */
/* Allocates n_slots (one per full-attention layer) K and V caches of `cap` tokens (rounded up to a
 * multiple of 32, at most max_ctx rounded up), zero-filled. Any previous caches are freed. On failure
 * (QWATTN_ENOMEM) no cache is left allocated. Reference: alloc_state, src/qwen4_vk.cpp:565-574. */
int qwattn_kv_alloc(qwattn_ctx* ctx, int n_slots, int cap);
/* Grows every slot to hold `tokens` positions: new capacity max(2*cap, tokens), at most max_ctx,
 * copying each slot's rows; no-op when tokens <= cap. Synchronizes `stream`. Same contract as
 * ensure_kv (src/qwen4_vk.cpp:657-685): call between passes. All or nothing: on QWATTN_ENOMEM (the
 * reference's "out of VRAM growing the K/V caches") or another error every slot, its contents and the
 * capacity are as before the call. */
int qwattn_kv_grow(qwattn_ctx* ctx, void* stream, int tokens);
/* Current capacity in tokens and the device addresses of one slot's caches. */
int qwattn_kv_slot(const qwattn_ctx* ctx, int slot, void** kcache, void** vcache, int* cap);

/* ---- Kernels (one entry point per reference dispatch) ---- */

/* Fused QK-RMSNorm + partial RoPE + KV append (reference: shaders/qk_norm_rope.comp, pipeline
 * qk_norm_rope_kv16, dispatched at src/qwen4_vk.cpp:968-972 with PcQkRope). For each token t < n at
 * position p = pos + t and each head: y = x * rsqrt(mean(x^2) + eps) * (1 + w), rotate-half RoPE on
 * the first R dims from `rope` row p; query heads write q_out[t][h], key heads write K cache row p
 * and V is copied to V cache row p. `q_dtype` is QWATTN_F32 (the reference's q_out) or QWATTN_F16
 * (prefill operand: fp16, pre-multiplied by log2(e)/sqrt(D)). `q_out` may be NULL: then only the key
 * and value rows are normalized, rotated and appended (qwattn_attend_prefill_qg does the query rows
 * itself). `kv_cap` is the caches' capacity; pos + n must not exceed it. */
int qwattn_qk_norm_rope_append(qwattn_ctx* ctx, void* stream, const void* qg, const void* k,
                               const void* v, int in_dtype, const float* qn, const float* kn,
                               const float* rope, void* kcache, void* vcache, int kv_cap, void* q_out,
                               int q_dtype, int pos, int n);

/* Split-KV causal GQA attention partials (reference: shaders/attention.comp, pipeline
 * attention_kv16, dispatched at src/qwen4_vk.cpp:985-988 with PcAttn). Token t attends to keys
 * [0, pos+t+1); the nb = ceil((pos+n)/32) 32-key blocks of keys [0, pos+n) are cut into `n_split`
 * parts (0 = automatic: one workgroup per CU). A requested count is used as given, capped at max_splits
 * and at nb, so that every part holds at least one block. With up to 8 query rows per KV head
 * (n * NH/NKV <= 8: decode) part z holds the blocks z, z + n_split, z + 2 n_split, ... (the parts of a KV
 * head read neighbouring blocks at every step); with more rows (verify) part z is a contiguous chunk, the
 * first nb % n_split chunks one block longer than the others. The reference cuts ceil(len/n_split)
 * contiguous keys per chunk (src/qwen4_vk.cpp:974-978); every partition gives the same output up to fp32
 * rounding.
 * Each workgroup serves all NH/NKV query heads of all n tokens of one KV head for one chunk,
 * so every K/V row is read from HBM once. `q` is the normalized, rotated query [n][NH][D] fp32 (the
 * reference's q_out) and rows [pos, pos+n) must already be in the caches. Requires n * NH/NKV <= 32
 * (decode n=1, MTP verify n<=4 at NH/NKV=8). Partials (running max in log2 units, sum, unnormalized
 * o[D]) go to the context's scratch; returns the split count actually used in *used_splits (may be
 * NULL). */
int qwattn_attend_partial(qwattn_ctx* ctx, void* stream, const float* q, const void* kcache,
                          const void* vcache, int kv_cap, int pos, int n, int n_split,
                          int* used_splits);

/* The reference's qk_norm_rope + attention dispatches of one decode / verify pass in one launch
 * (src/qwen4_vk.cpp:968-988): from the projection outputs qg, k, v of the n new tokens it applies the
 * QK-RMSNorm (1 + w) and partial RoPE, appends the new K/V rows at positions pos.. pos+n-1 of the
 * caches, and writes the split-KV partials exactly as qwattn_attend_partial would for the normalized
 * query. Requires n <= 8 and n * NH/NKV <= 32. Follow with qwattn_combine. */
int qwattn_decode_partial(qwattn_ctx* ctx, void* stream, const void* qg, const void* k, const void* v,
                          int in_dtype, const float* qn, const float* kn, const float* rope,
                          void* kcache, void* vcache, int kv_cap, int pos, int n, int n_split,
                          int* used_splits);

/* All three of the reference's decode dispatches (src/qwen4_vk.cpp:968-992: qk_norm_rope,
 * attention, attn_combine): qwattn_decode_partial followed, inside the same kernel, by the log-sum-exp
 * combine and the sigmoid gate of qwattn_combine, writing out[n][NH][D]. One workgroup per output row,
 * one of the last chunks of its KV head (n * NH/NKV <= 8: decode) or 16-row slice (above: MTP verify) once
 * its own partials are out, merges the split partials as their records (in the context, tagged with a
 * per-launch epoch) arrive; the combine launch follows instead only when a head or slice has fewer chunks
 * than rows. Nothing needs clearing between launches, so the call
 * allocates and clears nothing and can be captured into a graph. Calls on one context must not overlap
 * (one stream, or ordered streams). The merge order is fixed, so the output does not depend on which
 * workgroup finishes first. Same limits as qwattn_decode_partial (n <= 8, n * NH/NKV <= 32: decode and
 * MTP verify). `n_split` as in qwattn_attend_partial, except that for n * NH/NKV <= 8 a requested count
 * is capped at the automatic one (one streaming workgroup per CU): its partials never leave the launch,
 * and more parts would only add workgroup prologues and partials to merge. *used_splits (may be NULL)
 * returns the count used. */
int qwattn_decode(qwattn_ctx* ctx, void* stream, const void* qg, const void* k, const void* v,
                  int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache,
                  void* vcache, int kv_cap, float* out, int pos, int n, int n_split, int* used_splits);

/* Log-sum-exp merge of the partials of the last qwattn_attend_partial / qwattn_decode_partial plus the
 * sigmoid output gate
 * (reference: shaders/attn_combine.comp, dispatched at src/qwen4_vk.cpp:990-992 with
 * PcAttnCombine): out[t][h][d] = (sum_z o_z e^{m_z-M}) / (sum_z l_z e^{m_z-M}) * sigmoid(gate),
 * gate = qg[t][h][D + d]; splits with l = 0 are skipped. */
int qwattn_combine(qwattn_ctx* ctx, void* stream, const void* qg, int in_dtype, float* out, int n,
                   int n_split);

/* Causal chunked prefill on MFMA: out = softmax(q K^T / sqrt(D)) V * sigmoid(gate) for n tokens at
 * positions pos.. pos+n-1 against keys [0, pos+t+1), in one kernel. The reference runs prefill
 * chunks through the same split-K shader (src/qwen4_vk.cpp:974-978); this is its matrix-core
 * replacement. `q` is QWATTN_F16 pre-scaled (see qwattn_qk_norm_rope_append) or QWATTN_F32 unscaled
 * (`q_dtype`; converted to the fp16 operand in the context's query buffer by one more launch).
 * Query tiles are paired short with long, the long tile's key range split between the pair's two
 * workgroups; when two workgroups per tile fit the CUs (small chunks), every tile's key range is split
 * over two workgroups instead. Split tiles are merged in the launch through the context's partials
 * and arrival counters,
 * which are back at zero when the launch ends. The merge order is fixed, so repeated calls give the
 * same bits. Calls on one context that overlap in time race on those buffers. */
int qwattn_attend_prefill(qwattn_ctx* ctx, void* stream, const void* q, int q_dtype,
                          const void* kcache, const void* vcache, int kv_cap, const void* qg,
                          int in_dtype, float* out, int pos, int n);

/* qwattn_attend_prefill on the raw projection output: the kernel applies the query half of the
 * reference's qk_norm_rope dispatch (RMSNorm with weights (1 + qn), rotate-half RoPE from `rope`, the
 * fp16 operand pre-multiplied by log2(e)/sqrt(D)) to the query half of qg as it loads each query row,
 * so no query buffer is written or read. The n tokens' key and value rows must already be in the caches
 * (qwattn_qk_norm_rope_append with q_out = NULL). Needs rope_dim in {0, 32, 64, 128, 256} and
 * rope_dim <= head_dim (QWATTN_EINVAL otherwise; qwattn_prefill then takes the two-buffer path). */
int qwattn_attend_prefill_qg(qwattn_ctx* ctx, void* stream, const void* qg, int in_dtype, const float* qn,
                             const float* rope, const void* kcache, const void* vcache, int kv_cap,
                             float* out, int pos, int n);

/* The reference's prefill dispatches of one chunk (src/qwen4_vk.cpp:968-992) in two launches:
 * qwattn_qk_norm_rope_append of the key and value rows, then qwattn_attend_prefill_qg, which normalizes
 * and rotates the query rows in the attention kernel; with a rope_dim that kernel does not take, the
 * query rows go through the context's fp16 query buffer (qwattn_qk_norm_rope_append, then
 * qwattn_attend_prefill). n <= max_tokens. */
int qwattn_prefill(qwattn_ctx* ctx, void* stream, const void* qg, const void* k, const void* v,
                   int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache,
                   void* vcache, int kv_cap, float* out, int pos, int n);

/* The whole attention body between the projections, for one full-attention layer `slot` of the
 * context's caches (reference: the dispatches of Qwen4Vulkan::attention, src/qwen4_vk.cpp:968-992;
 * Qwen4Cpu::attention src/qwen4_cpu.cpp:306-372 without the projections): qwattn_decode when
 * n <= 8 and n * NH/NKV <= 32 (decode, MTP verify); norm + rope + append, split attend and combine
 * when n > 8 and n * NH/NKV <= 32 (small GQA groups); qwattn_prefill otherwise. `n_split` as in
 * qwattn_attend_partial. Rollback after a rejected speculative draft (the reference's accept(keep),
 * src/qwen4_vk.cpp:286-300) needs no call: the next pass is made at the smaller pos, and the rows
 * beyond it are overwritten as they are appended again. */
int qwattn_layer_attention(qwattn_ctx* ctx, void* stream, int slot, const void* qg, const void* k,
                           const void* v, int in_dtype, const float* qn, const float* kn, float* out,
                           int pos, int n, int n_split);

/* qwattn_decode without a context and without allocating: no reference counterpart. It is for callers
 * that cannot allocate device memory — code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same work, kernels and results as qwattn_decode for the same shape and splits, but the
 * per-KV-head launch counters, split records and split partials live in a library-static scratch array of
 * 32 MiB per GPU (held until the process ends) instead of a context; the call allocates nothing and
 * frees nothing. `cfg` gives the shape and limits as for qwattn_create (max_splits caps the split count;
 * the rope table is the caller's, e.g. filled once by qwattn_fill_rope). A split count whose partials do
 * not fit the scratch (n * NH rows x splits x (D + 6) floats beyond about 32 MiB) is rejected with
 * QWATTN_EINVAL. `wait_status` (device int, may be NULL): a kernel whose bounded wait gives up stores a
 * nonzero code there (left untouched otherwise; the caller clears it). Errors are reported through
 * qwattn_last_error(NULL). Calls that overlap in time on one GPU share the scratch and race: issue them
 * on one stream, or ordered streams. */
int qwattn_decode_noalloc(int device, void* stream, const qwattn_config* cfg, const void* qg, const void* k,
                          const void* v, int in_dtype, const float* qn, const float* kn, const float* rope,
                          void* kcache, void* vcache, int kv_cap, float* out, int pos, int n, int n_split,
                          int* wait_status, int* used_splits);

/* ---- QSA block-sparse attention: the indexer ------------------------------------------------------------
 * A full-attention layer with a compress ratio `cr` scores blocks of cr consecutive positions with one pooled
 * key each; past its budget a token attends only to its budget/cr best complete blocks and to the incomplete
 * tail block (reference: class QsaIndexer, src/qwen4_qsa.h:17-115, run on the CPU there; here on the GPU). */

/* QsaIndexer::update (src/qwen4_qsa.h:38-54): caches the raw indexer keys ik[n][idx_dim] (in_dtype) of
 * positions pos.. pos+n-1 into raw[cap][idx_dim] fp32 and pools every block the call completes, blocks
 * [pos/cr, (pos+n)/cr), into pooled[cap/cr + 1][idx_dim] fp32: the mean of the block's raw keys, RMS-normed
 * with k_gamma as stored (not 1 + gamma) and rotated (rotate-half over the context's rope_dim) to the
 * block's first position. Positions below pos must have been cached by earlier calls; a pass redone at a
 * smaller pos (rollback) rewrites what it covers. idx_dim: a multiple of 64, <= 256, >= rope_dim; cr >= 2;
 * pos + n <= cap <= max_ctx. */
int qwattn_qsa_pool(qwattn_ctx* ctx, void* stream, const void* ik, int in_dtype, const float* k_gamma,
                    int idx_dim, int cr, float* raw, float* pooled, int cap, int pos, int n);

/* QsaIndexer::select (src/qwen4_qsa.h:58-91) with the bitmask the Vulkan backend builds from it
 * (src/qwen4_vk.cpp:952-960). Token t (position p = pos + t) sees nblk = (p + 1) / cr complete blocks. With
 * nblk <= budget / cr it selects nothing: its mask row is all ones (dense). Otherwise its idx_heads indexer
 * query heads iq[t][h][idx_dim] (in_dtype) are RMS-normed with q_gamma as stored and rotated to p, block b
 * scores sum_h max(0, q_h . pooled[b]), and the budget/cr best blocks (higher score first, the lower block id
 * on a tie) get their bit in mask[t][mask_words] (the other words zero). key_bits[t][kb_words] (either output
 * may be NULL) receives the per-key form the _qsa attention entry points take: bit j set when key j lies in
 * a selected block or at or past nblk * cr (the tail block). mask_words * 32 >= (pos+n)/cr; kb_words * 32 >=
 * pos + n; (pos+n)/cr <= 147,456 blocks; n <= max_tokens; idx_dim as for qwattn_qsa_pool, idx_heads x
 * idx_dim <= 8192. Calls on one context must not overlap. */
int qwattn_qsa_select(qwattn_ctx* ctx, void* stream, const void* iq, int in_dtype, const float* q_gamma,
                      int idx_heads, int idx_dim, int cr, int budget, const float* pooled, int pos, int n,
                      uint32_t* mask, int mask_words, uint32_t* key_bits, int kb_words);

/* qwattn_qsa_pool then qwattn_qsa_select (the reference's update then select, src/qwen4_vk.cpp:942-964) in
 * one call, with the same results and arguments as the two (ik and iq in one in_dtype). When the call
 * completes no block ((pos + n) / cr == pos / cr: every decode step but one in cr) there is nothing to pool
 * and the select launch appends the raw keys itself, so the pair costs one launch; otherwise the two
 * launches run as they would. No reference counterpart of its own: it fuses two that the reference calls
 * back to back. */
int qwattn_qsa_index(qwattn_ctx* ctx, void* stream, const void* ik, const void* iq, int in_dtype,
                     const float* k_gamma, const float* q_gamma, int idx_heads, int idx_dim, int cr, int budget,
                     float* raw, float* pooled, int cap, int pos, int n, uint32_t* mask, int mask_words,
                     uint32_t* key_bits, int kb_words);

/* The projections either side of the attention layer: Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856) on its
 * matrix-vector pipelines q4_matmul_q8 / q4_matmul_f32 (shaders/q4_matmul.comp, codecs C_Q8 / C_F32 of
 * shaders/q4_codec.glsl) and, from 16 tokens, its tiled GEMM pipelines q4_gemm_q8 / q4_gemm_f32
 * (shaders/q4_gemm.comp; here on MFMA with fp32-level accuracy: a skinny kernel for Q8 up to 64 tokens and
 * for Q8 matrices of up to 1,024 rows, a tiled GEMM otherwise). y[t][r] (row stride y_stride) = sum_c W[r][c] x[t][c] (row stride x_stride) for
 * t < n, r < rows, with W planar Q8_0 when q8 != 0 (w: int8 [rows][cols], s: float [rows][cols/32], one
 * scale per 32 consecutive weights of a row, as qwattn_q8_unpack writes them) or float [rows][cols] (s
 * unused); post 1 then applies y = silu(y * post_scale) (the shader's `post`). fp32 arithmetic. cols a
 * multiple of 32 (q8) or 16 (f32); x_stride >= cols and a multiple of 4; y_stride >= rows; w and x 16-byte
 * aligned. */
int qwattn_mat(qwattn_ctx* ctx, void* stream, const void* w, const float* s, int q8, int rows, int cols,
               const float* x, int x_stride, float* y, int y_stride, int n, int post, float post_scale);

/* One output of qwattn_mat_multi: a matrix (w, s, rows as in qwattn_mat) and where its y goes. */
typedef struct qwattn_mat_out {
    const void* w;
    const float* s;
    int rows;
    float* y;
    int y_stride;
    int post;
    float post_scale;
} qwattn_mat_out;

/* count (1..4) projections of the same input x in one call, with the results of count qwattn_mat calls.
 * No counterpart in the reference, which issues one Qwen4Vulkan::mat per matrix (the query, key and value
 * projections of a full-attention layer: src/qwen4_vk.cpp:965-967); for callers that project one input
 * several ways: below 16 tokens one matrix-vector launch streams every matrix (one launch's latency
 * instead of count), from 16 tokens each matrix runs as its own qwattn_mat call. All matrices share cols, q8, x,
 * x_stride and n; each is checked as qwattn_mat checks it. */
int qwattn_mat_multi(qwattn_ctx* ctx, void* stream, const qwattn_mat_out* mats, int count, int q8, int cols,
                     const float* x, int x_stride, int n);

/* GGUF Q8_0 rows (per 32 weights: a binary16 scale, then 32 int8) to the planar form qwattn_mat takes
 * (host memory, no GPU): the reference's upload repacking, unpack_q8_row (src/qwen4_vk.cpp:98-106). Each
 * scale is widened as ck::half_to_f32 widens it (src/cpu_kernels.cpp:20-34), bit for bit: exponent 31 is an
 * ordinary exponent there (0x7C00 gives 65536, not inf). cols a multiple of 32. Returns QWATTN_OK or
 * QWATTN_EINVAL. */
int qwattn_q8_unpack(const uint8_t* blocks, int rows, int cols, int8_t* w, float* s);

/* The per-key visibility bits from a block mask in the reference's format (mask[t][mask_words], as the
 * reference's attention_qsa_kv16 pipeline takes it: shaders/attention.comp:35-43): bit j of key_bits[t] is
 * set when block j / cr has its bit set or j >= ((pos + t + 1) / cr) * cr. */
int qwattn_qsa_key_bits(qwattn_ctx* ctx, void* stream, const uint32_t* mask, int mask_words, int cr, int pos,
                        int n, uint32_t* key_bits, int kb_words);

/* qwattn_attend_partial restricted to the keys QSA leaves visible (reference: the attention_qsa_kv16
 * pipeline, shaders/attention.comp:35-43, dispatched at src/qwen4_vk.cpp:980-984): token t attends to key j
 * only when bit j of key_bits[t][kb_words] is set (qwattn_qsa_select or qwattn_qsa_key_bits write them;
 * kb_words * 32 >= pos + n), within its causal range as always. With at most 8 query rows per KV head
 * (decode) a workgroup reads only the 32-key tiles some token sees, so the bytes streamed fall with the
 * selection; the split count is raised, if needed, until no workgroup has more than 256 tiles. Partials
 * and qwattn_combine as for qwattn_attend_partial. */
int qwattn_attend_partial_qsa(qwattn_ctx* ctx, void* stream, const float* q, const void* kcache,
                              const void* vcache, int kv_cap, int pos, int n, int n_split,
                              const uint32_t* key_bits, int kb_words, int* used_splits);

/* qwattn_decode (norm, RoPE and append of the new rows, split attention, combine and gate) with the QSA key
 * visibility of qwattn_attend_partial_qsa. The new rows are appended whether or not any token sees them. */
int qwattn_decode_qsa(qwattn_ctx* ctx, void* stream, const void* qg, const void* k, const void* v,
                      int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache,
                      void* vcache, int kv_cap, float* out, int pos, int n, int n_split,
                      const uint32_t* key_bits, int kb_words, int* used_splits);

/* The MFMA prefill (qwattn_attend_prefill / qwattn_prefill) with the QSA key visibility of
 * qwattn_attend_partial_qsa: query row t attends to key j < pos + t + 1 only when bit j of key_bits[t] is
 * set (the reference runs QSA prefill chunks through the same attention_qsa_kv16 dispatch,
 * src/qwen4_vk.cpp:980-984). The masked scores are taken out per element; every key tile is still read. */
int qwattn_attend_prefill_qsa(qwattn_ctx* ctx, void* stream, const void* q, int q_dtype,
                              const void* kcache, const void* vcache, int kv_cap, const void* qg,
                              int in_dtype, float* out, int pos, int n, const uint32_t* key_bits,
                              int kb_words);
int qwattn_prefill_qsa(qwattn_ctx* ctx, void* stream, const void* qg, const void* k, const void* v,
                       int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache,
                       void* vcache, int kv_cap, float* out, int pos, int n, const uint32_t* key_bits,
                       int kb_words);

/* qwattn_layer_attention of a QSA layer past its budget (reference: Qwen4Vulkan::attention with `masked`,
 * src/qwen4_vk.cpp:942-984): the same dispatch (decode, verify, small-group split path, prefill) with the
 * key visibility bits key_bits[n][kb_words] that qwattn_qsa_select wrote for the pass. */
int qwattn_layer_attention_qsa(qwattn_ctx* ctx, void* stream, int slot, const void* qg, const void* k,
                               const void* v, int in_dtype, const float* qn, const float* kn, float* out,
                               int pos, int n, int n_split, const uint32_t* key_bits, int kb_words);

#ifdef __cplusplus
}
#endif

#endif /* QWATTN_H */
