// qwattn.hpp — C++ wrapper of the qwattn C ABI (include/qwattn.h) for the reference engine's backends.
//
// The reference engine reports failures by throwing std::runtime_error (src/vk_common.h:19-23, the
// "context overflow" of src/qwen4_vk.cpp:304); the C ABI returns status codes and never throws. This
// header turns a nonzero status into a qwattn::Error (a std::runtime_error carrying the status) and owns
// a context with RAII, so a HipBackend : Backend (src/backend.h:9-41) can call the attention layer the way
// the Vulkan backend calls its dispatches (src/qwen4_vk.cpp:937-996).
#pragma once

#include <stdexcept>
#include <string>
#include <utility>

#include "qwattn.h"

namespace qwattn {

// A nonzero status of a qwattn call, with the library's message (qwattn_last_error).
class Error : public std::runtime_error {
public:
    Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
    int code() const noexcept { return code_; }

private:
    int code_;
};

// Throws qwattn::Error when rc is not QWATTN_OK; `ctx` is the context the call was made on (NULL for
// qwattn_create and qwattn_decode_noalloc, whose message is the thread's last creation error).
inline void check(const qwattn_ctx* ctx, int rc, const char* call) {
    if (rc != QWATTN_OK) {
        const char* msg = qwattn_last_error(ctx);
        throw Error(rc, std::string(call) + ": " + (msg ? msg : "") + " (status " + std::to_string(rc) + ")");
    }
}

// One context: attention shape, rope table, split partials and the K/V caches of its layer slots.
// Not copyable; one host thread drives it at a time, as the reference backends.
class Context {
public:
    Context(int device, const qwattn_config& cfg) { check(nullptr, qwattn_create(&ctx_, device, &cfg), "qwattn_create"); }
    ~Context() {
        if (ctx_) qwattn_destroy(ctx_);
    }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    Context(Context&& o) noexcept : ctx_(std::exchange(o.ctx_, nullptr)) {}
    Context& operator=(Context&& o) noexcept {
        if (this != &o) {
            if (ctx_) qwattn_destroy(ctx_);
            ctx_ = std::exchange(o.ctx_, nullptr);
        }
        return *this;
    }

    qwattn_ctx* get() const noexcept { return ctx_; }
    qwattn_config config() const {
        qwattn_config c{};
        check(ctx_, qwattn_get_config(ctx_, &c), "qwattn_get_config");
        return c;
    }
    const float* rope_table() const {
        const float* r = nullptr;
        check(ctx_, qwattn_rope_table(ctx_, &r), "qwattn_rope_table");
        return r;
    }

    // K/V caches, one slot per full-attention layer (alloc_state / ensure_kv, src/qwen4_vk.cpp:565-574,
    // 657-685)
    void kv_alloc(int n_slots, int cap) { check(ctx_, qwattn_kv_alloc(ctx_, n_slots, cap), "qwattn_kv_alloc"); }
    void kv_grow(void* stream, int tokens) { check(ctx_, qwattn_kv_grow(ctx_, stream, tokens), "qwattn_kv_grow"); }

    // The attention body of one full-attention layer between its projections, for n tokens at positions
    // pos.. pos+n-1 of layer slot `slot` (the three dispatches of Qwen4Vulkan::attention). A speculative
    // pass is the same call with n = 1 + drafts; rejecting drafts needs no call: the next pass is made at
    // the smaller pos and the rows beyond it are rewritten.
    void layer_attention(void* stream, int slot, const void* qg, const void* k, const void* v, int in_dtype,
                         const float* qn, const float* kn, float* out, int pos, int n, int n_split = 0) {
        check(ctx_, qwattn_layer_attention(ctx_, stream, slot, qg, k, v, in_dtype, qn, kn, out, pos, n, n_split),
              "qwattn_layer_attention");
    }

    // A projection, Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856): y[n][y_stride] = x[n][x_stride] W^T, W planar
    // Q8_0 (w int8 [rows][cols], s fp32 [rows][cols/32]) or fp32 (s unused); post 1: silu(y * post_scale).
    void mat(void* stream, const void* w, const float* s, bool q8, int rows, int cols, const float* x, int x_stride,
             float* y, int y_stride, int n, int post = 0, float post_scale = 0.f) {
        check(ctx_, qwattn_mat(ctx_, stream, w, s, q8 ? 1 : 0, rows, cols, x, x_stride, y, y_stride, n, post, post_scale),
              "qwattn_mat");
    }

    // count projections of one input (qwattn_mat_multi: one launch below 16 tokens).
    void mat_multi(void* stream, const qwattn_mat_out* mats, int count, bool q8, int cols, const float* x, int x_stride,
                   int n) {
        check(ctx_, qwattn_mat_multi(ctx_, stream, mats, count, q8 ? 1 : 0, cols, x, x_stride, n), "qwattn_mat_multi");
    }

    // A QSA layer past its budget (Qwen4Vulkan::attention with `masked`, src/qwen4_vk.cpp:942-984): cache
    // and pool the pass's projected indexer keys, select each token's blocks into per-key visibility bits,
    // and run the layer's attention over the visible keys. raw [max_ctx][idx_dim] and pooled
    // [max_ctx/cr + 1][idx_dim] are the layer's indexer arrays; key_bits [n][kb_words], kb_words >=
    // ceil((pos + n) / 32).
    void qsa_layer_attention(void* stream, int slot, const void* qg, const void* k, const void* v, int in_dtype,
                             const float* qn, const float* kn, const void* iq, const void* ik, int idx_dtype,
                             const float* iq_gamma, const float* ik_gamma, int idx_heads, int idx_dim, int cr,
                             int budget, float* raw, float* pooled, int cap, uint32_t* key_bits, int kb_words,
                             float* out, int pos, int n, int n_split = 0) {
        check(ctx_, qwattn_qsa_index(ctx_, stream, ik, iq, idx_dtype, ik_gamma, iq_gamma, idx_heads, idx_dim, cr, budget,
                                     raw, pooled, cap, pos, n, nullptr, 0, key_bits, kb_words),
              "qwattn_qsa_index");
        check(ctx_, qwattn_layer_attention_qsa(ctx_, stream, slot, qg, k, v, in_dtype, qn, kn, out, pos, n, n_split,
                                               key_bits, kb_words),
              "qwattn_layer_attention_qsa");
    }

    // Waits for `stream` and throws if a bounded in-kernel wait of an earlier decode launch gave up.
    void sync(void* stream) { check(ctx_, qwattn_sync_status(ctx_, stream), "qwattn_sync_status"); }

private:
    qwattn_ctx* ctx_ = nullptr;
};

}  // namespace qwattn
