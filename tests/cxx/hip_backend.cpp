// The reference-side binding of libqwattn: the attention layers of a HIP backend for the qwen4exp engine,
// written against the reference's own interfaces (class Backend, src/backend.h:9-41; Q4Config and
// Q4Weights, src/qwen4.h:22-107). Compiled by tests/test_integration_cxx.py with -fsyntax-only, against
// include/qwattn.hpp alone and, where the reference sources are present, with -DQW_WITH_REFERENCE against
// the reference's headers. The full-attention layers' projections run through qwattn_mat; the rest of a
// backend — weight upload, DeltaNet, MoE, hyper-connections, sampling — is not part of libqwattn and is
// left declared, not defined.
#include <algorithm>
#include <vector>

#include "qwattn.hpp"

#ifdef QW_WITH_REFERENCE
#include "qwen4.h"

class HipBackend : public Backend {
public:
    // One qwattn context per model, one K/V slot per full-attention layer, 16,384 tokens to start and
    // grown by doubling (QW_KV_START and ensure_kv, src/qwen4_vk.cpp:52, 657-685).
    HipBackend(const Q4Config& c, const Q4Weights& w, int max_ctx, void* stream)
        : cfg_(c), w_(w), max_ctx_(max_ctx), stream_(stream),
          att_(/*device*/ 0, qwattn_config{c.n_heads, c.n_kv_heads, c.head_dim, c.rope_dim, c.rope_theta, c.rms_eps,
                                           max_ctx, /*max_tokens: the reference's NMAX chunk*/ 1024,
                                           /*max_splits*/ 1024}) {
        slot_.assign(c.n_layers, -1);
        int n_full = 0;
        for (int l = 0; l < c.n_layers; l++)
            if (c.is_full_attn[l]) slot_[l] = n_full++;
        att_.kv_alloc(std::max(1, n_full), std::min(max_ctx, 16384));
        upload_norms();
    }

    void reset() override {
        pos_ = 0;
        reset_recurrent();
    }
    void forward(const int* tokens, int n, float* logits) override {
        run(tokens, n, logits, /*all_logits*/ false);
        pos_ += n;
    }
    int pos() const override { return pos_; }
    // K/V rows below pos are never rewritten, so the attention layers need only the position
    // (src/backend.h:17-20); the recurrent state is the DeltaNet part's
    void save_state() override {
        saved_pos_ = pos_;
        save_recurrent();
    }
    void restore_state() override {
        pos_ = saved_pos_;
        restore_recurrent();
    }
    int max_ctx() const override { return max_ctx_; }
    const char* name() const override { return "hip (gfx950, attention through libqwattn)"; }

    // Speculative verify: one pass over 1 + drafts tokens; accept(keep) moves the position back, and the
    // K/V rows past it are rewritten by the next pass (Qwen4Vulkan::forward_all / accept,
    // src/qwen4_vk.cpp:278-300)
    int max_draft() const override { return w_.has_mtp ? 3 : 0; }
    void forward_all(const int* tokens, int n, float* logits) override {
        spec_pos0_ = pos_;
        run(tokens, n, logits, /*all_logits*/ true);
        pos_ += n;
    }
    void accept(int keep) override { pos_ = spec_pos0_ + keep; }

private:
    // A matrix as uploaded: planar Q8_0 (int8 weights, fp32 scale per 32) as the reference's upload repacks
    // GGUF Q8_0 (src/qwen4_vk.cpp:98-106; qwattn_q8_unpack on the host), or fp32.
    struct DevMat {
        const void* w = nullptr;
        const float* s = nullptr;
        bool q8 = false;
        int rows = 0, cols = 0;
    };
    // Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856)
    void mat(const DevMat& m, const float* x, float* y, int n, int x_stride) {
        att_.mat(stream_, m.w, m.s, m.q8, m.rows, m.cols, x, x_stride, y, m.rows, n);
    }
    // A full-attention layer l for n tokens on its normed input xn [n][hidden]: the q (query | gate), k and v
    // projections, the attention body, then o_proj into h [n][hidden] (src/qwen4_vk.cpp:965-967, 994). The
    // layer's matrices are all Q8_0 or all fp32, as the reference's upload makes them.
    void full_attention_layer(int l, int n, const float* xn, float* h) {
        const LayerMats& m = mats_[l];
        // q, k and v share xn: one qwattn_mat_multi call (one launch for decode and verify passes)
        const qwattn_mat_out qkv[3] = {{m.q.w, m.q.s, m.q.rows, qg_, m.q.rows, 0, 0.f},
                                       {m.k.w, m.k.s, m.k.rows, k_, m.k.rows, 0, 0.f},
                                       {m.v.w, m.v.s, m.v.rows, v_, m.v.rows, 0, 0.f}};
        att_.mat_multi(stream_, qkv, 3, m.q.q8, cfg_.hidden, xn, cfg_.hidden, n);
        attention(l, n, qg_, k_, v_, att_out_);
        mat(m.o, att_out_, h, n, cfg_.n_heads * cfg_.head_dim);
    }

    // The body of one full-attention layer l for n tokens at the current position, between its q/k/v
    // projections (qg [n][NH][2D] = query | gate per head, k and v [n][NKV][D], fp32 device buffers)
    // and o_proj (out [n][NH][D]), where src/qwen4_vk.cpp:1198/1255 call attention(l, n, pos_).
    void attention(int l, int n, const float* qg, const float* k, const float* v, float* out) {
        att_.kv_grow(stream_, pos_ + n);  // ensure_kv: between passes, a no-op while the slots fit
        att_.layer_attention(stream_, slot_[l], qg, k, v, QWATTN_F32, q_norm_dev_[l], k_norm_dev_[l], out, pos_, n,
                             /*n_split: one workgroup per CU*/ 0);
    }

    // the rest of the backend (not libqwattn): weights upload — the norm gammas minus one, as
    // up_norm_minus1 (src/qwen4_vk.cpp:444-448), into q_norm_dev_/k_norm_dev_, the q/k/v/o matrices into
    // mats_ and the layer buffers qg_, k_, v_, att_out_ — the layer stack calling full_attention_layer() for
    // the full-attention layers, and the recurrent state
    void upload_norms();
    void run(const int* tokens, int n, float* logits, bool all_logits);
    void reset_recurrent();
    void save_recurrent();
    void restore_recurrent();

    const Q4Config& cfg_;
    const Q4Weights& w_;
    int max_ctx_;
    void* stream_;
    qwattn::Context att_;
    std::vector<int> slot_;  // K/V slot of each layer (-1: not a full-attention layer)
    std::vector<const float*> q_norm_dev_, k_norm_dev_;
    struct LayerMats {
        DevMat q, k, v, o;
    };
    std::vector<LayerMats> mats_;
    float *qg_ = nullptr, *k_ = nullptr, *v_ = nullptr, *att_out_ = nullptr;  // [max_tokens][...] device buffers
    int pos_ = 0, saved_pos_ = 0, spec_pos0_ = 0;
};

std::unique_ptr<Backend> make_hip_backend(const Q4Config& c, const Q4Weights& w, int max_ctx, void* stream) {
    return std::make_unique<HipBackend>(c, w, max_ctx, stream);
}

#else  // without the reference headers: the same calls on a context alone

struct AttentionLayers {
    qwattn::Context att;
    int pos = 0;
    AttentionLayers(const qwattn_config& c, int n_full, int start_cap) : att(0, c) { att.kv_alloc(n_full, start_cap); }
    void layer(void* stream, int slot, const float* qg, const float* k, const float* v, const float* qn,
               const float* kn, float* out, int n) {
        att.kv_grow(stream, pos + n);
        att.layer_attention(stream, slot, qg, k, v, QWATTN_F32, qn, kn, out, pos, n);
    }
    void project(void* stream, const void* w8, const float* s, int rows, int cols, const float* x, float* y, int n) {
        att.mat(stream, w8, s, true, rows, cols, x, cols, y, rows, n);
    }
};

#endif
