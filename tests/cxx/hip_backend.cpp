// The reference-side binding of libqwattn: a HIP backend for the qwen4exp engine whose attention layers run
// through the C ABI, written against the reference's own interfaces (class Backend, src/backend.h:9-41;
// Q4Config and Q4Weights, src/qwen4.h:22-107).
//
// With -DQW_WITH_REFERENCE (the reference's headers on the include path) this file defines HipBackend and
// make_hip_backend. tests/cxx/build.py compiles it into tests/cxx/_build/backend_driver (with
// backend_driver.cpp) where the reference sources are present; tests/test_hip_backend.py drives that program
// on the GPU through every Backend entry point (forward, forward_all / accept, save_state / restore_state,
// reset) and checks its logits against the CPU oracle. Without the reference headers the same calls compile
// against include/qwattn.hpp alone (tests/test_integration_cxx.py).
//
// What runs where:
//  - the full-attention layers on the GPU through libqwattn: the q|gate, k and v projections (and a QSA
//    layer's indexer projections) in qwattn_mat_multi, the layer body in qwattn_layer_attention, or, on a
//    QSA layer (compress > 0), qwattn_qsa_index + qwattn_layer_attention_qsa as the reference's masked
//    dispatch (src/qwen4_vk.cpp:942-984), then o_proj in qwattn_mat; the K/V caches grow by doubling
//    (ensure_kv, src/qwen4_vk.cpp:657-685);
//  - the lm_head (Q4Weights::output) on the GPU in qwattn_mat;
//  - the residual stream, the block-input norms and the final norm on the host, for an attention-only
//    stack with one residual stream (Q4Config::hc == 1): the mixer then reduces to an RMSNorm with the
//    mixer's gamma (Q4Hc::norm). DeltaNet, MoE, PLE and multi-stream hyper-connections are not part of
//    libqwattn: a model that has them is refused at construction.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "qwattn.hpp"

#ifdef QW_WITH_REFERENCE
#include "qwen4.h"

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Device memory owned by the backend (weights as uploaded, layer buffers).
class DevBuf {
public:
    DevBuf() = default;
    explicit DevBuf(size_t bytes) { hip_check(hipMalloc(&p_, std::max<size_t>(bytes, 16)), "hipMalloc"); }
    ~DevBuf() {
        if (p_) (void)hipFree(p_);
    }
    DevBuf(DevBuf&& o) noexcept : p_(std::exchange(o.p_, nullptr)) {}
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) {
            if (p_) (void)hipFree(p_);
            p_ = std::exchange(o.p_, nullptr);
        }
        return *this;
    }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    template <class T>
    T* as() const {
        return static_cast<T*>(p_);
    }

private:
    void* p_ = nullptr;
};

DevBuf upload(const void* src, size_t bytes) {
    DevBuf b(bytes);
    hip_check(hipMemcpy(b.as<void>(), src, bytes, hipMemcpyHostToDevice), "hipMemcpy to device");
    return b;
}

// y = x * rsqrt(mean(x^2) + eps) * g over n values (the engine's rms_mul, src/qwen4_cpu.cpp:19-23)
void rms_mul(const float* x, const float* g, float* y, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float r = 1.0f / std::sqrt((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * r * g[i];
}

}  // namespace

class HipBackend : public Backend {
public:
    // One qwattn context per model, one K/V slot per full-attention layer, 16,384 tokens to start and grown
    // by doubling (QW_KV_START and ensure_kv, src/qwen4_vk.cpp:52, 657-685). Passes longer than kNMax tokens
    // run in chunks of kNMax (the reference's NMAX, src/qwen4_vk.cpp:50).
    static constexpr int kNMax = 1024;

    HipBackend(const Q4Config& c, const Q4Weights& w, int max_ctx, void* stream)
        : cfg_(c), w_(w), max_ctx_(max_ctx), stream_(stream),
          att_(/*device*/ 0, qwattn_config{c.n_heads, c.n_kv_heads, c.head_dim, c.rope_dim, c.rope_theta, c.rms_eps,
                                           max_ctx, kNMax, /*max_splits*/ 1024}) {
        if (c.hc != 1 || c.n_experts != 0)
            throw std::runtime_error("HipBackend: only attention-only stacks with one residual stream run here "
                                     "(hyper-connections, DeltaNet and MoE are outside libqwattn)");
        slot_.assign(c.n_layers, -1);
        int n_full = 0;
        for (int l = 0; l < c.n_layers; l++) {
            if (!c.is_full_attn[l] || !w.layers[l].full_attn)
                throw std::runtime_error("HipBackend: layer " + std::to_string(l) + " is not a full-attention layer");
            slot_[l] = n_full++;
        }
        att_.kv_alloc(std::max(1, n_full), std::min(max_ctx, 16384));
        upload_weights();
        const int H = c.hidden, AD = c.n_heads * c.head_dim;
        xn_ = DevBuf((size_t)kNMax * H * 4);
        h_ = DevBuf((size_t)kNMax * std::max(H, c.vocab) * 4);
        qg_ = DevBuf((size_t)kNMax * 2 * AD * 4);
        k_ = DevBuf((size_t)kNMax * c.n_kv_heads * c.head_dim * 4);
        v_ = DevBuf((size_t)kNMax * c.n_kv_heads * c.head_dim * 4);
        att_out_ = DevBuf((size_t)kNMax * AD * 4);
        if (c.idx_heads > 0) {
            iq_ = DevBuf((size_t)kNMax * c.idx_heads * c.idx_dim * 4);
            ik_ = DevBuf((size_t)kNMax * c.idx_dim * 4);
            kb_words_ = (max_ctx + 31) / 32;
            key_bits_ = DevBuf((size_t)kNMax * kb_words_ * 4);
        }
    }

    void reset() override { pos_ = 0; }
    void forward(const int* tokens, int n, float* logits) override {
        run(tokens, n, logits, /*all_logits*/ false);
        pos_ += n;
    }
    int pos() const override { return pos_; }
    // K/V rows below pos are never rewritten (src/backend.h:17-20), and an attention-only stack has no
    // recurrent state: the snapshot is the position
    void save_state() override { saved_pos_ = pos_; }
    void restore_state() override { pos_ = saved_pos_; }
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
    void accept(int keep) override {
        if (keep < 1 || spec_pos0_ + keep > pos_) throw std::runtime_error("HipBackend::accept: bad keep");
        pos_ = spec_pos0_ + keep;
    }

private:
    // A matrix as uploaded: planar Q8_0 (int8 weights, fp32 scale per 32) as the reference's upload repacks
    // GGUF Q8_0 (src/qwen4_vk.cpp:98-106; qwattn_q8_unpack on the host), or fp32.
    struct DevMat {
        DevBuf w, s;
        bool q8 = false;
        int rows = 0, cols = 0;
    };
    struct LayerMats {
        DevMat q, k, v, o, idx_q, idx_k;
        DevBuf qn, kn, iqn, ikn;  // norm weights: (gamma - 1) for q/k (the kernels multiply by 1 + w), the
                                  // indexer's as they are
        DevBuf raw, pooled;       // QSA: the indexer's raw and pooled keys
    };

    static DevMat upload_mat(const gq::GMat& m) {
        DevMat d;
        d.rows = m.rows;
        d.cols = m.cols;
        if (m.type == GType::Q8_0) {
            std::vector<int8_t> w8((size_t)m.rows * m.cols);
            std::vector<float> sc((size_t)m.rows * (m.cols / 32));
            if (qwattn_q8_unpack(m.data, m.rows, m.cols, w8.data(), sc.data()) != QWATTN_OK)
                throw std::runtime_error("HipBackend: bad Q8_0 matrix");
            d.w = upload(w8.data(), w8.size());
            d.s = upload(sc.data(), sc.size() * 4);
            d.q8 = true;
        } else if (m.type == GType::F32) {
            d.w = upload(m.data, (size_t)m.rows * m.cols * 4);
        } else {
            throw std::runtime_error("HipBackend: matrix type not uploaded (F32 and Q8_0 only)");
        }
        return d;
    }

    // The upload: the norm gammas minus one, as up_norm_minus1 (src/qwen4_vk.cpp:444-448), and the matrices
    void upload_weights() {
        mats_.resize(cfg_.n_layers);
        for (int l = 0; l < cfg_.n_layers; l++) {
            const Q4Layer& L = w_.layers[l];
            LayerMats& m = mats_[l];
            m.q = upload_mat(L.q);
            m.k = upload_mat(L.k);
            m.v = upload_mat(L.v);
            m.o = upload_mat(L.o);
            if (m.q.q8 != m.k.q8 || m.q.q8 != m.v.q8)
                throw std::runtime_error("HipBackend: a layer's q, k, v matrices must share one type");
            std::vector<float> g(L.q_norm.size());
            for (size_t i = 0; i < g.size(); i++) g[i] = L.q_norm[i] - 1.0f;
            m.qn = upload(g.data(), g.size() * 4);
            for (size_t i = 0; i < g.size(); i++) g[i] = L.k_norm[i] - 1.0f;
            m.kn = upload(g.data(), g.size() * 4);
            if (L.compress > 0) {
                m.idx_q = upload_mat(L.idx_q);
                m.idx_k = upload_mat(L.idx_k);
                if (m.idx_q.q8 != m.idx_k.q8) throw std::runtime_error("HipBackend: indexer matrices of two types");
                m.iqn = upload(L.idx_q_norm.data(), L.idx_q_norm.size() * 4);
                m.ikn = upload(L.idx_k_norm.data(), L.idx_k_norm.size() * 4);
                m.raw = DevBuf((size_t)max_ctx_ * cfg_.idx_dim * 4);
                m.pooled = DevBuf((size_t)(max_ctx_ / L.compress + 1) * cfg_.idx_dim * 4);
            }
        }
        lm_head_ = upload_mat(w_.output);
    }

    // Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856)
    void mat(const DevMat& m, const float* x, float* y, int n, int x_stride) {
        att_.mat(stream_, m.w.as<void>(), m.s.as<float>(), m.q8, m.rows, m.cols, x, x_stride, y, m.rows, n);
    }

    // A full-attention layer l for n tokens at position pos on its normed input xn [n][hidden]: the q (query |
    // gate), k and v projections, the attention body, then o_proj into h [n][hidden] (src/qwen4_vk.cpp:937-996).
    void full_attention_layer(int l, int n, int pos, const float* xn, float* h) {
        const LayerMats& m = mats_[l];
        const int H = cfg_.hidden;
        // q, k and v share xn: one qwattn_mat_multi call (one launch for decode and verify passes)
        const qwattn_mat_out qkv[3] = {{m.q.w.as<void>(), m.q.s.as<float>(), m.q.rows, qg_.as<float>(), m.q.rows, 0, 0.f},
                                       {m.k.w.as<void>(), m.k.s.as<float>(), m.k.rows, k_.as<float>(), m.k.rows, 0, 0.f},
                                       {m.v.w.as<void>(), m.v.s.as<float>(), m.v.rows, v_.as<float>(), m.v.rows, 0, 0.f}};
        att_.mat_multi(stream_, qkv, 3, m.q.q8, H, xn, H, n);
        att_.kv_grow(stream_, pos + n);  // ensure_kv: between passes, a no-op while the slots fit
        const int cr = w_.layers[l].compress;
        if (cr > 0) {
            // the reference's masked path: the indexer caches and pools this pass's keys and selects each token's
            // blocks (dense for a token that sees no more than budget / cr complete blocks), then the layer's
            // attention runs over the visible keys
            const qwattn_mat_out idx[2] = {{m.idx_q.w.as<void>(), m.idx_q.s.as<float>(), m.idx_q.rows, iq_.as<float>(),
                                            m.idx_q.rows, 0, 0.f},
                                           {m.idx_k.w.as<void>(), m.idx_k.s.as<float>(), m.idx_k.rows, ik_.as<float>(),
                                            m.idx_k.rows, 0, 0.f}};
            att_.mat_multi(stream_, idx, 2, m.idx_q.q8, H, xn, H, n);
            att_.qsa_layer_attention(stream_, slot_[l], qg_.as<float>(), k_.as<float>(), v_.as<float>(), QWATTN_F32,
                                     m.qn.as<float>(), m.kn.as<float>(), iq_.as<float>(), ik_.as<float>(), QWATTN_F32,
                                     m.iqn.as<float>(), m.ikn.as<float>(), cfg_.idx_heads, cfg_.idx_dim, cr,
                                     cfg_.idx_budget, m.raw.as<float>(), m.pooled.as<float>(), max_ctx_,
                                     key_bits_.as<uint32_t>(), kb_words_, att_out_.as<float>(), pos, n);
        } else {
            att_.layer_attention(stream_, slot_[l], qg_.as<float>(), k_.as<float>(), v_.as<float>(), QWATTN_F32,
                                 m.qn.as<float>(), m.kn.as<float>(), att_out_.as<float>(), pos, n,
                                 /*n_split: one workgroup per CU*/ 0);
        }
        mat(m.o, att_out_.as<float>(), h, n, cfg_.n_heads * cfg_.head_dim);
    }

    // The token rows of the embedding as floats: F32, or Q8_0 widened as the upload widens it
    void embed_rows(const int* tokens, int n, float* x) const {
        const gq::GMat& e = w_.embed;
        const int H = cfg_.hidden;
        std::vector<int8_t> w8(H);
        std::vector<float> sc(H / 32 + 1);
        for (int t = 0; t < n; t++) {
            if (tokens[t] < 0 || tokens[t] >= cfg_.vocab) throw std::runtime_error("token id out of range");
            const uint8_t* row = e.row(tokens[t]);
            if (e.type == GType::F32) {
                std::memcpy(x + (size_t)t * H, row, (size_t)H * 4);
            } else if (e.type == GType::Q8_0) {
                if (qwattn_q8_unpack(row, 1, H, w8.data(), sc.data()) != QWATTN_OK)
                    throw std::runtime_error("HipBackend: bad Q8_0 embedding row");
                for (int i = 0; i < H; i++) x[(size_t)t * H + i] = (float)w8[i] * sc[i / 32];
            } else {
                throw std::runtime_error("HipBackend: embedding type not read (F32 and Q8_0 only)");
            }
        }
    }

    // n tokens at pos_: logits of the last token (vocab floats), or of every token (n * vocab)
    void run(const int* tokens, int n, float* logits, bool all_logits) {
        if (n <= 0 || pos_ + n > max_ctx_) throw std::runtime_error("context overflow");
        for (int t0 = 0; t0 < n; t0 += kNMax) {
            const int m = std::min(kNMax, n - t0);
            const bool last = t0 + m == n;
            chunk(tokens + t0, m, pos_ + t0, all_logits ? logits + (size_t)t0 * cfg_.vocab : (last ? logits : nullptr),
                  all_logits);
        }
    }

    void chunk(const int* tokens, int n, int pos, float* logits, bool all_logits) {
        const int H = cfg_.hidden, V = cfg_.vocab;
        std::vector<float> x((size_t)n * H), xn((size_t)n * H), h((size_t)n * H);
        embed_rows(tokens, n, x.data());
        for (int l = 0; l < cfg_.n_layers; l++) {
            const std::vector<float>& g = w_.layers[l].hc_attn.norm;
            for (int t = 0; t < n; t++) rms_mul(&x[(size_t)t * H], g.data(), &xn[(size_t)t * H], H, cfg_.rms_eps);
            hip_check(hipMemcpyAsync(xn_.as<void>(), xn.data(), xn.size() * 4, hipMemcpyHostToDevice,
                                     (hipStream_t)stream_), "hipMemcpyAsync");
            full_attention_layer(l, n, pos, xn_.as<float>(), h_.as<float>());
            hip_check(hipMemcpyAsync(h.data(), h_.as<void>(), h.size() * 4, hipMemcpyDeviceToHost, (hipStream_t)stream_),
                      "hipMemcpyAsync");
            att_.sync(stream_);  // also reports a bounded in-kernel wait that gave up
            for (size_t i = 0; i < x.size(); i++) x[i] += h[i];
        }
        if (!logits) return;
        // the final norm (the head mixer's gamma) and the lm_head, for the last token or every token
        const int t0 = all_logits ? 0 : n - 1, m = n - t0;
        const std::vector<float>& g = w_.hc_head.norm;
        for (int t = 0; t < m; t++) rms_mul(&x[(size_t)(t0 + t) * H], g.data(), &xn[(size_t)t * H], H, cfg_.rms_eps);
        hip_check(hipMemcpyAsync(xn_.as<void>(), xn.data(), (size_t)m * H * 4, hipMemcpyHostToDevice, (hipStream_t)stream_),
                  "hipMemcpyAsync");
        mat(lm_head_, xn_.as<float>(), h_.as<float>(), m, H);
        hip_check(hipMemcpyAsync(logits, h_.as<void>(), (size_t)m * V * 4, hipMemcpyDeviceToHost, (hipStream_t)stream_),
                  "hipMemcpyAsync");
        att_.sync(stream_);
    }

    const Q4Config& cfg_;
    const Q4Weights& w_;
    int max_ctx_;
    void* stream_;
    qwattn::Context att_;
    std::vector<int> slot_;  // K/V slot of each layer
    std::vector<LayerMats> mats_;
    DevMat lm_head_;
    DevBuf xn_, h_, qg_, k_, v_, att_out_, iq_, ik_, key_bits_;  // [kNMax][...] layer buffers
    int kb_words_ = 0;
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
