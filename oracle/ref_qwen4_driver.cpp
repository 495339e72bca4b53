// CPU ORACLE (reference build) — test infrastructure only, see oracle.cpp.
//
// Runs the reference's own qwen4exp CPU engine (class Qwen4Cpu, src/qwen4_cpu.cpp, behind
// make_qwen4_cpu_backend; weights and config from src/qwen4.cpp and src/gguf.cpp; projections from
// src/quant.cpp), compiled in place, on a GGUF model file: the end-to-end path the reference's own tiny-model
// check exercises (tests/check_gguf.py:35-48 on tests/make_tiny_gguf.py output).
//
// The full-attention layer body is observed at the one seam the engine exposes without changing a line of
// it: every projection goes through gq::run_jobs (src/quant.cpp:343), which this library is linked to
// intercept (-Wl,--wrap; oracle/Makefile). Inside Qwen4Cpu::attention (src/qwen4_cpu.cpp:291-374) the
// engine calls run_jobs for the layer's q|gate, k and v projections (one call of three jobs), for the QSA
// indexer's key and query projections (QsaIndexer::update / select, src/qwen4_qsa.h:38-91), and last for
// o_proj, whose input is the attention body's output. A registered callback receives each of those arrays
// as the engine produced them, and for the o_proj input it may overwrite the attention output before the
// engine projects it: the test that runs the GPU attention inside the reference engine uses that.
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "qwen4.h"

namespace {

// kinds passed to the callback
enum { kQG = 0, kK = 1, kV = 2, kIK = 3, kIQ = 4, kATT = 5 };
typedef void (*rq4_cb)(void* user, int layer, int kind, int pos, int n, float* data, long count);

struct Engine {
    std::unique_ptr<Gguf> g;
    Q4Config c;
    Q4Weights w;
    std::unique_ptr<Backend> be;
    rq4_cb cb = nullptr;
    void* user = nullptr;
    int pos = 0;  // position of the forward call in progress
    std::string err;
};

Engine* g_active = nullptr;  // the engine whose forward call is in progress (one at a time)

}  // namespace

// The engine's projections, intercepted (-Wl,--wrap=<this symbol>): the real gq::run_jobs runs unchanged;
// jobs on a full-attention layer's matrices are reported to the active engine's callback.
extern "C" void __real__ZN2gq8run_jobsER10ThreadPoolRKSt6vectorINS_3JobESaIS3_EE(ThreadPool& pool,
                                                                              const std::vector<gq::Job>& jobs);

extern "C" void __wrap__ZN2gq8run_jobsER10ThreadPoolRKSt6vectorINS_3JobESaIS3_EE(ThreadPool& pool,
                                                                              const std::vector<gq::Job>& jobs) {
    Engine* e = g_active;
    auto role = [&](const gq::GMat* m, int& layer) -> int {
        if (!e) return -1;
        for (size_t l = 0; l < e->w.layers.size() && (int)l < e->c.n_layers; l++) {
            const Q4Layer& L = e->w.layers[l];
            if (!L.full_attn) continue;
            layer = (int)l;
            if (m == &L.q) return kQG;
            if (m == &L.k) return kK;
            if (m == &L.v) return kV;
            if (m == &L.idx_k) return kIK;
            if (m == &L.idx_q) return kIQ;
            if (m == &L.o) return kATT;
        }
        return -1;
    };
    if (e && e->cb) {  // the attention output, before o_proj reads it (the callback may replace it)
        for (const gq::Job& j : jobs) {
            int layer = -1;
            if (role(j.m, layer) == kATT)
                e->cb(e->user, layer, kATT, e->pos, j.n, const_cast<float*>(j.x), (long)j.n * j.m->cols);
        }
    }
    __real__ZN2gq8run_jobsER10ThreadPoolRKSt6vectorINS_3JobESaIS3_EE(pool, jobs);
    if (e && e->cb) {  // the projection outputs, as the engine will use them
        for (const gq::Job& j : jobs) {
            int layer = -1;
            const int k = role(j.m, layer);
            if (k >= 0 && k != kATT) e->cb(e->user, layer, k, e->pos, j.n, j.y, (long)j.n * j.m->rows);
        }
    }
}

extern "C" {

// Loads the GGUF model and creates the reference's CPU engine (max_ctx positions, `threads` workers).
// Returns a handle, or nullptr with the reason in rq4_error(nullptr).
static std::string g_open_err;

void* rq4_open(const char* path, int max_ctx, int threads) {
    try {
        auto e = std::make_unique<Engine>();
        e->g = std::make_unique<Gguf>(path);
        e->g->check_complete();
        e->c = Q4Config::load(*e->g);
        e->w.load(*e->g, e->c);
        e->be = make_qwen4_cpu_backend(e->c, e->w, max_ctx, threads);
        return e.release();
    } catch (const std::exception& ex) {
        g_open_err = ex.what();
        return nullptr;
    }
}

const char* rq4_error(void* h) { return h ? static_cast<Engine*>(h)->err.c_str() : g_open_err.c_str(); }

void rq4_close(void* h) { delete static_cast<Engine*>(h); }

// Shape of the model: out[0..11] = hidden, n_layers, vocab, n_heads, n_kv_heads, head_dim, rope_dim,
// idx_heads, idx_dim, idx_budget; fout[0..1] = rms_eps, rope_theta.
int rq4_info(void* h, int* out, float* fout) {
    const Q4Config& c = static_cast<Engine*>(h)->c;
    const int v[10] = {c.hidden, c.n_layers, c.vocab, c.n_heads, c.n_kv_heads, c.head_dim, c.rope_dim,
                       c.idx_heads, c.idx_dim, c.idx_budget};
    std::memcpy(out, v, sizeof v);
    fout[0] = c.rms_eps;
    fout[1] = c.rope_theta;
    return 0;
}

// Layer l: out[0] = full attention, out[1] = QSA compress ratio (0 = dense).
int rq4_layer(void* h, int l, int* out) {
    const Engine* e = static_cast<Engine*>(h);
    if (l < 0 || l >= e->c.n_layers) return -1;
    out[0] = e->w.layers[l].full_attn ? 1 : 0;
    out[1] = e->w.layers[l].compress;
    return 0;
}

// The norm gammas of full-attention layer l as the engine holds them (already folded to 1 + w):
// q_norm, k_norm [head_dim]; idx_q_norm, idx_k_norm [idx_dim] (QSA layers).
int rq4_norms(void* h, int l, float* qn, float* kn, float* iqn, float* ikn) {
    const Engine* e = static_cast<Engine*>(h);
    if (l < 0 || l >= e->c.n_layers || !e->w.layers[l].full_attn) return -1;
    const Q4Layer& L = e->w.layers[l];
    std::memcpy(qn, L.q_norm.data(), L.q_norm.size() * 4);
    std::memcpy(kn, L.k_norm.data(), L.k_norm.size() * 4);
    if (L.compress > 0) {
        std::memcpy(iqn, L.idx_q_norm.data(), L.idx_q_norm.size() * 4);
        std::memcpy(ikn, L.idx_k_norm.data(), L.idx_k_norm.size() * 4);
    }
    return 0;
}

void rq4_set_callback(void* h, rq4_cb cb, void* user) {
    Engine* e = static_cast<Engine*>(h);
    e->cb = cb;
    e->user = user;
}

// Backend::forward (src/backend.h:14-15): n tokens at the current position, logits of the last one.
int rq4_forward(void* h, const int* tokens, int n, float* logits) {
    Engine* e = static_cast<Engine*>(h);
    try {
        e->pos = e->be->pos();
        g_active = e;
        e->be->forward(tokens, n, logits);
        g_active = nullptr;
        return 0;
    } catch (const std::exception& ex) {
        g_active = nullptr;
        e->err = ex.what();
        return -1;
    }
}

int rq4_pos(void* h) { return static_cast<Engine*>(h)->be->pos(); }
void rq4_reset(void* h) { static_cast<Engine*>(h)->be->reset(); }
void rq4_save_state(void* h) { static_cast<Engine*>(h)->be->save_state(); }
void rq4_restore_state(void* h) { static_cast<Engine*>(h)->be->restore_state(); }

}  // extern "C"
