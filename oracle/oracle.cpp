// CPU ORACLE — test infrastructure only. Nothing in the product links, loads or calls this file; only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker and as the
// timed CPU baseline.
//
// A restatement (not a copy) of the reference engine's CPU full-attention path, in plain C++:
//   - rms_mul            src/qwen4_cpu.cpp:19-23  (fp32 dot accumulation, folded gamma)
//   - rmsnorm(one_plus)  src/cpu_kernels.cpp:306-314 (double accumulation, (1+w))
//   - dot_f32            src/cpu_kernels.cpp:103-119 (two 16-lane accumulators over 32-wide steps)
//   - axpy               src/cpu_kernels.cpp:297-304
//   - sigmoid            src/cpu_kernels.h:14
//   - inv_freq           src/qwen4_cpu.cpp:38-39 (double, cast to float)
//   - rope               src/qwen4_cpu.cpp:281-289 (rotate-half on the first R dims, fp32 angle)
//   - attention          src/qwen4_cpu.cpp:291-374 and src/cpu_backend.cpp:218-274: norm + rope +
//                        cache write per token, then one task per (token, head): scores, max,
//                        exp/sum, axpy over V, sigmoid gate
//   - parallel_for       src/threadpool.h:25-37 (spinning pool, one contiguous chunk per thread)
//   - split partials     shaders/attention.comp:26-75 and shaders/attn_combine.comp:13-29 (the
//                        split-K online softmax and its log-sum-exp merge, on the CPU)
//   - QSA indexer        src/qwen4_qsa.h:38-54 (pooled block keys), :58-91 (block selection), the
//                        bitmask of src/qwen4_vk.cpp:952-960, and the masked attention of
//                        src/qwen4_cpu.cpp:325-344 (runs of visible keys) / shaders/attention.comp:35-43
//   - projections        Y = X W^T of Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856, shaders/q4_matmul.comp with
//                        the C_Q8 / C_F32 codecs of shaders/q4_codec.glsl): planar Q8_0 (int8 weights, one
//                        f32 scale per 32, src/qwen4_vk.cpp:98-106) or f32 rows, optional silu(y * scale)
// plus an fp64 brute-force attention used to write golden fixtures.
//
// Parity pins for every function here live in tests/test_oracle.py (closed forms, invariants,
// fp64 brute force, the reference's own primitives compiled under oracle/_ref, and an independent
// fixture from the installed Hugging Face Qwen3-Next attention).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

namespace {

// ---- primitives -------------------------------------------------------------------------------

// Two 16-lane partial sums advanced 32 elements at a time, then a tail (src/cpu_kernels.cpp:103-119).
float dot_f32(const float* a, const float* b, int n) {
    float acc0[16] = {0}, acc1[16] = {0};
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 16; j++) {
            acc0[j] += a[i + j] * b[i + j];
            acc1[j] += a[i + 16 + j] * b[i + 16 + j];
        }
    float s = 0;
    for (int j = 0; j < 16; j++) s += acc0[j] + acc1[j];
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

inline void axpy(float* out, float p, const float* v, int n) {
    for (int i = 0; i < n; i++) out[i] += p * v[i];
}

inline float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// out = x * rsqrt(mean(x^2) + eps) * gamma, gamma already folded to (1 + w) (src/qwen4_cpu.cpp:19-23).
void rms_mul(const float* x, const float* gamma, float* out, int n, float eps) {
    const float r = 1.0f / std::sqrt(dot_f32(x, x, n) / n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * r * gamma[i];
}

// Rotate-half on pairs (i, i + R/2) of the first R dims, angle (float)p * inv_freq[i]
// (src/qwen4_cpu.cpp:281-289).
void rope(float* v, int p, const float* inv_freq, int R) {
    const int half = R / 2;
    for (int i = 0; i < half; i++) {
        const float ang = (float)p * inv_freq[i], cs = std::cos(ang), sn = std::sin(ang);
        const float a = v[i], b = v[i + half];
        v[i] = a * cs - b * sn;
        v[i + half] = b * cs + a * sn;
    }
}

// ---- spinning thread pool (src/threadpool.h:25-37 semantics) ----------------------------------

class Pool {
public:
    explicit Pool(int n) : n_(std::max(1, n)) {
        for (int i = 1; i < n_; i++) workers_.emplace_back([this, i] { loop(i); });
    }
    ~Pool() {
        stop_ = true;
        gen_.fetch_add(1, std::memory_order_release);
        for (auto& t : workers_) t.join();
    }
    int size() const { return n_; }
    // fn(b, e) over [0, n) in contiguous chunks, one per thread; every worker acknowledges every
    // dispatch so that a late worker never reads the parameters of a newer one.
    void parallel_for(int64_t n, const std::function<void(int64_t, int64_t)>& fn, int64_t min_chunk = 1) {
        const int nt = (int)std::min<int64_t>(n_, (n + min_chunk - 1) / min_chunk);
        if (nt <= 1) {
            if (n > 0) fn(0, n);
            return;
        }
        fn_ = &fn;
        n_items_ = n;
        n_threads_ = nt;
        pending_.store(n_ - 1, std::memory_order_relaxed);
        gen_.fetch_add(1, std::memory_order_release);
        chunk(0);
        while (pending_.load(std::memory_order_acquire) != 0) std::this_thread::yield();
    }

private:
    void chunk(int i) {
        const int64_t b = n_items_ * i / n_threads_, e = n_items_ * (i + 1) / n_threads_;
        if (b < e) (*fn_)(b, e);
    }
    void loop(int i) {
        uint64_t seen = 0;
        for (;;) {
            uint64_t g;
            int spins = 0;
            while ((g = gen_.load(std::memory_order_acquire)) == seen) {
                if (++spins > 2000000) std::this_thread::sleep_for(std::chrono::microseconds(200));
                else if (spins > 20000) std::this_thread::yield();
            }
            seen = g;
            if (stop_) return;
            if (i < n_threads_) chunk(i);
            pending_.fetch_sub(1, std::memory_order_acq_rel);
        }
    }
    int n_;
    std::vector<std::thread> workers_;
    std::atomic<uint64_t> gen_{0};
    std::atomic<int> pending_{0};
    std::atomic<bool> stop_{false};
    const std::function<void(int64_t, int64_t)>* fn_ = nullptr;
    int64_t n_items_ = 0;
    int n_threads_ = 0;
};

Pool* g_pool = nullptr;
Pool& pool() {
    if (!g_pool) g_pool = new Pool((int)std::thread::hardware_concurrency());
    return *g_pool;
}

}  // namespace

extern "C" {

// Sets the pool size (0 = hardware_concurrency, as ThreadPool's default); returns the size.
int orc_set_threads(int n) {
    delete g_pool;
    g_pool = new Pool(n > 0 ? n : (int)std::thread::hardware_concurrency());
    return g_pool->size();
}

float orc_dot_f32(const float* a, const float* b, int n) { return dot_f32(a, b, n); }

// inv_freq[i] = (float)(1 / theta^(2i/R)) in double (src/qwen4_cpu.cpp:38-39).
void orc_inv_freq(float* out, int R, double theta) {
    for (int i = 0; i < R / 2; i++) out[i] = (float)(1.0 / std::pow(theta, (2.0 * i) / R));
}

// rope table [n_pos][R/2][2] of (cos, sin) (src/qwen4_vk.cpp:494-504).
void orc_rope_table(float* out, int n_pos, int R, double theta) {
    std::vector<float> inv(R / 2);
    orc_inv_freq(inv.data(), R, theta);
    for (int p = 0; p < n_pos; p++)
        for (int i = 0; i < R / 2; i++) {
            const float ang = (float)p * inv[i];
            out[((size_t)p * (R / 2) + i) * 2] = std::cos(ang);
            out[((size_t)p * (R / 2) + i) * 2 + 1] = std::sin(ang);
        }
}

void orc_rms_mul(const float* x, const float* gamma, float* out, int n, float eps) { rms_mul(x, gamma, out, n, eps); }

// rmsnorm with double accumulation and (1 + w) (src/cpu_kernels.cpp:306-314).
void orc_rmsnorm_one_plus(const float* x, const float* w, float* out, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float r = 1.0f / std::sqrt((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * r * (1.0f + w[i]);
}

void orc_rope(float* v, int p, int R, double theta) {
    std::vector<float> inv(R / 2);
    orc_inv_freq(inv.data(), R, theta);
    rope(v, p, inv.data(), R);
}

// Norm + rope + cache write for n tokens at positions pos.. (src/qwen4_cpu.cpp:306-322).
//   qg [n][NH][2D] (query | gate), k/v [n][NKV][D]; gammas folded (1 + w).
//   q_out [n][NH][D]; kcache/vcache [>= pos+n][NKV][D] fp32 (the reference CPU cache is fp32).
void orc_qk_norm_rope(const float* qg, const float* k, const float* v, const float* q_gamma,
                      const float* k_gamma, float* q_out, float* kcache, float* vcache, int pos, int n,
                      int NH, int NKV, int D, int R, double theta, float eps) {
    std::vector<float> inv(R / 2), tmp(D);
    orc_inv_freq(inv.data(), R, theta);
    for (int t = 0; t < n; t++) {
        const int p = pos + t;
        for (int h = 0; h < NH; h++) {
            float* qo = &q_out[((size_t)t * NH + h) * D];
            rms_mul(&qg[((size_t)t * NH + h) * 2 * D], q_gamma, qo, D, eps);
            rope(qo, p, inv.data(), R);
        }
        for (int h = 0; h < NKV; h++) {
            rms_mul(&k[((size_t)t * NKV + h) * D], k_gamma, tmp.data(), D, eps);
            rope(tmp.data(), p, inv.data(), R);
            std::memcpy(&kcache[((size_t)p * NKV + h) * D], tmp.data(), D * sizeof(float));
            std::memcpy(&vcache[((size_t)p * NKV + h) * D], &v[((size_t)t * NKV + h) * D], D * sizeof(float));
        }
    }
}

// Causal GQA attention with the sigmoid gate (src/qwen4_cpu.cpp:346-372, src/cpu_backend.cpp:248-272):
// one task per (t, h) over the pool, two-pass softmax with a stored score vector.
//   q [n][NH][D] normalized queries (stride q_stride floats between heads: D for a packed q_out, 2D
//   when q points into qg), gate: qg-style [n][NH][2D] whose second half is the gate (NULL = no gate),
//   caches fp32 [rows][NKV][D], out [n][NH][D].
void orc_attention(const float* q, int q_stride, const float* qg_gate, const float* kcache,
                   const float* vcache, float* out, int pos, int n, int NH, int NKV, int D) {
    const float scale = 1.0f / std::sqrt((float)D);
    const int group = NH / NKV;
    pool().parallel_for((int64_t)n * NH, [&](int64_t b, int64_t e) {
        std::vector<float> sc;
        for (int64_t i = b; i < e; i++) {
            const int t = (int)(i / NH), h = (int)(i % NH), kvh = h / group, len = pos + t + 1;
            const float* qh = &q[((size_t)t * NH + h) * q_stride];
            sc.resize(len);
            float mx = -1e30f;
            for (int j = 0; j < len; j++) {
                sc[j] = dot_f32(qh, &kcache[((size_t)j * NKV + kvh) * D], D) * scale;
                mx = std::max(mx, sc[j]);
            }
            float sum = 0;
            for (int j = 0; j < len; j++) {
                sc[j] = std::exp(sc[j] - mx);
                sum += sc[j];
            }
            float* o = &out[((size_t)t * NH + h) * D];
            std::fill(o, o + D, 0.f);
            for (int j = 0; j < len; j++) axpy(o, sc[j] / sum, &vcache[((size_t)j * NKV + kvh) * D], D);
            if (qg_gate) {
                const float* gate = &qg_gate[((size_t)t * NH + h) * 2 * D + D];
                for (int d = 0; d < D; d++) o[d] *= sigmoid(gate[d]);
            }
        }
    });
}

// Split-K form of the same attention (shaders/attention.comp:26-75 then attn_combine.comp:13-29):
// keys [0, pos+n) cut into chunks of `chunk`; each (t, h, z) keeps an online softmax (m, l, o[D]) over
// its keys, and the merge skips splits with l <= 0. Natural-log units, scores pre-scaled.
void orc_attention_split(const float* q, int q_stride, const float* qg_gate, const float* kcache,
                         const float* vcache, float* out, int pos, int n, int NH, int NKV, int D, int chunk) {
    const float scale = 1.0f / std::sqrt((float)D);
    const int group = NH / NKV, maxlen = pos + n, n_split = (maxlen + chunk - 1) / chunk;
    std::vector<float> M((size_t)n_split), L((size_t)n_split), O((size_t)n_split * D);
    for (int t = 0; t < n; t++)
        for (int h = 0; h < NH; h++) {
            const int kvh = h / group, len = pos + t + 1;
            const float* qh = &q[((size_t)t * NH + h) * q_stride];
            for (int z = 0; z < n_split; z++) {
                float m = -1e30f, l = 0;
                float* o = &O[(size_t)z * D];
                std::fill(o, o + D, 0.f);
                const int jb = z * chunk, je = std::min(len, jb + chunk);
                for (int j = jb; j < je; j++) {
                    const float s = dot_f32(qh, &kcache[((size_t)j * NKV + kvh) * D], D) * scale;
                    const float mn = std::max(m, s), corr = std::exp(m - mn), p = std::exp(s - mn);
                    l = l * corr + p;
                    for (int d = 0; d < D; d++) o[d] = o[d] * corr + p * vcache[((size_t)j * NKV + kvh) * D + d];
                    m = mn;
                }
                M[z] = m;
                L[z] = l;
            }
            float Mx = -1e30f;
            for (int z = 0; z < n_split; z++)
                if (L[z] > 0) Mx = std::max(Mx, M[z]);
            float Ls = 0;
            float* res = &out[((size_t)t * NH + h) * D];
            std::fill(res, res + D, 0.f);
            for (int z = 0; z < n_split; z++) {
                if (L[z] <= 0) continue;
                const float c = std::exp(M[z] - Mx);
                Ls += L[z] * c;
                axpy(res, c, &O[(size_t)z * D], D);
            }
            for (int d = 0; d < D; d++) {
                res[d] /= Ls;
                if (qg_gate) res[d] *= sigmoid(qg_gate[((size_t)t * NH + h) * 2 * D + D + d]);
            }
        }
}

// ---- QSA indexer and block-sparse attention ------------------------------------------------------

// Pooled keys of the blocks [b0, b1) of `cr` consecutive positions (src/qwen4_qsa.h:44-53): the mean of
// the blocks' raw indexer keys raw[pos][ID] accumulated one key at a time (axpy with 1/cr), RMS-normed
// with the gamma as stored (no 1 + w) and rotated to the block's first position.
void orc_qsa_pool(const float* raw, const float* gamma, float* pooled, int b0, int b1, int ID, int cr, int R,
                  double theta, float eps) {
    std::vector<float> inv(R / 2);
    for (int i = 0; i < R / 2; i++) inv[i] = (float)(1.0 / std::pow(theta, (2.0 * i) / R));
    for (int b = b0; b < b1; b++) {
        float* pk = pooled + (size_t)b * ID;
        std::fill(pk, pk + ID, 0.f);
        for (int i = 0; i < cr; i++) axpy(pk, 1.0f / cr, raw + ((size_t)b * cr + i) * ID, ID);
        rms_mul(pk, gamma, pk, ID, eps);
        rope(pk, b * cr, inv.data(), R);
    }
}

// Block selection for n tokens at positions pos.. (src/qwen4_qsa.h:58-91) written as the per-token
// bitmask the attention consumes (src/qwen4_vk.cpp:952-960). Token t (position p = pos + t) sees
// nblk = (p + 1) / cr complete blocks; with nblk <= top it selects nothing and its row is all ones
// (dense). Otherwise its IH indexer query heads iq[t][h][ID] are RMS-normed (gamma as stored) and rotated
// to p, block b scores sum_h max(0, q_h . pooled_b), and the `top` best blocks (higher score first, the
// lower block id on a tie) have their bits set. scores (NULL or [n][stride]) receives the scores of
// the tokens that select.
void orc_qsa_select(const float* iq, const float* gamma, const float* pooled, uint32_t* mask, int mask_words,
                    float* scores, int stride, int pos, int n, int IH, int ID, int cr, int top, int R,
                    double theta, float eps) {
    std::vector<float> inv(R / 2);
    for (int i = 0; i < R / 2; i++) inv[i] = (float)(1.0 / std::pow(theta, (2.0 * i) / R));
    std::vector<float> q((size_t)IH * ID), sc;
    std::vector<int> order;
    for (int t = 0; t < n; t++) {
        const int p = pos + t, nblk = (p + 1) / cr;
        uint32_t* m = mask + (size_t)t * mask_words;
        if (nblk <= top) {
            std::fill(m, m + mask_words, 0xFFFFFFFFu);
            continue;
        }
        std::fill(m, m + mask_words, 0u);
        for (int h = 0; h < IH; h++) {
            rms_mul(iq + ((size_t)t * IH + h) * ID, gamma, &q[(size_t)h * ID], ID, eps);
            rope(&q[(size_t)h * ID], p, inv.data(), R);
        }
        sc.assign(nblk, 0.f);
        for (int b = 0; b < nblk; b++) {
            float s = 0;
            for (int h = 0; h < IH; h++) s += std::max(0.f, dot_f32(&q[(size_t)h * ID], pooled + (size_t)b * ID, ID));
            sc[b] = s;
        }
        if (scores) std::copy(sc.begin(), sc.end(), scores + (size_t)t * stride);
        order.resize(nblk);
        for (int b = 0; b < nblk; b++) order[b] = b;
        std::partial_sort(order.begin(), order.begin() + top, order.end(),
                          [&](int x, int y) { return sc[x] > sc[y] || (sc[x] == sc[y] && x < y); });
        for (int i = 0; i < top; i++) m[order[i] >> 5] |= 1u << (order[i] & 31);
    }
}

// Causal GQA attention restricted to the keys the QSA mask leaves visible (src/qwen4_cpu.cpp:325-372,
// shaders/attention.comp:35-43): token t (len = pos + t + 1) attends to the keys of the complete blocks
// whose bit is set in mask[t][mask_words] and to the incomplete tail block, keys [(len / cr) * cr, len),
// in key order. Arguments otherwise as orc_attention.
void orc_attention_qsa(const float* q, int q_stride, const float* qg_gate, const float* kcache,
                       const float* vcache, float* out, int pos, int n, int NH, int NKV, int D,
                       const uint32_t* mask, int mask_words, int cr) {
    const float scale = 1.0f / std::sqrt((float)D);
    const int group = NH / NKV;
    pool().parallel_for((int64_t)n * NH, [&](int64_t b, int64_t e) {
        std::vector<float> sc;
        std::vector<int> keys;
        for (int64_t i = b; i < e; i++) {
            const int t = (int)(i / NH), h = (int)(i % NH), kvh = h / group, len = pos + t + 1;
            const int tail = len / cr * cr;
            const uint32_t* m = mask + (size_t)t * mask_words;
            keys.clear();
            for (int j = 0; j < len; j++) {
                const int blk = j / cr;
                if (j >= tail || (m[blk >> 5] >> (blk & 31)) & 1u) keys.push_back(j);
            }
            const float* qh = &q[((size_t)t * NH + h) * q_stride];
            sc.resize(keys.size());
            float mx = -1e30f;
            for (size_t k = 0; k < keys.size(); k++) {
                sc[k] = dot_f32(qh, &kcache[((size_t)keys[k] * NKV + kvh) * D], D) * scale;
                mx = std::max(mx, sc[k]);
            }
            float sum = 0;
            for (float& s : sc) {
                s = std::exp(s - mx);
                sum += s;
            }
            float* o = &out[((size_t)t * NH + h) * D];
            std::fill(o, o + D, 0.f);
            for (size_t k = 0; k < keys.size(); k++) axpy(o, sc[k] / sum, &vcache[((size_t)keys[k] * NKV + kvh) * D], D);
            if (qg_gate) {
                const float* gate = &qg_gate[((size_t)t * NH + h) * 2 * D + D];
                for (int d = 0; d < D; d++) o[d] *= sigmoid(gate[d]);
            }
        }
    });
}

// Projection Y[n][y_stride] = X[n][x_stride] W^T (Qwen4Vulkan::mat, src/qwen4_vk.cpp:848-856; per element as
// shaders/q4_matmul.comp with q4_codec.glsl's C_Q8 / C_F32): row r of W is w8[r][cols] * s[r][cols/32] (q8) or
// wf[r][cols] (f32); each output is accumulated in double over the dequantized weights and rounded to float
// once (fp32-order-independent); post 1: y = silu(y * post_scale) as the shader applies it.
void orc_mat(const int8_t* w8, const float* s, const float* wf, int q8, int rows, int cols, const float* x,
             int x_stride, float* y, int y_stride, int n, int post, float post_scale) {
    for (int t = 0; t < n; t++)
        for (int r = 0; r < rows; r++) {
            double acc = 0.0;
            for (int c = 0; c < cols; c++) {
                const float wv = q8 ? (float)w8[(size_t)r * cols + c] * s[(size_t)r * (cols / 32) + c / 32]
                                    : wf[(size_t)r * cols + c];
                acc += (double)wv * (double)x[(size_t)t * x_stride + c];
            }
            float v = (float)acc;
            if (post == 1) {
                const float u = v * post_scale;
                v = u / (1.0f + std::exp(-u));
            }
            y[(size_t)t * y_stride + r] = v;
        }
}

}  // extern "C"
