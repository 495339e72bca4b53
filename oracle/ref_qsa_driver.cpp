// CPU ORACLE (reference build) — test infrastructure only, see oracle.cpp.
//
// Also drives the reference's CPU projection (gq::run_jobs over a GGUF Q8_0 matrix, src/quant.cpp:343-...),
// which the planar Q8 projection restated in oracle.cpp is pinned against.
//
// Runs the reference's own QSA indexer (class QsaIndexer, src/qwen4_qsa.h:17-115, header-only) compiled
// in place, with its projections (gq::run_jobs, src/quant.cpp) and primitives (src/cpu_kernels.cpp).
// The indexer takes the layer's block input xn[n][hidden] and projects it with idx_q / idx_k; here those
// are F32 selection matrices over xn = [iq (IH*ID) | ik (ID)], so the projections hand the indexer the
// test's raw indexer queries and keys exactly (each output is one input times 1.0 plus zeros). The
// selection is turned into the per-token bitmask the Vulkan backend uploads (src/qwen4_vk.cpp:952-960).
#include <cstdint>
#include <cstring>
#include <vector>

#include "qwen4_qsa.h"

extern "C" {

// One layer, `n_calls` indexer calls in order: call c covers tokens [pos_c, pos_c + n_c) whose inputs are
// the next n_c rows of iq_all [.][IH][ID] and ik_all [.][ID]. For each call the indexer caches the keys
// (update) and, when some token sees more than budget/CR complete blocks, selects (select); every token's
// mask row [mask_words] is written to mask_out in call order (all ones: no selection, dense).
// Returns 0, or -1 on a bad argument.
int ref_qsa_run(int IH, int ID, int CR, int budget, int R, float theta, float eps, const float* q_gamma,
                const float* k_gamma, int max_ctx, int threads, int n_calls, const int* call_pos,
                const int* call_n, const float* iq_all, const float* ik_all, uint32_t* mask_out, int mask_words) {
    if (IH <= 0 || ID <= 0 || CR < 2 || budget % CR || R > ID || n_calls < 0) return -1;
    const int H = IH * ID + ID;
    Q4Config c;
    c.hidden = H;
    c.n_layers = 1;
    c.rms_eps = eps;
    c.rope_dim = R;
    c.rope_theta = theta;
    c.idx_heads = IH;
    c.idx_dim = ID;
    c.idx_budget = budget;
    c.compress = {CR};
    std::vector<float> wq((size_t)IH * ID * H, 0.f), wk((size_t)ID * H, 0.f);
    for (int i = 0; i < IH * ID; i++) wq[(size_t)i * H + i] = 1.f;
    for (int i = 0; i < ID; i++) wk[(size_t)i * H + IH * ID + i] = 1.f;
    Q4Weights w;
    w.layers.resize(1);
    Q4Layer& L = w.layers[0];
    L.full_attn = true;
    L.compress = CR;
    L.idx_q.type = GType::F32;
    L.idx_q.data = reinterpret_cast<const uint8_t*>(wq.data());
    L.idx_q.rows = IH * ID;
    L.idx_q.cols = H;
    L.idx_q.row_bytes = (size_t)H * 4;
    L.idx_k.type = GType::F32;
    L.idx_k.data = reinterpret_cast<const uint8_t*>(wk.data());
    L.idx_k.rows = ID;
    L.idx_k.cols = H;
    L.idx_k.row_bytes = (size_t)H * 4;
    L.idx_q_norm.assign(q_gamma, q_gamma + ID);
    L.idx_k_norm.assign(k_gamma, k_gamma + ID);
    ThreadPool pool(threads);
    QsaIndexer qsa(c, w, max_ctx, pool);
    size_t row = 0;
    std::vector<float> xn;
    std::vector<std::vector<int>> blocks;
    for (int k = 0; k < n_calls; k++) {
        const int pos = call_pos[k], n = call_n[k];
        if (pos < 0 || n <= 0 || pos + n > max_ctx) return -1;
        xn.assign((size_t)n * H, 0.f);
        for (int t = 0; t < n; t++) {
            std::memcpy(&xn[(size_t)t * H], iq_all + (row + t) * IH * ID, sizeof(float) * IH * ID);
            std::memcpy(&xn[(size_t)t * H + IH * ID], ik_all + (row + t) * ID, sizeof(float) * ID);
        }
        blocks.assign(n, {});
        qsa.update(0, xn.data(), n, pos);
        if (qsa.needs_select(0, pos, n)) qsa.select(0, xn.data(), n, pos, blocks);
        for (int t = 0; t < n; t++) {
            uint32_t* m = mask_out + (row + t) * mask_words;
            std::fill(m, m + mask_words, blocks[t].empty() ? 0xFFFFFFFFu : 0u);
            for (int b : blocks[t]) {
                if ((b >> 5) >= mask_words) return -1;
                m[b >> 5] |= 1u << (b & 31);
            }
        }
        row += n;
    }
    return 0;
}

// Y[n][rows] = X[n][cols] W^T for W in GGUF Q8_0 blocks (34 bytes per 32 weights: f16 scale, 32 int8), through
// the reference's own CPU path (gq::run_jobs on a thread pool of `threads`). Returns 0, or -1 on bad shapes.
int ref_mat_q8(const uint8_t* blocks, int rows, int cols, const float* x, int n, float* y, int threads) {
    if (rows <= 0 || cols <= 0 || cols % 32 || n <= 0) return -1;
    gq::GMat m;
    m.type = GType::Q8_0;
    m.data = blocks;
    m.rows = rows;
    m.cols = cols;
    m.row_bytes = (size_t)cols / 32 * 34;
    ThreadPool pool(threads);
    gq::Job j;
    j.m = &m;
    j.x = x;
    j.y = y;
    j.n = n;
    gq::run_jobs(pool, {j});
    return 0;
}

}  // extern "C"
