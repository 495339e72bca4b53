// CPU ORACLE (reference build) — test infrastructure only, see oracle.cpp.
//
// Links the reference's own CPU primitives, compiled from /root/reference/src/cpu_kernels.cpp where
// they lie (ck::dot_f32 :103-119, ck::axpy :297-304, ck::rmsnorm :306-314, ck::half_to_f32 :20-34,
// ck::sigmoid cpu_kernels.h:14) and its spinning ThreadPool (src/threadpool.h), and drives them with
// the loop of Qwen4Cpu::attention (src/qwen4_cpu.cpp:306-372), which is a private member of a class
// that needs a whole GGUF model and so cannot be called on its own. The loop below restates it;
// every arithmetic operation inside it is the reference's compiled code.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

#include "cpu_kernels.h"
#include "threadpool.h"

namespace {
std::unique_ptr<ThreadPool> g_pool;
ThreadPool& pool() {
    if (!g_pool) g_pool.reset(new ThreadPool(0));
    return *g_pool;
}
}  // namespace

extern "C" {

int ref_set_threads(int n) {
    g_pool.reset(new ThreadPool(n));
    return g_pool->size();
}

float ref_dot_f32(const float* a, const float* b, int n) { return ck::dot_f32(a, b, n); }
void ref_axpy(float* out, float p, const float* v, int n) { ck::axpy(out, p, v, n); }
float ref_sigmoid(float x) { return ck::sigmoid(x); }
float ref_half_to_f32(uint16_t h) { return ck::half_to_f32(h); }

void ref_rmsnorm_one_plus(const float* x, const float* w, float* out, int n, float eps) {
    BMat m;
    m.rows = 1;
    m.cols = n;
    m.f32.assign(w, w + n);
    ck::rmsnorm(x, m, out, n, eps, true);
}

// Causal GQA attention with the sigmoid gate; one pool task per (token, head) like
// src/qwen4_cpu.cpp:346-372. Arguments as orc_attention.
void ref_attention(const float* q, int q_stride, const float* qg_gate, const float* kcache,
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
                sc[j] = ck::dot_f32(qh, &kcache[((size_t)j * NKV + kvh) * D], D) * scale;
                mx = std::max(mx, sc[j]);
            }
            float sum = 0;
            for (int j = 0; j < len; j++) {
                sc[j] = std::exp(sc[j] - mx);
                sum += sc[j];
            }
            float* o = &out[((size_t)t * NH + h) * D];
            std::fill(o, o + D, 0.f);
            for (int j = 0; j < len; j++) ck::axpy(o, sc[j] / sum, &vcache[((size_t)j * NKV + kvh) * D], D);
            if (qg_gate) {
                const float* gate = &qg_gate[((size_t)t * NH + h) * 2 * D + D];
                for (int d = 0; d < D; d++) o[d] *= ck::sigmoid(gate[d]);
            }
        }
    });
}

}  // extern "C"
