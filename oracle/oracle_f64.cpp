// CPU ORACLE (fp64 part) — test infrastructure only, see oracle.cpp. Compiled without -ffast-math:
// these functions write and check golden fixtures, so every operation is IEEE double.
#include <cmath>
#include <cstddef>
#include <vector>

extern "C" void orc_inv_freq(float* out, int R, double theta);

extern "C" {

// fp64 brute force: softmax(q.k / sqrt(D)) v * sigmoid(gate), every quantity in double.
void orc_attention_f64(const double* q, int q_stride, const double* qg_gate, const double* kcache,
                       const double* vcache, double* out, int pos, int n, int NH, int NKV, int D) {
    const double scale = 1.0 / std::sqrt((double)D);
    const int group = NH / NKV;
    std::vector<double> sc;
    for (int t = 0; t < n; t++)
        for (int h = 0; h < NH; h++) {
            const int kvh = h / group, len = pos + t + 1;
            const double* qh = &q[((size_t)t * NH + h) * q_stride];
            sc.resize(len);
            double mx = -1e300;
            for (int j = 0; j < len; j++) {
                double s = 0;
                for (int d = 0; d < D; d++) s += qh[d] * kcache[((size_t)j * NKV + kvh) * D + d];
                sc[j] = s * scale;
                mx = std::max(mx, sc[j]);
            }
            double sum = 0;
            for (int j = 0; j < len; j++) sum += (sc[j] = std::exp(sc[j] - mx));
            double* o = &out[((size_t)t * NH + h) * D];
            for (int d = 0; d < D; d++) {
                double acc = 0;
                for (int j = 0; j < len; j++) acc += sc[j] * vcache[((size_t)j * NKV + kvh) * D + d];
                acc /= sum;
                if (qg_gate) acc *= 1.0 / (1.0 + std::exp(-qg_gate[((size_t)t * NH + h) * 2 * D + D + d]));
                o[d] = acc;
            }
        }
}

// fp64 norm + rope: y = x / sqrt(mean(x^2) + eps) * gamma (gamma folded), then rotate-half on the first
// R dims with inv_freq[i] = (float)(1/theta^(2i/R)) as the engine computes it.
void orc_qk_norm_rope_f64(const double* x, const double* gamma, double* out, int n_rows, int D, int R,
                          const int* row_pos, double theta, double eps, int fp32_angle) {
    std::vector<float> inv(R / 2);
    orc_inv_freq(inv.data(), R, theta);
    for (int r = 0; r < n_rows; r++) {
        const double* xr = &x[(size_t)r * D];
        double* o = &out[(size_t)r * D];
        double ss = 0;
        for (int d = 0; d < D; d++) ss += xr[d] * xr[d];
        const double rs = 1.0 / std::sqrt(ss / D + eps);
        for (int d = 0; d < D; d++) o[d] = xr[d] * rs * gamma[d];
        for (int i = 0; i < R / 2; i++) {
            // the engine's angle is the fp32 product (float)p * inv_freq (src/qwen4_cpu.cpp:284); with
            // fp32_angle = 0 the exact product is used instead
            const double ang = fp32_angle ? (double)((float)row_pos[r] * inv[i]) : (double)row_pos[r] * (double)inv[i];
            const double a = o[i], b = o[i + R / 2];
            o[i] = a * std::cos(ang) - b * std::sin(ang);
            o[i + R / 2] = b * std::cos(ang) + a * std::sin(ang);
        }
    }
}

}  // extern "C"
