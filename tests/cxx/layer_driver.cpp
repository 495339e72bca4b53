// A C++ caller of libqwattn through include/qwattn.hpp: runs a sequence of attention passes of one
// full-attention layer (prefill chunk, speculative verify, decode steps) on device 0 and writes the
// outputs, so tests/test_integration_cxx.py can check them against the CPU oracle. It allocates its
// buffers with the HIP runtime, grows the context's K/V slot between passes (ensure_kv) and turns every
// nonzero status into a qwattn::Error, the way a HipBackend would.
//
// Input (little-endian): int32 NH, NKV, D, R, npass, then npass int32 token counts, float32 theta, eps,
// qn[D], kn[D], then per pass qg[n][NH][2D], k[n][NKV][D], v[n][NKV][D] (fp32). A negative count -r is a
// speculative rollback, not a pass: the position moves back r tokens (accept(keep) after a verify pass,
// src/qwen4_vk.cpp:278-300; no call into the library, the next pass rewrites the rows). Output: per pass
// out[n][NH][D] (fp32). Exit status: 0 ok, 2 bad input, 3 a qwattn::Error (message on stderr), 4 a HIP
// runtime failure.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <vector>

#include "qwattn.hpp"

namespace {

template <typename T>
bool read(std::ifstream& f, T* p, size_t n) {
    return static_cast<bool>(f.read(reinterpret_cast<char*>(p), sizeof(T) * n));
}

struct HipError {
    const char* what;
};

void hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw HipError{what};
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s input.bin output.bin\n", argv[0]);
        return 2;
    }
    std::ifstream in(argv[1], std::ios::binary);
    int32_t hdr[5];
    if (!read(in, hdr, 5)) return 2;
    const int NH = hdr[0], NKV = hdr[1], D = hdr[2], R = hdr[3], npass = hdr[4];
    if (NH <= 0 || NKV <= 0 || D <= 0 || npass <= 0 || npass > 64) return 2;
    std::vector<int32_t> ns(npass);
    float te[2];
    std::vector<float> qn(D), kn(D);
    if (!read(in, ns.data(), npass) || !read(in, te, 2) || !read(in, qn.data(), D) || !read(in, kn.data(), D)) return 2;
    int total = 0, nmax = 0;
    for (int n : ns) {
        if (n == 0 || n > 1024 || n < -1024) return 2;
        if (n < 0) continue;
        total += n;
        nmax = std::max(nmax, n);
    }
    if (nmax == 0) return 2;
    std::vector<float> out_all;
    try {
        qwattn::Context att(0, qwattn_config{NH, NKV, D, R, te[0], te[1], /*max_ctx*/ 4096, /*max_tokens*/ 1024,
                                             /*max_splits*/ 1024});
        att.kv_alloc(1, 64);  // grown between passes
        hipStream_t s = nullptr;
        hip(hipStreamCreate(&s), "hipStreamCreate");
        float *qg = nullptr, *k = nullptr, *v = nullptr, *out = nullptr, *qn_d = nullptr, *kn_d = nullptr;
        hip(hipMalloc(&qg, sizeof(float) * nmax * NH * 2 * D), "hipMalloc");
        hip(hipMalloc(&k, sizeof(float) * nmax * NKV * D), "hipMalloc");
        hip(hipMalloc(&v, sizeof(float) * nmax * NKV * D), "hipMalloc");
        hip(hipMalloc(&out, sizeof(float) * nmax * NH * D), "hipMalloc");
        hip(hipMalloc(&qn_d, sizeof(float) * D), "hipMalloc");
        hip(hipMalloc(&kn_d, sizeof(float) * D), "hipMalloc");
        hip(hipMemcpy(qn_d, qn.data(), sizeof(float) * D, hipMemcpyHostToDevice), "hipMemcpy");
        hip(hipMemcpy(kn_d, kn.data(), sizeof(float) * D, hipMemcpyHostToDevice), "hipMemcpy");
        int pos = 0;
        for (int p = 0; p < npass; p++) {
            const int n = ns[p];
            if (n < 0) {  // rollback: reject the last -n tokens
                if (pos + n < 0) return 2;
                pos += n;
                continue;
            }
            std::vector<float> hqg((size_t)n * NH * 2 * D), hk((size_t)n * NKV * D), hv((size_t)n * NKV * D),
                hout((size_t)n * NH * D);
            if (!read(in, hqg.data(), hqg.size()) || !read(in, hk.data(), hk.size()) || !read(in, hv.data(), hv.size()))
                return 2;
            hip(hipMemcpyAsync(qg, hqg.data(), sizeof(float) * hqg.size(), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
            hip(hipMemcpyAsync(k, hk.data(), sizeof(float) * hk.size(), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
            hip(hipMemcpyAsync(v, hv.data(), sizeof(float) * hv.size(), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
            att.kv_grow(s, pos + n);  // ensure_kv
            att.layer_attention(s, 0, qg, k, v, QWATTN_F32, qn_d, kn_d, out, pos, n);
            hip(hipMemcpyAsync(hout.data(), out, sizeof(float) * hout.size(), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
            att.sync(s);
            out_all.insert(out_all.end(), hout.begin(), hout.end());
            pos += n;
        }
        // the error path: a pass past the context limit throws with the library's status
        bool threw = false;
        try {
            att.layer_attention(s, 0, qg, k, v, QWATTN_F32, qn_d, kn_d, out, 4096, 1);
        } catch (const qwattn::Error& e) {
            threw = e.code() == QWATTN_ERANGE && std::strstr(e.what(), "context overflow") != nullptr;
        }
        if (!threw) {
            std::fprintf(stderr, "a pass past max_ctx did not throw qwattn::Error(QWATTN_ERANGE)\n");
            return 5;
        }
        for (float* p : {qg, k, v, out, qn_d, kn_d}) (void)hipFree(p);
        (void)hipStreamDestroy(s);
    } catch (const qwattn::Error& e) {
        std::fprintf(stderr, "qwattn::Error %d: %s\n", e.code(), e.what());
        return 3;
    } catch (const HipError& e) {
        std::fprintf(stderr, "HIP runtime failure: %s\n", e.what);
        return 4;
    }
    std::ofstream o(argv[2], std::ios::binary);
    o.write(reinterpret_cast<const char*>(out_all.data()), sizeof(float) * out_all.size());
    std::printf("layer_driver: %d passes, %d tokens\n", npass, total);
    return o ? 0 : 4;
}
