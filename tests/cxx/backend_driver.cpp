// Runs HipBackend (tests/cxx/hip_backend.cpp) through the reference's Backend interface (src/backend.h:9-41)
// on an attention-only model and a schedule of Backend calls, both read from a file that
// tests/test_hip_backend.py writes; every logit the calls return goes to the output file, in order.
//
// Input (little-endian):
//   "QWHB", int32 hidden, n_layers, vocab, n_heads, n_kv_heads, head_dim, rope_dim, idx_heads, idx_dim,
//   idx_budget, max_ctx, q8 (matrices as GGUF Q8_0 blocks when 1, fp32 rows when 0); float32 rms_eps, rope_theta
//   per layer: int32 compress; float32 norm[hidden], q_norm[head_dim], k_norm[head_dim] (gammas, 1 + w);
//     matrices q [NH*2D][hidden], k and v [NKV*D][hidden], o [hidden][NH*D]; when compress > 0: idx_q
//     [idx_heads*idx_dim][hidden], idx_k [idx_dim][hidden], float32 idx_q_norm[idx_dim], idx_k_norm[idx_dim]
//   float32 final_norm[hidden], embed [vocab][hidden] (fp32), output matrix [vocab][hidden]
//   int32 n_ops; per op: int32 code, int32 n, then n int32 tokens for codes 0 and 1
//     code 0 forward(n tokens), 1 forward_all(n tokens), 2 accept(n), 3 save_state, 4 restore_state, 5 reset
// Output: float32 logits of every forward (vocab) and forward_all (n * vocab) call; then int32 pos() after
// each op. Exit status 0, or 3 with the exception's text on stderr.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "qwen4.h"

std::unique_ptr<Backend> make_hip_backend(const Q4Config& c, const Q4Weights& w, int max_ctx, void* stream);

namespace {

struct Reader {
    std::vector<char> buf;
    size_t off = 0;
    explicit Reader(const char* path) {
        std::ifstream f(path, std::ios::binary);
        if (!f) throw std::runtime_error(std::string("cannot open ") + path);
        buf.assign(std::istreambuf_iterator<char>(f), {});
    }
    const char* take(size_t n) {
        if (off + n > buf.size()) throw std::runtime_error("input file too short");
        const char* p = buf.data() + off;
        off += n;
        return p;
    }
    int i32() {
        int v;
        std::memcpy(&v, take(4), 4);
        return v;
    }
    float f32() {
        float v;
        std::memcpy(&v, take(4), 4);
        return v;
    }
    std::vector<float> floats(size_t n) {
        std::vector<float> v(n);
        std::memcpy(v.data(), take(n * 4), n * 4);
        return v;
    }
};

// A matrix view into the input buffer (which outlives the backend), as the GGUF loader's views into the
// mapped file (gq::make_mat, src/quant.h:29-30)
gq::GMat mat(Reader& r, int rows, int cols, bool q8) {
    gq::GMat m;
    m.type = q8 ? GType::Q8_0 : GType::F32;
    m.rows = rows;
    m.cols = cols;
    m.row_bytes = q8 ? (size_t)cols / 32 * 34 : (size_t)cols * 4;
    m.data = reinterpret_cast<const uint8_t*>(r.take(m.nbytes()));
    return m;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s input.bin output.bin\n", argv[0]);
        return 2;
    }
    try {
        Reader r(argv[1]);
        if (std::memcmp(r.take(4), "QWHB", 4) != 0) throw std::runtime_error("not a QWHB file");
        Q4Config c;
        c.hidden = r.i32();
        c.n_layers = r.i32();
        c.vocab = r.i32();
        c.n_heads = r.i32();
        c.n_kv_heads = r.i32();
        c.head_dim = r.i32();
        c.rope_dim = r.i32();
        c.idx_heads = r.i32();
        c.idx_dim = r.i32();
        c.idx_budget = r.i32();
        const int max_ctx = r.i32();
        const bool q8 = r.i32() != 0;
        c.rms_eps = r.f32();
        c.rope_theta = r.f32();
        c.hc = 1;  // one residual stream: the block-input mixers are RMSNorms
        const int H = c.hidden, NH = c.n_heads, NKV = c.n_kv_heads, D = c.head_dim;
        Q4Weights w;
        w.layers.resize(c.n_layers);
        for (int l = 0; l < c.n_layers; l++) {
            Q4Layer& L = w.layers[l];
            L.full_attn = true;
            L.compress = r.i32();
            c.is_full_attn.push_back(true);
            c.compress.push_back(L.compress);
            L.hc_attn.norm = r.floats(H);
            L.q_norm = r.floats(D);
            L.k_norm = r.floats(D);
            L.q = mat(r, NH * 2 * D, H, q8);
            L.k = mat(r, NKV * D, H, q8);
            L.v = mat(r, NKV * D, H, q8);
            L.o = mat(r, H, NH * D, q8);
            if (L.compress > 0) {
                L.idx_q = mat(r, c.idx_heads * c.idx_dim, H, q8);
                L.idx_k = mat(r, c.idx_dim, H, q8);
                L.idx_q_norm = r.floats(c.idx_dim);
                L.idx_k_norm = r.floats(c.idx_dim);
            }
        }
        w.hc_head.norm = r.floats(H);
        w.embed = mat(r, c.vocab, H, false);
        w.output = mat(r, c.vocab, H, q8);

        std::unique_ptr<Backend> be = make_hip_backend(c, w, max_ctx, /*stream*/ nullptr);
        std::vector<float> out;
        std::vector<int> positions;
        const int n_ops = r.i32();
        for (int i = 0; i < n_ops; i++) {
            const int code = r.i32(), n = r.i32();
            std::vector<int> toks;
            if (code == 0 || code == 1) {
                toks.resize(n);
                std::memcpy(toks.data(), r.take((size_t)n * 4), (size_t)n * 4);
            }
            switch (code) {
                case 0: {
                    std::vector<float> lg(c.vocab);
                    be->forward(toks.data(), n, lg.data());
                    out.insert(out.end(), lg.begin(), lg.end());
                    break;
                }
                case 1: {
                    std::vector<float> lg((size_t)n * c.vocab);
                    be->forward_all(toks.data(), n, lg.data());
                    out.insert(out.end(), lg.begin(), lg.end());
                    break;
                }
                case 2: be->accept(n); break;
                case 3: be->save_state(); break;
                case 4: be->restore_state(); break;
                case 5: be->reset(); break;
                default: throw std::runtime_error("unknown op code");
            }
            positions.push_back(be->pos());
        }
        std::ofstream f(argv[2], std::ios::binary);
        f.write(reinterpret_cast<const char*>(out.data()), (std::streamsize)(out.size() * 4));
        f.write(reinterpret_cast<const char*>(positions.data()), (std::streamsize)(positions.size() * 4));
        std::fprintf(stderr, "backend_driver: %s, %d ops\n", be->name(), n_ops);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "backend_driver: %s\n", e.what());
        return 3;
    }
}
