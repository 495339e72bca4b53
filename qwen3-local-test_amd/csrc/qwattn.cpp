// C ABI of the MI355X attention hot path (declared in include/qwattn.h).
//
// Host-side counterpart of the reference's attention dispatch (src/qwen4_vk.cpp:937-996): it owns
// what the Vulkan backend owns around the three dispatches — rope table (:494-504), split partials
// (:540), fp16 K/V caches with grow-by-doubling (:565-574, 657-685) — checks every shape, pointer
// and range on the host before a kernel is launched (a kernel never sees an out-of-range position),
// and turns failures into status codes plus qwattn_last_error text instead of exceptions.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/qwattn.h"
#include "kernels.hpp"

struct qwattn_ctx {
    int device = 0;
    int n_cu = 0;
    qwattn_config cfg{};
    float* inv_freq = nullptr;   // [R/2]
    float* rope = nullptr;       // [max_ctx][R/2][2]
    float* part_o = nullptr;     // [split_rows][max_splits][D]
    float* part_ml = nullptr;    // [split_rows][max_splits][2]
    unsigned long long* ep = nullptr;  // qwattn_decode: per KV head launch counters (epochs, qw::kEpochStep)
    float* rec = nullptr;        // qwattn_decode: [split_rows][max_splits][4] split records (m, l, tag, 0)
    float* q32 = nullptr;        // [max_tokens][NH][D] layer-path query (fp32)
    void* q16 = nullptr;         // [max_tokens][NH][D] layer-path query (fp16, pre-scaled)
    float* pf_part = nullptr;    // prefill: partials of split query tiles (qw::PrefillArgs::part)
    int* pf_cnt = nullptr;       // prefill: their arrival counters, zero between launches
    int pf_slots_per_head = 0;   // prefill: split slots per KV head in pf_part / pf_cnt
    float* qsa_scores = nullptr; // QSA select: block scores of the tokens of one launch (kQsaScoreBytes)
    int* qsa_cnt = nullptr;      // QSA select: per-token arrival counters [max_tokens], zero between launches
    unsigned* qsa_hist = nullptr; // QSA select: first-digit histograms [qsa_hist_n][2048], zero between launches
    int qsa_hist_n = 0;           // histograms in qsa_hist: a select launch holds that many tokens x copies
    unsigned* qsa_cand = nullptr; // QSA select, two-launch form: candidates handed to the last workgroup
    int* qsa_cand_n = nullptr;    //   and their counts (qw::kQsaCandTokens tokens)
    int split_rows = 0;          // rows the split kernel handles: 32 * NKV (n * G <= 32)
    int last_splits = 0;         // split count of the last qwattn_attend_partial / qwattn_decode_partial
    int last_n = 0;
    std::vector<uint16_t*> kc, vc;
    int kv_cap = 0;
    int* wait_err_host = nullptr;  // pinned host word a kernel's bounded wait writes when it gives up
    int* wait_err_dev = nullptr;   // its device address
    int spin_max = qw::kSpinDefault;
    int epoch_skew = 0;
    int alloc_fault = 0;         // test hook: the alloc_fault-th K/V buffer allocation of the next call fails
    std::string err;
};

namespace {

thread_local std::string g_create_err;
// QSA select workspace per context: the block scores of the tokens one select launch handles (a call's
// tokens go in as many launches as the scores need: 512 tokens at 8,192 blocks)
constexpr size_t kQsaScoreBytes = (size_t)16 << 20;

int fail(qwattn_ctx* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    else g_create_err = buf;
    return code;
}

// Makes the context's device current for the duration of a call and restores the caller's.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

#define HIP_TRY(c, expr)                                                                             \
    do {                                                                                             \
        hipError_t e_ = (expr);                                                                      \
        if (e_ != hipSuccess) return fail((c), QWATTN_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)


int check_shape(qwattn_ctx* c, const qwattn_config& g) {
    if (g.n_heads <= 0 || g.n_kv_heads <= 0 || g.n_heads % g.n_kv_heads)
        return fail(c, QWATTN_EINVAL, "unsupported attention head counts (%d, %d)", g.n_heads, g.n_kv_heads);
    if (g.head_dim != 64 && g.head_dim != 128 && g.head_dim != 256)
        return fail(c, QWATTN_EINVAL, "head_dim %d not supported (64, 128, 256)", g.head_dim);
    // RoPE pairs (d, d + R/2) are exchanged between lanes that hold D/32 consecutive dims each
    const int dpl = g.head_dim / 32;
    if (g.rope_dim < 0 || g.rope_dim > g.head_dim || g.rope_dim % 2 || (g.rope_dim / 2) % dpl)
        return fail(c, QWATTN_EINVAL, "unsupported rope dimension %d (R/2 must be a multiple of %d)", g.rope_dim, dpl);
    const int G = g.n_heads / g.n_kv_heads;
    if (G > 32 || 128 % G)
        return fail(c, QWATTN_EINVAL, "GQA group %d not supported (a power of two <= 32)", G);
    if (g.n_kv_heads > 32) return fail(c, QWATTN_EINVAL, "%d KV heads: at most 32 are supported", g.n_kv_heads);
    if (g.max_ctx <= 0 || g.max_tokens <= 0 || g.max_splits <= 0 || g.max_ctx > (1 << 26))
        return fail(c, QWATTN_EINVAL, "bad limits (max_ctx %d, max_tokens %d, max_splits %d)", g.max_ctx, g.max_tokens, g.max_splits);
    if (!(g.rms_eps >= 0.f) || !(g.rope_theta > 0.f)) return fail(c, QWATTN_EINVAL, "bad eps/theta");
    return QWATTN_OK;
}

// A bounded in-kernel wait of an earlier launch gave up: report it once (QWATTN_ETIMEOUT) and clear it.
int take_wait_error(qwattn_ctx* c) {
    if (!c->wait_err_host) return QWATTN_OK;
    const int code = __atomic_exchange_n(c->wait_err_host, 0, __ATOMIC_ACQ_REL);
    if (code == 0) return QWATTN_OK;
    static const char* what[] = {"", "a split's record never arrived at the in-launch combine", "",
                                 "a loader wave's slot was never released", "a compute wave's tile was never published"};
    return fail(c, QWATTN_ETIMEOUT, "a bounded wait in an earlier decode launch gave up (%s); its output is not valid",
                code >= 1 && code <= 4 ? what[code] : "unknown wait");
}

// Position and capacity checks of a call (c may be NULL: the text then goes to qwattn_last_error(NULL)).
int check_range(qwattn_ctx* c, const qwattn_config& g, int pos, int n, int kv_cap) {
    if (n < 1) return fail(c, QWATTN_EINVAL, "n = %d", n);
    if (pos < 0) return fail(c, QWATTN_EINVAL, "pos = %d", pos);
    if (n > g.max_tokens) return fail(c, QWATTN_EINVAL, "n = %d exceeds max_tokens %d", n, g.max_tokens);
    if ((long long)pos + n > g.max_ctx) return fail(c, QWATTN_ERANGE, "context overflow (%d + %d > %d)", pos, n, g.max_ctx);
    if ((long long)pos + n > kv_cap) return fail(c, QWATTN_ERANGE, "context overflow: %d + %d rows exceed the K/V cache capacity %d", pos, n, kv_cap);
    if (kv_cap % 32) return fail(c, QWATTN_EINVAL, "K/V cache capacity %d is not a multiple of 32", kv_cap);
    // the kernels address one KV head's part of a cache with 32-bit byte offsets
    if ((long long)kv_cap * g.head_dim * 2 >= (1ll << 31))
        return fail(c, QWATTN_EINVAL, "K/V cache capacity %d: a KV head's part exceeds 2 GiB", kv_cap);
    return QWATTN_OK;
}

int check_call(qwattn_ctx* c, int pos, int n, int kv_cap) {
    if (int rc = check_range(c, c->cfg, pos, n, kv_cap)) return rc;
    return take_wait_error(c);
}

// Split of the key axis [0, maxlen) for the decode kernels into S parts of whole 32-key blocks, of the
// nb = ceil(maxlen / 32) blocks that hold keys. Up to 8 query rows per KV head (k_decode_ld) part z takes
// the blocks z, z + S, z + 2S, ...; more rows (k_decode) take contiguous chunks, chunk z the blocks
// [z*cq + min(z, cr), (z+1)*cq + min(z+1, cr)) with cq = nb / S, cr = nb % S (the first cr chunks one block
// longer). A requested count n_split > 0 is used as given (the reference's 64, src/qwen4_vk.cpp:974-978,
// or 1,024 at 256K), capped at max_splits and at nb: a part holds at least one block. n_split = 0 picks
// one workgroup per CU: CUs / (NKV x the decode kernel's 16-row slices) parts. `fill_cap` (the
// one-launch decode up to 8 rows, whose partials never leave the launch) also caps a requested count at
// that number: more parts than streaming workgroups that fit the CUs at once only add workgroup
// prologues and partials to merge, and the output is the same up to fp32 rounding.
struct Split {
    int S, cq, cr;
};

// The one-launch decode combines in the launch on the last chunks of each KV head (up to 8 query rows)
// or 16-row slice (more rows), one output row each, once their own partials are out: every CU streams
// (1,024 blocks at 32K split evenly over 128 chunks a head). This needs at least as many chunks as rows
// per head / slice; otherwise the combine kernel follows.
bool tail_launch(const qwattn_config& g, int n, int S) {
    const int rows = n * (g.n_heads / g.n_kv_heads);
    return S >= std::min(rows, 16);
}

// Dim slices per output row of that combine: the most of 4, 2, 1 that keeps the combiners at half of a
// head's (slice's) chunks or fewer (4 at decode: 32 of 128 chunks; 2 at the 4-token verify: 32 of 64);
// each combiner then loads and sums D / slices dims of every split.
int combine_slices(const qwattn_config& g, int n, int S) {
    const int rows = std::min(n * (g.n_heads / g.n_kv_heads), 16);
    for (int k : {4, 2})
        if (k > 0 && 2 * rows * k <= S && g.head_dim / k >= 16) return k;
    return 1;
}

// more than 8 rows go to the decode kernel's 16-row slices (grid.z)
Split pick_split(int n_cu, const qwattn_config& g, int maxlen, int n, int n_split, bool fill_cap = false) {
    const int nb = (maxlen + 31) / 32;
    const int rows = n * (g.n_heads / g.n_kv_heads);
    const int slices = rows <= 8 ? 1 : (rows + 15) / 16;
    const int fill = std::max(1, n_cu / (g.n_kv_heads * slices));
    int S = n_split > 0 ? (fill_cap ? std::min(n_split, fill) : n_split) : fill;
    S = std::max(1, std::min({S, g.max_splits, nb}));
    return Split{S, nb / S, nb % S};
}

Split pick_split(const qwattn_ctx* c, int maxlen, int n, int n_split, bool fill_cap = false) {
    return pick_split(c->n_cu, c->cfg, maxlen, n, n_split, fill_cap);
}

// Arguments of the decode kernels: shape and split (partials and wait settings: decode_args below).
qw::DecodeArgs decode_shape_args(const qwattn_config& g, const void* q, const void* knew, const void* vnew,
                                 const float* qn, const float* kn, const float* rope, const void* kcache,
                                 const void* vcache, int kv_cap, int pos, int n, const Split& sp) {
    qw::DecodeArgs a{};
    a.q = q, a.knew = knew, a.vnew = vnew, a.qn = qn, a.kn = kn, a.rope = rope;
    a.kc = (uint16_t*)kcache, a.vc = (uint16_t*)vcache, a.part_o = nullptr, a.part_ml = nullptr;
    a.pos = pos, a.n = n, a.NH = g.n_heads, a.NKV = g.n_kv_heads, a.R = g.rope_dim;
    a.cq = sp.cq, a.cr = sp.cr, a.n_split = sp.S;
    a.eps = g.rms_eps, a.q_scale = qw::kLog2eHost / std::sqrt((float)g.head_dim);
    a.out = nullptr, a.ep = nullptr, a.rec = nullptr, a.ncomb = 0, a.cap = kv_cap;
    a.err = nullptr, a.spin_max = qw::kSpinDefault, a.epoch_skew = 0;
    return a;
}

// ... with the context's partials and wait settings.
qw::DecodeArgs decode_args(const qwattn_ctx* c, const void* q, const void* knew, const void* vnew, const float* qn,
                           const float* kn, const float* rope, const void* kcache, const void* vcache, int kv_cap, int pos, int n,
                           const Split& sp) {
    qw::DecodeArgs a = decode_shape_args(c->cfg, q, knew, vnew, qn, kn, rope, kcache, vcache, kv_cap, pos, n, sp);
    a.part_o = c->part_o, a.part_ml = c->part_ml;
    a.err = c->wait_err_dev, a.spin_max = c->spin_max, a.epoch_skew = c->epoch_skew;
    return a;
}


}  // namespace

extern "C" {

const char* qwattn_last_error(const qwattn_ctx* ctx) { return ctx ? ctx->err.c_str() : g_create_err.c_str(); }

int qwattn_create(qwattn_ctx** out, int device, const qwattn_config* cfg) {
    if (!out || !cfg) return fail(nullptr, QWATTN_EINVAL, "null argument");
    *out = nullptr;
    int rc = check_shape(nullptr, *cfg);
    if (rc) return rc;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return fail(nullptr, QWATTN_EINVAL, "device %d not available (%d devices)", device, ndev);
    qwattn_ctx* c = new qwattn_ctx;
    c->device = device;
    c->cfg = *cfg;
    DeviceGuard dg(device);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        delete c;
        return fail(nullptr, QWATTN_EHIP, "hipGetDeviceProperties failed");
    }
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
        delete c;
        return fail(nullptr, QWATTN_EINVAL, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    }
    c->n_cu = prop.multiProcessorCount;
    const int NH = cfg->n_heads, NKV = cfg->n_kv_heads, D = cfg->head_dim, R = cfg->rope_dim;
    c->split_rows = 32 * NKV;
    // + 64 floats: the decode kernel's lanes outside the rotated dims read (and discard) the table start
    const size_t rope_n = (size_t)cfg->max_ctx * std::max(1, R / 2) * 2 + 64;
    const size_t part = (size_t)c->split_rows * cfg->max_splits;
    if (part * D * sizeof(float) >= ((size_t)1 << 31)) {  // the kernels address the partials with 32-bit offsets
        delete c;
        return fail(nullptr, QWATTN_EINVAL, "max_splits %d: the split partials would exceed 2 GiB", cfg->max_splits);
    }
    const size_t qn = (size_t)cfg->max_tokens * NH * D;
    // prefill split slots per KV head: a pair of query tiles each (paired schedule) or a tile each (split
    // schedule, only while two workgroups per tile fit the CUs), at least one so the pointers are never
    // null; kPfWaves waves each, a partial region per half of the split tile
    const int qt_max = qw::pf_query_tiles(cfg->max_tokens, NH / NKV);
    c->pf_slots_per_head = std::max(1, std::max(qt_max / 2, std::min(qt_max, c->n_cu / (2 * NKV))));
    const size_t pf_slots = (size_t)NKV * c->pf_slots_per_head * qw::kPfWaves;
    c->qsa_hist_n = std::min(cfg->max_tokens, qw::kQsaHistTokens);
    const size_t hist_tokens = (size_t)c->qsa_hist_n;
    bool ok = hipMalloc(&c->pf_part, sizeof(float) * 2 * pf_slots * qw::pf_part_floats(D)) == hipSuccess &&
              hipMalloc(&c->pf_cnt, sizeof(int) * pf_slots) == hipSuccess &&
              hipMalloc(&c->inv_freq, sizeof(float) * std::max(1, R / 2)) == hipSuccess &&
              hipMalloc(&c->rope, sizeof(float) * rope_n) == hipSuccess &&
              hipMalloc(&c->part_o, sizeof(float) * part * D) == hipSuccess &&
              hipMalloc(&c->part_ml, sizeof(float) * part * 2) == hipSuccess &&
              hipMalloc(&c->ep, sizeof(unsigned long long) * NKV) == hipSuccess &&
              hipMalloc(&c->rec, sizeof(float) * 4 * part) == hipSuccess &&
              hipMalloc(&c->q32, sizeof(float) * qn) == hipSuccess && hipMalloc(&c->q16, 2 * qn) == hipSuccess &&
              hipMalloc(&c->qsa_scores, kQsaScoreBytes) == hipSuccess &&
              hipMalloc(&c->qsa_cnt, sizeof(int) * cfg->max_tokens) == hipSuccess &&
              hipMalloc(&c->qsa_hist, sizeof(unsigned) * 2048 * hist_tokens) == hipSuccess &&
              hipMalloc(&c->qsa_cand, sizeof(unsigned) * qw::kQsaCandTokens * qw::kQsaSelWgMax * 2 * qw::kQsaCandWg) ==
                  hipSuccess &&
              hipMalloc(&c->qsa_cand_n, sizeof(int) * qw::kQsaCandTokens * qw::kQsaSelWgMax) == hipSuccess &&
              hipHostMalloc(&c->wait_err_host, 64, hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess &&
              hipHostGetDevicePointer((void**)&c->wait_err_dev, c->wait_err_host, 0) == hipSuccess;
    if (!ok) {
        qwattn_destroy(c);
        return fail(nullptr, QWATTN_ENOMEM, "out of device memory creating the context");
    }
    // inv_freq[i] = (float)(1 / theta^(2i/R)) in double, as src/qwen4_vk.cpp:499 / src/qwen4_cpu.cpp:38-39
    std::vector<float> inv(std::max(1, R / 2), 0.f);
    for (int i = 0; i < R / 2; i++) inv[i] = (float)(1.0 / std::pow((double)cfg->rope_theta, (2.0 * i) / R));
    if (hipMemcpy(c->inv_freq, inv.data(), sizeof(float) * inv.size(), hipMemcpyHostToDevice) != hipSuccess ||
        (R > 0 && qw::launch_rope_table(c->rope, c->inv_freq, cfg->max_ctx, R, nullptr) != hipSuccess) ||
        hipMemset(c->part_ml, 0, sizeof(float) * part * 2) != hipSuccess ||
        hipMemset(c->pf_cnt, 0, sizeof(int) * pf_slots) != hipSuccess ||
        hipMemset(c->qsa_cnt, 0, sizeof(int) * cfg->max_tokens) != hipSuccess ||
        hipMemset(c->qsa_hist, 0, sizeof(unsigned) * 2048 * hist_tokens) != hipSuccess ||
        hipMemset(c->ep, 0, sizeof(unsigned long long) * NKV) != hipSuccess ||
        hipMemset(c->rec, 0, sizeof(float) * 4 * part) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        qwattn_destroy(c);
        return fail(nullptr, QWATTN_EHIP, "initializing the rope table failed");
    }
    *c->wait_err_host = 0;
    *out = c;
    return QWATTN_OK;
}

int qwattn_destroy(qwattn_ctx* c) {
    if (!c) return QWATTN_OK;
    DeviceGuard dg(c->device);
    (void)hipDeviceSynchronize();
    for (void* p : {(void*)c->inv_freq, (void*)c->rope, (void*)c->part_o, (void*)c->part_ml, (void*)c->ep, (void*)c->rec,
                    (void*)c->q32, c->q16, (void*)c->pf_part, (void*)c->pf_cnt, (void*)c->qsa_scores, (void*)c->qsa_cnt,
                    (void*)c->qsa_hist, (void*)c->qsa_cand, (void*)c->qsa_cand_n})
        if (p) (void)hipFree(p);
    for (auto* p : c->kc) (void)hipFree(p);
    for (auto* p : c->vc) (void)hipFree(p);
    if (c->wait_err_host) (void)hipHostFree(c->wait_err_host);
    delete c;
    return QWATTN_OK;
}

int qwattn_sync_status(qwattn_ctx* c, void* stream) {
    if (!c) return QWATTN_EINVAL;
    DeviceGuard dg(c->device);
    HIP_TRY(c, hipStreamSynchronize((hipStream_t)stream));
    return take_wait_error(c);
}

int qwattn_set_wait_limits(qwattn_ctx* c, int spin_max, int epoch_skew) {
    if (!c) return QWATTN_EINVAL;
    if (spin_max < 0) return fail(c, QWATTN_EINVAL, "qwattn_set_wait_limits: spin_max %d", spin_max);
    c->spin_max = spin_max ? spin_max : qw::kSpinDefault;
    c->epoch_skew = epoch_skew;
    return QWATTN_OK;
}

int qwattn_get_config(const qwattn_ctx* c, qwattn_config* cfg) {
    if (!c || !cfg) return QWATTN_EINVAL;
    *cfg = c->cfg;
    return QWATTN_OK;
}

int qwattn_rope_table(const qwattn_ctx* c, const float** rope) {
    if (!c || !rope) return QWATTN_EINVAL;
    *rope = c->rope;
    return QWATTN_OK;
}

int qwattn_fill_rope(qwattn_ctx* c, void* stream, float* rope, int n_pos) {
    if (!c) return QWATTN_EINVAL;
    if (!rope || n_pos <= 0) return fail(c, QWATTN_EINVAL, "qwattn_fill_rope: bad table");
    if (c->cfg.rope_dim == 0) return QWATTN_OK;
    DeviceGuard dg(c->device);
    HIP_TRY(c, qw::launch_rope_table(rope, c->inv_freq, n_pos, c->cfg.rope_dim, (hipStream_t)stream));
    return QWATTN_OK;
}

// ---- KV cache ---------------------------------------------------------------------------------------

// One K/V cache buffer; fails as hipMalloc does when the test hook qwattn_set_alloc_fault names this
// allocation (counted from 1 within the calling qwattn_kv_alloc / qwattn_kv_grow).
static hipError_t kv_malloc(qwattn_ctx* c, uint16_t** p, size_t bytes, int& nth) {
    *p = nullptr;
    if (c->alloc_fault && ++nth == c->alloc_fault) {
        c->alloc_fault = 0;
        return hipErrorOutOfMemory;
    }
    return hipMalloc((void**)p, bytes);
}

static void free_all(std::vector<uint16_t*>& v) {
    for (auto*& p : v) {
        if (p) (void)hipFree(p);
        p = nullptr;
    }
}

int qwattn_kv_alloc(qwattn_ctx* c, int n_slots, int cap) {
    if (!c) return QWATTN_EINVAL;
    if (n_slots <= 0 || cap <= 0) return fail(c, QWATTN_EINVAL, "qwattn_kv_alloc: %d slots of %d tokens", n_slots, cap);
    cap = std::min((cap + 31) / 32 * 32, (c->cfg.max_ctx + 31) / 32 * 32);
    DeviceGuard dg(c->device);
    free_all(c->kc);
    free_all(c->vc);
    c->kc.assign(n_slots, nullptr);
    c->vc.assign(n_slots, nullptr);
    c->kv_cap = 0;
    const size_t bytes = (size_t)cap * c->cfg.n_kv_heads * c->cfg.head_dim * 2;
    int nth = 0;
    hipError_t e = hipSuccess;
    for (int s = 0; s < n_slots && e == hipSuccess; s++) {
        e = kv_malloc(c, &c->kc[s], bytes, nth);
        if (e == hipSuccess) e = kv_malloc(c, &c->vc[s], bytes, nth);
        if (e == hipSuccess) e = hipMemset(c->kc[s], 0, bytes);
        if (e == hipSuccess) e = hipMemset(c->vc[s], 0, bytes);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {  // nothing half-allocated stays behind: no cache at all, as before the first call
        free_all(c->kc);
        free_all(c->vc);
        c->kc.clear();
        c->vc.clear();
        return e == hipErrorOutOfMemory ? fail(c, QWATTN_ENOMEM, "out of device memory allocating the K/V caches")
                                        : fail(c, QWATTN_EHIP, "qwattn_kv_alloc: %s", hipGetErrorString(e));
    }
    c->kv_cap = cap;
    return QWATTN_OK;
}

// All or nothing, as src/qwen4_vk.cpp:657-685 throws before touching the old caches: every slot's new
// buffers are allocated and filled first; any failure frees them and leaves every slot and kv_cap as they
// were. Only then are the old buffers freed and the new ones swapped in.
int qwattn_kv_grow(qwattn_ctx* c, void* stream, int tokens) {
    if (!c) return QWATTN_EINVAL;
    if (c->kc.empty()) return fail(c, QWATTN_ESTATE, "qwattn_kv_grow: no K/V cache allocated");
    if (tokens <= c->kv_cap) return QWATTN_OK;
    if (tokens > c->cfg.max_ctx) return fail(c, QWATTN_ERANGE, "context overflow growing the K/V caches to %d", tokens);
    long long cap = std::max<long long>(2ll * c->kv_cap, tokens);
    cap = std::min<long long>(cap, (c->cfg.max_ctx + 31) / 32 * 32);
    cap = (cap + 31) / 32 * 32;
    DeviceGuard dg(c->device);
    hipStream_t s = (hipStream_t)stream;
    const int nkv = c->cfg.n_kv_heads;
    const size_t per = (size_t)c->cfg.head_dim * 2;  // bytes per position and KV head
    const size_t old_head = (size_t)c->kv_cap * per, new_head = (size_t)cap * per, bytes = nkv * new_head;
    const size_t slots = c->kc.size();
    std::vector<uint16_t*> nk(slots, nullptr), nv(slots, nullptr);
    int nth = 0;
    hipError_t e = hipSuccess;
    for (size_t i = 0; i < slots && e == hipSuccess; i++) {
        e = kv_malloc(c, &nk[i], bytes, nth);
        if (e == hipSuccess) e = kv_malloc(c, &nv[i], bytes, nth);
    }
    // the blocked layout keeps each KV head's 32-position blocks in order, so a head's old region is a
    // prefix of its new one; the rest starts at zero
    for (size_t i = 0; i < slots && e == hipSuccess; i++) {
        e = hipMemsetAsync(nk[i], 0, bytes, s);
        if (e == hipSuccess) e = hipMemsetAsync(nv[i], 0, bytes, s);
        for (int h = 0; h < nkv && e == hipSuccess; h++) {
            e = hipMemcpyAsync(reinterpret_cast<char*>(nk[i]) + h * new_head,
                               reinterpret_cast<char*>(c->kc[i]) + h * old_head, old_head, hipMemcpyDeviceToDevice, s);
            if (e == hipSuccess)
                e = hipMemcpyAsync(reinterpret_cast<char*>(nv[i]) + h * new_head,
                                   reinterpret_cast<char*>(c->vc[i]) + h * old_head, old_head, hipMemcpyDeviceToDevice,
                                   s);
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);  // no copy may still read or write the buffers freed here
        free_all(nk);
        free_all(nv);
        return e == hipErrorOutOfMemory ? fail(c, QWATTN_ENOMEM, "out of VRAM growing the K/V caches")
                                        : fail(c, QWATTN_EHIP, "qwattn_kv_grow: %s", hipGetErrorString(e));
    }
    free_all(c->kc);
    free_all(c->vc);
    c->kc.swap(nk);
    c->vc.swap(nv);
    c->kv_cap = (int)cap;
    return QWATTN_OK;
}

int qwattn_set_alloc_fault(qwattn_ctx* c, int nth) {
    if (!c) return QWATTN_EINVAL;
    if (nth < 0) return fail(c, QWATTN_EINVAL, "qwattn_set_alloc_fault: %d", nth);
    c->alloc_fault = nth;
    return QWATTN_OK;
}

int qwattn_kv_slot(const qwattn_ctx* c, int slot, void** kcache, void** vcache, int* cap) {
    if (!c || slot < 0 || slot >= (int)c->kc.size()) return QWATTN_EINVAL;
    if (kcache) *kcache = c->kc[slot];
    if (vcache) *vcache = c->vc[slot];
    if (cap) *cap = c->kv_cap;
    return QWATTN_OK;
}

// ---- kernels ----------------------------------------------------------------------------------------

int qwattn_qk_norm_rope_append(qwattn_ctx* c, void* stream, const void* qg, const void* k, const void* v,
                               int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache,
                               void* vcache, int kv_cap, void* q_out, int q_dtype, int pos, int n) {
    if (!c) return QWATTN_EINVAL;
    if (!qg || !k || !v || !qn || !kn || !kcache || !vcache || (!rope && c->cfg.rope_dim))
        return fail(c, QWATTN_EINVAL, "qwattn_qk_norm_rope_append: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    if (q_out && q_dtype != QWATTN_F32 && q_dtype != QWATTN_F16) return fail(c, QWATTN_EINVAL, "q_dtype %d", q_dtype);
    int rc = check_call(c, pos, n, kv_cap);
    if (rc) return rc;
    DeviceGuard dg(c->device);
    const qwattn_config& g = c->cfg;
    qw::NormRopeArgs a{qg, k, v, qn, kn, rope ? rope : c->rope, (uint16_t*)kcache, (uint16_t*)vcache, q_out,
                       pos, n, g.n_heads, g.n_kv_heads, g.rope_dim, g.rms_eps,
                       qw::kLog2eHost / std::sqrt((float)g.head_dim), kv_cap};
    HIP_TRY(c, qw::launch_qk_norm_rope(a, g.head_dim, in_dtype, q_dtype == QWATTN_F16 ? 1 : 0, (hipStream_t)stream));
    return QWATTN_OK;
}

// QSA key bits of a call (NULL: dense): checks the row width and raises the split count until no workgroup
// has more tiles than its kernel holds key words for (kQsaTiles: the loader-wave kernel, at most 8 query rows
// per KV head; kQsaChunkTiles: the 16-row-slice kernel)
// Histogram copies a token of a select launch of n tokens takes: up to 8 (the scoring workgroups add their
// counts into the copies in turn), within the context's histograms.
static int qsa_hist_copies(const qwattn_ctx* c, int n) { return std::max(1, std::min(8, c->qsa_hist_n / std::max(1, n))); }

static int qsa_args(qwattn_ctx* c, const char* fn, const uint32_t* kbits, int kb_words, int pos, int n, Split* sp,
                    qw::DecodeArgs* a) {
    if (!kbits) return QWATTN_OK;
    const qwattn_config& g = c->cfg;
    if (kb_words * 32 < pos + n)
        return fail(c, QWATTN_EINVAL, "%s: kb_words %d < %d keys / 32", fn, kb_words, pos + n);
    const int nb = (pos + n + 31) / 32;
    const int cap_tiles = n * (g.n_heads / g.n_kv_heads) <= 8 ? qw::kQsaTiles : qw::kQsaChunkTiles;
    if ((nb + sp->S - 1) / sp->S > cap_tiles) {
        const int S = (nb + cap_tiles - 1) / cap_tiles;
        if (S > g.max_splits)
            return fail(c, QWATTN_EINVAL, "%s: %d keys need %d splits, more than max_splits %d", fn, pos + n, S,
                        g.max_splits);
        *sp = Split{S, nb / S, nb % S};
    }
    a->kbits = kbits, a->kb_words = kb_words;
    a->n_split = sp->S, a->cq = sp->cq, a->cr = sp->cr;
    return QWATTN_OK;
}

static int attend_partial_impl(qwattn_ctx* c, const char* fn, void* stream, const float* q, const void* kcache,
                               const void* vcache, int kv_cap, int pos, int n, int n_split, const uint32_t* kbits,
                               int kb_words, int* used_splits) {
    if (!c) return QWATTN_EINVAL;
    if (!q || !kcache || !vcache) return fail(c, QWATTN_EINVAL, "%s: null pointer", fn);
    int rc = check_call(c, pos, n, kv_cap);
    if (rc) return rc;
    const qwattn_config& g = c->cfg;
    const int G = g.n_heads / g.n_kv_heads;
    if (n * G > 32) return fail(c, QWATTN_EINVAL, "%s: n * NH/NKV = %d > 32 rows (use the prefill kernel)", fn, n * G);
    Split sp = pick_split(c, pos + n, n, n_split);
    qw::DecodeArgs a = decode_args(c, q, nullptr, nullptr, nullptr, nullptr, nullptr, kcache, vcache, kv_cap, pos, n, sp);
    if ((rc = qsa_args(c, fn, kbits, kb_words, pos, n, &sp, &a))) return rc;
    const int used = sp.S;
    DeviceGuard dg(c->device);
    HIP_TRY(c, qw::launch_decode(a, g.head_dim, false, QWATTN_F32, (hipStream_t)stream));
    c->last_splits = used;
    c->last_n = n;
    if (used_splits) *used_splits = used;
    return QWATTN_OK;
}

int qwattn_attend_partial(qwattn_ctx* c, void* stream, const float* q, const void* kcache, const void* vcache,
                          int kv_cap, int pos, int n, int n_split, int* used_splits) {
    return attend_partial_impl(c, "qwattn_attend_partial", stream, q, kcache, vcache, kv_cap, pos, n, n_split, nullptr,
                               0, used_splits);
}

int qwattn_attend_partial_qsa(qwattn_ctx* c, void* stream, const float* q, const void* kcache, const void* vcache,
                              int kv_cap, int pos, int n, int n_split, const uint32_t* key_bits, int kb_words,
                              int* used_splits) {
    if (c && !key_bits) return fail(c, QWATTN_EINVAL, "qwattn_attend_partial_qsa: null key_bits");
    return attend_partial_impl(c, "qwattn_attend_partial_qsa", stream, q, kcache, vcache, kv_cap, pos, n, n_split,
                               key_bits, kb_words, used_splits);
}

int qwattn_decode_partial(qwattn_ctx* c, void* stream, const void* qg, const void* k, const void* v, int in_dtype,
                          const float* qn, const float* kn, const float* rope, void* kcache, void* vcache, int kv_cap,
                          int pos, int n, int n_split, int* used_splits) {
    if (!c) return QWATTN_EINVAL;
    if (!qg || !k || !v || !qn || !kn || !kcache || !vcache || (!rope && c->cfg.rope_dim))
        return fail(c, QWATTN_EINVAL, "qwattn_decode_partial: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    int rc = check_call(c, pos, n, kv_cap);
    if (rc) return rc;
    const qwattn_config& g = c->cfg;
    const int G = g.n_heads / g.n_kv_heads;
    if (n * G > 32 || n > 8)
        return fail(c, QWATTN_EINVAL, "qwattn_decode_partial: n = %d tokens (n * NH/NKV = %d) exceeds the fused decode "
                    "kernel (n <= 8 and n * NH/NKV <= 32)", n, n * G);
    const Split sp = pick_split(c, pos + n, n, n_split);
    const int used = sp.S;
    DeviceGuard dg(c->device);
    const qw::DecodeArgs a = decode_args(c, qg, k, v, qn, kn, rope ? rope : c->rope, kcache, vcache, kv_cap, pos, n,
                                         sp);
    HIP_TRY(c, qw::launch_decode(a, g.head_dim, true, in_dtype, (hipStream_t)stream));
    c->last_splits = used;
    c->last_n = n;
    if (used_splits) *used_splits = used;
    return QWATTN_OK;
}

static int decode_impl(qwattn_ctx* c, const char* fn, void* stream, const void* qg, const void* k, const void* v,
                       int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache, void* vcache,
                       int kv_cap, float* out, int pos, int n, int n_split, const uint32_t* kbits, int kb_words,
                       int* used_splits) {
    if (!c) return QWATTN_EINVAL;
    if (!qg || !k || !v || !qn || !kn || !kcache || !vcache || !out || (!rope && c->cfg.rope_dim))
        return fail(c, QWATTN_EINVAL, "%s: null pointer", fn);
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    int rc = check_call(c, pos, n, kv_cap);
    if (rc) return rc;
    const qwattn_config& g = c->cfg;
    const int G = g.n_heads / g.n_kv_heads;
    if (n * G > 32 || n > 8)
        return fail(c, QWATTN_EINVAL, "qwattn_decode: n = %d tokens (n * NH/NKV = %d) exceeds the fused decode "
                    "kernel (n <= 8 and n * NH/NKV <= 32)", n, n * G);
    // the combine runs inside the attend launch (tail_launch); otherwise the combine kernel follows. Up to 8
    // rows a requested split count is capped at one streaming workgroup per CU: its partials never leave
    // the launch, and more parts would only add workgroup prologues and partials to merge
    const int ncomb = n * g.n_heads;
    Split sp = pick_split(c, pos + n, n, n_split, n * G <= 8);
    qw::DecodeArgs a = decode_args(c, qg, k, v, qn, kn, rope ? rope : c->rope, kcache, vcache, kv_cap, pos, n, sp);
    if ((rc = qsa_args(c, fn, kbits, kb_words, pos, n, &sp, &a))) return rc;
    const bool one = tail_launch(g, n, sp.S);
    const int used = sp.S;
    DeviceGuard dg(c->device);
    if (one) a.out = out, a.ep = c->ep, a.rec = c->rec, a.ncomb = ncomb, a.nds = combine_slices(g, n, sp.S);
    HIP_TRY(c, qw::launch_decode(a, g.head_dim, true, in_dtype, (hipStream_t)stream));
    if (!one) {
        qw::CombineArgs ca{c->part_o, c->part_ml, qg, out, n, g.n_heads, used};
        HIP_TRY(c, qw::launch_combine(ca, g.head_dim, in_dtype, (hipStream_t)stream));
    }
    // the partials are consumed in the launch: a following qwattn_combine has nothing to merge
    c->last_splits = 0;
    if (used_splits) *used_splits = used;
    return QWATTN_OK;
}

int qwattn_decode(qwattn_ctx* c, void* stream, const void* qg, const void* k, const void* v, int in_dtype,
                  const float* qn, const float* kn, const float* rope, void* kcache, void* vcache, int kv_cap,
                  float* out, int pos, int n, int n_split, int* used_splits) {
    return decode_impl(c, "qwattn_decode", stream, qg, k, v, in_dtype, qn, kn, rope, kcache, vcache, kv_cap, out, pos,
                       n, n_split, nullptr, 0, used_splits);
}

int qwattn_decode_qsa(qwattn_ctx* c, void* stream, const void* qg, const void* k, const void* v, int in_dtype,
                      const float* qn, const float* kn, const float* rope, void* kcache, void* vcache, int kv_cap,
                      float* out, int pos, int n, int n_split, const uint32_t* key_bits, int kb_words,
                      int* used_splits) {
    if (c && !key_bits) return fail(c, QWATTN_EINVAL, "qwattn_decode_qsa: null key_bits");
    return decode_impl(c, "qwattn_decode_qsa", stream, qg, k, v, in_dtype, qn, kn, rope, kcache, vcache, kv_cap, out,
                       pos, n, n_split, key_bits, kb_words, used_splits);
}

int qwattn_combine(qwattn_ctx* c, void* stream, const void* qg, int in_dtype, float* out, int n, int n_split) {
    if (!c) return QWATTN_EINVAL;
    if (!qg || !out) return fail(c, QWATTN_EINVAL, "qwattn_combine: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    if (c->last_splits == 0)
        return fail(c, QWATTN_ESTATE, "qwattn_combine: no partials (call qwattn_attend_partial or qwattn_decode_partial first)");
    if (n != c->last_n || n_split != c->last_splits)
        return fail(c, QWATTN_EINVAL, "qwattn_combine: n=%d splits=%d do not match the last partials (n=%d splits=%d)", n,
                    n_split, c->last_n, c->last_splits);
    if (int rc = take_wait_error(c)) return rc;
    DeviceGuard dg(c->device);
    qw::CombineArgs a{c->part_o, c->part_ml, qg, out, n, c->cfg.n_heads, n_split};
    HIP_TRY(c, qw::launch_combine(a, c->cfg.head_dim, in_dtype, (hipStream_t)stream));
    return QWATTN_OK;
}

// the launch arguments shared by both prefill entry points (split layout sized for n)
static int prefill_args(qwattn_ctx* c, const void* q, const void* kcache, const void* vcache, int kv_cap,
                        const void* qg, float* out, int pos, int n, qw::PrefillArgs* a) {
    const qwattn_config& g = c->cfg;
    // Few query tiles (two workgroups per tile still fit the CUs): every tile's keys are split over two
    // workgroups; otherwise short and long tiles are paired. Either way the split tiles fit the slots
    // sized at creation (n <= max_tokens by check_call; split_all only when 2 * n_qt * NKV <= n_cu).
    const int n_qt = qw::pf_query_tiles(n, g.n_heads / g.n_kv_heads);
    const int split_all = 2 * n_qt * g.n_kv_heads <= c->n_cu ? 1 : 0;
    *a = qw::PrefillArgs{q, (const uint16_t*)kcache, (const uint16_t*)vcache, qg, out, pos, n, g.n_heads,
                         g.n_kv_heads, qw::kLog2eHost / std::sqrt((float)g.head_dim), kv_cap, c->pf_part, c->pf_cnt,
                         qw::pf_split_slots(n_qt, split_all), split_all, nullptr, nullptr, 0, g.rms_eps};
    if (a->slots > c->pf_slots_per_head) return fail(c, QWATTN_EINVAL, "prefill: %d split slots > %d", a->slots, c->pf_slots_per_head);
    return QWATTN_OK;
}

static int kbits_ok(qwattn_ctx* c, const char* fn, const uint32_t* kbits, int kb_words, int pos, int n) {
    if (kbits && kb_words * 32 < pos + n)
        return fail(c, QWATTN_EINVAL, "%s: kb_words %d < %d keys / 32", fn, kb_words, pos + n);
    return QWATTN_OK;
}

static int attend_prefill_impl(qwattn_ctx* c, const char* fn, void* stream, const void* q, int q_dtype,
                               const void* kcache, const void* vcache, int kv_cap, const void* qg, int in_dtype,
                               float* out, int pos, int n, const uint32_t* kbits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    if (!q || !kcache || !vcache || !qg || !out) return fail(c, QWATTN_EINVAL, "%s: null pointer", fn);
    if (q_dtype != QWATTN_F32 && q_dtype != QWATTN_F16) return fail(c, QWATTN_EINVAL, "q_dtype %d", q_dtype);
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    int rc = check_call(c, pos, n, kv_cap);
    if (rc || (rc = kbits_ok(c, fn, kbits, kb_words, pos, n))) return rc;
    const qwattn_config& g = c->cfg;
    DeviceGuard dg(c->device);
    qw::PrefillArgs a;
    if ((rc = prefill_args(c, q, kcache, vcache, kv_cap, qg, out, pos, n, &a))) return rc;
    a.kbits = kbits, a.kb_words = kb_words;
    if (q_dtype == QWATTN_F32) {  // the kernel's operand: fp16(q * log2(e)/sqrt(D)) in the context's query buffer
        HIP_TRY(c, qw::launch_q_f16(static_cast<const float*>(q), c->q16, a.q_scale, (size_t)n * g.n_heads * g.head_dim,
                                    (hipStream_t)stream));
        a.q = c->q16;
    }
    HIP_TRY(c, qw::launch_prefill(a, g.head_dim, 2, in_dtype, (hipStream_t)stream));
    return QWATTN_OK;
}

int qwattn_attend_prefill(qwattn_ctx* c, void* stream, const void* q, int q_dtype, const void* kcache,
                          const void* vcache, int kv_cap, const void* qg, int in_dtype, float* out, int pos, int n) {
    return attend_prefill_impl(c, "qwattn_attend_prefill", stream, q, q_dtype, kcache, vcache, kv_cap, qg, in_dtype,
                               out, pos, n, nullptr, 0);
}

int qwattn_attend_prefill_qsa(qwattn_ctx* c, void* stream, const void* q, int q_dtype, const void* kcache,
                              const void* vcache, int kv_cap, const void* qg, int in_dtype, float* out, int pos, int n,
                              const uint32_t* key_bits, int kb_words) {
    if (c && !key_bits) return fail(c, QWATTN_EINVAL, "qwattn_attend_prefill_qsa: null key_bits");
    return attend_prefill_impl(c, "qwattn_attend_prefill_qsa", stream, q, q_dtype, kcache, vcache, kv_cap, qg,
                               in_dtype, out, pos, n, key_bits, kb_words);
}

static int attend_prefill_qg_impl(qwattn_ctx* c, const char* fn, void* stream, const void* qg, int in_dtype,
                                  const float* qn, const float* rope, const void* kcache, const void* vcache,
                                  int kv_cap, float* out, int pos, int n, const uint32_t* kbits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    const qwattn_config& g = c->cfg;
    if (!qg || !qn || !kcache || !vcache || !out || (!rope && g.rope_dim))
        return fail(c, QWATTN_EINVAL, "%s: null pointer", fn);
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    if (!qw::pf_fused_rope_ok(g.rope_dim, g.head_dim))
        return fail(c, QWATTN_EINVAL, "%s: rope_dim %d (needs 0, 32, 64, 128 or 256, <= head_dim %d)", fn, g.rope_dim,
                    g.head_dim);
    int rc = check_call(c, pos, n, kv_cap);
    if (rc || (rc = kbits_ok(c, fn, kbits, kb_words, pos, n))) return rc;
    DeviceGuard dg(c->device);
    qw::PrefillArgs a;
    if ((rc = prefill_args(c, nullptr, kcache, vcache, kv_cap, qg, out, pos, n, &a))) return rc;
    a.qn = qn;
    a.rope = rope;
    a.R = g.rope_dim;
    a.kbits = kbits, a.kb_words = kb_words;
    HIP_TRY(c, qw::launch_prefill(a, g.head_dim, 2, in_dtype, (hipStream_t)stream));
    return QWATTN_OK;
}

int qwattn_attend_prefill_qg(qwattn_ctx* c, void* stream, const void* qg, int in_dtype, const float* qn,
                             const float* rope, const void* kcache, const void* vcache, int kv_cap, float* out,
                             int pos, int n) {
    return attend_prefill_qg_impl(c, "qwattn_attend_prefill_qg", stream, qg, in_dtype, qn, rope, kcache, vcache,
                                  kv_cap, out, pos, n, nullptr, 0);
}

static int prefill_impl(qwattn_ctx* c, const char* fn, void* stream, const void* qg, const void* k, const void* v,
                        int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache, void* vcache,
                        int kv_cap, float* out, int pos, int n, const uint32_t* kbits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    if (!out) return fail(c, QWATTN_EINVAL, "%s: null pointer", fn);
    int rc = kbits_ok(c, fn, kbits, kb_words, pos, n);
    if (rc) return rc;
    if (qw::pf_fused_rope_ok(c->cfg.rope_dim, c->cfg.head_dim)) {
        // the key and value rows appended, then the MFMA prefill normalizing the query rows itself
        rc = qwattn_qk_norm_rope_append(c, stream, qg, k, v, in_dtype, qn, kn, rope, kcache, vcache, kv_cap, nullptr,
                                        QWATTN_F16, pos, n);
        if (rc) return rc;
        return attend_prefill_qg_impl(c, fn, stream, qg, in_dtype, qn, rope ? rope : c->rope, kcache, vcache, kv_cap,
                                      out, pos, n, kbits, kb_words);
    }
    // norm + rope + append into the context's fp16 query buffer, then the MFMA prefill on it
    rc = qwattn_qk_norm_rope_append(c, stream, qg, k, v, in_dtype, qn, kn, rope, kcache, vcache, kv_cap, c->q16,
                                    QWATTN_F16, pos, n);
    if (rc) return rc;
    return attend_prefill_impl(c, fn, stream, c->q16, QWATTN_F16, kcache, vcache, kv_cap, qg, in_dtype, out, pos, n,
                               kbits, kb_words);
}

int qwattn_prefill(qwattn_ctx* c, void* stream, const void* qg, const void* k, const void* v, int in_dtype,
                   const float* qn, const float* kn, const float* rope, void* kcache, void* vcache, int kv_cap,
                   float* out, int pos, int n) {
    return prefill_impl(c, "qwattn_prefill", stream, qg, k, v, in_dtype, qn, kn, rope, kcache, vcache, kv_cap, out,
                        pos, n, nullptr, 0);
}

int qwattn_prefill_qsa(qwattn_ctx* c, void* stream, const void* qg, const void* k, const void* v, int in_dtype,
                       const float* qn, const float* kn, const float* rope, void* kcache, void* vcache, int kv_cap,
                       float* out, int pos, int n, const uint32_t* key_bits, int kb_words) {
    if (c && !key_bits) return fail(c, QWATTN_EINVAL, "qwattn_prefill_qsa: null key_bits");
    return prefill_impl(c, "qwattn_prefill_qsa", stream, qg, k, v, in_dtype, qn, kn, rope, kcache, vcache, kv_cap, out,
                        pos, n, key_bits, kb_words);
}

static int layer_impl(qwattn_ctx* c, const char* fn, void* stream, int slot, const void* qg, const void* k,
                      const void* v, int in_dtype, const float* qn, const float* kn, float* out, int pos, int n,
                      int n_split, const uint32_t* kbits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    if (slot < 0 || slot >= (int)c->kc.size())
        return fail(c, QWATTN_ESTATE, "%s: slot %d of %d allocated K/V caches", fn, slot, (int)c->kc.size());
    const int G = c->cfg.n_heads / c->cfg.n_kv_heads;
    int rc, used = 0;
    if (n * G <= 32 && n <= 8)  // decode / verify: one launch (norm + rope + append + split attend + combine)
        return decode_impl(c, fn, stream, qg, k, v, in_dtype, qn, kn, c->rope, c->kc[slot], c->vc[slot], c->kv_cap, out,
                           pos, n, n_split, kbits, kb_words, &used);
    if (n * G <= 32) {  // more than 8 tokens in small groups: norm + rope + append, split attend, combine
        rc = qwattn_qk_norm_rope_append(c, stream, qg, k, v, in_dtype, qn, kn, c->rope, c->kc[slot], c->vc[slot],
                                        c->kv_cap, c->q32, QWATTN_F32, pos, n);
        if (rc) return rc;
        rc = attend_partial_impl(c, fn, stream, c->q32, c->kc[slot], c->vc[slot], c->kv_cap, pos, n, n_split, kbits,
                                 kb_words, &used);
        if (rc) return rc;
        return qwattn_combine(c, stream, qg, in_dtype, out, n, used);
    }
    return prefill_impl(c, fn, stream, qg, k, v, in_dtype, qn, kn, c->rope, c->kc[slot], c->vc[slot], c->kv_cap, out,
                        pos, n, kbits, kb_words);
}

int qwattn_layer_attention(qwattn_ctx* c, void* stream, int slot, const void* qg, const void* k, const void* v,
                           int in_dtype, const float* qn, const float* kn, float* out, int pos, int n, int n_split) {
    return layer_impl(c, "qwattn_layer_attention", stream, slot, qg, k, v, in_dtype, qn, kn, out, pos, n, n_split,
                      nullptr, 0);
}

int qwattn_layer_attention_qsa(qwattn_ctx* c, void* stream, int slot, const void* qg, const void* k, const void* v,
                               int in_dtype, const float* qn, const float* kn, float* out, int pos, int n, int n_split,
                               const uint32_t* key_bits, int kb_words) {
    if (c && !key_bits) return fail(c, QWATTN_EINVAL, "qwattn_layer_attention_qsa: null key_bits");
    return layer_impl(c, "qwattn_layer_attention_qsa", stream, slot, qg, k, v, in_dtype, qn, kn, out, pos, n, n_split,
                      key_bits, kb_words);
}

// ---- the decode without allocation ------------------------------------------------------------------
// qwattn_decode_noalloc keeps what qwattn_decode keeps in the context — the per-KV-head launch counters,
// the split records and the split partials — in `scratch`, one static array per GPU the library runs on,
// held until the process ends. Layout: [0, 256) the launch counters (32 u64, one per KV head index; they
// only grow and are never cleared: static device memory starts at zero), then the records and the
// partials of the call, laid out per call. In host code `scratch` names a host-side stand-in: its device
// address, per device, comes from hipGetSymbolAddress (scratch_base) and only that address is used.
constexpr size_t kScratchBytes = (size_t)32 << 20;
constexpr size_t kScratchData = 256;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_at[kMaxDevices] = {};  // device address of `scratch`, per device (nullptr: not yet)
int g_scratch_cu[kMaxDevices] = {};            // the device's compute units

// Device address of `scratch` on `device` (made current by the caller) and its CU count, looked up on the
// first call on that device (the device must be a gfx950).
int scratch_base(int device, unsigned char** base, int* n_cu) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_at[device]) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, device) != hipSuccess)
            return fail(nullptr, QWATTN_EHIP, "hipGetDeviceProperties failed on device %d", device);
        if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
            return fail(nullptr, QWATTN_EINVAL, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
        void* at = nullptr;
        const hipError_t e = hipGetSymbolAddress(&at, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !at)
            return fail(nullptr, QWATTN_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
        g_scratch_cu[device] = prop.multiProcessorCount;
        g_scratch_at[device] = static_cast<unsigned char*>(at);
    }
    *base = g_scratch_at[device];
    *n_cu = g_scratch_cu[device];
    return QWATTN_OK;
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

int qwattn_decode_noalloc(int device, void* stream, const qwattn_config* cfg, const void* qg, const void* k,
                          const void* v, int in_dtype, const float* qn, const float* kn, const float* rope, void* kcache,
                          void* vcache, int kv_cap, float* out, int pos, int n, int n_split, int* wait_status,
                          int* used_splits) {
    if (!cfg) return fail(nullptr, QWATTN_EINVAL, "qwattn_decode_noalloc: null config");
    const qwattn_config& g = *cfg;
    if (int rc = check_shape(nullptr, g)) return rc;
    if (!qg || !k || !v || !qn || !kn || !kcache || !vcache || !out || (!rope && g.rope_dim))
        return fail(nullptr, QWATTN_EINVAL, "qwattn_decode_noalloc: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(nullptr, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    if (int rc = check_range(nullptr, g, pos, n, kv_cap)) return rc;
    const int G = g.n_heads / g.n_kv_heads;
    if (n * G > 32 || n > 8)
        return fail(nullptr, QWATTN_EINVAL, "qwattn_decode_noalloc: n = %d tokens (n * NH/NKV = %d) exceeds the fused "
                    "decode kernel (n <= 8 and n * NH/NKV <= 32)", n, n * G);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev || device >= kMaxDevices)
        return fail(nullptr, QWATTN_EINVAL, "device %d not available (%d devices)", device, ndev);
    DeviceGuard dg(device);
    unsigned char* base = nullptr;
    int n_cu = 0;
    if (int rc = scratch_base(device, &base, &n_cu)) return rc;
    const int ncomb = n * g.n_heads;
    const Split sp = pick_split(n_cu, g, pos + n, n, n_split, n * G <= 8);
    const bool one = tail_launch(g, n, sp.S);
    const size_t parts = (size_t)ncomb * sp.S;  // split partial rows
    const size_t rec_b = align256(parts * 16), ml_b = align256(parts * 8), o_b = align256(parts * g.head_dim * 4);
    if (kScratchData + rec_b + ml_b + o_b > kScratchBytes)
        return fail(nullptr, QWATTN_EINVAL, "qwattn_decode_noalloc: %d splits x %d rows of %d dims need %zu bytes of "
                    "partials, more than its %zu-byte scratch (ask for fewer splits)", sp.S, ncomb, g.head_dim,
                    rec_b + ml_b + o_b, kScratchBytes - kScratchData);
    qw::DecodeArgs a = decode_shape_args(g, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, pos, n, sp);
    a.rec = reinterpret_cast<float*>(base + kScratchData);
    a.part_ml = reinterpret_cast<float*>(base + kScratchData + rec_b);
    a.part_o = reinterpret_cast<float*>(base + kScratchData + rec_b + ml_b);
    a.err = wait_status;
    if (one) a.out = out, a.ep = reinterpret_cast<unsigned long long*>(base), a.ncomb = ncomb, a.nds = combine_slices(g, n, sp.S);
    else a.rec = nullptr;
    hipError_t e = qw::launch_decode(a, g.head_dim, true, in_dtype, (hipStream_t)stream);
    if (e == hipSuccess && !one) {
        qw::CombineArgs ca{a.part_o, a.part_ml, qg, out, n, g.n_heads, sp.S};
        e = qw::launch_combine(ca, g.head_dim, in_dtype, (hipStream_t)stream);
    }
    if (e != hipSuccess) return fail(nullptr, QWATTN_EHIP, "qwattn_decode_noalloc: launch failed: %s", hipGetErrorString(e));
    if (used_splits) *used_splits = sp.S;
    return QWATTN_OK;
}

// ---- QSA indexer ----------------------------------------------------------------------------------------

int qwattn_qsa_pool(qwattn_ctx* c, void* stream, const void* ik, int in_dtype, const float* k_gamma, int idx_dim,
                    int cr, float* raw, float* pooled, int cap, int pos, int n) {
    if (!c) return QWATTN_EINVAL;
    if (!ik || !k_gamma || !raw || !pooled) return fail(c, QWATTN_EINVAL, "qwattn_qsa_pool: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    const qwattn_config& g = c->cfg;
    if (idx_dim <= 0 || idx_dim % 64 || idx_dim > 256 || idx_dim < g.rope_dim)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_pool: idx_dim %d (a multiple of 64, <= 256, >= rope_dim %d)", idx_dim,
                    g.rope_dim);
    if (cr < 2) return fail(c, QWATTN_EINVAL, "qwattn_qsa_pool: compress ratio %d (>= 2)", cr);
    if (n <= 0 || pos < 0 || pos + n > cap || cap > g.max_ctx)
        return fail(c, QWATTN_ERANGE, "qwattn_qsa_pool: positions [%d, %d) beyond the capacity %d (max_ctx %d)", pos,
                    pos + n, cap, g.max_ctx);
    if (int rc = take_wait_error(c)) return rc;
    DeviceGuard dg(c->device);
    qw::QsaPoolArgs a{ik, k_gamma, c->rope, raw, pooled, pos, n, idx_dim, cr, g.rope_dim, g.rms_eps};
    HIP_TRY(c, qw::launch_qsa_pool(a, in_dtype, (hipStream_t)stream));
    return QWATTN_OK;
}

int qwattn_qsa_select(qwattn_ctx* c, void* stream, const void* iq, int in_dtype, const float* q_gamma, int idx_heads,
                      int idx_dim, int cr, int budget, const float* pooled, int pos, int n, uint32_t* mask,
                      int mask_words, uint32_t* key_bits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    if (!iq || !q_gamma || !pooled || (!mask && !key_bits))
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_select: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    const qwattn_config& g = c->cfg;
    if (idx_dim <= 0 || idx_dim % 64 || idx_dim > 256 || idx_dim < g.rope_dim || idx_heads <= 0 ||
        idx_heads * idx_dim > 8192)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_select: %d heads of %d dims (idx_dim a multiple of 64, <= 256, >= "
                    "rope_dim %d; heads x dims <= 8192)", idx_heads, idx_dim, g.rope_dim);
    if (cr < 2 || budget <= 0 || budget % cr)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_select: budget %d with compress ratio %d (a positive multiple)",
                    budget, cr);
    if (n <= 0 || pos < 0 || pos + n > g.max_ctx || n > g.max_tokens)
        return fail(c, QWATTN_ERANGE, "qwattn_qsa_select: tokens [%d, %d) (max_ctx %d, max_tokens %d)", pos, pos + n,
                    g.max_ctx, g.max_tokens);
    const int nmax = (pos + n) / cr;  // complete blocks of the last token
    if ((nmax + 31) / 32 > qw::qsa_mask_lds_words())
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_select: %d complete blocks exceed the %d a launch holds", nmax,
                    32 * qw::qsa_mask_lds_words());
    if (mask && mask_words * 32 < nmax)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_select: mask_words %d < %d blocks / 32", mask_words, nmax);
    if (key_bits && kb_words * 32 < pos + n)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_select: kb_words %d < %d keys / 32", kb_words, pos + n);
    if (int rc = take_wait_error(c)) return rc;
    DeviceGuard dg(c->device);
    const int stride = (std::max(1, nmax) + 3) & ~3;  // score rows padded to whole 16-byte loads
    const int per = (int)std::min<size_t>(std::min(c->qsa_hist_n, qw::qsa_select_tokens(nmax)),
                                          std::max<size_t>(1, kQsaScoreBytes / ((size_t)stride * sizeof(float))));
    for (int t0 = 0; t0 < n; t0 += per) {
        const int nt = std::min(per, n - t0);
        qw::QsaSelectArgs a{(const char*)iq + (size_t)t0 * idx_heads * idx_dim * (in_dtype == QWATTN_F32 ? 4 : 2),
                            q_gamma, c->rope, pooled, c->qsa_scores, c->qsa_cnt, c->qsa_hist, c->qsa_cand,
                            c->qsa_cand_n, mask ? mask + (size_t)t0 * mask_words : nullptr,
                            key_bits ? key_bits + (size_t)t0 * kb_words : nullptr, nullptr, nullptr, mask_words,
                            kb_words, stride, pos + t0, nt, idx_heads, idx_dim, cr, budget / cr, g.rope_dim,
                            g.rms_eps, qsa_hist_copies(c, nt)};
        HIP_TRY(c, qw::launch_qsa_select(a, in_dtype, (hipStream_t)stream));
    }
    return QWATTN_OK;
}

int qwattn_qsa_index(qwattn_ctx* c, void* stream, const void* ik, const void* iq, int in_dtype, const float* k_gamma,
                     const float* q_gamma, int idx_heads, int idx_dim, int cr, int budget, float* raw, float* pooled,
                     int cap, int pos, int n, uint32_t* mask, int mask_words, uint32_t* key_bits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    if (!ik || !k_gamma || !raw) return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: null pointer");
    if (n <= 0 || pos < 0 || pos + n > cap || cap > c->cfg.max_ctx)
        return fail(c, QWATTN_ERANGE, "qwattn_qsa_index: positions [%d, %d) beyond the capacity %d (max_ctx %d)", pos,
                    pos + n, cap, c->cfg.max_ctx);
    const int nmax = (pos + n) / std::max(cr, 1);
    const int stride = (std::max(1, nmax) + 3) & ~3;  // score rows padded to whole 16-byte loads
    const int per = (int)std::min<size_t>(std::min(c->qsa_hist_n, qw::qsa_select_tokens(nmax)),
                                          std::max<size_t>(1, kQsaScoreBytes / ((size_t)stride * sizeof(float))));
    if (cr < 2 || nmax != pos / cr || n > per) {
        // a block completes (or the tokens take several select launches): the pooling launch, then the select
        if (int rc = qwattn_qsa_pool(c, stream, ik, in_dtype, k_gamma, idx_dim, cr, raw, pooled, cap, pos, n)) return rc;
        return qwattn_qsa_select(c, stream, iq, in_dtype, q_gamma, idx_heads, idx_dim, cr, budget, pooled, pos, n,
                                 mask, mask_words, key_bits, kb_words);
    }
    // no block completes: nothing to pool, and the select launch appends the raw keys itself
    if (!iq || !q_gamma || !pooled || (!mask && !key_bits))
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: null pointer");
    if (in_dtype != QWATTN_F32 && in_dtype != QWATTN_BF16) return fail(c, QWATTN_EINVAL, "in_dtype %d", in_dtype);
    const qwattn_config& g = c->cfg;
    if (idx_dim <= 0 || idx_dim % 64 || idx_dim > 256 || idx_dim < g.rope_dim || idx_heads <= 0 ||
        idx_heads * idx_dim > 8192)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: %d heads of %d dims (idx_dim a multiple of 64, <= 256, >= "
                    "rope_dim %d; heads x dims <= 8192)", idx_heads, idx_dim, g.rope_dim);
    if (budget <= 0 || budget % cr)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: budget %d with compress ratio %d (a positive multiple)",
                    budget, cr);
    if (n > g.max_tokens) return fail(c, QWATTN_ERANGE, "qwattn_qsa_index: n %d > max_tokens %d", n, g.max_tokens);
    if ((nmax + 31) / 32 > qw::qsa_mask_lds_words())
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: %d complete blocks exceed the %d a launch holds", nmax,
                    32 * qw::qsa_mask_lds_words());
    if (mask && mask_words * 32 < nmax)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: mask_words %d < %d blocks / 32", mask_words, nmax);
    if (key_bits && kb_words * 32 < pos + n)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_index: kb_words %d < %d keys / 32", kb_words, pos + n);
    if (int rc = take_wait_error(c)) return rc;
    DeviceGuard dg(c->device);
    qw::QsaSelectArgs a{iq, q_gamma, c->rope, pooled, c->qsa_scores, c->qsa_cnt, c->qsa_hist, c->qsa_cand,
                        c->qsa_cand_n, mask, key_bits, ik, raw, mask_words, kb_words, stride, pos, n, idx_heads,
                        idx_dim, cr, budget / cr, g.rope_dim, g.rms_eps, qsa_hist_copies(c, n)};
    HIP_TRY(c, qw::launch_qsa_select(a, in_dtype, (hipStream_t)stream));
    return QWATTN_OK;
}

}  // extern "C"

// binary16 bits to float as the reference's upload widens Q8_0 scales (ck::half_to_f32,
// src/cpu_kernels.cpp:20-34): sign, 5-bit exponent (bias 15), 10-bit fraction; subnormals scale the
// fraction by 2^-24. Exponent 31 has no inf / NaN case there: it is a normal exponent, so 0x7C00 widens to
// 65536 and 0x7FFF to 131008, and the planar scales stay bit-identical to the reference's.
static float half_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, f = h & 1023u;
    float v;
    if (e == 0) v = std::ldexp((float)f, -24);
    else v = std::ldexp((float)(f | 1024u), (int)e - 25);
    uint32_t b;
    std::memcpy(&b, &v, 4);
    b |= sign;
    std::memcpy(&v, &b, 4);
    return v;
}

extern "C" {

int qwattn_mat(qwattn_ctx* c, void* stream, const void* w, const float* s, int q8, int rows, int cols, const float* x,
               int x_stride, float* y, int y_stride, int n, int post, float post_scale) {
    if (!c) return QWATTN_EINVAL;
    if (!w || !x || !y || (q8 && !s)) return fail(c, QWATTN_EINVAL, "qwattn_mat: null pointer");
    if (rows <= 0 || cols <= 0 || n <= 0 || cols % (q8 ? 32 : 16))
        return fail(c, QWATTN_EINVAL, "qwattn_mat: %d x %d weights (cols a multiple of %d), n %d", rows, cols,
                    q8 ? 32 : 16, n);
    if (x_stride < cols || x_stride % 4 || y_stride < rows || post < 0 || post > 1)
        return fail(c, QWATTN_EINVAL, "qwattn_mat: x_stride %d (>= cols, a multiple of 4), y_stride %d (>= rows), post %d",
                    x_stride, y_stride, post);
    if (((uintptr_t)w | (uintptr_t)x) & 15) return fail(c, QWATTN_EINVAL, "qwattn_mat: w and x must be 16-byte aligned");
    DeviceGuard dg(c->device);
    qw::MatArgs a{w, s, x, y, rows, cols, n, x_stride, y_stride, post, post_scale};
    HIP_TRY(c, qw::launch_mat(a, q8 != 0, (hipStream_t)stream));
    return QWATTN_OK;
}

int qwattn_mat_multi(qwattn_ctx* c, void* stream, const qwattn_mat_out* mats, int count, int q8, int cols,
                     const float* x, int x_stride, int n) {
    if (!c) return QWATTN_EINVAL;
    if (!mats || count < 1 || count > qw::kMatMulti)
        return fail(c, QWATTN_EINVAL, "qwattn_mat_multi: %d matrices (1..%d)", count, qw::kMatMulti);
    if (!x || cols <= 0 || n <= 0 || cols % (q8 ? 32 : 16) || x_stride < cols || x_stride % 4 || ((uintptr_t)x & 15))
        return fail(c, QWATTN_EINVAL, "qwattn_mat_multi: cols %d (a multiple of %d), n %d, x_stride %d (>= cols, a multiple "
                    "of 4), x 16-byte aligned", cols, q8 ? 32 : 16, n, x_stride);
    qw::MatMultiArgs a{};
    a.count = count;
    for (int i = 0; i < count; i++) {
        const qwattn_mat_out& m = mats[i];
        if (!m.w || !m.y || (q8 && !m.s) || m.rows <= 0 || m.y_stride < m.rows || m.post < 0 || m.post > 1 ||
            ((uintptr_t)m.w & 15))
            return fail(c, QWATTN_EINVAL, "qwattn_mat_multi: matrix %d: rows %d, y_stride %d (>= rows), post %d, w and y set "
                        "(w 16-byte aligned), s set for q8", i, m.rows, m.y_stride, m.post);
        a.m[i] = qw::MatArgs{m.w, m.s, x, m.y, m.rows, cols, n, x_stride, m.y_stride, m.post, m.post_scale};
    }
    DeviceGuard dg(c->device);
    HIP_TRY(c, qw::launch_mat_multi(a, q8 != 0, (hipStream_t)stream));
    return QWATTN_OK;
}

int qwattn_q8_unpack(const uint8_t* blocks, int rows, int cols, int8_t* w, float* s) {
    if (!blocks || !w || !s || rows <= 0 || cols <= 0 || cols % 32) return QWATTN_EINVAL;
    for (int r = 0; r < rows; r++) {
        const uint8_t* src = blocks + (size_t)r * (cols / 32) * 34;
        for (int b = 0; b < cols / 32; b++, src += 34) {
            uint16_t h;
            std::memcpy(&h, src, 2);
            s[(size_t)r * (cols / 32) + b] = half_bits_to_float(h);
            std::memcpy(w + (size_t)r * cols + 32 * b, src + 2, 32);
        }
    }
    return QWATTN_OK;
}

int qwattn_qsa_key_bits(qwattn_ctx* c, void* stream, const uint32_t* mask, int mask_words, int cr, int pos, int n,
                        uint32_t* key_bits, int kb_words) {
    if (!c) return QWATTN_EINVAL;
    if (!mask || !key_bits) return fail(c, QWATTN_EINVAL, "qwattn_qsa_key_bits: null pointer");
    if (cr < 2) return fail(c, QWATTN_EINVAL, "qwattn_qsa_key_bits: compress ratio %d (>= 2)", cr);
    if (n <= 0 || pos < 0) return fail(c, QWATTN_ERANGE, "qwattn_qsa_key_bits: tokens [%d, %d)", pos, pos + n);
    if (mask_words * 32 < (pos + n) / cr || kb_words * 32 < pos + n)
        return fail(c, QWATTN_EINVAL, "qwattn_qsa_key_bits: mask_words %d / kb_words %d too small for %d keys",
                    mask_words, kb_words, pos + n);
    DeviceGuard dg(c->device);
    qw::QsaKeyBitsArgs a{mask, key_bits, mask_words, kb_words, pos, n, cr};
    HIP_TRY(c, qw::launch_qsa_key_bits(a, (hipStream_t)stream));
    return QWATTN_OK;
}

}  // extern "C"
