// The projections on either side of the attention layer for gfx950: Y[n][rows] = X[n][cols] W^T with W in
// planar Q8_0 (int8 weights, one f32 scale per 32 consecutive weights of a row) or plain f32 rows.
//
// Replaces Qwen4Vulkan::mat (src/qwen4_vk.cpp:848-856) on its matrix-vector pipelines q4_matmul_q8 /
// q4_matmul_f32 (shaders/q4_matmul.comp with the C_Q8 / C_F32 codecs of shaders/q4_codec.glsl; the planar
// repacking of GGUF Q8_0 is src/qwen4_vk.cpp:98-106) below 16 tokens, and on its tiled GEMM pipelines
// q4_gemm_q8 / q4_gemm_f32 from 16 (further down: a skinny MFMA kernel for Q8 up to 64 tokens, a tiled
// MFMA GEMM beyond): every output is the fp32 dot product of a dequantized
// weight row (int8 times its block's scale) with a token's input row, then optionally silu(y * post_scale).
//
// MI355X design of the matrix-vector kernels: the weights are read once per launch and are the bound (a
// decode step's projections are memory-bound); a wave owns RW rows and a workgroup NTP tokens (one for a single token), lane l covering the
// 16 consecutive columns 16 l + 1,024 k of every row, so a wave reads a kilobyte of each row per chunk in
// one 16-byte load a lane (plus one scale a lane pair), and every weight load of a wave's rows is issued
// before the first is used. A 16-column group never crosses a 32-weight block, so the lane applies its
// block scale once per group and token. The partial dot products are summed over the wave with DPP row
// operations and permlane swaps.
#include "common.hpp"
#include "kernels.hpp"

namespace qw {

namespace {

constexpr int kMatNTP = 4;  // tokens a workgroup

// Sum over the 64 lanes, in every lane.
__device__ __forceinline__ float mat_wave_sum(float x) {
    x = sum32(x);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// f32 weights: a wave's RW rows a 16-column group at a time (f32 projections are the small ones)
template <int NTP, int RW>
__device__ __forceinline__ void mat_f32_body(const MatArgs& a, int bx) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = (bx * 4 + wave) * RW;
    const int t0 = blockIdx.y * NTP;
    const int nt = min(NTP, a.n - t0);
    if (r0 >= a.rows) return;  // whole waves
    float acc[RW][NTP];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) acc[r][t] = 0.f;
    for (int c = lane * 16; c < a.cols; c += 1024) {
        float xv[NTP][16];
#pragma unroll
        for (int t = 0; t < NTP; t++) {
            const float* xr = a.x + (size_t)(t0 + (t < nt ? t : 0)) * a.x_stride + c;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xr + i);
                xv[t][i] = v[0], xv[t][i + 1] = v[1], xv[t][i + 2] = v[2], xv[t][i + 3] = v[3];
            }
        }
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const float* wr = static_cast<const float*>(a.w) + (size_t)min(r0 + r, a.rows - 1) * a.cols + c;
            float wv[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(wr + i);
                wv[i] = v[0], wv[i + 1] = v[1], wv[i + 2] = v[2], wv[i + 3] = v[3];
            }
#pragma unroll
            for (int t = 0; t < NTP; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[r][t] = __builtin_fmaf(wv[i], xv[t][i], acc[r][t]);
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) {
            float v = mat_wave_sum(acc[r][t]);
            if (a.post == 1) {
                const float u = v * a.post_scale;
                v = u / (1.0f + __expf(-u));
            }
            if (lane == 0 && r0 + r < a.rows && t < nt) a.y[(size_t)(t0 + t) * a.y_stride + r0 + r] = v;
        }
}

// planar Q8: every weight load of a batch of up to kMatK 1,024-column chunks (RW rows x kMatK 16-byte
// loads a lane, with their scales) is issued before any is used, so a wave has its whole share of the
// matrix in flight at once (the stream is the bound: the loads have to overlap); then per chunk the token
// rows' 16 columns (cached: every wave reads them) and the dot products
constexpr int kMatK = 4;
template <int NTP, int RW>
__device__ __forceinline__ void mat_q8_body(const MatArgs& a, int bx) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = (bx * 4 + wave) * RW;
    const int t0 = blockIdx.y * NTP;
    const int nt = min(NTP, a.n - t0);
    if (r0 >= a.rows) return;  // whole waves
    const int8_t* w8 = static_cast<const int8_t*>(a.w);
    const int nsb = a.cols >> 5;  // scales a row
    float acc[RW][NTP];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) acc[r][t] = 0.f;
    for (int cb = 0; cb < a.cols; cb += kMatK * 1024) {
        u32x4 q[RW][kMatK];
        float sc[RW][kMatK];
#pragma unroll
        for (int k = 0; k < kMatK; k++) {
            if (cb + k * 1024 >= a.cols) break;  // the whole chunk lies past the row (wave-uniform)
            const int c = min(cb + k * 1024 + lane * 16, a.cols - 16);  // past the row: a valid group, unused
#pragma unroll
            for (int r = 0; r < RW; r++) {
                const int row = min(r0 + r, a.rows - 1);  // past the last row: a valid row, result not stored
                q[r][k] = *reinterpret_cast<const u32x4*>(w8 + (size_t)row * a.cols + c);
                sc[r][k] = a.s[(size_t)row * nsb + (c >> 5)];
            }
        }
#pragma unroll
        for (int k = 0; k < kMatK; k++) {
            if (cb + k * 1024 >= a.cols) break;
            const int c = cb + k * 1024 + lane * 16;
            if (c >= a.cols) continue;  // this lane's group lies past the row
            float xv[NTP][16];
#pragma unroll
            for (int t = 0; t < NTP; t++) {
                const float* xr = a.x + (size_t)(t0 + (t < nt ? t : 0)) * a.x_stride + c;
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + i);
                    xv[t][i] = v[0], xv[t][i + 1] = v[1], xv[t][i + 2] = v[2], xv[t][i + 3] = v[3];
                }
            }
#pragma unroll
            for (int r = 0; r < RW; r++) {
                float wv[16];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int v = (int)q[r][k][j];
                    wv[4 * j] = (float)((v << 24) >> 24);
                    wv[4 * j + 1] = (float)((v << 16) >> 24);
                    wv[4 * j + 2] = (float)((v << 8) >> 24);
                    wv[4 * j + 3] = (float)(v >> 24);
                }
#pragma unroll
                for (int t = 0; t < NTP; t++) {
                    float d = 0.f;
#pragma unroll
                    for (int i = 0; i < 16; i++) d = __builtin_fmaf(wv[i], xv[t][i], d);
                    acc[r][t] = __builtin_fmaf(d, sc[r][k], acc[r][t]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int t = 0; t < NTP; t++) {
            float v = mat_wave_sum(acc[r][t]);
            if (a.post == 1) {
                const float u = v * a.post_scale;
                v = u / (1.0f + __expf(-u));
            }
            if (lane == 0 && r0 + r < a.rows && t < nt) a.y[(size_t)(t0 + t) * a.y_stride + r0 + r] = v;
        }
}

template <int NTP, int RW>
__global__ __launch_bounds__(256) void k_mat_q8(MatArgs a) {
    mat_q8_body<NTP, RW>(a, blockIdx.x);
}
template <int NTP, int RW>
__global__ __launch_bounds__(256) void k_mat_f32(MatArgs a) {
    mat_f32_body<NTP, RW>(a, blockIdx.x);
}

// Several matrices on one input in one launch: workgroups [wg_end[i-1], wg_end[i]) run matrix i (a
// wave-uniform choice), so a decode step's query, key and value projections stream as one burst.
template <bool Q8, int NTP, int RW>
__global__ __launch_bounds__(256) void k_mat_multi(MatMultiArgs a) {
    int i = 0;
    while (i + 1 < a.count && (int)blockIdx.x >= a.wg_end[i]) i++;
    const int bx = (int)blockIdx.x - (i ? a.wg_end[i - 1] : 0);
    if constexpr (Q8) mat_q8_body<NTP, RW>(a.m[i], bx);
    else mat_f32_body<NTP, RW>(a.m[i], bx);
}

// ---- many tokens: tiled MFMA GEMM ------------------------------------------------------------------
// Replaces the q4_gemm_q8 / q4_gemm_f32 pipelines (shaders/q4_gemm.comp) that Qwen4Vulkan::mat selects from
// nine tokens on (src/qwen4_vk.cpp:852-853). A workgroup owns a 128-row x BN-token tile of Y, walks the
// columns one 32-column step at a time (one Q8 block) through two LDS stages, and its four waves each own a
// 64-row x BN/2-token quarter as 4 x BN/32 v_mfma_f32_16x16x32_bf16 tiles (A = weight rows, B = token rows).
// fp32 accuracy from bf16 products: an int8 weight is exact in bf16, and an fp32 x is split into
// x_hi = bf16(x) and x_lo = bf16(x - x_hi), which leaves |x - x_hi - x_lo| <= 2^-18 |x|; a product's two
// MFMAs then carry it to within 2^-18 |w x| before the fp32 accumulation. Q8: each 32-column step's
// product (a fresh accumulator) is scaled by its rows' block scales into the running sum, as the reference
// applies the scale per block. f32 weights are split the same way (four MFMAs a tile: hi.hi, hi.lo,
// lo.hi, lo.lo). The next step's global loads are in flight while the current step's MFMAs run; tiles are
// assigned so that each XCD takes a contiguous range of row tiles (its weights stay in its L2).
constexpr int kGemmBM = 128;  // rows a workgroup
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Byte offset of 16-byte chunk g (k = 8 g .. 8 g + 7) of tile row r in an LDS tile of [rows][32] bf16: the
// chunk index is XORed with (r / 2) % 4, so any 8 consecutive rows' chunk g (an MFMA operand read) and any
// 4 rows' chunk pairs (the loaders' writes) land in 8 distinct 16-byte bank groups (no bank conflicts,
// counted by SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ int gemm_off(int r, int g) { return r * 64 + ((g ^ ((r >> 1) & 3)) << 4); }

__device__ __forceinline__ void split_bf16(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        hi[i] = (__bf16)v[i];
        lo[i] = (__bf16)(v[i] - (float)hi[i]);
    }
}

// ---- a few tokens (16 to a few hundred), Q8: skinny MFMA kernel ------------------------------------
// The tiled GEMM keeps too little in flight there (its 128-row tiles give the 8,192-row projection only 64
// workgroups below 32 tokens). Here a workgroup owns 32 rows x 16 tokens and its four waves split the
// columns; a wave loads its weights straight from HBM in the MFMA operand layout (lane (c, g): row c, the
// 8 columns 8 g .. 8 g + 7 of a 32-column block, one 8-byte load), kSkK blocks at a time, all issued before
// the first is used, with the token rows (fp32, split into bf16 hi / lo as in the GEMM) and the block
// scales of its accumulator rows. Per block and 16-row tile: two MFMAs (hi, lo) into a fresh accumulator,
// scaled into the running sum. The four waves' sums meet in LDS.
constexpr int kSkinnyMaxN = 64;  // token counts the skinny kernel takes (from 16)
constexpr int kSkinnyMaxRows = 1024;         // row counts it takes at any token count
// TT 16-token tiles a workgroup, KK blocks a batch
template <int TT, int KK>
__global__ __launch_bounds__(256) void k_mat_skinny(MatArgs a) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __shared__ f32x4 s_acc[3][2][TT][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int r0 = blockIdx.x * 32, t0 = blockIdx.y * 16 * TT;
    const int nkb = a.cols >> 5;
    const int kb0 = wave * nkb / 4, kb1 = (wave + 1) * nkb / 4;  // this wave's blocks
    const int8_t* w8 = static_cast<const int8_t*>(a.w);
    const size_t arow[2] = {(size_t)min(r0 + c, a.rows - 1) * a.cols, (size_t)min(r0 + 16 + c, a.rows - 1) * a.cols};
    int srow[2][4];  // accumulator rows of this lane: 16 m + 4 g + i
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) srow[m][i] = min(r0 + 16 * m + 4 * g + i, a.rows - 1);
    const float* xrow[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) xrow[t] = a.x + (size_t)min(t0 + 16 * t + c, a.n - 1) * a.x_stride + 8 * g;
    f32x4 acc[2][TT];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kb = kb0; kb < kb1; kb += KK) {
        u32x2 wq[2][KK];
        f32x4 xv[KK][TT][2];
        float sc[2][4][KK];
#pragma unroll
        for (int j = 0; j < KK; j++) {
            const int b = min(kb + j, kb1 - 1);  // past this wave's range: a repeat, unused
#pragma unroll
            for (int m = 0; m < 2; m++) wq[m][j] = *reinterpret_cast<const u32x2*>(w8 + arow[m] + b * 32 + 8 * g);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                xv[j][t][0] = *reinterpret_cast<const f32x4*>(xrow[t] + b * 32);
                xv[j][t][1] = *reinterpret_cast<const f32x4*>(xrow[t] + b * 32 + 4);
            }
#pragma unroll
            for (int m = 0; m < 2; m++)
#pragma unroll
                for (int i = 0; i < 4; i++) sc[m][i][j] = a.s[(size_t)srow[m][i] * nkb + b];
        }
#pragma unroll
        for (int j = 0; j < KK; j++) {
            if (kb + j >= kb1) break;  // uniform
            bf16x8 av[2];
#pragma unroll
            for (int m = 0; m < 2; m++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int q = (int)wq[m][j][e / 4];
                    av[m][e] = (__bf16)(float)((q << (24 - 8 * (e % 4))) >> 24);
                }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                float v8[8] = {xv[j][t][0][0], xv[j][t][0][1], xv[j][t][0][2], xv[j][t][0][3],
                               xv[j][t][1][0], xv[j][t][1][1], xv[j][t][1][2], xv[j][t][1][3]};
                bf16x8 bh, bl;
                split_bf16(v8, bh, bl);
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[m], bh, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[m], bl, p, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[m][t][i] = __builtin_fmaf(sc[m][i][j], p[i], acc[m][t][i]);
                }
            }
        }
    }
    // the four waves' column ranges: sum in LDS, wave 0 writes (lane (c, g): token 16 t + c, rows 16 m + 4 g + i)
    if (wave > 0) {
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int t = 0; t < TT; t++) s_acc[wave - 1][m][t][lane] = acc[m][t];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const int tok = t0 + 16 * t + c;
#pragma unroll
            for (int m = 0; m < 2; m++) {
                f32x4 v = acc[m][t];
#pragma unroll
                for (int w = 0; w < 3; w++) v += s_acc[w][m][t][lane];  // waves 1..3 in order
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int row = r0 + 16 * m + 4 * g + i;
                    float y = v[i];
                    if (a.post == 1) {
                        const float u = y * a.post_scale;
                        y = u / (1.0f + __expf(-u));
                    }
                    if (tok < a.n && row < a.rows) a.y[(size_t)tok * a.y_stride + row] = y;
                }
            }
        }
    }
}

template <bool Q8, int BN>
__global__ __launch_bounds__(256, 2) void k_gemm(MatArgs a) {
    constexpr int NT = BN / 32;                      // 16-token tiles a wave (BN = 32, 64 or 128)
    constexpr int W_B = kGemmBM * 64;                // one bf16 weight plane of a stage
    constexpr int X_B = BN * 64;                     // one bf16 token plane
    constexpr int STAGE = (Q8 ? W_B + kGemmBM * 4 : 2 * W_B) + 2 * X_B;
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * STAGE];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int wr = wave & 1, wt = wave >> 1;

    const int RT = (a.rows + kGemmBM - 1) / kGemmBM, TT = (a.n + BN - 1) / BN, T = RT * TT;
    const int b = blockIdx.x;
    const int idx = (T & 7) ? b : (b & 7) * (T >> 3) + (b >> 3);  // XCD b % 8 takes tiles [x T/8, (x+1) T/8)
    const int r0 = (idx / TT) * kGemmBM, t0 = (idx % TT) * BN;
    const int nkb = a.cols >> 5;

    // loader roles: weight row lr (two threads a row, 16 columns each); token row lt
    const int lr = tid >> 1, lh = tid & 1;
    const size_t wrow = (size_t)min(r0 + lr, a.rows - 1);
    constexpr int XT = BN >= 64 ? 256 / BN : 4;       // threads a token row (2 or 4)
    constexpr int XC = 32 / XT;                       // columns a thread (16 or 8)
    const int lt = tid / XT, lq = tid % XT;
    const bool xl = BN * XT == 256 || tid < BN * XT;  // BN = 32: threads 0..127 load the token rows
    const float* xrow = a.x + (size_t)min(t0 + min(lt, BN - 1), a.n - 1) * a.x_stride + lq * XC;

    // one step's global data in registers
    struct Pre {
        u32x4 w;       // Q8: 16 int8 weights
        float f[16];   // f32: 16 weights
        float sc;      // Q8: block scale of row `tid` (threads 0..127)
        float x[XC];
    };
    auto load = [&](Pre& P, int kb) {
        const int k0 = kb * 32;
        if constexpr (Q8) {
            P.w = *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(a.w) + wrow * a.cols + k0 + 16 * lh);
            if (tid < kGemmBM) P.sc = a.s[(size_t)min(r0 + tid, a.rows - 1) * nkb + kb];
        } else {
            const float* wp = static_cast<const float*>(a.w) + wrow * a.cols + k0 + 16 * lh;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(wp + i);
                P.f[i] = v[0], P.f[i + 1] = v[1], P.f[i + 2] = v[2], P.f[i + 3] = v[3];
            }
        }
        if (xl) {
#pragma unroll
            for (int i = 0; i < XC; i += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xrow + k0 + i);
                P.x[i] = v[0], P.x[i + 1] = v[1], P.x[i + 2] = v[2], P.x[i + 3] = v[3];
            }
        }
    };
    auto store = [&](const Pre& P, int st) {
        unsigned char* S = smem + st * STAGE;
        if constexpr (Q8) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                bf16x8 v;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int q = (int)P.w[2 * h + j / 4];
                    v[j] = (__bf16)(float)((q << (24 - 8 * (j % 4))) >> 24);
                }
                *reinterpret_cast<bf16x8*>(S + gemm_off(lr, 2 * lh + h)) = v;
            }
            if (tid < kGemmBM) reinterpret_cast<float*>(S + W_B + 2 * X_B)[tid] = P.sc;
        } else {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float v8[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v8[j] = P.f[8 * h + j];
                bf16x8 hi, lo;
                split_bf16(v8, hi, lo);
                *reinterpret_cast<bf16x8*>(S + gemm_off(lr, 2 * lh + h)) = hi;
                *reinterpret_cast<bf16x8*>(S + W_B + 2 * X_B + gemm_off(lr, 2 * lh + h)) = lo;
            }
        }
#pragma unroll
        for (int h = 0; h < XC / 8; h++) {
            if (!xl) break;
            float v8[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v8[j] = P.x[8 * h + j];
            bf16x8 hi, lo;
            split_bf16(v8, hi, lo);
            const int gc = lq * (XC / 8) + h;
            *reinterpret_cast<bf16x8*>(S + W_B + gemm_off(lt, gc)) = hi;
            *reinterpret_cast<bf16x8*>(S + W_B + X_B + gemm_off(lt, gc)) = lo;
        }
    };

    f32x4 acc[4][NT];
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int st) {
        const unsigned char* S = smem + st * STAGE;
        bf16x8 A[4], Bh[NT], Bl[NT];
#pragma unroll
        for (int m = 0; m < 4; m++) A[m] = *reinterpret_cast<const bf16x8*>(S + gemm_off(wr * 64 + m * 16 + c, g));
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int r = wt * (BN / 2) + t * 16 + c;
            Bh[t] = *reinterpret_cast<const bf16x8*>(S + W_B + gemm_off(r, g));
            Bl[t] = *reinterpret_cast<const bf16x8*>(S + W_B + X_B + gemm_off(r, g));
        }
        if constexpr (Q8) {
            const float* sS = reinterpret_cast<const float*>(S + W_B + 2 * X_B);
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const f32x4 sc = *reinterpret_cast<const f32x4*>(sS + wr * 64 + m * 16 + 4 * g);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[m], Bh[t], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[m], Bl[t], p, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[m][t][i] = __builtin_fmaf(sc[i], p[i], acc[m][t][i]);
                }
            }
        } else {
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const bf16x8 Al = *reinterpret_cast<const bf16x8*>(S + W_B + 2 * X_B + gemm_off(wr * 64 + m * 16 + c, g));
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[m], Bh[t], acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[m], Bl[t], acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bh[t], acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bl[t], acc[m][t], 0, 0, 0);
                }
            }
        }
    };

    // stage kb % 2 holds step kb; step kb + 1's global loads are in flight while its MFMAs run, then
    // converted into the other stage (whose last readers passed the previous barrier)
    Pre P;
    load(P, 0);
    store(P, 0);
    __syncthreads();
    for (int kb = 0; kb < nkb; kb++) {
        if (kb + 1 < nkb) load(P, kb + 1);
        compute(kb & 1);
        if (kb + 1 < nkb) store(P, (kb + 1) & 1);
        __syncthreads();
    }

    // lane (c, g) holds rows 4 g .. 4 g + 3 of each tile for token c
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tok = t0 + wt * (BN / 2) + t * 16 + c;
        if (tok >= a.n) continue;
        float* yr = a.y + (size_t)tok * a.y_stride;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int row = r0 + wr * 64 + m * 16 + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = acc[m][t][i];
                if (a.post == 1) {
                    const float u = v * a.post_scale;
                    v = u / (1.0f + __expf(-u));
                }
                if (row + i < a.rows) yr[row + i] = v;
            }
        }
    }
}

}  // namespace

hipError_t launch_mat(const MatArgs& a, bool q8, hipStream_t s) {
    // the skinny kernel up to 64 tokens, at any token count for matrices of up to 1,024 rows, and wherever
    // the GEMM would have fewer than 256 tiles of 128 rows x 32 tokens (it would leave most CUs idle:
    // 512 x 2,048 at 2,048 tokens 51 -> 45 us, at 256 tokens 39 -> 26 us; 2,048 x 4,096 at 256 tokens
    // 89 -> 48 us)
    const int t32 = ((a.rows + kGemmBM - 1) / kGemmBM) * ((a.n + 31) / 32);
    if (q8 && a.n >= kGemmMinN && (a.n <= kSkinnyMaxN || a.rows <= kSkinnyMaxRows || t32 < 256) && a.cols % 32 == 0) {
        // 16 tokens a workgroup up to 16, 32 up to 32, then 64 (the weights re-read once per token group)
        const int tt = a.n <= 16 ? 1 : a.n <= 32 ? 2 : 4;
        const dim3 grid((a.rows + 31) / 32, (a.n + 16 * tt - 1) / (16 * tt));
        if (tt == 1) hipLaunchKernelGGL((k_mat_skinny<1, 8>), grid, dim3(256), 0, s, a);
        else if (tt == 2) hipLaunchKernelGGL((k_mat_skinny<2, 4>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_mat_skinny<4, 2>), grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    if (a.n >= kGemmMinN && a.cols % 32 == 0) {
        // the widest token tile that still gives two workgroups a CU (fewer weight re-reads), else the
        // narrowest (the most workgroups)
        const int rt = (a.rows + kGemmBM - 1) / kGemmBM;
        const auto tiles = [&](int bn) { return rt * ((a.n + bn - 1) / bn); };
        const int bn = tiles(128) >= 512 ? 128 : tiles(64) >= 512 ? 64 : 32;
        const dim3 grid(tiles(bn)), block(256);
        if (bn == 128) {
            if (q8) hipLaunchKernelGGL((k_gemm<true, 128>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_gemm<false, 128>), grid, block, 0, s, a);
        } else if (bn == 64) {
            if (q8) hipLaunchKernelGGL((k_gemm<true, 64>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_gemm<false, 64>), grid, block, 0, s, a);
        } else {
            if (q8) hipLaunchKernelGGL((k_gemm<true, 32>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_gemm<false, 32>), grid, block, 0, s, a);
        }
        return hipGetLastError();
    }
    // matrix-vector: one token a workgroup for a decode step, else four; four rows a wave when that still
    // gives 256 workgroups a token group, else one (small matrices: more rows in flight at once)
    const int ntp = a.n == 1 ? 1 : kMatNTP;
    const bool rw4 = a.rows >= 4096;
    if ((a.n + ntp - 1) / ntp > 65535) return hipErrorInvalidConfiguration;  // grid y limit (f32, cols % 32 != 0)
    const dim3 grid((a.rows + (rw4 ? 15 : 3)) / (rw4 ? 16 : 4), (a.n + ntp - 1) / ntp), block(256);
    if (q8) {
        if (ntp == 1) {
            if (rw4) hipLaunchKernelGGL((k_mat_q8<1, 4>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_mat_q8<1, 1>), grid, block, 0, s, a);
        } else {
            if (rw4) hipLaunchKernelGGL((k_mat_q8<kMatNTP, 4>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_mat_q8<kMatNTP, 1>), grid, block, 0, s, a);
        }
    } else {
        if (ntp == 1) {
            if (rw4) hipLaunchKernelGGL((k_mat_f32<1, 4>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_mat_f32<1, 1>), grid, block, 0, s, a);
        } else {
            if (rw4) hipLaunchKernelGGL((k_mat_f32<kMatNTP, 4>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((k_mat_f32<kMatNTP, 1>), grid, block, 0, s, a);
        }
    }
    return hipGetLastError();
}

hipError_t launch_mat_multi(const MatMultiArgs& a0, bool q8, hipStream_t s) {
    const MatArgs& f = a0.m[0];
    if (f.n >= kGemmMinN && f.cols % 32 == 0) {  // the GEMM: one launch a matrix (each fills the chip)
        for (int i = 0; i < a0.count; i++) {
            const hipError_t e = launch_mat(a0.m[i], q8, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    MatMultiArgs a = a0;
    int rows = 0;
    for (int i = 0; i < a.count; i++) rows += a.m[i].rows;
    const int ntp = f.n == 1 ? 1 : kMatNTP;
    const bool rw4 = rows >= 4096;
    if ((f.n + ntp - 1) / ntp > 65535) return hipErrorInvalidConfiguration;  // grid y limit (f32, cols % 32 != 0)
    int wg = 0;
    for (int i = 0; i < a.count; i++) {
        wg += (a.m[i].rows + (rw4 ? 15 : 3)) / (rw4 ? 16 : 4);
        a.wg_end[i] = wg;
    }
    const dim3 grid(wg, (f.n + ntp - 1) / ntp), block(256);
#define QW_MULTI(Q, N, R) hipLaunchKernelGGL((k_mat_multi<Q, N, R>), grid, block, 0, s, a)
    if (q8) {
        if (ntp == 1) { if (rw4) QW_MULTI(true, 1, 4); else QW_MULTI(true, 1, 1); }
        else { if (rw4) QW_MULTI(true, kMatNTP, 4); else QW_MULTI(true, kMatNTP, 1); }
    } else {
        if (ntp == 1) { if (rw4) QW_MULTI(false, 1, 4); else QW_MULTI(false, 1, 1); }
        else { if (rw4) QW_MULTI(false, kMatNTP, 4); else QW_MULTI(false, kMatNTP, 1); }
    }
#undef QW_MULTI
    return hipGetLastError();
}

}  // namespace qw
