# Builds qwen3-local-test_amd/_build/timeline/libqwattn_timeline.so: libqwattn with a stamped copy of
# k_decode_ld (each wave writes s_memrealtime timestamps at the phase ends of the one-launch decode, plus its
# XCC and CU ids, into a device buffer that probe_set points to). Measurement tooling: the product library
# is built from the unmodified sources; this copy only serves run.py.
import os, subprocess, sys, concurrent.futures
ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
CSRC = os.path.join(ROOT, "qwen3-local-test_amd", "csrc")
OUT = os.path.join(ROOT, "qwen3-local-test_amd", "_build", "timeline")
os.makedirs(OUT, exist_ok=True)
src = open(os.path.join(CSRC, "decode.hip")).read()

def rep(old, new, cnt=1):
    global src
    assert src.count(old) == cnt, (old[:80], src.count(old))
    src = src.replace(old, new)

# global probe buffer + stamp helper
rep('namespace qw {\n\n// k_decode: a slice', '''namespace qw {
__device__ unsigned long long* g_probe;
// slot layout per wave: 32 u64
#define PSTAMP(k) do { const unsigned long long t_ = __builtin_amdgcn_s_memrealtime(); \
    const uint32_t a_ = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&s_stamp[threadIdx.x >> 6][(k)])); \
    asm volatile("ds_write_b64 %0, %1" :: "v"(a_), "v"(t_) : "memory"); } while (0)
#define PFLUSH() do { __syncthreads(); if (g_probe && (threadIdx.x & 63) < 32) g_probe[pbase + (threadIdx.x & 63)] = s_stamp[threadIdx.x >> 6][threadIdx.x & 63]; } while (0)

// k_decode: a slice''')
rep('''template <int D, int FUSED, int IN_DT, int QSA>
__global__ __launch_bounds__(256, 1) void k_decode_ld(DecodeArgs a) {''', '''template <int D, int FUSED, int IN_DT, int QSA>
__global__ __launch_bounds__(256, 1) void k_decode_ld(DecodeArgs a) {
    const size_t pbase = (((size_t)blockIdx.x * 4) + (threadIdx.x >> 6)) * 32;
    __shared__ unsigned long long s_stamp[4][32];
    if ((threadIdx.x & 63) < 32) s_stamp[threadIdx.x >> 6][threadIdx.x & 63] = 0;
    PSTAMP(0);
    if (g_probe && (threadIdx.x & 63) == 0) {
        const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);
        const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
        s_stamp[threadIdx.x >> 6][31] = ((unsigned long long)xcc << 32) | hw;
    }''')
# prologue barrier passed (the bare barrier before m_run init)
rep('''    asm volatile("" ::: "memory");

    float m_run = kNegInf, l_run = 0.f;
    f32x4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (loader) {''', '''    asm volatile("" ::: "memory");
    PSTAMP(1);

    float m_run = kNegInf, l_run = 0.f;
    f32x4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (loader) {''')
# loader: tile landed stamps (slots 8..23)
rep("""            asm volatile("ds_write_b32 %0, %1" ::"v"(raddr), "v"(i + 1) : "memory");""", """            asm volatile("ds_write_b32 %0, %1" ::"v"(raddr), "v"(i + 1) : "memory");
            if (i < 16) PSTAMP(8 + i);""")
rep("""            __hip_atomic_store(&freed[wave], i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);""",
    """            __hip_atomic_store(&freed[wave], i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (i < 16) PSTAMP(8 + i);""")
rep("""        l_run += __shfl_xor(l_run, 16, 64);  // the column's sum over the lane groups""", """        { float s0 = acc[0][0]; asm volatile("" :: "v"(s0)); PSTAMP(2); }
        l_run += __shfl_xor(l_run, 16, 64);  // the column's sum over the lane groups""")
rep("""        m_run = M, l_run = L;
    }
""", """        m_run = M, l_run = L;
        PSTAMP(3);
    }
""")
rep("""                                                   rr, row * 16, 0, kScDevice);
        }
    }
}""", """                                                   rr, row * 16, 0, kScDevice);
        }
        PSTAMP(4);
    }
    PFLUSH();
}""")
rep('void combine_row(const DecodeArgs& a, unsigned char* smem, int r) {', 'void combine_row(const DecodeArgs& a, unsigned char* smem, int r, size_t pbase, unsigned long long (*s_stamp)[32]) {')
rep('combine_row<D, IN_DT>(a, smem, blockIdx.x);', 'combine_row<D, IN_DT>(a, smem, blockIdx.x, pbase, s_stamp);\n            PFLUSH();')
rep("""        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        // the group's max and weights""", """        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        if (wb == 0) PSTAMP(5);
        // the group's max and weights""")
rep("""        *reinterpret_cast<fDL*>(&s_go[wave * D + lane * DL]) = og;""", """        *reinterpret_cast<fDL*>(&s_go[wave * D + lane * DL]) = og;
        if (wb == 0) PSTAMP(6);""")
rep("""    if (tid < D) a.out[((size_t)t * a.NH + h) * D + tid] = (L > 0.f ? O / L : 0.f) * sigmoid(gate);""", """    if (tid < D) a.out[((size_t)t * a.NH + h) * D + tid] = (L > 0.f ? O / L : 0.f) * sigmoid(gate);
    PSTAMP(7);
    if (lane == 0) s_stamp[wave][30] = spins;""")
src += '''
extern "C" int probe_set(void* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(qw::g_probe), &buf, sizeof(buf));
}
'''
open(os.path.join(OUT, "decode.hip"), "w").write(src)
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", CSRC]
def cc(path):
    obj = os.path.join(OUT, os.path.basename(path) + ".o")
    r = subprocess.run(["/opt/rocm/bin/hipcc", *FLAGS, "-x", "hip", "-c", path, "-o", obj], capture_output=True, text=True)
    if r.returncode:
        print(r.stderr[-3000:]); sys.exit(1)
    return obj
srcs = [os.path.join(OUT, "decode.hip")] + [os.path.join(CSRC, f) for f in ("norm_rope.hip", "prefill.hip", "qsa.hip", "mat.hip", "qwattn.cpp")]
with concurrent.futures.ThreadPoolExecutor(4) as ex:
    objs = list(ex.map(cc, srcs))
r = subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", os.path.join(OUT, "libqwattn_timeline.so")], capture_output=True, text=True)
if r.returncode:
    print(r.stderr); sys.exit(1)
print("built", os.path.join(OUT, "libqwattn_timeline.so"))
