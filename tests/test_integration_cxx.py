"""The drop-in boundary from C++: include/qwattn.hpp (the throwing wrapper) and the reference-side binding
tests/cxx/hip_backend.cpp compile — against the wrapper alone and, where the reference sources are
present, against the reference's own Backend / Q4Config headers (src/backend.h:9-41, src/qwen4.h:22-25) —
and a C++ caller (tests/cxx/layer_driver.cpp) runs the layer attention through the wrapper: on a machine
without a GPU its context creation throws qwattn::Error; on the GPU its outputs over a prefill chunk, a
4-token verify pass and decode steps match the CPU oracle, and a pass past the context limit throws."""
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

from common import QWEN3_NEXT, assert_parity, projections

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CXX = os.path.join(ROOT, "tests", "cxx")
REF_SRC = "/root/reference/src"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
sys.path.insert(0, CXX)
import build as cxx_build  # noqa: E402


def _syntax(extra, std):
    cmd = ["g++", f"-std={std}", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"), *extra, os.path.join(CXX, "hip_backend.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("std", ["c++17", "c++20"])
def test_wrapper_compiles(std):
    _syntax([], std)


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "backend.h")), reason="reference sources not present")
def test_binding_compiles_against_reference_headers():
    """HipBackend : Backend overrides every pure virtual and uses Q4Config's own field names."""
    r = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-DQW_WITH_REFERENCE",
                        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"),
                        "-I", REF_SRC, os.path.join(CXX, "hip_backend.cpp")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def _driver():
    if not os.path.exists(cxx_build.OUT):
        cxx_build.build()
    return cxx_build.OUT


def _write_input(path, s, ns, seed=0):
    qg_all, k_all, v_all = [], [], []
    _, _, _, qn, kn = projections(seed, 1, s)
    with open(path, "wb") as f:
        f.write(struct.pack("<5i", s.NH, s.NKV, s.D, s.R, len(ns)))
        f.write(struct.pack(f"<{len(ns)}i", *ns))
        f.write(struct.pack("<2f", s.theta, s.eps))
        f.write(qn.astype("<f4").tobytes())
        f.write(kn.astype("<f4").tobytes())
        for i, n in enumerate(ns):
            if n < 0:  # a rollback entry carries no data
                qg_all.append(None), k_all.append(None), v_all.append(None)
                continue
            qg, k, v, _, _ = projections(seed + 10 + i, n, s)
            f.write(qg.astype("<f4").tobytes())
            f.write(k.astype("<f4").tobytes())
            f.write(v.astype("<f4").tobytes())
            qg_all.append(qg), k_all.append(k), v_all.append(v)
    return qg_all, k_all, v_all, qn, kn


def test_driver_throws_without_gpu(tmp_path):
    """No usable gfx950: qwattn_create fails and the wrapper turns the status into qwattn::Error."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    _write_input(inp, QWEN3_NEXT, [3, 1])
    r = subprocess.run([_driver(), str(inp), str(outp)], capture_output=True, text=True)
    assert r.returncode == 3, (r.returncode, r.stderr)
    assert "qwattn::Error" in r.stderr and "qwattn_create" in r.stderr


@pytest.mark.gpu
def test_driver_matches_oracle(oracle, tmp_path):
    s = QWEN3_NEXT
    ns = [300, 4, -2, 1, 1]  # prefill chunk, 1 + 3 drafts, accept(2) (two drafts rejected), then decode steps
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    qgs, ks, vs, qn, kn = _write_input(inp, s, ns, seed=5)
    print(f"layer_driver over {ns}", flush=True)
    r = subprocess.run([_driver(), str(inp), str(outp)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stderr)
    got = np.fromfile(outp, dtype="<f4")
    rows = sum(n for n in ns if n > 0)
    ref_k = np.zeros((rows, s.NKV, s.D), np.float32)
    ref_v = np.zeros((rows, s.NKV, s.D), np.float32)
    pos, off = 0, 0
    for i, n in enumerate(ns):
        if n < 0:  # rollback: the next pass rewrites the rejected rows
            pos += n
            continue
        rq, rk, rv = oracle.qk_norm_rope(qgs[i], ks[i], vs[i], 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
        ref_k[pos:pos + n] = rk[pos:pos + n].astype(np.float16)
        ref_v[pos:pos + n] = rv[pos:pos + n].astype(np.float16)
        ref = oracle.attention(rq, ref_k[:pos + n], ref_v[:pos + n], pos, qgs[i])
        out = got[off:off + n * s.NH * s.D].reshape(n, s.NH, s.D)
        assert_parity(out, ref, f"pass {i} pos={pos} n={n}")
        off += n * s.NH * s.D
        pos += n
