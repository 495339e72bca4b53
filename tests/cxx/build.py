"""Builds the C++ callers of libqwattn (g++ with the HIP runtime API only; linked against the in-tree
libqwattn.so):
  tests/cxx/_build/layer_driver    the layer attention through include/qwattn.hpp
  tests/cxx/_build/backend_driver  HipBackend : Backend (hip_backend.cpp + backend_driver.cpp), compiled
                                   against the reference's own headers (src/backend.h, src/qwen4.h), so only
                                   where the reference sources are present; the binary travels with the tree"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "_build", "layer_driver")
BACKEND_OUT = os.path.join(HERE, "_build", "backend_driver")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
REF_SRC = "/root/reference/src"


def _link_flags():
    return ["-L", os.path.join(ROOT, "qwen3-local-test_amd", "lib"), "-lqwattn", "-L", os.path.join(ROCM, "lib"),
            "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../../qwen3-local-test_amd/lib", "-Wl,-rpath," + os.path.join(ROCM, "lib")]


def _run(cmd, what, out):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {what} failed:\n{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


def build():
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROCM, "include"), os.path.join(HERE, "layer_driver.cpp"), "-o", OUT + ".tmp",
           *_link_flags()]
    _run(cmd, "layer_driver", OUT)
    if os.path.exists(os.path.join(REF_SRC, "qwen4.h")):
        build_backend()
    return OUT


def build_backend():
    cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", "-DQW_WITH_REFERENCE",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"), "-I", REF_SRC,
           os.path.join(HERE, "hip_backend.cpp"), os.path.join(HERE, "backend_driver.cpp"), "-o", BACKEND_OUT + ".tmp",
           *_link_flags()]
    return _run(cmd, "backend_driver", BACKEND_OUT)


if __name__ == "__main__":
    print(build())
