"""Builds tests/cxx/_build/layer_driver, the C++ caller of libqwattn through include/qwattn.hpp (g++ with
the HIP runtime API only; linked against the in-tree libqwattn.so)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "_build", "layer_driver")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build():
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROCM, "include"), os.path.join(HERE, "layer_driver.cpp"), "-o", OUT + ".tmp",
           "-L", os.path.join(ROOT, "qwen3-local-test_amd", "lib"), "-lqwattn", "-L", os.path.join(ROCM, "lib"),
           "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../../qwen3-local-test_amd/lib", "-Wl,-rpath," + os.path.join(ROCM, "lib")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building layer_driver failed:\n{r.stderr}")
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build())
