"""Build libgptoss_moe.so and libgptoss_attn.so in-tree for gfx950 (hipcc, no
JIT cache)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in any kernel.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]

SOURCES = [os.path.join(HERE, "csrc", "gptoss_moe.hip"), os.path.join(HERE, "csrc", "bin_loader.cpp")]
LIB = os.path.join(HERE, "libgptoss_moe.so")
ATTN_SOURCES = [os.path.join(HERE, "csrc", "gptoss_attn.hip"), os.path.join(HERE, "csrc", "gptoss_decoder.hip")]
ATTN_LIB = os.path.join(HERE, "libgptoss_attn.so")


# A C++ caller of the library and of the moe_gpu shim (csrc/moe_gpu_shim.hpp),
# run by tests/test_gpu_cpp_shim.py; links the in-tree library by rpath.
SHIM_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "moe_gpu_test.cpp")
SHIM_TEST_BIN = os.path.join(HERE, "bin", "moe_gpu_test")
# The same for the attention shim (csrc/attn_gpu_shim.hpp), run by
# tests/wip_gpu_attn.py.
ATTN_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "attn_gpu_test.cpp")
ATTN_TEST_BIN = os.path.join(HERE, "bin", "attn_gpu_test")


def _run(cmd, verbose):
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)


def build(verbose: bool = False) -> str:
    _run([HIPCC, *HIP_FLAGS, *SOURCES, "-o", LIB], verbose)
    _run([HIPCC, *HIP_FLAGS, *ATTN_SOURCES, "-o", ATTN_LIB], verbose)
    os.makedirs(os.path.dirname(SHIM_TEST_BIN), exist_ok=True)
    _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
          "-x", "hip", SHIM_TEST_SRC, "-L", HERE, "-lgptoss_moe",
          "-Wl,-rpath,$ORIGIN/..", "-o", SHIM_TEST_BIN], verbose)
    _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
          "-x", "hip", ATTN_TEST_SRC, "-L", HERE, "-lgptoss_attn",
          "-Wl,-rpath,$ORIGIN/..", "-o", ATTN_TEST_BIN], verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
