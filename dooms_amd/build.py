"""Builds the gfx950 attention library libmx_attn.so in-tree with hipcc (no CUDA, no torch in the ABI)."""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libmx_attn.so")
SOURCES = ["api.hip", "decode.hip", "prefill.hip", "rope.hip", "linear.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: the compiler must not emit packed f32 arithmetic (its host pass warns that it does not know
# the feature; that warning is filtered below).
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Werror", "-Wno-unused-function",
    "-fvisibility=hidden",
]


def build(verbose: bool = False) -> str:
    """Compiles every HIP source into dooms_amd/libmx_attn.so; returns its path. Raises on a compile error."""
    cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           *[os.path.join(CSRC, s) for s in SOURCES], "-lhipblaslt", "-o", LIB + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{msg}")
    if verbose and msg.strip():
        print(msg, file=sys.stderr)
    os.replace(LIB + ".tmp", LIB)
    return LIB


TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_host_attention.cpp")
TEST_BIN = os.path.join(ROOT, "tests", "cpp", "test_host_attention")


def build_host_test() -> str:
    """Compiles the C++ host-layer test (tests/cpp) against libmx_attn.so and the CPU oracle (oracle/liboracle.so)."""
    oracle_dir = os.path.join(ROOT, "oracle")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall", "-Werror",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "host"), TEST_SRC,
           "-L", PKG, "-lmx_attn", "-L", oracle_dir, "-loracle",
           "-Wl,-rpath,$ORIGIN/../../dooms_amd", "-Wl,-rpath,$ORIGIN/../../oracle", "-o", TEST_BIN + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on the host test ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(TEST_BIN + ".tmp", TEST_BIN)
    return TEST_BIN


if __name__ == "__main__":
    print(build(verbose=True))
