"""Builds the gfx950 attention library libmx_attn.so in-tree with hipcc (no CUDA, no torch in the ABI)."""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libmx_attn.so")
SOURCES = ["api.hip", "decode.hip", "prefill.hip", "rope.hip", "small.hip", "linear.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: the compiler must not emit packed f32 arithmetic (its host pass warns that it does not know
# the feature; that warning is filtered below).
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Werror", "-Wno-unused-function",
    "-fvisibility=hidden",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    return r.returncode, "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)


def build(verbose: bool = False, out: str = LIB, defines=()) -> str:
    """Compiles every HIP source (one hipcc per source, in parallel) and links dooms_amd/libmx_attn.so; returns its
    path. Raises on a compile error. `out` and `defines` (extra -D macros) serve experiments that build variants."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = os.path.join(os.path.dirname(out), "_build", os.path.splitext(os.path.basename(out))[0])
    os.makedirs(objdir, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC, *[f"-D{d}" for d in defines]]
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    jobs = [[HIPCC, *compile_flags, *inc, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        results = list(ex.map(_run, jobs))
    msgs = "\n".join(m for _, m in results if m.strip())
    if any(rc != 0 for rc, _ in results):
        raise RuntimeError(f"hipcc failed:\n{msgs}")
    rc, msg = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", out + ".tmp"])
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{msg}")
    if verbose and (msgs + msg).strip():
        print(msgs + msg, file=sys.stderr)
    os.replace(out + ".tmp", out)
    return out


LIB_TRACE = os.path.join(os.path.dirname(LIB), "libmx_attn_trace.so")


def build_trace(verbose: bool = False) -> str:
    """The phase-trace variant of the library (MX_ATTN_TRACE: the decode kernel stamps its phases per workgroup and
    exports mx_attn_trace_read), used by `bench.py --trace-decode`; the product library compiles the stamps away."""
    return build(verbose=verbose, out=LIB_TRACE, defines=("MX_ATTN_TRACE=1",))


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


SAN_DIR = os.path.join(ROOT, "tests", "cpp", "_san")


def build_sanitized_abi_check() -> str:
    """The library's host code with AddressSanitizer and UndefinedBehaviorSanitizer (device code unchanged), linked
    into tests/cpp/abi_checks_sanitized.cpp's driver of every entry point's argument checks; returns the binary."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(SAN_DIR, exist_ok=True)
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
           "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all"]
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    compile_flags = [f for f in FLAGS if f not in ("-shared", "-fvisibility=hidden")]
    objs = [os.path.join(SAN_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    jobs = [[HIPCC, *compile_flags, *san, *inc, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
    driver = os.path.join(ROOT, "tests", "cpp", "abi_checks_sanitized.cpp")
    dobj = os.path.join(SAN_DIR, "driver.o")
    jobs.append([HIPCC, "-std=c++17", "-O1", "-g", *san, *inc, "-c", driver, "-o", dobj])
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        results = list(ex.map(_run, jobs))
    if any(rc != 0 for rc, _ in results):
        raise RuntimeError("hipcc failed:\n" + "\n".join(m for _, m in results))
    exe = os.path.join(SAN_DIR, "abi_checks_sanitized")
    rc, msg = _run([HIPCC, "--offload-arch=gfx950", "-fsanitize=address,undefined", *objs, dobj, "-o", exe])
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{msg}")
    return exe
