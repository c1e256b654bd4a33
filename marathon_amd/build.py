"""In-tree build of the HIP library (gfx950 only).

``python -m marathon_amd.build`` (or ``__graft_entry__.build()``) compiles
``csrc/kvshift.hip`` into ``_lib/libmarathon_kvshift.so`` with hipcc.  It always
recompiles: the build is a few seconds and a stale library is worse than a slow one.
:func:`build_test_libraries` compiles the GPU tests' own HIP helpers (``tests/hip``)
into ``tests/_lib`` with the same flags.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "kvshift.hip")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "_lib")
OUT = os.path.join(OUT_DIR, "libmarathon_kvshift.so")
TEST_SRC_DIR = os.path.join(ROOT, "tests", "hip")
TEST_OUT_DIR = os.path.join(ROOT, "tests", "_lib")

ARCH = "gfx950"

# -ffp-contract=off: the rotation is mul, mul, add with one rounding each (the
#   reference torch path's order); a fused multiply-add would change the low bits.
# -fno-gpu-flush-denormals-to-zero: bf16/fp32 denormals must survive like on the CPU.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 anywhere in this library.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(src: str, out: str, verbose: bool, extra: list | None = None) -> str:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *(extra or []), f"-I{INCLUDE}",
           f"-I{os.path.join(HERE, 'csrc')}", src, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is
    # expected and harmless, everything else is shown
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    os.replace(tmp, out)
    return out


#: Extra preprocessor definitions for the library's compile-time tuning knobs (the
#: ``MKV_*`` macros at the top of ``csrc/kvshift.hip``), space-separated ``NAME=VALUE``
#: pairs, e.g. ``MARATHON_KVSHIFT_DEFINES="MKV_STORE_CPOL=2 MKV_PASSES_2B=2"``: a build
#: for an A/B of a default.  Empty: the defaults.
DEFINES_ENV = "MARATHON_KVSHIFT_DEFINES"
DEFINES_FILE = os.path.join(OUT_DIR, "build_defines.txt")


def build_library(verbose: bool = False) -> str:
    extra = [f"-D{d}" for d in os.environ.get(DEFINES_ENV, "").split() if d]
    for d in extra:
        if not d[2:].startswith("MKV_"):
            raise ValueError(f"{DEFINES_ENV}: {d[2:]!r} is not an MKV_ tuning knob")
    out = _compile(SRC, OUT, verbose, extra)
    # beside the library, what it was built with (bench.py reports it)
    with open(DEFINES_FILE, "w") as f:
        f.write(" ".join(d[2:] for d in extra) + "\n")
    return out


def _compile_c_host(src: str, out: str, verbose: bool) -> str:
    """A C host program against the library's C ABI and the HIP runtime, built by gcc
    (no HIP compiler involved: this is what an outside C caller does)."""
    os.makedirs(os.path.dirname(out), exist_ok=True)
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(hipcc())))
    rel = os.path.relpath(OUT_DIR, os.path.dirname(out))
    cmd = ["gcc", "-std=c11", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__",
           f"-I{os.path.join(rocm, 'include')}", f"-I{INCLUDE}", src, f"-L{OUT_DIR}",
           "-lmarathon_kvshift", f"-L{os.path.join(rocm, 'lib')}", "-lamdhip64", "-lm",
           f"-Wl,-rpath,$ORIGIN/{rel}", f"-Wl,-rpath,{os.path.join(rocm, 'lib')}",
           "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("gcc failed:\n" + res.stderr)
    os.replace(out + ".tmp", out)
    return out


def build_test_libraries(verbose: bool = False) -> list:
    """The GPU tests' own native helpers (test infrastructure only):
    ``tests/hip/<name>.hip`` -> ``tests/_lib/lib<name>.so`` and
    ``tests/c/<name>.c`` -> ``tests/_lib/<name>`` (C programs on the C ABI)."""
    outs = []
    if os.path.isdir(TEST_SRC_DIR):
        for fn in sorted(os.listdir(TEST_SRC_DIR)):
            if fn.endswith(".hip"):
                out = os.path.join(TEST_OUT_DIR, f"lib{fn[:-4]}.so")
                outs.append(_compile(os.path.join(TEST_SRC_DIR, fn), out, verbose))
    c_dir = os.path.join(ROOT, "tests", "c")
    if os.path.isdir(c_dir):
        for fn in sorted(os.listdir(c_dir)):
            if fn.endswith(".c"):
                out = os.path.join(TEST_OUT_DIR, fn[:-2])
                outs.append(_compile_c_host(os.path.join(c_dir, fn), out, verbose))
    return outs


if __name__ == "__main__":
    print(build_library(verbose=True))
    for path in build_test_libraries(verbose=True):
        print(path)
