"""Build recipes for libmtg.so (gfx950) and the oracle's liboracle.so.

hipcc compiles the HIP kernels and the host runtime for gfx950 only; packed FP32
instructions are disabled for the device pass. Outputs stay in-tree:
  moss-transcribe.cpp_amd/libmtg.so   (product)
  oracle/liboracle.so                  (test infrastructure)
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libmtg.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["kernels.hip", "kernels_wt.hip", "step_kernel.hip", "noalloc.hip", "prefill.hip", "prefill_wt.hip", "generate.hip", "encoder.hip", "runtime.cpp", "capi.cpp",
           "synth.cpp", "gguf.cpp", "reference_api.cpp"]
# -ffp-contract=off: elementwise ops round like the reference's scalar code;
# fused multiply-adds are written explicitly (fmaf) where they are wanted.
COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-pass-failed", "-Wno-unused-parameter", "-Wno-unused-value", "-Wno-unused-result",
          "--offload-arch=gfx950",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError("command failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build_lib(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    jobs = []
    for src in SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        cmd = [HIPCC] + COMMON + ["-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        jobs.append(cmd)
    with ThreadPoolExecutor(max_workers=4) as ex:
        outs = list(ex.map(_run, jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-pthread", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


CPP_TESTS = os.path.join(ROOT, "tests", "cpp")


def build_cpp_tests():
    """The C++ test drivers of the reference-named interface (tests/cpp), linked
    against libmtg.so; binaries go to tests/cpp/bin (git-ignored)."""
    out_dir = os.path.join(CPP_TESTS, "bin")
    os.makedirs(out_dir, exist_ok=True)
    outs = []
    for name in sorted(os.listdir(CPP_TESTS)):
        if not name.endswith(".cpp"):
            continue
        exe = os.path.join(out_dir, name[:-4])
        _run(["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "include"),
              os.path.join(CPP_TESTS, name), "-o", exe, "-L", PKG, "-lmtg",
              "-Wl,-rpath," + PKG, "-Wl,-rpath-link,/opt/rocm/lib"])
        outs.append(exe)
    return outs


def build_oracle():
    _run(["make", "-s", "-C", ORACLE_DIR, "liboracle.so"])
    return ORACLE_LIB


def build_all(verbose=False):
    build_lib(verbose)
    build_oracle()
    build_cpp_tests()


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", LIB, ORACLE_LIB)
