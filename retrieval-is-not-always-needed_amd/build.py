"""Build the gfx950 HIP library, the C++ engine and the CPU oracle in-tree.

    lib/librina_hip.so     hand-written HIP kernels + the C-ABI of include/rina_hip.h
    lib/librina_engine.so  host C++ engine (ops / Layer / Inference), links librina_hip.so
    ../oracle/build/librina_oracle.so   CPU parity checker (tests only)

Run as a script or call build().  Every call recompiles (sources are few).
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INC = os.path.join(ROOT, "include")
HIP_SRC = os.path.join(PKG, "csrc", "hip")
ENG_SRC = os.path.join(PKG, "csrc", "engine")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    "-O3", "--offload-arch=gfx950", "-fPIC", "-std=c++17",
    # no packed fp32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-Wall", "-Wno-unused-function"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), out))
    return out


def _hip_objects(jobs):
    srcs = sorted(f for f in os.listdir(HIP_SRC) if f.endswith(".hip"))
    cmds = []
    for f in srcs:
        o = os.path.join(OBJ, f[:-4] + ".o")
        cmds.append(([os.path.join(ROCM, "bin", "hipcc")] + HIPCC_FLAGS +
                     ["-I", INC, "-I", HIP_SRC, "-c", os.path.join(HIP_SRC, f), "-o", o], o))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda c: _run(c[0]), cmds))
    return [o for _, o in cmds]


def _engine_objects(jobs):
    srcs = []
    for d, _, fs in os.walk(ENG_SRC):
        srcs += [os.path.join(d, f) for f in fs if f.endswith(".cpp")]
    srcs.sort()
    cmds = []
    for s in srcs:
        rel = os.path.relpath(s, ENG_SRC).replace(os.sep, "_")
        o = os.path.join(OBJ, "eng_" + rel[:-4] + ".o")
        cmds.append((["g++"] + CXX_FLAGS + ["-I", INC, "-I", ENG_SRC, "-I", os.path.join(ROCM, "include"),
                                            "-c", s, "-o", o], o))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda c: _run(c[0]), cmds))
    return [o for _, o in cmds]


def build_oracle():
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])


SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]


def build_sanitized(jobs=None):
    """AddressSanitizer + UBSan builds of the host code: the engine's C++
    (g++, no HIP sources; linked against the uninstrumented librina_hip.so)
    into _build/asan/librina_engine.so and the oracle into
    oracle/build/asan/librina_oracle.so.  Used by tests/test_sanitizers.py
    through RINA_ENGINE_SO / RINA_ORACLE_SO."""
    jobs = jobs or min(8, os.cpu_count() or 4)
    out = os.path.join(OBJ, "asan")
    os.makedirs(out, exist_ok=True)
    srcs = []
    for d, _, fs in os.walk(ENG_SRC):
        srcs += [os.path.join(d, f) for f in fs if f.endswith(".cpp")]
    srcs.sort()
    cmds = []
    for s in srcs:
        o = os.path.join(out, os.path.relpath(s, ENG_SRC).replace(os.sep, "_")[:-4] + ".o")
        cmds.append(["g++"] + CXX_FLAGS + SAN_FLAGS + ["-I", INC, "-I", ENG_SRC, "-I", os.path.join(ROCM, "include"),
                                                      "-c", s, "-o", o])
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_run, cmds))
    so = os.path.join(out, "librina_engine.so")
    _run(["g++", "-shared", "-fsanitize=address,undefined", "-o", so] + [c[-1] for c in cmds] +
         ["-L", LIB, "-lrina_hip", "-Wl,-rpath," + LIB, "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
          "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"])
    return so, os.path.join(ROOT, "oracle", "build", "asan", "librina_oracle.so")


def build(verbose=False, jobs=None):
    jobs = jobs or min(8, os.cpu_count() or 4)
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    hip_objs = _hip_objects(jobs)
    hip_so = os.path.join(LIB, "librina_hip.so")
    tmp = hip_so + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + hip_objs)
    os.replace(tmp, hip_so)
    eng_objs = _engine_objects(jobs)
    eng_so = os.path.join(LIB, "librina_engine.so")
    tmp = eng_so + ".tmp"
    _run(["g++", "-shared", "-o", tmp] + eng_objs +
         ["-L", LIB, "-lrina_hip", "-Wl,-rpath,$ORIGIN", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
          "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, eng_so)
    build_oracle()
    if verbose:
        print("built", hip_so, eng_so)
    return hip_so, eng_so


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
