"""The engine's Layer / Inference ABI keeps the reference's shape
(rina-engine/src/core/layer.h:50-57, infer/infer_base.h:10-22): a
translation unit written the reference's way (six-slot vtable initializer,
void forward) compiles against the engine headers, links the engine
library and runs on the CPU."""
import os
import subprocess

import pytest

from conftest import PKG_DIR, ROOT, load_pkg


def test_reference_shaped_layer_and_inference(tmp_path):
    rina = load_pkg()
    rina.load_engine()   # built
    lib = os.path.join(PKG_DIR, "lib")
    exe = str(tmp_path / "ref_shaped")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(PKG_DIR, "csrc", "engine"), "-I", os.path.join(rocm, "include"),
           os.path.join(ROOT, "tests", "abi", "ref_shaped_engine.cpp"), "-o", exe, "-L", lib, "-lrina_engine",
           "-Wl,-rpath," + lib]
    c = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert c.returncode == 0, c.stdout
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 0 and "ref-shaped ABI ok" in r.stdout, r.stdout
