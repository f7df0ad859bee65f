"""The C-ABI libraries load on a host without a GPU and export every entry
point declared in include/*.h (no compute calls here)."""
import ctypes as C
import os
import re

from conftest import ROOT

HEADERS = {"rina_hip.h": "hip", "rina_engine.h": "engine"}


def declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(rina_[a-z0-9_]+)\s*\(", src)))


def test_headers_declare_entry_points():
    assert "rina_hip_linear" in declared("rina_hip.h")
    assert "rina_hip_gqa_attention" in declared("rina_hip.h")
    assert "rina_infer_forward" in declared("rina_engine.h")


def test_libraries_export_declared_symbols(rina):
    libs = {"hip": rina.load_hip(), "engine": rina.load_engine()}
    for h, which in HEADERS.items():
        lib = libs[which]
        missing = [s for s in declared(h) if not hasattr(lib, s)]
        assert not missing, "%s: not exported: %s" % (h, missing)


def test_version_string(rina):
    v = rina.load_hip().rina_hip_version()
    assert b"gfx950" in v


def test_argument_errors_without_device(rina):
    # argument validation happens before any HIP call
    hip = rina.load_hip()
    assert hip.rina_hip_linear(None, 7, None, None, 1, 1, 32, None) == -1
    assert hip.rina_hip_linear(C.c_void_p(16), 99, C.c_void_p(16), C.c_void_p(16), 1, 1, 32, None) == -2
    assert hip.rina_hip_kv_quantize(9, C.c_void_p(16), C.c_void_p(16), 32, None) == -2
    assert hip.rina_hip_kv_quantize(1, C.c_void_p(16), C.c_void_p(16), 33, None) == -3
    assert hip.rina_hip_pack_weights(5, C.c_void_p(16), 31, C.c_void_p(16), None) == -3
    assert hip.rina_hip_kv_region_bytes(5, 1, 4096, 512) == 4096 * 16 * 6
    assert hip.rina_hip_kv_region_bytes(1, 0, 4096, 512) == 4096 * 16 * 34
    assert hip.rina_hip_kv_region_bytes(0, 0, 10, 512) == 10 * 512 * 4


def test_engine_config_errors(rina):
    eng = rina.load_engine()
    assert not eng.rina_model_create(b"{not json")
    m = eng.rina_model_create(b'{"name": "llama3.2-1b", "dim": 64, "layers": [{"type": "standard_attention"}]}')
    assert m
    eng.rina_model_destroy(m)
