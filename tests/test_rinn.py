"""The .rinn format (rina-engine/src/loader.cpp:14-152 reads it,
tools/convert_llama_to_rinn.py:97-123 writes it): the package's writer
against an independent reader restated from loader.cpp, and the engine
reader's error paths (no device memory is touched before they fail)."""
import json
import os
import struct

import numpy as np
import pytest

from conftest import load_pkg

QT_Q4_0, QT_FP32, QT_Q4_0F = 5, 6, 7


def read_rinn(path):
    """Header, config and index as loader.cpp:19-26,90-103 read them."""
    with open(path, "rb") as f:
        raw = f.read()
    hdr = raw[:512]
    assert hdr[:4] == b"RINN"
    version, n_tensors = struct.unpack_from("<II", hdr, 4)
    cfg_off, cfg_sz, idx_off, idx_sz, data_off = struct.unpack_from("<5Q", hdr, 16)
    config = json.loads(raw[cfg_off:cfg_off + cfg_sz].decode())
    idx = raw[idx_off:idx_off + idx_sz]
    specs, p = [], 0
    while p < len(idx):
        (nl,) = struct.unpack_from("<H", idx, p)
        p += 2
        name = idx[p:p + nl].decode()
        p += nl
        shape = list(struct.unpack_from("<4i", idx, p))
        p += 16
        qt, bs, off, size = struct.unpack_from("<BHQQ", idx, p)
        p += 1 + 2 + 8 + 8
        specs.append(dict(name=name, shape=shape, qt=qt, block_size=bs, offset=off, size=size,
                          data=raw[off:off + size]))
    return dict(version=version, n_tensors=n_tensors, cfg_off=cfg_off, cfg_sz=cfg_sz, idx_off=idx_off,
                idx_sz=idx_sz, data_off=data_off, config=config, specs=specs, file_size=len(raw))


def sample_tensors():
    r = np.random.default_rng(3)
    q4 = r.integers(0, 256, 3 * 18, dtype=np.uint8)          # 3 Q4_0 blocks: a [2, 48] tensor
    q4f = r.integers(0, 256, 2 * 20, dtype=np.uint8)         # 2 Q4_0F blocks: [64]
    f32 = r.standard_normal((5, 7)).astype(np.float32)
    return [("transformer.wte.weight", (5, 7), QT_FP32, f32),
            ("transformer.h.0.attn.w_q.weight", (2, 48), QT_Q4_0, q4),
            ("transformer.h.0.mlp.w1.weight", (64,), QT_Q4_0F, q4f)]


def test_writer_layout(tmp_path):
    import importlib
    load_pkg()
    synth = importlib.import_module("rina_amd.synth")
    cfg = {"name": "llama-tiny", "dim": 7, "n_layers": 1, "block_size": 16, "layers": [{"type": "standard_attention"}]}
    tens = sample_tensors()
    path = str(tmp_path / "m.rinn")
    synth.write_rinn(path, cfg, tens)
    f = read_rinn(path)
    assert f["version"] == 1 and f["n_tensors"] == len(tens)
    assert f["cfg_off"] == 512 and f["idx_off"] == 512 + f["cfg_sz"]
    assert f["config"] == cfg
    # index entry size of the writer: 2 + name + 4*4 + 1 + 2 + 8 + 8
    assert f["idx_sz"] == sum(2 + len(n) + 35 for n, _, _, _ in tens)
    assert f["data_off"] % 256 == 0 and f["data_off"] >= f["idx_off"] + f["idx_sz"]
    assert f["data_off"] - (f["idx_off"] + f["idx_sz"]) < 256
    off = f["data_off"]
    for (name, shape, qt, data), sp in zip(tens, f["specs"]):
        assert sp["name"] == name and sp["qt"] == qt
        assert sp["shape"] == list(shape) + [0] * (4 - len(shape))
        assert sp["block_size"] == (32 if qt in (QT_Q4_0, QT_Q4_0F) else 1)
        assert sp["offset"] == off                                   # back to back, in order
        assert sp["data"] == np.ascontiguousarray(data).tobytes()
        off += sp["size"]
    assert off == f["file_size"]


def _write(path, cfg, tens, corrupt=None):
    import importlib
    load_pkg()
    synth = importlib.import_module("rina_amd.synth")
    synth.write_rinn(path, cfg, tens)
    if corrupt:
        with open(path, "r+b") as f:
            corrupt(f)


@pytest.mark.parametrize("case", ["missing", "magic", "index_count", "data_past_end", "qtype", "negative_dim",
                                  "zero_dim", "overflow"])
def test_load_errors(tmp_path, case):
    rina = load_pkg()
    eng = rina.load_engine()
    cfg = {"name": "llama-tiny", "dim": 7, "n_layers": 1, "layers": [{"type": "standard_attention"}]}
    tens = sample_tensors()
    path = str(tmp_path / "m.rinn")
    want = {"missing": "cannot open", "magic": "bad magic", "index_count": "tensor count",
            "data_past_end": "past the end", "qtype": "unsupported quant_type",
            "negative_dim": "non-positive or oversized", "zero_dim": "non-positive or oversized",
            "overflow": "non-positive or oversized"}[case]
    if case == "magic":
        _write(path, cfg, tens, lambda f: f.write(b"RINX"))
    elif case == "index_count":
        _write(path, cfg, tens, lambda f: (f.seek(8), f.write(struct.pack("<I", 9))))
    elif case == "data_past_end":
        # first tensor: fp32 [5, 7] claims a larger shape than its bytes in the file
        _write(path, cfg, [("transformer.wte.weight", (5000, 7000), QT_FP32, tens[0][3])] + tens[1:])
    elif case == "qtype":
        _write(path, cfg, [("transformer.h.0.x.weight", (256,), 10, np.zeros(84, np.uint8))] + tens)
    elif case == "negative_dim":
        # [-5, -7] has a positive product: the reader must look at each dim
        _write(path, cfg, [("transformer.wte.weight", (-5, -7), QT_FP32, tens[0][3])] + tens[1:])
    elif case == "zero_dim":
        _write(path, cfg, [("transformer.wte.weight", (5, 0, 7), QT_FP32, tens[0][3])] + tens[1:])
    elif case == "overflow":
        big = (1 << 31) - 1
        _write(path, cfg, [("transformer.wte.weight", (big, big, big, big), QT_FP32, tens[0][3])] + tens[1:])
    m = eng.rina_model_load(path.encode())
    assert not m
    assert want in eng.rina_engine_last_error().decode()


def test_load_directory_form_needs_weights_rinn(tmp_path):
    rina = load_pkg()
    eng = rina.load_engine()
    assert not eng.rina_model_load(str(tmp_path).encode())          # a directory without weights.rinn
    assert "weights.rinn" in eng.rina_engine_last_error().decode()


def _tiny_header(**kw):
    h = {"name": "llama-tiny", "dim": 64, "n_layers": 1, "n_heads": 2, "n_kv_heads": 1, "head_dim": 32,
         "vocab_size": 50, "max_seq_len": 16, "hidden_dim": 128, "layers": [{"type": "standard_attention"}]}
    h.update(kw)
    return h


def _add_fake(eng, m, name, qt, shape):
    """Register a tensor at a fake device address: no kernel reads it on the
    CPU, the engine only borrows the pointer."""
    import ctypes as C
    shp = (C.c_int64 * len(shape))(*shape)
    return eng.rina_model_add_tensor(m, name.encode(), qt, len(shape), shp, C.c_void_p(0x1000))


def test_add_tensor_rejects_bad_shapes():
    import json
    eng = load_pkg().load_engine()
    m = eng.rina_model_create(json.dumps(_tiny_header()).encode())
    assert m
    try:
        for shape in ((-4, 16), (4, 0), (0,), (1 << 40, 1 << 20)):
            assert _add_fake(eng, m, "transformer.wte.weight", QT_FP32, shape) == -1
            assert "shape" in eng.rina_engine_last_error().decode()
        assert _add_fake(eng, m, "transformer.wte.weight", QT_FP32, (50, 64)) == 0
    finally:
        eng.rina_model_destroy(m)


@pytest.mark.parametrize("bad", [None, "transformer.h.0.attn.w_k.weight", "transformer.h.0.mlp.w2.weight",
                                 "transformer.h.0.attn.rope.cos", "transformer.wte.weight"])
def test_layer_init_checks_shapes(bad):
    """A tensor smaller than its config implies fails Inference init (the
    kernels would read past it); with every shape right, init gets past the
    layers and fails only at the device allocation (no GPU here)."""
    import json
    eng = load_pkg().load_engine()
    m = eng.rina_model_create(json.dumps(_tiny_header()).encode())
    d, H, Hkv, dh, hd, V, S = 64, 2, 1, 32, 128, 50, 16
    shapes = {"transformer.h.0.attn.w_q.weight": (H * dh, d), "transformer.h.0.attn.w_k.weight": (Hkv * dh, d),
              "transformer.h.0.attn.w_v.weight": (Hkv * dh, d), "transformer.h.0.attn.w_o.weight": (d, H * dh),
              "transformer.h.0.mlp.w1.weight": (hd, d), "transformer.h.0.mlp.w3.weight": (hd, d),
              "transformer.h.0.mlp.w2.weight": (d, hd), "transformer.h.0.ln1.weight": (d,),
              "transformer.h.0.ln2.weight": (d,), "transformer.h.0.attn.rope.cos": (S, dh // 2),
              "transformer.h.0.attn.rope.sin": (S, dh // 2), "transformer.wte.weight": (V, d),
              "transformer.ln_f.weight": (d,)}
    try:
        for name, shp in shapes.items():
            if name == bad:
                shp = (shp[0] - 1,) + tuple(shp[1:])
            qt = QT_FP32 if ("ln" in name or "rope" in name or "wte" in name) else 7
            assert _add_fake(eng, m, name, qt, shp) == 0
        inf = eng.rina_infer_create(m, b"gqa", b"fp32", 0)
        assert not inf
        msg = eng.rina_engine_last_error().decode()
        if bad is None:
            assert "allocation failed" in msg, msg
        elif bad == "transformer.wte.weight":
            assert "wte" in msg, msg
        else:
            assert "layer init failed" in msg, msg
    finally:
        eng.rina_model_destroy(m)
