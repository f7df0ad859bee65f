"""A model written as .rinn (the converter's layout) and read back by the
engine's loader (rina_model_load, loader.cpp:14-152) runs exactly as the
model registered tensor by tensor: the same logits bit for bit and the same
greedy tokens, and its tensors are the written bytes."""
import ctypes as C
import importlib

import numpy as np
import pytest

from _util import d2h, empty, host, stream

pytestmark = pytest.mark.gpu

TINY = dict(name="llama-tiny", dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, hidden_dim=512,
            vocab_size=1000, rope_theta=500000.0)


def run(rina, eng, model, prompt, steps):
    import torch
    inf = eng.rina_infer_create(model, b"gqa", b"fp32", 64)
    assert inf, eng.rina_engine_last_error().decode()
    ids = torch.tensor(prompt, dtype=torch.int32, device="cuda")
    lg = empty(len(prompt) * TINY["vocab_size"])
    rina.check(eng.rina_infer_forward(inf, ids.data_ptr(), lg.data_ptr(), 1, len(prompt), 0, stream()), "forward")
    logits = host(lg)
    out = (C.c_int * steps)()
    p = (C.c_int * len(prompt))(*prompt)
    rina.check(eng.rina_infer_generate(inf, p, len(prompt), steps, out, 1, stream(), None), "generate")
    eng.rina_infer_destroy(inf)
    return logits, list(out)


@pytest.mark.parametrize("qt", [5, 7])
@pytest.mark.parametrize("as_dir", [False, True])
def test_rinn_round_trip(rina, tmp_path, qt, as_dir):
    synth = importlib.import_module("rina_amd.synth")
    eng = rina.load_engine()
    sm = synth.SynthLlama(TINY, qt=qt, seed=11, max_seq=64, keep_host=True)
    try:
        path = tmp_path / "weights.rinn"
        sm.save_rinn(str(path))
        m = eng.rina_model_load(str(tmp_path if as_dir else path).encode())
        assert m, eng.rina_engine_last_error().decode()
        try:
            prompt = [3, 14, 15, 92, 65, 35]
            lg_a, tok_a = run(rina, eng, sm.model, prompt, 12)
            lg_b, tok_b = run(rina, eng, m, prompt, 12)
            assert np.array_equal(lg_a.view(np.uint32), lg_b.view(np.uint32))
            assert tok_a == tok_b
        finally:
            eng.rina_model_destroy(m)
    finally:
        sm.close()
