"""Config 2 at its full shape: the Llama-3.2-1B-shaped Q4_0F model with an
fp32 KV cache, a 512-token seeded prompt, then 64 greedy steps.  The GPU
prefills and decodes (device loop, one graph per step); the CPU oracle
takes over the GPU's cache rows 0..511 and its first token (the oracle's
own 512-token prefill would take many minutes) and decodes the same 64
steps, which must give the same tokens."""
import ctypes as C
import importlib
import os

import numpy as np
import pytest

from _util import d2h, stream

pytestmark = pytest.mark.gpu

N_PROMPT = 512
STEPS = 64
MAX_SEQ = N_PROMPT + STEPS + 8


def test_config2_greedy_64_steps(rina, orc):
    synth = importlib.import_module("rina_amd.synth")
    sm = synth.SynthLlama(synth.LLAMA_1B, qt=rina.QT_Q4_0F, seed=1, max_seq=MAX_SEQ, keep_host=True)
    try:
        eng = rina.load_engine()
        c = sm.cfg
        L, kvd, V = c["n_layers"], c["n_kv_heads"] * c["head_dim"], c["vocab_size"]
        inf = sm.infer("fp32", MAX_SEQ)
        prompt = np.random.default_rng(3).integers(0, V, N_PROMPT).astype(np.int32)
        out = (C.c_int * (STEPS + 1))()
        rina.check(eng.rina_infer_generate(inf, prompt.ctypes.data_as(C.POINTER(C.c_int)), N_PROMPT, STEPS + 1, out,
                                           1, stream(), None), "generate")
        got = list(out)
        m, hold = orc.gqa_from_tensors(c, sm.host, sm.qt, MAX_SEQ, "fp32", min(os.cpu_count() or 1, 16))
        Lo = orc.load()
        keep = N_PROMPT * kvd * 4
        for layer in range(L):
            for which in (0, 1):
                ptr, nb = C.c_void_p(), C.c_size_t()
                rina.check(eng.rina_infer_kv_region(inf, layer, which, C.byref(ptr), C.byref(nb)), "region")
                cache = d2h(ptr.value, keep)
                onb = C.c_size_t()
                optr = Lo.orc_gqa_cache(m, layer, which, C.byref(onb))
                assert onb.value >= keep
                C.memmove(optr, cache.ctypes.data, keep)
        eng.rina_infer_destroy(inf)
        lg = np.zeros(V, np.float32)
        ref = []
        tok, pos = got[0], N_PROMPT
        for s in range(STEPS):
            t = np.array([tok], np.int32)
            assert Lo.orc_gqa_forward(m, t.ctypes.data, 1, pos, lg.ctypes.data, 1) == 0
            tok = Lo.orc_argmax(lg.ctypes.data, V)
            ref.append(tok)
            pos += 1
        Lo.orc_gqa_destroy(m)
        assert got[1:] == ref
    finally:
        sm.close()
