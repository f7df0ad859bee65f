"""Config 3: the Llama-3.2-1B-shaped model at context 4096 with the KV cache
in q8, q4 and q2k_q1v.  The GPU prefills a 4032-token seeded prompt and
decodes 64 greedy steps (positions 4032..4095); every K/V row the model
appended is re-packed by the oracle and compared with the cache bytes
(bit-exact), and the oracle, started from those same cache rows and the
first generated token, decodes the same 64 tokens (its own prefill of 4032
tokens on the CPU would take hours; the first token comes from the
prefill, which attends over the fp32 rows, not the packed cache).  Every
step's top-2 logit margin must clear twice the 1e-5 tolerance."""
import ctypes as C
import importlib
import os

import numpy as np
import pytest

from _util import REL_TOL, d2h, stream

pytestmark = pytest.mark.gpu

N_PROMPT = 4032
STEPS = 65          # the prefill's token, then 64 decode steps
MAX_SEQ = 4104


@pytest.fixture(scope="module")
def llama(rina):
    synth = importlib.import_module("rina_amd.synth")
    sm = synth.SynthLlama(synth.LLAMA_1B, qt=rina.QT_Q4_0F, seed=1, max_seq=MAX_SEQ, keep_host=True)
    yield sm
    sm.close()


@pytest.mark.parametrize("kv_mode", ["q8", "q4", "q2k_q1v"])
def test_ctx4096_packs_and_greedy(rina, orc, llama, kv_mode):
    import torch
    eng = rina.load_engine()
    c = llama.cfg
    L, kvd, S, V = c["n_layers"], c["n_kv_heads"] * c["head_dim"], MAX_SEQ, c["vocab_size"]
    inf = llama.infer(kv_mode, MAX_SEQ)
    tap = torch.zeros(L * 2 * S * kvd, dtype=torch.float32, device="cuda")
    rina.check(eng.rina_infer_set_kv_tap(inf, tap.data_ptr()), "tap")
    prompt = np.random.default_rng(3).integers(0, V, N_PROMPT).astype(np.int32)
    out = (C.c_int * STEPS)()
    rina.check(eng.rina_infer_generate(inf, prompt.ctypes.data_as(C.POINTER(C.c_int)), N_PROMPT, STEPS, out, 1,
                                       stream(), None), "generate")
    got = list(out)
    tp = tap.cpu().numpy().reshape(L, 2, S, kvd)
    kf, vf = orc.kv_mode_formats(orc.KV_MODES[kv_mode])
    m, hold = orc.gqa_from_tensors(c, llama.host, llama.qt, MAX_SEQ, kv_mode, min(os.cpu_count() or 1, 16))
    Lo = orc.load()
    for layer in range(L):
        for which, fmt in ((0, kf), (1, vf)):
            ptr, nb = C.c_void_p(), C.c_size_t()
            rina.check(eng.rina_infer_kv_region(inf, layer, which, C.byref(ptr), C.byref(nb)), "region")
            cache = d2h(ptr.value, nb.value)
            want = orc.kv_quantize(fmt, tp[layer, which, :N_PROMPT])
            assert np.array_equal(cache[: want.size], want), "pack layer %d %s" % (layer, "V" if which else "K")
            # the oracle continues from the same cache rows 0..n-1
            onb = C.c_size_t()
            optr = Lo.orc_gqa_cache(m, layer, which, C.byref(onb))
            keep = N_PROMPT * (kvd // 32) * orc.kv_block_bytes(fmt)
            C.memmove(optr, cache.ctypes.data, keep)
    eng.rina_infer_destroy(inf)
    lg = np.zeros(V, np.float32)
    ref, margins = [], []
    tok, pos = got[0], N_PROMPT
    for s in range(STEPS - 1):
        t = np.array([tok], np.int32)
        assert Lo.orc_gqa_forward(m, t.ctypes.data, 1, pos, lg.ctypes.data, 1) == 0
        top = np.argsort(lg)[::-1][:2]
        margins.append(float(lg[top[0]] - lg[top[1]]) / float(np.max(np.abs(lg))))
        tok = Lo.orc_argmax(lg.ctypes.data, V)
        ref.append(tok)
        pos += 1
    Lo.orc_gqa_destroy(m)
    assert got[1:] == ref, "first divergence at step %d" % next(i for i in range(STEPS - 1) if got[1 + i] != ref[i])
    assert min(margins) > 2 * REL_TOL, "near tie at step %d (%.2e)" % (int(np.argmin(margins)), min(margins))
    assert len(set(got)) >= 16
