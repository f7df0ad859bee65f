"""Config 4 at its full shape: the DeepSeek-V2-Lite-shaped MLA + MoE model
(27 layers, 64 experts top-6 + 2 shared, vocab 102400) with random zero-mean
Q2_K weights, a 2000-token seeded prompt, then 64 greedy steps at positions
2000..2063, which run the engine's decode graph for positions >= 256 (the
chunked latent attention).

The oracle cannot prefill 2000 DeepSeek tokens in minutes, so:
  * layer 0's 2000 latent records (RMSNorm(c_kv)*k_norm | RoPE(k_pe)), which
    depend only on the prompt, are recomputed with the oracle's primitives
    and compared with the GPU's (the prompt path at full shape);
  * the oracle takes over every layer's 2000 records (orc_mla_load_latent
    expands them through W_kv_b as its own forward would) and the GPU's
    first token, then decodes the same 64 steps.
Every step's top-2 logit margin must clear twice the 1e-5 tolerance, so the
identity is a stable requirement; the tokens must be varied (a degenerate
random model would emit one token forever) and the last step's logits
agree within 1e-5."""
import ctypes as C
import importlib
import os

import numpy as np
import pytest

from _util import REL_TOL, assert_close, d2h, empty, host, stream

pytestmark = pytest.mark.gpu

N_PROMPT = 2000
STEPS = 64
MAX_SEQ = N_PROMPT + STEPS + 8


def test_config4_greedy_64_steps_at_2000(rina, orc):
    import torch
    synth = importlib.import_module("rina_amd.synth")
    sm = synth.SynthDeepSeek(seed=1, max_seq=MAX_SEQ, keep_host=True)
    try:
        eng = rina.load_engine()
        c = sm.cfg
        L, V, d, dc, rope = c["n_layers"], c["vocab_size"], c["dim"], c["dc"], c["rope"]
        R = dc + rope
        nt = min(os.cpu_count() or 1, 16)
        inf = sm.infer(MAX_SEQ)
        prompt = np.random.default_rng(3).integers(0, V, N_PROMPT).astype(np.int32)
        out = (C.c_int * (STEPS + 1))()
        rina.check(eng.rina_infer_generate(inf, prompt.ctypes.data_as(C.POINTER(C.c_int)), N_PROMPT, STEPS + 1, out,
                                           1, stream(), None), "generate")
        got = list(out)
        recs = []
        for layer in range(L):
            ptr, nb = C.c_void_p(), C.c_size_t()
            rina.check(eng.rina_infer_kv_region(inf, layer, 0, C.byref(ptr), C.byref(nb)), "region")
            recs.append(d2h(ptr.value, N_PROMPT * R * 4).view(np.float32).reshape(N_PROMPT, R))
        Lo = orc.load()
        # layer 0's records from the oracle's primitives
        h0 = np.zeros((N_PROMPT, d), np.float32)
        wte = sm.host["transformer.wte.weight"]
        Lo.orc_embedding(wte.ctypes.data, 10, prompt.ctypes.data, h0.ctypes.data, N_PROMPT, d)
        ln1 = sm.host["transformer.h.0.ln1.weight"]
        Lo.orc_rms_norm(h0.ctypes.data, ln1.ctypes.data, N_PROMPT, d, np.float32(1e-5))
        kva = orc.linear(sm.host["transformer.h.0.attn.w_kv_a.weight"], 10, h0, R, d, nt)
        cn = np.ascontiguousarray(kva[:, :dc])
        kn = sm.host["transformer.h.0.attn.k_norm.weight"]
        Lo.orc_rms_norm(cn.ctypes.data, kn.ctypes.data, N_PROMPT, dc, np.float32(1e-5))
        kpe = np.ascontiguousarray(kva[:, dc:])
        cos, sin = sm.host["transformer.h.0.attn.rope_q.cos"], sm.host["transformer.h.0.attn.rope_q.sin"]
        for t in range(N_PROMPT):
            Lo.orc_rope_neox(kpe[t].ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, 1, rope, t)
        want0 = np.concatenate([cn, kpe], axis=1)
        row_err = np.max(np.abs(recs[0] - want0), axis=1) / np.maximum(np.max(np.abs(want0), axis=1), 1e-30)
        assert row_err.max() <= REL_TOL, "layer-0 record %d: %.3e" % (int(row_err.argmax()), row_err.max())
        # the oracle continues from the GPU's cache rows and first token
        m, hold = orc.mla_from_tensors(c, sm.host, sm.qts, MAX_SEQ, nt)
        for layer in range(L):
            assert Lo.orc_mla_load_latent(m, layer, np.ascontiguousarray(recs[layer]).ctypes.data, N_PROMPT) == 0
        lg = np.zeros(V, np.float32)
        ref, margins = [], []
        tok, pos = got[0], N_PROMPT
        for s in range(STEPS):
            t = np.array([tok], np.int32)
            assert Lo.orc_mla_forward(m, t.ctypes.data, 1, pos, lg.ctypes.data, 1) == 0
            top = np.argsort(lg)[::-1][:2]
            margins.append(float(lg[top[0]] - lg[top[1]]) / float(np.max(np.abs(lg))))
            tok = Lo.orc_argmax(lg.ctypes.data, V)
            ref.append(tok)
            pos += 1
        Lo.orc_mla_destroy(m)
        assert got[1:] == ref, "first divergence at step %d" % next(i for i in range(STEPS) if got[1 + i] != ref[i])
        assert min(margins) > 2 * REL_TOL, "near tie at step %d (%.2e)" % (int(np.argmin(margins)), min(margins))
        assert len(set(got)) >= 16, "degenerate model: %d distinct tokens" % len(set(got))
        # the last step's logits: the GPU recomputes position N_PROMPT+STEPS-1
        ids = torch.tensor([got[STEPS - 1]], dtype=torch.int32, device="cuda")
        glg = empty(V)
        rina.check(eng.rina_infer_forward(inf, ids.data_ptr(), glg.data_ptr(), 1, 1, N_PROMPT + STEPS - 1, stream()),
                   "forward")
        assert_close(host(glg), lg, what="config-4 logits at position %d" % (N_PROMPT + STEPS - 1))
        eng.rina_infer_destroy(inf)
    finally:
        sm.close()
