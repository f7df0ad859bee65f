"""End-to-end parity of the C++ engine (Inference "gqa") on the GPU against
the CPU oracle model: logits (1e-5 relative), greedy token identity, and
bit-exact KV packs of the rows the model appended (config 3's check)."""
import ctypes as C
import importlib

import numpy as np
import pytest

from _util import assert_close, d2h, empty, host, stream

pytestmark = pytest.mark.gpu

TINY = dict(name="llama-tiny", dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, hidden_dim=512,
            vocab_size=1000, rope_theta=500000.0)


def synth(rina):
    return importlib.import_module("rina_amd.synth")


def oracle_for(orc, sm, kv_mode, nthreads=0):
    """CPU oracle model over the same (downloaded) packed tensors."""
    return orc.gqa_from_tensors(sm.cfg, sm.host, sm.qt, sm.max_seq, kv_mode, nthreads)


def gen_gpu(rina, sm, kv_mode, prompt, steps, use_graph):
    eng = rina.load_engine()
    inf = sm.infer(kv_mode)
    out = (C.c_int * steps)()
    p = (C.c_int * len(prompt))(*prompt)
    ms = C.c_float()
    rina.check(eng.rina_infer_generate(inf, p, len(prompt), steps, out, 1 if use_graph else 0, stream(),
                                       C.byref(ms)), "generate")
    eng.rina_infer_destroy(inf)
    return list(out)


@pytest.fixture(scope="module")
def tiny(rina):
    sm = synth(rina).SynthLlama(TINY, qt=rina.QT_Q4_0F, seed=3, max_seq=128, keep_host=True)
    yield sm
    sm.close()


def test_forward_logits_all_rows(rina, orc, tiny):
    eng = rina.load_engine()
    inf = tiny.infer("fp32")
    ids = np.array([5, 17, 3, 999, 42, 7], np.int32)
    import torch
    idd = torch.from_numpy(ids).cuda()
    lg = empty(len(ids) * 1000)
    rina.check(eng.rina_infer_forward(inf, idd.data_ptr(), lg.data_ptr(), 1, len(ids), 0, stream()), "forward")
    got = host(lg).reshape(len(ids), 1000)
    m, hold = oracle_for(orc, tiny, "fp32")
    ref = np.zeros((len(ids), 1000), np.float32)
    assert orc.load().orc_gqa_forward(m, ids.ctypes.data, len(ids), 0, ref.ctypes.data, 0) == 0
    assert_close(got, ref, what="prefill logits")
    # one decode step at host position 6
    nxt = np.array([11], np.int32)
    nd = torch.from_numpy(nxt).cuda()
    rina.check(eng.rina_infer_forward(inf, nd.data_ptr(), lg.data_ptr(), 1, 1, 6, stream()), "decode")
    ref1 = np.zeros(1000, np.float32)
    orc.load().orc_gqa_forward(m, nxt.ctypes.data, 1, 6, ref1.ctypes.data, 0)
    assert_close(host(lg)[:1000], ref1, what="decode logits")
    orc.load().orc_gqa_destroy(m)
    eng.rina_infer_destroy(inf)


@pytest.mark.parametrize("kv_mode", ["fp32", "q8", "q4", "q4k_q2v", "q2", "q2k_q1v"])
def test_greedy_tokens_identical(rina, orc, tiny, kv_mode):
    prompt = [3, 141, 59, 265, 358, 979, 323, 846]
    steps = 24
    got = gen_gpu(rina, tiny, kv_mode, prompt, steps, use_graph=True)
    m, hold = oracle_for(orc, tiny, kv_mode)
    p = np.array(prompt, np.int32)
    ref = np.zeros(steps, np.int32)
    assert orc.load().orc_gqa_generate(m, p.ctypes.data, len(prompt), steps, ref.ctypes.data) == 0
    orc.load().orc_gqa_destroy(m)
    assert got == list(ref)
    assert gen_gpu(rina, tiny, kv_mode, prompt, steps, use_graph=False) == got


@pytest.mark.parametrize("kv_mode", ["q8", "q4", "q2k_q1v"])
def test_kv_pack_bitexact_from_model(rina, orc, tiny, kv_mode):
    """Config 3's check on the tiny model: K/V rows produced by the model are
    re-packed by the oracle and compared with the cache bytes."""
    import torch
    eng = rina.load_engine()
    inf = tiny.infer(kv_mode)
    c = tiny.cfg
    L, kvd, S = c["n_layers"], c["n_kv_heads"] * c["head_dim"], tiny.max_seq
    tap = torch.zeros(L * 2 * S * kvd, dtype=torch.float32, device="cuda")
    rina.check(eng.rina_infer_set_kv_tap(inf, tap.data_ptr()), "tap")
    ids = [7, 8, 9, 10, 11]
    idd = torch.tensor(ids + [0] * 20, dtype=torch.int32, device="cuda")
    lg = empty(len(ids) * 1000)
    rina.check(eng.rina_infer_forward(inf, idd.data_ptr(), lg.data_ptr(), 1, len(ids), 0, stream()), "prefill")
    pos = len(ids)
    for _ in range(6):   # host-driven decode loop of main.cpp:666-690
        nxt = int(np.argmax(host(lg).reshape(-1, 1000)[-1]))
        idd[pos] = nxt
        rina.check(eng.rina_infer_forward(inf, idd.data_ptr() + 4 * pos, lg.data_ptr(), 1, 1, pos, stream()), "step")
        pos += 1
    tp = host(tap).reshape(L, 2, S, kvd)
    kf, vf = orc.kv_mode_formats(orc.KV_MODES[kv_mode])
    for layer in range(L):
        for which, fmt in ((0, kf), (1, vf)):
            ptr, nb = C.c_void_p(), C.c_size_t()
            rina.check(eng.rina_infer_kv_region(inf, layer, which, C.byref(ptr), C.byref(nb)), "region")
            cache = d2h(ptr.value, nb.value)
            rows = tp[layer, which, :pos]
            want = orc.kv_quantize(fmt, rows)
            assert np.array_equal(cache[: want.size], want), "layer %d %s" % (layer, "V" if which else "K")
    eng.rina_infer_destroy(inf)


def test_graph_recaptured_after_buffer_growth(rina):
    """A decode graph captured at one activation capacity must not be
    replayed after a longer prompt re-allocates the activations: generate
    with a short prompt (graph captured), then with a prompt past the
    512-row capacity on the same Inference; the tokens equal a fresh
    Inference's, and a prompt id outside the vocabulary is rejected before
    anything is launched."""
    eng = rina.load_engine()
    sm = synth(rina).SynthLlama(TINY, qt=rina.QT_Q4_0F, seed=5, max_seq=600)
    try:
        steps = 6
        short = [3, 1, 4, 1, 5, 9, 2, 6]
        long_prompt = list(np.random.default_rng(7).integers(0, TINY["vocab_size"], 530))
        inf = sm.infer("q8")
        out = (C.c_int * steps)()
        rina.check(eng.rina_infer_generate(inf, (C.c_int * len(short))(*short), len(short), steps, out, 1,
                                           stream(), None), "generate short")
        first = list(out)
        rina.check(eng.rina_infer_generate(inf, (C.c_int * len(long_prompt))(*long_prompt), len(long_prompt), steps,
                                           out, 1, stream(), None), "generate long")
        reused = list(out)
        bad = list(short)
        bad[3] = TINY["vocab_size"]
        assert eng.rina_infer_generate(inf, (C.c_int * len(bad))(*bad), len(bad), 2, out, 1, stream(), None) == -1
        assert "outside the vocabulary" in eng.rina_engine_last_error().decode()
        eng.rina_infer_destroy(inf)
        assert gen_gpu(rina, sm, "q8", long_prompt, steps, True) == reused
        assert gen_gpu(rina, sm, "q8", short, steps, True) == first
    finally:
        sm.close()
