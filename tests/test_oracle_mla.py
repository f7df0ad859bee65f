"""Pin the CPU oracle's DeepSeek MLA + MoE path: router top-k properties and
a tiny model against a float64 numpy restatement (expanded attention)."""
import numpy as np

import _mla_tiny as mt


def test_moe_topk_properties(orc):
    r = np.random.default_rng(3)
    for trial in range(50):
        E, k = 64, 6
        lg = (r.standard_normal(E) * 2).astype(np.float32)
        ids, pr = orc.moe_topk(lg, k)
        p64 = np.exp(lg.astype(np.float64) - lg.max())
        p64 /= p64.sum()
        # the k largest probabilities, in ascending order, each within fp32 rounding of the softmax
        assert sorted(ids.tolist()) == sorted(np.argsort(-p64, kind="stable")[:k].tolist())
        assert np.all(np.diff(pr) >= 0)
        assert np.allclose(pr, p64[ids], rtol=1e-5, atol=0)
    # ties: equal logits -> the lower expert index is kept (strict ">")
    lg = np.zeros(8, np.float32)
    lg[[1, 2, 5, 6]] = 3.0
    ids, pr = orc.moe_topk(lg, 3)
    assert sorted(ids.tolist()) == [1, 2, 5]
    # fewer finite candidates than k is impossible for a softmax; k == E keeps all
    ids, pr = orc.moe_topk(np.arange(4, dtype=np.float32), 4)
    assert ids.tolist() == [0, 1, 2, 3] and abs(pr.sum() - 1) < 1e-6


def _model(orc, seed, max_seq=32):
    tensors, qts, mats = mt.build(seed=seed, max_pos=max_seq)
    m, hold = orc.mla_from_tensors(mt.CFG, tensors, qts, max_seq, nthreads=1)
    return m, hold, mats


def test_tiny_mla_vs_float64(orc):
    m, hold, mats = _model(orc, 11)
    L = orc.load()
    ids = np.array([5, 17, 3, 90, 42, 7], np.int32)
    lg = np.zeros(mt.CFG["vocab_size"], np.float32)
    assert L.orc_mla_forward(m, ids.ctypes.data, len(ids), 0, lg.ctypes.data, 1) == 0
    margins = []
    ref = mt.forward(mats, ids, margin=margins)
    assert min(margins) > 2e-5, "router near tie: choose another seed"
    assert np.max(np.abs(lg - ref)) <= 1e-4 * np.max(np.abs(ref))
    # incremental decode over the expanded cache equals the full recompute
    m2, hold2, _ = _model(orc, 11)
    L.orc_mla_forward(m2, ids.ctypes.data, 3, 0, lg.ctypes.data, 1)
    for t in range(3, 6):
        L.orc_mla_forward(m2, ids[t:].ctypes.data, 1, t, lg.ctypes.data, 1)
    assert np.max(np.abs(lg - ref)) <= 1e-4 * np.max(np.abs(ref))
    L.orc_mla_destroy(m)
    L.orc_mla_destroy(m2)


def test_tiny_mla_greedy_matches_float64(orc):
    m, hold, mats = _model(orc, 12)
    prompt = [3, 1, 4, 1]
    got = orc.mla_generate(m, prompt, 5)
    ids = list(prompt)
    for s in range(5):
        margins = []
        ref = mt.forward(mats, np.array(ids, np.int32), margin=margins)
        top = np.argsort(ref)[::-1]
        assert ref[top[0]] - ref[top[1]] > 1e-6 and min(margins) > 1e-5, "near tie: choose another seed"
        ids.append(int(top[0]))
    assert got == ids[4:]
    orc.load().orc_mla_destroy(m)


def test_load_latent_reproduces_the_forward_cache(orc):
    """orc_mla_load_latent, fed the latent records a prefill stored, gives
    a second model the same expanded cache: every cached float equal and the
    next decode step's logits equal bit for bit.  A wrong record offset, a
    swapped K_nope / V half or a missing k_pe rotation fails here."""
    L = orc.load()
    max_seq = 32
    c = mt.CFG
    R = c["dc"] + c["rope"]
    m, hold, _ = _model(orc, 11, max_seq)
    m2, hold2, _ = _model(orc, 11, max_seq)
    tap = np.zeros((c["n_layers"], max_seq, R), np.float32)
    L.orc_mla_set_latent_tap(m, tap.ctypes.data)
    ids = np.array([5, 17, 3, 90, 42, 7, 11, 60, 2], np.int32)
    n = len(ids) - 1
    lg = np.zeros(c["vocab_size"], np.float32)
    assert L.orc_mla_forward(m, ids.ctypes.data, n, 0, lg.ctypes.data, 1) == 0
    L.orc_mla_set_latent_tap(m, None)
    assert np.any(tap[:, :n] != 0) and not np.any(tap[:, n:])
    for layer in range(c["n_layers"]):
        assert L.orc_mla_load_latent(m2, layer, tap[layer].ctypes.data, n) == 0
        sizes = (max_seq * c["rope"], max_seq * c["n_heads"] * c["nope"], max_seq * c["n_heads"] * c["v_dim"])
        for which, sz in enumerate(sizes):
            a = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_float * sz).from_address(L.orc_mla_cache(m, layer, which)))
            b = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_float * sz).from_address(L.orc_mla_cache(m2, layer, which)))
            assert np.array_equal(a, b), (layer, which)
    lg1 = np.zeros_like(lg)
    lg2 = np.zeros_like(lg)
    assert L.orc_mla_forward(m, ids[n:].ctypes.data, 1, n, lg1.ctypes.data, 1) == 0
    assert L.orc_mla_forward(m2, ids[n:].ctypes.data, 1, n, lg2.ctypes.data, 1) == 0
    assert np.array_equal(lg1, lg2)
    assert L.orc_mla_load_latent(m2, c["n_layers"], tap[0].ctypes.data, n) != 0   # bad layer rejected
    L.orc_mla_destroy(m)
    L.orc_mla_destroy(m2)
