"""Pin the CPU oracle's RINA Jamba hybrid: a tiny model against a float64
numpy restatement of the reference's full-recompute forward, and the
incremental (state-carrying) form against the full recompute, bit for bit."""
import numpy as np

import _jamba_tiny as jt


def _model(orc, seed=21, max_seq=48):
    tensors, mats, shapes = jt.build(orc, seed=seed, max_pos=max_seq)
    m, hold = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq, nthreads=1)
    return m, hold, mats


def test_tiny_jamba_vs_float64(orc):
    m, hold, mats = _model(orc)
    L = orc.load()
    ids = np.array([5, 17, 3, 90, 42, 7, 66, 1], np.int32)
    lg = np.zeros(jt.CFG["vocab_size"], np.float32)
    assert L.orc_jamba_forward(m, ids.ctypes.data, len(ids), 0, lg.ctypes.data, 1) == 0
    ref = jt.forward(mats, ids)
    assert np.max(np.abs(lg - ref)) <= 1e-4 * np.max(np.abs(ref))
    L.orc_jamba_destroy(m)


def test_incremental_equals_full_recompute(orc):
    m, hold, mats = _model(orc, seed=22)
    L = orc.load()
    ids = np.array([9, 4, 77, 3, 12, 5, 60, 2, 8], np.int32)
    V = jt.CFG["vocab_size"]
    full = np.zeros(V, np.float32)
    inc = np.zeros(V, np.float32)
    L.orc_jamba_forward(m, ids.ctypes.data, len(ids), 0, full.ctypes.data, 1)
    L.orc_jamba_forward(m, ids.ctypes.data, 4, 0, inc.ctypes.data, 1)       # resets the state
    for t in range(4, len(ids)):
        L.orc_jamba_forward(m, ids[t:].ctypes.data, 1, t, inc.ctypes.data, 1)
    assert np.array_equal(inc.view(np.uint32), full.view(np.uint32))
    # greedy: incremental decode == the reference's recompute-every-step loop
    prompt = [3, 1, 4, 1, 5]
    assert orc.jamba_generate(m, prompt, 6) == orc.jamba_generate(m, prompt, 6, recompute=True)
    L.orc_jamba_destroy(m)


def test_tiny_jamba_greedy_matches_float64(orc):
    m, hold, mats = _model(orc, seed=23)
    prompt = [2, 7, 1, 8]
    got = orc.jamba_generate(m, prompt, 5)
    ids = list(prompt)
    for s in range(5):
        ref = jt.forward(mats, np.array(ids, np.int32))
        top = np.argsort(ref)[::-1]
        assert ref[top[0]] - ref[top[1]] > 1e-6, "near tie: choose another seed"
        ids.append(int(top[0]))
    assert got == ids[4:]
    orc.load().orc_jamba_destroy(m)
