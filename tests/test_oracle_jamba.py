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


def _qmodel(orc, seed, kv_mode, max_seq=48, nthreads=1):
    tensors, mats, shapes = jt.build(orc, seed=seed, max_pos=max_seq)
    m, hold = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq, nthreads=nthreads, kv_mode=kv_mode)
    return m, hold, mats


def _arr(addr, n, dtype):
    import ctypes as C
    ct = {np.uint8: C.c_uint8, np.float32: C.c_float}[dtype]
    return np.ctypeslib.as_array((ct * n).from_address(addr)).copy()


def test_q2k_q1v_rmla_cache(orc):
    """The q2 K / q1 V RINA-MLA cache (rina/model_jamba_qw2.py:175-177):
    (1) a prompt equals the same tokens as single steps, bit for bit (every
    position reads earlier positions through the packed cache); (2) the
    first RINA-MLA layer, whose inputs only SSM layers shape, packs exactly
    the fp32 rows an fp32-cache model computes (KV packers of
    kernels/quantize.cu); (3) the logits equal a float64 restatement whose
    attention reads earlier positions from the dequantized packs and the
    own position, and the RoPE part, unquantized."""
    L = orc.load()
    c = jt.CFG
    H, Hkv, dh, dhr, V, ms = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["d_h_r"], c["vocab_size"], 48
    ids = np.array([9, 4, 77, 3, 12, 5, 60, 2, 8, 31, 14], np.int32)
    T = len(ids)
    mq, hq, mats = _qmodel(orc, 24, "q2k_q1v")
    full = np.zeros(V, np.float32)
    L.orc_jamba_forward(mq, ids.ctypes.data, T, 0, full.ctypes.data, 1)
    ms2, hs2, _ = _qmodel(orc, 24, "q2k_q1v")
    inc = np.zeros(V, np.float32)
    for t in range(T):
        L.orc_jamba_forward(ms2, ids[t:].ctypes.data, 1, t, inc.ctypes.data, 1)
    assert np.array_equal(inc.view(np.uint32), full.view(np.uint32))
    # the prompt's query rows split over 3 worker threads: the same logits, bit for bit
    mt, ht, _ = _qmodel(orc, 24, "q2k_q1v", nthreads=3)
    par = np.zeros(V, np.float32)
    L.orc_jamba_forward(mt, ids.ctypes.data, T, 0, par.ctypes.data, 1)
    assert np.array_equal(par.view(np.uint32), full.view(np.uint32))
    L.orc_jamba_destroy(mt)
    rmla = [l for l, ty in enumerate(jt.TYPES) if ty not in ("inertia_wave_ssm", "ssm")]
    nb = T * Hkv * (dh // 32)
    mf, hf, _ = _qmodel(orc, 24, "fp32")
    L.orc_jamba_forward(mf, ids.ctypes.data, T, 0, full.ctypes.data, 1)
    first = rmla[0]
    kf = _arr(L.orc_jamba_fp32_cache(mf, first, 0), T * Hkv * (dh + dhr), np.float32).reshape(T, Hkv, dh + dhr)
    vf = _arr(L.orc_jamba_fp32_cache(mf, first, 1), T * Hkv * dh, np.float32).reshape(T, Hkv, dh)
    kq = _arr(L.orc_jamba_packed_cache(mq, first, 0), nb * 10, np.uint8)
    vq = _arr(L.orc_jamba_packed_cache(mq, first, 1), nb * 6, np.uint8)
    assert np.array_equal(kq, orc.kv_quantize(3, np.ascontiguousarray(kf[:, :, :dh]).reshape(-1)))
    assert np.array_equal(vq, orc.kv_quantize(4, vf.reshape(-1)))
    # (3) float64 with the oracle's packs as the history
    hist = {}
    for l in rmla:
        kql = _arr(L.orc_jamba_packed_cache(mq, l, 0), nb * 10, np.uint8)
        vql = _arr(L.orc_jamba_packed_cache(mq, l, 1), nb * 6, np.uint8)
        hist[l] = (orc.kv_dequant(3, kql, T * Hkv * dh).reshape(T, Hkv, dh).astype(np.float64),
                   orc.kv_dequant(4, vql, T * Hkv * dh).reshape(T, Hkv, dh).astype(np.float64))
    L.orc_jamba_forward(mq, ids.ctypes.data, T, 0, full.ctypes.data, 1)   # the same tokens again: same packs
    ref = jt.forward(mats, ids, history=hist)
    assert np.max(np.abs(full - ref)) <= 1e-4 * np.max(np.abs(ref))
    plain = jt.forward(mats, ids)
    assert np.max(np.abs(plain - ref)) > 1e-3 * np.max(np.abs(ref))      # the packed history matters
    for m in (mq, ms2, mf):
        L.orc_jamba_destroy(m)
