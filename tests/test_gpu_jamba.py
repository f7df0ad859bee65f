"""RINA Jamba hybrid on the GPU: the RINA-MLA decode attention against a
float64 restatement, and the engine (SSM + RINA-MLA layers through the
"gqa" Inference) against the CPU oracle: logits and greedy tokens, tiny
and at the config-5 shape."""
import ctypes as C
import importlib
import os

import numpy as np
import pytest

import _jamba_tiny as jt
import _numpy_ref as nr
from _util import REL_TOL, assert_close, assert_close_elem, dev, empty, host, ok, rng, stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("P,use_dpos", [(0, False), (9, False), (70, True), (300, False)])
@pytest.mark.parametrize("H,Hkv,da,db", [(10, 5, 64, 32), (4, 2, 64, 16)])
def test_dq_decode_attention(rina, P, use_dpos, H, Hkv, da, db):
    hip = rina.load_hip()
    dq, dv = da + db, 64
    max_seq = P + 5
    r = rng(P + H + db)
    ck = r.standard_normal((max_seq, Hkv, dq)).astype(np.float32)
    cv = r.standard_normal((max_seq, Hkv, dv)).astype(np.float32)
    qa = r.standard_normal((H, da)).astype(np.float32)
    qb = r.standard_normal((H, db)).astype(np.float32)
    ka = r.standard_normal((Hkv, da)).astype(np.float32)
    kb = r.standard_normal((Hkv, db)).astype(np.float32)
    v = r.standard_normal((Hkv, dv)).astype(np.float32)
    ang = np.outer(np.arange(max_seq), 1.0 / 10000 ** (np.arange(0, db, 2) / db)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

    def rope(x):   # HF pairs at position P, reference fma form in fp32
        c, s = cos[P], sin[P]
        y = x.copy()
        x0, x1 = x[..., 0::2], x[..., 1::2]
        y[..., 0::2] = (x0.astype(np.float64) * c - (x1 * s).astype(np.float32)).astype(np.float32)
        y[..., 1::2] = (x0.astype(np.float64) * s + (x1 * c).astype(np.float32)).astype(np.float32)
        return y

    qf = np.concatenate([qa, rope(qb)], axis=1).astype(np.float64)
    kn = np.concatenate([ka, rope(kb)], axis=1)
    K = ck.astype(np.float64).copy()
    V = cv.astype(np.float64).copy()
    K[P], V[P] = kn, v
    rep = H // Hkv
    ref = np.concatenate([nr.softmax_attn(qf[h], K[: P + 1, h // rep], V[: P + 1, h // rep], 1 / np.sqrt(dq))
                          for h in range(H)])
    wsb = hip.rina_hip_dq_attention_workspace(H, dq, max_seq)
    ws = empty(wsb, "uint8")
    ckd, cvd = dev(ck), dev(cv)
    od = empty(H * dv)
    cd, sd = dev(cos), dev(sin)
    pos = dev(np.array([P], np.int32)) if use_dpos else None
    ok(hip.rina_hip_dq_decode_attention(dev(qa).data_ptr(), dev(qb).data_ptr(), dev(ka).data_ptr(),
                                        dev(kb).data_ptr(), dev(v).data_ptr(), cd.data_ptr(), sd.data_ptr(),
                                        cd.data_ptr(), sd.data_ptr(), ckd.data_ptr(), cvd.data_ptr(), H, Hkv, da, db,
                                        dv, 0 if use_dpos else P, pos.data_ptr() if use_dpos else None, max_seq,
                                        od.data_ptr(), ws.data_ptr(), wsb, stream()), "dq attention")
    assert_close_elem(host(od), ref, what="dq attention P %d" % P)
    gk = host(ckd).reshape(max_seq, Hkv, dq)
    assert np.max(np.abs(gk[P] - kn)) <= 2e-6 * np.max(np.abs(kn))          # appended K row (rotated)
    assert np.array_equal(host(cvd).reshape(max_seq, Hkv, dv)[P], v)
    keep = np.ones(max_seq, bool)
    keep[P] = False
    assert np.array_equal(gk[keep], ck[keep])


@pytest.mark.parametrize("T", [2, 19, 300])
@pytest.mark.parametrize("H,Hkv,da,db", [(10, 5, 64, 32), (4, 2, 64, 16)])
def test_dq_prompt_attention_matches_decode_rows(rina, T, H, Hkv, da, db):
    """A prompt of T rows from position 0 in one call (every row's key and
    value appended, then one causal attention over the rows) against the
    same rows fed to the fp32-cache decode attention one position at a
    time: both caches bit for bit, every output row within tolerance."""
    hip = rina.load_hip()
    dq, dv = da + db, 64
    max_seq = T + 4
    r = rng(T + H + db)
    qa = r.standard_normal((T, H * da)).astype(np.float32)
    qb = r.standard_normal((T, H * db)).astype(np.float32)
    ka = r.standard_normal((T, Hkv * da)).astype(np.float32)
    kb = r.standard_normal((T, Hkv * db)).astype(np.float32)
    v = r.standard_normal((T, Hkv * dv)).astype(np.float32)
    ang = np.outer(np.arange(max_seq), 1.0 / 10000 ** (np.arange(0, db, 2) / db)).astype(np.float32)
    cd, sd = dev(np.cos(ang).astype(np.float32)), dev(np.sin(ang).astype(np.float32))
    qad, qbd, kad, kbd, vd = dev(qa), dev(qb), dev(ka), dev(kb), dev(v)
    ck1, cv1 = dev(np.zeros((max_seq, Hkv, dq), np.float32)), dev(np.zeros((max_seq, Hkv, dv), np.float32))
    wsb = hip.rina_hip_dq_attention_workspace(H, dq, max_seq)
    ws = empty(wsb, "uint8")
    od = empty(H * dv)
    one = np.zeros((T, H * dv), np.float32)
    for t in range(T):
        ok(hip.rina_hip_dq_decode_attention(qad.data_ptr() + 4 * t * H * da, qbd.data_ptr() + 4 * t * H * db,
                                            kad.data_ptr() + 4 * t * Hkv * da, kbd.data_ptr() + 4 * t * Hkv * db,
                                            vd.data_ptr() + 4 * t * Hkv * dv, cd.data_ptr(), sd.data_ptr(),
                                            cd.data_ptr(), sd.data_ptr(), ck1.data_ptr(), cv1.data_ptr(), H, Hkv, da,
                                            db, dv, t, None, max_seq, od.data_ptr(), ws.data_ptr(), wsb, stream()),
           "decode row %d" % t)
        one[t] = host(od)
    ck2, cv2 = dev(np.zeros((max_seq, Hkv, dq), np.float32)), dev(np.zeros((max_seq, Hkv, dv), np.float32))
    pwb = hip.rina_hip_dq_prompt_workspace(T, H, Hkv, da, db, dv)
    pw = empty(pwb, "uint8")
    o2 = empty(T * H * dv)
    ok(hip.rina_hip_dq_prompt_attention(qad.data_ptr(), qbd.data_ptr(), kad.data_ptr(), kbd.data_ptr(), vd.data_ptr(),
                                        cd.data_ptr(), sd.data_ptr(), cd.data_ptr(), sd.data_ptr(), ck2.data_ptr(),
                                        cv2.data_ptr(), H, Hkv, da, db, dv, T, max_seq, o2.data_ptr(), pw.data_ptr(),
                                        pwb, stream()), "prompt attention")
    assert np.array_equal(host(ck2).view(np.uint32), host(ck1).view(np.uint32))
    assert np.array_equal(host(cv2).view(np.uint32), host(cv1).view(np.uint32))
    got = host(o2).reshape(T, H * dv)
    for t in range(T):
        assert_close_elem(got[t], one[t], what="prompt row %d vs decode row" % t)


@pytest.mark.parametrize("mode", [5, 0])
@pytest.mark.parametrize("T,start", [(1, 0), (2, 0), (19, 0), (300, 0), (40, 37), (260, 700)])
@pytest.mark.parametrize("H,Hkv,da,db", [(10, 5, 64, 32), (4, 2, 64, 16), (4, 1, 64, 0)])
def test_dq_prompt_attention_kv_matches_decode_rows(rina, T, start, H, Hkv, da, db, mode):
    """A prompt of T rows at positions start .. start+T-1 in one call (every
    row appended, then each row reads the rows before it through the cache)
    against the same rows fed to the decode attention of the same cache one
    position at a time: over the q2k_q1v cache (mode 5) the packed key
    content, the RoPE'd key part and the packed values, over fp32 caches
    (mode 0) the key and value rows, bit for bit over the whole cache; every
    output row within tolerance.  Rows before start come from decode calls
    in both runs (a prompt that continues a cache); 260 rows from 700 take
    32-position chunks on both sides of a chunk boundary."""
    hip = rina.load_hip()
    dv = 64
    max_seq = start + T + 4
    r = rng(T + H + db + start)
    n = start + T
    qa = r.standard_normal((n, H * da)).astype(np.float32)
    qb = r.standard_normal((n, H * max(db, 1))).astype(np.float32)[:, :H * db].copy()
    ka = r.standard_normal((n, Hkv * da)).astype(np.float32)
    kb = r.standard_normal((n, Hkv * max(db, 1))).astype(np.float32)[:, :Hkv * db].copy()
    v = r.standard_normal((n, Hkv * dv)).astype(np.float32)
    hb = max(db // 2, 1)
    ang = np.outer(np.arange(max_seq), 1.0 / 10000 ** (np.arange(0, 2 * hb, 2) / max(db, 2))).astype(np.float32)
    cd, sd = dev(np.cos(ang).astype(np.float32)), dev(np.sin(ang).astype(np.float32))
    qad, kad, vd = dev(qa), dev(ka), dev(v)
    qbd = dev(qb) if db else None
    kbd = dev(kb) if db else None
    sizes = [hip.rina_hip_dq_kv_region_bytes(mode, part, max_seq, Hkv, da, db, dv) for part in range(3)]
    assert sizes[0] > 0 and sizes[1] > 0 and (sizes[2] > 0) == (mode == 5 and db > 0)

    def caches():
        return [dev(np.zeros(max(sz, 4), np.uint8)) for sz in sizes]

    wsb = hip.rina_hip_dq_attention_workspace(H, da + db, max_seq)
    ws = empty(wsb, "uint8")
    od = empty(H * dv)
    ptr = lambda x, off: x.data_ptr() + off if x is not None else None

    def decode_row(c, t):
        ok(hip.rina_hip_dq_decode_attention_kv(ptr(qad, 4 * t * H * da), ptr(qbd, 4 * t * H * db),
                                               ptr(kad, 4 * t * Hkv * da), ptr(kbd, 4 * t * Hkv * db),
                                               ptr(vd, 4 * t * Hkv * dv), cd.data_ptr(), sd.data_ptr(), cd.data_ptr(),
                                               sd.data_ptr(), mode, c[0].data_ptr(), c[1].data_ptr(),
                                               c[2].data_ptr() if sizes[2] else None, H, Hkv, da, db, dv, t, None,
                                               max_seq,
                                               od.data_ptr(), ws.data_ptr(), wsb, stream()), "decode row %d" % t)
        return host(od)

    c1, c2 = caches(), caches()
    for t in range(start):
        decode_row(c1, t)
        decode_row(c2, t)
    one = np.stack([decode_row(c1, t) for t in range(start, n)])
    o2 = empty(T * H * dv)
    ok(hip.rina_hip_dq_prompt_attention_kv(ptr(qad, 4 * start * H * da), ptr(qbd, 4 * start * H * db),
                                           ptr(kad, 4 * start * Hkv * da), ptr(kbd, 4 * start * Hkv * db),
                                           ptr(vd, 4 * start * Hkv * dv), cd.data_ptr(), sd.data_ptr(), cd.data_ptr(),
                                           sd.data_ptr(), mode, c2[0].data_ptr(), c2[1].data_ptr(),
                                           c2[2].data_ptr() if sizes[2] else None, H, Hkv, da, db, dv, start, T,
                                           max_seq, o2.data_ptr(), stream()), "prompt attention mode %d" % mode)
    for part in range(3):
        if sizes[part]:
            assert np.array_equal(host(c2[part]), host(c1[part])), "cache part %d" % part
    got = host(o2).reshape(T, H * dv)
    for t in range(T):
        assert_close_elem(got[t], one[t], what="prompt row %d vs decode row" % (start + t))


def test_dq_prompt_attention_kv_rejects(rina):
    """Argument checks of the batched prompt entry, before any launch: a GQA
    cache mode (-2, RINA_ERR_QTYPE), q2k_q1v key content or values other than
    64 wide (-3, RINA_ERR_SHAPE), rows past the cache (-4, RINA_ERR_RANGE),
    no rows (-1, RINA_ERR_ARG)."""
    hip = rina.load_hip()
    buf = empty(1 << 16, "uint8")
    p = buf.data_ptr()
    call = lambda mode, da, dv, start, T, max_seq: hip.rina_hip_dq_prompt_attention_kv(
        p, p, p, p, p, None, None, None, None, mode, p, p, p, 4, 2, da, 16, dv, start, T, max_seq, p, stream())
    assert call(1, 64, 64, 0, 4, 8) == -2
    assert call(5, 32, 64, 0, 4, 8) == -3
    assert call(5, 64, 32, 0, 4, 8) == -3
    assert call(5, 64, 64, 6, 4, 8) == -4
    assert call(5, 64, 64, 0, 0, 8) == -1


def header(max_seq, cfg=jt.CFG, types=jt.TYPES):
    c = cfg
    return {"name": c["name"], "dim": c["dim"], "n_layers": c["n_layers"], "n_heads": c["n_heads"],
            "n_kv_heads": c["n_kv_heads"], "head_dim": c["head_dim"], "d_h_r": c["d_h_r"], "d_c": c["d_c"],
            "ssm_steps": c["ssm_steps"], "vocab_size": c["vocab_size"], "max_seq_len": max_seq,
            "hidden_dim": c["hidden_dim"], "layers": [{"type": t} for t in types]}


@pytest.fixture(scope="module")
def tiny_jamba(rina, orc):
    synth = importlib.import_module("rina_amd.synth")
    max_seq = 48
    tensors, mats, shapes = jt.build(orc, seed=21, max_pos=max_seq)
    qts = {n: (6 if a.dtype == np.float32 else jt.Q4_0) for n, a in tensors.items()}
    up = {n: (qts[n], shapes[n], tensors[n]) for n in tensors}
    hm = synth.HostModel(header(max_seq), up)
    yield hm, tensors, max_seq
    hm.close()


def test_jamba_engine_forward_logits(rina, orc, tiny_jamba):
    import torch
    hm, tensors, max_seq = tiny_jamba
    eng = rina.load_engine()
    inf = hm.infer("gqa", max_seq=max_seq)
    V = jt.CFG["vocab_size"]
    ids = np.array([5, 17, 3, 90, 42, 7], np.int32)
    lg = empty(len(ids) * V)
    rina.check(eng.rina_infer_forward(inf, torch.from_numpy(ids).cuda().data_ptr(), lg.data_ptr(), 1, len(ids), 0,
                                      stream()), "forward")
    m, hold = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq)
    L = orc.load()
    ref = np.zeros((len(ids), V), np.float32)
    assert L.orc_jamba_forward(m, ids.ctypes.data, len(ids), 0, ref.ctypes.data, 0) == 0
    assert_close(host(lg).reshape(len(ids), V), ref, what="jamba prefill logits")
    for t, nxt in enumerate([11, 64, 2]):
        x = np.array([nxt], np.int32)
        rina.check(eng.rina_infer_forward(inf, torch.from_numpy(x).cuda().data_ptr(), lg.data_ptr(), 1, 1, 6 + t,
                                          stream()), "decode")
        r1 = np.zeros(V, np.float32)
        L.orc_jamba_forward(m, x.ctypes.data, 1, 6 + t, r1.ctypes.data, 0)
        assert_close(host(lg)[:V], r1, what="jamba decode logits %d" % t)
    L.orc_jamba_destroy(m)
    eng.rina_infer_destroy(inf)


def test_jamba_prompt_rows_match_single_positions(rina, orc, tiny_jamba):
    """A prompt of T rows (the matvecs as T-row products, the SSM scan over
    the T positions in one launch, the RINA-MLA attention row by row) against
    the same ids fed one position at a time: every row's logits, and the
    decode steps after the prompt (which read the caches and scan state the
    two paths left), within tolerance."""
    import torch
    hm, tensors, max_seq = tiny_jamba
    eng = rina.load_engine()
    V = jt.CFG["vocab_size"]
    ids = np.array([5, 17, 3, 90, 42, 7, 8, 1, 33, 64, 2, 71, 19, 4, 6, 50, 12, 99, 23], np.int32)
    T = len(ids)
    rows_inf, one_inf = hm.infer("gqa", max_seq=max_seq), hm.infer("gqa", max_seq=max_seq)
    lg = empty(T * V)
    rina.check(eng.rina_infer_forward(rows_inf, torch.from_numpy(ids).cuda().data_ptr(), lg.data_ptr(), 1, T, 0,
                                      stream()), "prompt rows")
    rows = host(lg).reshape(T, V)
    one = np.zeros((T, V), np.float32)
    l1 = empty(V)
    for t in range(T):
        x = torch.from_numpy(ids[t:t + 1].copy()).cuda()
        rina.check(eng.rina_infer_forward(one_inf, x.data_ptr(), l1.data_ptr(), 1, 1, t, stream()), "position %d" % t)
        one[t] = host(l1)
    assert_close(rows, one, what="prompt rows vs one position at a time")
    for t, nxt in enumerate([11, 64, 2]):
        x = torch.from_numpy(np.array([nxt], np.int32)).cuda()
        got = []
        for inf in (rows_inf, one_inf):
            rina.check(eng.rina_infer_forward(inf, x.data_ptr(), l1.data_ptr(), 1, 1, T + t, stream()), "decode")
            got.append(host(l1))
        assert_close(got[0], got[1], what="decode %d after the prompt" % t)
    eng.rina_infer_destroy(rows_inf)
    eng.rina_infer_destroy(one_inf)


@pytest.mark.parametrize("use_graph", [True, False])
def test_jamba_engine_greedy_identical(rina, orc, tiny_jamba, use_graph):
    hm, tensors, max_seq = tiny_jamba
    eng = rina.load_engine()
    inf = hm.infer("gqa", max_seq=max_seq)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    steps = 24
    out = (C.c_int * steps)()
    rina.check(eng.rina_infer_generate(inf, (C.c_int * len(prompt))(*prompt), len(prompt), steps, out,
                                       1 if use_graph else 0, stream(), None), "generate")
    eng.rina_infer_destroy(inf)
    m, hold = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq)
    ref = orc.jamba_generate(m, prompt, steps, recompute=True)     # the reference's semantics
    orc.load().orc_jamba_destroy(m)
    assert list(out) == ref


def test_jamba_config5_shape_greedy(rina, orc):
    """config-5 widths (640d, 10/5 heads, d_c 160, 12 SSM + 4 RINA-MLA,
    vocab 128256, Q4_0): greedy tokens identical to the oracle."""
    synth = importlib.import_module("rina_amd.synth")
    sm = synth.SynthJamba(seed=3, max_seq=64, keep_host=True)
    try:
        eng = rina.load_engine()
        inf = sm.infer()
        prompt = [101, 2047, 9, 55555, 3, 777, 12, 40000]
        steps = 8
        out = (C.c_int * steps)()
        rina.check(eng.rina_infer_generate(inf, (C.c_int * len(prompt))(*prompt), len(prompt), steps, out, 1,
                                           stream(), None), "generate")
        eng.rina_infer_destroy(inf)
        m, hold = orc.jamba_from_tensors(sm.cfg, sm.host, sm.types, jt.Q4_0, 64)
        ref = orc.jamba_generate(m, prompt, steps)
        orc.load().orc_jamba_destroy(m)
        assert list(out) == ref
    finally:
        sm.close()


@pytest.mark.parametrize("kv_mode", ["fp32", "q2k_q1v"])
def test_jamba_config5_full_context_128_steps(rina, orc, kv_mode):
    """Config 5 as specified: the full Jamba shape at context 2048, a
    1900-token seeded prompt, then 128 greedy steps (positions 1900..2027),
    with the fp32 RINA-MLA cache (the reference's numerics) and with the q2 K
    / q1 V cache (rina_mla_kv_mode "q2k_q1v": key content q2_1, values q1_0,
    packed on append; queries and the current position fp32).  The oracle
    runs its own 1900-token prefill in the same mode and its state-carrying
    decode (proven equal to the reference's full recompute); all 129 tokens
    must match, every step's top-2 margin must clear twice the 1e-5
    tolerance, and the tokens must be varied."""
    synth = importlib.import_module("rina_amd.synth")
    n_prompt, steps, max_seq = 1900, 128, 2048
    sm = synth.SynthJamba(seed=3, max_seq=max_seq, keep_host=True, kv_mode=kv_mode)
    try:
        eng = rina.load_engine()
        V = sm.cfg["vocab_size"]
        prompt = np.random.default_rng(5).integers(0, V, n_prompt).astype(np.int32)
        inf = sm.infer()
        out = (C.c_int * (steps + 1))()
        rina.check(eng.rina_infer_generate(inf, prompt.ctypes.data_as(C.POINTER(C.c_int)), n_prompt, steps + 1, out,
                                           1, stream(), None), "generate")
        eng.rina_infer_destroy(inf)
        got = list(out)
        m, hold = orc.jamba_from_tensors(sm.cfg, sm.host, sm.types, jt.Q4_0, max_seq,
                                         min(os.cpu_count() or 1, 16), kv_mode=kv_mode)
        L = orc.load()
        lg = np.zeros(V, np.float32)
        ref, margins = [], []
        ids, T, pos = prompt, n_prompt, 0
        for s in range(steps + 1):
            assert L.orc_jamba_forward(m, ids.ctypes.data, T, pos, lg.ctypes.data, 1) == 0
            top = np.argsort(lg)[::-1][:2]
            margins.append(float(lg[top[0]] - lg[top[1]]) / float(np.max(np.abs(lg))))
            tok = L.orc_argmax(lg.ctypes.data, V)
            ref.append(tok)
            pos += T
            ids, T = np.array([tok], np.int32), 1
        L.orc_jamba_destroy(m)
        print("config 5 %s: tokens %s, min top-2 margin %.2e" % (kv_mode, got[:8], min(margins)))
        assert got == ref, "first divergence at step %d" % next(i for i in range(steps + 1) if got[i] != ref[i])
        assert min(margins) > 2 * REL_TOL, "near tie at step %d (%.2e)" % (int(np.argmin(margins)), min(margins))
        assert len(set(got)) >= 16
    finally:
        sm.close()


@pytest.mark.parametrize("mode", ["q8", "q4", "q4k_q2v", "q2", "q2k_q1v"])
def test_jamba_kv_quant_mode_keeps_fp32_rmla(rina, tiny_jamba, mode):
    """kv_quant_mode names the GQA cache; the reference's RINA-MLA layer keeps
    fp32 rows whatever it says (rina_mla_layer.cu:65-98, infer_gqa.cpp).  A
    hybrid created with each reference mode initializes and gives the
    fp32-cache model's logits, bit for bit."""
    import torch
    hm, tensors, max_seq = tiny_jamba
    eng = rina.load_engine()
    V = jt.CFG["vocab_size"]
    ids = np.array([5, 17, 3, 90, 42, 7], np.int32)
    outs = []
    for kv in (None, mode):
        inf = hm.infer("gqa", kv_mode=kv, max_seq=max_seq)
        lg = empty(len(ids) * V)
        rina.check(eng.rina_infer_forward(inf, torch.from_numpy(ids).cuda().data_ptr(), lg.data_ptr(), 1, len(ids),
                                          0, stream()), "forward")
        x = np.array([11], np.int32)
        l1 = empty(V)
        rina.check(eng.rina_infer_forward(inf, torch.from_numpy(x).cuda().data_ptr(), l1.data_ptr(), 1, 1, len(ids),
                                          stream()), "decode")
        outs.append(np.concatenate([host(lg), host(l1)]))
        eng.rina_infer_destroy(inf)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("P,use_dpos", [(0, False), (9, False), (70, True), (300, False)])
@pytest.mark.parametrize("H,Hkv,db", [(10, 5, 32), (4, 2, 16)])
def test_dq_decode_attention_q2k_q1v(rina, orc, P, use_dpos, H, Hkv, db):
    """The q2 K / q1 V RINA-MLA cache: earlier positions are read through
    their packs (key content q2_1, values q1_0, the RoPE part fp32), the
    current one from its fp32 rows, which are appended packed: the appended
    bytes equal the KV packers' (bit-exact), the RoPE part is stored as
    rotated, no other position changes, and the output is within 1e-5 of a
    float64 softmax over that history."""
    hip = rina.load_hip()
    da, dv = 64, 64
    dq = da + db
    max_seq = P + 5
    r = rng(P + H + db + 1000)
    ckf = r.standard_normal((max_seq, Hkv, da)).astype(np.float32)    # history before packing
    cvf = r.standard_normal((max_seq, Hkv, dv)).astype(np.float32)
    ckr = r.standard_normal((max_seq, Hkv, db)).astype(np.float32)
    ckq = orc.kv_quantize(3, ckf.reshape(-1))
    cvq = orc.kv_quantize(4, cvf.reshape(-1))
    Kc = orc.kv_dequant(3, ckq, ckf.size).reshape(max_seq, Hkv, da).astype(np.float64)
    Vh = orc.kv_dequant(4, cvq, cvf.size).reshape(max_seq, Hkv, dv).astype(np.float64)
    qa = r.standard_normal((H, da)).astype(np.float32)
    qb = r.standard_normal((H, db)).astype(np.float32)
    ka = r.standard_normal((Hkv, da)).astype(np.float32)
    kb = r.standard_normal((Hkv, db)).astype(np.float32)
    v = r.standard_normal((Hkv, dv)).astype(np.float32)
    ang = np.outer(np.arange(max_seq), 1.0 / 10000 ** (np.arange(0, db, 2) / db)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

    def rope(x):   # HF pairs at position P, reference fma form in fp32
        c, s = cos[P], sin[P]
        y = x.copy()
        x0, x1 = x[..., 0::2], x[..., 1::2]
        y[..., 0::2] = (x0.astype(np.float64) * c - (x1 * s).astype(np.float32)).astype(np.float32)
        y[..., 1::2] = (x0.astype(np.float64) * s + (x1 * c).astype(np.float32)).astype(np.float32)
        return y

    qf = np.concatenate([qa, rope(qb)], axis=1).astype(np.float64)
    krot = rope(kb)
    K = np.concatenate([Kc, ckr.astype(np.float64)], axis=2)
    V = Vh.copy()
    K[P] = np.concatenate([ka, krot], axis=1)
    V[P] = v
    rep = H // Hkv
    ref = np.concatenate([nr.softmax_attn(qf[h], K[: P + 1, h // rep], V[: P + 1, h // rep], 1 / np.sqrt(dq))
                          for h in range(H)])
    wsb = hip.rina_hip_dq_attention_workspace(H, dq, max_seq)
    ws = empty(wsb, "uint8")
    for part, arr in ((0, ckq), (1, cvq), (2, ckr)):
        assert hip.rina_hip_dq_kv_region_bytes(5, part, max_seq, Hkv, da, db, dv) == arr.nbytes
    ckd, cvd, krd = dev(ckq), dev(cvq), dev(ckr)
    od = empty(H * dv)
    cd, sd = dev(cos), dev(sin)
    pos = dev(np.array([P], np.int32)) if use_dpos else None
    ok(hip.rina_hip_dq_decode_attention_kv(dev(qa).data_ptr(), dev(qb).data_ptr(), dev(ka).data_ptr(),
                                           dev(kb).data_ptr(), dev(v).data_ptr(), cd.data_ptr(), sd.data_ptr(),
                                           cd.data_ptr(), sd.data_ptr(), 5, ckd.data_ptr(), cvd.data_ptr(),
                                           krd.data_ptr(), H, Hkv, da, db, dv, 0 if use_dpos else P,
                                           pos.data_ptr() if use_dpos else None, max_seq, od.data_ptr(),
                                           ws.data_ptr(), wsb, stream()), "dq attention q2k_q1v")
    assert_close_elem(host(od), ref, what="dq attention q2k_q1v P %d" % P)
    gk, gv, gr = host(ckd), host(cvd), host(krd).reshape(max_seq, Hkv, db)
    kbytes, vbytes = Hkv * (da // 32) * 10, Hkv * (dv // 32) * 6
    assert np.array_equal(gk[P * kbytes:(P + 1) * kbytes], orc.kv_quantize(3, ka.reshape(-1)))
    assert np.array_equal(gv[P * vbytes:(P + 1) * vbytes], orc.kv_quantize(4, v.reshape(-1)))
    assert np.max(np.abs(gr[P] - krot)) <= 2e-6 * np.max(np.abs(krot))
    keep = np.ones(max_seq, bool)
    keep[P] = False
    assert np.array_equal(gk.reshape(max_seq, -1)[keep], ckq.reshape(max_seq, -1)[keep])
    assert np.array_equal(gv.reshape(max_seq, -1)[keep], cvq.reshape(max_seq, -1)[keep])
    assert np.array_equal(gr[keep], ckr[keep])


@pytest.mark.parametrize("use_graph", [True, False])
def test_jamba_q2k_q1v_cache_greedy(rina, orc, use_graph):
    """The tiny hybrid with the q2 K / q1 V RINA-MLA cache: the engine's
    greedy tokens equal the oracle's in the same cache mode, and so do the
    logits of a prefill and of three host-position decode steps (1e-5),
    which differ from the fp32-cache model's by far more (the packed
    history is what the steps read)."""
    import torch
    synth = importlib.import_module("rina_amd.synth")
    max_seq = 48
    tensors, mats, shapes = jt.build(orc, seed=21, max_pos=max_seq)
    qts = {n: (6 if a.dtype == np.float32 else jt.Q4_0) for n, a in tensors.items()}
    up = {n: (qts[n], shapes[n], tensors[n]) for n in tensors}
    hdr = header(max_seq)
    hdr["rina_mla_kv_mode"] = "q2k_q1v"
    hm = synth.HostModel(hdr, up)
    try:
        eng = rina.load_engine()
        inf = hm.infer("gqa", max_seq=max_seq)
        prompt = [3, 1, 4, 1, 5, 9, 2, 6]
        steps = 20
        out = (C.c_int * steps)()
        rina.check(eng.rina_infer_generate(inf, (C.c_int * len(prompt))(*prompt), len(prompt), steps, out,
                                           1 if use_graph else 0, stream(), None), "generate")
        eng.rina_infer_destroy(inf)
        m, hold = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq, kv_mode="q2k_q1v")
        ref = orc.jamba_generate(m, prompt, steps)
        orc.load().orc_jamba_destroy(m)
        assert list(out) == ref
        # logits: prefill of 6 tokens, then 3 decode steps at host positions
        L = orc.load()
        V = jt.CFG["vocab_size"]
        mq, hq = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq, kv_mode="q2k_q1v")
        mf, hf = orc.jamba_from_tensors(jt.CFG, tensors, jt.TYPES, jt.Q4_0, max_seq)
        inf = hm.infer("gqa", max_seq=max_seq)
        ids = np.array([5, 17, 3, 90, 42, 7], np.int32)
        lg = empty(len(ids) * V)
        rina.check(eng.rina_infer_forward(inf, torch.from_numpy(ids).cuda().data_ptr(), lg.data_ptr(), 1, len(ids), 0,
                                          stream()), "forward")
        rq, rf = np.zeros(V, np.float32), np.zeros(V, np.float32)
        L.orc_jamba_forward(mq, ids.ctypes.data, len(ids), 0, rq.ctypes.data, 1)
        L.orc_jamba_forward(mf, ids.ctypes.data, len(ids), 0, rf.ctypes.data, 1)
        assert_close(host(lg).reshape(len(ids), V)[-1], rq, what="q2k_q1v prefill logits")
        far = 0.0
        for t, nxt in enumerate([11, 64, 2]):
            x = np.array([nxt], np.int32)
            rina.check(eng.rina_infer_forward(inf, torch.from_numpy(x).cuda().data_ptr(), lg.data_ptr(), 1, 1, 6 + t,
                                              stream()), "decode")
            L.orc_jamba_forward(mq, x.ctypes.data, 1, 6 + t, rq.ctypes.data, 1)
            L.orc_jamba_forward(mf, x.ctypes.data, 1, 6 + t, rf.ctypes.data, 1)
            assert_close(host(lg)[:V], rq, what="q2k_q1v decode logits %d" % t)
            far = max(far, float(np.max(np.abs(rq - rf)) / np.max(np.abs(rf))))
        eng.rina_infer_destroy(inf)
        L.orc_jamba_destroy(mq)
        L.orc_jamba_destroy(mf)
        assert far > 1e-3, far
    finally:
        hm.close()
