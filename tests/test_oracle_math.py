"""Pin the CPU oracle's arithmetic: matvec, attention, glue and a tiny GQA
model against float64 numpy restatements, closed forms and invariants."""
import ctypes as C

import numpy as np
import pytest

import _numpy_ref as nr

# test_linear_q4.cu:106-124 shapes (M, N, K)
Q4_SHAPES = [(4, 160, 640), (2, 2048, 2048), (1, 640, 640), (8, 64, 4096)]


@pytest.mark.parametrize("qt", [5, 7])
@pytest.mark.parametrize("M,N,K", Q4_SHAPES)
def test_q4_linear_vs_float64(orc, qt, M, N, K):
    r = np.random.default_rng(M * 7 + N + K)
    w = (r.standard_normal(N * K) * 0.02).astype(np.float32)
    x = r.uniform(-1, 1, (M, K)).astype(np.float32)
    p = orc.pack(qt, w)
    W = nr.dequant_q4(p, N * K, qt == 7).reshape(N, K).astype(np.float64)
    ref = x.astype(np.float64) @ W.T
    got = orc.linear(p, qt, x, N, K)
    # fp32 serial accumulation of K terms: |err| <= K * eps * sum|w x| bound, far below 1e-5 rel
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    # single-thread and multi-thread results are the same numbers
    assert np.array_equal(got, orc.linear(p, qt, x, N, K, nthreads=1))


@pytest.mark.parametrize("K", [2048, 1408, 512])
def test_q2k_linear_flat_indexing(orc, K):
    N = 48
    r = np.random.default_rng(K)
    nb = (N * K + 255) // 256
    blk = r.integers(0, 256, (nb, 84), dtype=np.uint8)
    blk[:, 80:82] = np.frombuffer(np.float16(0.0025).tobytes() * nb, np.uint8).reshape(nb, 2)
    blk[:, 82:84] = np.frombuffer(np.float16(0.00125).tobytes() * nb, np.uint8).reshape(nb, 2)
    w = blk.reshape(-1)
    x = r.standard_normal(K).astype(np.float32)
    # flat element order: row n = elements [nK, nK+K) of the block stream
    W = nr.dequant_q2k_blocks(w)[: N * K].reshape(N, K).astype(np.float64)
    ref = W @ x.astype(np.float64)
    got = orc.linear(w, orc.Q2_K, x, N, K)[0]
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_fp32_linear_vs_float64(orc):
    r = np.random.default_rng(9)
    N, K = 1000, 640
    w = (r.standard_normal(N * K) * 0.02).astype(np.float32)
    x = r.standard_normal((3, K)).astype(np.float32)
    ref = x.astype(np.float64) @ w.reshape(N, K).T.astype(np.float64)
    got = orc.linear(w, orc.FP32, x, N, K)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def _attn_rows(orc, q, K, V):
    L = orc.load()
    T, dq = K.shape
    dh = V.shape[1]
    o = np.zeros(dh, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    L.orc_attn_rows(q.ctypes.data, dq, K.ctypes.data, dq, V.ctypes.data, dh, o.ctypes.data, dh, T - 1, 1, dq, dh)
    return o


def test_attention_vs_textbook_softmax(orc):
    r = np.random.default_rng(11)
    for T, dq, dh in [(1, 64, 64), (7, 64, 64), (100, 192, 128), (513, 64, 64)]:
        q = r.standard_normal(dq).astype(np.float32)
        K = r.standard_normal((T, dq)).astype(np.float32)
        V = r.standard_normal((T, dh)).astype(np.float32)
        got = _attn_rows(orc, q, K, V)
        ref = nr.softmax_attn(q, K, V, 1 / np.sqrt(dq))
        assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_attention_invariants(orc):
    r = np.random.default_rng(12)
    q = r.standard_normal(64).astype(np.float32)
    K = r.standard_normal((1, 64)).astype(np.float32)
    V = r.standard_normal((1, 64)).astype(np.float32)
    assert np.array_equal(_attn_rows(orc, q, K, V), V[0])           # one key: the V row
    K = np.repeat(r.standard_normal((1, 64)).astype(np.float32), 9, 0)
    V = r.standard_normal((9, 64)).astype(np.float32)
    assert np.allclose(_attn_rows(orc, q, K, V), V.mean(0), atol=1e-6)   # equal keys: mean of V


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4, 5])
def test_gqa_attention_quant_cache(orc, mode):
    L = orc.load()
    r = np.random.default_rng(20 + mode)
    H, Hkv, dh, P = 8, 2, 64, 37
    kvd = Hkv * dh
    kc = r.standard_normal((P, kvd)).astype(np.float32)
    vc = r.standard_normal((P, kvd)).astype(np.float32)
    q = r.standard_normal(H * dh).astype(np.float32)
    kcur = r.standard_normal(kvd).astype(np.float32)
    vcur = r.standard_normal(kvd).astype(np.float32)
    out = np.zeros(H * dh, np.float32)
    if mode == 0:
        Kd, Vd = kc, vc
        L.orc_gqa_attention(q.ctypes.data, kcur.ctypes.data, vcur.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                            None, None, 0, 0, None, None, 1, P, H, Hkv, dh, out.ctypes.data)
    else:
        kf, vf = orc.kv_mode_formats(mode)
        kq, vq = nr.kv_quantize(kf, kc), nr.kv_quantize(vf, vc)
        Kd, Vd = nr.kv_dequant(kf, kq, kc.size).reshape(P, kvd), nr.kv_dequant(vf, vq, vc.size).reshape(P, kvd)
        L.orc_gqa_attention(q.ctypes.data, kcur.ctypes.data, vcur.ctypes.data, None, None, kq.ctypes.data,
                            vq.ctypes.data, mode, 0, None, None, 1, P, H, Hkv, dh, out.ctypes.data)
    Kall = np.concatenate([Kd, kcur[None]], 0)
    Vall = np.concatenate([Vd, vcur[None]], 0)
    for h in range(H):
        g = h // (H // Hkv)
        ref = nr.softmax_attn(q[h * dh:(h + 1) * dh], Kall[:, g * dh:(g + 1) * dh], Vall[:, g * dh:(g + 1) * dh],
                              1 / np.sqrt(dh))
        assert np.max(np.abs(out[h * dh:(h + 1) * dh] - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_glue_vs_float64(orc):
    L = orc.load()
    r = np.random.default_rng(30)
    n, d = 3, 2048
    x = r.standard_normal((n, d)).astype(np.float32)
    w = r.uniform(0.5, 1.5, d).astype(np.float32)
    y = x.copy()
    L.orc_rms_norm(y.ctypes.data, w.ctypes.data, n, d, np.float32(1e-5))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    y = x.copy()
    L.orc_layer_norm(y.ctypes.data, w.ctypes.data, n, d, np.float32(1e-5))
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    # RoPE: NeoX pairs (i, i+d/2) at start_pos
    T, H, hd = 3, 4, 64
    ang = np.outer(np.arange(40), 1.0 / 500000 ** (np.arange(0, hd, 2) / hd)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    xr = r.standard_normal((T, H, hd)).astype(np.float32)
    y = xr.copy()
    L.orc_rope_neox(y.ctypes.data, cos.ctypes.data, sin.ctypes.data, T, H, hd, 17)
    assert np.max(np.abs(y - nr.rope_neox(xr, cos, sin, 17))) <= 1e-6
    # HF pairs (2i, 2i+1)
    y = xr.copy()
    L.orc_rope_hf(y.ctypes.data, cos.ctypes.data, sin.ctypes.data, T, H, hd, 0)
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])
    ref = nr.rope_neox(xr[..., perm], cos, sin, 0)
    back = np.empty_like(ref)
    back[..., perm] = ref
    assert np.max(np.abs(y - back)) <= 1e-6
    # silu * up
    g = r.standard_normal(1000).astype(np.float32)
    u = r.standard_normal(1000).astype(np.float32)
    o = np.zeros(1000, np.float32)
    L.orc_silu_mul(o.ctypes.data, g.ctypes.data, u.ctypes.data, 1000)
    gd = g.astype(np.float64)
    assert np.max(np.abs(o - gd / (1 + np.exp(-gd)) * u)) <= 1e-6


def test_argmax_rule(orc):
    L = orc.load()
    a = np.array([-1e11, 3.0, 5.0, 5.0, np.nan, 1.0], np.float32)
    assert L.orc_argmax(a.ctypes.data, a.size) == 2           # lowest index on ties, NaN skipped
    b = np.full(5, -2e10, np.float32)
    assert L.orc_argmax(b.ctypes.data, b.size) == 0           # nothing above -1e10 -> 0


def test_embedding_rows(orc):
    L = orc.load()
    r = np.random.default_rng(31)
    V, d = 50, 512
    w = (r.standard_normal(V * d) * 0.02).astype(np.float32)
    ids = np.array([3, 0, -5, 49], np.int32)
    for qt in (orc.Q4_0, orc.Q4_0F, orc.FP32):
        p = w if qt == orc.FP32 else orc.pack(qt, w)
        out = np.zeros((4, d), np.float32)
        L.orc_embedding(p.ctypes.data, qt, ids.ctypes.data, out.ctypes.data, 4, d)
        full = w.reshape(V, d) if qt == orc.FP32 else nr.dequant_q4(p, V * d, qt == orc.Q4_0F).reshape(V, d)
        assert np.array_equal(out, full[np.maximum(ids, 0)])


# ---- tiny model: oracle forward vs a float64 numpy restatement ----------------

def tiny_cfg():
    return dict(dim=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, hidden=256, vocab=97)


def build_tiny(orc, qt=7, seed=5):
    c = tiny_cfg()
    r = np.random.default_rng(seed)
    d, H, Hkv, dh, hd, V = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["hidden"], c["vocab"]
    ang = np.outer(np.arange(64), 1.0 / 500000 ** (np.arange(0, dh, 2) / dh)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    keep = {"cos": cos, "sin": sin}
    layers = []
    for l in range(c["n_layers"]):
        Lw = {}
        for nm, rows, cols in (("q", H * dh, d), ("k", Hkv * dh, d), ("v", Hkv * dh, d), ("o", d, H * dh),
                               ("1", hd, d), ("2", d, hd), ("3", hd, d)):
            w = (r.standard_normal(rows * cols) * 0.05).astype(np.float32)
            p = orc.pack(qt, w)
            Lw[nm] = (p, nr.dequant_q4(p, rows * cols, qt == 7).reshape(rows, cols))
        Lw["ln1"] = r.uniform(0.8, 1.2, d).astype(np.float32)
        Lw["ln2"] = r.uniform(0.8, 1.2, d).astype(np.float32)
        layers.append(Lw)
    keep["wte"] = (r.standard_normal(V * d) * 0.5).astype(np.float32)
    keep["ln_f"] = np.ones(d, np.float32)
    return c, layers, keep


def oracle_model(orc, c, layers, keep, kv_mode=0, qt=7, max_seq=64):
    LW = orc.GQALayerW * c["n_layers"]
    lw = LW()
    for i, Lw in enumerate(layers):
        o = lw[i]
        for f in ("q", "k", "v", "o", "1", "2", "3"):
            setattr(o, "w_" + f if f in "qkvo" else "w" + f, Lw[f][0].ctypes.data)
            setattr(o, "qt_" + f, qt)
        o.ln1, o.ln2 = Lw["ln1"].ctypes.data, Lw["ln2"].ctypes.data
        o.rope_q_cos = o.rope_k_cos = keep["cos"].ctypes.data
        o.rope_q_sin = o.rope_k_sin = keep["sin"].ctypes.data
    cfg = orc.GQACfg(dim=c["dim"], n_layers=c["n_layers"], n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"],
                     head_dim=c["head_dim"], hidden=c["hidden"], vocab=c["vocab"], max_seq=max_seq, use_rms_norm=1,
                     kv_mode=kv_mode, pre_rope=0, nthreads=1, wte=keep["wte"].ctypes.data, qt_wte=orc.FP32,
                     ln_f=keep["ln_f"].ctypes.data, lm_head=None, qt_lm=0, layers=lw)
    m = orc.load().orc_gqa_create(C.byref(cfg))
    return m, (lw, cfg)


def numpy_forward(c, layers, keep, ids):
    """float64 restatement of GQAImpl::forward + GQAInference::forward (fp32 KV,
    prefill of all ids, logits of the last row)."""
    d, H, Hkv, dh, V = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["vocab"]
    T = len(ids)
    h = keep["wte"].reshape(V, d)[ids].astype(np.float64)

    def rms(x, w):
        return x / np.sqrt((x ** 2).mean(1, keepdims=True) + 1e-5) * w

    for Lw in layers:
        a = rms(h, Lw["ln1"])
        q = (a @ Lw["q"][1].T).reshape(T, H, dh)
        k = (a @ Lw["k"][1].T).reshape(T, Hkv, dh)
        v = (a @ Lw["v"][1].T).reshape(T, Hkv, dh)
        q = nr.rope_neox(q, keep["cos"], keep["sin"], 0)
        k = nr.rope_neox(k, keep["cos"], keep["sin"], 0)
        att = np.zeros((T, H, dh))
        for t in range(T):
            for hh in range(H):
                g = hh // (H // Hkv)
                att[t, hh] = nr.softmax_attn(q[t, hh], k[: t + 1, g], v[: t + 1, g], 1 / np.sqrt(dh))
        h = h + att.reshape(T, H * dh) @ Lw["o"][1].T
        a = rms(h, Lw["ln2"])
        gg = a @ Lw["1"][1].T
        uu = a @ Lw["3"][1].T
        h = h + (gg / (1 + np.exp(-gg)) * uu) @ Lw["2"][1].T
    hl = rms(h[-1:], keep["ln_f"])
    return (hl @ keep["wte"].reshape(V, d).T)[0]


def test_tiny_model_vs_float64(orc):
    c, layers, keep = build_tiny(orc)
    m, hold = oracle_model(orc, c, layers, keep)
    L = orc.load()
    ids = np.array([5, 17, 3, 90, 42, 7], np.int32)
    logits = np.zeros(c["vocab"], np.float32)
    assert L.orc_gqa_forward(m, ids.ctypes.data, len(ids), 0, logits.ctypes.data, 1) == 0
    ref = numpy_forward(c, layers, keep, ids)
    assert np.max(np.abs(logits - ref)) <= 1e-4 * np.max(np.abs(ref))
    # incremental decode over the fp32 cache equals the full recompute
    m2, hold2 = oracle_model(orc, c, layers, keep)
    L.orc_gqa_forward(m2, ids.ctypes.data, 4, 0, logits.ctypes.data, 1)
    L.orc_gqa_forward(m2, ids[4:].ctypes.data, 1, 4, logits.ctypes.data, 1)
    L.orc_gqa_forward(m2, ids[5:].ctypes.data, 1, 5, logits.ctypes.data, 1)
    assert np.max(np.abs(logits - ref)) <= 1e-4 * np.max(np.abs(ref))
    L.orc_gqa_destroy(m)
    L.orc_gqa_destroy(m2)


def test_tiny_model_greedy_matches_float64(orc):
    c, layers, keep = build_tiny(orc, seed=6)
    m, hold = oracle_model(orc, c, layers, keep)
    L = orc.load()
    prompt = np.array([1, 2, 3, 4], np.int32)
    out = np.zeros(6, np.int32)
    assert L.orc_gqa_generate(m, prompt.ctypes.data, 4, 6, out.ctypes.data) == 0
    ids = list(prompt)
    for s in range(6):
        ref = numpy_forward(c, layers, keep, np.array(ids, np.int32))
        top = np.argsort(ref)[::-1]
        assert ref[top[0]] - ref[top[1]] > 1e-6, "near tie: choose another seed"
        ids.append(int(top[0]))
    assert list(out) == ids[4:]
    L.orc_gqa_destroy(m)
