"""DeepSeek MLA + MoE on the GPU: the latent decode attention and the MoE
kernels against float64 restatements of the intended math, the router
top-k against the oracle, and the engine's "mla" Inference (logits and
greedy tokens) against the CPU oracle model."""
import ctypes as C
import importlib

import numpy as np
import pytest

import _mla_tiny as mt
import _numpy_ref as nr
from _util import assert_close, assert_close_elem, dev, empty, host, ok, rng, stream

pytestmark = pytest.mark.gpu

Q2K, Q4F, FP32, Q40 = 10, 7, 6, 5


def rope_tables(rope, n, theta=10000.0):
    ang = np.outer(np.arange(n), 1.0 / theta ** (np.arange(0, rope, 2) / rope)).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def weight(orc, qt, rows, cols, r):
    """packed weight + its float64 matrix (numpy restatement dequant)"""
    if qt == Q2K:
        w = mt.q2k_random(r, rows * cols)
        return w, nr.dequant_q2k_blocks(w)[: rows * cols].reshape(rows, cols).astype(np.float64)
    wf = (r.standard_normal(rows * cols) * 0.05).astype(np.float32)
    if qt == FP32:
        return wf, wf.reshape(rows, cols).astype(np.float64)
    w = orc.pack(qt, wf)
    return w, nr.dequant_q4(w, rows * cols, qt == Q4F).reshape(rows, cols).astype(np.float64)


@pytest.mark.parametrize("shape,T", [("tiny", 2), ("tiny", 37), ("dsv2lite", 17), ("dsv2lite", 300)])
@pytest.mark.parametrize("qt", [Q2K, Q4F, Q40])
def test_mla_prompt_attention_matches_decode_rows(rina, orc, shape, T, qt):
    """A prompt of T rows from position 0 in one call (the prefill's causal
    attention in the expanded form: T-row products of W_kb / W_vb, one causal
    attention over the rows) against the same rows fed to the decode
    attention one position at a time: the T appended latent records bit for
    bit, every output row within tolerance, and row T-1 against the float64
    expanded form."""
    hip = rina.load_hip()
    H, nope, rope, vd, dc = (4, 32, 16, 32, 64) if shape == "tiny" else (16, 128, 64, 128, 512)
    R = dc + rope
    max_seq = T + 5
    r = rng(T * 7 + H + qt)
    wkvb, W = weight(orc, qt, H * (nope + vd), dc, r)
    q = r.standard_normal((T, H * (nope + rope))).astype(np.float32)
    kva = r.standard_normal((T, R)).astype(np.float32)
    knorm = r.uniform(0.8, 1.2, dc).astype(np.float32)
    cos, sin = rope_tables(rope, max_seq)
    qd, kd, nd, cdv, sdv, wd = dev(q), dev(kva), dev(knorm), dev(cos), dev(sin), dev(wkvb)
    # one position at a time
    c1 = dev(np.zeros((max_seq, R), np.float32))
    ws_bytes = hip.rina_hip_mla_attention_workspace(H, dc, rope, max_seq)
    ws = empty(ws_bytes, "uint8")
    o1 = np.zeros((T, H * vd), np.float32)
    od = empty(H * vd)
    for t in range(T):
        ok(hip.rina_hip_mla_decode_attention_ex(qd.data_ptr() + 4 * t * q.shape[1], kd.data_ptr() + 4 * t * R,
                                                nd.data_ptr(), np.float32(1e-5), cdv.data_ptr(), sdv.data_ptr(),
                                                wd.data_ptr(), qt, c1.data_ptr(), H, nope, rope, vd, dc, t, None,
                                                max_seq, -1, od.data_ptr(), ws.data_ptr(), ws_bytes, stream()),
           "decode row %d" % t)
        o1[t] = host(od)
    # the prompt in one call
    c2 = dev(np.zeros((max_seq, R), np.float32))
    pws = hip.rina_hip_mla_prompt_workspace(T, H, nope, rope, vd, dc)
    pw = empty(pws, "uint8")
    o2 = empty(T * H * vd)
    ok(hip.rina_hip_mla_prompt_attention(qd.data_ptr(), kd.data_ptr(), nd.data_ptr(), np.float32(1e-5),
                                         cdv.data_ptr(), sdv.data_ptr(), wd.data_ptr(), qt, c2.data_ptr(), H, nope,
                                         rope, vd, dc, T, max_seq, o2.data_ptr(), pw.data_ptr(), pws, stream()),
       "prompt attention")
    assert np.array_equal(host(c2).view(np.uint32), host(c1).view(np.uint32))
    got = host(o2).reshape(T, H * vd)
    for t in range(T):
        assert_close_elem(got[t], o1[t], what="prompt row %d vs decode row" % t)
    # row T-1 against the float64 expanded form over the appended records
    allc = host(c2).reshape(max_seq, R).astype(np.float64)
    L = orc.load()
    qr = q[T - 1].copy()
    L.orc_rope_neox(qr[H * nope:].ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, H, rope, T - 1)
    ref = np.zeros(H * vd)
    for hh in range(H):
        Kn = allc[:T, :dc] @ W[hh * nope:(hh + 1) * nope].T
        K = np.concatenate([Kn, allc[:T, dc:]], axis=1)
        V = allc[:T, :dc] @ W[H * nope + hh * vd: H * nope + (hh + 1) * vd].T
        qh = np.concatenate([qr[hh * nope:(hh + 1) * nope], qr[H * nope + hh * rope: H * nope + (hh + 1) * rope]])
        ref[hh * vd:(hh + 1) * vd] = nr.softmax_attn(qh.astype(np.float64), K, V, 1 / np.sqrt(nope + rope))
    assert_close_elem(got[T - 1], ref, what="prompt last row vs float64")


def test_mla_prompt_attention_rejects(rina):
    """Shapes the prompt path does not take return before any launch."""
    hip = rina.load_hip()
    buf = empty(1 << 16)
    p = buf.data_ptr()
    ws = hip.rina_hip_mla_prompt_workspace(4, 2, 32, 16, 32, 64)
    assert hip.rina_hip_mla_prompt_attention(p, p, p, np.float32(1e-5), p, p, p, FP32, p, 2, 32, 16, 32, 1024, 4, 8,
                                             p, p, 1 << 18, stream()) == -3        # RINA_ERR_SHAPE: dc > 512
    assert hip.rina_hip_mla_prompt_attention(p, p, p, np.float32(1e-5), p, p, p, FP32, p, 2, 32, 16, 64, 64, 4, 8,
                                             p, p, 1 << 18, stream()) == -3        # v_dim > nope + rope
    assert hip.rina_hip_mla_prompt_attention(p, p, p, np.float32(1e-5), p, p, p, FP32, p, 2, 32, 16, 32, 64, 9, 8,
                                             p, p, 1 << 18, stream()) == -4        # RINA_ERR_RANGE: T > max_seq
    assert hip.rina_hip_mla_prompt_attention(p, p, p, np.float32(1e-5), p, p, p, FP32, p, 2, 32, 16, 32, 64, 4, 8,
                                             p, p, ws - 4, stream()) == -6   # RINA_ERR_WORKSPACE


@pytest.mark.parametrize("shape", ["tiny", "dsv2lite"])
@pytest.mark.parametrize("qt", [Q2K, Q4F, Q40])
# (position, device position, pos_hint, minimum max_seq).  At the
# DeepSeek-V2-Lite shape: one-launch path below 256 positions (one and
# several 64-position blocks, a device position past its hint); above it the
# chunk + combine launches, whose chunks follow the position count: 257
# (5 slots, the last chunk 2 positions), 300, 700 (11 one-block chunks),
# 1100 with a 4100-position cache (16 slots, 9 chunks of two blocks) and a
# device position with no usable bound.  The tiny shape takes the
# three-launch path above 256.
@pytest.mark.parametrize("P,use_dpos,hint,min_seq", [(0, False, -1, 0), (5, False, -1, 0), (40, True, -1, 0),
                                                     (40, True, -1, 400), (40, True, 63, 400), (100, False, -1, 0),
                                                     (200, True, 10, 0), (257, True, -1, 0), (300, False, -1, 0),
                                                     (700, False, -1, 0), (1100, True, -1, 4100)])
def test_mla_decode_attention(rina, orc, shape, qt, P, use_dpos, hint, min_seq):
    hip = rina.load_hip()
    L = orc.load()
    H, nope, rope, vd, dc = (4, 32, 16, 32, 64) if shape == "tiny" else (16, 128, 64, 128, 512)
    R = dc + rope
    max_seq = max(P + 7, min_seq)
    r = rng(P * 3 + H + qt)
    wkvb, W = weight(orc, qt, H * (nope + vd), dc, r)
    q = r.standard_normal(H * (nope + rope)).astype(np.float32)
    kva = r.standard_normal(R).astype(np.float32)
    knorm = r.uniform(0.8, 1.2, dc).astype(np.float32)
    cos, sin = rope_tables(rope, max_seq)
    cache = r.standard_normal((max_seq, R)).astype(np.float32)     # records of earlier positions
    # expected record at P: RMSNorm(c)*k_norm (oracle fp32 rule), RoPE(k_pe) (oracle, bit-exact)
    rec = np.zeros(R, np.float32)
    c = kva[:dc].copy()
    L.orc_rms_norm(c.ctypes.data, knorm.ctypes.data, 1, dc, np.float32(1e-5))
    kpe = kva[dc:].copy()
    L.orc_rope_neox(kpe.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, 1, rope, P)
    rec[:dc], rec[dc:] = c, kpe
    # float64 reference over the expanded form
    qr = q.copy()
    L.orc_rope_neox(qr[H * nope:].ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, H, rope, P)
    allc = cache.astype(np.float64).copy()
    allc[P] = rec
    ref = np.zeros(H * vd)
    for hh in range(H):
        Kn = allc[: P + 1, :dc] @ W[hh * nope:(hh + 1) * nope].T            # [P+1, nope]
        K = np.concatenate([Kn, allc[: P + 1, dc:]], axis=1)
        V = allc[: P + 1, :dc] @ W[H * nope + hh * vd: H * nope + (hh + 1) * vd].T
        qh = np.concatenate([qr[hh * nope:(hh + 1) * nope], qr[H * nope + hh * rope: H * nope + (hh + 1) * rope]])
        ref[hh * vd:(hh + 1) * vd] = nr.softmax_attn(qh.astype(np.float64), K, V, 1 / np.sqrt(nope + rope))
    ws_bytes = hip.rina_hip_mla_attention_workspace(H, dc, rope, max_seq)
    ws = empty(ws_bytes, "uint8")
    cd = dev(cache)
    od = empty(H * vd)
    pos = dev(np.array([P], np.int32)) if use_dpos else None
    ok(hip.rina_hip_mla_decode_attention_ex(dev(q).data_ptr(), dev(kva).data_ptr(), dev(knorm).data_ptr(),
                                            np.float32(1e-5), dev(cos).data_ptr(), dev(sin).data_ptr(),
                                            dev(wkvb).data_ptr(), qt, cd.data_ptr(), H, nope, rope, vd, dc,
                                            0 if use_dpos else P, pos.data_ptr() if use_dpos else None, max_seq,
                                            hint, od.data_ptr(), ws.data_ptr(), ws_bytes, stream()), "mla attention")
    assert_close_elem(host(od), ref, what="mla %s qt %d P %d" % (shape, qt, P))
    gc = host(cd).reshape(max_seq, R)
    assert np.array_equal(gc[P, dc:].view(np.uint32), kpe.view(np.uint32))     # RoPE: same fma form
    assert np.max(np.abs(gc[P, :dc] - c)) <= 1e-6 * np.max(np.abs(c))          # norm: sum order differs
    others = np.ones(max_seq, bool)
    others[P] = False
    assert np.array_equal(gc[others], cache[others])


def test_moe_topk_matches_oracle(rina, orc):
    hip = rina.load_hip()
    r = rng(77)
    checked = 0
    for trial in range(40):
        E, k = (64, 6) if trial % 2 == 0 else (8, 3)
        lg = (r.standard_normal(E) * 1.5).astype(np.float32)
        p = np.sort(np.exp(lg - lg.max()) / np.exp(lg - lg.max()).sum())[::-1]
        if p[k - 1] - p[k] < 1e-5:
            continue
        ids_o, pr_o = orc.moe_topk(lg, k)
        ids, pr = empty(k, "int32"), empty(k)
        ok(hip.rina_hip_moe_topk(dev(lg).data_ptr(), E, k, ids.data_ptr(), pr.data_ptr(), stream()), "topk")
        assert host(ids).tolist() == ids_o.tolist()
        assert np.allclose(host(pr), pr_o, rtol=2e-6, atol=0)
        checked += 1
    assert checked >= 30


def packed_only(orc, qt, rows, cols, r):
    if qt == Q2K:
        return mt.q2k_random(r, rows * cols)
    return orc.pack(qt, (r.standard_normal(rows * cols) * 0.05).astype(np.float32))


def as_f64(qt, w, rows, cols):
    if qt == Q2K:
        return nr.dequant_q2k_blocks(w)[: rows * cols].reshape(rows, cols).astype(np.float64)
    return nr.dequant_q4(w, rows * cols, qt == Q4F).reshape(rows, cols).astype(np.float64)


@pytest.mark.parametrize("d,F,E,k,qt", [(256, 48, 8, 3, Q2K), (2048, 1408, 64, 6, Q2K), (512, 96, 4, 2, Q4F)])
def test_moe_ffn_vs_float64(rina, orc, d, F, E, k, qt):
    hip = rina.load_hip()
    r = rng(d + F + k)
    parts = {nm: [packed_only(orc, qt, *shp, r) for _ in range(E)] for nm, shp in
             (("g", (F, d)), ("u", (F, d)), ("dn", (d, F)))}
    gate, up, down = (np.concatenate(parts[nm]) for nm in ("g", "u", "dn"))
    sgu, sdn = gate.nbytes // E, down.nbytes // E
    x = r.standard_normal(d).astype(np.float32)
    ids = np.sort(r.choice(E, k, replace=False)).astype(np.int32)
    ids[0] = -1 if k > 2 else ids[0]                                    # a skipped slot
    probs = np.sort(r.uniform(0.05, 0.3, k)).astype(np.float32)
    shared = r.standard_normal(d).astype(np.float32)
    h0 = r.standard_normal(d).astype(np.float32)
    acc = shared.astype(np.float64).copy()
    for j in range(k):
        e = ids[j]
        if e < 0:
            continue
        g = as_f64(qt, parts["g"][e], F, d) @ x
        u = as_f64(qt, parts["u"][e], F, d) @ x
        acc += probs[j] * (as_f64(qt, parts["dn"][e], d, F) @ (g / (1 + np.exp(-g)) * u))
    ref = h0 + acc
    hd = dev(h0)
    wsb = hip.rina_hip_moe_workspace(k, F)
    ws = empty(wsb, "uint8")
    ok(hip.rina_hip_moe_ffn(dev(x).data_ptr(), dev(gate).data_ptr(), dev(up).data_ptr(), dev(down).data_ptr(), qt,
                            sgu, sdn, E, dev(ids).data_ptr(), dev(probs).data_ptr(), k, d, F, dev(shared).data_ptr(),
                            hd.data_ptr(), ws.data_ptr(), wsb, stream()), "moe ffn")
    assert_close(host(hd), ref, what="moe d %d F %d" % (d, F))


@pytest.mark.parametrize("d,F,S,E,k", [(2048, 1408, 2816, 64, 6), (256, 64, 128, 8, 3), (512, 96, 192, 16, 4),
                                       (1024, 2048, 64, 32, 2),
                                       # shared and expert widths multiples of 128 (the down
                                       # kernel's quad column loads)
                                       (256, 128, 256, 8, 3), (512, 256, 128, 16, 4)])
def test_moe_block_vs_float64(rina, orc, d, F, S, E, k):
    """Fused MoE block (norm, router, top-k, shared + routed experts, residual)
    against a float64 restatement of forward_moe; selected ids and probs
    against the oracle's top-k of the float64 logits."""
    hip = rina.load_hip()
    r = rng(d + F + S + k)
    parts = {nm: [packed_only(orc, Q2K, *shp, r) for _ in range(E)] for nm, shp in
             (("g", (F, d)), ("u", (F, d)), ("dn", (d, F)))}
    gate, up, down = (np.concatenate(parts[nm]) for nm in ("g", "u", "dn"))
    sgu, sdn = gate.nbytes // E, down.nbytes // E
    sg, sg64 = weight(orc, Q2K, S, d, r)
    su, su64 = weight(orc, Q2K, S, d, r)
    sd, sd64 = weight(orc, Q2K, d, S, r)
    wr = (r.standard_normal((E, d)) * 0.05).astype(np.float32)
    ln2 = r.uniform(0.8, 1.2, d).astype(np.float32)
    h0 = (r.standard_normal(d) * 2).astype(np.float32)
    h64 = h0.astype(np.float64)
    a2 = h64 / np.sqrt((h64 ** 2).mean() + 1e-5) * ln2
    lg = wr.astype(np.float64) @ a2
    p = np.exp(lg - lg.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    assert p[order[k - 1]] - p[order[k]] > 1e-4, "router near tie: choose another seed"
    ids_o, pr_o = orc.moe_topk(lg.astype(np.float32), k)

    def silu(v):
        return v / (1 + np.exp(-v))

    acc = sd64 @ (silu(sg64 @ a2) * (su64 @ a2))
    for j in range(k):
        e = ids_o[j]
        g = as_f64(Q2K, parts["g"][e], F, d) @ a2
        u = as_f64(Q2K, parts["u"][e], F, d) @ a2
        acc = acc + p[e] * (as_f64(Q2K, parts["dn"][e], d, F) @ (silu(g) * u))
    ref = h64 + acc
    hd = dev(h0)
    wsb = hip.rina_hip_moe_block_workspace(d, E, k, F, S)
    ws = empty(wsb // 4 + 4)
    keep = [dev(t) for t in (ln2, wr, sg, su, sd, gate, up, down)]
    ok(hip.rina_hip_moe_block(hd.data_ptr(), keep[0].data_ptr(), np.float32(1e-5), keep[1].data_ptr(), FP32,
                              keep[2].data_ptr(), keep[3].data_ptr(), keep[4].data_ptr(), S, keep[5].data_ptr(),
                              keep[6].data_ptr(), keep[7].data_ptr(), Q2K, sgu, sdn, E, k, d, F, ws.data_ptr(), wsb,
                              stream()), "moe block")
    assert_close(host(hd), ref, what="moe block d %d F %d S %d" % (d, F, S))
    wh = host(ws)
    n = S + k * F
    got_ids = wh[n + d + E: n + d + E + k].view(np.int32)
    assert got_ids.tolist() == ids_o.tolist()
    assert np.allclose(wh[n + d + E + k: n + d + E + 2 * k], pr_o, rtol=1e-5, atol=0)
    # a second call on the updated stream reuses the workspace
    ok(hip.rina_hip_moe_block(hd.data_ptr(), keep[0].data_ptr(), np.float32(1e-5), keep[1].data_ptr(), FP32,
                              keep[2].data_ptr(), keep[3].data_ptr(), keep[4].data_ptr(), S, keep[5].data_ptr(),
                              keep[6].data_ptr(), keep[7].data_ptr(), Q2K, sgu, sdn, E, k, d, F, ws.data_ptr(), wsb,
                              stream()), "moe block 2")
    assert np.all(np.isfinite(host(hd)))


@pytest.mark.parametrize("d,F,S,E,k,T", [(2048, 1408, 2816, 64, 6, 40), (256, 64, 128, 8, 3, 1), (256, 64, 128, 8, 3, 33),
                                         (512, 96, 192, 16, 4, 17)])
def test_moe_rows_matches_block_rows(rina, orc, d, F, S, E, k, T):
    """The MoE block over a prompt's T rows in one call (T-row products, rows
    grouped by expert) against the fused single-row block applied to each
    row, within tolerance; row 0 against a float64 restatement of
    forward_moe."""
    hip = rina.load_hip()
    r = rng(d + F + S + k + T)
    parts = {nm: [packed_only(orc, Q2K, *shp, r) for _ in range(E)] for nm, shp in
             (("g", (F, d)), ("u", (F, d)), ("dn", (d, F)))}
    gate, up, down = (np.concatenate(parts[nm]) for nm in ("g", "u", "dn"))
    sgu, sdn = gate.nbytes // E, down.nbytes // E
    sg, sg64 = weight(orc, Q2K, S, d, r)
    su, su64 = weight(orc, Q2K, S, d, r)
    sd, sd64 = weight(orc, Q2K, d, S, r)
    wr = (r.standard_normal((E, d)) * 0.05).astype(np.float32)
    ln2 = r.uniform(0.8, 1.2, d).astype(np.float32)
    h0 = (r.standard_normal((T, d)) * 2).astype(np.float32)
    keep = [dev(t) for t in (ln2, wr, sg, su, sd, gate, up, down)]
    # one row at a time through the fused block
    hb = dev(h0)
    wsb = hip.rina_hip_moe_block_workspace(d, E, k, F, S)
    ws = empty(wsb // 4 + 4)
    for t in range(T):
        ok(hip.rina_hip_moe_block(hb.data_ptr() + 4 * t * d, keep[0].data_ptr(), np.float32(1e-5), keep[1].data_ptr(),
                                  FP32, keep[2].data_ptr(), keep[3].data_ptr(), keep[4].data_ptr(), S,
                                  keep[5].data_ptr(), keep[6].data_ptr(), keep[7].data_ptr(), Q2K, sgu, sdn, E, k, d, F,
                                  ws.data_ptr(), wsb, stream()), "moe block row %d" % t)
    # all rows at once
    hr = dev(h0)
    mwb = hip.rina_hip_moe_rows_workspace(T, d, E, k, F, S)
    mws = empty(mwb // 4 + 4)
    ok(hip.rina_hip_moe_rows(hr.data_ptr(), T, keep[0].data_ptr(), np.float32(1e-5), keep[1].data_ptr(), FP32,
                             keep[2].data_ptr(), keep[3].data_ptr(), keep[4].data_ptr(), S, Q2K, keep[5].data_ptr(),
                             keep[6].data_ptr(), keep[7].data_ptr(), Q2K, sgu, sdn, E, k, d, F, mws.data_ptr(), mwb,
                             stream()), "moe rows")
    got, want = host(hr).reshape(T, d), host(hb).reshape(T, d)
    for t in range(T):
        assert_close(got[t], want[t], what="moe rows, row %d" % t)
    # row 0 against float64 forward_moe (skipped at a router near tie)
    h64 = h0[0].astype(np.float64)
    a2 = h64 / np.sqrt((h64 ** 2).mean() + 1e-5) * ln2
    lg = wr.astype(np.float64) @ a2
    p = np.exp(lg - lg.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    if p[order[k - 1]] - p[order[k]] > 1e-4:
        def silu(v):
            return v / (1 + np.exp(-v))
        acc = sd64 @ (silu(sg64 @ a2) * (su64 @ a2))
        for e in order[:k]:
            g = as_f64(Q2K, parts["g"][e], F, d) @ a2
            u = as_f64(Q2K, parts["u"][e], F, d) @ a2
            acc = acc + p[e] * (as_f64(Q2K, parts["dn"][e], d, F) @ (silu(g) * u))
        assert_close(got[0], h64 + acc, what="moe rows, row 0 vs float64")


def test_moe_block_rejects_unsupported(rina):
    hip = rina.load_hip()
    buf = empty(1 << 16)
    ptr = buf.data_ptr()
    args = lambda d, F, S, E, k, qt, qr: (ptr, ptr, np.float32(1e-5), ptr, qr, ptr, ptr, ptr, S, ptr, ptr, ptr, qt,
                                          256, 256, E, k, d, F, ptr, 1 << 18, stream())
    assert hip.rina_hip_moe_block(*args(256, 48, 64, 8, 3, Q2K, FP32)) == -3    # F % 32
    assert hip.rina_hip_moe_block(*args(160, 64, 64, 8, 3, Q2K, FP32)) == -3    # d % 128
    assert hip.rina_hip_moe_block(*args(256, 64, 64, 8, 3, Q4F, FP32)) == -2
    assert hip.rina_hip_moe_block(*args(256, 64, 64, 8, 3, Q2K, Q2K)) == -2    # router not fp32
    assert hip.rina_hip_moe_block(*args(4096, 64, 64, 8, 3, Q2K, FP32)) == -3
    assert hip.rina_hip_moe_block(*args(256, 64, 64, 128, 3, Q2K, FP32)) == -3  # E > 64
    assert hip.rina_hip_moe_block(*args(256, 64, 64 * 300, 8, 7, Q2K, FP32)) == -3   # shared + k ffn > 16384


# ---- engine ---------------------------------------------------------------

def header(max_seq):
    c = mt.CFG
    return {"name": c["name"], "dim": c["dim"], "n_layers": c["n_layers"], "n_heads": c["n_heads"],
            "n_kv_heads": c["n_heads"], "head_dim": c["nope"], "qk_nope_head_dim": c["nope"],
            "qk_rope_head_dim": c["rope"], "v_head_dim": c["v_dim"], "kv_lora_rank": c["dc"],
            "vocab_size": c["vocab_size"], "max_seq_len": max_seq, "n_routed_experts": c["n_experts"],
            "num_experts_per_tok": c["top_k"], "moe_intermediate_size": c["expert_ffn"],
            "layers": [{"type": "deepseek_mla_dense"}] + [{"type": "deepseek_mla_moe"}] * (c["n_layers"] - 1)}


def shape_of(name, arr, qt):
    c = mt.CFG
    if qt == FP32:
        return arr.shape if arr.ndim > 1 else (arr.size,)
    rows = {"w_q": c["n_heads"] * (c["nope"] + c["rope"]), "w_kv_a": c["dc"] + c["rope"],
            "w_kv_b": c["n_heads"] * (c["nope"] + c["v_dim"]), "w_o": c["dim"], "w1": c["dense_ffn"],
            "w3": c["dense_ffn"], "w2": c["dim"], "gate_exps": c["expert_ffn"], "up_exps": c["expert_ffn"],
            "down_exps": c["dim"], "gate_shexp": c["shared_ffn"], "up_shexp": c["shared_ffn"],
            "down_shexp": c["dim"], "wte": c["vocab_size"], "lm_head": c["vocab_size"]}
    key = name.split(".")[-2]
    n = rows[key]
    if key.endswith("exps"):
        return (c["n_experts"], n, -1)
    return (n, -1)


@pytest.fixture(scope="module")
def tiny_mla(rina):
    synth = importlib.import_module("rina_amd.synth")
    max_seq = 48
    tensors, qts, mats = mt.build(seed=11, max_pos=max_seq)
    up = {}
    for nm, arr in tensors.items():
        shp = list(shape_of(nm, arr, qts[nm]))
        if shp[-1] == -1:       # cols of a packed matrix
            c = mt.CFG
            cols = {"w_kv_b": c["dc"], "w_o": c["n_heads"] * c["v_dim"], "w2": c["dense_ffn"],
                    "down_exps": c["expert_ffn"], "down_shexp": c["shared_ffn"]}.get(nm.split(".")[-2], c["dim"])
            shp[-1] = cols
        up[nm] = (qts[nm], tuple(shp), arr)
    hm = synth.HostModel(header(max_seq), up)
    yield hm, tensors, qts, max_seq
    hm.close()


def test_mla_engine_forward_logits(rina, orc, tiny_mla):
    import torch
    hm, tensors, qts, max_seq = tiny_mla
    eng = rina.load_engine()
    inf = hm.infer("mla", max_seq=max_seq)
    V = mt.CFG["vocab_size"]
    ids = np.array([5, 17, 3, 90, 42, 7], np.int32)
    lg = empty(len(ids) * V)
    rina.check(eng.rina_infer_forward(inf, torch.from_numpy(ids).cuda().data_ptr(), lg.data_ptr(), 1, len(ids), 0,
                                      stream()), "forward")
    m, hold = orc.mla_from_tensors(mt.CFG, tensors, qts, max_seq)
    ref = np.zeros((len(ids), V), np.float32)
    assert orc.load().orc_mla_forward(m, ids.ctypes.data, len(ids), 0, ref.ctypes.data, 0) == 0
    assert_close(host(lg).reshape(len(ids), V), ref, what="mla prefill logits")
    nxt = np.array([11], np.int32)
    rina.check(eng.rina_infer_forward(inf, torch.from_numpy(nxt).cuda().data_ptr(), lg.data_ptr(), 1, 1, 6,
                                      stream()), "decode")
    ref1 = np.zeros(V, np.float32)
    orc.load().orc_mla_forward(m, nxt.ctypes.data, 1, 6, ref1.ctypes.data, 0)
    assert_close(host(lg)[:V], ref1, what="mla decode logits")
    orc.load().orc_mla_destroy(m)
    eng.rina_infer_destroy(inf)


@pytest.mark.parametrize("use_graph", [True, False])
def test_mla_engine_greedy_identical(rina, orc, tiny_mla, use_graph):
    hm, tensors, qts, max_seq = tiny_mla
    eng = rina.load_engine()
    inf = hm.infer("mla", max_seq=max_seq)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    steps = 20
    out = (C.c_int * steps)()
    rina.check(eng.rina_infer_generate(inf, (C.c_int * len(prompt))(*prompt), len(prompt), steps, out,
                                       1 if use_graph else 0, stream(), None), "generate")
    eng.rina_infer_destroy(inf)
    m, hold = orc.mla_from_tensors(mt.CFG, tensors, qts, max_seq)
    ref = orc.mla_generate(m, prompt, steps)
    orc.load().orc_mla_destroy(m)
    assert list(out) == ref


def test_mla_engine_full_width_greedy(rina, orc):
    """DeepSeek-V2-Lite widths (3 layers: dense + 2 MoE, vocab 102400, 64
    experts of 1408): greedy tokens identical to the oracle."""
    synth = importlib.import_module("rina_amd.synth")
    sm = synth.SynthDeepSeek(seed=5, max_seq=64, keep_host=True, n_layers=3)
    try:
        eng = rina.load_engine()
        inf = sm.infer()
        prompt = [101, 2047, 9, 55555, 3, 777]
        steps = 5
        out = (C.c_int * steps)()
        rina.check(eng.rina_infer_generate(inf, (C.c_int * len(prompt))(*prompt), len(prompt), steps, out, 1,
                                           stream(), None), "generate")
        eng.rina_infer_destroy(inf)
        m, hold = orc.mla_from_tensors(sm.cfg, sm.host, sm.qts, 64)
        ref = orc.mla_generate(m, prompt, steps)
        orc.load().orc_mla_destroy(m)
        assert list(out) == ref
    finally:
        sm.close()


def test_mla_graph_recaptured_after_buffer_growth(rina, orc):
    """The MLA Inference starts with 64 activation rows: a graph captured
    after a short prompt must be dropped when a 70-token prompt grows them.
    Tokens after the long prompt equal a fresh Inference's and the oracle's."""
    synth = importlib.import_module("rina_amd.synth")
    max_seq = 96
    tensors, qts, mats = mt.build(seed=11, max_pos=max_seq)
    up = {}
    for nm, arr in tensors.items():
        shp = list(shape_of(nm, arr, qts[nm]))
        if shp[-1] == -1:
            c = mt.CFG
            shp[-1] = {"w_kv_b": c["dc"], "w_o": c["n_heads"] * c["v_dim"], "w2": c["dense_ffn"],
                       "down_exps": c["expert_ffn"], "down_shexp": c["shared_ffn"]}.get(nm.split(".")[-2], c["dim"])
        up[nm] = (qts[nm], tuple(shp), arr)
    hm = synth.HostModel(header(max_seq), up)
    try:
        eng = rina.load_engine()
        steps = 5
        short = [3, 1, 4, 1, 5]
        long_prompt = [int(x) for x in np.random.default_rng(2).integers(0, mt.CFG["vocab_size"], 70)]
        out = (C.c_int * steps)()

        def gen(inf, prompt):
            rina.check(eng.rina_infer_generate(inf, (C.c_int * len(prompt))(*prompt), len(prompt), steps, out, 1,
                                               stream(), None), "generate")
            return list(out)

        inf = hm.infer("mla", max_seq=max_seq)
        gen(inf, short)
        reused = gen(inf, long_prompt)
        eng.rina_infer_destroy(inf)
        fresh = hm.infer("mla", max_seq=max_seq)
        assert gen(fresh, long_prompt) == reused
        eng.rina_infer_destroy(fresh)
        m, hold = orc.mla_from_tensors(mt.CFG, tensors, qts, max_seq)
        ref = orc.mla_generate(m, long_prompt, steps)
        orc.load().orc_mla_destroy(m)
        assert reused == ref
    finally:
        hm.close()
