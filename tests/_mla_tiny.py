"""A tiny DeepSeek-MLA + MoE model (1 dense + 2 MoE layers) with Q2_K
linears, and a float64 numpy restatement of its forward pass (the intended
math of arch/mla/deepseek_mla_layer.cu:171-350 at any start_pos).  Shared by
the oracle tests and the GPU engine tests."""
import numpy as np

import _numpy_ref as nr

Q2K, FP32 = 10, 6

CFG = dict(dim=256, n_layers=3, n_heads=4, nope=32, rope=16, v_dim=32, dc=64, vocab_size=97, dense_ffn=96,
           n_experts=8, top_k=3, expert_ffn=48, shared_ffn=64, name="deepseek-tiny")


def q2k_random(r, n, std=0.05):
    """Zero-mean Q2_K blocks: min nibble = scale nibble, dmin = 1.5 d, so an
    element is d*sc*(q - 1.5) (the rule of rina_amd.synth.random_q2k)."""
    nb = (n + 255) // 256
    blk = np.zeros((nb, 84), np.uint8)
    blk[:, 0:80] = r.integers(0, 256, (nb, 80), dtype=np.uint8)
    sc = blk[:, 0:16] & 15
    blk[:, 0:16] = sc | (sc << 4)
    d = np.float16(std / 9.84)
    dmin = np.float16(np.float32(d) * np.float32(1.5))
    blk[:, 80:82] = np.frombuffer(np.array([d], np.float16).tobytes(), np.uint8)
    blk[:, 82:84] = np.frombuffer(np.array([dmin], np.float16).tobytes(), np.uint8)
    return blk.reshape(-1)


def build(seed=11, max_pos=64, cfg=CFG):
    """tensors: name -> packed bytes / fp32; qts: name -> quant type;
    mats: name -> float64 matrix (dequantized with the numpy restatement)."""
    c = cfg
    r = np.random.default_rng(seed)
    d, H, nope, rope, vd, dc = c["dim"], c["n_heads"], c["nope"], c["rope"], c["v_dim"], c["dc"]
    E, F, S, hd, V = c["n_experts"], c["expert_ffn"], c["shared_ffn"], c["dense_ffn"], c["vocab_size"]
    tensors, qts, mats = {}, {}, {}

    def q2(name, rows, cols, experts=1):
        n = rows * cols
        nb = (n + 255) // 256
        parts = [q2k_random(r, n) for _ in range(experts)]
        w = np.concatenate(parts)
        tensors[name], qts[name] = w, Q2K
        deq = [nr.dequant_q2k_blocks(p)[:n].reshape(rows, cols).astype(np.float64) for p in parts]
        mats[name] = deq[0] if experts == 1 else np.stack(deq)
        assert w.size == experts * nb * 84

    def f32(name, a):
        tensors[name], qts[name] = a.astype(np.float32), FP32
        mats[name] = a.astype(np.float64)

    ang = np.outer(np.arange(max_pos), 1.0 / 10000 ** (np.arange(0, rope, 2) / rope)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    for l in range(c["n_layers"]):
        p = "transformer.h.%d." % l
        q2(p + "attn.w_q.weight", H * (nope + rope), d)
        q2(p + "attn.w_kv_a.weight", dc + rope, d)
        f32(p + "attn.k_norm.weight", r.uniform(0.8, 1.2, dc))
        q2(p + "attn.w_kv_b.weight", H * (nope + vd), dc)
        q2(p + "attn.w_o.weight", d, H * vd)
        f32(p + "ln1.weight", r.uniform(0.8, 1.2, d))
        f32(p + "ln2.weight", r.uniform(0.8, 1.2, d))
        f32(p + "attn.rope_q.cos", cos)
        f32(p + "attn.rope_q.sin", sin)
        if l == 0:
            q2(p + "mlp.w1.weight", hd, d)
            q2(p + "mlp.w2.weight", d, hd)
            q2(p + "mlp.w3.weight", hd, d)
        else:
            f32(p + "mlp.gate_inp.weight", r.standard_normal((E, d)) * 0.06)
            q2(p + "mlp.gate_exps.weight", F, d, E)
            q2(p + "mlp.up_exps.weight", F, d, E)
            q2(p + "mlp.down_exps.weight", d, F, E)
            q2(p + "mlp.gate_shexp.weight", S, d)
            q2(p + "mlp.up_shexp.weight", S, d)
            q2(p + "mlp.down_shexp.weight", d, S)
    q2("transformer.wte.weight", V, d)
    f32("transformer.ln_f.weight", np.ones(d))
    q2("lm_head.weight", V, d)
    return tensors, qts, mats


def rms(x, w):
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-5) * w


def silu(x):
    return x / (1 + np.exp(-x))


def topk64(logits, k):
    p = np.exp(logits - logits.max())
    p = p / p.sum()
    order = sorted(range(len(p)), key=lambda e: (-p[e], e))
    return order[:k], p


def forward(mats, ids, cfg=CFG, margin=None):
    """float64 logits of the last row after a full prefill of ids.  If
    margin is a list, the router's k-th / (k+1)-th probability gaps are
    appended to it (to reject seeds with near ties)."""
    c = cfg
    d, H, nope, rope, vd = c["dim"], c["n_heads"], c["nope"], c["rope"], c["v_dim"]
    dq = nope + rope
    T = len(ids)
    h = mats["transformer.wte.weight"][ids].copy()
    cos = mats["transformer.h.0.attn.rope_q.cos"]
    sin = mats["transformer.h.0.attn.rope_q.sin"]
    for l in range(c["n_layers"]):
        p = "transformer.h.%d." % l
        a = rms(h, mats[p + "ln1.weight"])
        Q = a @ mats[p + "attn.w_q.weight"].T
        qn = Q[:, :H * nope].reshape(T, H, nope)
        qr = nr.rope_neox(Q[:, H * nope:].reshape(T, H, rope), cos, sin, 0)
        kva = a @ mats[p + "attn.w_kv_a.weight"].T
        cn = rms(kva[:, :c["dc"]], mats[p + "attn.k_norm.weight"])
        kpe = nr.rope_neox(kva[:, c["dc"]:].reshape(T, 1, rope), cos, sin, 0)[:, 0]
        kvb = cn @ mats[p + "attn.w_kv_b.weight"].T
        kn = kvb[:, :H * nope].reshape(T, H, nope)
        vv = kvb[:, H * nope:].reshape(T, H, vd)
        att = np.zeros((T, H, vd))
        for t in range(T):
            for hh in range(H):
                q = np.concatenate([qn[t, hh], qr[t, hh]])
                K = np.concatenate([kn[: t + 1, hh], kpe[: t + 1]], axis=1)
                att[t, hh] = nr.softmax_attn(q, K, vv[: t + 1, hh], 1 / np.sqrt(dq))
        h = h + att.reshape(T, H * vd) @ mats[p + "attn.w_o.weight"].T
        a = rms(h, mats[p + "ln2.weight"])
        if (p + "mlp.w1.weight") in mats:
            g = a @ mats[p + "mlp.w1.weight"].T
            u = a @ mats[p + "mlp.w3.weight"].T
            h = h + (silu(g) * u) @ mats[p + "mlp.w2.weight"].T
            continue
        for t in range(T):
            at = a[t]
            acc = (silu(at @ mats[p + "mlp.gate_shexp.weight"].T) * (at @ mats[p + "mlp.up_shexp.weight"].T)) \
                @ mats[p + "mlp.down_shexp.weight"].T
            sel, prob = topk64(at @ mats[p + "mlp.gate_inp.weight"].T, c["top_k"])
            if margin is not None:
                srt = np.sort(prob)[::-1]
                margin.append(srt[c["top_k"] - 1] - srt[c["top_k"]])
            for e in sel:
                g = at @ mats[p + "mlp.gate_exps.weight"][e].T
                u = at @ mats[p + "mlp.up_exps.weight"][e].T
                acc = acc + prob[e] * ((silu(g) * u) @ mats[p + "mlp.down_exps.weight"][e].T)
            h[t] = h[t] + acc
    hl = rms(h[-1:], mats["transformer.ln_f.weight"])
    return (hl @ mats["lm_head.weight"].T)[0]
