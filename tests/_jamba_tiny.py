"""A tiny RINA Jamba hybrid (SSM + RINA-MLA layers, Q4_0 linears, LayerNorm)
and a float64 numpy restatement of the reference's full-recompute forward
(arch/ssm/rina_ssm_layer.cu:90-126, kernels/ssm_kernels_fp32.cu:6-47,
arch/mla/rina_mla_layer.cu:65-98).  Shared by the oracle and GPU tests."""
import numpy as np

import _numpy_ref as nr

Q4_0, FP32 = 5, 6
CFG = dict(name="rina-jamba-tiny", dim=128, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=64, d_h_r=16, d_c=64,
           ssm_steps=3, hidden_dim=256, vocab_size=101)
TYPES = ["inertia_wave_ssm", "inertia_wave_ssm", "inertia_wave_ssm", "sparse_gather_fa"]


def build(orc, seed=21, max_pos=64, cfg=CFG, types=TYPES, qt=Q4_0, std=0.05):
    c = cfg
    r = np.random.default_rng(seed)
    d, H, Hkv, dh, dhr, dc, hd, V = (c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["d_h_r"], c["d_c"],
                                     c["hidden_dim"], c["vocab_size"])
    tensors, mats, shapes = {}, {}, {}

    def lin(name, rows, cols, s=std):
        w = (r.standard_normal(rows * cols) * s).astype(np.float32)
        p = orc.pack(qt, w)
        tensors[name] = p
        shapes[name] = (rows, cols)
        mats[name] = nr.dequant_q4(p, rows * cols, qt == 7).reshape(rows, cols).astype(np.float64)

    def f32(name, a):
        tensors[name] = np.ascontiguousarray(a, np.float32)
        shapes[name] = a.shape
        mats[name] = a.astype(np.float64)

    ang = np.outer(np.arange(max_pos), 1.0 / 10000 ** (np.arange(0, dhr, 2) / dhr)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    for l, t in enumerate(types):
        p = "transformer.h.%d." % l
        f32(p + "ln1.weight", r.uniform(0.8, 1.2, d))
        f32(p + "ln2.weight", r.uniform(0.8, 1.2, d))
        f32(p + "path.q_norm.weight", r.uniform(0.8, 1.2, dc))
        if t in ("inertia_wave_ssm", "ssm"):
            lin(p + "path.w_dq.weight", dc, d)
            for k in range(c["ssm_steps"]):
                lin(p + "path.w_mem.%d.weight" % k, H * dh, dc)
                lin(p + "path.w_decay.%d.weight" % k, H, dc, s=0.3)
            lin(p + "path.w_out.weight", d, d + H * dh)
        else:
            lin(p + "path.w_dqkv.weight", dc, d)
            lin(p + "path.w_uq.weight", H * dh, dc)
            lin(p + "path.w_uk.weight", Hkv * dh, dc)
            lin(p + "path.w_k2v.weight", Hkv * dh, Hkv * dh)
            lin(p + "path.w_qr.weight", H * dhr, d)
            lin(p + "path.w_kr.weight", Hkv * dhr, d)
            lin(p + "path.c_proj.weight", d, H * dh)
            for nm, a in (("rope_q.cos", cos), ("rope_q.sin", sin), ("rope.cos", cos), ("rope.sin", sin)):
                f32(p + "path." + nm, a)
        lin(p + "mlp.w1.weight", hd, d)
        lin(p + "mlp.w2.weight", d, hd)
        lin(p + "mlp.w3.weight", hd, d)
    f32("transformer.wte.weight", r.standard_normal((V, d)) * 0.5)
    f32("transformer.ln_f.weight", np.ones(d))
    return tensors, mats, shapes


def ln(x, w):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * w


def rope_hf(x, cos, sin):
    """x [T, nh, d] at positions 0..T-1, pairs (2i, 2i+1)"""
    T = x.shape[0]
    c, s = cos[:T][:, None, :].astype(np.float64), sin[:T][:, None, :].astype(np.float64)
    y = x.copy()
    y[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    y[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return y


def forward(mats, ids, cfg=CFG, types=TYPES, history=None):
    """float64 logits of the last row, full recompute over ids.  history:
    layer -> (K content [T, Hkv, dh], V [T, Hkv, dh]) that position tt's
    attention reads for positions < tt instead of the computed rows (the
    q2k_q1v RINA-MLA cache: earlier positions dequantized, the own position
    from its computed rows; the RoPE part never quantized)."""
    c = cfg
    d, H, Hkv, dh, dhr = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["d_h_r"]
    T = len(ids)
    V = c["vocab_size"]
    h = mats["transformer.wte.weight"].reshape(V, d)[ids].copy()
    for l, t in enumerate(types):
        p = "transformer.h.%d." % l
        a = ln(h, mats[p + "ln1.weight"])
        if t in ("inertia_wave_ssm", "ssm"):
            cq = ln(a @ mats[p + "path.w_dq.weight"].T, mats[p + "path.q_norm.weight"])
            mem = [(cq @ mats[p + "path.w_mem.%d.weight" % k].T).reshape(T, H, dh) for k in range(3)]
            dec = [1 / (1 + np.exp(-(cq @ mats[p + "path.w_decay.%d.weight" % k].T))) for k in range(3)]
            da = np.maximum(dec[0] * dec[1] * dec[2], 1e-38)                     # [T, H]
            ma = mem[0] * (dec[1] * dec[2])[..., None] + mem[1] * dec[2][..., None] + mem[2]
            lcs = np.cumsum(np.log(da), axis=0)                                    # [T, H]
            ca = np.exp(lcs)
            wcs = np.cumsum(ma / np.maximum(ca, 1e-30)[..., None], axis=0)
            sf = (ca[..., None] * wcs).reshape(T, H * dh)
            h = h + np.concatenate([a, sf], axis=1) @ mats[p + "path.w_out.weight"].T
        else:
            cq = ln(a @ mats[p + "path.w_dqkv.weight"].T, mats[p + "path.q_norm.weight"])
            q = (cq @ mats[p + "path.w_uq.weight"].T).reshape(T, H, dh)
            k = cq @ mats[p + "path.w_uk.weight"].T
            v = (k @ mats[p + "path.w_k2v.weight"].T).reshape(T, Hkv, dh)
            k = k.reshape(T, Hkv, dh)
            qr = rope_hf((a @ mats[p + "path.w_qr.weight"].T).reshape(T, H, dhr), mats[p + "path.rope_q.cos"],
                         mats[p + "path.rope_q.sin"])
            kr = rope_hf((a @ mats[p + "path.w_kr.weight"].T).reshape(T, Hkv, dhr), mats[p + "path.rope.cos"],
                         mats[p + "path.rope.sin"])
            att = np.zeros((T, H, dh))
            rep = H // Hkv
            kh, vh = (k, v) if history is None or l not in history else history[l]
            for tt in range(T):
                for hh in range(H):
                    g = hh // rep
                    qq = np.concatenate([q[tt, hh], qr[tt, hh]])
                    kc_rows = np.concatenate([kh[:tt, g], k[tt:tt + 1, g]], axis=0)
                    v_rows = np.concatenate([vh[:tt, g], v[tt:tt + 1, g]], axis=0)
                    K = np.concatenate([kc_rows, kr[: tt + 1, g]], axis=1)
                    att[tt, hh] = nr.softmax_attn(qq, K, v_rows, 1 / np.sqrt(dh + dhr))
            h = h + att.reshape(T, H * dh) @ mats[p + "path.c_proj.weight"].T
        a = ln(h, mats[p + "ln2.weight"])
        g = a @ mats[p + "mlp.w1.weight"].T
        u = a @ mats[p + "mlp.w3.weight"].T
        h = h + (g / (1 + np.exp(-g)) * u) @ mats[p + "mlp.w2.weight"].T
    hl = ln(h[-1:], mats["transformer.ln_f.weight"])
    return (hl @ mats["transformer.wte.weight"].reshape(V, d).T)[0]
