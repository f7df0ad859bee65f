"""ctypes binding of the CPU oracle (oracle/rina_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "build", "librina_oracle.so")

Q4_0, FP32, Q4_0F, Q2_K = 5, 6, 7, 10
KVF_Q8_0, KVF_Q4_0, KVF_Q2_1, KVF_Q1_0 = 1, 2, 3, 4
KV_MODES = {"fp32": 0, "q8": 1, "q4": 2, "q4k_q2v": 3, "q2": 4, "q2k_q1v": 5}

VP, I32, I64, F32, SZ = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t


class GQALayerW(C.Structure):
    _fields_ = [("w_q", VP), ("qt_q", I32), ("w_k", VP), ("qt_k", I32), ("w_v", VP), ("qt_v", I32),
                ("w_o", VP), ("qt_o", I32), ("w1", VP), ("qt_1", I32), ("w2", VP), ("qt_2", I32),
                ("w3", VP), ("qt_3", I32), ("ln1", VP), ("ln2", VP),
                ("rope_q_cos", VP), ("rope_q_sin", VP), ("rope_k_cos", VP), ("rope_k_sin", VP)]


class GQACfg(C.Structure):
    _fields_ = [("dim", I32), ("n_layers", I32), ("n_heads", I32), ("n_kv_heads", I32), ("head_dim", I32),
                ("hidden", I32), ("vocab", I32), ("max_seq", I32), ("use_rms_norm", I32), ("kv_mode", I32),
                ("pre_rope", I32), ("nthreads", I32), ("wte", VP), ("qt_wte", I32), ("ln_f", VP),
                ("lm_head", VP), ("qt_lm", I32), ("layers", C.POINTER(GQALayerW))]


class MLALayerW(C.Structure):
    _fields_ = [("w_q", VP), ("qt_q", I32), ("w_kv_a", VP), ("qt_kv_a", I32), ("k_norm", VP),
                ("w_kv_b", VP), ("qt_kv_b", I32), ("w_o", VP), ("qt_o", I32), ("ln1", VP), ("ln2", VP),
                ("rope_cos", VP), ("rope_sin", VP), ("is_moe", I32),
                ("w1", VP), ("qt_1", I32), ("w2", VP), ("qt_2", I32), ("w3", VP), ("qt_3", I32), ("hidden", I32),
                ("gate_inp", VP), ("qt_gate_inp", I32), ("gate_exps", VP), ("up_exps", VP), ("qt_gu", I32),
                ("down_exps", VP), ("qt_dn", I32), ("stride_gu", I64), ("stride_dn", I64),
                ("gate_sh", VP), ("up_sh", VP), ("qt_sh_gu", I32), ("down_sh", VP), ("qt_sh_dn", I32),
                ("shared_hidden", I32)]


class MLACfg(C.Structure):
    _fields_ = [("dim", I32), ("n_layers", I32), ("n_heads", I32), ("nope", I32), ("rope", I32), ("v_dim", I32),
                ("dc", I32), ("vocab", I32), ("max_seq", I32), ("n_experts", I32), ("top_k", I32),
                ("expert_ffn", I32), ("nthreads", I32), ("wte", VP), ("qt_wte", I32), ("ln_f", VP),
                ("lm_head", VP), ("qt_lm", I32), ("layers", C.POINTER(MLALayerW))]


class JambaLayerW(C.Structure):
    _fields_ = [("type", I32), ("qt", I32), ("ln1", VP), ("ln2", VP), ("w_dq", VP), ("q_norm", VP),
                ("w_mem", VP * 3), ("w_decay", VP * 3), ("w_out", VP), ("w_uq", VP), ("w_uk", VP),
                ("w_k2v", VP), ("w_qr", VP), ("w_kr", VP), ("c_proj", VP), ("rope_q_cos", VP),
                ("rope_q_sin", VP), ("rope_k_cos", VP), ("rope_k_sin", VP), ("w1", VP), ("w2", VP), ("w3", VP)]


class JambaCfg(C.Structure):
    _fields_ = [("dim", I32), ("n_layers", I32), ("n_heads", I32), ("n_kv_heads", I32), ("head_dim", I32),
                ("dhr", I32), ("dc", I32), ("ssm_steps", I32), ("hidden", I32), ("vocab", I32), ("max_seq", I32),
                ("nthreads", I32), ("wte", VP), ("qt_wte", I32), ("ln_f", VP), ("lm_head", VP), ("qt_lm", I32),
                ("layers", C.POINTER(JambaLayerW)), ("rmla_kv_mode", I32)]


_lib = None


def load(build=True):
    global _lib
    if _lib is not None:
        return _lib
    so = os.environ.get("RINA_ORACLE_SO") or SO     # a sanitizer build of the same source, for tests
    if so == SO and not os.path.exists(SO) and build:
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    L = C.CDLL(so)
    sigs = {
        "orc_f32_to_f16": (C.c_uint16, [F32]),
        "orc_f32_to_f16_trunc": (C.c_uint16, [F32]),
        "orc_f16_to_f32": (F32, [C.c_uint16]),
        "orc_quantized_size": (SZ, [I64, I32]),
        "orc_pack_q4_0": (None, [VP, I64, VP]),
        "orc_pack_q4_0f": (None, [VP, I64, VP]),
        "orc_pack_q4_0_hf": (None, [VP, I64, VP]),
        "orc_dequant_weights": (None, [VP, I32, I64, VP]),
        "orc_linear": (I32, [VP, I32, VP, VP, I32, I32, I32, I32]),
        "orc_kv_block_bytes": (I32, [I32]),
        "orc_kv_quantize": (None, [I32, VP, VP, I64]),
        "orc_kv_dequant": (None, [I32, VP, VP, I64]),
        "orc_rms_norm": (None, [VP, VP, I32, I32, F32]),
        "orc_layer_norm": (None, [VP, VP, I32, I32, F32]),
        "orc_rope_neox": (None, [VP, VP, VP, I32, I32, I32, I32]),
        "orc_rope_hf": (None, [VP, VP, VP, I32, I32, I32, I32]),
        "orc_embedding": (None, [VP, I32, VP, VP, I32, I32]),
        "orc_silu_mul": (None, [VP, VP, VP, I32]),
        "orc_argmax": (I32, [VP, I32]),
        "orc_attn_rows": (None, [VP, I32, VP, I32, VP, I32, VP, I32, I32, I32, I32, I32]),
        "orc_gqa_attention": (None, [VP, VP, VP, VP, VP, VP, VP, I32, I32, VP, VP, I32, I32, I32, I32, I32, VP]),
        "orc_gqa_create": (VP, [C.POINTER(GQACfg)]),
        "orc_gqa_destroy": (None, [VP]),
        "orc_gqa_forward": (I32, [VP, VP, I32, I32, VP, I32]),
        "orc_gqa_cache": (VP, [VP, I32, I32, C.POINTER(SZ)]),
        "orc_gqa_last_kv": (VP, [VP, I32, I32]),
        "orc_gqa_generate": (I32, [VP, VP, I32, I32, VP]),
        "orc_num_threads": (I32, []),
        "orc_moe_topk": (None, [VP, I32, I32, VP, VP]),
        "orc_jamba_create": (VP, [C.POINTER(JambaCfg)]),
        "orc_jamba_destroy": (None, [VP]),
        "orc_jamba_forward": (I32, [VP, VP, I32, I32, VP, I32]),
        "orc_jamba_generate": (I32, [VP, VP, I32, I32, VP]),
        "orc_jamba_generate_recompute": (I32, [VP, VP, I32, I32, VP]),
        "orc_jamba_packed_cache": (VP, [VP, I32, I32]),
        "orc_jamba_fp32_cache": (VP, [VP, I32, I32]),
        "orc_mla_create": (VP, [C.POINTER(MLACfg)]),
        "orc_mla_destroy": (None, [VP]),
        "orc_mla_forward": (I32, [VP, VP, I32, I32, VP, I32]),
        "orc_mla_generate": (I32, [VP, VP, I32, I32, VP]),
        "orc_mla_cache": (VP, [VP, I32, I32]),
        "orc_mla_load_latent": (I32, [VP, I32, VP, I32]),
        "orc_mla_set_latent_tap": (None, [VP, VP]),
    }
    for n, (r, a) in sigs.items():
        f = getattr(L, n)
        f.restype = r
        f.argtypes = a
    _lib = L
    return L


def ptr(a):
    return a.ctypes.data if a is not None else None


# ---- convenience wrappers (numpy in, numpy out) ----------------------------

def f32_to_f16(x):
    L = load()
    return np.array([L.orc_f32_to_f16(float(v)) for v in np.asarray(x, np.float32).ravel()], np.uint16)


def quantized_size(n, qt):
    return load().orc_quantized_size(n, qt)


def pack(qt, x, hf=False):
    L = load()
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(quantized_size(x.size, qt), np.uint8)
    if qt == Q4_0 and hf:
        L.orc_pack_q4_0_hf(ptr(x), x.size, ptr(out))
    elif qt == Q4_0:
        L.orc_pack_q4_0(ptr(x), x.size, ptr(out))
    elif qt == Q4_0F:
        L.orc_pack_q4_0f(ptr(x), x.size, ptr(out))
    else:
        raise ValueError(qt)
    return out


def dequant(qt, w, n):
    out = np.zeros(n, np.float32)
    load().orc_dequant_weights(ptr(np.ascontiguousarray(w)), qt, n, ptr(out))
    return out


def linear(w, qt, x, N, K, nthreads=0):
    x = np.ascontiguousarray(x, np.float32)
    M = x.size // K
    out = np.zeros((M, N), np.float32)
    rc = load().orc_linear(ptr(np.ascontiguousarray(w)), qt, ptr(x), ptr(out), M, N, K, nthreads)
    assert rc == 0, rc
    return out


def kv_quantize(fmt, x):
    L = load()
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(x.size // 32 * L.orc_kv_block_bytes(fmt), np.uint8)
    L.orc_kv_quantize(fmt, ptr(x), ptr(out), x.size)
    return out


def kv_dequant(fmt, b, n):
    out = np.zeros(n, np.float32)
    load().orc_kv_dequant(fmt, ptr(np.ascontiguousarray(b)), ptr(out), n)
    return out


def kv_block_bytes(fmt):
    return load().orc_kv_block_bytes(fmt)


def kv_mode_formats(mode):
    return {1: (KVF_Q8_0, KVF_Q8_0), 2: (KVF_Q4_0, KVF_Q4_0), 3: (KVF_Q4_0, KVF_Q2_1), 4: (KVF_Q2_1, KVF_Q2_1),
            5: (KVF_Q2_1, KVF_Q1_0)}[mode]


def gqa_from_tensors(cfg, tensors, qt, max_seq, kv_mode, nthreads=0, pre_rope=False):
    """Oracle GQA model over host copies of an engine model's tensors.

    cfg: dict with name, dim, n_layers, n_heads, n_kv_heads, head_dim,
    hidden_dim, vocab_size; tensors: name -> numpy array (packed bytes or
    fp32), reference tensor names.  Returns (handle, keepalive)."""
    hold = []

    def h(name):
        a = np.ascontiguousarray(tensors[name])
        hold.append(a)
        return a.ctypes.data

    lw = (GQALayerW * cfg["n_layers"])()
    for l in range(cfg["n_layers"]):
        p = "transformer.h.%d." % l
        o = lw[l]
        o.w_q, o.w_k, o.w_v, o.w_o = (h(p + "attn.w_%s.weight" % x) for x in "qkvo")
        o.w1, o.w2, o.w3 = (h(p + "mlp.w%d.weight" % i) for i in (1, 2, 3))
        o.qt_q = o.qt_k = o.qt_v = o.qt_o = o.qt_1 = o.qt_2 = o.qt_3 = qt
        o.ln1, o.ln2 = h(p + "ln1.weight"), h(p + "ln2.weight")
        o.rope_q_cos, o.rope_q_sin = h(p + "attn.rope_q.cos"), h(p + "attn.rope_q.sin")
        o.rope_k_cos, o.rope_k_sin = h(p + "attn.rope.cos"), h(p + "attn.rope.sin")
    c = GQACfg(dim=cfg["dim"], n_layers=cfg["n_layers"], n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
               head_dim=cfg["head_dim"], hidden=cfg["hidden_dim"], vocab=cfg["vocab_size"], max_seq=max_seq,
               use_rms_norm=1 if "llama" in cfg["name"] else 0, kv_mode=KV_MODES[kv_mode],
               pre_rope=1 if pre_rope else 0, nthreads=nthreads, wte=h("transformer.wte.weight"), qt_wte=FP32,
               ln_f=h("transformer.ln_f.weight"), lm_head=None, qt_lm=0, layers=lw)
    m = load().orc_gqa_create(C.byref(c))
    return m, (hold, lw, c)


def gqa_generate(m, prompt, steps):
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.zeros(steps, np.int32)
    rc = load().orc_gqa_generate(m, p.ctypes.data, p.size, steps, out.ctypes.data)
    assert rc == 0, rc
    return [int(v) for v in out]


def moe_topk(logits, k):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(k, np.int32)
    pr = np.zeros(k, np.float32)
    load().orc_moe_topk(lg.ctypes.data, lg.size, k, ids.ctypes.data, pr.ctypes.data)
    return ids, pr


def mla_from_tensors(cfg, tensors, qts, max_seq, nthreads=0):
    """Oracle DeepSeek MLA + MoE model over host copies of an engine model's
    tensors.  cfg: dict with dim, n_layers, n_heads, nope, rope, v_dim, dc,
    vocab_size, n_experts, top_k, expert_ffn; tensors: name -> numpy array
    (packed bytes or fp32) under the reference names; qts: name -> quant
    type.  Returns (handle, keepalive)."""
    hold = []

    def h(name):
        if name not in tensors:
            return None
        a = np.ascontiguousarray(tensors[name])
        hold.append(a)
        return a.ctypes.data

    def q(name):
        return qts.get(name, FP32)

    nl = cfg["n_layers"]
    lw = (MLALayerW * nl)()
    for l in range(nl):
        p = "transformer.h.%d." % l
        o = lw[l]
        for f, nm in (("w_q", "attn.w_q"), ("w_kv_a", "attn.w_kv_a"), ("w_kv_b", "attn.w_kv_b"), ("w_o", "attn.w_o")):
            setattr(o, f, h(p + nm + ".weight"))
            setattr(o, "qt_" + f[2:], q(p + nm + ".weight"))
        o.k_norm = h(p + "attn.k_norm.weight")
        o.ln1, o.ln2 = h(p + "ln1.weight"), h(p + "ln2.weight")
        o.rope_cos, o.rope_sin = h(p + "attn.rope_q.cos"), h(p + "attn.rope_q.sin")
        if (p + "mlp.gate_inp.weight") in tensors:
            o.is_moe = 1
            o.gate_inp, o.qt_gate_inp = h(p + "mlp.gate_inp.weight"), q(p + "mlp.gate_inp.weight")
            o.gate_exps, o.up_exps = h(p + "mlp.gate_exps.weight"), h(p + "mlp.up_exps.weight")
            o.qt_gu = q(p + "mlp.gate_exps.weight")
            o.down_exps, o.qt_dn = h(p + "mlp.down_exps.weight"), q(p + "mlp.down_exps.weight")
            o.stride_gu = tensors[p + "mlp.gate_exps.weight"].nbytes // cfg["n_experts"]
            o.stride_dn = tensors[p + "mlp.down_exps.weight"].nbytes // cfg["n_experts"]
            o.gate_sh, o.up_sh = h(p + "mlp.gate_shexp.weight"), h(p + "mlp.up_shexp.weight")
            o.qt_sh_gu = q(p + "mlp.gate_shexp.weight")
            o.down_sh, o.qt_sh_dn = h(p + "mlp.down_shexp.weight"), q(p + "mlp.down_shexp.weight")
            o.shared_hidden = cfg["shared_ffn"]
        else:
            o.w1, o.qt_1 = h(p + "mlp.w1.weight"), q(p + "mlp.w1.weight")
            o.w2, o.qt_2 = h(p + "mlp.w2.weight"), q(p + "mlp.w2.weight")
            o.w3, o.qt_3 = h(p + "mlp.w3.weight"), q(p + "mlp.w3.weight")
            o.hidden = cfg["dense_ffn"]
    c = MLACfg(dim=cfg["dim"], n_layers=nl, n_heads=cfg["n_heads"], nope=cfg["nope"], rope=cfg["rope"],
               v_dim=cfg["v_dim"], dc=cfg["dc"], vocab=cfg["vocab_size"], max_seq=max_seq,
               n_experts=cfg.get("n_experts", 0), top_k=cfg.get("top_k", 0), expert_ffn=cfg.get("expert_ffn", 0),
               nthreads=nthreads, wte=h("transformer.wte.weight"), qt_wte=q("transformer.wte.weight"),
               ln_f=h("transformer.ln_f.weight"), lm_head=h("lm_head.weight"), qt_lm=q("lm_head.weight"),
               layers=lw)
    m = load().orc_mla_create(C.byref(c))
    return m, (hold, lw, c)


def mla_generate(m, prompt, steps):
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.zeros(steps, np.int32)
    rc = load().orc_mla_generate(m, p.ctypes.data, p.size, steps, out.ctypes.data)
    assert rc == 0, rc
    return [int(v) for v in out]


JAMBA_SSM_TYPES = ("inertia_wave_ssm", "ssm")


def jamba_from_tensors(cfg, tensors, layer_types, qt, max_seq, nthreads=0, kv_mode="fp32"):
    """Oracle RINA Jamba model over host tensors (reference names).  cfg:
    dim, n_layers, n_heads, n_kv_heads, head_dim, d_h_r, d_c, ssm_steps,
    hidden_dim, vocab_size; layer_types: per-layer type strings; qt: quant
    type of every linear; kv_mode: the RINA-MLA cache form ("fp32" or
    "q2k_q1v").  Returns (handle, keepalive)."""
    hold = []

    def h(name):
        if name not in tensors:
            return None
        a = np.ascontiguousarray(tensors[name])
        hold.append(a)
        return a.ctypes.data

    nl = cfg["n_layers"]
    lw = (JambaLayerW * nl)()
    for l in range(nl):
        p = "transformer.h.%d." % l
        o = lw[l]
        o.qt = qt
        o.ln1, o.ln2 = h(p + "ln1.weight"), h(p + "ln2.weight")
        o.w1, o.w2, o.w3 = (h(p + "mlp.w%d.weight" % i) for i in (1, 2, 3))
        o.q_norm = h(p + "path.q_norm.weight")
        if layer_types[l] in JAMBA_SSM_TYPES:
            o.type = 0
            o.w_dq = h(p + "path.w_dq.weight")
            for k in range(3):
                o.w_mem[k] = h(p + "path.w_mem.%d.weight" % k)
                o.w_decay[k] = h(p + "path.w_decay.%d.weight" % k)
            o.w_out = h(p + "path.w_out.weight")
        else:
            o.type = 1
            o.w_dq = h(p + "path.w_dqkv.weight")
            for f in ("w_uq", "w_uk", "w_k2v", "w_qr", "w_kr", "c_proj"):
                setattr(o, f, h(p + "path.%s.weight" % f))
            o.rope_q_cos, o.rope_q_sin = h(p + "path.rope_q.cos"), h(p + "path.rope_q.sin")
            o.rope_k_cos, o.rope_k_sin = h(p + "path.rope.cos"), h(p + "path.rope.sin")
    c = JambaCfg(dim=cfg["dim"], n_layers=nl, n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
                 head_dim=cfg["head_dim"], dhr=cfg["d_h_r"], dc=cfg["d_c"], ssm_steps=cfg["ssm_steps"],
                 hidden=cfg["hidden_dim"], vocab=cfg["vocab_size"], max_seq=max_seq, nthreads=nthreads,
                 wte=h("transformer.wte.weight"), qt_wte=FP32, ln_f=h("transformer.ln_f.weight"),
                 lm_head=h("lm_head.weight"), qt_lm=FP32, layers=lw, rmla_kv_mode=KV_MODES[kv_mode])
    m = load().orc_jamba_create(C.byref(c))
    return m, (hold, lw, c)


def jamba_generate(m, prompt, steps, recompute=False):
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.zeros(steps, np.int32)
    f = load().orc_jamba_generate_recompute if recompute else load().orc_jamba_generate
    rc = f(m, p.ctypes.data, p.size, steps, out.ctypes.data)
    assert rc == 0, rc
    return [int(v) for v in out]
