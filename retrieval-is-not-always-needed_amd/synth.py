"""Random-init models for the decode path (no checkpoints exist offline).

Weights are fp32 ~ N(0, std) from numpy's PCG64 (one seed per tensor, so a
tensor's values do not depend on which others are built), packed on the GPU
by rina_hip_pack_weights (the tools/q4_pack.py rules), and registered in an
engine model under the reference's tensor names
(rina-engine/tools/convert_llama_to_rinn.py:97-123): transformer.wte.weight
(fp32, tied LM head), transformer.h.{l}.attn.w_{q,k,v,o}.weight,
transformer.h.{l}.mlp.w{1,2,3}.weight, transformer.h.{l}.ln{1,2}.weight,
transformer.h.{l}.attn.rope_q.{cos,sin} / rope.{cos,sin}, transformer.ln_f.weight.
"""
import ctypes as C
import json
import math

import numpy as np

from . import QT_FP32, QT_Q4_0, QT_Q4_0F, QT_Q2_K, check, load_engine, load_hip

LLAMA_1B = dict(name="llama3.2-1b", dim=2048, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64,
                hidden_dim=8192, vocab_size=128256, rope_theta=500000.0)


def make_rope(dim, max_pos, theta=500000.0):
    """cos/sin tables [max_pos, dim/2] (convert_llama_to_rinn.py:19-34, no scaling)."""
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim)))).astype(np.float32)
    t = np.arange(max_pos, dtype=np.float32)
    ang = np.outer(t, inv).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def normal(seed, n, std):
    return (np.random.default_rng(seed).standard_normal(n, dtype=np.float32) * np.float32(std)).astype(np.float32)


def q2k_scales(target_std):
    """fp16 (d, dmin) of the zero-mean Q2_K blocks below: with the min nibble
    equal to the scale nibble sc and dmin = 1.5 d, an element is
    d*sc*q - 1.5*d*sc = d*sc*(q - 1.5), symmetric around 0 for uniform
    2-bit q.  Its rms over uniform sc in 0..15 is d*sqrt(77.5*1.25) = 9.84 d."""
    d = np.float16(target_std / 9.84)
    return d, np.float16(np.float32(d) * np.float32(1.5))


def random_q2k(seed, n_elems, target_std=0.02):
    """Random valid Q2_K blocks (84 B / 256 values) with zero-mean values:
    random 4-bit scale nibbles, each sub-block's min nibble equal to its
    scale nibble, random 2-bit q, fp16 d / dmin from q2k_scales (the
    reference ships no Q2_K quantizer).  Uniform independent min nibbles
    would give every weight a mean of about +0.6 of its spread, and a random
    model built from them emits the same token at every step."""
    nb = (n_elems + 255) // 256
    rng = np.random.default_rng(seed)
    blk = np.zeros((nb, 84), np.uint8)
    sc = rng.integers(0, 16, (nb, 16), dtype=np.uint8)
    blk[:, 0:16] = sc | (sc << 4)
    blk[:, 16:80] = rng.integers(0, 256, (nb, 64), dtype=np.uint8)
    d, dmin = q2k_scales(target_std)
    blk[:, 80:82] = np.frombuffer(np.array([d], np.float16).tobytes(), np.uint8)
    blk[:, 82:84] = np.frombuffer(np.array([dmin], np.float16).tobytes(), np.uint8)
    return blk.reshape(-1)


class DeviceArena:
    """Keeps the torch device tensors that back borrowed engine tensors alive."""

    def __init__(self):
        self.keep = []

    def put(self, t):
        self.keep.append(t)
        return t


def _torch():
    import torch
    return torch


def pack_on_device(x_host, qt, stream=None):
    """fp32 host array -> packed device tensor (uint8) via rina_hip_pack_weights."""
    torch = _torch()
    hip = load_hip()
    n = x_host.size
    x = torch.from_numpy(np.ascontiguousarray(x_host, np.float32).reshape(-1)).cuda()
    if qt == QT_FP32:
        return x
    nbytes = (n // 32) * (18 if qt == QT_Q4_0 else 20)
    out = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    check(hip.rina_hip_pack_weights(qt, x.data_ptr(), n, out.data_ptr(), s), "rina_hip_pack_weights")
    return out


def write_rinn(path, config, tensors):
    """Write a .rinn file in the layout of tools/convert_llama_to_rinn.py:97-123
    (read by loader.cpp:14-141): a 512-byte header ("RINN", version 1, the
    tensor count, config / index / data offsets), the config as JSON, the
    tensor index (u16 name length, name, 4 x i32 shape padded with zeros,
    u8 quant type, u16 block size (32 for Q4 types, 1 for fp32), u64 offset,
    u64 size), then the tensor bytes from the first 256-byte boundary after
    the index, back to back.  tensors: (name, shape, quant_type, bytes-like)
    in file order."""
    import struct
    cj = json.dumps(config).encode("utf-8")
    entries = []
    for name, shape, qt, data in tensors:
        nb = name.encode()
        b = bytes(memoryview(np.ascontiguousarray(data)).cast("B"))
        shp = list(shape) + [0] * (4 - len(shape))
        entries.append((nb, shp, int(qt), 32 if qt in (QT_Q4_0, QT_Q4_0F) else 1, b))
    idx_sz = sum(2 + len(nb) + 16 + 1 + 2 + 8 + 8 for nb, _, _, _, _ in entries)
    data_off = ((512 + len(cj) + idx_sz + 255) // 256) * 256
    hdr = bytearray(512)
    hdr[0:4] = b"RINN"
    struct.pack_into("<I", hdr, 4, 1)
    struct.pack_into("<I", hdr, 8, len(entries))
    struct.pack_into("<QQQQQ", hdr, 16, 512, len(cj), 512 + len(cj), idx_sz, data_off)
    with open(path, "wb") as f:
        f.write(hdr)
        f.write(cj)
        off = data_off
        for nb, shp, qt, bs, b in entries:
            f.write(struct.pack("<H", len(nb)) + nb + struct.pack("<4i", *shp) + struct.pack("<BHQQ", qt, bs, off, len(b)))
            off += len(b)
        f.write(b"\x00" * (data_off - f.tell()))
        for _, _, _, _, b in entries:
            f.write(b)


class SynthLlama:
    """A Llama-shaped GQA model with random weights, built on the device.

    keep_host: also keep host copies of the packed tensors (for the oracle).
    """

    def __init__(self, cfg, qt=QT_Q4_0F, seed=1, max_seq=1024, std=0.02, keep_host=False, kv_mode="fp32"):
        torch = _torch()
        self.cfg = dict(cfg)
        self.qt = qt
        self.max_seq = max_seq
        self.kv_mode = kv_mode
        self.arena = DeviceArena()
        self.host = {}
        self.dev = {}
        self.shapes, self.qts, self.order = {}, {}, []
        eng = load_engine()
        c = self.cfg
        d, H, Hkv, dh, hd, V, L = (c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["hidden_dim"],
                                   c["vocab_size"], c["n_layers"])
        header = {"name": c["name"], "dim": d, "n_layers": L, "n_heads": H, "n_kv_heads": Hkv, "head_dim": dh,
                  "vocab_size": V, "max_seq_len": max_seq, "hidden_dim": hd, "weight_tying": True,
                  "kv_quant_mode": kv_mode, "layers": [{"type": "standard_attention"} for _ in range(L)]}
        self.model = eng.rina_model_create(json.dumps(header).encode())
        if not self.model:
            raise RuntimeError(eng.rina_engine_last_error().decode())
        self._eng = eng
        idx = [0]

        def add(name, shape, qt_, data_dev, host=None):
            shp = (C.c_int64 * len(shape))(*shape)
            check(eng.rina_model_add_tensor(self.model, name.encode(), qt_, len(shape), shp, data_dev.data_ptr()),
                  "add_tensor " + name)
            self.arena.put(data_dev)
            self.dev[name] = data_dev
            self.shapes[name], self.qts[name] = tuple(shape), qt_
            self.order.append(name)
            if keep_host:
                self.host[name] = host if host is not None else data_dev.cpu().numpy()

        def weight(name, rows, cols):
            idx[0] += 1
            x = normal(seed * 1000003 + idx[0], rows * cols, std)
            dev = pack_on_device(x, qt)
            add(name, (rows, cols), qt, dev)

        wte = normal(seed * 1000003, V * d, std)
        add("transformer.wte.weight", (V, d), QT_FP32, torch.from_numpy(wte).cuda(), wte if keep_host else None)
        cos, sin = make_rope(dh, max_seq, c.get("rope_theta", 500000.0))
        cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        ones = np.ones(d, np.float32)
        for l in range(L):
            p = "transformer.h.%d." % l
            weight(p + "attn.w_q.weight", H * dh, d)
            weight(p + "attn.w_k.weight", Hkv * dh, d)
            weight(p + "attn.w_v.weight", Hkv * dh, d)
            weight(p + "attn.w_o.weight", d, H * dh)
            weight(p + "mlp.w1.weight", hd, d)
            weight(p + "mlp.w2.weight", d, hd)
            weight(p + "mlp.w3.weight", hd, d)
            add(p + "ln1.weight", (d,), QT_FP32, torch.from_numpy(ones.copy()).cuda(), ones)
            add(p + "ln2.weight", (d,), QT_FP32, torch.from_numpy(ones.copy()).cuda(), ones)
            for nm, t, h in (("attn.rope_q.cos", cos_d, cos), ("attn.rope_q.sin", sin_d, sin),
                             ("attn.rope.cos", cos_d, cos), ("attn.rope.sin", sin_d, sin)):
                add(p + nm, (max_seq, dh // 2), QT_FP32, t, h)
        add("transformer.ln_f.weight", (d,), QT_FP32, torch.from_numpy(ones.copy()).cuda(), ones)
        self.cos, self.sin = cos, sin

    def save_rinn(self, path):
        """The model as a .rinn file (write_rinn; needs keep_host=True), with
        the converter's config keys (convert_llama_to_rinn.py:46-53) plus
        hidden_dim and the KV mode."""
        if not self.host:
            raise RuntimeError("save_rinn needs a model built with keep_host=True")
        c = self.cfg
        L = c["n_layers"]
        config = {"name": c["name"], "dim": c["dim"], "n_layers": L, "n_heads": c["n_heads"],
                  "n_kv_heads": c["n_kv_heads"], "head_dim": c["head_dim"], "d_c": 0, "d_h_r": c["head_dim"],
                  "vocab_size": c["vocab_size"], "block_size": self.max_seq, "ssm_steps": 0, "weight_tying": True,
                  "quant_mode": "", "ssm_qbits": 0, "hidden_dim": c["hidden_dim"], "kv_quant_mode": self.kv_mode,
                  "layers": [{"type": "standard_attention"} for _ in range(L)]}
        tensors = [(n, self.shapes[n], self.qts[n], self.host[n]) for n in self.order]
        write_rinn(path, config, tensors)

    def weight_bytes_per_token(self):
        c = self.cfg
        d, H, Hkv, dh, hd, V, L = (c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["hidden_dim"],
                                   c["vocab_size"], c["n_layers"])
        bpb = {QT_Q4_0: 18, QT_Q4_0F: 20}[self.qt]
        per_layer = ((H * dh + 2 * Hkv * dh) * d + d * H * dh + 2 * hd * d + d * hd) // 32 * bpb
        return L * per_layer + V * d * 4 + (2 * L + 1) * d * 4

    def infer(self, kv_mode=None, max_seq=None):
        eng = self._eng
        h = eng.rina_infer_create(self.model, b"gqa", (kv_mode or self.kv_mode).encode(), max_seq or self.max_seq)
        if not h:
            raise RuntimeError(eng.rina_engine_last_error().decode())
        return h

    def close(self):
        if self.model:
            self._eng.rina_model_destroy(self.model)
            self.model = None
        self.arena.keep.clear()


class HostModel:
    """An engine model uploaded from host tensors: header is the config
    dict (JSON keys of the engine's ModelConfig), tensors maps reference
    names to (quant_type, shape, ndarray of packed bytes or fp32)."""

    def __init__(self, header, tensors):
        torch = _torch()
        self.header = dict(header)
        self.arena = DeviceArena()
        self.dev = {}
        eng = load_engine()
        self._eng = eng
        self.model = eng.rina_model_create(json.dumps(self.header).encode())
        if not self.model:
            raise RuntimeError(eng.rina_engine_last_error().decode())
        for name, (qt, shape, arr) in tensors.items():
            t = torch.from_numpy(np.ascontiguousarray(arr)).cuda()
            shp = (C.c_int64 * len(shape))(*shape)
            check(eng.rina_model_add_tensor(self.model, name.encode(), qt, len(shape), shp, t.data_ptr()),
                  "add_tensor " + name)
            self.arena.put(t)
            self.dev[name] = t

    def infer(self, arch, kv_mode=None, max_seq=0):
        h = self._eng.rina_infer_create(self.model, arch.encode(), kv_mode.encode() if kv_mode else None, max_seq)
        if not h:
            raise RuntimeError(self._eng.rina_engine_last_error().decode())
        return h

    def close(self):
        if self.model:
            self._eng.rina_model_destroy(self.model)
            self.model = None
        self.arena.keep.clear()


DSV2_LITE = dict(name="deepseek-v2-lite", dim=2048, n_layers=27, n_heads=16, nope=128, rope=64, v_dim=128, dc=512,
                 vocab_size=102400, dense_ffn=10944, n_experts=64, top_k=6, expert_ffn=1408, shared_ffn=2816,
                 rope_theta=10000.0)


def q2k_device(n_elems, seed, std=0.02):
    """Random valid zero-mean Q2_K blocks generated on the device (the rule
    of random_q2k)."""
    torch = _torch()
    nb = (n_elems + 255) // 256
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    blk = torch.randint(0, 256, (nb, 84), dtype=torch.uint8, device="cuda", generator=g)
    sc = blk[:, 0:16] & 15
    blk[:, 0:16] = sc | (sc << 4)
    d, dmin = q2k_scales(std)
    dd = np.frombuffer(np.array([d, dmin], np.float16).tobytes(), np.uint8)
    blk[:, 80:84] = torch.from_numpy(dd.copy()).cuda()
    return blk.reshape(-1)


class SynthDeepSeek:
    """DeepSeek-V2-Lite-shaped MLA + MoE model with random Q2_K weights
    (fp32 router, norms 1, NeoX RoPE tables), built on the device.  Layer 0
    is dense, the rest MoE (config 4 of the benchmark set)."""

    def __init__(self, cfg=DSV2_LITE, seed=1, max_seq=2048, keep_host=False, n_layers=None):
        torch = _torch()
        c = self.cfg = dict(cfg)
        if n_layers is not None:
            c["n_layers"] = n_layers
        self.max_seq = max_seq
        self.host, self.qts, self.dev = {}, {}, {}
        d, H, nope, rope, vd, dc = c["dim"], c["n_heads"], c["nope"], c["rope"], c["v_dim"], c["dc"]
        E, F, S, hd, V, L = c["n_experts"], c["expert_ffn"], c["shared_ffn"], c["dense_ffn"], c["vocab_size"], c["n_layers"]
        header = {"name": c["name"], "dim": d, "n_layers": L, "n_heads": H, "n_kv_heads": H, "head_dim": nope,
                  "qk_nope_head_dim": nope, "qk_rope_head_dim": rope, "v_head_dim": vd, "kv_lora_rank": dc,
                  "vocab_size": V, "max_seq_len": max_seq, "n_routed_experts": E, "num_experts_per_tok": c["top_k"],
                  "moe_intermediate_size": F,
                  "layers": [{"type": "deepseek_mla_dense"}] + [{"type": "deepseek_mla_moe"}] * (L - 1)}
        eng = load_engine()
        self._eng = eng
        self.arena = DeviceArena()
        self.model = eng.rina_model_create(json.dumps(header).encode())
        if not self.model:
            raise RuntimeError(eng.rina_engine_last_error().decode())
        idx = [0]

        def add(name, shape, qt, t):
            shp = (C.c_int64 * len(shape))(*shape)
            check(eng.rina_model_add_tensor(self.model, name.encode(), qt, len(shape), shp, t.data_ptr()),
                  "add_tensor " + name)
            self.arena.put(t)
            self.dev[name] = t
            self.qts[name] = qt
            if keep_host:
                self.host[name] = t.cpu().numpy()

        def q2(name, shape):
            idx[0] += 1
            n = int(np.prod(shape))
            if len(shape) == 3:   # stacked experts: whole blocks per expert
                per = (shape[1] * shape[2] + 255) // 256 * 256
                t = q2k_device(shape[0] * per, seed * 7919 + idx[0])
            else:
                t = q2k_device(n, seed * 7919 + idx[0])
            add(name, shape, QT_Q2_K, t)

        def f32(name, a):
            add(name, a.shape, QT_FP32, torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda())

        cos, sin = make_rope(rope, max_seq, c.get("rope_theta", 10000.0))
        ones = np.ones(d, np.float32)
        for l in range(L):
            p = "transformer.h.%d." % l
            q2(p + "attn.w_q.weight", (H * (nope + rope), d))
            q2(p + "attn.w_kv_a.weight", (dc + rope, d))
            f32(p + "attn.k_norm.weight", np.ones(dc, np.float32))
            q2(p + "attn.w_kv_b.weight", (H * (nope + vd), dc))
            q2(p + "attn.w_o.weight", (d, H * vd))
            f32(p + "ln1.weight", ones)
            f32(p + "ln2.weight", ones)
            f32(p + "attn.rope_q.cos", cos)
            f32(p + "attn.rope_q.sin", sin)
            if l == 0:
                q2(p + "mlp.w1.weight", (hd, d))
                q2(p + "mlp.w2.weight", (d, hd))
                q2(p + "mlp.w3.weight", (hd, d))
            else:
                f32(p + "mlp.gate_inp.weight", normal(seed * 31 + l, E * d, 0.02).reshape(E, d))
                q2(p + "mlp.gate_exps.weight", (E, F, d))
                q2(p + "mlp.up_exps.weight", (E, F, d))
                q2(p + "mlp.down_exps.weight", (E, d, F))
                q2(p + "mlp.gate_shexp.weight", (S, d))
                q2(p + "mlp.up_shexp.weight", (S, d))
                q2(p + "mlp.down_shexp.weight", (d, S))
        q2("transformer.wte.weight", (V, d))
        f32("transformer.ln_f.weight", ones)
        q2("lm_head.weight", (V, d))

    def bytes_per_token(self, pos):
        """HBM bytes one decode step reads at cache position pos: all
        attention / dense / shared weights, top_k experts per MoE layer, the
        router, the LM head row block, and the latent cache."""
        c = self.cfg
        d, H, nope, rope, vd, dc = c["dim"], c["n_heads"], c["nope"], c["rope"], c["v_dim"], c["dc"]
        q2 = lambda n: (n + 255) // 256 * 84
        attn = q2(H * (nope + rope) * d) + q2((dc + rope) * d) + q2(H * (nope + vd) * dc) + q2(d * H * vd)
        dense = 3 * q2(c["dense_ffn"] * d)
        moe = c["top_k"] * 3 * q2(c["expert_ffn"] * d) + 3 * q2(c["shared_ffn"] * d) + c["n_experts"] * d * 4
        L = c["n_layers"]
        return (L * attn + dense + (L - 1) * moe + q2(c["vocab_size"] * d) + L * (pos + 1) * (dc + rope) * 4)

    def infer(self, max_seq=None):
        h = self._eng.rina_infer_create(self.model, b"mla", None, max_seq or self.max_seq)
        if not h:
            raise RuntimeError(self._eng.rina_engine_last_error().decode())
        return h

    def close(self):
        if self.model:
            self._eng.rina_model_destroy(self.model)
            self.model = None
        self.arena.keep.clear()


JAMBA = dict(name="rina-gen6-jamba", dim=640, n_layers=16, n_heads=10, n_kv_heads=5, head_dim=64, d_h_r=32, d_c=160,
             ssm_steps=3, hidden_dim=1536, vocab_size=128256)


def jamba_types(n_layers, every=4):
    """12 SSM + 4 attention layers for 16: attention at every 4th layer."""
    return ["sparse_gather_fa" if l % every == every - 1 else "inertia_wave_ssm" for l in range(n_layers)]


class SynthJamba:
    """RINA Gen6 Jamba hybrid at random init (config 5): InertiaWave SSM and
    RINA-MLA layers with Q4_0 linears packed on the device, LayerNorm, fp32
    tied embedding / LM head, HF RoPE tables."""

    def __init__(self, cfg=JAMBA, seed=1, max_seq=2048, keep_host=False, std=0.02, kv_mode="fp32"):
        torch = _torch()
        c = self.cfg = dict(cfg)
        self.max_seq = max_seq
        self.kv_mode = kv_mode
        self.types = jamba_types(c["n_layers"])
        self.host, self.dev = {}, {}
        d, H, Hkv, dh, dhr, dc, hd, V = (c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["d_h_r"], c["d_c"],
                                         c["hidden_dim"], c["vocab_size"])
        header = {"name": c["name"], "dim": d, "n_layers": c["n_layers"], "n_heads": H, "n_kv_heads": Hkv,
                  "head_dim": dh, "d_h_r": dhr, "d_c": dc, "ssm_steps": c["ssm_steps"], "vocab_size": V,
                  "max_seq_len": max_seq, "hidden_dim": hd, "rina_mla_kv_mode": kv_mode,
                  "layers": [{"type": t} for t in self.types]}
        eng = load_engine()
        self._eng = eng
        self.arena = DeviceArena()
        self.model = eng.rina_model_create(json.dumps(header).encode())
        if not self.model:
            raise RuntimeError(eng.rina_engine_last_error().decode())
        idx = [0]

        def add(name, shape, qt, t, host=None):
            shp = (C.c_int64 * len(shape))(*shape)
            check(eng.rina_model_add_tensor(self.model, name.encode(), qt, len(shape), shp, t.data_ptr()),
                  "add_tensor " + name)
            self.arena.put(t)
            self.dev[name] = t
            if keep_host:
                self.host[name] = host if host is not None else t.cpu().numpy()

        def lin(name, rows, cols, s=std):
            idx[0] += 1
            add(name, (rows, cols), QT_Q4_0, pack_on_device(normal(seed * 1000003 + idx[0], rows * cols, s), QT_Q4_0))

        def f32(name, a):
            a = np.ascontiguousarray(a, np.float32)
            add(name, a.shape, QT_FP32, torch.from_numpy(a).cuda(), a)

        ang = np.outer(np.arange(max_seq, dtype=np.float32),
                       (1.0 / (10000.0 ** (np.arange(0, dhr, 2, dtype=np.float32) / dhr))).astype(np.float32))
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        ones = np.ones(d, np.float32)
        for l, t in enumerate(self.types):
            p = "transformer.h.%d." % l
            f32(p + "ln1.weight", ones)
            f32(p + "ln2.weight", ones)
            f32(p + "path.q_norm.weight", np.ones(dc, np.float32))
            if t == "inertia_wave_ssm":
                lin(p + "path.w_dq.weight", dc, d)
                for k in range(c["ssm_steps"]):
                    lin(p + "path.w_mem.%d.weight" % k, H * dh, dc)
                    lin(p + "path.w_decay.%d.weight" % k, H, dc)
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
        f32("transformer.wte.weight", normal(seed * 1000003, V * d, std).reshape(V, d))
        f32("transformer.ln_f.weight", ones)

    def bytes_per_token(self, pos):
        c = self.cfg
        d, H, Hkv, dh, dhr, dc, hd, V = (c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["d_h_r"], c["d_c"],
                                         c["hidden_dim"], c["vocab_size"])
        q4 = lambda n: n // 32 * 18
        mlp = 3 * q4(hd * d)
        ssm = q4(dc * d) + c["ssm_steps"] * (q4(H * dh * dc) + q4(H * dc)) + q4(d * (d + H * dh))
        # cache bytes per position and KV head: fp32 [k | kr] and v, or the
        # packed form (two q2_1 blocks of k, kr in fp32, two q1_0 records of v)
        rec = (dh + dhr + dh) * 4 if self.kv_mode != "q2k_q1v" else dh // 32 * 10 + dhr * 4 + dh // 32 * 6
        att = (q4(dc * d) + q4(H * dh * dc) + q4(Hkv * dh * dc) + q4(Hkv * dh * Hkv * dh) + q4(H * dhr * d) +
               q4(Hkv * dhr * d) + q4(d * H * dh) + (pos + 1) * Hkv * rec)
        n_att = sum(1 for t in self.types if t != "inertia_wave_ssm")
        n_ssm = len(self.types) - n_att
        return n_ssm * (ssm + mlp) + n_att * (att + mlp) + V * d * 4

    def infer(self, max_seq=None):
        h = self._eng.rina_infer_create(self.model, b"gqa", None, max_seq or self.max_seq)
        if not h:
            raise RuntimeError(self._eng.rina_engine_last_error().decode())
        return h

    def close(self):
        if self.model:
            self._eng.rina_model_destroy(self.model)
            self.model = None
        self.arena.keep.clear()
