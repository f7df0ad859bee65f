"""Decode-step benchmark of the MI355X RINA hot path (one GPU).

Workload: Llama-3.2-1B-shaped model, random-init
Q4_0F linears, fp32 tied LM head, fp32 KV cache, 512-token seeded prompt,
greedy decode.  A step is one decoded token (the whole hot path: embedding,
16 x [RMSNorm, fused q/k/v Q4_0F matvec, RoPE + KV append, decode attention,
W_o + residual, RMSNorm, W1/W3 + SiLU*up, W2 + residual], final norm, fp32
LM head, device argmax), replayed as one HIP graph.  The timed region is
exactly --steps decode steps with all inputs resident in HBM.

The headline roofline is the metric's own kernels: config 2's quant matvecs
and decode attention over all 16 layers (the layer stack, one graph replay
per token, HIP events on the stream it runs on), algorithmic bytes per token
over device time per token.  Also reported: the fp32 LM head, the Q4_0F
SwiGLU matvec and config 1's Q4_0 GEMV over weight rings larger than the
256 MB MALL, decode attention and config 4's stages on their own, configs
3-5 end to end, and the CPU oracle's decode rate on a bounded sample
(cpu_baseline).
"""
import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "retrieval-is-not-always-needed_amd")
HBM_PEAK = 8.0e12
METRIC = "quant GEMV + decode-attn achieved HBM GB/s (% of 8 TB/s); decode tokens/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pkg():
    if "rina_amd" in sys.modules:
        return sys.modules["rina_amd"]
    spec = importlib.util.spec_from_file_location("rina_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["rina_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def time_kernel(torch, fn, iters, replays=3):
    """Average device time (s) per fn(i) launch on torch's current stream:
    `iters` launches are captured once as a HIP graph and the graph is
    replayed between two HIP events on that stream, so the host's launch
    rate does not enter the figure."""
    st = torch.cuda.current_stream()
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(replays):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / 1e3 / (iters * replays)


def roofline(bytes_per_launch, seconds, traffic=None):
    a = bytes_per_launch / seconds
    return {"bound": "hbm", "achieved": round(a / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": round(a / HBM_PEAK, 4), "traffic": traffic}


def plain_read_time(torch, hip, st, nbytes, iters):
    """Device time (s) of one launch that only streams nbytes from HBM: the
    rina_hip_read_probe kernel over a ring of buffers larger than the
    256 MB MALL, best of four grid sizes.  A kernel's ceiling_frac is this
    time over its own at the same byte count."""
    n = min(64, max(2, -(-640_000_000 // nbytes)))   # every entry read once per graph replay
    ring = [torch.empty(nbytes // 4 + 4, device="cuda") for _ in range(n)]
    sink = torch.empty(8192, device="cuda")
    best = None
    for grid in (256, 512, 1024, 2048):
        t = time_kernel(torch, lambda i=0: hip.rina_hip_read_probe(ring[i % n].data_ptr(), nbytes, grid,
                                                                   sink.data_ptr(), st), max(iters, n))
        best = t if best is None else min(best, t)
    del ring
    return best


def with_ceiling(roof, t_kernel, t_plain):
    roof = dict(roof)
    roof["plain_read_us"] = round(t_plain * 1e6, 3)
    roof["ceiling_frac"] = round(t_plain / t_kernel, 4)
    return roof


_hiprt = None


def d2h_f32(ptr, n):
    """n floats of engine-owned device memory to a numpy array."""
    global _hiprt
    if _hiprt is None:
        _hiprt = C.CDLL("libamdhip64.so")
        _hiprt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hiprt.hipMemcpy.restype = C.c_int
    out = np.empty(n, np.float32)
    assert _hiprt.hipMemcpy(out.ctypes.data, ptr, n * 4, 2) == 0   # hipMemcpyDeviceToHost
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_lm_head_fp32.json")
STACK_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_decode_layers_config2.json")
COPY_BYTES = 512 << 20          # calibration copy: 512 MiB read + 512 MiB written (> the 256 MB MALL)
STACK_POS = 543                 # traffic probe of the layer stack: the average config-2 decode position


def _probe_setup():
    import torch
    rina = pkg()
    hip = rina.load_hip()
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    return torch, rina, hip, stream.cuda_stream


def traffic_probe(iters):
    """Run under rocprofv3 --pmc: the LM head matvec (128256 x 2048 fp32) and
    a plain device copy of COPY_BYTES, `iters` launches each."""
    torch, rina, hip, st = _probe_setup()
    d, V = 2048, 128256
    w = torch.randn(V * d, device="cuda") * 0.02
    x = torch.randn(d, device="cuda")
    y = torch.empty(V, device="cuda")
    src = torch.randn(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(iters):
        rina.check(hip.rina_hip_linear(w.data_ptr(), rina.QT_FP32, x.data_ptr(), y.data_ptr(), 1, V, d, st), "lm head")
        dst.copy_(src)
    torch.cuda.synchronize()
    print("probe done", flush=True)


def traffic_probe_stack(iters):
    """Run under rocprofv3 --pmc: `iters` tokens of config 2's decode layer
    stack (LayerStack at STACK_POS) and as many plain copies of COPY_BYTES."""
    torch, rina, hip, st = _probe_setup()
    synth = importlib.import_module("rina_amd.synth")
    sm = synth.SynthLlama(dict(synth.LLAMA_1B), qt=rina.QT_Q4_0F, seed=1, max_seq=STACK_POS + 8)
    ls = LayerStack(torch, hip, rina, sm, sm.cfg, STACK_POS, st)
    src = torch.randn(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(iters):
        ls.token()
        dst.copy_(src)
    torch.cuda.synchronize()
    print("probe done: %d tokens, %d bytes per token" % (iters, ls.bytes_per_token()), flush=True)


STACK_KERNELS = ("gemv_direct_kernel", "attn_vsplit_kernel", "attn_split_kernel", "attn_combine_kernel")


def _pmc_sum(db, counter, kernels, ncopy):
    """Per-dispatch sums of `counter` (KiB): over every dispatch of a kernel
    whose name contains one of `kernels`, and over the `ncopy` largest
    dispatches of the copy kernel (the calibration copies; the probe's set-up
    makes smaller device copies of its own)."""
    import sqlite3
    c = sqlite3.connect(db)
    cols = [r[1] for r in c.execute("pragma table_info(counters_collection)")]
    ix = {n: i for i, n in enumerate(cols)}
    tot = {"k": 0.0, "copy": 0.0}
    n = {"k": 0, "copy": 0}
    per = {}
    copies = []
    for r in c.execute("select * from counters_collection").fetchall():
        if r[ix["counter_name"]] != counter:
            continue
        name = r[ix["kernel_name"]]
        v = float(r[ix["value"]])
        if any(k in name for k in kernels):
            tot["k"] += v
            n["k"] += 1
            short = next(k for k in kernels if k in name)
            per[short] = per.get(short, 0.0) + v
        elif "copyBuffer" in name:
            copies.append(v)
    copies = sorted(copies, reverse=True)[:ncopy]
    if len(copies) < ncopy or copies[-1] < 0.9 * copies[0]:
        raise RuntimeError("%s: %d calibration copies expected, largest copy dispatches read %s" %
                           (counter, ncopy, copies))
    tot["copy"], n["copy"] = sum(copies), len(copies)
    return tot, n, per


def _pmc_runs(probe_flag, iters, kernels):
    import subprocess
    import tempfile
    out = {}
    env = dict(os.environ, TMPDIR="/tmp")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="rina_pmc_", dir="/tmp")
        cmd = ["timeout", "-s", "KILL", "170", "rocprofv3", "--pmc", counter, "-d", d, "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), probe_flag, str(iters)]
        log("running: " + " ".join(cmd))
        subprocess.run(cmd, cwd="/tmp", env=env, check=True, timeout=180)
        db = [os.path.join(r, f) for r, _, fs in os.walk(d) for f in fs if f.endswith("_results.db")][0]
        tot, n, per = _pmc_sum(db, counter, kernels, iters)
        log("%s KiB: %s (dispatches %s)" % (counter, tot, n))
        factor = COPY_BYTES / (tot["copy"] / n["copy"] * 1024.0)       # bytes per counted KiB
        out[counter] = {"kernel_kib_total": tot["k"], "kernel_dispatches": n["k"],
                        "copy_kib": tot["copy"] / n["copy"], "factor": factor,
                        "per_kernel_kib_total": per}
    return out


def measure_traffic(iters=10):
    """rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE, one run each)
    over two probes: the LM head and config 2's decode layer stack.  Each
    counter is scaled by its reading on a plain copy of known size in the
    same run.  Writes TRAFFIC_FILE and STACK_TRAFFIC_FILE.  The profiler runs
    as a child process."""
    out = _pmc_runs("--traffic-probe", iters, ("gemv_f32_kernel",))
    lmb = {c: out[c]["kernel_kib_total"] / out[c]["kernel_dispatches"] * 1024.0 * out[c]["factor"] for c in out}
    lm_alg = 128256 * 2048 * 4 + 2048 * 4 + 128256 * 4
    res = {"kernel": "gemv_f32_kernel (tied LM head 128256x2048 fp32)", "algorithmic_bytes": lm_alg,
           "fetch_bytes": round(lmb["FETCH_SIZE"]), "write_bytes": round(lmb["WRITE_SIZE"]),
           "hbm_bytes": round(lmb["FETCH_SIZE"] + lmb["WRITE_SIZE"]),
           "calibration": "plain device copy of %d bytes (reads and writes %d bytes)" % (COPY_BYTES, COPY_BYTES),
           "counters": out, "command": "python bench.py --measure-traffic"}
    res["traffic_over_algorithmic"] = round(res["hbm_bytes"] / lm_alg, 4)
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res), flush=True)
    tokens = 4
    out = _pmc_runs("--traffic-probe-stack", tokens, STACK_KERNELS)
    tb = {c: out[c]["kernel_kib_total"] / tokens * 1024.0 * out[c]["factor"] for c in out}
    pkg()
    synth = importlib.import_module("rina_amd.synth")
    alg = 16 * sum(stack_bytes(synth.LLAMA_1B, STACK_POS).values())
    res = {"kernel": "config-2 decode layer stack (%s; 16 layers, fp32 KV at position %d)"
                     % (", ".join(k for k in STACK_KERNELS if out["FETCH_SIZE"]["per_kernel_kib_total"].get(k)), STACK_POS),
           "algorithmic_bytes": alg, "tokens": tokens,
           "fetch_bytes": round(tb["FETCH_SIZE"]), "write_bytes": round(tb["WRITE_SIZE"]),
           "hbm_bytes": round(tb["FETCH_SIZE"] + tb["WRITE_SIZE"]),
           "calibration": "plain device copy of %d bytes (reads and writes %d bytes)" % (COPY_BYTES, COPY_BYTES),
           "counters": out, "command": "python bench.py --measure-traffic"}
    res["traffic_over_algorithmic"] = round(res["hbm_bytes"] / alg, 4)
    with open(STACK_TRAFFIC_FILE, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res), flush=True)


def committed_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch (per token for the layer stack) from a committed
    PMC measurement."""
    try:
        with open(path) as f:
            t = json.load(f)
        return t["hbm_bytes"], {
            "fetch_bytes": t["fetch_bytes"], "write_bytes": t["write_bytes"],
            "over_algorithmic": t["traffic_over_algorithmic"],
            "source": "profiles/%s (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, each scaled by the same counter on a "
                      "plain copy of known size)" % os.path.basename(path)}
    except (OSError, KeyError, ValueError):
        return None, None


STACK_KINDS = ("qkv", "attn", "wo", "w13", "w2")
STACK_NOTES = {"qkv": "fused q/k/v Q4_0F matvec with the ln1 RMSNorm prologue (N 3072, K 2048)",
               "attn": "RoPE + fp32 KV append + decode attention (one launch up to rina_hip_gqa_one_launch_positions(), "
                       "else split + merge)",
               "wo": "W_o Q4_0F matvec + residual (N 2048, K 2048)",
               "w13": "W1/W3 Q4_0F matvec pair with the ln2 RMSNorm prologue and SiLU*up (N 8192, K 2048)",
               "w2": "W2 Q4_0F matvec + residual (N 2048, K 8192)"}


def stack_bytes(cfg, pos):
    """Algorithmic bytes of one layer's decode launches at position pos
    (Q4_0F weights, 20 B per 32 values; fp32 activations, norm weights and
    K/V rows): weights once, every vector read or written once."""
    d, H, Hkv, dh, hd = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["hidden_dim"]
    kvd = Hkv * dh
    bq = lambda n, k: n * k // 32 * 20
    return {"qkv": bq(H * dh + 2 * kvd, d) + 2 * d * 4 + (H * dh + 2 * kvd) * 4,
            "attn": pos * kvd * 8 + (2 * H * dh + 2 * kvd) * 4,
            "wo": bq(d, H * dh) + H * dh * 4 + 2 * d * 4,
            "w13": 2 * bq(hd, d) + 2 * d * 4 + hd * 4,
            "w2": bq(d, hd) + hd * 4 + 2 * d * 4}


class LayerStack:
    """Config 2's decode layers, issued through the C-ABI exactly as
    gqa_layer.cpp's decode step issues them, over the model's own 16 layers
    of weights (608 MB, larger than the 256 MB MALL): per layer the quant
    matvecs and the decode attention, the launches the metric names.  The
    embedding, the fp32 LM head and the argmax are not part of it.  Each
    layer has its own fp32 K/V cache filled with N(0,1) rows; the attention
    appends at host position `pos` and reads positions 0..pos."""

    def __init__(self, torch, hip, rina, sm, cfg, pos, st):
        self.hip, self.rina, self.st, self.pos = hip, rina, st, pos
        d, H, Hkv, dh, hd, L = (cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["hidden_dim"],
                                cfg["n_layers"])
        self.d, self.H, self.Hkv, self.dh, self.hd, self.L = d, H, Hkv, dh, hd, L
        kvd = Hkv * dh
        self.msq = pos + 8
        self.kc = [torch.randn(self.msq * kvd, device="cuda") for _ in range(L)]
        self.vc = [torch.randn(self.msq * kvd, device="cuda") for _ in range(L)]
        self.h = torch.randn(d, device="cuda")
        self.q, self.k, self.v = (torch.empty(n, device="cuda") for n in (H * dh, kvd, kvd))
        self.a, self.g = torch.empty(H * dh, device="cuda"), torch.empty(hd, device="cuda")
        self.wsb = int(hip.rina_hip_gqa_attention_workspace(1, H, dh, self.msq))
        self.ws = torch.empty(self.wsb // 4 + 4, device="cuda")
        W = lambda l, n: sm.dev["transformer.h.%d.%s" % (l, n)].data_ptr()
        LS = rina.LinearSeg
        self.lay = []
        for l in range(L):
            self.lay.append(dict(
                qkv=(LS * 3)(LS(W(l, "attn.w_q.weight"), None, self.q.data_ptr(), H * dh),
                             LS(W(l, "attn.w_k.weight"), None, self.k.data_ptr(), kvd),
                             LS(W(l, "attn.w_v.weight"), None, self.v.data_ptr(), kvd)),
                wo=LS(W(l, "attn.w_o.weight"), None, self.h.data_ptr(), d),
                w13=LS(W(l, "mlp.w1.weight"), W(l, "mlp.w3.weight"), self.g.data_ptr(), hd),
                w2=LS(W(l, "mlp.w2.weight"), None, self.h.data_ptr(), d),
                ln1=W(l, "ln1.weight"), ln2=W(l, "ln2.weight"),
                rope=[W(l, "attn.%s" % n) for n in ("rope_q.cos", "rope_q.sin", "rope.cos", "rope.sin")]))
        self.bytes = stack_bytes(cfg, pos)

    def call(self, kind, l):
        hip, r, st, w = self.hip, self.rina, self.st, self.lay[l % self.L]
        if kind == "qkv":
            return hip.rina_hip_linear_fused(w["qkv"], 3, r.QT_Q4_0F, self.h.data_ptr(), 1, self.d, r.EPI_STORE,
                                             r.PRO_RMSNORM, w["ln1"], 1e-5, st)
        if kind == "attn":
            c = w["rope"]
            return hip.rina_hip_gqa_decode_attention(
                self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), c[0], c[1], c[2], c[3],
                self.kc[l % self.L].data_ptr(), self.vc[l % self.L].data_ptr(), 0, self.H, self.Hkv, self.dh,
                self.pos, None, self.msq, self.a.data_ptr(), None, self.ws.data_ptr(), self.wsb, st)
        if kind == "wo":
            return hip.rina_hip_linear_fused(C.byref(w["wo"]), 1, r.QT_Q4_0F, self.a.data_ptr(), 1, self.H * self.dh,
                                             r.EPI_ADD, r.PRO_NONE, None, 0.0, st)
        if kind == "w13":
            return hip.rina_hip_linear_fused(C.byref(w["w13"]), 1, r.QT_Q4_0F, self.h.data_ptr(), 1, self.d,
                                             r.EPI_SWIGLU, r.PRO_RMSNORM, w["ln2"], 1e-5, st)
        return hip.rina_hip_linear_fused(C.byref(w["w2"]), 1, r.QT_Q4_0F, self.g.data_ptr(), 1, self.hd, r.EPI_ADD,
                                         r.PRO_NONE, None, 0.0, st)

    def token(self, i=0):
        for l in range(self.L):
            for kind in STACK_KINDS:
                self.rina.check(self.call(kind, l), kind)
        return 0

    def bytes_per_token(self):
        return self.L * sum(self.bytes.values())


def layer_stack_roofline(torch, hip, rina, sm, cfg, pos, st, iters):
    """The headline roofline: config 2's decode layer stack (the quant
    matvecs and decode attention of all 16 layers) as one graph replay per
    token, its algorithmic bytes per token over its device time per token;
    plus each launch class timed on its own over the 16 layers."""
    ls = LayerStack(torch, hip, rina, sm, cfg, pos, st)
    t_tok = time_kernel(torch, ls.token, max(2, iters // 8))
    per = {}
    for kind in STACK_KINDS:
        t = time_kernel(torch, lambda i=0, k=kind: ls.call(k, i), ls.L * max(1, iters // 8))
        b = ls.bytes[kind]
        per[kind] = {"bytes_per_launch": b, "avg_us": round(t * 1e6, 3), "frac": round(b / t / HBM_PEAK, 4),
                     "note": STACK_NOTES[kind]}
    tb = ls.bytes_per_token()
    traffic, detail = committed_traffic(STACK_TRAFFIC_FILE)
    roof = roofline(tb, t_tok, traffic)
    one = pos + 1 <= hip.rina_hip_gqa_one_launch_positions()
    roof.update({"kernel": "config-2 decode layer stack: 16 x [q/k/v + ln1, RoPE + KV append + attention "
                           "(%s), W_o + residual, W1/W3 + ln2 + SiLU*up, W2 + residual], Q4_0F, fp32 "
                           "KV at position %d" % ("one launch" if one else "split + merge", pos),
                 "bytes_per_token": tb, "us_per_token": round(t_tok * 1e6, 2),
                 "launches_per_token": (5 if one else 6) * ls.L, "per_launch": per})
    if detail:
        roof["traffic_detail"] = detail
    log("layer stack at position %d: %.1f us per token, %.0f GB/s (%.3f of peak)" %
        (pos, t_tok * 1e6, tb / t_tok / 1e9, tb / t_tok / HBM_PEAK))
    for kind in STACK_KINDS:
        log("  %-5s %7.2f us  %.3f" % (kind, per[kind]["avg_us"], per[kind]["frac"]))
    del ls
    return roof


def config4_kernel_roofs(torch, hip, rina, synth, st, pos, iters):
    """Live device times of config 4's two largest per-layer stages at its
    decode context, over rings larger than the 256 MB MALL (as between the
    layers of a decode step): the latent attention at position `pos`
    (RMSNorm + RoPE append, q_lat, softmax over pos+1 latent records, W_vb)
    and the MoE block (router, top-6 of 64, shared + routed gate/up, down)."""
    H, nope, rope, vd, dc, d = 16, 128, 64, 128, 512, 2048
    E, K, F, S = 64, 6, 1408, 2816
    R = dc + rope
    q2b = lambda n: n // 256 * 84
    out = {}
    ms = pos + 8
    nr = 64                                   # 64 x (4.7 MB cache + 0.7 MB W_kv_b) > MALL
    caches = [torch.randn(ms * R, device="cuda") for _ in range(nr)]
    wkvb = [synth.q2k_device(H * (nope + vd) * dc, 100 + i) for i in range(nr)]
    q = torch.randn(H * (nope + rope), device="cuda")
    kva = torch.randn(R, device="cuda")
    kn = torch.ones(dc, device="cuda")
    cos, sin = synth.make_rope(rope, ms, 10000.0)
    cd, sd = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    o = torch.empty(H * vd, device="cuda")
    pd = torch.tensor([pos], dtype=torch.int32, device="cuda")
    wsb = int(hip.rina_hip_mla_attention_workspace(H, dc, rope, ms))
    ws = torch.empty(wsb // 4 + 4, device="cuda")
    t = time_kernel(torch, lambda i=0: hip.rina_hip_mla_decode_attention_ex(
        q.data_ptr(), kva.data_ptr(), kn.data_ptr(), 1e-5, cd.data_ptr(), sd.data_ptr(), wkvb[i % nr].data_ptr(),
        rina.QT_Q2_K, caches[i % nr].data_ptr(), H, nope, rope, vd, dc, 0, pd.data_ptr(), ms, ms - 1,
        o.data_ptr(), ws.data_ptr(), wsb, st), max(iters, nr))   # every ring entry once per replay
    nb = (pos + 1) * R * 4 + q2b(H * (nope + vd) * dc) + (H * (nope + rope) + R + H * vd) * 4
    out["decode_mla_latent_p%d" % pos] = dict(
        with_ceiling(roofline(nb, t), t, plain_read_time(torch, hip, st, nb, iters)), bytes_per_launch=nb,
        avg_us=round(t * 1e6, 3), note="config 4 latent attention, device position (graph replay): "
                                       "mla_chunk_kernel + mla_combine_kernel")
    log("config-4 latent attention at %d: %.2f us" % (pos, t * 1e6))
    del caches, wkvb
    # MoE block: 4 layers' weights (4 x 187 MB), h updated in place by every
    # call, so the selected experts change from call to call
    nl = 4
    lay = [dict(wr=torch.randn(E * d, device="cuda") * 0.02, sg=synth.q2k_device(S * d, 10 * l + 1),
                su=synth.q2k_device(S * d, 10 * l + 2), sd=synth.q2k_device(d * S, 10 * l + 3),
                wg=synth.q2k_device(E * F * d, 10 * l + 4), wu=synth.q2k_device(E * F * d, 10 * l + 5),
                wd=synth.q2k_device(E * d * F, 10 * l + 6)) for l in range(nl)]
    h = torch.randn(d, device="cuda")
    ln2 = torch.ones(d, device="cuda")
    wsb = int(hip.rina_hip_moe_block_workspace(d, E, K, F, S))
    ws = torch.empty(wsb // 4 + 4, device="cuda")
    sgu, sdn = q2b(F * d), q2b(d * F)
    def moe(i=0):
        w = lay[i % nl]
        return hip.rina_hip_moe_block(h.data_ptr(), ln2.data_ptr(), 1e-5, w["wr"].data_ptr(), rina.QT_FP32,
                                      w["sg"].data_ptr(), w["su"].data_ptr(), w["sd"].data_ptr(), S,
                                      w["wg"].data_ptr(), w["wu"].data_ptr(), w["wd"].data_ptr(), rina.QT_Q2_K,
                                      sgu, sdn, E, K, d, F, ws.data_ptr(), wsb, st)
    t = time_kernel(torch, moe, iters)
    nb = E * d * 4 + 3 * q2b(S * d) + 3 * K * q2b(F * d) + 2 * d * 4
    out["decode_moe_block_q2k"] = dict(
        with_ceiling(roofline(nb, t), t, plain_read_time(torch, hip, st, nb, iters)), bytes_per_launch=nb,
        avg_us=round(t * 1e6, 3), note="config 4 MoE block (64 experts, top-6 of 1408, 2 shared): "
                                       "moe_router_kernel + moe_gate_up_q2_kernel + moe_down_q2_kernel")
    log("config-4 MoE block: %.2f us" % (t * 1e6))
    del lay
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-steps", type=int, default=4)
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--no-config4", action="store_true", help="skip the DeepSeek MLA + MoE (config 4) decode line")
    ap.add_argument("--config4-steps", type=int, default=32)
    ap.add_argument("--config4-prompt", type=int, default=2040,
                    help="config 4 prompt length (decode context); shorter for counter runs, where every dispatch "
                         "of the per-token prompt path is serialized")
    ap.add_argument("--no-config5", action="store_true", help="skip the RINA Jamba (config 5) decode line")
    ap.add_argument("--no-config3", action="store_true", help="skip the context-4096 quantized-KV (config 3) line")
    ap.add_argument("--config3-steps", type=int, default=8)
    ap.add_argument("--traffic-probe", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--traffic-probe-stack", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--measure-traffic", action="store_true",
                    help="run the two rocprofv3 --pmc passes for the LM head's HBM traffic and write them to profiles/")
    args = ap.parse_args()
    if args.traffic_probe:
        traffic_probe(args.traffic_probe)
        return
    if args.traffic_probe_stack:
        traffic_probe_stack(args.traffic_probe_stack)
        return
    if args.measure_traffic:
        measure_traffic()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X in this build "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    rina = pkg()
    synth = importlib.import_module("rina_amd.synth")
    hip = rina.load_hip()
    eng = rina.load_engine()
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()          # default priority
    torch.cuda.set_stream(stream)
    st = stream.cuda_stream

    cfg = dict(synth.LLAMA_1B)
    cfg["n_layers"] = args.layers
    max_seq = args.prompt + args.warmup + args.steps + 8
    t0 = time.time()
    want_cpu = not args.no_cpu
    sm = synth.SynthLlama(cfg, qt=rina.QT_Q4_0F, seed=1, max_seq=max_seq, keep_host=want_cpu)
    log("model built in %.1fs" % (time.time() - t0))
    inf = sm.infer("fp32", max_seq)
    prompt = np.random.default_rng(3).integers(0, cfg["vocab_size"], args.prompt).astype(np.int32)
    first = (C.c_int * (1 + args.warmup))()
    rina.check(eng.rina_infer_generate(inf, prompt.ctypes.data_as(C.POINTER(C.c_int)), args.prompt,
                                       1 + args.warmup, first, 1, st, None), "prefill + warmup")
    log("prefill + %d warmup steps done" % args.warmup)
    out = (C.c_int * args.steps)()
    ms = C.c_float()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    rina.check(eng.rina_infer_decode(inf, args.steps, out, 1, st, C.byref(ms)), "decode")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    tok_s = args.steps / wall
    log("decode: %d steps, %.3f ms/step (device %.3f ms/step), %.1f tok/s" %
        (args.steps, wall * 1e3 / args.steps, ms.value / args.steps, tok_s))
    tokens = list(first) + list(out)
    # prompt phase of the same model (context only; not the metric): the
    # 512-token prefill with the last row's logits and its argmax, timed on
    # its second run (the first sizes the activation buffers)
    pre_ms = []
    one = (C.c_int * 1)()
    for _ in range(2):
        torch.cuda.synchronize()
        t_p = time.perf_counter()
        rina.check(eng.rina_infer_generate(inf, prompt.ctypes.data_as(C.POINTER(C.c_int)), args.prompt, 1, one, 0,
                                           st, None), "prefill")
        torch.cuda.synchronize()
        pre_ms.append((time.perf_counter() - t_p) * 1e3)
    prefill = {"prompt": args.prompt, "ms": round(pre_ms[-1], 3),
               "tokens_per_s": round(args.prompt / (pre_ms[-1] / 1e3), 1),
               "note": "Q4 linears on v_mfma_f32_16x16x32_bf16 with x split exactly into three bf16 parts "
                       "(fp32 products, fp32 sums); prompt attention from position 0 on "
                       "v_mfma_f32_16x16x4f32 in 64-position blocks (one softmax rescale per block)"}
    log("prefill: %d tokens in %.2f ms (%.0f tok/s)" % (args.prompt, pre_ms[-1], prefill["tokens_per_s"]))
    # the GPU's K/V rows of the prompt, so the CPU baseline decodes at the
    # GPU's positions from the same cache
    cache_rows = []
    if want_cpu:
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        torch.cuda.synchronize()
        for layer in range(cfg["n_layers"]):
            for which in (0, 1):
                ptr, nb = C.c_void_p(), C.c_size_t()
                rina.check(eng.rina_infer_kv_region(inf, layer, which, C.byref(ptr), C.byref(nb)), "kv region")
                cache_rows.append(d2h_f32(ptr.value, args.prompt * kvd))
    eng.rina_infer_destroy(inf)

    # ---- dominant kernel: fp32 tied LM head GEMV (128256 x 2048), HIP events on our stream
    d, V = cfg["dim"], cfg["vocab_size"]
    wte = sm.dev["transformer.wte.weight"]
    x = torch.randn(d, device="cuda")
    y = torch.empty(V, device="cuda")
    lm_bytes = V * d * 4 + d * 4 + V * 4
    t_lm = time_kernel(torch, lambda i=0: hip.rina_hip_linear(wte.data_ptr(), rina.QT_FP32, x.data_ptr(), y.data_ptr(),
                                                              1, V, d, st), args.kernel_iters)
    traffic, traffic_detail = committed_traffic()
    lm_roof = with_ceiling(roofline(lm_bytes, t_lm, traffic), t_lm,
                           plain_read_time(torch, hip, st, lm_bytes, max(4, args.kernel_iters // 5)))
    log("lm_head fp32 GEMV: %.1f us, %.0f GB/s (plain read %.1f us)" %
        (t_lm * 1e6, lm_bytes / t_lm / 1e9, lm_roof["plain_read_us"]))

    # ---- headline roofline: the metric's kernels, config 2's quant matvecs
    # and decode attention over all 16 layers, at the timed run's middle position
    stack_roof = layer_stack_roofline(torch, hip, rina, sm, cfg, args.prompt + 1 + args.warmup + args.steps // 2, st,
                                      args.kernel_iters)

    # ---- Q4_0F SwiGLU matvec over the model's own layers (ring > MALL)
    hd = cfg["hidden_dim"]
    w1s = [sm.dev["transformer.h.%d.mlp.w1.weight" % l] for l in range(cfg["n_layers"])]
    w3s = [sm.dev["transformer.h.%d.mlp.w3.weight" % l] for l in range(cfg["n_layers"])]
    g = torch.empty(hd, device="cuda")
    segs = [rina.LinearSeg(w1s[i].data_ptr(), w3s[i].data_ptr(), g.data_ptr(), hd) for i in range(len(w1s))]
    nl = len(segs)

    def swiglu(i=0):
        return hip.rina_hip_linear_fused(C.byref(segs[i % nl]), 1, rina.QT_Q4_0F, x.data_ptr(), 1, d,
                                         rina.EPI_SWIGLU, rina.PRO_NONE, None, 0.0, st)
    t_sw = time_kernel(torch, swiglu, args.kernel_iters)
    sw_bytes = 2 * hd * d // 32 * 20 + d * 4 + hd * 4
    sw_roof = with_ceiling(roofline(sw_bytes, t_sw), t_sw, plain_read_time(torch, hip, st, sw_bytes, args.kernel_iters))
    log("Q4_0F W1/W3 SwiGLU matvec: %.1f us, %.0f GB/s" % (t_sw * 1e6, sw_bytes / t_sw / 1e9))

    # ---- prompt phase: the same W1/W3 SwiGLU at M = args.prompt rows on the
    # matrix cores, HIP events on our stream.  The kernel forms fp32 products
    # from three bf16 MFMAs each (x split exactly into three bf16 parts), so
    # its peak in fp32-product flop is the dense bf16 peak / 3 (2500 / 3
    # TFLOP/s); the flop counted are the algorithmic 2 per multiply-add.
    Mp = args.prompt
    xp = torch.randn(Mp * d, device="cuda")
    gp = torch.empty(Mp * hd, device="cuda")
    segp = [rina.LinearSeg(w1s[i].data_ptr(), w3s[i].data_ptr(), gp.data_ptr(), hd) for i in range(len(w1s))]

    def swiglu_p(i=0):
        return hip.rina_hip_linear_fused(C.byref(segp[i % nl]), 1, rina.QT_Q4_0F, xp.data_ptr(), Mp, d,
                                         rina.EPI_SWIGLU, rina.PRO_NONE, None, 0.0, st)
    t_swp = time_kernel(torch, swiglu_p, 8, replays=2)
    swp_flop = 2 * 2 * Mp * hd * d
    swp_peak = 2500.0 / 3
    swp_roof = {"bound": "mfma", "achieved": round(swp_flop / t_swp / 1e12, 2), "peak": round(swp_peak, 1),
                "unit": "TFLOP/s", "frac": round(swp_flop / t_swp / (swp_peak * 1e12), 4), "traffic": None,
                "fp32_mfma_frac": round(swp_flop / t_swp / 157.3e12, 4)}
    log("prompt W1/W3 SwiGLU (M %d): %.1f us, %.1f TFLOP/s" % (Mp, t_swp * 1e6, swp_flop / t_swp / 1e12))
    del xp, gp

    # ---- config 1: Q4_0 GEMV 8192 x 2048 over a ring of 64 weight copies (~604 MB)
    N1, K1 = 8192, 2048
    w0 = synth.normal(1, N1 * K1, 0.02)
    ring = [synth.pack_on_device(w0, rina.QT_Q4_0)]
    for i in range(63):
        ring.append(ring[0].clone())
    x1 = torch.from_numpy(np.random.default_rng(2).standard_normal(K1).astype(np.float32)).cuda()
    y1 = torch.empty(N1, device="cuda")
    t_q4 = time_kernel(torch, lambda i=0: hip.rina_hip_linear(ring[i % 64].data_ptr(), rina.QT_Q4_0, x1.data_ptr(),
                                                              y1.data_ptr(), 1, N1, K1, st), args.kernel_iters * 4)
    q4_bytes = N1 * K1 // 32 * 18 + K1 * 4 + N1 * 4
    del ring
    q4_roof = with_ceiling(roofline(q4_bytes, t_q4), t_q4, plain_read_time(torch, hip, st, q4_bytes, args.kernel_iters))
    log("config-1 Q4_0 GEMV: %.2f us, %.0f GB/s (plain read %.2f us)" %
        (t_q4 * 1e6, q4_bytes / t_q4 / 1e9, q4_roof["plain_read_us"]))

    # ---- decode attention of one layer (RoPE, append, attention), the
    # metric's other kernel: config 2's fp32 cache at position 530 and
    # config 3's q8 cache at position 4095, over rings of caches larger than
    # the MALL (as between the layers of a decode step)
    attn_roofs = {}
    H, Hkv, dh = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    kvd = Hkv * dh
    for name, mode, pos, kb, vb in (("decode_attention_fp32_p530", 0, 530, 4.0, 4.0),
                                    ("decode_attention_q8_p4095", 1, 4095, 34 / 32, 34 / 32)):
        msq = pos + 8
        region = int(hip.rina_hip_kv_region_bytes(mode, 0, msq, kvd))
        nring = min(128, max(2, -(-640_000_000 // (2 * region))))
        kc = [torch.zeros(region // 4 + 4, device="cuda") for _ in range(nring)]
        vc = [torch.zeros(region // 4 + 4, device="cuda") for _ in range(nring)]
        if mode:   # valid q8 blocks: pack random rows once, copy into every ring entry
            rows = torch.randn(msq * kvd, device="cuda")
            hip.rina_hip_kv_quantize(rina.KVF_Q8_0, rows.data_ptr(), kc[0].data_ptr(), msq * kvd, st)
            hip.rina_hip_kv_quantize(rina.KVF_Q8_0, rows.data_ptr(), vc[0].data_ptr(), msq * kvd, st)
        else:
            kc[0].normal_()
            vc[0].normal_()
        for i in range(1, nring):
            kc[i].copy_(kc[0])
            vc[i].copy_(vc[0])
        cos, sin = synth.make_rope(dh, msq, cfg.get("rope_theta", 500000.0))
        cd, sd = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        qa, ka, va = torch.randn(H * dh, device="cuda"), torch.randn(kvd, device="cuda"), torch.randn(kvd, device="cuda")
        oa = torch.empty(H * dh, device="cuda")
        wsb = int(hip.rina_hip_gqa_attention_workspace(1, H, dh, msq))
        wsa = torch.empty(wsb // 4 + 4, device="cuda")
        t_at = time_kernel(torch, lambda i=0: hip.rina_hip_gqa_decode_attention(
            qa.data_ptr(), ka.data_ptr(), va.data_ptr(), cd.data_ptr(), sd.data_ptr(), cd.data_ptr(), sd.data_ptr(),
            kc[i % nring].data_ptr(), vc[i % nring].data_ptr(), mode, H, Hkv, dh, pos, None, msq, oa.data_ptr(), None,
            wsa.data_ptr(), wsb, st), max(args.kernel_iters, nring))   # every ring entry once per replay
        at_bytes = int(pos * kvd * (kb + vb)) + (2 * H * dh + 2 * kvd) * 4
        attn_roofs[name] = dict(with_ceiling(roofline(at_bytes, t_at), t_at,
                                             plain_read_time(torch, hip, st, at_bytes, args.kernel_iters)),
                                bytes_per_launch=at_bytes, avg_us=round(t_at * 1e6, 3),
                                note="RoPE + append + attention: one launch"
                                if mode == 0 and pos + 1 <= hip.rina_hip_gqa_one_launch_positions()
                                else "RoPE + append + split-sequence attention + chunk merge, two launches")
        log("%s: %.2f us, %.0f GB/s" % (name, t_at * 1e6, at_bytes / t_at / 1e9))
        del kc, vc

    # ---- config 4: DeepSeek-V2-Lite-shaped MLA + MoE decode, random Q2_K weights
    cfg4 = None
    if not args.no_config4:
        t4 = time.time()
        p4, s4 = args.config4_prompt, args.config4_steps   # context 2048: decode steps at positions 2041..
        ds = synth.SynthDeepSeek(seed=1, max_seq=p4 + s4 + 8)
        log("config 4 model built in %.1fs" % (time.time() - t4))
        inf4 = ds.infer()
        pr4 = np.random.default_rng(4).integers(0, ds.cfg["vocab_size"], p4).astype(np.int32)
        first4 = (C.c_int * 2)()
        rina.check(eng.rina_infer_generate(inf4, pr4.ctypes.data_as(C.POINTER(C.c_int)), p4, 2, first4, 1, st, None),
                   "config 4 prefill")
        out4 = (C.c_int * s4)()
        torch.cuda.synchronize()
        tq = time.perf_counter()
        rina.check(eng.rina_infer_decode(inf4, s4, out4, 1, st, None), "config 4 decode")
        torch.cuda.synchronize()
        w4 = time.perf_counter() - tq
        eng.rina_infer_destroy(inf4)
        b4 = ds.bytes_per_token(p4 + 1 + s4 // 2)
        cfg4 = {"workload": "DeepSeek-V2-Lite-shaped MLA + MoE decode: 27 layers (1 dense + 26 MoE, 64 experts top-6 "
                            "of 1408, 2 shared), d 2048, 16 heads, kv_lora_rank 512, rope 64, vocab 102400, random "
                            "zero-mean Q2_K weights, latent fp32 cache, %d-token seeded prompt (prefill untimed), "
                            "greedy steps at positions %d..%d" % (p4, p4 + 1, p4 + s4),
                "latent_kv_bytes_per_token": ds.cfg["n_layers"] * (p4 + 1 + s4 // 2) * (ds.cfg["dc"] + ds.cfg["rope"]) * 4,
                "tokens_per_s": round(s4 / w4, 2), "ms_per_step": round(w4 * 1e3 / s4, 4), "steps": s4,
                "bytes_per_token": b4, "hbm_gbps": round(b4 * s4 / w4 / 1e9, 1),
                "hbm_frac": round(b4 * s4 / w4 / HBM_PEAK, 4), "tokens_head": list(first4) + list(out4)[:6]}
        log("config 4: %.3f ms/step, %.1f tok/s" % (w4 * 1e3 / s4, s4 / w4))
        ds.close()
        del ds
        torch.cuda.empty_cache()
        attn_roofs.update(config4_kernel_roofs(torch, hip, rina, synth, st, p4, args.kernel_iters))

    # ---- config 5: RINA Gen6 Jamba hybrid at context 2048, 1900-token prompt
    # then 128 greedy steps: with its q2 K / q1 V RINA-MLA cache (the
    # config's stated cache, rina_mla_kv_mode "q2k_q1v"), and with the fp32
    # cache (the reference engine's RINA-MLA numerics)
    cfg5 = {}
    if not args.no_config5:
        p5, s5 = 1900, 128   # context 2048: steps at positions 1901..2028
        for key, kvm in (("config5_rina_jamba", "q2k_q1v"), ("config5_rina_jamba_fp32_cache", "fp32")):
            jm = synth.SynthJamba(seed=1, max_seq=2048, kv_mode=kvm)
            inf5 = jm.infer()
            pr5 = np.random.default_rng(5).integers(0, jm.cfg["vocab_size"], p5).astype(np.int32)
            # two generated tokens: the second step captures the decode graph
            # outside the timed region (as for config 4)
            first5 = (C.c_int * 2)()
            rina.check(eng.rina_infer_generate(inf5, pr5.ctypes.data_as(C.POINTER(C.c_int)), p5, 2, first5, 1, st,
                                               None), "config 5 prefill")
            out5 = (C.c_int * s5)()
            torch.cuda.synchronize()
            tq = time.perf_counter()
            rina.check(eng.rina_infer_decode(inf5, s5, out5, 1, st, None), "config 5 decode")
            torch.cuda.synchronize()
            w5 = time.perf_counter() - tq
            eng.rina_infer_destroy(inf5)
            b5 = jm.bytes_per_token(p5 + 1 + s5 // 2)
            cache = ("q2 K / q1 V RINA-MLA cache (q2_1 key content, fp32 RoPE part, q1_0 values; queries and the "
                     "current position fp32)" if kvm == "q2k_q1v" else "fp32 RINA-MLA cache")
            cfg5[key] = {
                "workload": "RINA Gen6 Jamba hybrid at random init: 640d, 16 layers (12 InertiaWave SSM + 4 RINA-MLA), "
                            "10/5 heads, d_c 160, LayerNorm + SwiGLU 1536, vocab 128256, Q4_0 linears, fp32 tied LM "
                            "head, %s, context 2048, %d-token seeded prompt (prefill untimed), %d greedy steps at "
                            "positions %d..%d" % (cache, p5, s5, p5 + 1, p5 + s5),
                "rina_mla_kv_mode": kvm,
                "tokens_per_s": round(s5 / w5, 2), "ms_per_step": round(w5 * 1e3 / s5, 4), "steps": s5,
                "bytes_per_token": b5, "hbm_gbps": round(b5 * s5 / w5 / 1e9, 1),
                "hbm_frac": round(b5 * s5 / w5 / HBM_PEAK, 4), "tokens_head": list(first5) + list(out5)[:7]}
            log("config 5 (%s cache): %.3f ms/step, %.1f tok/s" % (kvm, w5 * 1e3 / s5, s5 / w5))
            jm.close()
            del jm
            torch.cuda.empty_cache()

    # ---- config 3: the same model at context 4096, KV cache q8 / q4 / q2k_q1v.
    # A 4090-token seeded prompt is prefilled (untimed; the second generated
    # token captures the decode graph), then greedy steps at positions
    # 4092.. are timed.
    cfg3 = None
    if not args.no_config3:
        n3, s3, ms3 = 4090, args.config3_steps, 4104
        t3 = time.time()
        sm3 = synth.SynthLlama(cfg, qt=rina.QT_Q4_0F, seed=1, max_seq=ms3)
        log("config 3 model built in %.1fs" % (time.time() - t3))
        pr3 = np.random.default_rng(3).integers(0, cfg["vocab_size"], n3).astype(np.int32)
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        rec = {"q8": (34, 34), "q4": (18, 18), "q2k_q1v": (10, 6)}     # K / V bytes per 32 values
        modes = {}
        for mode in ("q8", "q4", "q2k_q1v"):
            inf3 = sm3.infer(mode, ms3)
            f3 = (C.c_int * 2)()
            rina.check(eng.rina_infer_generate(inf3, pr3.ctypes.data_as(C.POINTER(C.c_int)), n3, 2, f3, 1, st, None),
                       "config 3 prefill")
            o3 = (C.c_int * s3)()
            torch.cuda.synchronize()
            tq = time.perf_counter()
            rina.check(eng.rina_infer_decode(inf3, s3, o3, 1, st, None), "config 3 decode")
            torch.cuda.synchronize()
            w3 = time.perf_counter() - tq
            eng.rina_infer_destroy(inf3)
            kv_tok = cfg["n_layers"] * (n3 + 2 + s3 // 2) * (kvd // 32) * sum(rec[mode])
            modes[mode] = {"tokens_per_s": round(s3 / w3, 2), "ms_per_step": round(w3 * 1e3 / s3, 4),
                           "kv_bytes_per_token": kv_tok, "tokens_head": list(f3) + list(o3)[:4]}
            log("config 3 %s: %.3f ms/step, %.1f tok/s" % (mode, w3 * 1e3 / s3, s3 / w3))
        sm3.close()
        del sm3
        torch.cuda.empty_cache()
        cfg3 = {"workload": "Llama-3.2-1B-shaped decode at context 4096 (4090-token seeded prompt, steps at positions "
                            "%d..%d), Q4_0F linears, fp32 tied LM head, KV cache q8 / q4 / q2k_q1v" % (n3 + 2, n3 + 1 + s3),
                "steps": s3, "modes": modes}

    # ---- CPU baseline: the oracle (scalar C restatement of the reference's
    # loops) decoding the same model at the GPU's positions: it takes the
    # GPU's prompt K/V rows and first token, then decodes greedily; timed on
    # the job's CPU share (all of it) and on one core.
    cpu = None
    if want_cpu:
        sys.path.insert(0, ROOT)
        import oracle
        try:
            share = len(os.sched_getaffinity(0))
        except AttributeError:
            share = os.cpu_count() or 1
        cores = max(1, min(share, 16))   # this pool gives one GPU job a 16-core CPU share
        L = oracle.load()
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        ms_cpu = args.prompt + 16

        def cpu_model_at_prompt(nthreads):
            m, hold = oracle.gqa_from_tensors(cfg, sm.host, sm.qt, ms_cpu, "fp32", nthreads)
            for layer in range(cfg["n_layers"]):
                for which in (0, 1):
                    onb = C.c_size_t()
                    optr = L.orc_gqa_cache(m, layer, which, C.byref(onb))
                    src = cache_rows[2 * layer + which]
                    C.memmove(optr, src.ctypes.data, src.nbytes)
            return m, hold

        def decode(m, steps):
            lg = np.zeros(V, np.float32)
            tok = np.array([tokens[0]], np.int32)
            ids = []
            tc = time.perf_counter()
            for k in range(steps):
                L.orc_gqa_forward(m, tok.ctypes.data, 1, args.prompt + k, lg.ctypes.data, 1)
                tok[0] = L.orc_argmax(lg.ctypes.data, V)
                ids.append(int(tok[0]))
            return time.perf_counter() - tc, ids

        m, hold = cpu_model_at_prompt(cores)
        dt, ids_cpu = decode(m, args.cpu_steps)
        L.orc_gqa_destroy(m)
        m1, hold1 = cpu_model_at_prompt(1)
        dt1, _ = decode(m1, 1)
        L.orc_gqa_destroy(m1)
        cpu = {"value": round(args.cpu_steps / dt, 4), "unit": "tokens/s", "cores": cores, "kind": "port",
               "value_1core": round(1.0 / dt1, 4), "cpu_model": cpu_model(), "host_cores_visible": os.cpu_count(),
               "matches_gpu_tokens": ids_cpu == tokens[1:1 + args.cpu_steps],
               "sample": "%d greedy decode steps (and 1 step on one core) of the same config-2 model at the GPU's "
                         "positions %d..%d, the oracle starting from the GPU's %d prompt K/V rows and first token "
                         "(1.66 GB of weights and ~34 MB of fp32 KV per token)"
                         % (args.cpu_steps, args.prompt, args.prompt + args.cpu_steps - 1, args.prompt)}
        log("cpu oracle: %.3f tok/s on %d threads, %.3f tok/s on 1 (%s)" %
            (cpu["value"], cores, cpu["value_1core"], cpu["cpu_model"]))

    per_token = sm.weight_bytes_per_token() + cfg["n_layers"] * 2 * (args.prompt + args.warmup + args.steps // 2) * \
        cfg["n_kv_heads"] * cfg["head_dim"] * 4
    res = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Llama-3.2-1B-shaped decode: %d layers, d 2048, 32/8 heads, dh 64, ffn 8192, "
                               "vocab 128256, Q4_0F linears, fp32 tied LM head, fp32 KV, %d-token seeded prompt, "
                               "greedy" % (cfg["n_layers"], args.prompt),
                   "prompt": args.prompt, "kv": "fp32", "weights": "Q4_0F"},
        "roofline": stack_roof,
        "roofline_other": {
            "lm_head_fp32": dict(lm_roof, kernel="gemv_f32_kernel (tied LM head 128256x2048 fp32)",
                                 bytes_per_launch=lm_bytes, avg_us=round(t_lm * 1e6, 2), traffic_detail=traffic_detail),
            "q4_0f_swiglu_w1w3": dict(sw_roof, bytes_per_launch=sw_bytes, avg_us=round(t_sw * 1e6, 2)),
            "config1_q4_0_gemv_8192x2048": dict(q4_roof, bytes_per_launch=q4_bytes, avg_us=round(t_q4 * 1e6, 3)),
            "prefill_q4_0f_swiglu_m%d" % Mp: dict(swp_roof, flop_per_launch=swp_flop, avg_us=round(t_swp * 1e6, 2),
                                                  kernel="gemm_bf3_kernel (v_mfma_f32_16x16x32_bf16, "
                                                         "three per fp32 product)"),
            **attn_roofs,
        },
        "decode_hbm_gbps": round(per_token * tok_s / 1e9, 1),
        "decode_hbm_frac": round(per_token * tok_s / HBM_PEAK, 4),
        "prefill_config2": prefill,
        "config3_ctx4096_quant_kv": cfg3,
        "config4_deepseek_mla_moe": cfg4,
        "config5_rina_jamba": cfg5.get("config5_rina_jamba"),
        "config5_rina_jamba_fp32_cache": cfg5.get("config5_rina_jamba_fp32_cache"),
        "cpu_baseline": cpu,
        "tokens_head": tokens[:8],
    }
    sm.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
