"""GPU parity of every C-ABI kernel entry point against the CPU oracle.

Bit-exact: weight packing, weight/KV dequant, KV quantize-on-append.
1e-5 relative (REL_TOL, fp32 accumulate): matvec, attention, glue.
"""
import ctypes as C

import numpy as np
import pytest

import _numpy_ref as nr
from _util import (REL_TOL, assert_close, assert_close_attn, assert_close_elem, attention_f64, dev, empty, host, ok, rng,
                   stream)

pytestmark = pytest.mark.gpu

Q4_SHAPES = [(4, 160, 640), (2, 2048, 2048), (1, 640, 640), (8, 64, 4096),      # test_linear_q4.cu:106-124
             (1, 8192, 2048), (1, 2048, 8192), (1, 512, 2048), (1, 100, 96), (1, 33, 160), (3, 77, 320),
             (1, 2048, 16384),
             # direct-load matvec: 2 waves per row with several row groups per
             # workgroup, and a ragged 4-row-group shape that loops
             (1, 12289, 4096), (1, 70001, 2048)]


def q2k_blocks(seed, n):
    nb = (n + 255) // 256
    r = rng(seed)
    blk = r.integers(0, 256, (nb, 84), dtype=np.uint8)
    blk[:, 80:82] = np.frombuffer(np.float16(0.0025).tobytes() * nb, np.uint8).reshape(nb, 2)
    blk[:, 82:84] = np.frombuffer(np.float16(0.00125).tobytes() * nb, np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def gpu_pack(rina, qt, x):
    xd = dev(x)
    out = empty((x.size // 32) * (18 if qt == 5 else 20), "uint8")
    ok(rina.load_hip().rina_hip_pack_weights(qt, xd.data_ptr(), x.size, out.data_ptr(), stream()), "pack")
    return out


@pytest.mark.parametrize("qt", [5, 7])
def test_pack_weights_bitexact(rina, orc, qt):
    r = rng(qt)
    x = (r.standard_normal(32 * 20000) * 0.02).astype(np.float32)
    x[:32] = 0
    x[32:64] = np.float32(7.0)
    x[64:96] = 0
    x[64] = 7.0
    x[65] = np.float32(0.49999997)
    x[96:128] = r.uniform(-1e-12, 1e-12, 32)
    x[128:160] = np.float32(1e5) * r.standard_normal(32)
    assert np.array_equal(host(gpu_pack(rina, qt, x)), orc.pack(qt, x))


@pytest.mark.parametrize("n", [32 * 4001, 32 * 57 + 13, 5])
def test_pack_weights_hf_bitexact(rina, orc, n):
    """HF-loader quantizer: roundf, truncating fp16 (flush and saturate
    classes), ragged last block, the 0.49999997f rounding edge."""
    r = rng(n)
    x = (r.standard_normal(n) * 0.05).astype(np.float32)
    if n > 32 * 8:
        x[:32] = 0.0                                             # scale clamp 1e-10 -> exponent <= 0
        x[32:64] = r.uniform(-1e-4, 1e-4, 32)                    # tiny scale: flushed fp16
        x[64:96] = r.uniform(-1e6, 1e6, 32)                      # scale > 65504: 0x7FFF class
        x[96:128] = np.float32(7.0) * np.arange(32, dtype=np.float32) / 31
        x[100] = np.float32(0.49999997) * (x[96:128].max() / 7)  # near-.5 tie
    out = empty((n + 31) // 32 * 18, "uint8")
    ok(rina.load_hip().rina_hip_pack_weights_hf(dev(x).data_ptr(), n, out.data_ptr(), stream()), "pack hf")
    assert np.array_equal(host(out), orc.pack(5, x, hf=True))


@pytest.mark.parametrize("qt", [5, 7, 10, 6])
def test_dequant_weights_bitexact(rina, orc, qt):
    n = 256 * 300
    if qt == 10:
        w = q2k_blocks(1, n)
    elif qt == 6:
        w = rng(2).standard_normal(n).astype(np.float32)
    else:
        w = orc.pack(qt, (rng(3).standard_normal(n) * 0.02).astype(np.float32))
    out = empty(n)
    ok(rina.load_hip().rina_hip_dequant_weights(qt, dev(w).data_ptr(), n, out.data_ptr(), stream()))
    assert np.array_equal(host(out).view(np.uint32), orc.dequant(qt, w, n).view(np.uint32))


def run_linear(rina, w, qt, x, N, K):
    M = x.size // K
    y = empty(M * N)
    ok(rina.load_hip().rina_hip_linear(dev(w).data_ptr(), qt, dev(x).data_ptr(), y.data_ptr(), M, N, K, stream()),
       "linear")
    return host(y).reshape(M, N)


@pytest.mark.parametrize("qt", [5, 7])
@pytest.mark.parametrize("M,N,K", Q4_SHAPES)
def test_linear_q4(rina, orc, qt, M, N, K):
    r = rng(M + N + K + qt)
    w = orc.pack(qt, (r.standard_normal(N * K) * 0.02).astype(np.float32))
    x = r.standard_normal((M, K)).astype(np.float32)
    assert_close(run_linear(rina, w, qt, x, N, K), orc.linear(w, qt, x, N, K), what="q%d %s" % (qt, (M, N, K)))


@pytest.mark.parametrize("M,N,K", [(1, 64, 2048), (1, 576, 2048), (1, 2048, 1408), (1, 1408, 2048),
                                   (1, 96, 10944), (1, 4096, 512), (3, 64, 1408), (1, 77, 1408),
                                   (1, 300, 2816), (1, 200, 4096), (1, 96, 8192), (1, 50, 160), (1, 33, 96),
                                   (1, 40, 48), (1, 102400 // 8, 2048)])
def test_linear_q2k(rina, orc, M, N, K):
    w = q2k_blocks(N + K, N * K)
    x = rng(K).standard_normal((M, K)).astype(np.float32)
    assert_close(run_linear(rina, w, 10, x, N, K), orc.linear(w, 10, x, N, K), what="q2k %s" % ((M, N, K),))


@pytest.mark.parametrize("M,N,K", [(1, 32000, 2048), (1, 1000, 640), (2, 300, 2050), (1, 64, 2048)])
def test_linear_fp32(rina, orc, M, N, K):
    r = rng(N)
    w = (r.standard_normal(N * K) * 0.02).astype(np.float32)
    x = r.standard_normal((M, K)).astype(np.float32)
    assert_close(run_linear(rina, w, 6, x, N, K), orc.linear(w, 6, x, N, K), what="fp32 %s" % ((M, N, K),))


@pytest.mark.parametrize("K", [128, 384, 640, 896])
def test_linear_fp32_half_rows(rina, orc, K):
    # K/4 an odd multiple of 32: one row per half wave; three segments of
    # row counts that are not multiples of the rows per wave, add and SwiGLU
    hip = rina.load_hip()
    r = rng(K + 5)
    Ns = (1001, 37, 130)
    ws = [(r.standard_normal(n * K) * 0.05).astype(np.float32) for n in Ns]
    x = r.standard_normal(K).astype(np.float32)
    xd = dev(x)
    wd = [dev(w) for w in ws]
    outs = [empty(n) for n in Ns]
    segs = (rina.LinearSeg * 3)(*[rina.LinearSeg(wd[i].data_ptr(), None, outs[i].data_ptr(), Ns[i]) for i in range(3)])
    ok(hip.rina_hip_linear_fused(segs, 3, 6, xd.data_ptr(), 1, K, rina.EPI_STORE, 0, None, 0.0, stream()), "store")
    for i in range(3):
        assert_close(host(outs[i]), orc.linear(ws[i], 6, x, Ns[i], K)[0], what="K %d seg %d" % (K, i))
    base = r.standard_normal(Ns[0]).astype(np.float32)
    yd = dev(base)
    seg = rina.LinearSeg(wd[0].data_ptr(), None, yd.data_ptr(), Ns[0])
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, 6, xd.data_ptr(), 1, K, rina.EPI_ADD, 0, None, 0.0, stream()), "add")
    assert_close(host(yd), base + orc.linear(ws[0], 6, x, Ns[0], K)[0], what="K %d add" % K)
    w3 = (r.standard_normal(Ns[0] * K) * 0.05).astype(np.float32)
    gd = empty(Ns[0])
    seg = rina.LinearSeg(wd[0].data_ptr(), dev(w3).data_ptr(), gd.data_ptr(), Ns[0])
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, 6, xd.data_ptr(), 1, K, rina.EPI_SWIGLU, 0, None, 0.0, stream()),
       "swiglu")
    g = orc.linear(ws[0], 6, x, Ns[0], K)[0]
    u = orc.linear(w3, 6, x, Ns[0], K)[0]
    ref = np.zeros(Ns[0], np.float32)
    orc.load().orc_silu_mul(ref.ctypes.data, g.ctypes.data, u.ctypes.data, Ns[0])
    assert_close(host(gd), ref, what="K %d swiglu" % K)


@pytest.mark.parametrize("qt", [7, 6])
def test_linear_in_place(rina, orc, qt):
    # input == output: defined as out of place (the reference's in-place w_o call races)
    N = K = 2048
    r = rng(77)
    wf = (r.standard_normal(N * K) * 0.02).astype(np.float32)
    w = wf if qt == 6 else orc.pack(qt, wf)
    x = r.standard_normal(K).astype(np.float32)
    xd = dev(x)
    ok(rina.load_hip().rina_hip_linear(dev(w).data_ptr(), qt, xd.data_ptr(), xd.data_ptr(), 1, N, K, stream()))
    assert_close(host(xd), orc.linear(w, qt, x, N, K)[0], what="in-place")


@pytest.mark.parametrize("qt", [7, 5, 10, 6])
def test_linear_fused_epilogues(rina, orc, qt):
    hip = rina.load_hip()
    r = rng(qt + 100)
    K, Ns = 2048, (2048, 512, 512)

    def mk(n):
        if qt == 10:
            return q2k_blocks(int(r.integers(1 << 30)), n * K)
        wf = (r.standard_normal(n * K) * 0.02).astype(np.float32)
        return wf if qt == 6 else orc.pack(qt, wf)

    ws = [mk(n) for n in Ns]
    x = r.standard_normal(K).astype(np.float32)
    xd = dev(x)
    wd = [dev(w) for w in ws]
    outs = [empty(n) for n in Ns]
    segs = (rina.LinearSeg * 3)(*[rina.LinearSeg(wd[i].data_ptr(), None, outs[i].data_ptr(), Ns[i]) for i in range(3)])
    ok(hip.rina_hip_linear_fused(segs, 3, qt, xd.data_ptr(), 1, K, rina.EPI_STORE, 0, None, 0.0, stream()),
       "fused store")
    for i in range(3):
        assert_close(host(outs[i]), orc.linear(ws[i], qt, x, Ns[i], K)[0], what="seg %d" % i)
    # residual add
    base = r.standard_normal(2048).astype(np.float32)
    yd = dev(base)
    seg = rina.LinearSeg(wd[0].data_ptr(), None, yd.data_ptr(), 2048)
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, qt, xd.data_ptr(), 1, K, rina.EPI_ADD, 0, None, 0.0, stream()),
       "fused add")
    assert_close(host(yd), base + orc.linear(ws[0], qt, x, 2048, K)[0], what="add")
    # SiLU(W1 x) * (W3 x)
    w3 = mk(2048)
    gd = empty(2048)
    seg = rina.LinearSeg(wd[0].data_ptr(), dev(w3).data_ptr(), gd.data_ptr(), 2048)
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, qt, xd.data_ptr(), 1, K, rina.EPI_SWIGLU, 0, None, 0.0,
                                 stream()), "swiglu")
    g = orc.linear(ws[0], qt, x, 2048, K)[0]
    u = orc.linear(w3, qt, x, 2048, K)[0]
    ref = np.zeros(2048, np.float32)
    orc.load().orc_silu_mul(ref.ctypes.data, g.ctypes.data, u.ctypes.data, 2048)
    assert_close(host(gd), ref, what="swiglu")


@pytest.mark.parametrize("qt,K", [(5, 640), (7, 2048), (10, 2048), (10, 1408), (6, 640), (5, 10240)])
@pytest.mark.parametrize("pro", [0, 1, 2])
def test_linear_fused_six_segments_and_norm_out(rina, orc, qt, K, pro):
    """Up to 6 segments on one input (one launch on the direct path, 3 per
    launch elsewhere) and the normalized row stored by the prologue."""
    hip = rina.load_hip()
    L = orc.load()
    r = rng(qt * 1000 + K + pro)
    Ns = (200, 37, 64, 150, 10, 96)

    def mk(n):
        if qt == 10:
            return q2k_blocks(int(r.integers(1 << 30)), n * K)
        wf = (r.standard_normal(n * K) * 0.02).astype(np.float32)
        return wf if qt == 6 else orc.pack(qt, wf)

    ws = [mk(n) for n in Ns]
    x = (r.standard_normal(K) * 2 + 0.3).astype(np.float32)
    nw = r.uniform(0.5, 1.5, K).astype(np.float32)
    wd = [dev(w) for w in ws]
    outs = [empty(n) for n in Ns]
    xn = empty(K)
    segs = (rina.LinearSeg * 6)(*[rina.LinearSeg(wd[i].data_ptr(), None, outs[i].data_ptr(), Ns[i]) for i in range(6)])
    ok(hip.rina_hip_linear_fused_ex(segs, 6, qt, dev(x).data_ptr(), 1, K, rina.EPI_STORE, pro,
                                    dev(nw).data_ptr() if pro else None, np.float32(1e-5),
                                    xn.data_ptr() if pro else None, stream()), "six segments")
    xr = x.copy()
    if pro:
        (L.orc_rms_norm if pro == 1 else L.orc_layer_norm)(xr.ctypes.data, nw.ctypes.data, 1, K, np.float32(1e-5))
        assert_close(host(xn), xr, what="normalized row")
    for i in range(6):
        assert_close(host(outs[i]), orc.linear(ws[i], qt, xr, Ns[i], K)[0], what="segment %d" % i)


def test_linear_fused_ex_rejects(rina):
    hip = rina.load_hip()
    buf = empty(1 << 16)
    seg = (rina.LinearSeg * 7)(*[rina.LinearSeg(buf.data_ptr(), None, buf.data_ptr(), 4) for _ in range(7)])
    p = buf.data_ptr()
    assert hip.rina_hip_linear_fused_ex(seg, 7, 5, p, 1, 64, 0, 0, None, 0.0, None, stream()) == -1   # > 6 segments
    assert hip.rina_hip_linear_fused_ex(seg, 1, 5, p, 1, 64, 0, 0, None, 0.0, p, stream()) == -1      # norm_out w/o prologue
    assert hip.rina_hip_linear_fused_ex(seg, 1, 5, p, 2, 64, 0, 1, p, 0.0, p, stream()) == -1         # norm_out with M > 1


@pytest.mark.parametrize("fmt", [1, 2, 3, 4])
def test_kv_quantize_bitexact(rina, orc, fmt):
    hip = rina.load_hip()
    r = rng(fmt)
    x = r.standard_normal(32 * 5000).astype(np.float32)
    x[:32] = 0
    x[32:64] = r.uniform(-1e-11, 1e-11, 32)
    x[64:96] = np.arange(32, dtype=np.float32) - 15.5
    x[96:128] = np.float32(3e5) * r.standard_normal(32)
    out = empty(x.size // 32 * nr.KV_BB[fmt], "uint8")
    ok(hip.rina_hip_kv_quantize(fmt, dev(x).data_ptr(), out.data_ptr(), x.size, stream()))
    got = host(out)
    assert np.array_equal(got, orc.kv_quantize(fmt, x))
    d = empty(x.size)
    ok(hip.rina_hip_kv_dequant(fmt, out.data_ptr(), d.data_ptr(), x.size, stream()))
    ref = orc.kv_dequant(fmt, got, x.size)
    dh = host(d)
    fin = np.isfinite(ref)
    assert np.array_equal(dh[fin], ref[fin]) and np.array_equal(np.isfinite(dh), fin)


def rope_tables(dh, n):
    ang = np.outer(np.arange(n, dtype=np.float32),
                   (1.0 / (500000.0 ** (np.arange(0, dh, 2, dtype=np.float32) / dh))).astype(np.float32))
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("pre_rope", [0, 1])
def test_rope_append(rina, orc, mode, pre_rope):
    hip = rina.load_hip()
    H, Hkv, dh, T, P, max_seq = 8, 4, 64, 3, 10, 32
    kvd = Hkv * dh
    r = rng(mode * 2 + pre_rope)
    q = r.standard_normal((T, H * dh)).astype(np.float32)
    k = r.standard_normal((T, kvd)).astype(np.float32)
    v = r.standard_normal((T, kvd)).astype(np.float32)
    cos, sin = rope_tables(dh, max_seq)
    nbytes = hip.rina_hip_kv_region_bytes(mode, 0, max_seq, kvd)
    vbytes = hip.rina_hip_kv_region_bytes(mode, 1, max_seq, kvd)
    ck, cv = empty(nbytes, "uint8"), empty(vbytes, "uint8")
    qd, kd, vd = dev(q), dev(k), dev(v)
    cd, sd = dev(cos), dev(sin)
    ok(hip.rina_hip_rope_append(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cd.data_ptr(), sd.data_ptr(),
                                cd.data_ptr(), sd.data_ptr(), ck.data_ptr(), cv.data_ptr(), mode, pre_rope, T, H, Hkv,
                                dh, P, None, max_seq, stream()), "rope_append")
    qr = nr.rope_neox(q.reshape(T, H, dh), cos, sin, P).reshape(T, -1)
    kr = nr.rope_neox(k.reshape(T, Hkv, dh), cos, sin, P).reshape(T, -1)
    assert np.max(np.abs(host(qd) - qr)) <= 1e-5 and np.max(np.abs(host(kd) - kr)) <= 1e-5
    kc_src = k if pre_rope else host(kd)        # what went into the cache, in fp32
    if mode == 0:
        got_k = host(ck).view(np.float32).reshape(max_seq, kvd)[P:P + T]
        got_v = host(cv).view(np.float32).reshape(max_seq, kvd)[P:P + T]
        assert np.array_equal(got_k, kc_src) and np.array_equal(got_v, v)
    else:
        kf, vf = orc.kv_mode_formats(mode)
        kb, vb = nr.KV_BB[kf], nr.KV_BB[vf]
        nbp = kvd // 32
        got_k = host(ck)[P * nbp * kb:(P + T) * nbp * kb]
        got_v = host(cv)[P * nbp * vb:(P + T) * nbp * vb]
        assert np.array_equal(got_k, orc.kv_quantize(kf, kc_src))
        assert np.array_equal(got_v, orc.kv_quantize(vf, v))
        assert not host(ck)[: P * nbp * kb].any()        # nothing written outside the rows


def attention_case(rina, orc, mode, P, T, H=32, Hkv=8, dh=64, pre_rope=0, use_dpos=False, seed=0):
    hip = rina.load_hip()
    L = orc.load()
    kvd = Hkv * dh
    max_seq = max(P + T, 8)
    r = rng(seed * 1000 + mode * 31 + P + T)
    kc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    vc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    q = r.standard_normal((T, H * dh)).astype(np.float32)
    kcur = r.standard_normal((T, kvd)).astype(np.float32)
    vcur = r.standard_normal((T, kvd)).astype(np.float32)
    cos, sin = rope_tables(dh, max_seq)
    if mode == 0:
        ckb, cvb = kc.view(np.uint8).reshape(-1), vc.view(np.uint8).reshape(-1)
    else:
        kf, vf = orc.kv_mode_formats(mode)
        ckb, cvb = orc.kv_quantize(kf, kc), orc.kv_quantize(vf, vc)
    out = np.zeros((T, H * dh), np.float32)
    if mode == 0:
        L.orc_gqa_attention(q.ctypes.data, kcur.ctypes.data, vcur.ctypes.data, kc.ctypes.data, vc.ctypes.data, None,
                            None, 0, pre_rope, cos.ctypes.data, sin.ctypes.data, T, P, H, Hkv, dh, out.ctypes.data)
    else:
        L.orc_gqa_attention(q.ctypes.data, kcur.ctypes.data, vcur.ctypes.data, None, None, ckb.ctypes.data,
                            cvb.ctypes.data, mode, pre_rope, cos.ctypes.data, sin.ctypes.data, T, P, H, Hkv, dh,
                            out.ctypes.data)
    ws_bytes = hip.rina_hip_gqa_attention_workspace(T, H, dh, max_seq)
    ws = empty(ws_bytes, "uint8")
    od = empty(T * H * dh)
    cd, sd = dev(cos), dev(sin)
    pos = dev(np.array([P], np.int32)) if use_dpos else None
    ok(hip.rina_hip_gqa_attention(dev(q).data_ptr(), dev(kcur).data_ptr(), dev(vcur).data_ptr(), dev(ckb).data_ptr(),
                                  dev(cvb).data_ptr(), mode, pre_rope, cd.data_ptr(), sd.data_ptr(), T, H, Hkv, dh,
                                  0 if use_dpos else P, pos.data_ptr() if use_dpos else None, max_seq, od.data_ptr(),
                                  ws.data_ptr(), ws_bytes, stream()), "attention")
    return host(od).reshape(T, -1), out


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("P", [0, 1, 31, 32, 33, 100, 543, 1000])
def test_attention_decode(rina, orc, mode, P):
    got, ref = attention_case(rina, orc, mode, P, 1)
    assert_close_elem(got, ref, what="decode mode %d pos %d" % (mode, P))


@pytest.mark.parametrize("mode", [0, 1, 5])
def test_attention_decode_device_pos(rina, orc, mode):
    got, ref = attention_case(rina, orc, mode, 70, 1, use_dpos=True)
    assert_close_elem(got, ref, what="d_pos mode %d" % mode)


@pytest.mark.parametrize("mode,P,T", [(0, 0, 7), (0, 5, 4), (2, 9, 3), (5, 0, 33), (1, 40, 2)])
def test_attention_multi_row(rina, orc, mode, P, T):
    got, ref = attention_case(rina, orc, mode, P, T)
    assert_close_elem(got, ref, what="rows mode %d P %d T %d" % (mode, P, T))


@pytest.mark.parametrize("T,H,Hkv", [(100, 32, 8), (300, 32, 8), (512, 32, 8), (17, 8, 2), (250, 16, 2),
                                     (129, 10, 5), (64, 8, 8)])
def test_attention_prompt_from_zero(rina, orc, T, H, Hkv):
    """Prompt rows from position 0: several 64-position blocks, ragged row
    groups, causal against the oracle.  H / Hkv a multiple of 4 takes the
    matrix-core kernel (config 2's 512 x 32 / 8 among them), the others the
    one-wave block kernel."""
    got, ref = attention_case(rina, orc, 0, 0, T, H=H, Hkv=Hkv)
    assert_close_elem(got, ref, what="prompt T %d H %d/%d" % (T, H, Hkv))


@pytest.mark.parametrize("H,Hkv,dh", [(10, 5, 64), (16, 16, 128), (4, 2, 32)])
def test_attention_other_shapes(rina, orc, H, Hkv, dh):
    got, ref = attention_case(rina, orc, 0, 20, 1, H=H, Hkv=Hkv, dh=dh)
    assert_close_elem(got, ref, what="shape %s" % ((H, Hkv, dh),))


def edge_row(r, n, t):
    """n values (n % 32 == 0) made of 32-value blocks on the quantizers'
    edges, in an order and power-of-two scale that depend on t: all zeros;
    -0 with values under the 1e-10 scale clamp; exact roundf ties on the q8
    grid (amax 127, scale 1), the q4 grid (amax 7) and the q2_1 grid (amax 2,
    v / amax = +-0.5); one outlier over normals; plain normals."""
    blocks = [np.zeros(32),
              np.concatenate([[-0.0, 1e-12, -3e-11], np.full(29, -0.0)]),
              np.array([127.0] + [(j % 9 - 4) + 0.5 for j in range(31)]),
              np.array([7.0] + [(j % 7 - 3) + 0.5 for j in range(31)]),
              np.array([2.0] + [(-1.0) ** j for j in range(31)]),
              np.concatenate([[3e5], r.standard_normal(31)]),
              r.standard_normal(32)]
    out = [blocks[(t + 3 * b) % len(blocks)] * 2.0 ** ((t + b) % 5 - 2) for b in range(n // 32)]
    return np.concatenate(out).astype(np.float32)


def gpu_kv_quantize(hip, fmt, x):
    """rina_hip_kv_quantize: one thread packs each 32-value block."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = empty(x.size // 32 * nr.KV_BB[fmt], "uint8")
    ok(hip.rina_hip_kv_quantize(fmt, dev(x).data_ptr(), out.data_ptr(), x.size, stream()), "kv_quantize")
    return host(out)


@pytest.mark.parametrize("mode", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("pre_rope,Hkv,dh", [(1, 4, 64), (0, 4, 64), (1, 3, 32), (0, 3, 32)])
def test_rope_append_cache_bytes(rina, orc, mode, pre_rope, Hkv, dh):
    """The records rope_append writes (a half wave packs each block) are the
    bytes of rina_hip_kv_quantize (one thread per block) on the same rows,
    inf and NaN included, and the oracle's bytes on the finite rows; with
    3 x 32 dims a wave holds K blocks in one half and V blocks in the other."""
    hip = rina.load_hip()
    H, T, P, max_seq = 2 * Hkv, 4, 6, 16
    kvd = Hkv * dh
    r = rng(300 + 10 * mode + pre_rope + Hkv)
    k = np.stack([edge_row(r, kvd, t) for t in range(T)])
    v = np.stack([edge_row(r, kvd, t + 2) for t in range(T)])
    k[3, 5], k[3, 40], v[3, 70], v[3, kvd - 3] = np.inf, np.nan, -np.inf, np.nan
    q = r.standard_normal((T, H * dh)).astype(np.float32)
    cos, sin = rope_tables(dh, max_seq)
    ck = empty(hip.rina_hip_kv_region_bytes(mode, 0, max_seq, kvd), "uint8")
    cv = empty(hip.rina_hip_kv_region_bytes(mode, 1, max_seq, kvd), "uint8")
    kd = dev(k)
    cd, sd = dev(cos), dev(sin)
    ok(hip.rina_hip_rope_append(dev(q).data_ptr(), kd.data_ptr(), dev(v).data_ptr(), cd.data_ptr(), sd.data_ptr(),
                                cd.data_ptr(), sd.data_ptr(), ck.data_ptr(), cv.data_ptr(), mode, pre_rope, T, H, Hkv,
                                dh, P, None, max_seq, stream()), "rope_append")
    kf, vf = orc.kv_mode_formats(mode)
    ks = k if pre_rope else host(kd).reshape(T, kvd)      # the cache holds raw keys under pre_rope
    kb, vb = kvd // 32 * nr.KV_BB[kf], kvd // 32 * nr.KV_BB[vf]
    gk, gv = host(ck)[P * kb:(P + T) * kb], host(cv)[P * vb:(P + T) * vb]
    assert np.array_equal(gk, gpu_kv_quantize(hip, kf, ks))
    assert np.array_equal(gv, gpu_kv_quantize(hip, vf, v))
    assert np.array_equal(gk[:3 * kb], orc.kv_quantize(kf, ks[:3]))
    assert np.array_equal(gv[:3 * vb], orc.kv_quantize(vf, v[:3]))


@pytest.mark.parametrize("mode", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("P,H,Hkv", [(0, 32, 8), (45, 32, 8), (0, 10, 5), (300, 16, 16)])
def test_decode_attention_fused_edge_blocks(rina, orc, mode, P, H, Hkv):
    """The fused decode append packs the current K / V row with a half wave
    per block: on blocks at the quantizers' edges its records equal the
    oracle's bytes for the rotated key row the call returns and the value
    row, and no other cache row changes."""
    hip = rina.load_hip()
    dh = 64
    kvd = Hkv * dh
    max_seq = P + 3
    r = rng(500 + 10 * mode + P + H)
    kc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    vc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    q = r.standard_normal(H * dh).astype(np.float32)
    k, v = edge_row(r, kvd, P), edge_row(r, kvd, P + 1)
    cos, sin = rope_tables(dh, max_seq)
    kf, vf = orc.kv_mode_formats(mode)
    ckb, cvb = orc.kv_quantize(kf, kc), orc.kv_quantize(vf, vc)
    ws_bytes = hip.rina_hip_gqa_attention_workspace(1, H, dh, max_seq)
    ws = empty(ws_bytes, "uint8")
    ckd, cvd = dev(ckb), dev(cvb)
    od, krot = empty(H * dh), empty(kvd)
    cd, sd = dev(cos), dev(sin)
    ok(hip.rina_hip_gqa_decode_attention(dev(q).data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), cd.data_ptr(),
                                         sd.data_ptr(), cd.data_ptr(), sd.data_ptr(), ckd.data_ptr(), cvd.data_ptr(),
                                         mode, H, Hkv, dh, P, None, max_seq, od.data_ptr(), krot.data_ptr(),
                                         ws.data_ptr(), ws_bytes, stream()), "decode attention")
    kr = host(krot)
    if P == 0:        # cos 1, sin 0: the rotation leaves the edge blocks as they are
        assert np.array_equal(kr, k)
    want_k, want_v = kc.copy(), vc.copy()
    want_k[P], want_v[P] = kr, v
    assert np.array_equal(host(ckd), orc.kv_quantize(kf, want_k))
    assert np.array_equal(host(cvd), orc.kv_quantize(vf, want_v))


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("P,H,Hkv,use_dpos", [(0, 32, 8, False), (37, 32, 8, False), (543, 32, 8, True),
                                              (1500, 32, 8, False), (70, 10, 5, False), (16, 8, 8, True),
                                              (300, 32, 4, True), (1500, 32, 4, False),
                                              (1023, 32, 8, False), (1015, 32, 8, True), (1024, 32, 8, False),
                                              (255, 32, 8, False), (256, 32, 8, False), (600, 32, 8, True),
                                              (4095, 32, 8, True), (6000, 32, 8, False), (8200, 32, 4, True)])
def test_decode_attention_fused(rina, orc, mode, P, H, Hkv, use_dpos):
    """RoPE + K/V append + attention in one call == rope_append then attention
    (oracle): the rotated K row and the appended cache bytes bit-exact, the
    output within tolerance, and no other cache row touched.  fp32 caches of
    up to 1024 positions take the one-launch kernel in steps of 256 positions
    (1023, and 1015 with a 1024-row cache and a device position, fill its
    last step; 255 / 256 end and start a step), 1024 the split + combine
    pair.  On split + combine, chunks of up to 5 steps of 16 positions run
    scores first (4095: 5 steps), longer ones the running softmax after the
    5 entry steps (6000: 6 steps per chunk; 8200 with 4 KV heads: 9 steps,
    3 entry steps for fp32).

    Past 2048 positions the per-element check is against float64 attention
    over the same (dequantized) rows, with the floor set by the magnitude
    of the values each output averages (assert_close_attn): the fp32
    oracle itself misses 1e-6 max|out| by one element in most of these
    cases (its error is at most 6.9e-7 of that magnitude, while the flat
    softmax over 4k-8k random rows leaves max|out| near 0.08).  The oracle
    still bounds the output normwise."""
    hip = rina.load_hip()
    L = orc.load()
    dh = 64
    kvd = Hkv * dh
    max_seq = P + 9
    r = rng(mode * 7 + P + H)
    kc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    vc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    q = r.standard_normal(H * dh).astype(np.float32)
    k = r.standard_normal(kvd).astype(np.float32)
    v = r.standard_normal(kvd).astype(np.float32)
    cos, sin = rope_tables(dh, max_seq)
    qr, kr = q.copy(), k.copy()
    L.orc_rope_neox(qr.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, H, dh, P)
    L.orc_rope_neox(kr.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, Hkv, dh, P)
    if mode == 0:
        ckb, cvb = kc.view(np.uint8).reshape(-1).copy(), vc.view(np.uint8).reshape(-1).copy()
    else:
        kf, vf = orc.kv_mode_formats(mode)
        ckb, cvb = orc.kv_quantize(kf, kc), orc.kv_quantize(vf, vc)
    ref = np.zeros(H * dh, np.float32)
    if mode == 0:
        L.orc_gqa_attention(qr.ctypes.data, kr.ctypes.data, v.ctypes.data, kc.ctypes.data, vc.ctypes.data, None,
                            None, 0, 0, None, None, 1, P, H, Hkv, dh, ref.ctypes.data)
    else:
        L.orc_gqa_attention(qr.ctypes.data, kr.ctypes.data, v.ctypes.data, None, None, ckb.ctypes.data,
                            cvb.ctypes.data, mode, 0, None, None, 1, P, H, Hkv, dh, ref.ctypes.data)
    ws_bytes = hip.rina_hip_gqa_attention_workspace(1, H, dh, max_seq)
    ws = empty(ws_bytes, "uint8")
    ckd, cvd = dev(ckb), dev(cvb)
    od, krot = empty(H * dh), empty(kvd)
    cd, sd = dev(cos), dev(sin)
    pos = dev(np.array([P], np.int32)) if use_dpos else None
    ok(hip.rina_hip_gqa_decode_attention(dev(q).data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), cd.data_ptr(),
                                         sd.data_ptr(), cd.data_ptr(), sd.data_ptr(), ckd.data_ptr(), cvd.data_ptr(),
                                         mode, H, Hkv, dh, 0 if use_dpos else P,
                                         pos.data_ptr() if use_dpos else None, max_seq, od.data_ptr(),
                                         krot.data_ptr(), ws.data_ptr(), ws_bytes, stream()), "decode attention")
    assert np.array_equal(host(krot).view(np.uint32), kr.view(np.uint32))
    if P <= 2048:
        assert_close_elem(host(od), ref, what="fused decode mode %d P %d" % (mode, P))
    else:
        assert_close(host(od), ref, what="fused decode mode %d P %d" % (mode, P))
        if mode == 0:
            Kh, Vh = kc[:P], vc[:P]
        else:
            Kh = orc.kv_dequant(kf, ckb, max_seq * kvd).reshape(max_seq, kvd)[:P]
            Vh = orc.kv_dequant(vf, cvb, max_seq * kvd).reshape(max_seq, kvd)[:P]
        o64, mag = attention_f64(qr, np.vstack([Kh, kr[None]]), np.vstack([Vh, v[None]]), H, Hkv, dh)
        assert_close_attn(host(od), o64, mag, what="fused decode mode %d P %d vs float64" % (mode, P))
    gk, gv = host(ckd), host(cvd)
    if mode == 0:
        want_k = kc.copy(); want_k[P] = kr
        want_v = vc.copy(); want_v[P] = v
        assert np.array_equal(gk.view(np.float32).reshape(max_seq, kvd), want_k)
        assert np.array_equal(gv.view(np.float32).reshape(max_seq, kvd), want_v)
    else:
        want_k = kc.copy(); want_k[P] = kr
        want_v = vc.copy(); want_v[P] = v
        assert np.array_equal(gk, orc.kv_quantize(kf, want_k))
        assert np.array_equal(gv, orc.kv_quantize(vf, want_v))


@pytest.mark.parametrize("mode", [1, 2, 5])
@pytest.mark.parametrize("P,max_seq", [(100, 109), (1200, 1201), (4095, 4096)])
def test_decode_attention_cache_at_2_mod_4(rina, orc, mode, P, max_seq):
    """Packed caches whose base lies 2 bytes past a 4-byte boundary (the
    entry point asks for 2-byte alignment): the q8 slices are read as
    12-byte windows from the dword at or below them, whose offset then
    flips between the even and odd blocks of a record.  Output against the
    oracle (per element below 2048 positions, else against float64 with
    the averaged values' magnitude as floor), appended bytes bit-exact, the
    bytes around the cache untouched; P = max_seq - 1 writes the last row
    and reads every row before it."""
    hip = rina.load_hip()
    L = orc.load()
    H, Hkv, dh = 32, 8, 64
    kvd = Hkv * dh
    r = rng(77 + mode + P)
    kc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    vc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    q = r.standard_normal(H * dh).astype(np.float32)
    k = r.standard_normal(kvd).astype(np.float32)
    v = r.standard_normal(kvd).astype(np.float32)
    cos, sin = rope_tables(dh, max_seq)
    qr, kr = q.copy(), k.copy()
    L.orc_rope_neox(qr.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, H, dh, P)
    L.orc_rope_neox(kr.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, Hkv, dh, P)
    kf, vf = orc.kv_mode_formats(mode)
    ckb, cvb = orc.kv_quantize(kf, kc), orc.kv_quantize(vf, vc)
    ref = np.zeros(H * dh, np.float32)
    L.orc_gqa_attention(qr.ctypes.data, kr.ctypes.data, v.ctypes.data, None, None, ckb.ctypes.data,
                        cvb.ctypes.data, mode, 0, None, None, 1, P, H, Hkv, dh, ref.ctypes.data)
    guard = np.arange(16, dtype=np.uint8) + 200
    kbuf = dev(np.concatenate([guard[:2], ckb, guard]))     # cache at base + 2
    vbuf = dev(np.concatenate([guard[:2], cvb, guard]))
    assert kbuf.data_ptr() % 4 == 0
    ws_bytes = hip.rina_hip_gqa_attention_workspace(1, H, dh, max_seq)
    ws = empty(ws_bytes, "uint8")
    od = empty(H * dh)
    cd, sd = dev(cos), dev(sin)
    ok(hip.rina_hip_gqa_decode_attention(dev(q).data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), cd.data_ptr(),
                                         sd.data_ptr(), cd.data_ptr(), sd.data_ptr(), kbuf.data_ptr() + 2,
                                         vbuf.data_ptr() + 2, mode, H, Hkv, dh, P, None, max_seq, od.data_ptr(),
                                         None, ws.data_ptr(), ws_bytes, stream()), "decode attention")
    got = host(od)
    if P <= 2048:
        assert_close_elem(got, ref, what="cache at 2 mod 4, mode %d P %d" % (mode, P))
    else:
        assert_close(got, ref, what="cache at 2 mod 4, mode %d P %d" % (mode, P))
        Kh = orc.kv_dequant(kf, ckb, max_seq * kvd).reshape(max_seq, kvd)[:P]
        Vh = orc.kv_dequant(vf, cvb, max_seq * kvd).reshape(max_seq, kvd)[:P]
        o64, mag = attention_f64(qr, np.vstack([Kh, kr[None]]), np.vstack([Vh, v[None]]), H, Hkv, dh)
        assert_close_attn(got, o64, mag, what="cache at 2 mod 4, mode %d P %d vs float64" % (mode, P))
    gk, gv = host(kbuf), host(vbuf)
    want_k, want_v = kc.copy(), vc.copy()
    want_k[P], want_v[P] = kr, v
    assert np.array_equal(gk[2:2 + ckb.size], orc.kv_quantize(kf, want_k))
    assert np.array_equal(gv[2:2 + cvb.size], orc.kv_quantize(vf, want_v))
    assert np.array_equal(gk[:2], guard[:2]) and np.array_equal(gk[2 + ckb.size:], guard)
    assert np.array_equal(gv[:2], guard[:2]) and np.array_equal(gv[2 + cvb.size:], guard)


def test_decode_attention_sequence(rina, orc):
    """40 consecutive decode calls at a device position (the decode loop):
    every output against the oracle over the cache as it grows, so each call
    starts from the completion counters the previous call left."""
    hip = rina.load_hip()
    L = orc.load()
    H, Hkv, dh, max_seq, P0, n = 32, 8, 64, 600, 500, 40
    kvd = Hkv * dh
    r = rng(4242)
    kc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    vc = r.standard_normal((max_seq, kvd)).astype(np.float32)
    cos, sin = rope_tables(dh, max_seq)
    ws_bytes = hip.rina_hip_gqa_attention_workspace(1, H, dh, max_seq)
    ws = empty(ws_bytes, "uint8")
    ckd, cvd = dev(kc), dev(vc)
    cd, sd = dev(cos), dev(sin)
    od = empty(H * dh)
    pos = dev(np.array([P0], np.int32))
    for i in range(n):
        P = P0 + i
        q = r.standard_normal(H * dh).astype(np.float32)
        k = r.standard_normal(kvd).astype(np.float32)
        v = r.standard_normal(kvd).astype(np.float32)
        pos.copy_(dev(np.array([P], np.int32)))
        ok(hip.rina_hip_gqa_decode_attention(dev(q).data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), cd.data_ptr(),
                                             sd.data_ptr(), cd.data_ptr(), sd.data_ptr(), ckd.data_ptr(),
                                             cvd.data_ptr(), 0, H, Hkv, dh, 0, pos.data_ptr(), max_seq,
                                             od.data_ptr(), None, ws.data_ptr(), ws_bytes, stream()), "decode")
        qr, kr = q.copy(), k.copy()
        L.orc_rope_neox(qr.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, H, dh, P)
        L.orc_rope_neox(kr.ctypes.data, cos.ctypes.data, sin.ctypes.data, 1, Hkv, dh, P)
        ref = np.zeros(H * dh, np.float32)
        L.orc_gqa_attention(qr.ctypes.data, kr.ctypes.data, v.ctypes.data, kc.ctypes.data, vc.ctypes.data, None,
                            None, 0, 0, None, None, 1, P, H, Hkv, dh, ref.ctypes.data)
        assert_close_elem(host(od), ref, what="decode call %d (P %d)" % (i, P))
        kc[P], vc[P] = kr, v


@pytest.mark.parametrize("mode", [0, 2])
def test_attention_pre_rope(rina, orc, mode):
    got, ref = attention_case(rina, orc, mode, 12, 1, pre_rope=1)
    assert_close_elem(got, ref, what="pre_rope mode %d" % mode)


@pytest.mark.parametrize("d", [64, 102, 640, 2048, 3000, 8192, 10000])
def test_rms_norm_shapes(rina, orc, d):
    """rina_hip_rms_norm at row widths of each of its launch forms (16-byte
    loads held in registers for d % 4 == 0 up to 8192, one to eight float4 per
    thread; the scalar kernel for the others), out of place and in place."""
    hip = rina.load_hip()
    L = orc.load()
    r = rng(d)
    n = 5
    x = (r.standard_normal((n, d)) * np.float32(3.0)).astype(np.float32)
    w = r.uniform(0.5, 1.5, d).astype(np.float32)
    ref = x.copy()
    L.orc_rms_norm(ref.ctypes.data, w.ctypes.data, n, d, np.float32(1e-5))
    xd, od, wd = dev(x), empty(n * d), dev(w)
    ok(hip.rina_hip_rms_norm(xd.data_ptr(), od.data_ptr(), wd.data_ptr(), n, d, np.float32(1e-5), stream()))
    assert_close_elem(host(od).reshape(n, d), ref, what="rms_norm d %d" % d)
    ok(hip.rina_hip_rms_norm(xd.data_ptr(), xd.data_ptr(), wd.data_ptr(), n, d, np.float32(1e-5), stream()))
    assert_close_elem(host(xd).reshape(n, d), ref, what="rms_norm in place d %d" % d)


def test_glue(rina, orc):
    hip = rina.load_hip()
    L = orc.load()
    r = rng(5)
    n, d = 3, 2048
    x = r.standard_normal((n, d)).astype(np.float32)
    w = r.uniform(0.5, 1.5, d).astype(np.float32)
    for fn_h, fn_o in ((hip.rina_hip_rms_norm, L.orc_rms_norm), (hip.rina_hip_layer_norm, L.orc_layer_norm)):
        xd, od = dev(x), empty(n * d)
        ok(fn_h(xd.data_ptr(), od.data_ptr(), dev(w).data_ptr(), n, d, np.float32(1e-5), stream()))
        ref = x.copy()
        fn_o(ref.ctypes.data, w.ctypes.data, n, d, np.float32(1e-5))
        assert_close_elem(host(od).reshape(n, d), ref, what="norm")
    T, H, hd = 3, 4, 64
    cos, sin = rope_tables(hd, 64)
    xr = r.standard_normal((T, H, hd)).astype(np.float32)
    for hf, fn in ((0, L.orc_rope_neox), (1, L.orc_rope_hf)):
        xd = dev(xr)
        ok(hip.rina_hip_rope(xd.data_ptr(), dev(cos).data_ptr(), dev(sin).data_ptr(), T, H, hd, 9, None, hf, stream()))
        ref = xr.copy()
        fn(ref.ctypes.data, cos.ctypes.data, sin.ctypes.data, T, H, hd, 9)
        assert np.max(np.abs(host(xd) - ref)) <= 1e-6
    g = r.standard_normal(5000).astype(np.float32)
    u = r.standard_normal(5000).astype(np.float32)
    od = empty(5000)
    ok(hip.rina_hip_silu_mul(od.data_ptr(), dev(g).data_ptr(), dev(u).data_ptr(), 5000, stream()))
    ref = np.zeros(5000, np.float32)
    L.orc_silu_mul(ref.ctypes.data, g.ctypes.data, u.ctypes.data, 5000)
    assert_close_elem(host(od), ref, what="silu")
    ok(hip.rina_hip_add(od.data_ptr(), dev(g).data_ptr(), dev(u).data_ptr(), 5000, stream()))
    assert np.array_equal(host(od), g + u)
    dd = dev(g)
    ok(hip.rina_hip_saxpy(dd.data_ptr(), dev(u).data_ptr(), np.float32(0.5), 5000, stream()))
    assert_close_elem(host(dd), g + np.float32(0.5) * u, what="saxpy")


@pytest.mark.parametrize("qt", [6, 5, 7, 10])
def test_embedding(rina, orc, qt):
    hip = rina.load_hip()
    V, d = 300, 512
    if qt == 10:
        w = q2k_blocks(9, V * d)
    else:
        wf = (rng(qt).standard_normal(V * d) * 0.02).astype(np.float32)
        w = wf if qt == 6 else orc.pack(qt, wf)
    ids = np.array([0, 299, -4, 17, 150], np.int32)
    od = empty(5 * d)
    ok(hip.rina_hip_embedding(dev(w).data_ptr(), qt, dev(ids).data_ptr(), None, od.data_ptr(), 5, d, 0, stream()))
    ref = np.zeros((5, d), np.float32)
    orc.load().orc_embedding(w.ctypes.data, qt, ids.ctypes.data, ref.ctypes.data, 5, d)
    assert np.array_equal(host(od).reshape(5, d), ref)
    # with the vocabulary bound, ids past the table are clamped to its last row
    big = np.array([300, 7, 1 << 30, -1, 299], np.int32)
    ok(hip.rina_hip_embedding(dev(w).data_ptr(), qt, dev(big).data_ptr(), None, od.data_ptr(), 5, d, V, stream()))
    want = np.clip(big, 0, V - 1).astype(np.int32)
    orc.load().orc_embedding(w.ctypes.data, qt, want.ctypes.data, ref.ctypes.data, 5, d)
    assert np.array_equal(host(od).reshape(5, d), ref)


def test_argmax(rina, orc):
    hip = rina.load_hip()
    cases = [np.array([-1e11, 3.0, 5.0, 5.0, np.nan, 1.0], np.float32),
             np.full(7, -2e10, np.float32),
             rng(1).standard_normal(128256).astype(np.float32)]
    c3 = cases[2].copy()
    c3[[100, 90000, 128255]] = 50.0
    cases.append(c3)
    for a in cases:
        out = empty(1, "int32")
        ok(hip.rina_hip_argmax(dev(a).data_ptr(), a.size, out.data_ptr(), None, None, stream()))
        assert int(host(out)[0]) == orc.load().orc_argmax(a.ctypes.data, a.size)
    # ragged length (scalar tail) and an unaligned start (scalar path)
    c4 = rng(2).standard_normal(100003).astype(np.float32)
    c4[100002] = 9.0
    d4 = dev(np.concatenate([np.zeros(1, np.float32), c4]))
    for ptr, arr in ((d4.data_ptr() + 4, c4), (d4.data_ptr(), np.concatenate([np.zeros(1, np.float32), c4]))):
        out = empty(1, "int32")
        ok(hip.rina_hip_argmax(ptr, arr.size, out.data_ptr(), None, None, stream()))
        assert int(host(out)[0]) == orc.load().orc_argmax(arr.ctypes.data, arr.size)
    # device-loop form: ids[pos+1] = argmax, pos += 1
    ids = empty(16, "int32")
    pos = dev(np.array([4], np.int32))
    ok(hip.rina_hip_argmax(dev(c3).data_ptr(), c3.size, None, ids.data_ptr(), pos.data_ptr(), stream()))
    assert int(host(pos)[0]) == 5 and int(host(ids)[5]) == 100


def test_argmax_signed_zero_and_key_slots(rina, orc):
    """+0 and -0 are equal under the reference's strict ">" (main.cpp:139-146),
    so the lower index wins either way round; two caller key slots give each
    call its own answer."""
    hip = rina.load_hip()
    cases = [np.array([-0.0, 0.0, -1.0], np.float32), np.array([0.0, -0.0], np.float32),
             np.array([-3.0, -0.0, -1.0, 0.0], np.float32), np.full(2000, -0.0, np.float32)]
    slots = empty(4, "int32")   # two 8-byte slots, zero
    for i, a in enumerate(cases):
        want = orc.load().orc_argmax(a.ctypes.data, a.size)
        out = empty(1, "int32")
        ok(hip.rina_hip_argmax(dev(a).data_ptr(), a.size, out.data_ptr(), None, None, stream()))
        assert int(host(out)[0]) == want, (a[:4], want)
        ok(hip.rina_hip_argmax_ws(dev(a).data_ptr(), a.size, out.data_ptr(), None, None,
                                  slots.data_ptr() + 8 * (i % 2), stream()))
        assert int(host(out)[0]) == want
    assert not host(slots).any()   # each call leaves its slot zero
    bad = hip.rina_hip_argmax_ws(dev(cases[0]).data_ptr(), 3, empty(1, "int32").data_ptr(), None, None,
                                 slots.data_ptr() + 4, stream())
    assert bad == -1   # misaligned slot rejected before launch


@pytest.mark.parametrize("N,K,pro", [(128256, 2048, 1), (128256, 640, 2), (5000, 4096, 0), (333, 1000, 1)])
def test_linear_argmax_and_embed(rina, orc, N, K, pro):
    """The fused decode tail: rina_hip_linear_argmax writes the same logits
    as rina_hip_linear_fused (bit for bit: the same row arithmetic) plus
    per-workgroup argmax keys; rina_hip_argmax_embed picks the oracle's
    greedy id from them (strict ">", lowest index among ties, planted at
    three indices), writes it after the device position, advances the
    position and writes that id's embedding row (fp32 and Q4_0F tables,
    bit-exact against the oracle's row dequant).  The keys-slot form
    (rina_hip_argmax_partial + reset) leaves its slot zero."""
    hip = rina.load_hip()
    L = orc.load()
    r = rng(N + K + pro)
    w = (r.standard_normal(N * K) * 0.02).astype(np.float32)
    x = (r.standard_normal(K) * 2 + 0.3).astype(np.float32)
    nw = r.uniform(0.5, 1.5, K).astype(np.float32)
    wd, xd, nwd = dev(w), dev(x), dev(nw)
    y0, y1 = empty(N), empty(N)
    s0 = rina.LinearSeg(wd.data_ptr(), None, y0.data_ptr(), N)
    s1 = rina.LinearSeg(wd.data_ptr(), None, y1.data_ptr(), N)
    ok(hip.rina_hip_linear_fused(C.byref(s0), 1, 6, xd.data_ptr(), 1, K, rina.EPI_STORE, pro,
                                 nwd.data_ptr() if pro else None, 1e-5, stream()))
    keys = empty(2 * 8192, "int32")
    nk = C.c_int()
    ok(hip.rina_hip_linear_argmax(C.byref(s1), 6, xd.data_ptr(), K, pro, nwd.data_ptr() if pro else None, 1e-5,
                                  keys.data_ptr(), 8192, C.byref(nk), stream()))
    logits = host(y1)
    assert np.array_equal(logits.view(np.uint32), host(y0).view(np.uint32))
    assert 1 <= nk.value <= 8192
    want = L.orc_argmax(logits.ctypes.data, N)
    # ties at the maximum: the lowest index must win
    top = float(logits.max())
    tied = logits.copy()
    tied[[N // 3, N - 1, N // 7]] = top
    want_tied = L.orc_argmax(tied.ctypes.data, N)
    for qt_e in (6, 7):
        d_e = 64
        V = N
        ef = (r.standard_normal(V * d_e) * 0.5).astype(np.float32)
        emb = ef if qt_e == 6 else orc.pack(qt_e, ef)
        ed = dev(emb)
        ids = empty(16, "int32")
        pos = dev(np.array([6], np.int32))
        h = empty(d_e)
        ok(hip.rina_hip_argmax_embed(keys.data_ptr(), nk.value, 0, None, ids.data_ptr(), pos.data_ptr(), ed.data_ptr(),
                                     qt_e, h.data_ptr(), d_e, V, stream()))
        assert int(host(pos)[0]) == 7 and int(host(ids)[7]) == want
        row = ef[want * d_e:(want + 1) * d_e] if qt_e == 6 else orc.dequant(qt_e, emb, V * d_e)[want * d_e:(want + 1) * d_e]
        assert np.array_equal(host(h), row)
    # the key-slot form over the tied logits, then the slot is zero again
    slot = empty(2, "int32")
    out = empty(1, "int32")
    ok(hip.rina_hip_argmax_partial(dev(tied).data_ptr(), N, slot.data_ptr(), stream()))
    ok(hip.rina_hip_argmax_embed(slot.data_ptr(), 1, 1, out.data_ptr(), None, None, ed.data_ptr(), 7, h.data_ptr(),
                                 d_e, V, stream()))
    assert int(host(out)[0]) == want_tied
    assert not host(slot).any()


@pytest.mark.parametrize("qt", [7, 5, 10, 6])
@pytest.mark.parametrize("pro", [1, 2])
@pytest.mark.parametrize("M,K", [(1, 2048), (1, 640), (2, 2048), (1, 8192), (1, 4096)])
def test_linear_norm_prologue(rina, orc, qt, pro, M, K):
    """norm(x) fused into the matvec == oracle norm followed by oracle matvec"""
    hip = rina.load_hip()
    L = orc.load()
    r = rng(qt * 10 + pro + K)
    N = 256
    if qt == 10:
        w = q2k_blocks(K, N * K)
    else:
        wf = (r.standard_normal(N * K) * 0.02).astype(np.float32)
        w = wf if qt == 6 else orc.pack(qt, wf)
    x = (r.standard_normal((M, K)) * 3 + 0.5).astype(np.float32)
    nw = r.uniform(0.5, 1.5, K).astype(np.float32)
    y = empty(M * N)
    seg = rina.LinearSeg(dev(w).data_ptr(), None, y.data_ptr(), N)
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, qt, dev(x).data_ptr(), M, K, rina.EPI_STORE, pro,
                                 dev(nw).data_ptr(), np.float32(1e-5), stream()), "prologue")
    xn = x.copy()
    (L.orc_rms_norm if pro == 1 else L.orc_layer_norm)(xn.ctypes.data, nw.ctypes.data, M, K, np.float32(1e-5))
    assert_close(host(y).reshape(M, N), orc.linear(w, qt, xn, N, K), what="prologue %d qt %d" % (pro, qt))


@pytest.mark.parametrize("qt", [5, 7, 10])
@pytest.mark.parametrize("N,K,epi,pro", [(2048, 8192, 1, 0),    # W2 + residual: 8 rows per wave, 4 waves per row
                                         (2048, 2048, 1, 0),    # W_o + residual: 2 rows per wave
                                         (640, 1536, 1, 0),     # Jamba W2 + residual
                                         (4100, 2048, 0, 1),    # Q2_K LM-head form: 4 rows per wave, loops
                                         (2049, 2048, 1, 2)])   # ragged last row group, LayerNorm prologue
def test_linear_single_segment_decode_shapes(rina, orc, qt, N, K, epi, pro):
    """One matrix in one segment at the decode step's shapes (the direct
    kernel without a segment table): the residual-add epilogue, with the old
    output words loaded with the weights, and the norm prologues.  Normwise
    against the oracle's norm and matvec, and per element against float64
    products of the dequantized weights with the oracle's normalized row,
    within 1e-5 of the element's magnitude scale sum_k |w_ik x_k| (the
    bound fp32 accumulation of a K-term sum is held to) plus the rounding of
    the final residual add."""
    hip = rina.load_hip()
    L = orc.load()
    r = rng(qt * 7 + N + K + epi * 3 + pro)
    if qt == 10:
        w = q2k_blocks(N + K, N * K)
    else:
        w = orc.pack(qt, (r.standard_normal(N * K) * 0.02).astype(np.float32))
    x = (r.standard_normal(K) * 2 + 0.3).astype(np.float32)
    nw = r.uniform(0.5, 1.5, K).astype(np.float32)
    base = r.standard_normal(N).astype(np.float32)
    yd = dev(base)
    seg = rina.LinearSeg(dev(w).data_ptr(), None, yd.data_ptr(), N)
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, qt, dev(x).data_ptr(), 1, K, epi, pro,
                                 dev(nw).data_ptr() if pro else None, np.float32(1e-5), stream()), "single segment")
    xn = x.copy()
    if pro:
        (L.orc_rms_norm if pro == 1 else L.orc_layer_norm)(xn.ctypes.data, nw.ctypes.data, 1, K, np.float32(1e-5))
    ref = orc.linear(w, qt, xn, N, K)[0]
    if epi == 1:
        ref = base + ref
    got = host(yd)
    assert_close(got, ref, what="single segment qt %d N %d K %d" % (qt, N, K))
    W = orc.dequant(qt, w, N * K).reshape(N, K).astype(np.float64)
    ref64 = W @ xn.astype(np.float64) + (base.astype(np.float64) if epi == 1 else 0.0)
    scale = np.abs(W) @ np.abs(xn.astype(np.float64))
    err = np.abs(got.astype(np.float64) - ref64) - 1.2e-7 * np.abs(ref64)
    worst = int(np.argmax(err / scale))
    assert err[worst] <= REL_TOL * scale[worst], "element %d: %.9g against %.9g (scale %.3g)" % (
        worst, got[worst], ref64[worst], scale[worst])


def _prefill_weights(orc, qt, r, n):
    if qt == 10:   # zero-mean Q2_K blocks (flat element order; rows may straddle blocks)
        import importlib
        return importlib.import_module("rina_amd.synth").random_q2k(int(r.integers(1 << 30)), n)
    return orc.pack(qt, (r.standard_normal(n) * 0.02).astype(np.float32))


@pytest.mark.parametrize("qt", [5, 7, 10])
@pytest.mark.parametrize("M,N,K", [(16, 64, 32), (100, 200, 512), (64, 2048, 2048), (130, 77, 320), (512, 96, 1024),
                                   (520, 4096, 64), (256, 8192, 256),    # 64-row tiles; the others take 32-row tiles
                                   (512, 2048, 512),   # Q4 at 32 rows in 128-column tiles of eight waves (with 256 CUs)
                                   (48, 1408, 2048), (100, 2048, 1408), (33, 96, 10944)])   # DeepSeek-V2-Lite rows
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_linear_prefill_mfma(rina, orc, qt, M, N, K, epi):
    """Prompt-sized M on the matrix-core path: store, residual add and
    SiLU*up epilogues against the oracle's per-row matvec (fp32 products of
    the dequantized weights, fp32 sums).  Q2_K rows in flat element order
    (K = 320, 1408, 10944 straddle 256-value blocks) are the M > 1 analogue
    of the fused Q2_K kernel (ops/linear.cu:445-483)."""
    hip = rina.load_hip()
    r = rng(M * 7 + N + K + qt * 3 + epi)
    w = _prefill_weights(orc, qt, r, N * K)
    w3 = _prefill_weights(orc, qt, r, N * K)
    x = r.standard_normal((M, K)).astype(np.float32)
    y0 = r.standard_normal((M, N)).astype(np.float32)
    y = dev(y0)
    seg = rina.LinearSeg(dev(w).data_ptr(), dev(w3).data_ptr() if epi == 2 else None, y.data_ptr(), N)
    ok(hip.rina_hip_linear_fused(C.byref(seg), 1, qt, dev(x).data_ptr(), M, K, epi, 0, None, 0.0, stream()),
       "prefill")
    g = orc.linear(w, qt, x, N, K).astype(np.float64)
    if epi == 0:
        ref = g
    elif epi == 1:
        ref = y0.astype(np.float64) + g
    else:
        u = orc.linear(w3, qt, x, N, K).astype(np.float64)
        ref = g / (1.0 + np.exp(-g)) * u
    assert_close(host(y).reshape(M, N), ref, what="prefill q%d epi %d %s" % (qt, epi, (M, N, K)))


@pytest.mark.parametrize("qt", [5, 7, 10])
@pytest.mark.parametrize("Ns,epi", [((256, 64, 64), 0), ((100, 37), 1), ((2048, 512, 512), 0)])
def test_linear_prefill_segments(rina, orc, qt, Ns, epi):
    """Several weight segments on one prompt (q / k / v) in one matrix-core
    launch: each segment's rows against the oracle."""
    hip = rina.load_hip()
    r = rng(sum(Ns) + qt + epi)
    M, K = 100, 512
    ws = [_prefill_weights(orc, qt, r, n * K) for n in Ns]
    x = r.standard_normal((M, K)).astype(np.float32)
    y0 = [r.standard_normal((M, n)).astype(np.float32) for n in Ns]
    ys = [dev(y) for y in y0]
    wd = [dev(w) for w in ws]
    segs = (rina.LinearSeg * len(Ns))(*[rina.LinearSeg(wd[i].data_ptr(), None, ys[i].data_ptr(), Ns[i])
                                        for i in range(len(Ns))])
    ok(hip.rina_hip_linear_fused(segs, len(Ns), qt, dev(x).data_ptr(), M, K, epi, 0, None, 0.0, stream()), "segs")
    for i, n in enumerate(Ns):
        ref = orc.linear(ws[i], qt, x, n, K).astype(np.float64) + (y0[i] if epi == 1 else 0.0)
        assert_close(host(ys[i]).reshape(M, n), ref, what="segment %d of %s" % (i, Ns))


@pytest.mark.parametrize("qt", [5, 7, 10, 6])
@pytest.mark.parametrize("N,K", [(2048, 2048), (512, 8192), (1024, 1408)])
def test_linear_outlier_activations(rina, orc, qt, N, K):
    """Activation columns carrying 1e4x outliers (the decode matvec holds x
    to 22 bits of each 32-value column's maximum, weakest when one value of
    a column dwarfs the rest).  Per element, the error against a float64
    matvec of the same dequantized weights must stay within 1e-5 of the
    element's magnitude scale sum_k |w_ik x_k| (the bound fp32 accumulation
    itself obeys); the oracle's fp32 result is checked the same way, and the
    largest error relative to |y_i| is reported."""
    if qt in (5, 7) and K % 32:
        pytest.skip("Q4 rows need K % 32 == 0")
    hip = rina.load_hip()
    r = rng(qt * 7 + K)
    x = r.standard_normal(K).astype(np.float32)
    cols = K // 32
    hot = r.choice(cols, max(1, cols // 8), replace=False)
    for cidx in hot:                       # one 1e4x value in every eighth column
        x[cidx * 32 + int(r.integers(32))] = np.float32(1e4 * (1 if r.integers(2) else -1))
    x[:32] = np.float32(1e4) * r.standard_normal(32).astype(np.float32)   # a column of outliers only
    if qt == 10:
        import importlib
        w = importlib.import_module("rina_amd.synth").random_q2k(K, N * K)
    elif qt == 6:
        w = (r.standard_normal(N * K) * 0.02).astype(np.float32)
    else:
        w = orc.pack(qt, (r.standard_normal(N * K) * 0.02).astype(np.float32))
    W = orc.dequant(qt, w, N * K).reshape(N, K).astype(np.float64)
    ref64 = W @ x.astype(np.float64)
    scale = np.abs(W) @ np.abs(x.astype(np.float64))
    yd = empty(N)
    ok(hip.rina_hip_linear(dev(w).data_ptr(), qt, dev(x).data_ptr(), yd.data_ptr(), 1, N, K, stream()), "linear")
    got = host(yd).astype(np.float64)
    ora = orc.linear(w, qt, x, N, K)[0].astype(np.float64)
    e_gpu = np.abs(got - ref64) / scale
    e_ora = np.abs(ora - ref64) / scale
    rel_y = np.abs(got - ref64) / np.maximum(np.abs(ref64), 1e-30)
    print("qt %d N %d K %d: max |err|/sum|wx| gpu %.2e oracle %.2e; max |err|/|y| gpu %.2e (median %.2e)"
          % (qt, N, K, e_gpu.max(), e_ora.max(), rel_y.max(), np.median(rel_y)))
    assert e_ora.max() <= REL_TOL
    assert e_gpu.max() <= REL_TOL, "element %d: %.3e" % (int(e_gpu.argmax()), e_gpu.max())
    assert_close(got, ora, what="outlier matvec vs oracle")
