"""InertiaWave SSM step on the GPU: rina_hip_ssm_step after the projections
(rina_hip_linear_fused) and the fused rina_hip_ssm_proj_step, each against
a float64 restatement of the reference's step (arch/ssm/rina_ssm_layer.cu:
97-109, kernels/ssm_kernels_fp32.cu:6-47) over several positions of one
scan, and against each other."""
import ctypes as C

import numpy as np
import pytest

import _numpy_ref as nr
from _util import assert_close, dev, empty, host, ok, rng, stream

pytestmark = pytest.mark.gpu


def ln(x, w):
    mu = x.mean()
    var = ((x - mu) ** 2).mean()
    return (x - mu) / np.sqrt(var + 1e-5) * w


def ref_scan(cqs, qn, wm, wd, steps, H, dh):
    """sf [T, H*dh] and the final (lcs, wcs) of the reference's scan over T
    positions; steps < 3 leave decay 1 and memory 0 for the missing steps."""
    lcs = np.zeros((H, 1))
    wcs = np.zeros((H, dh))
    sfs = []
    for cq in cqs:
        x = ln(cq.astype(np.float64), qn.astype(np.float64))
        mem = [(x @ wm[k].T).reshape(H, dh) if k < steps else np.zeros((H, dh)) for k in range(3)]
        dec = [1 / (1 + np.exp(-(x @ wd[k].T))) if k < steps else np.ones(H) for k in range(3)]
        da = np.maximum(dec[0] * dec[1] * dec[2], 1e-38)[:, None]
        ma = mem[0] * (dec[1] * dec[2])[:, None] + mem[1] * dec[2][:, None] + mem[2]
        lcs = lcs + np.log(da)
        ca = np.exp(lcs)
        wcs = wcs + ma / np.maximum(ca, 1e-30)
        sfs.append((ca * wcs).reshape(-1))
    return np.array(sfs), np.broadcast_to(lcs, (H, dh)).reshape(-1), wcs.reshape(-1)


def make(qt, H, dh, dc, steps, seed):
    r = rng(seed)
    fp32s = qt == 7
    packed, mats = [], []
    for k in range(steps):
        for rows, s in ((H * dh, 0.05), (H, 0.3)):
            w = (r.standard_normal(rows * dc) * s).astype(np.float32)
            p = nr.pack_q4(w, fp32s)
            packed.append(p)
            mats.append(nr.dequant_q4(p, rows * dc, fp32s).reshape(rows, dc).astype(np.float64))
    wm_p, wd_p = packed[0::2], packed[1::2]
    wm, wd = mats[0::2], mats[1::2]
    qn = r.uniform(0.8, 1.2, dc).astype(np.float32)
    return wm_p, wd_p, wm, wd, qn, r


SHAPES = [  # H, dh, dc, steps
    (10, 64, 160, 3),    # config-5 widths
    (4, 64, 64, 3),
    (3, 6, 160, 2),      # dh not a multiple of 4: 2 elements per wave
    (2, 5, 96, 1),       # odd dh: 1 element per wave
    (2, 32, 256, 3),     # 8 columns
    (1, 8, 32, 3),
]


@pytest.mark.parametrize("qt", [5, 7])
@pytest.mark.parametrize("H,dh,dc,steps", SHAPES)
def test_ssm_step_paths_against_reference(rina, qt, H, dh, dc, steps):
    hip = rina.load_hip()
    wm_p, wd_p, wm, wd, qn, r = make(qt, H, dh, dc, steps, H * 1000 + dh * 10 + dc + steps + qt)
    T = 6
    cqs = (r.standard_normal((T, dc)) * 1.5 + 0.2).astype(np.float32)
    sf_ref, lcs_ref, wcs_ref = ref_scan(cqs, qn, wm, wd, steps, H, dh)
    wmd, wdd = [dev(w) for w in wm_p], [dev(w) for w in wd_p]
    qnd = dev(qn)
    VP = C.c_void_p
    pm = (VP * 3)(*[w.data_ptr() for w in wmd] + [None] * (3 - steps))
    pd = (VP * 3)(*[w.data_ptr() for w in wdd] + [None] * (3 - steps))
    n = H * dh
    # two launches: LN prologue + 2*steps projections, then the scan step
    lcs2, wcs2, sf2 = empty(n), empty(n), empty(n)
    mem, dec, xn = empty(3 * n), empty(3 * H), empty(dc)
    segs = (rina.LinearSeg * 6)()
    for k in range(steps):
        segs[k] = rina.LinearSeg(wmd[k].data_ptr(), None, mem.data_ptr() + 4 * k * n, n)
        segs[steps + k] = rina.LinearSeg(wdd[k].data_ptr(), None, dec.data_ptr() + 4 * k * H, H)
    # fused
    lcs1, wcs1, sf1 = empty(n), empty(n), empty(n)
    for t in range(T):
        cqd = dev(cqs[t])
        ok(hip.rina_hip_linear_fused(segs, 2 * steps, qt, cqd.data_ptr(), 1, dc, rina.EPI_STORE,
                                     rina.PRO_LAYERNORM, qnd.data_ptr(), np.float32(1e-5), stream()), "projections")
        ok(hip.rina_hip_ssm_step(mem.data_ptr(), dec.data_ptr(), steps, H, dh, lcs2.data_ptr(), wcs2.data_ptr(),
                                 sf2.data_ptr(), 1 if t == 0 else 0, stream()), "ssm_step")
        ok(hip.rina_hip_ssm_proj_step(cqd.data_ptr(), qnd.data_ptr(), np.float32(1e-5), pm, pd, qt, steps, H, dh, dc,
                                      lcs1.data_ptr(), wcs1.data_ptr(), sf1.data_ptr(), 1 if t == 0 else 0,
                                      stream()), "ssm_proj_step")
        assert_close(host(sf2), sf_ref[t], what="ssm_step sf, position %d" % t)
        assert_close(host(sf1), sf_ref[t], what="ssm_proj_step sf, position %d" % t)
        assert_close(host(sf1), host(sf2), what="fused vs two launches, position %d" % t)
    for name, got in (("two launches", (lcs2, wcs2)), ("fused", (lcs1, wcs1))):
        assert_close(host(got[0]), lcs_ref, what=name + " lcs")
        assert_close(host(got[1]), wcs_ref, what=name + " wcs")


@pytest.mark.parametrize("H,dh,steps,T,reset", [(4, 64, 3, 37, 1), (3, 6, 2, 5, 0), (2, 5, 1, 1, 1), (10, 64, 3, 300, 0)])
def test_ssm_scan_equals_steps(rina, H, dh, steps, T, reset):
    """rina_hip_ssm_scan over T positions (a prompt's scan in one launch)
    equals T calls of rina_hip_ssm_step, bit for bit: every sf row (written
    with a row stride wider than H*dh, the gaps untouched) and the final
    state, from a zero start (reset) and from a carried state.  The step
    kernel is pinned against the float64 scan above."""
    hip = rina.load_hip()
    r = rng(7 * H + dh + 11 * steps + T + reset)
    n = H * dh
    mem = (r.standard_normal((steps, T, n)) * 0.7).astype(np.float32)
    dec = (r.standard_normal((steps, T, H)) * 1.5 + 1.0).astype(np.float32)
    l0 = r.uniform(-3.0, 0.0, n).astype(np.float32)
    w0 = r.standard_normal(n).astype(np.float32)
    # T one-position launches
    lcs1, wcs1 = dev(l0), dev(w0)
    sf1 = np.zeros((T, n), np.float32)
    out = empty(n)
    for t in range(T):
        md, dd = dev(np.ascontiguousarray(mem[:, t, :])), dev(np.ascontiguousarray(dec[:, t, :]))
        ok(hip.rina_hip_ssm_step(md.data_ptr(), dd.data_ptr(), steps, H, dh, lcs1.data_ptr(), wcs1.data_ptr(),
                                 out.data_ptr(), reset if t == 0 else 0, stream()), "ssm_step")
        sf1[t] = host(out)
    # one scan launch
    stride = n + 7
    lcs2, wcs2 = dev(l0), dev(w0)
    sf2 = dev(np.full(T * stride, 123.0, np.float32))
    ok(hip.rina_hip_ssm_scan(dev(mem).data_ptr(), dev(dec).data_ptr(), steps, H, dh, T, lcs2.data_ptr(),
                             wcs2.data_ptr(), sf2.data_ptr(), stride, reset, stream()), "ssm_scan")
    got = host(sf2).reshape(T, stride)
    assert np.array_equal(got[:, :n].view(np.uint32), sf1.view(np.uint32))
    assert np.all(got[:, n:] == 123.0)
    assert np.array_equal(host(lcs2).view(np.uint32), host(lcs1).view(np.uint32))
    assert np.array_equal(host(wcs2).view(np.uint32), host(wcs1).view(np.uint32))


def test_ssm_proj_step_rejects(rina):
    hip = rina.load_hip()
    buf = empty(1 << 16)
    p = buf.data_ptr()
    VP = C.c_void_p
    w3 = (VP * 3)(p, p, p)
    args = lambda qt, H, dh, dc, steps, w=w3: (p, p, np.float32(1e-5), w, w, qt, steps, H, dh, dc, p, p, p, 0,
                                               stream())
    assert hip.rina_hip_ssm_proj_step(*args(10, 2, 8, 256, 3)) == -2        # Q2_K
    assert hip.rina_hip_ssm_proj_step(*args(6, 2, 8, 64, 3)) == -2         # fp32
    assert hip.rina_hip_ssm_proj_step(*args(5, 2, 8, 48, 3)) == -3         # dc % 32
    assert hip.rina_hip_ssm_proj_step(*args(5, 2, 8, 288, 3)) == -3        # dc > 256
    assert hip.rina_hip_ssm_proj_step(*args(5, 2, 8, 64, 4)) == -1         # steps > 3
    assert hip.rina_hip_ssm_proj_step(*args(5, 2, 8, 64, 2, (VP * 3)(p, None, p))) == -1
    torch = __import__("torch")
    torch.cuda.synchronize()
