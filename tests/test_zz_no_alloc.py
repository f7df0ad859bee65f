"""The allocation-free decode attention (rina_hip_gqa_decode_attention_noalloc)
against the workspace entry point it shares its kernels with: same outputs
and the same appended cache bytes, bit for bit, on two calls in a row (the
second smaller), and the size limit rejected before anything is launched."""
import numpy as np
import pytest

from _util import dev, empty, host, ok, rng, stream

pytestmark = pytest.mark.gpu


def rope(dh, n, theta=500000.0):
    inv = 1.0 / theta ** (np.arange(0, dh, 2, dtype=np.float64) / dh)
    ang = np.outer(np.arange(n), inv)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def one_call(rina, mode, H, Hkv, pos, max_seq, seed):
    hip = rina.load_hip()
    dh = 64
    kvd = Hkv * dh
    r = rng(seed)
    q = r.standard_normal(H * dh).astype(np.float32)
    k = r.standard_normal(kvd).astype(np.float32)
    v = r.standard_normal(kvd).astype(np.float32)
    cos, sin = rope(dh, max_seq)
    region = int(hip.rina_hip_kv_region_bytes(mode, 0, max_seq, kvd))
    if mode == 0:
        ck = r.standard_normal(region // 4).astype(np.float32)
        cv = r.standard_normal(region // 4).astype(np.float32)
    else:   # valid packed rows: quantize random values with the library's packer
        kf, vf = {1: (1, 1), 2: (2, 2), 5: (3, 4)}[mode]
        ckd, cvd = empty(region, "uint8"), empty(int(hip.rina_hip_kv_region_bytes(mode, 1, max_seq, kvd)), "uint8")
        ok(hip.rina_hip_kv_quantize(kf, dev(r.standard_normal(max_seq * kvd).astype(np.float32)).data_ptr(),
                                    ckd.data_ptr(), max_seq * kvd, stream()))
        ok(hip.rina_hip_kv_quantize(vf, dev(r.standard_normal(max_seq * kvd).astype(np.float32)).data_ptr(),
                                    cvd.data_ptr(), max_seq * kvd, stream()))
        ck, cv = host(ckd), host(cvd)
    args = [dev(q).data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(), dev(cos).data_ptr(), dev(sin).data_ptr(),
            dev(cos).data_ptr(), dev(sin).data_ptr()]
    ck1, cv1, ck2, cv2 = dev(ck), dev(cv), dev(ck), dev(cv)
    o1, o2 = empty(H * dh), empty(H * dh)
    wsb = int(hip.rina_hip_gqa_attention_workspace(1, H, dh, max_seq))
    ws = empty(wsb, "uint8")
    ok(hip.rina_hip_gqa_decode_attention(*args, ck1.data_ptr(), cv1.data_ptr(), mode, H, Hkv, dh, pos, None, max_seq,
                                         o1.data_ptr(), None, ws.data_ptr(), wsb, stream()), "workspace form")
    ok(hip.rina_hip_gqa_decode_attention_noalloc(*args, ck2.data_ptr(), cv2.data_ptr(), mode, H, Hkv, dh, pos, None,
                                                 max_seq, o2.data_ptr(), None, stream()), "allocation-free form")
    a, b = host(o1), host(o2)
    assert np.all(np.isfinite(a))
    assert np.array_equal(a, b)
    assert np.array_equal(host(ck1), host(ck2)) and np.array_equal(host(cv1), host(cv2))


def test_noalloc_matches_workspace_form_twice(rina):
    # config-2 shape at position 530, then a smaller call (fewer heads, shorter
    # cache, another KV format): the second call runs over the first's leftovers
    one_call(rina, 1, 32, 8, 530, 600, 1)
    one_call(rina, 2, 8, 2, 100, 128, 2)
    one_call(rina, 0, 8, 2, 37, 64, 3)


def test_noalloc_rejects_oversized_partials(rina):
    hip = rina.load_hip()
    lim = int(hip.rina_hip_noalloc_scratch_bytes())
    assert lim == 1 << 20
    H, Hkv, ms = 64, 8, 4096
    assert int(hip.rina_hip_gqa_attention_workspace(1, H, 64, ms)) > lim
    x = empty(64 * 64)
    rc = hip.rina_hip_gqa_decode_attention_noalloc(x.data_ptr(), x.data_ptr(), x.data_ptr(), None, None, None, None,
                                                   x.data_ptr(), x.data_ptr(), 1, H, Hkv, 64, 5, None, ms,
                                                   x.data_ptr(), None, stream())
    assert rc == -6   # RINA_ERR_WORKSPACE, nothing launched
