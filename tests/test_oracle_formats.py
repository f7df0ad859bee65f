"""Pin the CPU oracle's format rules: fp16, weight packers, Q2_K, KV blocks.

Checks are against numpy's IEEE float16 conversion, the reference's known
answers (rina-engine/tests/test_layers.cu:29,41,84), independent numpy
restatements (tests/_numpy_ref.py) and closed-form bounds.
"""
import numpy as np
import pytest

import _numpy_ref as nr


def test_f16_to_f32_exhaustive(orc):
    L = orc.load()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne(orc):
    L = orc.load()
    r = np.random.default_rng(0)
    vals = [r.standard_normal(20000).astype(np.float32) * 10 ** r.uniform(-9, 5, 20000).astype(np.float32)]
    # every f16 value, midpoints between neighbours (ties to even), overflow edge, subnormal edges
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    hv = h.view(np.float16).astype(np.float32)
    vals.append(hv)
    nxt = np.arange(1, 0x7c01, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((hv.astype(np.float64) + nxt) / 2).astype(np.float32)
    vals.append(mid[np.isfinite(mid)])
    vals.append(np.array([65504, 65519.99, 65520, 65536, 1e30, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0000001, 2 ** -26,
                          1e-10, 0.0, -0.0, np.inf, -np.inf], np.float32))
    x = np.concatenate(vals).astype(np.float32)
    x = np.concatenate([x, -x])
    got = np.array([L.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_trunc_closed_form(orc):
    L = orc.load()
    x = np.random.default_rng(1).standard_normal(5000).astype(np.float32) * np.float32(1000)
    x = np.concatenate([x, np.float32([1e-10, 7e-6, 7e5, -3.0])])
    b = x.view(np.uint32).astype(np.int64)
    e = ((b >> 23) & 0xFF) - 127 + 15
    m = (b >> 13) & 0x3FF
    m = np.where(e <= 0, 0, np.where(e >= 31, 0x3FF, m))
    e = np.clip(e, 0, 31)
    ref = (((b >> 31) & 1) << 15) | (e << 10) | m
    got = np.array([L.orc_f32_to_f16_trunc(float(v)) for v in x], np.int64)
    assert np.array_equal(got, ref)


def test_q4_known_answers(orc):
    # test_layers.cu:29,41 — nibble 0xEE with scale 1 is +7; dot with 1/K is 7.0
    blk = np.full(32, 7.0, np.float32)
    p = orc.pack(orc.Q4_0, blk)
    assert p[:2].view(np.uint16)[0] == np.float16(1.0).view(np.uint16)
    assert np.all(p[2:] == 0xEE)
    K = 256
    w = np.tile(p, K // 32 * 3).reshape(3, -1)
    y = orc.linear(w.reshape(-1), orc.Q4_0, np.full(K, 1.0 / K, np.float32), 3, K)
    assert np.all(y == 7.0)
    # test_layers.cu:84 — nibble 0x77 is 0: an all-zero block packs to scale 0 (1e-10 underflows fp16)
    z = orc.pack(orc.Q4_0, np.zeros(32, np.float32))
    assert np.all(z[2:] == 0x77) and z[0] == 0 and z[1] == 0
    assert np.all(orc.dequant(orc.Q4_0, z, 32) == 0)


def test_q4_pack_matches_numpy_restatement(orc):
    r = np.random.default_rng(2)
    x = (r.standard_normal(32 * 4096) * 0.02).astype(np.float32)
    x[:32] = 0
    x[32:64] = r.uniform(-1e-12, 1e-12, 32)
    assert np.array_equal(orc.pack(orc.Q4_0, x), nr.pack_q4(x))
    assert np.array_equal(orc.pack(orc.Q4_0F, x), nr.pack_q4(x, fp32_scale=True))


def test_q4_rounding_edges(orc):
    # y = 0.49999997f: q4_pack's floor(|y|+0.5) rounds the fp32 sum up to 1,
    # loader_hf's roundf gives 0 (both scale 1.0 from amax 7)
    x = np.zeros(32, np.float32)
    x[0] = 7.0
    x[1] = np.float32(0.49999997)
    x[2] = 2.5
    x[3] = -2.5
    a = orc.pack(orc.Q4_0, x)
    b = orc.pack(orc.Q4_0, x, hf=True)
    assert (a[2] >> 4) == 8 and (b[2] >> 4) == 7
    assert (a[3] & 0xF) == 10 and (a[3] >> 4) == 4      # +-2.5 -> +-3
    assert (b[3] & 0xF) == 10 and (b[3] >> 4) == 4


def test_q4_roundtrip_bound(orc):
    x = (np.random.default_rng(3).standard_normal(32 * 2000) * 0.02).astype(np.float32)
    for qt, fp32 in ((orc.Q4_0, False), (orc.Q4_0F, True)):
        d = orc.dequant(qt, orc.pack(qt, x), x.size)
        s = np.abs(x.reshape(-1, 32)).max(1, keepdims=True) / 7
        bound = s * 0.5 + (0 if fp32 else s * 7 * 2.0 ** -11) + 1e-12
        assert np.all(np.abs(d.reshape(-1, 32) - x.reshape(-1, 32)) <= bound)
        assert np.array_equal(d, nr.dequant_q4(orc.pack(qt, x), x.size, fp32))


def test_q2k_dequant_two_statements_agree(orc):
    # flat-element form (ops/linear.cu:413-431, the oracle) vs the page/thread
    # form (ops/linear.cu:322-338, the numpy restatement): values are exact in
    # fp32, so they must agree bit for bit
    r = np.random.default_rng(4)
    nb = 64
    blk = r.integers(0, 256, (nb, 84), dtype=np.uint8)
    blk[:, 80:82] = np.frombuffer(np.float16(0.0025).tobytes() * nb, np.uint8).reshape(nb, 2)
    blk[:, 82:84] = np.frombuffer(np.float16(0.00125).tobytes() * nb, np.uint8).reshape(nb, 2)
    w = blk.reshape(-1)
    got = orc.dequant(orc.Q2_K, w, nb * 256)
    ref = nr.dequant_q2k_blocks(w)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fmt", [1, 2, 3, 4])
def test_kv_quantize_matches_restatement(orc, fmt):
    r = np.random.default_rng(10 + fmt)
    x = r.standard_normal(32 * 3000).astype(np.float32)
    x[:32] = 0                                   # all-zero block
    x[32:64] = r.uniform(-1e-11, 1e-11, 32)      # amax <= 1e-10
    x[64:96] = np.float32(1e30) * np.sign(r.standard_normal(32)).astype(np.float32)   # fp16 overflow
    x[96:128] = np.arange(32, dtype=np.float32) - 15.5                                # ties
    assert orc.kv_block_bytes(fmt) == nr.KV_BB[fmt]
    got = orc.kv_quantize(fmt, x)
    assert np.array_equal(got, nr.kv_quantize(fmt, x))
    d = orc.kv_dequant(fmt, got, x.size)
    ref = nr.kv_dequant(fmt, got, x.size)
    assert np.array_equal(np.isnan(d), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(d[ok], ref[ok])


def test_kv_invariants(orc):
    x = np.random.default_rng(5).standard_normal(32 * 500).astype(np.float32)
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(1, keepdims=True)
    d8 = orc.kv_dequant(1, orc.kv_quantize(1, x), x.size).reshape(-1, 32)
    s8 = amax / 127
    assert np.all(np.abs(d8 - b) <= s8 * 0.5 + np.abs(b) * 2.0 ** -10 + 1e-7)
    d1 = orc.kv_dequant(4, orc.kv_quantize(4, x), x.size).reshape(-1, 32)
    assert np.all((d1 > 0) == (b > 0))
    assert np.allclose(np.abs(d1), np.float16(amax).astype(np.float32))
    # all-zero q2_1 block dequantizes to -fp16(amax) everywhere (quantize.cu:92-103)
    z = np.zeros(32, np.float32)
    z[5] = 1e-11
    dz = orc.kv_dequant(3, orc.kv_quantize(3, z), 32)
    assert np.all(dz == -np.float32(np.float16(np.float32(1e-11))))
