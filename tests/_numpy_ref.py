"""Independent numpy restatements used to pin the C oracle.

They are written from the reference's published rules with different
primitives than the oracle (vectorized numpy, numpy's own float16 RNE
conversion, the page/thread form of the Q2_K rule instead of the flat form),
so a slip in the oracle's bit handling or loop indexing shows up as a
mismatch.  Reference paths are relative to rina-engine/.
"""
import numpy as np

F32 = np.float32


def roundf(y):
    """C roundf (half away from zero) on float32 values, exact."""
    y = np.asarray(y, F32)
    t = np.trunc(y)
    frac = (y - t).astype(F32)
    return (t + np.where(np.abs(frac) >= F32(0.5), np.sign(y), F32(0))).astype(F32)


def f16_bits(x):
    return np.asarray(x, F32).astype(np.float16).view(np.uint16)


def f16_val(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(F32)


# ---- weights ------------------------------------------------------------

def pack_q4(x, fp32_scale=False):
    """tools/q4_pack.py:11-23,71-118, vectorized as the torch code is."""
    b = np.asarray(x, F32).reshape(-1, 32)
    amax = np.abs(b).max(axis=1, keepdims=True)
    scale = np.maximum((amax / F32(7.0)).astype(F32), F32(1e-10)).astype(F32)
    y = (b / scale).astype(F32)
    q = (np.clip(np.floor((np.abs(y) + F32(0.5)).astype(F32)), 0, 7).astype(np.int32) * np.sign(y).astype(np.int32))
    qu = (np.clip(q, -7, 7) + 7).astype(np.uint8)
    packed = (qu[:, 0::2] | (qu[:, 1::2] << 4)).astype(np.uint8)
    if fp32_scale:
        head = scale.astype(F32).view(np.uint8).reshape(-1, 4)
    else:
        head = f16_bits(scale[:, 0]).view(np.uint8).reshape(-1, 2)
    return np.concatenate([head, packed], axis=1).reshape(-1)


def dequant_q4(w, n, fp32_scale=False):
    bb = 20 if fp32_scale else 18
    so = 4 if fp32_scale else 2
    blk = np.asarray(w, np.uint8).reshape(-1, bb)[: n // 32]
    if fp32_scale:
        s = blk[:, :4].copy().view(F32)[:, 0]
    else:
        s = f16_val(blk[:, :2].copy().view(np.uint16)[:, 0])
    data = blk[:, so:so + 16]
    q = np.empty((blk.shape[0], 32), np.int32)
    q[:, 0::2] = data & 0xF
    q[:, 1::2] = data >> 4
    return ((q - 7).astype(F32) * s[:, None]).astype(F32).reshape(-1)


def dequant_q2k_blocks(w):
    """dequant_block_q2_K_gpu form (ops/linear.cu:322-338): thread tid of 64
    covers l = tid%32 in page n = tid/32 and writes 4 values 32 apart."""
    blk = np.asarray(w, np.uint8).reshape(-1, 84)
    nb = blk.shape[0]
    sc = blk[:, 0:16].astype(np.int32)
    qs = blk[:, 16:80].astype(np.int32)
    d = f16_val(blk[:, 80:82].copy().view(np.uint16)[:, 0])
    dmin = f16_val(blk[:, 82:84].copy().view(np.uint16)[:, 0])
    y = np.zeros((nb, 256), F32)
    for tid in range(64):
        n, l = tid // 32, tid % 32
        is_ = 8 * n + l // 16
        q = qs[:, 32 * n + l]
        for g in range(4):
            s = sc[:, is_ + 2 * g]
            a = (d * (s & 0xF).astype(F32)).astype(F32) * ((q >> (2 * g)) & 3).astype(F32)
            m = (dmin * (s >> 4).astype(F32)).astype(F32)
            y[:, 128 * n + l + 32 * g] = (a.astype(F32) - m).astype(F32)
    return y.reshape(-1)


# ---- KV blocks (kernels/quantize.cu) -------------------------------------

def kv_quantize(fmt, x):
    b = np.asarray(x, F32).reshape(-1, 32)
    nb = b.shape[0]
    amax = np.abs(b).max(axis=1)
    if fmt == 1:   # q8_0
        scale = np.maximum((amax / F32(127.0)).astype(F32), F32(1e-10)).astype(F32)
        q = np.clip(roundf(b / scale[:, None]), -127, 127).astype(np.int8)
        return np.concatenate([f16_bits(scale).view(np.uint8).reshape(-1, 2), q.view(np.uint8)], 1).reshape(-1)
    if fmt == 2:   # q4_0
        scale = np.maximum((amax / F32(7.0)).astype(F32), F32(1e-10)).astype(F32)
        q = (np.clip(roundf(b / scale[:, None]), -7, 7) + 7).astype(np.uint8)
        packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
        return np.concatenate([f16_bits(scale).view(np.uint8).reshape(-1, 2), packed], 1).reshape(-1)
    if fmt == 3:   # q2_1
        ok = amax > F32(1e-10)
        safe = np.where(ok, amax, F32(1)).astype(F32)
        q = (np.clip(roundf(b / safe[:, None]), -1, 1) + 1).astype(np.uint8)
        q[~ok] = 0
        packed = (q[:, 0::4] | (q[:, 1::4] << 2) | (q[:, 2::4] << 4) | (q[:, 3::4] << 6)).astype(np.uint8)
        return np.concatenate([f16_bits(amax).view(np.uint8).reshape(-1, 2), packed], 1).reshape(-1)
    if fmt == 4:   # q1_0, 6-byte record
        ok = amax > F32(1e-10)
        bits = ((b > 0).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1).astype(np.uint32)
        bits[~ok] = 0
        return np.concatenate([f16_bits(amax).view(np.uint8).reshape(-1, 2),
                               bits.view(np.uint8).reshape(-1, 4)], 1).reshape(-1)
    raise ValueError(fmt)


KV_BB = {1: 34, 2: 18, 3: 10, 4: 6}


def kv_dequant(fmt, data, n):
    blk = np.asarray(data, np.uint8).reshape(-1, KV_BB[fmt])[: n // 32]
    s = f16_val(blk[:, :2].copy().view(np.uint16)[:, 0])[:, None]
    if fmt == 1:
        return (blk[:, 2:].view(np.int8).astype(F32) * s).astype(F32).reshape(-1)
    if fmt == 2:
        q = np.empty((blk.shape[0], 32), np.int32)
        q[:, 0::2] = blk[:, 2:] & 0xF
        q[:, 1::2] = blk[:, 2:] >> 4
        return ((q - 7).astype(F32) * s).astype(F32).reshape(-1)
    if fmt == 3:
        q = np.empty((blk.shape[0], 32), np.int32)
        for k in range(4):
            q[:, k::4] = (blk[:, 2:] >> (2 * k)) & 3
        return ((q - 1).astype(F32) * s).astype(F32).reshape(-1)
    bits = blk[:, 2:6].copy().view(np.uint32)[:, 0]
    on = ((bits[:, None] >> np.arange(32, dtype=np.uint32)) & 1).astype(bool)
    return np.where(on, s, -s).astype(F32).reshape(-1)


# ---- float64 references ----------------------------------------------------

def softmax_attn(q, K, V, scale):
    """textbook softmax(q K^T * scale) V in float64"""
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ V.astype(np.float64)


def rope_neox(x, cos, sin, pos0):
    """x [T, H, d]: pairs (i, i+d/2), row t at table row pos0+t (float64)"""
    x = np.asarray(x, np.float64).copy()
    T, H, d = x.shape
    h = d // 2
    c = cos[pos0:pos0 + T][:, None, :].astype(np.float64)
    s = sin[pos0:pos0 + T][:, None, :].astype(np.float64)
    a, b = x[..., :h].copy(), x[..., h:].copy()
    x[..., :h] = a * c - b * s
    x[..., h:] = a * s + b * c
    return x
