"""Shared test helpers: device arrays through torch (plumbing only) and
tolerance checks stated once."""
import numpy as np

# Matvec / attention tolerance of the north star: fp32 accumulate, 1e-5
# relative, measured against the largest output magnitude of the case.
REL_TOL = 1e-5


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got - ref))) / scale


# Per-element form (attention, norms and the other glue): every element is
# also held to its own magnitude, |got - ref| <= tol |ref| + ELEM_FLOOR
# max|ref|.  The floor covers elements that are sums with cancellation,
# whose rounding error is set by the size of their terms and not by the
# (small) result.  Long matvec rows (K in the thousands) and whole-model
# logits are held to the normwise bound only: there the oracle's own serial
# fp32 sum differs from the exact one by more than 1e-5 of a cancelled
# element.
ELEM_FLOOR = 1e-6


def elem_violations(got, ref, tol=REL_TOL, floor=ELEM_FLOOR):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    bad = ~(np.abs(got - ref) <= tol * np.abs(ref) + floor * scale)   # NaN counts as a violation
    return np.flatnonzero(bad), got, ref


def assert_close(got, ref, tol=REL_TOL, what=""):
    e = rel_err(got, ref)
    assert e <= tol, "%s: relative error %.3e > %.1e" % (what, e, tol)


def assert_close_elem(got, ref, tol=REL_TOL, what=""):
    assert_close(got, ref, tol, what)
    idx, g, r = elem_violations(got, ref, tol)
    assert idx.size == 0, "%s: %d elements outside %.0e |ref| + %.0e max|ref| (first at %d: %.9g against %.9g)" % (
        what, idx.size, tol, ELEM_FLOOR, idx[0], g[idx[0]], r[idx[0]])


def attention_f64(q, K, V, H, Hkv, dh):
    """Softmax attention of one query row (scale 1/sqrt(dh)) in float64 over
    K, V [n][Hkv * dh]: the outputs, and per output element the weighted
    mean magnitude sum_p w_p |v_p,i| of the values it averages."""
    q = np.asarray(q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    out, mag = np.zeros(H * dh), np.zeros(H * dh)
    for h in range(H):
        g = h // (H // Hkv)
        s = K[:, g * dh:(g + 1) * dh] @ q[h * dh:(h + 1) * dh] / np.sqrt(dh)
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h * dh:(h + 1) * dh] = w @ V[:, g * dh:(g + 1) * dh]
        mag[h * dh:(h + 1) * dh] = w @ np.abs(V[:, g * dh:(g + 1) * dh])
    return out, mag


# Per-element form for long-context attention against the float64 result:
# an output averaging n values carries fp32 rounding of the size of the
# values it averages (mag_i above), not of the output, which cancels to
# about mag / sqrt(n).  |got - ref| <= tol |ref| + ELEM_FLOOR mag_i.
def assert_close_attn(got, ref64, mag, tol=REL_TOL, what=""):
    got = np.asarray(got, np.float64).reshape(-1)
    bad = np.flatnonzero(~(np.abs(got - ref64) <= tol * np.abs(ref64) + ELEM_FLOOR * mag))
    assert bad.size == 0, "%s: %d elements outside %.0e |ref| + %.0e mag (first at %d: %.9g against %.9g, mag %.3g)" % (
        what, bad.size, tol, ELEM_FLOOR, bad[0], got[bad[0]], ref64[bad[0]], mag[bad[0]])


def torch():
    import torch as t
    return t


# Device tensors created by dev()/empty() stay referenced until the next
# test starts (conftest clears the list): a temporary whose only use is
# .data_ptr() would otherwise return its block to torch's caching allocator
# before the kernel runs, and the next upload would alias it.
LIVE = []


def dev(a):
    t = torch()
    x = t.from_numpy(np.ascontiguousarray(a)).cuda()
    LIVE.append(x)
    return x


def empty(n, dtype="float32"):
    t = torch()
    dt = {"float32": t.float32, "uint8": t.uint8, "int32": t.int32}[dtype]
    x = t.zeros(n, dtype=dt, device="cuda")
    LIVE.append(x)
    return x


def host(t):
    torch().cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return torch().cuda.current_stream().cuda_stream


_hiprt = None


def d2h(ptr, nbytes):
    """Copy nbytes of device memory owned by the engine to a numpy array."""
    global _hiprt
    import ctypes as C
    if _hiprt is None:
        _hiprt = C.CDLL("libamdhip64.so")
        _hiprt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hiprt.hipMemcpy.restype = C.c_int
    torch().cuda.synchronize()
    out = np.empty(nbytes, np.uint8)
    assert _hiprt.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0   # hipMemcpyDeviceToHost
    return out


def rng(seed):
    return np.random.default_rng(seed)


def ok(rc, what=""):
    assert rc == 0, "%s returned %d" % (what, rc)
