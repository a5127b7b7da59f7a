"""ctypes wrapper of the RefineKV CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, as the checker or the timed CPU baseline.  The
product package never imports it.  The C sources in ``rkv_oracle.c`` restate
the reference's torch path (src/refinekv/summary.py:35-113,
src/refinekv/reference.py:10-73); this module only moves numpy arrays.

Array conventions: fp32 arrays hold exact values of the caller's dtype;
bfloat16 data is passed as its uint16 bit pattern.
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liborc.so")
TILE = 64  # LSE tile (blocks), shared with the HIP kernels
REDUCTIONS = {"mean": 0, "max": 1, "any": 2}

_lib = None
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build():
    """Compile the oracle with its Makefile (gcc)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_summary.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64p, _u16p, _u16p,
                                  _u16p, _f32p, _f32p]
        L.orc_summary.restype = ctypes.c_int
        L.orc_select_stats.argtypes = [_f32p, _u16p, _u16p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                       _i64, _i64, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_select_stats.restype = ctypes.c_int
        L.orc_select.argtypes = [_f32p, _u16p, _u16p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                 _i64, ctypes.c_float, ctypes.c_int, ctypes.c_void_p, _u8p, _f32p,
                                 _f32p]
        L.orc_select.restype = ctypes.c_int
        L.orc_sparse_attention.argtypes = [_f32p, _u16p, _u16p, _u16p, _f32p, _f32p, _u16p, _u16p,
                                           _u16p, _u16p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                           ctypes.c_float, ctypes.c_int, ctypes.c_void_p, _u8p,
                                           _f32p]
        L.orc_sparse_attention.restype = ctypes.c_int
        L.orc_dense_attention.argtypes = [_f32p, _u16p, _u16p, _i64, _i64, _i64, _i64, _f32p]
        L.orc_dense_attention.restype = ctypes.c_int
        for name in ("orc_expf_n", "orc_logf_n"):
            getattr(L, name).argtypes = [_f32p, _f32p, _i64]
        L.orc_bf16_n.argtypes = [_f32p, _u16p, _i64]
        L.orc_risk_n.argtypes = [_f32p] * 7 + [_i64]
        _lib = L
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _u16(x):
    x = np.ascontiguousarray(x)
    if x.dtype != np.uint16:
        raise TypeError("bfloat16 data must be passed as uint16 bit patterns")
    return x


def expf(x):
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().orc_expf_n(x, y, x.size)
    return y


def logf(x):
    x = _f32(x).ravel()
    y = np.empty_like(x)
    lib().orc_logf_n(x, y, x.size)
    return y


def risk(z, delta, log_z, log_c, vmax, vnorm):
    """Elementwise risk (reference.py:26-34) from given statistics (broadcast)."""
    arrs = np.broadcast_arrays(*[_f32(a) for a in (z, delta, log_z, log_c, vmax, vnorm)])
    arrs = [np.ascontiguousarray(a, dtype=np.float32).ravel() for a in arrs]
    out = np.empty_like(arrs[0])
    lib().orc_risk_n(*arrs, out, out.size)
    return out


def bf16_bits(x):
    """Round fp32 to bfloat16 (nearest-even); returns uint16 bit patterns."""
    x = _f32(x)
    y = np.empty(x.shape, np.uint16)
    lib().orc_bf16_n(x.ravel(), y.reshape(-1), x.size)
    return y


def bf16_value(bits):
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def num_blocks(length, block):
    return (length + block - 1) // block


def summary(keys, values, block):
    """build_summary on (H, L, D) arrays.  Returns a dict of numpy arrays."""
    keys, values = _f32(keys), _f32(values)
    H, L, D = keys.shape
    N = num_blocks(L, block)
    out = dict(
        counts=np.empty(N, np.int64),
        key_mean=np.empty((H, N, D), np.uint16),
        value_mean=np.empty((H, N, D), np.uint16),
        ellipsoid=np.empty((H, N, D), np.uint16),
        value_norm=np.empty((H, N), np.float32),
        max_value_norm=np.empty(H, np.float32),
    )
    rc = lib().orc_summary(keys, values, H, L, D, block, out["counts"], out["key_mean"],
                           out["value_mean"], out["ellipsoid"], out["value_norm"],
                           out["max_value_norm"])
    if rc:
        raise ValueError(f"orc_summary rejected shape {keys.shape} block {block}")
    out.update(prompt_length=L, block_size=block)
    return out


def select_stats(query, summ):
    """selection_statistics: query (H, G, D) -> z, delta, risk (H,G,N), log_z, log_c (H,G)."""
    q = _f32(query)
    H, G, D = q.shape
    N = summ["counts"].shape[0]
    z = np.empty((H, G, N), np.float32)
    delta = np.empty_like(z)
    risk = np.empty_like(z)
    lz = np.empty((H, G), np.float32)
    lc = np.empty_like(lz)
    rc = lib().orc_select_stats(q, _u16(summ["key_mean"]), _u16(summ["ellipsoid"]),
                                _f32(summ["value_norm"]), _f32(summ["max_value_norm"]), H, G, D,
                                N, summ["block_size"], summ["prompt_length"], z, delta, risk, lz,
                                lc)
    if rc:
        raise ValueError("orc_select_stats rejected its inputs")
    return dict(z=z, delta=delta, risk=risk, log_z=lz, log_c=lc)


def _anchor_ptr(anchor, H, N):
    if anchor is None:
        return None, None
    a = np.ascontiguousarray(anchor, dtype=np.uint8).reshape(H, N)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def select(query, summ, eps, reduction, anchor=None):
    """select_blocks_reference (+ optional anchor union): mask (H, N) uint8, z, risk."""
    q = _f32(query)
    H, G, D = q.shape
    N = summ["counts"].shape[0]
    keep, aptr = _anchor_ptr(anchor, H, N)
    mask = np.empty((H, N), np.uint8)
    z = np.empty((H, G, N), np.float32)
    risk = np.empty_like(z)
    rc = lib().orc_select(q, _u16(summ["key_mean"]), _u16(summ["ellipsoid"]),
                          _f32(summ["value_norm"]), _f32(summ["max_value_norm"]), H, G, D, N,
                          summ["block_size"], summ["prompt_length"], float(eps),
                          REDUCTIONS[reduction], aptr, mask, z, risk)
    if rc:
        raise ValueError("orc_select rejected its inputs")
    return mask, z, risk


def sparse_attention(query, summ, key_pages, value_pages, key_suffix, value_suffix, eps,
                     reduction, anchor=None):
    """sparse_attention_reference: returns (out (H, G, D) fp32, mask (H, N) uint8).

    key_pages/value_pages: (H, N, B, D) bf16 bits; suffix: (H, S, D) bf16 bits.
    """
    q = _f32(query)
    H, G, D = q.shape
    N = summ["counts"].shape[0]
    B = summ["block_size"]
    kp, vp = _u16(key_pages).reshape(H, N, B, D), _u16(value_pages).reshape(H, N, B, D)
    ks, vs = _u16(key_suffix), _u16(value_suffix)
    S = ks.shape[1]
    if ks.size == 0:
        ks = vs = np.zeros((H, 1, D), np.uint16)
    keep, aptr = _anchor_ptr(anchor, H, N)
    mask = np.empty((H, N), np.uint8)
    out = np.empty((H, G, D), np.float32)
    rc = lib().orc_sparse_attention(q, _u16(summ["key_mean"]), _u16(summ["value_mean"]),
                                    _u16(summ["ellipsoid"]), _f32(summ["value_norm"]),
                                    _f32(summ["max_value_norm"]), kp, vp, ks, vs, S, H, G, D, N,
                                    B, summ["prompt_length"], float(eps), REDUCTIONS[reduction],
                                    aptr, mask, out)
    if rc:
        raise ValueError("orc_sparse_attention rejected its inputs")
    return out, mask


def dense_attention(query, keys, values):
    """Dense decode (transformers.py:510-520's SDPA over the cache): returns
    out (H, G, D) fp32.  query (H, G, D); keys/values (H, L, D) bf16 bits."""
    q = _f32(query)
    H, G, D = q.shape
    k, v = _u16(keys), _u16(values)
    L = k.shape[1]
    out = np.empty((H, G, D), np.float32)
    if lib().orc_dense_attention(q, k, v, H, G, D, L, out):
        raise ValueError("orc_dense_attention rejected its inputs")
    return out


def access_blocks(mask, counts):
    """Per-step block term of the access counter (transformers.py:590-594):
    sum over (head, block) of count if expanded else 1."""
    mask = np.asarray(mask).astype(bool)
    counts = np.asarray(counts, dtype=np.int64)
    return int((mask * counts[None, :]).sum() + (~mask).sum())
