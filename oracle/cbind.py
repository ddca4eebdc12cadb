"""ctypes binding of ``oracle/liboracle.so`` (the C restatement) -- test infrastructure.

``attend_q8`` runs the reference's two-pass split-K decode (locals/qkv.py:30-87,
179-208, 232) in fp32 on the host cores; ``quantize`` runs MLX's affine quantizer;
``sdpa`` / ``sdpa_q8`` run masked multi-query attention with sinks (MLX SDPA as
locals/qkv.py:270-272, locals/fuse.py:131-144 and locals/treedec.py:56-79 call it),
for full-size parity where the float64 oracle would take minutes.
Build with ``make -C oracle`` (``__graft_entry__.build()`` does).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from .quant import from_f32, to_f32

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/liboracle.so is not built (run: make -C oracle)")
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        L.orc_attend_q8.argtypes = [P] * 9 + [ctypes.c_float] + [ctypes.c_int] * 7 + [P]
        L.orc_attend_q8.restype = ctypes.c_int
        L.orc_quantize.argtypes = [P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P]
        L.orc_quantize.restype = None
        L.orc_sdpa.argtypes = [P, P, P, P, ctypes.c_int, P, P, ctypes.c_int, P, ctypes.c_float] + \
            [ctypes.c_int] * 7 + [P]
        L.orc_sdpa.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def quantize(w, dtype: str = "float16", group: int = 64, round_mode: str = "away"):
    x = np.ascontiguousarray(to_f32(w, dtype), dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D
    codes = np.empty(x.shape, dtype=np.uint8)
    sc = np.empty(x.shape[:-1] + (D // group,), dtype=np.float32)
    bi = np.empty_like(sc)
    lib().orc_quantize(_p(x), rows, D, group, 0 if round_mode == "away" else 1, _p(codes), _p(sc), _p(bi))
    words = codes.reshape(-1, D).view("<u4").reshape(x.shape[:-1] + (D // 4,))
    return words, from_f32(sc, dtype), from_f32(bi, dtype)


def attend_q8(q, keys, values, n: int, sinks, scale: float, start, dtype: str = "float16", block: int = 0,
              threads: int | None = None):
    """fp32 two-pass split-K decode on the host.  Returns float32 (B, H, 1, HD)."""
    qf = np.ascontiguousarray(to_f32(q, dtype), dtype=np.float32)
    B, H, _, HD = qf.shape
    kw, ks, kb = keys
    vw, vs, vb = values
    KVH, cap = kw.shape[1], kw.shape[2]
    f = lambda a: np.ascontiguousarray(to_f32(a, dtype), dtype=np.float32)  # noqa: E731
    kw, vw = np.ascontiguousarray(kw, dtype=np.uint32), np.ascontiguousarray(vw, dtype=np.uint32)
    ks, kb, vs, vb = f(ks), f(kb), f(vs), f(vb)
    st = np.ascontiguousarray(start, dtype=np.int32)
    sk = None if sinks is None else np.ascontiguousarray(to_f32(sinks, dtype), dtype=np.float32)
    out = np.empty((B, H, HD), dtype=np.float32)
    if threads is not None:
        os.environ["OMP_NUM_THREADS"] = str(threads)
    rc = lib().orc_attend_q8(_p(qf), _p(kw), _p(ks), _p(kb), _p(vw), _p(vs), _p(vb), _p(st), _p(sk),
                             ctypes.c_float(scale), B, H, KVH, HD, cap, n, block, _p(out))
    if rc:
        raise ValueError(f"orc_attend_q8 failed ({rc})")
    return out.reshape(B, H, 1, HD)


MASKS = {None: 0, "causal": 1, "tree": 2, "dense": 3, "window": 4}


def sdpa(q, k, v, scale: float, mask=None, sinks=None, start=None, tree=None, dense=None, window: int = 0,
         n: int | None = None, threads: int | None = None):
    """Masked SDPA over fp32 values: q (B, H, L, D), k/v (B, KVH, cap, D) of which the first ``n`` keys (default
    cap) are attended.  ``mask``: None, "causal", "tree" (``tree`` (B, L) uint64 bits of the new keys each query
    sees; the first N - L keys are visible to all), "dense" (``dense`` (B, L, N) bool) or "window" (``window``).
    Returns float32 (B, H, L, D)."""
    qf = np.ascontiguousarray(q, dtype=np.float32)
    kf = np.ascontiguousarray(k, dtype=np.float32)
    vf = np.ascontiguousarray(v, dtype=np.float32)
    B, H, L, D = qf.shape
    KVH, cap = kf.shape[1], kf.shape[2]
    N = cap if n is None else int(n)
    tr = None if tree is None else np.ascontiguousarray(tree, dtype=np.uint64)
    de = None if dense is None else np.ascontiguousarray(dense, dtype=np.uint8)
    st = None if start is None else np.ascontiguousarray(start, dtype=np.int32)
    sk = None if sinks is None else np.ascontiguousarray(sinks, dtype=np.float32)
    out = np.empty((B, H, L, D), dtype=np.float32)
    if threads is not None:
        os.environ["OMP_NUM_THREADS"] = str(threads)
    rc = lib().orc_sdpa(_p(qf), _p(kf), _p(vf), _p(st), MASKS[mask], _p(tr), _p(de), int(window), _p(sk),
                        ctypes.c_float(scale), B, H, KVH, L, N, D, cap, _p(out))
    if rc:
        raise ValueError(f"orc_sdpa failed ({rc})")
    return out


def sdpa_q8(q, keys, values, scale: float, mask=None, sinks=None, n: int | None = None, dtype: str = "float16",
            **kw):
    """``sdpa`` over 8-bit triples dequantized as the reference's prompt path feeds MLX's attention: fp32
    ``scale * code + bias`` rounded to the activation dtype (``mx.dequantize`` returns it, locals/qkv.py:272)."""
    from .quant import dequantize

    def dq(t):
        x = dequantize(*t, dtype=dtype, out=np.float32).astype(np.float32)
        return to_f32(from_f32(x, dtype), dtype)

    sk = None if sinks is None else to_f32(sinks, dtype)
    return sdpa(to_f32(q, dtype), dq(keys), dq(values), scale, mask, sk, n=n, **kw)
