"""Keys and values in 8 bits, attended to without unpacking them -- MI355X drop-in for ``locals/qkv.py``.

Same names, argument orders and semantics as the reference module (locals/qkv.py), on torch tensors in GPU memory:

* ``attend(q, keys, values, n, sinks, scale, start)`` -- one query a row over whole-buffer 8-bit
  (words, scales, biases) triples read in place, keys ``[start[b], n)`` of row b, a softmax with each head's sink
  (locals/qkv.py:213-249).  Backed by ``lcl_qkv_attend`` (split-K flash decode on MFMA, include/locals_amd.h).
* ``dequantized``, ``quantized``, ``attention``, ``QuantizedKVCache8``, ``BatchQuantizedKVCache``, ``BITS``,
  ``GROUP``, ``BLOCK``, ``wants_8bit``, ``opt_in`` -- see their docstrings.

Nothing here synchronises with the GPU except where the reference itself reads values back on the host
(``filter``/``extract`` read ``left_padding``, locals/qkv.py:376,415-416).
"""

from __future__ import annotations

import os
from typing import List, Optional

import torch

from . import _lib

BITS, GROUP = 8, 64
BLOCK = 0  # keys a pass-1 workgroup reads (a multiple of 64); 0: the library's choice (locals/qkv.py:28)

_U32 = getattr(torch, "uint32", None)


def _words_ok(t: torch.Tensor) -> bool:
    return t.dtype in (torch.int32,) or (_U32 is not None and t.dtype == _U32)


def _check_triple(t, name):
    if not isinstance(t, (tuple, list)) or len(t) != 3:
        raise ValueError(f"{name} must be a (words, scales, biases) triple")
    w, s, b = t
    if not _words_ok(w):
        raise ValueError(f"{name} words must be int32/uint32, got {w.dtype}")
    if s.dtype not in (torch.float16, torch.bfloat16) or b.dtype != s.dtype:
        raise ValueError(f"{name} scales/biases must be float16 or bfloat16 (same dtype)")
    for x in t:
        if not x.is_contiguous():
            raise ValueError(f"{name} buffers must be contiguous (they are read in place)")
    if w.dim() != 4 or s.dim() != 4 or b.dim() != 4:
        raise ValueError(f"{name} buffers must be (B, KVH, cap, .)")
    if s.shape[:3] != w.shape[:3] or b.shape != s.shape or s.shape[3] * 16 != w.shape[3]:
        raise ValueError(f"{name} triple shapes disagree: {tuple(w.shape)}, {tuple(s.shape)}, {tuple(b.shape)}")


def workspace_bytes(R: int, H: int, extent: int, block: int = 0) -> int:
    return int(_lib.load().lcl_decode_workspace_bytes(R, H, extent, block))


def attend(q: torch.Tensor, keys, values, n: int, sinks: Optional[torch.Tensor], scale: float,
           start: Optional[torch.Tensor]) -> torch.Tensor:
    """One query per row against 8-bit keys and values (locals/qkv.py:213-249).

    ``q`` (B, H, 1, HD) with HD = 128; ``keys``/``values`` a cache's whole buffers, (words, scales, biases) of shape
    (B, KVH, capacity, ...), read in place; positions ``start[b]`` to ``n`` are row b's.  Softmax over those keys and
    the head's sink (``sinks`` (H,), any float dtype, or None for no sink).  Returns (B, H, 1, HD) in q's dtype.
    """
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError("attend takes one query a row: q (B, H, 1, HD)")
    B, H, _, HD = q.shape
    _check_triple(keys, "keys")
    _check_triple(values, "values")
    kw, ks, kb = keys
    vw, vs, vb = values
    if kw.shape != vw.shape or ks.shape != vs.shape or ks.dtype != vs.dtype:
        raise ValueError("keys and values buffers must have the same shapes and dtypes")
    if kw.shape[0] != B:
        raise ValueError("keys rows must match q rows")
    KVH, cap = kw.shape[1], kw.shape[2]
    if kw.shape[3] * 4 != HD:
        raise ValueError("head_dim of q and of the 8-bit buffers differ")
    if H % KVH:
        raise ValueError("query heads must be a multiple of key/value heads")
    n = int(n)
    if not 0 <= n <= cap:
        raise ValueError(f"n={n} outside the buffers' capacity {cap}")
    dev = _lib.require_gpu(q, kw, ks, kb, vw, vs, vb, start, sinks)
    q = q.contiguous()
    st = None
    if start is not None:
        st = start.to(device=dev, dtype=torch.int32).contiguous()
        if st.numel() != B:
            raise ValueError("start must have one entry a row")
    sk = None
    if sinks is not None:
        sk = sinks.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if sk.numel() != H:
            raise ValueError("sinks must have one entry a query head")
    lib = _lib.load()
    blk = int(BLOCK)
    nbytes = int(lib.lcl_decode_workspace_bytes(B, H, n, blk))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    out = torch.empty((B, H, 1, HD), dtype=q.dtype, device=dev)
    rc = lib.lcl_qkv_attend(_lib.ptr(q), _lib.dtype_code(q.dtype), _lib.ptr(kw), _lib.ptr(ks), _lib.ptr(kb),
                            _lib.ptr(vw), _lib.ptr(vs), _lib.ptr(vb), _lib.dtype_code(ks.dtype), _lib.ptr(st),
                            _lib.ptr(sk), float(scale), B, H, KVH, HD, cap, n, blk, _lib.ptr(out), _lib.ptr(ws),
                            nbytes, _lib.stream_of(dev))
    _lib.check(rc, "lcl_qkv_attend")
    return out
