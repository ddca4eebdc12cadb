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

import ctypes
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
    """Decode attention of a single query token per row over an 8-bit cache (locals/qkv.py:213-249).

    ``q`` is (B, H, 1, 128).  ``keys`` and ``values`` are the cache's full (words, scales, biases) buffers,
    (B, KVH, capacity, ...); they are consumed where they lie, without copying out the live part.  Row b uses
    buffer positions ``start[b]`` up to ``n`` (``start`` None means 0).  Each head's softmax also counts its sink
    logit ``sinks[h]`` in the denominator (``sinks`` (H,) of any float dtype, or None).  The result is
    (B, H, 1, 128) in q's dtype.
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


ROUND_MODE = os.environ.get("LOCALS_AMD_ROUND", "away")  # "away": MLX's Metal mx.quantize; "even": its CPU path


def _round_code(mode: Optional[str] = None) -> int:
    m = ROUND_MODE if mode is None else mode
    if m not in ("away", "even"):
        raise ValueError("round mode must be 'away' or 'even'")
    return 0 if m == "away" else 1


def quantize_into(keys: torch.Tensor, values: Optional[torch.Tensor], kbuf, vbuf, prev: int,
                  round_mode: Optional[str] = None) -> None:
    """Quantize (B, KVH, L, D) ``keys`` (and ``values``) with MLX's affine 8 bits (group 64) into positions
    [prev, prev + L) of the (B, KVH, cap, .) triples ``kbuf``/``vbuf`` (locals/qkv.py:320-325), one launch."""
    if keys.dim() != 4:
        raise ValueError("keys must be (B, KVH, L, D)")
    B, KVH, L, D = keys.shape
    if keys.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("8-bit caches take float16 or bfloat16 keys and values")
    _check_triple(kbuf, "key buffers")
    cap = kbuf[0].shape[2]
    if kbuf[0].shape[:2] != (B, KVH) or kbuf[0].shape[3] * 4 != D or kbuf[1].dtype != keys.dtype:
        raise ValueError("key buffers do not match the keys")
    if values is not None:
        _check_triple(vbuf, "value buffers")
        if values.shape != keys.shape or values.dtype != keys.dtype or vbuf[0].shape != kbuf[0].shape:
            raise ValueError("values must match keys")
    if not 0 <= prev <= cap - L:
        raise ValueError("write past the buffers' capacity")
    dev = _lib.require_gpu(keys, values, *kbuf, *(vbuf or ()))
    keys = keys.contiguous()
    values = values.contiguous() if values is not None else None
    v3 = vbuf if values is not None else (None, None, None)
    rc = _lib.load().lcl_quantize_append(
        _lib.ptr(keys), _lib.ptr(values), _lib.dtype_code(keys.dtype), _lib.ptr(kbuf[0]), _lib.ptr(kbuf[1]),
        _lib.ptr(kbuf[2]), _lib.ptr(v3[0]), _lib.ptr(v3[1]), _lib.ptr(v3[2]), B, KVH, L, D, cap, prev,
        _round_code(round_mode), _lib.stream_of(dev))
    _lib.check(rc, "lcl_quantize_append")


def quantize(x: torch.Tensor, group_size: int = GROUP, bits: int = BITS, round_mode: Optional[str] = None):
    """``mx.quantize(x, group_size=64, bits=8)`` (affine) of a 16-bit (..., D) tensor: (words int32 (..., D/4),
    scales (..., D/64), biases (..., D/64)), bit-exact with MLX's closed form."""
    if group_size != GROUP or bits != BITS:
        raise ValueError("only group_size=64, bits=8 (the reference's 8-bit KV)")
    shape = x.shape
    D = shape[-1]
    x4 = x.reshape(1, 1, -1, D)
    out = _zeros_like_shape(1, 1, x4.shape[2], D, x.dtype, x.device, empty=True)
    quantize_into(x4, None, out, None, 0, round_mode)
    return tuple(a.reshape(*shape[:-1], a.shape[-1]) for a in out)


def dequantized(t, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``mx.dequantize(*t, group_size=64, bits=8)`` (locals/qkv.py:252-253): scale * code + bias in the scales'
    dtype (or ``dtype``)."""
    w, s, b = t
    if not _words_ok(w) or s.dtype not in (torch.float16, torch.bfloat16) or b.dtype != s.dtype:
        raise ValueError("dequantized takes an 8-bit (words, scales, biases) triple")
    D = w.shape[-1] * 4
    odt = dtype or s.dtype
    dev = _lib.require_gpu(w, s, b)
    w, s, b = w.contiguous(), s.contiguous(), b.contiguous()
    out = torch.empty(*w.shape[:-1], D, dtype=odt, device=dev)
    rows = w.numel() // w.shape[-1] if w.numel() else 0
    rc = _lib.load().lcl_dequantize(_lib.ptr(w), _lib.ptr(s), _lib.ptr(b), _lib.dtype_code(s.dtype), rows, D,
                                    _lib.ptr(out), _lib.dtype_code(odt), _lib.stream_of(dev))
    _lib.check(rc, "lcl_dequantize")
    return out


def quantized(cache) -> bool:
    """Whether ``cache`` keeps 8-bit keys and values (locals/qkv.py:256-257)."""
    return getattr(cache, "bits", None) == BITS and getattr(cache, "group_size", None) == GROUP


def attention(q, k, v, cache, scale: float, mask, sinks) -> torch.Tensor:
    """Append this step's ``k``/``v`` (B, KVH, L, HD) to the 8-bit ``cache``, then attend (locals/qkv.py:260-272):
    single-token decode (L == 1, head size 128) goes to ``attend``; a prompt chunk, span or tree (L > 1) goes to the
    masked kernel, which reads the 8-bit cache without a dequantized copy."""
    cache.update_and_fetch(k, v)
    return attend_cache(q, cache, scale, mask, sinks)


def attend_cache(q, cache, scale: float, mask, sinks) -> torch.Tensor:
    """The read half of ``attention`` (locals/qkv.py:264-272): ``q`` against a quantized cache that already holds
    this step's keys and values (written by ``update_and_fetch`` or ``qk_kernel.qk_norm_rope_append``)."""
    keys, values = cache.keys_and_values() if hasattr(cache, "keys_and_values") else cache.state
    if q.shape[2] == 1 and q.shape[3] == 128:
        start = getattr(cache, "left_padding", None)
        if start is None:
            start = torch.zeros((q.shape[0],), dtype=torch.int32, device=q.device)
        n = cache._idx if hasattr(cache, "_idx") else cache.offset
        return attend(q, cache.keys, cache.values, n, sinks, scale, start)
    from .fuse import attend_few_q8

    # the prompt branch hands the sinks over in the queries' dtype (locals/qkv.py:272: sinks.astype(q.dtype))
    return attend_few_q8(q, keys, values, scale, mask, None if sinks is None else sinks.to(q.dtype))


def _zeros_like_shape(B, H, n, D, dtype, device, empty=False):
    mk = torch.empty if empty else torch.zeros
    return (mk((B, H, n, D * BITS // 32), dtype=torch.int32, device=device),
            mk((B, H, n, D // GROUP), dtype=dtype, device=device),
            mk((B, H, n, D // GROUP), dtype=dtype, device=device))


def _zeros(B, H, n, D, dtype, device=None):
    """Empty 8-bit buffers (locals/qkv.py:275-277)."""
    return _zeros_like_shape(B, H, n, D, dtype, device)


def _head_dim(t):
    return t[0].shape[-1] * 32 // BITS


def _slice(t, lo=None, hi=None):
    return tuple(a[..., lo:hi, :] for a in t)


def create_causal_mask(N: int, offset: int = 0, window_size: Optional[int] = None, right_padding=None,
                       left_padding=None, device=None) -> torch.Tensor:
    """mlx-lm's ``create_causal_mask`` as BatchQuantizedKVCache.make_mask uses it (locals/qkv.py:367-368):
    (N, offset + N) bool, or (B, 1, N, offset + N) with per-row padding."""
    rinds = torch.arange(offset + N, device=device)
    linds = torch.arange(offset, offset + N, device=device)[:, None]
    mask = linds >= rinds[None]
    if window_size is not None:
        mask = mask & (linds < rinds[None] + window_size)
    if right_padding is not None:
        rp = torch.as_tensor(right_padding, device=device).reshape(-1, 1, 1, 1)
        mask = mask & (rinds < (offset + N) - rp)
    if left_padding is not None:
        lp = torch.as_tensor(left_padding, device=device).reshape(-1, 1, 1, 1)
        mask = mask & (lp <= rinds)
    return mask


def move_rows(rows, cap: int, like):
    """New (keys, values) triples of ``len(rows)`` rows and ``cap`` positions, built on the GPU by ``lcl_kv_gather``
    (one launch a triple).  ``rows[r] = (keys, values, row, shift, n, wrap)``: destination row r takes row ``row``
    of the source triples at position t - shift -- copied where it lies in [0, n), 0 elsewhere; with ``wrap``
    modulo n (a roll).  A source of None (or n == 0) gives a zero row.  ``like`` is a (keys, values) pair whose
    kv heads, head dims and dtypes the result takes."""
    lk, lv = like
    KVH, dt, dev = lk[0].shape[1], lk[1].dtype, lk[0].device
    out = []
    for which, ref in ((0, lk), (1, lv)):
        D = _head_dim(ref)
        dst = _zeros_like_shape(len(rows), KVH, cap, D, dt, dev, empty=True)
        n_ = len(rows)
        PP = ctypes.c_void_p * n_
        sw, ss, sb = PP(), PP(), PP()
        scap = (ctypes.c_longlong * n_)()
        sh, ln, wr = (ctypes.c_int * n_)(), (ctypes.c_int * n_)(), (ctypes.c_int * n_)()
        for r, (keys, values, row, shift, n, wrap) in enumerate(rows):
            src = keys if which == 0 else values
            n = int(n) if src is not None else 0
            if n:
                if src[0].device != dev or not all(a.is_contiguous() for a in src):
                    raise ValueError("row moves need contiguous buffers on the same GPU")
                sw[r], ss[r], sb[r] = (ctypes.c_void_p(a[row].data_ptr()) for a in src)
                scap[r] = src[0].shape[2]
            sh[r], ln[r], wr[r] = int(shift), n, int(bool(wrap))
        if n_ and cap:
            _lib.require_gpu(*dst)
            rc = _lib.load().lcl_kv_gather(_lib.ptr(dst[0]), _lib.ptr(dst[1]), _lib.ptr(dst[2]), n_, KVH, cap, D, sw,
                                           ss, sb, scap, sh, ln, wr, _lib.stream_of(dev))
            _lib.check(rc, "lcl_kv_gather")
        out.append(dst)
    return out[0], out[1]


def _grow(cache, B: int, H: int, prev: int, S: int, D: int, dtype, device, keep_aligned: bool = False) -> None:
    """Room for S positions at ``prev``: when the buffers are missing or too short, the kept positions are followed
    by ``ceil(S / step) * step`` zeroed ones.  The batch cache keeps exactly ``prev`` (locals/qkv.py:311-319), so its
    capacity becomes prev + ceil(S / step) * step; the one-request cache follows mlx-lm's QuantizedKVCache
    (``keep_aligned``): it drops the positions past ``prev`` only when ``prev`` is not a multiple of ``step``, and
    otherwise keeps its whole buffer."""
    if cache.keys is not None and prev + S <= cache.keys[0].shape[2]:
        return
    grow = (S + cache.step - 1) // cache.step * cache.step
    if cache.keys is None:
        keep = 0
    elif keep_aligned and prev % cache.step == 0:
        keep = cache.keys[0].shape[2]
    else:
        keep = prev
    nk = _zeros(B, H, keep + grow, D, dtype, device)
    nv = _zeros(B, H, keep + grow, D, dtype, device)
    if keep:
        for a, z in zip(cache.keys + cache.values, nk + nv):
            z[..., :keep, :] = a[..., :keep, :]
    cache.keys, cache.values = nk, nv


class QuantizedKVCache8:
    """Cache of one request in 8-bit triples, with mlx-lm's QuantizedKVCache bookkeeping at bits 8, group 64
    (locals/qkv.py:284-292).  Buffers grow in units of ``step`` positions; ``merge`` of several of these builds a
    BatchQuantizedKVCache."""

    step = 256
    bits, group_size = BITS, GROUP

    def __init__(self):
        self.keys = self.values = None
        self.offset = 0

    def _reserve(self, B: int, H: int, S: int, D: int, dtype, device) -> int:
        """Grow the buffers to hold S more positions and advance the offset; returns where the S positions go."""
        prev = self.offset
        _grow(self, B, H, prev, S, D, dtype, device, keep_aligned=True)
        self.offset += S
        return prev

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        B, H, S, D = keys.shape
        if values.shape != keys.shape:
            raise ValueError("values must match keys")
        prev = self._reserve(B, H, S, D, keys.dtype, keys.device)
        quantize_into(keys, values, self.keys, self.values, prev)
        return _slice(self.keys, None, self.offset), _slice(self.values, None, self.offset)

    @property
    def state(self):
        if self.keys is None:
            return self.keys, self.values
        return _slice(self.keys, None, self.offset), _slice(self.values, None, self.offset)

    @state.setter
    def state(self, v):
        self.keys, self.values = v
        self.offset = self.keys[0].shape[2]

    @property
    def meta_state(self):
        """(step, offset, group_size, bits) as strings, as mlx-lm's QuantizedKVCache records them in a snapshot."""
        return tuple(map(str, (self.step, self.offset, self.group_size, self.bits)))

    @meta_state.setter
    def meta_state(self, v):
        self.step, self.offset, self.group_size, self.bits = map(int, v)

    @classmethod
    def from_state(cls, state, meta_state):
        c = cls.__new__(cls)
        c.keys = c.values = None
        c.state = state
        c.meta_state = meta_state
        return c

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        return n

    def make_mask(self, N: int, return_array: bool = False, window_size: Optional[int] = None, **kwargs):
        if N == 1 and not return_array:
            return None
        if window_size is None and not return_array:
            return "causal"
        dev = self.keys[0].device if self.keys is not None else None
        return create_causal_mask(N, offset=self.offset, window_size=window_size, device=dev)

    def size(self):
        return self.offset

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        return sum(a.numel() * a.element_size() for a in self.keys + self.values)

    @classmethod
    def merge(cls, caches):
        return BatchQuantizedKVCache.merge(caches)


class BatchQuantizedKVCache:
    """Cache of a batch of requests in 8-bit triples (locals/qkv.py:295-452), kept as mlx-lm's BatchKVCache keeps
    its rows: rows are aligned on the right with ``left_padding`` blank positions in front, all rows share the write
    position ``_idx`` (a host int), and ``offset`` (int32 device tensor, like ``left_padding``) is each row's own
    token count.  Growth appends whole ``step``s after the used positions."""

    step = 256
    bits, group_size = BITS, GROUP

    def __init__(self, left_padding: List[int], device=None):
        self.keys = self.values = None
        self.left_padding = torch.as_tensor(left_padding, dtype=torch.int32, device=device)
        self.offset = -self.left_padding.clone()
        self._idx = 0
        self._right_padding = None

    def _dev(self):
        return self.left_padding.device

    def _reserve(self, B: int, H: int, S: int, D: int, dtype, device) -> int:
        """Grow the buffers to hold S more positions and advance ``offset`` and ``_idx``; returns where the S
        positions go (the shared buffer index)."""
        prev = self._idx
        if self.left_padding.device != device:
            self.left_padding = self.left_padding.to(device)
            self.offset = self.offset.to(device)
        _grow(self, B, H, prev, S, D, dtype, device)
        self.offset = self.offset + S
        self._idx += S
        return prev

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        B, H, S, D = keys.shape
        if values.shape != keys.shape:
            raise ValueError("values must match keys")
        prev = self._reserve(B, H, S, D, keys.dtype, keys.device)
        quantize_into(keys, values, self.keys, self.values, prev)
        return self.keys_and_values()

    def keys_and_values(self):
        return _slice(self.keys, None, self._idx), _slice(self.values, None, self._idx)

    def prepare(self, *, left_padding=None, lengths=None, right_padding=None):
        if left_padding is not None:
            if self.keys is not None:
                raise ValueError("left padding can only be added to an empty cache")
            lp = torch.as_tensor(left_padding, dtype=torch.int32, device=self._dev())
            self.left_padding = self.left_padding + lp
            self.offset = self.offset - lp
        if right_padding is not None and max(right_padding) > 0:
            self._right_padding = [int(x) for x in right_padding]  # host values: the roll's shifts

    def finalize(self):
        """Rows prepared with right padding are rolled right by it (mlx-lm's dynamic_roll along the positions), so
        their padding moves to the left (locals/qkv.py:340-346)."""
        if self._right_padding is not None:
            p = self._right_padding
            if self.keys is not None:
                n = self.keys[0].shape[2]
                self.keys, self.values = move_rows([(self.keys, self.values, b, p[b], n, True) for b in range(len(p))],
                                                   n, (self.keys, self.values))
            pt = torch.as_tensor(p, dtype=torch.int32, device=self._dev())
            self.offset = self.offset - pt
            self.left_padding = self.left_padding + pt
            self._right_padding = None

    @property
    def state(self):
        return self.keys, self.values, self.offset, self.left_padding, self._idx

    @state.setter
    def state(self, v):
        self.keys, self.values, self.offset, self.left_padding, self._idx = v

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def make_mask(self, N: int, return_array: bool = False, **kwargs):
        return create_causal_mask(N, offset=self._idx, left_padding=self.left_padding, device=self._dev(), **kwargs)

    def filter(self, batch_indices):
        """Keep the rows ``batch_indices`` (in that order) and drop the left padding they all share
        (locals/qkv.py:370-380): one gather of the kept rows shifted left by that padding."""
        keep = [int(i) for i in (batch_indices.tolist() if isinstance(batch_indices, torch.Tensor) else batch_indices)]
        idx = torch.as_tensor(keep, device=self._dev(), dtype=torch.long)
        self.offset = self.offset[idx]
        self.left_padding = self.left_padding[idx]
        drop = int(self.left_padding.min().item()) if self.left_padding.numel() else 0
        drop = max(drop, 0)
        if self.keys is not None:
            n = self.keys[0].shape[2]
            self.keys, self.values = move_rows([(self.keys, self.values, i, -drop, n, False) for i in keep], n - drop,
                                               (self.keys, self.values))
        if drop > 0:
            self._idx -= drop
            self.left_padding = self.left_padding - drop

    def extend(self, other):
        if self.keys is None and other.keys is None:
            self.left_padding = torch.cat([self.left_padding, other.left_padding.to(self._dev())])
            self.offset = torch.cat([self.offset, other.offset.to(self._dev())])
            return
        ref = self if self.keys is not None else other
        dev = ref.keys[0].device
        max_idx = max(self._idx, other._idx)
        size = max(c.keys[0].shape[2] for c in (self, other) if c.keys is not None)
        # each side's rows move right by max_idx - _idx; what passes `size` is cut, the rest is zero-filled
        # (locals/qkv.py:388-401)
        rows = []
        for c in (self, other):
            left = max_idx - c._idx
            n = min(c.keys[0].shape[2], size - left) if c.keys is not None else 0
            rows += [(c.keys, c.values, b, left, n, False) for b in range(c.offset.shape[0])]
        self.keys, self.values = move_rows(rows, size, (ref.keys, ref.values))
        self.offset = torch.cat([self.offset.to(dev), other.offset.to(dev)])
        self.left_padding = torch.cat([self.left_padding.to(dev) + (max_idx - self._idx),
                                       other.left_padding.to(dev) + (max_idx - other._idx)])
        self._idx = max_idx

    def extract(self, idx):
        """Row ``idx`` as a one-request cache holding exactly its positions [left_padding, _idx)
        (locals/qkv.py:408-415)."""
        c = QuantizedKVCache8()
        p = int(self.left_padding[idx].item())
        c.keys, c.values = move_rows([(self.keys, self.values, int(idx), -p, self._idx, False)], self._idx - p,
                                     (self.keys, self.values))
        c.offset = self._idx - p
        return c

    @classmethod
    def merge(cls, caches):
        lengths = [c.offset if c.keys is not None else 0 for c in caches]
        L = max(lengths)
        ref = next((c for c in caches if c.keys is not None), None)
        dev = ref.keys[0].device if ref is not None else None
        out = cls([L - n for n in lengths], device=dev)
        if L == 0:
            return out
        # request i's first n_i positions, right-aligned in L (locals/qkv.py:419-430)
        out.keys, out.values = move_rows([(c.keys, c.values, 0, L - n, n, False) for n, c in zip(lengths, caches)],
                                         L, (ref.keys, ref.values))
        out._idx = L
        out.offset = out.offset + L
        return out

    def size(self):
        return self._idx

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        return sum(a.numel() * a.element_size() for a in self.keys + self.values)


def wants_8bit(model) -> bool:
    """Whether full-attention layers keep 8-bit keys and values: LOCALS_KV_BITS=8 (locals/qkv.py:455-460)."""
    return os.environ.get("LOCALS_KV_BITS", "16") == "8"


def opt_in(model) -> Optional[bool]:
    """Full-attention layers of a model in QuantizedKVCache8 (its make_cache replaced); True if done
    (locals/qkv.py:463-472).  Sliding-window layers keep whatever cache ``model.make_cache`` made for them."""
    if not wants_8bit(model):
        return False
    layers = model.layers
    base = getattr(model, "make_cache", None)

    def make_cache():
        made = base() if base is not None else [None] * len(layers)
        return [c if getattr(l, "use_sliding", False) else QuantizedKVCache8() for l, c in zip(layers, made)]

    model.make_cache = make_cache
    return True


# ---- prompt-cache snapshots (the reference's DiskPromptCache, locals/hybrid_batch.py:332-455, writes them with
# mlx-lm's save_prompt_cache / load_prompt_cache): one safetensors file, each layer cache's ``state`` arrays under
# "<layer>.<i>.<j>" and, in the metadata, its ``meta_state`` under "0.<layer>.<k>", the caller's metadata under
# "1.<key>" and its class name under "2.<layer>".  The 8-bit words are stored as uint32, as MLX holds them.

_SNAPSHOT_CLASSES = {"QuantizedKVCache8": QuantizedKVCache8}


def _flatten(tree, prefix=""):
    if isinstance(tree, (list, tuple)):
        out = []
        for i, t in enumerate(tree):
            out += _flatten(t, f"{prefix}.{i}" if prefix else str(i))
        return out
    if isinstance(tree, dict):
        out = []
        for k, t in tree.items():
            out += _flatten(t, f"{prefix}.{k}" if prefix else str(k))
        return out
    return [(prefix, tree)]


def _unflatten(items):
    """The nested lists of _flatten's numeric paths (and dicts of the others)."""
    root: dict = {}
    for key, val in items:
        node = root
        parts = key.split(".")
        for part in parts[:-1]:
            node = node.setdefault(part, {})
        node[parts[-1]] = val

    def build(node):
        if not isinstance(node, dict):
            return node
        if node and all(k.isdigit() for k in node):  # a list; an empty one leaves no key behind
            return [build(node.get(str(i), {})) for i in range(max(int(k) for k in node) + 1)]
        return {k: build(v) for k, v in node.items()}

    return build(root)


def save_prompt_cache(path: str, caches, metadata: Optional[dict] = None) -> None:
    """Write the layer caches ``caches`` (QuantizedKVCache8) to ``path`` in mlx-lm's snapshot layout."""
    from safetensors.torch import save_file

    arrays = {}
    for key, t in _flatten([c.state for c in caches]):
        t = t.detach().contiguous().cpu()
        if t.dtype == torch.int32:  # 8-bit words
            t = t.view(torch.uint32)
        arrays[key] = t
    meta = dict(_flatten([[c.meta_state for c in caches], metadata or {}, [type(c).__name__ for c in caches]]))
    save_file(arrays, path, metadata={k: str(v) for k, v in meta.items()})


def load_prompt_cache(path: str, device=None, return_metadata: bool = False):
    """The layer caches of a snapshot written by ``save_prompt_cache`` (or mlx-lm's, for 8-bit layers), on
    ``device`` (default cuda:0)."""
    from safetensors import safe_open

    dev = torch.device(device) if device is not None else torch.device("cuda", 0)
    with safe_open(path, "pt") as f:
        meta = f.metadata() or {}
        arrays = []
        for k in f.keys():
            t = f.get_tensor(k)
            if t.dtype == getattr(torch, "uint32", None):
                t = t.view(torch.int32)
            arrays.append((k, t.to(dev)))
    state = _unflatten(arrays)
    info, user_meta, classes = (_unflatten(list(meta.items())) + [None, None, None])[:3]
    caches = []
    for i, name in enumerate(classes):
        cls = _SNAPSHOT_CLASSES.get(name)
        if cls is None:
            raise ValueError(f"snapshot layer {i}: cache class {name!r} is not one of {sorted(_SNAPSHOT_CLASSES)}")
        st = state[i]
        caches.append(cls.from_state((tuple(st[0]), tuple(st[1])), info[i]))
    if return_metadata:
        return caches, (user_meta if isinstance(user_meta, dict) else {})
    return caches
