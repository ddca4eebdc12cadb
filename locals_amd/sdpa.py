"""MLX's ``scaled_dot_product_attention`` contract on the MI355X kernels, for the reference's multi-query calls.

The reference routes chunked prefill, spans, packed segments and tree verification through
``mx.fast.scaled_dot_product_attention(q, k, v, scale=, mask=, sinks=)`` (locals/fuse.py:139,144;
locals/treedec.py:79; locals/packed.py:141; locals/tree.py:95), over K/V dequantized from the 8-bit cache for
Flint's full-attention layers (locals/qkv.py:270-272).  ``scaled_dot_product_attention`` here takes the same
arguments and, in place of dequantized tensors, the 8-bit (words, scales, biases) triples themselves (read in
place, dequantized in LDS by ``lcl_sdpa``).

Masks: ``None``; ``"causal"`` (the last query aligned with the last key, locals/fuse.py:131-137); a boolean tensor
broadcastable to (B, H, L, N); or a ``TreeMask`` (the prefix visible to every new token, ancestor-only within the
new tokens, locals/treedec.py:56-67) which the kernel reads as one 64-bit word a query; or a ``WindowMask`` (the
sliding-window layers' mask: causal within the last W keys, locals/fuse.py:113-125).  ``sinks`` (H,) are logits
in the denominator only.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib
from .qkv import _words_ok

BLOCK = 0  # keys a pass-1 workgroup reads (a multiple of 64); 0: the library's choice
# 8-bit K/V with many row blocks per (row, KV head): give the library room to dequantize K and V once and run the
# 16-bit kernel (the reference's own prompt path dequantizes first too); False keeps the fused 8-bit kernel
DEQUANTIZE_FIRST = True

MASK_NONE, MASK_CAUSAL, MASK_TREE, MASK_DENSE, MASK_WINDOW = 0, 1, 2, 3, 4


class WindowMask:
    """The mask a sliding-window layer gives a prompt chunk (mlx-lm's ``create_causal_mask(..., window_size=W)``
    for a ``RotatingKVCache``, locals/models/flint.py:157,197): query i of L, at position N - L + i, sees the keys
    (N - L + i - W, N - L + i].  The reference computes it as bands of queries over the keys each band reaches
    (locals/fuse.py:113-125, locals/models/flint_streamed.py:114-128); the kernel reads each workgroup's band."""

    def __init__(self, window: int):
        if int(window) < 1:
            raise ValueError("a window holds at least the query's own key")
        self.window = int(window)


class TreeMask:
    """Ancestor-only attention among the last L keys, the earlier keys visible to all: ``bits[b, i]`` has bit d set
    iff new token i sees new token d (L <= 64).  ``bits`` is (B, L) or (1, L) int64 on the GPU."""

    def __init__(self, bits: torch.Tensor):
        if bits.dim() != 2 or bits.shape[1] > 64:
            raise ValueError("TreeMask bits must be (B or 1, L <= 64)")
        self.bits = bits.to(torch.int64).contiguous()

    @property
    def L(self) -> int:
        return self.bits.shape[1]

    @classmethod
    def from_local(cls, local, device=None) -> "TreeMask":
        """From a (L, L) or (B, L, L) boolean "token i sees token j" matrix over the new tokens."""
        m = torch.as_tensor(local, dtype=torch.bool)
        if m.dim() == 2:
            m = m[None]
        L = m.shape[-1]
        if L > 64 or m.shape[-2] != L:
            raise ValueError("tree masks cover at most 64 new tokens (an L x L matrix)")
        w = torch.zeros(m.shape[:2], dtype=torch.int64)
        for d in range(L):
            bit = (1 << d) if d < 63 else -(1 << 63)
            w |= m[..., d].to(torch.int64) * bit
        return cls(w.to(device) if device is not None else w)

    @classmethod
    def from_parents(cls, parents: Sequence[int], device=None) -> "TreeMask":
        """From a tree in preorder: parents[i] < i, -1 for a root; token i sees itself and its ancestors."""
        L = len(parents)
        local = torch.zeros(L, L, dtype=torch.bool)
        for i in range(L):
            j = i
            while j >= 0:
                local[i, j] = True
                j = int(parents[j])
        return cls.from_local(local, device)

    @classmethod
    def from_branches(cls, br: Sequence[int], device=None) -> "TreeMask":
        """The reference's layout (locals/treedec.py:56-67, locals/packed.py:176-181): token i sees token j iff
        j <= i and (same branch or j on the main path, br[j] < 0)."""
        b = torch.as_tensor(list(br))
        L = b.numel()
        qi, kj = torch.arange(L)[:, None], torch.arange(L)[None, :]
        local = (kj <= qi) & ((b[:, None] == b[None, :]) | (b[None, :] < 0))
        return cls.from_local(local, device)


def _kv_view(t: torch.Tensor, name: str):
    """(tensor, cap): a (B, KVH, N, D) tensor that is the first N positions of a contiguous (B, KVH, cap, D) buffer
    (a cache's ``keys_and_values()`` slice) is read in place."""
    if t.dim() != 4:
        raise ValueError(f"{name} must be (B, KVH, N, .)")
    B, KVH, N, D = t.shape
    st = t.stride()
    if st[3] != 1 or st[2] != D or st[1] % D or st[0] != KVH * st[1] or st[1] // D < N:
        t = t.contiguous()
        st = t.stride()
    return t, st[1] // D


def scaled_dot_product_attention(q: torch.Tensor, k, v, *, scale: float, mask=None,
                                 sinks: Optional[torch.Tensor] = None, start: Optional[torch.Tensor] = None):
    """Attention of ``q`` (B, H, L, D) over ``k``/``v`` -- (B, KVH, N, D) fp16/bf16 tensors, or 8-bit
    (words, scales, biases) triples of N positions -- with MLX's mask and sink semantics.  ``start`` (B,) masks the
    keys before start[b] (a left-padded batch).  Returns (B, H, L, D) in q's dtype.  D = 128 runs on the tiled MFMA
    kernels; other head sizes (a multiple of 16 up to 512 for 16-bit K/V, of 64 for 8-bit) on a general kernel."""
    if q.dim() != 4:
        raise ValueError("q must be (B, H, L, D)")
    B, H, L, D = q.shape
    q8 = isinstance(k, (tuple, list))
    if not (0 < D <= 512 and D % (64 if q8 else 16) == 0):
        raise ValueError(f"head_dim {D} not supported (a multiple of {64 if q8 else 16} up to 512)")
    if q8:
        kt = tuple(_kv_view(a, "keys") for a in k)
        vt = tuple(_kv_view(a, "values") for a in v)
        kw, ks, kb = (a for a, _ in kt)
        vw, vs, vb = (a for a, _ in vt)
        if not _words_ok(kw) or kw.shape[3] * 4 != D or ks.shape[3] * 64 != D:
            raise ValueError("8-bit keys must be (B, KVH, N, D / 4) words with scales/biases (B, KVH, N, D / 64)")
        caps = {c for _, c in kt + vt}
        if len(caps) != 1:
            raise ValueError("8-bit buffers of different capacities")
        cap = caps.pop()
        KVH, N = kw.shape[1], kw.shape[2]
        kvdt = ks.dtype
        if ks.dtype not in (torch.float16, torch.bfloat16) or kb.dtype != ks.dtype:
            raise ValueError("8-bit scales/biases must be float16 or bfloat16")
        kf = vf = None
        tensors = (kw, ks, kb, vw, vs, vb)
        fmt = 0
    else:
        kf, cap = _kv_view(k, "keys")
        vf, capv = _kv_view(v, "values")
        if capv != cap or vf.shape != kf.shape:
            raise ValueError("keys and values differ in shape or capacity")
        if kf.dtype not in (torch.float16, torch.bfloat16) or vf.dtype != kf.dtype:
            raise ValueError("keys/values must be float16 or bfloat16")
        KVH, N = kf.shape[1], kf.shape[2]
        kvdt = kf.dtype
        kw = ks = kb = vw = vs = vb = None
        tensors = (kf, vf)
        fmt = 1
    if kw is not None and (kw.shape[:3] != vw.shape[:3] or ks.dtype != vs.dtype):
        raise ValueError("keys and values buffers differ")
    if H % KVH or (kw is not None and kw.shape[0] != B) or (kf is not None and kf.shape[0] != B):
        raise ValueError("q and k/v disagree on rows or heads")
    dev = _lib.require_gpu(q, *tensors, sinks, start)
    q = q.contiguous()
    mk, window, tree, tree_bs, dense, strides = MASK_NONE, 0, None, 0, None, (0, 0, 0, 0)
    if mask is None:
        pass
    elif isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask {mask!r}")
        if L > N:
            raise ValueError("a causal mask needs at least as many keys as queries")
        mk = MASK_CAUSAL
    elif isinstance(mask, TreeMask):
        if mask.L != L or mask.bits.shape[0] not in (1, B) or L > N:
            raise ValueError("TreeMask must cover the L queries, one row or one for all")
        mk, tree = MASK_TREE, mask.bits.to(dev)
        tree_bs = L if mask.bits.shape[0] == B and B > 1 else 0
    elif isinstance(mask, WindowMask):
        if L > N:
            raise ValueError("a window mask needs at least as many keys as queries")
        mk, window = MASK_WINDOW, mask.window
    elif isinstance(mask, torch.Tensor):
        if mask.dtype != torch.bool:
            raise ValueError("array masks must be boolean (additive masks are not part of the reference's calls)")
        m = mask
        while m.dim() < 4:
            m = m[None]
        m = m.to(dev).expand(B, H, L, N)
        dense = m.view(torch.uint8)
        strides = tuple(dense.stride())
        mk = MASK_DENSE
    else:
        raise ValueError("mask must be None, 'causal', a boolean tensor, a TreeMask or a WindowMask")
    sk = None if sinks is None else sinks.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if sk is not None and sk.numel() != H:
        raise ValueError("sinks must have one entry a query head")
    st = None if start is None else start.to(device=dev, dtype=torch.int32).contiguous()
    lib = _lib.load()
    blk = int(BLOCK)
    if DEQUANTIZE_FIRST:
        nbytes = int(lib.lcl_sdpa_workspace_bytes_kv(B, H, KVH, L, N, cap, blk, fmt, mk))
    else:
        nbytes = int(lib.lcl_sdpa_workspace_bytes(B, H, L, N, blk))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    out = torch.empty((B, H, L, D), dtype=q.dtype, device=dev)
    P = _lib.ptr
    rc = lib.lcl_sdpa(P(q), _lib.dtype_code(q.dtype), fmt, P(kw), P(ks), P(kb), P(vw), P(vs), P(vb), P(kf), P(vf),
                      _lib.dtype_code(kvdt), P(st), mk, window, P(tree), tree_bs, P(dense), *strides, P(sk), float(scale),
                      B, H, KVH, L, N, D, cap, blk, P(out), P(ws), nbytes, _lib.stream_of(dev))
    _lib.check(rc, "lcl_sdpa")
    return out
