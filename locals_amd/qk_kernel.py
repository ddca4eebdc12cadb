"""Per-head q/k RMS norms and RoPE in one launch (``locals/qk_kernel.py`` on the MI355X kernel ``lcl_qk_norm_rope``).

``qk_norm_rope(qkv, attn, offset)`` and ``fits(attn, qkv)`` keep the reference's names, arguments and results
(locals/qk_kernel.py:74-109): ``attn`` is any object with the attention layer's attributes (``n_heads``,
``n_kv_heads``, ``head_dim``, ``q_norm``/``k_norm`` with ``weight`` and ``eps``, ``rope`` None or with ``base``,
``dims``, ``traditional`` and optionally ``scale``).

``qk_norm_rope_append(qkv, attn, cache)`` is the fused form of the reference's next step
(locals/fuse.py:80-83): it returns q and stores the normed/rotated k and the raw v straight into an 8-bit
cache, as ``cache.update_and_fetch(k, v)`` does after ``qk_norm_rope``, in the same launch.
"""

from __future__ import annotations

import math
import os

import torch

from . import _lib
from .qkv import _round_code, quantized

USE_QK_KERNEL = os.environ.get("LOCALS_QK_KERNEL", "1") != "0"

HEAD_DIMS = tuple(128 * k for k in range(1, 9))  # the head sizes the kernel is built for: multiples of 128 to 1024


def fits(attn, qkv: torch.Tensor) -> bool:
    """True when the fused kernel can take this layer (the predicate of locals/qk_kernel.py:74-82): fp16 or bf16
    activations with norm weights of the same dtype, a head size the kernel handles (``HEAD_DIMS``), one eps shared
    by the q and k norms, and either no RoPE or a non-traditional RoPE of unit scale over the full head."""
    hd = attn.head_dim
    rope = attn.rope
    return (USE_QK_KERNEL and qkv.dtype in (torch.bfloat16, torch.float16) and hd in HEAD_DIMS
            and attn.q_norm.weight.dtype == qkv.dtype and attn.k_norm.weight.dtype == qkv.dtype
            and abs(attn.q_norm.eps - attn.k_norm.eps) < 1e-12
            and (rope is None or (not rope.traditional and rope.dims == hd and getattr(rope, "scale", 1.0) == 1.0)))


def _offsets(offset, B: int, dev: torch.device):
    """(int32 device tensor, per_row) as locals/qk_kernel.py:99-100."""
    if isinstance(offset, torch.Tensor):
        o = offset.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
        if o.numel() not in (1, B):
            raise ValueError("offset must be an int or one value a row")
        return o, o.numel() > 1
    return torch.full((1,), int(offset), dtype=torch.int32, device=dev), False


def _common(qkv: torch.Tensor, attn):
    if qkv.dim() != 3:
        raise ValueError("qkv must be (B, L, (H + 2 KV) * head_dim)")
    B, L, W = qkv.shape
    H, KV, HD = int(attn.n_heads), int(attn.n_kv_heads), int(attn.head_dim)
    if W != (H + 2 * KV) * HD:
        raise ValueError("qkv's last axis is not (H + 2 KV) * head_dim")
    if not fits(attn, qkv):
        raise ValueError("layer not covered by qk_norm_rope (see fits)")
    qw, kw = attn.q_norm.weight, attn.k_norm.weight
    if qw.numel() != HD or kw.numel() != HD:
        raise ValueError("norm weights must have head_dim entries")
    dev = _lib.require_gpu(qkv, qw, kw)
    base = attn.rope.base if attn.rope is not None else 10000.0
    return (B, L, H, KV, HD, dev, qkv.contiguous(), qw.contiguous(), kw.contiguous(), float(attn.q_norm.eps),
            float(math.log2(base)), attn.rope is not None)


def qk_norm_rope(qkv: torch.Tensor, attn, offset):
    """Split the fused projection ``qkv`` (B, L, (H + 2 KV) * HD) into q (B, H, L, HD), k and v (B, KV, L, HD).
    q and k get their per-head RMS norm and, when the layer has ``attn.rope``, RoPE at positions ``offset + l``;
    ``offset`` is an int or a per-row tensor (a batch cache's ``offset``).  v is a fresh tensor, not a view of
    ``qkv`` (locals/qk_kernel.py:85-109)."""
    B, L, H, KV, HD, dev, x, qw, kw, eps, lb, rope = _common(qkv, attn)
    offs, per_row = _offsets(offset, B, dev)
    q = torch.empty((B, H, L, HD), dtype=qkv.dtype, device=dev)
    k = torch.empty((B, KV, L, HD), dtype=qkv.dtype, device=dev)
    v = torch.empty((B, KV, L, HD), dtype=qkv.dtype, device=dev)
    P = _lib.ptr
    rc = _lib.load().lcl_qk_norm_rope(P(x), _lib.dtype_code(qkv.dtype), P(qw), P(kw), P(offs), int(per_row), eps, lb,
                                      int(rope), B, L, H, KV, HD, P(q), P(k), P(v), _lib.stream_of(dev))
    _lib.check(rc, "lcl_qk_norm_rope")
    return q, k, v


def qk_norm_rope_append(qkv: torch.Tensor, attn, cache, round_mode=None) -> torch.Tensor:
    """q of ``qk_norm_rope(qkv, attn, cache.offset)``, with its k and v stored into the 8-bit ``cache`` exactly as
    ``cache.update_and_fetch(k, v)`` stores them (locals/fuse.py:80-83, locals/qkv.py:309-326), in one launch.
    The cache's offset (and ``_idx``) advance by L as with ``update_and_fetch``."""
    if not quantized(cache):
        raise ValueError("qk_norm_rope_append writes an 8-bit cache (BatchQuantizedKVCache / QuantizedKVCache8)")
    B, L, H, KV, HD, dev, x, qw, kw, eps, lb, rope = _common(qkv, attn)
    offs, per_row = _offsets(cache.offset, B, dev)  # positions before this step's keys
    prev = cache._reserve(B, KV, L, HD, qkv.dtype, dev)
    kb, vb = cache.keys, cache.values
    if kb[0].shape[:2] != (B, KV) or kb[1].dtype != qkv.dtype:
        raise ValueError("the cache's buffers do not match qkv")
    q = torch.empty((B, H, L, HD), dtype=qkv.dtype, device=dev)
    P = _lib.ptr
    rc = _lib.load().lcl_qk_norm_rope_append(
        P(x), _lib.dtype_code(qkv.dtype), P(qw), P(kw), P(offs), int(per_row), eps, lb, int(rope), B, L, H, KV, HD,
        P(q), P(kb[0]), P(kb[1]), P(kb[2]), P(vb[0]), P(vb[1]), P(vb[2]), kb[0].shape[2], prev,
        _round_code(round_mode), _lib.stream_of(dev))
    _lib.check(rc, "lcl_qk_norm_rope_append")
    return q
