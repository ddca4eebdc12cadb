"""Ragged batch decode attention: one launch for all rows of all requests -- drop-in for ``locals/attention.py``.

Row r of the packed batch belongs to KV slot ``slots[r]`` and may see the first ``nkeys[r]`` keys of that slot
(its prefix plus the earlier new tokens of its own segment, which gives the causal mask for multi-token segments);
K/V live in slot-major buffers (n_slots, n_kv_heads, cap, D) (locals/attention.py:1-8).  Backed by
``lcl_ragged_attention`` (split-K flash decode on MFMA over fp16/bf16 K/V).
"""

from __future__ import annotations

import torch

from . import _lib
from .qkv import workspace_bytes  # noqa: F401  (same workspace rule)

BLOCK = 0  # keys a pass-1 workgroup reads (a multiple of 64); 0: the library's choice


def ragged_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, slots: torch.Tensor,
                     nkeys: torch.Tensor, scale) -> torch.Tensor:
    """q: (R, H, D); keys/values: (n_slots, Hkv, cap, D); slots/nkeys: (R,) int32; scale: (1,) float32 tensor or a
    float.  Returns (R, H, D) (locals/attention.py:200-224).  A row with no keys gives 0."""
    if q.dim() != 3 or keys.dim() != 4 or values.shape != keys.shape:
        raise ValueError("q (R, H, D), keys/values (n_slots, Hkv, cap, D) expected")
    R, H, D = q.shape
    n_slots, Hkv, cap, D2 = keys.shape
    if D2 != D:
        raise ValueError("head dims differ")
    if D % 32 or H % Hkv:
        raise ValueError("D must be a multiple of 32 and H a multiple of Hkv (locals/attention.py preconditions)")
    if keys.dtype not in (torch.float16, torch.bfloat16) or values.dtype != keys.dtype:
        raise ValueError("keys/values must be float16 or bfloat16")
    if slots.numel() != R or nkeys.numel() != R:
        raise ValueError("slots and nkeys need one entry a row")
    dev = _lib.require_gpu(q, keys, values, slots, nkeys)
    q, keys, values = q.contiguous(), keys.contiguous(), values.contiguous()
    sl = slots.to(device=dev, dtype=torch.int32).contiguous()
    nk = nkeys.to(device=dev, dtype=torch.int32).contiguous()
    scale_dev = None
    if isinstance(scale, torch.Tensor):
        if scale.is_cuda:
            scale_dev = scale.to(device=dev, dtype=torch.float32).reshape(-1)[:1].contiguous()
            scale_f = 0.0
        else:
            scale_f = float(scale.reshape(-1)[0])
    else:
        scale_f = float(scale)
    lib = _lib.load()
    blk = int(BLOCK)
    nbytes = int(lib.lcl_decode_workspace_bytes(R, H, cap, blk))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    out = torch.empty((R, H, D), dtype=q.dtype, device=dev)
    rc = lib.lcl_ragged_attention(_lib.ptr(q), _lib.dtype_code(q.dtype), _lib.ptr(keys), _lib.ptr(values),
                                  _lib.dtype_code(keys.dtype), _lib.ptr(sl), _lib.ptr(nk), scale_f, _lib.ptr(scale_dev),
                                  R, H, n_slots, Hkv, D, cap, blk, _lib.ptr(out), _lib.ptr(ws), nbytes,
                                  _lib.stream_of(dev))
    _lib.check(rc, "lcl_ragged_attention")
    return out
