"""``ragged_attention`` on the MI355X: decode attention over 16-bit K/V for a packed batch in a single launch.

The call surface is the reference's (locals/attention.py:200-224).  Each query row names the KV slot it reads
(``slots``) and how many of that slot's leading keys it sees (``nkeys``); a multi-token segment gets its causal
mask by giving each of its rows one more key than the row before.  K and V are slot-major buffers
(n_slots, Hkv, cap, D).  The work runs in ``lcl_ragged_attention``: a split-K pass 1 on MFMA and a log-sum-exp
join.
"""

from __future__ import annotations

import torch

from . import _lib
from .qkv import workspace_bytes  # noqa: F401  (same workspace rule)

BLOCK = 0  # keys a pass-1 workgroup reads (a multiple of 64); 0: the library's choice


def ragged_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, slots: torch.Tensor,
                     nkeys: torch.Tensor, scale) -> torch.Tensor:
    """Attention of R query rows (q (R, H, D)) over slot-major K/V (n_slots, Hkv, cap, D): row r reads slot
    ``slots[r]``, keys [0, ``nkeys[r]``).  ``scale`` is a float or a (1,) float32 tensor (a GPU tensor is read on
    the device).  Returns (R, H, D) in q's dtype; a row whose ``nkeys`` is 0 comes back as zeros
    (locals/attention.py:200-224)."""
    if q.dim() != 3 or keys.dim() != 4 or values.shape != keys.shape:
        raise ValueError("q (R, H, D), keys/values (n_slots, Hkv, cap, D) expected")
    R, H, D = q.shape
    n_slots, Hkv, cap, D2 = keys.shape
    if D2 != D:
        raise ValueError("head dims differ")
    if D % 32 or D > 512 or H % Hkv:
        raise ValueError("D must be a multiple of 32 (at most 512) and H a multiple of Hkv (locals/attention.py "
                         "preconditions)")
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
