"""Seeded synthetic inputs shared by the tests and the bench (numpy PCG64; the same arrays feed oracle and kernel)."""

from __future__ import annotations

import numpy as np

from oracle import quant


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal16(g: np.random.Generator, shape, scale: float = 1.0, dtype: str = "float16"):
    x = (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)
    return quant.from_f32(x, dtype)


def q8_cache(g: np.random.Generator, B, KVH, cap, HD=128, kscale=1.0, vscale=1.0, dtype="float16"):
    """K/V drawn N(0, scale^2) in dtype and quantized with MLX's affine 8-bit (group 64)."""
    K = normal16(g, (B, KVH, cap, HD), kscale, dtype)
    V = normal16(g, (B, KVH, cap, HD), vscale, dtype)
    return quant.quantize(K, dtype), quant.quantize(V, dtype)


def to_torch(a, dev, dtype: str = "float16"):
    """numpy array -> torch tensor on dev; uint32 words as int32, bf16 bit patterns as bfloat16."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(dev)
    if a.dtype == np.uint16 and dtype == "bfloat16":
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(a).to(dev)


def triple_to_torch(t, dev, dtype="float16"):
    return tuple(to_torch(x, dev, dtype) for x in t)
