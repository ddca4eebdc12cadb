"""Seeded synthetic inputs shared by the tests and the bench (numpy PCG64; the same arrays feed oracle and kernel)."""

from __future__ import annotations

import numpy as np

from oracle import quant
from oracle.quant import from_f32, to_f32


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


def peaked_inputs(g: np.random.Generator, B, H, KVH, L, cap, lo, hi, scale=1 / np.sqrt(128), gap=(6.0, 14.0),
                  n_dom=1, tail=0.5, v_offset=(0.75, 1.5), dtype="float16", HD=128):
    """Queries and 8-bit K/V whose softmax is peaked: per (row b, kv head) a direction u shared by the group's
    queries (q = 0.6 u + 0.8 N(0, 1) per head and query), ``n_dom`` keys in [lo[b], hi[b]) equal to a u with a set so
    their logit is ``gap`` nats (U[gap]) above the rest, whose keys are N(0, tail^2) (logits ~ N(0, tail^2)), i.e.
    one or a few dominant keys over a tail ~9..20 log2 below.  V = N(0, 0.5^2) + a per-(row, kv head, 64-dim group)
    offset of random sign and magnitude U[v_offset], so each group's MLX scale has one sign (|max| > |min|) and the
    rounding of the V weights cannot cancel; |V| stays below 4, where an fp16 output's own rounding (<= 2^-10) leaves
    room under the 2e-3 bar.  Returns (q (B, H, L, HD), K triple, V triple, dominant positions (B, KVH, n_dom))."""
    G = H // KVH
    u = g.standard_normal((B, KVH, HD)).astype(np.float32)
    u *= np.float32(np.sqrt(HD)) / np.linalg.norm(u, axis=-1, keepdims=True)
    qf = (0.6 * u[:, :, None, None, :] + 0.8 * g.standard_normal((B, KVH, G, L, HD))).astype(np.float32)
    q = from_f32(qf.reshape(B, H, L, HD), dtype)
    qv = to_f32(q, dtype).reshape(B, KVH, G, L, HD).astype(np.float64)
    kf = (tail * g.standard_normal((B, KVH, cap, HD))).astype(np.float32)
    dom = np.zeros((B, KVH, n_dom), dtype=np.int64)
    for b in range(B):
        for h in range(KVH):
            pos = g.choice(np.arange(lo[b], hi[b]), size=min(n_dom, hi[b] - lo[b]), replace=False)
            dom[b, h, :len(pos)] = pos
            # logit of a*u against the group's queries: scale * a * mean(q . u)
            qu = float((qv[b, h] @ u[b, h]).mean()) * scale
            for p_ in pos:
                kf[b, h, p_] = u[b, h] * np.float32(g.uniform(*gap) / qu)
    off = g.uniform(*v_offset, (B, KVH, 1, HD // 64)) * g.choice([-1.0, 1.0], (B, KVH, 1, HD // 64))
    vf = (0.5 * g.standard_normal((B, KVH, cap, HD)) + np.repeat(off, 64, axis=-1)).astype(np.float32)
    K = quant.quantize(from_f32(kf, dtype), dtype)
    V = quant.quantize(from_f32(vf, dtype), dtype)
    return q, K, V, dom


def peaked_inputs_torch(gen, dev, B, H, KVH, L, cap, lo, hi, scale=1 / np.sqrt(128), gap=(6.0, 14.0), n_dom=1,
                        tail=0.5, v_offset=(0.75, 1.5), HD=128):
    """``peaked_inputs`` drawn on the GPU with a torch Generator, for full-size cases: fp16 q (B, H, L, HD) and 8-bit
    K/V triples (B, KVH, cap, .) quantized by the library's quantize kernel (bit-exact with oracle.quant, a GPU test
    of its own).  Same recipe: a direction u per (row, kv head) shared by its queries, ``n_dom`` keys in
    [lo[b], hi[b]) set to a u with their logit ``gap`` nats above a N(0, tail^2) tail, V = N(0, 0.5^2) plus a
    per-(row, kv head, group) offset of random sign."""
    import torch

    from locals_amd import qkv

    G = H // KVH
    f = dict(generator=gen, device=dev, dtype=torch.float32)
    u = torch.randn((B, KVH, HD), **f)
    u = u * (HD ** 0.5) / u.norm(dim=-1, keepdim=True)
    q = (0.6 * u[:, :, None, None, :] + 0.8 * torch.randn((B, KVH, G, L, HD), **f)).to(torch.float16)
    qu = (q.float() @ u[:, :, None, :, None]).mean(dim=(2, 3, 4)) * scale  # (B, KVH): logit of u against the queries
    K = qkv._zeros(B, KVH, cap, HD, torch.float16, dev)
    V = qkv._zeros(B, KVH, cap, HD, torch.float16, dev)
    for b in range(B):  # a row at a time keeps the temporaries small
        kf = tail * torch.randn((1, KVH, cap, HD), **f)
        for h in range(KVH):
            span = int(hi[b]) - int(lo[b])
            pos = int(lo[b]) + torch.randperm(span, generator=gen, device=dev)[:n_dom]
            a = (gap[0] + (gap[1] - gap[0]) * torch.rand((n_dom,), **f)) / qu[b, h]
            kf[0, h, pos] = a[:, None] * u[b, h][None, :]
        sgn = torch.where(torch.rand((1, KVH, 1, HD // 64), **f) < 0.5, -1.0, 1.0)
        off = sgn * (v_offset[0] + (v_offset[1] - v_offset[0]) * torch.rand((1, KVH, 1, HD // 64), **f))
        vf = 0.5 * torch.randn((1, KVH, cap, HD), **f) + off.repeat_interleave(64, dim=-1)
        qkv.quantize_into(kf.to(torch.float16), vf.to(torch.float16), tuple(t[b:b + 1] for t in K),
                          tuple(t[b:b + 1] for t in V), 0)
    return q.reshape(B, H, L, HD), K, V
