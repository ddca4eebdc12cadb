"""Head sizes other than 128 on the GPU, against the float64 oracle.

The reference's ragged decode kernels are templated on D (any multiple of 32, locals/attention.py:14-20,100-106)
and its quantized cache sends every head size but 128 to MLX's attention over the dequantized cache
(locals/qkv.py:264-272); MLX's attention takes any head size.  Here those shapes run on the general kernel
(locals_amd/csrc/generic.hip).  Cases: ragged fp16/bf16 decode at D = 32, 64, 256; masked attention over 16-bit
K/V at D = 16, 64, 256 under every mask kind with sinks and left padding; over 8-bit triples at D = 64, 256;
qkv.attention's single-token call on a D = 64 cache.  Bars: 2e-3 max-abs (fp16), 2^-7 (1 + max|ref|) (bf16).
"""

import numpy as np
import pytest
import torch

from oracle import attn as oa
from oracle import quant as oq
from tests.inputs import normal16, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _tol(ref, dtype):
    return 2e-3 if dtype == "float16" else 2 ** -7 * (1 + np.abs(ref).max())


@pytest.mark.parametrize("D", [32, 64, 256])
@pytest.mark.parametrize("kvdt", ["float16", "bfloat16"])
def test_ragged_head_dims(dev, D, kvdt):
    from locals_amd.attention import ragged_attention

    g = rng(400 + D)
    n_slots, cap, R, H, Hkv = 3, 700, 5, 16, 4
    q = normal16(g, (R, H, D), dtype=kvdt)
    Kf = normal16(g, (n_slots, Hkv, cap, D), dtype=kvdt)
    Vf = normal16(g, (n_slots, Hkv, cap, D), dtype=kvdt)
    slots = np.array([0, 2, 1, 2, 0], dtype=np.int32)
    nkeys = np.array([700, 1, 0, 333, 64], dtype=np.int32)
    scale = np.array([D ** -0.5], dtype=np.float32)
    got = ragged_attention(to_torch(q, dev, kvdt), to_torch(Kf, dev, kvdt), to_torch(Vf, dev, kvdt),
                           to_torch(slots, dev), to_torch(nkeys, dev), torch.from_numpy(scale).to(dev))
    torch.cuda.synchronize()
    f = lambda a: oq.to_f32(a, kvdt)  # noqa: E731
    ref = oa.ragged_attention(f(q), f(Kf), f(Vf), slots, nkeys, scale)
    assert np.abs(_np(got) - ref).max() <= _tol(ref, kvdt)
    assert (_np(got)[2] == 0).all()


@pytest.mark.parametrize("D", [16, 64, 256])
@pytest.mark.parametrize("mask", ["causal", "tree", "dense", "window", None])
def test_sdpa_16bit_head_dims(dev, D, mask):
    from locals_amd.sdpa import TreeMask, WindowMask, scaled_dot_product_attention

    print(f"sdpa 16-bit D={D} mask={mask}", flush=True)
    g = rng(410 + D)
    B, H, KVH, L, N = 2, 8, 2, 12, 200
    q = normal16(g, (B, H, L, D))
    k = normal16(g, (B, KVH, N, D))
    v = normal16(g, (B, KVH, N, D))
    sinks = normal16(g, (H,), 1.0)
    start = np.array([0, 30], dtype=np.int32)
    vis = np.ones((B, L, N), bool)
    if mask == "causal":
        m, vis = "causal", np.broadcast_to(oa.causal_mask(L, N), (B, L, N)).copy()
    elif mask == "tree":
        parents = [[-1] + [int(g.integers(max(0, i - 3), i)) for i in range(1, L)] for _ in range(B)]
        local = np.stack([oa.ancestor_mask(p) for p in parents])
        m = TreeMask.from_local(torch.from_numpy(local), device=dev)
        vis = np.stack([oa.tree_full_mask(x, N - L) for x in local])
    elif mask == "dense":
        vis = g.random((B, L, N)) < 0.5
        m = torch.from_numpy(vis[:, None]).to(dev)
    elif mask == "window":
        m, vis = WindowMask(37), np.broadcast_to(oa.window_mask(L, N, 37), (B, L, N)).copy()
    else:
        m = None
    vis = vis & (np.arange(N)[None, None] >= start[:, None, None])
    got = scaled_dot_product_attention(to_torch(q, dev), to_torch(k, dev), to_torch(v, dev), scale=D ** -0.5,
                                       mask=m, sinks=to_torch(sinks, dev), start=to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oa.sdpa(q, k, v, D ** -0.5, vis[:, None], sinks)
    assert np.abs(_np(got) - ref).max() <= 2e-3


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_sdpa_q8_head_dims(dev, D, dtype):
    from locals_amd.sdpa import scaled_dot_product_attention

    g = rng(420 + D)
    B, H, KVH, L, N, cap = 2, 8, 4, 20, 300, 320
    q = normal16(g, (B, H, L, D), dtype=dtype)
    K = oq.quantize(normal16(g, (B, KVH, cap, D), 2.0, dtype), dtype)
    V = oq.quantize(normal16(g, (B, KVH, cap, D), 1.0, dtype), dtype)
    sinks = normal16(g, (H,), 2.0, dtype=dtype)
    Kt, Vt = triple_to_torch(K, dev, dtype), triple_to_torch(V, dev, dtype)
    got = scaled_dot_product_attention(to_torch(q, dev, dtype), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.09, mask="causal",
                                       sinks=to_torch(sinks, dev, dtype))
    torch.cuda.synchronize()
    ref = oa.sdpa_q8(q, K, V, 0.09, "causal", sinks, n=N, dtype=dtype)
    assert np.abs(_np(got) - ref).max() <= _tol(ref, dtype)


def test_qkv_attention_decode_head_dim_64(dev):
    """A D = 64 layer's decode step through the 8-bit cache: the reference's attention() takes its attend_few
    branch for any head size but 128 (locals/qkv.py:264-272), here the general kernel over the triples."""
    from locals_amd import qkv

    g = rng(430)
    B, H, KVH, D = 2, 8, 2, 64
    cache = qkv.BatchQuantizedKVCache([0, 3], device=dev)
    ks, vs = [], []
    for L in (50, 1):
        k, v = normal16(g, (B, KVH, L, D)), normal16(g, (B, KVH, L, D))
        ks.append(k)
        vs.append(v)
        q = normal16(g, (B, H, L, D))
        mask = cache.make_mask(L)  # made before the step, as mlx-lm's create_attention_mask is: left padding too
        out = qkv.attention(to_torch(q, dev), to_torch(k, dev), to_torch(v, dev), cache, D ** -0.5, mask, None)
    torch.cuda.synchronize()
    K = oq.quantize(np.concatenate(ks, 2))
    V = oq.quantize(np.concatenate(vs, 2))
    vis = np.ones((B, 1, 1, 51), bool)
    vis[1, ..., :3] = False  # the second row's left padding
    ref = oa.sdpa_q8(q, K, V, D ** -0.5, vis, None, n=51)
    assert np.abs(_np(out) - ref).max() <= 2e-3
