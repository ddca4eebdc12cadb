"""GPU qk_norm_rope (and its fused 8-bit cache store) against the oracle, through the C ABI.

The kernel evaluates the reference's formula (locals/qk_kernel.py:50-62) at its rounding points -- an fp32 value,
then T -- with the angle in fp32 and the rest correctly rounded, as the oracle does, so q, k and v are compared bit
for bit (fp16 midpoints included: a merged fp64 -> T rounding would fail at about 1 value in 10^4).  The reference's own check (tests/test_flint.py:221-238: norm then RoPE within
0.02 max|ref|, v exact) is repeated against a plain torch float32 formula.  The fused form must equal
qk_norm_rope followed by the quantize-append kernel bit for bit.
"""

import math
import types

import numpy as np
import pytest
import torch

from oracle import attn as oa
from oracle import quant as oq
from tests.inputs import normal16, rng, to_torch

pytestmark = pytest.mark.gpu

TDT = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def _layer(H, KV, HD, dtype, dev, rope=True, base=10000.0, eps=1e-6, seed=0):
    g = rng(100 + seed)
    qw = normal16(g, (HD,), 0.05, dtype)
    kw = normal16(g, (HD,), 0.05, dtype)
    qw = oq.from_f32(oq.to_f32(qw, dtype) + 1.0, dtype)
    kw = oq.from_f32(oq.to_f32(kw, dtype) + 1.0, dtype)
    a = types.SimpleNamespace(
        n_heads=H, n_kv_heads=KV, head_dim=HD,
        q_norm=types.SimpleNamespace(weight=to_torch(qw, dev, dtype), eps=eps),
        k_norm=types.SimpleNamespace(weight=to_torch(kw, dev, dtype), eps=eps),
        rope=types.SimpleNamespace(base=base, dims=HD, traditional=False, scale=1.0) if rope else None)
    return a, oq.to_f32(qw, dtype), oq.to_f32(kw, dtype)


def _f32(t):
    return t.float().cpu().numpy()


def _ulps(got, ref, dtype):
    """|got - ref| in units of T's last place at |ref|."""
    p = 10 if dtype == "float16" else 7
    e = np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14)))
    return np.abs(got - ref) / 2.0 ** (e - p)


CASES = [  # B, L, H, KV, HD, offset
    (1, 1, 4, 2, 128, 300),
    (3, 1, 4, 2, 128, [4, 0, 77]),
    (2, 6, 4, 2, 128, 0),
    (16, 1, 32, 8, 128, list(range(1024, 32768, 2048))),
    (1, 64, 32, 8, 128, 16384),
    (2, 5, 4, 2, 256, [-3, 9000]),
    (1, 3, 2, 1, 512, 7),
    (2, 2, 2, 1, 384, [11, 2048]),
    (1, 2, 2, 2, 1024, 5),
]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("rope", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_qk_norm_rope_vs_oracle(dev, dtype, rope, case):
    from locals_amd import qk_kernel

    B, L, H, KV, HD, off = case
    print(f"qk_norm_rope B={B} L={L} H={H} KV={KV} HD={HD} rope={rope} {dtype}", flush=True)
    a, qw, kw = _layer(H, KV, HD, dtype, dev, rope)
    x = normal16(rng(sum(case[:5])), (B, L, (H + 2 * KV) * HD), 2.0, dtype)
    offset = torch.tensor(off, dtype=torch.int32, device=dev) if isinstance(off, list) else off
    q, k, v = qk_kernel.qk_norm_rope(to_torch(x, dev, dtype), a, offset)
    torch.cuda.synchronize()
    assert q.shape == (B, H, L, HD) and k.shape == v.shape == (B, KV, L, HD)
    q0, k0, v0 = oa.qk_norm_rope(oq.to_f32(x, dtype), qw, kw, 1e-6, off, H, KV, HD, rope, 10000.0, dtype)
    assert np.array_equal(_f32(v), v0)
    for got, ref in ((_f32(q), q0), (_f32(k), k0)):
        assert np.array_equal(got, ref), (_ulps(got, ref, dtype).max(), (got != ref).mean())


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_qk_norm_rope_is_norm_then_rope(dev, dtype):
    """The reference's test (tests/test_flint.py:221-238) against torch float32 RMS norm + RoPE over halves: within
    0.02 max|ref|, v exact; a layer without RoPE (norms only) and one with."""
    from locals_amd import qk_kernel

    for rope in (False, True):
        a, _, _ = _layer(4, 2, 128, dtype, dev, rope)
        for B, L, off in ((1, 1, 300), (3, 1, [4, 0, 77]), (2, 6, 0)):
            x = to_torch(normal16(rng(B * 10 + L), (B, L, 8 * 128), 2.0, dtype), dev, dtype)
            offset = torch.tensor(off, dtype=torch.int32, device=dev) if isinstance(off, list) else off

            def norm(t, w, eps=1e-6):
                t = t.float()
                n = (t * torch.rsqrt((t * t).mean(-1, keepdim=True) + eps)).to(x.dtype)
                return (w.float() * n.float()).to(x.dtype)

            q0 = norm(x[..., :512].reshape(B, L, 4, 128), a.q_norm.weight).transpose(1, 2)
            k0 = norm(x[..., 512:768].reshape(B, L, 2, 128), a.k_norm.weight).transpose(1, 2)
            if rope:
                pos = (torch.tensor(off if isinstance(off, list) else [off] * B, device=dev).float()[:, None]
                       + torch.arange(L, device=dev).float()[None])  # (B, L)
                inv = torch.exp2(-torch.arange(64, device=dev).float() * 2 / 128 * math.log2(10000.0))
                th = pos[:, None, :, None] * inv  # (B, 1, L, 64)
                c, s = torch.cos(th), torch.sin(th)

                def rot(t):
                    lo, hi = t[..., :64].float(), t[..., 64:].float()
                    return torch.cat([lo * c - hi * s, lo * s + hi * c], -1).to(x.dtype)

                q0, k0 = rot(q0), rot(k0)
            q, k, v = qk_kernel.qk_norm_rope(x, a, offset)
            assert torch.equal(v, x[..., 768:].reshape(B, L, 2, 128).transpose(1, 2))
            for got, ref in ((q, q0), (k, k0)):
                tol = 0.02 * float(ref.float().abs().max())
                assert float((got.float() - ref.float()).abs().max()) <= tol


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("mode", ["away", "even"])
def test_fused_append_equals_norm_rope_then_quantize(dev, dtype, mode):
    """qk_norm_rope_append == qk_norm_rope + update_and_fetch (quantize-append), bit for bit, over a left-padded
    batch cache: a prompt chunk, then two decode steps (the second crossing the 256-position growth step)."""
    from locals_amd import qk_kernel, qkv

    H, KV, HD = 8, 2, 128
    a, _, _ = _layer(H, KV, HD, dtype, dev, True)
    pads = [3, 0, 250]
    fused = qkv.BatchQuantizedKVCache(pads, device=dev)
    plain = qkv.BatchQuantizedKVCache(pads, device=dev)
    g = rng(7)
    for step, L in enumerate((253, 1, 3)):
        x = to_torch(normal16(g, (3, L, (H + 2 * KV) * HD), 2.0, dtype), dev, dtype)
        q1 = qk_kernel.qk_norm_rope_append(x, a, fused, round_mode=mode)
        q0, k0, v0 = qk_kernel.qk_norm_rope(x, a, plain.offset)
        k_prev = plain._idx
        plain._reserve(3, KV, L, HD, x.dtype, dev)
        qkv.quantize_into(k0, v0, plain.keys, plain.values, k_prev, round_mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(q1, q0), step
        assert fused._idx == plain._idx and torch.equal(fused.offset, plain.offset)
        for f, p in zip(fused.keys + fused.values, plain.keys + plain.values):
            assert f.shape == p.shape and torch.equal(f, p), step


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("mode", ["away", "even"])
def test_fused_append_vs_oracle(dev, dtype, mode):
    """qk_norm_rope_append against the oracle directly (locals/fuse.py:80-83 -> locals/qkv.py:309-326): q equals
    oracle.attn.qk_norm_rope bit for bit, and the cache's new positions hold oracle.quant.quantize of the oracle's
    normed/rotated k and of the raw v, bit for bit, in both tie modes.  A left-padded batch: a prompt chunk at
    per-row offsets, then a decode step; positions outside [prev, prev + L) keep their earlier contents."""
    from locals_amd import qk_kernel, qkv

    H, KV, HD, B = 8, 2, 128, 3
    a, qw, kw = _layer(H, KV, HD, dtype, dev, True, base=1000000.0, seed=3)
    pads = [5, 0, 60]
    cache = qkv.BatchQuantizedKVCache(pads, device=dev)
    g = rng(9)
    for L in (61, 1):
        print(f"fused append vs oracle {dtype} {mode} L={L}", flush=True)
        x = normal16(g, (B, L, (H + 2 * KV) * HD), 2.0, dtype)
        offs = cache.offset.cpu().numpy().copy()  # positions of this step's first token, per row
        prev = cache._idx
        before = None if cache.keys is None else [t.clone() for t in cache.keys + cache.values]
        q = qk_kernel.qk_norm_rope_append(to_torch(x, dev, dtype), a, cache, round_mode=mode)
        torch.cuda.synchronize()
        q0, k0, v0 = oa.qk_norm_rope(oq.to_f32(x, dtype), qw, kw, 1e-6, offs, H, KV, HD, True, 1000000.0, dtype)
        assert np.array_equal(_f32(q), q0)
        for buf, ref in ((cache.keys, k0), (cache.values, v0)):
            rw, rs, rb = oq.quantize(oq.from_f32(ref, dtype), dtype, round_mode=mode)
            w, s_, b_ = (t[:, :, prev:prev + L].cpu() for t in buf)
            assert np.array_equal(w.numpy().view(np.uint32), rw)
            assert np.array_equal(s_.view(torch.int16).numpy().view(np.uint16), np.asarray(rs).view(np.uint16))
            assert np.array_equal(b_.view(torch.int16).numpy().view(np.uint16), np.asarray(rb).view(np.uint16))
        if before is not None:
            for t, o in zip(cache.keys + cache.values, before):
                assert torch.equal(t[:, :, :prev], o[:, :, :prev])


def test_fused_append_single_cache_and_attention(dev):
    """QuantizedKVCache8 (int offset) through the fused store, then attend_cache: equals the unfused
    qkv.attention(q, k, v, cache, ...) path on a twin cache."""
    from locals_amd import qk_kernel, qkv

    dtype = "bfloat16"
    H, KV, HD = 8, 2, 128
    a, _, _ = _layer(H, KV, HD, dtype, dev, True, base=500000.0)
    c1, c2 = qkv.QuantizedKVCache8(), qkv.QuantizedKVCache8()
    g = rng(8)
    sinks = torch.randn(H, device=dev) * 2
    for L in (17, 1, 1):
        x = to_torch(normal16(g, (1, L, (H + 2 * KV) * HD), 2.0, dtype), dev, dtype)
        q1 = qk_kernel.qk_norm_rope_append(x, a, c1)
        mask = "causal" if L > 1 else None
        o1 = qkv.attend_cache(q1, c1, 0.0883, mask, sinks)
        q0, k0, v0 = qk_kernel.qk_norm_rope(x, a, c2.offset)
        o0 = qkv.attention(q0, k0, v0, c2, 0.0883, mask, sinks)
        torch.cuda.synchronize()
        assert c1.offset == c2.offset
        assert torch.equal(o1, o0)


def test_qk_rejects_what_fits_rejects(dev):
    from locals_amd import qk_kernel

    a, _, _ = _layer(4, 2, 128, "float16", dev, True)
    x = torch.zeros((1, 1, 8 * 128), dtype=torch.float16, device=dev)
    q, k, v = qk_kernel.qk_norm_rope(x[:0], a, 0)  # B = 0: nothing to launch
    assert q.shape == (0, 4, 1, 128)
    a.rope.traditional = True
    assert not qk_kernel.fits(a, x)
    with pytest.raises(ValueError):
        qk_kernel.qk_norm_rope(x, a, 0)
