"""GPU quantize / quantize-append / dequantize against the oracle: codes, scales and biases bit-exact.

Inputs: N(0,1) and N(0,1)*2 fp16/bf16 tensors (the reference test's K scale, tests/test_flint.py:284-285), plus
known-answer groups (constant, exact 255-step grids on either side, max == 0, min == 0, symmetric, ties).
"""

import numpy as np
import pytest
import torch

from oracle import quant as oq
from tests.inputs import normal16, rng, to_torch

pytestmark = pytest.mark.gpu


def _np(t, dtype):
    a = t.cpu()
    if a.dtype == torch.int32:
        return a.numpy().view(np.uint32)
    if a.dtype == torch.bfloat16:
        return a.view(torch.int16).numpy().view(np.uint16)
    return a.numpy()


def _special_groups(dtype):
    """(R, 128) rows whose 64-groups hit the closed form's corners."""
    rows = []
    grid = (np.arange(64, dtype=np.float32) * np.float32(0.25))  # min 0, max 15.75
    rows.append(np.concatenate([np.full(64, 1.5, np.float32), np.full(64, -3.0, np.float32)]))  # constant groups
    rows.append(np.concatenate([grid - 8.0, -(grid - 8.0)]))  # side and non-side grids
    rows.append(np.concatenate([grid, -grid]))  # min == 0 / max == 0
    rows.append(np.concatenate([np.linspace(-1, 1, 64, dtype=np.float32), np.zeros(64, np.float32)]))  # symmetric, zeros
    ties = np.zeros(64, np.float32)
    ties[0], ties[1] = 0.0, 255.0
    ties[2:] = np.arange(62, dtype=np.float32) + 0.5  # (w - 0) / 1 = k + 0.5: a tie for every value
    rows.append(np.concatenate([ties, ties - 255.0]))
    x = np.stack(rows)
    return oq.from_f32(x, dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("mode", ["away", "even"])
def test_quantize_bit_exact(dev, dtype, mode):
    from locals_amd import qkv

    g = rng(3)
    x = normal16(g, (3, 5, 77, 128), 2.0, dtype)
    sp = _special_groups(dtype)
    for arr in (x, sp):
        got = qkv.quantize(to_torch(arr, dev, dtype), round_mode=mode)
        torch.cuda.synchronize()
        ref = oq.quantize(arr, dtype, round_mode=mode)
        for a, b in zip(got, ref):
            assert np.array_equal(_np(a, dtype), b)


def test_tie_modes_differ_where_ties_exist(dev):
    from locals_amd import qkv

    sp = to_torch(_special_groups("float16"), dev)
    a = qkv.quantize(sp, round_mode="away")[0]
    e = qkv.quantize(sp, round_mode="even")[0]
    torch.cuda.synchronize()
    assert not torch.equal(a, e)  # the tie row rounds differently


def test_quantize_append_writes_only_its_positions(dev):
    from locals_amd import qkv

    g = rng(4)
    B, KVH, cap, L, prev = 2, 3, 512, 37, 200
    k = normal16(g, (B, KVH, L, 128))
    v = normal16(g, (B, KVH, L, 128))
    K = qkv._zeros(B, KVH, cap, 128, torch.float16, dev)
    V = qkv._zeros(B, KVH, cap, 128, torch.float16, dev)
    for t in K + V:
        t.fill_(7)
    qkv.quantize_into(to_torch(k, dev), to_torch(v, dev), K, V, prev)
    torch.cuda.synchronize()
    rk, rv = oq.quantize(k), oq.quantize(v)
    for got, ref in ((K, rk), (V, rv)):
        for a, b in zip(got, ref):
            a_cpu = a.cpu()
            keep = torch.ones(cap, dtype=torch.bool)
            keep[prev:prev + L] = False
            assert torch.equal(a_cpu[:, :, keep], torch.full_like(a_cpu, 7)[:, :, keep])
            assert np.array_equal(_np(a, "float16")[:, :, prev:prev + L], b)


@pytest.mark.parametrize("odt", [torch.float16, torch.float32])
def test_dequantize(dev, odt):
    from locals_amd import qkv

    g = rng(5)
    x = normal16(g, (2, 4, 100, 128), 2.0)
    t = oq.quantize(x)
    got = qkv.dequantized(tuple(to_torch(a, dev) for a in t), dtype=odt)
    torch.cuda.synchronize()
    ref = oq.dequantize(*t)
    err = np.abs(got.float().cpu().numpy().astype(np.float64) - ref)
    ulp = np.maximum(np.abs(ref), 2.0 ** -14) * (2.0 ** -10 if odt == torch.float16 else 2.0 ** -22)
    assert (err <= ulp).all()


@pytest.mark.parametrize("D,sdt,odt", [(64, "float16", torch.float16), (128, "bfloat16", torch.float32),
                                        (192, "float16", torch.float32), (256, "bfloat16", torch.bfloat16),
                                        (512, "float16", torch.float16), (192, "bfloat16", torch.bfloat16)])
def test_dequantize_is_one_fused_multiply_add(dev, D, sdt, odt):
    """lcl_dequantize computes each value as one fp32 fused multiply-add scale * code + bias, then rounds it to the
    output dtype.  That is pinned bit for bit for the kernel of D = 64 / 128 / 256 / 512 (row and group by shifts)
    and the general one (D = 192).  The exact value is formed in float64 (scale * code has at most 19 significant
    bits, so for these groups the sum is exact) and rounded once to fp32, as the fused operation does."""
    from locals_amd import _lib

    g = rng(6 + D)
    rows = 333
    x = normal16(g, (rows, D), 3.0, dtype=sdt)
    w, sc, bi = oq.quantize(x, dtype=sdt)
    s_t, b_t, w_t = to_torch(sc, dev, sdt), to_torch(bi, dev, sdt), to_torch(w, dev)
    out = torch.empty((rows, D), dtype=odt, device=dev)
    lib = _lib.load()
    rc = lib.lcl_dequantize(_lib.ptr(w_t), _lib.ptr(s_t), _lib.ptr(b_t), _lib.dtype_code(s_t.dtype), rows, D,
                            _lib.ptr(out), _lib.dtype_code(odt), _lib.stream_of(dev))
    _lib.check(rc, "lcl_dequantize")
    torch.cuda.synchronize()
    codes = w.view(np.uint8).reshape(rows, D).astype(np.float64)
    s64 = np.repeat(oq.to_f32(sc, sdt).astype(np.float64), 64, axis=1)
    b64 = np.repeat(oq.to_f32(bi, sdt).astype(np.float64), 64, axis=1)
    v32 = (s64 * codes + b64).astype(np.float32)
    if odt == torch.float32:
        want = torch.from_numpy(v32)
    elif odt == torch.float16:
        want = torch.from_numpy(v32.astype(np.float16))
    else:
        want = torch.from_numpy(oq.from_f32(v32, "bfloat16").view(np.int16)).view(torch.bfloat16)
    assert torch.equal(out.cpu(), want)


def test_batch_cache_decode_step_equals_oracle(dev):
    """A BatchQuantizedKVCache built by update_and_fetch then attended (qkv.attention, one query a row) equals the
    oracle over the oracle-quantized keys: the cache's codes are bit-exact and the attention within 2e-3."""
    from locals_amd import qkv
    from oracle import attn as oa

    g = rng(6)
    B, H, KVH, L0 = 3, 8, 2, 300
    pads = [0, 5, 40]
    cache = qkv.BatchQuantizedKVCache(pads, device=dev)
    k0 = normal16(g, (B, KVH, L0, 128))
    v0 = normal16(g, (B, KVH, L0, 128))
    cache.update_and_fetch(to_torch(k0, dev), to_torch(v0, dev))
    q = normal16(g, (B, H, 1, 128))
    k1 = normal16(g, (B, KVH, 1, 128))
    v1 = normal16(g, (B, KVH, 1, 128))
    sinks = normal16(g, (H,), 2.0)
    out = qkv.attention(to_torch(q, dev), to_torch(k1, dev), to_torch(v1, dev), cache, 0.0884, None,
                        to_torch(sinks, dev))
    torch.cuda.synchronize()
    K = oq.quantize(np.concatenate([k0, k1], axis=2))
    V = oq.quantize(np.concatenate([v0, v1], axis=2))
    for got, ref in zip(cache.keys, K):
        assert np.array_equal(_np(got, "float16")[:, :, :L0 + 1], ref)
    ref = oa.attend(q, K, V, L0 + 1, sinks, 0.0884, np.array(pads))
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-3
