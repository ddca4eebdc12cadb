"""GPU parity on peaked softmaxes: one or a few dominant keys over a long tail 9..20 log2 below them, V groups with a
common offset (one MLX scale sign per group), so rounding of the attention weights adds up instead of cancelling.

The 8-bit decode kernels multiply V by w = p * v_scale split into fp16 hi + lo; this is the input family where a
weight that loses bits (an fp16 subnormal lo) shows.  Cases: G = 2, 4, 8, 32 (both quad pass-1 forms and the
register-fed kernel), contexts up to 32k, sinks on and off, fp16 and bf16; the fp16/bf16 ragged decode; masked
multi-query attention over 8-bit K/V (causal prefill chunk, tree verification).  The oracle is the float64 closed
form (oracle/attn.py), which follows locals/qkv.py:213-249 and the MLX SDPA the reference calls for prompts
(locals/qkv.py:270-272).  Bars: 2e-3 max-abs (fp16), 2^-7 (1 + max|ref|) (bf16, tests/test_flint.py:295).
"""

import numpy as np
import pytest
import torch

from oracle import attn as oa
from oracle import quant as oq
from tests.inputs import normal16, peaked_inputs, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _tol(ref, dtype):
    return 2e-3 if dtype == "float16" else 2 ** -7 * (1 + np.abs(ref).max())


DECODE = [
    # (H, KVH, B, cap, n, n_dom, sinks)
    (16, 8, 3, 4096, 4000, 1, True),     # G = 2
    (32, 8, 3, 4096, 4000, 1, False),    # G = 4 (C2's heads)
    (32, 8, 2, 4096, 4000, 3, True),     # G = 4, three dominant keys
    (32, 4, 3, 4096, 4000, 1, True),     # G = 8 (two head groups)
    (32, 1, 2, 4096, 4000, 1, False),    # G = 32 (register-fed kernel)
    (8, 2, 1, 32768, 32768, 1, True),    # G = 4 over 32k keys
    (16, 2, 1, 32768, 32768, 2, False),  # G = 8 over 32k keys
]


@pytest.mark.parametrize("H,KVH,B,cap,n,n_dom,sinks", DECODE)
def test_attend_peaked(dev, H, KVH, B, cap, n, n_dom, sinks):
    from locals_amd import qkv

    print(f"peaked attend H={H} KVH={KVH} B={B} n={n} n_dom={n_dom} sinks={sinks}", flush=True)
    g = rng(300 + H + KVH + n + n_dom)
    start = np.array([0, n // 3, n - 1000][:B], dtype=np.int32)
    q, K, V, _ = peaked_inputs(g, B, H, KVH, 1, cap, start, np.full(B, n), scale=0.0884, n_dom=n_dom)
    sk = normal16(g, (H,), 2.0) if sinks else None
    got = qkv.attend(to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev), n,
                     None if sk is None else to_torch(sk, dev), 0.0884, to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oa.attend(q, K, V, n, sk, 0.0884, start)
    err = np.abs(_np(got) - ref).max()
    print(f"  max |err| {err:.3g}", flush=True)
    assert err <= 2e-3, err


def test_attend_peaked_bf16(dev):
    from locals_amd import qkv

    g = rng(311)
    B, H, KVH, cap, n = 2, 32, 8, 8192, 8000
    start = np.array([0, 2500], dtype=np.int32)
    q, K, V, _ = peaked_inputs(g, B, H, KVH, 1, cap, start, np.full(B, n), scale=0.0884, dtype="bfloat16")
    sk = normal16(g, (H,), 2.0, dtype="bfloat16")
    got = qkv.attend(to_torch(q, dev, "bfloat16"), triple_to_torch(K, dev, "bfloat16"),
                     triple_to_torch(V, dev, "bfloat16"), n, to_torch(sk, dev, "bfloat16"), 0.0884,
                     to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oa.attend(q, K, V, n, sk, 0.0884, start, dtype="bfloat16")
    assert np.abs(_np(got) - ref).max() <= _tol(ref, "bfloat16")


def test_attend_large_bf16_v_scales(dev):
    """bf16 V whose groups span ~1e6 (scales ~4e3): w = p * v_scale would pass fp16's 65504 without the prescale."""
    from locals_amd import qkv

    g = rng(312)
    B, H, KVH, cap, n = 1, 32, 8, 2048, 2000
    start = np.zeros(B, dtype=np.int32)
    q, K, V, _ = peaked_inputs(g, B, H, KVH, 1, cap, start, np.full(B, n), scale=0.0884, dtype="bfloat16")
    vf = oq.dequantize(*V, dtype="bfloat16").astype(np.float32) * np.float32(2.0 ** 18)
    V = oq.quantize(oq.from_f32(vf, "bfloat16"), "bfloat16")
    assert np.abs(oq.to_f32(V[1], "bfloat16")).max() > 1024.0
    got = qkv.attend(to_torch(q, dev, "bfloat16"), triple_to_torch(K, dev, "bfloat16"),
                     triple_to_torch(V, dev, "bfloat16"), n, None, 0.0884, to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oa.attend(q, K, V, n, None, 0.0884, start, dtype="bfloat16")
    out = _np(got)
    assert np.isfinite(out).all()
    assert np.abs(out - ref).max() <= _tol(ref, "bfloat16")


@pytest.mark.parametrize("kvdt", ["float16", "bfloat16"])
def test_ragged_peaked(dev, kvdt):
    from locals_amd.attention import ragged_attention

    g = rng(320)
    n_slots, H, Hkv, cap = 3, 16, 8, 4096
    q, K, V, _ = peaked_inputs(g, n_slots, H, Hkv, 1, cap, np.zeros(n_slots, int), np.full(n_slots, 1234),
                               scale=1 / np.sqrt(128), dtype=kvdt)
    Kf = oq.from_f32(oq.dequantize(*K, dtype=kvdt).astype(np.float32), kvdt)
    Vf = oq.from_f32(oq.dequantize(*V, dtype=kvdt).astype(np.float32), kvdt)
    slots = np.array([0, 2, 1, 2], dtype=np.int32)
    nkeys = np.array([4096, 3000, 4096, 1234], dtype=np.int32)
    qr = q[slots, :, 0]
    scale = np.array([1 / np.sqrt(128)], dtype=np.float32)
    got = ragged_attention(to_torch(qr, dev, kvdt), to_torch(Kf, dev, kvdt), to_torch(Vf, dev, kvdt),
                           to_torch(slots, dev), to_torch(nkeys, dev), torch.from_numpy(scale).to(dev))
    torch.cuda.synchronize()
    f = lambda a: oq.to_f32(a, kvdt)  # noqa: E731
    ref = oa.ragged_attention(f(qr), f(Kf), f(Vf), slots, nkeys, scale)
    assert np.abs(_np(got) - ref).max() <= _tol(ref, kvdt)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_causal_prefill_q8_peaked(dev, dtype):
    """A prompt chunk of 96 queries, causal over 2,000 8-bit keys: the dominant keys sit in the prefix every query
    sees."""
    from locals_amd.sdpa import scaled_dot_product_attention

    g = rng(330)
    B, H, KVH, L, N = 2, 32, 8, 96, 2000
    cap = 2048
    q, K, V, _ = peaked_inputs(g, B, H, KVH, L, cap, np.zeros(B, int), np.full(B, N - L), scale=0.0884, n_dom=2,
                               dtype=dtype)
    sk = normal16(g, (H,), 2.0, dtype=dtype)
    Kt, Vt = triple_to_torch(K, dev, dtype), triple_to_torch(V, dev, dtype)
    got = scaled_dot_product_attention(to_torch(q, dev, dtype), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.0884, mask="causal",
                                       sinks=to_torch(sk, dev, dtype))
    torch.cuda.synchronize()
    ref = oa.sdpa_q8(q, K, V, 0.0884, "causal", sk, n=N, dtype=dtype)
    assert np.abs(_np(got) - ref).max() <= _tol(ref, dtype)


def test_tree_verify_q8_peaked(dev):
    from locals_amd.sdpa import TreeMask, scaled_dot_product_attention

    g = rng(331)
    B, H, KVH, L, P = 4, 32, 8, 16, 3000
    N, cap = P + L, 3072
    q, K, V, _ = peaked_inputs(g, B, H, KVH, L, cap, np.zeros(B, int), np.full(B, P), scale=0.0884)
    parents = [[-1] + [int(g.integers(max(0, i - 3), i)) for i in range(1, L)] for _ in range(B)]
    local = np.stack([oa.ancestor_mask(pp) for pp in parents])
    tm = TreeMask.from_local(torch.from_numpy(local), device=dev)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    got = scaled_dot_product_attention(to_torch(q, dev), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.0884, mask=tm)
    torch.cuda.synchronize()
    vis = np.stack([oa.tree_full_mask(m, P) for m in local])[:, None]
    ref = oa.sdpa_q8(q, K, V, 0.0884, vis, None, n=N)
    assert np.abs(_np(got) - ref).max() <= 2e-3
