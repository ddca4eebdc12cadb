"""GPU parity of the split-K decode kernels (lcl_qkv_attend, lcl_ragged_attention) against the float64 oracle.

Cases follow the reference's own test (tests/test_flint.py:278-295: (B, n, cap, pads) =
(1,1,256,[0]), (1,13,256,[0]), (1,2100,2304,[0]), (3,700,768,[0,37,300]), K ~ 2 N(0,1), sinks ~ 2 N(0,1), scale
0.0884) over the head layouts (32,4) and (4,2) it uses plus the BASELINE shapes (32/8, 16/8) and G = 1, 5, 6, 7, 16, 32
(G <= 4 takes the one-head-group quad pass 1, 5 <= G <= 8 the two-group one, larger G the register-fed kernel).
Bar: max |got - oracle| <= 2e-3 for fp16 outputs; bf16 uses the reference's 2^-7 (1 + max|ref|).
"""

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from tests.inputs import normal16, q8_cache, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu

CASES = [(1, 1, 256, [0]), (1, 13, 256, [0]), (1, 2100, 2304, [0]), (3, 700, 768, [0, 37, 300])]
HEADS = [(32, 4), (24, 4), (20, 4), (28, 4), (4, 2), (32, 8), (16, 8), (8, 8), (16, 1), (32, 1)]


def _out(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("H,KVH", HEADS)
@pytest.mark.parametrize("case", CASES)
def test_attend_matches_oracle(dev, H, KVH, case):
    from locals_amd import qkv

    B, n, cap, pads = case
    print(f"attend H={H} KVH={KVH} case={case}", flush=True)
    g = rng(1000 + H * 7 + KVH + n)
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0)
    sinks = normal16(g, (H,), 2.0)
    start = np.array(pads, dtype=np.int32)
    got = qkv.attend(to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev), n, to_torch(sinks, dev),
                     0.0884, to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oattn.attend(q, K, V, n, sinks, 0.0884, start)
    err = np.abs(_out(got) - ref).max()
    assert err <= 2e-3, err


@pytest.mark.parametrize("block", [64, 256, 1024])
def test_attend_block_size_does_not_matter(dev, block):
    from locals_amd import qkv

    g = rng(7)
    B, H, KVH, cap, n = 2, 32, 8, 4096, 3001
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap)
    start = np.array([0, 1234], dtype=np.int32)
    ref = oattn.attend(q, K, V, n, None, 1 / np.sqrt(128), start)
    old = qkv.BLOCK
    try:
        qkv.BLOCK = block
        got = qkv.attend(to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev), n, None,
                         1 / np.sqrt(128), to_torch(start, dev))
        torch.cuda.synchronize()
    finally:
        qkv.BLOCK = old
    assert np.abs(_out(got) - ref).max() <= 2e-3


def test_attend_ignores_garbage_outside_range(dev):
    """Keys before start[b] and at/after n never matter, even NaN/inf there (scales, biases and codes)."""
    from locals_amd import qkv

    g = rng(11)
    B, H, KVH, cap, n = 2, 16, 8, 512, 300
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap)
    start = np.array([5, 77], dtype=np.int32)
    ref = oattn.attend(q, K, V, n, None, 0.1, start)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    for t in (Kt, Vt):
        for b, s in enumerate(start):
            t[1][b, :, :s] = float("nan")
            t[2][b, :, :s] = float("inf")
        t[1][:, :, n:] = float("nan")
        t[2][:, :, n:] = float("-inf")
        t[0][:, :, n:] = -1
    got = qkv.attend(to_torch(q, dev), Kt, Vt, n, None, 0.1, to_torch(start, dev))
    torch.cuda.synchronize()
    assert np.isfinite(_out(got)).all()
    assert np.abs(_out(got) - ref).max() <= 2e-3


def test_attend_empty_rows_and_sinks(dev):
    """n == start gives 0 (with or without a sink); a single key with sink -inf gives v exactly."""
    from locals_amd import qkv

    g = rng(12)
    B, H, KVH, cap = 3, 8, 4, 256
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap)
    sinks = normal16(g, (H,), 2.0)
    n = 100
    start = np.array([100, 250, 99], dtype=np.int32)  # empty, empty (start > n), one key
    got = qkv.attend(to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev), n, to_torch(sinks, dev),
                     0.09, to_torch(start, dev))
    got_ns = qkv.attend(to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev), n, None, 0.09,
                        to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oattn.attend(q, K, V, n, sinks, 0.09, start)
    assert np.abs(_out(got) - ref).max() <= 2e-3
    assert (_out(got)[:2] == 0).all() and (_out(got_ns)[:2] == 0).all()
    from oracle.quant import dequantize

    vd = dequantize(*V)
    for h in range(H):
        assert np.abs(_out(got_ns)[2, h, 0] - vd[2, h // 2, 99]).max() <= 2e-3


def test_attend_bf16(dev):
    from locals_amd import qkv

    g = rng(13)
    B, H, KVH, cap, n = 2, 32, 4, 768, 700
    q = normal16(g, (B, H, 1, 128), dtype="bfloat16")
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0, dtype="bfloat16")
    sinks = normal16(g, (H,), 2.0, dtype="bfloat16")
    start = np.array([0, 300], dtype=np.int32)
    got = qkv.attend(to_torch(q, dev, "bfloat16"), triple_to_torch(K, dev, "bfloat16"),
                     triple_to_torch(V, dev, "bfloat16"), n, to_torch(sinks, dev, "bfloat16"), 0.0884,
                     to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oattn.attend(q, K, V, n, sinks, 0.0884, start, dtype="bfloat16")
    assert got.dtype == torch.bfloat16
    assert np.abs(_out(got) - ref).max() <= 2 ** -7 * (1 + np.abs(ref).max())


@pytest.mark.parametrize("H,KVH", [(32, 8), (32, 4), (32, 1)])
def test_attend_fp32_query(dev, H, KVH):
    """fp32 queries (staged at 4 bytes a dim by the quad pass 1), fp16-representable so the oracle's fp16 q is the
    same query; the output is fp32."""
    from locals_amd import qkv

    g = rng(15 + H + KVH)
    B, cap, n = 3, 768, 700
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0)
    sinks = normal16(g, (H,), 2.0)
    start = np.array([0, 37, 300], dtype=np.int32)
    qt = to_torch(q, dev).float()
    got = qkv.attend(qt, triple_to_torch(K, dev), triple_to_torch(V, dev), n, to_torch(sinks, dev), 0.0884,
                     to_torch(start, dev))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    ref = oattn.attend(q, K, V, n, sinks, 0.0884, start)
    assert np.abs(_out(got) - ref).max() <= 2e-3


@pytest.mark.parametrize("H,Hkv", [(16, 8), (8, 8), (32, 4)])
@pytest.mark.parametrize("kvdt", ["float16", "bfloat16"])
def test_ragged_matches_oracle(dev, H, Hkv, kvdt):
    from locals_amd.attention import ragged_attention

    g = rng(20 + H + Hkv)
    n_slots, cap, R = 3, 2048, 5
    q = normal16(g, (R, H, 128), dtype=kvdt)
    Kf = normal16(g, (n_slots, Hkv, cap, 128), dtype=kvdt)
    Vf = normal16(g, (n_slots, Hkv, cap, 128), dtype=kvdt)
    slots = np.array([0, 2, 1, 2, 0], dtype=np.int32)
    nkeys = np.array([2048, 1, 0, 777, 1500], dtype=np.int32)
    scale = np.array([1 / np.sqrt(128)], dtype=np.float32)
    got = ragged_attention(to_torch(q, dev, kvdt), to_torch(Kf, dev, kvdt), to_torch(Vf, dev, kvdt),
                           to_torch(slots, dev), to_torch(nkeys, dev), torch.from_numpy(scale).to(dev))
    torch.cuda.synchronize()
    from oracle.quant import to_f32

    ref = oattn.ragged_attention(to_f32(q, kvdt), to_f32(Kf, kvdt), to_f32(Vf, kvdt), slots, nkeys, scale)
    tol = 2e-3 if kvdt == "float16" else 2 ** -7 * (1 + np.abs(ref).max())
    assert np.abs(_out(got) - ref).max() <= tol
    assert (_out(got)[2] == 0).all()


@pytest.mark.parametrize("H,KVH,B", [(8, 2, 100), (24, 4, 100), (32, 8, 37), (32, 4, 64)])
def test_attend_many_rows(dev, H, KVH, B):
    """Many rows with ragged left padding, empty rows and a row whose keys start mid-tile.  Past 64 rows the quad
    pass 1 scans the rows 64 at a time; up to 64 it holds one a lane, read 16 at a time by scalar loads (37 ends
    inside a group of 16, 64 fills four)."""
    from locals_amd import qkv

    g = rng(14 + H + B)
    cap, n = 640, 600
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0)
    sinks = normal16(g, (H,), 2.0)
    start = g.integers(0, n + 1, size=B).astype(np.int32)
    empty = [3, B * 2 // 5, B * 3 // 4]
    start[empty] = n  # empty rows
    start[[5, B - 2]] = 0
    got = qkv.attend(to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev), n, to_torch(sinks, dev),
                     0.0884, to_torch(start, dev))
    torch.cuda.synchronize()
    ref = oattn.attend(q, K, V, n, sinks, 0.0884, start)
    assert np.abs(_out(got) - ref).max() <= 2e-3
    assert not _out(got)[empty].any()


def test_attend_c2_full_size_vs_c_restatement(dev):
    """BASELINE config 2 at its full size (16 rows, contexts U[1024, 32768] seeded as bench.py draws them, 32/8
    heads, 8-bit K/V made by the quantize kernel on the GPU) against the C restatement of the reference's two
    passes (oracle/c, fp32, the reference's block sizes), with sinks."""
    import bench
    from locals_amd import qkv
    from oracle import cbind

    cfg = bench.config("c2")
    B, H, KVH, nb = cfg["B"], cfg["H"], cfg["KVH"], cfg["nb"]
    n = int(nb.max())
    cap = (n + 255) // 256 * 256
    print(f"c2 full size: sum n_b = {int(nb.sum())}, cap = {cap}", flush=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    K = qkv._zeros(B, KVH, cap, 128, torch.float16, dev)
    V = qkv._zeros(B, KVH, cap, 128, torch.float16, dev)
    for b in range(B):
        kf = torch.randn((1, KVH, cap, 128), generator=gen, device=dev, dtype=torch.float16)
        vf = torch.randn((1, KVH, cap, 128), generator=gen, device=dev, dtype=torch.float16)
        qkv.quantize_into(kf, vf, tuple(a[b:b + 1] for a in K), tuple(a[b:b + 1] for a in V), 0)
    q = torch.randn((B, H, 1, 128), generator=gen, device=dev, dtype=torch.float16)
    sinks = torch.randn((H,), generator=gen, device=dev, dtype=torch.float16) * 2
    start = torch.tensor(n - nb, dtype=torch.int32, device=dev)
    got = qkv.attend(q, K, V, n, sinks, 1 / np.sqrt(128), start)
    torch.cuda.synchronize()
    host = lambda t: t.cpu().numpy()  # noqa: E731
    Kn = (host(K[0]).view(np.uint32), host(K[1]), host(K[2]))
    Vn = (host(V[0]).view(np.uint32), host(V[1]), host(V[2]))
    ref = cbind.attend_q8(host(q), Kn, Vn, n, host(sinks), 1 / np.sqrt(128), host(start), threads=16)
    err = float(np.abs(_out(got) - ref.astype(np.float64)).max())
    print(f"c2 full size max |gpu - C| = {err:.3g}", flush=True)
    assert err <= 2e-3
