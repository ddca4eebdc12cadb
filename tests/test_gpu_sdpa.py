"""GPU parity of lcl_sdpa (multi-query masked attention, split-K on MFMA) against the float64 oracle.

Cases: the chunked-prefill shape (causal over an 8-bit prefix, the last query aligned with the last key,
locals/fuse.py:131-137), tree verification (prefix visible, ancestor-only among the new tokens,
locals/treedec.py:56-67), dense boolean masks (locals/fuse.py:139), sinks, left padding, fp16 and bf16, and the
reference's invariants: a chunk equals decoding its tokens one by one (tests/test_flint.py:420-455), a chain tree
equals the causal mask, 5 to 8 queries unpadded equal the reference's padded pass (tests/test_flint.py:534-552);
the sliding-window mask of the banded prompt chunks (locals/fuse.py:113-125) over 16-bit and 8-bit K/V, with left
padding; a query with no visible key gives 0.
Bars: 2e-3 max-abs for fp16 outputs; bf16 2^-7 (1 + max|ref|) (tests/test_flint.py:295).
"""

import numpy as np
import pytest
import torch

from oracle import attn as oa
from oracle import quant as oq
from tests.inputs import normal16, q8_cache, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=[0, 64, 1 << 20], ids=["auto-chunks", "chunk64", "one-chunk"])
def sdpa_block(request):
    """Every case runs with the library's chunking, with 64-key chunks (many parts, pass 2 joins them) and with a
    single chunk (pass 1 writes the output itself)."""
    from locals_amd import sdpa

    old = sdpa.BLOCK
    sdpa.BLOCK = request.param
    yield request.param
    sdpa.BLOCK = old


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _tol(ref, dtype):
    return 2e-3 if dtype == "float16" else 2 ** -7 * (1 + np.abs(ref).max())


@pytest.mark.parametrize("H,KVH,L,N", [(32, 8, 64, 600), (16, 8, 37, 300), (4, 2, 9, 9), (8, 8, 130, 1100),
                                       (32, 4, 16, 2100)])
def test_causal_prefill_q8(dev, H, KVH, L, N):
    from locals_amd.sdpa import scaled_dot_product_attention

    print(f"causal q8 H={H} KVH={KVH} L={L} N={N}", flush=True)
    g = rng(100 + H + L + N)
    B, cap = 2, (N + 255) // 256 * 256
    q = normal16(g, (B, H, L, 128))
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0)
    sinks = normal16(g, (H,), 2.0)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    got = scaled_dot_product_attention(to_torch(q, dev), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.0884, mask="causal",
                                       sinks=to_torch(sinks, dev))
    torch.cuda.synchronize()
    ref = oa.sdpa_q8(q, K, V, 0.0884, "causal", sinks, n=N)
    assert np.abs(_np(got) - ref).max() <= 2e-3


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_causal_prefill_q8_eight_waves(dev, sdpa_block, dtype):
    """8-bit K/V, causal, 512 rows a (row, KV head) (128 queries x 4 heads): the fused kernel in eight-wave
    workgroups of 256 rows, each thread feeding 16 dims of one key's K and V through registers, with left padding
    and sinks, in fp16 and bf16, at every chunking."""
    from locals_amd.sdpa import scaled_dot_product_attention

    B, H, KVH, L, N = 2, 32, 8, 128, 1100
    print(f"causal q8 eight waves {dtype} B={B} H={H} KVH={KVH} L={L} N={N} block={sdpa_block}", flush=True)
    g = rng(211 if dtype == "float16" else 212)
    cap = (N + 255) // 256 * 256
    q = normal16(g, (B, H, L, 128), dtype=dtype)
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0, dtype=dtype)
    sinks = normal16(g, (H,), 2.0, dtype=dtype)
    start = np.array([0, 61], np.int32)
    Kt, Vt = triple_to_torch(K, dev, dtype), triple_to_torch(V, dev, dtype)
    got = scaled_dot_product_attention(to_torch(q, dev, dtype), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.0884, mask="causal",
                                       sinks=to_torch(sinks, dev, dtype), start=to_torch(start, dev))
    torch.cuda.synchronize()
    vis = oa.causal_mask(L, N)[None, None] & (np.arange(N)[None, None, None, :] >= start[:, None, None, None])
    ref = oa.sdpa_q8(q, K, V, 0.0884, vis, sinks, n=N, dtype=dtype)
    assert np.abs(_np(got) - ref).max() <= _tol(ref, dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_tree_verify_q8(dev, dtype):
    from locals_amd.sdpa import TreeMask, scaled_dot_product_attention

    g = rng(7)
    B, H, KVH, L, P = 3, 32, 8, 16, 500
    N, cap = P + L, 768
    q = normal16(g, (B, H, L, 128), dtype=dtype)
    K, V = q8_cache(g, B, KVH, cap, dtype=dtype)
    parents = [[-1] + [int(g.integers(max(0, i - 3), i)) for i in range(1, L)] for _ in range(B)]
    local = np.stack([oa.ancestor_mask(pp) for pp in parents])
    tm = TreeMask.from_local(torch.from_numpy(local), device=dev)
    Kt, Vt = triple_to_torch(K, dev, dtype), triple_to_torch(V, dev, dtype)
    got = scaled_dot_product_attention(to_torch(q, dev, dtype), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.0884, mask=tm)
    torch.cuda.synchronize()
    vis = np.stack([oa.tree_full_mask(m, P) for m in local])[:, None]
    ref = oa.sdpa_q8(q, K, V, 0.0884, vis, None, n=N, dtype=dtype)
    assert np.abs(_np(got) - ref).max() <= _tol(ref, dtype)


@pytest.mark.parametrize("kvdt", ["float16", "bfloat16"])
@pytest.mark.parametrize("masked", ["causal", "dense", None])
def test_sdpa_16bit(dev, kvdt, masked):
    from locals_amd.sdpa import scaled_dot_product_attention

    g = rng(8)
    B, H, KVH, L, N = 2, 16, 4, 24, 333
    q = normal16(g, (B, H, L, 128), dtype=kvdt)
    k = normal16(g, (B, KVH, N, 128), dtype=kvdt)
    v = normal16(g, (B, KVH, N, 128), dtype=kvdt)
    sinks = normal16(g, (H,), 1.0, dtype=kvdt)
    if masked == "dense":
        vis = g.random((B, 1, L, N)) < 0.5
        vis[..., 0] = True
        mask, ref_mask = torch.from_numpy(vis).to(dev), vis
    else:
        mask, ref_mask = masked, masked
    got = scaled_dot_product_attention(to_torch(q, dev, kvdt), to_torch(k, dev, kvdt), to_torch(v, dev, kvdt),
                                       scale=0.09, mask=mask, sinks=to_torch(sinks, dev, kvdt))
    torch.cuda.synchronize()
    f = lambda a: oq.to_f32(a, kvdt)  # noqa: E731
    ref = oa.sdpa(f(q), f(k), f(v), 0.09, ref_mask, f(sinks), dtype="float64")
    assert np.abs(_np(got) - ref).max() <= _tol(ref, kvdt)


@pytest.mark.parametrize("case", ["causal-float16", "dense-bfloat16"])
def test_dequantize_first_route(dev, sdpa_block, case):
    """8-bit K/V with many row blocks per (row, KV head) (12 or more of 256 rows under a causal mask, 16 or more of
    64 rows under a dense one): given the room (lcl_sdpa_workspace_bytes_kv) the library dequantizes K and V once
    and runs the 16-bit kernel.  Its output equals the fused 8-bit kernel's bit for
    bit -- the same 16-bit operand values through the same products -- and the oracle within the bar, here with left
    padding and sinks."""
    from locals_amd import _lib, sdpa

    masked, dtype = case.split("-")
    g = rng(31 if masked == "causal" else 32)
    if masked == "causal":  # 768 queries x 4 heads = 12 blocks of 256 rows
        B, H, KVH, L, N = 1, 32, 8, 768, 900
    else:  # dense masks take 64-row blocks: 256 queries x 4 heads = 16
        B, H, KVH, L, N = 2, 16, 4, 256, 400
    cap = (N + 255) // 256 * 256
    print(f"dequantize-first {case} B={B} H={H} KVH={KVH} L={L} N={N} block={sdpa_block}", flush=True)
    lib = _lib.load()
    mk = sdpa.MASK_CAUSAL if masked == "causal" else sdpa.MASK_DENSE
    assert lib.lcl_sdpa_workspace_bytes_kv(B, H, KVH, L, N, cap, sdpa_block, 0, mk) > \
        lib.lcl_sdpa_workspace_bytes(B, H, L, N, sdpa_block)
    q = normal16(g, (B, H, L, 128), dtype=dtype)
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0, dtype=dtype)
    sinks = normal16(g, (H,), 2.0, dtype=dtype)
    start = np.array([37, 0][:B], np.int32)
    if masked == "causal":
        mask = "causal"
        vis = oa.causal_mask(L, N)[None, None]
    else:
        vis = g.random((B, 1, L, N)) < 0.6
        vis[..., N - 1] = True
        mask = torch.from_numpy(vis).to(dev)
    vis = vis & (np.arange(N)[None, None, None, :] >= start[:, None, None, None])
    Kt, Vt = triple_to_torch(K, dev, dtype), triple_to_torch(V, dev, dtype)
    args = (to_torch(q, dev, dtype), tuple(a[:, :, :N] for a in Kt), tuple(a[:, :, :N] for a in Vt))
    kw = dict(scale=0.0884, mask=mask, sinks=to_torch(sinks, dev, dtype), start=to_torch(start, dev))
    got = sdpa.scaled_dot_product_attention(*args, **kw)
    old = sdpa.DEQUANTIZE_FIRST
    sdpa.DEQUANTIZE_FIRST = False
    try:
        fused = sdpa.scaled_dot_product_attention(*args, **kw)
    finally:
        sdpa.DEQUANTIZE_FIRST = old
    torch.cuda.synchronize()
    assert torch.equal(got, fused)
    if sdpa_block == 0:  # the oracle once per case (the chunkings are tied to it by the other tests)
        ref = oa.sdpa_q8(q, K, V, 0.0884, vis, sinks, n=N, dtype=dtype)
        assert np.abs(_np(got) - ref).max() <= _tol(ref, dtype)


def test_left_padding_start(dev):
    """start[b] masks the keys before it, like the batch cache's left padding."""
    from locals_amd.sdpa import scaled_dot_product_attention

    g = rng(9)
    B, H, KVH, L, N, cap = 3, 8, 2, 5, 200, 256
    q = normal16(g, (B, H, L, 128))
    K, V = q8_cache(g, B, KVH, cap)
    start = np.array([0, 17, 150], np.int32)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    got = scaled_dot_product_attention(to_torch(q, dev), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.1, mask="causal",
                                       start=to_torch(start, dev))
    torch.cuda.synchronize()
    vis = oa.causal_mask(L, N)[None, None] & (np.arange(N)[None, None, None, :] >= start[:, None, None, None])
    ref = oa.sdpa_q8(q, K, V, 0.1, vis, None, n=N)
    assert np.abs(_np(got) - ref).max() <= 2e-3


def test_chunk_equals_tokens_one_by_one(dev):
    """A causal chunk of L queries equals L one-query passes over the growing prefix (the 8-bit decode kernel)."""
    from locals_amd import qkv
    from locals_amd.sdpa import scaled_dot_product_attention

    g = rng(10)
    B, H, KVH, L, N, cap = 1, 32, 8, 12, 400, 512
    q = normal16(g, (B, H, L, 128))
    K, V = q8_cache(g, B, KVH, cap)
    sinks = normal16(g, (H,), 2.0)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    qt, st = to_torch(q, dev), to_torch(sinks, dev)
    chunk = scaled_dot_product_attention(qt, tuple(a[:, :, :N] for a in Kt), tuple(a[:, :, :N] for a in Vt),
                                         scale=0.0884, mask="causal", sinks=st)
    for i in range(L):
        one = qkv.attend(qt[:, :, i:i + 1].contiguous(), Kt, Vt, N - L + i + 1, st, 0.0884,
                         torch.zeros(B, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        assert np.abs(_np(one)[:, :, 0] - _np(chunk)[:, :, i]).max() <= 2e-3


def test_chain_tree_is_causal(dev):
    from locals_amd.sdpa import TreeMask, scaled_dot_product_attention

    g = rng(11)
    B, H, KVH, L, N = 2, 8, 2, 10, 90
    q = normal16(g, (B, H, L, 128))
    k = normal16(g, (B, KVH, N, 128))
    v = normal16(g, (B, KVH, N, 128))
    args = (to_torch(q, dev), to_torch(k, dev), to_torch(v, dev))
    a = scaled_dot_product_attention(*args, scale=0.1, mask="causal")
    b = scaled_dot_product_attention(*args, scale=0.1, mask=TreeMask.from_parents(list(range(-1, L - 1)), dev))
    c = scaled_dot_product_attention(*args, scale=0.1, mask=TreeMask.from_branches([-1] * L, dev))
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("L", [5, 6, 7, 8])
def test_attend_few_five_to_eight(dev, L):
    """attend_few needs no padding: the real queries get what unpadded MLX attention gives them, under the causal
    mask, a window mask (2-D and per row), or none (the reference test's cases)."""
    from locals_amd.fuse import attend_few

    g = rng(20 + L)
    B, H, KVH, n = 2, 8, 2, 40
    q = normal16(g, (B, H, L, 128), dtype="bfloat16")
    k = normal16(g, (B, KVH, n, 128), dtype="bfloat16")
    v = normal16(g, (B, KVH, n, 128), dtype="bfloat16")
    sinks = normal16(g, (H,), 1.0, dtype="bfloat16")
    window = (np.arange(n)[None, :] <= (n - L + np.arange(L))[:, None]) & \
             (np.arange(n)[None, :] > (n - L + np.arange(L))[:, None] - 9)
    f = lambda a: oq.to_f32(a, "bfloat16")  # noqa: E731
    for mask, ref_mask in (("causal", "causal"), (None, None), (torch.from_numpy(window).to(dev), window[None, None]),
                           (torch.from_numpy(np.broadcast_to(window, (B, 1, L, n)).copy()).to(dev),
                            np.broadcast_to(window, (B, 1, L, n)))):
        got = attend_few(to_torch(q, dev, "bfloat16"), to_torch(k, dev, "bfloat16"), to_torch(v, dev, "bfloat16"),
                         0.09, mask, to_torch(sinks, dev, "bfloat16"))
        torch.cuda.synchronize()
        ref = oa.sdpa(f(q), f(k), f(v), 0.09, ref_mask, f(sinks), dtype="float64")
        assert np.abs(_np(got) - ref).max() <= 1e-2 * (1 + np.abs(ref).max())


def test_qkv_attention_prompt_branch(dev):
    """qkv.attention with L > 1 stores the chunk in the 8-bit cache and attends through the masked kernel."""
    from locals_amd import qkv

    g = rng(12)
    B, H, KVH, L0, L = 1, 8, 2, 100, 7
    cache = qkv.QuantizedKVCache8()
    k0, v0 = normal16(g, (B, KVH, L0, 128)), normal16(g, (B, KVH, L0, 128))
    cache.update_and_fetch(to_torch(k0, dev), to_torch(v0, dev))
    q = normal16(g, (B, H, L, 128))
    k1, v1 = normal16(g, (B, KVH, L, 128)), normal16(g, (B, KVH, L, 128))
    sinks = normal16(g, (H,), 1.0)
    out = qkv.attention(to_torch(q, dev), to_torch(k1, dev), to_torch(v1, dev), cache, 0.0884, "causal",
                        to_torch(sinks, dev))
    torch.cuda.synchronize()
    K = oq.quantize(np.concatenate([k0, k1], 2))
    V = oq.quantize(np.concatenate([v0, v1], 2))
    ref = oa.sdpa_q8(q, K, V, 0.0884, "causal", sinks)
    assert np.abs(_np(out) - ref).max() <= 2e-3


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_qkv_attention_prompt_branch_fp32_sinks(dev, dtype):
    """A model's sinks are fp32 parameters; the prompt branch hands them over cast to q's dtype (locals/qkv.py:272),
    so the output equals the call given the rounded sinks, bit for bit, and the oracle of that branch."""
    from locals_amd import qkv

    g = rng(13)
    B, H, KVH, L0, L = 1, 8, 2, 300, 9
    cache = qkv.QuantizedKVCache8()
    k0, v0 = normal16(g, (B, KVH, L0, 128), dtype=dtype), normal16(g, (B, KVH, L0, 128), dtype=dtype)
    cache.update_and_fetch(to_torch(k0, dev, dtype), to_torch(v0, dev, dtype))
    q = normal16(g, (B, H, L, 128), dtype=dtype)
    k1, v1 = normal16(g, (B, KVH, L, 128), dtype=dtype), normal16(g, (B, KVH, L, 128), dtype=dtype)
    s32 = (3.0 + g.standard_normal(H)).astype(np.float32)  # sinks that carry a tenth of the softmax weight
    qt = to_torch(q, dev, dtype)
    out = qkv.attention(qt, to_torch(k1, dev, dtype), to_torch(v1, dev, dtype), cache, 0.0884, "causal",
                        torch.from_numpy(s32).to(dev))
    again = qkv.attend_cache(qt, cache, 0.0884, "causal", torch.from_numpy(s32).to(dev).to(qt.dtype))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    K = oq.quantize(np.concatenate([k0, k1], 2), dtype)
    V = oq.quantize(np.concatenate([v0, v1], 2), dtype)
    ref = oa.attention_prompt(q, K, V, 0.0884, "causal", s32, n=L0 + L, dtype=dtype)
    assert np.abs(_np(out) - ref).max() <= _tol(ref, dtype)


@pytest.mark.parametrize("kvdt", ["float16", "bfloat16"])
@pytest.mark.parametrize("W", [1, 37, 129, 513, 100000])
def test_window_16bit(dev, kvdt, W):
    """A sliding-window layer's prompt chunk (fuse.banded, the reference's _banded, locals/fuse.py:113-125) over
    16-bit K/V: Flint's head ratio (G = 8), the chunk after a ring of 512 earlier keys; windows from the query alone
    to wider than every key (then the causal mask)."""
    from locals_amd import fuse

    print(f"window 16-bit W={W} {kvdt}", flush=True)
    g = rng(30 + W)
    B, H, KVH, L, N = 1, 16, 2, 300, 812
    q = normal16(g, (B, H, L, 128), dtype=kvdt)
    k = normal16(g, (B, KVH, N, 128), dtype=kvdt)
    v = normal16(g, (B, KVH, N, 128), dtype=kvdt)
    sinks = normal16(g, (H,), 1.0, dtype=kvdt)
    got = fuse.banded(to_torch(q, dev, kvdt), to_torch(k, dev, kvdt), to_torch(v, dev, kvdt), W, 0.09,
                      to_torch(sinks, dev, kvdt))
    torch.cuda.synchronize()
    f = lambda a: oq.to_f32(a, kvdt)  # noqa: E731
    ref = oa.sdpa(f(q), f(k), f(v), 0.09, oa.window_mask(L, N, W)[None, None], f(sinks), dtype="float64")
    assert np.abs(_np(got) - ref).max() <= _tol(ref, kvdt)


@pytest.mark.parametrize("W", [7, 100, 700])
def test_window_q8_left_padded(dev, W):
    """The window over 8-bit K/V (two row tiles a wave), with left padding: row 2's first queries have their whole
    window before its start and give 0; sinks present."""
    from locals_amd.sdpa import WindowMask, scaled_dot_product_attention

    print(f"window q8 W={W}", flush=True)
    g = rng(40 + W)
    B, H, KVH, L, N, cap = 3, 32, 4, 64, 700, 768
    q = normal16(g, (B, H, L, 128))
    K, V = q8_cache(g, B, KVH, cap)
    sinks = normal16(g, (H,), 2.0)
    start = np.array([0, 17, 690], np.int32)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    got = scaled_dot_product_attention(to_torch(q, dev), tuple(a[:, :, :N] for a in Kt),
                                       tuple(a[:, :, :N] for a in Vt), scale=0.0884, mask=WindowMask(W),
                                       sinks=to_torch(sinks, dev), start=to_torch(start, dev))
    torch.cuda.synchronize()
    vis = oa.window_mask(L, N, W)[None, None] & (np.arange(N)[None, None, None, :] >= start[:, None, None, None])
    ref = oa.sdpa_q8(q, K, V, 0.0884, vis, sinks, n=N)
    assert np.abs(_np(got) - ref).max() <= 2e-3
    blind = ~vis[2, 0].any(-1)  # row 2's queries that see no key
    assert blind.any() and not np.abs(_np(got)[2][:, blind]).any()


def test_query_with_no_visible_key_is_zero(dev):
    """A query whose mask row is all false gives 0, sink or not, in every chunking (with one chunk pass 1 writes
    the output itself)."""
    from locals_amd.sdpa import scaled_dot_product_attention

    g = rng(13)
    B, H, KVH, L, N = 2, 8, 2, 6, 150
    q = normal16(g, (B, H, L, 128))
    k = normal16(g, (B, KVH, N, 128))
    v = normal16(g, (B, KVH, N, 128))
    vis = g.random((B, 1, L, N)) < 0.3
    vis[:, :, 2] = False
    vis[1, :, 4] = False
    for sinks in (None, normal16(g, (H,), 1.0)):
        got = scaled_dot_product_attention(to_torch(q, dev), to_torch(k, dev), to_torch(v, dev), scale=0.1,
                                           mask=torch.from_numpy(vis).to(dev),
                                           sinks=None if sinks is None else to_torch(sinks, dev))
        torch.cuda.synchronize()
        out = _np(got)
        assert not np.abs(out[:, :, 2]).any() and not np.abs(out[1, :, 4]).any()
        ref = oa.sdpa(q, k, v, 0.1, vis, sinks, dtype="float16")
        assert np.abs(out - ref).max() <= 2e-3
