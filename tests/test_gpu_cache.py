"""GPU row moves of the 8-bit caches (lcl_kv_gather behind merge / extend / filter / extract / finalize,
locals/qkv.py:340-440) compared byte for byte with the oracle's restatement (oracle/cache.py, pinned by hand in
tests/test_oracle.py), and prompt-cache snapshots (the reference's DiskPromptCache, locals/hybrid_batch.py:332-455)
saved and loaded back: the restored caches decode bit-identically to the originals."""

import numpy as np
import pytest
import torch

from oracle import cache as oc
from tests.inputs import normal16, rng, to_torch

pytestmark = pytest.mark.gpu


def _rand_triple(B, KVH, cap, seed, dev, dtype=torch.float16):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (B, KVH, cap, 32), generator=g, device=dev, dtype=torch.int64)
    s = torch.randint(-2 ** 15, 2 ** 15 - 1, (B, KVH, cap, 2), generator=g, device=dev, dtype=torch.int64)
    b = torch.randint(-2 ** 15, 2 ** 15 - 1, (B, KVH, cap, 2), generator=g, device=dev, dtype=torch.int64)
    return (w.to(torch.int32), s.to(torch.int16).view(dtype), b.to(torch.int16).view(dtype))


def _np(t):
    return (t[0].cpu().numpy().view(np.uint32), t[1].cpu().view(torch.int16).numpy().view(np.uint16),
            t[2].cpu().view(torch.int16).numpy().view(np.uint16))


def _same(got, want):
    g = _np(got)
    assert len(g) == len(want)
    for a, b in zip(g, want):
        assert a.shape == b.shape and np.array_equal(a, b)


def _single(dev, n, cap, seed):
    from locals_amd import qkv

    c = qkv.QuantizedKVCache8()
    c.keys, c.values = _rand_triple(1, 2, cap, seed, dev), _rand_triple(1, 2, cap, seed + 100, dev)
    c.offset = n
    return c


def test_merge_extend_filter_extract_match_oracle(dev):
    from locals_amd import qkv

    singles = [_single(dev, 700, 768, 1), _single(dev, 300, 512, 2), qkv.QuantizedKVCache8(), _single(dev, 1, 256, 3)]
    b = qkv.QuantizedKVCache8.merge(singles)
    ok = oc.merge([(None if c.keys is None else _np(c.keys), c.offset) for c in singles], KVH=2)
    ov = oc.merge([(None if c.keys is None else _np(c.values), c.offset) for c in singles], KVH=2)
    _same(b.keys, ok["keys"])
    _same(b.values, ov["keys"])
    assert b._idx == ok["idx"] and b.left_padding.tolist() == ok["left_padding"].tolist()
    assert b.offset.tolist() == ok["offset"].tolist()
    # a decode step grows it to 700 + 256 positions (locals/qkv.py:311-319); the step's keys land at 700 on every row
    g = rng(5)
    k1, v1 = normal16(g, (4, 2, 1, 128)), normal16(g, (4, 2, 1, 128))
    b.update_and_fetch(to_torch(k1, dev), to_torch(v1, dev))
    assert b.keys[0].shape[2] == 956
    for o, buf in ((ok, b.keys), (ov, b.values)):
        o["keys"] = oc.grow(o["keys"], 700, 1, KVH=2, B=4)
        for a, x in zip(o["keys"], _np(tuple(t[:, :, 700:701] for t in buf))):  # the quantized step itself
            a[:, :, 700:701] = x
        o["idx"], o["offset"] = 701, o["offset"] + 1
    _same(b.keys, ok["keys"])
    _same(b.values, ov["keys"])
    # extend with a batch of a longer request (1000 keys): every row moves right by 299, the capacity is 1000 and
    # what passes it is cut
    other = qkv.QuantizedKVCache8.merge([_single(dev, 1000, 1024, 7)])
    okb = {"keys": _np(other.keys), "left_padding": np.array([0]), "offset": np.array([1000]), "idx": 1000}
    ovb = {"keys": _np(other.values), "left_padding": np.array([0]), "offset": np.array([1000]), "idx": 1000}
    b.extend(other)
    ok = oc.extend(ok, okb, KVH=2)
    ov = oc.extend(ov, ovb, KVH=2)
    _same(b.keys, ok["keys"])
    _same(b.values, ov["keys"])
    assert b._idx == ok["idx"] == 1000 and b.left_padding.tolist() == ok["left_padding"].tolist()
    # filter rows 2, 1 (reordered; their common padding, 699, goes)
    b.filter([2, 1])
    ok, ov = oc.filter_rows(ok, [2, 1]), oc.filter_rows(ov, [2, 1])
    assert ok["idx"] == 301
    _same(b.keys, ok["keys"])
    _same(b.values, ov["keys"])
    assert b._idx == ok["idx"] and b.left_padding.tolist() == ok["left_padding"].tolist()
    # extract row 1: exactly its live positions
    e = b.extract(1)
    ek, n = oc.extract(ok, 1)
    ev, _ = oc.extract(ov, 1)
    _same(e.keys, ek)
    _same(e.values, ev)
    assert e.offset == n


def test_finalize_rolls_right_padding(dev):
    """prepare(right_padding) + a prompt chunk + finalize: each row's keys rolled right by its padding
    (locals/qkv.py:340-346), the padding moved to the left."""
    from locals_amd import qkv

    c = qkv.BatchQuantizedKVCache([0, 0, 0], device=dev)
    c.prepare(right_padding=[0, 5, 37])
    g = rng(6)
    k, v = normal16(g, (3, 2, 100, 128)), normal16(g, (3, 2, 100, 128))
    c.update_and_fetch(to_torch(k, dev), to_torch(v, dev))
    before = {"keys": _np(c.keys), "left_padding": np.zeros(3, int), "offset": np.full(3, 100), "idx": 100}
    beforev = {"keys": _np(c.values), "left_padding": np.zeros(3, int), "offset": np.full(3, 100), "idx": 100}
    c.finalize()
    want, wantv = oc.finalize(before, [0, 5, 37]), oc.finalize(beforev, [0, 5, 37])
    _same(c.keys, want["keys"])
    _same(c.values, wantv["keys"])
    assert c.left_padding.tolist() == [0, 5, 37] and c.offset.tolist() == [100, 95, 63]


def test_snapshot_round_trip_decodes_identically(dev, tmp_path):
    """A request's 8-bit caches (two layers) written by save_prompt_cache and read by load_prompt_cache hold the
    same bytes, and decode the next token bit-identically, alone and merged into a batch."""
    from locals_amd import qkv

    g = rng(8)
    layers = [qkv.QuantizedKVCache8() for _ in range(2)]
    for c in layers:
        for L in (300, 1, 1):  # a prompt chunk, then two decode steps
            k, v = normal16(g, (1, 2, L, 128), dtype="bfloat16"), normal16(g, (1, 2, L, 128), dtype="bfloat16")
            c.update_and_fetch(to_torch(k, dev, "bfloat16"), to_torch(v, dev, "bfloat16"))
    path = str(tmp_path / "prompt.safetensors")
    qkv.save_prompt_cache(path, layers, {"tokens": "302"})
    back, meta = qkv.load_prompt_cache(path, device=dev, return_metadata=True)
    assert meta == {"tokens": "302"}
    q = to_torch(normal16(g, (1, 8, 1, 128), dtype="bfloat16"), dev, "bfloat16")
    sinks = torch.randn(8, device=dev)
    for c0, c1 in zip(layers, back):
        assert c1.offset == c0.offset == 302
        for a, x in zip(c0.state[0] + c0.state[1], c1.keys + c1.values):
            assert torch.equal(a, x)
        o0 = qkv.attend_cache(q, c0, 0.0884, None, sinks)
        o1 = qkv.attend_cache(q, c1, 0.0884, None, sinks)
        assert torch.equal(o0.view(torch.int16), o1.view(torch.int16))
    m0 = qkv.QuantizedKVCache8.merge([layers[0], layers[1]])
    m1 = qkv.QuantizedKVCache8.merge([back[0], back[1]])
    qq = torch.cat([q, q])
    assert torch.equal(qkv.attend_cache(qq, m0, 0.0884, None, sinks).view(torch.int16),
                       qkv.attend_cache(qq, m1, 0.0884, None, sinks).view(torch.int16))


@pytest.mark.parametrize("D", [128, 64])
def test_move_rows_every_case(dev, D):
    """qkv.move_rows (lcl_kv_gather) on its own, byte for byte against its definition: 40 destination rows (two
    launches of 32 + 8), sources of different capacities, shifts below 0, 0 and above, lengths 0 / partial / whole,
    rolls with every shift sign, a missing source, and a second kv-head layout (D = 64: 16 words, one scale)."""
    from locals_amd import qkv

    g = np.random.default_rng(77 + D)
    KVH, cap = 3, 300

    def rand_triple(B, c, seed):
        t = _rand_triple(B, KVH, c, seed, dev)
        if D == 64:
            t = (t[0][..., :16].contiguous(), t[1][..., :1].contiguous(), t[2][..., :1].contiguous())
        return t

    srcs = [(rand_triple(4, c, 10 + i), rand_triple(4, c, 50 + i)) for i, c in enumerate((256, 300, 512))]
    rows = []
    for r in range(40):
        si = int(g.integers(0, 3))
        keys, values = srcs[si]
        scap = keys[0].shape[2]
        n = int(g.choice([0, 1, scap // 3, scap]))
        shift = int(g.integers(-scap, cap))
        wrap = bool(g.integers(0, 2))
        if r == 7:
            keys = values = None
        rows.append((keys, values, int(g.integers(0, 4)), shift, n, wrap))
    like = srcs[0]
    got_k, got_v = qkv.move_rows(rows, cap, like)
    torch.cuda.synchronize()
    for which, got in ((0, got_k), (1, got_v)):
        g_np = _np(got)
        for a in range(3):
            want = np.zeros_like(g_np[a])
            for r, (keys, values, row, shift, n, wrap) in enumerate(rows):
                src = keys if which == 0 else values
                if src is None or n == 0:
                    continue
                s = _np(src)[a][row]  # (KVH, scap, per)
                t = np.arange(cap) - shift
                if wrap:
                    want[r] = s[:, np.mod(t, n)]
                else:
                    ok = (t >= 0) & (t < n)
                    want[r][:, ok] = s[:, t[ok]]
            assert np.array_equal(g_np[a], want), (which, a)
