"""Pins the CPU oracle (oracle/) against checks that do not restate it.

Quantizer: hand-derived MLX closed-form groups (tests/golden/quant_known.npz), both tie modes, the
dequantization error bound, edge-to-code-0, and agreement with the independent C restatement.
Attention: torch's CPU float64 scaled_dot_product_attention (sink = extra zero key with additive mask) on the
golden cases and on random ones; invariants of the reference's split-K algebra (block size, key permutation,
GQA == MHA with repeated K/V, single key, empty range, garbage outside [start, n)).
Masks: chain tree == causal, the reference's branch formula == ancestor-or-self of the parent array, brute force;
the sliding window against a brute-force ring buffer, and banded == whole under the window mask.
qk_norm_rope: torch RMS norm + complex RoPE in float64 within the reference's bar 0.02 max|ref|
(tests/test_flint.py:235-236); v bit-exact.
"""

import os

import numpy as np
import pytest
import torch

from oracle import attn as oa
from oracle import cbind
from oracle import quant as oq

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ------------------------------------------------------------------ quantizer
@pytest.mark.parametrize("mode", ["away", "even"])
def test_quantize_known_groups(mode):
    g = _gold("quant_known.npz")
    w, s, b = oq.quantize(g["x"], round_mode=mode)
    assert np.array_equal(oq.codes_of(w), g["codes"])
    assert np.array_equal(s.view(np.uint16), g["scales"].view(np.uint16))
    assert np.array_equal(b.view(np.uint16), g["biases"].view(np.uint16))


def test_quantize_tie_modes():
    g = _gold("quant_known.npz")
    assert np.array_equal(oq.codes_of(oq.quantize(g["tie"], round_mode="away")[0]), g["tie_away"])
    assert np.array_equal(oq.codes_of(oq.quantize(g["tie"], round_mode="even")[0]), g["tie_even"])
    assert not np.array_equal(g["tie_away"], g["tie_even"])


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("mode", ["away", "even"])
def test_quantize_error_bound_and_edge(dtype, mode):
    g = np.random.default_rng(1)
    x = oq.from_f32((g.standard_normal((500, 128)) * np.exp(g.uniform(-4, 4, (500, 1)))).astype(np.float32), dtype)
    w, s, b = oq.quantize(x, dtype, round_mode=mode)
    xf = oq.to_f32(x, dtype).astype(np.float64).reshape(500, 2, 64)
    c = oq.codes_of(w).astype(np.float64).reshape(500, 2, 64)
    sf = oq.to_f32(s, dtype).astype(np.float64)[..., None]
    bf = oq.to_f32(b, dtype).astype(np.float64)[..., None]
    # the fp32 scale/bias put an interior code within half a step; MLX's zero-point step (scale = edge / q0 with
    # |q0| >= 128) can push the far extreme at most one step past 255, where it is clamped (1.5 steps).  The
    # 16-bit rounding of scale and bias adds at most 255 half-ulps of the scale and a half-ulp of the bias.
    ulp = 2.0 ** (-10 if dtype == "float16" else -7)
    fp16_terms = 255 * np.abs(sf) * ulp / 2 + np.abs(bf) * ulp / 2 + 1e-30
    err = np.abs(c * sf + bf - xf)
    interior = (c > 0) & (c < 255)
    assert (err <= (np.abs(sf) / 2 * (1 + 1e-5) + fp16_terms) * 1.0001)[interior].all()
    assert (err <= (np.abs(sf) * 1.5 * (1 + 1e-5) + fp16_terms) * 1.0001).all()
    # the edge (the extreme of larger magnitude) maps to code 0, the other extreme near 255
    edge = np.where(np.abs(xf.min(-1)) > np.abs(xf.max(-1)), xf.argmin(-1), xf.argmax(-1))
    assert (np.take_along_axis(c, edge[..., None], -1) == 0).all()
    assert (c.max(-1) >= 254).all()


@pytest.mark.parametrize("mode", ["away", "even"])
def test_quantize_numpy_equals_c(mode):
    g = np.random.default_rng(2)
    x = (g.standard_normal((3, 7, 50, 128)) * 3).astype(np.float16)
    a = oq.quantize(x, round_mode=mode)
    b = cbind.quantize(x, round_mode=mode)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


# ------------------------------------------------------------------ attention
def _sdpa64(q, k, v, scale, vis, sinks):
    from tests.golden.make_golden import sdpa64

    return sdpa64(q, k, v, scale, vis, sinks)


def test_sdpa_golden_cases():
    g = _gold("attn_sdpa.npz")
    out = oa.sdpa(g["dec_q"], g["dec_k"], g["dec_v"], 0.0884,
                  mask=(np.arange(40)[None, None, None, :] >= g["dec_start"][:, None, None, None]),
                  sinks=g["dec_sinks"])
    assert np.abs(out - g["dec_out"]).max() < 1e-9
    out = oa.sdpa(g["cau_q"], g["cau_k"], g["cau_v"], 0.1, mask="causal")
    assert np.abs(out - g["cau_out"]).max() < 1e-9
    local = oa.ancestor_mask(g["tree_parents"])
    out = oa.sdpa(g["tree_q"], g["tree_k"], g["tree_v"], 0.0884, mask=oa.tree_full_mask(local, 9)[None, None],
                  sinks=g["tree_sinks"])
    assert np.abs(out - g["tree_out"]).max() < 1e-9


def _q8_case(seed, B=3, H=8, KVH=2, cap=300):
    g = np.random.default_rng(seed)
    q = g.standard_normal((B, H, 1, 128)).astype(np.float16)
    K = oq.quantize((g.standard_normal((B, KVH, cap, 128)) * 2).astype(np.float16))
    V = oq.quantize(g.standard_normal((B, KVH, cap, 128)).astype(np.float16))
    sinks = (g.standard_normal(H) * 2).astype(np.float16)
    return g, q, K, V, sinks


def test_attend_equals_torch_sdpa_over_dequantized():
    g, q, K, V, sinks = _q8_case(3)
    n, start = 257, np.array([0, 13, 200], np.int32)
    kd, vd = oq.dequantize(*K), oq.dequantize(*V)
    vis = np.arange(n)[None, None, None, :] >= start[:, None, None, None]
    ref = _sdpa64(q, kd[:, :, :n], vd[:, :, :n], float(np.float32(0.0884)), vis, sinks.astype(np.float64))
    assert np.abs(oa.attend(q, K, V, n, sinks, 0.0884, start) - ref).max() < 1e-9


def test_attend_invariants():
    g, q, K, V, sinks = _q8_case(4, B=2)
    n, start = 290, np.array([0, 31], np.int32)
    base = oa.attend(q, K, V, n, sinks, 0.0884, start)
    # key permutation inside each row's range
    perm = np.arange(K[0].shape[2])
    perm[31:n] = 31 + g.permutation(n - 31)
    perm[:31] = g.permutation(31)
    Kp, Vp = tuple(a[:, :, perm] for a in K), tuple(a[:, :, perm] for a in V)
    start0 = np.array([0, 31], np.int32)
    # row 0 sees [0, n): permuting [0,31) and [31,n) separately keeps its key set
    assert np.abs(oa.attend(q, Kp, Vp, n, sinks, 0.0884, start0) - base).max() < 1e-9
    # GQA == MHA with K/V repeated G times
    G = q.shape[1] // K[0].shape[1]
    Kr, Vr = tuple(np.repeat(a, G, axis=1) for a in K), tuple(np.repeat(a, G, axis=1) for a in V)
    assert np.abs(oa.attend(q, Kr, Vr, n, sinks, 0.0884, start) - base).max() < 1e-12
    # sinks = -inf is plain softmax, i.e. torch SDPA without the extra key
    kd, vd = oq.dequantize(*K), oq.dequantize(*V)
    vis = np.arange(n)[None, None, None, :] >= start[:, None, None, None]
    ref = _sdpa64(q, kd[:, :, :n], vd[:, :, :n], float(np.float32(0.0884)), vis, None)
    assert np.abs(oa.attend(q, K, V, n, None, 0.0884, start) - ref).max() < 1e-9
    # empty range -> 0; a single key without a sink -> that key's value
    e = oa.attend(q, K, V, 5, None, 0.0884, np.array([5, 4], np.int32))
    assert (e[0] == 0).all()
    assert np.abs(e[1] - vd[1, np.arange(q.shape[1]) // G, 4][:, None]).max() < 1e-12


@pytest.mark.parametrize("block", [64, 128, 1024, 0])
def test_c_split_k_matches_closed_form(block):
    """The C restatement of qkv.py's two passes equals the float64 closed form for any block size, and ignores
    NaN/inf garbage outside each row's [start, n)."""
    g, q, K, V, sinks = _q8_case(5, B=3, H=16, KVH=4, cap=768)
    n, start = 700, np.array([0, 37, 300], np.int32)
    ref = oa.attend(q, K, V, n, sinks, 0.0884, start)
    Kg = (K[0], K[1].copy(), K[2].copy())
    Kg[1][0, :, n:] = np.float16(np.nan)
    Kg[2][2, :, :300] = np.float16(np.inf)
    got = cbind.attend_q8(q, Kg, V, n, sinks, 0.0884, start, block=block)
    assert np.abs(got - ref).max() < 2e-5


def test_causal_alignment_and_chain_tree():
    # the last query of "causal" sees every key; query i sees N - L + i + 1 keys
    m = oa.causal_mask(5, 12)
    assert m[-1].all() and [int(r.sum()) for r in m] == [8, 9, 10, 11, 12]
    # a chain tree (parents i-1) is the causal mask over the new tokens
    assert np.array_equal(oa.ancestor_mask(np.arange(-1, 6)), oa.causal_mask(7, 7))


def test_branch_mask_is_ancestor_mask():
    """The reference's formula (locals/treedec.py:56-67): main path then branches laid out contiguously; as a
    tree, each branch hangs off the last main token."""
    g = np.random.default_rng(6)
    for _ in range(20):
        m = int(g.integers(1, 5))
        lens = g.integers(1, 4, size=int(g.integers(1, 4)))
        br = [-1] * m
        parents = list(range(-1, m - 1))
        for i, ln in enumerate(lens):
            for j in range(ln):
                parents.append(m - 1 if j == 0 else len(br) - 1)
                br.append(i)
        assert np.array_equal(oa.branch_mask(br), oa.ancestor_mask(parents))


def test_ancestor_mask_brute_force():
    g = np.random.default_rng(7)
    for _ in range(20):
        L = int(g.integers(1, 17))
        parents = [-1] + [int(g.integers(0, i)) for i in range(1, L)]
        m = oa.ancestor_mask(parents)
        for i in range(L):
            anc = {i}
            j = parents[i]
            while j >= 0:
                anc.add(j)
                j = parents[j]
            assert set(np.nonzero(m[i])[0].tolist()) == anc


def test_window_mask_is_the_rotating_ring():
    """The sliding-window mask against a brute-force ring of W slots (what a RotatingKVCache of max_size W holds
    after writing positions 0..pos: the keys query pos attends to), its closed-form row counts, W >= N being the
    causal mask, and the host mask builder (mlx-lm's create_causal_mask with window_size)."""
    from locals_amd import qkv

    for L, N, W in ((5, 12, 3), (12, 12, 1), (7, 30, 9), (16, 16, 40), (9, 9, 9)):
        m = oa.window_mask(L, N, W)
        for i in range(L):
            pos = N - L + i
            ring = [-1] * W
            for t in range(pos + 1):
                ring[t % W] = t
            assert set(np.nonzero(m[i])[0].tolist()) == {t for t in ring if t >= 0}
            assert int(m[i].sum()) == min(W, pos + 1) and m[i, pos] and not m[i, pos + 1:].any()
        if W >= N:
            assert np.array_equal(m, oa.causal_mask(L, N))
        host = qkv.create_causal_mask(L, offset=N - L, window_size=W, device="cpu").numpy()
        assert np.array_equal(host, m)


@pytest.mark.parametrize("band", [1, 4, 7, 64])
def test_banded_window_equals_whole_masked(band):
    """The reference's own check (tests/test_flint.py:458-476): the chunk's attention band by band over the keys
    each band's window reaches equals one attention over every key under the window's mask; and a window of one
    key gives the query's own value (no sink)."""
    g = np.random.default_rng(10)
    B, H, KVH, L, N = 2, 4, 2, 13, 20
    q = g.standard_normal((B, H, L, 128))
    k = g.standard_normal((B, KVH, N, 128))
    v = g.standard_normal((B, KVH, N, 128))
    s = g.standard_normal(H)
    for W in (1, 3, 9, 100):
        whole = oa.sdpa(q, k, v, 0.09, oa.window_mask(L, N, W)[None, None], s, dtype="float64")
        assert np.abs(oa.banded_sdpa(q, k, v, 0.09, W, s, band=band, dtype="float64") - whole).max() < 1e-12
        ref = _sdpa64(q, k, v, 0.09, oa.window_mask(L, N, W)[None, None], s)
        assert np.abs(whole - ref).max() < 1e-9
    one = oa.sdpa(q, k, v, 0.09, oa.window_mask(L, N, 1)[None, None], None, dtype="float64")
    assert np.abs(one - np.repeat(v[:, :, N - L:], H // KVH, axis=1)).max() < 1e-12


def test_sdpa_random_masks_vs_torch():
    g = np.random.default_rng(8)
    q = g.standard_normal((2, 8, 5, 128))
    k = g.standard_normal((2, 4, 23, 128))
    v = g.standard_normal((2, 4, 23, 128))
    vis = g.random((2, 1, 5, 23)) < 0.6
    vis[..., 0] = True
    s = g.standard_normal(8)
    ref = _sdpa64(q, k, v, 0.09, vis, s)
    assert np.abs(oa.sdpa(q, k, v, 0.09, mask=vis, sinks=s, dtype="float64") - ref).max() < 1e-9


def test_ragged_vs_torch():
    g = np.random.default_rng(9)
    q = g.standard_normal((4, 8, 128))
    K = g.standard_normal((3, 2, 50, 128))
    V = g.standard_normal((3, 2, 50, 128))
    slots, nkeys = np.array([2, 0, 1, 2]), np.array([50, 1, 0, 17])
    out = oa.ragged_attention(q, K, V, slots, nkeys, np.array([0.125], np.float32))
    for r in range(4):
        if nkeys[r] == 0:
            assert (out[r] == 0).all()
            continue
        kk, vv = K[slots[r]][:, :nkeys[r]][None], V[slots[r]][:, :nkeys[r]][None]
        ref = _sdpa64(q[r][None, :, None], kk, vv, 0.125, np.ones((1, 1, 1, nkeys[r]), bool), None)
        assert np.abs(out[r] - ref[0, :, 0]).max() < 1e-9


# ------------------------------------------------------------------ qk_norm_rope
@pytest.mark.parametrize("rope", [True, False])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("HD,offs", [(128, [4, 0, 77]), (256, [-3, 1000, 9])])
def test_qk_norm_rope_vs_torch(rope, dtype, HD, offs):
    """The oracle against torch's RMS norm and a complex-exponential RoPE in float64: within four rounding steps of
    T relative to each (lo, hi) pair's size (a dropped term, a swapped half or a wrong sign is O(1) off); v exact."""
    g = np.random.default_rng(10)
    B, L, H, KV = 3, 4, 4, 2
    x = oq.to_f32(oq.from_f32((g.standard_normal((B, L, (H + 2 * KV) * HD)) * 2).astype(np.float32), dtype), dtype)
    qw = oq.to_f32(oq.from_f32((1 + 0.05 * g.standard_normal(HD)).astype(np.float32), dtype), dtype)
    kw = oq.to_f32(oq.from_f32((1 + 0.05 * g.standard_normal(HD)).astype(np.float32), dtype), dtype)
    offs = np.array(offs)
    q, k, v = oa.qk_norm_rope(x, qw, kw, 1e-6, offs, H, KV, HD, rope, 10000.0, dtype)
    t = torch.from_numpy(x.astype(np.float64)).reshape(B, L, H + 2 * KV, HD)

    def norm(a, w):
        return a * torch.rsqrt((a * a).mean(-1, keepdim=True) + 1e-6) * torch.from_numpy(w.astype(np.float64))

    def rot(a):
        pos = torch.from_numpy(offs)[:, None].double() + torch.arange(L)[None].double()  # (B, L)
        inv = 10000.0 ** (-torch.arange(HD // 2).double() * 2 / HD)
        ang = pos[:, :, None, None] * inv  # (B, L, 1, HD/2)
        z = torch.complex(a[..., :HD // 2], a[..., HD // 2:]) * torch.exp(1j * ang)
        return torch.cat([z.real, z.imag], -1)

    q0 = norm(t[:, :, :H], qw)
    k0 = norm(t[:, :, H:H + KV], kw)
    if rope:
        q0, k0 = rot(q0), rot(k0)
    q0, k0 = q0.permute(0, 2, 1, 3).numpy(), k0.permute(0, 2, 1, 3).numpy()
    ulp = 2.0 ** (-11 if dtype == "float16" else -8)
    for got, ref in ((q, q0), (k, k0)):
        pair = np.maximum(np.abs(ref[..., :HD // 2]), np.abs(ref[..., HD // 2:]))
        bound = 4 * ulp * np.concatenate([pair, pair], -1) + 1e-6
        assert np.all(np.abs(got - ref) <= bound), np.abs(got - ref).max()
    assert np.array_equal(v, x.reshape(B, L, H + 2 * KV, HD)[:, :, H + KV:].transpose(0, 2, 1, 3))


def test_qk_norm_rope_position_zero_is_the_norm_and_rope_is_relative():
    """At position 0 RoPE is the identity; and rotating q and k by the same extra distance leaves q.k unchanged
    (the angle depends on the position difference only), up to T rounding."""
    g = np.random.default_rng(11)
    B, L, H, KV, HD = 1, 1, 2, 1, 128
    x = oq.to_f32(oq.from_f32((g.standard_normal((B, L, (H + 2 * KV) * HD)) * 2).astype(np.float32), "float16"),
                  "float16")
    w = np.ones(HD, np.float32)
    q0, k0, _ = oa.qk_norm_rope(x, w, w, 1e-6, [0], H, KV, HD, True)
    qn, kn, _ = oa.qk_norm_rope(x, w, w, 1e-6, [0], H, KV, HD, False)
    assert np.array_equal(q0, qn) and np.array_equal(k0, kn)
    dots = []
    for p in (5, 5 + 64):  # q at p, k at p - 5
        qp, _, _ = oa.qk_norm_rope(x, w, w, 1e-6, [p], H, KV, HD, True)
        _, kp, _ = oa.qk_norm_rope(x, w, w, 1e-6, [p - 5], H, KV, HD, True)
        dots.append(float((qp[0, 0, 0].astype(np.float64) * kp[0, 0, 0]).sum()))
    assert abs(dots[0] - dots[1]) < 0.05 and abs(dots[0] - float((qn[0, 0, 0] * kn[0, 0, 0]).sum())) > 0.05


@pytest.mark.parametrize("mask", [None, "causal", "tree", "dense", "window"])
def test_c_sdpa_matches_float64_oracle(mask):
    """The C masked SDPA (used for full-size GPU parity) against the float64 closed form on small cases: every mask
    kind, sinks, left padding, G = 4, queries that cross its 16-query blocks; and the 8-bit form against sdpa_q8."""
    g = np.random.default_rng(40)
    B, H, KVH, L, N, D = 2, 8, 2, 21, 150, 128
    cap = 160
    q = g.standard_normal((B, H, L, D)).astype(np.float32)
    k = g.standard_normal((B, KVH, cap, D)).astype(np.float32)
    v = g.standard_normal((B, KVH, cap, D)).astype(np.float32)
    sinks = (2 * g.standard_normal(H)).astype(np.float32)
    start = np.array([0, 17], dtype=np.int32)
    vis = np.broadcast_to(oa.causal_mask(L, N), (B, L, N)).copy()
    kw = {}
    if mask == "tree":
        parents = [[-1] + [int(g.integers(max(0, i - 3), i)) for i in range(1, L)] for _ in range(B)]
        local = np.stack([oa.ancestor_mask(p) for p in parents])
        vis = np.stack([oa.tree_full_mask(m, N - L) for m in local])
        bits = (local.astype(np.uint64) << np.arange(L, dtype=np.uint64)).sum(-1).astype(np.uint64)
        kw["tree"] = bits
    elif mask == "dense":
        vis = g.random((B, L, N)) < 0.4
        kw["dense"] = vis
    elif mask == "window":
        vis = np.broadcast_to(oa.window_mask(L, N, 37), (B, L, N)).copy()
        kw["window"] = 37
    elif mask is None:
        vis = np.ones((B, L, N), bool)
    vis = vis & (np.arange(N)[None, None, :] >= start[:, None, None])
    got = cbind.sdpa(q, k, v, 0.0884, mask, sinks, start=start, n=N, **kw)
    ref = oa.sdpa(q, k[:, :, :N], v[:, :, :N], 0.0884, vis[:, None], sinks, dtype="float64")
    assert np.abs(got - ref).max() < 2e-6
    if mask in ("causal", "tree"):
        K, V = oq.quantize(k.astype(np.float16)), oq.quantize(v.astype(np.float16))
        q16, s16 = q.astype(np.float16), sinks.astype(np.float16)
        got8 = cbind.sdpa_q8(q16, K, V, 0.0884, mask, s16, n=N, start=start, **kw)
        ref8 = oa.sdpa_q8(q16, K, V, 0.0884, vis[:, None], s16, n=N)
        assert np.abs(got8 - ref8).max() < 2e-6


def _triple(B, KVH, cap, seed):
    g = np.random.default_rng(seed)
    return (g.integers(0, 2 ** 32, (B, KVH, cap, 32), dtype=np.uint32),
            g.integers(0, 2 ** 16, (B, KVH, cap, 2), dtype=np.uint16),
            g.integers(0, 2 ** 16, (B, KVH, cap, 2), dtype=np.uint16))


def test_cache_row_bookkeeping_oracle():
    """oracle.cache against positions worked out by hand from locals/qkv.py:340-440: requests of 20 and 11 keys
    merge right-aligned; extend with a 30-key request pads the older rows by 10; filter drops the shared padding;
    extract returns a row's own keys; finalize rolls rows right by their right padding; growth keeps prev and
    appends whole steps."""
    from oracle import cache as oc

    t1, t2, t3 = _triple(1, 2, 256, 1), _triple(1, 2, 256, 2), _triple(1, 2, 64, 3)
    b = oc.merge([(t1, 20), (t2, 11), (None, 0)], KVH=2)
    assert b["idx"] == 20 and b["left_padding"].tolist() == [0, 9, 20] and b["offset"].tolist() == [20, 11, 0]
    for a, x in zip(b["keys"], t2):
        assert np.array_equal(a[1, :, 9:20], x[0, :, :11]) and not a[1, :, :9].any() and not a[2].any()
    e, n = oc.extract(b, 1)
    assert n == 11 and all(np.array_equal(a[0], x[0, :, :11]) for a, x in zip(e, t2))
    b3 = oc.merge([(t3, 30)], KVH=2)
    x = oc.extend(b, b3, KVH=2)
    assert x["idx"] == 30 and x["left_padding"].tolist() == [10, 19, 30, 0] and x["keys"][0].shape[2] == 30
    for a, y in zip(x["keys"], t1):
        assert np.array_equal(a[0, :, 10:30], y[0, :, :20]) and not a[0, :, :10].any()
    f = oc.filter_rows(x, [1, 0])
    assert f["idx"] == 20 and f["left_padding"].tolist() == [9, 0] and f["keys"][0].shape[2] == 20
    for a, y in zip(f["keys"], t1):
        assert np.array_equal(a[1, :, :20], y[0, :, :20])
    r = oc.finalize({"keys": tuple(a[:, :, :5] for a in t1), "left_padding": np.array([0]), "offset": np.array([5]),
                     "idx": 5}, [2])
    assert r["left_padding"].tolist() == [2] and r["offset"].tolist() == [3]
    assert np.array_equal(r["keys"][0][0, 0, :, 0], t1[0][0, 0, [3, 4, 0, 1, 2], 0])
    g = oc.grow(tuple(a[:, :, :700] for a in _triple(2, 2, 700, 4)), 700, 1, KVH=2, B=2)
    assert g[0].shape[2] == 956 and not g[0][:, :, 700:].any()
