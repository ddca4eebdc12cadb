"""The hot-path entry points under HIP graph capture: they allocate nothing, never synchronise and clear nothing with
memset, so a serving loop can capture a decode step once and replay it.

Each test captures the calls on torch's capture stream, replays the graph several times with new inputs copied
into the captured tensors (eager work and synchronisations between the replays), and compares every replay with
the same calls run eagerly, bit for bit (same kernels, same inputs).
"""

import numpy as np
import pytest
import torch

from tests.inputs import normal16, q8_cache, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu


def _replays(dev, graph_fn, eager_fn, refill, n=3):
    """Capture graph_fn, then n times: refill the inputs, replay, run eager_fn, compare."""
    graph_fn()  # warm-up outside capture (library load, workspace sizes)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = graph_fn()
    for i in range(n):
        refill(i)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]  # eager_fn may write the same buffers
        want = eager_fn()
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), i


@pytest.mark.parametrize("H,KVH", [(32, 8), (32, 4)])
def test_decode_step_replays(dev, H, KVH):
    """qkv.attend over a left-padded batch (stream-K pass 1 + combine; one and two head groups)."""
    from locals_amd import qkv

    g = rng(50 + KVH)
    B, cap, n = 4, 1024, 1000
    K, V = q8_cache(g, B, KVH, cap)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    q = to_torch(normal16(g, (B, H, 1, 128)), dev)
    sinks = to_torch(normal16(g, (H,), 2.0), dev)
    start = torch.tensor([0, 10, 500, 999], dtype=torch.int32, device=dev)

    def call():
        return (qkv.attend(q, Kt, Vt, n, sinks, 0.0884, start),)

    def refill(i):
        q.copy_(to_torch(normal16(rng(60 + i), (B, H, 1, 128)), dev))
        start.copy_(torch.tensor([i, 10 * i, 500 - i, 999 - i], dtype=torch.int32, device=dev))

    _replays(dev, call, call, refill)


@pytest.mark.parametrize("block", [0, 64])
def test_prefill_chunk_replays(dev, block):
    """scaled_dot_product_attention over 8-bit triples with a causal mask: one chunk (pass 1 writes the output) and
    64-key chunks (pass 2 joins them)."""
    from locals_amd import sdpa

    old = sdpa.BLOCK
    sdpa.BLOCK = block
    try:
        g = rng(51)
        B, H, KVH, L, N, cap = 1, 16, 4, 40, 700, 768
        K, V = q8_cache(g, B, KVH, cap)
        Kt = tuple(a[:, :, :N] for a in triple_to_torch(K, dev))
        Vt = tuple(a[:, :, :N] for a in triple_to_torch(V, dev))
        q = to_torch(normal16(g, (B, H, L, 128)), dev)

        def call():
            return (sdpa.scaled_dot_product_attention(q, Kt, Vt, scale=0.0884, mask="causal"),)

        def refill(i):
            q.copy_(to_torch(normal16(rng(70 + i), (B, H, L, 128)), dev))

        _replays(dev, call, call, refill)
    finally:
        sdpa.BLOCK = old


def test_qk_norm_rope_append_replays(dev):
    """The fused norms + RoPE + 8-bit cache store of a decode step, into fixed cache buffers."""
    import types

    from locals_amd import _lib, qk_kernel

    g = rng(52)
    B, H, KV, HD, cap = 2, 8, 2, 128, 256
    w = lambda: to_torch(normal16(g, (HD,), 0.05), dev) + 1.0  # noqa: E731
    attn = types.SimpleNamespace(n_heads=H, n_kv_heads=KV, head_dim=HD,
                                 q_norm=types.SimpleNamespace(weight=w(), eps=1e-6),
                                 k_norm=types.SimpleNamespace(weight=w(), eps=1e-6),
                                 rope=types.SimpleNamespace(base=10000.0, dims=HD, traditional=False, scale=1.0))
    qkv_in = to_torch(normal16(g, (B, 1, (H + 2 * KV) * HD), 2.0), dev)
    offs = torch.tensor([5, 77], dtype=torch.int32, device=dev)
    kw = torch.zeros((B, KV, cap, HD // 4), dtype=torch.int32, device=dev)
    ks = torch.zeros((B, KV, cap, HD // 64), dtype=torch.float16, device=dev)
    kb, vw, vs, vb = torch.zeros_like(ks), torch.zeros_like(kw), torch.zeros_like(ks), torch.zeros_like(ks)
    qout = torch.empty((B, H, 1, HD), dtype=torch.float16, device=dev)
    P = _lib.ptr

    def call():
        rc = _lib.load().lcl_qk_norm_rope_append(
            P(qkv_in), 0, P(attn.q_norm.weight), P(attn.k_norm.weight), P(offs), 1, 1e-6, float(np.log2(10000.0)), 1,
            B, 1, H, KV, HD, P(qout), P(kw), P(ks), P(kb), P(vw), P(vs), P(vb), cap, 100, 0, _lib.stream_of(dev))
        _lib.check(rc, "lcl_qk_norm_rope_append")
        return (qout,) + tuple(t[:, :, 100] for t in (kw, ks, kb, vw, vs, vb))  # the step's cache position

    def eager():
        qout.fill_(-7.0)  # the eager run must write everything compared
        for t in (kw, ks, kb, vw, vs, vb):
            t[:, :, 100].fill_(-7)
        out = call()
        q1, _, _ = qk_kernel.qk_norm_rope(qkv_in, attn, offs)  # the unfused q, bit for bit
        assert torch.equal(q1, qout)
        return out

    def refill(i):
        qkv_in.copy_(to_torch(normal16(rng(80 + i), (B, 1, (H + 2 * KV) * HD), 2.0), dev))

    _replays(dev, call, eager, refill)
