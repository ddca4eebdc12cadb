"""Outputs written through the C ABI at addresses that are not 8-byte (16-bit) or 16-byte (fp32) aligned.

The kernels store a lane's 4 consecutive output elements as one vector store when the address allows it and as
four element stores otherwise.  These tests call the entry points with the output pointer moved by one element
into a larger buffer and compare, bit for bit, with the aligned call (same kernels, same arithmetic: only the
store path differs).
"""

import numpy as np
import pytest
import torch

from tests.inputs import normal16, q8_cache, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu


def _shifted(shape, dtype, dev):
    """A tensor of `shape` starting one element into a fresh buffer (so 2 or 4 bytes past an aligned address)."""
    n = int(np.prod(shape))
    buf = torch.full((n + 8,), float("nan"), dtype=dtype, device=dev)
    return buf[1:1 + n].view(shape)


@pytest.mark.parametrize("qdtype", ["float16", "float32"])
def test_decode_unaligned_output(dev, qdtype):
    from locals_amd import _lib, qkv

    g = rng(90)
    B, H, KVH, cap, n = 3, 16, 4, 768, 700
    q = to_torch(normal16(g, (B, H, 1, 128)), dev)
    if qdtype == "float32":
        q = q.float()
    K, V = q8_cache(g, B, KVH, cap)
    Kt, Vt = triple_to_torch(K, dev), triple_to_torch(V, dev)
    start = torch.tensor([0, 37, 300], dtype=torch.int32, device=dev)
    want = qkv.attend(q, Kt, Vt, n, None, 0.0884, start)
    out = _shifted((B, H, 1, 128), q.dtype, dev)
    lib = _lib.load()
    nbytes = int(lib.lcl_decode_workspace_bytes(B, H, n, qkv.BLOCK))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    P = _lib.ptr
    rc = lib.lcl_qkv_attend(P(q), _lib.dtype_code(q.dtype), P(Kt[0]), P(Kt[1]), P(Kt[2]), P(Vt[0]), P(Vt[1]),
                            P(Vt[2]), _lib.dtype_code(Kt[1].dtype), P(start), None, 0.0884, B, H, KVH, 128, cap, n,
                            qkv.BLOCK, P(out), P(ws), nbytes, _lib.stream_of(dev))
    _lib.check(rc, "lcl_qkv_attend")
    torch.cuda.synchronize()
    assert torch.equal(out, want)


@pytest.mark.parametrize("block", [0, 64])
@pytest.mark.parametrize("qdtype", ["float16", "float32"])
def test_sdpa_unaligned_output(dev, block, qdtype):
    """16-bit K/V, no mask: one chunk (the pass-1 kernel writes the output) and 64-key chunks (the join does)."""
    from locals_amd import _lib, sdpa

    g = rng(91)
    B, H, KVH, L, N, cap = 2, 8, 2, 24, 300, 320
    q = to_torch(normal16(g, (B, H, L, 128)), dev)
    if qdtype == "float32":
        q = q.float()
    kf = to_torch(normal16(g, (B, KVH, cap, 128)), dev)
    vf = to_torch(normal16(g, (B, KVH, cap, 128)), dev)
    old = sdpa.BLOCK
    sdpa.BLOCK = block
    try:
        want = sdpa.scaled_dot_product_attention(q, kf[:, :, :N], vf[:, :, :N], scale=0.0884)
    finally:
        sdpa.BLOCK = old
    out = _shifted((B, H, L, 128), q.dtype, dev)
    lib = _lib.load()
    nbytes = int(lib.lcl_sdpa_workspace_bytes(B, H, L, N, block))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    P = _lib.ptr
    rc = lib.lcl_sdpa(P(q), _lib.dtype_code(q.dtype), 1, None, None, None, None, None, None, P(kf), P(vf),
                      _lib.dtype_code(kf.dtype), None, 0, 0, None, 0, None, 0, 0, 0, 0, None, 0.0884,
                      B, H, KVH, L, N, 128, cap, block, P(out), P(ws), nbytes, _lib.stream_of(dev))
    _lib.check(rc, "lcl_sdpa")
    torch.cuda.synchronize()
    assert torch.equal(out, want)
