"""The allocation-free decode entry point (lcl_qkv_attend_noalloc) through the C ABI: its output equals
lcl_qkv_attend's with a caller workspace, bit for bit (the same kernels and split), on two calls in a row, the
second with a smaller input than the first (the shared scratch keeps the first call's parts), and both match the
float64 oracle (locals/qkv.py:213-249) within 2e-3.  (The refusal of calls beyond the scratch is checked on the
CPU, tests/test_abi_host.py.)"""

import numpy as np
import pytest
import torch

from oracle import attn as oattn
from tests.inputs import normal16, q8_cache, rng, to_torch, triple_to_torch

pytestmark = pytest.mark.gpu


def _call(lib, fn, q, K, V, n, sinks, scale, start, ws=None):
    from locals_amd import _lib

    B, H, _, HD = q.shape
    kw, ks, kb = K
    vw, vs, vb = V
    KVH, cap = kw.shape[1], kw.shape[2]
    out = torch.full((B, H, 1, HD), float("nan"), dtype=q.dtype, device=q.device)
    args = [_lib.ptr(q), _lib.dtype_code(q.dtype), _lib.ptr(kw), _lib.ptr(ks), _lib.ptr(kb), _lib.ptr(vw),
            _lib.ptr(vs), _lib.ptr(vb), _lib.dtype_code(ks.dtype), _lib.ptr(start), _lib.ptr(sinks), float(scale),
            B, H, KVH, HD, cap, n, 0, _lib.ptr(out)]
    if ws is not None:
        args += [_lib.ptr(ws), ws.numel() * 4]
    rc = getattr(lib, fn)(*args, _lib.stream_of(q.device))
    assert rc == 0, (fn, rc)
    return out


def _case(dev, seed, B, H, KVH, cap, n):
    g = rng(seed)
    q = normal16(g, (B, H, 1, 128))
    K, V = q8_cache(g, B, KVH, cap, kscale=2.0)
    sinks = normal16(g, (H,), 2.0)
    start = g.integers(0, max(1, n // 2), size=B).astype(np.int32)
    return q, K, V, sinks, start, (to_torch(q, dev), triple_to_torch(K, dev), triple_to_torch(V, dev),
                                   to_torch(sinks.astype(np.float32), dev), to_torch(start, dev))


def test_noalloc_equals_workspace_entry_on_two_calls(dev):
    from locals_amd import _lib

    lib = _lib.load()
    # the second call is smaller (fewer rows, fewer keys, other heads) than the first
    for seed, (B, H, KVH, cap, n) in [(1, (16, 32, 8, 8192, 8000)), (2, (3, 16, 8, 768, 700))]:
        print(f"noalloc B={B} H={H} KVH={KVH} n={n}", flush=True)
        q, K, V, sinks, start, t = _case(dev, seed, B, H, KVH, cap, n)
        nbytes = int(lib.lcl_decode_workspace_bytes(B, H, n, 0))
        ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
        want = _call(lib, "lcl_qkv_attend", t[0], t[1], t[2], n, t[3], 0.0884, t[4], ws=ws)
        got = _call(lib, "lcl_qkv_attend_noalloc", t[0], t[1], t[2], n, t[3], 0.0884, t[4])
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        ref = oattn.attend(q, K, V, n, sinks, 0.0884, start)
        assert np.abs(got.float().cpu().numpy() - ref).max() <= 2e-3
