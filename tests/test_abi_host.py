"""CPU checks of the boundary: the C-ABI library loads and exports every entry point include/*.h declares, the
Python signature table matches the header, entry points reject bad arguments before touching the GPU, and the
host-side cache bookkeeping (mlx-lm BatchKVCache semantics, locals/qkv.py:295-452) is right on CPU tensors."""

import ctypes
import glob
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        names |= set(re.findall(r"^\s*(?:int|size_t|void)\s+(lcl_\w+)\s*\(", src, re.M))
    return names


def test_library_exports_every_declared_symbol():
    from locals_amd import _lib

    lib = _lib.load()
    declared = _declared()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_signature_arity_matches_header():
    from locals_amd import _lib

    src = "".join(open(h).read() for h in glob.glob(os.path.join(ROOT, "include", "*.h")))
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(r"(?:int|size_t|void)\s+" + name + r"\s*\(([^;]*)\);", src, re.S)
        assert m, name
        assert len([a for a in m.group(1).split(",") if a.strip()]) == len(args), name


def test_entry_points_reject_bad_arguments_without_a_gpu():
    from locals_amd import _lib

    lib = _lib.load()
    P = ctypes.c_void_p
    one = P(16)  # never dereferenced: validation fails first
    # head_dim 64 -> unsupported (-2); null q -> invalid (-1); missing workspace -> -3
    rc = lib.lcl_qkv_attend(one, 0, one, one, one, one, one, one, 0, None, None, 0.1, 1, 8, 2, 64, 256, 10, 0,
                            one, one, 1 << 20, None)
    assert rc == -2
    rc = lib.lcl_qkv_attend(None, 0, one, one, one, one, one, one, 0, None, None, 0.1, 1, 8, 2, 128, 256, 10, 0,
                            one, one, 1 << 20, None)
    assert rc == -1
    rc = lib.lcl_qkv_attend(one, 0, one, one, one, one, one, one, 0, None, None, 0.1, 1, 8, 2, 128, 256, 10, 0,
                            one, None, 0, None)
    assert rc == -3
    # the allocation-free decode checks its arguments as lcl_qkv_attend does, and refuses a call whose split-K parts
    # would not fit its fixed scratch (64 rows x 64 heads over 128k keys need ~550 MB), before touching the GPU
    rc = lib.lcl_qkv_attend_noalloc(None, 0, one, one, one, one, one, one, 0, None, None, 0.1, 1, 8, 2, 128, 256, 10,
                                    0, one, None)
    assert rc == -1
    assert lib.lcl_decode_workspace_bytes(64, 64, 131072, 0) > (32 << 20)
    rc = lib.lcl_qkv_attend_noalloc(one, 0, one, one, one, one, one, one, 0, None, None, 0.1, 64, 64, 8, 128, 131072,
                                    131072, 0, one, None)
    assert rc == -4
    rc = lib.lcl_quantize_append(one, None, 0, one, one, one, None, None, None, 1, 1, 4, 100, 8, 0, 0, None)
    assert rc == -1  # D not a multiple of 64
    # parts a (row, head): max(key chunks of 512, stream-K slots: ceil(16 tiles / 8 a wave) + 1) = 3, each with m, l
    # and 128 o; then one int32 part count a (row, head)
    assert lib.lcl_decode_workspace_bytes(2, 4, 1000, 512) == 2 * 4 * 3 * (2 + 128) * 4 + 2 * 4 * 4
    # qk_norm_rope: head_dim 64 unsupported; f32 unsupported; null q invalid; H not a multiple of KV invalid;
    # an empty call (B * L == 0) is a no-op even with null pointers; the fused store past the capacity is invalid
    qk = lambda qkv, dt, H, KV, hd, B=1, L=1, q=one: lib.lcl_qk_norm_rope(qkv, dt, one, one, one, 0, 1e-6, 13.3, 1, B, L,
                                                                         H, KV, hd, q, one, one, None)
    assert qk(one, 0, 4, 2, 64) == -2
    assert qk(one, 2, 4, 2, 128) == -2
    assert qk(one, 0, 4, 2, 128, q=None) == -1
    assert qk(one, 0, 4, 3, 128) == -1
    assert qk(None, 0, 4, 2, 128, B=0, q=None) == 0
    rc = lib.lcl_qk_norm_rope_append(one, 0, one, one, one, 0, 1e-6, 13.3, 1, 1, 5, 4, 2, 128, one, one, one, one,
                                     one, one, one, 256, 254, 0, None)
    assert rc == -1
    rc = lib.lcl_qk_norm_rope_append(one, 0, one, one, one, 0, 1e-6, 13.3, 1, 1, 5, 4, 2, 128, one, one, one, one,
                                     one, one, one, 256, 0, 2, None)
    assert rc == -1  # round mode
    # lcl_sdpa: the sliding window needs window >= 1 and L <= N; unknown mask kinds are invalid
    sd = lambda mk, W, L=4, N=10: lib.lcl_sdpa(one, 0, 1, None, None, None, None, None, None, one, one, 0, None, mk,
                                              W, None, 0, None, 0, 0, 0, 0, None, 0.1, 1, 8, 2, L, N, 128, 16, 0, one,
                                              None, 0, None)
    assert sd(4, 0) == -1 and sd(4, -3) == -1 and sd(4, 5, L=11) == -1 and sd(5, 5) == -1


def test_prompt_route_threshold_without_a_gpu():
    """Where the library dequantizes 8-bit K/V once before the masked-attention pass (its workspace then has room
    for the 16-bit copy): with eight-wave workgroups (causal or no mask, rows a multiple of 256 or more than 128 in
    the last 256-row block) from 12 row blocks of 256 rows per (row, KV head), so C4's 512-query chunk (8 blocks)
    stays on the fused kernel; otherwise from 16 blocks of 128 (or, under a dense mask, 64) rows; never under a
    window, for 16-bit K/V, or when the buffers hold over 512 positions past N."""
    from locals_amd import _lib, sdpa

    lib = _lib.load()
    B, H, KVH, P = 1, 32, 8, 16384

    def dq(L, mk, kvfmt=0, extra_cap=0):
        N = P + L
        cap = (N + 255) // 256 * 256 + extra_cap
        split = lib.lcl_sdpa_workspace_bytes(B, H, L, N, 0)
        kv = lib.lcl_sdpa_workspace_bytes_kv(B, H, KVH, L, N, cap, 0, kvfmt, mk)
        assert kv >= split
        if kv > split:  # room for K and V as (B, KVH, cap, 128) 16-bit values after the split-K parts
            assert kv >= split + 2 * B * KVH * cap * 128 * 2
        return kv > split

    causal, none, dense, window = sdpa.MASK_CAUSAL, sdpa.MASK_NONE, sdpa.MASK_DENSE, sdpa.MASK_WINDOW
    assert not dq(512, causal)   # 2048 rows: 8 blocks of 256 (C4)
    assert not dq(704, causal)   # 2816 rows: 11 blocks
    assert dq(768, causal)       # 3072 rows: 12 blocks
    assert dq(1024, causal)      # 16 blocks
    assert dq(768, none) and not dq(704, none)
    # rows leaving at most 128 in a last 256-row block keep four-wave workgroups (no padding rows added), and with
    # them the 128-row threshold of 16 blocks
    assert not dq(576, causal)   # 2304 rows: 9 blocks of 256, eight waves
    assert dq(544, causal)       # 2176 rows: 17 blocks of 128, four waves
    assert dq(256, dense)        # 1024 rows: 16 blocks of 64
    assert not dq(240, dense)    # 15 blocks
    assert not dq(1024, window)
    assert not dq(1024, causal, kvfmt=1)
    assert not dq(1024, causal, extra_cap=768)


def test_python_wrappers_refuse_cpu_tensors():
    from locals_amd import qkv

    q = torch.zeros(1, 8, 1, 128, dtype=torch.float16)
    K = qkv._zeros(1, 2, 64, 128, torch.float16)
    with pytest.raises(ValueError):
        qkv.attend(q, K, K, 10, None, 0.1, None)


def test_create_causal_mask():
    from locals_amd import qkv

    m = qkv.create_causal_mask(3, offset=4)
    assert m.shape == (3, 7) and m[0].tolist() == [True] * 5 + [False] * 2 and m[2].all()
    mp = qkv.create_causal_mask(2, offset=3, left_padding=torch.tensor([0, 2]))
    assert mp.shape == (2, 1, 2, 5) and not mp[1, 0, :, :2].any() and mp[0, 0, 1].all()


def _filled(B, H, n, seed):
    from locals_amd import qkv

    g = torch.Generator().manual_seed(seed)
    t = qkv._zeros(B, H, n, 128, torch.float16)
    t[0].copy_(torch.randint(-2 ** 31, 2 ** 31 - 1, t[0].shape, generator=g, dtype=torch.int64).to(torch.int32))
    t[1].copy_(torch.randn(t[1].shape, generator=g))
    t[2].copy_(torch.randn(t[2].shape, generator=g))
    return t


def test_batch_cache_growth_follows_the_reference_rule():
    """BatchQuantizedKVCache grows to prev + ceil(S / 256) * 256 positions, keeping exactly the first prev
    (locals/qkv.py:311-319: concatenate(a[..., :prev, :], zeros(ceil(S / step) * step))).  Capacities below are
    worked out by hand from that rule; nbytes is 272 B a position and kv head (128 + 4 + 4 for K and for V)."""
    from locals_amd import qkv

    def step(c, S):
        c._reserve(c.left_padding.numel(), 2, S, 128, torch.float16, torch.device("cpu"))
        return c.keys[0].shape[2]

    # as merge leaves two requests of 700 and 300 keys (buffers of exactly 700 positions), then decode steps
    b = qkv.BatchQuantizedKVCache([0, 400])
    b.keys, b.values, b._idx = _filled(2, 2, 700, 1), _filled(2, 2, 700, 2), 700
    b.offset = torch.tensor([700, 300], dtype=torch.int32)
    assert step(b, 1) == 956  # 700 + 256
    assert step(b, 255) == 956  # 956 positions used, no growth
    assert step(b, 1) == 1212  # 956 + 256
    assert b._idx == 957 and b.offset.tolist() == [957, 557]
    assert b.nbytes == 2 * 2 * 1212 * 272
    keys, values, offset, lp, idx = b.state
    assert keys[0].shape == (2, 2, 1212, 32) and keys[1].shape == (2, 2, 1212, 2) and idx == 957
    # a prompt chunk, a step, a longer chunk
    e = qkv.BatchQuantizedKVCache([0, 0])
    assert step(e, 700) == 768  # 0 + 3 * 256
    assert step(e, 1) == 768
    assert step(e, 300) == 1213  # 701 + 2 * 256
    # the kept positions are copied, the new ones are zero
    e2 = qkv.BatchQuantizedKVCache([0])
    e2.keys, e2.values, e2._idx = _filled(1, 2, 300, 7), _filled(1, 2, 300, 8), 300
    e2.offset = torch.tensor([300], dtype=torch.int32)
    old = [a.clone() for a in e2.keys]
    assert step(e2, 10) == 556
    assert all(torch.equal(a[..., :300, :], o) for a, o in zip(e2.keys, old))
    assert not any(a[..., 300:, :].any() for a in e2.keys)


def test_single_cache_growth_follows_mlx_lm():
    """QuantizedKVCache8 (mlx-lm's QuantizedKVCache): grows by ceil(S / 256) * 256, dropping positions past the
    offset first only when the offset is not a multiple of 256."""
    from locals_amd import qkv

    c = qkv.QuantizedKVCache8()
    cpu = torch.device("cpu")
    c._reserve(1, 2, 300, 128, torch.float16, cpu)
    assert c.keys[0].shape[2] == 512 and c.offset == 300
    c._reserve(1, 2, 100, 128, torch.float16, cpu)
    assert c.keys[0].shape[2] == 512
    c._reserve(1, 2, 200, 128, torch.float16, cpu)  # 400 % 256 != 0: keep 400, add 256
    assert c.keys[0].shape[2] == 656 and c.offset == 600
    c.trim(88)  # offset 512, a multiple of 256: the whole buffer is kept on the next growth
    c._reserve(1, 2, 200, 128, torch.float16, cpu)
    assert c.keys[0].shape[2] == 912 and c.offset == 712
    assert c.nbytes == 2 * 912 * 272


def test_prompt_branch_hands_sinks_over_in_the_query_dtype(monkeypatch):
    """qkv.attention's prompt branch casts the sinks to q's dtype (locals/qkv.py:272) before the masked kernel."""
    from locals_amd import fuse, qkv

    seen = {}

    def fake(q, keys, values, scale, mask, sinks):
        seen["sinks"] = sinks
        return q

    monkeypatch.setattr(fuse, "attend_few_q8", fake)
    c = qkv.QuantizedKVCache8()
    c.keys, c.values, c.offset = _filled(1, 2, 256, 1), _filled(1, 2, 256, 2), 10
    q = torch.zeros(1, 4, 3, 128, dtype=torch.bfloat16)
    s32 = torch.tensor([0.1234567, -3.3333333, 2.0000001, 7.7777777], dtype=torch.float32)
    qkv.attend_cache(q, c, 0.1, "causal", s32)
    assert seen["sinks"].dtype == torch.bfloat16 and torch.equal(seen["sinks"], s32.to(torch.bfloat16))
    qkv.attend_cache(q, c, 0.1, "causal", None)
    assert seen["sinks"] is None


def test_prompt_cache_snapshot_layout_on_host(tmp_path):
    """save_prompt_cache writes mlx-lm's layout (state arrays under "<layer>.<i>.<j>", meta_state, metadata and
    class names in the safetensors metadata; 8-bit words as uint32) and load_prompt_cache reads it back exactly."""
    from safetensors import safe_open

    from locals_amd import qkv

    caches = []
    for i, n in enumerate((300, 17)):
        c = qkv.QuantizedKVCache8()
        c.keys, c.values, c.offset = _filled(1, 2, 512, 10 + i), _filled(1, 2, 512, 20 + i), n
        caches.append(c)
    path = str(tmp_path / "snap.safetensors")
    qkv.save_prompt_cache(path, caches, {"model": "flint"})
    with safe_open(path, "pt") as f:
        meta = f.metadata()
        assert f.get_tensor("0.0.0").dtype == torch.uint32 and f.get_tensor("1.1.2").shape == (1, 2, 17, 2)
    assert meta["0.0.1"] == "300" and meta["0.1.1"] == "17" and meta["0.0.0"] == "256" and meta["0.0.3"] == "8"
    assert meta["1.model"] == "flint" and meta["2.0"] == meta["2.1"] == "QuantizedKVCache8"
    back, md = qkv.load_prompt_cache(path, device="cpu", return_metadata=True)
    assert md == {"model": "flint"} and [c.offset for c in back] == [300, 17]
    for c0, c1 in zip(caches, back):
        for a, x in zip(c0.state[0] + c0.state[1], c1.keys + c1.values):
            assert a.dtype == x.dtype and torch.equal(a, x)
    qkv.save_prompt_cache(path, caches[:1])  # no metadata
    assert qkv.load_prompt_cache(path, device="cpu")[0].offset == 300
