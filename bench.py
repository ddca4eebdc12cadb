"""Benchmark of the batched-attention hot path on one MI355X: 8-bit-KV GQA flash-decode.

    python bench.py [--steps K] [--warmup W] [--config c2|c1|c3|c4|c5|w1|f2|qk] [--cpu-seconds S] [--no-cpu]

A step is one ``qkv.attend`` over the whole batch (pass 1 + the log-sum-exp combine) with K/V already resident in
HBM.  Workload (default, "c2"): B=16 rows, 32 query / 8 KV heads, head_dim 128, row contexts n_b ~ U[1024, 32768]
(seeded), left-padded in one buffer of capacity n = max n_b rounded up to 256 (start_b = n - n_b), K/V ~ N(0,1) fp16
quantized with MLX's affine 8 bits (group 64), Q ~ N(0,1) fp16, no sink.  Two independent buffer sets (2 x 1.14 GB)
alternate so the 256 MB MALL cannot serve a step.

Prints one JSON line.  ``value`` = algorithmic bytes a step (sum_b n_b * KVH * 272 + Q + O) / step time, GB/s.
``roofline`` = the pass-1 kernel: its algorithmic bytes (K/V codes, scales, biases and Q) / its own average
duration, timed by hipEvents recorded by its dispatch (lcl_qkv_attend_ex) inside the timed region, against the
8 TB/s HBM peak.  ``cpu_baseline`` = the reference's two-pass split-K algorithm restated in C (oracle/, OpenMP) on
this host's cores over a bounded sample of the same workload (kind "port").
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))


def _hip():
    """The HIP runtime torch loaded (so events and streams are the same runtime's)."""
    import torch  # noqa: F401

    path = None
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                path = line.split()[-1]
                break
    lib = ctypes.CDLL(path or "libamdhip64.so")
    lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return lib


class Events:
    def __init__(self, n):
        self.hip = _hip()
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = self.hip.hipEventCreate(ctypes.byref(e))
            if rc:
                raise RuntimeError(f"hipEventCreate failed {rc}")
            self.ev.append(e)

    def ms(self, a, b):
        t = ctypes.c_float()
        rc = self.hip.hipEventElapsedTime(ctypes.byref(t), self.ev[a], self.ev[b])
        if rc:
            raise RuntimeError(f"hipEventElapsedTime failed {rc}")
        return t.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def dist(us):
    """median / p10 / p90 / mean of a sample of µs values"""
    a = np.asarray(us, dtype=np.float64)
    return {"median": round(float(np.median(a)), 2), "p10": round(float(np.percentile(a, 10)), 2),
            "p90": round(float(np.percentile(a, 90)), 2), "mean": round(float(a.mean()), 2), "n": int(a.size)}


def timed_loop(run, steps, warmup, stream, every):
    """``warmup`` untimed calls, then ``steps`` timed ones.  Returns (µs a step over the region, pass-1 µs of the
    sampled dispatches or None).  With ``every`` > 0 the pass-1 dispatch of every ``every``-th call records its own
    start/stop events; that costs step time (so the region time of such a loop is not reported), and bracketing
    back-to-back dispatches lengthens what their events measure (C2 pass 1: ~106 us every call against ~101 us every
    4th call, the rocprofv3 figure), so samples are taken every 4th call.  With ``every`` = 0 the region has no other
    events."""
    import torch

    for i in range(warmup):
        run(i)
    torch.cuda.synchronize()
    ev = Events(2 * steps + 2)
    hip = ev.hip
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventRecord(ev.ev[-2], stream)
    for i in range(steps):
        if every and i % every == 0:
            run(i, ev.ev[2 * i], ev.ev[2 * i + 1])
        else:
            run(i)
    hip.hipEventRecord(ev.ev[-1], stream)
    torch.cuda.synchronize()
    step_us = ev.ms(2 * steps, 2 * steps + 1) * 1e3 / steps
    p1 = [ev.ms(2 * i, 2 * i + 1) * 1e3 for i in range(0, steps, every)] if every else None
    ev.close()
    return step_us, p1


def config(name: str, seed: int = 0):
    g = np.random.default_rng(seed)
    if name == "c1":
        return dict(name="c1", workload="fp16 ragged decode: 4 rows x 2,048 keys, 16 query / 8 KV heads "
                    "(ragged_attention, BASELINE config 1)", B=4, H=16, KVH=8, nb=np.array([2048] * 4))
    if name == "c2":
        B, H, KVH = 16, 32, 8
        nb = g.integers(1024, 32768, size=B, endpoint=True)
        return dict(name="c2", workload="8-bit KV GQA flash-decode, mixed contexts (BASELINE config 2)",
                    B=B, H=H, KVH=KVH, nb=nb)
    if name == "qk":
        return dict(name="qk", workload="qk_norm_rope, quantize_append and the fused qk_norm_rope_append at C2's "
                    "decode step (16 x 1 token) and at a 512-token prompt chunk, 32 / 8 heads, bf16")
    if name == "f2":
        B, H, KVH = 16, 32, 4
        nb = g.integers(1024, 32768, size=B, endpoint=True)
        return dict(name="f2", workload="8-bit KV flash-decode with Flint's head layout (32 query / 4 KV heads, G = 8), "
                    "the rows and contexts of BASELINE config 2", B=B, H=H, KVH=KVH, nb=nb)
    if name == "c3":
        return dict(name="c3", workload="long-context single-row split-K decode (BASELINE config 3)",
                    B=1, H=16, KVH=8, nb=np.array([245760]))
    if name == "c4d":
        B = 15
        return dict(name="c4d", workload="hybrid batch: the 15 decode rows (BASELINE config 4, decode part)",
                    B=B, H=32, KVH=8, nb=g.integers(2048, 16384, size=B, endpoint=True))
    if name == "c4":
        return dict(name="c4", workload="hybrid batch: 512-token causal prefill chunk over a 16,384-token 8-bit "
                    "prefix + 15 decode rows with contexts U[2k, 16k] (BASELINE config 4)", B=15, H=32, KVH=8,
                    nb=g.integers(2048, 16384, size=15, endpoint=True), L=512, prefix=16384)
    if name == "c5":
        return dict(name="c5", workload="speculative tree verification: 8 rows x 16 draft tokens (random trees, "
                    "branching 1-3, depth <= 8) over 8,192 cached 8-bit keys (BASELINE config 5)", B=8, H=32, KVH=8,
                    L=16, prefix=8192)
    if name == "w1":
        return dict(name="w1", workload="sliding-window prompt chunk: 2,048 queries after a ring of 512 keys, window "
                    "513, Flint's 32 query / 4 KV heads, bf16 K/V (the banded attention, locals/fuse.py:113-125)",
                    B=1, H=32, KVH=4, L=2048, prefix=512, window=513)
    raise SystemExit(f"unknown config {name}")


def random_tree(g, L=16, max_depth=8):
    """Preorder parent array of a random tree: each node has 1-3 children while depth <= max_depth."""
    parents, depth = [-1], [1]
    frontier = [0]
    while len(parents) < L and frontier:
        node = frontier.pop(0)
        for _ in range(int(g.integers(1, 4))):
            if len(parents) >= L or depth[node] >= max_depth:
                break
            parents.append(node)
            depth.append(depth[node] + 1)
            frontier.append(len(parents) - 1)
    while len(parents) < L:  # chain the rest under the last node that may still grow
        parents.append(len(parents) - 1)
        depth.append(depth[-1] + 1)
    # renumber to preorder
    children = {i: [] for i in range(L)}
    for i, p in enumerate(parents[1:], 1):
        children[p].append(i)
    order, stack = [], [0]
    while stack:
        n = stack.pop()
        order.append(n)
        stack.extend(reversed(children[n]))
    new = {o: i for i, o in enumerate(order)}
    return [-1 if parents[o] < 0 else new[parents[o]] for o in order]


def _depth(parents, i):
    d = 0
    while parents[i] >= 0:
        i, d = parents[i], d + 1
    return d


def bench_multi(cfg, args, dev, return_runner=False):
    """C4 (decode rows + causal prefill chunk), C5 (tree verification) and W1 (sliding-window chunk over 16-bit K/V):
    pass-1 times from the dispatch events, FLOPs and bytes from the shapes."""
    import torch

    from locals_amd import _lib, qkv, sdpa

    lib = _lib.load()
    stream = _lib.stream_of(dev)
    H, KVH, L, P = cfg["H"], cfg["KVH"], cfg["L"], cfg["prefix"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    Bp = 1 if cfg["name"] == "c4" else cfg["B"]
    N = P + L
    cap = (N + 255) // 256 * 256
    W = cfg.get("window", 0)
    sets = []
    kv_set = Bp * KVH * N * (512 if W else 272)
    nsets = max(args.sets, -(-(1 << 30) // kv_set))  # >= 1 GiB of K/V in rotation, so the 256 MB MALL cannot hold it
    for s in range(nsets):
        if W:  # 16-bit K/V, the rotating cache's dtype
            K = torch.randn((Bp, KVH, cap, 128), generator=gen, device=dev, dtype=torch.bfloat16)
            V = torch.randn((Bp, KVH, cap, 128), generator=gen, device=dev, dtype=torch.bfloat16)
            q = torch.randn((Bp, H, L, 128), generator=gen, device=dev, dtype=torch.bfloat16)
            sets.append((q, K, V))
            continue
        K = qkv._zeros(Bp, KVH, cap, 128, torch.float16, dev)
        V = qkv._zeros(Bp, KVH, cap, 128, torch.float16, dev)
        for b in range(Bp):
            kf = torch.randn((1, KVH, cap, 128), generator=gen, device=dev, dtype=torch.float16)
            vf = torch.randn((1, KVH, cap, 128), generator=gen, device=dev, dtype=torch.float16)
            qkv.quantize_into(kf, vf, tuple(a[b:b + 1] for a in K), tuple(a[b:b + 1] for a in V), 0)
        q = torch.randn((Bp, H, L, 128), generator=gen, device=dev, dtype=torch.float16)
        sets.append((q, K, V))
    g = np.random.default_rng(7)
    if cfg["name"] == "c5":
        trees = [random_tree(g, L) for _ in range(Bp)]
        local = np.zeros((Bp, L, L), bool)
        for b, par in enumerate(trees):
            for i in range(L):
                j = i
                while j >= 0:
                    local[b, i, j] = True
                    j = par[j]
        mask = sdpa.TreeMask.from_local(torch.from_numpy(local), device=dev)
        mk, tree, tree_bs = 2, mask.bits, L
        pairs = int(Bp * (L * P + local.sum()))
    elif W:
        mk, tree, tree_bs = 4, None, 0
        pairs = Bp * sum(min(W, P + i + 1) for i in range(L))
    else:
        mk, tree, tree_bs = 1, None, 0
        pairs = sum(P + i + 1 for i in range(L))
    flops = pairs * H * 4 * 128
    kv_bytes = Bp * KVH * N * (512 if W else 272)
    split = int(lib.lcl_sdpa_workspace_bytes(Bp, H, L, N, sdpa.BLOCK))
    nbytes = int(lib.lcl_sdpa_workspace_bytes_kv(Bp, H, KVH, L, N, cap, sdpa.BLOCK, 1 if W else 0, mk))
    if not sdpa.DEQUANTIZE_FIRST:
        nbytes = split
    # with room for it the library dequantizes K/V once and runs the 16-bit kernel; the events bracket pass 1 alone,
    # the call time covers the dequantization, pass 1 and the join
    route = "dequantize K/V, 16-bit pass 1" if nbytes > split else ("16-bit pass 1" if W else "fused 8-bit pass 1")
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    out = torch.empty((Bp, H, L, 128), dtype=torch.bfloat16 if W else torch.float16, device=dev)
    P_ = _lib.ptr

    def run(i, e0=None, e1=None, st=None):
        q, K, V = sets[i % len(sets)]
        st = stream if st is None else st
        if W:
            rc = lib.lcl_sdpa_ex(P_(q), 1, 1, None, None, None, None, None, None, P_(K), P_(V), 1, None, mk, W, None,
                                 0, None, 0, 0, 0, 0, None, float(1 / np.sqrt(128)), Bp, H, KVH, L, N, 128, cap,
                                 sdpa.BLOCK, P_(out), P_(ws), nbytes, st, e0, e1)
        else:
            rc = lib.lcl_sdpa_ex(P_(q), 0, 0, P_(K[0]), P_(K[1]), P_(K[2]), P_(V[0]), P_(V[1]), P_(V[2]), None, None,
                                 0, None, mk, 0, P_(tree), tree_bs, None, 0, 0, 0, 0, None, float(1 / np.sqrt(128)), Bp,
                                 H, KVH, L, N, 128, cap, sdpa.BLOCK, P_(out), P_(ws), nbytes, st, e0, e1)
        _lib.check(rc, "lcl_sdpa_ex")

    if return_runner:
        return run

    # the whole call (dequantization, pass 1, join) unbracketed; then pass 1 of every 4th call by its own events
    step_us, _ = timed_loop(run, args.steps, args.warmup, stream, 0)
    _, p1 = timed_loop(run, 4 * args.steps, 2, stream, 4)
    us = float(np.mean(p1))
    res = {"kernel": "sdpa_pass1", "route": route, "L": L, "N": N, "rows": Bp, "avg_us": round(us, 2),
           "pass1_us": dist(p1), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
           "mfma_frac_of_2.5PF": round(flops / (us * 1e-6) / 2.5e15, 4),
           "kv_GBs": round(kv_bytes / (us * 1e-6) / 1e9, 1), "hbm_frac": round(kv_bytes / (us * 1e-6) / 8e12, 4),
           "us_per_call": round(step_us, 2),
           "mfma_frac_call": round(flops / (step_us * 1e-6) / 2.5e15, 4),
           "hbm_frac_call": round(kv_bytes / (step_us * 1e-6) / 8e12, 4),
           "flops": flops, "kv_bytes": kv_bytes, "buffer_sets": nsets}
    if cfg["name"] == "c5":
        res["tree_depths"] = [1 + max(_depth(t, i) for i in range(L)) for t in trees]
    if W:
        res["window"] = W
    return res


def bench_c1(cfg, args, dev):
    """C1: attention.ragged_attention over fp16 slot-major K/V, one row a slot.  33.6 MB of K/V a step sits in the
    256 MB MALL, so 10 buffer sets (336 MB) rotate.  Pass-1 times from its dispatch events; the step time from
    events around the whole timed region."""
    import torch

    from locals_amd import _lib

    lib = _lib.load()
    stream = _lib.stream_of(dev)
    R, H, KVH, n = cfg["B"], cfg["H"], cfg["KVH"], int(cfg["nb"][0])
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    nsets = max(args.sets, 10)
    sets = [(torch.randn((R, H, 128), generator=gen, device=dev, dtype=torch.float16),
             torch.randn((R, KVH, n, 128), generator=gen, device=dev, dtype=torch.float16),
             torch.randn((R, KVH, n, 128), generator=gen, device=dev, dtype=torch.float16)) for _ in range(nsets)]
    slots = torch.arange(R, dtype=torch.int32, device=dev)
    nkeys = torch.full((R,), n, dtype=torch.int32, device=dev)
    blk = args.block or 0
    nbytes = int(lib.lcl_decode_workspace_bytes(R, H, n, blk))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    out = torch.empty((R, H, 128), dtype=torch.float16, device=dev)
    P_ = _lib.ptr
    ev = Events(2 * args.steps + 2)

    def run(i, e0=None, e1=None):
        q, K, V = sets[i % nsets]
        rc = lib.lcl_ragged_attention_ex(P_(q), 0, P_(K), P_(V), 0, P_(slots), P_(nkeys), float(1 / np.sqrt(128)),
                                         None, R, H, R, KVH, 128, n, blk, P_(out), P_(ws), nbytes, stream, e0, e1)
        _lib.check(rc, "lcl_ragged_attention_ex")

    for i in range(args.warmup):
        run(i)
    torch.cuda.synchronize()
    hip = ev.hip
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventRecord(ev.ev[-2], stream)
    every = max(1, args.p1_every)
    for i in range(args.steps):
        if i % every == 0:
            run(i, ev.ev[2 * i], ev.ev[2 * i + 1])
        else:
            run(i)
    hip.hipEventRecord(ev.ev[-1], stream)
    torch.cuda.synchronize()
    step_us = ev.ms(2 * args.steps, 2 * args.steps + 1) * 1e3 / args.steps
    p1 = np.array([ev.ms(2 * i, 2 * i + 1) for i in range(0, args.steps, every)]) * 1e3
    ev.close()
    kv = R * KVH * n * 512
    b_step = kv + 2 * R * H * 128 * 2
    return {"kernel": "ragged_pass1_16", "us_per_step": round(step_us, 2), "GBs_step": round(b_step / step_us / 1e3, 1),
            "hbm_frac_step": round(b_step / step_us / 1e3 / HBM_PEAK_GBS, 4), "pass1_avg_us": round(float(p1.mean()), 2),
            "pass1_GBs": round((kv + R * H * 256) / float(p1.mean()) / 1e3, 1), "bytes_per_step": b_step,
            "buffer_sets": nsets}


def bench_qk(args, dev):
    """The per-step kernels around attention in Flint's full-attention layers, at C2's decode step (16 rows x 1
    token) and at a 512-token prompt chunk, 32 / 8 heads: qk_norm_rope (q/k norms + RoPE, v split out),
    quantize_append (8-bit cache store of k and v) and the fused qk_norm_rope_append.  Each is one launch; the bytes
    are what the call must move: bf16 activations in and out, 272 B of cache a token and kv head.  The calls are replayed from a HIP
    graph of 20, so the time per call is the GPU's (with the gaps between the graph's launches), not the host's."""
    import types

    import torch

    from locals_amd import _lib, qk_kernel, qkv

    H, KV, HD = 32, 8, 128
    res = {}
    for name, B, L in (("decode_step", 16, 1), ("prompt_chunk", 1, 512)):
        gen = torch.Generator(device=dev)
        gen.manual_seed(5)
        dt = torch.bfloat16
        x = torch.randn((B, L, (H + 2 * KV) * HD), generator=gen, device=dev, dtype=dt)
        wq = (torch.randn(HD, generator=gen, device=dev) * 0.05 + 1).to(dt)
        wk = (torch.randn(HD, generator=gen, device=dev) * 0.05 + 1).to(dt)
        attn = types.SimpleNamespace(n_heads=H, n_kv_heads=KV, head_dim=HD,
                                     q_norm=types.SimpleNamespace(weight=wq, eps=1e-6),
                                     k_norm=types.SimpleNamespace(weight=wk, eps=1e-6),
                                     rope=types.SimpleNamespace(base=10000.0, dims=HD, traditional=False, scale=1.0))
        offs = torch.full((B,), 1000, dtype=torch.int32, device=dev)
        cap = 1024 + L
        K = qkv._zeros(B, KV, cap, HD, dt, dev)
        V = qkv._zeros(B, KV, cap, HD, dt, dev)
        q, k, v = qk_kernel.qk_norm_rope(x, attn, offs)
        lib = _lib.load()
        P = _lib.ptr
        qo = torch.empty((B, H, L, HD), dtype=dt, device=dev)

        def fused():  # the stream is read at each call: under capture it is the capturing one
            rc = lib.lcl_qk_norm_rope_append(P(x), 1, P(wq), P(wk), P(offs), 1, 1e-6, float(np.log2(10000.0)), 1, B, L,
                                             H, KV, HD, P(qo), P(K[0]), P(K[1]), P(K[2]), P(V[0]), P(V[1]), P(V[2]),
                                             cap, 1000, 0, _lib.stream_of(dev))
            _lib.check(rc, "lcl_qk_norm_rope_append")

        act = B * L * (H + 2 * KV) * HD * 2  # bf16 qkv
        cache = B * L * KV * 272  # K and V triples
        calls = {
            "qk_norm_rope": (lambda: qk_kernel.qk_norm_rope(x, attn, offs), 2 * act),
            "quantize_append": (lambda: qkv.quantize_into(k, v, K, V, 1000), B * L * KV * HD * 2 * 2 + cache),
            "qk_norm_rope_append": (fused, act + B * L * H * HD * 2 + cache),
        }
        out = {}
        per_graph = 20
        for cname, (fn, nbytes) in calls.items():
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            # 20 calls captured in one HIP graph, so the host's launch cost is not what is timed
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(per_graph):
                    fn()
            g.replay()
            torch.cuda.synchronize()
            reps = max(1, args.steps // per_graph)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
            out[cname] = {"us_per_call": round(us, 2), "bytes": nbytes, "GBs": round(nbytes / us / 1e3, 1),
                          "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        res[name] = {"B": B, "L": L, **out}
    return res


def build_sets(cfg, nsets, dev):
    import torch

    from locals_amd import qkv

    B, H, KVH = cfg["B"], cfg["H"], cfg["KVH"]
    nb = cfg["nb"]
    n = int(nb.max())
    cap = (n + 255) // 256 * 256
    start = torch.tensor(n - nb, dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev)
    sets = []
    for s in range(nsets):
        gen.manual_seed(1234 + s)
        K = qkv._zeros(B, KVH, cap, 128, torch.float16, dev)
        V = qkv._zeros(B, KVH, cap, 128, torch.float16, dev)
        for b in range(B):  # a row at a time keeps the fp16 temporaries small
            kf = torch.randn((1, KVH, cap, 128), generator=gen, device=dev, dtype=torch.float16)
            vf = torch.randn((1, KVH, cap, 128), generator=gen, device=dev, dtype=torch.float16)
            qkv.quantize_into(kf, vf, tuple(a[b:b + 1] for a in K), tuple(a[b:b + 1] for a in V), 0)
        q = torch.randn((B, H, 1, 128), generator=gen, device=dev, dtype=torch.float16)
        sets.append((q, K, V))
    torch.cuda.synchronize()
    return sets, start, n, cap


def bench_decode_extra(cfg, args, dev, return_runner=False):
    """A decode config beside the headline (C3, C4's decode rows): the whole lcl_qkv_attend (pass 1 + join) over
    >= 1 GiB of rotating buffer sets unbracketed, then pass 1 with its own dispatch events."""
    import torch

    from locals_amd import _lib, qkv

    B, H, KVH = cfg["B"], cfg["H"], cfg["KVH"]
    b_step, b_p1 = step_bytes(cfg)
    nsets = max(2, -(-(1 << 30) // b_p1))
    sets, start, n, cap = build_sets(cfg, nsets, dev)
    lib = _lib.load()
    nbytes = int(lib.lcl_decode_workspace_bytes(B, H, n, qkv.BLOCK))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    out = torch.empty((B, H, 1, 128), dtype=torch.float16, device=dev)
    stream = _lib.stream_of(dev)

    def run(i, e0=None, e1=None, st=None):
        q, K, V = sets[i % len(sets)]
        rc = lib.lcl_qkv_attend_ex(_lib.ptr(q), 0, _lib.ptr(K[0]), _lib.ptr(K[1]), _lib.ptr(K[2]), _lib.ptr(V[0]),
                                   _lib.ptr(V[1]), _lib.ptr(V[2]), 0, _lib.ptr(start), None, float(1 / np.sqrt(128)),
                                   B, H, KVH, 128, cap, n, qkv.BLOCK, _lib.ptr(out), _lib.ptr(ws), nbytes,
                                   stream if st is None else st, e0, e1)
        _lib.check(rc, "lcl_qkv_attend_ex")

    if return_runner:
        return run

    steps, warmup = max(args.steps, 20), max(args.warmup, 3)
    step_us, _ = timed_loop(run, steps, warmup, stream, 0)
    _, p1 = timed_loop(run, 4 * steps, 2, stream, 4)
    del sets
    G = H // KVH
    return {"workload": cfg["workload"], "B": B, "H": H, "KVH": KVH, "sum_n": int(cfg["nb"].sum()),
            "us_per_step": round(step_us, 2), "hbm_frac_step": round(b_step / step_us / 1e3 / HBM_PEAK_GBS, 4),
            "pass1": {"kernel": "qkv_pass1_q8_quad" if G <= 8 else "qkv_pass1_q8", "us": dist(p1),
                      "hbm_frac": round(b_p1 / float(np.mean(p1)) / 1e3 / HBM_PEAK_GBS, 4)},
            "bytes_per_step": b_step, "buffer_sets": nsets, "steps": steps}


def c4_overlap(args, dev):
    """C4's two attention calls (the 15 decode rows, the 512-query prompt chunk) in sequence on one stream, and
    concurrently on two streams of the default priority forked from and joined to it by events (what a
    co-scheduled mixed.forward layer would launch, locals/mixed.py:108-110).  µs a step of both, over the region."""
    import torch

    from locals_amd import _lib

    dec = bench_decode_extra(config("c4d"), args, dev, return_runner=True)
    pre = bench_multi(config("c4"), args, dev, return_runner=True)
    s0 = torch.cuda.current_stream(dev)
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    h1, h2 = ctypes.c_void_p(s1.cuda_stream), ctypes.c_void_p(s2.cuda_stream)

    def seq(i, e0=None, e1=None):
        dec(i)
        pre(i)

    def conc(i, e0=None, e1=None):
        fork = torch.cuda.Event()
        fork.record(s0)
        s1.wait_event(fork)
        s2.wait_event(fork)
        dec(i, st=h1)
        pre(i, st=h2)
        d1, d2 = torch.cuda.Event(), torch.cuda.Event()
        d1.record(s1)
        d2.record(s2)
        s0.wait_event(d1)
        s0.wait_event(d2)

    stream = _lib.stream_of(dev)
    steps, warmup = max(args.steps, 20), max(args.warmup, 3)
    out = {}
    for rep_ in range(2):  # interleaved, twice
        out.setdefault("sequential_us", []).append(round(timed_loop(seq, steps, warmup, stream, 0)[0], 2))
        out.setdefault("concurrent_us", []).append(round(timed_loop(conc, steps, warmup, stream, 0)[0], 2))
    torch.cuda.synchronize()
    return out


def extras(args, dev):
    """The other BASELINE configurations measured in the same run: C3 (long-context split-K decode), C4 (the decode
    rows and the 512-query prompt chunk of the hybrid batch) and C5 (tree verification), with kernel medians and
    p10 / p90, HBM and MFMA fractions."""
    import torch

    a = argparse.Namespace(**vars(args))
    a.steps, a.warmup = max(args.steps, 20), max(args.warmup, 3)
    res = {"c3": bench_decode_extra(config("c3"), a, dev)}
    torch.cuda.empty_cache()
    c4d = bench_decode_extra(config("c4d"), a, dev)
    torch.cuda.empty_cache()
    c4p = bench_multi(config("c4"), a, dev)
    torch.cuda.empty_cache()
    res["c4"] = {"decode_rows": c4d, "prefill": c4p,
                 "us_per_step_decode_then_prefill": round(c4d["us_per_step"] + c4p["us_per_call"], 2),
                 "two_streams": c4_overlap(a, dev)}
    torch.cuda.empty_cache()
    res["c5"] = bench_multi(config("c5"), a, dev)
    torch.cuda.empty_cache()
    return res


def step_bytes(cfg):
    B, H, KVH = cfg["B"], cfg["H"], cfg["KVH"]
    kv = int(cfg["nb"].sum()) * KVH * 272
    return kv + 2 * B * H * 128 + 2 * B * H * 128, kv + 2 * B * H * 128  # whole step, pass 1 (KV + Q)


def cpu_baseline(cfg, sets, start, n, seconds, gpu_out):
    """The C port of the reference algorithm on the host cores over the same inputs (set 0): whole steps repeated
    until ``seconds`` of CPU time; also its max |difference| from the GPU's output of the same step."""
    import torch

    threads = min(16, len(os.sched_getaffinity(0)))
    os.environ["OMP_NUM_THREADS"] = str(threads)
    sys.path.insert(0, ROOT)
    from oracle import cbind

    q, K, V = sets[0]
    tonp = lambda t: t.cpu().numpy()  # noqa: E731
    qn = tonp(q)
    Kn = (tonp(K[0]).view(np.uint32), tonp(K[1]), tonp(K[2]))
    Vn = (tonp(V[0]).view(np.uint32), tonp(V[1]), tonp(V[2]))
    st = tonp(start)
    reps, t0 = 0, time.perf_counter()
    out = None
    while True:
        out = cbind.attend_q8(qn, Kn, Vn, n, None, 1 / np.sqrt(128), st, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / reps
    err = float(np.abs(out.astype(np.float64) - gpu_out.float().cpu().numpy()).max())
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return per, reps, threads, cpu, err


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # 500 untimed steps (~55 ms at C2): the first few hundred decode steps after set-up run 2-3 us slower (C2 on
    # one box: 116.7-117.6 us a step after 20 warm-up steps, 113.8-114.3 after 300, 1000 or 3000)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--sets", type=int, default=2)
    ap.add_argument("--block", type=int, default=None, help="keys a pass-1 workgroup reads (qkv.BLOCK)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip C3 / C4 / C5 beside the headline")
    ap.add_argument("--p1-every", type=int, default=4, metavar="K",
                    help="bracket every K-th step's pass-1 dispatch with HIP events (the roofline sample)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the bench: K device copies of MIB MiB (the known-size kernel that scales the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    sys.path.insert(0, ROOT)
    from locals_amd import _lib, qkv

    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        ms = copy_ms(n, args.steps, dev)
        print(json.dumps({"calibrate_copy_bytes": n, "dispatches": args.steps, "ms_per_copy": round(ms, 4),
                          "copy_GBs_read_plus_write": round(2 * n / ms / 1e6, 1)}), flush=True)
        return
    cfg = config(args.config)
    if args.block is not None:
        qkv.BLOCK = args.block
    if cfg["name"] == "c1":
        print(json.dumps({"config": cfg["workload"], "ragged_decode": bench_c1(cfg, args, dev)}), flush=True)
        return
    if cfg["name"] == "qk":
        print(json.dumps({"config": cfg["workload"], "qk_and_cache_store": bench_qk(args, dev)}), flush=True)
        return
    if cfg["name"] in ("c4", "c5", "w1"):
        from locals_amd import sdpa

        if args.block is not None:
            sdpa.BLOCK = args.block
        multi = bench_multi(cfg, args, dev)
        if cfg["name"] in ("c5", "w1"):
            key = "tree_verify" if cfg["name"] == "c5" else "window_prefill"
            print(json.dumps({"config": cfg["workload"], key: multi}), flush=True)
            return
        cfg = dict(cfg, workload=cfg["workload"])  # the decode rows below; the prefill part reported beside them
    sets, start, n, cap = build_sets(cfg, args.sets, dev)
    B, H, KVH = cfg["B"], cfg["H"], cfg["KVH"]
    lib = _lib.load()
    nbytes = int(lib.lcl_decode_workspace_bytes(B, H, n, qkv.BLOCK))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=dev)
    outs = [torch.empty((B, H, 1, 128), dtype=torch.float16, device=dev) for _ in sets]
    stream = _lib.stream_of(dev)
    scale = 1 / np.sqrt(128)
    K_ = args.steps
    ev = Events(2 * K_ + 2)

    def step(i, e0=None, e1=None):
        q, K, V = sets[i % len(sets)]
        rc = lib.lcl_qkv_attend_ex(_lib.ptr(q), 0, _lib.ptr(K[0]), _lib.ptr(K[1]), _lib.ptr(K[2]), _lib.ptr(V[0]),
                                   _lib.ptr(V[1]), _lib.ptr(V[2]), 0, _lib.ptr(start), None, float(scale), B, H, KVH,
                                   128, cap, n, qkv.BLOCK, _lib.ptr(outs[i % len(sets)]), _lib.ptr(ws), nbytes,
                                   stream, e0, e1)
        _lib.check(rc, "lcl_qkv_attend_ex")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # timed region: K steps; the pass-1 dispatch of each records its own start/stop events
    t0 = time.perf_counter()
    hip = ev.hip
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventRecord(ev.ev[-2], stream)
    every = max(1, args.p1_every)
    for i in range(K_):
        if i % every == 0:
            step(i, ev.ev[2 * i], ev.ev[2 * i + 1])
        else:
            step(i)
    hip.hipEventRecord(ev.ev[-1], stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    region_ms = ev.ms(2 * K_, 2 * K_ + 1)
    p1 = np.array([ev.ms(2 * i, 2 * i + 1) for i in range(0, K_, every)])
    ev.close()
    # after the timed region, for pass 1's distribution: 80 more steps, every 4th dispatch bracketed
    _, p1_more = timed_loop(step, 80, 2, stream, 4)
    # secondary rooflines, outside the timed region: what a plain 1 GiB device copy and a plain streaming read of
    # 1 GiB move per second on this part
    copy_gbs = 2 * (1 << 30) / copy_ms(1 << 30, 20, dev) / 1e6
    read_gbs, read_how = read_probe(1 << 30, 20, dev)

    ms_step = region_ms / K_
    # the pass-1 kernel the library runs for this head ratio (4x4x4-MFMA stream-K kernel for G <= 8)
    kernel = "qkv_pass1_q8_quad" if H // KVH <= 8 else "qkv_pass1_q8"
    b_step, b_p1 = step_bytes(cfg)
    value = b_step / (ms_step * 1e-3) / 1e9
    p1_us = float(p1.mean() * 1e3)
    achieved = b_p1 / (p1.mean() * 1e-3) / 1e9
    line = {
        "metric": "decode-attn µs/step + HBM GB/s (% peak), B=16 8-bit KV GQA 32/8 D=128",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K_,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "us_per_step": round(ms_step * 1e3, 2),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "B": B, "H": H, "KVH": KVH, "head_dim": 128,
                   "contexts": [int(x) for x in cfg["nb"]], "sum_n": int(cfg["nb"].sum()), "cap": cap,
                   "bytes_per_step": b_step, "buffer_sets": len(sets), "kv": "MLX affine 8-bit, group 64",
                   "compute": "u8 codes -> fp16 MFMA (exact), fp32 accumulate", "block": qkv.BLOCK or "auto",
                   "wall_s_timed": round(wall, 4)},
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "avg_us": round(p1_us, 2), "median_us": round(float(np.median(p1)) * 1e3, 2),
                     "p10_us": round(float(np.percentile(p1, 10)) * 1e3, 2),
                     "p90_us": round(float(np.percentile(p1, 90)) * 1e3, 2), "samples": int(p1.size),
                     "sampled_every": every, "after_region_us": dist(p1_more),
                     "bytes_per_launch": b_p1,
                     "traffic": _traffic(cfg["name"], kernel),
                     "measured_copy_GBs": round(copy_gbs, 1), "frac_of_measured_copy": round(achieved / copy_gbs, 4),
                     "measured_read_GBs": round(read_gbs, 1), "measured_read_setting": read_how,
                     "frac_of_measured_read": round(achieved / read_gbs, 4)},
        "cpu_baseline": None,
    }
    if cfg["name"] == "c4":
        line["prefill"] = multi
        line["us_per_step_decode_plus_prefill"] = round(ms_step * 1e3 + multi["avg_us"], 2)
    if not args.no_cpu:
        per, reps, threads, cpu, err = cpu_baseline(cfg, sets, start, n, args.cpu_seconds, outs[0])
        line["cpu_baseline"] = {"value": round(b_step / per / 1e9, 3), "unit": "GB/s", "cores": threads,
                                "kind": "port", "us_per_step": round(per * 1e6, 1), "cpu": cpu,
                                "sample": f"{reps} whole steps of buffer set 0 (the same inputs as the GPU), "
                                          f"C restatement of qkv.py's two passes (oracle/c/oracle.c), OpenMP",
                                "max_abs_diff_vs_gpu": err}
    if cfg["name"] == "c2" and not args.no_extras:
        del sets, outs, ws
        torch.cuda.empty_cache()
        line["extras"] = extras(args, dev)
    print(json.dumps(line), flush=True)


def copy_ms(nbytes, reps, dev):
    """Average ms of a device-to-device copy of `nbytes` (torch's copy kernel; bytes read + written = 2 * nbytes)."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return ms


def read_probe(nbytes, reps, dev):
    """Best streaming-read rate of the probes in locals_amd/libread_probe.so over `nbytes` (GB/s), and the setting
    that gave it.  Tried: direct buffer->LDS loads (the decode kernels' method) by 2048 / 4096 single-wave
    workgroups with rings of 2, 3 and 4 16-KiB tiles, and plain 16-byte vector loads by 4096 workgroups of 256."""
    import torch

    from locals_amd import _lib

    path = os.path.join(ROOT, "locals_amd", "libread_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run python -m locals_amd.build")
    lib = ctypes.CDLL(path)
    V = ctypes.c_void_p
    lib.lcl_probe_read_lds.argtypes = [V, ctypes.c_size_t, V, ctypes.c_int, ctypes.c_int, V]
    lib.lcl_probe_read_vec.argtypes = [V, ctypes.c_size_t, V, ctypes.c_int, V]
    lib.lcl_probe_out_words.restype = ctypes.c_size_t
    lib.lcl_probe_out_words.argtypes = [ctypes.c_int]
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    out = torch.empty(int(lib.lcl_probe_out_words(4096)), dtype=torch.int32, device=dev)
    stream = _lib.stream_of(dev)
    settings = [("lds", w, d) for w in (2048, 4096) for d in (2, 3, 4)] + [("vec", 4096, 0)]
    best = (0.0, None)
    for kind, w, d in settings:
        def launch():
            if kind == "lds":
                rc = lib.lcl_probe_read_lds(src.data_ptr(), nbytes, out.data_ptr(), w, d, stream)
            else:
                rc = lib.lcl_probe_read_vec(src.data_ptr(), nbytes, out.data_ptr(), w, stream)
            if rc:
                raise RuntimeError(f"read probe {kind} returned {rc}")

        launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        gbs = nbytes / (e0.elapsed_time(e1) / reps) / 1e6
        print(f"read probe {kind} {w} {d}: {gbs:.1f} GB/s", file=sys.stderr, flush=True)
        if gbs > best[0]:
            what = f"{w} waves, LDS ring of {d} tiles" if kind == "lds" else f"{w} x 256 threads, vector loads"
            best = (gbs, what)
    del src, out
    return best


def _traffic(name, kernel):
    """HBM bytes a pass-1 launch moved, from the committed rocprofv3 --pmc summary of this kernel, or None."""
    path = os.path.join(ROOT, "profiles", f"decode_q8_{name}_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    return d.get("traffic_bytes_per_launch") if d.get("kernel") == kernel else None


if __name__ == "__main__":
    main()
