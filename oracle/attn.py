"""float64 closed forms of the attention variants on the hot path (test infrastructure).

Every function returns float64; the HIP path is compared against these on the same
seeded inputs.  Each follows a reference file:line; all keep the reference's
conventions:

* the sink is a logit in the softmax denominator only (locals/qkv.py:198-207,
  tests/test_flint_streamed.py:167-184);
* ``"causal"`` aligns the last query with the last key: query i of L sees key j of
  N iff j <= N - L + i (locals/fuse.py:131-137);
* GQA: query head h reads key/value head h // (H / KVH) (locals/qkv.py:43,49);
* a row with no visible key and no sink gives 0 (locals/attention.py:82,182 do so
  for ragged rows; the same convention is used everywhere here).
"""

from __future__ import annotations

import numpy as np

from .quant import dequantize, from_f32, to_f32


def _f64(x, dtype="float16"):
    return to_f32(x, dtype).astype(np.float64) if dtype == "bfloat16" else np.asarray(x).astype(np.float64)


def _softmax_rows(s: np.ndarray, v: np.ndarray, sink: float) -> np.ndarray:
    """sum_j softmax([s_j] U {sink})_j v_j for one row of scores s (N,) and values v (N, D)."""
    m = max(float(s.max()) if s.size else -np.inf, sink)
    if m == -np.inf:
        return np.zeros(v.shape[-1])
    e = np.exp(s - m)
    den = e.sum() + (np.exp(sink - m) if sink != -np.inf else 0.0)
    return (e @ v) / den


def attend(q, keys, values, n: int, sinks, scale: float, start, dtype: str = "float16") -> np.ndarray:
    """``qkv.attend`` (locals/qkv.py:213-249): one query a row over 8-bit K/V triples.

    q (B, H, 1, HD); keys/values = (words, scales, biases) of shape (B, KVH, cap, .);
    row b attends to keys [max(start[b], 0), n) (locals/qkv.py:40); ``sinks`` (H,) or
    None; ``scale`` is rounded to fp32 as the reference passes it
    (locals/qkv.py:241).  Split-K is an implementation detail of the reference
    (A.3 algebra, locals/qkv.py:40-86,185-207); its result is this softmax.
    """
    kd = dequantize(*keys, dtype=dtype)
    vd = dequantize(*values, dtype=dtype)
    qf = _f64(q, dtype)
    B, H, _, HD = qf.shape
    KVH = kd.shape[1]
    G = H // KVH
    sc = float(np.float32(scale))
    sk = None if sinks is None else _f64(sinks, dtype)
    st = np.asarray(start).astype(np.int64)
    out = np.zeros((B, H, 1, HD))
    for b in range(B):
        lo, hi = max(int(st[b]), 0), int(n)
        for h in range(H):
            kv = h // G
            s = sc * (kd[b, kv, lo:hi] @ qf[b, h, 0]) if hi > lo else np.zeros(0)
            sink = -np.inf if sk is None else float(sk[h])
            out[b, h, 0] = _softmax_rows(s, vd[b, kv, lo:hi] if hi > lo else np.zeros((0, HD)), sink)
    return out


def causal_mask(L: int, N: int) -> np.ndarray:
    """MLX's ``"causal"``: (L, N) bool, query i sees key j iff j <= N - L + i (locals/fuse.py:131-137)."""
    return np.arange(N)[None, :] <= (N - L + np.arange(L))[:, None]


def window_mask(L: int, N: int, W: int) -> np.ndarray:
    """A sliding-window layer's mask over a prompt chunk (mlx-lm's create_causal_mask with window_size W, as a
    RotatingKVCache layer gets it, locals/models/flint.py:157): (L, N) bool, query i at position N - L + i sees key
    j iff N - L + i - W < j <= N - L + i.  The lower bound is the one the reference's band slicing assumes
    (locals/fuse.py:122: a band's first query reaches back W - 1 keys)."""
    pos = (N - L + np.arange(L))[:, None]
    j = np.arange(N)[None, :]
    return (j <= pos) & (j > pos - W)


def banded_sdpa(q, k, v, scale: float, W: int, sinks=None, band: int = 512, dtype: str = "float16") -> np.ndarray:
    """``FusedFlintAttention._banded`` (locals/fuse.py:113-125): the chunk's L queries (the last L of the N keys) in
    bands of ``band``, each band attending over the slice of keys its window reaches, with the matching slice of
    the window mask; the bands' outputs concatenated along the queries."""
    L, N = np.shape(q)[2], np.shape(k)[2]
    P = N - L
    mask = window_mask(L, N, W)
    outs = []
    for a in range(0, L, band):
        b = min(L, a + band)
        lo, hi = max(0, P + a - (W - 1)), P + b
        outs.append(sdpa(q[:, :, a:b], k[:, :, lo:hi], v[:, :, lo:hi], scale, mask[a:b, lo:hi][None, None], sinks,
                         dtype))
    return np.concatenate(outs, axis=2)


def branch_mask(br) -> np.ndarray:
    """The reference's tree mask over the new tokens (locals/treedec.py:56-67, locals/packed.py:176-181):
    token i sees token j iff j <= i and (same branch or j on the main path, br[j] < 0)."""
    br = np.asarray(br)
    L = br.size
    qi, kj = np.arange(L)[:, None], np.arange(L)[None, :]
    return (kj <= qi) & ((br[:, None] == br[None, :]) | (br[None, :] < 0))


def ancestor_mask(parents) -> np.ndarray:
    """Ancestor-or-self mask of a tree in preorder (parent[i] < i, -1 for a root): (L, L) bool."""
    p = np.asarray(parents)
    L = p.size
    m = np.zeros((L, L), dtype=bool)
    for i in range(L):
        j = i
        while j >= 0:
            m[i, j] = True
            j = int(p[j])
    return m


def tree_full_mask(local: np.ndarray, prefix: int) -> np.ndarray:
    """(L, prefix + L): the prefix is visible to every new token (locals/treedec.py:66)."""
    L = local.shape[0]
    return np.concatenate([np.ones((L, prefix), dtype=bool), np.asarray(local, dtype=bool)], axis=1)


def sdpa(q, k, v, scale: float, mask=None, sinks=None, dtype: str = "float16") -> np.ndarray:
    """MLX ``scaled_dot_product_attention(q, k, v, scale, mask, sinks)`` as the reference calls it
    (locals/fuse.py:139,144; locals/treedec.py:79; locals/packed.py:141; locals/tree.py:95).

    q (B, H, L, D); k, v (B, KVH, N, D); mask None, "causal", or a bool array
    broadcastable to (B, H, L, N); sinks (H,) or None.
    """
    qf, kf, vf = _f64(q, dtype), _f64(k, dtype), _f64(v, dtype)
    B, H, L, D = qf.shape
    KVH, N = kf.shape[1], kf.shape[2]
    G = H // KVH
    if mask is None:
        vis = np.ones((1, 1, L, N), dtype=bool)
    elif isinstance(mask, str):
        if mask != "causal":
            raise ValueError(mask)
        vis = causal_mask(L, N)[None, None]
    else:
        vis = np.asarray(mask, dtype=bool)
    vis = np.broadcast_to(vis, (B, H, L, N))
    sk = None if sinks is None else _f64(sinks, dtype)
    out = np.zeros((B, H, L, D))
    for b in range(B):
        for h in range(H):
            kv = h // G
            s = scale * (qf[b, h] @ kf[b, kv].T)  # (L, N)
            sink = -np.inf if sk is None else float(sk[h])
            for i in range(L):
                sel = vis[b, h, i]
                out[b, h, i] = _softmax_rows(s[i, sel], vf[b, kv][sel], sink)
    return out


def sdpa_q8(q, keys, values, scale: float, mask=None, sinks=None, n: int | None = None, dtype: str = "float16",
            round_kv: bool = True):
    """``attend_few(q, dequantized(K), dequantized(V), ...)`` (locals/qkv.py:270-272): SDPA over the first
    ``n`` keys of 8-bit triples.  The reference dequantizes into T (``mx.dequantize`` returns the scales' dtype)
    before MLX's attention; ``round_kv`` rounds the fp32 dequantized values to T likewise."""
    kd = dequantize(*keys, dtype=dtype, out=np.float32 if round_kv else np.float64)
    vd = dequantize(*values, dtype=dtype, out=np.float32 if round_kv else np.float64)
    if round_kv:
        kd = _round_t(kd, dtype).astype(np.float64)
        vd = _round_t(vd, dtype).astype(np.float64)
    if n is not None:
        kd, vd = kd[:, :, :n], vd[:, :, :n]
    sk = None if sinks is None else _f64(sinks, dtype)
    return sdpa(_f64(q, dtype), kd, vd, scale, mask, sk, dtype="float64")


def attention_prompt(q, keys, values, scale: float, mask, sinks_f32, n: int, dtype: str = "float16"):
    """``qkv.attention``'s prompt branch (locals/qkv.py:270-272) after the store: the sinks, given as float32 values
    (a model's parameter), are cast to the queries' dtype (``sinks.astype(q.dtype)``) before ``attend_few`` over the
    dequantized cache; the rest is ``sdpa_q8``."""
    sk = None if sinks_f32 is None else from_f32(np.asarray(sinks_f32, dtype=np.float32), dtype)
    return sdpa_q8(q, keys, values, scale, mask, sk, n=n, dtype=dtype)


def ragged_attention(q, keys, values, slots, nkeys, scale) -> np.ndarray:
    """``attention.ragged_attention`` (locals/attention.py:200-224): row r of the packed batch reads KV slot
    ``slots[r]`` and its first ``nkeys[r]`` keys; fp32 scale; output 0 for a row with no keys
    (locals/attention.py:82,182).  q (R, H, D); keys/values (n_slots, Hkv, cap, D)."""
    qf, kf, vf = (np.asarray(x).astype(np.float64) for x in (q, keys, values))
    R, H, D = qf.shape
    Hkv = kf.shape[1]
    G = H // Hkv
    sc = float(np.float32(np.asarray(scale).reshape(-1)[0]))
    out = np.zeros((R, H, D))
    for r in range(R):
        sl, N = int(slots[r]), int(nkeys[r])
        for h in range(H):
            kv = h // G
            s = sc * (kf[sl, kv, :N] @ qf[r, h])
            out[r, h] = _softmax_rows(s, vf[sl, kv, :N], -np.inf)
    return out


def _round_t(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to the 16-bit activation dtype and back to float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "bfloat16":
        from .quant import bf16_round, bf16_to_f32

        return bf16_to_f32(bf16_round(x))
    return x.astype(np.float16).astype(np.float32)


def qk_norm_rope(qkv, q_w, k_w, eps: float, offsets, H: int, KV: int, HD: int, rope: bool,
                 base: float = 10000.0, dtype: str = "float16"):
    """``qk_kernel.qk_norm_rope`` (locals/qk_kernel.py:24-109) with its rounding points.

    qkv (B, L, (H + 2 KV) * HD) as float32 values of ``dtype``; q_w, k_w (HD,) likewise.
    Per head: r = 1/sqrt(mean(x^2) + eps) with eps the fp32 value the reference passes
    (qk_kernel.py:50,103); a = T(w * T(x * r)) (qk_kernel.py:56-57); RoPE over halves at
    position offsets[b] + l (qk_kernel.py:51) with the angle in the reference's fp32 steps
    (qk_kernel.py:59): e = fp32(-2i) / fp32(HD) * fp32(log2 base), inv = fp32(2^e),
    theta = fp32(pos * inv); cos/sin of theta and the rotation in float64, rounded to fp32
    and then to T (qk_kernel.py:60-62); v copied exactly (qk_kernel.py:33-37).
    Everything else is float64 (sum of squares, r, x * r), rounded to fp32 then T.
    Returns float32 arrays q (B, H, L, HD), k and v (B, KV, L, HD) holding T values.
    """
    x = np.asarray(qkv, dtype=np.float32)
    B, L, _ = x.shape
    x = x.reshape(B, L, H + 2 * KV, HD)
    offs = np.asarray(offsets, dtype=np.int64).reshape(-1)
    qw, kw = np.asarray(q_w, dtype=np.float32), np.asarray(k_w, dtype=np.float32)
    half = HD // 2
    eps32 = float(np.float32(eps))
    e = (np.float32(-2.0) * np.arange(half, dtype=np.float32)) / np.float32(HD) * np.float32(np.log2(base))
    inv = np.exp2(e.astype(np.float64)).astype(np.float32)  # (half,) fp32

    def norm(t, w):
        ss = (t.astype(np.float64) ** 2).sum(-1, keepdims=True)
        r = 1.0 / np.sqrt(ss / HD + eps32)
        n = _round_t((t * r).astype(np.float32), dtype)
        return _round_t(w * n, dtype).astype(np.float64)

    def rot(a, pos):
        th = (pos.astype(np.float32)[..., None] * inv).astype(np.float64)  # fp32 product, (..., half)
        c, s = np.cos(th), np.sin(th)
        lo, hi = a[..., :half], a[..., half:]
        return _round_t(np.concatenate([lo * c - hi * s, lo * s + hi * c], -1).astype(np.float32), dtype)

    qn = norm(x[:, :, :H], qw)
    kn = norm(x[:, :, H:H + KV], kw)
    pos = (offs[:, None] if offs.size > 1 else np.full((B, 1), offs[0])) + np.arange(L)[None, :]  # (B, L)
    if rope:
        qn = rot(qn, pos[:, :, None])
        kn = rot(kn, pos[:, :, None])
    q = np.asarray(qn, dtype=np.float32).transpose(0, 2, 1, 3)
    k = np.asarray(kn, dtype=np.float32).transpose(0, 2, 1, 3)
    v = x[:, :, H + KV:].transpose(0, 2, 1, 3).copy()
    return q, k, v
