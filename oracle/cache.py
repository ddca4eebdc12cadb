"""The 8-bit cache's row bookkeeping restated on numpy triples (test infrastructure).

Follows BatchQuantizedKVCache in the reference (locals/qkv.py:295-452; mlx-lm's BatchKVCache semantics) and
QuantizedKVCache8's growth (mlx-lm QuantizedKVCache, as pinned by uv.lock:428-430): a triple is
(words uint32 (B, KVH, cap, D/4), scales, biases (B, KVH, cap, D/64)) of any 16-bit dtype carried as uint16 bits
here, since the operations only move bytes.  A cache is a dict with keys "keys", "values" (triples or None),
"offset" (B,), "left_padding" (B,), "idx" (int) -- the reference's ``_idx``.

* ``grow``      qkv.py:311-319: keep the first prev positions, append ceil(S / step) * step zero positions
* ``merge``     qkv.py:417-431: right-align each request's first n_i positions in L = max n_i
* ``extend``    qkv.py:382-406: both sides moved right to the larger ``_idx``, cut or zero-padded to the larger capacity
* ``filter``    qkv.py:370-380: keep rows, then drop their common left padding
* ``extract``   qkv.py:408-415: one row's positions [left_padding, _idx)
* ``finalize``  qkv.py:340-346: each row rolled right by its right padding (mlx-lm dynamic_roll, numpy.roll)
"""

from __future__ import annotations

import numpy as np

STEP = 256


def zeros(B, KVH, cap, D=128):
    return (np.zeros((B, KVH, cap, D // 4), np.uint32), np.zeros((B, KVH, cap, D // 64), np.uint16),
            np.zeros((B, KVH, cap, D // 64), np.uint16))


def _cat(ts, axis):
    return tuple(np.concatenate(x, axis=axis) for x in zip(*ts))


def grow(t, prev: int, S: int, KVH: int, B: int, D: int = 128, step: int = STEP):
    """The triple after making room for S positions at prev (None: a new buffer)."""
    if t is not None and prev + S <= t[0].shape[2]:
        return t
    new = zeros(B, KVH, (S + step - 1) // step * step, D)
    if t is None:
        return new
    return _cat([tuple(a[:, :, :prev] for a in t), new], axis=2)


def merge(caches, KVH: int, D: int = 128):
    """caches: list of (triple or None, n) single-request caches (rows of 1) -> batch cache."""
    lengths = [n if t is not None else 0 for t, n in caches]
    L = max(lengths)
    out = {"left_padding": np.array([L - n for n in lengths]), "offset": np.array(lengths), "idx": L}
    if L == 0:
        out["keys"] = None
        return out
    k = zeros(len(caches), KVH, L, D)
    for i, ((t, _), n) in enumerate(zip(caches, lengths)):
        if n:
            for a, x in zip(k, t):
                a[i, :, L - n:] = x[0, :, :n]
    out["keys"] = k
    return out


def extend(a: dict, b: dict, KVH: int, D: int = 128):
    """Batch cache a followed by the rows of b."""
    if a["keys"] is None and b["keys"] is None:
        return {"keys": None, "left_padding": np.concatenate([a["left_padding"], b["left_padding"]]),
                "offset": np.concatenate([a["offset"], b["offset"]]), "idx": a["idx"]}
    max_idx = max(a["idx"], b["idx"])
    size = max(c["keys"][0].shape[2] for c in (a, b) if c["keys"] is not None)

    def pad(c):
        t = c["keys"] if c["keys"] is not None else zeros(len(c["offset"]), KVH, 0, D)
        left = max_idx - c["idx"]
        right = size - t[0].shape[2] - left
        if right < 0:
            t = tuple(x[:, :, :right] for x in t)
            right = 0
        t = tuple(np.pad(x, ((0, 0), (0, 0), (left, right), (0, 0))) for x in t)
        return t, c["left_padding"] + left

    (ta, pa), (tb, pb) = pad(a), pad(b)
    return {"keys": _cat([ta, tb], axis=0), "left_padding": np.concatenate([pa, pb]),
            "offset": np.concatenate([a["offset"], b["offset"]]), "idx": max_idx}


def filter_rows(c: dict, idx):
    idx = list(idx)
    t = None if c["keys"] is None else tuple(x[idx] for x in c["keys"])
    lp, off, i = c["left_padding"][idx], c["offset"][idx], c["idx"]
    drop = int(lp.min()) if len(lp) else 0
    if drop > 0:
        if t is not None:
            t = tuple(x[:, :, drop:] for x in t)
        i -= drop
        lp = lp - drop
    return {"keys": t, "left_padding": lp, "offset": off, "idx": i}


def extract(c: dict, row: int):
    p = int(c["left_padding"][row])
    t = tuple(x[row:row + 1, :, p:c["idx"]] for x in c["keys"])
    return t, c["idx"] - p


def finalize(c: dict, right_padding):
    rp = np.asarray(right_padding)
    t = c["keys"]
    if t is not None:
        t = tuple(np.stack([np.roll(x[b], int(rp[b]), axis=1) for b in range(x.shape[0])]) for x in t)
    return {"keys": t, "left_padding": c["left_padding"] + rp, "offset": c["offset"] - rp, "idx": c["idx"]}
