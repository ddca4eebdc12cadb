"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference holds no fixtures or golden vectors for this path (its hot-path tests compare against MLX at run time,
tests/test_flint.py:278-295), so the expected values here come from sources independent of this repo's oracle:

* quant_known.npz -- MLX affine 8-bit groups whose codes, scales and biases follow by hand from the closed form
  (exact 255-step grids on either side of zero, constant groups, zero-ended groups, a tie group), built with
  exactly representable fp16 values.
* attn_sdpa.npz   -- small decode / masked-prefill / tree cases (with sinks) whose expected outputs come from
  torch's CPU float64 scaled_dot_product_attention, the sink entered as an extra zero key whose additive mask
  is the sink logit.
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def known_groups():
    """(rows of 128 fp16 values, expected codes (rows, 128) uint8, scales, biases (rows, 2) fp16) + tie rows."""
    rows, codes, scales, biases = [], [], [], []
    k = np.arange(64)
    step = 0.0625
    # 1. |min| > |max|: min = -255/16, values min + k step  ->  scale = +step, bias = min, code = k
    g1 = (-255 * step + k * 4 * step).astype(np.float32)
    g1[-1] = 0.0  # max = 0 exactly (code 255)
    c1 = (k * 4).astype(np.int64)
    c1[-1] = 255
    # 2. |min| <= |max|: max = 255/16, values max - k step -> scale = -step, bias = max, code = k
    g2 = (255 * step - k * 4 * step).astype(np.float32)
    g2[-1] = 0.0
    c2 = (k * 4).astype(np.int64)
    c2[-1] = 255
    rows.append(np.concatenate([g1, g2]))
    codes.append(np.concatenate([c1, c2]))
    scales.append([step, -step])
    biases.append([-255 * step, 255 * step])
    # 3. constant groups: codes 0, bias = the value, scale = value / round(value / -1e-7) (fp32 then fp16)
    for v in (1.5, -3.0):
        pass
    g3 = np.full(64, 1.5, np.float32)
    g4 = np.full(64, -3.0, np.float32)
    rows.append(np.concatenate([g3, g4]))
    codes.append(np.zeros(128, np.int64))
    s3 = np.float32(1.5) / np.float32(np.rint(np.float32(1.5) / np.float32(-1e-7)))
    s4 = np.float32(-3.0) / np.float32(np.rint(np.float32(-3.0) / np.float32(-1e-7)))
    scales.append([float(s3), float(s4)])
    biases.append([1.5, -3.0])
    # 4. all-zero group: q0 = 0 -> bias 0, scale = -1e-7, codes 0
    rows.append(np.concatenate([np.zeros(64, np.float32), g1]))
    codes.append(np.concatenate([np.zeros(64, np.int64), c1]))
    scales.append([float(np.float32(-1e-7)), step])
    biases.append([0.0, -255 * step])
    x = np.stack(rows).astype(np.float16)
    assert np.array_equal(x.astype(np.float32), np.stack(rows))  # exactly representable
    # tie row: min 0, max 255, scale = -1, bias = 255, code = round(255 - w); w = j + 0.5 is a tie for every j
    t = np.zeros(64, np.float32)
    t[1] = 255.0
    t[2:] = np.arange(62, dtype=np.float32) * 4 + 0.5
    tie_row = np.concatenate([t, t]).astype(np.float16)
    y = 255.0 - t
    away = np.where(np.abs(y - np.trunc(y)) >= 0.5, np.trunc(y) + 1, np.trunc(y))
    even = np.rint(y)
    return (x, np.stack(codes).astype(np.uint8), np.array(scales, np.float16), np.array(biases, np.float16),
            tie_row[None], np.tile(away, 2)[None].astype(np.uint8), np.tile(even, 2)[None].astype(np.uint8))


def sdpa64(q, k, v, scale, vis, sinks):
    """torch float64 SDPA with GQA by repetition and the sink as an extra zero key (additive mask = sink)."""
    q, k, v = (torch.from_numpy(np.asarray(a, np.float64)) for a in (q, k, v))
    B, H, L, D = q.shape
    KVH, N = k.shape[1], k.shape[2]
    k = k.repeat_interleave(H // KVH, 1)
    v = v.repeat_interleave(H // KVH, 1)
    mask = torch.zeros(B, H, L, N + 1, dtype=torch.float64)
    mask[..., :N] = torch.where(torch.from_numpy(np.broadcast_to(vis, (B, H, L, N)).copy()), 0.0, -np.inf)
    if sinks is None:
        mask[..., N] = -np.inf
    else:
        mask[..., N] = torch.from_numpy(np.asarray(sinks, np.float64))[None, :, None]
    k = torch.cat([k, torch.zeros(B, H, 1, D, dtype=torch.float64)], 2)
    v = torch.cat([v, torch.zeros(B, H, 1, D, dtype=torch.float64)], 2)
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)
    return out.numpy()


def attn_cases():
    g = np.random.default_rng(20261201)
    out = {}
    # decode: B=2, H=8, KVH=2, N=40, row 1 starts at key 7 (left padding), sinks
    q = g.standard_normal((2, 8, 1, 128)).astype(np.float16)
    k = (g.standard_normal((2, 2, 40, 128)) * 2).astype(np.float16)
    v = g.standard_normal((2, 2, 40, 128)).astype(np.float16)
    s = (g.standard_normal(8) * 2).astype(np.float16)
    vis = np.ones((2, 1, 1, 40), bool)
    vis[1, ..., :7] = False
    out.update(dec_q=q, dec_k=k, dec_v=v, dec_sinks=s, dec_start=np.array([0, 7], np.int32),
               dec_out=sdpa64(q, k, v, 0.0884, vis, s.astype(np.float64)))
    # causal prefill: L=6 queries over N=20 keys (the last query sees every key), no sink
    q = g.standard_normal((1, 4, 6, 128)).astype(np.float16)
    k = g.standard_normal((1, 2, 20, 128)).astype(np.float16)
    v = g.standard_normal((1, 2, 20, 128)).astype(np.float16)
    vis = (np.arange(20)[None, :] <= (20 - 6 + np.arange(6))[:, None])[None, None]
    out.update(cau_q=q, cau_k=k, cau_v=v, cau_out=sdpa64(q, k, v, 0.1, vis, None))
    # tree: prefix 9 keys + 7 new tokens; parents (preorder) -> ancestor-or-self mask
    parents = np.array([-1, 0, 1, 1, 0, 4, 5], np.int32)
    L = 7
    anc = np.zeros((L, L), bool)
    for i in range(L):
        j = i
        while j >= 0:
            anc[i, j] = True
            j = parents[j]
    vis = np.concatenate([np.ones((L, 9), bool), anc], 1)[None, None]
    q = g.standard_normal((1, 8, L, 128)).astype(np.float16)
    k = g.standard_normal((1, 2, 9 + L, 128)).astype(np.float16)
    v = g.standard_normal((1, 2, 9 + L, 128)).astype(np.float16)
    s = g.standard_normal(8).astype(np.float16)
    out.update(tree_q=q, tree_k=k, tree_v=v, tree_parents=parents, tree_sinks=s,
               tree_out=sdpa64(q, k, v, 0.0884, vis, s.astype(np.float64)))
    return out


def main():
    x, c, s, b, tie, away, even = known_groups()
    np.savez_compressed(os.path.join(HERE, "quant_known.npz"), x=x, codes=c, scales=s, biases=b, tie=tie,
                        tie_away=away, tie_even=even)
    np.savez_compressed(os.path.join(HERE, "attn_sdpa.npz"), **attn_cases())
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
