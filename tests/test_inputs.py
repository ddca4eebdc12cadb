"""The seeded input generators shared by the GPU tests and the bench do what their docstrings claim (CPU)."""

import numpy as np

from oracle import quant as oq
from tests.inputs import peaked_inputs, rng


def test_peaked_inputs_have_one_dominant_key_and_a_deep_tail():
    g = rng(1)
    B, H, KVH, cap = 2, 8, 2, 1024
    lo, hi = np.array([0, 100]), np.array([1000, 1000])
    q, K, V, dom = peaked_inputs(g, B, H, KVH, 1, cap, lo, hi, scale=0.0884)
    kd = oq.dequantize(*K)
    G = H // KVH
    for b in range(B):
        for h in range(H):
            s = 0.0884 * (kd[b, h // G, lo[b]:hi[b]] @ q[b, h, 0].astype(np.float64))
            l2 = (s - s.max()) / np.log(2.0)
            assert int(np.argmax(s)) + lo[b] == dom[b, h // G, 0]
            tail = np.sort(l2)[:-1]
            assert tail.max() < -6.0  # the dominant key carries > 98% of the weight
            assert np.median(tail) < -8.0 and tail.min() > -30.0


def test_peaked_inputs_fix_the_v_scale_sign_per_group():
    g = rng(2)
    _, _, V, _ = peaked_inputs(g, 2, 8, 2, 1, 512, np.zeros(2, int), np.full(2, 512))
    sc = V[1].astype(np.float32)  # (B, KVH, cap, 2)
    assert ((sc > 0).all(axis=2) | (sc < 0).all(axis=2)).all()
