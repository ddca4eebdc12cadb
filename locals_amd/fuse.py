"""``attend_few`` -- drop-in for locals/fuse.py:128-144 on the MI355X kernels.

The reference pads a pass of 5 to 8 queries a row in front to 9, because MLX's attention runs a path twice as slow
for 5 to 8 (locals/fuse.py:131-137), and drops the padding's outputs.  ``lcl_sdpa`` has no such regime (every L
goes through the same MFMA tiles), so nothing is padded here; the outputs are what the padded reference returns
for the real queries (tests/test_flint.py:534-552 pins that the padding is invisible).

``banded`` is the sliding-window layers' prompt-chunk attention (``FusedFlintAttention._banded``,
locals/fuse.py:113-125; ``Attention._windowed``, locals/models/flint_streamed.py:114-128): the reference slices
FLINT_BAND queries at a time against the keys their window reaches; here one launch does it, each workgroup
reading its own queries' band of keys.
"""

from __future__ import annotations

import os

from .sdpa import WindowMask, scaled_dot_product_attention

FEW_PAD = os.environ.get("LOCALS_FEW_QUERY_PAD", "1") != "0"  # kept for the reference's flag; no effect here
FLINT_BAND = int(os.environ.get("LOCALS_FLINT_BAND", "512"))  # the reference's band size; no effect here


def attend_few(q, k, v, scale: float, mask, sinks):
    """Attention of a prompt chunk, span or tree (several queries a row) over 16-bit K/V (locals/fuse.py:131)."""
    return scaled_dot_product_attention(q, k, v, scale=scale, mask=mask, sinks=sinks)


def attend_few_q8(q, keys, values, scale: float, mask, sinks, start=None):
    """The same over a cache's 8-bit triples, dequantized in LDS (the reference's
    ``attend_few(q, dequantized(keys), dequantized(values), ...)``, locals/qkv.py:270-272)."""
    return scaled_dot_product_attention(q, keys, values, scale=scale, mask=mask, sinks=sinks, start=start)


def banded(q, k, v, W: int, scale: float, sinks):
    """A prompt chunk's attention in a sliding-window layer of window W (locals/fuse.py:113-125): q (B, H, L, D) is
    the last L of the N keys of k/v (B, KVH, N, D); query i sees keys (N - L + i - W, N - L + i].  The same
    scores as the whole chunk under the window's mask array, reading only the keys each query's window reaches."""
    return scaled_dot_product_attention(q, k, v, scale=scale, mask=WindowMask(W), sinks=sinks)
