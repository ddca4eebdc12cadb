"""CPU oracle for the batched-attention hot path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import, call, link or run anything under
``oracle/``, and only as the checker (or the timed CPU baseline), never as the
thing measured or shipped.  The product path (``locals_amd``) never imports it and
fails loudly when its HIP library is missing.

Contents
--------
``quant``   MLX affine 8-bit quantize / dequantize (group 64), numpy float32.
``attn``    float64 closed forms of the attention variants: 8-bit split-K
            decode with sinks (``attend``), masked SDPA with sinks (``sdpa``),
            ragged fp16 decode (``ragged_attention``), the mask builders, and
            ``qk_norm_rope``.
``c/``      a C (OpenMP) restatement of the reference's two-pass split-K
            decode and of the quantizer; built into ``oracle/liboracle.so``.
            It is the CPU baseline ``bench.py`` times (kind "port").

Pinning (what checks each function, all in ``tests/test_oracle.py``):

* ``quant.quantize`` -- known-answer groups that follow from the MLX closed form
  (constant group, exact 255-step grids on either side, max==0 / min==0,
  +-symmetric, tie cases for both rounding modes), the dequantization error
  bound ``|w - dq(q(w))| <= |scale|/2 + fp16 rounding``, edge-to-code-0, and
  agreement with the independent C restatement.
* ``attn.attend`` / ``attn.sdpa`` / ``attn.ragged_attention`` -- torch's CPU
  float64 ``scaled_dot_product_attention`` (an independent library routine) with
  the sink expressed as an extra zero key whose additive mask is the sink,
  block-size independence of the C split-K restatement, key permutation
  invariance, GQA == MHA with repeated K/V, single-key and empty-range closed
  forms, garbage outside ``[start, n)``.
* masks -- chain tree == causal; branch formula of the reference equals the
  ancestor-or-self mask of the equivalent parent array; brute-force ancestor
  walk on small random trees.
* ``attn.qk_norm_rope`` -- torch RMS norm + a complex-number RoPE in float64
  within the reference's own bar (0.02 * max|ref|, tests/test_flint.py:235-236).

Parity unpinned: MLX's exact tie rounding and its treatment of an all-negative
group inside ``mx.quantize`` (MLX 0.32.3 is not installed and no reference
fixture holds codes); the oracle implements MLX's published affine closed form
(``quant.quantize`` docstring) with a selectable tie mode.
"""

from . import attn, quant  # noqa: F401
