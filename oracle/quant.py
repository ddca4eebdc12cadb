"""MLX affine 8-bit quantization, group 64 -- CPU restatement (test infrastructure).

The reference never quantizes by itself: ``BatchQuantizedKVCache.update_and_fetch``
calls ``mx.quantize(x, group_size=64, bits=8)`` (locals/qkv.py:322-323) and
``dequantized`` calls ``mx.dequantize`` (locals/qkv.py:252-253).  The arithmetic is
MLX 0.32.3's (pinned at uv.lock:376-378, not vendored in the reference), restated
here from MLX's public affine quantizer:

    per group of 64 values w (input dtype T, widened to fp32):
        w_max, w_min = max(w), min(w)
        scale = max((w_max - w_min) / 255, 1e-7)
        side  = |w_min| > |w_max|
        scale = side ? scale : -scale
        edge  = side ? w_min : w_max
        q0    = round(edge / scale)
        if q0 != 0: scale = edge / q0 ; bias = edge     else: bias = 0
        code  = clamp(round((w - bias) / scale), 0, 255)  (fp32 scale and bias)
        store scale, bias as T (round to nearest even)

All arithmetic is IEEE fp32 with correctly rounded division (numpy float32).
``round`` ties away from zero on MLX's Metal GPU path (Metal ``round``) and to
even on its CPU path (``std::rint``); ``round_mode`` selects it ("away" is the
default: the reference runs ``mx.quantize`` on the Apple GPU).

Layout (locals/qkv.py:35,48,52-58,275-277): ``words`` uint32 (..., D/4), dim 4w+i
in byte i of word w (little endian); ``scales``/``biases`` (..., D/64), group g
covering dims [64g, 64g+64).  Dequantization is ``scale * code + bias``
(locals/qkv.py:57-58).

bfloat16 is carried as uint16 bit patterns (numpy has no bf16); see ``bf16_round``.
"""

from __future__ import annotations

import numpy as np

BITS, GROUP = 8, 64
N_BINS = np.float32(255.0)
EPS = np.float32(1e-7)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = np.where(nan, (u >> np.uint64(16)) | np.uint64(0x40), r)
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_f32(x, dtype: str) -> np.ndarray:
    """Values of a 16-bit tensor as float32: fp16 arrays, or bf16 bit patterns."""
    if dtype == "bfloat16":
        return bf16_to_f32(x)
    return np.asarray(x).astype(np.float32)


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> the 16-bit storage of ``dtype`` (fp16 array, or bf16 bits), RNE."""
    if dtype == "bfloat16":
        return bf16_round(x)
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def _round(x: np.ndarray, mode: str) -> np.ndarray:
    """fp32 rounding to an integer value: "even" = rint, "away" = C roundf (Metal round)."""
    if mode == "even":
        return np.rint(x).astype(np.float32)
    if mode != "away":
        raise ValueError(f"round_mode must be 'away' or 'even', not {mode!r}")
    t = np.trunc(x).astype(np.float32)
    frac = (x - t).astype(np.float32)  # exact in fp32
    return np.where(np.abs(frac) >= np.float32(0.5), t + np.sign(x).astype(np.float32), t).astype(np.float32)


def quantize(w, dtype: str = "float16", group: int = GROUP, round_mode: str = "away"):
    """MLX ``mx.quantize(w, group_size=64, bits=8)`` (affine) of ``w`` (..., D).

    ``w`` is a float16 array, or bf16 bit patterns when ``dtype == "bfloat16"``.
    Returns ``(words uint32 (..., D/4), scales, biases)`` with scales/biases in the
    16-bit storage of ``dtype``.
    """
    x = to_f32(w, dtype)
    shape = x.shape
    D = shape[-1]
    if D % group:
        raise ValueError("last dim must be a multiple of the group size")
    g = x.reshape(-1, D // group, group)
    with np.errstate(divide="ignore", invalid="ignore"):
        w_max = g.max(-1, keepdims=True)
        w_min = g.min(-1, keepdims=True)
        scale = np.maximum((w_max - w_min) / N_BINS, EPS).astype(np.float32)
        side = np.abs(w_min) > np.abs(w_max)
        scale = np.where(side, scale, -scale).astype(np.float32)
        edge = np.where(side, w_min, w_max).astype(np.float32)
        q0 = _round((edge / scale).astype(np.float32), round_mode)
        at_zero = q0 == 0
        scale = np.where(at_zero, scale, (edge / np.where(at_zero, np.float32(1), q0)).astype(np.float32))
        bias = np.where(at_zero, np.float32(0), edge).astype(np.float32)
        codes = _round(((g - bias) / scale).astype(np.float32), round_mode)
    codes = np.clip(codes, 0, 255).astype(np.uint8).reshape(-1, D)
    words = np.ascontiguousarray(codes).view("<u4").reshape(shape[:-1] + (D // 4,))
    scales = from_f32(scale.reshape(shape[:-1] + (D // group,)), dtype)
    biases = from_f32(bias.reshape(shape[:-1] + (D // group,)), dtype)
    return words, scales, biases


def codes_of(words: np.ndarray) -> np.ndarray:
    """uint32 words (..., D/4) -> uint8 codes (..., D)."""
    w = np.ascontiguousarray(words, dtype="<u4")
    return w.view(np.uint8).reshape(w.shape[:-1] + (w.shape[-1] * 4,))


def dequantize(words, scales, biases, dtype: str = "float16", group: int = GROUP, out=np.float64) -> np.ndarray:
    """``scale * code + bias`` per group (locals/qkv.py:57-58), in ``out`` precision.

    In float64 the products are exact, which is what the float64 attention oracle
    consumes.  ``out=np.float32`` gives the reference kernels' fp32 value when they
    do not fuse the multiply-add.
    """
    c = codes_of(words).astype(out)
    s = to_f32(scales, dtype).astype(out)
    b = to_f32(biases, dtype).astype(out)
    D = c.shape[-1]
    c = c.reshape(c.shape[:-1] + (D // group, group))
    v = c * s[..., None] + b[..., None]
    return v.reshape(v.shape[:-2] + (D,))
