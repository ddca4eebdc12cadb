"""CPU emulation of the 8-bit decode kernels' P.V arithmetic, one head over one wave's run of 64-key tiles.

The 8-bit pass-1 kernels (locals_amd/csrc/decode.hip) multiply V on MFMA with A = w = p * v_scale (per key and
64-dim group) as an fp16 hi + lo pair and B = 1024 + code (exact in fp16); the 1024 offset and the bias go into an
fp32 side sum, so a head's output is

    o_d = (sum_t w^_t (1024 + c_td) + sum_t (p_t b_t - 1024 w_t)) / sum_t p_t          (w^ = hi + lo)

and its error is sum_t (w^_t - w_t)(1024 + c_td) / l.  These tests run that arithmetic in numpy (fp16 casts, fp32
products and sums; the MFMA's own sums in float64) against the float64 closed form of the reference's pass 1
(locals/qkv.py:50-66: p = exp(s - m), o += p * (scale * code + bias) in fp32) on the case the split is worst at: one
dominant key over a long tail 10..18 log2 below it, and V groups with a common offset, so MLX's scale has one sign
in every group and rounding errors of w add up instead of cancelling.

* ``scheme="rtz"`` is the earlier arithmetic: w split with round-toward-zero at the softmax's own reference
  (p <= 2^6), so for |w| < 2^-3 the lo half is an fp16 subnormal, and the (1024 + code) factor multiplies what it
  drops.  The test shows this misses the 2e-3 bar.
* ``scheme="scaled"`` is the kernels' arithmetic: the softmax reference moves down by a wave-uniform E (p' = 2^E p),
  with E = 9 - e(S), S < 2^e(S) the largest |V scale| of the tile, lowered (never raised) when a later tile's
  scales need it, so max w' <= 2^15 and the weights that matter have normal hi and lo; both halves round to
  nearest.  Every product and sum is scaled by the same 2^E, so the partial (m_ref, l', o') keeps o'/l' = o/l.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quant

TILE = 64
THR = 6.0  # lazy softmax rescale threshold (log2), as in the kernels


def _f16_rtz(x: np.ndarray) -> np.ndarray:
    """float32 -> fp16 rounded toward zero (v_cvt_pkrtz_f16_f32), as float32 values."""
    x = np.asarray(x, dtype=np.float32)
    h = x.astype(np.float16)
    over = np.abs(h.astype(np.float32)) > np.abs(x)
    h = np.where(over, np.nextafter(h, np.float16(0)), h)
    return h.astype(np.float32)


def _f16_rne(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def _exp2(x):
    with np.errstate(over="ignore"):
        return np.exp2(np.asarray(x, dtype=np.float64)).astype(np.float32)


def _scale_exponent(sc: np.ndarray) -> int:
    """e with max|sc| < 2^e from the fp16 bits (the kernels take the largest magnitude's exponent field)."""
    bits = np.asarray(sc, dtype=np.float16).view(np.uint16) & np.uint16(0x7FFF)
    hm = int(bits.max()) if bits.size else 0
    return (hm >> 10) - 14


def emulate(s, codes, sc, b, scheme: str):
    """One wave's partial of one head: s (N,) base-2 logits, codes (N, 128) uint8, sc / b (N, 2) fp16 of V.

    Returns (m, l, o[128]) with o already divided by l."""
    N = s.shape[0]
    m_run = -np.inf
    E = 40  # upper bound of the prescale exponent; the first tile lowers it
    mref = np.float32(-np.inf)
    l_acc = np.float32(0)
    wb = np.zeros(2, np.float32)
    O = np.zeros(128, np.float32)
    c = codes.astype(np.float64)
    scf = sc.astype(np.float32)
    bf = b.astype(np.float32)
    for t0 in range(0, N, TILE):
        sl = slice(t0, min(N, t0 + TILE))
        st = s[sl].astype(np.float32)
        tmax = float(st.max())
        need_m = tmax > m_run + THR
        if scheme == "scaled":
            et = 9 - _scale_exponent(sc[sl])
            need_e = et < E
        else:
            need_e = False
        if need_m or need_e:
            if need_e:
                E = et
            if need_m:
                m_run = tmax
            new_ref = np.float32(m_run - (E if scheme == "scaled" else 0))
            corr = np.float32(0) if mref == -np.inf else _exp2(mref - new_ref)
            mref = new_ref
            l_acc = np.float32(l_acc * corr)
            wb = (wb * corr).astype(np.float32)
            O = (O * corr).astype(np.float32)
        p = _exp2(st - mref)
        x = (p[:, None] * scf[sl]).astype(np.float32)  # w' (keys, group)
        y = (p[:, None] * bf[sl]).astype(np.float32)
        if scheme == "rtz":
            hi = _f16_rtz(x)
            lo = _f16_rtz((x - hi).astype(np.float32))
        else:
            hi = _f16_rne(x)
            lo = _f16_rne((x - hi).astype(np.float32))
        w_hat = hi.astype(np.float64) + lo.astype(np.float64)
        for g in range(2):
            prod = (w_hat[:, g:g + 1] * (1024.0 + c[sl, 64 * g:64 * g + 64])).sum(0)
            O[64 * g:64 * g + 64] = (O[64 * g:64 * g + 64] + prod).astype(np.float32)
        for k in range(st.shape[0]):
            l_acc = np.float32(l_acc + p[k])
            for g in range(2):
                wb[g] = np.float32(wb[g] + np.float32(np.float64(-1024.0) * x[k, g] + y[k, g]))
    o = (O.astype(np.float64) + np.repeat(wb.astype(np.float64), 64)) / np.float64(l_acc)
    return float(mref), float(l_acc), o


def exact(s, codes, sc, b):
    """float64: sum_t 2^s_t (sc c + b) / sum_t 2^s_t."""
    p = np.exp2(s.astype(np.float64) - s.max())
    v = codes.astype(np.float64).reshape(-1, 2, 64) * sc.astype(np.float64)[:, :, None] + \
        b.astype(np.float64)[:, :, None]
    return (p @ v.reshape(-1, 128)) / p.sum()


def peaked_case(seed: int, N: int = 1088, offset: float = 3.0, lo: float = 10.0, hi: float = 18.0, first=True):
    """A dominant key (logit 0) and N - 1 keys lo..hi log2 below it; V = N(0, 1) + offset quantized by MLX's
    affine rule (one scale sign per group when the offset dominates)."""
    g = np.random.default_rng(seed)
    s = -g.uniform(lo, hi, N).astype(np.float32)
    s[0 if first else N // 2] = 0.0
    V = (g.standard_normal((N, 128)) + offset).astype(np.float16)
    w, scales, biases = quant.quantize(V)
    return s, quant.codes_of(w), scales, biases


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_round_toward_zero_split_misses_the_bar_on_peaked_softmax(seed):
    s, c, sc, b = peaked_case(seed)
    assert (sc.astype(np.float32) < 0).all()  # the offset fixes the scale sign
    _, _, o = emulate(s, c, sc, b, "rtz")
    err = np.abs(o - exact(s, c, sc, b)).max()
    assert err > 1e-2, err


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("N,first", [(1088, True), (1088, False), (4096, True)])
def test_scaled_split_is_fp32_grade_on_peaked_softmax(seed, N, first):
    s, c, sc, b = peaked_case(seed, N=N, first=first)
    _, _, o = emulate(s, c, sc, b, "scaled")
    err = np.abs(o - exact(s, c, sc, b)).max()
    # what is left is the fp32 rounding of the side sum -1024 w' + p b, which cancels the MFMA's 1024 w' terms:
    # ~2^-24 * 1024 * |w'| a step, i.e. ~2^-14 S over a run of keys (S ~ 0.03 here), with or without the split
    assert err < 1e-4, err


def test_scaled_split_flat_softmax_and_zero_mean_v():
    g = np.random.default_rng(5)
    N = 2048
    s = (g.standard_normal(N) * 1.5).astype(np.float32)
    V = g.standard_normal((N, 128)).astype(np.float16)
    w, sc, b = quant.quantize(V)
    c = quant.codes_of(w)
    for scheme in ("rtz", "scaled"):
        _, _, o = emulate(s, c, sc, b, scheme)
        assert np.abs(o - exact(s, c, sc, b)).max() < 2e-4


def test_scaled_split_tracks_growing_scales():
    """Later tiles with 2^12 x larger V scales lower E (w' stays within fp16: no inf / NaN) and the result keeps its
    precision; smaller later scales leave E alone."""
    g = np.random.default_rng(6)
    N = 1024
    s = (g.standard_normal(N) * 2).astype(np.float32)
    V = g.standard_normal((N, 128)).astype(np.float32)
    V[N // 2:] *= 4096.0
    V[N // 4:N // 2] /= 4096.0
    w, sc, b = quant.quantize(V.astype(np.float16))
    c = quant.codes_of(w)
    _, _, o = emulate(s, c, sc, b, "scaled")
    ref = exact(s, c, sc, b)
    assert np.isfinite(o).all()
    # the side sum's fp32 rounding scales with the largest |V scale| S (~2^-14 S a run of keys)
    S = np.abs(sc.astype(np.float64)).max()
    assert np.abs(o - ref).max() <= 2.0 ** -12 * S


def test_gpu_peaked_inputs_would_fail_the_old_split():
    """The GPU tests' peaked generator (tests/inputs.py) is a case the earlier arithmetic gets wrong: one wave's run
    of 17 tiles starting at the dominant key of one (row, kv head), scores and V exactly as the kernel sees them."""
    from oracle.quant import dequantize
    from tests.inputs import peaked_inputs, rng

    g = rng(301)
    q, K, V, dom = peaked_inputs(g, 1, 4, 1, 1, 4096, np.array([0]), np.array([4000]), scale=0.0884)
    t0 = int(dom[0, 0, 0]) // TILE * TILE
    run = slice(t0, t0 + 17 * TILE)
    kd = dequantize(*K)[0, 0, run]
    s = (0.0884 * (kd @ q[0, 0, 0].astype(np.float64)) / np.log(2.0)).astype(np.float32)
    c = quant.codes_of(V[0])[0, 0, run]
    sc, b = V[1][0, 0, run], V[2][0, 0, run]
    ref = exact(s, c, sc, b)
    err_old = np.abs(emulate(s, c, sc, b, "rtz")[2] - ref).max()
    err_new = np.abs(emulate(s, c, sc, b, "scaled")[2] - ref).max()
    assert err_old > 2e-3 and err_new < 1e-4, (err_old, err_new)
