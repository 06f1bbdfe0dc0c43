"""Pins the oracle's speech-decoder restatement (oracle/qtts_oracle_decoder.c)
primitive by primitive, against closed forms and a float64 brute force
written from the reference's definitions (tests/numpy_decoder.py), and the
whole decode_to_audio of a small decoder (every stage, the window exceeded)
against the float64 model.  The cases are chosen so a dropped term, a wrong
sign, a shifted tap, an off-by-one window or a transposed weight fails one.

Tolerances: each primitive within 1e-5 of its float64 value (relative to the
output's largest magnitude; f32 sums of <= a few hundred terms); the whole
decode within 1e-4."""
import numpy as np
import pytest

import numpy_decoder as nd
import qtts
from oracle import oracle
from qtts_file_writer import SMALL_DECODER

dec = oracle.dec
TOL = 1e-5


def rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(1e-30, float(np.max(np.abs(ref)))))


def rnd(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


@pytest.mark.parametrize("k,dil", [(1, 1), (3, 1), (7, 1), (7, 3), (7, 9)])
def test_causal_conv(k, dil):
    cin, cout, L = 5, 6, 40
    x, w, b = rnd(1, cin, L), rnd(2, cout, cin, k, scale=0.3), rnd(3, cout)
    got = dec.causal_conv(x, w, b, dil)
    assert got.shape == (cout, L)
    assert rel(got, nd.causal_conv(x, w, b, dil)) < TOL
    # causality: changing the last input sample moves only the last output
    x2 = x.copy()
    x2[:, -1] += 1.0
    d = np.abs(dec.causal_conv(x2, w, b, dil) - got).max(axis=0)
    assert np.all(d[:-1] == 0) and d[-1] > 0


def test_causal_conv_threads_and_impulse():
    """An impulse at t0 reproduces the kernel taps at t0 + (K-1-k)*dil; the
    channel split over threads changes nothing."""
    cin, cout, k, dil, L = 1, 3, 4, 2, 20
    w, b = rnd(4, cout, cin, k), np.zeros(cout, np.float32)
    x = np.zeros((cin, L), np.float32)
    x[0, 5] = 1.0
    y = dec.causal_conv(x, w, b, dil, nthreads=1)
    for kk in range(k):
        assert np.array_equal(y[:, 5 + (k - 1 - kk) * dil], w[:, 0, kk])
    x = rnd(5, 4, 33)
    w4 = rnd(6, 7, 4, 3)
    assert np.array_equal(dec.causal_conv(x, w4, rnd(7, 7), 1, nthreads=1),
                          dec.causal_conv(x, w4, rnd(7, 7), 1, nthreads=3))


@pytest.mark.parametrize("k,s", [(2, 2), (4, 2), (6, 3), (16, 8), (5, 5)])
def test_transposed_conv(k, s):
    cin, cout, L = 4, 3, 9
    x, w, b = rnd(8, cin, L), rnd(9, cin, cout, k, scale=0.4), rnd(10, cout)
    got = dec.transposed_conv(x, w, b, s)
    ref = nd.transposed_conv(x, w, b, s)
    assert got.shape == ref.shape == (cout, L * s)  # (L-1)s + k cropped by k - s
    assert rel(got, ref) < TOL


def test_transposed_conv_skips_zero_inputs_exactly():
    """The reference skips exact-zero inputs; zeros contribute nothing, so
    the output is the bias there."""
    w, b = rnd(11, 2, 2, 4), rnd(12, 2)
    y = dec.transposed_conv(np.zeros((2, 6), np.float32), w, b, 2)
    assert np.array_equal(y, np.repeat(b[:, None], 12, axis=1))


@pytest.mark.parametrize("pad", [0, 3])
def test_depthwise_conv_is_causal_whatever_its_padding(pad):
    c, k, L = 6, 7, 25
    x, w, b = rnd(13, c, L), rnd(14, c, k), rnd(15, c)
    got = dec.depthwise_conv(x, w, b, padding=pad)
    assert rel(got, nd.depthwise_conv(x, w, b)) < TOL
    x2 = x.copy()
    x2[:, 10] += 1.0
    d = np.abs(dec.depthwise_conv(x2, w, b, padding=pad) - got).max(axis=0)
    assert np.all(d[:10] == 0) and np.all(d[10:17] > 0) and np.all(d[17:] == 0)


def test_snake_closed_form():
    c, L = 5, 64
    x = np.linspace(-6, 6, c * L, dtype=np.float32).reshape(c, L)
    a, b = rnd(16, c, scale=0.5), rnd(17, c, scale=0.5)
    got = dec.snake(x, a, b)
    ref = x.astype(np.float64) + np.exp(-b.astype(np.float64))[:, None] * np.sin(
        np.exp(a.astype(np.float64))[:, None] * x) ** 2
    assert np.max(np.abs(got - ref)) < 4e-6 * np.max(np.abs(ref))
    # alpha = beta = 0: x + sin(x)^2; x = 0 stays 0
    z = dec.snake(x, np.zeros(c, np.float32), np.zeros(c, np.float32))
    assert np.max(np.abs(z - (x + np.sin(x.astype(np.float64)) ** 2))) < 4e-6
    assert dec.snake(np.zeros((1, 3), np.float32), a[:1], b[:1]).tolist() == [[0.0, 0.0, 0.0]]


def test_gelu_tanh_form():
    for x in (-8.0, -3.0, -1.0, -0.25, 0.0, 0.5, 1.0, 2.0, 7.5):
        ref = x * 0.5 * (1.0 + np.tanh(x / np.sqrt(2.0)))
        assert abs(dec.gelu(x) - ref) <= 2e-7 * max(1.0, abs(ref)), x
    # the tanh form, not erf: at x = 1 the two differ by ~0.04
    assert abs(dec.gelu(1.0) - 0.8413447) > 0.01


def test_layer_norm_and_rms_norm():
    c, L = 16, 11
    x, g, b = rnd(18, c, L, scale=3.0), rnd(19, c), rnd(20, c)
    assert rel(dec.layer_norm_cf(x, g, b), nd.layer_norm_cf(x, g, b)) < TOL
    # a constant column normalises to beta
    const = np.full((c, 2), 4.0, np.float32)
    assert np.array_equal(dec.layer_norm_cf(const, g, b), np.repeat(b[:, None], 2, axis=1))
    v, gv = rnd(21, 64, scale=2.0), rnd(22, 64)
    assert rel(dec.rms_norm(v, gv), nd.rms_norm(v, gv)) < TOL
    ones = np.ones(64, np.float32)
    assert np.allclose(dec.rms_norm(np.full(64, 3.0, np.float32), ones), 3.0 / np.sqrt(9.0 + 1e-5), rtol=1e-7)


def test_rope_split_half():
    heads, hd, rows = 3, 16, 10
    half = hd // 2
    ang = np.arange(rows)[:, None] * (1.0 / 10000.0 ** (np.arange(half) * 2 / hd))[None, :]
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x = rnd(23, heads * hd)
    assert np.array_equal(dec.rope(x, heads, hd, 0, cs, sn), x)  # position 0: identity
    assert np.array_equal(dec.rope(x, heads, hd, rows, cs, sn), x)  # past the table: unchanged
    for pos in (1, 5, 9):
        got = dec.rope(x, heads, hd, pos, cs, sn)
        assert rel(got, nd.rope_split_half(x, heads, hd, pos, cs, sn)) < TOL
        # each pair (i, i + half) keeps its norm
        g, r = got.reshape(heads, hd).astype(np.float64), x.reshape(heads, hd).astype(np.float64)
        assert np.allclose(g[:, :half] ** 2 + g[:, half:] ** 2, r[:, :half] ** 2 + r[:, half:] ** 2, rtol=1e-5)


@pytest.mark.parametrize("T,window", [(1, 4), (10, 4), (10, 72), (9, 1)])
def test_window_attention(T, window):
    heads, hd = 2, 8
    q, k, v = rnd(24, T, heads * hd), rnd(25, T, heads * hd), rnd(26, T, heads * hd)
    got = dec.window_attention(q, k, v, heads, hd, window)
    assert rel(got, nd.window_attention(q, k, v, heads, hd, window)) < TOL
    # the first row, and every row of a window of 1, is its own v
    assert np.array_equal(got[0], v[0])
    if window == 1:
        assert np.array_equal(got, v)


def test_codebook_lookup():
    w = qtts.DecoderWeights(27, SMALL_DECODER)
    codes = w.synthetic_codes(28, 6)
    got = dec.codebook_lookup(w, codes)
    assert rel(got, nd.codebook_lookup(w, codes)) < TOL


@pytest.mark.parametrize("frames", [1, 12])
def test_decode_to_audio_matches_float64(frames):
    """The whole decoder: codebooks, pre-conv, the windowed transformer (12
    frames exceed its window of 8), ConvNeXt upsampling and the Vocos blocks."""
    w = qtts.DecoderWeights(29, SMALL_DECODER)
    codes = w.synthetic_codes(30 + frames, frames)
    got = oracle.decode_to_audio(w, codes)
    ref = nd.decode_to_audio(w, codes)
    assert got.shape == ref.shape
    assert np.max(np.abs(ref)) < 1.0  # the clamp does not hide differences
    assert rel(got, ref) < 1e-4
