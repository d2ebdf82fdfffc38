"""The encoder conv stem's oracle (build_encoder_kv_graph, src/voxtral.cpp:
2094-2126; causal_conv1d_graph :1767-1816; compute_causal_conv1d_dims
:1670-1687): against an independent fp64 im2col of the same f16-rounded
operands, the dependence window the reference states (encoder frame e reads
Mel[2e-3 .. 2e+1], :3678-3680), and bit-exact frames from different plans'
windows past the stream start (the property the plan's window relies on)."""
import math

import numpy as np
import pytest
from scipy.special import erf

import oracle

N_MEL, DIM = 128, 256   # the reference's 128 bins; a narrow channel count keeps it fast


def weights(rng, dim=DIM):
    w0 = (rng.standard_normal((dim, N_MEL, 3)) * 0.05).astype(np.float16)
    w1 = (rng.standard_normal((dim, dim, 3)) * 0.05).astype(np.float16)
    b0 = (rng.standard_normal(dim) * 0.1).astype(np.float32)
    b1 = (rng.standard_normal(dim) * 0.1).astype(np.float32)
    return w0.view(np.uint16), b0, w1.view(np.uint16), b1


def test_conv_dims_closed_form():
    for n in range(1, 300):
        # stride 1: same length, pad 2; stride 2: ceil(n / 2), pad 1
        assert oracle.conv_dims(n, 3, 1) == (2, n)
        assert oracle.conv_dims(n, 3, 2) == (1, math.ceil(n / 2))


def gelu64(v):
    return 0.5 * v * (1 + erf(v / np.sqrt(2.0)))


def conv64(inp, w, b, stride):
    """fp64 causal conv of [t][ch] input (f16-rounded), weights [oc][ic][3]"""
    n, ch = inp.shape
    pad = 3 - stride
    out_len = (n + pad - 3) // stride + 1 if stride == 1 else math.ceil(n / 2)
    x = np.zeros((n + pad + 3, ch))
    x[pad:pad + n] = inp.astype(np.float16).astype(np.float64)
    wf = w.view(np.float16).astype(np.float64)
    y = np.empty((out_len, wf.shape[0]))
    for t in range(out_len):
        win = x[t * stride:t * stride + 3]          # [3][ch]
        y[t] = np.einsum("oik,ki->o", wf, win) + b
    return gelu64(y)


def test_conv_stem_against_fp64():
    rng = np.random.default_rng(2094)
    w0, b0, w1, b1 = weights(rng)
    conv_len, n_new = 36, 16
    mel = rng.standard_normal((N_MEL, conv_len)).astype(np.float32)
    got = oracle.conv_stem(mel, 2, n_new, w0, b0, w1, b1)
    y0 = conv64(mel.T, w0, b0, 1).astype(np.float32)
    want = conv64(y0, w1, b1, 2)[2:2 + n_new]
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-4)   # y0 is re-rounded to f16


def test_dependence_window():
    rng = np.random.default_rng(3678)
    w0, b0, w1, b1 = weights(rng)
    conv_len = 40
    mel = rng.standard_normal((N_MEL, conv_len)).astype(np.float32)
    base = oracle.conv_stem(mel, 0, conv_len // 2, w0, b0, w1, b1)
    e = 8
    for m, changes in ((2 * e - 4, False), (2 * e - 3, True), (2 * e + 1, True), (2 * e + 2, False)):
        mp = mel.copy()
        mp[:, m] += 1.0
        got = oracle.conv_stem(mp, 0, conv_len // 2, w0, b0, w1, b1)
        assert (not np.array_equal(got[e], base[e])) == changes, m


@pytest.mark.parametrize("q_start,n_new", [(2, 4), (30, 16), (57, 5)])
def test_plan_windows_give_the_same_frames(q_start, n_new):
    """frames from a plan's window [2(q-2), 2(q+n)) equal those of one big
    window from the stream start, bit for bit"""
    rng = np.random.default_rng(q_start)
    w0, b0, w1, b1 = weights(rng)
    total = 2 * (q_start + n_new)
    mel = rng.standard_normal((N_MEL, total)).astype(np.float32)
    big = oracle.conv_stem(mel, 0, total // 2, w0, b0, w1, b1)
    start = max(0, 2 * (q_start - 2))
    slice_start = q_start - start // 2
    part = oracle.conv_stem(np.ascontiguousarray(mel[:, start:total]), slice_start, n_new,
                            w0, b0, w1, b1)
    assert np.array_equal(part, big[q_start:q_start + n_new])
