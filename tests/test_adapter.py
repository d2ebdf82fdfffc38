"""The realtime rows rings and the adapter on the CPU oracle
(voxtral_ctx_adapter_commit src/voxtral.cpp:5424-5485,
build_adapter_ring_graph_reusable :2589-2620, copy_chunk_to_enc_out_ring
:4018-4043, read_realtime_ring_rows :5530-5554; ring capacities :42-55).

Checks that do not restate the oracle: GELU against math.erf; the rings
against a dictionary of logical rows; the adapter's gather against the batch
adapter's reshape of a contiguous frame run (build_adapter_graph :2531-2534)
and its products against fp64 products of the dequantized weights, bounded by
the Q8_K rounding of the inputs (|x - dq(q8k(x))| <= d/2 per element)."""
import math

import numpy as np
import pytest

import oracle
from kq_util import random_matrix

ENC, DEC, DOWN, CAP = 1280, 3072, 4, 256


def test_gelu_erf_closed_form():
    xs = np.concatenate([np.linspace(-8, 8, 4001), [0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0]])
    got = oracle.gelu_erf(xs.astype(np.float32)).astype(np.float64)
    want = np.array([0.5 * x * (1 + math.erf(x / math.sqrt(2))) for x in xs.astype(np.float32)])
    # f32 evaluation of 0.5 x (1 + erf): 1 + erf cancels for x << 0, so the
    # error is relative to |x| there (ggml's own formula, not a defect)
    xf = np.abs(xs.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4e-7 * np.abs(want) + 1.2e-7 * xf + 1e-37)
    assert got[-2] == np.float32(30.0) and got[-1] == 0.0
    # not the tanh approximation (ggml_gelu): they differ by ~1e-4 near |x| = 2
    x = np.float32(2.0)
    tanh_approx = 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    assert abs(oracle.gelu_erf(np.array([x]))[0] - tanh_approx) > 1e-5


def test_ring_rows_match_a_dictionary_of_logical_rows():
    rng = np.random.default_rng(4018)
    cap, width = 12, 5
    ring = np.zeros((cap, width), np.float32)
    logical = {}
    pos = 0
    for _ in range(40):
        n = int(rng.integers(0, cap + 1))
        rows = rng.standard_normal((n, width)).astype(np.float32)
        oracle.row_ring_write(ring, pos, rows)
        for i in range(n):
            logical[pos + i] = rows[i]
        pos += n
        if pos == 0:
            continue
        lo = max(0, pos - cap)
        k = int(rng.integers(1, pos - lo + 1))
        start = int(rng.integers(lo, pos - k + 1))
        got = oracle.row_ring_read(ring, start, k)
        assert np.array_equal(got, np.stack([logical[r] for r in range(start, start + k)]))
    with pytest.raises(ValueError):
        oracle.row_ring_write(ring, 0, np.zeros((cap + 1, width), np.float32))
    with pytest.raises(ValueError):
        oracle.row_ring_read(ring, 0, cap + 1)
    with pytest.raises(ValueError):
        oracle.row_ring_read(ring, -1, 1)


def q8k_image(x):
    return oracle.dequantize(oracle.Q8_K, oracle.q8_k_quantize(x), x.size).astype(np.float64)


def q8k_half_step(x):
    """d/2 of each element's Q8_K block: the rounding bound of the image"""
    d = np.abs(oracle.q8_k_quantize(x).reshape(-1, 292)[:, :4].copy().view(np.float32)[:, 0])
    return np.repeat(d.astype(np.float64) / 2, 256)


@pytest.fixture(scope="module")
def adapter_weights():
    rng = np.random.default_rng(2589)
    w0 = random_matrix(rng, oracle.Q4_K, DEC, ENC * DOWN, 0.03)
    w2 = random_matrix(rng, oracle.Q6_K, DEC, DEC, 0.5)
    w0d = oracle.dequantize(oracle.Q4_K, w0, DEC * ENC * DOWN).reshape(DEC, -1).astype(np.float64)
    w2d = oracle.dequantize(oracle.Q6_K, w2, DEC * DEC).reshape(DEC, DEC).astype(np.float64)
    return w0, w2, w0d, w2d


def gelu64(x):
    from scipy.special import erf
    return 0.5 * x * (1 + erf(x / math.sqrt(2)))


def test_adapter_gathers_four_frames_and_applies_both_products(adapter_weights):
    """groups 60..67 straddle the 256-frame ring's wrap (frames 240..271)"""
    w0, w2, w0d, w2d = adapter_weights
    rng = np.random.default_rng(5424)
    n_frames = 272
    frames = rng.standard_normal((n_frames, ENC)).astype(np.float32)
    enc = np.zeros((CAP, ENC), np.float32)
    for f0 in range(0, n_frames, 16):
        oracle.row_ring_write(enc, f0, frames[f0:f0 + 16])
    aemb = np.full((CAP, DEC), np.nan, np.float32)
    g0, n = 60, 8
    oracle.adapter_commit(enc, aemb, g0, n, oracle.Q4_K, w0, oracle.Q6_K, w2)
    # the batch adapter's view: frames [4g, 4g + 4) reshaped into one row
    xs = frames.reshape(-1, ENC * DOWN)[g0:g0 + n]
    for i in range(n):
        x = xs[i]
        xq, hx = q8k_image(x), q8k_half_step(x)
        pre = w0d @ xq
        pre_err = 1e-5 * (np.abs(w0d) @ np.abs(xq))
        h = gelu64(pre)
        # gelu is 1.13-Lipschitz; the second input's own Q8_K rounding adds d_h / 2
        h_err = 1.13 * pre_err
        hq_bound = np.abs(h).max() / 127 / 2 + h_err.max()
        y = w2d @ h
        bound = np.abs(w2d) @ (h_err + hq_bound) + 1e-5 * (np.abs(w2d) @ np.abs(h))
        got = aemb[(g0 + i) % CAP].astype(np.float64)
        assert np.all(np.abs(got - y) <= bound), i
        # the unquantized input would miss by up to the Q8_K rounding: the
        # input was quantized (the bound above is not met by chance)
        assert np.all(np.abs(w0d @ x.astype(np.float64) - pre) <= np.abs(w0d) @ hx + pre_err)
    untouched = np.ones(CAP, bool)
    untouched[[(g0 + i) % CAP for i in range(n)]] = False
    assert np.isnan(aemb[untouched]).all()


def test_adapter_is_the_composition_of_pinned_steps(adapter_weights):
    """bit for bit: gather (reshape rule) -> matvec -> gelu -> matvec, rows
    stored at g % capacity, later groups overwriting earlier ones"""
    w0, w2, _, _ = adapter_weights
    rng = np.random.default_rng(5433)
    enc = rng.standard_normal((16, ENC)).astype(np.float32)      # a 16-frame ring: 4 groups
    aemb = np.zeros((3, DEC), np.float32)                         # a 3-row audio ring
    oracle.adapter_commit(enc, aemb, 5, 4, oracle.Q4_K, w0, oracle.Q6_K, w2)
    want = {}
    for g in range(5, 9):
        x = enc.reshape(-1, ENC * DOWN)[g % 4]
        h = oracle.gelu_erf(oracle.matvec(oracle.Q4_K, w0, DEC, ENC * DOWN, x, n_threads=8))
        want[g % 3] = oracle.matvec(oracle.Q6_K, w2, DEC, DEC, h, n_threads=8)
    for slot, y in want.items():
        assert np.array_equal(aemb[slot], y)


def test_adapter_rejects_a_ring_that_splits_groups(adapter_weights):
    w0, w2, _, _ = adapter_weights
    enc = np.zeros((10, ENC), np.float32)
    with pytest.raises(ValueError):
        oracle.adapter_commit(enc, np.zeros((4, DEC), np.float32), 0, 1, oracle.Q4_K, w0,
                              oracle.Q6_K, w2)


def test_time_embedding_closed_form():
    """compute_time_embedding (src/voxtral.cpp:729-740): cos of the first half,
    sin of the second, frequencies exp(-ln(10000) i / half); at t = 6 (the
    delay tokens, :1535) and a few other times"""
    for t in (6.0, 0.0, 1.0, 37.5):
        e = oracle.time_embedding(t, 3072).astype(np.float64)
        i = np.arange(1536)
        ang = t * np.exp(-np.log(10000.0) * i / 1536)
        assert np.allclose(e[:1536], np.cos(ang), rtol=0, atol=3e-6)
        assert np.allclose(e[1536:], np.sin(ang), rtol=0, atol=3e-6)
    assert np.all(oracle.time_embedding(0.0, 3072)[:1536] == 1) and \
        np.all(oracle.time_embedding(0.0, 3072)[1536:] == 0)


def ada_w0(rng, ad, dim):
    """Q4_K rows whose products with e(t) straddle GELU's bend: small
    scales, and the sign of d flipped on odd rows (a negative fp16 d is a
    valid block)"""
    w0 = random_matrix(rng, oracle.Q4_K, ad, dim, 0.004).reshape(ad, dim // 256, 144)
    w0[1::2, :, 1] |= 0x80
    return w0.reshape(-1)


def test_ada_scale_against_fp64():
    """build_decoder_layer's ada MLP (:2864-2874): W2 gelu(W0 e(t)), W0 Q4_K
    [32][3072] through the Q8_K product, W2 f16 [3072][32] with its input
    rounded to f16"""
    rng = np.random.default_rng(2864)
    dim, ad = 3072, 32
    w0 = ada_w0(rng, ad, dim)
    w2 = (rng.standard_normal((dim, ad)) * 0.1).astype(np.float16)
    got = oracle.ada_scale(oracle.Q4_K, w0, w2.view(np.uint16), dim, ad, 6.0).astype(np.float64)
    e = oracle.time_embedding(6.0, dim)
    w0d = oracle.dequantize(oracle.Q4_K, w0, ad * dim).reshape(ad, dim).astype(np.float64)
    eq = q8k_image(e)
    pre = w0d @ eq
    h = gelu64(pre)
    dh = 1.13 * 1e-5 * (np.abs(w0d) @ np.abs(eq)) + 1e-7 * np.abs(h)
    hf = h.astype(np.float16).astype(np.float64)   # the f16 vec-dot input
    w2d = w2.astype(np.float64)
    want = w2d @ hf
    # a change of h within dh may move its f16 rounding by one ulp
    bound = np.abs(w2d) @ (dh + np.abs(hf) * 2.0 ** -10) + 1e-6 * np.abs(want)
    assert np.all(np.abs(got - want) <= bound)
    # not the unrounded product and not without GELU: both miss by more
    assert np.abs(w2d @ gelu64(pre) - w2d @ pre).max() > 100 * bound.max()
