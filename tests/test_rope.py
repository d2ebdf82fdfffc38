"""The oracle's restatement of the decoder's RoPE (ggml_rope_ext mode 0,
src/voxtral.cpp:2667-2671), pinned by what the mathematics fixes: the identity
at position 0, the fp64 closed form x'_{2i} = x_{2i} cos(p w_i) - x_{2i+1}
sin(p w_i), x'_{2i+1} = x_{2i} sin(p w_i) + x_{2i+1} cos(p w_i) with
w_i = theta^(-2i/d) at small positions (a swapped pair, a wrong sign or a
wrong frequency index fails it), norm preservation of every pair, and the
relative-position property q(p1).k(p2) = q(p1+s).k(p2+s).  ggml's f32 running
product for theta_i is followed as recalled from its public source (ggml is
not vendored), and the cos/sin of every angle the decoder and encoder use are
checked against the C library's cosf/sinf, which ggml's CPU rope calls: within
one ulp everywhere, equal for ~99% (the C library's are not correctly rounded,
so bit-equality with a ggml build depends on its libm)."""
import numpy as np

import oracle

THETA, D = 1.0e6, 128


def closed_form(x, pos, theta=THETA, d=D):
    x = np.asarray(x, np.float64)
    i = np.arange(d // 2)
    w = theta ** (-2.0 * i / d)
    out = x.copy()
    for r in range(x.shape[0]):
        a = (pos + r) * w
        c, s = np.cos(a), np.sin(a)
        for h0 in range(0, x.shape[1], d):
            x0, x1 = x[r, h0 + 2 * i], x[r, h0 + 2 * i + 1]
            out[r, h0 + 2 * i] = x0 * c - x1 * s
            out[r, h0 + 2 * i + 1] = x0 * s + x1 * c
    return out


def rows(n, width, seed):
    return np.random.default_rng(seed).standard_normal((n, width)).astype(np.float32)


def test_position_zero_is_identity():
    x = rows(1, 4 * D, 1)
    assert np.array_equal(oracle.rope(x, D, 0, THETA), x)


def test_closed_form_at_small_positions():
    x = rows(17, 2 * D, 2)
    got = oracle.rope(x, D, 0, THETA)
    want = closed_form(x, 0)
    assert np.max(np.abs(got - want)) <= 2e-5


def test_theta_and_head_width_matter():
    x = rows(4, D, 3)
    got = oracle.rope(x, D, 5, 10000.0)
    assert np.max(np.abs(got - closed_form(x, 5, theta=10000.0))) <= 2e-5
    assert np.max(np.abs(got - closed_form(x, 5))) > 1e-2
    y = rows(4, 128, 4)
    assert np.max(np.abs(oracle.rope(y, 64, 3, THETA) - closed_form(y, 3, d=64))) <= 2e-5


def test_pair_norms_preserved():
    x = rows(8, 4 * D, 5)
    y = oracle.rope(x, D, 30000, THETA).astype(np.float64)
    n0 = x.astype(np.float64).reshape(8, -1, 2)
    n1 = y.reshape(8, -1, 2)
    assert np.allclose((n1 ** 2).sum(-1), (n0 ** 2).sum(-1), rtol=1e-5, atol=1e-6)


def test_relative_position():
    q, k = rows(1, D, 6), rows(1, D, 7)
    for p1, p2, shift in ((3, 1, 5), (40, 17, 29), (100, 0, 60)):
        a = float(oracle.rope(q, D, p1, THETA)[0] @ oracle.rope(k, D, p2, THETA)[0])
        b = float(oracle.rope(q, D, p1 + shift, THETA)[0] @ oracle.rope(k, D, p2 + shift, THETA)[0])
        assert abs(a - b) <= 1e-3 * max(1.0, abs(a))


def test_rows_take_consecutive_positions():
    x = rows(6, D, 8)
    whole = oracle.rope(x, D, 1000, THETA)
    for r in range(6):
        assert np.array_equal(whole[r], oracle.rope(x[r:r + 1], D, 1000 + r, THETA)[0])


def test_cos_sin_against_the_c_library():
    """ggml's CPU rope evaluates cosf/sinf of each f32 angle (the C
    library's, glibc here).  Rotating (1, 0) pairs makes the oracle return its
    cos and sin of every angle; against glibc's cosf/sinf of the same angles
    (ggml's f32 running product restated in numpy) they agree to within one
    ulp at every angle of positions 0..8191 for the decoder's and the
    encoder's head widths, and are equal for all but ~1% (glibc's cosf/sinf
    are accurate to < 1 ulp, not correctly rounded, while the oracle rounds
    the double result).  A wrong angle (frequency index, running product, a
    swapped cos/sin) would miss by far more than one ulp."""
    import ctypes

    libm = ctypes.CDLL("libm.so.6")
    for fn in (libm.cosf, libm.sinf):
        fn.restype, fn.argtypes = ctypes.c_float, [ctypes.c_float]
    libm.powf.restype, libm.powf.argtypes = ctypes.c_float, [ctypes.c_float, ctypes.c_float]
    cosf = np.frompyfunc(lambda v: libm.cosf(float(v)), 1, 1)
    sinf = np.frompyfunc(lambda v: libm.sinf(float(v)), 1, 1)
    npos = 8192
    for d in (128, 64):
        ts = np.float32(libm.powf(THETA, np.float32(-2.0) / np.float32(d)))
        ang = np.empty((npos, d // 2), np.float32)
        ang[:, 0] = np.arange(npos, dtype=np.float32)
        for i in range(1, d // 2):
            ang[:, i] = ang[:, i - 1] * ts
        unit = np.tile(np.array([1.0, 0.0], np.float32), d // 2)[None, :].repeat(npos, 0)
        got = oracle.rope(unit, d, 0, THETA)
        got_c, got_s = got[:, 0::2], got[:, 1::2]
        want_c = cosf(ang).astype(np.float32)
        want_s = sinf(ang).astype(np.float32)
        for g, w in ((got_c, want_c), (got_s, want_s)):
            ulp = np.abs(g.view(np.int32).astype(np.int64) - w.view(np.int32).astype(np.int64))
            same_sign = np.sign(g) == np.sign(w)
            assert np.all(same_sign | (g == 0) | (w == 0))
            assert ulp.max() <= 1, d
            assert np.mean(ulp != 0) < 0.02, d
