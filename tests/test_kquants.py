"""Decoder weight formats and the CPU matrix-vector product (ggml Q4_K / Q6_K
weights, Q8_K activations; ggml_mul_mat at src/voxtral.cpp:2656-2659, 2857,
2878-2882, quantization mix src/voxtral-quantize.cpp:148-159).

Checks of the oracle that do not restate it: blocks are packed here from
chosen scales and codes by an independent writer of the byte layout, and
dequantized values must equal the closed form; the integer dot products must
agree with fp64 dots of the dequantized operands; the Q8_K quantizer is held to
its closed forms (extreme element -> -127, first-occurrence tie, half-even
rounding, error <= d/2)."""
import numpy as np
import pytest

import oracle

F16 = np.float16


def f16_bits(v):
    return np.asarray(v, dtype=np.float16).view(np.uint16)


def pack_q4_k(d, dmin, sc, m, q):
    """One Q4_K block from d, dmin (f16-representable), sc[8], m[8] (0..63)
    and codes q[256] (0..15)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(f16_bits(d).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(f16_bits(dmin).tobytes(), np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= m[j] & 63
        else:
            s[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    blk[4:16] = s.astype(np.uint8)
    q = np.asarray(q).reshape(4, 2, 32)           # [pair c][sub-block parity][l]
    blk[16:] = (q[:, 0, :] | (q[:, 1, :] << 4)).astype(np.uint8).ravel()
    return blk


def pack_q6_k(d, scales, q):
    """One Q6_K block from d, scales[16] (int8) and codes q[256] (0..63)."""
    q = np.asarray(q).reshape(2, 4, 32)           # [half n][group g][l]
    ql = np.zeros((2, 64), np.int64)
    qh = np.zeros((2, 32), np.int64)
    for g in range(4):
        lo = q[:, g, :] & 15
        half = 32 * (g & 1)
        ql[:, half:half + 32] |= lo << (4 * (g >> 1))
        qh[:, :] |= (q[:, g, :] >> 4) << (2 * g)
    blk = np.zeros(210, np.uint8)
    blk[0:128] = ql.astype(np.uint8).ravel()
    blk[128:192] = qh.astype(np.uint8).ravel()
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = np.frombuffer(f16_bits(d).tobytes(), np.uint8)
    return blk


def random_q4_k(rng, n_blocks):
    """Blocks, their f32 dequantization by the closed form, and the exact
    (fp64) weight values."""
    out, ref, exact = [], [], []
    for _ in range(n_blocks):
        d = F16(rng.uniform(1e-3, 3e-2))
        dmin = F16(rng.uniform(1e-3, 3e-2))
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        out.append(pack_q4_k(d, dmin, sc, m, q))
        d1 = np.float32(d) * sc.astype(np.float32)
        m1 = np.float32(dmin) * m.astype(np.float32)
        ref.append(np.repeat(d1, 32) * q.astype(np.float32) - np.repeat(m1, 32))
        exact.append(float(d) * np.repeat(sc, 32) * q - float(dmin) * np.repeat(m, 32))
    return np.concatenate(out), np.concatenate(ref).astype(np.float32), np.concatenate(exact)


def random_q6_k(rng, n_blocks):
    out, ref, exact = [], [], []
    for _ in range(n_blocks):
        d = F16(rng.uniform(1e-4, 2e-3))
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, 256)
        out.append(pack_q6_k(d, sc, q))
        ds = np.float32(d) * sc.astype(np.float32)
        ref.append(np.repeat(ds, 16) * (q - 32).astype(np.float32))
        exact.append(float(d) * np.repeat(sc, 16) * (q - 32))
    return np.concatenate(out), np.concatenate(ref).astype(np.float32), np.concatenate(exact)


def test_q4_k_unpack_matches_the_layout():
    rng = np.random.default_rng(1)
    blocks, want, _ = random_q4_k(rng, 24)
    got = oracle.dequantize(oracle.Q4_K, blocks, want.size)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4_k_scale_bits_are_independent():
    # one non-zero 6-bit field at a time: every other sub-block dequantizes to 0
    for j in range(8):
        for which in ("sc", "m"):
            for v in (1, 16, 32, 63):
                sc, m = np.zeros(8, np.int64), np.zeros(8, np.int64)
                (sc if which == "sc" else m)[j] = v
                blk = pack_q4_k(1.0, 1.0, sc, m, np.full(256, 1))
                y = oracle.dequantize(oracle.Q4_K, blk, 256).reshape(8, 32)
                want = np.zeros((8, 32), np.float32)
                want[j] = v if which == "sc" else -v
                np.testing.assert_array_equal(y, want)


def test_q6_k_unpack_matches_the_layout():
    rng = np.random.default_rng(2)
    blocks, want, _ = random_q6_k(rng, 24)
    got = oracle.dequantize(oracle.Q6_K, blocks, want.size)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6_k_element_positions():
    # a single code of 33 (value +1) at element e, scale index e // 16 set to 1
    for e in (0, 15, 16, 31, 32, 63, 64, 95, 96, 127, 128, 200, 255):
        q = np.full(256, 32)
        q[e] = 33
        sc = np.zeros(16, np.int64)
        sc[e // 16] = 1
        y = oracle.dequantize(oracle.Q6_K, pack_q6_k(1.0, sc, q), 256)
        want = np.zeros(256, np.float32)
        want[e] = 1.0
        np.testing.assert_array_equal(y, want)


def q8k_fields(blocks, n):
    b = blocks.reshape(n // 256, 292)
    d = b[:, 0:4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].copy().view(np.int8)
    bs = b[:, 260:292].copy().view(np.int16)
    return d, qs, bs


def test_q8_k_closed_forms():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256 * 40) * rng.uniform(0.01, 50, 40).repeat(256)).astype(np.float32)
    blocks = oracle.q8_k_quantize(x)
    d, qs, bs = q8k_fields(blocks, x.size)
    xb = x.reshape(-1, 256)
    for i in range(xb.shape[0]):
        j = int(np.argmax(np.abs(xb[i])))              # first occurrence of the largest |x|
        assert qs[i, j] == -127
        assert np.all(np.abs(qs[i].astype(int)) <= 127)
        iscale = np.float32(-127.0) / xb[i, j]
        assert d[i] == np.float32(1.0) / iscale
        err = np.abs(d[i].astype(np.float64) * qs[i] - xb[i])
        assert np.all(err <= abs(float(d[i])) * (0.5 + 1e-5))
        np.testing.assert_array_equal(bs[i], qs[i].astype(int).reshape(16, 16).sum(1))


def test_q8_k_ties_rounding_and_zero():
    x = np.zeros(256 * 4, np.float32)
    # block 0: +3 at 5 then -3 at 9 -> the first one maps to -127
    x[5], x[9] = 3.0, -3.0
    # block 1: the mirror
    x[256 + 5], x[256 + 9] = -3.0, 3.0
    # block 2: max = -127 makes iscale = 1: half-way values round to even
    x[512 + 0] = -127.0
    x[512 + 1:512 + 7] = [2.5, 3.5, -2.5, -3.5, 0.5, 126.5]
    # block 3: all zero
    blocks = oracle.q8_k_quantize(x)
    d, qs, bs = q8k_fields(blocks, x.size)
    assert (qs[0, 5], qs[0, 9]) == (-127, 127)
    assert (qs[1, 5], qs[1, 9]) == (-127, 127)
    assert d[2] == 1.0
    assert list(qs[2, :7]) == [-127, 2, 4, -2, -4, 0, 126]
    assert d[3] == 0.0 and not qs[3].any() and not bs[3].any()


@pytest.mark.parametrize("dtype", [oracle.Q4_K, oracle.Q6_K])
@pytest.mark.parametrize("n", [256, 3072, 9216])
def test_vec_dot_against_fp64(dtype, n):
    rng = np.random.default_rng(n + dtype)
    maker = random_q4_k if dtype == oracle.Q4_K else random_q6_k
    w, _, wv = maker(rng, n // 256)
    x = rng.standard_normal(n).astype(np.float32)
    xq = oracle.q8_k_quantize(x)
    got = oracle.vec_dot(dtype, w, xq, n)
    # exact operands: both sides dequantized in fp64
    xv = oracle.dequantize(oracle.Q8_K, xq, n).astype(np.float64)
    terms = wv * xv
    assert abs(got - terms.sum()) <= 4e-6 * np.abs(terms).sum()


def pack_q8_0(d, q):
    """One block_q8_0 from d (f16-representable) and codes q[32] (int8)."""
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(f16_bits(d).tobytes(), np.uint8)
    blk[2:] = np.asarray(q, np.int8).view(np.uint8)
    return blk


def q8_0_fields(blocks):
    b = blocks.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).ravel().astype(np.float32)
    return d, b[:, 2:].copy().view(np.int8)


def random_q8_0(rng, n_blocks):
    """Q8_0 weight blocks (codes in [-127, 127], the quantizer's range) and the
    exact (fp64) weight values."""
    d = rng.uniform(1e-3, 3e-2, n_blocks).astype(np.float16)
    q = rng.integers(-127, 128, (n_blocks, 32))
    blocks = np.concatenate([pack_q8_0(d[i], q[i]) for i in range(n_blocks)])
    return blocks, (d.astype(np.float64)[:, None] * q).ravel()


def test_q8_0_weights_dequantize_to_d_times_q():
    rng = np.random.default_rng(95)
    blocks, exact = random_q8_0(rng, 40)
    got = oracle.dequantize(oracle.Q8_0, blocks, exact.size)
    np.testing.assert_array_equal(got, exact.astype(np.float32))   # d * q is exact in f32


def test_q8_0_activation_closed_forms():
    rng = np.random.default_rng(96)
    x = (rng.standard_normal(32 * 64) * rng.uniform(0.01, 50, 64).repeat(32)).astype(np.float32)
    d, qs = q8_0_fields(oracle.q8_0_quantize_x86(x))
    xb = x.reshape(-1, 32)
    for i in range(xb.shape[0]):
        j = int(np.argmax(np.abs(xb[i])))
        amax = np.abs(xb[i, j])
        assert qs[i, j] == (127 if xb[i, j] > 0 else -127)
        assert np.all(np.abs(qs[i].astype(int)) <= 127)
        # d: amax / 127 in f32, stored as f16 (numpy's conversion rounds to nearest even)
        assert d[i] == np.float32(np.float16(amax / np.float32(127)))
        # the codes come from 127 / amax, not from the stored d: |q d' - x| <= d' / 2
        # with d' = amax / 127, and the f16 rounding of d adds at most 127 d 2^-11
        err = np.abs(float(d[i]) * qs[i] - xb[i].astype(np.float64))
        assert np.all(err <= float(amax) / 127 * (0.5 + 1e-5) + 127 * abs(float(d[i])) * 2.0 ** -11)


def test_q8_0_activation_ties_scale_source_and_zero():
    x = np.zeros(32 * 4, np.float32)
    # block 0: amax = 127 gives id = 1 and d = 1: half-way values round to even
    # (the portable _ref quantizer would give 3, 4, -3, -4, 1, -1, 2, 127)
    x[0:9] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]
    # block 1: the largest magnitude negative
    x[32], x[33] = -127.0, 64.0
    # block 2: amax = 100: 50 * f32(127 / 100) = 63.5 exactly, a tie, -> 64;
    # a quantizer taking id from the stored f16 d (0.787598) would give 63
    x[64], x[65] = 100.0, 50.0
    # block 3: all zero
    d, qs = q8_0_fields(oracle.q8_0_quantize_x86(x))
    assert d[0] == 1.0
    assert list(qs[0, :9]) == [127, 2, 4, -2, -4, 0, 0, 2, 126]
    assert (qs[1, 0], qs[1, 1]) == (-127, 64)
    assert d[2] == np.float32(np.float16(np.float32(100) / np.float32(127)))
    assert (qs[2, 0], qs[2, 1]) == (127, 64)
    assert d[3] == 0.0 and not qs[3].any()


@pytest.mark.parametrize("n", [32, 256, 3072, 9216])
def test_vec_dot_q8_0_against_fp64(n):
    rng = np.random.default_rng(n + 8)
    w, wv = random_q8_0(rng, n // 32)
    x = rng.standard_normal(n).astype(np.float32)
    xq = oracle.q8_0_quantize_x86(x)
    got = oracle.vec_dot(oracle.Q8_0, w, xq, n)
    xv = oracle.dequantize(oracle.Q8_0, xq, n).astype(np.float64)
    terms = wv * xv
    assert abs(got - terms.sum()) <= 4e-6 * np.abs(terms).sum()


def test_vec_dot_q8_0_every_element_counts():
    # unit weights (d = 1, codes 1) against integer activations with amax 127
    # (d = 1, codes = values): the dot is the plain sum of the values
    n = 96
    w = np.concatenate([pack_q8_0(1.0, np.ones(32, int)) for _ in range(n // 32)])
    x = np.arange(-47, 49, dtype=np.float32)
    x[[0, 40, 80]] = [-127.0, 127.0, -127.0]
    for e in (0, 1, 3, 4, 31, 32, 35, 63, 64, 95):
        xe = x.copy()
        xe[e] += 0.0 if abs(xe[e]) == 127 else 1.0
        got = oracle.vec_dot(oracle.Q8_0, w, oracle.q8_0_quantize_x86(xe), n)
        assert got == float(xe.sum())


def test_matvec_q8_0_rows_and_threads():
    rng = np.random.default_rng(10)
    n_rows, n = 48, 3072
    w, _ = random_q8_0(rng, n_rows * n // 32)
    x = rng.standard_normal(n).astype(np.float32)
    y1 = oracle.matvec(oracle.Q8_0, w, n_rows, n, x, 1)
    np.testing.assert_array_equal(y1, oracle.matvec(oracle.Q8_0, w, n_rows, n, x, 4))
    xq = oracle.q8_0_quantize_x86(x)
    rb = oracle.wrow_bytes(oracle.Q8_0, n)
    assert rb == n // 32 * 34
    for r in (0, 17, 47):
        assert y1[r] == oracle.vec_dot(oracle.Q8_0, w[r * rb:(r + 1) * rb], xq, n)


def test_rms_norm_and_ada():
    rng = np.random.default_rng(7)
    for n in (256, 3072, 9216):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        a = rng.uniform(-0.3, 0.3, n).astype(np.float32)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5)
        y = oracle.norm_act(x, eps=1e-5)
        np.testing.assert_array_equal(y, x)                        # no norm weight: identity
        y = oracle.norm_act(x, w, eps=1e-5)
        np.testing.assert_allclose(y, ref * w, rtol=3e-7 * 4, atol=0)
        y2 = oracle.norm_act(x, w, a, eps=1e-5)
        np.testing.assert_allclose(y2, ref * w * (1 + a.astype(np.float64)), rtol=6e-7 * 4,
                                   atol=1e-12)


def test_matvec_rows_and_threads():
    rng = np.random.default_rng(9)
    n_rows, n = 64, 3072
    w, _, _ = random_q4_k(rng, n_rows * n // 256)
    x = rng.standard_normal(n).astype(np.float32)
    y1 = oracle.matvec(oracle.Q4_K, w, n_rows, n, x, 1)
    y4 = oracle.matvec(oracle.Q4_K, w, n_rows, n, x, 4)
    np.testing.assert_array_equal(y1, y4)
    xq = oracle.q8_k_quantize(x)
    rb = oracle.wrow_bytes(oracle.Q4_K, n)
    for r in (0, 17, 63):
        assert y1[r] == oracle.vec_dot(oracle.Q4_K, w[r * rb:(r + 1) * rb], xq, n)


def test_silu_closed_form():
    v = np.array([-20.0, -1.0, 0.0, 0.5, 3.0, 30.0], np.float32)
    want = v.astype(np.float64) / (1 + np.exp(-v.astype(np.float64)))
    np.testing.assert_allclose(oracle.silu(v), want, rtol=1e-6, atol=1e-12)


def test_argmax_last_index_of_the_maximum():
    x = np.array([1.0, 3.0, -2.0, 3.0, 0.5], np.float32)
    assert oracle.argmax(x) == 3                    # ties: the later index
    assert oracle.argmax(np.full(7, -np.inf, np.float32)) == 6
    assert oracle.argmax(np.array([2.0], np.float32)) == 0
    rng = np.random.default_rng(11)
    for _ in range(20):
        v = rng.integers(-50, 50, 4096).astype(np.float32)   # many ties
        want = v.size - 1 - int(np.argmax(v[::-1]))
        assert oracle.argmax(v) == want


def test_norm_bias_closed_form():
    rng = np.random.default_rng(1855)
    x = rng.standard_normal(1280).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1280).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, 1280).astype(np.float32)
    y = oracle.norm_act(x, w, eps=1e-5, norm_b=b)
    np.testing.assert_array_equal(y, oracle.norm_act(x, w, eps=1e-5) + b)   # f32 add after the weight
