"""Element formats and synthetic inputs of the oracle, pinned independently:
F16 against numpy's IEEE binary16 (RNE) conversion, q8_0 against closed-form
properties of the block quantizer, the generator against the published
splitmix64 sequence and N(0,1) moments.  CPU only."""
import numpy as np
import pytest

import oracle


def _np_f16_bits(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


class TestF16:
    def test_all_codes_to_f32(self):
        codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
        got = oracle.f16_bits_to_f32(codes)
        want = codes.view(np.float16).astype(np.float32)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))

    def test_roundtrip_every_finite_code(self):
        codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
        vals = codes.view(np.float16).astype(np.float32)
        fin = np.isfinite(vals)
        assert np.array_equal(oracle.f32_to_f16_bits(vals[fin]), codes[fin])

    def test_random_bit_patterns_match_numpy(self):
        rng = np.random.default_rng(7)
        bits = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        x = x[~np.isnan(x)]
        assert np.array_equal(oracle.f32_to_f16_bits(x), _np_f16_bits(x))

    def test_ties_subnormals_and_overflow(self):
        # every representable f16 midpoint (ties -> even), +-1 ulp of f32 around it
        codes = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
        lo = codes[:-1].view(np.float16).astype(np.float64)
        hi = codes[1:].view(np.float16).astype(np.float64)
        mid = ((lo + hi) / 2).astype(np.float32)       # exact in f32
        near = np.concatenate([mid, np.nextafter(mid, np.float32(0)),
                               np.nextafter(mid, np.float32(np.inf))])
        near = np.concatenate([near, -near])
        assert np.array_equal(oracle.f32_to_f16_bits(near), _np_f16_bits(near))
        special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e30, -1e30,
                            np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25, 1.5 * 2 ** -25, 2.0 ** -26,
                            2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1e-40], dtype=np.float32)
        assert np.array_equal(oracle.f32_to_f16_bits(special), _np_f16_bits(special))

    def test_nan_stays_nan(self):
        x = np.array([np.nan, -np.nan], dtype=np.float32)
        h = oracle.f32_to_f16_bits(x)
        assert np.all(np.isnan(h.view(np.float16)))


class TestQ8:
    def test_block_layout_and_scale(self):
        rng = np.random.default_rng(3)
        x = rng.standard_normal(32 * 64).astype(np.float32)
        blk = oracle.q8_0_quantize(x).reshape(64, 34)
        xb = x.reshape(64, 32)
        amax = np.abs(xb).max(axis=1)
        # d is fp16(RNE) of amax/127 computed in f32
        d_want = (amax.astype(np.float32) / np.float32(127)).astype(np.float16).view(np.uint16)
        assert np.array_equal(blk[:, :2].copy().view(np.uint16).ravel(), d_want)
        qs = blk[:, 2:].view(np.int8)
        # the element of largest magnitude maps to +-127 exactly
        i = np.abs(xb).argmax(axis=1)
        assert np.array_equal(np.abs(qs[np.arange(64), i]), np.full(64, 127))
        assert np.all(np.abs(qs.astype(np.int32)) <= 127)
        assert np.all(np.sign(qs) == np.where(np.abs(xb * 127 / amax[:, None]) >= 0.5, np.sign(xb), 0))

    def test_error_bound(self):
        rng = np.random.default_rng(4)
        x = (rng.standard_normal(32 * 4096) * rng.uniform(1e-3, 1e3, 4096).repeat(32)).astype(np.float32)
        y = oracle.q8_0_dequantize(oracle.q8_0_quantize(x), x.size)
        d = (np.abs(x.reshape(-1, 32)).max(axis=1) / 127.0).repeat(32)
        # half a quantum plus the fp16 rounding of the stored scale (<= 2^-11 rel. x 127)
        assert np.all(np.abs(x - y) <= d * (0.5 + 127 * 2.0 ** -11) * (1 + 1e-6))

    def test_round_half_away_from_zero(self):
        # amax = 127 -> d = 1, id = 1: x*id lands exactly on .5 ties
        x = np.zeros(32, dtype=np.float32)
        x[0] = 127.0
        x[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -3.5]
        qs = oracle.q8_0_quantize(x)[2:].view(np.int8)
        assert list(qs[:9]) == [127, 3, -3, 1, -1, 2, -2, 127, -4]

    def test_zero_block(self):
        blk = oracle.q8_0_quantize(np.zeros(32, dtype=np.float32))
        assert np.all(blk == 0)
        assert np.all(oracle.q8_0_dequantize(blk, 32) == 0)

    def test_dequant_closed_form(self):
        blk = np.zeros(34, dtype=np.uint8)
        blk[:2] = np.array([0.25], dtype=np.float16).view(np.uint8)
        blk[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
        y = oracle.q8_0_dequantize(blk, 32)
        assert np.array_equal(y, np.arange(-16, 16, dtype=np.float32) * 0.25)


class TestGenerator:
    def test_splitmix64_published_sequence(self):
        # splitmix64 (Steele, Lea & Flood 2014; Vigna's reference C code), seed 1234567
        want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                4593380528125082431, 16408922859458223821]
        g = 0x9E3779B97F4A7C15
        got = [oracle.lib.orc_mix64((1234567 + k * g) % 2 ** 64) for k in range(5)]
        assert got == want

    def test_moments_and_grid(self):
        x = np.concatenate([oracle.synth_row(42, oracle.TAG_K, 0, l, p, 1024)
                            for l in range(4) for p in range(256)])
        assert abs(x.mean()) < 0.005
        assert abs(x.var() - 1.0) < 0.01
        assert np.all(np.abs(x) <= 6.0)
        assert np.all(x * 65536 == np.round(x * 65536))      # exact multiples of 2^-16
        # fourth moment of Irwin-Hall(12) standardised: 3 - 1.2/12 = 2.9
        assert abs((x ** 4).mean() - 2.9) < 0.05

    def test_keys_separate_streams(self):
        a = oracle.synth_row(1, oracle.TAG_K, 0, 0, 0, 4096)
        for args in [(2, oracle.TAG_K, 0, 0, 0), (1, oracle.TAG_V, 0, 0, 0),
                     (1, oracle.TAG_K, 1, 0, 0), (1, oracle.TAG_K, 0, 1, 0),
                     (1, oracle.TAG_K, 0, 0, 1)]:
            b = oracle.synth_row(*args, 4096)
            assert abs(np.corrcoef(a, b)[0, 1]) < 0.06
        assert np.array_equal(a, oracle.synth_row(1, oracle.TAG_K, 0, 0, 0, 4096))


@pytest.mark.parametrize("dtype", [oracle.F32, oracle.F16, oracle.Q8_0])
def test_cache_image_append_and_expected_state(dtype):
    """Appending synthetic rows one position at a time through planner write
    segments produces the closed-form expected state (newest position per
    slot, untouched slots zero), and gather returns the logical window."""
    kv_dim, cap, backing, seed = 64, 16, 20, 9
    rb = oracle.row_bytes(dtype, kv_dim)
    img = np.zeros(backing * rb, dtype=np.uint8)
    ring = oracle.new_ring(cap)
    pos = 0
    for n in [3, 1, 7, 5, 16, 2, 9]:
        plan = oracle.decoder_plan(ring, pos, n)
        src = oracle.synth_rows(seed, oracle.TAG_K, 0, 0, range(pos, pos + n), kv_dim)
        oracle.append(dtype, img, rb, kv_dim, oracle.segs_of(plan.write_seg, plan.write_nseg), src)
        oracle.decoder_commit(ring, plan)
        pos += n
        want = oracle.expected_layer(dtype, backing, cap, kv_dim, pos, seed, oracle.TAG_K, 0, 0)
        assert np.array_equal(img, want)
        win = oracle.gather(img, rb, oracle.segs_of(plan.read_seg, plan.read_nseg))
        rows = range(plan.oldest_after, plan.next_after)
        want_win = oracle.rows_from_f32(dtype, oracle.synth_rows(seed, oracle.TAG_K, 0, 0, rows, kv_dim))
        assert np.array_equal(win, want_win)
    assert np.all(img[cap * rb:] == 0)
