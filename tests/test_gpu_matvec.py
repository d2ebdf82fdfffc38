"""GPU parity of the decoder projections on ggml k-quant weights
(ggml_mul_mat at src/voxtral.cpp:2656-2659 Q/K/V, :2857 O + residual,
:2878-2882 SwiGLU FFN, :2955/:2968 logits; RMSNorm :2653-2654, :2861-2862;
ada conditioning :2864-2874; get_rows :3008) against the oracle's restatement
of ggml's CPU path.

The Q8_K input image and the dequantized rows are bit-exact.  The products
are integer dot products per block on both sides; only the f32 combination of
the per-block partial sums is ordered differently (ggml: eight running lanes,
here a lane-per-quarter-block wave reduction), so each output is held to
1e-5 x sum_e |w_e| |x_e| (the magnitude the f32 rounding scales with)."""
import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import dev, stream_ptr
from kq_util import random_matrix

pytestmark = pytest.mark.gpu

EPS = 1e-5
REL = 1e-5


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def inputs(rng, n):
    x = (rng.standard_normal(n) * 2.0).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    a = rng.uniform(-0.4, 0.4, n).astype(np.float32)
    return x, w, a


def magnitude(dtype, w, n_rows, n_in, h):
    """sum_e |w_re| |x_e| per row, x the dequantized Q8_K image of h (q8_0 for
    Q8_0 weights)"""
    if dtype == vkv.Q8_0:
        ax = np.abs(oracle.dequantize(oracle.Q8_0, oracle.q8_0_quantize_x86(h), n_in))
    else:
        ax = np.abs(oracle.dequantize(oracle.Q8_K, oracle.q8_k_quantize(h), n_in))
    ax = ax.astype(np.float32)
    out = np.empty(n_rows, np.float64)
    rb = oracle.wrow_bytes(dtype, n_in)
    step = 4096
    for r0 in range(0, n_rows, step):
        r1 = min(n_rows, r0 + step)
        wd = oracle.dequantize(dtype, w[r0 * rb:r1 * rb], (r1 - r0) * n_in).reshape(r1 - r0, n_in)
        out[r0:r1] = np.abs(wd) @ ax
    return out


def check_rows(got, want, mag, extra=0.0):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = REL * mag + extra + 1e-30
    bad = np.flatnonzero(err > tol)
    assert bad.size == 0, (f"{bad.size} rows off; worst row {bad[np.argmax(err[bad] / tol[bad])]}: "
                           f"err {err[bad].max():.3e} tol {tol[bad].min():.3e}")


@pytest.mark.parametrize("n", [256, 3072, 9216, 12288])
@pytest.mark.parametrize("mode", ["plain", "norm", "norm_ada"])
def test_q8_k_input_image_is_bit_exact(n, mode):
    rng = np.random.default_rng(n + len(mode))
    x, w, a = inputs(rng, n)
    nw = w if mode != "plain" else None
    ad = a if mode == "norm_ada" else None
    xd, wd, adv = to_dev(x), to_dev(w), to_dev(a)
    out = torch.zeros(n // 256 * 292, dtype=torch.uint8, device=dev())
    vkv.quantize_q8_k(xd.data_ptr(), n, out.data_ptr(),
                      wd.data_ptr() if nw is not None else None,
                      adv.data_ptr() if ad is not None else None, EPS, hip_stream=stream_ptr())
    want = oracle.q8_k_quantize(oracle.norm_act(x, nw, ad, EPS))
    np.testing.assert_array_equal(host(out), want)


def test_q8_k_input_image_edge_blocks():
    n = 1024
    x = np.zeros(n, np.float32)
    x[5], x[9] = 3.0, -3.0                       # tie: the first one maps to -127
    x[256 + 5], x[256 + 9] = -3.0, 3.0
    x[512] = -127.0
    x[513:519] = [2.5, 3.5, -2.5, -3.5, 0.5, 126.5]   # half-way codes round to even
    # block 3 stays zero
    xd = to_dev(x)
    out = torch.zeros(n // 256 * 292, dtype=torch.uint8, device=dev())
    vkv.quantize_q8_k(xd.data_ptr(), n, out.data_ptr(), hip_stream=stream_ptr())
    np.testing.assert_array_equal(host(out), oracle.q8_k_quantize(x))


@pytest.mark.parametrize("dtype", [vkv.Q4_K, vkv.Q6_K, vkv.Q8_0])
def test_dequantize_is_bit_exact(dtype):
    rng = np.random.default_rng(dtype)
    rows, n_in = 37, 3072
    w = random_matrix(rng, dtype, rows, n_in)
    y = torch.empty(rows * n_in, dtype=torch.float32, device=dev())
    wd = to_dev(w)
    vkv.dequantize(dtype, wd.data_ptr(), rows * n_in, y.data_ptr(), hip_stream=stream_ptr())
    want = oracle.dequantize(dtype, w, rows * n_in)
    np.testing.assert_array_equal(host(y).view(np.uint32), want.view(np.uint32))


SHAPES = [
    (vkv.Q4_K, 4096, 3072),     # attn_q
    (vkv.Q4_K, 1024, 3072),     # attn_k
    (vkv.Q6_K, 1024, 3072),     # attn_v
    (vkv.Q4_K, 3072, 4096),     # attn_o
    (vkv.Q6_K, 3072, 9216),     # ffn_w2
    (vkv.Q4_K, 3072, 9216),
    (vkv.Q6_K, 777, 12288),     # largest input, rows not a multiple of the grid
    (vkv.Q4_K, 13, 256),        # one block per row
    (vkv.Q6_K, 1, 512),
    # a Q8_0 file (src/voxtral-quantize.cpp:95-96): every matrix Q8_0
    (vkv.Q8_0, 4096, 3072),     # attn_q
    (vkv.Q8_0, 1024, 3072),
    (vkv.Q8_0, 3072, 4096),     # attn_o
    (vkv.Q8_0, 3072, 5120),     # two steps per row (the adapter's input width)
    (vkv.Q8_0, 3072, 9216),     # ffn_w2
    (vkv.Q8_0, 777, 12288),
    (vkv.Q8_0, 13, 256),
    (vkv.Q8_0, 1, 512),
]


@pytest.mark.parametrize("dtype,n_rows,n_in", SHAPES)
def test_matvec_matches_oracle(dtype, n_rows, n_in):
    rng = np.random.default_rng(n_rows * 7 + n_in + dtype)
    w = random_matrix(rng, dtype, n_rows, n_in)
    x, _, _ = inputs(rng, n_in)
    xd, wd = to_dev(x), to_dev(w)
    y = torch.full((n_rows,), np.nan, dtype=torch.float32, device=dev())
    vkv.matvec(xd.data_ptr(), n_in, [(wd.data_ptr(), dtype, n_rows, y.data_ptr())],
               hip_stream=stream_ptr())
    want = oracle.matvec(dtype, w, n_rows, n_in, x, n_threads=8)
    check_rows(host(y), want, magnitude(dtype, w, n_rows, n_in, x))


def test_logits_matvec_full_vocab():
    """output / tied tok_embeddings: Q6_K [131072][3072] after the final norm"""
    rng = np.random.default_rng(131072)
    n_rows, n_in = 131072, 3072
    w = random_matrix(rng, vkv.Q6_K, n_rows, n_in)
    x, nw, _ = inputs(rng, n_in)
    xd, wd, nwd = to_dev(x), to_dev(w), to_dev(nw)
    y = torch.full((n_rows,), np.nan, dtype=torch.float32, device=dev())
    vkv.matvec(xd.data_ptr(), n_in, [(wd.data_ptr(), vkv.Q6_K, n_rows, y.data_ptr())],
               norm_w_ptr=nwd.data_ptr(), eps=EPS, hip_stream=stream_ptr())
    h = oracle.norm_act(x, nw, None, EPS)
    want = oracle.matvec(vkv.Q6_K, w, n_rows, n_in, h, n_threads=8)
    check_rows(host(y), want, magnitude(vkv.Q6_K, w, n_rows, n_in, h))


def test_qkv_in_one_call_with_norm():
    rng = np.random.default_rng(6144)
    n_in = 3072
    mats = [(vkv.Q4_K, 4096), (vkv.Q4_K, 1024), (vkv.Q6_K, 1024)]
    ws = [random_matrix(rng, dt, n, n_in) for dt, n in mats]
    x, nw, _ = inputs(rng, n_in)
    xd, nwd = to_dev(x), to_dev(nw)
    wds = [to_dev(w) for w in ws]
    ys = [torch.full((n,), np.nan, dtype=torch.float32, device=dev()) for _, n in mats]
    vkv.matvec(xd.data_ptr(), n_in,
               [(wd.data_ptr(), dt, n, y.data_ptr()) for wd, (dt, n), y in zip(wds, mats, ys)],
               norm_w_ptr=nwd.data_ptr(), eps=EPS, hip_stream=stream_ptr())
    h = oracle.norm_act(x, nw, None, EPS)
    for w, (dt, n), y in zip(ws, mats, ys):
        want = oracle.matvec(dt, w, n, n_in, h, n_threads=8)
        check_rows(host(y), want, magnitude(dt, w, n, n_in, h))


def test_residual_add_in_place():
    """x = residual + W_o attn (src/voxtral.cpp:2857-2858), y aliasing add"""
    rng = np.random.default_rng(2857)
    n_rows, n_in = 3072, 4096
    w = random_matrix(rng, vkv.Q4_K, n_rows, n_in)
    attn, _, _ = inputs(rng, n_in)
    res = rng.standard_normal(n_rows).astype(np.float32)
    ad, wd, r = to_dev(attn), to_dev(w), to_dev(res)
    vkv.matvec(ad.data_ptr(), n_in, [(wd.data_ptr(), vkv.Q4_K, n_rows, r.data_ptr(), r.data_ptr())],
               hip_stream=stream_ptr())
    proj = oracle.matvec(vkv.Q4_K, w, n_rows, n_in, attn, n_threads=8)
    want = res + proj
    mag = magnitude(vkv.Q4_K, w, n_rows, n_in, attn)
    check_rows(host(r), want, mag, extra=6e-8 * (np.abs(res) + np.abs(proj)))


def test_swiglu_ffn_with_norm_and_ada():
    """silu(W1 h) * (W3 h), h = rms_norm(x) * ffn_norm * (1 + ada)"""
    rng = np.random.default_rng(2879)
    n_rows, n_in = 9216, 3072
    w1 = random_matrix(rng, vkv.Q4_K, n_rows, n_in)
    w3 = random_matrix(rng, vkv.Q4_K, n_rows, n_in)
    x, nw, a = inputs(rng, n_in)
    xd, nwd, add, w1d, w3d = to_dev(x), to_dev(nw), to_dev(a), to_dev(w1), to_dev(w3)
    y = torch.full((n_rows,), np.nan, dtype=torch.float32, device=dev())
    vkv.matvec(xd.data_ptr(), n_in,
               [(w1d.data_ptr(), vkv.Q4_K, n_rows, y.data_ptr()),
                (w3d.data_ptr(), vkv.Q4_K, n_rows, None)],
               norm_w_ptr=nwd.data_ptr(), ada_ptr=add.data_ptr(), eps=EPS,
               epilogue=vkv.MV_SWIGLU, hip_stream=stream_ptr())
    h = oracle.norm_act(x, nw, a, EPS)
    g = oracle.matvec(vkv.Q4_K, w1, n_rows, n_in, h, n_threads=8).astype(np.float64)
    u = oracle.matvec(vkv.Q4_K, w3, n_rows, n_in, h, n_threads=8).astype(np.float64)
    sg = g / (1 + np.exp(-g))
    want = sg * u
    m1 = magnitude(vkv.Q4_K, w1, n_rows, n_in, h)
    m3 = magnitude(vkv.Q4_K, w3, n_rows, n_in, h)
    # d silu / dg <= 1.1; silu and the product each add a few f32 roundings
    err_bound = REL * (1.1 * m1 * np.abs(u) + np.abs(sg) * m3) + 1e-6 * np.abs(want)
    got = host(y).astype(np.float64)
    assert np.all(np.abs(got - want) <= err_bound + 1e-30)


def test_zero_input_gives_zero():
    n_rows, n_in = 256, 3072
    rng = np.random.default_rng(0)
    for dt in (vkv.Q4_K, vkv.Q6_K):
        w = to_dev(random_matrix(rng, dt, n_rows, n_in))
        x = torch.zeros(n_in, dtype=torch.float32, device=dev())
        y = torch.full((n_rows,), np.nan, dtype=torch.float32, device=dev())
        vkv.matvec(x.data_ptr(), n_in, [(w.data_ptr(), dt, n_rows, y.data_ptr())],
                   hip_stream=stream_ptr())
        assert np.all(host(y) == 0.0)


@pytest.mark.parametrize("n", [256, 3072, 5120, 9216])
@pytest.mark.parametrize("mode", ["plain", "norm_ada"])
def test_q8_0_input_image_through_unit_rows(n, mode):
    """Q8_0 rows with one code 1 (d = 1) at element r: y[r] is the q8_0 image's
    value at r, exactly (one non-zero block term, integer times d_x), so the
    kernel's q8_0 image of h must equal ggml's x86 quantize_row_q8_0 bit for
    bit; half-way and extreme values are planted in the input."""
    rng = np.random.default_rng(n + 80 + len(mode))
    x, nw, a = inputs(rng, n)
    if mode == "plain":
        x[:9] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]   # d = 1: ties to even
        x[32:64] = 0.0                                                 # an all-zero block
        x[64], x[65] = 100.0, 50.0                                     # 50 * f32(1.27) = 63.5
    nwv, adv = (nw, a) if mode == "norm_ada" else (None, None)
    rows = np.zeros((n, n // 32, 34), np.uint8)
    rows[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    r = np.arange(n)
    rows[r, r // 32, 2 + r % 32] = 1
    w = rows.reshape(-1)
    xd, wd, nwd, ad = to_dev(x), to_dev(w), to_dev(nw), to_dev(a)
    y = torch.full((n,), np.nan, dtype=torch.float32, device=dev())
    vkv.matvec(xd.data_ptr(), n, [(wd.data_ptr(), vkv.Q8_0, n, y.data_ptr())],
               norm_w_ptr=nwd.data_ptr() if nwv is not None else None,
               ada_ptr=ad.data_ptr() if adv is not None else None, eps=EPS,
               hip_stream=stream_ptr())
    h = oracle.norm_act(x, nwv, adv, EPS)
    want = oracle.dequantize(oracle.Q8_0, oracle.q8_0_quantize_x86(h), n)
    np.testing.assert_array_equal(host(y).view(np.uint32), want.view(np.uint32))
    if mode == "plain":
        assert list(host(y)[:9]) == [127, 2, 4, -2, -4, 0, 0, 2, 126]


def test_q8_0_mixed_with_k_quants_in_one_call():
    """each work group quantizes the input for its own matrix's format"""
    rng = np.random.default_rng(8012)
    n_in = 3072
    mats = [(vkv.Q8_0, 4096), (vkv.Q4_K, 1024), (vkv.Q8_0, 1024), (vkv.Q6_K, 512)]
    ws = [random_matrix(rng, dt, n, n_in) for dt, n in mats]
    x, nw, _ = inputs(rng, n_in)
    xd, nwd = to_dev(x), to_dev(nw)
    wds = [to_dev(w) for w in ws]
    ys = [torch.full((n,), np.nan, dtype=torch.float32, device=dev()) for _, n in mats]
    vkv.matvec(xd.data_ptr(), n_in,
               [(wd.data_ptr(), dt, n, y.data_ptr()) for wd, (dt, n), y in zip(wds, mats, ys)],
               norm_w_ptr=nwd.data_ptr(), eps=EPS, hip_stream=stream_ptr())
    h = oracle.norm_act(x, nw, None, EPS)
    for w, (dt, n), y in zip(ws, mats, ys):
        want = oracle.matvec(dt, w, n, n_in, h, n_threads=8)
        check_rows(host(y), want, magnitude(dt, w, n, n_in, h))


def test_q8_0_swiglu_and_residual():
    rng = np.random.default_rng(8013)
    n_rows, n_in = 9216, 3072
    w1, w3 = (random_matrix(rng, vkv.Q8_0, n_rows, n_in) for _ in range(2))
    x, nw, a = inputs(rng, n_in)
    xd, nwd, add, w1d, w3d = to_dev(x), to_dev(nw), to_dev(a), to_dev(w1), to_dev(w3)
    y = torch.full((n_rows,), np.nan, dtype=torch.float32, device=dev())
    vkv.matvec(xd.data_ptr(), n_in,
               [(w1d.data_ptr(), vkv.Q8_0, n_rows, y.data_ptr()),
                (w3d.data_ptr(), vkv.Q8_0, n_rows, None)],
               norm_w_ptr=nwd.data_ptr(), ada_ptr=add.data_ptr(), eps=EPS,
               epilogue=vkv.MV_SWIGLU, hip_stream=stream_ptr())
    h = oracle.norm_act(x, nw, a, EPS)
    g = oracle.matvec(vkv.Q8_0, w1, n_rows, n_in, h, n_threads=8).astype(np.float64)
    u = oracle.matvec(vkv.Q8_0, w3, n_rows, n_in, h, n_threads=8).astype(np.float64)
    sg = g / (1 + np.exp(-g))
    want = sg * u
    m1 = magnitude(vkv.Q8_0, w1, n_rows, n_in, h)
    m3 = magnitude(vkv.Q8_0, w3, n_rows, n_in, h)
    err_bound = REL * (1.1 * m1 * np.abs(u) + np.abs(sg) * m3) + 1e-6 * np.abs(want)
    assert np.all(np.abs(host(y).astype(np.float64) - want) <= err_bound + 1e-30)
    # W2 + residual, in place (src/voxtral.cpp:2882-2883)
    w2 = random_matrix(rng, vkv.Q8_0, n_in, n_rows)
    res = rng.standard_normal(n_in).astype(np.float32)
    f = host(y)
    fd, w2d, r = to_dev(f), to_dev(w2), to_dev(res)
    vkv.matvec(fd.data_ptr(), n_rows, [(w2d.data_ptr(), vkv.Q8_0, n_in, r.data_ptr(), r.data_ptr())],
               hip_stream=stream_ptr())
    proj = oracle.matvec(vkv.Q8_0, w2, n_in, n_rows, f, n_threads=8)
    check_rows(host(r), res + proj, magnitude(vkv.Q8_0, w2, n_in, n_rows, f),
               extra=6e-8 * (np.abs(res) + np.abs(proj)))


def test_q8_0_embedding_row():
    rng = np.random.default_rng(3008)
    vocab, dim = 64, 3072
    table = random_matrix(rng, vkv.Q8_0, vocab, dim)
    audio = rng.standard_normal(dim).astype(np.float32)
    td, ad = to_dev(table), to_dev(audio)
    y = torch.full((dim,), np.nan, dtype=torch.float32, device=dev())
    rb = oracle.wrow_bytes(oracle.Q8_0, dim)
    for token in (0, 37, vocab - 1):
        vkv.embed(vkv.Q8_0, td.data_ptr(), vocab, dim, token, y.data_ptr(), add_ptr=ad.data_ptr(),
                  hip_stream=stream_ptr())
        want = oracle.dequantize(oracle.Q8_0, table[token * rb:(token + 1) * rb], dim) + audio
        np.testing.assert_array_equal(host(y), want)
