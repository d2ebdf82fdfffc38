"""GPU parity of the multi-row products (the encoder's P frames per chunk,
build_encoder_kv_graph src/voxtral.cpp:2147-2370: Q/K/V with biases :2150-2152,
O + bias + residual :2358-2359, SwiGLU :2362-2366 with the optional W2 bias;
enc_apply_norm with its bias :1855-1861; the decoder prefill's projections)
against the oracle's restatement of ggml's CPU path, one input row at a time.

The Q8_K image of every input row is bit-exact; every output within
1e-5 x sum_e |w_e| |x_e| of the oracle (f32 combination of exact integer
block sums in another order), plus the f32 rounding of bias / residual adds."""
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


def workspace(n_cols, n_in):
    b = vkv.matmul_workspace(n_cols, n_in)
    assert b > 0
    t = torch.empty(b // 4 + 64, dtype=torch.float32, device=dev())
    return t, (t.data_ptr() + 255) & ~255, b


def x_image(dtype, h, n_in):
    """the dequantized input image a product on dtype rows multiplies"""
    if dtype == vkv.Q8_0:
        return oracle.dequantize(oracle.Q8_0, oracle.q8_0_quantize_x86(h), n_in)
    return oracle.dequantize(oracle.Q8_K, oracle.q8_k_quantize(h), n_in)


def rows_ref(dtype, w, n_rows, n_in, hs):
    """oracle outputs [n_cols][n_rows] and magnitudes sum |w||x| (x = Q8_K image)"""
    out = np.stack([oracle.matvec(dtype, w, n_rows, n_in, h, n_threads=8) for h in hs])
    wd = np.abs(oracle.dequantize(dtype, w, n_rows * n_in).reshape(n_rows, n_in))
    ax = np.stack([np.abs(x_image(dtype, h, n_in)) for h in hs])
    return out, ax @ wd.T


def check(got, want, mag, extra=0.0):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = REL * mag + extra + 1e-30
    assert np.all(err <= tol), f"{int((err > tol).sum())} outputs off, worst {float((err / tol).max()):.2f}x tol"


@pytest.mark.parametrize("P", [1, 4, 16, 17, 38, 128])
def test_encoder_qkv_with_norm_bias_and_biases(P):
    rng = np.random.default_rng(2150 + P)
    n_in = 1280
    mats = [(vkv.Q4_K, 1280, True), (vkv.Q4_K, 1280, False), (vkv.Q6_K, 1280, True)]
    ws = [random_matrix(rng, dt, n, n_in, 0.05) for dt, n, _ in mats]
    bs = [rng.standard_normal(n).astype(np.float32) if hb else None for _, n, hb in mats]
    x = rng.standard_normal((P, n_in)).astype(np.float32) * 3
    nw = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    nb = rng.uniform(-0.3, 0.3, n_in).astype(np.float32)
    xd, nwd, nbd = to_dev(x), to_dev(nw), to_dev(nb)
    wds = [to_dev(w) for w in ws]
    bds = [to_dev(b) if b is not None else None for b in bs]
    ys = [torch.full((P, n), np.nan, device=dev()) for _, n, _ in mats]
    t, ws_ptr, ws_b = workspace(P, n_in)
    vkv.matmul(xd.data_ptr(), P, n_in,
               [(wd.data_ptr(), dt, n, y.data_ptr(), None, bd.data_ptr() if bd is not None else None)
                for wd, (dt, n, _), y, bd in zip(wds, mats, ys, bds)],
               ws_ptr, ws_b, norm_w_ptr=nwd.data_ptr(), norm_b_ptr=nbd.data_ptr(), eps=EPS,
               hip_stream=stream_ptr())
    hs = [oracle.norm_act(x[p], nw, eps=EPS, norm_b=nb) for p in range(P)]
    # the Q8_K image (codes at the workspace start, [P][n_in], each 256-block
    # in the products' lane order: byte 64 q + 16 kg + 8 h + e holds code
    # 32 (2q + h) + 8 kg + e) is the oracle's, bit for bit
    raw = host(t).view(np.uint8)[ws_ptr - t.data_ptr():][:P * n_in]
    codes = raw.reshape(P, n_in // 256, 4, 4, 2, 8).transpose(0, 1, 2, 4, 3, 5).reshape(P, n_in)
    for p in range(P):
        want = oracle.q8_k_quantize(hs[p]).reshape(-1, 292)[:, 4:260].ravel()
        assert np.array_equal(codes[p], want)
    for w, (dt, n, _), y, b in zip(ws, mats, ys, bs):
        want, mag = rows_ref(dt, w, n, n_in, hs)
        if b is not None:
            want = want + b[None, :]
        check(host(y), want, mag, extra=6e-8 * np.abs(want))


@pytest.mark.parametrize("dtype,n_rows,n_in,P", [(vkv.Q4_K, 1280, 1280, 16),   # encoder O
                                                  (vkv.Q6_K, 1280, 5120, 16),   # encoder W2
                                                  (vkv.Q6_K, 1280, 5120, 5),
                                                  (vkv.Q4_K, 3072, 4096, 38)])  # decoder prefill O
def test_bias_and_residual_in_place(dtype, n_rows, n_in, P):
    rng = np.random.default_rng(n_rows + n_in + P)
    w = random_matrix(rng, dtype, n_rows, n_in, 0.05)
    b = rng.standard_normal(n_rows).astype(np.float32)
    x = rng.standard_normal((P, n_in)).astype(np.float32)
    res = rng.standard_normal((P, n_rows)).astype(np.float32)
    xd, wd, bd, r = to_dev(x), to_dev(w), to_dev(b), to_dev(res)
    t, ws_ptr, ws_b = workspace(P, n_in)
    vkv.matmul(xd.data_ptr(), P, n_in, [(wd.data_ptr(), dtype, n_rows, r.data_ptr(), r.data_ptr(),
                                          bd.data_ptr())], ws_ptr, ws_b, hip_stream=stream_ptr())
    proj, mag = rows_ref(dtype, w, n_rows, n_in, list(x))
    want = res + (proj + b[None, :])
    check(host(r), want, mag, extra=1.2e-7 * (np.abs(res) + np.abs(proj) + np.abs(b)[None, :]))


@pytest.mark.parametrize("P", [3, 16])
def test_encoder_swiglu(P):
    rng = np.random.default_rng(2362 + P)
    n_in, hid = 1280, 5120
    w1 = random_matrix(rng, vkv.Q4_K, hid, n_in, 0.02)
    w3 = random_matrix(rng, vkv.Q4_K, hid, n_in, 0.02)
    x = rng.standard_normal((P, n_in)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    xd, nwd, w1d, w3d = to_dev(x), to_dev(nw), to_dev(w1), to_dev(w3)
    y = torch.full((P, hid), np.nan, device=dev())
    t, ws_ptr, ws_b = workspace(P, n_in)
    vkv.matmul(xd.data_ptr(), P, n_in, [(w1d.data_ptr(), vkv.Q4_K, hid, y.data_ptr()),
                                        (w3d.data_ptr(), vkv.Q4_K, hid, None)],
               ws_ptr, ws_b, norm_w_ptr=nwd.data_ptr(), eps=EPS, epilogue=vkv.MV_SWIGLU,
               hip_stream=stream_ptr())
    hs = [oracle.norm_act(x[p], nw, eps=EPS) for p in range(P)]
    g, m1 = rows_ref(vkv.Q4_K, w1, hid, n_in, hs)
    u, m3 = rows_ref(vkv.Q4_K, w3, hid, n_in, hs)
    g, u = g.astype(np.float64), u.astype(np.float64)
    sg = g / (1 + np.exp(-g))
    want = sg * u
    bound = REL * (1.1 * m1 * np.abs(u) + np.abs(sg) * m3) + 1e-6 * np.abs(want)
    assert np.all(np.abs(host(y) - want) <= bound + 1e-30)


def test_matches_the_single_row_kernel():
    """n_cols = 1 agrees with vkv_matvec within the same bound"""
    rng = np.random.default_rng(1)
    n_rows, n_in = 4096, 3072
    w = random_matrix(rng, vkv.Q4_K, n_rows, n_in)
    x = rng.standard_normal(n_in).astype(np.float32)
    xd, wd = to_dev(x), to_dev(w)
    y1 = torch.empty(n_rows, device=dev())
    y2 = torch.empty(n_rows, device=dev())
    vkv.matvec(xd.data_ptr(), n_in, [(wd.data_ptr(), vkv.Q4_K, n_rows, y1.data_ptr())],
               hip_stream=stream_ptr())
    t, ws_ptr, ws_b = workspace(1, n_in)
    vkv.matmul(xd.data_ptr(), 1, n_in, [(wd.data_ptr(), vkv.Q4_K, n_rows, y2.data_ptr())],
               ws_ptr, ws_b, hip_stream=stream_ptr())
    _, mag = rows_ref(vkv.Q4_K, w, n_rows, n_in, [x])
    check(host(y2), host(y1), 2 * mag[0])


@pytest.mark.parametrize("norm", [False, True])
def test_fused_and_separate_input_images_agree(norm):
    """A call with few input rows quantizes them inside the products' work
    groups (at most two 16-lane tasks per group); a call with many rows takes
    the separate quantization launch.  The same rows must get the same Q8_K
    image bit for bit, and the same outputs, whatever the call's size: the
    encoder's outputs must not depend on how a stream is cut into chunks.
    Rows span a dynamic range of e^+-6 (the norm's double sums of f32
    squares), the Q/K/V shape of the encoder (three matrices over 1280)."""
    rng = np.random.default_rng(4242 + norm)
    n_in, P_big, P_small = 1280, 64, 4
    mats = [(vkv.Q4_K, 1280), (vkv.Q4_K, 1280), (vkv.Q6_K, 1280)]
    ws = [to_dev(random_matrix(rng, dt, n, n_in, 0.05)) for dt, n in mats]
    x = (rng.standard_normal((P_big, n_in)) *
         np.exp(rng.uniform(-6, 6, (P_big, 1)))).astype(np.float32)
    nw = to_dev(rng.uniform(0.5, 1.5, n_in).astype(np.float32)) if norm else None
    nb = to_dev(rng.uniform(-0.3, 0.3, n_in).astype(np.float32)) if norm else None
    xd = to_dev(x)
    runs = []
    for P in (P_small, P_big):
        ys = [torch.full((P, n), np.nan, device=dev()) for _, n in mats]
        t, ws_ptr, ws_b = workspace(P, n_in)
        vkv.matmul(xd.data_ptr(), P, n_in,
                   [(w.data_ptr(), dt, n, y.data_ptr()) for w, (dt, n), y in zip(ws, mats, ys)],
                   ws_ptr, ws_b, norm_w_ptr=nw.data_ptr() if norm else None,
                   norm_b_ptr=nb.data_ptr() if norm else None, eps=EPS, hip_stream=stream_ptr())
        raw = host(t).view(np.uint8)[ws_ptr - t.data_ptr():][:P * n_in].reshape(P, n_in)
        runs.append((raw.copy(), [host(y) for y in ys]))
    (img_s, out_s), (img_b, out_b) = runs
    assert np.array_equal(img_s, img_b[:P_small])
    for a, b in zip(out_s, out_b):
        assert np.array_equal(a.view(np.uint32), b[:P_small].view(np.uint32))
    # and the image is the oracle's
    for p in range(P_small):
        h = oracle.norm_act(x[p], host(nw), eps=EPS, norm_b=host(nb)) if norm else x[p]
        want = oracle.q8_k_quantize(h).reshape(-1, 292)[:, 4:260].ravel()
        codes = img_s[p].reshape(n_in // 256, 4, 4, 2, 8).transpose(0, 1, 3, 2, 4).reshape(n_in)
        assert np.array_equal(codes, want)


@pytest.mark.parametrize("n_in,ada", [(3072, False), (3072, True), (2048, True)])
def test_normed_input_wider_than_the_fused_norm(n_in, ada):
    """A normed call at the decoder's width (the Q/K/V and W1/W3 products of a
    prompt of a few tokens, RMSNorm x weight x (1 + ada)): each work group of
    a fused-input call stages the norm's vectors in LDS, 4 elements per
    thread, so a width above 4 x 64 x waves must take the separate
    quantization.  A run of 4 rows and a run of 64 rows give the same Q8_K
    image and the same outputs bit for bit, and both are the oracle's.  (2048
    fits the 8-wave fused norm exactly: the fused path is exercised at its
    limit.)"""
    rng = np.random.default_rng(3072 + n_in + ada)
    P_big, P_small = 64, 4
    mats = [(vkv.Q4_K, 4096), (vkv.Q4_K, 1024), (vkv.Q6_K, 1024)]
    ws_np = [random_matrix(rng, dt, n, n_in, 0.05) for dt, n in mats]
    ws = [to_dev(w) for w in ws_np]
    x = (rng.standard_normal((P_big, n_in)) *
         np.exp(rng.uniform(-3, 3, (P_big, 1)))).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    ad = rng.uniform(-0.5, 0.5, n_in).astype(np.float32) if ada else None
    xd, nwd = to_dev(x), to_dev(nw)
    add = to_dev(ad) if ada else None
    runs = []
    for P in (P_small, P_big):
        ys = [torch.full((P, n), np.nan, device=dev()) for _, n in mats]
        t, ws_ptr, ws_b = workspace(P, n_in)
        vkv.matmul(xd.data_ptr(), P, n_in,
                   [(w.data_ptr(), dt, n, y.data_ptr()) for w, (dt, n), y in zip(ws, mats, ys)],
                   ws_ptr, ws_b, norm_w_ptr=nwd.data_ptr(),
                   ada_ptr=add.data_ptr() if ada else None, eps=EPS, hip_stream=stream_ptr())
        raw = host(t).view(np.uint8)[ws_ptr - t.data_ptr():][:P * n_in].reshape(P, n_in)
        runs.append((raw.copy(), [host(y) for y in ys]))
    (img_s, out_s), (img_b, out_b) = runs
    assert np.array_equal(img_s, img_b[:P_small])
    for a, b in zip(out_s, out_b):
        assert np.array_equal(a.view(np.uint32), b[:P_small].view(np.uint32))
    hs = [oracle.norm_act(x[p], nw, ad, EPS) for p in range(P_small)]
    for p in range(P_small):
        want = oracle.q8_k_quantize(hs[p]).reshape(-1, 292)[:, 4:260].ravel()
        codes = img_s[p].reshape(n_in // 256, 4, 4, 2, 8).transpose(0, 1, 3, 2, 4).reshape(n_in)
        assert np.array_equal(codes, want)
    for w, (dt, n), y in zip(ws_np, mats, out_s):
        want, mag = rows_ref(dt, w, n, n_in, hs)
        check(y, want, mag)


def image_parts(t, ws_ptr, P, n_in):
    """codes [P][n_in] in natural order and the 16-bit words [P][n_in / 32]
    (Q8_K sums, or the fp16 d of a q8_0 image) from a call's workspace"""
    raw = host(t).view(np.uint8)[ws_ptr - t.data_ptr():]
    codes = raw[:P * n_in].reshape(P, n_in // 256, 4, 4, 2, 8).transpose(0, 1, 2, 4, 3, 5)
    off = -(-P * n_in // 256) * 256
    off += -(-P * (n_in // 256) * 4 // 256) * 256
    words = raw[off:off + P * (n_in // 32) * 2].copy().view(np.uint16).reshape(P, n_in // 32)
    return codes.reshape(P, n_in).copy(), words


@pytest.mark.parametrize("P", [1, 4, 16, 38, 64])
def test_q8_0_products_with_norm_bias_and_biases(P):
    """A Q8_0 file's encoder Q/K/V (all three Q8_0, src/voxtral-quantize.cpp:
    95-96): the q8_0 image of every row (codes in the products' lane order,
    the fp16 d of every 32-element block in the sums' place) is ggml's x86
    quantize_row_q8_0 of the normed row bit for bit, through the fused (P <= 4)
    and the separate quantization alike; the outputs are within the bound."""
    rng = np.random.default_rng(8000 + P)
    n_in = 1280
    mats = [(vkv.Q8_0, 1280, True), (vkv.Q8_0, 1280, False), (vkv.Q8_0, 1280, True)]
    ws = [random_matrix(rng, dt, n, n_in, 0.05) for dt, n, _ in mats]
    bs = [rng.standard_normal(n).astype(np.float32) if hb else None for _, n, hb in mats]
    x = (rng.standard_normal((P, n_in)) * np.exp(rng.uniform(-4, 4, (P, 1)))).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    nb = rng.uniform(-0.3, 0.3, n_in).astype(np.float32)
    xd, nwd, nbd = to_dev(x), to_dev(nw), to_dev(nb)
    wds = [to_dev(w) for w in ws]
    bds = [to_dev(b) if b is not None else None for b in bs]
    ys = [torch.full((P, n), np.nan, device=dev()) for _, n, _ in mats]
    t, ws_ptr, ws_b = workspace(P, n_in)
    vkv.matmul(xd.data_ptr(), P, n_in,
               [(wd.data_ptr(), dt, n, y.data_ptr(), None, bd.data_ptr() if bd is not None else None)
                for wd, (dt, n, _), y, bd in zip(wds, mats, ys, bds)],
               ws_ptr, ws_b, norm_w_ptr=nwd.data_ptr(), norm_b_ptr=nbd.data_ptr(), eps=EPS,
               hip_stream=stream_ptr())
    hs = [oracle.norm_act(x[p], nw, eps=EPS, norm_b=nb) for p in range(P)]
    codes, words = image_parts(t, ws_ptr, P, n_in)
    for p in range(P):
        blk = oracle.q8_0_quantize_x86(hs[p]).reshape(-1, 34)
        assert np.array_equal(codes[p], blk[:, 2:].view(np.int8).ravel().view(np.uint8))
        assert np.array_equal(words[p], blk[:, 0:2].copy().view(np.uint16).ravel())
    for w, (dt, n, _), y, b in zip(ws, mats, ys, bs):
        want, mag = rows_ref(dt, w, n, n_in, hs)
        if b is not None:
            want = want + b[None, :]
        check(host(y), want, mag, extra=6e-8 * np.abs(want))


@pytest.mark.parametrize("P", [3, 16])
def test_q8_0_swiglu_and_w2_residual(P):
    """the encoder FFN of a Q8_0 file: SwiGLU over 5120 rows, then W2 + bias +
    residual in place over a 5120-wide input (two passes of 256-blocks per wave)"""
    rng = np.random.default_rng(8362 + P)
    n_in, hid = 1280, 5120
    w1 = random_matrix(rng, vkv.Q8_0, hid, n_in, 0.02)
    w3 = random_matrix(rng, vkv.Q8_0, hid, n_in, 0.02)
    x = rng.standard_normal((P, n_in)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    xd, nwd, w1d, w3d = to_dev(x), to_dev(nw), to_dev(w1), to_dev(w3)
    y = torch.full((P, hid), np.nan, device=dev())
    t, ws_ptr, ws_b = workspace(P, n_in)
    vkv.matmul(xd.data_ptr(), P, n_in, [(w1d.data_ptr(), vkv.Q8_0, hid, y.data_ptr()),
                                        (w3d.data_ptr(), vkv.Q8_0, hid, None)],
               ws_ptr, ws_b, norm_w_ptr=nwd.data_ptr(), eps=EPS, epilogue=vkv.MV_SWIGLU,
               hip_stream=stream_ptr())
    hs = [oracle.norm_act(x[p], nw, eps=EPS) for p in range(P)]
    g, m1 = rows_ref(vkv.Q8_0, w1, hid, n_in, hs)
    u, m3 = rows_ref(vkv.Q8_0, w3, hid, n_in, hs)
    g, u = g.astype(np.float64), u.astype(np.float64)
    sg = g / (1 + np.exp(-g))
    want = sg * u
    bound = REL * (1.1 * m1 * np.abs(u) + np.abs(sg) * m3) + 1e-6 * np.abs(want)
    f = host(y)
    assert np.all(np.abs(f - want) <= bound + 1e-30)
    w2 = random_matrix(rng, vkv.Q8_0, n_in, hid, 0.05)
    b2 = rng.standard_normal(n_in).astype(np.float32)
    res = rng.standard_normal((P, n_in)).astype(np.float32)
    fd, w2d, b2d, r = to_dev(f), to_dev(w2), to_dev(b2), to_dev(res)
    t2, ws2, wsb2 = workspace(P, hid)
    vkv.matmul(fd.data_ptr(), P, hid, [(w2d.data_ptr(), vkv.Q8_0, n_in, r.data_ptr(), r.data_ptr(),
                                         b2d.data_ptr())], ws2, wsb2, hip_stream=stream_ptr())
    proj, mag = rows_ref(vkv.Q8_0, w2, n_in, hid, list(f))
    want2 = res + (proj + b2[None, :])
    check(host(r), want2, mag, extra=1.2e-7 * (np.abs(res) + np.abs(proj) + np.abs(b2)[None, :]))


def test_q8_0_matches_the_single_row_kernel_and_rejects_mixing():
    rng = np.random.default_rng(80)
    n_rows, n_in = 3072, 4096
    w = random_matrix(rng, vkv.Q8_0, n_rows, n_in)
    x = rng.standard_normal(n_in).astype(np.float32)
    xd, wd = to_dev(x), to_dev(w)
    y1 = torch.empty(n_rows, device=dev())
    y2 = torch.empty(n_rows, device=dev())
    vkv.matvec(xd.data_ptr(), n_in, [(wd.data_ptr(), vkv.Q8_0, n_rows, y1.data_ptr())],
               hip_stream=stream_ptr())
    t, ws_ptr, ws_b = workspace(1, n_in)
    vkv.matmul(xd.data_ptr(), 1, n_in, [(wd.data_ptr(), vkv.Q8_0, n_rows, y2.data_ptr())],
               ws_ptr, ws_b, hip_stream=stream_ptr())
    _, mag = rows_ref(vkv.Q8_0, w, n_rows, n_in, [x])
    check(host(y2), host(y1), 2 * mag[0])
    with pytest.raises(vkv.VkvError):
        vkv.matmul(xd.data_ptr(), 1, n_in, [(wd.data_ptr(), vkv.Q8_0, n_rows, y2.data_ptr()),
                                            (wd.data_ptr(), vkv.Q4_K, 16, y1.data_ptr())],
                   ws_ptr, ws_b, hip_stream=stream_ptr())
