"""GPU parity of the realtime rows rings and the adapter
(copy_chunk_to_enc_out_ring src/voxtral.cpp:4018-4043, read_realtime_ring_rows
:5530-5554, voxtral_ctx_adapter_commit :5424-5485 over
build_adapter_ring_graph_reusable :2589-2620) against the oracle.

Ring copies are bit-exact.  The adapter is checked stage by stage with the
oracle fed the device's own stage input (teacher forcing): h = gelu(W0 x)
within 1e-5 x sum |w||x| of the oracle's product (through GELU's 1.13
Lipschitz bound, plus f32 rounding of GELU itself), then W2 h within
1e-5 x sum |w||h|; end to end the rows differ from the oracle's only where
the two h round to different Q8_K codes (a few codes per row at most)."""
import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import dev, stream_ptr
from kq_util import random_matrix

pytestmark = pytest.mark.gpu

ENC, DEC, DOWN, CAP = 1280, 3072, 4, 256


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ring_of(t):
    return vkv.RowRing(t.data_ptr(), t.shape[0], t.shape[1])


def test_ring_write_read_round_trip_across_the_wrap():
    rng = np.random.default_rng(4018)
    ring_t = torch.full((CAP, ENC), np.nan, device=dev())
    ring = ring_of(ring_t)
    want = np.full((CAP, ENC), np.nan, np.float32)
    frames = rng.standard_normal((600, ENC)).astype(np.float32)
    fd = to_dev(frames)
    pos = 0
    for n in (16, 128, 100, 4, 16, 200, 136):   # wraps at 256 and 512
        vkv.row_ring_write(ring, pos, fd[pos].data_ptr(), n, hip_stream=stream_ptr())
        oracle.row_ring_write(want, pos, frames[pos:pos + n])
        pos += n
    assert np.array_equal(host(ring_t), want)
    # read back into host memory and into device memory, across the wrap
    out = np.empty((200, ENC), np.float32)
    vkv.row_ring_read(ring, pos - 200, 200, out.ctypes.data, hip_stream=stream_ptr())
    assert np.array_equal(out, frames[pos - 200:pos])
    od = torch.empty(256, ENC, device=dev())
    vkv.row_ring_read(ring, pos - 256, 256, od.data_ptr(), hip_stream=stream_ptr())
    assert np.array_equal(host(od), frames[pos - 256:pos])
    with pytest.raises(vkv.VkvError):
        vkv.row_ring_read(ring, 0, 257, od.data_ptr(), hip_stream=stream_ptr())


@pytest.fixture(scope="module")
def weights():
    rng = np.random.default_rng(2589)
    w0 = random_matrix(rng, vkv.Q4_K, DEC, ENC * DOWN, 0.03)
    w2 = random_matrix(rng, vkv.Q6_K, DEC, DEC, 0.5)
    w0d = oracle.dequantize(oracle.Q4_K, w0, DEC * ENC * DOWN).reshape(DEC, -1).astype(np.float64)
    w2d = oracle.dequantize(oracle.Q6_K, w2, DEC * DEC).reshape(DEC, DEC).astype(np.float64)
    return w0, w2, w0d, w2d, to_dev(w0), to_dev(w2)


def q8k_abs(x):
    return np.abs(oracle.dequantize(oracle.Q8_K, oracle.q8_k_quantize(x), x.size)).astype(np.float64)


@pytest.mark.parametrize("g0,n", [(0, 1), (63, 1), (7, 2), (60, 8), (0, 32), (40, 64)])
def test_adapter_commit(weights, g0, n):
    """the 256-frame encoder ring holds 64 groups: g0 = 60 and 40 read across
    its wrap"""
    w0, w2, w0d, w2d, w0t, w2t = weights
    rng = np.random.default_rng(g0 * 100 + n)
    # frames 4 g0 .. 4 (g0 + n) written into the ring as an encoder would
    f0, nf = DOWN * g0, DOWN * n
    frames = rng.standard_normal((nf, ENC)).astype(np.float32)
    enc_t = torch.full((CAP, ENC), np.nan, device=dev())
    enc_h = np.full((CAP, ENC), np.nan, np.float32)
    fd = to_dev(frames)
    for s in range(0, nf, CAP):
        k = min(CAP, nf - s)
        vkv.row_ring_write(ring_of(enc_t), f0 + s, fd[s].data_ptr(), k, hip_stream=stream_ptr())
    aemb_t = torch.full((CAP, DEC), np.nan, device=dev())
    ad = vkv.Adapter(w0t.data_ptr(), w2t.data_ptr(), vkv.Q4_K, vkv.Q6_K, ENC, DEC, DOWN)
    ws_b = vkv.adapter_workspace(ad, n)
    ws_t = torch.empty(ws_b // 4 + 64, device=dev())
    ws = (ws_t.data_ptr() + 255) & ~255
    vkv.adapter_commit(ad, ring_of(enc_t), ring_of(aemb_t), g0, n, ws, ws_b, hip_stream=stream_ptr())
    got = host(aemb_t)
    hid = host(ws_t).view(np.uint8)[ws - ws_t.data_ptr():][:n * DEC * 4].view(np.float32).reshape(n, DEC)
    xs = frames.reshape(n, ENC * DOWN)
    oracle.row_ring_write(enc_h, f0, frames)
    want_all = np.full((CAP, DEC), np.nan, np.float32)
    oracle.adapter_commit(enc_h, want_all, g0, n, oracle.Q4_K, w0, oracle.Q6_K, w2)
    for i in range(n):
        x = xs[i]
        pre = oracle.matvec(oracle.Q4_K, w0, DEC, ENC * DOWN, x, n_threads=8).astype(np.float64)
        mag1 = np.abs(w0d) @ q8k_abs(x)
        h_want = oracle.gelu_erf(pre.astype(np.float32)).astype(np.float64)
        dh = 1.13 * 1e-5 * mag1 + 4e-7 * np.abs(h_want) + 1.2e-7 * np.abs(pre) + 1e-30
        assert np.all(np.abs(hid[i] - h_want) <= dh), i
        # second product, fed the device's own h
        y_want = oracle.matvec(oracle.Q6_K, w2, DEC, DEC, hid[i], n_threads=8).astype(np.float64)
        mag2 = np.abs(w2d) @ q8k_abs(hid[i])
        row = got[(g0 + i) % CAP].astype(np.float64)
        assert np.all(np.abs(row - y_want) <= 1e-5 * mag2 + 1e-30), i
        # end to end: only Q8_K code flips of h separate the two
        d_h = np.abs(h_want).max() / 127
        e2e = 1e-5 * mag2 + np.abs(w2d) @ dh + 4 * d_h * np.abs(w2d).max()
        assert np.all(np.abs(row - want_all[(g0 + i) % CAP]) <= e2e), i
    touched = np.zeros(CAP, bool)
    touched[[(g0 + i) % CAP for i in range(n)]] = True
    assert np.isnan(got[~touched]).all()


def test_adapter_runs_that_wrap_both_rings(weights):
    """70 groups from group 30: the encoder ring (64 groups) wraps once and a
    32-row audio ring twice; the last group written to a row wins"""
    w0, w2, _, _, w0t, w2t = weights
    rng = np.random.default_rng(70)
    enc = rng.standard_normal((CAP, ENC)).astype(np.float32)
    enc_t = to_dev(enc)
    aemb_t = torch.full((32, DEC), np.nan, device=dev())
    ad = vkv.Adapter(w0t.data_ptr(), w2t.data_ptr(), vkv.Q4_K, vkv.Q6_K, ENC, DEC, DOWN)
    ws_b = vkv.adapter_workspace(ad, 70)
    ws_t = torch.empty(ws_b // 4 + 64, device=dev())
    ws = (ws_t.data_ptr() + 255) & ~255
    vkv.adapter_commit(ad, ring_of(enc_t), ring_of(aemb_t), 30, 70, ws, ws_b, hip_stream=stream_ptr())
    want = np.full((32, DEC), np.nan, np.float32)
    oracle.adapter_commit(enc, want, 30, 70, oracle.Q4_K, w0, oracle.Q6_K, w2)
    got = host(aemb_t)
    # the oracle writes group by group, so each row holds its last group; an
    # earlier group left in a row would miss by the rows' own scale
    assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max()
    first = np.full((32, DEC), np.nan, np.float32)
    oracle.adapter_commit(enc, first, 30, 32, oracle.Q4_K, w0, oracle.Q6_K, w2)
    assert np.abs(first - want).max() > 0.1 * np.abs(want).max()


def test_one_group_and_batched_paths_agree(weights):
    """n = 1 runs two single-row products, n > 1 the matrix-core products: the
    same rows within the products' bounds"""
    _, _, _, w2d, w0t, w2t = weights
    rng = np.random.default_rng(5)
    enc_t = to_dev(rng.standard_normal((CAP, ENC)).astype(np.float32))
    ad = vkv.Adapter(w0t.data_ptr(), w2t.data_ptr(), vkv.Q4_K, vkv.Q6_K, ENC, DEC, DOWN)
    ws_b = vkv.adapter_workspace(ad, 4)
    ws_t = torch.empty(ws_b // 4 + 64, device=dev())
    ws = (ws_t.data_ptr() + 255) & ~255
    a = torch.zeros(CAP, DEC, device=dev())
    b = torch.zeros(CAP, DEC, device=dev())
    vkv.adapter_commit(ad, ring_of(enc_t), ring_of(a), 10, 4, ws, ws_b, hip_stream=stream_ptr())
    for g in range(10, 14):
        vkv.adapter_commit(ad, ring_of(enc_t), ring_of(b), g, 1, ws, ws_b, hip_stream=stream_ptr())
    ga, gb = host(a)[10:14], host(b)[10:14]
    assert np.abs(ga - gb).max() <= 2e-3 * np.abs(gb).max()
    assert not np.array_equal(ga, np.zeros_like(ga))


def test_adapter_rejects_bad_rings(weights):
    _, _, _, _, w0t, w2t = weights
    enc_t = torch.zeros(258, ENC, device=dev())
    aemb_t = torch.zeros(CAP, DEC, device=dev())
    ad = vkv.Adapter(w0t.data_ptr(), w2t.data_ptr(), vkv.Q4_K, vkv.Q6_K, ENC, DEC, DOWN)
    ws_t = torch.empty(1 << 20, device=dev())
    with pytest.raises(vkv.VkvError):
        vkv.adapter_commit(ad, ring_of(enc_t), ring_of(aemb_t), 0, 1, ws_t.data_ptr(), 1 << 22,
                           hip_stream=stream_ptr())
    assert "multiple of 4" in vkv.last_error()


@pytest.mark.parametrize("f16", [True, False])
def test_ada_scale(f16):
    """vkv_ada_scale (build_decoder_layer's ada MLP, src/voxtral.cpp:2864-2874)
    against the oracle: the hidden rows within the Q4_K product's bound through
    GELU, the output within the second product's bound plus one f16 ulp of h"""
    from test_adapter import ada_w0
    rng = np.random.default_rng(2866 + f16)
    dim, ad = 3072, 32
    w0 = ada_w0(rng, ad, dim)
    w2 = (rng.standard_normal((dim, ad)) * 0.1).astype(np.float16 if f16 else np.float32)
    w2_arg = w2.view(np.uint16) if f16 else w2
    want = oracle.ada_scale(oracle.Q4_K, w0, w2_arg, dim, ad, 6.0).astype(np.float64)
    w0t, w2t = to_dev(w0), to_dev(w2_arg)
    out = torch.full((dim,), np.nan, device=dev())
    wb = vkv.ada_scale_workspace(dim, ad)
    ws_t = torch.empty(wb // 4 + 64, device=dev())
    ws = (ws_t.data_ptr() + 255) & ~255
    vkv.ada_scale(w0t.data_ptr(), vkv.Q4_K, w2t.data_ptr(), vkv.F16 if f16 else vkv.F32, dim, ad,
                  6.0, out.data_ptr(), ws, wb, hip_stream=stream_ptr())
    got = host(out).astype(np.float64)
    e = oracle.time_embedding(6.0, dim)
    w0d = np.abs(oracle.dequantize(oracle.Q4_K, w0, ad * dim).reshape(ad, dim).astype(np.float64))
    dh = 1.13 * 1e-5 * (w0d @ q8k_abs(e)) + 1e-6
    # the workspace keeps h after the time embedding (256-byte aligned)
    h = host(ws_t).view(np.uint8)[ws - ws_t.data_ptr() + dim * 4:][:ad * 4].view(np.float32).astype(np.float64)
    h_want = oracle.gelu_erf(oracle.matvec(oracle.Q4_K, w0, ad, dim, e)).astype(np.float64)
    assert np.all(np.abs(h - h_want) <= dh)
    w2d = np.abs(w2.astype(np.float64))
    ulp = np.abs(h) * 2.0 ** -10 if f16 else 0.0
    assert np.all(np.abs(got - want) <= w2d @ (dh + ulp) + 1e-6 * np.abs(want) + 1e-30)
