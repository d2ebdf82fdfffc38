"""GPU parity of the encoder conv stem (build_encoder_kv_graph, src/voxtral.cpp:
2094-2126) at the real shape (128 Mel bins -> 1280 channels, kernel 3, strides
1 then 2, GELU) against the oracle: conv0 over the plan's window and conv1 at
the kept frames, each checked with the GPU's own input (teacher forcing); the
frames of two plans with overlapping windows agree bit for bit."""
import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import dev, stream_ptr

pytestmark = pytest.mark.gpu

N_MEL, DIM, CAP, WIN = 128, 1280, 878, 750


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def weights(rng):
    w0 = (rng.standard_normal((DIM, N_MEL, 3)) * 0.05).astype(np.float16).view(np.uint16)
    w1 = (rng.standard_normal((DIM, DIM, 3)) * 0.02).astype(np.float16).view(np.uint16)
    b0 = (rng.standard_normal(DIM) * 0.1).astype(np.float32)
    b1 = (rng.standard_normal(DIM) * 0.1).astype(np.float32)
    return w0, b0, w1, b1


def run(mel_global, plan, wd):
    """GPU conv stem for a plan; returns (x, y0 from the workspace)"""
    w0d, b0d, w1d, b1d = wd
    win = np.ascontiguousarray(mel_global[:, plan.conv_mel_start:plan.conv_mel_end])
    conv_len = win.shape[1]
    md = to_dev(win)
    x = torch.full((plan.n_new, DIM), np.nan, device=dev())
    wb = vkv.enc_conv_stem_workspace(conv_len, N_MEL, DIM, plan.n_new)
    ws = torch.empty(wb // 4 + 64, device=dev())
    wp = (ws.data_ptr() + 255) & ~255
    vkv.enc_conv_stem(md.data_ptr(), N_MEL, plan, w0d.data_ptr(), b0d.data_ptr(), w1d.data_ptr(),
                      b1d.data_ptr(), DIM, x.data_ptr(), wp, wb, hip_stream=stream_ptr())
    # workspace: f16 im2col of conv0 (256-aligned), then conv0's output [frame][channel]
    off = (wp - ws.data_ptr()) // 4 + ((conv_len * N_MEL * 3 * 2 + 255) & ~255) // 4
    y0 = host(ws)[off:off + conv_len * DIM].reshape(conv_len, DIM)
    return host(x), y0, win


@pytest.mark.parametrize("q_start,n_new", [(0, 16), (1, 4), (2, 16), (500, 16), (1297, 4), (900, 128)])
def test_conv_stem(q_start, n_new):
    rng = np.random.default_rng(q_start * 7 + n_new)
    w0, b0, w1, b1 = weights(rng)
    wd = tuple(to_dev(a) for a in (w0, b0, w1, b1))
    plan = vkv.enc_plan(q_start, n_new, CAP, WIN)
    mel = rng.standard_normal((N_MEL, plan.conv_mel_end)).astype(np.float32)
    x, y0, win = run(mel, plan, wd)
    conv_len = win.shape[1]
    # conv0 over the window against the oracle
    want0 = oracle.conv1d(win, conv_len, 1, conv_len, N_MEL, w0, b0, 1, 2, 0, conv_len)
    np.testing.assert_allclose(y0, want0, rtol=1e-5, atol=1e-5)
    # conv1 at the kept frames from the GPU's conv0 output
    want1 = oracle.conv1d(y0, 1, DIM, conv_len, DIM, w1, b1, 2, 1, plan.conv_slice_start, n_new)
    np.testing.assert_allclose(x, want1, rtol=1e-5, atol=1e-5)


def test_overlapping_plans_agree_bitwise():
    rng = np.random.default_rng(3681)
    w0, b0, w1, b1 = weights(rng)
    wd = tuple(to_dev(a) for a in (w0, b0, w1, b1))
    mel = rng.standard_normal((N_MEL, 2 * 64)).astype(np.float32)
    xa, _, _ = run(mel, vkv.enc_plan(30, 16, CAP, WIN), wd)   # frames 30..45
    xb, _, _ = run(mel, vkv.enc_plan(38, 8, CAP, WIN), wd)    # frames 38..45
    assert np.array_equal(xa[8:16].view(np.uint32), xb.view(np.uint32))
