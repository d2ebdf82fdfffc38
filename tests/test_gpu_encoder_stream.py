"""Streaming-vs-batch gate of the encoder (tests/node/baseline/encoder-kv.test.js:
27, 50-95): one synthetic Mel of 4,272 frames (2,136 encoder frames with the
72-frame right pad: the 878-slot ring wraps twice) through vkv_enc_conv_stem +
vkv_encoder_chunk, run by run as vkv_enc_drive_next schedules it
(encoder_kv_drive, src/voxtral.cpp:4379-4426), under three schedules fed in
three plans:

  * 4/4 steady with the 8-frame terminal flush, fed 8 Mel frames (80 ms) at a time;
  * logical 8 / physical 32, fed 48 Mel frames (480 ms) at a time;
  * throughput 128 (the batch shape: logical = physical = 128), fed whole.

The 32 encoder layers at the real shape (dim 1280, hidden 5120, 32 heads x 64,
window 750) cycle four random Q4_K/Q6_K weight sets.  Each frame is computed
exactly once (the runs tile [0, frames) with no overlap and no replay), every
run's Mel window lies inside the Mel fed so far, and the encoder outputs of the
three schedules agree within 1e-5 over an F32 ring (the reference's gate) --
bit for bit, since the window tile's key blocks are absolute.  The F16 ring is
schedule-invariant too; its distance from the F32 ring is printed."""
import numpy as np
import pytest
import torch

import vkv
from gpu_util import dev, stream_ptr
from test_gpu_conv import weights as conv_weights
from test_gpu_encoder_chunk import make_model, upload

pytestmark = pytest.mark.gpu

N_MEL, DIM, CAP, WIN, LAYERS = 128, 1280, 878, 750, 32
MEL_TOTAL, RIGHT_PAD = 4200, 72
ENC_DELTA_GATE = 1e-5           # encoder-kv.test.js:27
SCHEDULES = {
    "4/4+finish8 @80ms": ((0, 0, 0, 0), 8, True),
    "8/32 @480ms": ((0, 0, 8, 32), 48, False),
    "throughput128 @full": ((1, 0, 0, 0), MEL_TOTAL, False),
}


@pytest.fixture(scope="module")
def encoder():
    rng = np.random.default_rng(2136)
    sets = [make_model(rng, 1) for _ in range(4)]
    m = dict(layers=[sets[i % 4]["layers"][0] for i in range(LAYERS)],
             out_norm=sets[0]["out_norm"], out_norm_b=sets[0]["out_norm_b"], types=sets[0]["types"])
    model, keep, arr = upload(m)
    w0, b0, w1, b1 = conv_weights(rng)
    conv = [torch.from_numpy(np.ascontiguousarray(a)).to(dev()) for a in (w0, b0, w1, b1)]
    mel = rng.standard_normal((N_MEL, MEL_TOTAL + RIGHT_PAD)).astype(np.float32)
    mel[:, MEL_TOTAL:] = -0.625      # the right pad: one constant (silence) column
    mel_d = torch.from_numpy(mel).to(dev())
    yield model, conv, mel_d
    del keep, arr


def run_stream(encoder, dtype, sched, feed, batch_terminal):
    """(outputs [frames][dim] on the device, runs [(q0, n)])"""
    model, conv, mel_d = encoder
    sc = vkv.enc_schedule(*sched)
    frames = vkv.enc_frames_realizable(MEL_TOTAL + RIGHT_PAD)
    out = torch.full((frames, DIM), np.nan, device=dev())
    x = torch.empty(128, DIM, device=dev())
    ws_b = vkv.encoder_chunk_workspace(model, 128)
    ws = torch.empty(ws_b // 4 + 64, device=dev())
    wsp = (ws.data_ptr() + 255) & ~255
    cw_b = vkv.enc_conv_stem_workspace(2 * 128 + 8, N_MEL, DIM, 128)
    cws = torch.empty(cw_b // 4 + 64, device=dev())
    cwp = (cws.data_ptr() + 255) & ~255
    runs = []
    emitted = 0
    with vkv.Cache(n_streams=1, n_layers=LAYERS, capacity=CAP, n_kv_heads=32, head_dim=64,
                   n_q_heads=32, dtype=dtype) as c:
        def drive(avail, final):
            nonlocal emitted
            target = vkv.enc_frames_realizable(avail)
            while True:
                r = vkv.enc_drive_next(emitted, target, final, sc, 8, batch_terminal and final)
                if r.n == 0:
                    return
                assert r.q0 == emitted and 0 < r.n <= 128
                plan = vkv.enc_plan(r.q0, r.n, CAP, WIN)
                assert plan.conv_mel_end <= avail, (r.q0, r.n, plan.conv_mel_end, avail)
                conv_len = plan.conv_mel_end - plan.conv_mel_start
                assert vkv.enc_conv_stem_workspace(conv_len, N_MEL, DIM, r.n) <= cw_b
                win = mel_d[:, plan.conv_mel_start:plan.conv_mel_end].contiguous()
                vkv.enc_conv_stem(win.data_ptr(), N_MEL, plan, conv[0].data_ptr(), conv[1].data_ptr(),
                                  conv[2].data_ptr(), conv[3].data_ptr(), DIM, x.data_ptr(), cwp, cw_b,
                                  hip_stream=stream_ptr())
                vkv.encoder_chunk(c, 0, plan, WIN, model, x.data_ptr(), wsp, ws_b,
                                  hip_stream=stream_ptr())
                out[r.q0:r.q0 + r.n].copy_(x[:r.n])
                runs.append((r.q0, r.n))
                emitted += r.n

        fed = 0
        while fed < MEL_TOTAL:
            fed = min(MEL_TOTAL, fed + feed)
            drive(fed, False)
        drive(MEL_TOTAL + RIGHT_PAD, True)
        torch.cuda.synchronize()
    return out, runs, frames


def test_encoder_outputs_agree_across_schedules(encoder):
    results = {}
    for name, (sched, feed, bt) in SCHEDULES.items():
        out, runs, frames = run_stream(encoder, vkv.F32, sched, feed, bt)
        # each frame computed exactly once: the runs tile [0, frames)
        starts = [q0 for q0, _ in runs]
        assert starts == sorted(starts)
        assert sum(n for _, n in runs) == frames and runs[-1][0] + runs[-1][1] == frames
        assert all(a[0] + a[1] == b[0] for a, b in zip(runs, runs[1:]))
        assert runs[0] == (0, 128)      # the startup block at the batch shape
        got = out.cpu().numpy()
        assert np.isfinite(got).all()
        results[name] = got
        print(f"F32 {name}: {len(runs)} runs, {frames} frames, max |x| {np.abs(got).max():.3f}",
              flush=True)
    names = list(results)
    base = results[names[0]]
    for name in names[1:]:
        d = float(np.max(np.abs(results[name] - base)))
        same = np.array_equal(results[name].view(np.uint32), base.view(np.uint32))
        print(f"F32 {name} vs {names[0]}: max |delta| {d:.3e}, bitwise {same}", flush=True)
        assert d <= ENC_DELTA_GATE, (name, d)
        assert same, name

    # the F16 ring: schedule-invariant as well; its distance from the F32 ring
    f16 = {}
    for name in (names[0], names[2]):
        sched, feed, bt = SCHEDULES[name]
        f16[name] = run_stream(encoder, vkv.F16, sched, feed, bt)[0].cpu().numpy()
    assert np.array_equal(f16[names[0]].view(np.uint32), f16[names[2]].view(np.uint32))
    d16 = np.abs(f16[names[2]].astype(np.float64) - base)
    print(f"F16 ring vs F32 ring: max |delta| {d16.max():.3e}, mean {d16.mean():.3e}, "
          f"frames past the first wrap max {d16[CAP:].max():.3e}", flush=True)
