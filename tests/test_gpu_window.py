"""GPU parity of the multi-query window attention: the encoder's causal
sliding window over the 878-slot ring (32 layers, 32 heads x 64, window 750,
16-frame chunks) and the decoder's causal prefill, against the oracle's fp64
window attention; ring state bit-exact.  The encoder chunks are also held to
the oracle's restatement of the reference's own CPU arithmetic for 16-row
blocks (src/voxtral.cpp:2259-2281: the query rounded to f16 against an F16
ring, softmax in f32, the weights rounded to f16 against an F16 V): within
2e-3 for an F16 ring and 1e-5 for an F32 ring at every checked chunk."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import SEED, empty_f32, layer_image, stream_ptr, synth

pytestmark = pytest.mark.gpu

POOL = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))
EH, ED, ECAP, EWIN, EL = 32, 64, 878, 750, 32
# F32: the reference's gate for the F32 encoder ring (encoder KV against the
# global batch within 1e-5, tests/node/baseline/encoder-kv.test.js:27)
TOL = {vkv.F16: 2e-3, vkv.F32: 1e-5, vkv.Q8_0: 1e-2}


def enc_inputs(layers, q_start, n):
    q = synth(None, EH * ED, vkv.TAG_EQ, nl=layers, p0=q_start, np_=n)
    k = synth(None, EH * ED, vkv.TAG_EK, nl=layers, p0=q_start, np_=n)
    v = synth(None, EH * ED, vkv.TAG_EV, nl=layers, p0=q_start, np_=n)
    return q, k, v


def oracle_window(c, layer, key_pos, q_rows, q_pos, n_q_heads, n_kv_heads, head_dim, window,
                  scale, ring_capacity, mimic=False):
    kimg = layer_image(c, 0, 0, layer)
    vimg = layer_image(c, 1, 0, layer)
    key_pos = np.asarray(key_pos, np.int64)
    fn = oracle.window_attn_mimic if mimic else oracle.window_attn_f64
    return fn(c.dtype, kimg, vimg, int(c.row_bytes), (key_pos % ring_capacity).astype(np.int32),
              key_pos, q_rows, np.asarray(q_pos, np.int64), n_q_heads, n_kv_heads, head_dim,
              window, scale)


@pytest.mark.parametrize("dtype,frames", [(vkv.F16, 6000), (vkv.F32, 6000), (vkv.Q8_0, 1200)])
def test_encoder_window_chunks(dtype, frames):
    """16 new frames per chunk as a 16-query block against the window."""
    P = 16
    n_chunks = frames // P
    checks = {0, 1, 46, 47, 54, 55, 56, n_chunks - 1}      # first wrap at frame 878 is in chunk 54
    with vkv.Cache(n_streams=1, n_layers=EL, capacity=ECAP, n_kv_heads=EH, head_dim=ED,
                   n_q_heads=EH, dtype=dtype) as c:
        out = empty_f32(EL, P, EH * ED)
        for ch in range(n_chunks):
            q_start = ch * P
            plan = vkv.enc_plan(q_start, P, ECAP, EWIN)
            q, k, v = enc_inputs(EL, q_start, P)
            c.enc_step(0, plan, EWIN, 0, EL, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                       out.data_ptr(), 0.125, hip_stream=stream_ptr())
            if ch not in checks:
                continue
            torch.cuda.synchronize()
            layers = [0, 13, 31]
            wants = list(POOL.map(lambda jw: oracle.expected_layer(
                dtype, ECAP, ECAP, EH * ED, plan.win_end, SEED,
                (vkv.TAG_EK, vkv.TAG_EV)[jw[1]], 0, jw[0]), [(l, w) for l in layers for w in (0, 1)]))
            for (l, w), want in zip([(l, w) for l in layers for w in (0, 1)], wants):
                assert np.array_equal(layer_image(c, w, 0, l), want), (ch, l, w)
            key_pos = np.arange(plan.win_start, plan.win_end)
            q_pos = np.arange(q_start, q_start + P)
            msg = []
            for l in (0, 31):
                q_rows = q[0, l].cpu().numpy().reshape(P, EH, ED)
                want = oracle_window(c, l, key_pos, q_rows, q_pos, EH, EH, ED, EWIN, 0.125, ECAP)
                got = out[l].cpu().numpy().reshape(P, EH, ED)
                e_exact = float(np.max(np.abs(got - want)))
                assert e_exact <= TOL[dtype], (ch, l, e_exact)
                if dtype != vkv.Q8_0:     # the reference's encoder ring is F16 or F32
                    mim = oracle_window(c, l, key_pos, q_rows, q_pos, EH, EH, ED, EWIN, 0.125, ECAP,
                                        mimic=True)
                    e_mimic = float(np.max(np.abs(got - mim)))
                    assert e_mimic <= TOL[dtype], (ch, l, e_mimic)
                    msg.append(f"layer {l}: gpu-fp64 {e_exact:.2e} gpu-mimic {e_mimic:.2e} "
                               f"mimic-fp64 {float(np.max(np.abs(mim - want))):.2e}")
            print(f"encoder chunk {ch} ok {'; '.join(msg)}", flush=True)


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.F32, vkv.Q8_0])
def test_decoder_prefill_then_steps(dtype):
    """38-token causal prefill at positions 0..37 (the stream prompt), a second
    10-token prefill, then a 300-token one (75 query tiles per kv head: its
    rows are appended in a launch of their own instead of the fused write),
    each against the oracle's ring image and fp64 causal attention."""
    L = 4
    with vkv.Cache(n_streams=1, n_layers=L, capacity=8192, dtype=dtype) as c:
        ring = vkv.new_ring(8192)
        for n in (38, 10, 300):
            start = ring.next_absolute_position
            q = synth(None, 4096, vkv.TAG_Q, nl=L, p0=start, np_=n)
            k = synth(None, 1024, vkv.TAG_K, nl=L, p0=start, np_=n)
            v = synth(None, 1024, vkv.TAG_V, nl=L, p0=start, np_=n)
            out = empty_f32(L, n, 4096)
            c.decoder_prefill(0, ring, 0, L, n, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                              out.data_ptr(), 1 / np.sqrt(128), hip_stream=stream_ptr())
            torch.cuda.synchronize()
            assert ring.next_absolute_position == start + n
            for l in range(L):
                for w in (0, 1):
                    want = oracle.expected_layer(dtype, 8192, 8192, 1024, start + n, SEED,
                                                 (vkv.TAG_K, vkv.TAG_V)[w], 0, l)
                    assert np.array_equal(layer_image(c, w, 0, l), want)
                want = oracle_window(c, l, np.arange(0, start + n), q[0, l].cpu().numpy().reshape(n, 32, 128),
                                     np.arange(start, start + n), 32, 8, 128, 0, 1 / np.sqrt(128), 8192)
                got = out[l].cpu().numpy().reshape(n, 32, 128)
                assert np.max(np.abs(got - want)) <= TOL[dtype], (start, l)


def test_window_attn_entry_point_over_wrapped_segments():
    """vkv_window_attn over an explicitly wrapped two-segment window with an
    arbitrary absolute key origin."""
    cap = 100
    with vkv.Cache(n_streams=1, n_layers=2, capacity=cap, n_kv_heads=4, head_dim=64,
                   n_q_heads=8, dtype=vkv.F16) as c:
        k = synth(None, 256, vkv.TAG_K, nl=2, p0=0, np_=cap)
        v = synth(None, 256, vkv.TAG_V, nl=2, p0=0, np_=cap)
        c.append(0, 0, 2, [(0, cap)], k.data_ptr(), v.data_ptr(), hip_stream=stream_ptr())
        segs = [(70, 30), (0, 50)]            # logical window of 80 keys, positions 1000..1079
        n_q = 7
        q = synth(None, 8 * 64, vkv.TAG_Q, nl=2, p0=0, np_=n_q)
        out = empty_f32(2, n_q, 8 * 64)
        c.window_attn(0, 0, 2, segs, 1000, 1070, n_q, 25, q.data_ptr(), out.data_ptr(), 0.125,
                      hip_stream=stream_ptr())
        torch.cuda.synchronize()
        slots = np.r_[np.arange(70, 100), np.arange(0, 50)].astype(np.int32)
        key_pos = np.arange(1000, 1080)
        for l in range(2):
            kimg, vimg = layer_image(c, 0, 0, l), layer_image(c, 1, 0, l)
            want = oracle.window_attn_f64(vkv.F16, kimg, vimg, int(c.row_bytes), slots, key_pos,
                                          q[0, l].cpu().numpy().reshape(n_q, 8, 64),
                                          np.arange(1070, 1070 + n_q), 8, 4, 64, 25, 0.125)
            got = out[l].cpu().numpy().reshape(n_q, 8, 64)
            assert np.max(np.abs(got - want)) <= 2e-3


@pytest.mark.parametrize("sched,batch_terminal", [((0, 0, 0, 0), True), ((0, 0, 8, 32), False)])
def test_encoder_stream_driven_by_the_schedule(sched, batch_terminal):
    """A streaming encoder over the ring, run by run as vkv_enc_drive_next
    schedules it: the 128-frame startup block (16-row tiles x 8), small feed
    batches, the finish flush, and the first ring wrap (frame 878); ring state
    bit-exact and attention within 2e-3 of the oracle at sampled runs."""
    L = 4
    sc = vkv.enc_schedule(*sched)
    mel_total, right_pad = 2000, 72
    with vkv.Cache(n_streams=1, n_layers=L, capacity=ECAP, n_kv_heads=EH, head_dim=ED,
                   n_q_heads=EH, dtype=vkv.F16) as c:
        emitted, runs_done = 0, 0
        chunks = [160] * (mel_total // 160) + [mel_total % 160]
        fed = 0

        def run_until_stop(target, final):
            nonlocal emitted, runs_done
            while True:
                r = vkv.enc_drive_next(emitted, target, final, sc, 8, batch_terminal)
                if r.n == 0:
                    return
                plan = vkv.enc_plan(r.q0, r.n, ECAP, EWIN)
                q, k, v = enc_inputs(L, r.q0, r.n)
                out = empty_f32(L, r.n, EH * ED)
                c.enc_step(0, plan, EWIN, 0, L, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           out.data_ptr(), 0.125, hip_stream=stream_ptr())
                emitted += r.n
                runs_done += 1
                if r.warmup or runs_done % 37 == 0 or (r.q0 < ECAP <= r.q0 + r.n) or final:
                    torch.cuda.synchronize()
                    for l in (0, L - 1):
                        for w in (0, 1):
                            want = oracle.expected_layer(vkv.F16, ECAP, ECAP, EH * ED, emitted,
                                                         SEED, (vkv.TAG_EK, vkv.TAG_EV)[w], 0, l)
                            assert np.array_equal(layer_image(c, w, 0, l), want), (r.q0, l, w)
                        want = oracle_window(c, l, np.arange(plan.win_start, plan.win_end),
                                             q[0, l].cpu().numpy().reshape(r.n, EH, ED),
                                             np.arange(r.q0, r.q0 + r.n), EH, EH, ED, EWIN, 0.125,
                                             ECAP)
                        got = out[l].cpu().numpy().reshape(r.n, EH, ED)
                        assert np.max(np.abs(got - want)) <= 2e-3, (r.q0, r.n, l)

        for ch in chunks:
            fed += ch
            run_until_stop(vkv.enc_frames_realizable(fed), False)
        target = vkv.enc_frames_realizable(mel_total + right_pad)
        run_until_stop(target, True)
        assert emitted == target
        print(f"encoder stream: {runs_done} runs, {emitted} frames", flush=True)


@pytest.mark.parametrize("head_dim,n_kv_heads,n_q_heads,per_layer",
                         [(64, 32, 32, False), (64, 32, 32, True), (128, 8, 32, False)])
def test_f32_matrix_core_tile_against_scalar_kernel(head_dim, n_kv_heads, n_q_heads, per_layer):
    """The F32 window tile on v_mfma_f32_16x16x4_f32 against the scalar-ALU
    kernel (VKV_KERNEL_WINDOW_VALU) over the same wrapped ring and queries:
    both f32 throughout, within 2e-6; ring bytes identical (the fused copy
    and the separate append store the same f32 rows).  per_layer: one call
    per layer (the encoder chunk's shape)."""
    cap, layers, n_q = 878, 2, 16
    kv_dim = n_kv_heads * head_dim
    outs, imgs = [], []
    for flags in (0, vkv.KERNEL_WINDOW_VALU):
        with vkv.Cache(n_streams=1, n_layers=layers, capacity=cap, n_kv_heads=n_kv_heads,
                       head_dim=head_dim, n_q_heads=n_q_heads, dtype=vkv.F32, kernel_flags=flags) as c:
            for ch in range(70):                     # 1120 frames: the ring wraps
                q_start = ch * n_q
                plan = vkv.enc_plan(q_start, n_q, cap, EWIN)
                q = synth(None, n_q_heads * head_dim, vkv.TAG_EQ, nl=layers, p0=q_start, np_=n_q)
                k = synth(None, kv_dim, vkv.TAG_EK, nl=layers, p0=q_start, np_=n_q)
                v = synth(None, kv_dim, vkv.TAG_EV, nl=layers, p0=q_start, np_=n_q)
                out = empty_f32(layers, n_q, n_q_heads * head_dim)
                if per_layer:
                    for l in range(layers):
                        c.enc_step(0, plan, EWIN, l, 1, q[0, l].data_ptr(), k[0, l].data_ptr(),
                                   v[0, l].data_ptr(), out[l].data_ptr(), 1 / np.sqrt(head_dim),
                                   hip_stream=stream_ptr())
                else:
                    c.enc_step(0, plan, EWIN, 0, layers, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               out.data_ptr(), 1 / np.sqrt(head_dim), hip_stream=stream_ptr())
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
            imgs.append([layer_image(c, w, 0, l).copy() for l in range(layers) for w in (0, 1)])
    for a, b in zip(*imgs):
        assert np.array_equal(a, b)
    d = float(np.max(np.abs(outs[0] - outs[1])))
    assert np.isfinite(outs[0]).all() and d <= 2e-6, d
    print(f"f32 tile head_dim {head_dim}: |mfma - valu| {d:.2e}", flush=True)


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.F32])
def test_per_layer_split_tile_is_schedule_invariant_across_tile_groups(dtype):
    """The one-layer window call at head_dim 64 and GQA 1 (the encoder's shape)
    splits each head's keys over 8 work groups and merges their partials in a
    second launch, in groups of at most 8 query tiles.  vkv_window_attn over a
    full 878-slot ring as two wrapped segments: one call of 200 queries (13
    tiles: groups of 8 and 5) against the same queries in 16-query calls, bit
    for bit, and against the oracle's fp64 window attention."""
    cap, n_q, win, k0, q0 = ECAP, 200, 300, 5000, 5678
    scale = 1.0 / np.sqrt(ED)
    with vkv.Cache(n_streams=1, n_layers=2, capacity=cap, n_kv_heads=EH, head_dim=ED,
                   n_q_heads=EH, dtype=dtype) as c:
        k = synth(None, EH * ED, vkv.TAG_K, nl=2, p0=0, np_=cap)
        v = synth(None, EH * ED, vkv.TAG_V, nl=2, p0=0, np_=cap)
        c.append(0, 0, 2, [(0, cap)], k.data_ptr(), v.data_ptr(), hip_stream=stream_ptr())
        segs = [(300, cap - 300), (0, 300)]      # key positions k0 .. k0 + cap - 1
        q = synth(None, EH * ED, vkv.TAG_Q, nl=2, p0=0, np_=n_q)
        one = empty_f32(2, n_q, EH * ED)
        parts = empty_f32(2, n_q, EH * ED)
        for l in range(2):
            c.window_attn(0, l, 1, segs, k0, q0, n_q, win, q[0, l].data_ptr(), one[l].data_ptr(),
                          scale, hip_stream=stream_ptr())
            for p0 in range(0, n_q, 16):
                n = min(16, n_q - p0)
                c.window_attn(0, l, 1, segs, k0, q0 + p0, n, win, q[0, l, p0:].data_ptr(),
                              parts[l, p0:].data_ptr(), scale, hip_stream=stream_ptr())
        torch.cuda.synchronize()
        a, b = one.cpu().numpy(), parts.cpu().numpy()
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        slots = np.r_[np.arange(300, cap), np.arange(0, 300)].astype(np.int32)
        key_pos = np.arange(k0, k0 + cap)
        for l in range(2):
            want = oracle.window_attn_f64(dtype, layer_image(c, 0, 0, l), layer_image(c, 1, 0, l),
                                          int(c.row_bytes), slots, key_pos,
                                          q[0, l].cpu().numpy().reshape(n_q, EH, ED),
                                          np.arange(q0, q0 + n_q), EH, EH, ED, win, scale)
            err = float(np.max(np.abs(a[l].reshape(n_q, EH, ED) - want)))
            assert err <= TOL[dtype], (l, err)
        print(f"split tile groups dtype {dtype}: 200-query call == 16-query calls bit for bit, "
              f"fp64 err {err:.2e}", flush=True)
