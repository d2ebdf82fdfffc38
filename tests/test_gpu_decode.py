"""GPU parity of the decoder KV step (append + single-query GQA attention)
against the oracle, at the decoder shapes: cache state bit-exact; attention
within 2e-3 (F16 KV) / 1e-2 (q8_0 KV) of the ggml-mimic, the oracle's
restatement of the reference's CPU flash-attention path (for q8_0 K that path
quantizes Q to q8_0 blocks and takes integer block sums, as the GPU does), and
close to the exact fp64 attention (EXACT_TOL)."""
import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import (SEED, empty_f32, expected_image, layer_image, oracle_decode, plan_slots,
                      step_inputs, stream_ptr, synth)

pytestmark = pytest.mark.gpu

TOL = {vkv.F16: 2e-3, vkv.F32: 1e-4, vkv.Q8_0: 1e-2}
# At the 26 x 8192 F16 shape the ggml mimic's f16 V accumulator is itself up
# to ~2.1e-3 from the exact attention (it rounds a running sum of ~300
# weighted rows to f16 at every key), so there the GPU is held to the exact
# result (1e-4) and to the mimic within the mimic's own distance from it.
F16_FULL_EXACT = 1e-4


# ggml's reduction with only its f16 V accumulator replaced by an f32 one
# (Q rounded to f16, f32 scores, the per-key online softmax) sits within this
# of the GPU at windows of 2048 keys and more (measured 1.3e-5 .. 3.4e-5 at
# 2048 .. 8192 keys, against 2e-5 .. 5.6e-5 from the exact attention): the
# GPU's remaining differences are the f16 rounding of its (lazily rescaled)
# softmax weights and the summation order.
F16_ACC32_TOL = 5e-5


def check_full_window_f16(got, exact, mimic, where, bound=F16_FULL_EXACT, acc32=None):
    """the F16 checks at windows where ggml's f16 V accumulator drifts: the
    GPU within `bound` of the exact attention, and within F16_ACC32_TOL of
    ggml's arithmetic with an f32 accumulator (`acc32`), which pins the
    query's f16 rounding and the softmax to the reference's path.  The full
    mimic's distance from the GPU is returned, not asserted: at these windows
    it is the f16 accumulator's drift from the exact result (~2.07e-3 at
    8192 keys), which the oracle's closed forms pin."""
    e_gpu = float(np.max(np.abs(got - exact)))
    e_mimic = float(np.max(np.abs(mimic - exact)))
    d = float(np.max(np.abs(got - mimic)))
    d32 = float("nan")
    assert e_gpu <= bound, (where, e_gpu)
    if acc32 is not None:
        d32 = float(np.max(np.abs(got - acc32)))
        assert d32 <= F16_ACC32_TOL, (where, d32)
    return e_gpu, e_mimic, d, d32
# Distance to the exact attention: for q8_0 the quantization of Q to q8_0
# blocks (ggml's q8_0 dot product) moves the output by up to ~1.5e-2 on
# windows of a few keys.
EXACT_TOL = {vkv.F16: 2e-3, vkv.F32: 1e-4, vkv.Q8_0: 3e-2}
SCALE = 1.0 / np.sqrt(128.0)
POOL = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))


def check_cache_state(c, streams, layers, ring_capacity, next_pos):
    """every listed (stream, layer, K|V) image equals the oracle's closed form"""
    jobs = [(s, l, w) for s in streams for l in layers for w in (0, 1)]
    wants = POOL.map(lambda j: expected_image(c, j[2], j[0], j[1], ring_capacity, next_pos[j[0]]), jobs)
    for (s, l, w), want in zip(jobs, wants):
        got = layer_image(c, w, s, l)
        assert np.array_equal(got, want), f"stream {s} layer {l} {'KV'[w]} differs at next={next_pos[s]}"


def prefill_by_append(c, ring, stream, n, layers):
    """positions [next, next+n) written through the planned append path"""
    start = ring.next_absolute_position
    plan = vkv.decoder_plan(ring, start, n)
    k = synth(None, c.kv_dim, vkv.TAG_K, s0=stream, l0=0, nl=layers, p0=start, np_=n)
    v = synth(None, c.kv_dim, vkv.TAG_V, s0=stream, l0=0, nl=layers, p0=start, np_=n)
    c.append(stream, 0, layers, vkv.plan_segs(plan.write_seg, plan.write_nseg), k.data_ptr(),
             v.data_ptr(), hip_stream=stream_ptr())
    vkv.decoder_commit(ring, plan)
    return plan


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.F32, vkv.Q8_0])
@pytest.mark.parametrize("capacity", [8192, 1025])
def test_single_layer_append_then_attend(dtype, capacity):
    """One decoder layer: 1024 positions prefilled, append position 1024, then
    1-query attention over all 1025 positions."""
    with vkv.Cache(n_streams=1, n_layers=1, capacity=capacity, dtype=dtype) as c:
        ring = vkv.new_ring(capacity)
        prefill_by_append(c, ring, 0, 1024, 1)
        q, k, v = step_inputs(c, [1024], n_layers=1)
        out = empty_f32(1, 1, 4096)
        rings = (vkv.Ring * 1)(ring)
        plans = c.decoder_step(0, rings, [1024], 0, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               out.data_ptr(), SCALE, hip_stream=stream_ptr())
        assert rings[0].next_absolute_position == 1025 and rings[0].used == 1025
        check_cache_state(c, [0], [0], capacity, {0: 1025})
        slots = plan_slots(plans[0])
        assert len(slots) == 1025
        q_row = q[0, 0].cpu().numpy()
        got = out[0, 0].cpu().numpy().reshape(32, 128)
        exact = oracle_decode(c, 0, 0, slots, q_row)
        mimic = oracle_decode(c, 0, 0, slots, q_row, mimic=True)
        assert np.max(np.abs(got - exact)) <= EXACT_TOL[dtype]
        assert np.max(np.abs(got - mimic)) <= TOL[dtype]
        # the unfused attention entry point over the same window agrees bit for bit
        out2 = empty_f32(1, 1, 4096)
        c.decode_attn(0, [plans[0]], 0, 1, q.data_ptr(), out2.data_ptr(), SCALE, hip_stream=stream_ptr())
        torch.cuda.synchronize()
        assert torch.equal(out, out2)


def test_empty_and_tiny_windows():
    with vkv.Cache(n_streams=1, n_layers=2, capacity=64, dtype=vkv.F16) as c:
        q = synth(None, 4096, vkv.TAG_Q, nl=2)
        out = empty_f32(2, 4096)
        empty = vkv.Plan()
        c.decode_attn(0, [empty], 0, 2, q.data_ptr(), out.data_ptr(), SCALE, hip_stream=stream_ptr())
        torch.cuda.synchronize()
        assert torch.count_nonzero(out) == 0          # no keys -> 0, as ggml's S=0 case
        ring = vkv.new_ring(64)
        rings = (vkv.Ring * 1)(ring)
        for pos in range(3):
            qq, k, v = step_inputs(c, [pos], n_layers=2)
            plans = c.decoder_step(0, rings, [pos], 0, 2, qq.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
            for layer in range(2):
                want = oracle_decode(c, 0, layer, plan_slots(plans[0]), qq[0, layer].cpu().numpy())
                got = out[layer].cpu().numpy().reshape(32, 128)
                assert np.max(np.abs(got - want)) <= 2e-3
        # one key: the output is that key's value row exactly (softmax weight 1)
        vrow = oracle.f16_bits_to_f32(np.frombuffer(c.read_rows(1, 0, 0, 0, 1), np.uint16))
        c.decode_attn(0, [vkv.decoder_plan(vkv.new_ring(64), 0, 1)], 0, 1, q.data_ptr(),
                      out.data_ptr(), SCALE, hip_stream=stream_ptr())
        torch.cuda.synchronize()
        got = out[0].cpu().numpy().reshape(32, 128)
        assert np.array_equal(got, np.repeat(vrow.reshape(8, 128), 4, axis=0))


def test_decoder_stream_4096_steps_no_wrap():
    """26 layers, 4096 consecutive steps from an empty 8192 ring."""
    with vkv.Cache(n_streams=1, n_layers=26, capacity=8192, dtype=vkv.F16) as c:
        rings = (vkv.Ring * 1)(vkv.new_ring(8192))
        out = empty_f32(1, 26, 4096)
        for pos in range(4096):
            q, k, v = step_inputs(c, [pos])
            plans = c.decoder_step(0, rings, [pos], 0, 26, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
            if pos in (0, 1, 4095):
                check_cache_state(c, [0], range(26), 8192, {0: pos + 1})
            if pos in (0, 1, 2047, 4095):
                for layer in (0, 13, 25):
                    slots, q_row = plan_slots(plans[0]), q[0, layer].cpu().numpy()
                    got = out[0, layer].cpu().numpy().reshape(32, 128)
                    exact = oracle_decode(c, 0, layer, slots, q_row)
                    mimic = oracle_decode(c, 0, layer, slots, q_row, mimic=True)
                    if pos < 1024:
                        # short windows: the literal bar against the ggml mimic
                        assert np.max(np.abs(got - mimic)) <= TOL[vkv.F16], (pos, layer)
                        assert np.max(np.abs(got - exact)) <= EXACT_TOL[vkv.F16], (pos, layer)
                        continue
                    acc32 = oracle_decode(c, 0, layer, slots, q_row, acc32=True)
                    errs = check_full_window_f16(got, exact, mimic, (pos, layer), acc32=acc32)
                    print(f"stream step {pos} layer {layer}: |gpu-fp64| {errs[0]:.2e}, "
                          f"|mimic-fp64| {errs[1]:.2e}, |gpu-mimic| {errs[2]:.2e}, "
                          f"|gpu-acc32| {errs[3]:.2e}", flush=True)
        assert rings[0].wraps == 0 and rings[0].used == 4096


def test_longform_ring_32768_steps():
    """26 layers, 8192-slot ring, 32768 single-token steps (the ring wraps 3x):
    ring metadata, full cache state and attention at steps 8191, 8192, 16500,
    32767."""
    meta = {8191: (8192, 0, 8192, 0, 0), 8192: (8192, 1, 8193, 1, 1),
            16500: (8192, 8309, 16501, 2, 8309), 32767: (8192, 24576, 32768, 3, 24576)}
    with vkv.Cache(n_streams=1, n_layers=26, capacity=8192, dtype=vkv.F16) as c:
        rings = (vkv.Ring * 1)(vkv.new_ring(8192))
        out = empty_f32(1, 26, 4096)
        for pos in range(32768):
            q, k, v = step_inputs(c, [pos])
            plans = c.decoder_step(0, rings, [pos], 0, 26, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
            if pos in meta:
                r = rings[0]
                assert (r.used, r.oldest_absolute_position, r.next_absolute_position, r.wraps,
                        r.evictions) == meta[pos]
                assert r.bytes_moved == 0 and r.full_buffer_moves == 0
                check_cache_state(c, [0], range(26), 8192, {0: pos + 1})
                for layer in (0, 25):
                    slots, q_row = plan_slots(plans[0]), q[0, layer].cpu().numpy()
                    got = out[0, layer].cpu().numpy().reshape(32, 128)
                    exact = oracle_decode(c, 0, layer, slots, q_row)
                    mimic = oracle_decode(c, 0, layer, slots, q_row, mimic=True)
                    acc32 = oracle_decode(c, 0, layer, slots, q_row, acc32=True)
                    errs = check_full_window_f16(got, exact, mimic, (pos, layer), acc32=acc32)
                    print(f"longform step {pos} layer {layer}: |gpu-fp64| {errs[0]:.2e}, "
                          f"|mimic-fp64| {errs[1]:.2e}, |gpu-mimic| {errs[2]:.2e}, "
                          f"|gpu-acc32| {errs[3]:.2e}", flush=True)
                print(f"longform step {pos} ok", flush=True)


def test_test_capacity_seam_64_of_8192():
    """A logical ring of 64 slots over the 8192-slot backing store
    (VOXTRAL_DECODER_KV_TEST_CAPACITY, src/voxtral.cpp:1537-1545): slots >= 64
    are never touched; wraps every 64 steps."""
    with vkv.Cache(n_streams=1, n_layers=2, capacity=8192, dtype=vkv.F16) as c:
        rings = (vkv.Ring * 1)(vkv.new_ring(64))
        out = empty_f32(1, 2, 4096)
        for pos in range(200):
            q, k, v = step_inputs(c, [pos], n_layers=2)
            plans = c.decoder_step(0, rings, [pos], 0, 2, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
            if pos in (63, 64, 130, 199):
                check_cache_state(c, [0], [0, 1], 64, {0: pos + 1})
                for layer in (0, 1):
                    want = oracle_decode(c, 0, layer, plan_slots(plans[0]), q[0, layer].cpu().numpy())
                    got = out[0, layer].cpu().numpy().reshape(32, 128)
                    assert np.max(np.abs(got - want)) <= 2e-3
        assert rings[0].wraps == 3 and rings[0].evictions == 200 - 64


def test_invalid_step_is_rejected_before_any_device_work():
    with vkv.Cache(n_streams=2, n_layers=1, capacity=16, dtype=vkv.F16) as c:
        rings = (vkv.Ring * 2)(vkv.new_ring(16), vkv.new_ring(16))
        q, k, v = step_inputs(c, [0, 0], n_layers=1)
        out = empty_f32(2, 1, 4096)
        with pytest.raises(vkv.VkvError) as ei:
            c.decoder_step(0, rings, [0, 5], 0, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           out.data_ptr(), SCALE, hip_stream=stream_ptr())
        assert ei.value.status == vkv.INVALID_ARGUMENT
        assert "stream 1" in ei.value.message
        assert rings[0].next_absolute_position == 0 and rings[1].next_absolute_position == 0
        assert not layer_image(c, 0, 0, 0).any() and not layer_image(c, 1, 1, 0).any()
        big = (vkv.Ring * 1)(vkv.new_ring(17))
        with pytest.raises(vkv.VkvError):
            c.decoder_step(0, big, [0], 0, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                           out.data_ptr(), SCALE, hip_stream=stream_ptr())


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.Q8_0])
def test_multi_stream_batch_mixed_fill(dtype):
    """Independent streams at different fill levels (one wrapped) in one launch."""
    ns, nl, cap = 5, 3, 512
    fills = [0, 1, 300, 512, 1500]
    with vkv.Cache(n_streams=ns, n_layers=nl, capacity=cap, dtype=dtype) as c:
        rings = (vkv.Ring * ns)(*[vkv.new_ring(cap) for _ in range(ns)])
        for s, n in enumerate(fills):
            left = n
            while left:
                m = min(cap, left)
                prefill_by_append(c, rings[s], s, m, nl)
                left -= m
        q, k, v = step_inputs(c, fills)
        out = empty_f32(ns, nl, 4096)
        plans = c.decoder_step(0, rings, fills, 0, nl, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               out.data_ptr(), SCALE, hip_stream=stream_ptr())
        check_cache_state(c, range(ns), range(nl), cap, {s: fills[s] + 1 for s in range(ns)})
        for s in range(ns):
            for layer in range(nl):
                slots, q_row = plan_slots(plans[s]), q[s, layer].cpu().numpy()
                got = out[s, layer].cpu().numpy().reshape(32, 128)
                mimic = oracle_decode(c, s, layer, slots, q_row, mimic=True)
                exact = oracle_decode(c, s, layer, slots, q_row)
                assert np.max(np.abs(got - mimic)) <= TOL[dtype], (s, layer)
                assert np.max(np.abs(got - exact)) <= EXACT_TOL[dtype], (s, layer)


def test_q8_0_eight_streams_full_window():
    """q8_0 KV, 8 independent streams, 26 layers, 8192 window: fast-forward each
    ring with planned multi-row appends to just before the checkpoints, then
    single decode steps; cache bit-exact and attention within 1e-2."""
    ns = 8
    with vkv.Cache(n_streams=ns, n_layers=26, capacity=8192, dtype=vkv.Q8_0) as c:
        rings = (vkv.Ring * ns)(*[vkv.new_ring(8192) for _ in range(ns)])
        out = empty_f32(ns, 26, 4096)
        pos = 0
        for target in (8191, 8192, 16500, 32767):
            while pos < target:
                m = min(8192, target - pos)
                for s in range(ns):
                    prefill_by_append(c, rings[s], s, m, 26)
                pos += m
            q, k, v = step_inputs(c, [pos] * ns)
            plans = c.decoder_step(0, rings, [pos] * ns, 0, 26, q.data_ptr(), k.data_ptr(),
                                   v.data_ptr(), out.data_ptr(), SCALE, hip_stream=stream_ptr())
            pos += 1
            check_cache_state(c, [0, ns - 1], range(0, 26, 5), 8192, {0: pos, ns - 1: pos})
            for s in (0, 3, ns - 1):
                slots, q_row = plan_slots(plans[s]), q[s, 25].cpu().numpy()
                got = out[s, 25].cpu().numpy().reshape(32, 128)
                mimic = oracle_decode(c, s, 25, slots, q_row, mimic=True)
                exact = oracle_decode(c, s, 25, slots, q_row)
                assert np.max(np.abs(got - mimic)) <= 1e-2, (target, s)
                assert np.max(np.abs(got - exact)) <= EXACT_TOL[vkv.Q8_0], (target, s)
            print(f"q8_0 8-stream step {target} ok", flush=True)


def test_q8_0_eight_streams_step_by_step_across_wraps():
    """Config 5 as a stream: q8_0 KV, 8 independent streams, 26 layers, 8192
    window, 512 consecutive fused steps (quantize-on-append + attention, every
    layer, every stream) across the first wrap (positions 7936 .. 8447) and 512
    across the second (16128 .. 16639), the rings fast-forwarded by planned
    appends in between.  After each run the whole cache of two streams (every
    layer, K and V) is bit-exact against the oracle's quantizer; attention of
    one stream's last layer within 1e-2 of the mimic every 64 steps."""
    ns, L, cap = 8, 26, 8192
    with vkv.Cache(n_streams=ns, n_layers=L, capacity=cap, dtype=vkv.Q8_0) as c:
        rings = (vkv.Ring * ns)(*[vkv.new_ring(cap) for _ in range(ns)])
        out = empty_f32(ns, L, 4096)
        pos = 0
        for first in (cap - 256, 2 * cap - 256):
            while pos < first:
                m = min(cap, first - pos)
                for s in range(ns):
                    prefill_by_append(c, rings[s], s, m, L)
                pos += m
            for step in range(512):
                q, k, v = step_inputs(c, [pos] * ns)
                plans = c.decoder_step(0, rings, [pos] * ns, 0, L, q.data_ptr(), k.data_ptr(),
                                       v.data_ptr(), out.data_ptr(), SCALE, hip_stream=stream_ptr())
                pos += 1
                if step % 64 == 63:
                    slots, q_row = plan_slots(plans[3]), q[3, L - 1].cpu().numpy()
                    got = out[3, L - 1].cpu().numpy().reshape(32, 128)
                    mimic = oracle_decode(c, 3, L - 1, slots, q_row, mimic=True)
                    assert np.max(np.abs(got - mimic)) <= TOL[vkv.Q8_0], (pos, step)
            assert all(rings[s].next_absolute_position == pos for s in range(ns))
            assert rings[0].wraps == pos // cap
            check_cache_state(c, [0, ns - 1], range(L), cap, {0: pos, ns - 1: pos})
            print(f"q8_0 8 streams: 512 steps up to position {pos - 1} ok (cache bit-exact, "
                  f"{rings[0].wraps} wraps)", flush=True)


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.F32, vkv.Q8_0])
def test_one_pass_full_ring(dtype):
    """26 layers x 8192 slots, one stream: F16 takes the whole-row kernel (a
    work group per (layer, 1024-slot chunk) + the merge), F32 and q8_0 the
    one-pass decode (one work group per (layer, kv head), no merge kernel).
    Three steps across the first wrap; cache bit-exact, attention against the
    oracle (F16: the full-window relation to fp64 and the mimic)."""
    with vkv.Cache(n_streams=1, n_layers=26, capacity=8192, dtype=dtype) as c:
        rings = (vkv.Ring * 1)(vkv.new_ring(8192))
        prefill_by_append(c, rings[0], 0, 8191, 26)
        out = empty_f32(1, 26, 4096)
        for pos in (8191, 8192, 8193):
            q, k, v = step_inputs(c, [pos])
            plans = c.decoder_step(0, rings, [pos], 0, 26, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
            check_cache_state(c, [0], [0, 25], 8192, {0: pos + 1})
            for layer in (0, 13, 25):
                slots, q_row = plan_slots(plans[0]), q[0, layer].cpu().numpy()
                got = out[0, layer].cpu().numpy().reshape(32, 128)
                mimic = oracle_decode(c, 0, layer, slots, q_row, mimic=True)
                exact = oracle_decode(c, 0, layer, slots, q_row)
                if dtype == vkv.F16:
                    check_full_window_f16(got, exact, mimic, (pos, layer),
                                          acc32=oracle_decode(c, 0, layer, slots, q_row, acc32=True))
                    continue
                assert np.max(np.abs(got - mimic)) <= TOL[dtype], (pos, layer)
                assert np.max(np.abs(got - exact)) <= EXACT_TOL[dtype], (pos, layer)
            print(f"one-pass {dtype} step {pos} ok", flush=True)


@pytest.mark.parametrize("rope", [False, True])
def test_whole_row_kernel_against_head_kernel(rope):
    """F16, 26 layers x 8192 slots: the default whole-row kernel (a work group
    per (layer, 1024-slot chunk) + the merge) and the per-head one-pass kernel
    (VKV_KERNEL_DECODE_HEADS) on the same steps across the first wrap: identical
    cache bytes, each within 1e-4 of the exact fp64 attention (both sit near
    3e-5; against the ggml mimic, whose f16 V accumulation is itself ~2e-3
    off here, both measure the same ~2.07e-3), and within 2e-4 of each other;
    with RoPE inside the step as well."""
    outs = {}
    for mode in ("default", "0"):
        flags = vkv.KERNEL_DECODE_HEADS if mode == "0" else 0
        with vkv.Cache(n_streams=1, n_layers=26, capacity=8192, dtype=vkv.F16,
                       kernel_flags=flags) as c:
            rings = (vkv.Ring * 1)(vkv.new_ring(8192))
            prefill_by_append(c, rings[0], 0, 8191, 26)
            out = empty_f32(1, 26, 4096)
            got = []
            for pos in (8191, 8192, 8193):
                q, k, v = step_inputs(c, [pos])
                if rope:
                    plans = c.decoder_step_rope(0, rings, [pos], 0, 26, q.data_ptr(), k.data_ptr(),
                                                v.data_ptr(), out.data_ptr(), SCALE, 1.0e6,
                                                hip_stream=stream_ptr())
                else:
                    plans = c.decoder_step(0, rings, [pos], 0, 26, q.data_ptr(), k.data_ptr(),
                                           v.data_ptr(), out.data_ptr(), SCALE,
                                           hip_stream=stream_ptr())
                torch.cuda.synchronize()
                got.append(out.cpu().numpy().copy())
                if not rope:
                    for layer in (0, 25):
                        slots, q_row = plan_slots(plans[0]), q[0, layer].cpu().numpy()
                        g = out[0, layer].cpu().numpy().reshape(32, 128)
                        assert np.max(np.abs(g - oracle_decode(c, 0, layer, slots, q_row))) <= 1e-4
            imgs = [layer_image(c, w, 0, layer).copy() for layer in (0, 12, 25) for w in (0, 1)]
        outs[mode] = (got, imgs)
    (ga, ia), (gb, ib) = outs["default"], outs["0"]
    for a, b in zip(ia, ib):
        assert np.array_equal(a, b)
    for a, b in zip(ga, gb):
        assert np.isfinite(a).all() and np.max(np.abs(a - b)) <= 2e-4


def ring_tuple(r):
    return (r.capacity, r.used, r.oldest_absolute_position, r.next_absolute_position, r.wraps,
            r.evictions, r.bytes_moved, r.full_buffer_moves)


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.Q8_0])
def test_clear_after_use_leaves_stale_slots_unreachable(dtype):
    """clear_kv_cache (src/voxtral.cpp:1590-1602), reached on every stream
    reset through voxtral_ctx_decoder_begin_incremental (:5489-5494), only
    resets the ring's metadata: the slots keep the previous stream's rows and
    reads stay bounded by `used`.  A 26 x 8192 ring is filled past its first
    wrap (the stale slots are non-zero), cleared, and stepped at positions
    0..3 with rows of another seed: attention equals the oracle over exactly
    the new keys, the image equals the pre-clear one with only the rewritten
    slots changed, and the metadata equals a fresh ring's after the same
    steps."""
    seed2 = SEED + 77
    layers = (0, 13, 25)
    with vkv.Cache(n_streams=1, n_layers=26, capacity=8192, dtype=dtype) as c:
        rings = (vkv.Ring * 1)(vkv.new_ring(8192))
        prefill_by_append(c, rings[0], 0, 8192, 26)
        prefill_by_append(c, rings[0], 0, 300, 26)      # positions 8192..8491: wrapped
        assert rings[0].wraps == 1 and rings[0].used == 8192
        before = {(w, l): layer_image(c, w, 0, l).copy() for l in layers for w in (0, 1)}
        assert all(np.any(img[:4 * int(c.row_bytes)]) for img in before.values())
        vkv.decoder_clear(rings[0], 8192)
        fresh = vkv.new_ring(8192)
        assert ring_tuple(rings[0]) == ring_tuple(fresh)
        out = empty_f32(1, 26, 4096)
        for pos in range(4):
            q, k, v = step_inputs(c, [pos], seed=seed2)
            plans = c.decoder_step(0, rings, [pos], 0, 26, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
            fplan = vkv.decoder_plan(fresh, pos, 1)
            vkv.decoder_commit(fresh, fplan)
            assert ring_tuple(rings[0]) == ring_tuple(fresh), pos
            slots = plan_slots(plans[0])
            assert list(slots) == list(range(pos + 1))
            for layer in layers:
                q_row = q[0, layer].cpu().numpy()
                got = out[0, layer].cpu().numpy().reshape(32, 128)
                exact = oracle_decode(c, 0, layer, slots, q_row)
                mimic = oracle_decode(c, 0, layer, slots, q_row, mimic=True)
                assert np.max(np.abs(got - exact)) <= EXACT_TOL[dtype], (pos, layer)
                assert np.max(np.abs(got - mimic)) <= TOL[dtype], (pos, layer)
        rb = int(c.row_bytes)
        for (w, l), img in before.items():
            new_rows = oracle.synth_rows(seed2, (vkv.TAG_K, vkv.TAG_V)[w], 0, l, range(4), c.kv_dim)
            want = img.copy()
            want[:4 * rb] = oracle.rows_from_f32(dtype, new_rows).view(np.uint8)
            assert np.array_equal(layer_image(c, w, 0, l), want), (w, l)


ROWS_CASES = {
    # streams x fills (the keys before the step); the kernel is forced with
    # VKV_KERNEL_DECODE_ROWS.  8 x 26: fill 1024 gives its stream a second,
    # one-slot chunk, so all 8 streams go through the partials and the merge
    # with empty second chunks (416 work groups); without it the grid is the
    # automatic range's 208 with direct output.
    "8x26_fills_le_1024": [0, 1, 2, 511, 1023, 1024, 700, 64],
    "8x26_one_chunk": [0, 1, 2, 511, 1023, 1000, 700, 64],          # direct output, 208 groups
    "2x26_empty_chunks": [1500, 3999],                             # stream 0: chunks 2, 3 empty
    "1x26_partial_last": [7200],                                   # chunk 7 holds 33 slots
}


def _rows_case_run(fills, flags, rope, dtype=vkv.F16):
    ns = len(fills)
    with vkv.Cache(n_streams=ns, n_layers=26, capacity=8192, dtype=dtype,
                   kernel_flags=flags) as c:
        rings = (vkv.Ring * ns)(*[vkv.new_ring(8192) for _ in range(ns)])
        for s, n in enumerate(fills):
            if n:
                prefill_by_append(c, rings[s], s, n, 26)
        q, k, v = step_inputs(c, fills)
        out = empty_f32(ns, 26, 4096)
        if rope:
            plans = c.decoder_step_rope(0, rings, fills, 0, 26, q.data_ptr(), k.data_ptr(),
                                        v.data_ptr(), out.data_ptr(), SCALE, 1.0e6,
                                        hip_stream=stream_ptr())
        else:
            plans = c.decoder_step(0, rings, fills, 0, 26, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), SCALE, hip_stream=stream_ptr())
        torch.cuda.synchronize()
        checks = []
        for s in range(ns):
            for layer in (0, 25):
                slots = plan_slots(plans[s])
                q_row = q[s, layer].cpu().numpy()
                if rope:
                    q_row = oracle.rope(q_row.reshape(1, 4096), 128, fills[s], 1.0e6)[0]
                got = out[s, layer].cpu().numpy().reshape(32, 128)
                checks.append((s, layer, got, oracle_decode(c, s, layer, slots, q_row),
                               oracle_decode(c, s, layer, slots, q_row, mimic=True)))
        imgs = [layer_image(c, w, s, l).copy() for s in range(ns) for l in (0, 25) for w in (0, 1)]
        return out.cpu().numpy(), imgs, checks


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("case", sorted(ROWS_CASES))
def test_whole_row_kernel_streams_and_partial_chunks(case, rope):
    """The whole-row F16 decode on the shapes its automatic choice covers
    beyond the one-stream headline: 8 streams at fills up to one chunk (the
    direct-output path, including a stream with no earlier keys) and with one
    stream a slot past it (every stream merged over an empty chunk), 2 streams
    whose shorter window leaves chunks empty (their -inf partials in the
    merge), and one stream whose last chunk is partial.  Against the oracle
    (exact and mimic) and against the per-head kernel on identical caches:
    identical cache bytes, outputs within 1e-3 (each kernel rounds the
    softmax weights to f16 against its own running maxima)."""
    fills = ROWS_CASES[case]
    out_r, img_r, checks = _rows_case_run(fills, vkv.KERNEL_DECODE_ROWS, rope)
    out_h, img_h, _ = _rows_case_run(fills, vkv.KERNEL_DECODE_HEADS, rope)
    for a, b in zip(img_r, img_h):
        assert np.array_equal(a, b)
    # both kernels round each softmax weight to f16 for the P.V products
    # relative to their own running maxima (different chunkings), so on
    # windows of a few keys with |v| ~ 2 they differ by a few 1e-4
    d_kernels = float(np.max(np.abs(out_r - out_h)))
    assert np.isfinite(out_r).all() and d_kernels <= 1e-3
    worst = np.zeros(3)
    for s, layer, got, exact, mimic in checks:
        bound = F16_FULL_EXACT if fills[s] + 1 > 1024 else TOL[vkv.F16]
        errs = check_full_window_f16(got, exact, mimic, (case, s, layer), bound)
        worst = np.maximum(worst, errs[:3])
    print(f"whole rows {case} rope={rope} ok: |rows-heads| {d_kernels:.2e}, |rows-fp64| "
          f"{worst[0]:.2e}, |mimic-fp64| {worst[1]:.2e}, |rows-mimic| {worst[2]:.2e}", flush=True)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("case", sorted(ROWS_CASES))
def test_q8_0_whole_row_kernel_streams_and_partial_chunks(case, rope):
    """The q8_0 whole-row decode (VKV_KERNEL_DECODE_ROWS: rows streamed flat
    into LDS, re-packed, the matrix-core arithmetic of the per-head kernel)
    on the same cases, against the oracle (mimic 1e-2, exact 3e-2) and
    against the default per-head matrix-core kernel on identical caches:
    identical cache bytes (the fused append quantizes the new row the same
    way), outputs within 5e-3 (the two round p * d_v to f16 against
    different running maxima)."""
    fills = ROWS_CASES[case]
    out_r, img_r, checks = _rows_case_run(fills, vkv.KERNEL_DECODE_ROWS, rope, vkv.Q8_0)
    out_h, img_h, _ = _rows_case_run(fills, vkv.KERNEL_DECODE_HEADS, rope, vkv.Q8_0)
    for a, b in zip(img_r, img_h):
        assert np.array_equal(a, b)
    d_kernels = float(np.max(np.abs(out_r - out_h)))
    assert np.isfinite(out_r).all() and d_kernels <= 5e-3
    worst = np.zeros(2)
    for s, layer, got, exact, mimic in checks:
        e_mimic = float(np.max(np.abs(got - mimic)))
        e_exact = float(np.max(np.abs(got - exact)))
        assert e_mimic <= TOL[vkv.Q8_0] and e_exact <= EXACT_TOL[vkv.Q8_0], (s, layer, e_mimic, e_exact)
        worst = np.maximum(worst, (e_mimic, e_exact))
    print(f"q8_0 whole rows {case} rope={rope} ok: |rows-heads| {d_kernels:.2e}, "
          f"|rows-mimic| {worst[0]:.2e}, |rows-fp64| {worst[1]:.2e}", flush=True)


@pytest.mark.parametrize("fill", [1, 36, 1024, 8191])
def test_q8_0_per_layer_call_in_ggml_query_arithmetic(fill):
    """A one-layer q8_0 step (the decoder's per-layer call: chunks of at most
    1024 slots) runs the VALU kernel in ggml's q8_0 arithmetic throughout: the
    query quantized per block as the cache is, exact block integer sums scaled
    by d_k d_q, V dequantised to f32 and accumulated in f32.  Against the ggml
    mimic (the same roundings, a per-key online softmax) within 5e-6 at
    windows of 2 to 8192 keys (measured 3e-7 .. 6e-7: the exp and summation
    orders); the matrix-core kernels, which round p * d_v to f16, are held to
    1e-2."""
    with vkv.Cache(n_streams=1, n_layers=1, capacity=8192, dtype=vkv.Q8_0) as c:
        ring = vkv.new_ring(8192)
        prefill_by_append(c, ring, 0, fill, 1)
        q, k, v = step_inputs(c, [fill], n_layers=1)
        out = empty_f32(1, 1, 4096)
        rings = (vkv.Ring * 1)(ring)
        plans = c.decoder_step(0, rings, [fill], 0, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               out.data_ptr(), SCALE, hip_stream=stream_ptr())
        torch.cuda.synchronize()
        slots = plan_slots(plans[0])
        q_row = q[0, 0].cpu().numpy()
        got = out[0, 0].cpu().numpy().reshape(32, 128)
        mimic = oracle_decode(c, 0, 0, slots, q_row, mimic=True)
        exact = oracle_decode(c, 0, 0, slots, q_row)
        d = float(np.max(np.abs(got - mimic)))
        assert np.isfinite(got).all() and d <= 5e-6, (fill, d)
        assert np.max(np.abs(got - exact)) <= EXACT_TOL[vkv.Q8_0]
        print(f"q8_0 per-layer call, {fill + 1} keys: |gpu - ggml mimic| {d:.2e}", flush=True)
