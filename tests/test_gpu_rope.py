"""GPU parity of the decoder's RoPE (ggml_rope_ext mode 0, src/voxtral.cpp:
2667-2671): the standalone kernel against the oracle, and the decode step with
RoPE fused in against the unfused step fed with rotated rows -- cache bytes and
attention outputs identical -- and against the oracle."""
import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import SEED, empty_f32, layer_image, oracle_decode, plan_slots, stream_ptr, synth

pytestmark = pytest.mark.gpu

THETA, D = 1.0e6, 128
SCALE = 1.0 / np.sqrt(128.0)


def assert_nearly_identical(got, want):
    """equal up to a rare last-ulp difference of cos/sin (double on the GPU
    and on the host, rounded to f32)"""
    diff = got != want
    assert diff.mean() <= 1e-5
    if diff.any():
        rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-30)
        assert rel.max() <= 4e-7


@pytest.mark.parametrize("pos0", [0, 1, 8191, 30000, (1 << 24) - 64])
def test_rope_kernel_matches_oracle(pos0):
    x = synth(None, 4096, vkv.TAG_Q, nl=3, p0=0, np_=64)          # [1][3][64][4096]
    host = x.cpu().numpy().reshape(3, 64, 4096)
    vkv.rope(x.data_ptr(), 3, 64, 4096, D, pos0, THETA, hip_stream=stream_ptr())
    torch.cuda.synchronize()
    want = oracle.rope(host, D, pos0, THETA)
    assert_nearly_identical(x.cpu().numpy().reshape(3, 64, 4096), want)


@pytest.mark.parametrize("dtype", [vkv.F16, vkv.Q8_0])
def test_fused_rope_step_equals_rope_then_step(dtype):
    L, cap = 26, 8192
    caches = [vkv.Cache(n_streams=1, n_layers=L, capacity=cap, dtype=dtype) for _ in range(2)]
    try:
        rings = [(vkv.Ring * 1)(vkv.new_ring(cap)) for _ in range(2)]
        for c, r in zip(caches, rings):
            plan = vkv.decoder_plan(r[0], 0, cap - 1)
            k = synth(None, 1024, vkv.TAG_K, nl=L, p0=0, np_=cap - 1)
            v = synth(None, 1024, vkv.TAG_V, nl=L, p0=0, np_=cap - 1)
            c.append(0, 0, L, vkv.plan_segs(plan.write_seg, plan.write_nseg), k.data_ptr(),
                     v.data_ptr(), hip_stream=stream_ptr())
            vkv.decoder_commit(r[0], plan)
        for pos in (cap - 1, cap, cap + 1):
            q = synth(None, 4096, vkv.TAG_Q, nl=L, p0=pos, np_=1)    # [1][L][1][4096]
            k = synth(None, 1024, vkv.TAG_K, nl=L, p0=pos, np_=1)
            v = synth(None, 1024, vkv.TAG_V, nl=L, p0=pos, np_=1)
            q_pre, k_pre = q.cpu().numpy().reshape(L, 4096), k.cpu().numpy().reshape(L, 1024)
            out_a, out_b = empty_f32(1, L, 4096), empty_f32(1, L, 4096)
            plans = caches[0].decoder_step_rope(0, rings[0], [pos], 0, L, q.data_ptr(), k.data_ptr(),
                                                v.data_ptr(), out_a.data_ptr(), SCALE, THETA,
                                                hip_stream=stream_ptr())
            q_rot, k_rot = q.clone(), k.clone()
            vkv.rope(q_rot.data_ptr(), L, 1, 4096, D, pos, THETA, hip_stream=stream_ptr())
            vkv.rope(k_rot.data_ptr(), L, 1, 1024, D, pos, THETA, hip_stream=stream_ptr())
            caches[1].decoder_step(0, rings[1], [pos], 0, L, q_rot.data_ptr(), k_rot.data_ptr(),
                                   v.data_ptr(), out_b.data_ptr(), SCALE, hip_stream=stream_ptr())
            torch.cuda.synchronize()
            assert torch.equal(out_a, out_b), pos
            for layer in (0, 12, 25):
                for w in (0, 1):
                    assert np.array_equal(layer_image(caches[0], w, 0, layer),
                                          layer_image(caches[1], w, 0, layer)), (pos, layer, w)
            # the stored K row is the oracle's rotation of the projected row
            slot = pos % cap
            rb = int(caches[0].row_bytes)
            for layer in (0, 25):
                want = np.frombuffer(oracle.rows_from_f32(dtype, oracle.rope(k_pre[layer:layer + 1], D, pos, THETA)), np.uint8)
                got = np.frombuffer(caches[0].read_rows(0, 0, layer, slot, 1), np.uint8)
                assert np.array_equal(got, want) or dtype == vkv.Q8_0 and np.mean(got != want) < 0.01
                q_row = oracle.rope(q_pre[layer:layer + 1], D, pos, THETA)[0]
                exact = oracle_decode(caches[0], 0, layer, plan_slots(plans[0]), q_row)
                got_o = out_a[0, layer].cpu().numpy().reshape(32, 128)
                assert np.max(np.abs(got_o - exact)) <= (2e-3 if dtype == vkv.F16 else 3e-2)
            print(f"fused rope {dtype} step {pos} ok", flush=True)
    finally:
        for c in caches:
            c.close()
