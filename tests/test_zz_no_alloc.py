"""The allocation-free decoder token, vkv_decoder_token_noalloc, whose
workspace is the library's static per-GPU scratch array, against
vkv_decoder_token with a workspace the caller allocated: two calls in a row
on one GPU, the second with a smaller model (narrower residual stream, FFN and
vocabulary, one layer), so the scratch still holds the first call's bytes when
the second starts.  Each call runs on its own copy of an identically filled
cache: logits bit for bit, the greedy token, the ring and the cache bytes
identical.  A model whose workspace exceeds the array is rejected before any
device work."""
import ctypes

import numpy as np
import pytest
import torch

import vkv
from gpu_util import dev, layer_image, stream_ptr, synth
from kq_util import random_matrix

pytestmark = pytest.mark.gpu

QH, KVH, HD = 32, 8, 128
QD, KD = QH * HD, KVH * HD
THETA, EPS = 1.0e6, 1e-5


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def device_model(rng, n_layers, dim, hidden, vocab):
    """random Q4_K / Q6_K decoder weights on the device + the vkv_dec_model"""
    keep = []

    def d(a):
        t = to_dev(a)
        keep.append(t)
        return t.data_ptr()

    arr = (vkv.DecLayer * n_layers)()
    for i in range(n_layers):
        arr[i] = vkv.DecLayer(
            d(rng.uniform(0.5, 1.5, dim).astype(np.float32)),
            d(random_matrix(rng, vkv.Q4_K, QD, dim, 0.005)),
            d(random_matrix(rng, vkv.Q4_K, KD, dim, 0.005)),
            d(random_matrix(rng, vkv.Q6_K, KD, dim, 0.1)),
            d(random_matrix(rng, vkv.Q4_K, dim, QD, 0.005)),
            vkv.Q4_K, vkv.Q4_K, vkv.Q6_K, vkv.Q4_K,
            d(rng.uniform(0.5, 1.5, dim).astype(np.float32)),
            d(rng.uniform(-0.3, 0.3, dim).astype(np.float32)),
            d(random_matrix(rng, vkv.Q4_K, hidden, dim, 0.003)),
            d(random_matrix(rng, vkv.Q6_K, dim, hidden, 0.05)),
            d(random_matrix(rng, vkv.Q4_K, hidden, dim, 0.003)),
            vkv.Q4_K, vkv.Q6_K, vkv.Q4_K)
    table = d(random_matrix(rng, vkv.Q6_K, vocab, dim, 0.5))
    model = vkv.DecModel(n_layers, dim, hidden, QH, KVH, HD, vocab, EPS, THETA, table, vkv.Q6_K,
                         d(rng.uniform(0.5, 1.5, dim).astype(np.float32)), table, vkv.Q6_K, arr)
    return model, (keep, arr)


def filled_cache(n_layers, capacity, n_pos):
    cache = vkv.Cache(n_streams=1, n_layers=n_layers, capacity=capacity, n_kv_heads=KVH,
                      head_dim=HD, n_q_heads=QH, dtype=vkv.F16)
    ring = vkv.new_ring(capacity)
    pos = 0
    while pos < n_pos:
        n = min(capacity, n_pos - pos)
        plan = vkv.decoder_plan(ring, pos, n)
        k = synth(None, KD, vkv.TAG_K, nl=n_layers, p0=pos, np_=n)
        v = synth(None, KD, vkv.TAG_V, nl=n_layers, p0=pos, np_=n)
        cache.append(0, 0, n_layers, vkv.plan_segs(plan.write_seg, plan.write_nseg), k.data_ptr(),
                     v.data_ptr(), hip_stream=stream_ptr())
        vkv.decoder_commit(ring, plan)
        pos += n
    torch.cuda.synchronize()
    return cache, ring


def ring_tuple(r):
    return (r.capacity, r.used, r.oldest_absolute_position, r.next_absolute_position, r.wraps,
            r.evictions, r.bytes_moved, r.full_buffer_moves)


# (layers, dim, hidden, vocab, ring capacity, positions already in the ring, token)
CALLS = [(2, 3072, 9216, 4096, 512, 700, 1234),
         (1, 1024, 2048, 1000, 256, 300, 777)]


def test_noalloc_token_equals_workspace_token_twice_second_smaller():
    rng = np.random.default_rng(20261202)
    sp = stream_ptr()
    sizes = []
    for n_layers, dim, hidden, vocab, cap, n_pos, token in CALLS:
        print(f"no-alloc token: {n_layers} layers, dim {dim}, hidden {hidden}, vocab {vocab}",
              flush=True)
        model, keep = device_model(rng, n_layers, dim, hidden, vocab)
        ws_bytes = vkv.decoder_token_workspace(model)
        assert 0 < ws_bytes <= vkv.TOKEN_SCRATCH_BYTES
        sizes.append(ws_bytes)
        audio = to_dev((rng.standard_normal(dim) * 0.1).astype(np.float32))
        ca, ra = filled_cache(n_layers, cap, n_pos)
        cb, rb = filled_cache(n_layers, cap, n_pos)
        ws = torch.empty(ws_bytes // 4 + 64, device=dev())
        ws_ptr = (ws.data_ptr() + 255) & ~255
        la = torch.full((vocab,), np.nan, device=dev())
        lb = torch.full((vocab,), np.nan, device=dev())
        ta = torch.full((1,), -1, dtype=torch.int32, device=dev())
        tb = torch.full((1,), -1, dtype=torch.int32, device=dev())
        pa = vkv.decoder_token(ca, 0, ra, model, token, audio.data_ptr(), la.data_ptr(),
                               ta.data_ptr(), ws_ptr, ws_bytes, hip_stream=sp)
        pb = vkv.decoder_token_noalloc(cb, 0, rb, model, token, audio.data_ptr(), lb.data_ptr(),
                                       tb.data_ptr(), hip_stream=sp)
        assert np.array_equal(host(la).view(np.uint32), host(lb).view(np.uint32))
        assert np.isfinite(host(lb)).all()
        assert int(host(ta)[0]) == int(host(tb)[0]) and 0 <= int(host(tb)[0]) < vocab
        assert ring_tuple(ra) == ring_tuple(rb) and rb.next_absolute_position == n_pos + 1
        assert bytes(pa) == bytes(pb)
        for layer in range(n_layers):
            for which in (0, 1):
                assert np.array_equal(layer_image(ca, which, 0, layer), layer_image(cb, which, 0, layer))
        ca.close()
        cb.close()
        del keep
    assert sizes[1] < sizes[0]


def test_noalloc_rejects_a_model_beyond_the_scratch():
    """hidden 262144: the FFN row alone fills the 1 MiB array; rejected with
    BUFFER_TOO_SMALL before the cache or any device is touched."""
    arr = (vkv.DecLayer * 1)()
    arr[0] = vkv.DecLayer(*([256] * 5), vkv.Q4_K, vkv.Q4_K, vkv.Q6_K, vkv.Q4_K, 256, None, 256,
                          256, 256, vkv.Q4_K, vkv.Q6_K, vkv.Q4_K)
    model = vkv.DecModel(1, 3072, 262144, QH, KVH, HD, 1000, EPS, THETA, 256, vkv.Q6_K, 256, 256,
                         vkv.Q6_K, arr)
    assert vkv.decoder_token_workspace(model) > vkv.TOKEN_SCRATCH_BYTES
    plan = vkv.Plan()
    plan.n_new = 9
    ring = vkv.new_ring(64)
    st = vkv.lib.vkv_decoder_token_noalloc(None, 0, ctypes.byref(ring), ctypes.byref(model), 0,
                                           None, 256, 256, ctypes.byref(plan), None)
    assert st == vkv.BUFFER_TOO_SMALL
    assert "static scratch" in vkv.last_error() and plan.n_new == 0
    assert ring.next_absolute_position == 0
