"""Helpers shared by the GPU parity tests: device buffers (torch is only the
allocator), synthetic inputs generated on the device by the product's
generator, cache images read back through the C ABI, and the oracle's expected
images and attention for comparison."""
import hashlib

import numpy as np
import torch

import oracle
import vkv

SEED = 20261201
DEC = dict(n_layers=26, capacity=8192, n_kv_heads=8, head_dim=128, n_q_heads=32)
ENC = dict(n_layers=32, capacity=878, n_kv_heads=32, head_dim=64, n_q_heads=32, window=750)


def dev():
    return torch.device("cuda:0")


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


def empty_f32(*shape):
    return torch.empty(*shape, dtype=torch.float32, device=dev())


def synth(shape_rows, row_len, tag, s0=0, ns=1, l0=0, nl=1, p0=0, np_=1, seed=SEED):
    """device f32 tensor [ns, nl, np_, row_len] of seeded rows"""
    t = empty_f32(ns, nl, np_, row_len)
    vkv.synth_rows(t.data_ptr(), row_len, seed, tag, s0=s0, ns=ns, l0=l0, nl=nl, p0=p0, np_=np_,
                   hip_stream=stream_ptr())
    return t


def step_inputs(cache, positions, layer0=0, n_layers=None, seed=SEED, tags=(vkv.TAG_Q, vkv.TAG_K, vkv.TAG_V)):
    """q [ns][nl][H*D], k/v [ns][nl][kv_dim] for one decode step per stream."""
    nl = n_layers or cache.n_layers
    ns = len(positions)
    q = empty_f32(ns, nl, cache.n_q_heads * cache.head_dim)
    k = empty_f32(ns, nl, cache.kv_dim)
    v = empty_f32(ns, nl, cache.kv_dim)
    for s, p in enumerate(positions):
        for t, tag, rl in ((q, tags[0], cache.n_q_heads * cache.head_dim), (k, tags[1], cache.kv_dim),
                           (v, tags[2], cache.kv_dim)):
            vkv.synth_rows(t[s].data_ptr(), rl, seed, tag, s0=s, ns=1, l0=layer0, nl=nl, p0=p,
                           np_=1, hip_stream=stream_ptr())
    return q, k, v


def layer_image(cache, which, stream, layer):
    torch.cuda.synchronize()
    return np.frombuffer(cache.read_rows(which, stream, layer, 0, cache.capacity), dtype=np.uint8)


def expected_image(cache, which, stream, layer, ring_capacity, next_pos, seed=SEED, tags=(vkv.TAG_K, vkv.TAG_V)):
    return oracle.expected_layer(cache.dtype, cache.capacity, ring_capacity, cache.kv_dim, next_pos,
                                 seed, tags[which], stream, layer)


def sha(b):
    return hashlib.sha256(np.ascontiguousarray(b).tobytes()).hexdigest()


def oracle_decode(cache, stream, layer, slots, q_row, mimic=False, acc32=False):
    """exact fp64 attention, the ggml mimic, or (acc32) the mimic with an f32
    V accumulator"""
    kimg = layer_image(cache, 0, stream, layer)
    vimg = layer_image(cache, 1, stream, layer)
    scale = 1.0 / np.sqrt(cache.head_dim)
    fn = (oracle.decode_attn_mimic_acc32 if acc32 else
          oracle.decode_attn_mimic if mimic else oracle.decode_attn_f64)
    return fn(cache.dtype, kimg, vimg, int(cache.row_bytes), np.asarray(slots, np.int32), q_row,
              cache.n_kv_heads, cache.head_dim, scale)


def plan_slots(plan):
    """physical slots of the plan's logical window, oldest -> newest"""
    out = []
    for i in range(plan.read_nseg):
        out.extend(range(plan.read_seg[i].slot, plan.read_seg[i].slot + plan.read_seg[i].len))
    return np.asarray(out, dtype=np.int32)
