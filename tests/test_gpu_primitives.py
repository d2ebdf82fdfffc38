"""GPU parity of the primitive kernels against the oracle, bit-exact:
synthetic generator, append (F16 RNE / F32 / q8_0) through <=2 write segments,
ring gather, q8_0 pack/unpack."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import SEED, empty_f32, layer_image, stream_ptr, synth

pytestmark = pytest.mark.gpu

DTYPES = [vkv.F16, vkv.F32, vkv.Q8_0]


def edge_rows(n, kv_dim, rng):
    """N(0,1) rows with f16 edge cases mixed in: ties, subnormals, overflow."""
    x = rng.standard_normal((n, kv_dim)).astype(np.float32)
    codes = rng.integers(0, 0x7BFF, size=n * kv_dim // 4).astype(np.uint16)
    lo = codes.view(np.float16).astype(np.float64)
    hi = (codes + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32) * np.where(rng.random(codes.size) < 0.5, -1, 1)
    flat = x.reshape(-1)
    flat[: ties.size] = ties
    specials = np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 7e4, -7e4, 2.0 ** -24, 2.0 ** -25,
                         3 * 2.0 ** -26, 1e-30, 6.1e-5, -6.1e-5], dtype=np.float32)
    flat[ties.size: ties.size + specials.size] = specials
    rng.shuffle(flat)
    return x


def test_synth_matches_oracle_generator():
    t = synth(None, 1024, vkv.TAG_K, s0=2, ns=2, l0=3, nl=3, p0=1000, np_=4)
    torch.cuda.synchronize()
    got = t.cpu().numpy()
    for i in range(2):
        for j in range(3):
            for k in range(4):
                want = oracle.synth_row(SEED, vkv.TAG_K, 2 + i, 3 + j, 1000 + k, 1024)
                assert np.array_equal(got[i, j, k], want)


@pytest.mark.parametrize("dtype", DTYPES)
def test_append_bit_exact_with_wrap(dtype):
    rng = np.random.default_rng(dtype + 1)
    kv_dim, backing, cap, layers = 1024, 40, 32, 3
    with vkv.Cache(n_streams=2, n_layers=layers, capacity=backing, n_kv_heads=8, head_dim=128,
                   n_q_heads=32, dtype=dtype) as c:
        rb = int(c.row_bytes)
        imgs = {(w, l): np.zeros(backing * rb, np.uint8) for w in (0, 1) for l in range(layers)}
        ring = vkv.new_ring(cap)
        pos = 0
        for n in (5, 20, 13, 32, 1, 7):
            plan = vkv.decoder_plan(ring, pos, n)
            segs = vkv.plan_segs(plan.write_seg, plan.write_nseg)
            k = edge_rows(layers * n, kv_dim, rng).reshape(layers, n, kv_dim)
            v = edge_rows(layers * n, kv_dim, rng).reshape(layers, n, kv_dim)
            kd, vd = torch.from_numpy(k).to("cuda"), torch.from_numpy(v).to("cuda")
            c.append(1, 0, layers, segs, kd.data_ptr(), vd.data_ptr(), hip_stream=stream_ptr())
            for l in range(layers):
                oracle.append(dtype, imgs[(0, l)], rb, kv_dim, segs, k[l])
                oracle.append(dtype, imgs[(1, l)], rb, kv_dim, segs, v[l])
            vkv.decoder_commit(ring, plan)
            pos += n
            for (w, l), want in imgs.items():
                got = layer_image(c, w, 1, l)
                assert np.array_equal(got, want), (n, w, l)
            # stream 0 untouched
            assert not layer_image(c, 0, 0, 0).any()


@pytest.mark.parametrize("dtype", DTYPES)
def test_gather_bit_exact(dtype):
    kv_dim, backing = 1024, 64
    rng = np.random.default_rng(5)
    with vkv.Cache(n_streams=1, n_layers=2, capacity=backing, dtype=dtype) as c:
        rb = int(c.row_bytes)
        k = rng.standard_normal((2, backing, kv_dim)).astype(np.float32)
        v = rng.standard_normal((2, backing, kv_dim)).astype(np.float32)
        kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
        c.append(0, 0, 2, [(0, backing)], kd.data_ptr(), vd.data_ptr(), hip_stream=stream_ptr())
        img_k = layer_image(c, 0, 0, 1)
        img_v = layer_image(c, 1, 0, 1)
        for segs in ([(10, 30)], [(50, 14), (0, 20)], [(63, 1), (0, 63)], [(0, 64)], []):
            n = sum(s[1] for s in segs)
            out_k = torch.zeros(max(n * rb, 16), dtype=torch.uint8, device="cuda")
            out_v = torch.zeros(max(n * rb, 16), dtype=torch.uint8, device="cuda")
            c.gather(0, 1, segs, out_k.data_ptr(), out_v.data_ptr(), hip_stream=stream_ptr())
            torch.cuda.synchronize()
            assert np.array_equal(out_k.cpu().numpy()[: n * rb], oracle.gather(img_k, rb, segs))
            assert np.array_equal(out_v.cpu().numpy()[: n * rb], oracle.gather(img_v, rb, segs))


def test_q8_0_pack_unpack_bit_exact():
    rng = np.random.default_rng(9)
    n = 32 * 5000
    x = (rng.standard_normal(n) * rng.uniform(1e-4, 1e4, n // 32).repeat(32)).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [0.0] * 24, np.float32)
    xd = torch.from_numpy(x).cuda()
    blocks = torch.zeros(n // 32 * 34, dtype=torch.uint8, device="cuda")
    vkv.q8_0_pack(xd.data_ptr(), blocks.data_ptr(), n, hip_stream=stream_ptr())
    y = empty_f32(n)
    vkv.q8_0_unpack(blocks.data_ptr(), y.data_ptr(), n, hip_stream=stream_ptr())
    torch.cuda.synchronize()
    want = oracle.q8_0_quantize(x)
    assert np.array_equal(blocks.cpu().numpy(), want)
    assert np.array_equal(y.cpu().numpy(), oracle.q8_0_dequantize(want, n))


def test_cache_is_zero_at_creation_and_after_zero():
    with vkv.Cache(n_streams=1, n_layers=2, capacity=16, dtype=vkv.F16) as c:
        assert not layer_image(c, 0, 0, 1).any()
        k = torch.ones(2, 16, c.kv_dim, device="cuda")
        c.append(0, 0, 2, [(0, 16)], k.data_ptr(), k.data_ptr(), hip_stream=stream_ptr())
        assert layer_image(c, 1, 0, 1).any()
        c.zero(hip_stream=stream_ptr())
        assert not layer_image(c, 1, 0, 1).any()


def test_invalid_arguments_leave_cache_untouched():
    with vkv.Cache(n_streams=1, n_layers=1, capacity=16, dtype=vkv.F16) as c:
        k = torch.ones(1, 16, c.kv_dim, device="cuda")
        for segs in ([(10, 7)], [(0, 8), (4, 9)], [(-1, 2)]):
            with pytest.raises(vkv.VkvError) as ei:
                c.append(0, 0, 1, segs, k.data_ptr(), k.data_ptr(), hip_stream=stream_ptr())
            assert ei.value.status == vkv.INVALID_ARGUMENT
        with pytest.raises(vkv.VkvError):
            c.append(0, 0, 1, [(0, 1)], k.data_ptr() + 4, k.data_ptr(), hip_stream=stream_ptr())
        with pytest.raises(vkv.VkvError):
            c.append(0, 1, 1, [(0, 1)], k.data_ptr(), k.data_ptr(), hip_stream=stream_ptr())
        assert not layer_image(c, 0, 0, 0).any()
