"""The oracle's attention functions, pinned without the reference (ggml is not
vendored): exact fp64 attention against torch's scaled_dot_product_attention in
float64 on the CPU, closed forms (all-equal scores -> mean of V, one key -> its
value), permutation equivariance (why attending over the physical ring after a
wrap equals the logical order, src/voxtral.cpp:2801-2807), the GQA head map,
and the ggml-mimic reduction order against the exact result.  CPU only."""
import numpy as np
import pytest
import torch

import oracle

D, G, H = 128, 8, 32
KV = G * D


def make_layer(dtype, rows):
    """cache image of one layer from f32 rows [n, kv_dim] and the rows as stored"""
    img = oracle.rows_from_f32(dtype, rows)
    return img, oracle.rows_to_f32(dtype, img, rows.shape[1]).astype(np.float64)


def sdpa_ref(q, kst, vst, slots, n_q_heads, n_kv_heads, head_dim, scale, mask=None):
    """torch SDPA in float64; q [n_q, H, D], kst/vst [slots, kv_dim] as stored."""
    grp = n_q_heads // n_kv_heads
    k = torch.from_numpy(kst[slots]).view(len(slots), n_kv_heads, head_dim).permute(1, 0, 2)
    v = torch.from_numpy(vst[slots]).view(len(slots), n_kv_heads, head_dim).permute(1, 0, 2)
    k = k.repeat_interleave(grp, dim=0).contiguous()
    v = v.repeat_interleave(grp, dim=0).contiguous()
    qt = torch.from_numpy(np.asarray(q, dtype=np.float64)).permute(1, 0, 2).contiguous()
    out = torch.nn.functional.scaled_dot_product_attention(
        qt.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), attn_mask=mask, scale=scale)
    return out[0].permute(1, 0, 2).numpy()


@pytest.mark.parametrize("dtype", [oracle.F32, oracle.F16, oracle.Q8_0])
@pytest.mark.parametrize("n", [1, 37, 1025])
def test_decode_f64_matches_sdpa(dtype, n):
    rng = np.random.default_rng(n)
    cap = n + 11
    kimg, kst = make_layer(dtype, rng.standard_normal((cap, KV)).astype(np.float32))
    vimg, vst = make_layer(dtype, rng.standard_normal((cap, KV)).astype(np.float32))
    q = rng.standard_normal((H, D)).astype(np.float32)
    slots = rng.permutation(cap)[:n].astype(np.int32)
    rb = oracle.row_bytes(dtype, KV)
    got = oracle.decode_attn_f64(dtype, kimg, vimg, rb, slots, q, G, D, 1 / np.sqrt(D))
    want = sdpa_ref(q[None], kst, vst, slots, H, G, D, 1 / np.sqrt(D))[0]
    assert np.max(np.abs(got - want)) < 1e-12


def test_closed_forms():
    rng = np.random.default_rng(0)
    n = 300
    vrows = rng.standard_normal((n, KV)).astype(np.float32)
    vimg, vst = make_layer(oracle.F16, vrows)
    kimg, _ = make_layer(oracle.F16, np.zeros((n, KV), np.float32))
    q = rng.standard_normal((H, D)).astype(np.float32)
    rb = oracle.row_bytes(oracle.F16, KV)
    slots = np.arange(n, dtype=np.int32)
    out = oracle.decode_attn_f64(oracle.F16, kimg, vimg, rb, slots, q, G, D, 0.088)
    mean = vst.mean(axis=0).reshape(G, D)
    assert np.max(np.abs(out - np.repeat(mean, H // G, axis=0))) < 1e-12   # equal scores
    one = oracle.decode_attn_f64(oracle.F16, kimg, vimg, rb, slots[7:8], q, G, D, 0.088)
    assert np.array_equal(one, np.repeat(vst[7].reshape(G, D), H // G, axis=0))  # one key
    assert np.all(oracle.decode_attn_f64(oracle.F16, kimg, vimg, rb, slots[:0], q, G, D, 1.0) == 0)


def test_permutation_equivariance_and_gqa_map():
    rng = np.random.default_rng(1)
    n = 500
    kimg, _ = make_layer(oracle.F16, rng.standard_normal((n, KV)).astype(np.float32))
    vimg, _ = make_layer(oracle.F16, rng.standard_normal((n, KV)).astype(np.float32))
    q = rng.standard_normal((H, D)).astype(np.float32)
    rb = oracle.row_bytes(oracle.F16, KV)
    slots = np.arange(n, dtype=np.int32)
    a = oracle.decode_attn_f64(oracle.F16, kimg, vimg, rb, slots, q, G, D, 0.088)
    rolled = np.roll(slots, 123)   # a wrapped ring read in physical order
    b = oracle.decode_attn_f64(oracle.F16, kimg, vimg, rb, rolled, q, G, D, 0.088)
    assert np.max(np.abs(a - b)) < 1e-13
    # perturb KV head 3 only: exactly query heads 12..15 change
    v2 = vimg.copy().reshape(n, -1)
    v2[:, 3 * D * 2:4 * D * 2] = 0
    c = oracle.decode_attn_f64(oracle.F16, kimg, v2.ravel(), rb, slots, q, G, D, 0.088)
    changed = np.any(a != c, axis=1)
    assert list(np.nonzero(changed)[0]) == [12, 13, 14, 15]


@pytest.mark.parametrize("dtype,tol", [(oracle.F32, 1e-5), (oracle.F16, 2e-3), (oracle.Q8_0, 1e-2)])
@pytest.mark.parametrize("n", [1025, 8192])
def test_mimic_within_tolerance_of_exact(dtype, tol, n):
    """ggml's reduction order (f16 Q, per-key online softmax, f16 V accumulator,
    q8_0 Q for q8_0 K) stays within the acceptance tolerance of the exact
    result on N(0,1) inputs at the decode shapes."""
    rng = np.random.default_rng(n + dtype)
    kimg, _ = make_layer(dtype, rng.standard_normal((n, KV)).astype(np.float32))
    vimg, _ = make_layer(dtype, rng.standard_normal((n, KV)).astype(np.float32))
    q = rng.standard_normal((H, D)).astype(np.float32)
    rb = oracle.row_bytes(dtype, KV)
    slots = np.arange(n, dtype=np.int32)
    ex = oracle.decode_attn_f64(dtype, kimg, vimg, rb, slots, q, G, D, 1 / np.sqrt(D))
    mi = oracle.decode_attn_mimic(dtype, kimg, vimg, rb, slots, q, G, D, 1 / np.sqrt(D))
    assert np.max(np.abs(ex - mi)) < tol


def test_mimic_exact_on_integer_sums():
    """All-equal scores and small-integer V: the f16 accumulator is exact, so
    the mimic returns exactly sum(V)/n."""
    n = 64
    rng = np.random.default_rng(5)
    vrows = rng.integers(-8, 8, size=(n, KV)).astype(np.float32)
    vimg, _ = make_layer(oracle.F16, vrows)
    kimg, _ = make_layer(oracle.F16, np.zeros((n, KV), np.float32))
    q = rng.standard_normal((H, D)).astype(np.float32)
    rb = oracle.row_bytes(oracle.F16, KV)
    mi = oracle.decode_attn_mimic(oracle.F16, kimg, vimg, rb, np.arange(n, dtype=np.int32), q, G, D, 0.1)
    want = (vrows.sum(axis=0, dtype=np.float64).astype(np.float32) * np.float32(1 / n)).reshape(G, D)
    assert np.array_equal(mi, np.repeat(want, H // G, axis=0))


@pytest.mark.parametrize("dtype", [oracle.F32, oracle.F16])
def test_window_f64_matches_masked_sdpa(dtype):
    """Encoder sliding window (MHA, head_dim 64, window 750) and the causal
    decoder prefill both reduce to SDPA with a boolean mask."""
    rng = np.random.default_rng(11)
    # encoder: 32 heads x 64, ring of 878, 16 queries at q_start=2000
    EH, ED, cap, win = 32, 64, 878, 750
    kimg, kst = make_layer(dtype, rng.standard_normal((cap, EH * ED)).astype(np.float32))
    vimg, vst = make_layer(dtype, rng.standard_normal((cap, EH * ED)).astype(np.float32))
    q_start, P = 2000, 16
    k_pos = np.arange(q_start - (win - 1), q_start + P, dtype=np.int64)
    k_slot = (k_pos % cap).astype(np.int32)
    q_pos = np.arange(q_start, q_start + P, dtype=np.int64)
    q = rng.standard_normal((P, EH, ED)).astype(np.float32)
    rb = oracle.row_bytes(dtype, EH * ED)
    got = oracle.window_attn_f64(dtype, kimg, vimg, rb, k_slot, k_pos, q, q_pos, EH, EH, ED, win, 0.125)
    mask = torch.from_numpy(np.array([[oracle.enc_mask_allows(int(k), int(qq), win) for k in k_pos]
                                      for qq in q_pos]))
    want = sdpa_ref(q, kst, vst, k_slot, EH, EH, ED, 0.125, mask=mask.unsqueeze(0))
    assert np.max(np.abs(got - want)) < 1e-12
    # decoder prefill: 38 tokens at positions 0..37, GQA 32/8, causal
    n = 38
    kimg, kst = make_layer(dtype, rng.standard_normal((n, KV)).astype(np.float32))
    vimg, vst = make_layer(dtype, rng.standard_normal((n, KV)).astype(np.float32))
    q = rng.standard_normal((n, H, D)).astype(np.float32)
    pos = np.arange(n, dtype=np.int64)
    got = oracle.window_attn_f64(dtype, kimg, vimg, oracle.row_bytes(dtype, KV), pos.astype(np.int32),
                                 pos, q, pos, H, G, D, 0, 1 / np.sqrt(D))
    mask = torch.tril(torch.ones(n, n, dtype=torch.bool))
    want = sdpa_ref(q, kst, vst, np.arange(n), H, G, D, 1 / np.sqrt(D), mask=mask.unsqueeze(0))
    assert np.max(np.abs(got - want)) < 1e-12
