"""The oracle's attention functions, pinned without the reference (ggml is not
vendored): exact fp64 attention against torch's scaled_dot_product_attention in
float64 on the CPU, closed forms (all-equal scores -> mean of V, one key -> its
value), permutation equivariance (why attending over the physical ring after a
wrap equals the logical order, src/voxtral.cpp:2801-2807), the GQA head map,
and the ggml-mimic reduction order against the exact result; the mimic's
closed-form pins hold for its scalar form and for the baseline's vector leg
(AVX2/FMA/F16C) alike.  CPU only."""
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


# ---------------------------------------------------------------------------
# Closed forms that pin the roundings which separate ggml's CPU flash
# attention (the mimic) from the exact result: the f16 V accumulator, Q
# rounded to f16 against an F16 K, and Q quantized to q8_0 blocks against a
# q8_0 K (integer block sums).  Each case is built so that the plausible
# alternative (f32 accumulator, unrounded Q, f16 Q against q8_0 K) lands
# many ulp away from the closed form.
# ---------------------------------------------------------------------------

def _ulps(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


def _f32(x):
    return np.float32(x)


LEGS = ["scalar", pytest.param("vector", marks=pytest.mark.skipif(
    not oracle.simd_available(), reason="host lacks AVX2/FMA/F16C"))]


def mimic(leg, dtype, kimg, vimg, rb, n, q, scale):
    """the mimic over slots [0, n): the scalar restatement, or the CPU
    baseline's vector leg (one layer of the threaded step, no append)"""
    if leg == "scalar":
        return oracle.decode_attn_mimic(dtype, kimg, vimg, rb, np.arange(n, dtype=np.int32), q, G,
                                        D, scale)
    _, out = oracle.decode_step_mimic_mt(dtype, kimg, vimg, len(kimg), rb, 1, n, q.reshape(1, -1),
                                         H, G, D, scale, 4, simd=True)
    return out[0]


@pytest.mark.parametrize("leg", LEGS)
def test_mimic_f16_accumulator_stalls_at_2048(leg):
    """4096 keys with equal scores (K = 0) and V = 1.0 everywhere: ggml adds
    each weight 1.0 into an f16 accumulator, which stops growing at 2048
    (2049 is a tie that rounds to even, 2048), while the weight sum S reaches
    4096 in f32; the output is exactly 0.5.  An f32 accumulator would give
    exactly 1.0, the exact attention 1.0."""
    n = 4096
    kimg, _ = make_layer(oracle.F16, np.zeros((n, KV), np.float32))
    vimg, _ = make_layer(oracle.F16, np.ones((n, KV), np.float32))
    q = np.random.default_rng(3).standard_normal((H, D)).astype(np.float32)
    rb = oracle.row_bytes(oracle.F16, KV)
    slots = np.arange(n, dtype=np.int32)
    mi = mimic(leg, oracle.F16, kimg, vimg, rb, n, q, 1 / np.sqrt(D))
    assert np.all(mi == np.float32(0.5))
    ex = oracle.decode_attn_f64(oracle.F16, kimg, vimg, rb, slots, q, G, D, 1 / np.sqrt(D))
    assert np.all(ex == 1.0)
    # below the stall every partial sum is an exact f16 integer
    mi = mimic(leg, oracle.F16, kimg, vimg, rb, 2048, q, 0.1)
    assert np.all(mi == np.float32(1.0))


# q values at f16 midpoints (ties) and just off them: RNE decides each
MIDPOINTS = [1 + 2 ** -11,          # tie -> 1.0 (even)
             1 + 3 * 2 ** -11,      # tie -> 1 + 2^-9 (even mantissa 2)
             2049.0 / 2048,         # 1 + 2^-11 again, written differently
             1.5 + 2 ** -11,        # tie -> 1.5 (mantissa 512, even)
             0.75 + 2 ** -12,       # tie below 1 -> 0.75
             0.75 + 3 * 2 ** -12,   # tie -> 0.75 + 2^-10
             1 + 2 ** -11 + 2 ** -20,  # just above a tie -> rounds up
             1.25 - 2 ** -12]       # tie -> 1.25 (mantissa 256, even)


@pytest.mark.parametrize("leg", LEGS)
def test_mimic_rounds_q_to_f16_against_f16_k(leg):
    """Two keys: key 0 has K = 1.0 in dimension 0 of every kv head and V = 1.0
    in dimension 0; key 1 has K = 0 and V = 1.0 in dimension 1.  Query head h
    holds a value q_h at or near an f16 midpoint in dimension 0 and zeros
    elsewhere.  ggml's CPU path converts Q to f16 (RNE) for the F16 K dot,
    so with s = scale * f16(q_h), w = expf(-s), S = 1 + w:
        out[h][0] = 1 / S,   out[h][1] = f16(w) / S   (f16 V accumulator)."""
    scale = 1.0
    krows = np.zeros((2, KV), np.float32)
    vrows = np.zeros((2, KV), np.float32)
    for g in range(G):
        krows[0, g * D] = 1.0
        vrows[0, g * D] = 1.0
        vrows[1, g * D + 1] = 1.0
    kimg, _ = make_layer(oracle.F16, krows)
    vimg, _ = make_layer(oracle.F16, vrows)
    q = np.zeros((H, D), np.float32)
    for h in range(H):
        q[h, 0] = MIDPOINTS[h % len(MIDPOINTS)] * (1 + h // len(MIDPOINTS))
    rb = oracle.row_bytes(oracle.F16, KV)
    mi = mimic(leg, oracle.F16, kimg, vimg, rb, 2, q, scale)
    for h in range(H):
        qh = oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(q[h, :1]))[0]
        assert qh == np.float16(q[h, 0]).astype(np.float32)         # numpy's RNE agrees
        s = _f32(_f32(qh) * _f32(scale))
        w = _f32(np.exp(-np.float64(s)))
        S = _f32(_f32(1.0) + w)
        inv = _f32(_f32(1.0) / S)
        want0 = inv
        want1 = _f32(np.float32(np.float16(w)) * inv)
        assert _ulps(mi[h, 0], want0) <= 2, h
        assert _ulps(mi[h, 1], want1) <= 2, h
        assert np.all(mi[h, 2:] == 0)
        # unrounded Q would move out[h][0] far beyond those 2 ulp when the
        # midpoint actually rounds
        if np.float32(q[h, 0]) != qh:
            s_alt = _f32(q[h, 0] * scale)
            alt = _f32(_f32(1.0) / _f32(_f32(1.0) + _f32(np.exp(-np.float64(s_alt)))))
            assert _ulps(alt, want0) >= 50, h
        # an f32 accumulator would keep w unrounded in out[h][1]
        assert _ulps(_f32(w * inv), want1) >= 50, h


@pytest.mark.parametrize("leg", LEGS)
def test_mimic_quantizes_q_to_q8_0_against_q8_0_k(leg):
    """Two keys over a q8_0 cache.  Key 0: block 0 of every kv head holds 1.0
    in all 32 places (codes 127, d_k = f16(1/127)); V has 1.0 in dimension 0.
    Key 1: K = 0, V = 1.0 in dimension 1.  Query block 0 is
    (127 c, c/2, ..., c/2) with c = 2^-6: its q8_0 form has d_q = c and codes
    (127, 1, ..., 1) (0.5 rounds half away from zero), so the score is the
    integer block sum 127*127 + 31*127 = 20066 times d_k*d_q, not the f16 dot
    product (which would weigh the 31 halves at 0.5)."""
    scale = 0.5
    krows = np.zeros((2, KV), np.float32)
    vrows = np.zeros((2, KV), np.float32)
    for g in range(G):
        krows[0, g * D:g * D + 32] = 1.0
        vrows[0, g * D] = 1.0
        vrows[1, g * D + 1] = 1.0
    kimg, _ = make_layer(oracle.Q8_0, krows)
    vimg, vst = make_layer(oracle.Q8_0, vrows)
    c = 2.0 ** -6
    q = np.zeros((H, D), np.float32)
    q[:, 0] = 127 * c
    q[:, 1:32] = c / 2
    blk = oracle.q8_0_quantize(q[0, :32])
    assert blk[2] == 127 and all(int(np.int8(b)) == 1 for b in blk[3:34])
    dk = oracle.f16_bits_to_f32(np.frombuffer(kimg[0:2].tobytes(), np.uint16))[0]
    assert dk == np.float32(np.float16(np.float32(1.0) / np.float32(127.0)))
    rb = oracle.row_bytes(oracle.Q8_0, KV)
    mi = mimic(leg, oracle.Q8_0, kimg, vimg, rb, 2, q, scale)
    v0 = np.float32(vst[0, 0])
    s = _f32(_f32(_f32(20066) * _f32(dk * _f32(c))) * _f32(scale))
    w = _f32(np.exp(-np.float64(s)))
    inv = _f32(_f32(1.0) / _f32(_f32(1.0) + w))
    want0 = _f32(v0 * inv)
    assert np.all(_ulps(mi[:, 0], want0) <= 2)
    # the f16 dot product of the unquantized Q would give a different score
    kdq = np.float32(127) * dk
    s_alt = _f32(_f32(np.float32(np.float16(127 * c)) * kdq + 31 * np.float32(np.float16(c / 2)) * kdq)
                 * _f32(scale))
    alt = _f32(v0 * _f32(_f32(1.0) / _f32(_f32(1.0) + _f32(np.exp(-np.float64(s_alt))))))
    assert _ulps(alt, want0) >= 1000


@pytest.mark.skipif(not oracle.simd_available(), reason="host lacks AVX2/FMA/F16C")
@pytest.mark.parametrize("dtype,tol", [(oracle.F32, 1e-6), (oracle.F16, 2e-4), (oracle.Q8_0, 1e-6)])
def test_vector_leg_against_scalar_mimic(dtype, tol):
    """The baseline's vector leg computes the mimic's function: two layers of
    1025 seeded keys, with the step's append of a new row at slot 700 first,
    within tol of the scalar step (only the K-row sum order differs: 8 lanes x
    4 f32 accumulators against one double sum; for F16 the per-key f16 V
    accumulator turns those differences into f16 ulps of the partial sums)."""
    L, n = 2, 1025
    rb = oracle.row_bytes(dtype, KV)
    imgs = [np.concatenate([oracle.expected_layer(dtype, n, n, KV, n, 11, tag, 0, l)
                            for l in range(L)]) for tag in (oracle.TAG_K, oracle.TAG_V)]
    rng = np.random.default_rng(int(dtype) + 5)
    q = rng.standard_normal((L, H * D)).astype(np.float32)
    kn = rng.standard_normal((L, KV)).astype(np.float32)
    vn = rng.standard_normal((L, KV)).astype(np.float32)
    outs = []
    for simd in (False, True):
        k, v = imgs[0].copy(), imgs[1].copy()
        _, o = oracle.decode_step_mimic_mt(dtype, k, v, rb * n, rb, L, n, q, H, G, D, 1 / np.sqrt(D),
                                           3, k_new=kn, v_new=vn, new_slot=700, simd=simd)
        outs.append(o)
    assert np.max(np.abs(outs[0] - outs[1])) <= tol


# ---------------------------------------------------------------------------
# The encoder's window attention in the reference's ggml CPU arithmetic
# (src/voxtral.cpp:2259-2281, fewer than 32 query rows): mul_mat of each K
# segment with the query (converted to f16 against an F16 ring), soft_max_ext
# in f32, mul_mat of each V^T segment with the weights (converted to f16
# against an F16 ring).  The closed forms below fail when either conversion
# is dropped; an F32 ring converts nothing.
# ---------------------------------------------------------------------------

EH, ED = 2, 64


def _enc_layer(dtype, krows, vrows):
    kimg, _ = make_layer(dtype, krows)
    vimg, _ = make_layer(dtype, vrows)
    return kimg, vimg, oracle.row_bytes(dtype, EH * ED)


def _two_key_closed_form(dtype, q, krows, vrows, scale):
    """ggml's manual softmax over keys 0 and 1 for one head: (out0, out1) where
    V0 = e_0 and V1 = e_1, so out_d = conv(p_d)"""
    f16 = lambda x: np.float32(np.float16(np.float32(x)))  # noqa: E731  (RNE, as numpy rounds)
    qc = np.array([f16(x) for x in q], np.float32) if dtype == oracle.F16 else q
    s = [np.float32(np.dot(krows[j, :ED].astype(np.float64), qc.astype(np.float64)))
         for j in range(2)]
    w = [_f32(sj * _f32(scale)) for sj in s]
    m = max(w)
    e = [_f32(np.exp(np.float64(_f32(wj - m)))) for wj in w]
    inv = _f32(1.0 / (np.float64(e[0]) + np.float64(e[1])))
    p = [_f32(ej * inv) for ej in e]
    return [f16(pj) if dtype == oracle.F16 else pj for pj in p], p, s


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.F32])
def test_window_mimic_rounds_weights_to_f16(dtype):
    """Two keys, K0 = a e_0, K1 = 0, V0 = e_0, V1 = e_1, queries e_0 (exact in
    f16): the softmax weights p0 = 1/(1+exp(-a/8)), p1 = 1 - p0 are not f16
    values, and an F16 ring's output is f16(p0), f16(p1) exactly, where the
    unrounded weights sit many ulp away; an F32 ring returns p0 and p1."""
    n_q = 12
    krows = np.zeros((2, EH * ED), np.float32)
    vrows = np.zeros((2, EH * ED), np.float32)
    for g in range(EH):
        vrows[0, g * ED] = 1.0
        vrows[1, g * ED + 1] = 1.0
    outs = []
    for i in range(n_q):
        a = 0.37 + 0.53 * i
        for g in range(EH):
            krows[0, g * ED] = a
        kimg, vimg, rb = _enc_layer(dtype, krows, vrows)
        a16 = np.float32(oracle.rows_to_f32(dtype, kimg, EH * ED)[0, 0])
        q = np.zeros((1, EH, ED), np.float32)
        q[0, :, 0] = 1.0
        got = oracle.window_attn_mimic(dtype, kimg, vimg, rb, np.array([0, 1]), np.array([0, 1]),
                                       q, np.array([1]), EH, EH, ED, 750, 0.125)
        kr = np.zeros((2, EH * ED), np.float32)
        kr[0, 0] = a16
        want, unrounded, _ = _two_key_closed_form(dtype, q[0, 0], kr, vrows, 0.125)
        for h in range(EH):
            assert _ulps(got[0, h, 0], want[0]) <= 1 and _ulps(got[0, h, 1], want[1]) <= 1, (i, h)
            assert np.all(got[0, h, 2:] == 0)
        if dtype == oracle.F16:
            outs.append(max(_ulps(unrounded[0], want[0]), _ulps(unrounded[1], want[1])))
    if dtype == oracle.F16:
        assert min(outs) >= 20      # the f32 weights are never f16 values here


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.F32])
def test_window_mimic_rounds_q_to_f16(dtype):
    """K0 = e_0, K1 = e_1, V0 = e_0, V1 = e_1, query (q0, 300, 0, ...) with q0
    near 300 off the f16 grid (ulp 0.25 there): against an F16 ring the
    scores are f16(q0) and 300, so q0 = 300.1 scores a tie and both outputs
    are exactly 0.5; unrounded, p0 = sigmoid(0.0125) = 0.5031, whose f16 is
    0.50293.  An F32 ring keeps q0."""
    krows = np.zeros((2, EH * ED), np.float32)
    vrows = np.zeros((2, EH * ED), np.float32)
    for g in range(EH):
        krows[0, g * ED] = 1.0
        krows[1, g * ED + 1] = 1.0
        vrows[0, g * ED] = 1.0
        vrows[1, g * ED + 1] = 1.0
    kimg, vimg, rb = _enc_layer(dtype, krows, vrows)
    q0s = [300.1, 300.2, 299.9, 300.05, 299.8, 300.37]
    q = np.zeros((len(q0s), EH, ED), np.float32)
    for i, q0 in enumerate(q0s):
        q[i, :, 0] = q0
        q[i, :, 1] = 300.0
    q_pos = np.arange(1, 1 + len(q0s))
    got = oracle.window_attn_mimic(dtype, kimg, vimg, rb, np.array([0, 1]), np.array([0, 1]), q,
                                   q_pos, EH, EH, ED, 750, 0.125)
    moved = 0
    for i in range(len(q0s)):
        want, _, _ = _two_key_closed_form(dtype, q[i, 0], krows, vrows, 0.125)
        # the same with the query left in f32
        alt, _, _ = _two_key_closed_form(oracle.F32, q[i, 0], krows, vrows, 0.125)
        alt = [np.float32(np.float16(x)) for x in alt] if dtype == oracle.F16 else alt
        for h in range(EH):
            assert _ulps(got[i, h, 0], want[0]) <= 1 and _ulps(got[i, h, 1], want[1]) <= 1, (i, h)
        if dtype == oracle.F16:
            moved += int(_ulps(alt[0], want[0]) >= 1000)
    if dtype == oracle.F16:
        assert got[0, 0, 0] == np.float32(0.5) and got[0, 0, 1] == np.float32(0.5)
        assert moved == len(q0s)      # every q0 here leaves the f16 grid by >= 0.05
    else:
        assert abs(float(got[0, 0, 0]) - 1 / (1 + np.exp(-0.0125))) < 1e-6


@pytest.mark.parametrize("dtype,tol", [(oracle.F16, 2e-3), (oracle.F32, 1e-5)])
def test_window_mimic_within_tolerance_of_exact(dtype, tol):
    """At the encoder's shape (32 heads x 64, window 750, a 16-frame block at
    q_start 2000 over a wrapped 878-slot ring) the reference's CPU arithmetic
    stays within the acceptance tolerance of exact attention; its distance is
    what the GPU tile is compared against."""
    rng = np.random.default_rng(2259 + dtype)
    H_, D_, cap, win, P, q_start = 32, 64, 878, 750, 16, 2000
    kimg, _ = make_layer(dtype, rng.standard_normal((cap, H_ * D_)).astype(np.float32))
    vimg, _ = make_layer(dtype, rng.standard_normal((cap, H_ * D_)).astype(np.float32))
    k_pos = np.arange(q_start - (win - 1), q_start + P, dtype=np.int64)
    k_slot = (k_pos % cap).astype(np.int32)
    q_pos = np.arange(q_start, q_start + P, dtype=np.int64)
    q = rng.standard_normal((P, H_, D_)).astype(np.float32)
    rb = oracle.row_bytes(dtype, H_ * D_)
    ex = oracle.window_attn_f64(dtype, kimg, vimg, rb, k_slot, k_pos, q, q_pos, H_, H_, D_, win, 0.125)
    mi = oracle.window_attn_mimic(dtype, kimg, vimg, rb, k_slot, k_pos, q, q_pos, H_, H_, D_, win,
                                  0.125)
    d = float(np.max(np.abs(mi - ex)))
    assert d < tol
    if dtype == oracle.F16:
        assert d > 1e-5       # the two f16 conversions are visible at this size
    # the flash form (32+ rows) is the decode mimic over each query's keys
    fl = oracle.window_attn_mimic(dtype, kimg, vimg, rb, k_slot, k_pos, q[:2], q_pos[:2], H_, H_,
                                  D_, win, 0.125, flash=True)
    for i in range(2):
        sl = k_slot[(k_pos <= q_pos[i]) & (k_pos >= q_pos[i] - (win - 1))]
        want = oracle.decode_attn_mimic(dtype, kimg, vimg, rb, sl, q[i].reshape(-1), H_, D_, 0.125)
        assert np.array_equal(fl[i], want)


def test_decode_mimic_acc32_differs_only_by_the_accumulator():
    """The f32-accumulator mimic keeps every other rounding: at the stall case
    (4096 equal weights of V = 1) it gives exactly 1.0 where the mimic gives
    0.5, and for an F32 cache (no f16 accumulator) both are the same bits."""
    n = 4096
    kimg, _ = make_layer(oracle.F16, np.zeros((n, KV), np.float32))
    vimg, _ = make_layer(oracle.F16, np.ones((n, KV), np.float32))
    q = np.random.default_rng(3).standard_normal((H, D)).astype(np.float32)
    rb = oracle.row_bytes(oracle.F16, KV)
    slots = np.arange(n, dtype=np.int32)
    a32 = oracle.decode_attn_mimic_acc32(oracle.F16, kimg, vimg, rb, slots, q, G, D, 1 / np.sqrt(D))
    assert np.all(a32 == np.float32(1.0))
    rng = np.random.default_rng(8)
    kimg, _ = make_layer(oracle.F32, rng.standard_normal((300, KV)).astype(np.float32))
    vimg, _ = make_layer(oracle.F32, rng.standard_normal((300, KV)).astype(np.float32))
    rb = oracle.row_bytes(oracle.F32, KV)
    sl = np.arange(300, dtype=np.int32)
    assert np.array_equal(oracle.decode_attn_mimic(oracle.F32, kimg, vimg, rb, sl, q, G, D, 0.09),
                          oracle.decode_attn_mimic_acc32(oracle.F32, kimg, vimg, rb, sl, q, G, D, 0.09))
