"""GPU parity of the decoder prefill of a prompt (run_decoder_prefill,
src/voxtral.cpp:5161-5213; graph build_decoder_prefill_graph :2893-2961,
layers build_decoder_layer :2629-2887):

  * vkv_decoder_prompt equals the entry points it composes called one by one
    (per-token embedding + audio row, multi-row products, vkv_rope,
    vkv_decoder_prefill per layer under one plan, last-row logits and
    argmax), bit for bit: logits, token, cache bytes, ring, residual rows;
  * every stage of that sequence matches the oracle's restatement of ggml's
    CPU path fed with the stage's own input (Q8_K products, RoPE, f16 K/V
    rows, causal attention in fp64), and the whole prompt matches the
    oracle's composition end to end;
  * the prompt at the stream start (positions 0..37, the reference's case),
    after a wrapped ring with evictions and an audio ring that wraps, and a
    prompt longer than one embedding launch;
  * argument errors leave the ring untouched.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import test_gpu_decoder_token as tok
import vkv
from gpu_util import dev, layer_image, stream_ptr

pytestmark = pytest.mark.gpu

DIM, HID, QH, KVH, HD = tok.DIM, tok.HID, tok.QH, tok.KVH, tok.HD
QD, KD = tok.QD, tok.KD
THETA, EPS, SCALE = tok.THETA, tok.EPS, tok.SCALE
host, to_dev, ring_tuple = tok.host, tok.to_dev, tok.ring_tuple


def rel(got, want):
    want = np.asarray(want, np.float64)
    return np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30)


def nearly_identical(got, want):
    diff = got != want
    assert diff.mean() <= 1e-5
    if diff.any():
        assert (np.abs(got - want) / np.maximum(np.abs(want), 1e-30)).max() <= 4e-7


def rows_matvec(dtype, w, n_rows, n_in, xs):
    return np.stack([oracle.matvec(dtype, w, n_rows, n_in, x, 8) for x in xs])


def copy_ring(r):
    c = vkv.Ring()
    ctypes.pointer(c)[0] = r
    return c


def audio_ring(rng, capacity, pos0, n):
    """a device rows ring of width DIM whose logical rows pos0 .. pos0+n-1
    hold random audio rows; returns (RowRing, tensor, rows[n][DIM])"""
    rows = (rng.standard_normal((n, DIM)) * 0.1).astype(np.float32)
    t = torch.full((capacity, DIM), np.nan, device=dev())
    ring = vkv.RowRing(t.data_ptr(), capacity, DIM)
    src = to_dev(rows)
    vkv.row_ring_write(ring, pos0, src.data_ptr(), n, hip_stream=stream_ptr())
    torch.cuda.synchronize()
    return ring, t, rows


def composed_prompt(cache, ring, model, tokens, aring, logits, tok_out, sp, m=None):
    """The entry points vkv_decoder_prompt composes, one by one; with m (the
    numpy weights) every stage is checked against the oracle's stage fed with
    this run's own input."""
    n = len(tokens)
    pos0 = ring.next_absolute_position
    plan = vkv.decoder_plan(ring, pos0, n)
    x = torch.empty(n, DIM, device=dev())
    q, k, v = (torch.empty(n, w, device=dev()) for w in (QD, KD, KD))
    attn = torch.empty(n, QD, device=dev())
    ffn = torch.empty(n, HID, device=dev())
    ws_b = vkv.matmul_workspace(n, HID)
    ws = torch.empty(ws_b // 4 + 64, device=dev())
    wp = (ws.data_ptr() + 255) & ~255
    row_b = int(cache.row_bytes)
    q_pos = np.arange(pos0, pos0 + n)
    for i, t in enumerate(tokens):
        a_ptr = None
        if aring is not None:
            a_ptr = aring.rows + ((pos0 + i) % aring.capacity) * DIM * 4
        vkv.embed(model.tok_embeddings_type, model.tok_embeddings, model.vocab, DIM, t,
                  x[i].data_ptr(), a_ptr, hip_stream=sp)
    xp = x.data_ptr()
    for layer in range(model.n_layers):
        L = model.layers[layer]
        x_in = host(x) if m else None
        vkv.matmul(xp, n, DIM, [(L.attn_q, L.attn_q_type, QD, q.data_ptr()),
                                (L.attn_k, L.attn_k_type, KD, k.data_ptr()),
                                (L.attn_v, L.attn_v_type, KD, v.data_ptr())],
                   wp, ws_b, norm_w_ptr=L.attn_norm, eps=EPS, hip_stream=sp)
        if m:
            M = m["layers"][layer]
            hs = [oracle.norm_act(x_in[p], M["attn_norm"], None, EPS) for p in range(n)]
            q_in, k_in, v_in = host(q), host(k), host(v)
            assert rel(q_in, rows_matvec(L.attn_q_type, M["attn_q"], QD, DIM, hs)) < 2e-6
            assert rel(k_in, rows_matvec(L.attn_k_type, M["attn_k"], KD, DIM, hs)) < 2e-6
            assert rel(v_in, rows_matvec(L.attn_v_type, M["attn_v"], KD, DIM, hs)) < 2e-6
        vkv.rope(q.data_ptr(), 1, n, QD, HD, pos0, THETA, hip_stream=sp)
        vkv.rope(k.data_ptr(), 1, n, KD, HD, pos0, THETA, hip_stream=sp)
        # every layer plans from the same ring state; the commit comes last
        cache.decoder_prefill(0, copy_ring(ring), layer, 1, n, q.data_ptr(), k.data_ptr(),
                              v.data_ptr(), attn.data_ptr(), SCALE, hip_stream=sp)
        if m:
            # RoPE: the oracle's up to a rare last ulp of cos/sin; the cached
            # rows are the f16 of this run's rotated k and of v, bit for bit
            qr, kr = host(q), host(k)
            nearly_identical(qr, oracle.rope(q_in, HD, pos0, THETA))
            nearly_identical(kr, oracle.rope(k_in, HD, pos0, THETA))
            kimg, vimg = layer_image(cache, 0, 0, layer), layer_image(cache, 1, 0, layer)
            for i in range(n):
                s = (pos0 + i) % ring.capacity
                assert np.array_equal(kimg[s * row_b:(s + 1) * row_b],
                                      np.frombuffer(oracle.rows_from_f32(oracle.F16, kr[i]), np.uint8))
                assert np.array_equal(vimg[s * row_b:(s + 1) * row_b],
                                      np.frombuffer(oracle.rows_from_f32(oracle.F16, v_in[i]), np.uint8))
            key_pos = np.arange(max(0, pos0 + n - ring.capacity), pos0 + n)
            want = oracle.window_attn_f64(oracle.F16, kimg, vimg, row_b,
                                          (key_pos % ring.capacity).astype(np.int32), key_pos,
                                          qr.reshape(n, QH, HD), q_pos, QH, KVH, HD, 0, SCALE)
            a_got = host(attn)
            assert np.abs(a_got - want.reshape(n, QD)).max() <= 2e-3
            x_mid = host(x)
        vkv.matmul(attn.data_ptr(), n, QD, [(L.attn_o, L.attn_o_type, DIM, xp, xp)], wp, ws_b,
                   hip_stream=sp)
        if m:
            x_o = host(x)
            assert rel(x_o, x_mid + rows_matvec(L.attn_o_type, M["attn_o"], DIM, QD, a_got)) < 2e-6
        vkv.matmul(xp, n, DIM, [(L.ffn_w1, L.ffn_w1_type, HID, ffn.data_ptr()),
                                (L.ffn_w3, L.ffn_w3_type, HID, None)],
                   wp, ws_b, norm_w_ptr=L.ffn_norm, ada_ptr=L.ada_scale, eps=EPS,
                   epilogue=vkv.MV_SWIGLU, hip_stream=sp)
        if m:
            h2 = [oracle.norm_act(x_o[p], M["ffn_norm"], M["ada"], EPS) for p in range(n)]
            g = rows_matvec(L.ffn_w1_type, M["ffn_w1"], HID, DIM, h2)
            u = rows_matvec(L.ffn_w3_type, M["ffn_w3"], HID, DIM, h2)
            f_got = host(ffn)
            assert rel(f_got, oracle.silu(g).reshape(g.shape) * u) < 2e-6
        vkv.matmul(ffn.data_ptr(), n, HID, [(L.ffn_w2, L.ffn_w2_type, DIM, xp, xp)], wp, ws_b,
                   hip_stream=sp)
        if m:
            assert rel(host(x), x_o + rows_matvec(L.ffn_w2_type, M["ffn_w2"], DIM, HID, f_got)) < 2e-6
    vkv.matvec(x[n - 1].data_ptr(), DIM, [(model.output, model.output_type, model.vocab,
                                           logits.data_ptr())],
               norm_w_ptr=model.out_norm, eps=EPS, hip_stream=sp)
    vkv.argmax(logits.data_ptr(), model.vocab, tok_out.data_ptr(), hip_stream=sp)
    vkv.decoder_commit(ring, plan)
    return plan, x


def oracle_prompt(m, k_imgs, v_imgs, row_b, capacity, pos0, tokens, audio, exact=False):
    """ggml's CPU path for the whole prompt (oracle restatements throughout,
    the attention in ggml's flash-attention arithmetic, or exact with
    `exact`): the last token's logits and greedy token"""
    n = len(tokens)
    T = m["types"]
    rb = oracle.wrow_bytes(T["table"], DIM)
    x = np.stack([oracle.dequantize(T["table"], m["table"][t * rb:(t + 1) * rb], DIM)
                  for t in tokens])
    if audio is not None:
        x = x + audio
    q_pos = np.arange(pos0, pos0 + n)
    key_pos = np.arange(max(0, pos0 + n - capacity), pos0 + n)
    for layer, L in enumerate(m["layers"]):
        hs = [oracle.norm_act(x[p], L["attn_norm"], None, EPS) for p in range(n)]
        q = oracle.rope(rows_matvec(T["attn_q"], L["attn_q"], QD, DIM, hs), HD, pos0, THETA)
        k = oracle.rope(rows_matvec(T["attn_k"], L["attn_k"], KD, DIM, hs), HD, pos0, THETA)
        v = rows_matvec(T["attn_v"], L["attn_v"], KD, DIM, hs)
        ki, vi = k_imgs[layer].copy(), v_imgs[layer].copy()
        for i in range(n):
            s = (pos0 + i) % capacity
            ki[s * row_b:(s + 1) * row_b] = np.frombuffer(oracle.rows_from_f32(oracle.F16, k[i]), np.uint8)
            vi[s * row_b:(s + 1) * row_b] = np.frombuffer(oracle.rows_from_f32(oracle.F16, v[i]), np.uint8)
        # the prefill's attention as ggml's CPU flash attention computes it
        # (src/voxtral.cpp:2763-2773: the query rounded to f16 against the F16
        # cache, per-key online softmax, f16 V accumulator over the causal keys)
        attn_fn = oracle.window_attn_f64 if exact else oracle.window_attn_mimic
        kw = {} if exact else {"flash": True}
        attn = attn_fn(oracle.F16, ki, vi, row_b, (key_pos % capacity).astype(np.int32), key_pos,
                       q.reshape(n, QH, HD), q_pos, QH, KVH, HD, 0, SCALE, **kw)
        attn = attn.reshape(n, QD).astype(np.float32)
        x = x + rows_matvec(T["attn_o"], L["attn_o"], DIM, QD, attn)
        hs = [oracle.norm_act(x[p], L["ffn_norm"], L["ada"], EPS) for p in range(n)]
        g = rows_matvec(T["ffn_w1"], L["ffn_w1"], HID, DIM, hs)
        u = rows_matvec(T["ffn_w3"], L["ffn_w3"], HID, DIM, hs)
        f = (oracle.silu(g).reshape(g.shape) * u).astype(np.float32)
        x = x + rows_matvec(T["ffn_w2"], L["ffn_w2"], DIM, HID, f)
    xn = oracle.norm_act(x[-1], m["out_norm"], None, EPS)
    logits = oracle.matvec(T["table"], m["table"], m["vocab"], DIM, xn, 8)
    return logits, oracle.argmax(logits)


def empty_cache(n_layers, capacity):
    cache = vkv.Cache(n_streams=1, n_layers=n_layers, capacity=capacity, n_kv_heads=KVH,
                      head_dim=HD, n_q_heads=QH, dtype=vkv.F16)
    return cache, vkv.new_ring(capacity)


def workspace_for(model, n):
    b = vkv.decoder_prompt_workspace(model, n)
    assert b > 0
    ws = torch.empty(b // 4 + 64, device=dev())
    return ws, (ws.data_ptr() + 255) & ~255, b


# (cache capacity, positions already in the ring, prompt tokens, audio ring
# capacity or None, weight file kind)
CASES = [(512, 0, 38, 64, "q4km"),          # the stream prompt at positions 0..37
         (512, 986, 38, 48, "q4km"),        # after a wrap: evictions, the audio ring wraps too
         (512, 0, 1, 64, "q4km"),           # prompts of a few tokens: the normed products at the
         (512, 40, 3, 64, "q4km"),          # decoder's width 3072 take the separate input
         (512, 300, 5, 48, "q4km"),         # quantization (a prompt's window is one segment)
         (512, 0, 38, 64, "q8_0"),          # a Q8_0 file: every product on q8_0 images
         (512, 40, 3, 64, "q8_0")]


@pytest.mark.parametrize("cap,P,N,acap,kind", CASES)
def test_prompt_two_layers(cap, P, N, acap, kind):
    rng = np.random.default_rng(7100 + P)
    n_layers, vocab = 2, 4096
    m = tok.make_model(rng, n_layers, vocab, kind)
    model, keep, arr = tok.upload_model(m)
    tokens = [int(t) for t in rng.integers(0, vocab, N)]
    tokens[0], tokens[-1] = 0, vocab - 1
    aring, at, audio = audio_ring(rng, acap, P, N)
    sp = stream_ptr()
    if P:
        ca, ra = tok.filled_cache(n_layers, cap, P)
        cb, rb = tok.filled_cache(n_layers, cap, P)
    else:
        ca, ra = empty_cache(n_layers, cap)
        cb, rb = empty_cache(n_layers, cap)
        torch.cuda.synchronize()
    row_b = int(ca.row_bytes)
    k_imgs = [layer_image(ca, 0, 0, layer).copy() for layer in range(n_layers)]
    v_imgs = [layer_image(ca, 1, 0, layer).copy() for layer in range(n_layers)]

    ws, wp, wb = workspace_for(model, N)
    la = torch.empty(vocab, device=dev())
    ta = torch.zeros(1, dtype=torch.int32, device=dev())
    plan = vkv.decoder_prompt(ca, 0, ra, model, tokens, aring, la.data_ptr(), ta.data_ptr(), wp,
                              wb, hip_stream=sp)
    lb = torch.empty(vocab, device=dev())
    tb = torch.zeros(1, dtype=torch.int32, device=dev())
    plan_b, xb = composed_prompt(cb, rb, model, tokens, aring, lb, tb, sp, m)
    print(f"prompt cap={cap} P={P} N={N} {kind}: composed stages ok", flush=True)

    assert np.array_equal(host(la).view(np.uint32), host(lb).view(np.uint32))
    assert int(host(ta)[0]) == int(host(tb)[0])
    assert ring_tuple(ra) == ring_tuple(rb) and ra.next_absolute_position == P + N
    assert plan.absolute_start == plan_b.absolute_start == P and plan.n_new == N
    off = (wp - ws.data_ptr()) // 4
    assert np.array_equal(host(ws[off:off + N * DIM]).view(np.uint32),
                          host(xb).reshape(-1).view(np.uint32))
    for layer in range(n_layers):
        for which in (0, 1):
            assert np.array_equal(layer_image(ca, which, 0, layer), layer_image(cb, which, 0, layer))

    # end to end against ggml's CPU path: within 1% of the logit range plus
    # the spread between that arithmetic and exact attention through the same
    # layers (on prompts of a few tokens each query averages few keys, so the
    # f16 roundings of the attention, ggml's V accumulator or the GPU's
    # softmax weights, are not averaged away: 1.1% of the range at 3 tokens)
    got = host(la).astype(np.float64)
    want, want_tok = oracle_prompt(m, k_imgs, v_imgs, row_b, cap, P, tokens, audio)
    want_x, _ = oracle_prompt(m, k_imgs, v_imgs, row_b, cap, P, tokens, audio, exact=True)
    scale = np.abs(want).max()
    spread = np.abs(want.astype(np.float64) - want_x).max()
    err = np.abs(got - want).max()
    corr = np.corrcoef(got, want)[0, 1]
    print(f"prompt cap={cap} P={P} N={N} {kind}: end to end {err:.3f}, mimic-exact spread {spread:.3f}, "
          f"range {scale:.2f}", flush=True)
    assert err <= 1e-2 * scale + spread and corr > 0.9999, (err, scale, spread, corr)
    top2 = np.sort(want)[-2:]
    if top2[1] - top2[0] > 2 * err:
        assert int(host(ta)[0]) == want_tok
    ca.close()
    cb.close()
    del keep, arr, at


def test_prompt_longer_than_one_embedding_launch():
    """300 tokens (two embedding launches), no audio: the same bits as the
    composed sequence."""
    rng = np.random.default_rng(300)
    n_layers, vocab, cap, N = 1, 2048, 512, 300
    m = tok.make_model(rng, n_layers, vocab)
    model, keep, arr = tok.upload_model(m)
    tokens = [int(t) for t in rng.integers(0, vocab, N)]
    sp = stream_ptr()
    ca, ra = empty_cache(n_layers, cap)
    cb, rb = empty_cache(n_layers, cap)
    torch.cuda.synchronize()
    ws, wp, wb = workspace_for(model, N)
    la, lb = torch.empty(vocab, device=dev()), torch.empty(vocab, device=dev())
    ta = torch.zeros(1, dtype=torch.int32, device=dev())
    tb = torch.zeros(1, dtype=torch.int32, device=dev())
    vkv.decoder_prompt(ca, 0, ra, model, tokens, None, la.data_ptr(), ta.data_ptr(), wp, wb,
                       hip_stream=sp)
    _, xb = composed_prompt(cb, rb, model, tokens, None, lb, tb, sp)
    assert np.array_equal(host(la).view(np.uint32), host(lb).view(np.uint32))
    assert int(host(ta)[0]) == int(host(tb)[0])
    off = (wp - ws.data_ptr()) // 4
    assert np.array_equal(host(ws[off:off + N * DIM]).view(np.uint32),
                          host(xb).reshape(-1).view(np.uint32))
    for which in (0, 1):
        assert np.array_equal(layer_image(ca, which, 0, 0), layer_image(cb, which, 0, 0))
    assert ring_tuple(ra) == ring_tuple(rb)
    ca.close()
    cb.close()
    del keep, arr


def test_prompt_errors_leave_the_ring():
    rng = np.random.default_rng(11)
    n_layers, vocab, cap = 1, 1024, 64
    m = tok.make_model(rng, n_layers, vocab)
    model, keep, arr = tok.upload_model(m)
    cache, ring = tok.filled_cache(n_layers, cap, 40)
    before = ring_tuple(ring)
    ws, wp, wb = workspace_for(model, 30)
    lg = torch.empty(vocab, device=dev())
    to = torch.zeros(1, dtype=torch.int32, device=dev())
    aring, at, _ = audio_ring(rng, 64, 40, 30)

    def call(tokens, ar=aring, bytes_=wb):
        return vkv.decoder_prompt(cache, 0, ring, model, tokens, ar, lg.data_ptr(), to.data_ptr(),
                                  wp, bytes_, hip_stream=stream_ptr())

    with pytest.raises(vkv.VkvError, match="outside"):
        call([1, 2, vocab])                               # a token outside the vocabulary
    with pytest.raises(vkv.VkvError, match="outside"):
        call([-1])
    with pytest.raises(vkv.VkvError, match="one segment"):
        call([1] * 30)                                    # 40 + 30 > 64: the window wraps
    with pytest.raises(vkv.VkvError, match="width"):
        call([1, 2], ar=vkv.RowRing(aring.rows, 64, DIM - 256))
    with pytest.raises(vkv.VkvError) as e:
        call([1, 2], bytes_=1024)
    assert e.value.status == vkv.BUFFER_TOO_SMALL
    with pytest.raises(vkv.VkvError):
        call([])
    assert ring_tuple(ring) == before
    # then a valid prompt still runs (24 tokens end the window at slot 63)
    call([5] * 24)
    assert ring.next_absolute_position == 64
    torch.cuda.synchronize()
    cache.close()
    del keep, arr, at


def test_prompt_on_a_q8_0_cache_then_tokens():
    """A q8_0 cache (quantize-on-append in the prefill attention), then three
    decoder tokens continuing from the prompt's ring: the entry points and the
    composed sequence agree bit for bit at every step."""
    rng = np.random.default_rng(808)
    n_layers, vocab, cap, N = 1, 1024, 256, 38
    m = tok.make_model(rng, n_layers, vocab)
    model, keep, arr = tok.upload_model(m)
    tokens = [int(t) for t in rng.integers(0, vocab, N)]
    aring, at, _ = audio_ring(rng, 64, 0, N + 3)
    sp = stream_ptr()
    caches = []
    for _ in range(2):
        c = vkv.Cache(n_streams=1, n_layers=n_layers, capacity=cap, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=vkv.Q8_0)
        caches.append((c, vkv.new_ring(cap)))
    torch.cuda.synchronize()
    (ca, ra), (cb, rb) = caches
    ws, wp, wb = workspace_for(model, N)
    la, lb = torch.empty(vocab, device=dev()), torch.empty(vocab, device=dev())
    ta = torch.zeros(1, dtype=torch.int32, device=dev())
    tb = torch.zeros(1, dtype=torch.int32, device=dev())
    vkv.decoder_prompt(ca, 0, ra, model, tokens, aring, la.data_ptr(), ta.data_ptr(), wp, wb,
                       hip_stream=sp)
    composed_prompt(cb, rb, model, tokens, aring, lb, tb, sp)
    assert np.array_equal(host(la).view(np.uint32), host(lb).view(np.uint32))
    assert int(host(ta)[0]) == int(host(tb)[0])
    tws_b = vkv.decoder_token_workspace(model)
    tws = torch.empty(tws_b // 4 + 64, device=dev())
    tws_p = (tws.data_ptr() + 255) & ~255
    for step in range(3):
        nxt = int(host(ta)[0])
        a_ptr = aring.rows + ((N + step) % aring.capacity) * DIM * 4
        vkv.decoder_token(ca, 0, ra, model, nxt, a_ptr, la.data_ptr(), ta.data_ptr(), tws_p, tws_b,
                          hip_stream=sp)
        tok.composed_token(cb, rb, model, nxt, a_ptr, lb, tb, sp)
        assert np.array_equal(host(la).view(np.uint32), host(lb).view(np.uint32)), step
        assert int(host(ta)[0]) == int(host(tb)[0])
        assert ring_tuple(ra) == ring_tuple(rb) and ra.next_absolute_position == N + step + 1
    for which in (0, 1):
        assert np.array_equal(layer_image(ca, which, 0, 0), layer_image(cb, which, 0, 0))
    assert np.isfinite(host(la)).all()
    ca.close()
    cb.close()
    del keep, arr, at
