"""GPU parity of one decoder token (run_decoder_step's graph, src/voxtral.cpp:
2981-3040, build_decoder_layer :2629-2887):

  * the per-layer planned step (vkv_decoder_layer_step, one plan per token,
    commit after the last layer) writes the same cache bytes as the
    all-layers step and the same attention up to summation order;
  * the embedding row (get_rows + audio add) is bit-exact and the argmax
    follows ggml_vec_argmax_f32 (last index of the maximum);
  * vkv_decoder_token equals the same entry points called one by one, bit
    for bit (cache, logits, token, ring), and matches the oracle's
    composition of ggml's CPU path (Q8_K matvecs, RoPE, f16 KV append,
    flash-attention mimic, SwiGLU) through two full-width layers, stage by
    stage (attention: no further from the exact attention of the f16-rounded
    query than ggml's CPU reduction order, the mimic, is) and end to end;
  * a greedy token sequence over a 64-slot ring that wraps three times keeps
    the oracle's logical-order token at every decisive step.
"""
import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import dev, layer_image, plan_slots, step_inputs, stream_ptr, synth
from kq_util import random_matrix

pytestmark = pytest.mark.gpu

DIM, HID, QH, KVH, HD = 3072, 9216, 32, 8, 128
QD, KD = QH * HD, KVH * HD
THETA, EPS = 1.0e6, 1e-5
SCALE = 1.0 / np.sqrt(HD)


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def filled_cache(n_layers, capacity, n_pos):
    """F16 cache + ring holding synthetic rows of positions [0, n_pos)."""
    cache = vkv.Cache(n_streams=1, n_layers=n_layers, capacity=capacity, n_kv_heads=KVH,
                      head_dim=HD, n_q_heads=QH, dtype=vkv.F16)
    ring = vkv.new_ring(capacity)
    sp = stream_ptr()
    pos = 0
    while pos < n_pos:
        n = min(capacity, n_pos - pos)
        plan = vkv.decoder_plan(ring, pos, n)
        k = synth(None, KD, vkv.TAG_K, nl=n_layers, p0=pos, np_=n)
        v = synth(None, KD, vkv.TAG_V, nl=n_layers, p0=pos, np_=n)
        cache.append(0, 0, n_layers, vkv.plan_segs(plan.write_seg, plan.write_nseg), k.data_ptr(),
                     v.data_ptr(), hip_stream=sp)
        vkv.decoder_commit(ring, plan)
        pos += n
    torch.cuda.synchronize()
    return cache, ring


def ring_tuple(r):
    return (r.capacity, r.used, r.oldest_absolute_position, r.next_absolute_position, r.wraps,
            r.evictions)


def test_layer_step_matches_all_layer_step():
    L, CAP, P = 26, 512, 700
    ca, ra = filled_cache(L, CAP, P)
    cb, rb = filled_cache(L, CAP, P)
    q, k, v = step_inputs(ca, [P])
    oa = torch.empty(1, L, QD, device=dev())
    ob = torch.empty(1, L, QD, device=dev())
    rings = (vkv.Ring * 1)(ra)
    ca.decoder_step_rope(0, rings, [P], 0, L, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                         oa.data_ptr(), SCALE, THETA, hip_stream=stream_ptr())
    plan = vkv.decoder_plan(rb, P, 1)
    for layer in range(L):
        cb.decoder_layer_step(0, plan, P, layer, 1, q[0, layer].data_ptr(), k[0, layer].data_ptr(),
                              v[0, layer].data_ptr(), ob[0, layer].data_ptr(), SCALE, THETA,
                              hip_stream=stream_ptr())
    vkv.decoder_commit(rb, plan)
    # one layer per call has 8 (layer, kv head) units: the window is split over
    # slot chunks and merged, while 26 layers run one pass per unit.  Both
    # round Q to f16 as ggml's CPU flash attention does and sit ~1e-4 from
    # fp64; the two summation orders differ by as much
    np.testing.assert_allclose(host(ob), host(oa), rtol=0, atol=3e-4)
    assert ring_tuple(rings[0]) == ring_tuple(rb)
    for layer in (0, 13, 25):
        for which in (0, 1):
            assert np.array_equal(layer_image(ca, which, 0, layer), layer_image(cb, which, 0, layer))
    ca.close()
    cb.close()


def test_layer_step_rejects_bad_plans():
    cache, ring = filled_cache(2, 64, 10)
    q, k, v = step_inputs(cache, [10])
    out = torch.empty(2, QD, device=dev())
    plan = vkv.decoder_plan(ring, 10, 1)
    with pytest.raises(vkv.VkvError):            # position is not the plan's
        cache.decoder_layer_step(0, plan, 11, 0, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                 out.data_ptr(), SCALE, THETA)
    two = vkv.decoder_plan(ring, 10, 2)
    with pytest.raises(vkv.VkvError):            # more than one row
        cache.decoder_layer_step(0, two, 10, 0, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                 out.data_ptr(), SCALE, THETA)
    with pytest.raises(vkv.VkvError):            # layer outside the cache
        cache.decoder_layer_step(0, plan, 10, 2, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                 out.data_ptr(), SCALE, THETA)
    cache.close()


def test_embed_row_plus_audio_is_bit_exact():
    rng = np.random.default_rng(3008)
    vocab = 1000
    table = random_matrix(rng, vkv.Q6_K, vocab, DIM)
    audio = rng.standard_normal(DIM).astype(np.float32)
    td, ad = to_dev(table), to_dev(audio)
    y = torch.empty(DIM, device=dev())
    rb = DIM // 256 * 210
    for token in (0, 777, vocab - 1):
        vkv.embed(vkv.Q6_K, td.data_ptr(), vocab, DIM, token, y.data_ptr(), ad.data_ptr(),
                  hip_stream=stream_ptr())
        want = oracle.dequantize(oracle.Q6_K, table[token * rb:(token + 1) * rb], DIM) + audio
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
    with pytest.raises(vkv.VkvError):
        vkv.embed(vkv.Q6_K, td.data_ptr(), vocab, DIM, vocab, y.data_ptr())


def test_argmax_matches_ggml_rule():
    rng = np.random.default_rng(2970)
    out = torch.zeros(1, dtype=torch.int32, device=dev())
    cases = [rng.standard_normal(131072).astype(np.float32),
             rng.integers(-40, 40, 131072).astype(np.float32),     # many ties of the maximum
             rng.integers(-40, 40, 131071).astype(np.float32),     # odd length (scalar tail)
             np.full(4097, -np.inf, np.float32),
             np.array([5.0], np.float32)]
    for x in cases:
        xd = to_dev(x)
        vkv.argmax(xd.data_ptr(), x.size, out.data_ptr(), hip_stream=stream_ptr())
        assert int(host(out)[0]) == oracle.argmax(x)


# ---- one full decoder token ----

# weight types of the two file kinds: the Q4_K_M mix (src/voxtral-quantize.cpp:
# 148-159) and a Q8_0 file (:95-96, every matrix Q8_0)
MIX = {"q4km": dict(attn_q=vkv.Q4_K, attn_k=vkv.Q4_K, attn_v=vkv.Q6_K, attn_o=vkv.Q4_K,
                    ffn_w1=vkv.Q4_K, ffn_w3=vkv.Q4_K, ffn_w2=vkv.Q6_K, table=vkv.Q6_K),
       "q8_0": dict(attn_q=vkv.Q8_0, attn_k=vkv.Q8_0, attn_v=vkv.Q8_0, attn_o=vkv.Q8_0,
                    ffn_w1=vkv.Q8_0, ffn_w3=vkv.Q8_0, ffn_w2=vkv.Q8_0, table=vkv.Q8_0)}


def wscale(dtype, slot):
    """random_matrix's scale factor for a Q8_0 matrix in a slot the Q4_K_M mix
    fills with Q4_K (typical |w| ~0.4 x scale) or Q6_K (~0.1 x scale): Q8_0
    blocks are ~1 x scale, so the activations keep the magnitudes the bounds
    below were set for"""
    if dtype != vkv.Q8_0:
        return 1.0
    return 0.11 if MIX["q4km"][slot] == vkv.Q6_K else 0.4


def make_model(rng, n_layers, vocab, kind="q4km"):
    """Random decoder weights (numpy) of one file kind, moderate magnitudes."""
    T = MIX[kind]
    layers = []
    for layer in range(n_layers):
        layers.append(dict(
            attn_norm=rng.uniform(0.5, 1.5, DIM).astype(np.float32),
            attn_q=random_matrix(rng, T["attn_q"], QD, DIM, 0.005 * wscale(T["attn_q"], "attn_q")),
            attn_k=random_matrix(rng, T["attn_k"], KD, DIM, 0.005 * wscale(T["attn_k"], "attn_k")),
            attn_v=random_matrix(rng, T["attn_v"], KD, DIM, 0.1 * wscale(T["attn_v"], "attn_v")),
            attn_o=random_matrix(rng, T["attn_o"], DIM, QD, 0.005 * wscale(T["attn_o"], "attn_o")),
            ffn_norm=rng.uniform(0.5, 1.5, DIM).astype(np.float32),
            ada=rng.uniform(-0.3, 0.3, DIM).astype(np.float32) if layer == 0 else None,
            ffn_w1=random_matrix(rng, T["ffn_w1"], HID, DIM, 0.003 * wscale(T["ffn_w1"], "ffn_w1")),
            ffn_w3=random_matrix(rng, T["ffn_w3"], HID, DIM, 0.003 * wscale(T["ffn_w3"], "ffn_w3")),
            ffn_w2=random_matrix(rng, T["ffn_w2"], DIM, HID, 0.05 * wscale(T["ffn_w2"], "ffn_w2"))))
    return dict(layers=layers, table=random_matrix(rng, T["table"], vocab, DIM,
                                                   0.5 * wscale(T["table"], "table")),
                out_norm=rng.uniform(0.5, 1.5, DIM).astype(np.float32), vocab=vocab, types=T)


def upload_model(m):
    """device tensors + the vkv_dec_model struct (keeps the tensors alive)."""
    keep = []

    def d(a):
        if a is None:
            return None
        t = to_dev(a)
        keep.append(t)
        return t.data_ptr()

    n = len(m["layers"])
    T = m["types"]
    arr = (vkv.DecLayer * n)()
    for i, L in enumerate(m["layers"]):
        arr[i] = vkv.DecLayer(d(L["attn_norm"]), d(L["attn_q"]), d(L["attn_k"]), d(L["attn_v"]),
                              d(L["attn_o"]), T["attn_q"], T["attn_k"], T["attn_v"], T["attn_o"],
                              d(L["ffn_norm"]), d(L["ada"]), d(L["ffn_w1"]), d(L["ffn_w2"]),
                              d(L["ffn_w3"]), T["ffn_w1"], T["ffn_w2"], T["ffn_w3"])
    table = d(m["table"])
    model = vkv.DecModel(n, DIM, HID, QH, KVH, HD, m["vocab"], EPS, THETA, table, T["table"],
                         d(m["out_norm"]), table, T["table"], arr)
    return model, keep, arr


stage_err = []   # (gpu, mimic) attention errors / scale of every checked stage


def composed_token(cache, ring, model, token, audio_ptr, logits, tok_out, hip_stream, m=None):
    """The same entry points vkv_decoder_token calls, one by one.  With m (the
    numpy weights) every stage is also checked against the oracle's stage fed
    with this run's own input (teacher forcing), so differences cannot
    compound."""
    pos = ring.next_absolute_position
    plan = vkv.decoder_plan(ring, pos, 1)
    x = torch.empty(DIM, device=dev())
    q, k, v = (torch.empty(n, device=dev()) for n in (QD, KD, KD))
    attn = torch.empty(QD, device=dev())
    ffn = torch.empty(HID, device=dev())
    row_b = int(cache.row_bytes)
    slot = plan.write_seg[0].slot

    def rel(got, want):
        want = np.asarray(want, np.float64)
        return np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30)

    vkv.embed(model.tok_embeddings_type, model.tok_embeddings, model.vocab, DIM, token, x.data_ptr(),
              audio_ptr, hip_stream=hip_stream)
    xp = x.data_ptr()
    for layer in range(model.n_layers):
        L = model.layers[layer]
        x_in = host(x) if m else None
        vkv.matvec(xp, DIM, [(L.attn_q, L.attn_q_type, QD, q.data_ptr()),
                             (L.attn_k, L.attn_k_type, KD, k.data_ptr()),
                             (L.attn_v, L.attn_v_type, KD, v.data_ptr())],
                   norm_w_ptr=L.attn_norm, eps=EPS, hip_stream=hip_stream)
        if m:
            M = m["layers"][layer]
            h = oracle.norm_act(x_in, M["attn_norm"], None, EPS)
            q_in, k_in, v_in = host(q), host(k), host(v)
            assert rel(q_in, oracle.matvec(L.attn_q_type, M["attn_q"], QD, DIM, h, 8)) < 2e-6
            assert rel(k_in, oracle.matvec(L.attn_k_type, M["attn_k"], KD, DIM, h, 8)) < 2e-6
            assert rel(v_in, oracle.matvec(L.attn_v_type, M["attn_v"], KD, DIM, h, 8)) < 2e-6
        cache.decoder_layer_step(0, plan, pos, layer, 1, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                 attn.data_ptr(), SCALE, THETA, hip_stream=hip_stream)
        if m:
            # appended rows: f16 of the RoPE'd k and of v, bit for bit
            kr = oracle.rope(k_in.reshape(1, KD), HD, pos, THETA).ravel()
            kimg, vimg = layer_image(cache, 0, 0, layer), layer_image(cache, 1, 0, layer)
            assert np.array_equal(kimg[slot * row_b:(slot + 1) * row_b],
                                  np.frombuffer(oracle.rows_from_f32(oracle.F16, kr), np.uint8))
            assert np.array_equal(vimg[slot * row_b:(slot + 1) * row_b],
                                  np.frombuffer(oracle.rows_from_f32(oracle.F16, v_in), np.uint8))
            qr = oracle.rope(q_in.reshape(1, QD), HD, pos, THETA).ravel()
            slots = plan_slots(plan)
            a_got = host(attn)
            # against the exact attention of the f16-rounded query (the
            # kernel's and ggml's dot type): no further from it than ggml's
            # CPU reduction order is (the mimic: f16 V accumulator), plus
            # 2e-5 of the output's scale (f32 scores of large magnitude)
            q16 = oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(qr.astype(np.float32)))
            exact = oracle.decode_attn_f64(oracle.F16, kimg, vimg, row_b, slots, q16, KVH, HD,
                                           SCALE).ravel()
            mimic = oracle.decode_attn_mimic(oracle.F16, kimg, vimg, row_b, slots, qr, KVH, HD,
                                             SCALE).ravel()
            mag = max(np.abs(exact).max(), 1e-30)
            e_gpu, e_mimic = np.abs(a_got - exact).max(), np.abs(mimic - exact).max()
            assert e_gpu <= e_mimic + 2e-5 * mag, (pos, layer, e_gpu, e_mimic, mag)
            stage_err.append((e_gpu / mag, e_mimic / mag))
            x_mid = host(x)
        vkv.matvec(attn.data_ptr(), QD, [(L.attn_o, L.attn_o_type, DIM, xp, xp)],
                   hip_stream=hip_stream)
        if m:
            x_o = host(x)
            assert rel(x_o, x_mid + oracle.matvec(L.attn_o_type, M["attn_o"], DIM, QD, a_got, 8)) < 2e-6
        vkv.matvec(xp, DIM, [(L.ffn_w1, L.ffn_w1_type, HID, ffn.data_ptr()),
                             (L.ffn_w3, L.ffn_w3_type, HID, None)],
                   norm_w_ptr=L.ffn_norm, ada_ptr=L.ada_scale, eps=EPS,
                   epilogue=vkv.MV_SWIGLU, hip_stream=hip_stream)
        if m:
            h2 = oracle.norm_act(x_o, M["ffn_norm"], M["ada"], EPS)
            g = oracle.matvec(L.ffn_w1_type, M["ffn_w1"], HID, DIM, h2, 8)
            u = oracle.matvec(L.ffn_w3_type, M["ffn_w3"], HID, DIM, h2, 8)
            f_got = host(ffn)
            assert rel(f_got, oracle.silu(g) * u) < 2e-6
        vkv.matvec(ffn.data_ptr(), HID, [(L.ffn_w2, L.ffn_w2_type, DIM, xp, xp)],
                   hip_stream=hip_stream)
        if m:
            assert rel(host(x), x_o + oracle.matvec(L.ffn_w2_type, M["ffn_w2"], DIM, HID, f_got, 8)) < 2e-6
    x_fin = host(x) if m else None
    vkv.matvec(xp, DIM, [(model.output, model.output_type, model.vocab, logits.data_ptr())],
               norm_w_ptr=model.out_norm, eps=EPS, hip_stream=hip_stream)
    vkv.argmax(logits.data_ptr(), model.vocab, tok_out.data_ptr(), hip_stream=hip_stream)
    if m:
        lg = host(logits)
        xn = oracle.norm_act(x_fin, m["out_norm"], None, EPS)
        assert rel(lg, oracle.matvec(model.output_type, m["table"], model.vocab, DIM, xn, 8)) < 2e-6
        assert int(host(tok_out)[0]) == oracle.argmax(lg)
    vkv.decoder_commit(ring, plan)
    return plan, x


def oracle_token(m, k_imgs, v_imgs, row_b, plan, pos, token, audio, attn_fn):
    """ggml's CPU path for the same token (oracle restatements throughout);
    attn_fn: the oracle's fp64 attention or its ggml flash-attention mimic."""
    T = m["types"]
    rb = oracle.wrow_bytes(T["table"], DIM)
    x = oracle.dequantize(T["table"], m["table"][token * rb:(token + 1) * rb], DIM) + audio
    slot = plan.write_seg[0].slot
    slots = plan_slots(plan)
    for layer, L in enumerate(m["layers"]):
        h = oracle.norm_act(x, L["attn_norm"], None, EPS)
        q = oracle.matvec(T["attn_q"], L["attn_q"], QD, DIM, h, 8)
        k = oracle.matvec(T["attn_k"], L["attn_k"], KD, DIM, h, 8)
        v = oracle.matvec(T["attn_v"], L["attn_v"], KD, DIM, h, 8)
        q = oracle.rope(q.reshape(1, QD), HD, pos, THETA).ravel()
        k = oracle.rope(k.reshape(1, KD), HD, pos, THETA).ravel()
        ki, vi = k_imgs[layer].copy(), v_imgs[layer].copy()
        ki[slot * row_b:(slot + 1) * row_b] = np.frombuffer(oracle.rows_from_f32(oracle.F16, k), np.uint8)
        vi[slot * row_b:(slot + 1) * row_b] = np.frombuffer(oracle.rows_from_f32(oracle.F16, v), np.uint8)
        attn = attn_fn(oracle.F16, ki, vi, row_b, slots, q, KVH, HD, SCALE).ravel()
        x = x + oracle.matvec(T["attn_o"], L["attn_o"], DIM, QD, attn, 8)
        h = oracle.norm_act(x, L["ffn_norm"], L["ada"], EPS)
        g = oracle.matvec(T["ffn_w1"], L["ffn_w1"], HID, DIM, h, 8)
        u = oracle.matvec(T["ffn_w3"], L["ffn_w3"], HID, DIM, h, 8)
        f = (oracle.silu(g) * u).astype(np.float32)
        x = x + oracle.matvec(T["ffn_w2"], L["ffn_w2"], DIM, HID, f, 8)
    xn = oracle.norm_act(x, m["out_norm"], None, EPS)
    logits = oracle.matvec(T["table"], m["table"], m["vocab"], DIM, xn, 8)
    return logits, oracle.argmax(logits)


@pytest.mark.parametrize("kind", ["q4km", "q8_0"])
def test_decoder_token_two_layers(kind):
    rng = np.random.default_rng(5219)
    n_layers, vocab, CAP, P, token = 2, 4096, 512, 700, 1234
    m = make_model(rng, n_layers, vocab, kind)
    model, keep, arr = upload_model(m)
    audio = (rng.standard_normal(DIM) * 0.1).astype(np.float32)
    ad = to_dev(audio)
    ws_bytes = vkv.decoder_token_workspace(model)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes // 4 + 64, device=dev())
    ws_ptr = (ws.data_ptr() + 255) & ~255
    sp = stream_ptr()

    ca, ra = filled_cache(n_layers, CAP, P)
    cb, rb_ = filled_cache(n_layers, CAP, P)
    row_b = int(ca.row_bytes)
    k_imgs = [layer_image(ca, 0, 0, layer).copy() for layer in range(n_layers)]
    v_imgs = [layer_image(ca, 1, 0, layer).copy() for layer in range(n_layers)]

    la = torch.empty(vocab, device=dev())
    ta = torch.zeros(1, dtype=torch.int32, device=dev())
    plan = vkv.decoder_token(ca, 0, ra, model, token, ad.data_ptr(), la.data_ptr(), ta.data_ptr(),
                             ws_ptr, ws_bytes, hip_stream=sp)
    lb = torch.empty(vocab, device=dev())
    tb = torch.zeros(1, dtype=torch.int32, device=dev())
    plan_b, xb = composed_token(cb, rb_, model, token, ad.data_ptr(), lb, tb, sp, m)

    # the C composition is the per-call sequence, bit for bit
    assert np.array_equal(host(la).view(np.uint32), host(lb).view(np.uint32))
    assert int(host(ta)[0]) == int(host(tb)[0])
    assert ring_tuple(ra) == ring_tuple(rb_) and ra.next_absolute_position == P + 1
    assert plan.write_seg[0].slot == plan_b.write_seg[0].slot == P % CAP
    # the workspace keeps the final residual stream at offset 0
    off = (ws_ptr - ws.data_ptr()) // 4
    assert np.array_equal(host(ws[off:off + DIM]).view(np.uint32), host(xb).view(np.uint32))
    for layer in range(n_layers):
        for which in (0, 1):
            assert np.array_equal(layer_image(ca, which, 0, layer), layer_image(cb, which, 0, layer))

    # end to end against ggml's CPU path: the stages agree as checked above;
    # composed over two layers, the f16 rounding of Q inside the attention
    # (ggml's CPU path rounds it too) is the only difference that grows
    # (with the mimic's f16 V accumulation as well, the bound is looser)
    got = host(la).astype(np.float64)
    for attn_fn, max_rel, min_corr in ((oracle.decode_attn_f64, 1e-2, 0.9999),
                                       (oracle.decode_attn_mimic, 4e-2, 0.999)):
        want, want_tok = oracle_token(m, k_imgs, v_imgs, row_b, plan, P, token, audio, attn_fn)
        scale = np.abs(want).max()
        err = np.abs(got - want).max()
        corr = np.corrcoef(got, want)[0, 1]
        print(f"{attn_fn.__name__}: max err {err:.4g} of scale {scale:.4g}, corr {corr:.6f}", flush=True)
        assert err <= max_rel * scale and corr > min_corr, (attn_fn.__name__, err, scale, corr)
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 2 * err:
            assert int(host(ta)[0]) == want_tok
    # the appended K rows are the RoPE'd projections, f16
    slot = P % CAP
    for layer in range(n_layers):
        kimg = layer_image(ca, 0, 0, layer)
        assert not np.array_equal(kimg[slot * row_b:(slot + 1) * row_b],
                                  k_imgs[layer][slot * row_b:(slot + 1) * row_b])
    ca.close()
    cb.close()
    del keep, arr


def test_token_sequence_across_capacity_64_wraps():
    """The reference's ring acceptance (tests/node/scripts/acceptance-decoder-
    kv-ring.js:54-117) runs the decoder at test capacity 64, so its ring
    wraps during real tokens, and requires the production (physical ring)
    token sequence to equal the logical-order oracle's.  Here: 160 greedy
    vkv_decoder_token steps (each output token is the next input) over a
    64-slot ring prefilled with positions 0..39, so positions 40..199 wrap it
    three times.  A second cache takes the same steps through the entry
    points one by one, each stage checked against the oracle fed that stage's
    input (attention in logical order, oldest -> newest slot): logits, token,
    ring and cache bytes of the two agree bit for bit at every step.  End to
    end, the oracle composes each token from the step's cache image with
    exact attention of the f16-rounded query; a last-bit difference can flip
    a code of a later product's Q8_K activations (ggml's CPU path quantizes
    them the same way) and compound, so the logits agree within 5e-2 of their
    scale at correlation > 0.998, and the token is the oracle's wherever its
    top-2 gap exceeds twice the logits' difference (at least half the steps)."""
    rng = np.random.default_rng(64)
    n_layers, vocab, CAP, P0, N = 2, 4096, 64, 40, 160
    m = make_model(rng, n_layers, vocab)
    model, keep, arr = upload_model(m)
    audio = (rng.standard_normal((N, DIM)) * 0.1).astype(np.float32)
    ad = to_dev(audio)
    ws_bytes = vkv.decoder_token_workspace(model)
    ws = torch.empty(ws_bytes // 4 + 64, device=dev())
    ws_ptr = (ws.data_ptr() + 255) & ~255
    sp = stream_ptr()
    cache, ring = filled_cache(n_layers, CAP, P0)
    cb, rb_ = filled_cache(n_layers, CAP, P0)
    row_b = int(cache.row_bytes)
    logits, lb = torch.empty(vocab, device=dev()), torch.empty(vocab, device=dev())
    tok, tb = (torch.zeros(1, dtype=torch.int32, device=dev()) for _ in range(2))
    token, decisive, wraps, rec = 7, 0, [], []

    def attn_f64_f16q(dtype, ki, vi, rb, slots, q, kvh, hd, scale):
        # exact attention of the f16-rounded query (ggml's CPU path converts
        # Q to K's f16 dot type; so does the decode kernel)
        q16 = oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(np.asarray(q, np.float32)))
        return oracle.decode_attn_f64(dtype, ki, vi, rb, slots, q16, kvh, hd, scale)

    for i in range(N):
        pos = ring.next_absolute_position
        assert pos == P0 + i
        k_imgs = [layer_image(cache, 0, 0, layer).copy() for layer in range(n_layers)]
        v_imgs = [layer_image(cache, 1, 0, layer).copy() for layer in range(n_layers)]
        plan = vkv.decoder_token(cache, 0, ring, model, token, ad[i].data_ptr(), logits.data_ptr(),
                                 tok.data_ptr(), ws_ptr, ws_bytes, hip_stream=sp)
        composed_token(cb, rb_, model, token, ad[i].data_ptr(), lb, tb, sp, m)
        got = host(logits)
        got_tok = int(host(tok)[0])
        assert np.array_equal(got.view(np.uint32), host(lb).view(np.uint32)), pos
        assert got_tok == int(host(tb)[0]) == oracle.argmax(got)
        assert ring_tuple(ring) == ring_tuple(rb_)
        for layer in range(n_layers):
            for which in (0, 1):
                assert np.array_equal(layer_image(cache, which, 0, layer),
                                      layer_image(cb, which, 0, layer)), (pos, layer, which)
        slots = plan_slots(plan)
        assert len(slots) == min(pos + 1, CAP) and slots[-1] == pos % CAP
        want, want_tok = oracle_token(m, k_imgs, v_imgs, row_b, plan, pos, token, audio[i],
                                      attn_f64_f16q)
        got = got.astype(np.float64)
        err = np.abs(got - want).max()
        corr = np.corrcoef(got, want)[0, 1]
        top2 = np.sort(want)[-2:]
        dec = top2[1] - top2[0] > 2 * err
        decisive += int(dec)
        rec.append((pos, err / np.abs(want).max(), corr, dec, got_tok, want_tok))
        wraps.append(ring.wraps)
        token = got_tok
    assert ring.next_absolute_position == P0 + N and ring.used == CAP
    assert ring.oldest_absolute_position == P0 + N - CAP
    assert wraps[-1] >= 3 and wraps[0] == 0
    errs, corrs = [r[1] for r in rec], [r[2] for r in rec]
    eg, em = np.array(stage_err[-2 * N:]).T
    print(f"attention stages: gpu error / scale max {eg.max():.2e} median {np.median(eg):.2e}; "
          f"mimic max {em.max():.2e} median {np.median(em):.2e}", flush=True)
    print(f"capacity 64: {N} tokens, {decisive} decisive, wraps {wraps[-1]}; logits error / scale "
          f"max {max(errs):.2e} median {np.median(errs):.2e}; correlation min {min(corrs):.6f} "
          f"median {np.median(corrs):.6f}", flush=True)
    for pos, e, corr, dec, gt, wt in rec:
        assert e <= 5e-2 and corr > 0.998, (pos, e, corr)
        assert not dec or gt == wt, (pos, gt, wt)
    assert decisive >= N // 2
    cache.close()
    cb.close()
    del keep, arr
