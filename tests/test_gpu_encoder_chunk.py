"""GPU parity of one encoder chunk through the transformer layers
(build_encoder_kv_graph, src/voxtral.cpp:2144-2370): vkv_encoder_chunk leaves
the same ring bytes as the same entry points called one by one, its output is
that run's rows through the final norm (within 2e-6 of the oracle's norm), and
each stage of that run matches the oracle's stage fed with the run's own input
(teacher forcing): projections with norm bias and biases, RoPE, the ring
append (bit-exact f16 rows) and window attention (fp64, 2e-3), O + bias +
residual, SwiGLU, W2 + bias + residual, the final norm."""
import numpy as np
import pytest
import torch

import oracle
import vkv
from gpu_util import dev, layer_image, stream_ptr, synth
from kq_util import random_matrix
from test_gpu_matmul import rows_ref

pytestmark = pytest.mark.gpu

DIM, HID, H, HD = 1280, 5120, 32, 64
QD = H * HD
CAP, WIN = 878, 750
THETA, EPS = 1.0e6, 1e-5
SCALE = 1.0 / np.sqrt(HD)


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# weight types of the two file kinds: the Q4_K_M mix (src/voxtral-quantize.cpp:
# 148-159) and a Q8_0 file (:95-96)
MIX = {"q4km": dict(attn_q=vkv.Q4_K, attn_k=vkv.Q4_K, attn_v=vkv.Q6_K, attn_o=vkv.Q4_K,
                    ffn_w1=vkv.Q4_K, ffn_w3=vkv.Q4_K, ffn_w2=vkv.Q6_K),
       "q8_0": dict(attn_q=vkv.Q8_0, attn_k=vkv.Q8_0, attn_v=vkv.Q8_0, attn_o=vkv.Q8_0,
                    ffn_w1=vkv.Q8_0, ffn_w3=vkv.Q8_0, ffn_w2=vkv.Q8_0)}


def wscale(dtype, slot):
    """a Q8_0 matrix's scale factor for the magnitudes of the slot's k-quant
    (Q4_K ~0.4 x scale, Q6_K ~0.1 x scale, Q8_0 ~1 x scale)"""
    if dtype != vkv.Q8_0:
        return 1.0
    return 0.11 if MIX["q4km"][slot] == vkv.Q6_K else 0.4


def make_model(rng, n_layers, kind="q4km"):
    T = MIX[kind]
    layers = []
    for _ in range(n_layers):
        layers.append(dict(
            attn_norm=rng.uniform(0.5, 1.5, DIM).astype(np.float32),
            attn_norm_b=rng.uniform(-0.1, 0.1, DIM).astype(np.float32),
            attn_q=random_matrix(rng, T["attn_q"], QD, DIM, 0.01 * wscale(T["attn_q"], "attn_q")),
            attn_k=random_matrix(rng, T["attn_k"], QD, DIM, 0.01 * wscale(T["attn_k"], "attn_k")),
            attn_v=random_matrix(rng, T["attn_v"], QD, DIM, 0.1 * wscale(T["attn_v"], "attn_v")),
            attn_o=random_matrix(rng, T["attn_o"], DIM, QD, 0.01 * wscale(T["attn_o"], "attn_o")),
            attn_q_b=rng.uniform(-0.1, 0.1, QD).astype(np.float32),
            attn_v_b=rng.uniform(-0.1, 0.1, QD).astype(np.float32),
            attn_o_b=rng.uniform(-0.1, 0.1, DIM).astype(np.float32),
            ffn_norm=rng.uniform(0.5, 1.5, DIM).astype(np.float32),
            ffn_norm_b=rng.uniform(-0.1, 0.1, DIM).astype(np.float32),
            ffn_w1=random_matrix(rng, T["ffn_w1"], HID, DIM, 0.005 * wscale(T["ffn_w1"], "ffn_w1")),
            ffn_w3=random_matrix(rng, T["ffn_w3"], HID, DIM, 0.005 * wscale(T["ffn_w3"], "ffn_w3")),
            ffn_w2=random_matrix(rng, T["ffn_w2"], DIM, HID, 0.05 * wscale(T["ffn_w2"], "ffn_w2")),
            ffn_w2_b=rng.uniform(-0.1, 0.1, DIM).astype(np.float32)))
    return dict(layers=layers, out_norm=rng.uniform(0.5, 1.5, DIM).astype(np.float32),
                out_norm_b=rng.uniform(-0.1, 0.1, DIM).astype(np.float32), types=T)


def upload(m):
    keep = []

    def d(a):
        t = to_dev(a)
        keep.append(t)
        return t.data_ptr()

    n = len(m["layers"])
    T = m["types"]
    arr = (vkv.EncLayer * n)()
    for i, L in enumerate(m["layers"]):
        arr[i] = vkv.EncLayer(d(L["attn_norm"]), d(L["attn_norm_b"]), d(L["attn_q"]), d(L["attn_k"]),
                              d(L["attn_v"]), d(L["attn_o"]), T["attn_q"], T["attn_k"], T["attn_v"],
                              T["attn_o"], d(L["attn_q_b"]), d(L["attn_v_b"]), d(L["attn_o_b"]),
                              d(L["ffn_norm"]), d(L["ffn_norm_b"]), d(L["ffn_w1"]), d(L["ffn_w2"]),
                              d(L["ffn_w3"]), T["ffn_w1"], T["ffn_w2"], T["ffn_w3"], d(L["ffn_w2_b"]))
    model = vkv.EncModel(n, DIM, HID, H, HD, EPS, THETA, d(m["out_norm"]), d(m["out_norm_b"]), arr)
    return model, keep, arr


def filled_ring(n_layers, n_pos):
    """encoder cache whose ring holds synthetic rows of frames [0, n_pos)"""
    c = vkv.Cache(n_streams=1, n_layers=n_layers, capacity=CAP, n_kv_heads=H, head_dim=HD,
                  n_q_heads=H, dtype=vkv.F16)
    pos = 0
    while pos < n_pos:
        n = min(128, n_pos - pos)
        plan = vkv.enc_plan(pos, n, CAP, WIN)
        k = synth(None, QD, vkv.TAG_EK, nl=n_layers, p0=pos, np_=n)
        v = synth(None, QD, vkv.TAG_EV, nl=n_layers, p0=pos, np_=n)
        c.append(0, 0, n_layers, vkv.plan_segs(plan.write_seg, plan.write_nseg), k.data_ptr(),
                 v.data_ptr(), hip_stream=stream_ptr())
        pos += n
    torch.cuda.synchronize()
    return c


def rel(got, want):
    want = np.asarray(want, np.float64)
    return np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30)


def composed(c, plan, model, m, x, check):
    """vkv_encoder_chunk's sequence of entry points; with check, every stage
    against the oracle fed this run's input"""
    N, sp = plan.n_new, stream_ptr()
    ws_b = vkv.matmul_workspace(N, HID)
    ws_t = torch.empty(ws_b // 4 + 64, device=dev())
    ws = (ws_t.data_ptr() + 255) & ~255
    qk = torch.empty(2, N, QD, device=dev())
    v = torch.empty(N, QD, device=dev())
    attn = torch.empty(N, QD, device=dev())
    ffn = torch.empty(N, HID, device=dev())
    xp = x.data_ptr()
    q_pos = np.arange(plan.q_start, plan.q_start + N)
    for layer in range(model.n_layers):
        L, M = model.layers[layer], m["layers"][layer]
        x_in = host(x)
        vkv.matmul(xp, N, DIM, [(L.attn_q, L.attn_q_type, QD, qk[0].data_ptr(), None, L.attn_q_b),
                                (L.attn_k, L.attn_k_type, QD, qk[1].data_ptr(), None, None),
                                (L.attn_v, L.attn_v_type, QD, v.data_ptr(), None, L.attn_v_b)],
                   ws, ws_b, norm_w_ptr=L.attn_norm, norm_b_ptr=L.attn_norm_b, eps=EPS, hip_stream=sp)
        if check:
            hs = [oracle.norm_act(x_in[p], M["attn_norm"], eps=EPS, norm_b=M["attn_norm_b"]) for p in range(N)]
            q_in, k_in, v_in = host(qk[0]), host(qk[1]), host(v)
            for got, w, dt, b in ((q_in, M["attn_q"], L.attn_q_type, M["attn_q_b"]),
                                  (k_in, M["attn_k"], L.attn_k_type, None),
                                  (v_in, M["attn_v"], L.attn_v_type, M["attn_v_b"])):
                want, mag = rows_ref(dt, w, QD, DIM, hs)
                if b is not None:
                    want = want + b[None, :]
                assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6 * np.abs(want) + 1e-30)
        vkv.rope(qk.data_ptr(), 2, N, QD, HD, plan.q_start, THETA, hip_stream=sp)
        if check:
            qr, kr = host(qk[0]), host(qk[1])
            assert rel(qr, oracle.rope(q_in, HD, plan.q_start, THETA)) <= 4e-7
            assert rel(kr, oracle.rope(k_in, HD, plan.q_start, THETA)) <= 4e-7
        c.enc_step(0, plan, WIN, layer, 1, qk[0].data_ptr(), qk[1].data_ptr(), v.data_ptr(),
                   attn.data_ptr(), SCALE, hip_stream=sp)
        if check:
            kimg, vimg = layer_image(c, 0, 0, layer), layer_image(c, 1, 0, layer)
            rb = int(c.row_bytes)
            for i in range(N):
                s = (plan.q_start + i) % CAP
                assert np.array_equal(kimg[s * rb:(s + 1) * rb],
                                      np.frombuffer(oracle.rows_from_f32(oracle.F16, kr[i]), np.uint8))
                assert np.array_equal(vimg[s * rb:(s + 1) * rb],
                                      np.frombuffer(oracle.rows_from_f32(oracle.F16, v_in[i]), np.uint8))
            key_pos = np.arange(plan.win_start, plan.win_end)
            want = oracle.window_attn_f64(oracle.F16, kimg, vimg, rb, (key_pos % CAP).astype(np.int32),
                                          key_pos, qr.reshape(N, H, HD), q_pos, H, H, HD, WIN, SCALE)
            a_got = host(attn)
            assert np.abs(a_got.reshape(N, H, HD) - want).max() <= 2e-3
            x_mid = host(x)
        vkv.matmul(attn.data_ptr(), N, QD, [(L.attn_o, L.attn_o_type, DIM, xp, xp, L.attn_o_b)],
                   ws, ws_b, hip_stream=sp)
        if check:
            x_o = host(x)
            proj, mag = rows_ref(L.attn_o_type, M["attn_o"], DIM, QD, list(a_got))
            want = x_mid + (proj + M["attn_o_b"][None, :])
            assert np.all(np.abs(x_o - want) <= 1e-5 * mag + 2e-7 * np.abs(want) + 1e-30)
        vkv.matmul(xp, N, DIM, [(L.ffn_w1, L.ffn_w1_type, HID, ffn.data_ptr()),
                                (L.ffn_w3, L.ffn_w3_type, HID, None)],
                   ws, ws_b, norm_w_ptr=L.ffn_norm, norm_b_ptr=L.ffn_norm_b, eps=EPS,
                   epilogue=vkv.MV_SWIGLU, hip_stream=sp)
        if check:
            hs = [oracle.norm_act(x_o[p], M["ffn_norm"], eps=EPS, norm_b=M["ffn_norm_b"]) for p in range(N)]
            g, m1 = rows_ref(L.ffn_w1_type, M["ffn_w1"], HID, DIM, hs)
            u, m3 = rows_ref(L.ffn_w3_type, M["ffn_w3"], HID, DIM, hs)
            g64, u64 = g.astype(np.float64), u.astype(np.float64)
            sg = g64 / (1 + np.exp(-g64))
            f_got = host(ffn)
            assert np.all(np.abs(f_got - sg * u64) <=
                          1e-5 * (1.1 * m1 * np.abs(u64) + np.abs(sg) * m3) + 1e-6 * np.abs(sg * u64) + 1e-30)
        vkv.matmul(ffn.data_ptr(), N, HID, [(L.ffn_w2, L.ffn_w2_type, DIM, xp, xp, L.ffn_w2_b)],
                   ws, ws_b, hip_stream=sp)
        if check:
            proj, mag = rows_ref(L.ffn_w2_type, M["ffn_w2"], DIM, HID, list(f_got))
            want = x_o + (proj + M["ffn_w2_b"][None, :])
            assert np.all(np.abs(host(x) - want) <= 1e-5 * mag + 2e-7 * np.abs(want) + 1e-30)
    return ws_t


@pytest.mark.parametrize("q_start,n_new,kind", [(800, 16, "q4km"), (1296, 4, "q4km"),
                                                (64, 16, "q4km"), (800, 16, "q8_0"),
                                                (1296, 4, "q8_0")])
def test_encoder_chunk(q_start, n_new, kind):
    rng = np.random.default_rng(q_start + n_new)
    n_layers = 2
    m = make_model(rng, n_layers, kind)
    model, keep, arr = upload(m)
    x0 = rng.standard_normal((n_new, DIM)).astype(np.float32)
    ca, cb = filled_ring(n_layers, q_start), filled_ring(n_layers, q_start)
    plan = vkv.enc_plan(q_start, n_new, CAP, WIN)
    xa, xb = to_dev(x0), to_dev(x0)
    ws_b = vkv.encoder_chunk_workspace(model, n_new)
    assert ws_b > 0
    ws = torch.empty(ws_b // 4 + 64, device=dev())
    vkv.encoder_chunk(ca, 0, plan, WIN, model, xa.data_ptr(), (ws.data_ptr() + 255) & ~255, ws_b,
                      hip_stream=stream_ptr())
    composed(cb, plan, model, m, xb, check=True)
    x_pre = host(xb)
    # the C call's output is the composed run's rows through the final norm
    # (rms_norm * w + b), and their rings are identical
    want = np.stack([oracle.norm_act(x_pre[p], m["out_norm"], eps=EPS, norm_b=m["out_norm_b"])
                     for p in range(n_new)])
    got = host(xa)
    assert rel(got, want) <= 2e-6
    for layer in range(n_layers):
        for which in (0, 1):
            assert np.array_equal(layer_image(ca, which, 0, layer), layer_image(cb, which, 0, layer))
    ca.close()
    cb.close()
    del keep, arr


@pytest.mark.parametrize("q_start,n_new", [(1276, 16), (4, 4)])
def test_encoder_chunk_into_the_output_ring(q_start, n_new):
    """vkv_encoder_chunk_ring stores exactly vkv_encoder_chunk's output rows at
    the 256-row encoder-output ring's logical rows q_start.. (across the wrap
    for 1276: rows 252..255, 0..11) and leaves every other row alone"""
    rng = np.random.default_rng(q_start)
    n_layers = 1
    m = make_model(rng, n_layers)
    model, keep, arr = upload(m)
    x0 = rng.standard_normal((n_new, DIM)).astype(np.float32)
    ca, cb = filled_ring(n_layers, q_start), filled_ring(n_layers, q_start)
    plan = vkv.enc_plan(q_start, n_new, CAP, WIN)
    xa, xb = to_dev(x0), to_dev(x0)
    ws_b = vkv.encoder_chunk_workspace(model, n_new)
    ws = torch.empty(ws_b // 4 + 64, device=dev())
    wsp = (ws.data_ptr() + 255) & ~255
    ring_t = torch.full((256, DIM), np.nan, device=dev())
    ring = vkv.RowRing(ring_t.data_ptr(), 256, DIM)
    vkv.encoder_chunk(ca, 0, plan, WIN, model, xa.data_ptr(), wsp, ws_b, hip_stream=stream_ptr())
    vkv.encoder_chunk_ring(cb, 0, plan, WIN, model, xb.data_ptr(), ring, wsp, ws_b,
                           hip_stream=stream_ptr())
    got, want = host(ring_t), host(xa)
    slots = [(q_start + i) % 256 for i in range(n_new)]
    assert np.array_equal(got[slots], want)
    rest = np.ones(256, bool)
    rest[slots] = False
    assert np.isnan(got[rest]).all()
    # x keeps the residual stream before the final norm
    assert rel(np.stack([oracle.norm_act(r, m["out_norm"], eps=EPS, norm_b=m["out_norm_b"])
                         for r in host(xb)]), want) <= 2e-6
    with pytest.raises(vkv.VkvError):
        vkv.encoder_chunk_ring(cb, 0, plan, WIN, model, xb.data_ptr(),
                               vkv.RowRing(ring_t.data_ptr(), 256, 1024), wsp, ws_b,
                               hip_stream=stream_ptr())
    ca.close()
    cb.close()
    del keep, arr
