"""GPU side of the GGUF loader (voxtral_model_load_from_file,
src/voxtral.cpp:1035-1316): vkv_model_load places every tensor's file bytes in
device memory unchanged, its view maps the reference's tensor names
(:1193-1265) with their types and shapes, and a realtime step run from the
loaded model (conv stem, encoder chunk into the output ring, adapter, decoder
token reading the audio row) equals, bit for bit, the same step run from the
tensors uploaded one by one outside the loader."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import oracle.gguf as og
import vkv
from gguf_util import gguf_bytes, realtime_model
from gpu_util import dev, stream_ptr

pytestmark = pytest.mark.gpu

ENC_L, DEC_L, VOCAB = 1, 2, 1024


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    kvs, tensors = realtime_model(np.random.default_rng(1035), enc_layers=ENC_L, dec_layers=DEC_L,
                                  vocab=VOCAB)
    data = gguf_bytes(kvs, tensors)
    p = tmp_path_factory.mktemp("gguf") / "realtime.gguf"
    p.write_bytes(data)
    return str(p), og.read(data)


@pytest.fixture(scope="module")
def q8_0_file(tmp_path_factory):
    """a Q8_0 file (src/voxtral-quantize.cpp:95-96): every matrix Q8_0"""
    kvs, tensors = realtime_model(np.random.default_rng(95), enc_layers=ENC_L, dec_layers=DEC_L,
                                  vocab=VOCAB, q4=8, q6=8)
    data = gguf_bytes(kvs, tensors)
    p = tmp_path_factory.mktemp("gguf") / "realtime_q8_0.gguf"
    p.write_bytes(data)
    return str(p), og.read(data)


def d2h(ptr, n):
    torch.cuda.synchronize()
    out = torch.empty(n, dtype=torch.uint8)
    hip = ctypes.CDLL("libamdhip64.so")   # the runtime torch has loaded
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(out.data_ptr(), ctypes.c_void_p(ptr), n, 2) == 0
    return out.numpy().tobytes()


def test_device_bytes_are_the_file_bytes(model_file):
    path, g = model_file
    m = vkv.Model(path, hip_stream=stream_ptr())
    base, t0 = m.tensor(g["tensors"][0]["name"])
    assert t0.offset == 0 and base % 256 == 0
    last = g["tensors"][-1]
    n = last["offset"] + last["nbytes"]
    assert m.view.device_bytes >= n
    assert d2h(base, n) == g["data"][g["data_offset"]:g["data_offset"] + n]
    for ti in g["tensors"]:
        p, info = m.tensor(ti["name"])
        assert p == base + ti["offset"] and info.nbytes == ti["nbytes"] and info.type == ti["type"]
    assert m.tensor("absent.weight") == (None, None)
    m.close()


def test_view_maps_the_reference_names(model_file):
    path, g = model_file
    m = vkv.Model(path, hip_stream=stream_ptr())
    v = m.view
    hp = og.hparams(g)
    for f, _ in vkv.Hparams._fields_:
        assert getattr(v.hp, f) == pytest.approx(hp[f], rel=1e-7), f

    def at(name):
        return m.tensor(name)[0]

    def typ(name):
        return m.tensor(name)[1].type

    assert (v.conv0_w, v.conv0_b, v.conv1_w, v.conv1_b) == (
        at("enc.conv0.weight"), at("enc.conv0.bias"), at("enc.conv1.weight"), at("enc.conv1.bias"))
    assert v.mel_filters == at("audio.mel_filters")
    e = v.enc
    assert (e.n_layers, e.dim, e.hidden, e.n_heads, e.head_dim) == (ENC_L, 1280, 5120, 32, 64)
    assert (e.out_norm, e.out_norm_b) == (at("enc.norm.weight"), None)
    for i in range(ENC_L):
        L, p = e.layers[i], f"enc.blk.{i}."
        for field, name in [("attn_norm", "attn_norm.weight"), ("attn_q", "attn_q.weight"),
                            ("attn_k", "attn_k.weight"), ("attn_v", "attn_v.weight"),
                            ("attn_o", "attn_o.weight"), ("attn_q_b", "attn_q.bias"),
                            ("attn_v_b", "attn_v.bias"), ("attn_o_b", "attn_o.bias"),
                            ("ffn_norm", "ffn_norm.weight"), ("ffn_w1", "ffn_w1.weight"),
                            ("ffn_w2", "ffn_w2.weight"), ("ffn_w3", "ffn_w3.weight"),
                            ("ffn_w2_b", "ffn_w2.bias")]:
            assert getattr(L, field) == at(p + name), field
        assert (L.attn_norm_b, L.ffn_norm_b) == (None, None)
        assert (L.attn_q_type, L.attn_v_type, L.ffn_w2_type) == (typ(p + "attn_q.weight"), 14, 14)
    a = v.adapter
    assert (a.w0, a.w2, a.w0_type, a.w2_type, a.enc_dim, a.dec_dim, a.downsample) == (
        at("adapter.0.weight"), at("adapter.2.weight"), 12, 12, 1280, 3072, 4)
    d = v.dec
    assert (d.n_layers, d.dim, d.hidden, d.n_q_heads, d.n_kv_heads, d.head_dim, d.vocab) == (
        DEC_L, 3072, 9216, 32, 8, 128, VOCAB)
    # the realtime model's output is tied to the embeddings
    assert d.tok_embeddings == d.output == at("tok_embeddings.weight")
    assert d.tok_embeddings_type == d.output_type == 14 and d.out_norm == at("norm.weight")
    for i in range(DEC_L):
        L, p = d.layers[i], f"dec.blk.{i}."
        for field, name in [("attn_norm", "attn_norm.weight"), ("attn_q", "attn_q.weight"),
                            ("attn_k", "attn_k.weight"), ("attn_v", "attn_v.weight"),
                            ("attn_o", "attn_o.weight"), ("ffn_norm", "ffn_norm.weight"),
                            ("ffn_w1", "ffn_w1.weight"), ("ffn_w2", "ffn_w2.weight"),
                            ("ffn_w3", "ffn_w3.weight")]:
            assert getattr(L, field) == at(p + name), field
        assert L.ada_scale is None
        assert (L.attn_v_type, L.ffn_w2_type, L.ffn_w1_type) == (14, 14, 12)
    m.close()


def independent(g):
    """the same tensors uploaded one by one (no loader), described by hand
    (types as the file records them)"""
    keep = {}
    types = {ti["name"]: ti["type"] for ti in g["tensors"]}
    for ti in g["tensors"]:
        b = np.frombuffer(og.tensor_bytes(g, ti), np.uint8).copy()
        keep[ti["name"]] = torch.from_numpy(b).to(dev())

    def at(n):
        return keep[n].data_ptr()

    def ty(p, *names):
        return [types[p + n + ".weight"] for n in names]

    el = (vkv.EncLayer * ENC_L)()
    for i in range(ENC_L):
        p = f"enc.blk.{i}."
        el[i] = vkv.EncLayer(at(p + "attn_norm.weight"), None, at(p + "attn_q.weight"),
                             at(p + "attn_k.weight"), at(p + "attn_v.weight"), at(p + "attn_o.weight"),
                             *ty(p, "attn_q", "attn_k", "attn_v", "attn_o"), at(p + "attn_q.bias"),
                             at(p + "attn_v.bias"), at(p + "attn_o.bias"), at(p + "ffn_norm.weight"),
                             None, at(p + "ffn_w1.weight"), at(p + "ffn_w2.weight"),
                             at(p + "ffn_w3.weight"), *ty(p, "ffn_w1", "ffn_w2", "ffn_w3"),
                             at(p + "ffn_w2.bias"))
    enc = vkv.EncModel(ENC_L, 1280, 5120, 32, 64, 1e-5, 1e6, at("enc.norm.weight"), None, el)
    dl = (vkv.DecLayer * DEC_L)()
    for i in range(DEC_L):
        p = f"dec.blk.{i}."
        dl[i] = vkv.DecLayer(at(p + "attn_norm.weight"), at(p + "attn_q.weight"), at(p + "attn_k.weight"),
                             at(p + "attn_v.weight"), at(p + "attn_o.weight"),
                             *ty(p, "attn_q", "attn_k", "attn_v", "attn_o"),
                             at(p + "ffn_norm.weight"), None, at(p + "ffn_w1.weight"),
                             at(p + "ffn_w2.weight"), at(p + "ffn_w3.weight"),
                             *ty(p, "ffn_w1", "ffn_w2", "ffn_w3"))
    tt = types["tok_embeddings.weight"]
    dec = vkv.DecModel(DEC_L, 3072, 9216, 32, 8, 128, VOCAB, 1e-5, 1e6, at("tok_embeddings.weight"), tt,
                       at("norm.weight"), at("tok_embeddings.weight"), tt, dl)
    ad = vkv.Adapter(at("adapter.0.weight"), at("adapter.2.weight"), types["adapter.0.weight"],
                     types["adapter.2.weight"], 1280, 3072, 4)
    conv = (at("enc.conv0.weight"), at("enc.conv0.bias"), at("enc.conv1.weight"), at("enc.conv1.bias"))
    return dict(enc=enc, dec=dec, adapter=ad, conv=conv, keep=(keep, el, dl))


def realtime_step(enc, dec, ad, conv, mel_window, plan):
    """conv stem -> encoder chunk into the output ring -> adapter groups ->
    a two-token decoder prompt over the first audio rows, then one decoder
    token per remaining group reading its audio row; returns the logits of
    the prompt's last token and of every token, and the rings"""
    sp = stream_ptr()
    n = plan.n_new
    ecache = vkv.Cache(n_streams=1, n_layers=ENC_L, capacity=878, n_kv_heads=32,
                       head_dim=64, n_q_heads=32, dtype=vkv.F16)
    dcache = vkv.Cache(n_streams=1, n_layers=DEC_L, capacity=512, n_kv_heads=8, head_dim=128,
                       n_q_heads=32, dtype=vkv.F16)
    ring = vkv.new_ring(512)
    x = torch.empty(n, 1280, device=dev())
    cb = vkv.enc_conv_stem_workspace(mel_window.shape[1], 128, 1280, n)
    cws = torch.empty(cb // 4 + 64, device=dev())
    vkv.enc_conv_stem(mel_window.data_ptr(), 128, plan, conv[0], conv[1], conv[2], conv[3], 1280,
                      x.data_ptr(), (cws.data_ptr() + 255) & ~255, cb, hip_stream=sp)
    enc_out = torch.full((256, 1280), np.nan, device=dev())
    aemb = torch.full((256, 3072), np.nan, device=dev())
    er = vkv.RowRing(enc_out.data_ptr(), 256, 1280)
    ar = vkv.RowRing(aemb.data_ptr(), 256, 3072)
    wb = vkv.encoder_chunk_workspace(enc, n)
    ws = torch.empty(wb // 4 + 64, device=dev())
    vkv.encoder_chunk_ring(ecache, 0, plan, 750, enc, x.data_ptr(), er, (ws.data_ptr() + 255) & ~255,
                           wb, hip_stream=sp)
    groups = n // 4
    ab = vkv.adapter_workspace(ad, groups)
    aws = torch.empty(ab // 4 + 64, device=dev())
    vkv.adapter_commit(ad, er, ar, 0, groups, (aws.data_ptr() + 255) & ~255, ab, hip_stream=sp)
    # the decoder: a two-token prompt at positions 0, 1 (audio rows 0, 1),
    # then one token per remaining group, as the stream decoder runs them
    logits = torch.zeros(groups, VOCAB, device=dev())
    tok = torch.zeros(groups + 1, dtype=torch.int32, device=dev())
    n_prompt = 2
    pb = vkv.decoder_prompt_workspace(dec, n_prompt)
    pws = torch.empty(pb // 4 + 64, device=dev())
    vkv.decoder_prompt(dcache, 0, ring, dec, [1, 5], ar, logits[n_prompt - 1].data_ptr(),
                       tok[n_prompt - 1].data_ptr(), (pws.data_ptr() + 255) & ~255, pb, hip_stream=sp)
    torch.cuda.synchronize()
    token = int(tok[n_prompt - 1].item())
    tb = vkv.decoder_token_workspace(dec)
    tws = torch.empty(tb // 4 + 64, device=dev())
    for p in range(n_prompt, groups):
        vkv.decoder_token(dcache, 0, ring, dec, token, aemb[p % 256].data_ptr(), logits[p].data_ptr(),
                          tok[p].data_ptr(), (tws.data_ptr() + 255) & ~255, tb, hip_stream=sp)
        torch.cuda.synchronize()
        token = int(tok[p].item())
    assert ring.next_absolute_position == groups
    torch.cuda.synchronize()
    out = (logits.cpu().numpy(), tok.cpu().numpy(), enc_out.cpu().numpy(), aemb.cpu().numpy())
    ecache.close()
    dcache.close()
    return out


def test_ada_scales_of_the_loaded_model(model_file):
    """vkv_model_set_ada: every layer's scale equals vkv_ada_scale on that
    layer's weights (bit for bit) and the oracle's within its bound; the
    view's layers point at the rows"""
    path, g = model_file
    m = vkv.Model(path, hip_stream=stream_ptr())
    scales = torch.full((DEC_L, 3072), np.nan, device=dev())
    m.set_ada(6.0, scales.data_ptr(), hip_stream=stream_ptr())
    got = scales.cpu().numpy()
    wb = vkv.ada_scale_workspace(3072, 32)
    ws = torch.empty(wb // 4 + 64, device=dev())
    one = torch.empty(3072, device=dev())
    for l in range(DEC_L):
        assert m.view.dec.layers[l].ada_scale == scales[l].data_ptr()
        a0, i0 = m.tensor(f"dec.blk.{l}.ada0.weight")
        a2, i2 = m.tensor(f"dec.blk.{l}.ada2.weight")
        vkv.ada_scale(a0, i0.type, a2, i2.type, 3072, 32, 6.0, one.data_ptr(),
                      (ws.data_ptr() + 255) & ~255, wb, hip_stream=stream_ptr())
        assert np.array_equal(one.cpu().numpy(), got[l])
        t0 = next(t for t in g["tensors"] if t["name"] == f"dec.blk.{l}.ada0.weight")
        t2 = next(t for t in g["tensors"] if t["name"] == f"dec.blk.{l}.ada2.weight")
        w0 = np.frombuffer(og.tensor_bytes(g, t0), np.uint8)
        w2 = np.frombuffer(og.tensor_bytes(g, t2), np.uint16)
        want = oracle.ada_scale(oracle.Q4_K, w0, w2, 3072, 32, 6.0)
        assert np.abs(got[l] - want).max() <= 1e-3 * max(np.abs(want).max(), 1e-3)
    m.close()


@pytest.mark.parametrize("kind", ["q4km", "q8_0"])
def test_a_realtime_step_from_the_loaded_model(kind, request):
    path, g = request.getfixturevalue("model_file" if kind == "q4km" else "q8_0_file")
    rng = np.random.default_rng(5424)
    plan = vkv.enc_plan(0, 16, 878, 750)
    win = plan.conv_mel_end - plan.conv_mel_start
    mel = torch.from_numpy(rng.uniform(-1.5, 1.5, (128, win)).astype(np.float32)).to(dev())
    m = vkv.Model(path, hip_stream=stream_ptr())
    scales = torch.empty(DEC_L, 3072, device=dev())
    m.set_ada(6.0, scales.data_ptr(), hip_stream=stream_ptr())
    v = m.view
    got = realtime_step(v.enc, v.dec, v.adapter, (v.conv0_w, v.conv0_b, v.conv1_w, v.conv1_b),
                        mel, plan)
    ind = independent(g)
    # the independent side computes its ada scales through vkv_ada_scale
    ind_scales = torch.empty(DEC_L, 3072, device=dev())
    wb = vkv.ada_scale_workspace(3072, 32)
    ws = torch.empty(wb // 4 + 64, device=dev())
    types = {ti["name"]: ti["type"] for ti in g["tensors"]}
    for l in range(DEC_L):
        k = ind["keep"][0]
        a0, a2 = f"dec.blk.{l}.ada0.weight", f"dec.blk.{l}.ada2.weight"
        vkv.ada_scale(k[a0].data_ptr(), types[a0], k[a2].data_ptr(), types[a2], 3072, 32, 6.0,
                      ind_scales[l].data_ptr(), (ws.data_ptr() + 255) & ~255, wb,
                      hip_stream=stream_ptr())
        ind["dec"].layers[l].ada_scale = ind_scales[l].data_ptr()
    want = realtime_step(ind["enc"], ind["dec"], ind["adapter"], ind["conv"], mel, plan)
    for a, b in zip(got, want):
        assert np.array_equal(a, b, equal_nan=True)
    logits, toks, enc_out, aemb = got
    assert np.isfinite(logits).all() and np.isfinite(enc_out[:16]).all() and np.isfinite(aemb[:4]).all()
    assert np.isnan(enc_out[16:]).all() and np.isnan(aemb[4:]).all()
    assert all(0 <= t < VOCAB for t in toks[:4])
    assert np.abs(logits[1:4]).max() > 0     # the prompt's and both tokens' logits were written
    m.close()


def small_file(tmp_path, name, edit=None, arch="voxtral_realtime"):
    from test_gguf import small_model
    kvs, tensors = small_model(np.random.default_rng(7))
    kvs = [(k, t, arch if k == "general.architecture" else v) for k, t, v in kvs]
    if edit:
        tensors = edit(tensors)
    p = tmp_path / name
    p.write_bytes(gguf_bytes(kvs, tensors))
    return str(p)


def test_model_errors(tmp_path):
    """the loader's model errors (voxtral_model_load's MODEL_ERROR): the
    offline architecture, a missing required tensor, a matrix of a type the
    products do not take, Q/K/V mixing Q8_0 with k-quants, a tensor of the
    wrong shape; a small realtime file loads"""
    m = vkv.Model(small_file(tmp_path, "ok.gguf"), hip_stream=stream_ptr())
    assert m.view.hp.dec_dim == 256 and m.view.dec.layers[1].attn_q is not None
    m.close()
    cases = {
        "offline.gguf": (None, "voxtral", "offline"),
        "missing.gguf": (lambda T: [t for t in T if t[0] != "dec.blk.1.ffn_w2.weight"], "voxtral_realtime",
                         "dec.blk.1.ffn_w2.weight"),
        "f16mat.gguf": (lambda T: [(n, 1, ne, np.zeros(ne[0] * ne[1] * 2, np.uint8).tobytes())
                                   if n == "enc.blk.0.attn_o.weight" else (n, t, ne, b)
                                   for n, t, ne, b in T], "voxtral_realtime", "Q6_K and Q8_0"),
        # one product call reads one input image: Q/K/V cannot mix Q8_0 and k-quants
        "mixed.gguf": (lambda T: [(n, 8, ne, np.zeros(ne[1] * (ne[0] // 32) * 34, np.uint8).tobytes())
                                  if n == "enc.blk.0.attn_v.weight" else (n, t, ne, b)
                                  for n, t, ne, b in T], "voxtral_realtime", "mixes Q8_0"),
        "shape.gguf": (lambda T: [(n, t, [ne[0] // 2], b[:len(b) // 2]) if n == "norm.weight"
                                  else (n, t, ne, b) for n, t, ne, b in T], "voxtral_realtime",
                       "norm.weight"),
    }
    for name, (edit, arch, msg) in cases.items():
        with pytest.raises(vkv.VkvError) as ei:
            vkv.Model(small_file(tmp_path, name, edit, arch), hip_stream=stream_ptr())
        assert ei.value.status == vkv.MODEL_ERROR, name
        assert msg in vkv.last_error(), (name, vkv.last_error())


def test_a_q8_0_file_maps_and_conditions(q8_0_file):
    """the view of a Q8_0 file carries Q8_0 for every matrix, and its ada
    scales (ada0 and ada2 both Q8_0) are vkv_ada_scale's and within the
    oracle's bound (ggml's product on q8_0 activations for both layers)"""
    path, g = q8_0_file
    m = vkv.Model(path, hip_stream=stream_ptr())
    v = m.view
    L = v.enc.layers[0]
    assert {L.attn_q_type, L.attn_k_type, L.attn_v_type, L.attn_o_type, L.ffn_w1_type,
            L.ffn_w2_type, L.ffn_w3_type} == {vkv.Q8_0}
    assert (v.adapter.w0_type, v.adapter.w2_type) == (vkv.Q8_0, vkv.Q8_0)
    assert v.dec.tok_embeddings_type == v.dec.output_type == vkv.Q8_0
    for l in range(DEC_L):
        D = v.dec.layers[l]
        assert {D.attn_q_type, D.attn_v_type, D.ffn_w1_type, D.ffn_w2_type} == {vkv.Q8_0}
    scales = torch.full((DEC_L, 3072), np.nan, device=dev())
    m.set_ada(6.0, scales.data_ptr(), hip_stream=stream_ptr())
    got = scales.cpu().numpy()
    for l in range(DEC_L):
        t0 = next(t for t in g["tensors"] if t["name"] == f"dec.blk.{l}.ada0.weight")
        t2 = next(t for t in g["tensors"] if t["name"] == f"dec.blk.{l}.ada2.weight")
        assert t0["type"] == t2["type"] == vkv.Q8_0
        w0 = np.frombuffer(og.tensor_bytes(g, t0), np.uint8)
        w2 = np.frombuffer(og.tensor_bytes(g, t2), np.uint8)
        want = oracle.ada_scale(oracle.Q8_0, w0, w2, 3072, 32, 6.0)
        assert np.abs(want).max() > 1e-3
        assert np.abs(got[l] - want).max() <= 1e-3 * np.abs(want).max()
    m.close()


def test_two_stream_pipelined_steps_equal_the_single_stream_order(model_file):
    """The realtime steps scheduled on two HIP streams, the decoder one group
    behind the encoder (step i's encoder + adapter on one stream while token
    i, on the other, reads step i-1's audio row; events order the chains):
    every token's logits, the tokens, the decoder cache and the rings equal
    the same steps issued in that order on one stream, bit for bit.  No host
    synchronization inside the loop, so a missing wait would show as a race."""
    path, g = model_file
    rng = np.random.default_rng(80)
    S = 12
    plans = [vkv.enc_plan(4 * i, 4, 878, 750) for i in range(S)]
    mel_all = rng.uniform(-1.5, 1.5, (128, plans[-1].conv_mel_end)).astype(np.float32)
    mels = [torch.from_numpy(np.ascontiguousarray(mel_all[:, p.conv_mel_start:p.conv_mel_end]))
            .to(dev()) for p in plans]
    m = vkv.Model(path, hip_stream=stream_ptr())
    scales = torch.empty(DEC_L, 3072, device=dev())
    m.set_ada(6.0, scales.data_ptr(), hip_stream=stream_ptr())
    v = m.view
    al = lambda t: (t.data_ptr() + 255) & ~255   # noqa: E731

    def run(two):
        s0 = torch.cuda.current_stream()
        s1 = torch.cuda.Stream() if two else s0
        ecache = vkv.Cache(n_streams=1, n_layers=ENC_L, capacity=878, n_kv_heads=32, head_dim=64,
                           n_q_heads=32, dtype=vkv.F16)
        dcache = vkv.Cache(n_streams=1, n_layers=DEC_L, capacity=512, n_kv_heads=8, head_dim=128,
                           n_q_heads=32, dtype=vkv.F16)
        ring = vkv.new_ring(512)
        x = torch.empty(4, 1280, device=dev())
        cb = max(vkv.enc_conv_stem_workspace(p.conv_mel_end - p.conv_mel_start, 128, 1280, 4)
                 for p in plans)
        cws = torch.empty(cb // 4 + 64, device=dev())
        enc_out = torch.full((256, 1280), np.nan, device=dev())
        aemb = torch.full((256, 3072), np.nan, device=dev())
        er, ar = vkv.RowRing(enc_out.data_ptr(), 256, 1280), vkv.RowRing(aemb.data_ptr(), 256, 3072)
        ewb = vkv.encoder_chunk_workspace(v.enc, 4)
        ews = torch.empty(ewb // 4 + 64, device=dev())
        awb = vkv.adapter_workspace(v.adapter, 1)
        aws = torch.empty(awb // 4 + 64, device=dev())
        twb = vkv.decoder_token_workspace(v.dec)
        tws = torch.empty(twb // 4 + 64, device=dev())
        logits = torch.zeros(S, VOCAB, device=dev())
        toks = torch.zeros(S, dtype=torch.int32, device=dev())
        ev_a = [torch.cuda.Event() for _ in range(S)]
        ev_d = [torch.cuda.Event() for _ in range(S)]
        torch.cuda.synchronize()
        for i, p in enumerate(plans):
            if two and i > 1:
                s0.wait_event(ev_d[i - 1])
            vkv.enc_conv_stem(mels[i].data_ptr(), 128, p, v.conv0_w, v.conv0_b, v.conv1_w, v.conv1_b,
                              1280, x.data_ptr(), al(cws), cb, hip_stream=s0.cuda_stream)
            vkv.encoder_chunk_ring(ecache, 0, p, 750, v.enc, x.data_ptr(), er, al(ews), ewb,
                                   hip_stream=s0.cuda_stream)
            vkv.adapter_commit(v.adapter, er, ar, i, 1, al(aws), awb, hip_stream=s0.cuda_stream)
            ev_a[i].record(s0)
            if i == 0:
                continue
            s1.wait_event(ev_a[i - 1])
            vkv.decoder_token(dcache, 0, ring, v.dec, 7 + i, aemb[i - 1].data_ptr(),
                              logits[i].data_ptr(), toks[i].data_ptr(), al(tws), twb,
                              hip_stream=s1.cuda_stream)
            ev_d[i].record(s1)
        torch.cuda.synchronize()
        out = (logits.cpu().numpy(), toks.cpu().numpy(), enc_out.cpu().numpy(), aemb.cpu().numpy(),
               [layer_bytes(dcache, w, l) for w in (0, 1) for l in range(DEC_L)])
        ecache.close()
        dcache.close()
        return out

    one, two = run(False), run(True)
    for a, b in zip(one[:4], two[:4]):
        assert np.array_equal(a, b, equal_nan=True)
    for a, b in zip(one[4], two[4]):
        assert np.array_equal(a, b)
    assert np.isfinite(one[0][1:]).all() and np.abs(one[0][1:]).max() > 0
    m.close()


def layer_bytes(cache, which, layer):
    from gpu_util import layer_image
    return layer_image(cache, which, 0, layer).copy()
