"""A GGUF v3 writer for the tests (the layout tools/convert_voxtral_to_gguf.py
writes: metadata, tensor infos, zero padding to the alignment, tensors at
their packed aligned offsets), and a synthetic realtime model with the
reference's tensor names and metadata keys."""
import struct

import numpy as np

from kq_util import random_matrix

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
TYPE_BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def _str(b):
    b = b.encode() if isinstance(b, str) else bytes(b)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, vals = v
        out = struct.pack("<IQ", et, len(vals))
        if et == STR:
            return out + b"".join(_str(x) for x in vals)
        return out + b"".join(struct.pack(_FMT[et], x) for x in vals)
    return struct.pack(_FMT[t], v)


def nbytes(ggml_type, ne):
    blk, bb = TYPE_BLOCK[ggml_type]
    n = 1
    for d in ne:
        n *= d
    return n // blk * bb


def gguf_bytes(kvs, tensors, alignment=32, version=3):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, ne, bytes)]"""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    off, offs = 0, []
    for name, t, ne, data in tensors:
        assert len(data) == nbytes(t, ne), name
        offs.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, t, ne, data), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", t, o)
    out = bytearray(head)
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (name, t, ne, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += data
    return bytes(out)


def realtime_model(rng, enc_layers=1, dec_layers=2, vocab=1024, enc=1280, dec=3072, n_mel=128,
                   enc_heads=32, enc_hd=64, enc_hidden=5120, dec_heads=32, dec_kv=8, dec_hd=128,
                   dec_hidden=9216, q4=12, q6=14):
    """kvs and tensors of a realtime model in the Q4_K_M mix
    (src/voxtral-quantize.cpp:148-159: attn_v, ffn_w2, tok_embeddings Q6_K;
    other matrices Q4_K), random valid blocks at sizes that keep the
    activations finite.  q4 = q6 = 8 gives a Q8_0 file (:95-96): every
    matrix Q8_0, ada2 included (its 32-wide rows are whole Q8_0 blocks,
    :161-164, :410)."""
    kvs = [("general.architecture", STR, "voxtral_realtime"),
           ("general.name", STR, "Voxtral-Mini-4B-Realtime-2602"),
           ("general.file_type", U32, 1),
           ("voxtral.decoder.dim", I32, dec), ("voxtral.decoder.n_layers", I32, dec_layers),
           ("voxtral.decoder.n_heads", I32, dec_heads), ("voxtral.decoder.head_dim", I32, dec_hd),
           ("voxtral.decoder.hidden_dim", I32, dec_hidden),
           ("voxtral.decoder.n_kv_heads", I32, dec_kv),
           ("voxtral.decoder.norm_eps", F32, 1e-5), ("voxtral.decoder.rope_theta", F32, 1e6),
           ("voxtral.encoder.dim", I32, enc), ("voxtral.encoder.n_layers", I32, enc_layers),
           ("voxtral.encoder.n_heads", I32, enc_heads), ("voxtral.encoder.head_dim", I32, enc_hd),
           ("voxtral.encoder.hidden_dim", I32, enc_hidden),
           ("voxtral.encoder.n_kv_heads", I32, enc_heads),
           ("voxtral.encoder.norm_eps", F32, 1e-5), ("voxtral.encoder.rope_theta", F32, 1e6),
           ("voxtral.encoder.causal", BOOL, True), ("voxtral.ada_rms_norm_t_cond", BOOL, True),
           ("voxtral.vocab_size", I32, vocab), ("voxtral.audio.downsample_factor", I32, 4),
           ("voxtral.token.bos", I32, 1), ("voxtral.token.eos", I32, 2),
           ("voxtral.token.audio", I32, 24), ("voxtral.token.begin_audio", I32, 25),
           ("voxtral.tokenizer.special_token_ranks", ARR, (I32, list(range(8)))),
           ("voxtral.tokenizer.vocab_token_bytes_b64", ARR, (STR, ["YQ==", "Yg==", "Yw=="]))]
    T = []

    def vec(name, n, lo=-0.1, hi=0.1):
        T.append((name, 0, [n], rng.uniform(lo, hi, n).astype(np.float32).tobytes()))

    def mat(name, t, rows, n_in, scale):
        T.append((name, t, [n_in, rows], random_matrix(rng, t, rows, n_in, scale).tobytes()))

    def conv(name, cin, cout):
        w = (rng.standard_normal((cout, cin, 3)) * 0.05).astype(np.float16)
        T.append((name, 1, [3, cin, cout], w.tobytes()))

    eq = enc_heads * enc_hd
    conv("enc.conv0.weight", n_mel, enc)
    vec("enc.conv0.bias", enc)
    conv("enc.conv1.weight", enc, enc)
    vec("enc.conv1.bias", enc)
    for i in range(enc_layers):
        p = f"enc.blk.{i}."
        vec(p + "attn_norm.weight", enc, 0.5, 1.5)
        mat(p + "attn_q.weight", q4, eq, enc, 0.01)
        vec(p + "attn_q.bias", eq)
        mat(p + "attn_k.weight", q4, eq, enc, 0.01)
        mat(p + "attn_v.weight", q6, eq, enc, 0.1)
        vec(p + "attn_v.bias", eq)
        mat(p + "attn_o.weight", q4, enc, eq, 0.01)
        vec(p + "attn_o.bias", enc)
        vec(p + "ffn_norm.weight", enc, 0.5, 1.5)
        mat(p + "ffn_w1.weight", q4, enc_hidden, enc, 0.005)
        mat(p + "ffn_w2.weight", q6, enc, enc_hidden, 0.05)
        vec(p + "ffn_w2.bias", enc)
        mat(p + "ffn_w3.weight", q4, enc_hidden, enc, 0.005)
    vec("enc.norm.weight", enc, 0.5, 1.5)
    mat("adapter.0.weight", q4, dec, enc * 4, 0.03)
    mat("adapter.2.weight", q4, dec, dec, 0.05)
    mat("tok_embeddings.weight", q6, vocab, dec, 1.0)
    vec("norm.weight", dec, 0.5, 1.5)
    for i in range(dec_layers):
        p = f"dec.blk.{i}."
        vec(p + "attn_norm.weight", dec, 0.5, 1.5)
        mat(p + "attn_q.weight", q4, dec_heads * dec_hd, dec, 0.01)
        mat(p + "attn_k.weight", q4, dec_kv * dec_hd, dec, 0.01)
        mat(p + "attn_v.weight", q6, dec_kv * dec_hd, dec, 0.1)
        mat(p + "attn_o.weight", q4, dec, dec_heads * dec_hd, 0.01)
        vec(p + "ffn_norm.weight", dec, 0.5, 1.5)
        mat(p + "ffn_w1.weight", q4, dec_hidden, dec, 0.005)
        mat(p + "ffn_w2.weight", q6, dec, dec_hidden, 0.05)
        mat(p + "ffn_w3.weight", q4, dec_hidden, dec, 0.005)
        mat(p + "ada0.weight", q4, 32, dec, 0.002)
        if q4 == 8:
            mat(p + "ada2.weight", 8, dec, 32, 0.02)
        else:
            T.append((p + "ada2.weight", 1, [32, dec],
                      (rng.standard_normal((dec, 32)) * 0.01).astype(np.float16).tobytes()))
    T.append(("audio.mel_filters", 0, [201, n_mel],
              rng.uniform(0, 0.01, 201 * n_mel).astype(np.float32).tobytes()))
    return kvs, T
