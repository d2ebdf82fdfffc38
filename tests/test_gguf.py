"""GGUF model files: the oracle's reader (oracle/gguf.py) and the library's
(vkv_gguf_*, vkv_model_load's file side), after voxtral_model_load_from_file
(src/voxtral.cpp:1035-1316) over ggml's gguf reader and the layout
tools/convert_voxtral_to_gguf.py:839-905 writes.

The oracle is pinned by a file assembled byte by byte here (each header field
a literal), by round trips through the tests' own writer for every value and
tensor type, and by rejecting every truncation and each malformation ggml's
reader rejects.  The library must agree with it on all of them, and its
hyperparameters with the reference's defaults and overrides."""
import os
import struct

import numpy as np
import pytest

import oracle.gguf as og
import vkv
from gguf_util import (ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64,
                       gguf_bytes, realtime_model)


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def le(v, n):
    return int(v).to_bytes(n, "little", signed=v < 0)


def hand_file():
    """one int32, one string, one f32 tensor [4, 2] -- every field a literal"""
    h = b"GGUF" + le(3, 4) + le(1, 8) + le(2, 8)
    h += le(11, 8) + b"voxtral.x.y" + le(5, 4) + b"\xff\xff\xff\xff"
    h += le(3, 8) + b"str" + le(8, 4) + le(2, 8) + b"hi"
    h += le(1, 8) + b"t" + le(2, 4) + le(4, 8) + le(2, 8) + le(0, 4) + le(0, 8)
    pad = (-len(h)) % 32
    body = struct.pack("<8f", *range(8))
    return h + b"\0" * pad + body, len(h) + pad


def test_oracle_reads_a_file_assembled_by_hand(tmp_path):
    data, data_off = hand_file()
    g = og.read(data)
    assert g["version"] == 3 and g["alignment"] == 32 and g["data_offset"] == data_off
    assert g["kv"] == {"voxtral.x.y": (5, -1), "str": (8, b"hi")}
    (t,) = g["tensors"]
    assert (t["name"], t["type"], t["ne"], t["n_dims"], t["offset"], t["nbytes"]) == ("t", 0, [4, 2, 1, 1], 2, 0, 32)
    assert og.tensor_bytes(g, t) == struct.pack("<8f", *range(8))
    G = vkv.Gguf(write(tmp_path, "hand.gguf", data))
    assert (G.version, G.alignment, G.data_offset) == (3, 32, data_off)
    assert G.keys() == ["voxtral.x.y", "str"]
    assert G.value("voxtral.x.y") == (5, -1) and G.value("str") == (8, b"hi")
    (ti,) = G.tensors()
    assert (ti.name, ti.type, ti.n_dims, list(ti.ne), ti.offset, ti.nbytes) == (b"t", 0, 2, [4, 2, 1, 1], 0, 32)
    assert G.tensor_bytes(0) == struct.pack("<8f", *range(8))
    G.close()


def every_type_file(alignment=64):
    rng = np.random.default_rng(7)
    kvs = [("general.alignment", U32, alignment), ("u8", U8, 255), ("i8", I8, -128),
           ("u16", U16, 65535), ("i16", I16, -32768), ("u32", U32, 2**32 - 1),
           ("i32", I32, -2**31), ("f32", F32, 1.5), ("bool", BOOL, True), ("bool0", BOOL, False),
           ("str", STR, "voxtral — ü"), ("u64", U64, 2**64 - 1), ("i64", I64, -2**63),
           ("f64", F64, -2.25), ("empty", STR, ""),
           ("arr_i32", ARR, (I32, [1, -2, 3])), ("arr_f32", ARR, (F32, [0.5, -1.0])),
           ("arr_u8", ARR, (U8, [1, 2, 3, 4, 5])), ("arr_i64", ARR, (I64, [-5])),
           ("arr_f64", ARR, (F64, [3.25, 4.5])), ("arr_bool", ARR, (BOOL, [True, False, True])),
           ("arr_str", ARR, (STR, ["a", "", "bcd"])), ("arr_empty", ARR, (I32, []))]
    tensors = [("f32v", 0, [5], rng.standard_normal(5).astype(np.float32).tobytes()),
               ("f16m", 1, [3, 2], rng.standard_normal(6).astype(np.float16).tobytes()),
               ("q8", 8, [64, 3], rng.integers(0, 256, 3 * 2 * 34, dtype=np.uint8).tobytes()),
               ("q4k", 12, [256, 2, 1], rng.integers(0, 256, 2 * 144, dtype=np.uint8).tobytes()),
               ("q6k", 14, [512, 1, 1, 2], rng.integers(0, 256, 2 * 2 * 210, dtype=np.uint8).tobytes())]
    return kvs, tensors


def test_round_trip_every_value_and_tensor_type(tmp_path):
    kvs, tensors = every_type_file()
    data = gguf_bytes(kvs, tensors, alignment=64)
    g = og.read(data)
    assert g["alignment"] == 64 and g["data_offset"] % 64 == 0
    G = vkv.Gguf(write(tmp_path, "all.gguf", data))
    assert G.alignment == 64 and G.data_offset == g["data_offset"]
    assert G.keys() == [k for k, _, _ in kvs]
    for k, t, v in kvs:
        ot, ov = g["kv"][k]
        ct, cv = G.value(k)
        assert ot == ct == t, k
        if t == STR:
            assert ov == cv == v.encode()
        elif t == ARR:
            et, vals = v
            assert ov[0] == cv[0] == et
            if et == STR:
                assert ov[1] == cv[1] == [x.encode() for x in vals]
            else:
                assert list(ov[1]) == list(cv[1]) == list(vals)
        else:
            assert ov == cv == v, k
    for i, (name, t, ne, b) in enumerate(tensors):
        ot, ct = g["tensors"][i], G.tensors()[i]
        assert ot["name"] == ct.name.decode() == name and ot["type"] == ct.type == t
        assert ot["ne"] == list(ct.ne) == ne + [1] * (4 - len(ne)) and ot["n_dims"] == ct.n_dims == len(ne)
        assert ot["offset"] == ct.offset and ot["offset"] % 64 == 0
        assert og.tensor_bytes(g, ot) == G.tensor_bytes(i) == b
    # typed getters reject other types, as ggml's gguf_get_val_* assert
    with pytest.raises(vkv.VkvError):
        vkv.check(vkv.lib.vkv_gguf_get_i32(G.handle, G.find_key("u32"), vkv.ctypes.byref(vkv.ctypes.c_int32())))
    assert G.find_key("absent") == -1 and vkv.lib.vkv_gguf_find_tensor(G.handle, b"absent") == -1
    G.close()


def rejected(tmp_path, data, name="bad.gguf"):
    with pytest.raises(og.GgufError):
        og.read(data)
    with pytest.raises(vkv.VkvError) as ei:
        vkv.Gguf(write(tmp_path, name, data))
    assert ei.value.status == vkv.MODEL_ERROR
    return vkv.last_error()


def test_every_truncation_is_rejected(tmp_path):
    kvs, tensors = every_type_file(alignment=32)
    data = gguf_bytes(kvs, tensors)
    g = og.read(data)
    last = g["tensors"][-1]
    end = g["data_offset"] + last["offset"] + last["nbytes"]
    assert end == len(data)   # no padding after the last tensor in this file
    for n in range(0, end, 7):
        rejected(tmp_path, data[:n], f"t{n}.gguf")
    rejected(tmp_path, data[:end - 1])
    # trailing padding of the last tensor is optional
    og.read(data + b"\0" * 5)
    vkv.Gguf(write(tmp_path, "pad.gguf", data + b"\0" * 5)).close()


def test_malformed_files_are_rejected(tmp_path):
    kvs, tensors = every_type_file(alignment=32)
    good = gguf_bytes(kvs, tensors)
    assert "magic" in rejected(tmp_path, b"GGUX" + good[4:])
    assert "version 1" in rejected(tmp_path, good[:4] + le(1, 4) + good[8:])
    rejected(tmp_path, good[:4] + le(4, 4) + good[8:])
    assert "duplicate key" in rejected(tmp_path, gguf_bytes(kvs + [("u8", U8, 1)], tensors))
    assert "duplicate tensor" in rejected(tmp_path, gguf_bytes(kvs, tensors + [tensors[0]]))
    five = [("t5", 0, [1, 1, 1, 1, 2], b"\0" * 8)]
    assert "dims" in rejected(tmp_path, gguf_bytes([], five))
    assert "alignment" in rejected(tmp_path, gguf_bytes([("general.alignment", U32, 48)], []))
    assert "alignment" in rejected(tmp_path, gguf_bytes([("general.alignment", I32, 64)], []))
    assert "63 bytes" in rejected(tmp_path, gguf_bytes([], [("n" * 64, 0, [1], b"\0" * 4)]))
    # an unknown ggml type and a misplaced offset, patched into a valid file
    one = gguf_bytes([], [("a", 0, [8], b"\0" * 32), ("b", 0, [8], b"\0" * 32)])
    i = one.index(b"\x01\x00\x00\x00\x00\x00\x00\x00b") + 9   # tensor "b": n_dims
    t_at = i + 4 + 8
    assert "type" in rejected(tmp_path, one[:t_at] + le(99, 4) + one[t_at + 4:])
    assert "offset" in rejected(tmp_path, one[:t_at + 4] + le(64, 8) + one[t_at + 12:])


def test_ne0_must_be_a_whole_number_of_blocks(tmp_path):
    # Q4_K [128, 2]: 128 is not a multiple of 256; written with the byte
    # count of one block so that only the ne[0] rule fails
    h = b"GGUF" + le(3, 4) + le(1, 8) + le(0, 8)
    h += le(1, 8) + b"q" + le(2, 4) + le(128, 8) + le(2, 8) + le(12, 4) + le(0, 8)
    data = h + b"\0" * ((-len(h)) % 32) + b"\0" * 144
    assert "multiple" in rejected(tmp_path, data)


def small_model(rng, **kw):
    return realtime_model(rng, enc_layers=2, dec_layers=2, vocab=256, enc=256, dec=256, n_mel=16,
                          enc_heads=4, enc_hd=64, enc_hidden=512, dec_heads=2, dec_kv=1,
                          dec_hd=128, dec_hidden=512, **kw)


def test_library_reader_matches_the_oracle_on_a_realtime_model(tmp_path):
    kvs, tensors = small_model(np.random.default_rng(1035))
    data = gguf_bytes(kvs, tensors)
    g = og.read(data)
    G = vkv.Gguf(write(tmp_path, "rt.gguf", data))
    assert G.keys() == list(g["kv"].keys())
    for k, (t, v) in g["kv"].items():
        ct, cv = G.value(k)
        assert ct == t
        if t == ARR:
            assert cv[0] == v[0] and list(cv[1]) == list(v[1])
        elif t == F32:
            assert cv == v
        else:
            assert cv == v, k
    for i, ot in enumerate(g["tensors"]):
        ct = G.tensors()[i]
        assert (ct.name.decode(), ct.type, list(ct.ne), ct.offset, ct.nbytes) == \
            (ot["name"], ot["type"], ot["ne"], ot["offset"], ot["nbytes"])
        assert G.tensor_bytes(i) == og.tensor_bytes(g, ot)
    hp = G.hparams()
    want = og.hparams(g)
    for f, _ in vkv.Hparams._fields_:
        assert getattr(hp, f) == pytest.approx(want[f], rel=0, abs=0), f
    names = {t["name"] for t in g["tensors"]}
    assert all(n in names for n, req in og.realtime_tensors(want) if req)
    G.close()


def hp_of(tmp_path, kvs):
    G = vkv.Gguf(write(tmp_path, "hp.gguf", gguf_bytes(kvs, [])))
    try:
        return {f: getattr(G.hparams(), f) for f, _ in vkv.Hparams._fields_}
    finally:
        G.close()


def test_hparams_defaults_and_overrides(tmp_path):
    # include/voxtral.h:38-78 when no key is present
    d = hp_of(tmp_path, [])
    assert d == pytest.approx(og.DEFAULTS)
    assert (d["enc_dim"], d["dec_layers"], d["dec_kv_heads"], d["vocab_size"], d["tok_audio"]) == \
        (1280, 26, 8, 131072, 24)
    assert d["enc_causal"] == 1 and d["ada_t_cond"] == 1 and d["is_offline"] == 0
    # the offline architecture flips the two defaults; explicit keys win
    off = hp_of(tmp_path, [("general.architecture", STR, "voxtral")])
    assert (off["is_offline"], off["enc_causal"], off["ada_t_cond"]) == (1, 0, 0)
    both = hp_of(tmp_path, [("general.architecture", STR, "voxtral"),
                            ("voxtral.encoder.causal", BOOL, True),
                            ("voxtral.ada_rms_norm_t_cond", BOOL, True)])
    assert (both["enc_causal"], both["ada_t_cond"]) == (1, 1)
    # the params.* key is read after voxtral.encoder.causal (src/voxtral.cpp:1093-1094)
    later = hp_of(tmp_path, [("voxtral.encoder.causal", BOOL, True),
                             ("voxtral.params.multimodal.whisper_model_args.encoder_args.causal", BOOL, False)])
    assert later["enc_causal"] == 0
    kv = [("voxtral.decoder.dim", I32, 512), ("voxtral.encoder.rope_theta", F32, 123.5),
          ("voxtral.token.begin_audio", I32, 99), ("voxtral.audio.downsample_factor", I32, 2)]
    o = hp_of(tmp_path, kv)
    assert (o["dec_dim"], o["enc_rope_theta"], o["tok_begin_audio"], o["downsample_factor"]) == (512, 123.5, 99, 2)
    assert o == pytest.approx(og.hparams(og.read(gguf_bytes(kv, []))))


def test_hparams_reject_a_key_of_another_type(tmp_path):
    data = gguf_bytes([("voxtral.decoder.dim", U32, 512)], [])
    G = vkv.Gguf(write(tmp_path, "ty.gguf", data))
    with pytest.raises(vkv.VkvError) as ei:
        G.hparams()
    assert ei.value.status == vkv.MODEL_ERROR and "type" in vkv.last_error()
    with pytest.raises(og.GgufError):
        og.hparams(og.read(data))
    G.close()


def test_model_load_rejects_bad_files_before_touching_a_device(tmp_path):
    with pytest.raises(vkv.VkvError) as ei:
        vkv.Model(str(tmp_path / "missing.gguf"))
    assert ei.value.status == vkv.MODEL_ERROR
    p = write(tmp_path, "ty.gguf", gguf_bytes([("voxtral.decoder.dim", U32, 512)], []))
    with pytest.raises(vkv.VkvError) as ei:
        vkv.Model(p)
    assert ei.value.status == vkv.MODEL_ERROR
    assert not os.path.exists(str(tmp_path / "missing.gguf"))


def test_huge_tensor_sizes_do_not_wrap(tmp_path):
    """An F32 tensor claiming 2^62 - 1 elements over no data bytes: its byte
    count (2^64 - 4) and its padded size would wrap a 64-bit sum; both
    readers reject the file instead of exposing the tensor."""
    for ne0 in (2 ** 62 - 1, 2 ** 62 - 8, 2 ** 61 + 3):
        h = b"GGUF" + le(3, 4) + le(1, 8) + le(0, 8)
        h += le(1, 8) + b"h" + le(1, 4) + le(ne0, 8) + le(0, 4) + le(0, 8)
        data = h + b"\0" * ((-len(h)) % 32) + b"\0" * 64
        msg = rejected(tmp_path, data, f"huge{ne0 % 97}.gguf")
        assert "too large" in msg or "past the end" in msg
