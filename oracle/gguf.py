"""Oracle: GGUF model files (TEST INFRASTRUCTURE ONLY).

A restatement of what voxtral_model_load_from_file (src/voxtral.cpp:1035-1316)
obtains from a file through ggml's gguf reader (ggml @ 5cecdad6, gguf.cpp, not
in the reference tree; its published GGUF v3 layout is also what
tools/convert_voxtral_to_gguf.py:839-905 writes and :907-957 reads back):

  "GGUF", u32 version, u64 n_tensors, u64 n_kv,
  n_kv x (string key, u32 type, value), n_tensors x (string name, u32 n_dims,
  u64 ne[n_dims], u32 ggml_type, u64 offset), zero padding to the alignment
  (general.alignment, u32, default 32), the data section: tensor i at offset
  sum_{j<i} pad(nbytes_j), nbytes = ne0 * ... / block * block_bytes.

Strings are u64 length + bytes.  Rejections follow ggml's reader: version 1
or > 3, duplicate keys or tensor names, more than 4 dims, ne[0] not a multiple
of the type's block, an offset other than the packed one, a tensor outside
the file.  hparams() restates the reference's metadata population with the
include/voxtral.h defaults (src/voxtral.cpp:1066-1113); realtime_tensors()
lists the tensors the realtime model maps (src/voxtral.cpp:1193-1265).

Pinned by tests/test_gguf.py: a file assembled byte by byte in the test
(every header field written as a literal), round trips through an independent
writer for every value type, and every prefix of a valid file rejected."""
import struct

BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
         14: (256, 210), 15: (256, 292), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8),
         28: (1, 8), 30: (1, 2)}
SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
          11: "<q", 12: "<d"}
STRING, ARRAY = 8, 9


class GgufError(ValueError):
    pass


def read(path_or_bytes):
    """dict(version, alignment, data_offset, kv={key: (type, value)},
    tensors=[dict(name, type, ne, offset, nbytes)], data=bytes of the file)"""
    data = path_or_bytes if isinstance(path_or_bytes, (bytes, bytearray)) else open(path_or_bytes, "rb").read()
    pos = 0

    def need(n):
        if pos + n > len(data):
            raise GgufError("truncated")

    def u(fmt):
        nonlocal pos
        n = struct.calcsize(fmt)
        need(n)
        v = struct.unpack_from(fmt, data, pos)[0]
        pos += n
        return v

    def s():
        nonlocal pos
        n = u("<Q")
        need(n)
        v = bytes(data[pos:pos + n])
        pos += n
        return v

    need(4)
    if data[:4] != b"GGUF":
        raise GgufError("bad magic")
    pos = 4
    version = u("<I")
    if version == 1 or version == 0 or version > 3:
        raise GgufError(f"version {version}")
    n_tensors, n_kv = u("<Q"), u("<Q")
    kv = {}
    for _ in range(n_kv):
        key = s().decode()
        t = u("<I")
        if t == STRING:
            val = s()
        elif t == ARRAY:
            et, n = u("<I"), u("<Q")
            if et == STRING:
                val = (et, [s() for _ in range(n)])
            elif et in SCALAR:
                val = (et, [u(SCALAR[et]) for _ in range(n)])
            else:
                raise GgufError(f"array of type {et}")
        elif t in SCALAR:
            val = u(SCALAR[t])
        else:
            raise GgufError(f"type {t}")
        if key in kv:
            raise GgufError(f"duplicate key {key}")
        kv[key] = (t, val)
    alignment = 32
    if "general.alignment" in kv:
        t, a = kv["general.alignment"]
        if t != 4 or a == 0 or a & (a - 1):
            raise GgufError("alignment")
        alignment = a
    tensors, names, packed = [], set(), 0
    for _ in range(n_tensors):
        name = s().decode()
        nd = u("<I")
        if nd > 4:
            raise GgufError(f"{name}: {nd} dims")
        ne = [u("<Q") for _ in range(nd)]
        t, off = u("<I"), u("<Q")
        if t not in BLOCK:
            raise GgufError(f"{name}: type {t}")
        blk, bb = BLOCK[t]
        if ne and ne[0] % blk:
            raise GgufError(f"{name}: ne0")
        elems = 1
        for d in ne:
            elems *= d
        nbytes = elems // blk * bb
        if off != packed:
            raise GgufError(f"{name}: offset {off} != {packed}")
        if name in names or len(name) >= 64:
            raise GgufError(f"tensor name {name}")
        names.add(name)
        packed += (nbytes + alignment - 1) // alignment * alignment
        tensors.append(dict(name=name, type=t, ne=ne + [1] * (4 - nd), n_dims=nd, offset=off,
                            nbytes=nbytes))
    data_offset = (pos + alignment - 1) // alignment * alignment
    for ti in tensors:
        if data_offset + ti["offset"] + ti["nbytes"] > len(data):
            raise GgufError(f"{ti['name']} past the end")
    return dict(version=version, alignment=alignment, data_offset=data_offset, kv=kv,
                tensors=tensors, data=bytes(data))


def tensor_bytes(g, ti):
    o = g["data_offset"] + ti["offset"]
    return g["data"][o:o + ti["nbytes"]]


DEFAULTS = dict(is_offline=0, enc_dim=1280, enc_layers=32, enc_heads=32, enc_head_dim=64,
                enc_hidden=5120, enc_kv_heads=32, enc_causal=1, enc_norm_eps=1e-5,
                enc_rope_theta=1e6, dec_dim=3072, dec_layers=26, dec_heads=32, dec_head_dim=128,
                dec_hidden=9216, dec_kv_heads=8, dec_norm_eps=1e-5, dec_rope_theta=1e6,
                ada_t_cond=1, vocab_size=131072, downsample_factor=4, tok_bos=1, tok_eos=2,
                tok_audio=24, tok_begin_audio=25)

_I32_KEYS = [("enc_dim", "voxtral.encoder.dim"), ("enc_layers", "voxtral.encoder.n_layers"),
             ("enc_heads", "voxtral.encoder.n_heads"), ("enc_head_dim", "voxtral.encoder.head_dim"),
             ("enc_hidden", "voxtral.encoder.hidden_dim"),
             ("enc_kv_heads", "voxtral.encoder.n_kv_heads"),
             ("dec_dim", "voxtral.decoder.dim"), ("dec_layers", "voxtral.decoder.n_layers"),
             ("dec_heads", "voxtral.decoder.n_heads"), ("dec_head_dim", "voxtral.decoder.head_dim"),
             ("dec_hidden", "voxtral.decoder.hidden_dim"),
             ("dec_kv_heads", "voxtral.decoder.n_kv_heads"), ("vocab_size", "voxtral.vocab_size"),
             ("downsample_factor", "voxtral.audio.downsample_factor"),
             ("tok_bos", "voxtral.token.bos"), ("tok_eos", "voxtral.token.eos"),
             ("tok_audio", "voxtral.token.audio"), ("tok_begin_audio", "voxtral.token.begin_audio")]
_F32_KEYS = [("enc_norm_eps", "voxtral.encoder.norm_eps"),
             ("enc_rope_theta", "voxtral.encoder.rope_theta"),
             ("dec_norm_eps", "voxtral.decoder.norm_eps"),
             ("dec_rope_theta", "voxtral.decoder.rope_theta")]


def hparams(g):
    """src/voxtral.cpp:1066-1113; a key of another type than the reader's is
    an error (ggml asserts)"""
    kv = g["kv"]

    def typed(key, t):
        if key not in kv:
            return None
        if kv[key][0] != t:
            raise GgufError(f"{key} has type {kv[key][0]}")
        return kv[key][1]

    hp = dict(DEFAULTS)
    arch = typed("general.architecture", STRING)
    hp["is_offline"] = int(arch == b"voxtral")
    for f, k in _I32_KEYS:
        v = typed(k, 5)
        if v is not None:
            hp[f] = v
    for f, k in _F32_KEYS:
        v = typed(k, 6)
        if v is not None:
            hp[f] = struct.unpack("<f", struct.pack("<f", v))[0]
    hp["enc_causal"] = int(not hp["is_offline"])
    for k in ("voxtral.encoder.causal", "voxtral.params.multimodal.whisper_model_args.encoder_args.causal"):
        v = typed(k, 7)
        if v is not None:
            hp["enc_causal"] = int(v)
    hp["ada_t_cond"] = int(not hp["is_offline"])
    v = typed("voxtral.ada_rms_norm_t_cond", 7)
    if v is not None:
        hp["ada_t_cond"] = int(v)
    return hp


def realtime_tensors(hp):
    """the names the realtime model maps (src/voxtral.cpp:1193-1265) as
    (name, required); optional ones may be absent"""
    out = [("enc.conv0.weight", True), ("enc.conv0.bias", True), ("enc.conv1.weight", True),
           ("enc.conv1.bias", True), ("enc.norm.weight", True), ("enc.norm.bias", False),
           ("output.weight", False)]
    for i in range(hp["enc_layers"]):
        for n in ("attn_norm.weight", "attn_q.weight", "attn_q.bias", "attn_k.weight",
                  "attn_v.weight", "attn_v.bias", "attn_o.weight", "attn_o.bias",
                  "ffn_norm.weight", "ffn_w1.weight", "ffn_w2.weight", "ffn_w2.bias",
                  "ffn_w3.weight"):
            out.append((f"enc.blk.{i}.{n}", True))
        out += [(f"enc.blk.{i}.attn_norm.bias", False), (f"enc.blk.{i}.ffn_norm.bias", False)]
    out += [("adapter.0.weight", True), ("adapter.2.weight", True),
            ("tok_embeddings.weight", True), ("norm.weight", True)]
    for i in range(hp["dec_layers"]):
        for n in ("attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                  "attn_o.weight", "ffn_norm.weight", "ffn_w1.weight", "ffn_w2.weight",
                  "ffn_w3.weight"):
            out.append((f"dec.blk.{i}.{n}", True))
        if hp["ada_t_cond"]:
            out += [(f"dec.blk.{i}.ada0.weight", True), (f"dec.blk.{i}.ada2.weight", True)]
    return out
