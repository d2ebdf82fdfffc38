"""CPU oracle for the KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (built by oracle/Makefile) and exposes numpy-friendly
wrappers.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import this package; the product (voxtral.cpp_amd/) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, Q8_0 = 0, 1, 8
Q4_K, Q6_K, Q8_K = 12, 14, 15
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q8_K: 292}
TAG_K, TAG_V, TAG_Q = 1, 2, 3
TAG_EK, TAG_EV, TAG_EQ = 11, 12, 13


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


if not os.path.exists(LIB_PATH):
    build()

lib = ctypes.CDLL(LIB_PATH)


class Ring(ctypes.Structure):
    _fields_ = [("capacity", ctypes.c_int64), ("used", ctypes.c_int64),
                ("oldest_absolute_position", ctypes.c_int64),
                ("next_absolute_position", ctypes.c_int64), ("wraps", ctypes.c_int64),
                ("evictions", ctypes.c_int64), ("bytes_moved", ctypes.c_int64),
                ("full_buffer_moves", ctypes.c_int64)]


class Seg(ctypes.Structure):
    _fields_ = [("slot", ctypes.c_int32), ("len", ctypes.c_int32)]


class Plan(ctypes.Structure):
    _fields_ = [("absolute_start", ctypes.c_int64), ("n_new", ctypes.c_int32),
                ("write_seg", Seg * 2), ("write_nseg", ctypes.c_int32),
                ("read_seg", Seg * 2), ("read_nseg", ctypes.c_int32),
                ("used_after", ctypes.c_int64), ("oldest_after", ctypes.c_int64),
                ("next_after", ctypes.c_int64), ("evicted", ctypes.c_int64),
                ("wrapped", ctypes.c_bool)]


class EncPlan(ctypes.Structure):
    _fields_ = [("q_start", ctypes.c_int64), ("n_new", ctypes.c_int32),
                ("win_start", ctypes.c_int64), ("win_end", ctypes.c_int64),
                ("win_len", ctypes.c_int32), ("read_seg", Seg * 2),
                ("read_nseg", ctypes.c_int32), ("read_wraps", ctypes.c_bool),
                ("write_seg", Seg * 2), ("write_nseg", ctypes.c_int32),
                ("write_wraps", ctypes.c_bool), ("conv_mel_start", ctypes.c_int64),
                ("conv_mel_end", ctypes.c_int64), ("conv_slice_start", ctypes.c_int32),
                ("evicted", ctypes.c_int64)]


class EncRun(ctypes.Structure):
    _fields_ = [("q0", ctypes.c_int64), ("n", ctypes.c_int32), ("physical", ctypes.c_int32),
                ("warmup", ctypes.c_int32)]


_P = ctypes.POINTER
_vp = ctypes.c_void_p
_i32, _i64, _u64, _u32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint32
_f32, _f64 = ctypes.c_float, ctypes.c_double

_protos = {
    "orc_decoder_plan": (ctypes.c_bool, [_P(Ring), _i64, _i32, _P(Plan)]),
    "orc_decoder_commit": (None, [_P(Ring), _P(Plan)]),
    "orc_decoder_clear": (None, [_P(Ring), _i64]),
    "orc_enc_plan": (ctypes.c_bool, [_i64, _i32, _i32, _i32, _P(EncPlan)]),
    "orc_enc_mask_allows": (ctypes.c_bool, [_i64, _i64, _i32]),
    "orc_rope_f32": (None, [_vp, _i64, _i64, _i32, _i32, _i64, _f32]),
    "orc_enc_normalize_physical": (_i32, [_i32]),
    "orc_enc_schedule": (None, [_i32, _i32, _i32, _i32, _P(_i32), _P(_i32)]),
    "orc_enc_frames_realizable": (_i64, [_i64]),
    "orc_enc_drive_next": (ctypes.c_bool, [_i64, _i64, ctypes.c_bool, _i32, _i32, _i32,
                                           ctypes.c_bool, _P(EncRun)]),
    "orc_f32_to_f16_n": (None, [_vp, _vp, _i64]),
    "orc_f16_to_f32_n": (None, [_vp, _vp, _i64]),
    "orc_q8_0_quantize": (None, [_vp, _vp, _i64]),
    "orc_q8_0_dequantize": (None, [_vp, _vp, _i64]),
    "orc_row_bytes": (_i64, [ctypes.c_int, _i64]),
    "orc_row_to_f32": (None, [ctypes.c_int, _vp, _vp, _i64]),
    "orc_row_from_f32": (None, [ctypes.c_int, _vp, _vp, _i64]),
    "orc_mix64": (_u64, [_u64]),
    "orc_row_key": (_u64, [_u64, _u32, _i64, _i64, _i64]),
    "orc_synth_value": (_f32, [_u64, _i64]),
    "orc_synth_row": (None, [_u64, _vp, _i64]),
    "orc_append": (None, [ctypes.c_int, _vp, _i64, _i32, _P(Seg), _i32, _vp]),
    "orc_gather": (None, [_vp, _i64, _P(Seg), _i32, _vp]),
    "orc_expected_layer": (None, [ctypes.c_int, _vp, _i64, _i64, _i32, _i64, _u64, _u32, _i64,
                                  _i64]),
    "orc_decode_attn_f64": (None, [ctypes.c_int, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32,
                                   _i32, _f64, _vp]),
    "orc_decode_attn_mimic": (None, [ctypes.c_int, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32,
                                     _i32, _f32, _vp]),
    "orc_decode_attn_mimic_acc32": (None, [ctypes.c_int, _vp, _vp, _i64, _vp, _i32, _vp, _i32,
                                           _i32, _i32, _f32, _vp]),
    "orc_window_attn_f64": (None, [ctypes.c_int, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32,
                                   _i32, _i32, _i32, _i32, _f64, _vp]),
    "orc_window_attn_mimic": (_i32, [ctypes.c_int, _vp, _vp, _i64, _vp, _vp, _i32, _i32, _vp, _vp,
                                     _i32, _i32, _i32, _i32, _i32, _f32, ctypes.c_int, _vp]),
    "orc_q4_k_dequantize": (None, [_vp, _vp, _i64]),
    "orc_q6_k_dequantize": (None, [_vp, _vp, _i64]),
    "orc_q8_k_quantize": (None, [_vp, _vp, _i64]),
    "orc_q8_k_dequantize": (None, [_vp, _vp, _i64]),
    "orc_vec_dot_q4_k_q8_k": (_f32, [_i64, _vp, _vp]),
    "orc_vec_dot_q6_k_q8_k": (_f32, [_i64, _vp, _vp]),
    "orc_rms_norm": (None, [_vp, _vp, _i64, _f32]),
    "orc_norm_act": (None, [_vp, _i64, _vp, _vp, _f32, _vp]),
    "orc_norm_act_b": (None, [_vp, _i64, _vp, _vp, _vp, _f32, _vp]),
    "orc_silu": (_f32, [_f32]),
    "orc_argmax": (_i32, [_vp, _i64]),
    "orc_conv_dims": (None, [_i32, _i32, _i32, _P(_i32), _P(_i32)]),
    "orc_conv1d": (None, [_vp, _i64, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                          _i32, _vp]),
    "orc_conv_stem": (None, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32, _vp]),
    "orc_gelu_erf": (_f32, [_f32]),
    "orc_time_embedding": (None, [_f32, _i32, _vp]),
    "orc_ada_scale": (_i32, [ctypes.c_int, _vp, ctypes.c_int, _vp, _i32, _i32, _f32, _vp]),
    "orc_row_ring_write": (_i32, [_vp, _i32, _i32, _i64, _vp, _i32]),
    "orc_row_ring_read": (_i32, [_vp, _i32, _i32, _i64, _i32, _vp]),
    "orc_adapter_commit": (_i32, [_vp, _i32, _i32, _i32, _vp, _i32, _i32, _i64, _i32,
                                  ctypes.c_int, _vp, ctypes.c_int, _vp, ctypes.c_int]),
    "orc_q8_0_quantize_x86": (None, [_vp, _vp, _i64]),
    "orc_vec_dot_q8_0_q8_0": (_f32, [_i64, _vp, _vp]),
    "orc_wrow_bytes": (_i64, [ctypes.c_int, _i64]),
    "orc_matvec": (None, [ctypes.c_int, _vp, _i64, _i64, _vp, _vp, ctypes.c_int]),
    "orc_decode_step_mimic_mt": (_f64, [ctypes.c_int, _vp, _vp, _i64, _i64, _i32, _i32, _vp,
                                        _i32, _i32, _i32, _f32, _vp, _vp, _vp, _i32, _i32]),
    "orc_decode_step_simd_mt": (_f64, [ctypes.c_int, _vp, _vp, _i64, _i64, _i32, _i32, _vp,
                                       _i32, _i32, _i32, _f32, _vp, _vp, _vp, _i32, _i32]),
    "orc_simd_available": (ctypes.c_int, []),
}
for _n, (_r, _a) in _protos.items():
    _f = getattr(lib, _n)
    _f.restype = _r
    _f.argtypes = _a


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(dtype, n):
    return int(lib.orc_row_bytes(dtype, n))


# ---- planners ----
def new_ring(capacity):
    r = Ring()
    lib.orc_decoder_clear(ctypes.byref(r), capacity)
    return r


def decoder_plan(ring, start, n_new):
    p = Plan()
    ok = lib.orc_decoder_plan(ctypes.byref(ring), start, n_new, ctypes.byref(p))
    return p if ok else None


def decoder_commit(ring, plan):
    lib.orc_decoder_commit(ctypes.byref(ring), ctypes.byref(plan))


def enc_plan(q_start, n_new, capacity, window):
    p = EncPlan()
    ok = lib.orc_enc_plan(q_start, n_new, capacity, window, ctypes.byref(p))
    return p if ok else None


def enc_mask_allows(kv, q, window):
    return bool(lib.orc_enc_mask_allows(kv, q, window))


def rope(x, head_dim, pos0, theta):
    """ggml mode-0 RoPE of float32 rows x[..., n_rows, row_len] (row r at
    position pos0 + r), returned as a new array."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    n_rows, row_len = y.shape[-2], y.shape[-1]
    n_outer = y.size // (n_rows * row_len) if y.size else 0
    lib.orc_rope_f32(_ptr(y), n_outer, n_rows, row_len, head_dim, pos0, theta)
    return y


def enc_normalize_physical(rows):
    return int(lib.orc_enc_normalize_physical(rows))


def enc_schedule(throughput=0, grid=0, logical=0, physical=0):
    lg, ph = _i32(), _i32()
    lib.orc_enc_schedule(throughput, grid, logical, physical, ctypes.byref(lg), ctypes.byref(ph))
    return lg.value, ph.value


def enc_frames_realizable(mel_frames):
    return int(lib.orc_enc_frames_realizable(mel_frames))


def enc_drive_next(emitted, target, final, logical, physical, finish_physical=8,
                   batch_terminal=False):
    """(q0, n, physical, warmup); n == 0: stop.  None where the reference fails."""
    r = EncRun()
    ok = lib.orc_enc_drive_next(emitted, target, bool(final), logical, physical, finish_physical,
                                bool(batch_terminal), ctypes.byref(r))
    return (r.q0, r.n, r.physical, r.warmup) if ok else None


def segs_of(segs, n):
    return [(segs[i].slot, segs[i].len) for i in range(n)]


# ---- numerics ----
def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib.orc_f32_to_f16_n(_ptr(x), _ptr(y), x.size)
    return y


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib.orc_f16_to_f32_n(_ptr(h), _ptr(y), h.size)
    return y


def q8_0_quantize(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib.orc_q8_0_quantize(_ptr(x), _ptr(out), x.size)
    return out


def q8_0_dequantize(blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, dtype=np.float32)
    lib.orc_q8_0_dequantize(_ptr(blocks), _ptr(y), n)
    return y


def rows_to_f32(dtype, raw, kv_dim):
    """raw row bytes (n_rows * row_bytes) -> float32 [n_rows, kv_dim]"""
    raw = np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray)) else raw
    rb = row_bytes(dtype, kv_dim)
    n = raw.size // rb
    out = np.empty((n, kv_dim), dtype=np.float32)
    raw = np.ascontiguousarray(raw)
    lib.orc_row_to_f32(dtype, _ptr(raw), _ptr(out), n * kv_dim)
    return out


def rows_from_f32(dtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    kv_dim = x.shape[-1]
    n = x.size // kv_dim
    out = np.empty(n * row_bytes(dtype, kv_dim), dtype=np.uint8)
    lib.orc_row_from_f32(dtype, _ptr(x), _ptr(out), x.size)
    return out


# ---- generator ----
def row_key(seed, tag, stream, layer, pos):
    return int(lib.orc_row_key(seed, tag, stream, layer, pos))


def synth_row(seed, tag, stream, layer, pos, n):
    out = np.empty(n, dtype=np.float32)
    lib.orc_synth_row(lib.orc_row_key(seed, tag, stream, layer, pos), _ptr(out), n)
    return out


def synth_rows(seed, tag, stream, layer, positions, n):
    return np.stack([synth_row(seed, tag, stream, layer, int(p), n) for p in positions])


# ---- cache image ----
def append(dtype, layer_img, row_b, kv_dim, segs, src):
    arr = (Seg * 2)()
    for i, (s, n) in enumerate(segs):
        arr[i].slot, arr[i].len = s, n
    src = np.ascontiguousarray(src, dtype=np.float32)
    lib.orc_append(dtype, _ptr(layer_img), row_b, kv_dim, arr, len(segs), _ptr(src))


def gather(layer_img, row_b, segs):
    arr = (Seg * 2)()
    total = 0
    for i, (s, n) in enumerate(segs):
        arr[i].slot, arr[i].len = s, n
        total += n
    out = np.empty(total * row_b, dtype=np.uint8)
    lib.orc_gather(_ptr(layer_img), row_b, arr, len(segs), _ptr(out))
    return out


def expected_layer(dtype, backing, capacity, kv_dim, next_pos, seed, tag, stream, layer):
    rb = row_bytes(dtype, kv_dim)
    out = np.empty(backing * rb, dtype=np.uint8)
    lib.orc_expected_layer(dtype, _ptr(out), backing, capacity, kv_dim, next_pos, seed, tag,
                           stream, layer)
    return out


# ---- attention ----
def decode_attn_f64(dtype, k_img, v_img, row_b, slots, q, n_kv_heads, head_dim, scale):
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q_heads = q.size // head_dim
    out = np.empty(n_q_heads * head_dim, dtype=np.float64)
    lib.orc_decode_attn_f64(dtype, _ptr(k_img), _ptr(v_img), row_b, _ptr(slots), slots.size,
                            _ptr(q), n_q_heads, n_kv_heads, head_dim, scale, _ptr(out))
    return out.reshape(n_q_heads, head_dim)


def decode_attn_mimic(dtype, k_img, v_img, row_b, slots, q, n_kv_heads, head_dim, scale):
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q_heads = q.size // head_dim
    out = np.empty(n_q_heads * head_dim, dtype=np.float32)
    lib.orc_decode_attn_mimic(dtype, _ptr(k_img), _ptr(v_img), row_b, _ptr(slots), slots.size,
                              _ptr(q), n_q_heads, n_kv_heads, head_dim, scale, _ptr(out))
    return out.reshape(n_q_heads, head_dim)


def decode_attn_mimic_acc32(dtype, k_img, v_img, row_b, slots, q, n_kv_heads, head_dim, scale):
    """the mimic with an f32 V accumulator: every other rounding of ggml's CPU
    flash attention kept"""
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q_heads = q.size // head_dim
    out = np.empty(n_q_heads * head_dim, dtype=np.float32)
    lib.orc_decode_attn_mimic_acc32(dtype, _ptr(k_img), _ptr(v_img), row_b, _ptr(slots),
                                    slots.size, _ptr(q), n_q_heads, n_kv_heads, head_dim, scale,
                                    _ptr(out))
    return out.reshape(n_q_heads, head_dim)


def window_attn_mimic(dtype, k_img, v_img, row_b, k_slot, k_pos, q, q_pos, n_q_heads,
                      n_kv_heads, head_dim, window, scale, new_start=None, flash=None):
    """orc_window_attn_f64's function in the reference encoder's ggml CPU
    arithmetic (segmented below 32 query rows, flash from 32 unless `flash`
    says otherwise); keys in logical order, the block's new rows from key
    index new_start (default: the first key at or past the first query)"""
    k_slot = np.ascontiguousarray(k_slot, dtype=np.int32)
    k_pos = np.ascontiguousarray(k_pos, dtype=np.int64)
    q_pos = np.ascontiguousarray(q_pos, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q = q_pos.size
    if new_start is None:
        new_start = int(np.searchsorted(k_pos, q_pos.min())) if n_q else k_slot.size
    if flash is None:
        flash = n_q >= 32
    out = np.empty(n_q * n_q_heads * head_dim, dtype=np.float32)
    st = lib.orc_window_attn_mimic(dtype, _ptr(k_img), _ptr(v_img), row_b, _ptr(k_slot),
                                   _ptr(k_pos), k_slot.size, new_start, _ptr(q), _ptr(q_pos), n_q,
                                   n_q_heads, n_kv_heads, head_dim, window, scale, int(flash),
                                   _ptr(out))
    if st != 0:
        raise ValueError("window_attn_mimic: F16 and F32 rings only")
    return out.reshape(n_q, n_q_heads, head_dim)


def window_attn_f64(dtype, k_img, v_img, row_b, k_slot, k_pos, q, q_pos, n_q_heads, n_kv_heads,
                    head_dim, window, scale):
    k_slot = np.ascontiguousarray(k_slot, dtype=np.int32)
    k_pos = np.ascontiguousarray(k_pos, dtype=np.int64)
    q_pos = np.ascontiguousarray(q_pos, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q = q_pos.size
    out = np.empty(n_q * n_q_heads * head_dim, dtype=np.float64)
    lib.orc_window_attn_f64(dtype, _ptr(k_img), _ptr(v_img), row_b, _ptr(k_slot), _ptr(k_pos),
                            k_slot.size, _ptr(q), _ptr(q_pos), n_q, n_q_heads, n_kv_heads,
                            head_dim, window, scale, _ptr(out))
    return out.reshape(n_q, n_q_heads, head_dim)


def simd_available():
    """whether this host runs the vector leg (AVX2, FMA and F16C)"""
    return bool(lib.orc_simd_available())


def decode_step_mimic_mt(dtype, k_cache, v_cache, layer_bytes, row_b, n_layers, n_valid, q,
                         n_q_heads, n_kv_heads, head_dim, scale, n_threads, k_new=None,
                         v_new=None, new_slot=0, simd=False):
    """One threaded decode step (append, then attention over slots [0, n_valid)
    of every layer) -> (wall seconds, out [n_layers][n_q_heads][head_dim]);
    simd: each head on AVX2/FMA/F16C lanes (orc_decode_step_simd_mt)."""
    if simd and not lib.orc_simd_available():
        raise RuntimeError("this host lacks AVX2, FMA or F16C")
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.empty(n_layers * n_q_heads * head_dim, dtype=np.float32)
    kn_arr = np.ascontiguousarray(k_new, dtype=np.float32) if k_new is not None else None
    vn_arr = np.ascontiguousarray(v_new, dtype=np.float32) if v_new is not None else None
    kn = _ptr(kn_arr) if kn_arr is not None else None
    vn = _ptr(vn_arr) if vn_arr is not None else None
    fn = lib.orc_decode_step_simd_mt if simd else lib.orc_decode_step_mimic_mt
    secs = fn(dtype, _ptr(k_cache), _ptr(v_cache), layer_bytes, row_b, n_layers, n_valid, _ptr(q),
              n_q_heads, n_kv_heads, head_dim, scale, _ptr(out), kn, vn, new_slot, n_threads)
    if secs < 0:
        raise ValueError(f"vector step: head_dim {head_dim} is not a multiple of 32 up to 512")
    return secs, out.reshape(n_layers, n_q_heads, head_dim)


# ---- decoder weights: ggml Q4_K / Q6_K, Q8_K activations ----
def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def _f32a(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def dequantize(dtype, blocks, n):
    """ggml dequantize_row_q4_K / _q6_K / _q8_K / _q8_0 of n elements -> f32."""
    blocks = _u8(blocks)
    y = np.empty(n, dtype=np.float32)
    fn = {Q4_K: lib.orc_q4_k_dequantize, Q6_K: lib.orc_q6_k_dequantize,
          Q8_K: lib.orc_q8_k_dequantize, Q8_0: lib.orc_q8_0_dequantize}[dtype]
    fn(_ptr(blocks), _ptr(y), n)
    return y


def q8_k_quantize(x):
    x = _f32a(x).ravel()
    out = np.empty(x.size // 256 * 292, dtype=np.uint8)
    lib.orc_q8_k_quantize(_ptr(x), _ptr(out), x.size)
    return out


def q8_0_quantize_x86(x):
    """q8_0 activation blocks (ggml's x86 quantize_row_q8_0: the input side of
    a product on Q8_0 weights)."""
    x = _f32a(x).ravel()
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib.orc_q8_0_quantize_x86(_ptr(x), _ptr(out), x.size)
    return out


def vec_dot(dtype, w_row, xq, n):
    """one row's dot: Q4_K / Q6_K against Q8_K blocks, Q8_0 against q8_0"""
    w_row, xq = _u8(w_row), _u8(xq)
    fn = {Q4_K: lib.orc_vec_dot_q4_k_q8_k, Q6_K: lib.orc_vec_dot_q6_k_q8_k,
          Q8_0: lib.orc_vec_dot_q8_0_q8_0}[dtype]
    return fn(n, _ptr(w_row), _ptr(xq))


def norm_act(x, norm_w=None, ada=None, eps=1e-5, norm_b=None):
    """rms_norm(x) * norm_w (+ norm_b) (then + h * ada); x itself without norm_w."""
    x = _f32a(x)
    y = np.empty_like(x)
    arrs = [_f32a(a) if a is not None else None for a in (norm_w, norm_b, ada)]
    ptrs = [_ptr(a) if a is not None else None for a in arrs]
    lib.orc_norm_act_b(_ptr(x), x.size, ptrs[0], ptrs[1], ptrs[2], eps, _ptr(y))
    return y


def silu(v):
    return np.array([lib.orc_silu(float(t)) for t in np.asarray(v, np.float32).ravel()],
                    dtype=np.float32)


def argmax(x):
    """ggml_argmax: the last index of the maximum (finite input)."""
    x = _f32a(x).ravel()
    return lib.orc_argmax(_ptr(x), x.size)


def wrow_bytes(dtype, n_in):
    return n_in // 32 * 34 if dtype == Q8_0 else n_in // 256 * BLOCK_BYTES[dtype]


def matvec(dtype, w, n_rows, n_in, x, n_threads=1):
    """ggml_mul_mat(W, x) as the CPU path computes it: x (already normalised)
    quantized to Q8_K (Q4_K / Q6_K weights) or q8_0 (Q8_0 weights), one
    vec_dot per row."""
    w, x = _u8(w), _f32a(x)
    assert w.size >= n_rows * wrow_bytes(dtype, n_in) and x.size == n_in
    y = np.empty(n_rows, dtype=np.float32)
    lib.orc_matvec(dtype, _ptr(w), n_rows, n_in, _ptr(x), _ptr(y), n_threads)
    return y


# ---- the encoder conv stem ----
def conv_dims(in_len, kernel, stride):
    pad, out = _i32(), _i32()
    lib.orc_conv_dims(in_len, kernel, stride, ctypes.byref(pad), ctypes.byref(out))
    return pad.value, out.value


def conv_stem(mel, slice_start, n_new, w0, b0, w1, b1):
    """mel [n_mel][conv_len] f32; w0 [dim][n_mel][3] / w1 [dim][dim][3] as f16
    bits (uint16); returns x [n_new][dim]."""
    mel = _f32a(mel)
    n_mel, conv_len = mel.shape
    w0 = np.ascontiguousarray(w0, np.uint16)
    w1 = np.ascontiguousarray(w1, np.uint16)
    dim = w0.shape[0]
    b0, b1 = _f32a(b0), _f32a(b1)
    x = np.empty((n_new, dim), np.float32)
    lib.orc_conv_stem(_ptr(mel), n_mel, conv_len, slice_start, n_new, _ptr(w0), _ptr(b0),
                      _ptr(w1), _ptr(b1), dim, _ptr(x))
    return x


def conv1d(inp, stride_c, stride_t, in_len, n_ch, w, b, stride, pad, t0, n_out, gelu=True):
    """one causal conv (f16 im2col of inp read with the given strides), y [n_out][out_ch]"""
    inp = _f32a(inp)
    w = np.ascontiguousarray(w, np.uint16)
    b = _f32a(b)
    y = np.empty((n_out, w.shape[0]), np.float32)
    lib.orc_conv1d(_ptr(inp), stride_c, stride_t, in_len, n_ch, _ptr(w), _ptr(b), w.shape[0],
                   stride, pad, t0, n_out, 1 if gelu else 0, _ptr(y))
    return y


# ---- the realtime rows rings and the adapter ----
def gelu_erf(x):
    """ggml_gelu_erf of f32 values, elementwise"""
    x = _f32a(x)
    return np.array([lib.orc_gelu_erf(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def row_ring_write(ring, row_start, src):
    """src rows -> logical rows row_start.. of ring [capacity][width] (in place)"""
    assert ring.dtype == np.float32 and ring.flags.c_contiguous
    src = _f32a(src).reshape(-1, ring.shape[1])
    rc = lib.orc_row_ring_write(_ptr(ring), ring.shape[0], ring.shape[1], row_start, _ptr(src),
                                src.shape[0])
    if rc != 0:
        raise ValueError("ring write rejected")


def row_ring_read(ring, row_start, n_rows):
    ring = _f32a(ring)
    dst = np.empty((n_rows, ring.shape[1]), np.float32)
    rc = lib.orc_row_ring_read(_ptr(ring), ring.shape[0], ring.shape[1], row_start, n_rows, _ptr(dst))
    if rc != 0:
        raise ValueError("ring read rejected")
    return dst


def adapter_commit(enc_ring, aemb_ring, group_start, n_groups, w0_type, w0, w2_type, w2,
                   down=4, n_threads=8):
    """the adapter over ring groups; aemb_ring [capacity][dec_dim] updated in place"""
    enc_ring = _f32a(enc_ring)
    assert aemb_ring.dtype == np.float32 and aemb_ring.flags.c_contiguous
    w0, w2 = _u8(w0), _u8(w2)
    enc_dim, dec_dim = enc_ring.shape[1], aemb_ring.shape[1]
    assert w0.size >= dec_dim * wrow_bytes(w0_type, enc_dim * down)
    assert w2.size >= dec_dim * wrow_bytes(w2_type, dec_dim)
    rc = lib.orc_adapter_commit(_ptr(enc_ring), enc_ring.shape[0], enc_dim, down, _ptr(aemb_ring),
                                aemb_ring.shape[0], dec_dim, group_start, n_groups, w0_type,
                                _ptr(w0), w2_type, _ptr(w2), n_threads)
    if rc != n_groups:
        raise ValueError("adapter commit rejected")


def time_embedding(t, dim):
    out = np.empty(dim, np.float32)
    lib.orc_time_embedding(t, dim, _ptr(out))
    return out


def ada_scale(w0_type, w0, w2, dim, ada_dim, t):
    """w2: uint16 (f16 bits) or float32 array [dim][ada_dim], or uint8 Q8_0
    blocks ([dim] rows of ada_dim / 32 blocks)"""
    w0 = _u8(w0)
    w2 = np.ascontiguousarray(w2)
    if w2.dtype == np.uint8:
        assert w2.size == dim * (ada_dim // 32) * 34
        w2_type = Q8_0
    else:
        assert w2.dtype in (np.uint16, np.float32) and w2.size == dim * ada_dim
        w2_type = F16 if w2.dtype == np.uint16 else F32
    out = np.empty(dim, np.float32)
    rc = lib.orc_ada_scale(w0_type, _ptr(w0), w2_type, _ptr(w2), dim, ada_dim, t, _ptr(out))
    if rc != 0:
        raise ValueError("ada scale rejected")
    return out
