"""ctypes binding of libvkv.so (include/vkv.h), the gfx950 KV-cache hot path.

Structures mirror the C ABI field for field; every wrapper raises VkvError on a
non-OK status with the library's own message.  Device pointers are plain
integers (e.g. torch's ``tensor.data_ptr()``); ``hip_stream`` is a raw
hipStream_t (``torch.cuda.current_stream().cuda_stream``) or 0.

There is no CPU fallback: if libvkv.so is missing, importing this module
raises.
"""
import ctypes
import os

try:
    # torch ships its own HIP runtime under the same soname (libamdhip64.so.7);
    # whichever loads first serves the whole process.  Load torch's first when
    # it is installed so that torch tensors and this library share one runtime.
    import torch  # noqa: F401
except ImportError:
    pass

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvkv.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python voxtral.cpp_amd/build.py` "
        "(or __graft_entry__.build()); the KV path has no fallback")

lib = ctypes.CDLL(LIB_PATH)

# status / dtype ---------------------------------------------------------
OK = 0
INVALID_ARGUMENT = 1
INVALID_STATE = 2
OUT_OF_MEMORY = 3
MODEL_ERROR = 8
BACKEND_ERROR = 9
INTERNAL_ERROR = 10
BUFFER_TOO_SMALL = 11

F32 = 0
F16 = 1
Q8_0 = 8
Q4_K = 12
Q6_K = 14
Q8_K = 15
MAX_BATCH_STREAMS = 32
KQ_BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q8_K: 292, Q8_0: 272}   # bytes per 256 elements
MV_MAX_IN = 12288
MV_MAX_OUTS = 4
MV_STORE, MV_SWIGLU, MV_GELU = 0, 1, 2


def row_bytes(dtype, n):
    return {F32: 4 * n, F16: 2 * n, Q8_0: (n // 32) * 34}[dtype]


class VkvError(RuntimeError):
    def __init__(self, status, message, backend_code=0):
        super().__init__(f"vkv status {status}: {message}")
        self.status = status
        self.message = message
        self.backend_code = backend_code


# structures (field-for-field with include/vkv.h) ---------------------------
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


class EncSchedule(ctypes.Structure):
    _fields_ = [("logical", ctypes.c_int32), ("physical", ctypes.c_int32)]


class EncRun(ctypes.Structure):
    _fields_ = [("q0", ctypes.c_int64), ("n", ctypes.c_int32), ("physical", ctypes.c_int32),
                ("warmup", ctypes.c_int32)]


class CacheParams(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("n_streams", ctypes.c_int32),
                ("n_layers", ctypes.c_int32), ("capacity", ctypes.c_int32),
                ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("n_q_heads", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("device", ctypes.c_int32), ("kernel_flags", ctypes.c_int32),
                ("decode_chunk", ctypes.c_int32), ("decode_waves", ctypes.c_int32),
                ("decode_stages", ctypes.c_int32)]


# vkv_cache_params.kernel_flags (cross-checks and A/B measurement only)
KERNEL_DECODE_HEADS = 0x1
KERNEL_DECODE_ROWS = 0x2
KERNEL_DECODE_VALU = 0x4
KERNEL_WINDOW_VALU = 0x8
KERNEL_XCD_SWIZZLE = 0x10
KERNEL_NO_XCD_SWIZZLE = 0x20


class CacheLayout(ctypes.Structure):
    _fields_ = [("row_bytes", ctypes.c_uint64), ("layer_bytes", ctypes.c_uint64),
                ("stream_bytes", ctypes.c_uint64), ("total_bytes", ctypes.c_uint64),
                ("k_base", ctypes.c_void_p), ("v_base", ctypes.c_void_p)]


_P = ctypes.POINTER
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float


class MvOut(ctypes.Structure):
    _fields_ = [("w", _vp), ("dtype", _i32), ("n_rows", _i32), ("y", _vp), ("add", _vp)]


class MmOut(ctypes.Structure):
    _fields_ = [("w", _vp), ("dtype", _i32), ("n_rows", _i32), ("y", _vp), ("add", _vp),
                ("bias", _vp)]


class EncLayer(ctypes.Structure):
    _fields_ = [("attn_norm", _vp), ("attn_norm_b", _vp), ("attn_q", _vp), ("attn_k", _vp),
                ("attn_v", _vp), ("attn_o", _vp), ("attn_q_type", _i32), ("attn_k_type", _i32),
                ("attn_v_type", _i32), ("attn_o_type", _i32), ("attn_q_b", _vp), ("attn_v_b", _vp),
                ("attn_o_b", _vp), ("ffn_norm", _vp), ("ffn_norm_b", _vp), ("ffn_w1", _vp),
                ("ffn_w2", _vp), ("ffn_w3", _vp), ("ffn_w1_type", _i32), ("ffn_w2_type", _i32),
                ("ffn_w3_type", _i32), ("ffn_w2_b", _vp)]


class EncModel(ctypes.Structure):
    _fields_ = [("n_layers", _i32), ("dim", _i32), ("hidden", _i32), ("n_heads", _i32),
                ("head_dim", _i32), ("norm_eps", _f32), ("rope_theta", _f32), ("out_norm", _vp),
                ("out_norm_b", _vp), ("layers", _P(EncLayer))]


class DecLayer(ctypes.Structure):
    _fields_ = [("attn_norm", _vp), ("attn_q", _vp), ("attn_k", _vp), ("attn_v", _vp),
                ("attn_o", _vp), ("attn_q_type", _i32), ("attn_k_type", _i32),
                ("attn_v_type", _i32), ("attn_o_type", _i32), ("ffn_norm", _vp),
                ("ada_scale", _vp), ("ffn_w1", _vp), ("ffn_w2", _vp), ("ffn_w3", _vp),
                ("ffn_w1_type", _i32), ("ffn_w2_type", _i32), ("ffn_w3_type", _i32)]


class DecModel(ctypes.Structure):
    _fields_ = [("n_layers", _i32), ("dim", _i32), ("hidden", _i32), ("n_q_heads", _i32),
                ("n_kv_heads", _i32), ("head_dim", _i32), ("vocab", _i32), ("norm_eps", _f32),
                ("rope_theta", _f32), ("tok_embeddings", _vp), ("tok_embeddings_type", _i32),
                ("out_norm", _vp), ("output", _vp), ("output_type", _i32),
                ("layers", _P(DecLayer))]


class RowRing(ctypes.Structure):
    _fields_ = [("rows", _vp), ("capacity", _i32), ("width", _i32)]


class Adapter(ctypes.Structure):
    _fields_ = [("w0", _vp), ("w2", _vp), ("w0_type", _i32), ("w2_type", _i32),
                ("enc_dim", _i32), ("dec_dim", _i32), ("downsample", _i32)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", _i32), ("n_dims", _i32), ("ne", _i64 * 4),
                ("offset", _u64), ("nbytes", _u64)]


class Hparams(ctypes.Structure):
    _fields_ = [("is_offline", _i32), ("enc_dim", _i32), ("enc_layers", _i32), ("enc_heads", _i32),
                ("enc_head_dim", _i32), ("enc_hidden", _i32), ("enc_kv_heads", _i32),
                ("enc_causal", _i32), ("enc_norm_eps", _f32), ("enc_rope_theta", _f32),
                ("dec_dim", _i32), ("dec_layers", _i32), ("dec_heads", _i32),
                ("dec_head_dim", _i32), ("dec_hidden", _i32), ("dec_kv_heads", _i32),
                ("dec_norm_eps", _f32), ("dec_rope_theta", _f32), ("ada_t_cond", _i32),
                ("vocab_size", _i32), ("downsample_factor", _i32), ("tok_bos", _i32),
                ("tok_eos", _i32), ("tok_audio", _i32), ("tok_begin_audio", _i32)]


class ModelView(ctypes.Structure):
    _fields_ = [("hp", Hparams), ("enc", EncModel), ("dec", DecModel), ("adapter", Adapter),
                ("conv0_w", _vp), ("conv1_w", _vp), ("conv0_b", _vp), ("conv1_b", _vp),
                ("mel_filters", _vp), ("device_bytes", _u64)]


# prototypes: name -> (restype, argtypes); exactly the functions of include/vkv.h
PROTOTYPES = {
    "vkv_decoder_plan": (_i32, [_P(Ring), _i64, _i32, _P(Plan)]),
    "vkv_decoder_commit": (_i32, [_P(Ring), _P(Plan)]),
    "vkv_decoder_clear": (_i32, [_P(Ring), _i64]),
    "vkv_enc_plan_build": (_i32, [_i64, _i32, _i32, _i32, _P(EncPlan)]),
    "vkv_enc_mask_allows": (_i32, [_i64, _i64, _i32]),
    "vkv_decoder_step_rope": (_i32, [_vp, _i32, _i32, _P(Ring), _P(_i64), _i32, _i32, _vp, _vp,
                                     _vp, _vp, _i32, ctypes.c_float, ctypes.c_float, _P(Plan),
                                     _vp]),
    "vkv_rope": (_i32, [_vp, _i64, _i64, _i32, _i32, _i64, ctypes.c_float, _vp]),
    "vkv_enc_normalize_physical": (_i32, [_i32]),
    "vkv_enc_schedule_make": (_i32, [_i32, _i32, _i32, _i32, _P(EncSchedule)]),
    "vkv_enc_frames_realizable": (_i64, [_i64]),
    "vkv_enc_drive_next": (_i32, [_i64, _i64, _i32, _P(EncSchedule), _i32, _i32, _P(EncRun)]),
    "vkv_cache_create": (_i32, [_P(CacheParams), _P(_vp)]),
    "vkv_cache_destroy": (_i32, [_vp]),
    "vkv_cache_get_layout": (_i32, [_vp, _P(CacheLayout)]),
    "vkv_cache_read_rows": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, ctypes.c_size_t]),
    "vkv_cache_zero": (_i32, [_vp, _vp]),
    "vkv_append": (_i32, [_vp, _i32, _i32, _i32, _P(Seg), _i32, _vp, _vp, _i64, _vp]),
    "vkv_gather": (_i32, [_vp, _i32, _i32, _P(Seg), _i32, _vp, _vp, _vp]),
    "vkv_decode_attn": (_i32, [_vp, _i32, _i32, _i32, _i32, _P(Plan), _vp, _vp, _i32, _f32, _vp]),
    "vkv_decoder_step": (_i32, [_vp, _i32, _i32, _P(Ring), _P(_i64), _i32, _i32, _vp, _vp, _vp,
                                _vp, _i32, _f32, _P(Plan), _vp]),
    "vkv_decoder_prefill": (_i32, [_vp, _i32, _P(Ring), _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                   _i32, _f32, _vp]),
    "vkv_enc_step": (_i32, [_vp, _i32, _P(EncPlan), _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i32,
                            _f32, _vp]),
    "vkv_window_attn": (_i32, [_vp, _i32, _i32, _i32, _P(Seg), _i32, _i64, _i64, _i32, _i32,
                               _vp, _vp, _i32, _f32, _vp]),
    "vkv_q8_0_pack": (_i32, [_vp, _vp, _i64, _vp]),
    "vkv_q8_0_unpack": (_i32, [_vp, _vp, _i64, _vp]),
    "vkv_matvec": (_i32, [_vp, _i64, _vp, _vp, _f32, _P(MvOut), _i32, _i32, _vp]),
    "vkv_matmul_workspace": (ctypes.c_size_t, [_i32, _i64]),
    "vkv_encoder_chunk_workspace": (ctypes.c_size_t, [_P(EncModel), _i32]),
    "vkv_enc_conv_stem_workspace": (ctypes.c_size_t, [_i32, _i32, _i32, _i32]),
    "vkv_enc_conv_stem": (_i32, [_vp, _i32, _P(EncPlan), _vp, _vp, _vp, _vp, _i32, _vp, _vp,
                                 ctypes.c_size_t, _vp]),
    "vkv_encoder_chunk": (_i32, [_vp, _i32, _P(EncPlan), _i32, _P(EncModel), _vp, _vp,
                                 ctypes.c_size_t, _vp]),
    "vkv_matmul": (_i32, [_vp, _i32, _i64, _vp, _vp, _vp, _f32, _P(MmOut), _i32, _i32, _vp,
                          ctypes.c_size_t, _vp]),
    "vkv_encoder_chunk_ring": (_i32, [_vp, _i32, _P(EncPlan), _i32, _P(EncModel), _vp,
                                      _P(RowRing), _vp, ctypes.c_size_t, _vp]),
    "vkv_row_ring_write": (_i32, [_P(RowRing), _i64, _vp, _i32, _vp]),
    "vkv_row_ring_read": (_i32, [_P(RowRing), _i64, _i32, _vp, _vp]),
    "vkv_adapter_workspace": (ctypes.c_size_t, [_P(Adapter), _i32]),
    "vkv_adapter_commit": (_i32, [_P(Adapter), _P(RowRing), _P(RowRing), _i64, _i32, _vp,
                                  ctypes.c_size_t, _vp]),
    "vkv_quantize_q8_k": (_i32, [_vp, _i64, _vp, _vp, _f32, _vp, _vp]),
    "vkv_dequantize": (_i32, [_i32, _vp, _i64, _vp, _vp]),
    "vkv_decoder_layer_step": (_i32, [_vp, _i32, _P(Plan), _i64, _i32, _i32, _vp, _vp, _vp, _vp,
                                      _i32, _f32, _f32, _vp]),
    "vkv_decoder_token_workspace": (ctypes.c_size_t, [_P(DecModel)]),
    "vkv_decoder_token": (_i32, [_vp, _i32, _P(Ring), _P(DecModel), _i32, _vp, _vp, _vp, _vp,
                                 ctypes.c_size_t, _P(Plan), _vp]),
    "vkv_decoder_token_noalloc": (_i32, [_vp, _i32, _P(Ring), _P(DecModel), _i32, _vp, _vp, _vp,
                                         _P(Plan), _vp]),
    "vkv_decoder_prompt_workspace": (ctypes.c_size_t, [_P(DecModel), _i32]),
    "vkv_decoder_prompt": (_i32, [_vp, _i32, _P(Ring), _P(DecModel), _P(ctypes.c_int32), _i32,
                                  _P(RowRing), _vp, _vp, _vp, ctypes.c_size_t, _P(Plan), _vp]),
    "vkv_ada_scale_workspace": (ctypes.c_size_t, [_i32, _i32]),
    "vkv_ada_scale": (_i32, [_vp, _i32, _vp, _i32, _i32, _i32, _f32, _vp, _vp, ctypes.c_size_t, _vp]),
    "vkv_model_set_ada": (_i32, [_vp, _f32, _vp, _vp]),
    "vkv_embed": (_i32, [_i32, _vp, _i32, _i64, _i32, _vp, _vp, _vp]),
    "vkv_argmax": (_i32, [_vp, _i64, _vp, _vp]),
    "vkv_gguf_open": (_i32, [ctypes.c_char_p, _P(_vp)]),
    "vkv_gguf_close": (_i32, [_vp]),
    "vkv_gguf_version": (_u32, [_vp]),
    "vkv_gguf_alignment": (_u64, [_vp]),
    "vkv_gguf_data_offset": (_u64, [_vp]),
    "vkv_gguf_n_kv": (_i64, [_vp]),
    "vkv_gguf_find_key": (_i64, [_vp, ctypes.c_char_p]),
    "vkv_gguf_key": (ctypes.c_char_p, [_vp, _i64]),
    "vkv_gguf_kv_type": (_i32, [_vp, _i64]),
    "vkv_gguf_get_i32": (_i32, [_vp, _i64, _P(_i32)]),
    "vkv_gguf_get_u32": (_i32, [_vp, _i64, _P(_u32)]),
    "vkv_gguf_get_i64": (_i32, [_vp, _i64, _P(_i64)]),
    "vkv_gguf_get_f32": (_i32, [_vp, _i64, _P(_f32)]),
    "vkv_gguf_get_f64": (_i32, [_vp, _i64, _P(ctypes.c_double)]),
    "vkv_gguf_get_bool": (_i32, [_vp, _i64, _P(_i32)]),
    "vkv_gguf_get_str": (_i32, [_vp, _i64, _P(_vp), _P(_u64)]),
    "vkv_gguf_get_scalar": (_i32, [_vp, _i64, _vp, _u64]),
    "vkv_gguf_get_arr": (_i32, [_vp, _i64, _P(_i32), _P(_u64), _P(_vp)]),
    "vkv_gguf_get_arr_str": (_i32, [_vp, _i64, _u64, _P(_vp), _P(_u64)]),
    "vkv_gguf_n_tensors": (_i64, [_vp]),
    "vkv_gguf_find_tensor": (_i64, [_vp, ctypes.c_char_p]),
    "vkv_gguf_tensor_info": (_i32, [_vp, _i64, _P(GgufTensor)]),
    "vkv_gguf_tensor_data": (_vp, [_vp, _i64]),
    "vkv_gguf_hparams": (_i32, [_vp, _P(Hparams)]),
    "vkv_model_load": (_i32, [ctypes.c_char_p, _i32, _vp, _P(_vp)]),
    "vkv_model_free": (_i32, [_vp]),
    "vkv_model_get_view": (_i32, [_vp, _P(ModelView)]),
    "vkv_model_tensor": (_vp, [_vp, ctypes.c_char_p, _P(GgufTensor)]),
    "vkv_synth_rows": (_i32, [_vp, _i32, _u64, _u32, _i64, _i32, _i64, _i64, _i32, _i64, _i64,
                              _i32, _i64, _vp]),
    "vkv_api_version": (_u32, []),
    "vkv_last_error": (ctypes.c_char_p, []),
    "vkv_last_backend_code": (_i32, []),
}

for _name, (_res, _args) in PROTOTYPES.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def last_error():
    return lib.vkv_last_error().decode()


def check(status):
    if status != OK:
        raise VkvError(status, last_error(), lib.vkv_last_backend_code())
    return status


def _segs(segs):
    arr = (Seg * 2)()
    for i, (slot, n) in enumerate(segs):
        arr[i].slot, arr[i].len = slot, n
    return arr, len(segs)


def plan_segs(segs, nseg):
    return [(segs[i].slot, segs[i].len) for i in range(nseg)]


# planners -----------------------------------------------------------------
def decoder_plan(ring, absolute_start, n_new):
    p = Plan()
    check(lib.vkv_decoder_plan(ctypes.byref(ring), absolute_start, n_new, ctypes.byref(p)))
    return p


def decoder_commit(ring, plan):
    check(lib.vkv_decoder_commit(ctypes.byref(ring), ctypes.byref(plan)))


def new_ring(capacity):
    r = Ring()
    check(lib.vkv_decoder_clear(ctypes.byref(r), capacity))
    return r


def decoder_clear(ring, capacity):
    """resets ring in place to an empty ring of the given capacity"""
    check(lib.vkv_decoder_clear(ctypes.byref(ring), capacity))


def enc_plan(q_start, n_new, capacity, window):
    p = EncPlan()
    check(lib.vkv_enc_plan_build(q_start, n_new, capacity, window, ctypes.byref(p)))
    return p


def enc_mask_allows(kv_abs, q_abs, window):
    return bool(lib.vkv_enc_mask_allows(kv_abs, q_abs, window))


ENC_WINDOW, ENC_MAX_NEW = 750, 128
ENC_KV_CAP = ENC_WINDOW + ENC_MAX_NEW


def enc_normalize_physical(rows):
    return int(lib.vkv_enc_normalize_physical(rows))


def enc_schedule(throughput=0, grid=0, logical=0, physical=0):
    sc = EncSchedule()
    check(lib.vkv_enc_schedule_make(throughput, grid, logical, physical, ctypes.byref(sc)))
    return sc


def enc_frames_realizable(mel_frames):
    return int(lib.vkv_enc_frames_realizable(mel_frames))


def enc_drive_next(emitted, target, final, schedule, finish_physical=8, batch_terminal=False):
    """Next encoder run (EncRun; n == 0: stop), as encoder_kv_drive."""
    r = EncRun()
    check(lib.vkv_enc_drive_next(emitted, target, int(bool(final)), ctypes.byref(schedule),
                                 finish_physical, int(bool(batch_terminal)), ctypes.byref(r)))
    return r


# cache --------------------------------------------------------------------
class Cache:
    """Owns one vkv_cache handle (K and V storage on the device)."""

    def __init__(self, n_streams=1, n_layers=26, capacity=8192, n_kv_heads=8, head_dim=128,
                 n_q_heads=32, dtype=F16, device=0, kernel_flags=0, decode_chunk=0,
                 decode_waves=0, decode_stages=0):
        p = CacheParams(ctypes.sizeof(CacheParams), n_streams, n_layers, capacity, n_kv_heads,
                        head_dim, n_q_heads, dtype, device, kernel_flags, decode_chunk,
                        decode_waves, decode_stages)
        h = _vp()
        check(lib.vkv_cache_create(ctypes.byref(p), ctypes.byref(h)))
        self.handle = h
        self.params = p
        self.n_streams, self.n_layers, self.capacity = n_streams, n_layers, capacity
        self.n_kv_heads, self.head_dim, self.n_q_heads = n_kv_heads, head_dim, n_q_heads
        self.kv_dim = n_kv_heads * head_dim
        self.dtype = dtype
        lay = CacheLayout()
        check(lib.vkv_cache_get_layout(h, ctypes.byref(lay)))
        self.layout = lay
        self.row_bytes = lay.row_bytes

    def close(self):
        if self.handle:
            check(lib.vkv_cache_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def read_rows(self, which, stream, layer, slot0, n_slots):
        """Synchronous copy of raw row bytes -> bytes object."""
        n = int(n_slots * self.row_bytes)
        buf = ctypes.create_string_buffer(max(n, 1))
        check(lib.vkv_cache_read_rows(self.handle, which, stream, layer, slot0, n_slots, buf, n))
        return buf.raw[:n]

    def zero(self, hip_stream=0):
        check(lib.vkv_cache_zero(self.handle, hip_stream))

    def append(self, stream, layer0, n_layers, segs, k_ptr, v_ptr, layer_stride=0, hip_stream=0):
        arr, n = _segs(segs)
        check(lib.vkv_append(self.handle, stream, layer0, n_layers, arr, n, k_ptr, v_ptr,
                             layer_stride, hip_stream))

    def gather(self, stream, layer, segs, k_dst, v_dst, hip_stream=0):
        arr, n = _segs(segs)
        check(lib.vkv_gather(self.handle, stream, layer, arr, n, k_dst, v_dst, hip_stream))

    def decode_attn(self, stream0, plans, layer0, n_layers, q_ptr, out_ptr, scale, hip_stream=0,
                    n_q_heads=None):
        arr = (Plan * len(plans))(*plans)
        check(lib.vkv_decode_attn(self.handle, stream0, len(plans), layer0, n_layers, arr, q_ptr,
                                  out_ptr, n_q_heads or self.n_q_heads, scale, hip_stream))

    def decoder_step(self, stream0, rings, positions, layer0, n_layers, q_ptr, k_ptr, v_ptr,
                     out_ptr, scale, hip_stream=0, n_q_heads=None):
        """rings: ctypes array of Ring (updated in place on success)."""
        ns = len(rings)
        pos = (_i64 * ns)(*positions)
        plans = (Plan * ns)()
        check(lib.vkv_decoder_step(self.handle, stream0, ns, rings, pos, layer0, n_layers, q_ptr,
                                   k_ptr, v_ptr, out_ptr, n_q_heads or self.n_q_heads, scale,
                                   plans, hip_stream))
        return plans

    def decoder_step_rope(self, stream0, rings, positions, layer0, n_layers, q_ptr, k_ptr, v_ptr,
                          out_ptr, scale, rope_theta, hip_stream=0, n_q_heads=None):
        """decoder_step with q/k before RoPE (rotated inside, ggml mode 0)."""
        ns = len(rings)
        pos = (_i64 * ns)(*positions)
        plans = (Plan * ns)()
        check(lib.vkv_decoder_step_rope(self.handle, stream0, ns, rings, pos, layer0, n_layers,
                                        q_ptr, k_ptr, v_ptr, out_ptr, n_q_heads or self.n_q_heads,
                                        scale, rope_theta, plans, hip_stream))
        return plans

    def decoder_layer_step(self, stream, plan, position, layer0, n_layers, q_ptr, k_ptr, v_ptr,
                           out_ptr, scale, rope_theta=0.0, hip_stream=0, n_q_heads=None):
        """One layer range of a token planned once with decoder_plan(ring,
        position, 1); commit after the last layer."""
        check(lib.vkv_decoder_layer_step(self.handle, stream, ctypes.byref(plan), position, layer0,
                                         n_layers, q_ptr, k_ptr, v_ptr, out_ptr,
                                         n_q_heads or self.n_q_heads, scale, rope_theta,
                                         hip_stream))

    def decoder_prefill(self, stream, ring, layer0, n_layers, n_tokens, q_ptr, k_ptr, v_ptr,
                        out_ptr, scale, hip_stream=0, n_q_heads=None):
        check(lib.vkv_decoder_prefill(self.handle, stream, ctypes.byref(ring), layer0, n_layers,
                                      n_tokens, q_ptr, k_ptr, v_ptr, out_ptr,
                                      n_q_heads or self.n_q_heads, scale, hip_stream))

    def enc_step(self, stream, plan, window, layer0, n_layers, q_ptr, k_ptr, v_ptr, out_ptr,
                 scale, hip_stream=0, n_q_heads=None):
        check(lib.vkv_enc_step(self.handle, stream, ctypes.byref(plan), window, layer0, n_layers,
                               q_ptr, k_ptr, v_ptr, out_ptr, n_q_heads or self.n_q_heads, scale,
                               hip_stream))

    def window_attn(self, stream, layer0, n_layers, segs, key_pos0, q_pos0, n_q, window, q_ptr,
                    out_ptr, scale, hip_stream=0, n_q_heads=None):
        arr, n = _segs(segs)
        check(lib.vkv_window_attn(self.handle, stream, layer0, n_layers, arr, n, key_pos0, q_pos0,
                                  n_q, window, q_ptr, out_ptr, n_q_heads or self.n_q_heads, scale,
                                  hip_stream))


def rope(x_ptr, n_outer, n_rows, row_len, head_dim, pos0, theta, hip_stream=0):
    """RoPE (ggml mode 0) in place on device f32 rows [n_outer][n_rows][row_len]."""
    check(lib.vkv_rope(x_ptr, n_outer, n_rows, row_len, head_dim, pos0, theta, hip_stream))


def q8_0_pack(x_ptr, blocks_ptr, n, hip_stream=0):
    check(lib.vkv_q8_0_pack(x_ptr, blocks_ptr, n, hip_stream))


def q8_0_unpack(blocks_ptr, y_ptr, n, hip_stream=0):
    check(lib.vkv_q8_0_unpack(blocks_ptr, y_ptr, n, hip_stream))


def matvec(x_ptr, n_in, outs, norm_w_ptr=None, ada_ptr=None, eps=1e-5, epilogue=MV_STORE,
           hip_stream=0):
    """y = W h for each (w_ptr, dtype, n_rows, y_ptr[, add_ptr]) in outs (device
    pointers); h = x, or rms_norm(x) * norm_w (* (1 + ada))."""
    arr = (MvOut * len(outs))()
    for i, o in enumerate(outs):
        w, dt, n, y = o[:4]
        add = o[4] if len(o) > 4 else None
        arr[i] = MvOut(w, dt, n, y, add)
    check(lib.vkv_matvec(x_ptr, n_in, norm_w_ptr, ada_ptr, eps, arr, len(outs), epilogue,
                         hip_stream))


def enc_conv_stem_workspace(conv_len, n_mel, dim, n_new):
    return lib.vkv_enc_conv_stem_workspace(conv_len, n_mel, dim, n_new)


def enc_conv_stem(mel_ptr, n_mel, plan, w0_ptr, b0_ptr, w1_ptr, b1_ptr, dim, x_ptr, ws_ptr,
                  ws_bytes, hip_stream=0):
    check(lib.vkv_enc_conv_stem(mel_ptr, n_mel, ctypes.byref(plan), w0_ptr, b0_ptr, w1_ptr,
                                b1_ptr, dim, x_ptr, ws_ptr, ws_bytes, hip_stream))


def encoder_chunk_workspace(model, n_new):
    return lib.vkv_encoder_chunk_workspace(ctypes.byref(model), n_new)


def encoder_chunk(cache, stream, plan, window, model, x_ptr, ws_ptr, ws_bytes, hip_stream=0):
    check(lib.vkv_encoder_chunk(cache.handle, stream, ctypes.byref(plan), window,
                                ctypes.byref(model), x_ptr, ws_ptr, ws_bytes, hip_stream))


def encoder_chunk_ring(cache, stream, plan, window, model, x_ptr, enc_out, ws_ptr, ws_bytes,
                       hip_stream=0):
    check(lib.vkv_encoder_chunk_ring(cache.handle, stream, ctypes.byref(plan), window,
                                     ctypes.byref(model), x_ptr, ctypes.byref(enc_out), ws_ptr,
                                     ws_bytes, hip_stream))


def row_ring_write(ring, row_start, src_ptr, n_rows, hip_stream=0):
    check(lib.vkv_row_ring_write(ctypes.byref(ring), row_start, src_ptr, n_rows, hip_stream))


def row_ring_read(ring, row_start, n_rows, dst_ptr, hip_stream=0):
    check(lib.vkv_row_ring_read(ctypes.byref(ring), row_start, n_rows, dst_ptr, hip_stream))


def adapter_workspace(adapter, n_groups):
    return lib.vkv_adapter_workspace(ctypes.byref(adapter), n_groups)


def adapter_commit(adapter, enc_out, audio_emb, group_start, n_groups, ws_ptr, ws_bytes,
                   hip_stream=0):
    check(lib.vkv_adapter_commit(ctypes.byref(adapter), ctypes.byref(enc_out),
                                 ctypes.byref(audio_emb), group_start, n_groups, ws_ptr, ws_bytes,
                                 hip_stream))


def matmul_workspace(n_cols, n_in):
    return lib.vkv_matmul_workspace(n_cols, n_in)


def matmul(x_ptr, n_cols, n_in, outs, ws_ptr, ws_bytes, norm_w_ptr=None, norm_b_ptr=None,
           ada_ptr=None, eps=1e-5, epilogue=MV_STORE, hip_stream=0):
    """Y = W h for n_cols input rows; outs: (w_ptr, dtype, n_rows, y_ptr[, add_ptr[, bias_ptr]])."""
    arr = (MmOut * len(outs))()
    for i, o in enumerate(outs):
        w, dt, n, y = o[:4]
        add = o[4] if len(o) > 4 else None
        bias = o[5] if len(o) > 5 else None
        arr[i] = MmOut(w, dt, n, y, add, bias)
    check(lib.vkv_matmul(x_ptr, n_cols, n_in, norm_w_ptr, norm_b_ptr, ada_ptr, eps, arr, len(outs),
                         epilogue, ws_ptr, ws_bytes, hip_stream))


def quantize_q8_k(x_ptr, n, blocks_ptr, norm_w_ptr=None, ada_ptr=None, eps=1e-5, hip_stream=0):
    check(lib.vkv_quantize_q8_k(x_ptr, n, norm_w_ptr, ada_ptr, eps, blocks_ptr, hip_stream))


def dequantize(dtype, blocks_ptr, n, y_ptr, hip_stream=0):
    check(lib.vkv_dequantize(dtype, blocks_ptr, n, y_ptr, hip_stream))


def embed(dtype, table_ptr, n_rows, n_cols, token, y_ptr, add_ptr=None, hip_stream=0):
    check(lib.vkv_embed(dtype, table_ptr, n_rows, n_cols, token, add_ptr, y_ptr, hip_stream))


def decoder_token_workspace(model):
    return lib.vkv_decoder_token_workspace(ctypes.byref(model))


def decoder_token(cache, stream, ring, model, token, audio_ptr, logits_ptr, token_out_ptr,
                  ws_ptr, ws_bytes, hip_stream=0):
    """One decoder token (embedding .. argmax) through vkv_decoder_token;
    returns the committed plan."""
    plan = Plan()
    check(lib.vkv_decoder_token(cache.handle, stream, ctypes.byref(ring), ctypes.byref(model),
                                token, audio_ptr, logits_ptr, token_out_ptr, ws_ptr, ws_bytes,
                                ctypes.byref(plan), hip_stream))
    return plan


TOKEN_SCRATCH_BYTES = 1 << 20   # VKV_TOKEN_SCRATCH_BYTES


def decoder_token_noalloc(cache, stream, ring, model, token, audio_ptr, logits_ptr, token_out_ptr,
                          hip_stream=0):
    """vkv_decoder_token with the library's static per-GPU scratch as its
    workspace (nothing allocated); returns the committed plan."""
    plan = Plan()
    check(lib.vkv_decoder_token_noalloc(cache.handle, stream, ctypes.byref(ring),
                                        ctypes.byref(model), token, audio_ptr, logits_ptr,
                                        token_out_ptr, ctypes.byref(plan), hip_stream))
    return plan


def decoder_prompt_workspace(model, n_tokens):
    return lib.vkv_decoder_prompt_workspace(ctypes.byref(model), n_tokens)


def decoder_prompt(cache, stream, ring, model, tokens, audio_ring, logits_ptr, token_out_ptr,
                   ws_ptr, ws_bytes, hip_stream=0):
    """The decoder prefill of a prompt (host token ids; audio_ring a RowRing
    or None) through vkv_decoder_prompt; returns the committed plan."""
    ids = (ctypes.c_int32 * max(len(tokens), 1))(*[int(t) for t in tokens])
    plan = Plan()
    check(lib.vkv_decoder_prompt(cache.handle, stream, ctypes.byref(ring), ctypes.byref(model),
                                 ids, len(tokens),
                                 ctypes.byref(audio_ring) if audio_ring is not None else None,
                                 logits_ptr, token_out_ptr, ws_ptr, ws_bytes, ctypes.byref(plan),
                                 hip_stream))
    return plan


def ada_scale_workspace(dim, ada_dim):
    return lib.vkv_ada_scale_workspace(dim, ada_dim)


def ada_scale(w0_ptr, w0_type, w2_ptr, w2_type, dim, ada_dim, t, out_ptr, ws_ptr, ws_bytes,
              hip_stream=0):
    check(lib.vkv_ada_scale(w0_ptr, w0_type, w2_ptr, w2_type, dim, ada_dim, t, out_ptr, ws_ptr,
                            ws_bytes, hip_stream))


def argmax(x_ptr, n, out_ptr, hip_stream=0):
    check(lib.vkv_argmax(x_ptr, n, out_ptr, hip_stream))


# tags of the synthetic inputs (shared with the oracle's generator)
TAG_K, TAG_V, TAG_Q = 1, 2, 3
TAG_EK, TAG_EV, TAG_EQ = 11, 12, 13


def synth_rows(dst_ptr, row_len, seed, tag, s0=0, ns=1, s_stride=0, l0=0, nl=1, l_stride=0,
               p0=0, np_=1, p_stride=0, hip_stream=0):
    """Rows (s0+i, l0+j, p0+k) at dst + (i*s_stride + j*l_stride + k*p_stride)*row_len.
    Zero strides default to a packed [s][l][p] layout."""
    if p_stride == 0:
        p_stride = 1
    if l_stride == 0:
        l_stride = np_ * p_stride
    if s_stride == 0:
        s_stride = nl * l_stride
    check(lib.vkv_synth_rows(dst_ptr, row_len, seed, tag, s0, ns, s_stride, l0, nl, l_stride, p0,
                             np_, p_stride, hip_stream))


# ---- GGUF files and models ----
GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32 = 0, 1, 2, 3, 4, 5
GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64 = 6, 7, 8, 9, 10, 11
GGUF_FLOAT64 = 12
_GGUF_NP = {GGUF_UINT8: "<u1", GGUF_INT8: "<i1", GGUF_UINT16: "<u2", GGUF_INT16: "<i2",
            GGUF_UINT32: "<u4", GGUF_INT32: "<i4", GGUF_FLOAT32: "<f4", GGUF_BOOL: "<u1",
            GGUF_UINT64: "<u8", GGUF_INT64: "<i8", GGUF_FLOAT64: "<f8"}


class Gguf:
    """A GGUF file opened by the library (metadata and tensor infos; the
    tensor bytes stay in the file mapping)."""

    def __init__(self, path):
        h = _vp()
        self.handle = None
        check(lib.vkv_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h
        self._close = lib.vkv_gguf_close   # still bound at interpreter exit

    def close(self):
        if self.handle:
            self._close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    @property
    def version(self):
        return lib.vkv_gguf_version(self.handle)

    @property
    def alignment(self):
        return lib.vkv_gguf_alignment(self.handle)

    @property
    def data_offset(self):
        return lib.vkv_gguf_data_offset(self.handle)

    def keys(self):
        return [lib.vkv_gguf_key(self.handle, i).decode() for i in range(lib.vkv_gguf_n_kv(self.handle))]

    def find_key(self, key):
        return lib.vkv_gguf_find_key(self.handle, key.encode())

    def kv_type(self, i):
        return lib.vkv_gguf_kv_type(self.handle, i)

    def value(self, key):
        """(type, value): scalars as Python numbers, strings as bytes, arrays
        as (element type, numpy array or list of bytes)"""
        import numpy as np
        i = self.find_key(key)
        if i < 0:
            raise KeyError(key)
        t = self.kv_type(i)
        if t == GGUF_STRING:
            p, n = _vp(), _u64()
            check(lib.vkv_gguf_get_str(self.handle, i, ctypes.byref(p), ctypes.byref(n)))
            return t, ctypes.string_at(p, n.value)
        if t == GGUF_ARRAY:
            et, n, d = _i32(), _u64(), _vp()
            check(lib.vkv_gguf_get_arr(self.handle, i, ctypes.byref(et), ctypes.byref(n),
                                       ctypes.byref(d)))
            if et.value == GGUF_STRING:
                out = []
                for j in range(n.value):
                    p, m = _vp(), _u64()
                    check(lib.vkv_gguf_get_arr_str(self.handle, i, j, ctypes.byref(p), ctypes.byref(m)))
                    out.append(ctypes.string_at(p, m.value))
                return t, (et.value, out)
            dt = np.dtype(_GGUF_NP[et.value])
            raw = ctypes.string_at(d, dt.itemsize * n.value) if n.value else b""
            return t, (et.value, np.frombuffer(raw, dt).copy())
        getters = {GGUF_INT32: (lib.vkv_gguf_get_i32, _i32), GGUF_UINT32: (lib.vkv_gguf_get_u32, _u32),
                   GGUF_INT64: (lib.vkv_gguf_get_i64, _i64), GGUF_FLOAT32: (lib.vkv_gguf_get_f32, _f32),
                   GGUF_FLOAT64: (lib.vkv_gguf_get_f64, ctypes.c_double),
                   GGUF_BOOL: (lib.vkv_gguf_get_bool, _i32)}
        if t in getters:
            fn, ct = getters[t]
            v = ct()
            check(fn(self.handle, i, ctypes.byref(v)))
            return t, v.value
        dt = np.dtype(_GGUF_NP[t])
        buf = ctypes.create_string_buffer(8)
        check(lib.vkv_gguf_get_scalar(self.handle, i, buf, 8))
        return t, np.frombuffer(buf.raw[:dt.itemsize], dt)[0].item()

    def tensors(self):
        out = []
        for i in range(lib.vkv_gguf_n_tensors(self.handle)):
            ti = GgufTensor()
            check(lib.vkv_gguf_tensor_info(self.handle, i, ctypes.byref(ti)))
            out.append(ti)
        return out

    def tensor_bytes(self, i):
        ti = GgufTensor()
        check(lib.vkv_gguf_tensor_info(self.handle, i, ctypes.byref(ti)))
        return ctypes.string_at(lib.vkv_gguf_tensor_data(self.handle, i), ti.nbytes)

    def hparams(self):
        hp = Hparams()
        check(lib.vkv_gguf_hparams(self.handle, ctypes.byref(hp)))
        return hp


class Model:
    """A GGUF model uploaded into one device allocation."""

    def __init__(self, path, device=0, hip_stream=0):
        h = _vp()
        self.handle = None
        check(lib.vkv_model_load(os.fsencode(path), device, hip_stream, ctypes.byref(h)))
        self.handle = h
        self._free = lib.vkv_model_free
        self.view = ModelView()
        check(lib.vkv_model_get_view(self.handle, ctypes.byref(self.view)))

    def set_ada(self, t, scales_ptr, hip_stream=0):
        """every decoder layer's ada scale at time t into scales [layers][dim];
        the view's layers point at them afterwards"""
        check(lib.vkv_model_set_ada(self.handle, t, scales_ptr, hip_stream))
        check(lib.vkv_model_get_view(self.handle, ctypes.byref(self.view)))

    def tensor(self, name):
        """(device address, GgufTensor) or (None, None)"""
        ti = GgufTensor()
        p = lib.vkv_model_tensor(self.handle, name.encode(), ctypes.byref(ti))
        return (p, ti) if p else (None, None)

    def close(self):
        if self.handle:
            self._free(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

