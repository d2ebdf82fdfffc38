"""The C ABI boundary without a GPU: libvkv.so loads, exports exactly the
functions include/vkv.h declares, its struct layouts match the ctypes mirror
(and the reference's field order), and argument errors come back as statuses
(never exceptions) with the out-parameters cleared."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

import oracle
import vkv

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "vkv.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vkv_\w+)\s*\(", text)))


def test_exports_match_header():
    declared = header_functions()
    out = subprocess.run(["nm", "-D", "--defined-only", vkv.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r" T (vkv_\w+)$", out, flags=re.M)))
    assert declared == exported
    assert sorted(vkv.PROTOTYPES) == declared
    for name in declared:
        assert hasattr(vkv.lib, name)


def test_struct_layout_matches_c():
    """sizeof/offsetof from a C compilation of vkv.h == the ctypes mirror ==
    the oracle's restatement of the reference structs."""
    structs = {
        "vkv_ring": (vkv.Ring, oracle.Ring),
        "vkv_seg": (vkv.Seg, oracle.Seg),
        "vkv_plan": (vkv.Plan, oracle.Plan),
        "vkv_enc_plan": (vkv.EncPlan, oracle.EncPlan),
        "vkv_enc_schedule": (vkv.EncSchedule, None),
        "vkv_enc_run": (vkv.EncRun, oracle.EncRun),
        "vkv_cache_params": (vkv.CacheParams, None),
        "vkv_cache_layout": (vkv.CacheLayout, None),
        "vkv_mv_out": (vkv.MvOut, None),
        "vkv_mm_out": (vkv.MmOut, None),
        "vkv_enc_layer": (vkv.EncLayer, None),
        "vkv_enc_model": (vkv.EncModel, None),
        "vkv_dec_layer": (vkv.DecLayer, None),
        "vkv_dec_model": (vkv.DecModel, None),
        "vkv_row_ring": (vkv.RowRing, None),
        "vkv_adapter": (vkv.Adapter, None),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "vkv.h"', "int main(void){"]
    for cname, (py, _) in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _t in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, "layout.c")
        exe = os.path.join(td, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), src, "-o", exe],
                       check=True)
        got = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    table = {}
    for line in got:
        if line:
            name, field, val = line.split()
            table[(name, field)] = int(val)
    for cname, (py, orc) in structs.items():
        assert table[(cname, "size")] == ctypes.sizeof(py), cname
        if orc is not None:
            assert ctypes.sizeof(orc) == ctypes.sizeof(py)
        for f, _t in py._fields_:
            assert table[(cname, f)] == getattr(py, f).offset, (cname, f)
            if orc is not None:
                assert getattr(orc, f).offset == getattr(py, f).offset


def test_api_version():
    assert vkv.lib.vkv_api_version() == 1


def test_error_statuses_without_device():
    L = vkv.lib
    # planner errors mirror the reference's `false` returns
    r = vkv.new_ring(8)
    p = vkv.Plan()
    p.n_new = 77
    assert L.vkv_decoder_plan(ctypes.byref(r), 1, 1, ctypes.byref(p)) == vkv.INVALID_ARGUMENT
    assert p.n_new == 0                                  # out-param cleared first
    assert "invalid absolute position" in vkv.last_error()
    assert L.vkv_decoder_plan(None, 0, 1, ctypes.byref(p)) == vkv.INVALID_ARGUMENT
    assert L.vkv_decoder_plan(ctypes.byref(r), 0, 1, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_decoder_commit(None, None) == vkv.INVALID_ARGUMENT
    e = vkv.EncPlan()
    assert L.vkv_enc_plan_build(0, 129, 878, 750, ctypes.byref(e)) == vkv.INVALID_ARGUMENT
    assert L.vkv_enc_plan_build(-1, 4, 878, 750, ctypes.byref(e)) == vkv.INVALID_ARGUMENT
    # cache creation: bad shapes are rejected before touching a device
    h = ctypes.c_void_p(1234)
    bad = vkv.CacheParams(ctypes.sizeof(vkv.CacheParams), 1, 1, 8, 8, 100, 32, vkv.Q8_0, 0)
    assert L.vkv_cache_create(ctypes.byref(bad), ctypes.byref(h)) == vkv.INVALID_ARGUMENT
    assert not h.value
    small = vkv.CacheParams(8, 1, 1, 8, 8, 128, 32, vkv.F16, 0)
    assert L.vkv_cache_create(ctypes.byref(small), ctypes.byref(h)) == vkv.INVALID_ARGUMENT
    odd = vkv.CacheParams(ctypes.sizeof(vkv.CacheParams), 1, 1, 8, 8, 128, 30, vkv.F16, 0)
    assert L.vkv_cache_create(ctypes.byref(odd), ctypes.byref(h)) == vkv.INVALID_ARGUMENT
    badtype = vkv.CacheParams(ctypes.sizeof(vkv.CacheParams), 1, 1, 8, 8, 128, 32, 2, 0)
    assert L.vkv_cache_create(ctypes.byref(badtype), ctypes.byref(h)) == vkv.INVALID_ARGUMENT
    # kernel selection fields: contradictory or unknown flags and out-of-range
    # tuning values are rejected before any device call
    full = ctypes.sizeof(vkv.CacheParams)
    for extra, what in (((vkv.KERNEL_DECODE_HEADS | vkv.KERNEL_DECODE_ROWS, 0, 0, 0), "kernel_flags"),
                        ((vkv.KERNEL_XCD_SWIZZLE | vkv.KERNEL_NO_XCD_SWIZZLE, 0, 0, 0), "kernel_flags"),
                        ((0x40, 0, 0, 0), "kernel_flags"),
                        ((0, 100, 0, 0), "decode_chunk"), ((0, 0, 6, 0), "decode_chunk"),
                        ((0, 0, 0, 5), "decode_chunk")):
        p = vkv.CacheParams(full, 1, 1, 8, 8, 128, 32, vkv.F16, 0, *extra)
        assert L.vkv_cache_create(ctypes.byref(p), ctypes.byref(h)) == vkv.INVALID_ARGUMENT
        assert what in vkv.last_error() and not h.value
    # a parameter block that ends at `device` is accepted (its shape is then checked)
    base = vkv.CacheParams(vkv.CacheParams.kernel_flags.offset, 1, 1, 8, 8, 100, 32, vkv.Q8_0, 0,
                           0x40, 0, 0, 0)
    assert L.vkv_cache_create(ctypes.byref(base), ctypes.byref(h)) == vkv.INVALID_ARGUMENT
    assert "invalid shape" in vkv.last_error()
    # hot-path calls on a null cache
    segs = (vkv.Seg * 2)()
    assert L.vkv_append(None, 0, 0, 1, segs, 1, None, None, 0, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_gather(None, 0, 0, segs, 1, None, None, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_decode_attn(None, 0, 1, 0, 1, None, None, None, 32, 1.0, None) == vkv.INVALID_ARGUMENT
    rings = (vkv.Ring * 1)()
    pos = (ctypes.c_int64 * 1)()
    plans = (vkv.Plan * 1)()
    plans[0].n_new = 5
    assert L.vkv_decoder_step(None, 0, 1, rings, pos, 0, 1, None, None, None, None, 32, 1.0,
                              plans, None) == vkv.INVALID_ARGUMENT
    assert plans[0].n_new == 0
    assert L.vkv_q8_0_pack(None, None, 33, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_q8_0_unpack(None, None, -32, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_synth_rows(None, 4, 1, 1, 0, 1, 1, 0, 1, 1, 0, 1, 1, None) == vkv.INVALID_ARGUMENT
    # matrix-vector products: shapes, dtypes and pointers checked on the host
    outs = (vkv.MvOut * 2)()
    outs[0] = vkv.MvOut(16, vkv.Q4_K, 8, 16, None)
    outs[1] = vkv.MvOut(16, vkv.Q6_K, 8, 16, None)
    x = ctypes.c_void_p(4096)
    assert L.vkv_matvec(x, 300, None, None, 1e-5, outs, 1, 0, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_matvec(x, 12288 + 256, None, None, 1e-5, outs, 1, 0, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_matvec(x, 3072, None, 4096, 1e-5, outs, 1, 0, None) == vkv.INVALID_ARGUMENT
    assert "ada requires norm_w" in vkv.last_error()
    assert L.vkv_matvec(ctypes.c_void_p(4100), 3072, None, None, 1e-5, outs, 1, 0,
                        None) == vkv.INVALID_ARGUMENT
    assert L.vkv_matvec(x, 3072, None, None, 1e-5, outs, 5, 0, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_matvec(x, 3072, None, None, 1e-5, outs, 2, 7, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_matvec(x, 3072, None, None, 1e-5, outs, 2, vkv.MV_SWIGLU,
                        None) == vkv.INVALID_ARGUMENT          # SwiGLU needs equal dtypes
    wrong = (vkv.MvOut * 1)(vkv.MvOut(16, 2, 8, 16, None))       # ggml Q4_0: not taken
    assert L.vkv_matvec(x, 3072, None, None, 1e-5, wrong, 1, 0, None) == vkv.INVALID_ARGUMENT
    huge = (vkv.MvOut * 1)(vkv.MvOut(16, vkv.Q6_K, 1 << 30, 16, None))
    assert L.vkv_matvec(x, 3072, None, None, 1e-5, huge, 1, 0, None) == vkv.INVALID_ARGUMENT
    assert "4 GiB" in vkv.last_error()
    assert L.vkv_quantize_q8_k(x, 3072, None, None, 1e-5, 4098, None) == vkv.INVALID_ARGUMENT
    mo = (vkv.MmOut * 1)(vkv.MmOut(16, vkv.Q4_K, 8, 16, None, None))
    assert L.vkv_matmul_workspace(16, 1280) > 16 * 1280
    assert L.vkv_matmul_workspace(0, 1280) == 0
    assert L.vkv_matmul(x, 16, 1280, None, None, None, 1e-5, mo, 1, 0, None, 0,
                        None) == vkv.INVALID_ARGUMENT                 # no workspace
    assert L.vkv_matmul(x, 16, 1280, None, 4096, None, 1e-5, mo, 1, 0, 4096, 1 << 20,
                        None) == vkv.INVALID_ARGUMENT                 # norm_b without norm_w
    assert L.vkv_matmul(x, 16, 1280, None, None, None, 1e-5, mo, 1, 0, 4096, 16,
                        None) == vkv.BUFFER_TOO_SMALL
    assert L.vkv_dequantize(vkv.F16, 16, 256, 16, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_embed(vkv.Q6_K, 16, 10, 3072, 10, None, 16, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_embed(vkv.Q6_K, 16, 10, 3072, -1, None, 16, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_argmax(x, 0, 16, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_argmax(ctypes.c_void_p(4100), 10, 16, None) == vkv.INVALID_ARGUMENT
    em = vkv.EncModel()
    assert L.vkv_encoder_chunk_workspace(ctypes.byref(em), 16) == 0
    assert L.vkv_encoder_chunk(None, 0, None, 750, ctypes.byref(em), None, None, 0,
                               None) == vkv.INVALID_ARGUMENT
    m = vkv.DecModel()
    assert L.vkv_decoder_token_workspace(ctypes.byref(m)) == 0
    assert L.vkv_decoder_token(None, 0, None, ctypes.byref(m), 0, None, None, None, None, 0,
                               None, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_decoder_prompt_workspace(ctypes.byref(m), 38) == 0
    ids = (ctypes.c_int32 * 2)(1, 2)
    plan = vkv.Plan()
    plan.n_new = 7
    assert L.vkv_decoder_prompt(None, 0, None, ctypes.byref(m), ids, 2, None, None, None, None, 0,
                                ctypes.byref(plan), None) == vkv.INVALID_ARGUMENT
    assert plan.n_new == 0                                        # out-parameter cleared
    assert L.vkv_decoder_layer_step(None, 0, None, 0, 0, 1, None, None, None, None, 32, 1.0,
                                    1e6, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_dequantize(vkv.Q4_K, 16, 255, 16, None) == vkv.INVALID_ARGUMENT
    # the rows rings and the adapter: validation precedes any device work
    enc = vkv.RowRing(4096, 256, 1280)
    aemb = vkv.RowRing(4096, 256, 3072)
    assert L.vkv_row_ring_write(ctypes.byref(enc), 0, 4096, 257, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_row_ring_write(ctypes.byref(enc), -1, 4096, 1, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_row_ring_read(ctypes.byref(enc), 0, 0, 4096, None) == vkv.INVALID_ARGUMENT
    assert L.vkv_row_ring_read(ctypes.byref(vkv.RowRing(4100, 256, 1280)), 0, 1, 4096,
                               None) == vkv.INVALID_ARGUMENT        # misaligned rows
    ad = vkv.Adapter(16, 16, vkv.Q4_K, vkv.Q4_K, 1280, 3072, 4)
    assert L.vkv_adapter_workspace(ctypes.byref(ad), 1) >= 3072 * 4
    assert L.vkv_adapter_workspace(ctypes.byref(ad), 32) > L.vkv_matmul_workspace(32, 5120)
    assert L.vkv_adapter_workspace(ctypes.byref(ad), 0) == 0
    assert L.vkv_adapter_commit(ctypes.byref(ad), ctypes.byref(enc), ctypes.byref(aemb), 0, 1,
                                4096, 16, None) == vkv.BUFFER_TOO_SMALL
    assert L.vkv_adapter_commit(ctypes.byref(ad), ctypes.byref(enc), ctypes.byref(aemb), 0, 0,
                                4096, 1 << 20, None) == vkv.INVALID_ARGUMENT
    odd = vkv.RowRing(4096, 258, 1280)
    assert L.vkv_adapter_commit(ctypes.byref(ad), ctypes.byref(odd), ctypes.byref(aemb), 0, 1,
                                4096, 1 << 20, None) == vkv.INVALID_ARGUMENT
    assert "multiple of 4" in vkv.last_error()
    assert L.vkv_adapter_commit(ctypes.byref(ad), ctypes.byref(aemb), ctypes.byref(enc), 0, 1,
                                4096, 1 << 20, None) == vkv.INVALID_ARGUMENT   # widths swapped
    bad = vkv.Adapter(16, 16, 2, vkv.Q4_K, 1280, 3072, 4)
    assert L.vkv_adapter_workspace(ctypes.byref(bad), 1) == 0
    assert L.vkv_encoder_chunk_ring(None, 0, None, 750, ctypes.byref(em), None, None, None, 0,
                                    None) == vkv.INVALID_ARGUMENT
    assert L.vkv_matvec(x, 3072, None, None, 1e-5,
                        (vkv.MvOut * 1)(vkv.MvOut(16, vkv.Q4_K, 8, 16, 16)), 1, vkv.MV_GELU,
                        None) == vkv.INVALID_ARGUMENT           # GELU has no residual
    assert L.vkv_cache_destroy(None) == vkv.OK
    with pytest.raises(vkv.VkvError) as ei:
        vkv.decoder_plan(r, 5, 1)
    assert ei.value.status == vkv.INVALID_ARGUMENT


def test_product_does_not_reference_the_oracle():
    """The shipped library and package neither link nor import the oracle."""
    out = subprocess.run(["ldd", vkv.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in out
    pkg = os.path.join(REPO, "voxtral.cpp_amd")
    for root, _dirs, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(root, f)).read()
                assert "import oracle" not in text and "liboracle" not in text, f
