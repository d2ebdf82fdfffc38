#!/usr/bin/env python3
"""KV-cache hot-path benchmark on one MI355X.

Default workload (the headline line): the longform streaming decoder -- 26
layers, an 8192-slot sliding ring that is full and wrapping (every step evicts
the oldest position), F16 KV, 32 query / 8 KV heads x 128, one stream.  One
step = one token = for every layer, append the token's K/V row (f32 -> f16) at
pos % 8192 and run the single-query GQA attention over all 8192 retained
positions, through the vkv_decoder_step C entry point: one k_decode_rows launch
(append fused in its prologue; a work group per (layer, 912-slot chunk) reads
whole 2 KiB rows for all 8 kv heads: 234 work groups, one per CU) and one
k_combine launch merging the 9 chunks per head.  Inputs (Q, K, V for every timed step) are generated on the
device before timing.

Other workloads (--workload), reported on the same contract:
  longform_rope_f16  the default workload through vkv_decoder_step_rope: Q and
               K arrive before RoPE (ggml mode 0, theta 1e6) and are rotated
               inside the step.
  stream4096_f16  the decoder from an empty ring: steps 0..4095 (append at
               pos, attend pos+1 keys; no wrap), every step timed; tokens/s
               over the whole run, bytes summed over the growing windows.
  layerwise_f16  the default workload in the decoder's own call shape: per
               token 26 vkv_decoder_layer_step calls, one layer each (layer
               l+1's Q depends on layer l's output), RoPE fused (theta 1e6),
               then the ring commit; tokens/s and the mean time per layer.
  layerwise_q8_0  the same call shape over a q8_0 cache (one stream).
  layer1_f16   one decoder layer, 1024 positions prefilled, then one step per
               token (append + attention over 1025 positions): a latency case.
  q8_0_batch8  the same decoder shape with q8_0 K/V (quantize-on-append,
               dequantize-in-register attention), 8 independent streams per
               step; tokens/s counts all 8 streams.
  encoder_f16  the encoder's streaming window: 32 layers, 32 heads x 64, an
               878-slot ring, window 750, 16 new frames per chunk appended and
               attended as a 16-query block (MFMA tile); frames/s.
  encoder_f32  the same with the reference's default F32 encoder ring (f32
               MFMA tile, 460 MB ring); frames/s.
  decoder_weights_q4km  the decoder step's projections on Q4_K_M weights
               (random valid blocks): per layer RMSNorm+Q/K/V (one call), O +
               residual, RMSNorm*(1+ada)+SwiGLU W1/W3, W2 + residual; then the
               final norm + the 131072-row Q6_K logits -- 105 vkv_matvec
               calls, 2.24 GB of weights per token; tokens/s.
  encoder_chunk_q4km  the encoder for one 16-frame chunk: the conv stem over
               the chunk's Mel window (vkv_enc_conv_stem), then
               vkv_encoder_chunk: 32 layers x (RMSNorm + Q/K/V with biases,
               RoPE, ring append + window-750 attention, O + bias + residual,
               RMSNorm + SwiGLU, W2 + bias + residual) + final norm, on Q4_K_M
               weights (539 MB per chunk), steady state; frames/s.
  adapter_q4km / adapter_group_q4km  the adapter over the rows rings: 32
               groups (the startup commit) or one group (the steady 80 ms
               commit); audio embeddings/s.
  model_load_q4km  a full-size realtime Q4_K_M GGUF file (the reference's
               tensor names, dims and quantization mix; synthetic bytes)
               written to $TMPDIR once, then vkv_model_load into one device
               allocation per step (file in the page cache); GB/s.
  realtime_step_q4km  one 80 ms step of the streaming path: conv stem +
               encoder over 4 new frames into the encoder-output ring, the
               adapter over the completed group, one decoder token reading its
               audio row (full 8192-slot ring); steps/s (x 0.08 = the
               realtime factor).
  realtime_pipelined_q4km  the same steps on two HIP streams, the decoder
               one group behind the encoder (token i reads step i-1's audio
               row while step i's encoder and adapter run); steps/s.
  decoder_token_q4km  one whole decoder token through vkv_decoder_token:
               embedding + audio row, 26 x (RMSNorm+QKV, RoPE + K/V append +
               attention over the full 8192-slot F16 ring, O + residual,
               RMSNorm*(1+ada) + SwiGLU, W2 + residual), final norm, logits,
               argmax; tokens/s.
  decoder_loop_q4km  the production token loop (run_decoder_step): per token
               vkv_decoder_token, the 4-byte token copied to pinned host
               memory, one stream synchronize, the token fed to the next
               step; tokens/s and per-token latency p50/p90/p99 (host wall
               clock; --steps tokens, 1000 by default for this workload).
  decoder_prompt_q4km  the decoder prefill of a 38-token prompt at the stream
               start through vkv_decoder_prompt: token + audio rows, 26 x
               (multi-row Q4_K_M products with RoPE in the epilogue, causal
               attention + K/V append, O, SwiGLU, W2), final norm, logits of
               the last token; prompt tokens/s.
  decoder_token_q8_0 / decoder_weights_q8_0  decoder_token_q4km and
               decoder_weights_q4km on a Q8_0 file's weights (every matrix
               Q8_0, src/voxtral-quantize.cpp:95-96; products on q8_0 input
               images).

Prints one JSON line: throughput, the roofline of the step (algorithmic bytes /
average step time from HIP events on the launch stream), the HBM traffic from
the committed rocprofv3 counter runs, and the CPU baseline (the oracle's
threaded restatement of ggml's CPU flash-attention step, timed on a bounded
sample on this host; decode workloads only).
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "voxtral.cpp_amd"))
sys.path.insert(0, ROOT)

LAYERS, CAP, KVH, HD, QH = 26, 8192, 8, 128, 32
KV_DIM, Q_DIM = KVH * HD, QH * HD
E_LAYERS, E_CAP, E_HEADS, E_HD, E_WIN, E_CHUNK = 32, 878, 32, 64, 750, 16
E_DIM = E_HEADS * E_HD
SEED = 20261201
HBM_PEAK_GBPS = 8000.0
METRIC = "decode attn+KV-append tokens/s and achieved HBM GB/s (% of peak) at 8192 window"

# F16 = 1, Q8_0 = 8 (ggml_type numbering, as in include/vkv.h)
WORKLOADS = {
    "longform_f16": dict(dtype=1, dtype_name="f16", streams=1,
                         pmc="decode_f16_26x8192_pmc.json", kern="k_decode_rows"),
    "longform_rope_f16": dict(dtype=1, dtype_name="f16", streams=1, pmc=""),
    "stream4096_f16": dict(dtype=1, dtype_name="f16", streams=1, pmc=""),
    "layer1_f16": dict(dtype=1, dtype_name="f16", streams=1, pmc=""),
    "layerwise_f16": dict(dtype=1, dtype_name="f16", streams=1,
                          pmc="decode_f16_26x8192_layerwise_pmc.json", kern=""),
    "layerwise_q8_0": dict(dtype=8, dtype_name="q8_0", streams=1, pmc=""),
    "q8_0_batch8": dict(dtype=8, dtype_name="q8_0", streams=8,
                        pmc="decode_q8_0_8x26x8192_pmc.json", kern="k_decode_q8rows"),
    "encoder_f16": dict(dtype=1, dtype_name="f16", streams=1,
                        pmc="encoder_f16_32x750_pmc.json", kern="k_window_mfma<64, 4, 4, 1>"),
    "encoder_f32": dict(dtype=0, dtype_name="f32", streams=1,
                        pmc="encoder_f32_32x750_pmc.json", kern="k_window_mfma_f32_64"),
    "encoder_chunk_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k weights (MFMA int8), f16 KV",
                               streams=1, pmc="encoder_chunk_q4km_pmc.json", kern="",
                               data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) frames and "
                                    "KV rows, generated on device)"),
    "decoder_token_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k weights, f16 KV",
                               streams=1, pmc="decoder_token_q4km_pmc.json", kern="",
                               data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) inputs and "
                                    "KV rows, generated on device)"),
    "decoder_loop_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k weights, f16 KV",
                              streams=1, pmc="",
                              data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) audio rows "
                                   "and KV rows, generated on device; tokens fed back greedily)"),
    "adapter_q4km": dict(dtype=12, dtype_name="q4_k x q8_k weights (MFMA int8), f32 rings",
                         streams=1, pmc="adapter_q4km_pmc.json", kern="", groups=32,
                         data="synthetic (random valid Q4_K blocks, N(0,1) encoder frames, "
                              "generated on device)"),
    "adapter_group_q4km": dict(dtype=12, dtype_name="q4_k x q8_k weights (int8 dot), f32 rings",
                               streams=1, pmc="", groups=1,
                               data="synthetic (random valid Q4_K blocks, N(0,1) encoder "
                                    "frames, generated on device)"),
    "model_load_q4km": dict(dtype=12, dtype_name="bytes (q4_k/q6_k/f16/f32 tensors copied verbatim)",
                            streams=1, pmc="",
                            data="synthetic (a full-size realtime Q4_K_M GGUF file of random "
                                 "bytes, written to local disk before timing)"),
    "realtime_step_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k weights, f16 KV, f32 rings",
                               streams=1, pmc="realtime_step_q4km_pmc.json", kern="",
                               data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) Mel windows "
                                    "and KV rows, generated on device)"),
    "realtime_pipelined_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k weights, f16 KV, f32 rings",
                                    streams=1, pmc="realtime_pipelined_q4km_pmc.json", kern="",
                                    data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) Mel "
                                         "windows and KV rows, generated on device)"),
    "decoder_prompt_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k weights (MFMA int8), f16 KV",
                                streams=1, pmc="decoder_prompt_q4km_pmc.json", kern="",
                                data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) audio rows, "
                                     "random prompt tokens, generated on device)"),
    "decoder_token_q8_0": dict(dtype=8, dtype_name="q8_0 x q8_0 weights, f16 KV", streams=1,
                               pmc="decoder_token_q8_0_pmc.json", kern="",
                               data="synthetic (random valid Q8_0 blocks, N(0,1) inputs and KV "
                                    "rows, generated on device)"),
    "decoder_weights_q8_0": dict(dtype=8, dtype_name="q8_0 x q8_0 (int8 dot)", streams=1,
                                 pmc="matvec_q8_0_26l_pmc.json", kern="",
                                 data="synthetic (random valid Q8_0 blocks, N(0,1) inputs, "
                                      "generated on device)"),
    "decoder_weights_q4km": dict(dtype=12, dtype_name="q4_k/q6_k x q8_k (int8 dot)", streams=1,
                                 pmc="matvec_q4km_26l_pmc.json", kern="",
                                 data="synthetic (random valid Q4_K/Q6_K blocks, N(0,1) inputs, "
                                      "generated on device)"),
}

# decoder projections: (name, dtype, rows, n_in); ggml Q8_0 = 8, Q4_K = 12, Q6_K = 14
DIM, HIDDEN, VOCAB = 3072, 9216, 131072
LAYER_MATS = [("attn_q", 12, Q_DIM, DIM), ("attn_k", 12, KV_DIM, DIM), ("attn_v", 14, KV_DIM, DIM),
              ("attn_o", 12, DIM, Q_DIM), ("ffn_w1", 12, HIDDEN, DIM), ("ffn_w3", 12, HIDDEN, DIM),
              ("ffn_w2", 14, DIM, HIDDEN)]
KQ_BLOCK = {8: 272, 12: 144, 14: 210}   # bytes per 256 weights
# the decoder's weight file kind: the Q4_K_M mix above (src/voxtral-quantize.cpp:
# 148-159; output Q6_K) or a Q8_0 file (:95-96, every matrix Q8_0); set from
# the workload's name
MIX = "q4km"


def layer_mats():
    return LAYER_MATS if MIX == "q4km" else [(nm, 8, r, n) for nm, _, r, n in LAYER_MATS]


def out_type():
    return 14 if MIX == "q4km" else 8


def mat_bytes(dtype, rows, n_in):
    return rows * (n_in // 256) * KQ_BLOCK[dtype]


def weights_bytes_per_token():
    per_layer = sum(mat_bytes(dt, r, n) for _, dt, r, n in layer_mats())
    return LAYERS * per_layer + mat_bytes(out_type(), VOCAB, DIM)


def random_blocks_np(rng, dtype, rows, n_in):
    """random_kq_device's blocks on the host (numpy), for the CPU legs"""
    import numpy as np
    if dtype == 8:
        nb = rows * (n_in // 32)
        w = np.empty((nb, 34), np.uint8)
        w[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
        w[:, 0:2] = rng.uniform(2e-4, 8e-3, nb).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return w.reshape(-1)
    w = rng.integers(0, 256, size=(rows * (n_in // 256), KQ_BLOCK[dtype]), dtype=np.uint8)
    if dtype == 12:
        w[:, 0:2] = rng.uniform(2e-4, 4e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        w[:, 2:4] = rng.uniform(1e-4, 2e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    else:
        w[:, 208:210] = rng.uniform(1e-5, 2e-4, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def random_kq_device(dtype, rows, n_in, gen):
    """Random valid k-quant (or Q8_0) blocks on the device: random bytes, fp16
    scales set to finite moderate values (Q8_0: codes in [-127, 127])."""
    import torch
    if dtype == 8:
        nb = rows * (n_in // 32)
        w = torch.randint(-127, 128, (nb, 34), dtype=torch.int8, device="cuda",
                          generator=gen).view(torch.uint8)
        w[:, 0:2] = torch.empty(nb, dtype=torch.float16, device="cuda").uniform_(
            2e-4, 8e-3, generator=gen).view(torch.uint8).view(nb, 2)
        return w.reshape(-1)
    nb = rows * (n_in // 256)
    w = torch.randint(0, 256, (nb, KQ_BLOCK[dtype]), dtype=torch.uint8, device="cuda",
                      generator=gen)
    if dtype == 12:
        w[:, 0:2] = torch.empty(nb, dtype=torch.float16, device="cuda").uniform_(
            2e-4, 4e-3, generator=gen).view(torch.uint8).view(nb, 2)
        w[:, 2:4] = torch.empty(nb, dtype=torch.float16, device="cuda").uniform_(
            1e-4, 2e-3, generator=gen).view(torch.uint8).view(nb, 2)
    else:
        w[:, 208:210] = torch.empty(nb, dtype=torch.float16, device="cuda").uniform_(
            1e-5, 2e-4, generator=gen).view(torch.uint8).view(nb, 2)
    return w.view(-1)


def gpu_weights(steps, warmup):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    mats = layer_mats()
    T = {name: dt for name, dt, _, _ in mats}
    layers = [{name: random_kq_device(dt, r, n, gen) for name, dt, r, n in mats}
              for _ in range(LAYERS)]
    logits_w = random_kq_device(out_type(), VOCAB, DIM, gen)
    norms = torch.empty(LAYERS * 2 + 1, DIM, device="cuda").uniform_(0.5, 1.5, generator=gen)
    ada = torch.empty(LAYERS, DIM, device="cuda").uniform_(-0.3, 0.3, generator=gen)
    x0 = torch.randn(DIM, device="cuda", generator=gen)
    attn = torch.randn(Q_DIM, device="cuda", generator=gen)   # stands in for attention output
    x = torch.empty(DIM, device="cuda")
    q, k, v = (torch.empty(n, device="cuda") for n in (Q_DIM, KV_DIM, KV_DIM))
    h = torch.empty(HIDDEN, device="cuda")
    logits = torch.empty(VOCAB, device="cuda")
    eps = 1e-5

    def step(_):
        x.copy_(x0)
        xp = x.data_ptr()
        for l, L in enumerate(layers):
            vkv.matvec(xp, DIM, [(L["attn_q"].data_ptr(), T["attn_q"], Q_DIM, q.data_ptr()),
                                 (L["attn_k"].data_ptr(), T["attn_k"], KV_DIM, k.data_ptr()),
                                 (L["attn_v"].data_ptr(), T["attn_v"], KV_DIM, v.data_ptr())],
                       norm_w_ptr=norms[2 * l].data_ptr(), eps=eps, hip_stream=sp)
            vkv.matvec(attn.data_ptr(), Q_DIM,
                       [(L["attn_o"].data_ptr(), T["attn_o"], DIM, xp, xp)], hip_stream=sp)
            vkv.matvec(xp, DIM, [(L["ffn_w1"].data_ptr(), T["ffn_w1"], HIDDEN, h.data_ptr()),
                                 (L["ffn_w3"].data_ptr(), T["ffn_w3"], HIDDEN, None)],
                       norm_w_ptr=norms[2 * l + 1].data_ptr(), ada_ptr=ada[l].data_ptr(),
                       eps=eps, epilogue=vkv.MV_SWIGLU, hip_stream=sp)
            vkv.matvec(h.data_ptr(), HIDDEN, [(L["ffn_w2"].data_ptr(), T["ffn_w2"], DIM, xp, xp)],
                       hip_stream=sp)
        vkv.matvec(xp, DIM, [(logits_w.data_ptr(), out_type(), VOCAB, logits.data_ptr())],
                   norm_w_ptr=norms[2 * LAYERS].data_ptr(), eps=eps, hip_stream=sp)

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    assert bool(torch.isfinite(logits).all()) and bool(torch.isfinite(x).all())
    return total_ms, step_ms, wall


E_HID = 5120
ENC_MATS = [("attn_q", 12, E_DIM, 1280), ("attn_k", 12, E_DIM, 1280), ("attn_v", 14, E_DIM, 1280),
            ("attn_o", 12, 1280, E_DIM), ("ffn_w1", 12, E_HID, 1280), ("ffn_w3", 12, E_HID, 1280),
            ("ffn_w2", 14, 1280, E_HID)]


A_ENC, A_DOWN, A_RING = 1280, 4, 256


def adapter_bytes(n_groups):
    """both adapter matrices (Q4_K) + the groups' encoder rows read and audio
    rows written"""
    return (mat_bytes(12, DIM, A_ENC * A_DOWN) + mat_bytes(12, DIM, DIM) +
            n_groups * (A_ENC * A_DOWN + DIM) * 4)


def gpu_adapter(n_groups, steps, warmup):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    w0 = random_kq_device(12, DIM, A_ENC * A_DOWN, gen)
    w2 = random_kq_device(12, DIM, DIM, gen)
    enc = torch.randn(A_RING, A_ENC, device="cuda", generator=gen)
    aemb = torch.zeros(A_RING, DIM, device="cuda")
    enc_r = vkv.RowRing(enc.data_ptr(), A_RING, A_ENC)
    aemb_r = vkv.RowRing(aemb.data_ptr(), A_RING, DIM)
    ad = vkv.Adapter(w0.data_ptr(), w2.data_ptr(), 12, 12, A_ENC, DIM, A_DOWN)
    ws_bytes = vkv.adapter_workspace(ad, n_groups)
    ws = torch.empty(ws_bytes // 4 + 64, device="cuda")
    ws_ptr = (ws.data_ptr() + 255) & ~255

    def step(i):
        vkv.adapter_commit(ad, enc_r, aemb_r, i * n_groups, n_groups, ws_ptr, ws_bytes,
                           hip_stream=sp)

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    assert bool(torch.isfinite(aemb).all())
    return total_ms, step_ms, wall


def cpu_adapter_leg(n_groups, target_seconds):
    """The oracle's adapter (gather, ggml's generic CPU q4_K x q8_K matvec,
    GELU, matvec) on the same shapes, threaded over rows."""
    import numpy as np

    import oracle

    threads = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(SEED)

    def mat(r, n):
        w = rng.integers(0, 256, size=(r * (n // 256), 144), dtype=np.uint8)
        w[:, 0:2] = rng.uniform(2e-4, 4e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        w[:, 2:4] = rng.uniform(1e-4, 2e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return w.reshape(-1)

    w0, w2 = mat(DIM, A_ENC * A_DOWN), mat(DIM, DIM)
    enc = rng.standard_normal((A_RING, A_ENC)).astype(np.float32)
    aemb = np.zeros((A_RING, DIM), np.float32)
    groups = 0
    t0 = time.perf_counter()
    while groups < 1 or (time.perf_counter() - t0 < target_seconds and groups < 4096):
        oracle.adapter_commit(enc, aemb, groups, 1, 12, w0, 12, w2, n_threads=threads)
        groups += 1
    secs = time.perf_counter() - t0
    return {"value": groups / secs, "unit": "audio embeddings/s", "cores": threads, "kind": "port",
            "sample": f"{groups} adapter groups (4 x 1280 -> 3072 -> 3072, Q4_K) of the oracle's "
                      f"restatement of ggml's CPU path, {threads} threads, {secs:.1f} s"}


def cpu_encoder_leg(P, target_seconds):
    """The oracle on one encoder execution of P new frames: the conv stem
    (C, one thread) over the frames' Mel window, then per layer the seven
    products (ggml's generic CPU q4_K/q6_K x q8_K mul_mat restated, threaded
    over rows) and the window attention of the P queries over the 750-frame
    window (the oracle's fp64 window attention, one thread); a chunk's time =
    conv + 32 x layer (sampled on one layer)."""
    import numpy as np

    import oracle

    threads = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(SEED)

    def mat(dt, r, k):
        w = rng.integers(0, 256, size=(r * (k // 256), KQ_BLOCK[dt]), dtype=np.uint8)
        if dt == 12:
            w[:, 0:2] = rng.uniform(2e-4, 4e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
            w[:, 2:4] = rng.uniform(1e-4, 2e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        else:
            w[:, 208:210] = rng.uniform(1e-5, 2e-4, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return w.reshape(-1)

    mats = [(dt, r, k, mat(dt, r, k)) for _, dt, r, k in ENC_MATS]
    xs = {k: rng.standard_normal((P, k)).astype(np.float32) for k in (1280, E_DIM, E_HID)}
    conv_len = 2 * P + 4
    mel = rng.standard_normal((128, conv_len)).astype(np.float32)
    w0 = (rng.standard_normal((1280, 128, 3)) * 0.05).astype(np.float16).view(np.uint16)
    w1 = (rng.standard_normal((1280, 1280, 3)) * 0.02).astype(np.float16).view(np.uint16)
    b0 = np.zeros(1280, np.float32)
    row_b = E_DIM * 2
    kimg = (rng.standard_normal(E_CAP * E_DIM) * 0.5).astype(np.float16).view(np.uint8)
    vimg = (rng.standard_normal(E_CAP * E_DIM) * 0.5).astype(np.float16).view(np.uint8)
    q0 = 768
    key_pos = np.arange(q0 + P - E_WIN, q0 + P)
    q = rng.standard_normal((P, E_HEADS, E_HD)).astype(np.float32)
    t_conv = t_proj = t_attn = 0.0
    reps = 0
    t0 = time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < target_seconds and reps < 10):
        a = time.perf_counter()
        oracle.conv_stem(mel, 2, P, w0, b0, w1, b0)
        b = time.perf_counter()
        for dt, r, k, w in mats:
            for c in range(P):
                oracle.matvec(dt, w, r, k, xs[k][c], n_threads=threads)
        c_ = time.perf_counter()
        oracle.window_attn_f64(1, kimg, vimg, row_b, (key_pos % E_CAP).astype(np.int32), key_pos, q,
                               np.arange(q0, q0 + P), E_HEADS, E_HEADS, E_HD, E_WIN, 0.125)
        d = time.perf_counter()
        t_conv += b - a
        t_proj += c_ - b
        t_attn += d - c_
        reps += 1
    chunk_s = (t_conv + E_LAYERS * (t_proj + t_attn)) / reps
    return {"value": P / chunk_s, "unit": "frames/s", "cores": threads, "kind": "port",
            "sample": f"{reps} x (conv stem over {P} frames + one layer's 7 projections over {P} "
                      f"rows + its window-750 attention of {P} queries) of the oracle, projections "
                      f"on {threads} threads; chunk = conv + 32 x layer"}


def cpu_realtime_leg(target_seconds):
    """One realtime step on the oracle: the encoder over 4 frames, one adapter
    group and one decoder token, each sampled as in its own workload; a step's
    time is their sum."""
    enc = cpu_encoder_leg(R_FRAMES, target_seconds / 3)
    ad = cpu_adapter_leg(1, target_seconds / 6)
    tok = cpu_token_leg(target_seconds / 2)
    step_s = R_FRAMES / enc["value"] + 1.0 / ad["value"] + 1.0 / tok["value"]
    return {"value": 1.0 / step_s, "unit": "steps/s", "cores": tok["cores"], "kind": "port",
            "sample": f"encoder: {enc['sample']}; adapter: {ad['sample']}; decoder token: "
                      f"{tok['sample']}; step = sum"}


def realtime_tensor_list():
    """(name, ggml type, ne) of the realtime model in the Q4_K_M mix
    (src/voxtral.cpp:1193-1265 names, src/voxtral-quantize.cpp:148-159 types)"""
    q4, q6 = 12, 14
    T = [("enc.conv0.weight", 1, [3, 128, 1280]), ("enc.conv0.bias", 0, [1280]),
         ("enc.conv1.weight", 1, [3, 1280, 1280]), ("enc.conv1.bias", 0, [1280])]
    for i in range(E_LAYERS):
        p = f"enc.blk.{i}."
        T += [(p + "attn_norm.weight", 0, [1280]), (p + "attn_q.weight", q4, [1280, 2048]),
              (p + "attn_q.bias", 0, [2048]), (p + "attn_k.weight", q4, [1280, 2048]),
              (p + "attn_v.weight", q6, [1280, 2048]), (p + "attn_v.bias", 0, [2048]),
              (p + "attn_o.weight", q4, [2048, 1280]), (p + "attn_o.bias", 0, [1280]),
              (p + "ffn_norm.weight", 0, [1280]), (p + "ffn_w1.weight", q4, [1280, 5120]),
              (p + "ffn_w2.weight", q6, [5120, 1280]), (p + "ffn_w2.bias", 0, [1280]),
              (p + "ffn_w3.weight", q4, [1280, 5120])]
    T += [("enc.norm.weight", 0, [1280]), ("adapter.0.weight", q4, [5120, DIM]),
          ("adapter.2.weight", q4, [DIM, DIM]), ("tok_embeddings.weight", q6, [DIM, VOCAB]),
          ("norm.weight", 0, [DIM])]
    for i in range(LAYERS):
        p = f"dec.blk.{i}."
        T += [(p + "attn_norm.weight", 0, [DIM]), (p + "attn_q.weight", q4, [DIM, Q_DIM]),
              (p + "attn_k.weight", q4, [DIM, KV_DIM]), (p + "attn_v.weight", q6, [DIM, KV_DIM]),
              (p + "attn_o.weight", q4, [Q_DIM, DIM]), (p + "ffn_norm.weight", 0, [DIM]),
              (p + "ffn_w1.weight", q4, [DIM, HIDDEN]), (p + "ffn_w2.weight", q6, [HIDDEN, DIM]),
              (p + "ffn_w3.weight", q4, [DIM, HIDDEN]), (p + "ada0.weight", q4, [DIM, 32]),
              (p + "ada2.weight", 1, [32, DIM])]
    T.append(("audio.mel_filters", 0, [201, 128]))
    return T


def write_synthetic_gguf(path):
    """the realtime model's GGUF layout with random bytes, streamed (GGUF v3,
    32-byte alignment); returns the data-section bytes"""
    import struct

    import numpy as np

    blk = {0: (1, 4), 1: (1, 2), 12: (256, 144), 14: (256, 210)}
    T = realtime_tensor_list()

    def sz(t, ne):
        n = 1
        for d in ne:
            n *= d
        return n // blk[t][0] * blk[t][1]

    def s(b):
        return struct.pack("<Q", len(b)) + b

    kvs = [(b"general.architecture", 8, s(b"voxtral_realtime")),
           (b"voxtral.vocab_size", 5, struct.pack("<i", VOCAB))]
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(T), len(kvs)))
    for k, t, v in kvs:
        head += s(k) + struct.pack("<I", t) + v
    off, offs = 0, []
    for name, t, ne in T:
        offs.append(off)
        off += (sz(t, ne) + 31) // 32 * 32
    for (name, t, ne), o in zip(T, offs):
        head += s(name.encode()) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", t, o)
    head += b"\0" * ((-len(head)) % 32)
    pool = np.random.default_rng(SEED).integers(0, 256, 64 << 20, dtype=np.uint8).tobytes()
    with open(path, "wb") as f:
        f.write(head)
        written = 0
        while written < off:
            n = min(len(pool), off - written)
            f.write(pool[:n])
            written += n
    return off


def gpu_model_load(steps, warmup):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    tmp = os.environ.get("TMPDIR", "/tmp")
    path = os.path.join(tmp, f"vkv_bench_realtime_q4km_{os.getpid()}.gguf")
    try:
        data_bytes = write_synthetic_gguf(path)
        torch.cuda.synchronize()
        for _ in range(warmup):
            vkv.Model(path, hip_stream=st.cuda_stream).close()
        times = []
        t0 = time.perf_counter()
        for _ in range(steps):
            a = time.perf_counter()
            m = vkv.Model(path, hip_stream=st.cuda_stream)
            times.append(time.perf_counter() - a)
            m.close()
        wall = time.perf_counter() - t0
    finally:
        if os.path.exists(path):
            os.remove(path)
    return sum(times) * 1e3, [t * 1e3 for t in times], wall, data_bytes


def cpu_load_leg(target_seconds):
    """The reference's weight upload on the CPU backend (src/voxtral.cpp:
    1160-1190): per tensor, seek + read into a staging vector + copy into the
    weight buffer, on a bounded prefix of the same synthetic file."""
    import numpy as np

    tmp = os.environ.get("TMPDIR", "/tmp")
    path = os.path.join(tmp, f"vkv_bench_cpu_load_{os.getpid()}.gguf")
    try:
        write_synthetic_gguf(path)
        import struct
        T = realtime_tensor_list()
        blk = {0: (1, 4), 1: (1, 2), 12: (256, 144), 14: (256, 210)}
        sizes = []
        for name, t, ne in T:
            n = 1
            for d in ne:
                n *= d
            sizes.append(n // blk[t][0] * blk[t][1])
        with open(path, "rb") as f:
            head = f.read(1 << 20)
        # data offset: end of the tensor infos, aligned (the writer pads to 32)
        pos = 24
        for _ in range(2):
            n = struct.unpack_from("<Q", head, pos)[0]
            pos += 8 + n
            t = struct.unpack_from("<I", head, pos)[0]
            pos += 4
            pos += 8 + struct.unpack_from("<Q", head, pos)[0] if t == 8 else 4
        offs = []
        for _ in T:
            n = struct.unpack_from("<Q", head, pos)[0]
            pos += 8 + n
            nd = struct.unpack_from("<I", head, pos)[0]
            pos += 4 + 8 * nd + 4
            offs.append(struct.unpack_from("<Q", head, pos)[0])
            pos += 8
        data0 = (pos + 31) // 32 * 32
        weights = np.empty(sum(sizes), np.uint8)
        moved, dst = 0, 0
        t0 = time.perf_counter()
        with open(path, "rb", buffering=0) as f:
            for o, n in zip(offs, sizes):
                f.seek(data0 + o)
                tmpv = bytearray(n)
                f.readinto(tmpv)
                weights[dst:dst + n] = np.frombuffer(tmpv, np.uint8)
                dst += n
                moved += n
                if time.perf_counter() - t0 > target_seconds:
                    break
        secs = time.perf_counter() - t0
    finally:
        if os.path.exists(path):
            os.remove(path)
    return {"value": moved / secs / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{moved / 1e9:.2f} GB of the same file (page cache) read tensor by tensor "
                      f"into a staging buffer and copied into host weight memory, as the "
                      f"reference's CPU-backend load does, 1 thread, {secs:.1f} s"}


def encoder_chunk_bytes(n_keys, P=E_CHUNK):
    """conv stem weights (f16) + 32 layers' weights + the window attention's
    bytes for one chunk"""
    conv = 2 * 1280 * 3 * (128 + 1280)
    w = E_LAYERS * sum(mat_bytes(dt, r, n) for _, dt, r, n in ENC_MATS)
    return conv + w + encoder_bytes_per_chunk(n_keys, P)


def encoder_setup(gen, sp):
    """Random Q4_K_M encoder weights on the device, their vkv_enc_model, and an
    encoder cache whose ring holds frames [0, 768) (the steady state); returns
    (model, cache, keep)."""
    import torch
    import vkv

    keep = []
    layers = (vkv.EncLayer * E_LAYERS)()

    def vec(n, lo, hi):
        t = torch.empty(n, device="cuda").uniform_(lo, hi, generator=gen)
        keep.append(t)
        return t.data_ptr()

    for l in range(E_LAYERS):
        w = {name: random_kq_device(dt, r, n, gen) for name, dt, r, n in ENC_MATS}
        keep.extend(w.values())
        layers[l] = vkv.EncLayer(vec(1280, 0.5, 1.5), vec(1280, -0.1, 0.1), w["attn_q"].data_ptr(),
                                 w["attn_k"].data_ptr(), w["attn_v"].data_ptr(),
                                 w["attn_o"].data_ptr(), 12, 12, 14, 12, vec(E_DIM, -0.1, 0.1),
                                 vec(E_DIM, -0.1, 0.1), vec(1280, -0.1, 0.1), vec(1280, 0.5, 1.5),
                                 vec(1280, -0.1, 0.1), w["ffn_w1"].data_ptr(),
                                 w["ffn_w2"].data_ptr(), w["ffn_w3"].data_ptr(), 12, 14, 12,
                                 vec(1280, -0.1, 0.1))
    model = vkv.EncModel(E_LAYERS, 1280, E_HID, E_HEADS, E_HD, 1e-5, 1.0e6, vec(1280, 0.5, 1.5),
                         vec(1280, -0.1, 0.1), layers)
    cache = vkv.Cache(n_streams=1, n_layers=E_LAYERS, capacity=E_CAP, n_kv_heads=E_HEADS,
                      head_dim=E_HD, n_q_heads=E_HEADS, dtype=vkv.F16)
    # steady state: the ring holds frames [0, 768) before the first timed chunk
    first = (E_WIN + E_CHUNK - 1) // E_CHUNK + 1
    for c in range(first):
        plan = vkv.enc_plan(c * E_CHUNK, E_CHUNK, E_CAP, E_WIN)
        k = torch.empty(E_LAYERS, E_CHUNK, E_DIM, device="cuda")
        v = torch.empty(E_LAYERS, E_CHUNK, E_DIM, device="cuda")
        vkv.synth_rows(k.data_ptr(), E_DIM, SEED, vkv.TAG_EK, nl=E_LAYERS, p0=c * E_CHUNK,
                       np_=E_CHUNK, hip_stream=sp)
        vkv.synth_rows(v.data_ptr(), E_DIM, SEED, vkv.TAG_EV, nl=E_LAYERS, p0=c * E_CHUNK,
                       np_=E_CHUNK, hip_stream=sp)
        cache.append(0, 0, E_LAYERS, vkv.plan_segs(plan.write_seg, plan.write_nseg), k.data_ptr(),
                     v.data_ptr(), hip_stream=sp)
    torch.cuda.synchronize()
    return model, cache, (keep, layers)


def gpu_encoder_chunk(steps, warmup):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    model, cache, keep = encoder_setup(gen, sp)
    first = (E_WIN + E_CHUNK - 1) // E_CHUNK + 1
    T = warmup + steps
    plans = [vkv.enc_plan((first + i) * E_CHUNK, E_CHUNK, E_CAP, E_WIN) for i in range(T)]
    # the conv stem's f16 weights and each chunk's Mel window [128][2 * 16 + 4]
    w0 = (torch.randn(1280, 128, 3, device="cuda", generator=gen) * 0.05).half()
    w1 = (torch.randn(1280, 1280, 3, device="cuda", generator=gen) * 0.02).half()
    b0 = torch.randn(1280, device="cuda", generator=gen) * 0.1
    b1 = torch.randn(1280, device="cuda", generator=gen) * 0.1
    conv_len = plans[0].conv_mel_end - plans[0].conv_mel_start
    mel = torch.randn(T, 128, conv_len, device="cuda", generator=gen)
    x = torch.empty(E_CHUNK, 1280, device="cuda")
    ws_bytes = vkv.encoder_chunk_workspace(model, E_CHUNK)
    ws = torch.empty(ws_bytes // 4 + 64, device="cuda")
    ws_ptr = (ws.data_ptr() + 255) & ~255
    cb = vkv.enc_conv_stem_workspace(conv_len, 128, 1280, E_CHUNK)
    cws = torch.empty(cb // 4 + 64, device="cuda")
    cws_ptr = (cws.data_ptr() + 255) & ~255

    def step(i):
        vkv.enc_conv_stem(mel[i].data_ptr(), 128, plans[i], w0.data_ptr(), b0.data_ptr(),
                          w1.data_ptr(), b1.data_ptr(), 1280, x.data_ptr(), cws_ptr, cb,
                          hip_stream=sp)
        vkv.encoder_chunk(cache, 0, plans[i], E_WIN, model, x.data_ptr(), ws_ptr, ws_bytes,
                          hip_stream=sp)

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    assert bool(torch.isfinite(x).all())
    n_keys = plans[0].win_end - plans[0].win_start
    cache.close()
    del keep
    return total_ms, step_ms, wall, n_keys


R_FRAMES = 4   # encoder frames per realtime step (the steady physical 4-row launch)


def gpu_realtime_step(steps, warmup, pipelined=False):
    """One 80 ms realtime step: the conv stem and the encoder over 4 new frames
    into the encoder-output ring, the adapter over the completed group into
    the audio-embedding ring, and one decoder token reading that row
    (26 layers, the full 8192-slot ring).

    pipelined: the same work on two HIP streams, the decoder one group
    behind: step i's encoder + adapter (group g_i) run on the timing stream
    while step i's decoder token, on a second stream, reads group g_{i-1}
    (it waits for step i-1's adapter through an event); the timing stream
    waits for token i-1 before step i+1's encoder, so at most one step of
    each chain is in flight beside the other, and the last step joins the
    decoder stream before the end event."""
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    dst = torch.cuda.Stream() if pipelined else st   # default priority
    dsp = dst.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    emodel, ecache, ekeep = encoder_setup(gen, sp)
    dmodel, dkeep = device_model(gen)
    dcache = vkv.Cache(n_streams=1, n_layers=LAYERS, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                       n_q_heads=QH, dtype=vkv.F16, **CACHE_KW)
    ring = vkv.new_ring(CAP)
    plan = vkv.decoder_plan(ring, 0, CAP)
    k0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    v0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    vkv.synth_rows(k0.data_ptr(), KV_DIM, SEED, vkv.TAG_K, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    vkv.synth_rows(v0.data_ptr(), KV_DIM, SEED, vkv.TAG_V, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    dcache.append(0, 0, LAYERS, vkv.plan_segs(plan.write_seg, plan.write_nseg), k0.data_ptr(),
                  v0.data_ptr(), hip_stream=sp)
    vkv.decoder_commit(ring, plan)
    torch.cuda.synchronize()
    del k0, v0
    ad_w0 = random_kq_device(12, DIM, 1280 * A_DOWN, gen)
    ad_w2 = random_kq_device(12, DIM, DIM, gen)
    ad = vkv.Adapter(ad_w0.data_ptr(), ad_w2.data_ptr(), 12, 12, 1280, DIM, A_DOWN)
    enc_out = torch.zeros(A_RING, 1280, device="cuda")
    aemb = torch.zeros(A_RING, DIM, device="cuda")
    er = vkv.RowRing(enc_out.data_ptr(), A_RING, 1280)
    ar = vkv.RowRing(aemb.data_ptr(), A_RING, DIM)
    q0 = ((E_WIN + E_CHUNK - 1) // E_CHUNK + 1) * E_CHUNK   # frames the ring already holds
    T = warmup + steps
    plans = [vkv.enc_plan(q0 + R_FRAMES * i, R_FRAMES, E_CAP, E_WIN) for i in range(T)]
    conv_len = plans[0].conv_mel_end - plans[0].conv_mel_start
    w0 = (torch.randn(1280, 128, 3, device="cuda", generator=gen) * 0.05).half()
    w1 = (torch.randn(1280, 1280, 3, device="cuda", generator=gen) * 0.02).half()
    b0 = torch.randn(1280, device="cuda", generator=gen) * 0.1
    b1 = torch.randn(1280, device="cuda", generator=gen) * 0.1
    mel = torch.randn(T, 128, conv_len, device="cuda", generator=gen)
    x = torch.empty(R_FRAMES, 1280, device="cuda")
    ewb = vkv.encoder_chunk_workspace(emodel, R_FRAMES)
    ews = torch.empty(ewb // 4 + 64, device="cuda")
    cb = vkv.enc_conv_stem_workspace(conv_len, 128, 1280, R_FRAMES)
    cws = torch.empty(cb // 4 + 64, device="cuda")
    awb = vkv.adapter_workspace(ad, 1)
    aws = torch.empty(awb // 4 + 64, device="cuda")
    twb = vkv.decoder_token_workspace(dmodel)
    tws = torch.empty(twb // 4 + 64, device="cuda")
    logits = torch.empty(VOCAB, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    al = lambda t: (t.data_ptr() + 255) & ~255
    ev_a = [torch.cuda.Event() for _ in range(T)]   # step i's adapter row is written
    ev_d = [torch.cuda.Event() for _ in range(T)]   # step i's token is done

    def step(i):
        p = plans[i]
        if pipelined and i > 0:
            st.wait_event(ev_d[i - 1])
        vkv.enc_conv_stem(mel[i].data_ptr(), 128, p, w0.data_ptr(), b0.data_ptr(), w1.data_ptr(),
                          b1.data_ptr(), 1280, x.data_ptr(), al(cws), cb, hip_stream=sp)
        vkv.encoder_chunk_ring(ecache, 0, p, E_WIN, emodel, x.data_ptr(), er, al(ews), ewb,
                               hip_stream=sp)
        g = (p.q_start + R_FRAMES) // A_DOWN - 1          # the group these frames complete
        vkv.adapter_commit(ad, er, ar, g, 1, al(aws), awb, hip_stream=sp)
        if not pipelined:
            vkv.decoder_token(dcache, 0, ring, dmodel, 32, aemb[g % A_RING].data_ptr(),
                              logits.data_ptr(), tok.data_ptr(), al(tws), twb, hip_stream=sp)
            return
        ev_a[i].record(st)
        if i > 0:
            dst.wait_event(ev_a[i - 1])
        gd = g - 1                                         # the previous step's group
        vkv.decoder_token(dcache, 0, ring, dmodel, 32, aemb[gd % A_RING].data_ptr(),
                          logits.data_ptr(), tok.data_ptr(), al(tws), twb, hip_stream=dsp)
        ev_d[i].record(dst)
        if i == T - 1:
            st.wait_event(ev_d[i])                         # join before the end event

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    assert bool(torch.isfinite(logits).all()) and bool(torch.isfinite(aemb).all())
    n_keys = plans[0].win_end - plans[0].win_start
    ecache.close()
    dcache.close()
    del ekeep, dkeep
    return total_ms, step_ms, wall, n_keys


def device_model(gen):
    """Random decoder weights of the MIX file kind on the device and the
    vkv_dec_model describing them (tied output = tok_embeddings)."""
    import torch
    import vkv
    keep = []
    layers = (vkv.DecLayer * LAYERS)()
    mats = layer_mats()
    T = {name: dt for name, dt, _, _ in mats}
    for l in range(LAYERS):
        w = {name: random_kq_device(dt, r, n, gen) for name, dt, r, n in mats}
        norms = torch.empty(2, DIM, device="cuda").uniform_(0.5, 1.5, generator=gen)
        ada = torch.empty(DIM, device="cuda").uniform_(-0.3, 0.3, generator=gen)
        keep += list(w.values()) + [norms, ada]
        layers[l] = vkv.DecLayer(norms[0].data_ptr(), w["attn_q"].data_ptr(), w["attn_k"].data_ptr(),
                                 w["attn_v"].data_ptr(), w["attn_o"].data_ptr(), T["attn_q"],
                                 T["attn_k"], T["attn_v"], T["attn_o"], norms[1].data_ptr(),
                                 ada.data_ptr(), w["ffn_w1"].data_ptr(), w["ffn_w2"].data_ptr(),
                                 w["ffn_w3"].data_ptr(), T["ffn_w1"], T["ffn_w2"], T["ffn_w3"])
    table = random_kq_device(out_type(), VOCAB, DIM, gen)
    out_norm = torch.empty(DIM, device="cuda").uniform_(0.5, 1.5, generator=gen)
    keep += [table, out_norm]
    model = vkv.DecModel(LAYERS, DIM, HIDDEN, QH, KVH, HD, VOCAB, 1e-5, 1.0e6, table.data_ptr(),
                         out_type(), out_norm.data_ptr(), table.data_ptr(), out_type(), layers)
    return model, (keep, layers)


def gpu_token(steps, warmup):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    model, keep = device_model(gen)
    cache = vkv.Cache(n_streams=1, n_layers=LAYERS, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=vkv.F16, **CACHE_KW)
    ring = vkv.new_ring(CAP)
    plan = vkv.decoder_plan(ring, 0, CAP)
    k0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    v0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    vkv.synth_rows(k0.data_ptr(), KV_DIM, SEED, vkv.TAG_K, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    vkv.synth_rows(v0.data_ptr(), KV_DIM, SEED, vkv.TAG_V, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    cache.append(0, 0, LAYERS, vkv.plan_segs(plan.write_seg, plan.write_nseg), k0.data_ptr(),
                 v0.data_ptr(), hip_stream=sp)
    vkv.decoder_commit(ring, plan)
    torch.cuda.synchronize()
    del k0, v0
    audio = torch.randn(warmup + steps, DIM, device="cuda", generator=gen) * 0.1
    logits = torch.empty(VOCAB, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_bytes = vkv.decoder_token_workspace(model)
    ws = torch.empty(ws_bytes // 4 + 64, device="cuda")
    ws_ptr = (ws.data_ptr() + 255) & ~255
    tokens = torch.randint(0, VOCAB, (warmup + steps,), generator=torch.Generator().manual_seed(1))

    def step(i):
        vkv.decoder_token(cache, 0, ring, model, int(tokens[i]), audio[i].data_ptr(),
                          logits.data_ptr(), tok.data_ptr(), ws_ptr, ws_bytes, hip_stream=sp)

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    assert bool(torch.isfinite(logits).all())
    assert ring.next_absolute_position == CAP + warmup + len(REP_MS) * steps
    cache.close()
    del keep
    return total_ms, step_ms, wall


LOOP_LAT_MS = []   # per-token latencies of the last gpu_token_loop run (ms)


def gpu_token_loop(steps, warmup):
    """The production token loop of run_decoder_step (src/voxtral.cpp:5219-5360:
    compute :5271, one synchronize :5273, the 4-byte token readback :5341):
    per token vkv_decoder_token on the stream, the token's 4 bytes copied to
    pinned host memory on the same stream, one hipStreamSynchronize, and the
    token fed to the next step (the greedy loop).  Every token's latency is
    the host's wall clock from the call to the synchronize's return; the
    repetitions are the K timed tokens, run once."""
    import ctypes

    import torch
    import vkv

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    hip.hipHostFree.argtypes = [ctypes.c_void_p]
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                   ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    model, keep = device_model(gen)
    cache = vkv.Cache(n_streams=1, n_layers=LAYERS, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=vkv.F16, **CACHE_KW)
    ring = vkv.new_ring(CAP)
    plan = vkv.decoder_plan(ring, 0, CAP)
    k0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    v0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    vkv.synth_rows(k0.data_ptr(), KV_DIM, SEED, vkv.TAG_K, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    vkv.synth_rows(v0.data_ptr(), KV_DIM, SEED, vkv.TAG_V, nl=LAYERS, p0=0, np_=CAP, hip_stream=sp)
    cache.append(0, 0, LAYERS, vkv.plan_segs(plan.write_seg, plan.write_nseg), k0.data_ptr(),
                 v0.data_ptr(), hip_stream=sp)
    vkv.decoder_commit(ring, plan)
    torch.cuda.synchronize()
    del k0, v0
    audio = torch.randn(warmup + steps, DIM, device="cuda", generator=gen) * 0.1
    logits = torch.empty(VOCAB, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_bytes = vkv.decoder_token_workspace(model)
    ws = torch.empty(ws_bytes // 4 + 64, device="cuda")
    ws_ptr = (ws.data_ptr() + 255) & ~255
    host = ctypes.c_void_p()
    if hip.hipHostMalloc(ctypes.byref(host), 64, 0) != 0:
        raise RuntimeError("hipHostMalloc failed")
    host_tok = ctypes.cast(host, ctypes.POINTER(ctypes.c_int32))

    def token(i, t):
        vkv.decoder_token(cache, 0, ring, model, t, audio[i].data_ptr(), logits.data_ptr(),
                          tok.data_ptr(), ws_ptr, ws_bytes, hip_stream=sp)
        if hip.hipMemcpyAsync(host, tok.data_ptr(), 4, 2, sp) != 0:   # device to host
            raise RuntimeError("hipMemcpyAsync failed")
        if hip.hipStreamSynchronize(sp) != 0:
            raise RuntimeError("hipStreamSynchronize failed")
        return int(host_tok[0])

    t = 1
    for i in range(warmup):
        t = token(i, t)
    lat = []
    wall0 = time.perf_counter()
    for i in range(steps):
        t0 = time.perf_counter()
        t = token(warmup + i, t)
        lat.append((time.perf_counter() - t0) * 1e3)
    wall = time.perf_counter() - wall0
    assert 0 <= t < VOCAB and bool(torch.isfinite(logits).all())
    assert ring.next_absolute_position == CAP + warmup + steps
    hip.hipHostFree(host)
    cache.close()
    del keep
    LOOP_LAT_MS[:] = lat
    REP_MS[:] = [sum(lat)]
    return sum(lat), lat, wall


P_TOKENS, P_AUDIO_CAP = 38, 256


def gpu_prompt(steps, warmup):
    """The decoder prefill of a 38-token prompt at the stream start, each
    token plus its audio row from a 256-row ring; the ring is cleared before
    every step (host bookkeeping only: the prompt rewrites slots 0..37 before
    any read)."""
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    model, keep = device_model(gen)
    cache = vkv.Cache(n_streams=1, n_layers=LAYERS, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=vkv.F16, **CACHE_KW)
    ring = vkv.new_ring(CAP)
    aemb = torch.randn(P_AUDIO_CAP, DIM, device="cuda", generator=gen) * 0.1
    aring = vkv.RowRing(aemb.data_ptr(), P_AUDIO_CAP, DIM)
    logits = torch.empty(VOCAB, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_bytes = vkv.decoder_prompt_workspace(model, P_TOKENS)
    ws = torch.empty(ws_bytes // 4 + 64, device="cuda")
    ws_ptr = (ws.data_ptr() + 255) & ~255
    g = torch.Generator().manual_seed(1)
    prompts = [[int(t) for t in torch.randint(0, VOCAB, (P_TOKENS,), generator=g)]
               for _ in range(warmup + steps)]

    def step(i):
        vkv.decoder_clear(ring, CAP)
        vkv.decoder_prompt(cache, 0, ring, model, prompts[i], aring, logits.data_ptr(),
                           tok.data_ptr(), ws_ptr, ws_bytes, hip_stream=sp)

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    assert bool(torch.isfinite(logits).all())
    assert ring.next_absolute_position == P_TOKENS
    cache.close()
    del keep
    return total_ms, step_ms, wall


def prompt_bytes(n=P_TOKENS):
    """The weights once (26 layers + the logits matrix), the token rows of the
    Q6_K table and the audio rows read, the K/V rows appended (f16); the
    activations between launches (n rows of at most 9216 floats) are not
    counted."""
    return (weights_bytes_per_token() + n * (DIM // 256 * 210 + DIM * 4) +
            LAYERS * n * 2 * KV_DIM * 2)


def cpu_prompt_leg(target_seconds, n=P_TOKENS):
    """The oracle's restatement of ggml's CPU mul_mat (one Q8_K vec_dot per
    (row, column)) on one layer's seven matrices over n input columns, and the
    logits of the last token; a prompt's time = 26 x layer + logits (the
    attention over at most 38 keys is left out: under 0.1% of the work)."""
    import numpy as np

    import oracle

    threads = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(SEED)

    def mat(dt, r, k):
        w = rng.integers(0, 256, size=(r * (k // 256), KQ_BLOCK[dt]), dtype=np.uint8)
        if dt == 12:
            w[:, 0:2] = rng.uniform(2e-4, 4e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
            w[:, 2:4] = rng.uniform(1e-4, 2e-3, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        else:
            w[:, 208:210] = rng.uniform(1e-5, 2e-4, len(w)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return w.reshape(-1)

    mats = [(dt, r, k, mat(dt, r, k)) for _, dt, r, k in LAYER_MATS]
    lw = mat(14, VOCAB, DIM)
    xs = {k: rng.standard_normal((n, k)).astype(np.float32) for k in (DIM, Q_DIM, HIDDEN)}
    t_layer = t_logits = 0.0
    reps = 0
    t0 = time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < target_seconds and reps < 10):
        a = time.perf_counter()
        for dt, r, k, w in mats:
            for c in range(n):
                oracle.matvec(dt, w, r, k, xs[k][c], n_threads=threads)
        b = time.perf_counter()
        oracle.matvec(14, lw, VOCAB, DIM, xs[DIM][n - 1], n_threads=threads)
        c_ = time.perf_counter()
        t_layer += b - a
        t_logits += c_ - b
        reps += 1
    prompt_s = (LAYERS * t_layer + t_logits) / reps
    return {"value": n / prompt_s, "unit": "prompt tokens/s", "cores": threads, "kind": "port",
            "sample": f"{reps} x (one layer's 7 projections over {n} columns + the 131072-row "
                      f"logits of one) of the oracle's restatement of ggml's generic CPU "
                      f"q4_K/q6_K x q8_K mul_mat, {threads} threads; prompt = 26 x layer + logits"}


def token_bytes():
    """Weights + the KV window read (26 layers x 8192 x 2 x 1024 f16) + the
    appended rows and the per-layer activations (small)."""
    return weights_bytes_per_token() + decode_bytes_per_stream_token(CAP, 1)


def cpu_token_leg(target_seconds):
    """The oracle's CPU restatement of a token: 26 x (one layer's projections +
    the attention step of one layer) + logits, from timed samples of each."""
    w = cpu_weights_leg(target_seconds / 2)
    a = cpu_leg(1, target_seconds / 2)
    t_proj = 1.0 / w["value"]           # 26 layers' projections + logits
    t_attn = 1.0 / a["value"]           # 26 layers' append + attention
    return {"value": 1.0 / (t_proj + t_attn), "unit": "tokens/s", "cores": w["cores"],
            "kind": "port",
            "sample": f"projections: {w['sample']}; attention: {a['sample']}; token = sum"}


def cpu_weights_leg(target_seconds):
    """The oracle's restatement of ggml's CPU matvec (Q8_K input, generic
    per-block integer dots), threaded over rows, on one layer's seven matrices
    and the logits matrix; a token's time = 26 x layer + logits."""
    import numpy as np

    import oracle

    threads = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(SEED)
    mats = [(dt, r, n, random_blocks_np(rng, dt, r, n)) for _, dt, r, n in layer_mats()]
    lw = random_blocks_np(rng, out_type(), VOCAB, DIM)
    xs = {n: rng.standard_normal(n).astype(np.float32) for n in (DIM, Q_DIM, HIDDEN)}
    t_layer = t_logits = 0.0
    reps = 0
    t0 = time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < target_seconds and reps < 20):
        a = time.perf_counter()
        for dt, r, n, w in mats:
            oracle.matvec(dt, w, r, n, xs[n], n_threads=threads)
        b = time.perf_counter()
        oracle.matvec(14, lw, VOCAB, DIM, xs[DIM], n_threads=threads)
        c = time.perf_counter()
        t_layer += b - a
        t_logits += c - b
        reps += 1
    token_s = (LAYERS * t_layer + t_logits) / reps
    return {"value": 1.0 / token_s, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{reps} x (one layer's 7 projections + the 131072-row logits) of the "
                      f"oracle's restatement of ggml's CPU "
                      f"{'q4_K/q6_K x q8_K' if MIX == 'q4km' else 'q8_0 x q8_0'} matvec, "
                      f"{threads} threads; token = 26 x layer + logits"}


def elem_bytes(dtype):
    return 2.0 if dtype == 1 else 34.0 / 32.0


def decode_bytes_per_stream_token(n_valid, dtype):
    """Per layer: K+V read of the window, new K/V f32 read, appended row write,
    Q read, output write -- times the layer count."""
    e = elem_bytes(dtype)
    per_layer = (n_valid * 2 * KV_DIM * e + 2 * KV_DIM * 4 + 2 * KV_DIM * e + Q_DIM * 4 +
                 Q_DIM * 4)
    return int(LAYERS * per_layer)


def encoder_bytes_per_chunk(n_keys, P=E_CHUNK, e=2):
    """Per layer: K+V read of the window keys, new K/V f32 read, appended rows
    write (e bytes per element: f16 2, f32 4), Q read, output write -- times
    the layer count."""
    per_layer = (n_keys * 2 * E_DIM * e + P * E_DIM * 4 * 2 + P * E_DIM * e * 2 + P * E_DIM * 4 +
                 P * E_DIM * 4)
    return E_LAYERS * per_layer


REPS = 5            # timed repetitions of the K steps; the median is reported
REPS_SET = [REPS]   # the run's repetitions (--reps)
REP_MS = []         # the last timed_loop's per-repetition totals (ms)


SPIN_CYCLES = 500_000   # GPU clock cycles of the pre-repetition spin (~0.2 ms)


def timed_loop(step, steps, warmup, st, every=8, reps=None):
    """W untimed steps, then `reps` repetitions of K timed steps, each between
    a synchronize and two events on the launch stream; returns the median
    repetition's total (ms), the per-group samples of every repetition and
    the wall time of all repetitions.  Each run of `every` consecutive timed
    steps is also bracketed by its own pair of events, and its duration /
    `every` is one sample of the step's GPU time: an event record costs the
    GPU a few microseconds, so bracketing single steps would add that to
    every sample (and events around every step would slow the timed region).
    A repetition replays the same step indices (their inputs); the state the
    steps advance (ring positions) keeps advancing.  Before each repetition's
    start event the stream gets a short spin (~0.2 ms, untimed) so the host
    has queued the first steps when the start event runs: the timed region
    then holds the K steps, not the host's latency in launching the first
    one after the synchronize (~1% of a 20-step region)."""
    import torch
    reps = REPS_SET[0] if reps is None else reps
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    every = max(1, min(every, steps))
    groups = [g for g in range(0, steps - every + 1, every)]
    totals, step_ms = [], []
    wall0 = time.perf_counter()
    for _ in range(reps):
        ev = {g: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for g in groups}
        t_start = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            torch.cuda._sleep(SPIN_CYCLES)
        t_start.record(st)
        for i in range(steps):
            if i in ev:
                ev[i][0].record(st)
            step(warmup + i)
            if i - every + 1 in ev:
                ev[i - every + 1][1].record(st)
        t_end.record(st)
        torch.cuda.synchronize()
        totals.append(t_start.elapsed_time(t_end))
        step_ms += [ev[g][0].elapsed_time(ev[g][1]) / every for g in groups]
    wall = time.perf_counter() - wall0
    REP_MS[:] = totals
    return sorted(totals)[len(totals) // 2], step_ms, wall


CACHE_KW = {}   # cache parameters from the command line (kernel selection for A/B runs)


def gpu_decode(dtype, ns, steps, warmup, rope_theta=None, layerwise=False):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    cache = vkv.Cache(n_streams=ns, n_layers=LAYERS, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=dtype, **CACHE_KW)
    rings = (vkv.Ring * ns)(*[vkv.new_ring(CAP) for _ in range(ns)])
    # fill every ring: positions [0, 8192) through the planned append path
    k0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    v0 = torch.empty(LAYERS, CAP, KV_DIM, device="cuda")
    for s in range(ns):
        plan = vkv.decoder_plan(rings[s], 0, CAP)
        vkv.synth_rows(k0.data_ptr(), KV_DIM, SEED, vkv.TAG_K, s0=s, nl=LAYERS, p0=0, np_=CAP,
                       hip_stream=sp)
        vkv.synth_rows(v0.data_ptr(), KV_DIM, SEED, vkv.TAG_V, s0=s, nl=LAYERS, p0=0, np_=CAP,
                       hip_stream=sp)
        cache.append(s, 0, LAYERS, vkv.plan_segs(plan.write_seg, plan.write_nseg), k0.data_ptr(),
                     v0.data_ptr(), hip_stream=sp)
        vkv.decoder_commit(rings[s], plan)
    torch.cuda.synchronize()
    del k0, v0
    # resident per-step inputs, [step][stream][layer][...]
    T = warmup + steps
    q = torch.empty(T, ns, LAYERS, Q_DIM, device="cuda")
    k = torch.empty(T, ns, LAYERS, KV_DIM, device="cuda")
    v = torch.empty(T, ns, LAYERS, KV_DIM, device="cuda")
    for t, tag, n in ((q, vkv.TAG_Q, Q_DIM), (k, vkv.TAG_K, KV_DIM), (v, vkv.TAG_V, KV_DIM)):
        vkv.synth_rows(t.data_ptr(), n, SEED, tag, s0=0, ns=ns, s_stride=LAYERS, nl=LAYERS,
                       l_stride=1, p0=CAP, np_=T, p_stride=ns * LAYERS, hip_stream=sp)
    out = torch.empty(T, ns, LAYERS, Q_DIM, device="cuda")
    scale = 1.0 / (HD ** 0.5)
    pos = [CAP]

    # the decoder's call shape: one plan per token, one C call per layer
    # (arguments prepared outside the loop, so the host keeps ahead of the GPU)
    layer_step = vkv.lib.vkv_decoder_layer_step
    ptrs = [t.data_ptr() for t in (q, k, v, out)]
    strides = [LAYERS * Q_DIM * 4, LAYERS * KV_DIM * 4, LAYERS * KV_DIM * 4, LAYERS * Q_DIM * 4]
    lstr = [Q_DIM * 4, KV_DIM * 4, KV_DIM * 4, Q_DIM * 4]

    def step_layers(i):
        plan = vkv.decoder_plan(rings[0], pos[0], 1)
        pref = ctypes.byref(plan)
        b = [p + i * st_ for p, st_ in zip(ptrs, strides)]
        for layer in range(LAYERS):
            rc = layer_step(cache.handle, 0, pref, pos[0], layer, 1, b[0] + layer * lstr[0],
                            b[1] + layer * lstr[1], b[2] + layer * lstr[2], b[3] + layer * lstr[3],
                            QH, scale, rope_theta, sp)
            if rc:
                vkv.check(rc)
        vkv.decoder_commit(rings[0], plan)
        pos[0] += 1

    def step(i):
        if layerwise:
            step_layers(i)
            return
        if rope_theta is None:
            cache.decoder_step(0, rings, [pos[0]] * ns, 0, LAYERS, q[i].data_ptr(),
                               k[i].data_ptr(), v[i].data_ptr(), out[i].data_ptr(), scale,
                               hip_stream=sp)
        else:
            cache.decoder_step_rope(0, rings, [pos[0]] * ns, 0, LAYERS, q[i].data_ptr(),
                                    k[i].data_ptr(), v[i].data_ptr(), out[i].data_ptr(), scale,
                                    rope_theta, hip_stream=sp)
        pos[0] += 1

    total_ms, step_ms, wall = timed_loop(step, steps, warmup, st)
    for s in range(ns):
        assert rings[s].used == CAP and rings[s].next_absolute_position == CAP + warmup + \
            len(REP_MS) * steps
    assert bool(torch.isfinite(out).all())
    cache.close()
    return total_ms, step_ms, wall


def gpu_stream_from_empty(n_steps, layers, prefill):
    """Decode steps at positions [prefill, prefill + n_steps) over an 8192 ring
    holding positions [0, prefill) (no wrap); every step is timed."""
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    cache = vkv.Cache(n_streams=1, n_layers=layers, capacity=CAP, n_kv_heads=KVH, head_dim=HD,
                      n_q_heads=QH, dtype=vkv.F16)
    rings = (vkv.Ring * 1)(vkv.new_ring(CAP))
    if prefill:
        plan = vkv.decoder_plan(rings[0], 0, prefill)
        k0 = torch.empty(layers, prefill, KV_DIM, device="cuda")
        v0 = torch.empty(layers, prefill, KV_DIM, device="cuda")
        vkv.synth_rows(k0.data_ptr(), KV_DIM, SEED, vkv.TAG_K, nl=layers, p0=0, np_=prefill,
                       hip_stream=sp)
        vkv.synth_rows(v0.data_ptr(), KV_DIM, SEED, vkv.TAG_V, nl=layers, p0=0, np_=prefill,
                       hip_stream=sp)
        cache.append(0, 0, layers, vkv.plan_segs(plan.write_seg, plan.write_nseg), k0.data_ptr(),
                     v0.data_ptr(), hip_stream=sp)
        vkv.decoder_commit(rings[0], plan)
    q = torch.empty(n_steps, layers, Q_DIM, device="cuda")
    k = torch.empty(n_steps, layers, KV_DIM, device="cuda")
    v = torch.empty(n_steps, layers, KV_DIM, device="cuda")
    for t, tag, n in ((q, vkv.TAG_Q, Q_DIM), (k, vkv.TAG_K, KV_DIM), (v, vkv.TAG_V, KV_DIM)):
        vkv.synth_rows(t.data_ptr(), n, SEED, tag, nl=layers, l_stride=1, p0=prefill, np_=n_steps,
                       p_stride=layers, hip_stream=sp)
    out = torch.empty(n_steps, layers, Q_DIM, device="cuda")
    scale = 1.0 / (HD ** 0.5)

    def step(i):
        cache.decoder_step(0, rings, [prefill + i], 0, layers, q[i].data_ptr(), k[i].data_ptr(),
                           v[i].data_ptr(), out[i].data_ptr(), scale, hip_stream=sp)

    total_ms, step_ms, wall = timed_loop(step, n_steps, 0, st, reps=1)
    assert rings[0].next_absolute_position == prefill + n_steps
    assert bool(torch.isfinite(out).all())
    cache.close()
    return total_ms, step_ms, wall


def gpu_encoder(steps, warmup, dtype=1):
    import torch
    import vkv

    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    cache = vkv.Cache(n_streams=1, n_layers=E_LAYERS, capacity=E_CAP, n_kv_heads=E_HEADS,
                      head_dim=E_HD, n_q_heads=E_HEADS, dtype=dtype)
    # chunks from frame 0; the window is full (765 keys) from frame 752 on
    first = (E_WIN + E_CHUNK - 1) // E_CHUNK + 1
    T = first + warmup + steps
    rows = E_LAYERS * E_CHUNK * E_DIM
    q = torch.empty(T, rows, device="cuda")
    k = torch.empty(T, rows, device="cuda")
    v = torch.empty(T, rows, device="cuda")
    for t, tag in ((q, vkv.TAG_EQ), (k, vkv.TAG_EK), (v, vkv.TAG_EV)):
        # [chunk][layer][frame][dim], one chunk of 16 frames at a time
        for c in range(T):
            vkv.synth_rows(t[c].data_ptr(), E_DIM, SEED, tag, nl=E_LAYERS, p0=c * E_CHUNK,
                           np_=E_CHUNK, hip_stream=sp)
    out = torch.empty(E_LAYERS, E_CHUNK, E_DIM, device="cuda")
    plans = [vkv.enc_plan(c * E_CHUNK, E_CHUNK, E_CAP, E_WIN) for c in range(T)]

    def chunk(c):
        cache.enc_step(0, plans[c], E_WIN, 0, E_LAYERS, q[c].data_ptr(), k[c].data_ptr(),
                       v[c].data_ptr(), out.data_ptr(), 1.0 / (E_HD ** 0.5), hip_stream=sp)

    for c in range(first):
        chunk(c)
    total_ms, step_ms, wall = timed_loop(lambda i: chunk(first + i), steps, warmup, st)
    n_keys = plans[first].win_end - plans[first].win_start
    assert n_keys == E_WIN + E_CHUNK - 1
    assert bool(torch.isfinite(out).all())
    cache.close()
    return total_ms, step_ms, wall, n_keys


def host_cpu():
    """The host's processor as the CPU legs see it: nproc, the CPUs this
    process may run on, the model name (lscpu's "Model name" line)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "model": model}


def cpu_leg(dtype, target_seconds, layers=LAYERS, n_keys=CAP, streams=1, label=None):
    """The oracle's threaded restatement of ggml's CPU flash-attention step
    (append + attention over n_keys positions, `layers` layers) on a bounded
    number of tokens, in four legs: the vector leg (AVX2/FMA/F16C lanes, the
    mimic's roundings; its threaded rate is the baseline's value) and the
    scalar mimic, each on min(usable CPUs, 16) threads and on one thread.  The
    scalar one-thread leg times a 2-layer sample and scales it to `layers`
    (the step's time is linear in the layers).  With several streams the CPU
    runs them one after another, so the aggregate rate is one stream's."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    host = host_cpu()
    threads = max(1, min(host["usable_cpus"] or 1, 16))
    rb = oracle.row_bytes(dtype, KV_DIM)
    layer_bytes = rb * n_keys
    kimg = np.empty(layers * layer_bytes, np.uint8)
    vimg = np.empty(layers * layer_bytes, np.uint8)

    def fill(job):
        img, tag, l = job
        img[l * layer_bytes:(l + 1) * layer_bytes] = oracle.expected_layer(
            dtype, n_keys, n_keys, KV_DIM, n_keys, SEED, tag, 0, l)

    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(fill, [(img, tag, l) for img, tag in ((kimg, oracle.TAG_K), (vimg, oracle.TAG_V))
                             for l in range(layers)]))
    scale = 1.0 / (HD ** 0.5)

    def leg(simd, n_threads, n_layers, budget):
        secs, n = 0.0, 0
        while n < 1 or (secs < budget and n < 64):
            pos = n_keys + n
            qs = np.stack([oracle.synth_row(SEED, oracle.TAG_Q, 0, l, pos, Q_DIM) for l in range(n_layers)])
            ks = np.stack([oracle.synth_row(SEED, oracle.TAG_K, 0, l, pos, KV_DIM) for l in range(n_layers)])
            vs = np.stack([oracle.synth_row(SEED, oracle.TAG_V, 0, l, pos, KV_DIM) for l in range(n_layers)])
            dt, _ = oracle.decode_step_mimic_mt(dtype, kimg, vimg, layer_bytes, rb, n_layers, n_keys,
                                                qs, QH, KVH, HD, scale, n_threads, ks, vs,
                                                pos % n_keys, simd=simd)
            secs += dt
            n += 1
        return n, secs, n * n_layers / (secs * layers)   # tokens/s of the full `layers`

    simd_ok = oracle.simd_available()
    legs = []
    plan = ([("vector avx2/fma/f16c", True, threads, layers, 0.3),
             ("vector avx2/fma/f16c", True, 1, layers, 0.2)] if simd_ok else []) + \
        [("scalar mimic", False, threads, layers, 0.3),
         ("scalar mimic", False, 1, min(layers, 2), 0.2)]
    for name, simd, nt, nl, share in plan:
        n, secs, rate = leg(simd, nt, nl, target_seconds * share)
        legs.append({"leg": name, "threads": nt, "value": round(rate, 4), "steps": n,
                     "layers_timed": nl, "seconds": round(secs, 2)})
    main = legs[0]
    dname = "f16" if dtype == 1 else "q8_0"
    what = label or f"{layers} layers, {n_keys}-position window, {dname} KV"
    return {"value": main["value"], "unit": "tokens/s", "cores": main["threads"], "kind": "port",
            "sample": f"{main['steps']} decode steps ({what}) of the oracle's {main['leg']} "
                      f"restatement of ggml's CPU flash-attention step, {main['threads']} threads, "
                      f"{main['seconds']:.1f} s; the other legs (one thread; the scalar mimic) "
                      f"are listed under legs"
                      + (f"; the {streams} streams run one after another on the CPU, so the "
                         f"aggregate rate equals one stream's" if streams > 1 else "")
                      + ("" if simd_ok else "; this host lacks AVX2/FMA/F16C: scalar legs only"),
            "host": host, "legs": legs}


RDREQ = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_64B_sum",
         "TCC_EA0_RDREQ_32B_sum")


def summarize_profiles(workload, d, out_dir):
    """profiles/<name>_kernel_trace.md, _pmc.md and _pmc.json from the runs
    of one session under directory d:
      tr_<w>/ and tr_<w>.log      rocprofv3 --kernel-trace --stats of the bench
                                  (its last line: the bench's JSON);
      pmc_<w>_FETCH_SIZE/, pmc_<w>_WRITE_SIZE/, pmc_<w>_RDREQ/ (+ .log)
                                  --pmc runs of the bench (RDREQ: the four
                                  TCC_EA0_RDREQ counters of RDREQ);
      calib_FETCH_SIZE/, calib_WRITE_SIZE/, calib_RDREQ/
                                  the same counters over --copy-calibration 512.
    A workload with a dominant kernel is summarized per launch of it; one
    whose step is many launches (kern "") per step, the step's kernels being
    the library's kernels dispatched a whole number of times per executed
    step (warmup + reps x steps).
    Read bytes two ways: FETCH_SIZE scaled by the copy's bytes / its
    FETCH_SIZE, and the request counts by size (128, 64, 32 bytes), which
    read the copy at 1.00x.  On gfx950 FETCH_SIZE's formula counts a
    128-byte request as 64 bytes (its TCC_BUBBLE term reads 0), so the copy
    scale is 2 and a kernel that also issues 64-byte requests is over-read by
    the scaled figure; the per-size figure is the traffic reported."""
    import csv
    import glob

    wl = WORKLOADS[workload]
    kern, prefix = wl["kern"], wl["pmc"][:-len("_pmc.json")]
    step_mode = not kern

    def csv_rows(sub, pattern):
        f = glob.glob(os.path.join(d, sub, "**", pattern), recursive=True)
        if not f:
            raise SystemExit(f"no {pattern} under {os.path.join(d, sub)}")
        with open(f[0]) as fh:
            return list(csv.DictReader(fh))

    def bench_line(log):
        with open(os.path.join(d, log)) as fh:
            return json.loads([x for x in fh.read().splitlines() if x.startswith("{")][-1])

    def executed(b):
        return b["warmup"] + b.get("reps", 1) * b["steps"]

    bl = bench_line(f"tr_{workload}.log")
    algo = bl["roofline"]["bytes_per_launch"]
    trace = csv_rows(f"tr_{workload}", "*kernel_trace.csv")
    stats = csv_rows(f"tr_{workload}", "*kernel_stats.csv")
    n_tr = executed(bl)
    calls = {}
    for r in trace:
        calls[r["Kernel_Name"]] = calls.get(r["Kernel_Name"], 0) + 1
    if step_mode:
        # the library's kernels dispatched a whole number of times per step
        # (setup kernels -- weight generation, fills -- run a count unrelated
        # to the steps)
        names = {k for k, v in calls.items() if "vkv::" in k and v >= n_tr and v % n_tr == 0}
    else:
        names = {k for k in calls if kern in k}

    def matches(name):
        return name in names

    # the step's time: kernel durations, and the span with the gaps between
    # consecutive step kernels (gaps over 200 us are the host's syncs and
    # the setup, not the step's)
    disp = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in trace
                  if matches(r["Kernel_Name"]))
    if not step_mode:
        # the dominant kernel's last warmup + reps x steps dispatches: a
        # workload that fills its ring with the same kernel first (the
        # encoder window's 48 chunks before the window is full) runs those
        # before, with fewer keys than the algorithmic bytes count
        disp = disp[-n_tr:]
    busy = sum(e - b for b, e in disp)
    gaps = sum(max(0, b2 - e1) for (_, e1), (b2, _) in zip(disp, disp[1:]) if b2 - e1 < 200_000)
    per = n_tr if step_mode else len(disp)
    kernel_us, span_us = busy / per / 1e3, (busy + gaps) / per / 1e3
    avg_us = kernel_us

    def pmc(c):
        b = bench_line(f"pmc_{workload}_{c}.log")
        rs = [r for r in csv_rows(f"pmc_{workload}_{c}", "*counter_collection.csv")
              if matches(r["Kernel_Name"])]
        if not step_mode:
            # as for the trace: the dominant kernel's last executed dispatches
            keep = set(sorted({int(r["Dispatch_Id"]) for r in rs})[-executed(b):])
            rs = [r for r in rs if int(r["Dispatch_Id"]) in keep]
        acc, seen = {}, set()
        for r in rs:
            acc[r["Counter_Name"]] = acc.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            seen.add(r["Dispatch_Id"])
        n = executed(b) if step_mode else len(seen)
        return {k: v / n for k, v in acc.items()}, len(seen)

    def calib(c):
        rs = csv_rows(f"calib_{c}", "*counter_collection.csv")
        tot = {}
        for r in rs:
            tot[r["Kernel_Name"]] = tot.get(r["Kernel_Name"], 0.0) + float(r["Counter_Value"])
        big = max(tot, key=tot.get)
        acc = {}
        for r in rs:
            if r["Kernel_Name"] == big:
                acc.setdefault(r["Counter_Name"], {})[r["Dispatch_Id"]] = float(r["Counter_Value"])
        return {k: sum(v.values()) / len(v) for k, v in acc.items()}

    kf, nd = pmc("FETCH_SIZE")
    kf = kf["FETCH_SIZE"]
    kw = pmc("WRITE_SIZE")[0]["WRITE_SIZE"]
    kr = pmc("RDREQ")[0]
    cf, cw, cr = calib("FETCH_SIZE")["FETCH_SIZE"], calib("WRITE_SIZE")["WRITE_SIZE"], calib("RDREQ")
    cal_bytes = 512 * (1 << 20)

    def req_bytes(c):
        return 128 * c[RDREQ[1]] + 64 * c[RDREQ[2]] + 32 * c[RDREQ[3]]

    f_scale, w_scale = cal_bytes / (cf * 1024), cal_bytes / (cw * 1024)
    rd_fetch = kf * 1024 * f_scale
    rd_req = req_bytes(kr)
    wr = kw * 1024 * w_scale
    unit = "step" if step_mode else "launch"
    j = {"workload": bl["config"]["workload"], "kernel": kern or "the step's kernels",
         "unit": unit, "dispatches_counted": nd, "algorithmic_bytes_per_launch": algo,
         "kernel_us_per_launch": kernel_us, "span_us_per_launch": span_us,
         "fetch_size_kib_per_launch": kf, "write_size_kib_per_launch": kw,
         "rdreq_per_launch": {c: kr[c] for c in RDREQ},
         "copy_calibration": {"bytes": cal_bytes, "fetch_size_kib": cf, "write_size_kib": cw,
                              "fetch_scale": f_scale, "write_scale": w_scale,
                              "rdreq_bytes": req_bytes(cr), "rdreq_scale": cal_bytes / req_bytes(cr)},
         "hbm_read_bytes_per_launch": rd_req, "hbm_read_bytes_per_launch_fetch_size": rd_fetch,
         "hbm_write_bytes_per_launch": wr, "traffic_bytes_per_launch": rd_req + wr,
         "traffic_bytes_per_launch_fetch_size": rd_fetch + wr}
    if step_mode:
        j["dispatches_per_step"] = len(disp) / n_tr
    with open(os.path.join(out_dir, f"{prefix}_pmc.json"), "w") as fh:
        json.dump(j, fh, indent=1)
    pb = bench_line(f"pmc_{workload}_FETCH_SIZE.log")

    def args_of(b):
        return f"--steps {b['steps']} --warmup {b['warmup']} --reps {b.get('reps', 1)}"

    run = f"python3 $R/bench.py {args_of(pb)} --no-cpu --workload {workload}"
    cal = "python3 $R/bench.py --copy-calibration 512"
    cmds = [f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/pmc_{workload}_FETCH_SIZE -o p -- {run} > $OUT/pmc_{workload}_FETCH_SIZE.log",
            f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/pmc_{workload}_WRITE_SIZE -o p -- {run} > $OUT/pmc_{workload}_WRITE_SIZE.log",
            f"rocprofv3 --pmc {' '.join(RDREQ)} --output-format csv -d $OUT/pmc_{workload}_RDREQ -o p -- {run} > $OUT/pmc_{workload}_RDREQ.log",
            f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/calib_FETCH_SIZE -o c -- {cal}",
            f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/calib_WRITE_SIZE -o c -- {cal}",
            f"rocprofv3 --pmc {' '.join(RDREQ)} --output-format csv -d $OUT/calib_RDREQ -o c -- {cal}",
            f"python3 $R/bench.py --summarize {workload} --prof-dir $OUT --summary-dir $R/profiles"]
    title = bl["config"]["workload"]
    what = "step" if step_mode else f"dispatch of `{kern}`"
    md = [f"# {title}: HBM traffic counters", "",
          "Commands, one session (run from /tmp with TMPDIR=/tmp; repo at $R, output under $OUT):",
          "", "```", *cmds, "```", "", f"Per {what}:", "", "| quantity | value |", "|---|---|",
          f"| dispatches counted | {nd} |",
          f"| FETCH_SIZE / WRITE_SIZE | {kf:.1f} / {kw:.1f} KiB |",
          "| read requests: all / 128 B / 64 B / 32 B | " +
          " / ".join(f"{kr[c]:,.0f}" for c in RDREQ) + " |",
          f"| copy calibration (512 MiB): FETCH_SIZE / WRITE_SIZE | {cf:.1f} / {cw:.1f} KiB |",
          f"| copy calibration: read bytes from request sizes | {req_bytes(cr):,.0f} "
          f"({req_bytes(cr) / cal_bytes:.4f}x the copy) |",
          f"| scale factors fetch, write (copy bytes / counter bytes) | {f_scale:.4f}, {w_scale:.4f} |",
          f"| HBM read bytes, from request sizes | {rd_req:,.0f} |",
          f"| HBM read bytes, scaled FETCH_SIZE | {rd_fetch:,.0f} |",
          f"| HBM write bytes (scaled WRITE_SIZE) | {wr:,.0f} |",
          f"| algorithmic bytes | {algo:,} |",
          f"| traffic / algorithmic (request sizes; scaled FETCH_SIZE) | "
          f"{(rd_req + wr) / algo:.4f}; {(rd_fetch + wr) / algo:.4f} |"]
    with open(os.path.join(out_dir, f"{prefix}_pmc.md"), "w") as fh:
        fh.write("\n".join(md) + "\n")
    tr = [f"# {title}: kernel trace", "",
          "Command (run from /tmp with TMPDIR=/tmp; repo at $R, output under $OUT):", "", "```",
          f"rocprofv3 --kernel-trace --stats --output-format csv -d $OUT/tr_{workload} -o trace -- "
          f"python3 $R/bench.py {args_of(bl)} --no-cpu --workload {workload} > $OUT/tr_{workload}.log",
          "```", ""]
    short = lambda n: n.replace("vkv::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    if step_mode:
        tr += [f"{n_tr} executed steps; the step's kernels by grid (one row per matrix or "
               f"launch shape):", "",
               "| kernel | grid (threads) | per step | avg us | us per step |", "|---|---|---|---|---|"]
        per_name = {}
        for r in trace:
            if matches(r["Kernel_Name"]):
                key = (r["Kernel_Name"], f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}")
                a = per_name.setdefault(key, [0, 0])
                a[0] += 1
                a[1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        for (n, g), (c, t) in sorted(per_name.items(), key=lambda kv: -kv[1][1]):
            tr.append(f"| {short(n)[:70]} | {g} | {c / n_tr:.2f} | {t / c / 1e3:.2f} | "
                      f"{t / n_tr / 1e3:.1f} |")
        tr += ["", f"Per step: {len(disp) / n_tr:.1f} dispatches, {kernel_us:.1f} us of kernels, "
                   f"{span_us:.1f} us from the first kernel's start to the last one's end "
                   f"(gaps {span_us - kernel_us:.1f} us); {algo:,} algorithmic bytes / {kernel_us:.1f} us "
                   f"of kernels = {algo / kernel_us / 1e3:.1f} GB/s ({100 * algo / kernel_us / 1e3 / HBM_PEAK_GBPS:.1f}% "
                   f"of 8 TB/s); the bench's own events over the same run: "
                   f"{bl['roofline']['avg_launch_ms'] * 1e3:.1f} us per step."]
    else:
        tr += ["| kernel | calls | avg us | min us | max us | % |", "|---|---|---|---|---|---|"]
        for r in stats:
            tr.append(f"| {short(r['Name'])[:80]} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                      f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                      f"{float(r['Percentage']):.2f} |")
        # the dominant kernel's mean over its last warmup + reps x steps
        # dispatches (the table above averages every call, ring fill included)
        avg_us = kernel_us
        tr += ["", f"Dominant kernel `{kern}`, mean of its last {len(disp)} dispatches (the "
                   f"bench's warmup and timed steps): {algo:,} algorithmic bytes / {avg_us:.2f} us = "
                   f"{algo / avg_us / 1e3:.1f} GB/s = {100 * algo / avg_us / 1e3 / HBM_PEAK_GBPS:.1f}% of "
                   f"8 TB/s (the bench's own events over the same run: "
                   f"{bl['roofline']['avg_launch_ms'] * 1e3:.2f} us per launch, frac "
                   f"{bl['roofline']['frac']})."]
    with open(os.path.join(out_dir, f"{prefix}_kernel_trace.md"), "w") as fh:
        fh.write("\n".join(tr) + "\n")
    print("\n".join(tr[-1:] + md[-9:]))


def load_traffic(name):
    """(traffic, traffic from scaled FETCH_SIZE) in HBM bytes per launch of
    the dominant kernel, from the committed rocprofv3 counter runs of this
    same workload (summarize_profiles)"""
    pmc = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(pmc):
        return None, None
    with open(pmc) as f:
        j = json.load(f)
    return j.get("traffic_bytes_per_launch"), j.get("traffic_bytes_per_launch_fetch_size")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="longform_f16")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--summarize", choices=sorted(w for w in WORKLOADS if "kern" in WORKLOADS[w]),
                    help="only write the workload's profiles/ summaries from the rocprofv3 runs "
                         "under --prof-dir")
    ap.add_argument("--prof-dir", default=".")
    ap.add_argument("--summary-dir", default=os.path.join(ROOT, "profiles"),
                    help="where --summarize writes its three files")
    ap.add_argument("--reps", type=int, default=REPS,
                    help="timed repetitions of the K steps (the median is reported)")
    ap.add_argument("--kernel-flags", type=lambda x: int(x, 0), default=0,
                    help="vkv_cache_params.kernel_flags of the decode workloads' cache "
                         "(VKV_KERNEL_* bits; kernel selection for A/B runs)")
    ap.add_argument("--decode-chunk", type=int, default=0)
    ap.add_argument("--decode-waves", type=int, default=0)
    ap.add_argument("--decode-stages", type=int, default=0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 20 times (scales rocprof "
                         "FETCH_SIZE/WRITE_SIZE counters to bytes)")
    args = ap.parse_args()
    if args.summarize:
        summarize_profiles(args.summarize, args.prof_dir, args.summary_dir)
        return
    if args.reps < 1:
        ap.error("--reps must be at least 1")
    REPS_SET[0] = args.reps
    CACHE_KW.update(kernel_flags=args.kernel_flags, decode_chunk=args.decode_chunk,
                    decode_waves=args.decode_waves, decode_stages=args.decode_stages)
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 20}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures the single-GPU KV step; --gpus {args.gpus} is not supported "
              "(this path has no multi-GPU leg)", file=sys.stderr)
        sys.exit(2)

    wl = WORKLOADS[args.workload]
    global MIX
    MIX = "q8_0" if args.workload.endswith("_q8_0") else "q4km"
    traffic, traffic_fetch = load_traffic(wl["pmc"]) if wl["pmc"] else (None, None)
    if args.workload in ("stream4096_f16", "layer1_f16"):
        layers, prefill = (LAYERS, 0) if args.workload == "stream4096_f16" else (1, 1024)
        n_steps = 4096 if args.workload == "stream4096_f16" else args.steps
        total_ms, step_ms, wall = gpu_stream_from_empty(n_steps, layers, prefill)
        args.steps, args.warmup = n_steps, 0
        per_layer_fixed = 2 * KV_DIM * 4 + 2 * KV_DIM * 2 + Q_DIM * 4 + Q_DIM * 4
        total_bytes = sum(layers * ((prefill + i + 1) * 2 * KV_DIM * 2 + per_layer_fixed)
                          for i in range(n_steps))
        bytes_step = total_bytes // n_steps
        units_per_step = 1
        res = {"metric": METRIC if args.workload == "stream4096_f16" else
               "single-layer decode step latency (append + attention over 1025 positions)",
               "unit": "tokens/s"}
        config = {"workload": ("decoder KV stream: 26 layers, 4096 consecutive steps from an "
                               "empty 8192-slot ring (no wrap), f16 KV, 32 q / 8 kv heads x 128")
                  if args.workload == "stream4096_f16" else
                  ("one decoder layer, 1024 positions prefilled, append position 1024.. and "
                   "attend 1025.. positions, f16 KV, 32 q / 8 kv heads x 128"),
                  "layers": layers, "window": CAP, "kv_heads": KVH, "q_heads": QH,
                  "head_dim": HD, "streams": 1, "bytes": "mean over the steps"}
        kernel = "k_decode<FmtF16> (append fused)"
    elif args.workload == "encoder_chunk_q4km":
        total_ms, step_ms, wall, n_keys = gpu_encoder_chunk(args.steps, args.warmup)
        bytes_step = encoder_chunk_bytes(n_keys)
        units_per_step = E_CHUNK
        res = {"metric": "encoder transformer frames/s (Q4_K_M projections on the matrix cores + "
                         "window-750 attention, 32 layers, 16-frame chunks) and HBM GB/s",
               "unit": "frames/s"}
        config = {"workload": "one 16-frame encoder chunk: conv stem (128 Mel bins -> 1280, "
                              "kernel 3, strides 1 and 2, GELU) + vkv_encoder_chunk: 32 x "
                              "(RMSNorm + Q/K/V + biases, RoPE, ring append + window-750 "
                              "attention, O + bias + residual, RMSNorm + SwiGLU, W2 + bias + "
                              "residual) + final norm; dim 1280, 32 heads x 64, hidden 5120",
                  "layers": E_LAYERS, "window": E_WIN, "frames_per_chunk": E_CHUNK,
                  "bytes_per_chunk": bytes_step, "keys_per_query_block": n_keys}
        kernel = ("conv stem (k_im2col_f16 + k_gemm_f16, x2) + 32 x (k_q8k_rows + k_gemm_kq, x4; "
                  "k_rope; k_window_mfma) + final norm")
    elif args.workload in ("adapter_q4km", "adapter_group_q4km"):
        ng = wl["groups"]
        total_ms, step_ms, wall = gpu_adapter(ng, args.steps, args.warmup)
        bytes_step = adapter_bytes(ng)
        units_per_step = ng
        res = {"metric": "adapter audio embeddings/s (4 encoder frames -> 3072, Q4_K_M adapter "
                         "on the device rings) and HBM GB/s", "unit": "audio embeddings/s"}
        config = {"workload": f"vkv_adapter_commit of {ng} group{'s' if ng > 1 else ''}: encoder-"
                              "output ring rows (4 x 1280 f32 per group) -> adapter.0 (3072 x "
                              "5120 Q4_K) -> GELU(erf) -> adapter.2 (3072 x 3072 Q4_K) -> "
                              "audio-embedding ring rows; 256-row rings",
                  "groups_per_commit": ng, "bytes_per_commit": bytes_step}
        kernel = ("k_q8k_rows + k_gemm_kq (GELU) + k_q8k_rows + k_gemm_kq" if ng > 1 else
                  "k_matvec (GELU) + k_matvec")
    elif args.workload == "model_load_q4km":
        args.steps, args.warmup = min(args.steps, 5), min(args.warmup, 1)
        total_ms, step_ms, wall, data_bytes = gpu_model_load(args.steps, args.warmup)
        bytes_step = data_bytes
        units_per_step = data_bytes / 1e9
        res = {"metric": "GGUF model load GB/s (file in the page cache -> one device allocation)",
               "unit": "GB/s"}
        config = {"workload": "vkv_model_load of a full-size realtime Q4_K_M GGUF (32 encoder "
                              "layers, 26 decoder layers, 131072-row Q6_K embeddings, adapter, "
                              "conv stem, ada weights, mel filters; "
                              f"{len(realtime_tensor_list())} tensors)",
                  "bytes_per_load": data_bytes, "staging": "3 x 64 MiB pinned buffers"}
        kernel = "hipMemcpyAsync host-to-device copies (no kernels)"
    elif args.workload in ("realtime_step_q4km", "realtime_pipelined_q4km"):
        piped = args.workload == "realtime_pipelined_q4km"
        total_ms, step_ms, wall, n_keys = gpu_realtime_step(args.steps, args.warmup, piped)
        bytes_step = (encoder_chunk_bytes(n_keys, R_FRAMES) + adapter_bytes(1) + token_bytes())
        units_per_step = 1
        res = {"metric": "realtime steps/s (one 80 ms audio step: 4 encoder frames, 1 adapter "
                         "group, 1 decoder token) and HBM GB/s", "unit": "steps/s"}
        config = {"workload": "one realtime step of the streaming path: conv stem + vkv_encoder_"
                              "chunk_ring over 4 new frames (32 layers, window 750), "
                              "vkv_adapter_commit of the completed group, vkv_decoder_token "
                              "reading its audio row (26 layers, full 8192-slot f16 ring, logits, "
                              "argmax); Q4_K_M weights",
                  "audio_ms_per_step": 80, "bytes_per_step": bytes_step}
        if piped:
            config["workload"] += ("; pipelined on two HIP streams: the decoder token of step i "
                                   "reads the previous step's audio row while step i's encoder "
                                   "and adapter run (events order the two chains)")
            config["streams"] = 2
        kernel = "whole step (encoder, adapter and decoder launches)"
    elif args.workload == "decoder_prompt_q4km":
        total_ms, step_ms, wall = gpu_prompt(args.steps, args.warmup)
        bytes_step = prompt_bytes()
        units_per_step = P_TOKENS
        res = {"metric": "decoder prefill prompt tokens/s (38-token prompt + audio rows through "
                         "26 Q4_K_M layers, causal attention with KV append, logits of the last "
                         "token) and HBM GB/s", "unit": "prompt tokens/s"}
        config = {"workload": "vkv_decoder_prompt of a 38-token prompt at the stream start: "
                              "embedding rows + audio rows, 26 x (RMSNorm + Q/K/V with RoPE, "
                              "causal attention + K/V append, O + residual, RMSNorm*(1+ada) + "
                              "SwiGLU, W2 + residual), final norm, 131072-row logits, argmax",
                  "layers": LAYERS, "dim": DIM, "hidden": HIDDEN, "vocab": VOCAB,
                  "prompt_tokens": P_TOKENS, "bytes_per_prompt": bytes_step}
        kernel = "whole prompt (k_gemm_kq, k_q8k_rows, k_window_mfma, k_matvec launches)"
    elif args.workload in ("decoder_token_q4km", "decoder_token_q8_0"):
        total_ms, step_ms, wall = gpu_token(args.steps, args.warmup)
        bytes_step = token_bytes()
        units_per_step = 1
        kind = "Q4_K_M" if MIX == "q4km" else "Q8_0"
        res = {"metric": f"decoder tokens/s (whole step: {kind} projections + f16 KV attention at "
                         "the 8192 window, 26 layers, logits, argmax) and HBM GB/s",
               "unit": "tokens/s"}
        config = {"workload": "one decoder token through vkv_decoder_token: embedding + audio, "
                              "26 x (RMSNorm + Q/K/V, RoPE + append + attention over the full "
                              "8192-slot f16 ring, O + residual, RMSNorm*(1+ada) + SwiGLU, W2 + "
                              "residual), final norm, 131072-row logits, argmax",
                  "layers": LAYERS, "dim": DIM, "hidden": HIDDEN, "vocab": VOCAB, "window": CAP,
                  "bytes_per_token": bytes_step, "launches_per_token": 6 * LAYERS + 2}
        kernel = ("k_kq_dequant + 26 x (4 k_matvec + k_decode + k_combine) + k_matvec "
                  "(158 launches per token)")
    elif args.workload == "decoder_loop_q4km":
        if not any(a == "--steps" or a.startswith("--steps=") for a in sys.argv[1:]):
            args.steps = 1000   # enough tokens for a p99
        total_ms, step_ms, wall = gpu_token_loop(args.steps, args.warmup)
        bytes_step = token_bytes()
        units_per_step = 1
        res = {"metric": "decoder tokens/s in the production loop (vkv_decoder_token + 4-byte "
                         "token readback + one synchronize per token) and per-token latency",
               "unit": "tokens/s"}
        config = {"workload": "the greedy token loop: per token vkv_decoder_token (26 layers, "
                              "Q4_K_M weights, f16 KV attention over the full 8192-slot ring, "
                              "logits, argmax), the token copied to pinned host memory, one "
                              "stream synchronize, the token fed to the next step",
                  "layers": LAYERS, "dim": DIM, "hidden": HIDDEN, "vocab": VOCAB, "window": CAP,
                  "bytes_per_token": bytes_step, "syncs_per_token": 1}
        kernel = "one decoder token (158 launches) + a 4-byte copy, then a synchronize"
        lat = sorted(LOOP_LAT_MS)
        pick = lambda q: lat[min(len(lat) - 1, int(round(q * (len(lat) - 1))))]  # noqa: E731
        res["latency_ms"] = {"p50": round(pick(0.50), 4), "p90": round(pick(0.90), 4),
                             "p99": round(pick(0.99), 4), "max": round(lat[-1], 4),
                             "mean": round(sum(lat) / len(lat), 4), "tokens": len(lat)}
    elif args.workload in ("decoder_weights_q4km", "decoder_weights_q8_0"):
        total_ms, step_ms, wall = gpu_weights(args.steps, args.warmup)
        bytes_step = weights_bytes_per_token()
        units_per_step = 1
        kind = ("Q4_K_M mix (attn_v, ffn_w2, output Q6_K; others Q4_K)" if MIX == "q4km" else
                "Q8_0 file (every matrix Q8_0, q8_0 input images)")
        res = {"metric": f"decoder projection tokens/s and HBM GB/s on {kind.split(' ')[0]} weights "
                         "(26 layers + logits)", "unit": "tokens/s"}
        config = {"workload": "decoder step projections, one token: 26 x (RMSNorm + Q/K/V, "
                              "O + residual, RMSNorm*(1+ada) + SwiGLU W1/W3, W2 + residual) + "
                              f"final norm + 131072-row logits; {kind}",
                  "layers": LAYERS, "dim": DIM, "hidden": HIDDEN, "vocab": VOCAB,
                  "weight_bytes_per_token": bytes_step, "calls_per_token": 4 * LAYERS + 1}
        kernel = "k_matvec (105 launches per token)"
    elif args.workload in ("encoder_f16", "encoder_f32"):
        total_ms, step_ms, wall, n_keys = gpu_encoder(args.steps, args.warmup, wl["dtype"])
        e = 2 if wl["dtype"] == 1 else 4
        bytes_step = encoder_bytes_per_chunk(n_keys, e=e)
        units_per_step = E_CHUNK
        res = {"metric": "encoder sliding-window attention + ring append frames/s at window 750",
               "unit": "frames/s"}
        config = {"workload": f"encoder streaming window: 32 layers, 32 heads x 64, 878-slot ring "
                              f"({wl['dtype_name']}), window 750, 16 new frames appended and "
                              f"attended per chunk as a 16-query block",
                  "layers": E_LAYERS, "window": E_WIN, "heads": E_HEADS, "head_dim": E_HD,
                  "ring": E_CAP, "frames_per_chunk": E_CHUNK, "keys_per_query_block": n_keys}
        kernel = ("k_window_mfma<64, 4, 4, 1> (4 kv heads per work group" if e == 2 else
                  "k_window_mfma_f32<64> (one kv head per work group") + \
            "; ring append fused; one launch per chunk)"
    else:
        ns = wl["streams"]
        layerwise = args.workload.startswith("layerwise_")
        rope = 1.0e6 if args.workload == "longform_rope_f16" or layerwise else None
        total_ms, step_ms, wall = gpu_decode(wl["dtype"], ns, args.steps, args.warmup, rope,
                                             layerwise)
        bytes_step = ns * decode_bytes_per_stream_token(CAP, wl["dtype"])
        units_per_step = ns
        res = {"metric": METRIC, "unit": "tokens/s"}
        config = {"workload": f"decoder KV step: 26 layers, 8192-slot ring full and wrapping, "
                              f"{wl['dtype_name']} KV, 32 q / 8 kv heads x 128, {ns} stream"
                              f"{'s' if ns > 1 else ''}, append + 1-query attention per layer",
                  "layers": LAYERS, "window": CAP, "kv_heads": KVH, "q_heads": QH,
                  "head_dim": HD, "streams": ns}
        if layerwise:
            config["workload"] = ("decoder KV step in the decoder's call shape: 26 "
                                  "vkv_decoder_layer_step calls per token (one layer each, RoPE "
                                  f"fused), 8192-slot ring full and wrapping, {wl['dtype_name']} KV, "
                                  "32 q / 8 kv heads x 128, 1 stream")
            kernel = ("26 x (k_decode + k_combine) (RoPE and append fused; 256-slot chunks, then "
                      "the merge" + ("; q8_0 blocks against the q8_0 query in integer dot "
                                     "products" if wl["dtype"] == 8 else "") + ")")
        elif wl["dtype"] == 1 and ns == 1:
            kernel = ("k_decode_rows + k_combine (append fused; a work group per (layer, 912-slot "
                      "chunk) reading whole rows, then the merge of the 9 chunks)")
        else:
            kernel = ("k_decode_q8rows + k_combine (append fused; a work group per (stream, layer, "
                      "1024-slot chunk) reading whole rows into LDS, then the merge of the 8 chunks)")
    # the load is bound by the host link, not HBM: PCIe 5.0 x16, 64 GB/s per direction
    bound, peak = ("host link (PCIe 5.0 x16)", 64.0) if args.workload == "model_load_q4km" else \
        ("hbm", HBM_PEAK_GBPS)
    ms_per_step = total_ms / args.steps
    step_avg = sum(step_ms) / len(step_ms)
    achieved = bytes_step / (step_avg * 1e-3) / 1e9
    res.update({
        "value": round(units_per_step * args.steps / (total_ms * 1e-3), 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "reps": len(REP_MS),
        "rep_ms_per_step": [round(t / args.steps, 5) for t in REP_MS],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype_name"],
        "data": wl.get("data", "synthetic (seeded integer Irwin-Hall N(0,1) Q/K/V, generated on "
                               "device)"),
        "config": config,
        "hbm_gbps": round(bytes_step / (ms_per_step * 1e-3) / 1e9, 1),
        "pct_hbm_peak": round(100 * bytes_step / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 2),
        "roofline": {"bound": bound, "achieved": round(achieved, 1), "peak": peak,
                     "unit": "GB/s", "frac": round(achieved / peak, 4),
                     "traffic": round(traffic) if traffic else None,
                     "traffic_scaled_fetch_size": round(traffic_fetch) if traffic_fetch else None,
                     "kernel": kernel,
                     "bytes_per_launch": bytes_step,
                     "avg_launch_ms": round(step_avg, 5)},
        "wall_s": round(wall, 3),
    })
    if not args.no_cpu and args.workload in ("decoder_weights_q4km", "decoder_weights_q8_0"):
        res["cpu_baseline"] = cpu_weights_leg(args.cpu_seconds)
    elif not args.no_cpu and args.workload == "encoder_chunk_q4km":
        res["cpu_baseline"] = cpu_encoder_leg(E_CHUNK, args.cpu_seconds)
    elif not args.no_cpu and args.workload in ("realtime_step_q4km", "realtime_pipelined_q4km"):
        res["cpu_baseline"] = cpu_realtime_leg(args.cpu_seconds)
    elif not args.no_cpu and args.workload == "decoder_prompt_q4km":
        res["cpu_baseline"] = cpu_prompt_leg(args.cpu_seconds)
    elif not args.no_cpu and args.workload in ("decoder_token_q4km", "decoder_loop_q4km",
                                               "decoder_token_q8_0"):
        res["cpu_baseline"] = cpu_token_leg(args.cpu_seconds)
    elif not args.no_cpu and args.workload in ("adapter_q4km", "adapter_group_q4km"):
        res["cpu_baseline"] = cpu_adapter_leg(wl["groups"], args.cpu_seconds)
    elif not args.no_cpu and args.workload == "model_load_q4km":
        res["cpu_baseline"] = cpu_load_leg(args.cpu_seconds)
    elif not args.no_cpu and args.workload == "layer1_f16":
        res["cpu_baseline"] = cpu_leg(1, args.cpu_seconds, layers=1, n_keys=1025,
                                      label="1 layer, 1025 positions, f16 KV")
    elif not args.no_cpu and args.workload == "stream4096_f16":
        # the CPU step's time is linear in the window: the run's mean window
        # (steps 0..4095 attend 1..4096 keys) stands for the run
        res["cpu_baseline"] = cpu_leg(1, args.cpu_seconds, n_keys=2048,
                                      label="26 layers at the run's mean window of 2048 positions, "
                                            "f16 KV")
    elif not args.no_cpu and args.workload not in ("encoder_f16", "encoder_f32", "encoder_chunk_q4km",
                                                   "adapter_q4km", "adapter_group_q4km",
                                                   "model_load_q4km", "realtime_step_q4km"):
        res["cpu_baseline"] = cpu_leg(wl["dtype"], args.cpu_seconds, streams=wl["streams"])
    if "cpu_baseline" in res:
        res["cpu_baseline"].setdefault("host", host_cpu())
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
