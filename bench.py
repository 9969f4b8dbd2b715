#!/usr/bin/env python3
"""Benchmark of the Qwen2 attention path on one MI355X.

Workloads (synthetic, seeded):
  prefill  Qwen2.5-7B attention (28 q heads / 4 kv heads, head_dim 128),
           causal prefill of 32768 tokens through all 28 layers: per layer the
           fused RoPE + KV append (bf16 Q/K/V in, F16 cache, theta 1e6) and the
           MFMA flash prefill.  One step = 28 layers.
           Throughput = 4 * Hq * d * sum_i (i + 1) FLOP per layer.
  decode   ASR transcript decode with CFG-style batch 2: 7B heads, one new
           token per step per stream, Q8_0 caches pre-filled to 32768
           positions, 28 layers (each with its own 2 x 71 MB of cache, 2 GB in
           all, so the 256 MB MALL cannot hold it).  One step = 28 layers of
           RoPE + append + split-K decode.
           Attention bytes per layer-step = K/V cache rows read (2 streams x L
           x Hkv x 2 x 136 B) + f32 Q read + f32 O write; the whole-step rate
           also counts the RoPE + append traffic.

  prefill_chunked  the ASR prefill as the reference runs it: 64 chunks of 512
           tokens over a growing past, 7B heads (same FLOPs as the single
           shot); reported beside the single-shot line.
  decode_small  the 0.5B TTS CFG decode step (B = 2, 14 q / 2 kv heads,
           d = 64, F16 caches at 1024, 24 layers), eager and as one captured
           HIP graph per step.

Prints one JSON line: `value` is the prefill throughput (TFLOP/s), `decode`
holds the decode throughput (GB/s); each carries a roofline entry measured
with HIP events around every attention launch on the library's stream.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "vibevoice.cpp_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

PEAK_F16_TFLOPS = 2500.0     # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E

D, HQ, HKV, LAYERS = 128, 28, 4, 28
T_PREFILL = 32768
L_DECODE = 32768
B_DECODE = 2
THETA = 1.0e6
CHUNK = 512                      # ASR prefill chunk (64 chunks cover 32768 tokens)
# 0.5B TTS CFG decode: 14 q / 2 kv heads, d = 64, F16 caches at 1024, 24 layers
S_D, S_HQ, S_HKV, S_LAYERS, S_L = 64, 14, 2, 24, 1024

# HBM bytes per launch of the dominant kernels, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# passes over this script (KiB per dispatch), each scaled by the counter's reading for a plain
# 1 GiB device-to-device copy (`--only copy`): FETCH_SIZE read 512 MiB for 1 GiB (x 2.0),
# WRITE_SIZE 1 GiB (x 1.0).  Counters and commands: profiles/prefill_kernel_7b_32k.md,
# profiles/decode_stream_q8_0_7b_32k.md.
TRAFFIC_PREFILL = (605956.9 * 2.0 + 459122.8 * 1.0) * 1024          # prefill_kernel<128,F16>
TRAFFIC_DECODE = ((35170.0 + 938.0) * 2.0 + (1904.0 + 28.0) * 1.0) * 1024    # stream + merge


def prefill_flops_per_layer(T: int, past: int = 0) -> float:
    # 2 * d for QK^T and 2 * d for PV per visible (query, key) pair
    return 4.0 * HQ * D * (T * past + T * (T + 1) / 2)


def decode_attn_bytes(lens) -> float:
    """Attention launch: K and V cache rows of every stream + f32 Q read + f32 O write."""
    q8_row = (D // 32) * 34
    return sum(L * HKV * 2 * q8_row for L in lens) + 2 * len(lens) * HQ * D * 4


def decode_append_bytes(B: int) -> float:
    """RoPE + append launch: f32 q, k, v read, f32 rotated q written, Q8_0 K and V rows written."""
    return B * ((HQ + 2 * HKV) * D * 4 + HQ * D * 4 + 2 * HKV * (D // 32) * 34)


def synth_weight(torch, vva, rng, m: int, k: int, wt: int):
    """Random weight bytes of m rows of k inputs as ggml stores them: F16
    values ~ N(0, 1/k), or GGUF Q8_0 blocks (fp16 scale of the same spread /
    127, int8 codes uniform in [-127, 127]) -- synthetic data, nothing is
    quantized."""
    if wt == vva.F16:
        raw = (rng.standard_normal((m, k)) * k ** -0.5).astype(np.float16).view(np.uint8).reshape(-1)
    else:
        nb = k // 32
        blk = np.empty((m, nb, 34), dtype=np.uint8)
        d = (rng.uniform(0.5, 1.5, (m, nb)) * 1.7 * k ** -0.5 / 127.0).astype(np.float16)
        blk[:, :, 0:2] = d.view(np.uint8).reshape(m, nb, 2)
        blk[:, :, 2:] = rng.integers(-127, 128, (m, nb, 32), dtype=np.int8).view(np.uint8)
        raw = blk.reshape(-1)
    return vva.Weight(torch.from_numpy(raw).cuda(), wt, k, m)


def run_prefill(torch, vva, ctx, steps: int, warmup: int, heavy: bool = False):
    rng = torch.Generator(device="cuda").manual_seed(1234)
    q = torch.randn((1, T_PREFILL, HQ, D), generator=rng, device="cuda").to(torch.bfloat16)
    k = torch.randn((1, T_PREFILL, HKV, D), generator=rng, device="cuda")
    if heavy:
        # heavy-tailed logits: K of tokens [1024 i, 1024 (i + 1)) scaled by 1 + 3.5 i, so each
        # row's running max rises by > 10 nats every 16 key tiles (up to 31 rescales per row)
        k = k * (1.0 + 3.5 * torch.div(torch.arange(T_PREFILL, device="cuda"), 1024,
                                       rounding_mode="floor")).view(1, -1, 1, 1)
    k = k.to(torch.bfloat16)
    v = torch.randn((1, T_PREFILL, HKV, D), generator=rng, device="cuda").to(torch.bfloat16)
    pos = torch.arange(T_PREFILL, dtype=torch.int32, device="cuda")
    qr = torch.empty((1, T_PREFILL, HQ, D), dtype=torch.float16, device="cuda")
    out = torch.empty((1, T_PREFILL, HQ, D), dtype=torch.float32, device="cuda")
    kv = vva.KVCache(ctx, LAYERS, HKV, D, T_PREFILL, 1, vva.F16)
    scale = D ** -0.5
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(LAYERS * steps)]

    def step(events=None):
        kv.set_len(0, 0)
        for layer in range(LAYERS):
            ctx.rope_append(kv, layer, q, k, v, pos, qr, freq_base=THETA)
            if events is not None:
                events[layer][0].record()
            ctx.attn(kv, layer, qr, out, scale)
            if events is not None:
                events[layer][1].record()
        kv.set_len(0, T_PREFILL)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        step(ev[s * LAYERS:(s + 1) * LAYERS])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    attn_ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    flops_layer = prefill_flops_per_layer(T_PREFILL)
    res = {
        "ms_per_step": wall * 1e3 / steps,
        "tflops": flops_layer * LAYERS * steps / wall / 1e12,
        "attn_ms": attn_ms,
        "attn_tflops": flops_layer / (attn_ms * 1e-3) / 1e12,
        "flops_per_layer": flops_layer,
    }
    return res, kv, qr, out


def run_decode(torch, vva, ctx, steps: int, warmup: int):
    rng = torch.Generator(device="cuda").manual_seed(4321)
    n_layer_steps = 32                  # per form, in the decode-step comparison below
    n_block_steps = 16                  # per form, in the attention-block comparison below
    kv = vva.KVCache(ctx, LAYERS, HKV, D, L_DECODE + steps + warmup + 2 * (n_layer_steps + n_block_steps) + 16,
                     B_DECODE, vva.Q8_0)
    # fill every layer's caches by appending L_DECODE random rows (RoPE'd K, raw V)
    chunk = 8192
    for layer in range(LAYERS):
        for c0 in range(0, L_DECODE, chunk):
            n = min(chunk, L_DECODE - c0)
            for s in range(B_DECODE):
                kv.set_len(s, c0)
            kk = torch.randn((B_DECODE, n, HKV, D), generator=rng, device="cuda")
            vv = torch.randn((B_DECODE, n, HKV, D), generator=rng, device="cuda")
            qq = torch.empty((B_DECODE, n, 1 * HKV, D), device="cuda")
            pos = torch.arange(c0, c0 + n, dtype=torch.int32, device="cuda")
            ctx.rope_append(kv, layer, qq, kk, vv, pos, qq, freq_base=THETA)
    torch.cuda.synchronize()
    for s in range(B_DECODE):
        kv.set_len(s, L_DECODE)
    q = torch.randn((B_DECODE, 1, HQ, D), generator=rng, device="cuda")
    k = torch.randn((B_DECODE, 1, HKV, D), generator=rng, device="cuda")
    v = torch.randn((B_DECODE, 1, HKV, D), generator=rng, device="cuda")
    qr = torch.empty_like(q)
    out = torch.empty((B_DECODE, 1, HQ, D), dtype=torch.float32, device="cuda")
    pos = torch.zeros((B_DECODE, 1), dtype=torch.int32, device="cuda")
    scale = D ** -0.5
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    lens_timed = []
    # The tensor descriptors do not change between steps: build them once and
    # call the C ABI directly, so the host enqueues faster than the GPU runs.
    # A step enqueues the 28 layers' RoPE + append, then their 28 attention
    # calls back to back between one event pair: an event pair around a
    # single launch costs several microseconds by itself at this kernel size,
    # a burst of 28 launches amortises it.  Each layer's append still precedes
    # its attention on the stream.
    lib, h, kvh = ctx.lib, ctx.h, kv.h
    byref = ctypes.byref
    qv, kv_, vv_, pv, qrv, ov = (vva.view(t) for t in (q, k, v, pos, qr, out))
    qv_r, kv_r, vv_r, pv_r, qrv_r, ov_r = (byref(t) for t in (qv, kv_, vv_, pv, qrv, ov))

    def step(events=None):
        cur = kv.get_len(0)
        pos.fill_(cur)
        for layer in range(LAYERS):
            ctx.check(lib.vva_rope_append(h, kvh, layer, qv_r, kv_r, vv_r, pv_r, None, THETA, qrv_r))
        if events is not None:
            events[0].record()
        for layer in range(LAYERS):
            ctx.check(lib.vva_attn(h, kvh, layer, qrv_r, None, None, scale, ov_r))
        if events is not None:
            events[1].record()
        for s in range(B_DECODE):
            kv.set_len(s, cur + 1)
        return cur + 1

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        lens_timed.append(step(ev[s]))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    attn_us = float(np.mean([a.elapsed_time(b) for a, b in ev])) * 1e3 / LAYERS

    # The decode step as the ASR loop runs it, layer after layer (RoPE +
    # append + attention of one new token per stream): vva_decode_step (the
    # streamed kernel in step mode, then its merge) against the
    # vva_rope_append + vva_attn pair, alternating, n_layer_steps steps each.
    def layer_step(fused, events):
        cur = kv.get_len(0)
        pos.fill_(cur)
        events[0].record()
        for layer in range(LAYERS):
            if fused:
                ctx.check(lib.vva_decode_step(h, kvh, layer, qv_r, kv_r, vv_r, pv_r, None, THETA, scale, qrv_r, ov_r))
            else:
                ctx.check(lib.vva_rope_append(h, kvh, layer, qv_r, kv_r, vv_r, pv_r, None, THETA, qrv_r))
                ctx.check(lib.vva_attn(h, kvh, layer, qrv_r, None, None, scale, ov_r))
        events[1].record()
        for s in range(B_DECODE):
            kv.set_len(s, cur + 1)
        return cur + 1

    layer_step(True, ev[0])
    layer_step(False, ev[0])
    torch.cuda.synchronize()
    ev_f = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_layer_steps)]
    ev_u = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_layer_steps)]
    lens_fused = []
    for i in range(n_layer_steps):
        lens_fused.append(layer_step(True, ev_f[i]))
        layer_step(False, ev_u[i])
    torch.cuda.synchronize()
    step_fused_us = float(np.mean([a.elapsed_time(b) for a, b in ev_f])) * 1e3 / LAYERS
    step_pair_us = float(np.mean([a.elapsed_time(b) for a, b in ev_u])) * 1e3 / LAYERS

    # The attention half of a decode layer (normed input to residual sum,
    # src/qwen2.cpp:273-350) with Q8_0 weights, 28 layers' weights in
    # rotation: the bare projections and the fused step (vva_qkv_proj +
    # vva_decode_step, which rotates and quantizes the new rows itself) against
    # vva_qkv_rope_append (projection, then RoPE and the Q8_0 append as a
    # second launch) + vva_attn; both end with vva_out_proj_residual.
    wrng = np.random.default_rng(23)
    hidden, m_qkv = HQ * D, (HQ + 2 * HKV) * D
    wshape = {"q": (HQ * D, hidden), "k": (HKV * D, hidden), "v": (HKV * D, hidden), "o": (hidden, HQ * D)}
    w0 = {key: synth_weight(torch, vva, wrng, m, k, vva.Q8_0) for key, (m, k) in wshape.items()}
    wsets = [w0] + [{key: vva.Weight(w.raw.clone(), w.w_type, w.K, w.M) for key, w in w0.items()}
                    for _ in range(LAYERS - 1)]
    wrefs = [tuple(byref(ws[key].t) for key in "qkvo") for ws in wsets]
    xb = torch.randn((B_DECODE, 1, hidden), generator=rng, device="cuda")
    hb = torch.empty_like(xb)
    yb = torch.empty((B_DECODE, 1, m_qkv), device="cuda")
    qy = yb[:, :, :HQ * D].view(B_DECODE, 1, HQ, D)
    ky = yb[:, :, HQ * D:(HQ + HKV) * D].view(B_DECODE, 1, HKV, D)
    vy = yb[:, :, (HQ + HKV) * D:].view(B_DECODE, 1, HKV, D)
    orows = out.view(B_DECODE, 1, HQ * D)
    bt = [vva.view(t) for t in (xb, hb, yb, qy, ky, vy, orows)]
    xr, hr, yr, qyr, kyr, vyr, orr = (byref(t) for t in bt)

    def block_step(fused, events):
        cur = kv.get_len(0)
        pos.fill_(cur)
        events[0].record()
        for layer in range(LAYERS):
            w = wrefs[layer]
            if fused:
                ctx.check(lib.vva_qkv_proj(h, xr, w[0], w[1], w[2], None, None, None, yr))
                ctx.check(lib.vva_decode_step(h, kvh, layer, qyr, kyr, vyr, pv_r, None, THETA, scale, qrv_r, ov_r))
            else:
                ctx.check(lib.vva_qkv_rope_append(h, kvh, layer, xr, w[0], w[1], w[2], None, None, None, pv_r, None,
                                                  THETA, qrv_r))
                ctx.check(lib.vva_attn(h, kvh, layer, qrv_r, None, None, scale, ov_r))
            ctx.check(lib.vva_out_proj_residual(h, orr, w[3], xr, hr))
        events[1].record()
        for s in range(B_DECODE):
            kv.set_len(s, cur + 1)

    block_step(True, ev[0])
    block_step(False, ev[0])
    torch.cuda.synchronize()
    ev_bf = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_block_steps)]
    ev_bu = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_block_steps)]
    for i in range(n_block_steps):
        block_step(True, ev_bf[i])
        block_step(False, ev_bu[i])
    torch.cuda.synchronize()
    block_fused_us = float(np.mean([a.elapsed_time(b) for a, b in ev_bf])) * 1e3 / LAYERS
    block_pair_us = float(np.mean([a.elapsed_time(b) for a, b in ev_bu])) * 1e3 / LAYERS
    del wsets, wrefs
    bytes_total = sum(decode_attn_bytes([L] * B_DECODE) + decode_append_bytes(B_DECODE)
                      for L in lens_timed) * LAYERS
    mean_L = float(np.mean(lens_timed))
    bytes_layer = decode_attn_bytes([mean_L] * B_DECODE)
    kv_bytes_layer = B_DECODE * mean_L * HKV * 2 * (D // 32) * 34
    res = {
        "ms_per_step": wall * 1e3 / steps,
        "gbs": bytes_total / wall / 1e9,
        "attn_us": attn_us,
        "attn_gbs": bytes_layer / (attn_us * 1e-6) / 1e9,
        "bytes_per_layer": bytes_layer,
        "kv_bytes_per_layer": kv_bytes_layer,
        "splits": ctx.last_decode_splits(),
        "mean_L": mean_L,
        "step_fused_us": step_fused_us,
        "step_pair_us": step_pair_us,
        "step_bytes": decode_attn_bytes([float(np.mean(lens_fused))] * B_DECODE) + decode_append_bytes(B_DECODE),
        "block_fused_us": block_fused_us,
        "block_pair_us": block_pair_us,
    }
    return res, kv


def run_prefill_chunked(torch, vva, ctx, layers: int, cache_type: int = None):
    """The ASR prefill as the reference runs it: 64 chunks of 512 tokens per
    layer, chunk c attending to its 512 rows plus the 512 c rows before it
    (same total FLOPs as the single-shot prefill).  HIP events around each
    chunk's attention launch."""
    rng = torch.Generator(device="cuda").manual_seed(99)
    q = torch.randn((1, CHUNK, HQ, D), generator=rng, device="cuda").to(torch.bfloat16)
    k = torch.randn((1, CHUNK, HKV, D), generator=rng, device="cuda").to(torch.bfloat16)
    v = torch.randn((1, CHUNK, HKV, D), generator=rng, device="cuda").to(torch.bfloat16)
    qr = torch.empty((1, CHUNK, HQ, D), dtype=torch.float16, device="cuda")
    out = torch.empty((1, CHUNK, HQ, D), dtype=torch.float32, device="cuda")
    ct = vva.F16 if cache_type is None else cache_type
    kv = vva.KVCache(ctx, layers + 1, HKV, D, T_PREFILL, 1, ct)
    n_chunks = T_PREFILL // CHUNK
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(layers * n_chunks)]
    scale = D ** -0.5
    pos_all = torch.arange(T_PREFILL, dtype=torch.int32, device="cuda")
    # chunk by chunk, the layer stack inside each chunk, as the reference's ASR
    # loop builds one graph per chunk (src/vibevoice_asr.cpp:554-652); layer 0
    # is untimed (it sizes the workspace).  The host settles a chunk's split
    # plan at its first call and the chunk's other layers reuse it (the
    # layer-major order measured the same: the host runs ahead of the GPU)
    for c in range(n_chunks):
        kv.set_len(0, c * CHUNK)
        for layer in range(layers + 1):
            ctx.rope_append(kv, layer, q, k, v, pos_all[c * CHUNK:(c + 1) * CHUNK], qr, freq_base=THETA)
            if layer > 0:
                ev[(layer - 1) * n_chunks + c][0].record()
            ctx.attn(kv, layer, qr, out, scale)
            if layer > 0:
                ev[(layer - 1) * n_chunks + c][1].record()
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in ev]
    attn_ms = float(np.sum(ms)) / layers
    flops = sum(4.0 * HQ * D * (CHUNK * c * CHUNK + CHUNK * (CHUNK + 1) / 2) for c in range(n_chunks))
    kv.free()
    tname = {vva.F16: "F16", vva.Q8_0: "Q8_0 (window converted to f16 per call)"}[ct]
    return {"workload": f"Qwen2.5-7B-shaped ASR prefill: {n_chunks} chunks of {CHUNK} tokens, past 0..{T_PREFILL - CHUNK}, "
                        f"{tname} cache, {layers} layers",
            "value": round(flops / (attn_ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s",
            "frac_of_mfma_peak": round(flops / (attn_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4),
            "attn_ms_per_layer": round(attn_ms, 3), "flop_per_layer": flops,
            "splits_last_chunk": ctx.last_decode_splits(),
            "first_chunk_ms": round(float(np.mean(ms[::n_chunks])), 4),
            "last_chunk_ms": round(float(np.mean(ms[n_chunks - 1::n_chunks])), 4),
            "timing": "HIP events around each chunk's attention launch"}


def run_decode_small(torch, vva, ctx, steps: int, vvo=None):
    """The 0.5B TTS CFG decode step (B = 2, 14 q / 2 kv heads, d = 64, F16
    caches at 1024, 24 layers of RoPE + append + attention), timed as eager
    launches from prebuilt descriptors and as one captured HIP graph per
    step.  The graph's kernel arguments (cache lengths) are fixed at capture,
    so each replay repeats the captured step at the same positions."""
    rng = torch.Generator(device="cuda").manual_seed(5)
    B = 2
    kv = vva.KVCache(ctx, S_LAYERS, S_HKV, S_D, S_L + 8, B, vva.F16)
    for layer in range(S_LAYERS):
        for s_ in range(B):
            kv.set_len(s_, 0)
        kk = torch.randn((B, S_L, S_HKV, S_D), generator=rng, device="cuda")
        vv = torch.randn((B, S_L, S_HKV, S_D), generator=rng, device="cuda")
        qq = torch.empty((B, S_L, S_HKV, S_D), device="cuda")
        pos = torch.arange(S_L, dtype=torch.int32, device="cuda")
        ctx.rope_append(kv, layer, qq, kk, vv, pos, qq, freq_base=THETA)
    for s_ in range(B):
        kv.set_len(s_, S_L)
    q = torch.randn((B, 1, S_HQ, S_D), generator=rng, device="cuda")
    k = torch.randn((B, 1, S_HKV, S_D), generator=rng, device="cuda")
    v = torch.randn((B, 1, S_HKV, S_D), generator=rng, device="cuda")
    qr = torch.empty_like(q)
    out = torch.empty((B, 1, S_HQ, S_D), dtype=torch.float32, device="cuda")
    pos = torch.full((B, 1), S_L, dtype=torch.int32, device="cuda")
    scale = S_D ** -0.5
    lib, h, kvh = ctx.lib, ctx.h, kv.h
    byref = ctypes.byref
    qv, kv_, vv_, pv, qrv, ov = (vva.view(t) for t in (q, k, v, pos, qr, out))

    def step_unfused():
        for layer in range(S_LAYERS):
            ctx.check(lib.vva_rope_append(h, kvh, layer, byref(qv), byref(kv_), byref(vv_), byref(pv), None, THETA,
                                          byref(qrv)))
            ctx.check(lib.vva_attn(h, kvh, layer, byref(qrv), None, None, scale, byref(ov)))

    def step():
        # vva_decode_step: RoPE + append + attention + split merge in one launch per layer
        for layer in range(S_LAYERS):
            ctx.check(lib.vva_decode_step(h, kvh, layer, byref(qv), byref(kv_), byref(vv_), byref(pv), None, THETA,
                                          scale, byref(qrv), byref(ov)))

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    unfused_us = timed(step_unfused)
    eager_us = timed(step)
    g = torch.cuda.CUDAGraph()
    default = torch.cuda.current_stream()
    try:
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream())
            step()
    finally:
        ctx.set_stream(default)
    g.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_us = e0.elapsed_time(e1) * 1e3 / steps
    del g
    L = S_L + 1
    # bytes per layer of the step: the K/V window read, f32 q/k/v in, rotated q and output out,
    # the appended K/V row
    attn_bytes = B * L * S_HKV * 2 * S_D * 2 + 2 * B * S_HQ * S_D * 4
    step_bytes = attn_bytes + B * ((S_HQ + 2 * S_HKV) * S_D * 4 + S_HQ * S_D * 4 + 2 * S_HKV * S_D * 2)
    cpu = None
    if vvo is not None:
        kraw = [kv.download(0, s_, L)[0].reshape(-1) for s_ in range(B)]
        vraw = [kv.download(0, s_, L)[1].reshape(-1) for s_ in range(B)]
        qn = qr.float().cpu().numpy()
        calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 5.0:
            vvo.attn(qn, kraw, vraw, vvo.F16, vvo.F16, [L] * B, n_kv_heads=S_HKV, scale=scale, mode=vvo.GGML)
            calls += 1
        dt = time.perf_counter() - t0
        cpu = {"value": round(calls * attn_bytes / dt / 1e9, 2), "unit": "GB/s", "cores": vvo.n_cores(),
               "kind": "port", "us_per_layer": round(dt / calls * 1e6, 2),
               "sample": f"{calls} attention calls of one layer (B=2, L={L}, F16 cache), ggml-order oracle, {dt:.1f} s"}
    kv.free()
    eager_layer, graph_layer = eager_us / S_LAYERS, graph_us / S_LAYERS
    return {"workload": f"Qwen2.5-0.5B-shaped TTS CFG decode: B=2, {S_HQ}q/{S_HKV}kv d={S_D}, F16 cache at {S_L}, "
                        f"{S_LAYERS} layers of RoPE + append + attention (vva_decode_step: one launch per layer; "
                        f"the rope_append + attn pair beside it)",
            "eager_us_per_step": round(eager_us, 2), "graph_us_per_step": round(graph_us, 2),
            "eager_us_per_layer": round(eager_layer, 3), "graph_us_per_layer": round(graph_layer, 3),
            "unfused_eager_us_per_layer": round(unfused_us / S_LAYERS, 3),
            "kernels_per_layer": 1,
            "attn_bytes_per_layer": attn_bytes, "step_bytes_per_layer": step_bytes, "steps": steps,
            "roofline": {"bound": "hbm", "achieved": round(step_bytes / eager_layer / 1e3, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(step_bytes / eager_layer / 1e3 / PEAK_HBM_GBS, 4),
                         "note": "a 1 MB window per layer is L2/MALL-resident: launch latency, not bandwidth, bounds it"},
            "cpu_baseline": cpu,
            "timing": "HIP events around `steps` back-to-back steps; graph: one captured step replayed"}


def run_proj(torch, vva, reps: int = 10, token_shapes=((4096, 1), (512, 1), (1, 2)), weight_types=None):
    """The fused projections at 7B shapes (hidden 3584, 28 q / 4 kv heads,
    d = 128), F16 and Q8_0 weights: vva_qkv_rope_append (q/k/v GEMM + bias +
    RoPE + F16 cache append) and vva_out_proj_residual.
      4096-token prefill and a 512-token ASR chunk: MFMA-bound (FLOP =
        2 N K M); HIP events around `reps` back-to-back calls.
      2-token CFG decode step: bound by streaming the weights (bytes = weight
        bytes); the calls rotate over 28 layers' weights, as a layer stack
        does (1.6 GB of F16 weights, beyond the 256 MB MALL), timed as one
        captured HIP graph of the 28 calls replayed (GPU time), and eagerly
        (launched one by one from Python, which bounds it)."""
    ctx = vva.Context(0)
    rng = np.random.default_rng(17)
    hidden, M_qkv = HQ * D, (HQ + 2 * HKV) * D
    shapes = {"q": (HQ * D, hidden), "k": (HKV * D, hidden), "v": (HKV * D, hidden), "o": (hidden, HQ * D)}
    out = {}
    n_layers = 28
    for wt, name in weight_types or ((vva.F16, "f16"), (vva.Q8_0, "q8_0")):
        sets = []
        for layer in range(n_layers):
            ws = {}
            for key, (m, k) in shapes.items():
                if layer == 0:
                    ws[key] = synth_weight(torch, vva, rng, m, k, wt)
                else:                                       # same bytes, another buffer
                    ws[key] = vva.Weight(sets[0][key].raw.clone(), wt, k, m)
            sets.append(ws)
        wbytes_qkv = sum(sets[0][k_].raw.numel() for k_ in "qkv")
        wbytes_o = sets[0]["o"].raw.numel()
        for T, B in token_shapes:
            kv = vva.KVCache(ctx, 1, HKV, D, T + 8, B, vva.F16)
            x = torch.randn((B, T, hidden), device="cuda")
            q_out = torch.empty((B, T, HQ, D), dtype=torch.float16, device="cuda")
            o = torch.randn((B, T, HQ * D), device="cuda")
            h = torch.empty((B, T, hidden), device="cuda")
            pos = torch.arange(T, dtype=torch.int32, device="cuda")
            calls = {
                "qkv": lambda w: ctx.qkv_rope_append(kv, 0, x, w["q"], w["k"], w["v"], pos, q_out),
                "o": lambda w: ctx.out_proj_residual(o, w["o"], x, h),
            }
            for op, fn in calls.items():
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                M = M_qkv if op == "qkv" else hidden
                flops = 2.0 * B * T * hidden * M
                if T > 1:
                    # untimed calls for >= 3 ms of GPU time: after the heavier shape
                    # before it the GPU's clock recovers over ~1 ms (kernel trace:
                    # the first 512-token calls after 4096-token ones run 8-10 % slow)
                    e0.record()
                    for _ in range(3):
                        fn(sets[0])
                    e1.record()
                    torch.cuda.synchronize()
                    n_more = int(3000.0 / max(e0.elapsed_time(e1) * 1e3 / 3, 1.0)) + 1
                    for _ in range(n_more):
                        fn(sets[0])
                    torch.cuda.synchronize()
                    e0.record()
                    for _ in range(reps):
                        fn(sets[0])
                    e1.record()
                    torch.cuda.synchronize()
                    us = e0.elapsed_time(e1) * 1e3 / reps
                    entry = {"us_per_call": round(us, 2), "tflops": round(flops / us / 1e6, 1),
                             "frac_of_mfma_peak": round(flops / us / 1e6 / PEAK_F16_TFLOPS, 4)}
                else:
                    for layer in range(n_layers):
                        fn(sets[layer])
                    torch.cuda.synchronize()
                    e0.record()
                    for r in range(4):
                        for layer in range(n_layers):
                            fn(sets[layer])
                    e1.record()
                    torch.cuda.synchronize()
                    eager = e0.elapsed_time(e1) * 1e3 / (4 * n_layers)
                    g = torch.cuda.CUDAGraph()
                    default = torch.cuda.current_stream()
                    try:
                        with torch.cuda.graph(g):
                            ctx.set_stream(torch.cuda.current_stream())
                            for layer in range(n_layers):
                                fn(sets[layer])
                    finally:
                        ctx.set_stream(default)
                    g.replay()
                    torch.cuda.synchronize()
                    e0.record()
                    for r in range(reps):
                        g.replay()
                    e1.record()
                    torch.cuda.synchronize()
                    us = e0.elapsed_time(e1) * 1e3 / (reps * n_layers)
                    del g
                    wb = wbytes_qkv if op == "qkv" else wbytes_o
                    entry = {"us_per_call": round(us, 2), "eager_us_per_call": round(eager, 2),
                             "weight_gbs": round(wb / us / 1e3, 1), "frac_of_hbm_peak": round(wb / us / 1e3 / PEAK_HBM_GBS, 4)}
                out[f"{op}_{name}_T{T}xB{B}"] = entry
            kv.free()
        del sets
    ctx.close()
    return {"workload": "Qwen2.5-7B-shaped projections: q/k/v GEMM + bias + RoPE + F16 cache append "
                        "(vva_qkv_rope_append) and output projection + residual (vva_out_proj_residual), "
                        "F16 and Q8_0 weights, 4096- and 512-token chunks and 2-token CFG decode step",
            "timing": f"4096 and 512 tokens: HIP events around {reps} back-to-back calls (prep + GEMM kernels); "
                      "2 tokens: 28 layers' weights in rotation, one captured HIP graph of the 28 calls replayed "
                      f"{reps} times (us_per_call), and the same calls launched eagerly", **out}


def run_small_prefills(torch, vva, reps: int = 20, vvo=None):
    """The two short prefill configurations, attention launch only (after the
    RoPE + append), HIP events around `reps` passes over the launches of a
    28- (or 24-) layer stack:
      C1  0.5B heads (14 q / 2 kv, d = 64), 256 tokens, F32 Q/K/V and F32
          cache: the fp32 eager branch (src/qwen2.cpp:336-344; the 1e-4
          tolerance), and beside it the flash branch, which casts the F32
          window to F16 (src/qwen2.cpp:328-331) and runs the MFMA prefill;
      C3  1.5B heads (12 q / 2 kv, d = 128), 4096 tokens, bf16 Q/K/V, F16
          cache: the MFMA flash prefill.
    With vvo, C1's eager line and C3 carry a cpu_baseline: the oracle on
    layer 0's cache and rotated Q (C1: every row, fp32 accumulation; C3: 512
    rows spread over the 4096, ggml order), repeated for about 2 s."""
    ctx = vva.Context(0)
    res = {}
    for name, (d, hq, hkv, T, layers, qt, ct, fa) in {
            "c1_0p5b_fp32_T256": (64, 14, 2, 256, 24, torch.float32, vva.F32, False),
            "c1_0p5b_f32cache_flash_T256": (64, 14, 2, 256, 24, torch.float32, vva.F32, True),
            "c3_1p5b_T4096": (128, 12, 2, 4096, 28, torch.bfloat16, vva.F16, True)}.items():
        ctx.set_flash_attn(fa)
        kv = vva.KVCache(ctx, layers, hkv, d, T, 1, ct)
        q = torch.randn((1, T, hq, d), device="cuda").to(qt)
        k = torch.randn((1, T, hkv, d), device="cuda").to(qt)
        v = torch.randn((1, T, hkv, d), device="cuda").to(qt)
        qr = torch.empty((1, T, hq, d), dtype=torch.float32 if ct == vva.F32 else torch.float16, device="cuda")
        out = torch.empty((1, T, hq, d), dtype=torch.float32, device="cuda")
        pos = torch.arange(T, dtype=torch.int32, device="cuda")
        kv.set_len(0, 0)
        for layer in range(layers):
            ctx.rope_append(kv, layer, q, k, v, pos, qr, freq_base=THETA)
        for rep in range(2):
            for layer in range(layers):
                ctx.attn(kv, layer, qr, out, d ** -0.5)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for rep in range(reps):
            for layer in range(layers):
                ctx.attn(kv, layer, qr, out, d ** -0.5)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (reps * layers)
        flops = 4.0 * hq * d * T * (T + 1) / 2
        peak = 157.3 if not fa else PEAK_F16_TFLOPS
        res[name] = {"attn_ms_per_layer": round(ms, 4), "tflops": round(flops / ms / 1e9, 2),
                     "peak_tflops": peak, "frac": round(flops / ms / 1e9 / peak, 4), "layers": layers,
                     "flop_per_layer": flops}
        if vvo is not None and name != "c1_0p5b_f32cache_flash_T256":
            res[name]["cpu_baseline"] = cpu_baseline_small(vvo, kv, qr, d, hq, hkv, T, ct)
        kv.free()
    ctx.close()
    res["timing"] = "HIP events around reps x layers back-to-back attention launches (the stack's order), per launch"
    return res


def cpu_baseline_small(vvo, kv, qr, d, hq, hkv, T, ct):
    """Oracle on layer 0 of a short prefill (all host cores), repeated for about 2 s: F32 caches
    every query row in fp32 accumulation, F16 caches 512 rows spread over [0, T) in ggml order."""
    kraw, vraw = kv.download(0, 0, T)
    q32 = qr.float().cpu().numpy()
    if ct == vvo.F32:
        rows, mode, what = np.arange(T, dtype=np.int32), vvo.GGML_F32ACC, "every row, fp32 accumulation, F32 K/V"
    else:
        rows, mode, what = np.linspace(0, T - 1, 512).astype(np.int32), vvo.GGML, "512 rows spread, ggml order, F16 K/V"
    calls = 0
    t0 = time.perf_counter()
    while True:
        vvo.attn(q32, [kraw.reshape(-1)], [vraw.reshape(-1)], ct, ct, [T], n_kv_heads=hkv, scale=d ** -0.5,
                 mode=mode, rows=rows)
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= 2.0:
            break
    flops = calls * float(sum(4.0 * hq * d * (int(r) + 1) for r in rows))
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": vvo.n_cores(), "kind": "port",
            "sample": f"1 layer, {len(rows)} query rows x {hq} heads ({what}), {calls} calls, {dt:.1f} s"}


def cpu_baseline_prefill(torch, vva, vvo, kv, qr):
    """Oracle (ggml-order mode, all host cores) on layer 0: 4096 query rows spread over [0, 32k)."""
    rows = np.linspace(0, T_PREFILL - 1, 4096).astype(np.int32)
    kraw, vraw = kv.download(0, 0, T_PREFILL)
    q32 = qr.float().cpu().numpy()
    t0 = time.perf_counter()
    vvo.attn(q32, [kraw.reshape(-1)], [vraw.reshape(-1)], vvo.F16, vvo.F16, [T_PREFILL], n_kv_heads=HKV,
             scale=D ** -0.5, mode=vvo.GGML, rows=rows)
    dt = time.perf_counter() - t0
    flops = float(sum(4.0 * HQ * D * (int(r) + 1) for r in rows))
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": vvo.n_cores(), "kind": "port",
            "sample": f"1 layer, {len(rows)} query rows spread over [0,{T_PREFILL}) x {HQ} heads, "
                      f"ggml-order oracle (F16 K/V), {dt:.1f} s"}


def cpu_baseline_decode(torch, vva, vvo, kv):
    """Oracle (ggml-order mode, Q8_0 integer dots): whole decode steps of both streams over the
    caches of 2 layers, repeated for about 10 s of CPU time."""
    rng = np.random.default_rng(9)
    L = kv.get_len(0)
    caches = [kv.download(layer, s, L) for layer in range(2) for s in range(B_DECODE)]
    q = rng.standard_normal((B_DECODE, 1, HQ, D)).astype(np.float32)
    ks = [[caches[layer * B_DECODE + s][0].reshape(-1) for s in range(B_DECODE)] for layer in range(2)]
    vs = [[caches[layer * B_DECODE + s][1].reshape(-1) for s in range(B_DECODE)] for layer in range(2)]
    calls = 0
    t0 = time.perf_counter()
    while True:
        layer = calls % 2
        vvo.attn(q, ks[layer], vs[layer], vvo.Q8_0, vvo.Q8_0, [L] * B_DECODE, n_kv_heads=HKV,
                 scale=D ** -0.5, mode=vvo.GGML)
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= 10.0:
            break
    nbytes = calls * decode_attn_bytes([L] * B_DECODE)
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": vvo.n_cores(), "kind": "port",
            "sample": f"{calls} layer-steps (2 layers' caches in turn), B=2, L={L}, Q8_0 cache, "
                      f"ggml-order oracle, {dt:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed prefill steps (28 layers each)")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--decode-steps", type=int, default=512)
    ap.add_argument("--decode-len", type=int, default=L_DECODE,
                    help="cache positions before the first decode step (the metric is quoted at 32768)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the chunked ASR prefill (64 x 512) and the 0.5B F16 decode step (eager and graph)")
    ap.add_argument("--only", choices=["prefill", "decode", "both", "copy", "proj", "small", "chunked"],
                    default="both",
                    help="copy: a plain 1 GiB device-to-device copy, the reference for FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention library has no multi-GPU mode "
              "(heads or CFG streams would shard with no exchange); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import vva
    import vvo

    torch.cuda.set_device(0)
    if args.only == "copy":
        n = 1 << 30
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": 3}), flush=True)
        return 0
    if args.only in ("proj", "small", "chunked"):
        if args.only == "chunked":
            c = vva.Context(0)
            r = {"f16": run_prefill_chunked(torch, vva, c, layers=2),
                 "q8_0": run_prefill_chunked(torch, vva, c, layers=2, cache_type=vva.Q8_0)}
            c.close()
        elif args.only == "proj":
            r = run_proj(torch, vva)
        else:
            r = run_small_prefills(torch, vva, vvo=None if args.no_cpu else vvo)
            c = vva.Context(0)
            r["c2_decode_small"] = run_decode_small(torch, vva, c, steps=200)
            c.close()
        print(json.dumps({args.only: r}), flush=True)
        return 0
    ctx = vva.Context(0)
    line = {
        "metric": "prefill attn TFLOP/s (% MFMA peak); decode attn HBM GB/s (% peak), 1 GPU",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "Qwen2.5-7B-shaped causal prefill, 32768 tokens, 28 layers, 28q/4kv d=128, "
                               "bf16 Q/K/V in, F16 KV cache, RoPE theta 1e6",
                   "global_batch": 1, "seq_len": T_PREFILL, "layers": LAYERS},
    }
    if args.only in ("prefill", "both"):
        pre, kv, qr, _ = run_prefill(torch, vva, ctx, args.steps, args.warmup)
        line["value"] = round(pre["tflops"], 2)
        line["ms_per_step"] = round(pre["ms_per_step"], 3)
        line["roofline"] = {"bound": "mfma", "achieved": round(pre["attn_tflops"], 2), "peak": PEAK_F16_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(pre["attn_tflops"] / PEAK_F16_TFLOPS, 4),
                            "traffic": TRAFFIC_PREFILL, "kernel": "prefill_kernel<128,F16>",
                            "avg_launch_ms": round(pre["attn_ms"], 4),
                            "flop_per_launch": pre["flops_per_layer"]}
        if not args.no_cpu:
            line["cpu_baseline"] = cpu_baseline_prefill(torch, vva, vvo, kv, qr)
        kv.free()
        torch.cuda.empty_cache()
        if not args.no_extra:
            hv, kvh_, _, _ = run_prefill(torch, vva, ctx, 1, 0, heavy=True)
            line["prefill_heavy_logits"] = {
                "workload": "as the prefill line, K of every 1024-token block scaled by 1 + 3.5 i: the running "
                            "max of a row rises by > 10 nats every 16 key tiles",
                "attn_ms": round(hv["attn_ms"], 4), "tflops": round(hv["attn_tflops"], 2),
                "frac_of_mfma_peak": round(hv["attn_tflops"] / PEAK_F16_TFLOPS, 4)}
            kvh_.free()
            torch.cuda.empty_cache()
    if args.only in ("decode", "both"):
        globals()["L_DECODE"] = args.decode_len      # read by run_decode
        dec, kvd = run_decode(torch, vva, ctx, args.decode_steps, max(1, args.warmup))
        line["decode"] = {
            "workload": f"Qwen2.5-7B-shaped CFG decode, batch 2, Q8_0 KV cache {args.decode_len} positions, 28 layers",
            "value": round(dec["gbs"], 1), "unit": "GB/s", "steps": args.decode_steps,
            "ms_per_step": round(dec["ms_per_step"], 4), "dtype": "q8_0/f32",
            "roofline": {"bound": "hbm", "achieved": round(dec["attn_gbs"], 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(dec["attn_gbs"] / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_DECODE,
                         "kernel": "decode_stream_kernel<128,2,2> + decode_merge_kernel<128>",
                         "avg_launch_us": round(dec["attn_us"], 3), "bytes_per_launch": dec["bytes_per_layer"],
                         "timing": "HIP events around each step's 28 back-to-back attention calls",
                         "splits": dec["splits"]},
            "step": {"workload": "the decode step as the ASR loop runs it: per layer RoPE + append + attention of "
                                 "one new token per stream, layer after layer",
                     "fused_us_per_layer": round(dec["step_fused_us"], 3),
                     "rope_append_plus_attn_us_per_layer": round(dec["step_pair_us"], 3),
                     "fused_gbs": round(dec["step_bytes"] / (dec["step_fused_us"] * 1e-6) / 1e9, 1),
                     "fused_frac_of_hbm_peak": round(dec["step_bytes"] / (dec["step_fused_us"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                     "timing": "HIP events around each step's 28 layers, 32 steps per form, alternating"},
            "block": {"workload": "the attention half of a decode layer, normed input to residual sum, Q8_0 "
                                  "weights (28 layers' in rotation): vva_qkv_proj + vva_decode_step against "
                                  "vva_qkv_rope_append + vva_attn, each followed by vva_out_proj_residual",
                      "fused_us_per_layer": round(dec["block_fused_us"], 3),
                      "unfused_us_per_layer": round(dec["block_pair_us"], 3),
                      "kernels_per_layer": {"fused": 4, "unfused": 5},
                      "timing": "HIP events around each step's 28 layers, 16 steps per form, alternating"},
        }
        if not args.no_cpu:
            line["decode"]["cpu_baseline"] = cpu_baseline_decode(torch, vva, vvo, kvd)
        kvd.free()
        if line["value"] is None:
            line["metric"] = "decode attn HBM GB/s (% peak), 1 GPU"
            line["value"], line["unit"] = line["decode"]["value"], "GB/s"
            line["ms_per_step"] = line["decode"]["ms_per_step"]
            line["roofline"] = line["decode"]["roofline"]
    if not args.no_extra and args.only in ("prefill", "decode", "both"):
        line["prefill_chunked"] = run_prefill_chunked(torch, vva, ctx, layers=2)
        torch.cuda.empty_cache()
        line["prefill_chunked_q8_0"] = run_prefill_chunked(torch, vva, ctx, layers=2, cache_type=vva.Q8_0)
        torch.cuda.empty_cache()
        line["decode_small"] = run_decode_small(torch, vva, ctx, steps=200, vvo=None if args.no_cpu else vvo)
        line["prefill_small"] = run_small_prefills(torch, vva, vvo=None if args.no_cpu else vvo)
        torch.cuda.empty_cache()
        line["proj"] = run_proj(torch, vva)
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
