#!/usr/bin/env python3
"""bench.py — MI355X measurement of the quantized-transformer hot path.

Workload (single GPU): the Whisper-large-v3 Q8_0
linear, out[M=1500, N=5120] = a[1500, 1280] . dequant(W[5120, 1280])^T with
a ~ N(0,1) f32 and W ~ N(0,0.02) packed to Q8_0 (synthetic, seeded). One step
= the whole gemm_q_f32 op on HBM-resident inputs: the INT8 activation pass
plus the MFMA block GEMM, f32 output written to HBM. The K timed steps are
captured into one HIP graph and replayed with one launch (the eager,
Python-issued loop is reported beside it as extra.eager_step_ms).

Prints ONE JSON line. `value` is whole-op throughput in TOPS (2*M*N*K per
step); `roofline` is the GEMM kernel alone, timed with HIP events on the
library's own stream; `cpu_baseline` is the oracle's restatement of the same
INT8 block GEMM on a bounded row sample, single thread (the reference's
INT8 quant route is single-threaded, kquant.rs:590-629).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quant-GEMM TOPS + paged-attn GB/s (% peak); decode tok/s, Whisper-large shape"
PEAK = {"int8_tops": 5000.0, "bf16_tflops": 2500.0, "fp32_tflops": 157.3, "hbm_gbs": 8000.0}


def timed_steps(ctx, hip, steps, warmup, launch, kernel_of_interest):
    """Runs warmup + steps; returns (wall ms per step, avg kernel ms)."""
    for _ in range(warmup):
        launch(None)
    ctx.synchronize()
    evs = [(hip.Event(ctx), hip.Event(ctx)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        launch(evs[i])
    ctx.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    kern_ms = float(np.mean([a.elapsed_ms(b) for a, b in evs]))
    return wall_ms, kern_ms


def bench_q8_gemm(ctx, hip, steps, warmup, act):
    M, N, K = 1500, 5120, 1280
    rng = np.random.default_rng(20261201)
    a = rng.standard_normal((M, K), dtype=np.float32)
    w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    wq = ctx.quantize_bytes(hip.KvQuant.Q8_0, w)
    W = ctx.upload_qweight(hip.WDtype.Q8_0, N, K, wq)
    d_a = hip.DeviceBuffer.from_array(ctx, a)
    d_out = hip.DeviceBuffer(ctx, M * N * 4)
    qa = ctx.qact(M, K)

    def launch(ev):
        qa.quantize(M, d_a, act)
        if ev is not None:
            ev[0].record()
        ctx.gemm_qact_dev(W, qa, d_out)
        if ev is not None:
            ev[1].record()

    eager_ms, _ = timed_steps(ctx, hip, steps, warmup, launch, "vk_gemm_qblock")
    # The timed steps: the same two launches (quantize, GEMM) per step, all
    # `steps` of them captured into one HIP graph and replayed with one launch,
    # the way a serving loop issues them, so the number is device time rather
    # than Python call overhead (about 8 us per graph launch from Python).
    warm = ctx.capture(lambda: [launch(None) for _ in range(max(warmup, 1))])
    timed = ctx.capture(lambda: [launch(None) for _ in range(steps)])
    warm.launch()
    ctx.synchronize()
    t0 = time.perf_counter()
    timed.launch()
    ctx.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    # the GEMM kernel alone: `steps` back-to-back launches replayed from one
    # graph on the library's stream, between two HIP events (the per-launch
    # average rocprof reports for this kernel)
    gemms = ctx.capture(lambda: [ctx.gemm_qact_dev(W, qa, d_out) for _ in range(steps)])
    gemms.launch()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    gemms.launch()
    e1.record()
    kern_ms = e0.elapsed_ms(e1) / steps
    ops = 2.0 * M * N * K
    return {"M": M, "N": N, "K": K, "wall_ms": wall_ms, "eager_ms": eager_ms, "gemm_ms": kern_ms,
            "tops": ops / (wall_ms * 1e-3) / 1e12, "gemm_tops": ops / (kern_ms * 1e-3) / 1e12,
            "a": a, "wq": wq}


def bench_q4_gemv(ctx, hip, n, k=1280, ms=(1, 8, 64), stream_bytes=600 << 20):
    """Q4_0 decode GEMV: back-to-back launches over distinct weight
    copies totalling > 512 MB, so weights come from HBM, not the 256 MB MALL;
    then the same linears as one grouped launch (vokra_hip_linear_group_run).
    GB/s counts the algorithmic bytes of one linear: Q4_0 weights
    n*(k/32)*18 + f32 activations m*k*4 + f32 outputs m*n*4."""
    rng = np.random.default_rng(7)
    wbytes = n * (k // 32) * 18
    copies = max(2, stream_bytes // wbytes)
    base = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    Ws = []
    for i in range(copies):
        wq = ctx.quantize_bytes(hip.KvQuant.Q4_0, base if i == 0 else np.roll(base, i, axis=1))
        Ws.append(ctx.upload_qweight(hip.WDtype.Q4_0, n, k, wq))
    res = {}
    for m in ms:
        a = rng.standard_normal((m, k), dtype=np.float32)
        d_a = hip.DeviceBuffer.from_array(ctx, a)
        d_out = hip.DeviceBuffer(ctx, m * n * 4)
        qa = ctx.qact(m, k)
        qa.quantize(m, d_a)
        # one graph replays all launches: host launch cost is not measured
        graph = ctx.capture(lambda: [ctx.gemm_qact_dev(W, qa, d_out) for W in Ws])
        graph.launch()
        e0, e1 = hip.Event(ctx), hip.Event(ctx)
        e0.record()
        graph.launch()
        e1.record()
        us = e0.elapsed_ms(e1) * 1e3 / len(Ws)
        nbytes = wbytes + m * k * 4 + m * n * 4
        gbs = nbytes / (us * 1e-6) / 1e9
        # the same linears as one grouped launch (one output buffer each): the
        # decode kernel's streaming rate without a launch per linear
        outs = [hip.DeviceBuffer(ctx, m * n * 4) for _ in Ws]
        group = hip.LinearGroup(ctx, Ws, outs)
        group.run(qa)
        ctx.synchronize()
        e0.record()
        for _ in range(3):
            group.run(qa)
        e1.record()
        gus = e0.elapsed_ms(e1) * 1e3 / (3 * len(Ws))
        ggbs = nbytes / (gus * 1e-6) / 1e9
        del group, outs
        res[f"M{m}"] = {"us_per_launch": round(us, 3), "bytes": nbytes, "gbs": round(gbs, 1),
                        "frac_hbm": round(gbs / PEAK["hbm_gbs"], 4),
                        "grouped": {"us_per_linear": round(gus, 3), "gbs": round(ggbs, 1),
                                    "frac_hbm": round(ggbs / PEAK["hbm_gbs"], 4)}}
    ctx.synchronize()
    del Ws
    return {"N": n, "K": k, "weight_copies": copies, **res}


Q4K_LAYER = [("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
             ("gate", 5632, 2048), ("up", 5632, 2048), ("down", 2048, 5632)]


def q4k_random_weight(rng, n, k):
    """Random Q4_K payload with the f16 d / dmin high bytes pinned small
    (as the reference's kquant_gemm_parity.rs:45-62 random_blocks)."""
    b = rng.integers(0, 256, size=(n * (k // 256), 144), dtype=np.uint8)
    b[:, 1] = 0x2C
    b[:, 3] = 0x24
    return b.reshape(-1)


def bench_q4k_decode(ctx, hip, m=32, layers=24):
    """Speech-LLM decode linears (config 4: d=2048, FFN 5632, 16/2 heads x 128)
    at batch m through the K-quant INT8 path: all 7 linears of `layers`
    distinct layers (24 x 24.8 MB = 594 MB > the 256 MB MALL) replayed as one
    graph. GB/s counts Q4_K weight bytes n*(k/256)*144 plus f32 activations
    and outputs per linear."""
    rng = np.random.default_rng(4)
    Ws = []
    for _ in range(layers):
        Ws.append([(name, n, k, ctx.upload_qweight(hip.WDtype.Q4_K, n, k, q4k_random_weight(rng, n, k)))
                   for (name, n, k) in Q4K_LAYER])
    qa = {}
    for k in (2048, 5632):
        a = rng.standard_normal((m, k), dtype=np.float32)
        q = ctx.qact(m, k)
        q.quantize(m, hip.DeviceBuffer.from_array(ctx, a), hip.ActQuant.KQUANT)
        qa[k] = q
    d_out = hip.DeviceBuffer(ctx, m * 5632 * 4)
    graph = ctx.capture(lambda: [ctx.gemm_qact_dev(W, qa[k], d_out) for layer in Ws for (_, _, k, W) in layer])
    graph.launch()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    graph.launch()
    e1.record()
    us_layer = e0.elapsed_ms(e1) * 1e3 / layers
    nbytes = sum(n * (k // 256) * 144 + m * k * 4 + m * n * 4 for (_, n, k) in Q4K_LAYER)
    ops = sum(2 * m * n * k for (_, n, k) in Q4K_LAYER)
    ctx.synchronize()
    del Ws
    return {"M": m, "layers": layers, "us_per_layer": round(us_layer, 3), "bytes_per_layer": nbytes,
            "gbs": round(nbytes / (us_layer * 1e-6) / 1e9, 1),
            "frac_hbm": round(nbytes / (us_layer * 1e-6) / 1e9 / PEAK["hbm_gbs"], 4),
            "tops": round(ops / (us_layer * 1e-6) / 1e12, 2)}


def bench_sdpa(ctx, hip, reps=20, T=1500, H=20, hd=64, batch=1):
    """Config 1 fused self-attention: 20 heads x 64, 1500 x 1500, non-causal,
    N(0,1) f32 q/k/v resident in HBM. Timed: the whole attn_f32_dev op (fp16
    hi/lo split pre-passes + the flash kernel). flops = 4*B*H*T^2*hd."""
    rng = np.random.default_rng(15)
    d = [hip.DeviceBuffer.from_array(ctx, rng.standard_normal((batch, T, H * hd), dtype=np.float32))
         for _ in range(3)]
    d_out = hip.DeviceBuffer(ctx, batch * T * H * hd * 4)

    def run():
        ctx.attn_f32_dev(batch, T, T, H, H, hd, d[0], d[1], d[2], hd ** -0.5, False, 0, d_out)

    run()
    ctx.synchronize()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    ms = e0.elapsed_ms(e1) / reps
    flops = 4.0 * batch * H * T * T * hd
    return {"B": batch, "T": T, "H": H, "hd": hd, "ms": round(ms, 4),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
            "frac_fp16_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK["bf16_tflops"], 4),
            "mfma_passes_per_product": 3}


def bench_paged_attn(ctx, hip, n_stream, H, hd, hq, len_lo, len_hi, max_time, n_layer=16, reps=10, seed=3):
    """Decode self-attention over the paged Q8_0 KV cache, 16-token pages placed
    at shuffled addresses, per-stream lengths U(len_lo..len_hi), for n_layer
    layers whose caches together exceed twice the 256 MB MALL; the timed loop
    launches the layers in rotation, so each launch reads its cache from HBM.
    GB/s counts per launch the K and V head slices read (int8 + f16 scale per
    32 values) for every (stream, key) plus f32 q and out. The same launch
    repeated on one layer (its cache then served from the MALL) is reported
    beside it as `single_layer_repeat`."""
    rng = np.random.default_rng(seed)
    bs = 16
    kv = ctx.kv_cache(n_layer, H, hd, n_stream, max_time, bs)
    ppl = (max_time + bs - 1) // bs
    kv.set_free_order(rng.permutation(n_layer * ppl).astype(np.int32))
    lens = rng.integers(len_lo, len_hi + 1, n_stream).astype(np.int32)
    w = H * hd
    st = np.concatenate([np.full(int(lens[s]), s, np.int32) for s in range(n_stream)])
    tt = np.concatenate([np.arange(int(lens[s]), dtype=np.int32) for s in range(n_stream)])
    for layer in range(n_layer):
        for i0 in range(0, st.size, 1024):
            i1 = min(st.size, i0 + 1024)
            rows = rng.standard_normal((i1 - i0, w), dtype=np.float32)
            kv.append(layer, st[i0:i1], tt[i0:i1], rows, rows[::-1].copy())
    d_st = hip.DeviceBuffer.from_array(ctx, np.arange(n_stream, dtype=np.int32))
    d_len = hip.DeviceBuffer.from_array(ctx, lens)
    d_q = hip.DeviceBuffer.from_array(ctx, rng.standard_normal((n_stream, hq * hd), dtype=np.float32))
    d_out = hip.DeviceBuffer(ctx, n_stream * hq * hd * 4)

    def run(layer):
        kv.attn_dev(layer, n_stream, d_st, d_len, int(lens.max()), hq, d_q, hd ** -0.5, d_out)

    for layer in range(n_layer):
        run(layer)
    ctx.synchronize()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for _ in range(reps):
        for layer in range(n_layer):
            run(layer)
    e1.record()
    us = e0.elapsed_ms(e1) * 1e3 / (reps * n_layer)
    e0.record()
    for _ in range(reps * n_layer):
        run(0)
    e1.record()
    us_one = e0.elapsed_ms(e1) * 1e3 / (reps * n_layer)
    nbytes = int(lens.sum()) * 2 * (w + (w // 32) * 2) + 2 * n_stream * hq * hd * 4
    del kv
    ctx.synchronize()
    return {"streams": n_stream, "kv_heads": H, "q_heads": hq, "head_dim": hd, "len_range": [len_lo, len_hi],
            "keys_total": int(lens.sum()), "layers_rotated": n_layer, "working_set_bytes": n_layer * nbytes,
            "us": round(us, 3), "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / PEAK["hbm_gbs"], 4),
            "single_layer_repeat": {"us": round(us_one, 3), "gbs": round(nbytes / (us_one * 1e-6) / 1e9, 1),
                                    "note": "one layer's cache, served from the MALL"}}


def random_block_weight(rng, wd, n, k, scale):
    """Random wire payload of n x k block-format weights: uniform quants and
    one f16 scale for every block (`scale`), i.e. random-init weights."""
    nb = n * (k // 32)
    if wd == 8:  # Q8_0: f16 d + 32 int8
        b = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    else:        # Q4_0: f16 d + 16 bytes of nibbles
        b = rng.integers(0, 256, size=(nb, 18), dtype=np.uint8)
    b[:, 0:2] = np.array([scale], np.float16).view(np.uint8)
    return b.reshape(-1)


def whisper_layer(rng, wd, d, ff, scale, decoder=False):
    one, zero = np.ones(d, np.float32), np.zeros(d, np.float32)
    L = {"ln1_gamma": one, "ln1_beta": zero, "ln2_gamma": one, "ln2_beta": zero}
    mats = [("wq", d, d), ("wk", d, d), ("wv", d, d), ("wo", d, d), ("w1", ff, d), ("w2", d, ff)]
    if decoder:
        L.update({"ln3_gamma": one, "ln3_beta": zero})
        mats += [("cwq", d, d), ("cwk", d, d), ("cwv", d, d), ("cwo", d, d)]
    for name, n, k in mats:
        L[name] = random_block_weight(rng, wd, n, k, scale)
    for name, n in (("bq", d), ("bv", d), ("bo", d), ("b1", ff), ("b2", d)):
        L[name] = (0.01 * rng.standard_normal(n)).astype(np.float32)
    return L


def bench_frontend(ctx, hip, batch=16, n_mels=128, d=1280, reps=5):
    """Config 2's front end: log-mel of `batch` 30 s clips (128 mels) and the
    conv stem (conv1 128->1280, conv2 1280->1280 stride 2, GELU, + positions)
    on device-resident arrays. FLOPs: STFT GEMM 2*3000*402*400 and mel GEMM
    2*3000*128*201 per clip; stem 2*3000*1280*384 + 2*1500*1280*3840."""
    rng = np.random.default_rng(5)
    n_samples = 480000
    d_pcm = hip.DeviceBuffer.from_array(ctx, (0.1 * rng.standard_normal((batch, n_samples))).astype(np.float32))
    d_mel = hip.DeviceBuffer(ctx, batch * n_mels * 3000 * 4)
    enc = hip.Encoder(ctx, 8, d, 20, 5120, [], np.ones(d, np.float32), np.zeros(d, np.float32), batch * 1500)
    enc.set_stem(n_mels, 3000, (0.02 * rng.standard_normal((d, n_mels, 3))).astype(np.float32),
                 np.zeros(d, np.float32), (0.02 * rng.standard_normal((d, d, 3))).astype(np.float32),
                 np.zeros(d, np.float32), (0.02 * rng.standard_normal((1500, d))).astype(np.float32))
    d_out = hip.DeviceBuffer(ctx, batch * 1500 * d * 4)
    ctx.log_mel_dev(d_pcm, batch, n_samples, n_mels, d_mel)
    enc.encode_dev(batch, d_mel, d_out)
    ctx.synchronize()
    e0, e1, e2 = hip.Event(ctx), hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for _ in range(reps):
        ctx.log_mel_dev(d_pcm, batch, n_samples, n_mels, d_mel)
    e1.record()
    for _ in range(reps):
        enc.encode_dev(batch, d_mel, d_out)  # no blocks: stem + ln_post
    e2.record()
    mel_ms, stem_ms = e0.elapsed_ms(e1) / reps, e1.elapsed_ms(e2) / reps
    mel_flop = batch * (2 * 3000 * 402 * 400 + 2 * 3000 * n_mels * 201)
    stem_flop = batch * (2 * 3000 * d * n_mels * 3 + 2 * 1500 * d * d * 3)
    return {"batch": batch, "n_mels": n_mels, "log_mel_ms": round(mel_ms, 3),
            "log_mel_clips_per_s": round(batch / (mel_ms * 1e-3), 1),
            "log_mel_tflops": round(mel_flop / (mel_ms * 1e-3) / 1e12, 2),
            "stem_ms": round(stem_ms, 3), "stem_tflops": round(stem_flop / (stem_ms * 1e-3) / 1e12, 2)}


def bench_encoder(ctx, hip, batch, n_layer=32, d=1280, H=20, ff=5120, T=1500, reps=3):
    """Config 2: Whisper-large-v3-shaped encoder blocks (32 x d=1280, 20 heads,
    FFN 5120, Q8_0 random-init weights) over 1500 frames, batch 1 or 16: one
    forward of the device-resident encoder session on resident input."""
    rng = np.random.default_rng(2)
    layers = [whisper_layer(rng, 8, d, ff, 2e-4) for _ in range(n_layer)]
    enc = hip.Encoder(ctx, 8, d, H, ff, layers, np.ones(d, np.float32), np.zeros(d, np.float32), batch * T)
    del layers
    d_x = hip.DeviceBuffer.from_array(ctx, rng.standard_normal((batch, T, d), dtype=np.float32))
    d_o = hip.DeviceBuffer(ctx, batch * T * d * 4)
    enc.forward_dev(batch, T, d_x, d_o)
    ctx.synchronize()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for _ in range(reps):
        enc.forward_dev(batch, T, d_x, d_o)
    e1.record()
    ms = e0.elapsed_ms(e1) / reps
    hd = d // H
    flops = n_layer * batch * (2.0 * T * (4 * d * d + 2 * d * ff) + 4.0 * H * T * T * hd)
    del enc
    ctx.synchronize()
    return {"batch": batch, "layers": n_layer, "frames": T, "ms": round(ms, 3),
            "frames_per_s": round(batch * T / (ms * 1e-3), 1), "tflops": round(flops / (ms * 1e-3) / 1e12, 2)}


def bench_decoder(ctx, hip, n_stream=64, n_layer=32, d=1280, H=20, ff=5120, V=51866, n_text=448, n_audio=1500,
                  steps=5, max_prefix=442):
    """Config 3: batched Whisper-large-v3-shaped decoder step, 64 streams with
    prefixes U(1..max_prefix) already in the paged Q8_0 self-KV cache (16-token
    pages), cross-attention over 1500 encoder frames per stream, Q4_0
    random-init weights, tied logits over a 51866-token vocabulary, greedy
    argmax. Timed: `steps` whole batched steps on device arrays. The prefix
    ceiling leaves room for the timed steps: prefix + 1 + steps <= 448
    positions (n_text_ctx), so the last timed step reaches position 447."""
    rng = np.random.default_rng(3)
    layers = [whisper_layer(rng, 2, d, ff, 5e-3, decoder=True) for _ in range(n_layer)]
    tok = (0.02 * rng.standard_normal((V, d))).astype(np.float32)
    pos = (0.02 * rng.standard_normal((n_text, d))).astype(np.float32)
    dec = hip.Decoder(ctx, 2, d, H, ff, V, n_text, n_audio, n_stream, layers, tok, pos,
                      np.ones(d, np.float32), np.zeros(d, np.float32), block_size=16)
    del layers, tok
    # the page table a long-running server ends up with: the self-KV pages
    # handed out in a seeded random order rather than LIFO from an empty arena
    dec.set_free_order(rng.permutation(sum(dec.kv_pages())).astype(np.int32))
    d_enc = hip.DeviceBuffer.from_array(ctx, rng.standard_normal((n_audio, d), dtype=np.float32))
    for s in range(n_stream):
        dec.set_encoder_dev(s, d_enc)
    lens = rng.integers(1, max_prefix + 1, n_stream)
    cur = rng.integers(0, V, n_stream).astype(np.int32)
    for t in range(int(lens.max())):   # prefill the caches one decode step at a time
        live = np.nonzero(lens > t)[0].astype(np.int32)
        nxt = dec.step(live, cur[live], np.full(live.size, t, np.int32))
        cur[live] = nxt
    streams = hip.DeviceBuffer.from_array(ctx, np.arange(n_stream, dtype=np.int32))
    toks = hip.DeviceBuffer.from_array(ctx, cur)
    posb = [hip.DeviceBuffer.from_array(ctx, (lens + k).astype(np.int32)) for k in range(steps + 1)]
    nxt = hip.DeviceBuffer(ctx, n_stream * 4)
    dec.step_dev(n_stream, streams, toks, posb[0], nxt)   # warm-up (positions lens)
    ctx.synchronize()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for k in range(1, steps + 1):
        dec.step_dev(n_stream, streams, nxt, posb[k], toks)
        nxt, toks = toks, nxt
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    # the same steps again with the half-precision cross-attention reads (a
    # performance mode: K/V as fp16, half the step's largest byte stream);
    # replaying positions rewrites the same cache rows
    dec.set_cross_precision(hip.CrossPrecision.F16)
    dec.step_dev(n_stream, streams, toks, posb[0], nxt)
    ctx.synchronize()
    e0.record()
    for k in range(1, steps + 1):
        dec.step_dev(n_stream, streams, nxt, posb[k], toks)
        nxt, toks = toks, nxt
    e1.record()
    ms_f16 = e0.elapsed_ms(e1) / steps
    keys = int((lens + 1 + steps // 2).sum())
    # a step reads 8 of the 10 d x d linears per layer (q, k, v, o, cross q,
    # cross o; cross k / v are applied once per utterance) and fc1 / fc2
    w_bytes = n_layer * (6 * d * d + 2 * d * ff) * 18 // 32
    kv_bytes = keys * n_layer * 2 * (d + d // 32 * 2)
    # cross K and V: fp16 high part + one-byte low part per value
    cross_bytes = n_stream * n_layer * n_audio * d * 3 * 2
    emb_bytes = V * d * 4
    total = w_bytes + kv_bytes + cross_bytes + emb_bytes
    del dec
    ctx.synchronize()
    return {"streams": n_stream, "layers": n_layer, "vocab": V, "prefix_range": [1, max_prefix],
            "page_table": "shuffled (seeded free order)",
            "last_position": int(lens.max()) + steps,
            "ms_per_step": round(ms, 3), "tokens_per_s": round(n_stream / (ms * 1e-3), 1),
            "cross_f16_mode": {"ms_per_step": round(ms_f16, 3), "tokens_per_s": round(n_stream / (ms_f16 * 1e-3), 1)},
            "bytes_per_step": {"weights_q4_0": w_bytes, "self_kv_q8_0": kv_bytes, "cross_kv_f16_q7": cross_bytes,
                               "tied_embedding_f32": emb_bytes},
            "gbs": round(total / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(total / (ms * 1e-3) / 1e9 / PEAK["hbm_gbs"], 4)}


def q4k_scaled_weight(rng, n, k, d_hi=0x10, dmin_hi=0x0C):
    """Random Q4_K payload (the reference's random_blocks pattern) with the
    f16 d / dmin high bytes pinned to give weights of a few 0.01 (random-init
    scale), so a 24-layer residual stream stays well inside f32 and fp16."""
    b = rng.integers(0, 256, size=(n * (k // 256), 144), dtype=np.uint8)
    b[:, 1] = d_hi
    b[:, 3] = dmin_hi
    return b.reshape(-1)


def bench_text_decoder(ctx, hip, n_stream=32, n_layer=24, d=2048, hq=16, hkv=2, hd=128, ff=5632, V=32000,
                       n_ctx=4096, len_lo=512, len_hi=4096, steps=10):
    """Config 4: batched speech-LLM decode step, 32 streams whose histories
    (rows restored into the paged Q8_0 cache, 16-token pages) are U(512..4096)
    positions, 24 layers of Q4_K linears (d=2048, GQA 16/2 x 128, SwiGLU FFN
    5632), Q4_K LM head over 32000 tokens, greedy argmax; seeded token IDs.
    Timed: `steps` whole batched steps on device arrays."""
    rng = np.random.default_rng(44)
    layers = []
    for _ in range(n_layer):
        L = {"attn_norm_gamma": np.ones(d, np.float32), "ffn_norm_gamma": np.ones(d, np.float32)}
        for name, n, k in (("wq", hq * hd, d), ("wk", hkv * hd, d), ("wv", hkv * hd, d), ("wo", d, hq * hd),
                           ("w_gate", ff, d), ("w_up", ff, d), ("w_down", d, ff)):
            L[name] = q4k_scaled_weight(rng, n, k)
        layers.append(L)
    tok = (0.02 * rng.standard_normal((V, d))).astype(np.float32)
    head = q4k_scaled_weight(rng, V, d)
    dec = hip.TextDecoder(ctx, 12, d, hq, hkv, hd, ff, V, n_ctx, n_stream, layers, tok, np.ones(d, np.float32),
                          head, rope_base=1e6, rms_norm_eps=1e-5, block_size=16)
    del layers
    dec.set_free_order(rng.permutation(sum(dec.kv_pages())).astype(np.int32))   # shuffled page table
    lens = rng.integers(len_lo, len_hi - steps, n_stream)
    kk = rng.standard_normal((n_layer, int(lens.max()), hkv * hd), dtype=np.float32)
    vv = rng.standard_normal((n_layer, int(lens.max()), hkv * hd), dtype=np.float32)
    for s in range(n_stream):
        dec.kv_restore(s, kk[:, :lens[s]], vv[:, :lens[s]])
    del kk, vv
    streams = hip.DeviceBuffer.from_array(ctx, np.arange(n_stream, dtype=np.int32))
    toks = hip.DeviceBuffer.from_array(ctx, rng.integers(0, V, n_stream).astype(np.int32))
    posb = [hip.DeviceBuffer.from_array(ctx, (lens + k).astype(np.int32)) for k in range(steps + 1)]
    nxt = hip.DeviceBuffer(ctx, n_stream * 4)
    dec.step_dev(n_stream, streams, toks, posb[0], nxt)   # warm-up
    dec.status()
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for k in range(1, steps + 1):
        dec.step_dev(n_stream, streams, nxt, posb[k], toks)
        nxt, toks = toks, nxt
    e1.record()
    dec.status()
    ms = e0.elapsed_ms(e1) / steps
    keys = int((lens + 1 + steps // 2).sum())
    w_layer = sum(n * (k // 256) * 144 for (_, n, k) in Q4K_LAYER)
    w_bytes = n_layer * w_layer + V * (d // 256) * 144
    kv_bytes = keys * n_layer * 2 * (hkv * hd + hkv * hd // 32 * 2)
    total = w_bytes + kv_bytes
    del dec
    ctx.synchronize()
    return {"streams": n_stream, "layers": n_layer, "vocab": V, "context_range": [len_lo, len_hi],
            "page_table": "shuffled (seeded free order)",
            "mean_context": round(float(lens.mean()), 1), "ms_per_step": round(ms, 3),
            "tokens_per_s": round(n_stream / (ms * 1e-3), 1),
            "bytes_per_step": {"weights_q4_k": w_bytes, "kv_q8_0": kv_bytes},
            "gbs": round(total / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(total / (ms * 1e-3) / 1e9 / PEAK["hbm_gbs"], 4)}


def bench_logits(ctx, hip, n=64, V=51866, d=1280, reps=20):
    """Config 3 tail: tied logits over the Whisper vocabulary (f32 embedding
    [V, d], 265.6 MB) for 64 streams and the greedy argmax, as one fused pass
    (vk_logits_argmax + the partial merge) with and without the logits
    written, beside the unfused route (f32 GEMM into logits, then argmax)."""
    rng = np.random.default_rng(5)
    d_x = hip.DeviceBuffer.from_array(ctx, rng.standard_normal((n, d), dtype=np.float32))
    d_e = hip.DeviceBuffer.from_array(ctx, (0.02 * rng.standard_normal((V, d))).astype(np.float32))
    d_l = hip.DeviceBuffer(ctx, n * V * 4)
    d_n = hip.DeviceBuffer(ctx, n * 4)
    runs = {
        "fused": lambda: ctx.logits_argmax_dev(n, V, d, d_x, d_e, None, d_n),
        "fused_with_logits": lambda: ctx.logits_argmax_dev(n, V, d, d_x, d_e, d_l, d_n),
        "gemm_then_argmax": lambda: (ctx.gemm_f32_dev(n, V, d, d_x, d_e, d_l, b_trans=True),
                                     ctx.argmax_f32_dev(d_l, n, V, d_n)),
    }
    out = {"streams": n, "vocab": V, "d": d, "emb_bytes": V * d * 4, "flop": 2 * n * V * d}
    for name, fn in runs.items():
        fn()
        ctx.synchronize()
        e0, e1 = hip.Event(ctx), hip.Event(ctx)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        ms = e0.elapsed_ms(e1) / reps
        out[name] = {"us": round(ms * 1e3, 2), "emb_gbs": round(V * d * 4 / (ms * 1e-3) / 1e9, 1),
                     "tflops": round(2 * n * V * d / (ms * 1e-3) / 1e12, 2)}
    out["fused"]["frac_f32_mfma_peak"] = round(out["fused"]["tflops"] / PEAK["fp32_tflops"], 4)
    out["fused"]["frac_hbm"] = round(out["fused"]["emb_gbs"] / PEAK["hbm_gbs"], 4)
    for b in (d_x, d_e, d_l, d_n):
        b.free()
    return out


def bench_copy(ctx, hip, nbytes=1 << 30, reps=5):
    """Plain streaming copy of 1 GiB (4x the 256 MB MALL): the
    achievable-HBM reference and the rocprof byte-counter calibration kernel."""
    src = hip.DeviceBuffer(ctx, nbytes)
    dst = hip.DeviceBuffer(ctx, nbytes)
    ctx.copy_dev(dst, src, nbytes)
    e0, e1 = hip.Event(ctx), hip.Event(ctx)
    e0.record()
    for _ in range(reps):
        ctx.copy_dev(dst, src, nbytes)
    e1.record()
    ms = e0.elapsed_ms(e1) / reps
    return {"bytes": nbytes, "ms": round(ms, 4), "gbs": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def _cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _host():
    return f"{_cpu_model()}, {os.cpu_count()} logical cores"


def _threads():
    """Host threads for the reference's pooled f32 work (VOKRA_CPU_THREADS
    semantics: every core, pool.rs:340-355)."""
    return max(1, os.cpu_count() or 1)


def _pool_map(fn, items, threads):
    """Runs fn over items on `threads` host threads (the oracle's ctypes calls
    release the interpreter lock, so the calls run in parallel)."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=threads) as ex:
        return list(ex.map(fn, items))


def _sdpa_heads(orc, t_q, t_kv, hd, q, k, v, heads, threads, causal=False, off=0):
    """attention_from_kv_into's per-head work (whisper/nn.rs:209-325) with the
    heads spread over the pool, as the reference's per-head GEMMs run on it."""
    return _pool_map(lambda h: orc.sdpa_whisper(t_q, t_kv, 1, hd, q, k, v, causal=causal, q_pos_offset=off),
                     range(heads), threads)


def cpu_baseline_q8(a, wq, N, K, budget_s=10.0):
    """The reference CPU's route for a Q8_0 GEMM (vokra-backend-cpu has no
    fused Q8_0 GEMM): A4 dequantize_bytes of the weight, transposed to [k, n],
    then gemm_f32 row-parallel on every host thread (kv_quant/mod.rs:307-359,
    kernels/mod.rs:305-325, scalar.rs:41-72, pool.rs:340-355), on as many
    activation rows as fit the budget; the weight dequant is inside every
    timed call. The single-thread route of dequant_gemv_scalar, one call per
    activation row (dequant_gemm.rs:49-98), is timed beside it."""
    from oracle import oracle as orc
    orc.lib()
    thr = _threads()
    rows, t_total, chunk = 0, 0.0, 64
    while rows < a.shape[0] and t_total < budget_s:
        blk = a[rows:rows + chunk]
        t0 = time.perf_counter()
        wt = orc.dequantize_bytes(orc.Q8_0, wq).reshape(N, K).T.copy()
        orc.gemm_f32(blk.shape[0], N, K, blk, wt, threads=thr)
        t_total += time.perf_counter() - t0
        rows += blk.shape[0]
    pooled = 2.0 * rows * N * K / t_total / 1e12
    # one thread, one dequant_gemv_scalar call per activation row
    g_rows, g_total = 0, 0.0
    while g_rows < 4 or (g_total < budget_s / 3 and g_rows < a.shape[0]):
        t0 = time.perf_counter()
        orc.dequant_gemv_scalar(orc.Q8_0, wq, N, K // 32, a[g_rows])
        g_total += time.perf_counter() - t0
        g_rows += 1
    return ({"value": pooled, "unit": "TOPS", "cores": thr, "kind": "port",
             "sample": f"{rows} of 1500 activation rows x N=5120, K=1280: dequantize_bytes (A4) + gemm_f32 on "
                       f"{thr} threads (vo_gemm_f32_mt), the weight dequant in every call; {t_total:.1f} s on "
                       f"{_host()}"},
            {"dequant_gemv_scalar_per_row": {"value": 2.0 * g_rows * N * K / g_total / 1e12, "unit": "TOPS",
                                             "cores": 1, "kind": "port",
                                             "sample": f"{g_rows} activation rows, one dequant_gemv_scalar call each "
                                                       f"(vo_dequant_gemv_scalar), {g_total:.1f} s on {_host()}"}})


def _per_call(fn, budget_s):
    """Median seconds per call of fn: one warm-up, then calls until the budget
    is spent (at least three)."""
    fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 50):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)


def cpu_baselines(budget_s=3.0):
    """Each leg's CPU column: the oracle's restatement of the reference's CPU
    route (oracle/vokra_oracle.c, the vokra-backend-cpu scalar tier) timed on
    this host on a bounded sample of the leg's workload, with the reference's
    threading: the block GEMV (dequant_gemv_scalar) and the K-quant INT8 route
    single-threaded, every f32 GEMM and the attention heads on the pool (all
    host threads). Values are in the leg's own unit."""
    from oracle import oracle as orc
    orc.lib()
    rng = np.random.default_rng(5)
    host = _host()
    thr = _threads()
    out = {}

    # Q4_0 GEMV (dequant_gemv_scalar, 1 thread): one activation vector, both config-1 widths
    gemv = []
    for n in (5120, 1280):
        k = 1280
        wq = rng.integers(0, 256, n * (k // 32) * 18, dtype=np.uint8)
        wq.reshape(-1, 18)[:, 0:2] = np.frombuffer(np.float16(0.002).tobytes(), np.uint8)
        x = rng.standard_normal(k, dtype=np.float32)
        sec, reps = _per_call(lambda: orc.dequant_gemv_scalar(1, wq, n, k // 32, x), budget_s / 2)
        nbytes = n * (k // 32) * 18 + k * 4 + n * 4
        gemv.append({"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "us_per_linear": round(sec * 1e6, 1),
                     "cores": 1, "kind": "port",
                     "sample": f"M=1 N={n} K={k}, dequant_gemv_scalar (vo_dequant_gemv_scalar), median of {reps} on "
                               f"{host}"})
    out["q4_0_gemv_streamed"] = gemv
    # Q4_K decode layer (kquant_gemm_i8, 1 thread: the reference does not pool it)
    total = 0.0
    for (_, n, k) in Q4K_LAYER:
        w = q4k_random_weight(rng, n, k)
        a = rng.standard_normal((32, k), dtype=np.float32)
        sec, _ = _per_call(lambda: orc.kquant_gemm_i8(12, n, k, 32, w, a), budget_s / 7)
        total += sec
    nbytes = sum(n * (k // 256) * 144 + 32 * k * 4 + 32 * n * 4 for (_, n, k) in Q4K_LAYER)
    out["q4_k_decode_layer_m32"] = {"value": round(nbytes / total / 1e9, 3), "unit": "GB/s",
                                    "us_per_layer": round(total * 1e6, 1), "cores": 1, "kind": "port",
                                    "sample": f"one config-4 layer (7 linears) at M=32 through kquant_gemm_i8 "
                                              f"(vo_kquant_gemm_i8) on {host}"}
    # fused SDPA config 1: the 20 heads of attention_from_kv_into on the pool
    T, hd = 1500, 64
    q, kk, v = (rng.standard_normal((T, hd), dtype=np.float32) for _ in range(3))
    sec, reps = _per_call(lambda: _sdpa_heads(orc, T, T, hd, q, kk, v, 20, thr), budget_s)
    flops = 4.0 * 20 * T * T * hd
    out["sdpa_config1"] = {"value": round(flops / sec / 1e12, 4), "unit": "TFLOP/s",
                           "ms_per_op": round(sec * 1e3, 1), "cores": min(thr, 20), "kind": "port",
                           "sample": f"all 20 heads (1500 x 1500 x 64, vo_sdpa_whisper per head) on {min(thr, 20)} "
                                     f"threads; median of {reps} on {host}"}
    # paged decode attention: config 3 (64 streams x 20 heads x 64, 224 keys each, the U(1..448) mean)
    # and config 4 (one stream, GQA 16/2 x 128, 2300 keys); dequantized rows, heads / streams on the pool
    t3 = 224
    K3 = rng.standard_normal((t3, 1280), dtype=np.float32)
    V3 = rng.standard_normal((t3, 1280), dtype=np.float32)
    q3 = rng.standard_normal((1, 1280), dtype=np.float32)
    sec, reps = _per_call(lambda: _pool_map(lambda s: orc.sdpa_whisper(1, t3, 20, 64, q3, K3, V3, causal=True,
                                                                       q_pos_offset=t3 - 1), range(64), thr),
                          budget_s / 2)
    nbytes = 64 * t3 * 2 * (1280 + 80)
    out["paged_attn_config3"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s",
                                 "us_per_layer": round(sec * 1e6, 1), "cores": thr, "kind": "port",
                                 "sample": f"64 streams x 224 keys, 20 heads x 64 over dequantized rows "
                                           f"(vo_sdpa_whisper per stream), streams on {thr} threads; median of "
                                           f"{reps} on {host}"}
    t_kv = 2300
    Kc = rng.standard_normal((t_kv, 256), dtype=np.float32)
    Vc = rng.standard_normal((t_kv, 256), dtype=np.float32)
    qg = rng.standard_normal((1, 2048), dtype=np.float32)
    sec, reps = _per_call(lambda: orc.gqa_attention(1, t_kv, 16, 2, 128, qg, Kc, Vc, 0.0884, t_kv - 1), budget_s / 2)
    nbytes = t_kv * 2 * (256 + 16)
    out["paged_attn_config4"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s",
                                 "us_per_stream": round(sec * 1e6, 1), "cores": 1, "kind": "port",
                                 "sample": f"one stream, 2300 keys, GQA 16/2 x 128 over dequantized rows "
                                           f"(vo_gqa_attention, text_decoder.rs:1302-1360 is a scalar loop), "
                                           f"median of {reps} on {host}"}
    # Whisper-large encoder block (config 2) on 96 of 1500 rows: Q8_0 linears through the
    # reference route (A4 dequant + gemm_f32 on the pool), attention heads on the pool
    rows, d, ff = 96, 1280, 5120
    a = rng.standard_normal((rows, d), dtype=np.float32)
    wdd = [orc.dequantize_bytes(orc.Q8_0, random_block_weight(rng, 8, d, d, 0.02)).reshape(d, d).T.copy()
           for _ in range(4)]
    w8f = random_block_weight(rng, 8, ff, d, 0.02)
    w8b = random_block_weight(rng, 8, d, ff, 0.02)
    af = rng.standard_normal((rows, ff), dtype=np.float32)
    qh = rng.standard_normal((rows, 64), dtype=np.float32)

    def enc_sample():
        for w in wdd:
            orc.gemm_f32(rows, d, d, a, w, threads=thr)
        orc.gemm_f32(rows, ff, d, a, orc.dequantize_bytes(orc.Q8_0, w8f).reshape(ff, d).T.copy(), threads=thr)
        orc.gemm_f32(rows, d, ff, af, orc.dequantize_bytes(orc.Q8_0, w8b).reshape(d, ff).T.copy(), threads=thr)
        _sdpa_heads(orc, rows, T, 64, qh, kk, v, 20, thr)
    sec, reps = _per_call(enc_sample, budget_s)
    per_block = sec * (1500 / rows)
    flops_block = 2 * 1500 * (4 * d * d + 2 * d * ff) + 4 * 20 * 1500 * 1500 * 64
    enc = {"value": round(flops_block / per_block / 1e12, 4), "unit": "TFLOP/s",
           "ms_per_utterance": round(per_block * 32 * 1e3, 0), "cores": thr, "kind": "port",
           "sample": f"one block for {rows} of 1500 rows (Q8_0 linears as dequantize_bytes + gemm_f32 on {thr} "
                     f"threads, 20 attention heads on the pool), scaled to 1500 rows x 32 blocks; an utterance "
                     f"batch runs one utterance after another (batch 16 = 16x); median of {reps} on {host}"}
    out["encoder_config2"] = [enc, dict(enc, sample=enc["sample"] + "; batch 16 line: same per-utterance rate")]
    # Whisper decoder step (config 3): one stream, one layer's 8 step linears (dequant_gemv_scalar,
    # 1 thread) + self / cross attention (heads on the pool) + the tied logits (gemm_f32 on the pool)
    Vv = 51866
    a1 = rng.standard_normal((1, d), dtype=np.float32)
    f1 = rng.standard_normal(ff, dtype=np.float32)
    w4 = random_block_weight(rng, 2, d, d, 0.02)
    w4f = random_block_weight(rng, 2, ff, d, 0.02)
    w4b = random_block_weight(rng, 2, d, ff, 0.02)
    ck = rng.standard_normal((1500, d), dtype=np.float32)
    sk = rng.standard_normal((224, d), dtype=np.float32)
    emb = rng.standard_normal((Vv, d), dtype=np.float32)
    embt = emb.T.copy()
    q64, sk64, ck64 = (np.ascontiguousarray(x[:, :64]) for x in (a1, sk, ck))

    def dec_layer():
        for _ in range(6):
            orc.dequant_gemv_scalar(1, w4, d, d // 32, a1[0])
        orc.dequant_gemv_scalar(1, w4f, ff, d // 32, a1[0])
        orc.dequant_gemv_scalar(1, w4b, d, ff // 32, f1)
        _pool_map(lambda h: orc.sdpa_whisper(1, 224, 1, 64, q64, sk64, sk64, causal=True, q_pos_offset=223),
                  range(20), thr)
        _pool_map(lambda h: orc.sdpa_whisper(1, 1500, 1, 64, q64, ck64, ck64), range(20), thr)
    sec_l, _ = _per_call(dec_layer, budget_s / 2)
    sec_g, _ = _per_call(lambda: orc.gemm_f32(1, Vv, d, a1, embt, threads=thr), budget_s / 2)
    step = 32 * sec_l + sec_g
    out["decoder_step_config3"] = {"value": round(1.0 / step, 2), "unit": "tokens/s",
                                   "ms_per_stream_step": round(step * 1e3, 1), "cores": thr, "kind": "port",
                                   "sample": f"one stream: one layer (8 Q4_0 step linears through "
                                             f"dequant_gemv_scalar, 1 thread; self-attention over 224 keys and "
                                             f"cross over 1500, 20 heads on {thr} threads) x 32, plus the tied "
                                             f"logits (gemm_f32 on {thr} threads); the reference has no batch "
                                             f"axis, so 64 streams take 64x; on {host}"}
    # speech-LLM step (config 4): one stream, one layer's 7 Q4_K linears + GQA over 2300 keys
    def td_layer():
        for (_, n, k) in Q4K_LAYER:
            orc.kquant_gemm_i8(12, n, k, 1, q4k_w[(n, k)], x4[k])
        orc.gqa_attention(1, t_kv, 16, 2, 128, qg, Kc, Vc, 0.0884, t_kv - 1)
    q4k_w = {(n, k): q4k_random_weight(rng, n, k) for (_, n, k) in Q4K_LAYER}
    x4 = {k: rng.standard_normal((1, k), dtype=np.float32) for k in (2048, 5632)}
    head = q4k_random_weight(rng, 32000, 2048)
    sec_l, _ = _per_call(td_layer, budget_s / 2)
    sec_h, _ = _per_call(lambda: orc.kquant_gemm_i8(12, 32000, 2048, 1, head, x4[2048]), budget_s / 2)
    step = 24 * sec_l + sec_h
    out["text_decoder_step_config4"] = {"value": round(1.0 / step, 2), "unit": "tokens/s",
                                        "ms_per_stream_step": round(step * 1e3, 1), "cores": 1, "kind": "port",
                                        "sample": f"one stream: one layer (7 Q4_K linears via kquant_gemm_i8, GQA "
                                                  f"over 2300 keys; the reference runs both single-threaded) x 24 "
                                                  f"plus the Q4_K LM head; on {host}"}
    # log-mel front end (one 30 s clip, 128 mels; the oracle's f64 DFT), clips on the pool
    pcm = rng.standard_normal(480000, dtype=np.float32) * 0.1
    sec, reps = _per_call(lambda: _pool_map(lambda i: orc.log_mel(pcm, 128), range(min(thr, 16)), thr), budget_s)
    out["frontend_config2_batch16"] = {"value": round(min(thr, 16) / sec, 2), "unit": "clips/s",
                                       "cores": min(thr, 16), "kind": "port",
                                       "sample": f"log-mel of {min(thr, 16)} 30 s clips, 128 mels (vo_log_mel, f64 "
                                                 f"DFT), one clip per thread; median of {reps} on {host}"}
    # tied logits + argmax (config 3): gemm_f32 over the embedding on every core
    xs = rng.standard_normal((8, d), dtype=np.float32)
    sec, reps = _per_call(lambda: orc.gemm_f32(8, Vv, d, xs, embt, threads=thr), budget_s)
    out["logits_argmax_config3"] = {"value": round(2.0 * 8 * Vv * d / sec / 1e12, 4), "unit": "TFLOP/s",
                                    "cores": thr, "kind": "port",
                                    "sample": f"8 of 64 stream rows x 51866 x 1280 (vo_gemm_f32_mt, {thr} threads), "
                                              f"median of {reps} on {host}"}
    return out


def load_traffic(name):
    """HBM bytes per launch of `name`, from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes recorded in profiles/traffic.json (calibrated on a 1 GiB copy)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        entry = json.load(open(path)).get(name)
        return None if entry is None else entry["bytes_per_launch"]
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default=None,
                    help="comma list of single legs to run, one JSON line each (for profiling): "
                         "gemm, gemm_pow2, copy, gemv, q4k, sdpa, paged, encoder, decoder, textdec, frontend, "
                         "logits, decoder_l2, textdec_l2 (2-layer steps for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(every configured workload fits one MI355X; the design shards decode batches by "
              "stream and GEMMs by output column, with no exchange)", file=sys.stderr)
        return 2

    from vokra_amd import hip
    ctx = hip.HipContext(0)
    if args.only:
        legs = {
            "gemm": lambda: bench_q8_gemm(ctx, hip, args.steps, args.warmup, hip.ActQuant.AMAX127),
            "gemm_pow2": lambda: bench_q8_gemm(ctx, hip, args.steps, args.warmup, hip.ActQuant.POW2),
            "copy": lambda: bench_copy(ctx, hip),
            "gemv": lambda: [bench_q4_gemv(ctx, hip, n) for n in (5120, 1280)],
            "q4k": lambda: bench_q4k_decode(ctx, hip),
            "sdpa": lambda: bench_sdpa(ctx, hip),
            "paged": lambda: [bench_paged_attn(ctx, hip, 64, 20, 64, 20, 1, 448, 448),
                              bench_paged_attn(ctx, hip, 32, 2, 128, 16, 512, 4096, 4096)],
            "encoder": lambda: [bench_encoder(ctx, hip, 1), bench_encoder(ctx, hip, 16)],
            "decoder": lambda: bench_decoder(ctx, hip),
            "textdec": lambda: bench_text_decoder(ctx, hip),
            # the two steps' per-layer kernels at their full shapes over 2
            # layers and short prefixes: a fast leg for counter runs (each
            # kernel's dispatches are those of the full legs)
            "decoder_l2": lambda: bench_decoder(ctx, hip, n_layer=2, max_prefix=16),
            "textdec_l2": lambda: bench_text_decoder(ctx, hip, n_layer=2),
            "frontend": lambda: bench_frontend(ctx, hip),
            "logits": lambda: bench_logits(ctx, hip),
        }
        for name in args.only.split(","):
            res = legs[name]()
            if isinstance(res, dict):
                res = {k: v for k, v in res.items() if not isinstance(v, np.ndarray)}
            print(json.dumps({"leg": name, "result": res}), flush=True)
        ctx.close()
        return 0
    main_run = bench_q8_gemm(ctx, hip, args.steps, args.warmup, hip.ActQuant.AMAX127)
    pow2_run = bench_q8_gemm(ctx, hip, args.steps, args.warmup, hip.ActQuant.POW2)
    copy_run = bench_copy(ctx, hip)
    gemv_runs = [bench_q4_gemv(ctx, hip, n) for n in (5120, 1280)]
    q4k_run = bench_q4k_decode(ctx, hip)
    sdpa_run = bench_sdpa(ctx, hip)
    paged_runs = [bench_paged_attn(ctx, hip, 64, 20, 64, 20, 1, 448, 448),
                  bench_paged_attn(ctx, hip, 32, 2, 128, 16, 512, 4096, 4096)]
    encoder_runs = [bench_encoder(ctx, hip, 1), bench_encoder(ctx, hip, 16)]
    frontend_run = bench_frontend(ctx, hip)
    logits_run = bench_logits(ctx, hip)
    decoder_run = bench_decoder(ctx, hip)
    textdec_run = bench_text_decoder(ctx, hip)

    M, N, K = main_run["M"], main_run["N"], main_run["K"]
    achieved = main_run["gemm_tops"]
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK["int8_tops"],
                "unit": "TFLOP/s", "frac": round(achieved / PEAK["int8_tops"], 4),
                "traffic": load_traffic("vk_gemm_qblock")}
    cpu, cpu_routes = None, None
    legs_cpu = {}
    if not args.no_cpu_baseline:
        cpu, cpu_routes = cpu_baseline_q8(main_run["a"], main_run["wq"], N, K)
        legs_cpu = cpu_baselines()
    line = {
        "metric": METRIC,
        "value": round(main_run["tops"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_run["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights packed to Q8_0 on the device)",
        "config": {"workload": "Q8_0 gemm_q_f32 M=1500 K=1280 N=5120 (Whisper-large-v3 linear, config 1)",
                   "act_quant": "amax127", "global_batch": M, "parallelism": "single-gpu"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": {
            "hbm_copy_reference": copy_run,
            "q4_0_gemv_streamed": gemv_runs,
            "q4_k_decode_layer_m32": q4k_run,
            "sdpa_config1": sdpa_run,
            "paged_attn_config3_config4": paged_runs,
            "encoder_config2": encoder_runs,
            "frontend_config2_batch16": frontend_run,
            "logits_argmax_config3": logits_run,
            "decoder_step_config3": decoder_run,
            "text_decoder_step_config4": textdec_run,
            "cpu_q8_gemm_other_routes": cpu_routes,
            "gemm_kernel_ms": round(main_run["gemm_ms"], 4),
            "eager_step_ms": round(main_run["eager_ms"], 4),
            "gemm_frac_of_bf16_mfma_peak": round(achieved / PEAK["bf16_tflops"], 4),
            "pow2_act": {"tops": round(pow2_run["tops"], 2), "gemm_tops": round(pow2_run["gemm_tops"], 2),
                         "gemm_ms": round(pow2_run["gemm_ms"], 4),
                         "frac_int8_peak": round(pow2_run["gemm_tops"] / PEAK["int8_tops"], 4)},
        },
    }
    for leg, base in legs_cpu.items():
        key = "paged_attn_config3_config4" if leg.startswith("paged_attn_config") else leg
        entry = line["extra"].get(key)
        if isinstance(entry, dict):
            entry["cpu_baseline"] = base
        elif isinstance(entry, list) and entry:
            if isinstance(base, list):   # one baseline per line (GEMV widths, encoder batches)
                for e, b in zip(entry, base):
                    e["cpu_baseline"] = b
            else:                        # the paged lines: config 3 first, config 4 last
                entry[0 if leg == "paged_attn_config3" else -1]["cpu_baseline"] = base
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
