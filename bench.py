#!/usr/bin/env python3
"""Encoder-attention step benchmark of the paged K/V-cache hot path on one MI355X.

A step = for every active stream of the batch and every layer: append the
chunk's K/V frames to the stream's pages, rel-pos attention of the chunk over
the stream's window read from its pages, sliding-window eviction and page
allocation on the host pool, streaming masks and state advance
(parakeet/engine/model_runner.py:254-304 minus the projections).

Default workload (the headline): large-model shape, 24 layers, d_model 1024,
8 heads x 128, bf16, a pool of 256 stream slots at 90% steady occupancy with
continuous arrivals/departures (lifetimes U(2, 30) s at 80 ms/frame), page size
16 frames, left context 70, 2 frames per step.  Inputs are seeded synthetic
tensors resident in HBM before timing.

The default run then adds, each under its own key with its roofline and CPU
baseline: the large model's own 14-frame chunk (``large_t14``), the small shape
at 64 streams (``small_64streams``), the fragmentation stress at 1024 streams
(``frag_1024streams``), the fp32 plumbing case of 4 streams and one layer
(``plumbing_4streams``) and the end-to-end pcm16 -> tokens step at 128 streams
of the small model (``e2e_pcm16_128streams``) and of the large one (128 mels,
24 layers, 14 frames a step, 2-layer predictor: ``e2e_pcm16_large_128streams``);
and, under ``concurrent_streams.measured_max``, a timed run at the largest batch
the GPU holds at the headline shape.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "parakeet-streaming_amd"))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FRAME_SECONDS = 0.08  # audio per encoder frame (10 ms hop x 8x subsampling)

CONFIGS = {
    "large": dict(shape="LARGE_BF16", slots=256, occupancy=0.9, durations=("uniform", 2.0, 30.0), shuffle=False, seed=3),
    "large-t14": dict(shape="LARGE_BF16_T14", slots=256, occupancy=0.9, durations=("uniform", 2.0, 30.0), shuffle=False, seed=3),
    "small": dict(shape="SMALL_FP16", slots=64, occupancy=1.0, durations=("uniform", 2.0, 30.0), shuffle=False, seed=1),
    "frag": dict(shape="SMALL_FP16", slots=1024, occupancy=1.0, durations=("loguniform", 1.0, 60.0), shuffle=True, seed=4),
    "plumbing": dict(shape="SMALL_FP32", slots=4, occupancy=1.0, durations=("uniform", 1e9, 1e9), shuffle=False, seed=0),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_runner(cfg, device, rows_per_lane=0):
    import numpy as np
    import torch

    from parakeet_amd import synth
    from parakeet_amd.pool import pages_per_slot
    from parakeet_amd.step import AttentionStep

    shape = getattr(synth, cfg["shape"])
    slots = cfg["slots"]
    seed = cfg["seed"]
    qkv = [synth.qkv_frames(slots, shape, device, seed=seed * 1000 + layer) for layer in range(shape.layers)]
    pos, bu, bv = synth.relpos_inputs(shape, device, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    bias_u = [(torch.randn(shape.heads, shape.head_dim, generator=g) * 0.02).to(shape.dtype).to(device) for _ in range(shape.layers)]
    bias_v = [(torch.randn(shape.heads, shape.head_dim, generator=g) * 0.02).to(shape.dtype).to(device) for _ in range(shape.layers)]
    del bu, bv
    order = None
    if cfg["shuffle"]:
        n = slots * pages_per_slot(shape.left, shape.chunk, shape.page_size)
        order = np.random.default_rng(seed).permutation(n)
    runner = AttentionStep(shape, slots, device, qkv, pos, bias_u, bias_v, page_order=order, rows_per_lane=rows_per_lane)
    churn = synth.Churn(num_slots=slots, chunk=shape.chunk, occupancy=cfg["occupancy"], durations=cfg["durations"], seed=seed)
    return shape, runner, churn


def churn_step(runner, churn, events=None, graph=False) -> int:
    import numpy as np

    departed, _arrived = churn.step()
    runner.reset_slots(departed)
    active = np.asarray(churn.active(), dtype=np.int32)
    runner.step(active, events, graph=graph)
    return int(active.shape[0])


TRAFFIC_SUMMARY = {
    "large": os.path.join(HERE, "profiles", "relpos_attn_large_bf16_230streams_hbm_counters.md"),
    "large-t14": os.path.join(HERE, "profiles", "relpos_attn_chunk_large_bf16_t14_230streams.md"),
    "small": os.path.join(HERE, "profiles", "relpos_attn_small_fp16_64streams.md"),
    "frag": os.path.join(HERE, "profiles", "relpos_attn_frag_fp16_1024streams.md"),
}


def measured_traffic(config_name: str, avg_streams: float):
    """HBM bytes per launch of the attention kernel on this workload, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), when
    that summary covers the same configuration and batch; None otherwise."""
    import re

    path = TRAFFIC_SUMMARY.get(config_name)
    if path is None or not os.path.exists(path):
        return None
    txt = open(path).read()
    m = re.search(r"^traffic_bytes_per_launch: (\d+)$", txt, re.M)
    n = re.search(r"^traffic_streams: (\d+)$", txt, re.M)
    if not m or not n or abs(avg_streams - int(n.group(1))) > 0.5:
        return None
    return int(m.group(1))


def copy_probe(megabytes: int, reps: int) -> dict:
    """A plain device copy of known size (reads and writes `megabytes` MiB per
    launch): the calibration run for the HBM byte counters, and the ceiling of
    one launch that moves the same bytes as an attention launch.  The copies
    cycle over enough buffer pairs (>= 1 GiB of sources) that the reads come
    from HBM, not from the 256 MB last-level cache; each copy is timed with
    HIP events on the launch stream."""
    import torch

    n = megabytes << 20
    pairs = max(2, -(-1024 // max(1, megabytes)))
    src = [torch.ones(n // 2, dtype=torch.bfloat16, device="cuda:0") for _ in range(pairs)]
    dst = [torch.empty_like(s) for s in src]
    for i in range(pairs):  # warm
        dst[i].copy_(src[i])
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    for r in range(reps):
        ev[r][0].record()
        dst[r % pairs].copy_(src[r % pairs])
        ev[r][1].record()
    torch.cuda.synchronize()
    us = 1000.0 * sum(a.elapsed_time(b) for a, b in ev) / reps
    return {
        "copy_probe_bytes_read": n,
        "copy_probe_bytes_written": n,
        "launches": reps,
        "avg_us": round(us, 3),
        "gbs": round(2 * n / (us * 1e-6) / 1e9, 1),
        "frac_of_peak": round(2 * n / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
    }


def cpu_baseline(shape, streams: int, budget_s: float, seed: int) -> dict:
    """The reference's dense fp32 path (oracle/dense_path.py) on the host cores,
    bounded to about ``budget_s`` seconds."""
    import torch

    from oracle.dense_path import DenseStatePool
    from parakeet_amd import synth

    cores = len(os.sched_getaffinity(0))  # every core of the affinity mask
    torch.set_num_threads(cores)
    T, D = shape.chunk, shape.d_model
    g = torch.Generator().manual_seed(seed)
    qkv = [torch.randn(streams, T, 3 * D, generator=g) for _ in range(shape.layers)]
    w = torch.randn(D, D, generator=g) / math.sqrt(D)
    pos = synth.sinusoid_slice(D, shape.left, T) @ w.T
    bu = torch.randn(shape.heads, shape.head_dim, generator=g) * 0.02
    bv = torch.randn(shape.heads, shape.head_dim, generator=g) * 0.02
    pool = DenseStatePool(streams, shape.layers, shape.left, shape.right, D)
    slots = list(range(streams))
    with torch.inference_mode():
        pool.step(slots, qkv, pos, bu, bv, shape.heads)  # untimed first step
        n = 0
        t0 = time.perf_counter()
        while True:
            pool.step(slots, qkv, pos, bu, bv, shape.heads)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s and n >= 2:
                break
    return {
        "value": round(n / el, 4),
        "unit": "steps/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"{n} steps x {streams} streams x {shape.layers} layers, d_model {D}, {T} frames a step, fp32 dense "
            "shift-buffer path (pack/unpack index_select/index_copy_, per-stream mask loop, clone+copy shift, "
            f"torch SDPA) in {el:.1f} s on {cores} threads, every core of the affinity mask"
        ),
        "ms_per_step": round(1000.0 * el / n, 2),
    }


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16

# pcm16 -> tokens models (config.py:5-31): mels, d_model, heads, layers, conv
# kernel, left / right context, subsampling channels, dtype, vocabulary,
# predictor layers; the first and the next pcm chunks (samples, model_runner.py:53-56)
# and the per-slot sample and mel rings that hold them; the bias added to the
# random-init joint's blank logit, so that frames end on blank or on tokens
E2E_MODELS = {
    "small": dict(n_mels=80, D=512, H=8, layers=17, K=9, left=70, right=1, C=256, dtype="fp16", vocab=1026,
                  pred_layers=1, first=1440, chunk=2560, ring=8192, mel_rows=64, blank_bias=3.0),
    "large": dict(n_mels=128, D=1024, H=8, layers=24, K=9, left=70, right=13, C=256, dtype="bf16", vocab=1024,
                  pred_layers=2, first=16800, chunk=17920, ring=32768, mel_rows=256, blank_bias=3.5),
}


def synth_pcm(streams: int, n: int, seed: int):
    """int16 pcm per stream: 3 sinusoids of random frequency (100-4000 Hz),
    amplitude and phase, plus Gaussian noise at 20 dB SNR."""
    import numpy as np

    rng = np.random.default_rng(seed)
    t = np.arange(n, dtype=np.float64) / 16000.0
    out = np.empty((streams, n), dtype=np.int16)
    for b in range(streams):
        f = rng.uniform(100.0, 4000.0, 3)
        a = rng.uniform(0.05, 0.3, 3)
        ph = rng.uniform(0.0, 2 * np.pi, 3)
        sig = (a[:, None] * np.sin(2 * np.pi * f[:, None] * t[None, :] + ph[:, None])).sum(0)
        sig += rng.standard_normal(n) * np.sqrt(np.mean(sig**2) / 100.0)
        out[b] = np.clip(np.round(sig * 32767.0), -32768, 32767).astype(np.int16)
    return out


def _graph_time_us(fn, device, reps: int = 20, inner: int = 10) -> float:
    """Average time of the launches ``fn`` makes: ``inner`` calls recorded in one
    HIP graph, replayed ``reps`` times, so neither the host's launch cost nor the
    graph's own launch shows in the per-call time."""
    import torch

    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        fn()  # warm outside the capture
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(inner):
            fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return 1000.0 * a.elapsed_time(b) / (reps * inner)


def front_end_cpu_baseline(sub_sd: dict, budget_s: float, seed: int, n_mels: int = 80, first: int = 1440,
                           chunk: int = 2560) -> dict:
    """The oracle's per-stream pre-encode (FeatureExtractor.push + ConvSubsampling
    on the [cache ; new] window + drop, model_runner.py:181-252) on one host core,
    on ``chunk``-sample chunks of one stream after a ``first``-sample one, for
    about ``budget_s`` seconds (at least two chunks)."""
    import numpy as np

    from oracle import frontend as ofe

    from threadpoolctl import threadpool_limits

    p = ofe.FeParams(n_mels=n_mels)
    st = ofe.PreEncodeState(ofe.FeState(p, noise_id=1, seed=1), sub_sd, store_dtype=None)
    n_chunks = max(2, min(400, int(400 * 2560 / chunk)))
    pcm = synth_pcm(1, first + chunk * n_chunks, seed)[0].astype(np.float32) / 32768.0
    with threadpool_limits(limits=1):  # one core, BLAS included
        st.push(pcm[:first])
        pos, chunks, t0 = first, 0, time.perf_counter()
        while (time.perf_counter() - t0 < budget_s or chunks < 2) and pos + chunk <= len(pcm):
            st.push(pcm[pos : pos + chunk])
            pos += chunk
            chunks += 1
        el = time.perf_counter() - t0
    return {"chunks_per_s": chunks / el, "chunks": chunks, "seconds": el}


def decode_cpu_baseline(pred, joint, vocab: int, budget_s: float, streams: int, frames: int = 2,
                        layers: int = 1) -> dict:
    """The oracle's greedy decoding (float64 numpy, one host core) of one stream
    on ``frames``-frame steps, for about ``budget_s`` seconds, scaled to
    ``streams`` streams."""
    import numpy as np
    import torch

    from oracle import rnnt
    from threadpoolctl import threadpool_limits

    P = rnnt.RnntParams(pred.state_dict(), joint.state_dict(), layers)
    sd = rnnt.StreamDecoder(P, vocab)
    g = np.random.default_rng(13)
    n, toks, t0 = 0, 0, time.perf_counter()
    with threadpool_limits(limits=1):
        while time.perf_counter() - t0 < budget_s:
            toks += len(sd.decode(g.standard_normal((frames, P.w_enc.shape[1]))))
            n += 1
    el = time.perf_counter() - t0
    return {
        "value": round(n / el / streams, 4),
        "unit": f"decode steps/s ({streams} streams x {frames} frames)",
        "cores": 1,
        "kind": "port",
        "sample": f"{n} {frames}-frame steps of one stream through the oracle's greedy loop (float64 numpy), "
        f"{toks} tokens, in {el:.1f} s, scaled to {streams} streams per step",
    }


def encoder_cpu_baseline(enc, budget_s: float, layers: int, heads: int, left: int, right: int, kernel: int,
                         d_model: int) -> dict:
    """The oracle's streaming encoder step (oracle/encoder.py: float64 numpy,
    encoder.py:229-267 with dense caches) on one stream and one host core, on
    random subsampled frames, for about ``budget_s`` seconds."""
    import numpy as np

    from oracle import encoder as oe
    from oracle import relpos
    from threadpoolctl import threadpool_limits

    sd = {k: v.detach().double().cpu().numpy() for k, v in enc.state_dict().items()}
    D, T = d_model, right + 1
    pe = relpos.sinusoid_table(5000, D).astype(np.float64)
    st = oe.EncoderState(1, layers, left, right, D, kernel)
    g = np.random.default_rng(14)
    n, t0 = 0, time.perf_counter()
    with threadpool_limits(limits=1):
        while time.perf_counter() - t0 < budget_s or n < 2:
            oe.encoder_step(g.standard_normal((1, T, D)), sd, st, np.full(1, T), layers, heads, pe)
            n += 1
    el = time.perf_counter() - t0
    return {"seconds_per_step": el / n, "steps": n}


def encoder_bench(args, device) -> dict:
    """``--config e2e``: one streaming step of a random-init FastConformer from
    pcm16 to tokens, ``--streams`` streams all live (E2E_MODELS; ``--model``):
    * small: 80 mels, 17 layers, d_model 512, fp16, each stream fed a 160 ms
      chunk (2560 samples) per step, 2 encoder frames per step;
    * large: 128 mels, 24 layers, d_model 1024, bf16, 1.12 s chunks (17920
      samples), 14 encoder frames per step (att_context (70, 13)), a 2-layer
      predictor.
    The step: the batched front end (pk_fe_step: sample ring, dither,
    pre-emphasis, FFT, Slaney mel, log; pk_subsample: the 8x convolution stack
    over each stream's [cached ; new] mel window; the ``out`` GEMM;
    model_runner.py:181-252), the encoder (8 heads, feed-forward x4, depthwise
    conv kernel 9, left context 70: torch projections and feed-forward GEMMs,
    pk_paged_relpos_attn, pk_conv_step, pk_streaming_mask; encoder.py:229-267),
    then greedy RNNT decoding (pk_rnnt_greedy_step: up to 5 symbols a frame,
    predictor state per slot on the device; model_runner.py:306-447) with one
    token copy per step.  Input: int16 pcm of 3 random sinusoids (100-4000 Hz)
    plus noise at 20 dB SNR, resident on the GPU.  Also times the front-end
    kernels, the decode step and the conv step alone."""
    import numpy as np
    import torch

    from parakeet_amd import ops
    from parakeet_amd.modules.decoder import GreedyDecoder, Joiner, Predictor
    from parakeet_amd.modules.encoder import ConformerEncoder, EncoderStepGraph
    from parakeet_amd.modules.frontend import ConvSubsampling, FeatureExtractor, PreEncoder

    model = getattr(args, "model", "small")
    m = E2E_MODELS[model]
    B, D, H, Ly, K, left, right = args.streams, m["D"], m["H"], m["layers"], m["K"], m["left"], m["right"]
    vocab, out_scale, blank_bias = m["vocab"], 4.0, m["blank_bias"]
    n_mels, C = m["n_mels"], m["C"]
    T = right + 1
    hop, first_chunk, chunk = 160, m["first"], m["chunk"]
    dt = {"fp16": torch.float16, "bf16": torch.bfloat16}[m["dtype"]]
    torch.manual_seed(4)
    enc = ConformerEncoder(
        feat_in=n_mels, hidden_size=D, ff_expansion_factor=4, num_layers=Ly, num_heads=H, subsampling_factor=8,
        pos_emb_max_len=5000, conv_kernel_size=K, att_context_size=[left, right], subsampling_conv_channels=C,
        use_bias=False,
    )
    sub = ConvSubsampling(D, C, n_mels, 8)
    with torch.no_grad():
        for layer in enc.layers:
            layer.self_attn.pos_bias_u.normal_(0.0, 0.02)
            layer.self_attn.pos_bias_v.normal_(0.0, 0.02)
        for mod in sub.conv:
            if isinstance(mod, torch.nn.Conv2d):
                mod.weight.normal_(0.0, mod.weight[0].numel() ** -0.5)
    # predictor and joiner (config.py:19-22), default init with the output layer
    # scaled and the blank logit biased so frames end on blank or on tokens
    # (the token rate is reported below)
    pred = Predictor(640, 640, m["pred_layers"], vocab)
    joint = Joiner(D, 640, 640, num_classes=vocab)
    with torch.no_grad():
        joint.joint_net[2].weight.mul_(out_scale)
        joint.joint_net[2].bias[vocab] += blank_bias
    enc = enc.to(dt).to(device).eval().requires_grad_(False)
    sub = sub.to(dt).to(device).eval().requires_grad_(False)
    pred = pred.to(dt).to(device).eval().requires_grad_(False)
    joint = joint.to(dt).to(device).eval().requires_grad_(False)
    dec = GreedyDecoder(pred, joint, blank_id=vocab, num_slots=B)
    dec.reset_slot(np.arange(B))
    fx = FeatureExtractor(n_mels=n_mels, seed=6, device=device)
    pre = PreEncoder(fx, sub, num_slots=B, device=device, ring_size=m["ring"], mel_rows=m["mel_rows"])
    slots = np.arange(B)
    for s in slots:
        pre.reset_slot(s)
    state = enc.init_streaming_state(batch_size=B, device=device, dtype=dt)
    pre_steps = -(-left // T) + 1 + args.warmup  # past the 70-frame window
    n_total = first_chunk + chunk * (pre_steps + args.steps)
    log(f"synthesising {B} x {n_total} pcm16 samples")
    # at most 256 distinct signals, repeated over larger batches (each stream's
    # dither still differs)
    base = synth_pcm(min(B, 256), n_total, seed=7)
    pcm = torch.from_numpy(base[np.arange(B) % base.shape[0]]).to(device)
    del base
    length = torch.full((B,), T, dtype=torch.int64, device=device)
    # the encoder step recorded once and replayed (the host page work and the
    # rows upload stay outside the recording), or issued op by op from Python
    enc_step = None if args.eager_encoder else EncoderStepGraph(enc, state, length)
    pos = 0
    n_tokens = n_frames = 0
    pending = None  # the previous step's tokens, split while the GPU runs this step
    last_enc = None  # the last step's encoder output, for the decode step timed alone

    def count_pending():
        nonlocal pending, n_tokens
        if pending is not None:
            n_tokens += pending.result().total()
            pending = None

    def step():
        nonlocal pos, n_tokens, n_frames, pending, last_enc
        n = first_chunk if pos == 0 else chunk
        rows, counts, first = pre.step(slots, pcm[:, pos : pos + n], n, False)
        pos += n
        if not (counts == T).all():
            raise RuntimeError(f"front end gave {counts.min()}..{counts.max()} frames per stream, expected {T}")
        if enc_step is not None:
            out = enc_step(rows.view(B, T, D))
        else:
            out, _ = enc(rows.view(B, T, D), state, length=length)
        last_enc = out.transpose(1, 2)
        res = dec.decode(slots, last_enc, graph=True, wait=False)
        count_pending()
        pending = res
        n_frames += B * T

    gc.collect()
    gc.freeze()
    with torch.inference_mode():
        for _ in range(pre_steps):  # past the 70-frame window
            step()
        count_pending()
        torch.cuda.synchronize()
        K_steps = args.steps
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(K_steps):
            step()
        count_pending()  # the last step's split is timed too: K splits in all
        stop.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = start.elapsed_time(stop) / K_steps
        log(f"timed {K_steps} steps from pcm16")
        tok_rate = n_tokens / max(n_frames, 1)
        # the decode step alone on the last step's encoder frames (the step's
        # launches replayed from its recording, one token copy back, the lazy
        # per-stream result); the predictor state keeps advancing, so the token
        # rate stays the model's
        enc_frames = last_enc.contiguous()
        dec.decode(slots, enc_frames, graph=True)
        torch.cuda.synchronize()
        a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        dec_reps = 20
        t1 = time.perf_counter()
        a_ev.record()
        for _ in range(dec_reps):
            dec.decode(slots, enc_frames, graph=True)
        b_ev.record()
        torch.cuda.synchronize()
        dec_wall_ms = 1000.0 * (time.perf_counter() - t1) / dec_reps
        dec_ms = a_ev.elapsed_time(b_ev) / dec_reps
        log("timed the decode step")

        # the front-end kernels alone on the last step's records (re-running a
        # step's records recomputes the same frames into the same ring rows)
        fe_args = dict(dither=fx.dither, seed=fx.seed, max_new=chunk, max_frames=chunk // hop)
        samples = pcm[:, pos - chunk : pos]
        flat = torch.empty((B * T, C * sub.final_freq_dim), dtype=dt, device=device)
        w = sub.conv_weights()
        fe_us = _graph_time_us(lambda: ops.fe_step(pre.hdr[: 32 * B], B, samples, pre.sample_ring, pre.mel_ring,
                                                   pre.tables, **fe_args), device)
        sub_us = _graph_time_us(lambda: ops.subsample(pre.hdr[32 * B :], B, pre.mel_ring, True, w, flat, max_out=T),
                                device)
        lin_us = _graph_time_us(lambda: torch.nn.functional.linear(flat, sub.out.weight, sub.out.bias), device)
        log("timed the front-end kernels")

        # the conv step alone on the same shape and cache
        conv = enc.layers[0].conv
        g = torch.Generator().manual_seed(5)
        h = torch.randn(B, T, 2 * D, generator=g).to(dt).to(device)
        frames = state.cache.conv_frames

        def conv_all_layers():
            for layer in range(Ly):
                ops.conv_step(h, frames, conv.depthwise_conv.weight, conv.batch_norm.weight, conv.batch_norm.bias,
                              layer=layer, eps=conv.batch_norm.eps)

        conv_us = _graph_time_us(conv_all_layers, device, inner=1) / Ly

        # the attention kernel alone on the step's own pages, every layer, with
        # the mask tensor the encoder passes it (full windows after the timed
        # steps), each launch between HIP events on its stream
        cache = state.cache
        pages = cache.paged()
        ga = torch.Generator().manual_seed(9)
        qkv_t = torch.randn(B, T, 3 * D, generator=ga).to(dt).to(device)
        q_t, k_t, v_t = qkv_t.chunk(3, dim=-1)
        pe = enc.pos_enc.pe[0]
        ctr = pe.shape[0] // 2 + 1
        pos_t = torch.nn.functional.linear(pe[ctr - (T + left) : ctr + T + left - 1].to(dt),
                                           enc.layers[0].self_attn.linear_pos.weight)
        bu_t = enc.layers[0].self_attn.pos_bias_u.to(dt).contiguous()
        bv_t = enc.layers[0].self_attn.pos_bias_v.to(dt).contiguous()
        _, mask_t = ops.streaming_mask(state.processed_frames - T, state.cache_lengths, T, chunk=T, left=left, chunk_size=T)
        att_out = torch.empty((B, T, D), dtype=dt, device=device)
        att_reps = 20
        att_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(att_reps * Ly)]
        for a_ev2, b_ev2 in att_ev:
            a_ev2.record()
            b_ev2.record()
        torch.cuda.synchronize()
        for r in range(att_reps):
            for layer in range(Ly):
                a_ev2, b_ev2 = att_ev[r * Ly + layer]
                ops.paged_relpos_attn(q_t, k_t, v_t, pos_t, bu_t, bv_t, mask_t, num_heads=H, left=left, pages=pages,
                                      layer=layer, append=True, out=att_out,
                                      start_event=ops._event_handle(a_ev2), stop_event=ops._event_handle(b_ev2))
        torch.cuda.synchronize()
        att_us = 1000.0 * sum(a_ev2.elapsed_time(b_ev2) for a_ev2, b_ev2 in att_ev) / len(att_ev)
        log("timed the attention kernel on the step's pages")
    s = 2
    conv_bytes = B * s * (T * 2 * D + 2 * (K - 1) * D + T * D) + s * D * (K + 2)
    # front-end algorithmic work per step (steady state: chunk / hop new mel frames)
    F1 = n_mels // 2 + 1
    F2 = F1 // 2 + 1
    F3 = F2 // 2 + 1
    fe_bytes = B * (chunk * 2 + chunk * 4 + (chunk // hop) * n_mels * 4)  # pcm in, ring write, mel rows out
    # the MACs the T kept output frames of each stream depend on: 4 T + 3 rows
    # of conv.0, 2 T + 1 of the first depthwise conv and conv.3, T of the second
    # depthwise conv and conv.6 (T = 2: conv.0 rows 2..12, first depthwise +
    # pointwise rows 2..6, second depthwise + pointwise rows 2..3)
    sub_macs = B * ((4 * T + 3) * F1 * C * 9 + (2 * T + 1) * F2 * C * 9 + (2 * T + 1) * F2 * C * C
                    + T * F3 * C * 9 + T * F3 * C * C)
    sub_tflops = 2 * sub_macs / (sub_us * 1e-6) / 1e12
    # attention: algorithmic bytes per launch (K/V window read, K/V append write,
    # query read and output write, block-table row, mask bytes) plus the shared
    # position rows and biases
    max_pages = cache.max_pages
    att_bytes = B * (s * D * (2 * (left + T) + 4 * T) + 4 * (1 + max_pages) + T * (left + T)) + s * D * (left + 2 * T - 1) + 2 * s * D
    att_gbs = att_bytes / (att_us * 1e-6) / 1e9
    cpu = dec_cpu = att_cpu = step_cpu = None
    if not args.no_cpu_baseline:
        from parakeet_amd import synth

        part_s = min(args.cpu_baseline_seconds, 10.0)
        att_cpu = cpu_baseline(synth.SMALL_FP16 if model == "small" else synth.LARGE_BF16_T14, B,
                               args.cpu_baseline_seconds, seed=5)
        att_cpu["sample"] = ("the reference's dense encoder-attention path only (not the whole pcm16 -> tokens step): "
                             + att_cpu["sample"])
        dec_cpu = decode_cpu_baseline(pred, joint, vocab, part_s, B, frames=T, layers=m["pred_layers"])
        sd = {k: v.detach().double().cpu().numpy() for k, v in sub.state_dict().items()}
        cb = front_end_cpu_baseline(sd, part_s, seed=8, n_mels=n_mels, first=first_chunk, chunk=chunk)
        chunk_ms = 1000.0 * chunk / 16000.0
        cpu = {
            "value": round(cb["chunks_per_s"] / B, 4),
            "unit": f"front-end steps/s ({B} streams x {chunk_ms:g} ms)",
            "cores": 1,
            "kind": "port",
            "sample": f"{cb['chunks']} chunks of {chunk_ms:g} ms of one stream through the oracle's FeatureExtractor.push + "
            f"ConvSubsampling (float64 numpy) in {cb['seconds']:.1f} s, scaled to {B} streams per step",
        }
        ec = encoder_cpu_baseline(enc, part_s, Ly, H, left, right, K, D)
        # the whole pcm16 -> tokens step of one stream on one core: front end +
        # encoder + greedy decode, each timed above, scaled to the batch
        per_stream_s = 1.0 / cb["chunks_per_s"] + ec["seconds_per_step"] + 1.0 / (dec_cpu["value"] * B)
        step_cpu = {
            "value": round(1.0 / (per_stream_s * B), 5),
            "unit": "steps/s",
            "cores": 1,
            "kind": "port",
            "sample": f"one stream's pcm16 -> tokens step on one core, the sum of the oracle's front end "
            f"({1000.0 / cb['chunks_per_s']:.2f} ms a {chunk_ms:g} ms chunk), encoder step ({Ly} layers, float64 numpy, "
            f"{1000.0 * ec['seconds_per_step']:.2f} ms over {ec['steps']} steps) and greedy decode "
            f"({1000.0 / (dec_cpu['value'] * B):.2f} ms a {T}-frame step), scaled to {B} streams per step",
        }
    result = {
        "metric": f"streaming steps/sec from pcm16 to tokens ({model} FastConformer: front end + {Ly} layers + greedy RNNT) at 1 GPU",
        "value": round(1000.0 / ms, 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": m["dtype"],
        "data": "synthetic pcm16 (3 random sinusoids 100-4000 Hz + noise at 20 dB SNR), random-init weights, pos biases N(0,0.02), joint output x4 with blank logit bias +3",
        "config": {
            "workload": f"{model} FastConformer step from pcm16: {1000.0 * chunk / 16000.0:g} ms per stream -> "
            f"log-mel ({n_mels}) -> 8x conv subsampling -> {Ly} layers x (FF/2, paged rel-pos MHA, conv module "
            f"with per-stream cache, FF/2, LN) -> greedy RNNT ({m['pred_layers']}-layer LSTM 640, joint 640, "
            f"{vocab + 1} classes, up to 5 symbols a frame), {B} streams all live, {T} encoder frames per step",
            "model": model,
            "layers": Ly,
            "d_model": D,
            "heads": H,
            "conv_kernel": K,
            "left_context": left,
            "frames_per_step": T,
            "streams": B,
            "n_mels": n_mels,
            "subsampling_channels": C,
            "parallelism": "single GPU",
            "encoder_launch": "eager: torch ops issued from Python"
            if args.eager_encoder
            else f"one HIP graph replay per step ({Ly} layers)",
        },
        "front_end": {
            "fe_kernel_us": round(fe_us, 3),
            "subsample_kernel_us": round(sub_us, 3),
            "out_gemm_us": round(lin_us, 3),
            "fe_bytes_per_launch": fe_bytes,
            "fe_gbs": round(fe_bytes / (fe_us * 1e-6) / 1e9, 1),
            "subsample_flops_per_launch": 2 * sub_macs,
            "roofline": {
                "bound": "mfma",
                "achieved": round(sub_tflops, 2),
                "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(sub_tflops / MFMA_F16_PEAK_TFLOPS, 5),
                "kernel": "subsample_kernel",
            },
            "cpu_baseline": cpu,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(att_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(att_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": ("relpos_attn_chunk_kernel (fused append + paged rel-pos attention over one read of the "
                       "window for all of the chunk's queries, mask tensor)" if T >= 3 else
                       "relpos_attn_mfma_kernel (fused append + paged rel-pos attention, mask tensor)"),
            "avg_kernel_us": round(att_us, 3),
            "bytes_per_launch": att_bytes,
            "launches_timed": len(att_ev),
            "cpu_baseline_attention_only": att_cpu,
        },
        "cpu_baseline": step_cpu,
        "realtime": {
            "audio_ms_per_step": 1000.0 * chunk / 16000.0,
            "streams": B,
            "x_realtime": round(1000.0 * chunk / 16000.0 / ms, 2),
            "keeps_up": bool(ms <= 1000.0 * chunk / 16000.0),
            # device memory at its peak in this run, and the part of it that is the
            # bench's own pcm input for every step (not state a server would hold)
            "device_gib_peak": round(torch.cuda.max_memory_allocated(device) / 2**30, 2),
            "device_gib_bench_pcm": round(pcm.numel() * pcm.element_size() / 2**30, 2),
        },
        "decode": {
            "step_ms": round(dec_ms, 4),
            "step_wall_ms": round(dec_wall_ms, 4),
            "tokens_per_frame": round(tok_rate, 3),
            "decisions_max_per_step": B * T * 5,
            "cpu_baseline": dec_cpu,
        },
        "conv_step": {
            "kernel": ("conv_chunk_kernel (GLU, pad mask, causal depthwise conv with cache, LayerNorm, SiLU; "
                       "the chunk's frames in parallel)" if T >= 3 and B * (-(-D // 512)) <
                       6 * torch.cuda.get_device_properties(device).multi_processor_count else
                       "conv_step_kernel (GLU, pad mask, causal depthwise conv with cache, LayerNorm, SiLU)"),
            "avg_kernel_us": round(conv_us, 3),
            "bytes_per_launch": conv_bytes,
            "gbs": round(conv_bytes / (conv_us * 1e-6) / 1e9, 1),
            "frac_of_peak": round(conv_bytes / (conv_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "wall_s": round(wall, 3),
    }
    return result


def read_probe(nbytes: int, reps: int) -> dict:
    """One launch of ``pk_hbm_read_probe`` reading ``nbytes`` (a launch's bytes),
    from buffers cycled past the 256 MB last-level cache (>= 1 GiB of them), each
    launch between HIP events on its stream: the read ceiling of a launch of that
    size on this GPU."""
    import torch

    from parakeet_amd import ops

    n = max(16, (int(nbytes) + 15) // 16 * 16)
    nbuf = max(2, -(-(1 << 30) // n))
    dev = torch.device("cuda:0")
    bufs = [torch.ones(n // 2, dtype=torch.bfloat16, device=dev) for _ in range(nbuf)]
    out = torch.empty(64 * 8 * torch.cuda.get_device_properties(dev).multi_processor_count, dtype=torch.uint8, device=dev)
    for b in bufs:  # warm
        ops.hbm_read_probe(b, out)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record()
        b.record()
    torch.cuda.synchronize()
    for r in range(reps):
        ops.hbm_read_probe(bufs[r % nbuf], out, start_event=ev[r][0], stop_event=ev[r][1])
    torch.cuda.synchronize()
    us = 1000.0 * sum(a.elapsed_time(b) for a, b in ev) / reps
    del bufs
    gbs = n / (us * 1e-6) / 1e9
    return {"bytes": n, "launches": reps, "buffers": nbuf, "avg_us": round(us, 3), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def _release(device) -> None:
    import torch

    gc.collect()
    torch.cuda.synchronize(device)
    torch.cuda.empty_cache()


def paged_bench(config_name: str, device, args, steps: int, warmup: int, event_steps: int, cpu_seconds: float,
                probes: bool = True) -> dict:
    """The encoder-attention step of one workload (CONFIGS): ``steps`` timed steps
    of host page work + upload + every layer's launch (replayed from a HIP graph
    with --graph), then ``event_steps`` steps with every kernel between HIP events
    for the roofline, the same-bytes read and copy probes and the CPU baseline."""
    import numpy as np
    import torch

    from parakeet_amd import ops

    cfg = CONFIGS[config_name]
    log(f"config {config_name}: building workload")
    shape, runner, churn = build_runner(cfg, device, args.rows_per_lane)
    Ly = shape.layers
    # the objects built so far live for the whole run: keep them out of the
    # collector's scans, so a full collection in the step loop stays short
    gc.collect()
    gc.freeze()
    with torch.inference_mode():
        for _ in range(args.preroll):
            churn_step(runner, churn)
        for _ in range(warmup):
            churn_step(runner, churn)
        torch.cuda.synchronize()
        log(f"{config_name}: preroll {args.preroll} + warmup {warmup} steps done")
        use_graph = args.graph
        if use_graph:
            runner.capture()
            for _ in range(max(1, warmup // 2)):
                churn_step(runner, churn, graph=True)
            torch.cuda.synchronize()
        # timed pass 1: the step loop as it serves
        batches = []
        step_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for k in range(steps):
            step_ev[k][0].record()
            batches.append(churn_step(runner, churn, graph=use_graph))
            step_ev[k][1].record()
        stop.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        log(f"{config_name}: timed {steps} steps")
        # timed pass 2: every kernel between its own HIP events (eager launches)
        ev_pairs, ev_batches = [], []
        for _ in range(event_steps):
            pairs = []
            for _ in range(Ly):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                b.record()
                pairs.append((a, b))
            ev_pairs.append(pairs)
        torch.cuda.synchronize()
        handles = [[(ops._event_handle(a), ops._event_handle(b)) for a, b in pairs] for pairs in ev_pairs]
        for k in range(event_steps):
            ev_batches.append(churn_step(runner, churn, handles[k]))
        torch.cuda.synchronize()
        log(f"{config_name}: {event_steps} steps with per-kernel events")
    gc.unfreeze()

    ms_per_step = start.elapsed_time(stop) / steps
    gpu_ms_per_step = sum(a.elapsed_time(b) for a, b in step_ev) / steps
    per_stream = runner.bytes_per_stream()
    shared = runner.bytes_shared_per_launch()
    total_bytes = sum(B * Ly * per_stream + Ly * shared for B in ev_batches)
    kern_ms = sum(a.elapsed_time(b) for pairs in ev_pairs for a, b in pairs)
    n_launch = max(1, len(ev_batches) * Ly)
    avg_us = 1000.0 * kern_ms / n_launch
    avg_B = float(np.mean(batches))
    ev_B = float(np.mean(ev_batches)) if ev_batches else avg_B
    per_stream_pool = runner.pool.max_pages * Ly * shape.page_size * shape.d_model * shape.elem_bytes * 2
    free_b, total_b = torch.cuda.mem_get_info(device)
    audio_ms = shape.chunk * FRAME_SECONDS * 1000.0
    if shape.dtype == torch.float32:
        kernel = ("relpos_attn_kernel (fp32 vector ALU; fused append + paged rel-pos attention, "
                  "each window split over 4 waves at small batches)")
    elif (3 <= shape.chunk <= 14 and args.rows_per_lane == 0) or args.rows_per_lane == -2:
        kernel = "relpos_attn_chunk_kernel (whole chunk; fused append + paged rel-pos attention)"
    else:
        kernel = "relpos_attn_mfma_kernel (fused append + paged rel-pos attention)"
    out = {
        "value": round(1000.0 / ms_per_step, 2),
        "unit": "steps/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "gpu_ms_per_step": round(gpu_ms_per_step, 4),
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[shape.dtype],
        "config": {
            "workload": f"{shape.name}: paged append+attention+eviction, {cfg['slots']} stream slots at "
            f"{int(cfg['occupancy'] * 100)}% occupancy with churn",
            "layers": Ly,
            "d_model": shape.d_model,
            "heads": shape.heads,
            "head_dim": shape.head_dim,
            "page_size": shape.page_size,
            "left_context": shape.left,
            "frames_per_step": shape.chunk,
            "stream_slots": cfg["slots"],
            "avg_active_streams": round(avg_B, 1),
            "parallelism": "single GPU",
            "launch": "one HIP graph replay per step (all layers)" if use_graph else "one host launch per layer",
        },
        "realtime": {
            "audio_ms_per_step": audio_ms,
            "x_realtime": round(audio_ms / ms_per_step, 1),
            "pool_capacity_hbm_streams": int((total_b * 0.9) // per_stream_pool),
            "pool_bytes_per_stream": per_stream_pool,
        },
        "wall_s": round(wall, 3),
    }
    achieved = total_bytes / (kern_ms * 1e-3) / 1e9 if kern_ms > 0 else 0.0  # 0: no launch was event-timed
    traffic = measured_traffic(config_name, ev_B) if args.rows_per_lane == 0 else None
    roof = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "kernel": kernel,
        "avg_kernel_us": round(avg_us, 3),
        "kernel_event_steps": len(ev_batches),
        "bytes_per_stream_layer": per_stream,
        "bytes_shared_per_launch": shared,
        "bytes_per_launch": int(round(total_bytes / n_launch)),
    }
    if traffic and avg_us > 0:
        # the same launch time over the bytes the HBM counters read
        roof["frac_counter_bytes"] = round(traffic / (avg_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    if probes and not args.no_copy_ceiling:
        launch_bytes = total_bytes / n_launch
        rp = read_probe(int(launch_bytes), 100)
        roof["read_same_bytes"] = rp
        roof["frac_of_read_ceiling"] = round(achieved / rp["gbs"], 4)
        log(f"{config_name}: same-bytes read {rp['avg_us']} us, {rp['gbs']} GB/s")
        mib = max(1, int(round(launch_bytes / 2 / (1 << 20))))
        cp = copy_probe(mib, 100)
        roof["copy_same_bytes"] = {"bytes": 2 * cp["copy_probe_bytes_read"], "avg_us": cp["avg_us"], "gbs": cp["gbs"],
                                   "frac": cp["frac_of_peak"]}
    out["roofline"] = roof
    out["paged_attn_hbm_gbs"] = round(achieved, 1)
    del runner, churn
    _release(device)
    if cpu_seconds > 0:
        log(f"{config_name}: cpu baseline ...")
        try:
            out["cpu_baseline"] = cpu_baseline(shape, max(1, int(round(avg_B))), cpu_seconds, cfg["seed"])
        except Exception as e:  # report, never hide
            out["cpu_baseline"] = {"error": repr(e)}
    return out


def capacity_bench(device, config_name: str, steps: int) -> dict:
    """The largest batch the GPU holds at a workload's shape, all streams live:
    the page pool sized to the free HBM (one qkv input shared by the layers),
    windows filled, then ``steps`` timed steps (host page work, upload, every
    layer's launch).  The step time against the chunk's audio says whether that
    batch keeps up with real time."""
    import numpy as np
    import torch

    from parakeet_amd import synth
    from parakeet_amd.pool import pages_per_slot
    from parakeet_amd.step import AttentionStep

    cfg = CONFIGS[config_name]
    shape = getattr(synth, cfg["shape"])
    Ly, T, D, s = shape.layers, shape.chunk, shape.d_model, shape.elem_bytes
    M = pages_per_slot(shape.left, T, shape.page_size)
    per_stream_pool = Ly * M * shape.page_size * D * s * 2
    per_stream_io = Ly * T * D * s + 3 * T * D * s  # outputs of every layer + the shared qkv input
    _release(device)
    free_b, total_b = torch.cuda.mem_get_info(device)
    reserve = 6 << 30
    S = int((free_b - reserve) // (per_stream_pool + per_stream_io)) // 256 * 256
    log(f"capacity {config_name}: {S} streams ({S * per_stream_pool / 2**30:.1f} GiB of pages, {free_b / 2**30:.1f} GiB free)")
    qkv = synth.qkv_frames(S, shape, device, seed=21)
    pos, bu, bv = synth.relpos_inputs(shape, device, seed=22)
    runner = AttentionStep(shape, S, device, [qkv] * Ly, pos, [bu] * Ly, [bv] * Ly)
    active = np.arange(S, dtype=np.int32)
    fill = -(-(shape.left + T) // T) + 1  # steps until every window is full
    with torch.inference_mode():
        for _ in range(fill):
            runner.step(active)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            runner.step(active)
        stop.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop) / steps
    nbytes = Ly * (S * runner.bytes_per_stream() + runner.bytes_shared_per_launch())
    audio_ms = T * FRAME_SECONDS * 1000.0
    peak_gib = torch.cuda.max_memory_allocated(device) / 2**30
    del runner, qkv
    _release(device)
    return {
        "workload": f"{shape.name}: {S} streams, all live, windows full",
        "streams": S,
        "steps": steps,
        "ms_per_step": round(ms, 3),
        "steps_per_s": round(1000.0 / ms, 2),
        "audio_ms_per_step": audio_ms,
        "x_realtime": round(audio_ms / ms, 2),
        "keeps_up": bool(ms <= audio_ms),
        "attention_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "pool_gib": round(S * per_stream_pool / 2**30, 1),
        "device_gib_total": round(total_b / 2**30, 1),
        "device_gib_peak": round(peak_gib, 1),
        "bound_by": "HBM capacity of the page pool" if ms <= audio_ms else "attention step time",
        "wall_s": round(wall, 2),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", choices=sorted(CONFIGS) + ["e2e"], default="large")
    ap.add_argument("--preroll", type=int, default=60, help="untimed steps before warmup to reach steady-state windows")
    ap.add_argument("--rows-per-lane", type=int, default=0, help="kernel choice (0 automatic; see pk_attn_args)")
    ap.add_argument("--kernel-event-steps", type=int, default=50, help="eager steps timed per kernel for the roofline")
    ap.add_argument("--graph", action="store_true", help="replay every step's launches from one HIP graph (grid sized for all slots)")
    ap.add_argument("--streams", type=int, default=128, help="e2e: streams in the batch (all live)")
    ap.add_argument("--model", choices=sorted(E2E_MODELS), default="small", help="e2e: the FastConformer size")
    ap.add_argument("--eager-encoder", action="store_true", help="e2e: issue the encoder's ops from Python instead of replaying a recorded step")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB", help="only run a device copy of MIB MiB (counter calibration)")
    ap.add_argument("--cpu-baseline-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-copy-ceiling", action="store_true", help="skip the same-bytes read and copy probes")
    ap.add_argument("--no-extras", action="store_true",
                    help="default config only: skip the other workloads and the capacity run")
    ap.add_argument("--no-kernel-events", action="store_true", help="no per-kernel event pass (for counter runs)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one GPU: the paged encoder-attention path has no cross-GPU work "
            "(streams are sharded per GPU with no per-step exchange); run with --gpus 1",
            file=sys.stderr,
        )
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    if args.copy_probe:
        print(json.dumps(copy_probe(args.copy_probe, max(1, args.steps))), flush=True)
        return 0
    if args.config == "e2e":
        print(json.dumps(encoder_bench(args, device)), flush=True)
        return 0
    cpu_s = 0.0 if args.no_cpu_baseline else args.cpu_baseline_seconds
    ev_steps = 0 if args.no_kernel_events else min(args.steps, args.kernel_event_steps)
    head = paged_bench(args.config, device, args, args.steps, args.warmup, ev_steps, cpu_s, probes=ev_steps > 0)
    result = {
        "metric": "encoder attn steps/sec & max concurrent streams at 1 GPU; paged-attn HBM GB/s",
        "value": head.pop("value"),
        "unit": head.pop("unit"),
        "n_gpus": 1,
        "steps": head.pop("steps"),
        "warmup": head.pop("warmup"),
        "ms_per_step": head.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head.pop("dtype"),
        "data": "synthetic (seeded N(0,1) Q/K/V, N(0,0.02) biases, linear_pos of the sinusoid table)",
        "config": head.pop("config"),
    }
    result.update(head)
    default_run = args.config == "large" and not args.no_extras and ev_steps > 0
    if default_run:
        # the other workloads, each with its roofline and CPU baseline, and the
        # largest batch the GPU holds at the headline shape
        extra_s = min(cpu_s, 8.0)
        extras = [
            ("large_t14", lambda: paged_bench("large-t14", device, args, 100, 10, 30, extra_s)),
            ("small_64streams", lambda: paged_bench("small", device, args, 100, 10, 30, extra_s)),
            ("frag_1024streams", lambda: paged_bench("frag", device, args, 100, 10, 30, extra_s)),
            ("plumbing_4streams", lambda: paged_bench("plumbing", device, args, 100, 10, 30, min(extra_s, 4.0))),
        ]
        for key, fn in extras:
            torch.cuda.reset_peak_memory_stats(device)
            try:
                result[key] = fn()
            except Exception as e:  # report, never hide
                result[key] = {"error": repr(e)}
        try:
            cap = capacity_bench(device, "large", 10)
        except Exception as e:
            cap = {"error": repr(e)}
        result["concurrent_streams"] = {
            "measured_max": cap,
            "headline_batch": result["config"]["avg_active_streams"],
            "reference_claim": "around 80 (small) / 60 (large) concurrent streams on an A100 (README.md:26-27)",
        }
        # pcm16 -> tokens, both model sizes at 128 streams
        for key, model, steps, warmup in (("e2e_pcm16_128streams", "small", 20, 5),
                                           ("e2e_pcm16_large_128streams", "large", 10, 3)):
            _release(device)
            torch.cuda.reset_peak_memory_stats(device)
            try:
                e2e_args = argparse.Namespace(**vars(args))
                e2e_args.steps, e2e_args.warmup = steps, warmup
                e2e_args.cpu_baseline_seconds = extra_s
                e2e_args.streams = 128
                e2e_args.model = model
                e2e = encoder_bench(e2e_args, device)
                for k in ("n_gpus", "higher_is_better", "scaling", "vs_baseline"):
                    e2e.pop(k, None)
                result[key] = e2e
            except Exception as e:
                result[key] = {"error": repr(e)}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
