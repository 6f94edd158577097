"""The streaming encoder step end to end, pcm16 in: the batched front end
(pk_fe_step, pk_subsample and the ``out`` GEMM; model_runner.py:181-252) feeds
the drop-in ConformerEncoder on the paged cache (torch projections and
feed-forward GEMMs, pk_paged_relpos_attn with the mask from the stream state,
pk_conv_step; encoder.py:11-81,229-267), run eagerly and as a recorded
EncoderStepGraph replay.  Each step's output of every stream is compared with
the float64 oracle composition on the CPU: oracle/frontend.py's per-stream
pre-encode of the same pcm (same dither stream) into oracle/encoder.py's
encoder step over dense caches, with the same (model-dtype-rounded) weights.

Workloads:
* small FastConformer (the 128-stream pcm16 workload's model at 4 streams):
  80 mels, 8x subsampling with 256 channels, d_model 512, 8 heads, all 17
  layers, conv kernel 9, left context 70, 2 frames a step, fp16, 45 steps (the
  window fills after 35, pages are evicted from then on);
* large FastConformer shape at its own chunking: 128 mels, d_model 1024,
  8 heads x 128, all 24 layers, chunk of 14 encoder frames (att_context
  (70, 13)), bf16, 4 streams, 9 steps (eviction from step 6).

Bar (stated per dtype in TOL): max |got - ref| over every output element, step
and stream, and the RMS of the error over a step.  The outputs leave the final
LayerNorm, so they are O(1).  The GPU computes in the model dtype with fp32
accumulation: every activation is rounded to fp16 (unit roundoff u = 2^-11)
or bf16 (2^-8) between operations.  Through the front end, the residual adds,
the five LayerNorms, the 2 feed-forward blocks and the attention and conv
branches of each layer, the roundings add up to 15-17 u at the worst element
and 2-4 u in RMS: measured fp16 (17 layers) max 8.35e-3 (17 u), RMS 1.84e-3;
bf16 (24 layers) max 4.57e-2 (12 u), RMS 8.5e-3 (at 6 layers 5.65e-2 and
6.6e-3).  The bars leave about a factor of two: fp16 max 1.6e-2 and RMS
3.5e-3, bf16 max 1e-1 and RMS 1.5e-2.  The GPU run compared with an oracle
carrying a plausible mistake in the composition (relative positions reversed:
max 0.42 / 0.47; conv taps shifted by one frame: 1.14 / 0.39; a feed-forward
branch without its 0.5: 0.26 / 0.24, fp16 / bf16) exceeds them by far, so they
catch those.  A mistake in a bias term (pos_bias_v
dropped) moves the stack's outputs by less than the dtype's rounding (fp16 max
1.04e-2 against 8.35e-3 clean; bf16 unchanged): the kernel-level bars catch it.
"""

import numpy as np
import pytest
import torch

from oracle import encoder as oe
from oracle import frontend as ofe
from oracle import relpos
from parakeet_amd.modules.encoder import ConformerEncoder, EncoderStepGraph
from parakeet_amd.modules.frontend import FeatureExtractor, PreEncoder

from _dense_encoder import init_attention

pytestmark = pytest.mark.gpu

CASES = {
    # D, H, layers, K, left, right, n_mels, C, dtype, streams, steps, first chunk, next chunks, ring, mel rows
    "small_fp16": (512, 8, 17, 9, 70, 1, 80, 256, torch.float16, 4, 45, 1440, 2560, 8192, 64),
    "large_bf16_t14": (1024, 8, 24, 9, 70, 13, 128, 256, torch.bfloat16, 4, 9, 16800, 17920, 32768, 256),
}
TOL = {torch.float16: (1.6e-2, 3.5e-3), torch.bfloat16: (1e-1, 1.5e-2)}  # (max abs, rms)


def _pcm(B, n, seed):
    """int16 pcm per stream: 3 sinusoids (100-4000 Hz) + noise at 20 dB SNR."""
    rng = np.random.default_rng(seed)
    t = np.arange(n) / 16000.0
    out = np.empty((B, n), dtype=np.int16)
    for b in range(B):
        f, a, ph = rng.uniform(100, 4000, 3), rng.uniform(0.05, 0.3, 3), rng.uniform(0, 2 * np.pi, 3)
        sig = (a[:, None] * np.sin(2 * np.pi * f[:, None] * t[None] + ph[:, None])).sum(0)
        sig += rng.standard_normal(n) * np.sqrt(np.mean(sig**2) / 100.0)
        out[b] = np.clip(np.round(sig * 32767.0), -32768, 32767).astype(np.int16)
    return out


def _model(case, seed):
    D, H, Ly, K, left, right, n_mels, C, dt = CASES[case][:9]
    torch.manual_seed(seed)
    enc = ConformerEncoder(
        feat_in=n_mels, hidden_size=D, ff_expansion_factor=4, num_layers=Ly, num_heads=H, subsampling_factor=8,
        pos_emb_max_len=5000, conv_kernel_size=K, att_context_size=[left, right], subsampling_conv_channels=C,
        use_bias=False,
    )
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for layer in enc.layers:
            init_attention(layer.self_attn, D, seed=seed + 10 + layer.layer_idx)
            for mod in layer.modules():
                if isinstance(mod, torch.nn.LayerNorm):
                    mod.weight.copy_(1.0 + 0.1 * torch.randn(mod.weight.shape, generator=g))
                    mod.bias.copy_(0.1 * torch.randn(mod.bias.shape, generator=g))
        for mod in enc.pre_encode.conv:
            if isinstance(mod, torch.nn.Conv2d):
                mod.weight.normal_(0.0, mod.weight[0].numel() ** -0.5, generator=g)
    enc = enc.to(dt).eval().requires_grad_(False)
    sd = {k: v.double().numpy() for k, v in enc.state_dict().items()}
    return enc, sd


_GPU_RUNS: dict = {}


def _gpu_run(cuda, case, replay, seed=21):
    """The GPU's outputs of every step and the oracle front end's frames for the
    same pcm (computed once per case and mode, shared by the parity check and the
    planted-mistake checks)."""
    key = (case, replay, seed)
    if key in _GPU_RUNS:
        return _GPU_RUNS[key]
    D, H, Ly, K, left, right, n_mels, C, dt, B, steps, n_first, n_next, ring, mrows = CASES[case]
    T = right + 1
    enc, sd = _model(case, seed)
    sub_sd = {k[len("pre_encode."):]: v for k, v in sd.items() if k.startswith("pre_encode.")}
    enc = enc.to(cuda)
    fx = FeatureExtractor(n_mels=n_mels, dither=1e-5, seed=seed, device=cuda)
    pre = PreEncoder(fx, enc.pre_encode, num_slots=B, device=cuda, ring_size=ring, mel_rows=mrows)
    slots = np.arange(B)
    for s in slots:
        pre.reset_slot(s)
    p = ofe.FeParams(n_mels=n_mels, dither=1e-5)
    fe_states = [ofe.PreEncodeState(ofe.FeState(p, noise_id=int(pre.noise_id[s]), seed=seed), sub_sd) for s in slots]
    state = enc.init_streaming_state(batch_size=B, device=cuda, dtype=dt)
    length = torch.full((B,), T, dtype=torch.int64, device=cuda)
    graph = EncoderStepGraph(enc, state, length) if replay else None
    pcm = _pcm(B, n_first + steps * n_next, seed)
    pos = 0
    outs, frames = [], []
    with torch.no_grad():
        for step in range(steps):
            n = n_first if step == 0 else n_next
            print(f"  [{case} replay={replay}] step {step}", flush=True)
            rows, counts, first = pre.step(slots, torch.from_numpy(pcm[:, pos : pos + n].copy()).to(cuda), n, False)
            assert (counts == T).all() and (first == T * slots).all(), (counts, first)
            x = rows.view(B, T, D)
            out = graph(x) if replay else enc(x, state, length=length)[0]
            outs.append(out.double().cpu().numpy())
            frames.append(np.stack([fe_states[b].push(pcm[b, pos : pos + n].astype(np.float32) / 32768.0)
                                    for b in range(B)]))
            pos += n
        assert state.processed_frames.tolist() == [steps * T] * B
        assert state.cache_lengths.tolist() == [min(steps * T, left)] * B
    torch.cuda.synchronize()
    _GPU_RUNS[key] = (outs, frames, sd)
    return _GPU_RUNS[key]


def _run(cuda, case, replay, seed=21, planted=None):
    """(worst max-abs, worst per-step RMS) of the GPU's outputs against the
    oracle's encoder steps over the same front-end frames (with ``planted``: an
    oracle carrying a mistake)."""
    D, H, Ly, K, left, right, n_mels, C, dt, B, steps = CASES[case][:11]
    T = right + 1
    outs, frames, sd = _gpu_run(cuda, case, replay, seed)
    ost = oe.EncoderState(B, Ly, left, right, D, K)
    pe = relpos.sinusoid_table(5000, D).astype(np.float64)
    if planted is not None:
        sd, pe = planted(sd, pe)
    worst = worst_rms = 0.0
    for got, X in zip(outs, frames):
        ref = oe.encoder_step(X, sd, ost, np.full(B, T), Ly, H, pe)
        err = np.abs(got - ref)
        worst = max(worst, float(err.max()))
        worst_rms = max(worst_rms, float(np.sqrt((err**2).mean())))
    return worst, worst_rms


@pytest.mark.parametrize("replay", [False, True])
@pytest.mark.parametrize("case", sorted(CASES))
def test_pcm16_encoder_step_matches_oracle(cuda, case, replay):
    print(f"\n[e2e] {case} replay={replay}", flush=True)
    worst, rms = _run(cuda, case, replay)
    tmax, trms = TOL[CASES[case][8]]
    print(f"  worst max-abs {worst:.3e} (bar {tmax:.1e}), worst step rms {rms:.3e} (bar {trms:.1e})", flush=True)
    assert worst <= tmax and rms <= trms, (worst, rms)


def _plant_reversed_positions(sd, pe):
    """Relative position r read as -r (the table flipped)."""
    return sd, pe[::-1].copy()


def _plant_conv_tap(sd, pe):
    """Depthwise taps applied one frame late."""
    sd = dict(sd)
    w = sd["layers.1.conv.depthwise_conv.weight"]
    sd["layers.1.conv.depthwise_conv.weight"] = np.concatenate([w[:, :, 1:], w[:, :, :1]], axis=2)
    return sd, pe


def _plant_ff_unscaled(sd, pe):
    """The second feed-forward branch of layer 1 added without its 0.5 (its
    output layer doubled)."""
    sd = dict(sd)
    sd["layers.1.feed_forward2.linear2.weight"] = 2.0 * sd["layers.1.feed_forward2.linear2.weight"]
    return sd, pe


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("planted", [_plant_reversed_positions, _plant_conv_tap, _plant_ff_unscaled],
                         ids=["positions_reversed", "conv_taps_shifted", "ff_unscaled"])
def test_planted_oracle_mistake_exceeds_the_bar(cuda, planted, case):
    """The same GPU run against an oracle carrying a plausible mistake: the
    difference must exceed the max-abs or the RMS bar, so the bars would catch
    it.  (A mistake in a bias term, pos_bias_v dropped, moves the outputs of the
    stack by less than the model dtype's rounding; it is caught at the kernel
    level, test_gpu_attention.py::test_planted_bias_mistakes_exceed_the_kernel_bar.)"""
    print(f"\n[e2e planted] {case} {planted.__name__}", flush=True)
    worst, rms = _run(cuda, case, False, planted=planted)
    tmax, trms = TOL[CASES[case][8]]
    print(f"  planted worst max-abs {worst:.3e} (bar {tmax:.1e}), worst step rms {rms:.3e} (bar {trms:.1e})", flush=True)
    assert worst > tmax or rms > trms, (worst, rms)
