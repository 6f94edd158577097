"""The batched pre-encode front end on the GPU (pk_fe_step, pk_subsample) against
the oracle (oracle/frontend.py, pinned in test_oracle_frontend.py).

Bars:
* log-mel (fp32 on both sides of the reference): per value
  |got - ref| <= 8e-6 + 128 eps32 sqrt(E_frame S_m / mel_m), where E_frame is the
  windowed frame's energy, S_m the filter's weight sum and eps32 = 2^-24 -- the
  first-order error of an fp32 FFT + filterbank; the reference's own fp32
  computation (torch.stft) reaches 42x that scale on these signals, so the bar
  leaves 3x;
* subsampling (every layer's output rounded to the model dtype):
  |got - ref| <= 4 eps (|ref| + rms(ref)), eps = 2^-10 fp16, 2^-7 bf16 (an
  fp32-accumulating emulation reaches 1.2 eps), 2^-17 fp32 (fp32 sums of 256
  products), against the oracle fed the GPU's own features;
* frame counts, windows, drops and row counts: exact.
"""

import numpy as np
import pytest
import torch

from oracle import frontend as fe
from parakeet_amd.modules.frontend import ConvSubsampling, FeatureExtractor, PreEncoder, stack_len

pytestmark = pytest.mark.gpu

EPS = {torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7, torch.float32: 2.0**-17}


def _pcm(n, seed, silence=0):
    """Sum of 3 sinusoids (100-4000 Hz) + noise at 20 dB SNR, as int16 pcm."""
    rng = np.random.default_rng(seed)
    t = np.arange(n) / 16000.0
    sig = sum(rng.uniform(0.05, 0.3) * np.sin(2 * np.pi * rng.uniform(100, 4000) * t + rng.uniform(0, 6)) for _ in range(3))
    sig = sig + rng.standard_normal(n) * np.sqrt(np.mean(sig**2) / 100.0)
    pcm = np.clip(np.round(sig * 32767.0), -32768, 32767).astype(np.int16)
    pcm[:silence] = 0
    return pcm


def _logmel_bound(x: np.ndarray, p, noise, ref: np.ndarray) -> np.ndarray:
    xd = np.asarray(x, dtype=np.float64) + (0.0 if noise is None else noise * p.dither)
    frames = fe.frames_of(fe.preemphasis(xd, p), p, 0, ref.shape[1])
    e_frame = (frames**2).sum(1)
    s_m = p.fb.astype(np.float64).sum(1)
    mel = np.exp(ref) - p.guard
    return 8e-6 + 128 * 2.0**-24 * np.sqrt(e_frame[None, :] * s_m[:, None] / np.maximum(mel + p.guard, 1e-300))


def _close_logmel(got, ref, bound, what):
    err = np.abs(got - ref)
    assert (err <= bound).all(), f"{what}: max excess {(err - bound).max():.3e} (max err {err.max():.3e})"


def _close_sub(got, ref, dt, what):
    rms = np.sqrt((ref**2).mean()) if ref.size else 0.0
    lim = 4 * EPS[dt] * (np.abs(ref) + rms)
    err = np.abs(got - ref)
    assert (err <= lim).all(), f"{what}: max excess {(err - lim).max():.3e}, max err {err.max():.3e}, rms {rms:.3e}"


SCHEDULES = [
    [1440] + [2560] * 5,  # the reference's chunking (model_runner.py:53-56)
    [100, 300, 17, 2600, 1, 5000, 640],  # pushes that emit nothing in between
    [256, 3000, 7000],
]


@pytest.mark.parametrize("n_mels", [80, 128])
@pytest.mark.parametrize("dither", [0.0, 1e-5])
def test_streamed_features_match_oracle(cuda, n_mels, dither):
    """Three streams with different push schedules in one batch per step; the
    last push of each is final (feature_extractor.py:111-112)."""
    fx = FeatureExtractor(n_mels=n_mels, dither=dither, seed=77, device=cuda)
    p = fe.FeParams(n_mels=n_mels, dither=dither)
    pre = PreEncoder(fx, None, num_slots=5, device=cuda)
    slots = [3, 0, 4]
    for s in slots:
        pre.reset_slot(s)
    sigs = [_pcm(sum(sc) + 10, seed=i, silence=2000 * (i == 1)) for i, sc in enumerate(SCHEDULES)]
    states = [fe.FeState(p, noise_id=int(pre.noise_id[s]), seed=77, dither=dither > 0) for s in slots]
    got = [[] for _ in slots]
    pos = [0] * 3
    for step in range(max(len(sc) for sc in SCHEDULES)):
        n_new = np.array([sc[step] if step < len(sc) else 0 for sc in SCHEDULES])
        final = np.array([step == len(sc) - 1 for sc in SCHEDULES])
        pcm = np.zeros((3, max(int(n_new.max()), 1)), dtype=np.int16)
        for i in range(3):
            pcm[i, : n_new[i]] = sigs[i][pos[i] : pos[i] + n_new[i]]
        plan, _, _ = pre._features(np.array(slots), torch.from_numpy(pcm).to(cuda), n_new, final)
        _, start, n_frames, *_ = plan
        torch.cuda.synchronize()
        for i, s in enumerate(slots):
            ref = states[i].push(sigs[i][pos[i] : pos[i] + n_new[i]].astype(np.float32) / 32768.0, bool(final[i]))
            assert (ref is None) == (n_frames[i] == 0), f"stream {i} step {step}: frame count"
            if ref is not None:
                assert ref.shape[1] == n_frames[i] and states[i].last_start == start[i]
                rows = (start[i] + np.arange(n_frames[i])) % pre.mel_rows
                got[i].append(pre.mel_ring[s].cpu().numpy()[rows].T)
            pos[i] += n_new[i]
        assert list(pre.emitted[slots]) == [st.emitted for st in states]
        assert list(pre.offset[slots]) == [st.offset for st in states]
    for i in range(3):
        x = sigs[i][: pos[i]].astype(np.float32) / 32768.0
        noise = fe.dither_normal(77, int(pre.noise_id[slots[i]]), np.arange(pos[i])) if dither else None
        ref = fe.log_mel(x, p, noise)
        g = np.concatenate(got[i], axis=1).astype(np.float64)
        assert g.shape == ref.shape
        _close_logmel(g, ref, _logmel_bound(x, p, noise, ref), f"stream {i}")


def test_dither_noise_matches_oracle(cuda):
    """Dither 1.0 on silence: the features are those of the Philox/Box-Muller
    noise alone, so a wrong generator, key or index shows at full scale."""
    fx = FeatureExtractor(n_mels=80, dither=1.0, seed=(5 << 32) | 9, device=cuda)
    p = fe.FeParams(n_mels=80, dither=1.0)
    x = np.zeros(4000, dtype=np.float32)
    got = fx._compute_features(x, noise_id=123)[0].cpu().numpy().astype(np.float64)
    noise = fe.dither_normal((5 << 32) | 9, 123, np.arange(4000))
    ref = fe.log_mel(x, p, noise)
    _close_logmel(got, ref, _logmel_bound(x, p, noise, ref), "noise features")
    assert np.std(ref) > 0.5  # the comparison is not on a flat floor


@pytest.mark.parametrize("n", [100, 16000, 48317])
def test_offline_call_matches_oracle(cuda, n):
    fx = FeatureExtractor(n_mels=128, dither=0.0, device=cuda)
    p = fe.FeParams(n_mels=128, dither=0.0)
    x = _pcm(n, seed=n).astype(np.float32) / 32768.0
    got = fx(x)[0].cpu().numpy().astype(np.float64)
    ref = fe.log_mel(x, p)
    assert got.shape == ref.shape == (128, 1 + n // 160)
    _close_logmel(got, ref, _logmel_bound(x, p, None, ref), "offline")


def _module(C, Fm, D, dt, cuda, seed):
    torch.manual_seed(seed)
    m = ConvSubsampling(D, C, Fm, 8)
    with torch.no_grad():
        for mod in m.conv:
            if isinstance(mod, torch.nn.Conv2d):
                fan = mod.weight[0].numel()
                mod.weight.normal_(0, fan**-0.5)
                mod.bias.normal_(0, 0.1)
    return m.requires_grad_(False).to(dt).to(cuda)


def _sd(m):
    return {k: v.detach().double().cpu().numpy() for k, v in m.state_dict().items()}


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Fm,C", [(80, 256), (128, 256), (80, 64), (40, 128)])
def test_subsampling_matches_oracle(cuda, dt, Fm, C):
    """ConvSubsampling.forward over a batch of feature sequences with partial
    lengths (subsample.py:140-152 with the masks of :30-57)."""
    D = 64
    m = _module(C, Fm, D, dt, cuda, seed=Fm + C)
    g = torch.Generator().manual_seed(Fm)
    B, T = 4, 41
    x = (torch.randn(B, T, Fm, generator=g) * 3 - 8).to(cuda)
    lengths = torch.tensor([41, 30, 7, 1])
    y, out_len = m(x, lengths)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (B, stack_len(T), D)
    sd = _sd(m)
    rec = np.zeros(B, dtype=[(n, "<i4") for n in ("slot", "row0", "rows", "length", "drop", "n_out", "out_row", "reserved")])
    for b in range(B):
        rec[b] = (b, 0, T, int(lengths[b]), 0, stack_len(T), b * stack_len(T), 0)
    flat = m.stack(x.float().contiguous(), rec, False, B * stack_len(T), stack_len(T)).double().cpu().numpy()
    for b in range(B):
        ref_flat, L = fe.conv_subsample(x[b].double().cpu().numpy(), int(lengths[b]), sd, dt, linear=False)
        assert int(out_len[b]) == L
        _close_sub(flat[b * stack_len(T) : (b + 1) * stack_len(T)], ref_flat, dt, f"stream {b} stack")
    # `out` is a plain GEMM on the stack output
    ref_y = flat @ sd["out.weight"].T + sd["out.bias"]
    _close_sub(y.double().cpu().numpy().reshape(-1, D), ref_y, dt, "out")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Fm", [80, 128])
@pytest.mark.parametrize("B", [64, 384])
def test_subsampling_tile_shapes_agree(cuda, dt, Fm, B):
    """The 16-bit stack kernel takes two output frames a workgroup when
    one-frame workgroups would not all fit on the CUs at once, one frame
    otherwise; with at least four two-frame tiles a CU (384 streams at 80 mels)
    it runs them in workgroups of 8 waves, two a CU, that take the second
    depthwise conv and conv.6 in two channel halves.  The same streams
    (partial lengths, frames dropped at the front of some) as one batch and in
    batches of 4 (one-frame tiles) give the same bits: every output is the same
    sums in the same order.  Three of them also match the oracle."""
    C, D = 256, 64
    m = _module(C, Fm, D, dt, cuda, seed=7 * Fm)
    T = 41
    T3 = stack_len(T)
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    assert B * T3 > cus >= 4 * T3, (B * T3, cus)  # one batch: two-frame tiles; 4 streams: one-frame
    g = torch.Generator().manual_seed(Fm + B)
    x = (torch.randn(B, T, Fm, generator=g) * 3 - 8).to(cuda).contiguous()
    rng = np.random.default_rng(Fm + B)
    lengths = rng.integers(1, T + 1, size=B)
    drops = rng.integers(0, 3, size=B)
    names = ("slot", "row0", "rows", "length", "drop", "n_out", "out_row", "reserved")
    def records(slots, first_row):
        rec = np.zeros(len(slots), dtype=[(n, "<i4") for n in names])
        for i, b in enumerate(slots):
            n_out = T3 - int(drops[b])
            rec[i] = (b, 0, T, int(lengths[b]), int(drops[b]), n_out, first_row + i * T3, 0)
        return rec
    whole = m.stack(x, records(range(B), 0), False, B * T3, T3)
    parts = torch.zeros_like(whole)
    for b0 in range(0, B, 4):
        rec = records(range(b0, b0 + 4), 0)
        parts[b0 * T3 : (b0 + 4) * T3] = m.stack(x, rec, False, 4 * T3, T3)
    torch.cuda.synchronize()
    for b in range(B):
        n_out = T3 - int(drops[b])
        got, ref = whole[b * T3 : b * T3 + n_out], parts[b * T3 : b * T3 + n_out]
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"stream {b}: tile shapes differ"
    sd = _sd(m)
    for b in (0, 17, B - 1):
        ref_flat, _ = fe.conv_subsample(x[b].double().cpu().numpy(), int(lengths[b]), sd, dt, linear=False)
        n_out = T3 - int(drops[b])
        got = whole[b * T3 : b * T3 + n_out].double().cpu().numpy()
        _close_sub(got, ref_flat[int(drops[b]) :], dt, f"stream {b} stack")


# (n_mels, d_model, first chunk, next chunk, frames per step, sample ring,
# mel ring, steps): the small model's chunking (right context 1: 9 then 16 mel
# frames) and the large model's (right context 13: 105 then 112 mel frames,
# 128 mels; config.py:5-31, model_runner.py:53-56) with rings sized for it
PRE_CONFIGS = {
    "small": (80, 512, 1440, 2560, 2, 8192, 64, 6),
    "large": (128, 1024, 16800, 17920, 14, 32768, 256, 5),
}


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cfg", sorted(PRE_CONFIGS))
def test_pre_encoder_stream_matches_oracle(cuda, dt, cfg):
    """_run_pre_encode (model_runner.py:181-252) for 6 streams: starts
    staggered, the reference's chunking (first chunk, then the next-chunk size),
    one stream finishing with a short final push.  Windows and row counts are
    exact; rows match the oracle's subsampling of the GPU's own window."""
    Fm, D, n_first, n_next, T_out, ring, mrows, steps = PRE_CONFIGS[cfg]
    C = 256
    fx = FeatureExtractor(n_mels=Fm, dither=1e-5, seed=3, device=cuda)
    m = _module(C, Fm, D, dt, cuda, seed=11)
    pre = PreEncoder(fx, m, num_slots=8, device=cuda, ring_size=ring, mel_rows=mrows)
    p = fe.FeParams(n_mels=Fm, dither=1e-5)
    sd = _sd(m)
    slots = np.array([5, 1, 7, 0, 2, 6])
    for s in slots:
        pre.reset_slot(s)
    start_step = [0, 0, 1, 2, 2, 3]
    sigs = [_pcm(n_first + steps * n_next, seed=20 + i) for i in range(6)]
    states = [fe.PreEncodeState(fe.FeState(p, noise_id=int(pre.noise_id[s]), seed=3), sd, store_dtype=dt) for s in slots]
    pos = [0] * 6
    for step in range(steps):
        live = [i for i in range(6) if step >= start_step[i]]
        n_new, final = [], []
        for i in live:
            k = step - start_step[i]
            n = n_first if k == 0 else n_next
            if i == 3 and k == 2:
                n, fin = 1000, True
            else:
                fin = False
            if i == 3 and k > 2:
                n = 0
            n_new.append(n)
            final.append(fin)
        pcm = np.zeros((len(live), n_next), dtype=np.int16)
        for r, i in enumerate(live):
            pcm[r, : n_new[r]] = sigs[i][pos[i] : pos[i] + n_new[r]]
        rows, counts, first = pre.step(slots[live], torch.from_numpy(pcm).to(cuda), np.array(n_new), np.array(final))
        torch.cuda.synchronize()
        rows = rows.double().cpu().numpy()
        mel = pre.mel_ring.cpu().numpy()
        for r, i in enumerate(live):
            x = sigs[i][pos[i] : pos[i] + n_new[r]].astype(np.float32) / 32768.0
            st = states[i]
            had_cache = st.cache is not None
            feats = st.fe.push(x, final[r]) if n_new[r] else None
            if feats is None:
                assert counts[r] == 0
            else:
                # the oracle's window bookkeeping, fed the GPU's features of that window
                win = feats if not had_cache else np.concatenate([st.cache, feats], axis=1)
                W = win.shape[1]
                w0, wl = pre.last_window[slots[i]]
                assert wl == W and w0 == st.fe.last_start - (W - feats.shape[1])
                gwin = mel[slots[i]][(w0 + np.arange(W)) % pre.mel_rows].astype(np.float64)  # [W, F]
                ref, _ = fe.conv_subsample(gwin, W, sd, dt, linear=False)
                ref = ref[2:] if had_cache else ref
                assert counts[r] == ref.shape[0]
                if not final[r]:
                    assert counts[r] == T_out  # 1 + 8R frames first, then 8 + 8R (model_runner.py:53-56)
                flat_ref = ref @ sd["out.weight"].T + sd["out.bias"]
                got = rows[first[r] : first[r] + counts[r]]
                _close_sub(got, flat_ref, dt, f"stream {i} step {step}")
                st.cache = win[:, -9:] if W >= 9 else win
            pos[i] += n_new[r]


def test_pre_encoder_rejects_oversized_pushes(cuda):
    fx = FeatureExtractor(n_mels=80, device=cuda)
    pre = PreEncoder(fx, None, num_slots=2, device=cuda, ring_size=4096, mel_rows=32)
    pcm = torch.zeros((1, 8000), dtype=torch.int16, device=cuda)
    with pytest.raises(RuntimeError, match="ring"):
        pre._features(np.array([0]), pcm, 8000, False)


def test_front_end_batch_over_one_launch(cuda):
    """65,540 streams in one step: pk_fe_step and pk_subsample take more
    streams than one launch grid holds (65,535 along its y / z extent) in
    several launches.  Every stream gets the same pcm without dither, so every
    stream's log-mel rows and subsampling output rows (before the ``out``
    Linear, whose library GEMM may round differently at another row count)
    equal those of the same signal run alone (4 streams in a batch), the
    streams past the first launch included."""
    from parakeet_amd import ops

    B, Fm, D, C = 65540, 80, 64, 256
    dt = torch.float16
    m = _module(C, Fm, D, dt, cuda, seed=5)
    sig = _pcm(1440 + 2 * 2560, seed=31)
    chunks = [sig[:1440], sig[1440:4000], sig[4000:6560]]

    def run(n):
        fx = FeatureExtractor(n_mels=Fm, dither=0.0, device=cuda)
        pre = PreEncoder(fx, m, num_slots=n, device=cuda)
        slots = np.arange(n)
        for s in slots:
            pre.reset_slot(s)
        out = []
        for ch in chunks:
            pcm = torch.from_numpy(np.ascontiguousarray(np.broadcast_to(ch, (n, len(ch))))).to(cuda)
            plan, sel, out_row = pre._features(slots, pcm, len(ch), False)
            n_out = plan[6]
            R = int(n_out.sum())
            flat = torch.empty((R, C * m.final_freq_dim), dtype=dt, device=cuda)
            if R:
                ops.subsample(pre.hdr[32 * n :], len(sel), pre.mel_ring, True, m.conv_weights(), flat,
                              max_out=int(n_out.max()))
            out.append((flat, n_out.copy(), out_row.copy()))
        torch.cuda.synchronize()
        return pre, out

    small_pre, small = run(4)
    big_pre, big = run(B)
    n_rows = 0
    for (fs_, cs, rs), (fb_, cb, rb) in zip(small, big):
        assert (cb == cs[0]).all()
        ref = fs_[rs[0] : rs[0] + cs[0]].view(torch.int16)
        for b in (0, 1, 65534, 65535, 65536, B - 1):
            got = fb_[rb[b] : rb[b] + cb[b]].view(torch.int16)
            assert torch.equal(got, ref), f"stream {b}: subsampling rows differ"
        n_rows += int(cs[0])
    assert n_rows > 0
    ref_mel = small_pre.mel_ring[0]
    for b in (65534, 65535, B - 1):
        assert torch.equal(big_pre.mel_ring[b], ref_mel), f"stream {b}: log-mel ring differs"


@pytest.mark.parametrize("dither", [0.0, 1e-5])
def test_features_four_frames_a_wave_form(cuda, dither):
    """With several workgroups a CU of 16 frames (here 2,100 streams of 16
    frames), pk_fe_step takes four frames a wave, so a workgroup stages its
    twiddles, window and filterbank once for 16 frames.  The log-mel rows of
    four streams equal, bit for bit, those of the same four streams stepped
    alone (one frame a wave), dither included (every stream's noise is a
    function of its own sample indices)."""
    S, Fm = 2100, 80
    sig = _pcm(1440 + 2 * 2560, seed=41)
    chunks = [sig[:1440], sig[1440:4000], sig[4000:6560]]
    probe = np.array([0, 1, 1000, S - 1])

    def run(slots):
        fx = FeatureExtractor(n_mels=Fm, dither=dither, seed=9, device=cuda)
        pre = PreEncoder(fx, None, num_slots=S, device=cuda)
        for s in range(S):
            pre.reset_slot(s)
        for ch in chunks:
            pcm = torch.from_numpy(np.ascontiguousarray(np.broadcast_to(ch, (len(slots), len(ch))))).to(cuda)
            plan, _, _ = pre._features(slots, pcm, len(ch), False)
        torch.cuda.synchronize()
        return pre

    big = run(np.arange(S))
    small = run(probe)
    assert int(big.emitted[0]) > 16  # three pushes emitted more frames than one
    for s in probe:
        assert torch.equal(big.mel_ring[s], small.mel_ring[s]), f"stream {s}: log-mel rows differ"
