"""Pins for the front-end oracle (oracle/frontend.py).

The reference ships no tests or fixtures for its feature extractor or its
subsampling; each restated function is checked against an independent
implementation or a property the algorithm fixes:

* Philox4x32-10 against the Random123 known-answer vectors;
* the Slaney filterbank against transformers' mel_filter_bank (its own
  restatement of librosa's algorithm); the window against torch.hann_window;
* log_mel against the reference's operator sequence run through torch.stft in
  float64 (feature_extractor.py:63-88);
* the streaming push against the offline features of the whole signal: every
  emitted frame equals the offline frame (the trim never cuts into a window);
* conv_subsample against the reference's layer stack rebuilt from torch's
  F.pad / F.conv2d with its masks (subsample.py:30-57,140-152,
  convolution.py:94-104), at full and partial lengths;
* the streaming pre-encode: the outputs kept after the drop do not depend on
  the zero padding in front of the window (a longer left history gives the
  same rows), and the reference's chunk schedule yields 2 rows per chunk.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import frontend as fe


def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds
    got = fe.philox4x32_10((0, 0, 0, 0), (0, 0))
    assert [int(v) for v in got] == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    got = fe.philox4x32_10((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0))
    assert [int(v) for v in got] == [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_dither_is_standard_normal_and_keyed():
    z = fe.dither_normal(7, 3, np.arange(200_000))
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1.0) < 0.02
    assert abs((np.abs(z) < 1.0).mean() - 0.6827) < 0.005
    # a function of (seed, stream, index): the same index gives the same value
    assert np.array_equal(fe.dither_normal(7, 3, [5, 100_000]), z[[5, 100_000]])
    assert not np.allclose(fe.dither_normal(7, 4, np.arange(16)), z[:16])
    assert not np.allclose(fe.dither_normal(8, 3, np.arange(16)), z[:16])
    # Box-Muller pairs: samples 4j, 4j+1 (and 4j+2, 4j+3) are the cos and sin of
    # one angle on one radius, the radius from the Philox draw of counter j
    # (pinned by the known answers above), so their squares sum to -2 ln u1;
    # within and across pairs the samples are uncorrelated
    j = np.arange(50_000)
    r0, _, r2, _ = fe.philox4x32_10((j, np.zeros_like(j), np.full_like(j, 3), np.zeros_like(j)), (7, 0))
    zz = z.reshape(-1, 4)
    for k, r in ((0, r0), (2, r2)):
        rad2 = -2.0 * np.log((r.astype(np.float64) + 1.0) * 2.0**-32)
        np.testing.assert_allclose(zz[:, k] ** 2 + zz[:, k + 1] ** 2, rad2, rtol=1e-12, atol=1e-12)
    for a, b in ((0, 1), (1, 2), (2, 3), (0, 2)):
        assert abs(np.corrcoef(zz[:, a], zz[:, b])[0, 1]) < 0.02


@pytest.mark.parametrize("n_mels,fmax", [(80, None), (128, None), (64, 6000.0)])
def test_mel_filterbank_matches_an_independent_slaney_implementation(n_mels, fmax):
    from transformers.audio_utils import mel_filter_bank

    ref = mel_filter_bank(
        num_frequency_bins=257, num_mel_filters=n_mels, min_frequency=0.0,
        max_frequency=fmax or 8000.0, sampling_rate=16000, norm="slaney", mel_scale="slaney",
    ).T
    got = fe.mel_filterbank(16000, 512, n_mels, 0.0, fmax)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-9)


def test_slaney_scale_round_trips_and_breaks_at_1khz():
    f = np.array([0.0, 200.0, 999.0, 1000.0, 4000.0, 8000.0])
    np.testing.assert_allclose(fe.mel_to_hz(fe.hz_to_mel(f)), f, rtol=1e-12, atol=1e-9)
    assert fe.hz_to_mel(1000.0) == pytest.approx(15.0)
    assert fe.hz_to_mel(6400.0) == pytest.approx(15.0 + 27.0)  # log step ln(6.4)/27


def test_hann_window_matches_torch():
    np.testing.assert_allclose(fe.hann(400), torch.hann_window(400, periodic=False).numpy(), atol=2.0**-22)


def _signal(n, seed=0):
    rng = np.random.default_rng(seed)
    t = np.arange(n) / 16000.0
    x = 0.3 * np.sin(2 * np.pi * 440 * t) + 0.1 * np.sin(2 * np.pi * 2500 * t) + 0.05 * rng.standard_normal(n)
    return x.astype(np.float32)


def _torch_features(x: np.ndarray, p, noise=None) -> np.ndarray:
    """feature_extractor.py:63-88 operator for operator, float64."""
    xt = torch.from_numpy(x.astype(np.float64))[None]
    if noise is not None:
        xt = xt + torch.from_numpy(noise)[None] * p.dither
    right = xt[:, 1:] - p.preemph * xt[:, :-1]
    xt = torch.cat((xt[:, :1], right), dim=-1)
    st = torch.stft(xt, n_fft=p.n_fft, hop_length=p.hop, win_length=p.win,
                    window=torch.from_numpy(p.window.astype(np.float64)),  # pinned on its own
                    center=True, return_complex=True, pad_mode="constant")
    spec = torch.view_as_real(st)
    spec = torch.sqrt(spec.pow(2).sum(-1)).pow(p.mag_power)
    mel = torch.matmul(torch.from_numpy(p.fb.astype(np.float64)), spec)
    return torch.log(mel + p.guard)[0].numpy()


@pytest.mark.parametrize("n_mels,n", [(80, 16000), (128, 3001), (128, 100)])
def test_log_mel_matches_the_reference_operator_sequence(n_mels, n):
    p = fe.FeParams(n_mels=n_mels)
    x = _signal(n)
    noise = fe.dither_normal(1, 2, np.arange(n))
    got = fe.log_mel(x, p, noise)
    ref = _torch_features(x, p, noise)
    assert got.shape == ref.shape == (n_mels, 1 + n // 160)
    np.testing.assert_allclose(got, ref, atol=1e-10)


def test_silence_is_the_log_guard():
    p = fe.FeParams(n_mels=80)
    got = fe.log_mel(np.zeros(1000, np.float32), p)
    assert np.all(got == np.log(2.0**-24))


def test_tone_lands_in_its_mel_band():
    p = fe.FeParams(n_mels=128)
    t = np.arange(8000) / 16000.0
    got = fe.log_mel(np.sin(2 * np.pi * 1000.0 * t).astype(np.float32), p)
    band = int(np.argmax(got[:, 25]))
    centre = fe.mel_to_hz(np.linspace(0, fe.hz_to_mel(8000.0), 130))[band + 1]
    assert abs(centre - 1000.0) < 60.0


SCHEDULES = [
    [1440] + [2560] * 6,  # the reference's chunking: 1 + 8 frames, then 16 frames
    [100, 100, 100, 17, 3000, 1, 2559, 640],  # pushes that emit nothing in between
    [7000],
    [256, 1, 4000],
]


@pytest.mark.parametrize("sched", SCHEDULES)
@pytest.mark.parametrize("dither", [False, True])
def test_streamed_push_equals_offline_features(sched, dither):
    p = fe.FeParams(n_mels=80)
    x = _signal(sum(sched) + 1000, seed=3)
    st = fe.FeState(p, noise_id=11, seed=5, dither=dither)
    outs, pos = [], 0
    for i, n in enumerate(sched):
        final = i == len(sched) - 1
        emitted_before = st.emitted
        o = st.push(x[pos : pos + n], final=final)
        pos += n
        if o is not None:
            assert st.last_start == emitted_before  # frames come out in order, none skipped
            outs.append(o)
        # the kept samples start at most one frame hop before what the next window needs
        assert st.offset <= max(0, st.emitted * p.hop - p.n_fft // 2)
    s = np.concatenate(outs, axis=1)
    noise = fe.dither_normal(5, 11, np.arange(pos)) if dither else None
    off = fe.log_mel(x[:pos], p, noise)
    assert s.shape == (80, pos // p.hop + 1)  # the final push emits through total // hop
    np.testing.assert_allclose(s, off, atol=1e-12)


def test_push_edge_cases():
    p = fe.FeParams(n_mels=80)
    st = fe.FeState(p, dither=False)
    assert st.push(np.zeros(0, np.float32)) is None
    assert st.push(np.ones(256, np.float32)) is None  # total <= n_fft/2
    assert st.push(np.ones(0, np.float32), final=True) is None  # an empty final push emits nothing
    o = st.push(np.ones(1, np.float32))
    assert o.shape == (80, 1) and st.emitted == 1  # (257 - 256) // 160 = 0


def _sub_params(C, Fm, D, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    F3 = fe.calc_length(Fm)
    sd = {
        "conv.0.weight": torch.randn(C, 1, 3, 3, generator=g) / 3,
        "conv.2.weight": torch.randn(C, 1, 3, 3, generator=g) / 3,
        "conv.3.weight": torch.randn(C, C, 1, 1, generator=g) / C**0.5,
        "conv.5.weight": torch.randn(C, 1, 3, 3, generator=g) / 3,
        "conv.6.weight": torch.randn(C, C, 1, 1, generator=g) / C**0.5,
        "out.weight": torch.randn(D, C * F3, generator=g) / (C * F3) ** 0.5,
        "out.bias": torch.randn(D, generator=g) * 0.1,
    }
    if bias:
        for k in ("conv.0", "conv.2", "conv.3", "conv.5", "conv.6"):
            sd[k + ".bias"] = torch.randn(C, generator=g) * 0.1
    return {k: v.double() for k, v in sd.items()}


def _torch_subsample(x, lengths, sd, C):
    """MaskedConvSequential + ConvSubsampling.forward rebuilt from torch ops
    (subsample.py:30-57,140-152; CausalConv2D = F.pad(2, 1, 2, 1) + conv2d)."""
    x = x.unsqueeze(1)

    def mask(t, L):
        return (torch.arange(t.shape[2])[None] < L[:, None]).double()[:, None, :, None]

    cur = lengths.clone()
    m = mask(x, cur)
    layers = [("conv.0", 2, 1, 3), None, ("conv.2", 2, C, 3), ("conv.3", 1, 1, 1), None,
              ("conv.5", 2, C, 3), ("conv.6", 1, 1, 1), None]
    for layer in layers:
        x = x * m
        if layer is None:
            x = torch.relu(x)
            continue
        name, stride, groups, k = layer
        if k == 3:
            x = F.pad(x, (2, 1, 2, 1))
        x = F.conv2d(x, sd[name + ".weight"], sd.get(name + ".bias"), stride=stride, groups=groups)
        if stride != 1:
            cur = (cur + 2 + 1 - 3) // 2 + 1
            m = mask(x, cur)
    x = x * m
    b, c, t, f = x.shape
    return x.transpose(1, 2).reshape(b, t, -1) @ sd["out.weight"].T + sd["out.bias"], cur


@pytest.mark.parametrize("Fm,bias", [(80, True), (128, False)])
def test_conv_subsample_matches_torch_layers(Fm, bias):
    C, D = 32, 48
    sd = _sub_params(C, Fm, D, seed=Fm, bias=bias)
    x = torch.randn(4, 25, Fm, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    lens = torch.tensor([25, 17, 4, 1])
    ref, ref_len = _torch_subsample(x, lens, sd, C)
    for b in range(4):
        y, L = fe.conv_subsample(x[b].numpy(), int(lens[b]), {k: v.numpy() for k, v in sd.items()})
        assert L == int(ref_len[b]) and y.shape == (4, D)
        np.testing.assert_allclose(y, ref[b].numpy(), atol=1e-12)


def test_lengths_closed_forms():
    assert fe.calc_length(80) == 11 and fe.calc_length(128) == 17
    for T in range(0, 40):
        L1 = fe.conv_out_len(T)
        assert L1 == (T + 3 - 3) // 2 + 1
        assert fe.calc_length(T, repeat_num=1) == L1
        # the padded conv's output length is the mask length at full input
        assert (T + 3 - 3) // 2 + 1 == fe.conv_out_len(T)


@pytest.mark.parametrize("store", [None, torch.float16])
def test_kept_rows_do_not_see_the_window_padding(store):
    """The drop of 2 leading outputs (model_runner.py:222-223) removes exactly
    the rows whose receptive field reaches the zero padding in front of the
    window: the kept rows equal the rows of a run over a longer history."""
    C, Fm, D = 16, 80, 32
    sd = {k: v.numpy() for k, v in _sub_params(C, Fm, D, seed=3).items()}
    rng = np.random.default_rng(4)
    hist = rng.standard_normal((25 + 64, Fm))
    win = hist[64:]
    y_win, _ = fe.conv_subsample(win, 25, sd, store)
    y_long, _ = fe.conv_subsample(hist, hist.shape[0], sd, store)
    # window row 0 is history row 64; layer-3 output t covers input rows from 8t - 14
    np.testing.assert_array_equal(y_win[2:], y_long[8 + 2 : 8 + 4])
    # the dropped rows do see the padding
    assert not np.allclose(y_win[1], y_long[8 + 1])


def test_pre_encode_chunk_schedule():
    """1440 samples, then 2560 per chunk (model_runner.py:53-56,94-95): 8 mel
    frames -> 2 rows, then windows of 24 and 25 frames -> 2 rows each."""
    C, Fm, D = 16, 80, 32
    sd = {k: v.numpy() for k, v in _sub_params(C, Fm, D, seed=5).items()}
    p = fe.FeParams(n_mels=Fm)
    st = fe.PreEncodeState(fe.FeState(p, dither=False), sd)
    x = _signal(1440 + 4 * 2560, seed=9)
    rows, windows = [], []
    pos = 0
    for n in [1440] + [2560] * 4:
        y = st.push(x[pos : pos + n])
        pos += n
        rows.append(y.shape[0])
        windows.append(st.last_window)
    assert rows == [2, 2, 2, 2, 2]
    assert windows == [(0, 8), (0, 24), (15, 25), (31, 25), (47, 25)]
    assert st.cache.shape == (Fm, 9)


# ---------------------------------------------------------------------------
# the front end's host bookkeeping (StreamCounters) against the oracle's push
# and pre-encode state machines, on random push schedules


@pytest.mark.parametrize("seed", range(6))
def test_stream_counters_follow_the_reference_bookkeeping(seed):
    from parakeet_amd.modules.frontend import StreamCounters

    rng = np.random.default_rng(seed)
    S, B, steps = 7, 4, 30
    p = fe.FeParams(n_mels=80, dither=0.0)
    C, D = 16, 8
    sd = {k: v.numpy() for k, v in _sub_params(C, 80, D, seed=1).items()}
    ctr = StreamCounters(S, 512, 400, 160, ring_size=8192, mel_rows=64)
    states = [None] * S
    for step in range(steps):
        slots = rng.permutation(S)[:B]
        for s in slots:
            if states[s] is None or rng.random() < 0.08:  # a new stream on this slot
                ctr.reset(int(s))
                states[s] = fe.PreEncodeState(fe.FeState(p, dither=False), sd)
        n_new = rng.choice([0, 1, 100, 257, 1440, 2560, 2560, 2560, 4000], size=B)
        final = rng.random(B) < 0.1
        x = [rng.standard_normal(int(n)).astype(np.float32) * 0.1 for n in n_new]
        total0, start, n_frames, c, W, drop, n_out, emit = ctr.plan(slots, n_new, final)
        for b, s in enumerate(slots):
            st = states[s]
            had_cache = st.cache is not None
            y = st.push(x[b], bool(final[b]), linear=False)
            assert bool(emit[b]) == (y is not None)
            assert ctr.emitted[s] == st.fe.emitted and ctr.offset[s] == st.fe.offset
            if y is None:
                continue
            assert start[b] == st.fe.last_start
            assert (int(ctr.last_window[s, 0]), int(ctr.last_window[s, 1])) == st.last_window
            assert drop[b] == (2 if had_cache else 0)
            assert n_out[b] == y.shape[0]
            assert c[b] + n_frames[b] == W[b]


def test_stream_counters_reject_what_the_rings_cannot_hold():
    from parakeet_amd.modules.frontend import StreamCounters

    ctr = StreamCounters(2, 512, 400, 160, ring_size=4096, mel_rows=32)
    with pytest.raises(RuntimeError, match="ring"):
        ctr.plan(np.array([0]), np.array([5000]), np.array([False]))
    ctr = StreamCounters(2, 512, 400, 160, ring_size=8192, mel_rows=16)
    with pytest.raises(RuntimeError, match="mel ring"):
        ctr.plan(np.array([1]), np.array([4000]), np.array([False]))  # 24 frames in one window
