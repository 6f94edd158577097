"""Pre-encode front end of the reference, restated: pcm -> log-mel -> 8x causal
convolution subsampling, streamed per chunk.

Test infrastructure only.

Feature extractor (parakeet/modules/feature_extractor.py):

* ``mel_filterbank``  librosa.filters.mel(sr, n_fft, n_mels, fmin, fmax,
  norm="slaney") as called at :49-56 (librosa is not installed here: its
  published algorithm is restated -- Slaney mel scale, triangular filters
  between n_mels+2 mel-spaced edges, area normalisation 2 / (f[m+2] - f[m]),
  float64 then cast to float32 as the reference does);
* ``hann``            torch.hann_window(win, periodic=False) (:46);
* ``log_mel``         _compute_features (:63-88): dither, pre-emphasis
  x[0], x[i] - 0.97 x[i-1], centred STFT with constant padding (n_fft // 2 each
  side, win_length zero-padded to n_fft in the middle), |X|^2, fb @ P,
  log(mel + 2^-24);
* ``FeState.push``    push + _trim_samples (:97-151): per-stream sample buffer,
  frames emitted up to (total - n_fft/2) // hop (total // hop on the final push).

The reference draws its dither from torch's global generator on every push, so
no two runs agree; here the noise is a function of the stream and of the global
sample index (Philox4x32-10, Salmon et al., SC'11, with the Box-Muller
transform), which the GPU kernel computes the same way.

Subsampling (parakeet/modules/subsample.py, convolution.py:55-104):

* ``conv_subsample``  ConvSubsampling.forward (:140-152) through
  MaskedConvSequential (:30-57): CausalConv2D (pad time and freq by kernel-1
  before, stride-1 after) 1 -> C, ReLU, then twice [depthwise 3x3 stride 2,
  pointwise 1x1, ReLU]; the time mask of the current lengths is applied before
  every layer and at the end; out = Linear(C * F3) over [t, c, f];
* ``calc_length``     calc_length (:9-15).

Streaming pre-encode (parakeet/engine/model_runner.py:181-252):

* ``PreEncodeState.push``  feature push, window = last pre_encode_cache_size
  cached mel frames + the new ones, subsample the window at its full length,
  drop drop_extra_pre_encoded leading outputs when a cache existed, keep the
  last pre_encode_cache_size frames of the window as the next cache.
"""

from __future__ import annotations

import math

import numpy as np
import torch

# ---------------------------------------------------------------------------
# Slaney mel filterbank (librosa.filters.mel, norm="slaney", htk=False)

_F_SP = 200.0 / 3.0
_MIN_LOG_HZ = 1000.0
_MIN_LOG_MEL = _MIN_LOG_HZ / _F_SP
_LOGSTEP = math.log(6.4) / 27.0


def hz_to_mel(f):
    """Slaney's auditory scale: linear below 1 kHz, logarithmic above."""
    f = np.asarray(f, dtype=np.float64)
    lin = f / _F_SP
    log = _MIN_LOG_MEL + np.log(np.maximum(f, 1e-300) / _MIN_LOG_HZ) / _LOGSTEP
    return np.where(f >= _MIN_LOG_HZ, log, lin)


def mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    lin = _F_SP * m
    log = _MIN_LOG_HZ * np.exp(_LOGSTEP * (m - _MIN_LOG_MEL))
    return np.where(m >= _MIN_LOG_MEL, log, lin)


def mel_filterbank(sr=16000, n_fft=512, n_mels=128, fmin=0.0, fmax=None) -> np.ndarray:
    """[n_mels, n_fft//2 + 1] float32 (feature_extractor.py:48-57)."""
    fmax = sr / 2.0 if fmax is None else float(fmax)
    fft_f = np.linspace(0.0, sr / 2.0, 1 + n_fft // 2)
    mel_f = mel_to_hz(np.linspace(hz_to_mel(fmin), hz_to_mel(fmax), n_mels + 2))
    fdiff = np.diff(mel_f)
    ramps = mel_f[:, None] - fft_f[None, :]
    w = np.zeros((n_mels, len(fft_f)))
    for i in range(n_mels):
        lower = -ramps[i] / fdiff[i]
        upper = ramps[i + 2] / fdiff[i + 1]
        w[i] = np.maximum(0.0, np.minimum(lower, upper))
    w *= (2.0 / (mel_f[2 : n_mels + 2] - mel_f[:n_mels]))[:, None]
    return w.astype(np.float32)


def hann(win: int) -> np.ndarray:
    """Symmetric Hann window, float32 (torch.hann_window(win, periodic=False))."""
    n = np.arange(win, dtype=np.float64)
    return (0.5 - 0.5 * np.cos(2.0 * np.pi * n / (win - 1))).astype(np.float32)


# ---------------------------------------------------------------------------
# Philox4x32-10 and Gaussian dither

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85
_U32 = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """Philox4x32 with 10 rounds on uint32 arrays: ctr = (c0, c1, c2, c3),
    key = (k0, k1); returns four uint32 arrays."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint64) & _U32 for c in ctr)
    k0, k1 = (np.asarray(k, dtype=np.uint64) & _U32 for k in key)
    for r in range(10):
        if r:
            k0 = (k0 + _W0) & _U32
            k1 = (k1 + _W1) & _U32
        p0 = c0 * np.uint64(_M0)
        p1 = c2 * np.uint64(_M1)
        hi0, lo0 = p0 >> np.uint64(32), p0 & _U32
        hi1, lo1 = p1 >> np.uint64(32), p1 & _U32
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return tuple(c.astype(np.uint32) for c in (c0, c1, c2, c3))


def dither_normal(seed: int, noise_id: int, idx) -> np.ndarray:
    """N(0, 1) for global sample indices ``idx`` of one stream.  Samples 4j ..
    4j + 3 share one Philox draw: counter (j lo, j hi, noise_id, 0), key (seed
    lo, seed hi).  Box-Muller on the word pairs (r0, r1) for samples 4j (cos)
    and 4j + 1 (sin) and (r2, r3) for 4j + 2 (cos) and 4j + 3 (sin), with
    u1 = (ra + 1) 2^-32 in (0, 1] and u2 = rb 2^-32."""
    idx = np.asarray(idx, dtype=np.int64)
    j, q = idx >> 2, idx & 3
    r0, r1, r2, r3 = philox4x32_10(
        (j & _U32, j >> 32, np.full_like(j, noise_id & _U32), np.zeros_like(j)),
        (seed & _U32, (seed >> 32) & _U32),
    )
    ra = np.where(q < 2, r0, r2).astype(np.float64)
    rb = np.where(q < 2, r1, r3).astype(np.float64)
    radius = np.sqrt(-2.0 * np.log((ra + 1.0) * 2.0**-32))
    angle = 2.0 * np.pi * rb * 2.0**-32
    return radius * np.where(q % 2 == 0, np.cos(angle), np.sin(angle))


# ---------------------------------------------------------------------------
# log-mel features


class FeParams:
    """The reference's FeatureExtractor constants (feature_extractor.py:11-57)."""

    def __init__(self, sampling_rate=16000, n_mels=128, n_fft=512, window_size=0.025, window_stride=0.01,
                 preemph=0.97, dither=1e-5, log_zero_guard_value=2**-24, lowfreq=0, highfreq=None,
                 mag_power=2.0):
        self.sr = sampling_rate
        self.n_mels = n_mels
        self.n_fft = n_fft or 2 ** math.ceil(math.log2(int(window_size * sampling_rate)))
        self.win = int(window_size * sampling_rate)
        self.hop = int(window_stride * sampling_rate)
        self.preemph = preemph
        self.dither = dither
        self.guard = float(log_zero_guard_value)
        self.mag_power = mag_power
        self.window = hann(self.win)
        self.fb = mel_filterbank(sampling_rate, self.n_fft, n_mels, lowfreq, highfreq or sampling_rate / 2)


def frames_of(y: np.ndarray, p: FeParams, first: int, count: int, offset: int = 0) -> np.ndarray:
    """Windowed n_fft frames ``first .. first+count-1`` (global frame indices) of
    the pre-emphasised signal ``y`` whose element 0 is global sample ``offset``:
    frame f covers samples f*hop - n_fft/2 + [0, n_fft) of the zero-extended
    signal (torch.stft center=True, pad_mode="constant"), the window sitting in
    the middle (n_fft - win) / 2 samples from the left edge."""
    nf, half = p.n_fft, p.n_fft // 2
    wpad = np.zeros(nf)
    left = (nf - p.win) // 2
    wpad[left : left + p.win] = p.window
    idx = (np.arange(first, first + count)[:, None] * p.hop - half + np.arange(nf)[None, :]) - offset
    ok = (idx >= 0) & (idx < len(y))
    fr = np.where(ok, y[np.clip(idx, 0, max(len(y) - 1, 0))] if len(y) else 0.0, 0.0)
    return fr * wpad


def power_to_logmel(fr: np.ndarray, p: FeParams) -> np.ndarray:
    """[count, n_fft] windowed frames -> [n_mels, count] log-mel
    (feature_extractor.py:81-86)."""
    spec = np.abs(np.fft.rfft(fr, axis=-1)) ** p.mag_power  # [count, n_fft/2+1]
    mel = p.fb.astype(np.float64) @ spec.T
    return np.log(mel + p.guard)


def preemphasis(x: np.ndarray, p: FeParams) -> np.ndarray:
    """x[0], x[i] - preemph * x[i-1] (feature_extractor.py:67-68)."""
    x = np.asarray(x, dtype=np.float64)
    if x.size == 0:
        return x
    return np.concatenate([x[:1], x[1:] - p.preemph * x[:-1]])


def log_mel(waveform: np.ndarray, p: FeParams, noise: np.ndarray | None = None) -> np.ndarray:
    """_compute_features (feature_extractor.py:63-88) for one waveform:
    [n_mels, 1 + len // hop] float64.  ``noise`` is the N(0,1) draw the dither
    scales (None: no dither)."""
    x = np.asarray(waveform, dtype=np.float64)
    if noise is not None:
        x = x + np.asarray(noise, dtype=np.float64) * p.dither
    y = preemphasis(x, p)
    count = 1 + len(y) // p.hop
    return power_to_logmel(frames_of(y, p, 0, count), p)


class FeState:
    """One stream's feature-extractor state (sequence.py:55-57) and
    FeatureExtractor.push / _trim_samples (feature_extractor.py:97-151).
    ``noise_id`` / ``seed`` select the dither noise; ``dither=False`` turns it
    off."""

    def __init__(self, p: FeParams, noise_id: int = 0, seed: int = 0, dither: bool = True):
        self.p = p
        self.samples = np.empty((0,), dtype=np.float32)
        self.emitted = 0
        self.offset = 0
        self.noise_id, self.seed, self.use_dither = noise_id, seed, dither
        self.last_start = None  # first frame of the last push that returned features

    def push(self, samples: np.ndarray, final: bool = False) -> np.ndarray | None:
        p = self.p
        samples = np.asarray(samples, dtype=np.float32)
        if not samples.size:
            return None
        self.samples = np.concatenate([self.samples, samples]) if self.samples.size else samples.copy()
        total = self.offset + self.samples.size
        hop, pad = p.hop, p.n_fft // 2
        offset_frames = self.offset // hop
        if final:
            max_frame = total // hop
        else:
            if total <= pad:
                return None
            max_frame = (total - pad) // hop
        min_frame = 0 if self.offset == 0 else (self.offset + pad + hop - 1) // hop
        start = max(self.emitted, min_frame)
        if start > max_frame:
            return None
        noise = None
        if self.use_dither and p.dither:
            noise = dither_normal(self.seed, self.noise_id, np.arange(self.offset, total))
        feats = log_mel(self.samples, p, noise)
        out = feats[:, start - offset_frames : max_frame - offset_frames + 1]
        self.last_start = start
        self.emitted = max_frame + 1
        self._trim()
        return out

    def _trim(self) -> None:
        if self.samples.size == 0:
            return
        hop, pad = self.p.hop, self.p.n_fft // 2
        min_keep = max(0, self.emitted * hop - pad)
        if min_keep <= self.offset:
            return
        aligned = (min_keep // hop) * hop
        if aligned <= self.offset:
            return
        drop = aligned - self.offset
        self.samples = self.samples[drop:] if drop < self.samples.size else np.empty((0,), dtype=np.float32)
        self.offset = aligned


# ---------------------------------------------------------------------------
# convolution subsampling


def round_to(x: np.ndarray, dtype: torch.dtype | None) -> np.ndarray:
    if dtype is None or dtype == torch.float64:
        return np.asarray(x, dtype=np.float64)
    return torch.from_numpy(np.asarray(x, dtype=np.float64)).to(dtype).double().numpy()


def calc_length(length: int, all_paddings: int = 3, kernel_size: int = 3, stride: int = 2, repeat_num: int = 3) -> int:
    """subsample.py:9-15 on one integer length."""
    for _ in range(repeat_num):
        length = math.floor((float(length) + all_paddings - kernel_size) / stride + 1.0)
    return int(length)


def conv_out_len(length: int) -> int:
    """calculate_conv_output_size for kernel 3, stride 2, padding (2, 1)
    (subsample.py:24-27) on integer lengths."""
    return (length + 2 + 1 - 3) // 2 + 1


def _pad_tf(x: np.ndarray) -> np.ndarray:
    """CausalConv2D's F.pad (convolution.py:94-103): time and freq get kernel-1 = 2
    zeros before and stride-1 = 1 after.  x: [C, T, F]."""
    return np.pad(x, ((0, 0), (2, 1), (2, 1)))


def _conv3x3_s2(x: np.ndarray, w: np.ndarray, b: np.ndarray | None, groups: int) -> np.ndarray:
    """nn.Conv2d(kernel 3, stride 2, padding 0) on the padded input.
    x: [Cin, T, F] (already padded); w: [Cout, Cin/groups, 3, 3]."""
    cin, T, F = x.shape
    To, Fo = (T - 3) // 2 + 1, (F - 3) // 2 + 1
    cout = w.shape[0]
    y = np.zeros((cout, To, Fo))
    for kt in range(3):
        for kf in range(3):
            patch = x[:, kt : kt + 2 * To - 1 : 2, kf : kf + 2 * Fo - 1 : 2]  # [Cin, To, Fo]
            if groups == 1:
                y += np.einsum("oc,ctf->otf", w[:, :, kt, kf], patch)
            else:  # depthwise, Cin == Cout == groups
                y += w[:, 0, kt, kf][:, None, None] * patch
    if b is not None:
        y += np.asarray(b, dtype=np.float64)[:, None, None]
    return y


def _time_mask(x: np.ndarray, length: int) -> np.ndarray:
    """apply_channel_mask with the time mask of one length (subsample.py:18-21,50-57)."""
    out = x.copy()
    out[:, length:, :] = 0.0
    return out


def conv_subsample(x: np.ndarray, length: int, params: dict, store_dtype=None, linear: bool = True):
    """ConvSubsampling.forward for one stream (subsample.py:140-152, 30-48).

    x: [T, F] features; length: valid frames (the mask length); params: the
    module's state dict as float64 numpy (keys ``conv.0.weight`` ...,
    ``out.weight``, ``out.bias``).  Each layer's output is rounded to
    ``store_dtype`` as a tensor of that dtype holds it.  Returns
    (y [T3, D] or the flattened [T3, C*F3] before ``out`` when linear=False,
    output length)."""
    g = {k: np.asarray(v, dtype=np.float64) for k, v in params.items()}
    a = round_to(np.asarray(x, dtype=np.float64), store_dtype)[None]  # [1, T, F]
    cur = int(length)
    a = _time_mask(a, cur)
    # conv.0: CausalConv2D 1 -> C (stride 2), conv.1: ReLU
    a = round_to(_conv3x3_s2(_pad_tf(a), g["conv.0.weight"], g.get("conv.0.bias"), 1), store_dtype)
    cur = conv_out_len(cur)
    a = np.maximum(_time_mask(a, cur), 0.0)
    for dw, pw in (("conv.2", "conv.3"), ("conv.5", "conv.6")):
        a = _time_mask(a, cur)
        a = round_to(_conv3x3_s2(_pad_tf(a), g[dw + ".weight"], g.get(dw + ".bias"), a.shape[0]), store_dtype)
        cur = conv_out_len(cur)
        a = _time_mask(a, cur)
        w = g[pw + ".weight"][:, :, 0, 0]  # [Cout, Cin]
        a = np.einsum("oc,ctf->otf", w, a)
        if pw + ".bias" in g:
            a = a + g[pw + ".bias"][:, None, None]
        a = round_to(a, store_dtype)
        a = np.maximum(_time_mask(a, cur), 0.0)
    a = _time_mask(a, cur)
    C, T3, F3 = a.shape
    flat = a.transpose(1, 0, 2).reshape(T3, C * F3)  # x.transpose(1, 2).reshape(b, t, -1)
    if not linear:
        return flat, cur
    y = flat @ g["out.weight"].T + g["out.bias"]
    return round_to(y, store_dtype), cur


class PreEncodeState:
    """One stream through _run_pre_encode (model_runner.py:181-252): feature
    push, [cache | new] window, subsampling at the window's full length, drop
    of the leading outputs when a cache existed, next cache = the window's last
    ``cache_size`` frames."""

    def __init__(self, fe: FeState, params: dict, cache_size: int = 9, drop: int = 2, store_dtype=None):
        self.fe = fe
        self.params = params
        self.cache_size, self.drop = cache_size, drop
        self.cache = None  # [n_mels, c]
        self.store_dtype = store_dtype
        self.last_window = None  # (first global frame, rows) of the last window

    def push(self, samples, final=False, linear=True):
        feats = self.fe.push(samples, final)
        if feats is None:
            return None
        if self.cache is None:
            win, has_cache = feats, False
        else:
            win, has_cache = np.concatenate([self.cache, feats], axis=1), True
        W = win.shape[1]
        self.last_window = (self.fe.last_start - (W - feats.shape[1]), W)
        y, _ = conv_subsample(win.T, W, self.params, self.store_dtype, linear=linear)
        if has_cache and self.drop > 0:
            y = y[self.drop :]
        if self.cache_size > 0:
            self.cache = win[:, -self.cache_size :] if W >= self.cache_size else win
        return y
