"""Drop-in for the streaming pre-encode front end, batched over streams.

* :class:`FeatureExtractor` -- parakeet/modules/feature_extractor.py:8-151: same
  constructor, ``__call__`` (offline features) and ``push(samples, state,
  final)``; the features are computed by the ``pk_fe_step`` HIP kernel.
* :class:`ConvSubsampling` -- parakeet/modules/subsample.py:60-179: same
  constructor and parameter names (``conv.0`` ... ``conv.6``, ``out``);
  ``forward(x, lengths)`` runs the convolution stack as the ``pk_subsample`` HIP
  kernel and ``out`` as a GEMM.
* :class:`PreEncoder` -- ModelRunner._run_pre_encode
  (parakeet/engine/model_runner.py:181-252) for every stream of a step at once:
  one feature launch and one subsampling launch for the whole batch.  Each
  stream's recent samples and mel frames live in device rings indexed by slot;
  the frame counters of FeatureExtractor.push / _trim_samples and the
  pre-encode cache bookkeeping are advanced on the host with integer arithmetic
  only (no device round trip).

There is no CPU path: without the HIP library the calls raise.
"""

from __future__ import annotations

import math

import numpy as np
import torch
from torch import Tensor, nn
from torch.nn import functional as F

from .. import ops

# 32-byte per-stream records read by the kernels (include/parakeet_paged.h)
FE_STREAM = np.dtype(
    [("slot", "<i4"), ("n_new", "<i4"), ("sample_base", "<i8"), ("frame0", "<i4"), ("n_frames", "<i4"),
     ("noise_id", "<u4"), ("reserved", "<i4")]
)
SUB_STREAM = np.dtype([(n, "<i4") for n in ("slot", "row0", "rows", "length", "drop", "n_out", "out_row", "reserved")])
assert FE_STREAM.itemsize == 32 and SUB_STREAM.itemsize == 32


def slaney_mel_filterbank(sr: int, n_fft: int, n_mels: int, fmin: float, fmax: float) -> np.ndarray:
    """Triangular filters on Slaney's mel scale (linear below 1 kHz, log step
    ln(6.4)/27 above) with area normalisation, as librosa.filters.mel(norm=
    "slaney") builds them for feature_extractor.py:49-56.  [n_mels, n_fft/2+1]
    float32."""
    f_sp, brk = 200.0 / 3.0, 1000.0
    step = math.log(6.4) / 27.0

    def to_mel(f):
        f = np.asarray(f, dtype=np.float64)
        return np.where(f < brk, f / f_sp, brk / f_sp + np.log(np.maximum(f, brk) / brk) / step)

    def to_hz(m):
        m = np.asarray(m, dtype=np.float64)
        return np.where(m < brk / f_sp, m * f_sp, brk * np.exp(step * (m - brk / f_sp)))

    edges = to_hz(np.linspace(to_mel(fmin), to_mel(fmax), n_mels + 2))  # [n_mels + 2]
    bins = np.linspace(0.0, sr / 2.0, n_fft // 2 + 1)
    lo, mid, hi = edges[:-2, None], edges[1:-1, None], edges[2:, None]
    rise = (bins[None, :] - lo) / (mid - lo)
    fall = (hi - bins[None, :]) / (hi - mid)
    tri = np.clip(np.minimum(rise, fall), 0.0, None)
    return (tri * (2.0 / (hi - lo))).astype(np.float32)


def _out_len(n: int) -> int:
    """Output length of a 3x3 stride-2 convolution padded (2, 1) (subsample.py:24-27)."""
    return n // 2 + 1


def stack_len(n: int) -> int:
    """Frames after the three stride-2 convolutions (subsample.py:9-15 for 8x)."""
    return _out_len(_out_len(_out_len(n)))


class _Staging:
    """Pinned host buffers for the per-step records, reused round-robin only
    after the copy that read them has completed."""

    def __init__(self, nbytes: int, depth: int = 4):
        self.bufs = [torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(depth)]
        self.events = [torch.cuda.Event() for _ in range(depth)]
        self.used = [False] * depth
        self.i = 0

    def take(self) -> tuple[int, torch.Tensor]:
        i = self.i
        self.i = (i + 1) % len(self.bufs)
        if self.used[i]:
            self.events[i].synchronize()
        return i, self.bufs[i]

    def upload(self, i: int, dst: Tensor, nbytes: int) -> None:
        dst[:nbytes].copy_(self.bufs[i][:nbytes], non_blocking=True)
        self.events[i].record()
        self.used[i] = True


class FeatureExtractor:
    """Log-mel front end (feature_extractor.py:8-151) on the GPU.

    Same constructor arguments; ``seed`` keys the dither noise (the reference
    draws torch.randn per push) and ``device`` is where features are computed.
    Only the reference's configuration is built: n_fft 512, power spectrum
    (mag_power 2), Slaney norm."""

    model_input_names = ["input_features"]

    def __init__(
        self,
        sampling_rate=16000,
        n_mels=128,
        n_fft=512,
        window_size=0.025,
        window_stride=0.01,
        normalize="NA",
        preemph=0.97,
        dither=1e-5,
        log_zero_guard_value=2**-24,
        lowfreq=0,
        highfreq=None,
        mag_power=2.0,
        pad_value=0.0,
        mel_norm="slaney",
        seed: int = 0,
        device=None,
    ):
        self.sampling_rate = sampling_rate
        self.feature_size = n_mels
        self.padding_value = pad_value
        self.normalize = normalize
        self.n_mels = n_mels
        self.n_fft = n_fft or 2 ** math.ceil(math.log2(int(window_size * sampling_rate)))
        self.win_length = int(window_size * sampling_rate)
        self.hop_length = int(window_stride * sampling_rate)
        self.preemph = preemph
        self.dither = dither
        self.log_zero_guard_value = float(log_zero_guard_value)
        self.mag_power = mag_power
        self.pad_value = pad_value
        if mag_power != 2.0 or mel_norm != "slaney" or self.n_fft != 512:
            raise NotImplementedError("the HIP front end computes the power spectrum (mag_power 2) of a "
                                      "512-point FFT with the Slaney-normalised filterbank")
        self.window = torch.hann_window(self.win_length, periodic=False)
        highfreq = highfreq or sampling_rate / 2
        self.fb = torch.from_numpy(slaney_mel_filterbank(sampling_rate, self.n_fft, n_mels, lowfreq, highfreq))
        self.seed = int(seed)
        self.device = torch.device(device) if device is not None else None
        self._tables: dict[torch.device, ops.FeTables] = {}

    # ------------------------------------------------------------ constants
    def tables(self, device: torch.device) -> ops.FeTables:
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        t = self._tables.get(device)
        if t is None:
            fb = self.fb.numpy()
            nz = fb != 0
            first = np.where(nz.any(1), nz.argmax(1), 0)
            end = np.where(nz.any(1), fb.shape[1] - nz[:, ::-1].argmax(1), 0)
            rng = np.stack([first, end], axis=1).astype(np.int32)
            t = ops.FeTables(
                window=self.window.to(device=device, dtype=torch.float32).contiguous(),
                fb=self.fb.to(device).contiguous(),
                fb_range=torch.from_numpy(rng).to(device),
                n_fft=self.n_fft,
                hop=self.hop_length,
                preemph=float(self.preemph),
                log_guard=self.log_zero_guard_value,
            )
            self._tables[device] = t
        return t

    def _device(self) -> torch.device:
        if self.device is not None:
            return self.device
        return torch.device("cuda", torch.cuda.current_device())

    def _get_seq_len(self, seq_len: int) -> int:
        return (seq_len + self.n_fft - self.n_fft) // self.hop_length

    # ------------------------------------------------------------ offline
    def _compute_features(self, waveform, noise_id: int = 0) -> Tensor:
        """[1, n_mels, 1 + len // hop] float32 on the device (feature_extractor.py:63-88)."""
        dev = self._device()
        x = torch.as_tensor(np.asarray(waveform, dtype=np.float32) if not isinstance(waveform, Tensor) else waveform)
        x = x.to(device=dev, dtype=torch.float32).reshape(1, -1).contiguous()
        n = int(x.shape[1])
        frames = 1 + n // self.hop_length
        ring = torch.empty((1, 1 << max(n, 1).bit_length()), dtype=torch.float32, device=dev)
        mel = torch.empty((1, 1 << max(frames - 1, 1).bit_length(), self.n_mels), dtype=torch.float32, device=dev)
        rec = np.zeros(1, dtype=FE_STREAM)
        rec["n_new"], rec["n_frames"], rec["noise_id"] = n, frames, noise_id
        hdr = torch.from_numpy(rec.view(np.uint8)).to(dev)
        ops.fe_step(hdr, 1, x, ring, mel, self.tables(dev), dither=self.dither, seed=self.seed,
                    max_new=n, max_frames=frames)
        return mel[0, :frames].t().unsqueeze(0)

    def __call__(self, audio, return_tensors: str | None = None, padding: bool = True):
        assert isinstance(audio, np.ndarray)
        assert audio.ndim == 1
        return self._compute_features(audio)

    # ------------------------------------------------------------ streaming
    def push(self, samples: np.ndarray, state, final: bool = False):
        """One stream's push (feature_extractor.py:97-133): returns the new frames
        [1, n_mels, n] (float32, on the device) or None.  ``state`` is any object;
        its device rings and counters are attached on first use."""
        st = getattr(state, "_fe_gpu", None)
        if st is None:
            st = state._fe_gpu = PreEncoder(self, None, num_slots=1, device=self._device())
        feats = st.push_features(0, samples, final)
        state._fe_emitted_frames = int(st.emitted[0])
        state._fe_sample_offset = int(st.offset[0])
        return feats


class ConvSubsampling(nn.Module):
    """8x convolution subsampling (subsample.py:60-179): same constructor and
    parameter names; the convolution stack runs as one HIP launch."""

    def __init__(
        self,
        hidden_size: int,
        subsampling_conv_channels: int,
        feat_in: int,
        subsampling_factor: int,
        stride: int = 2,
        kernel_size: int = 3,
    ):
        super().__init__()
        if subsampling_factor != 8 or stride != 2 or kernel_size != 3:
            raise NotImplementedError("the HIP subsampling is built for factor 8, stride 2, kernel 3 (config.py:15)")
        self._conv_channels = C = subsampling_conv_channels
        self.feat_in = feat_in
        self.sampling_num = int(math.log(subsampling_factor, 2))
        self.subsampling_factor = subsampling_factor
        self.subsampling_conv_chunking_factor = 1
        self._stride, self._kernel_size = stride, kernel_size
        self.ceil_mode = False
        self._left_padding, self._right_padding = kernel_size - 1, stride - 1
        act = nn.ReLU(inplace=True)
        self.conv = nn.Sequential(
            nn.Conv2d(1, C, kernel_size, stride),
            act,
            nn.Conv2d(C, C, kernel_size, stride, groups=C),
            nn.Conv2d(C, C, 1, 1),
            act,
            nn.Conv2d(C, C, kernel_size, stride, groups=C),
            nn.Conv2d(C, C, 1, 1),
            act,
        )
        self.final_freq_dim = stack_len(feat_in)
        self.out = nn.Linear(C * self.final_freq_dim, hidden_size, bias=True)

    def conv_weights(self) -> dict:
        return {f"conv.{i}.{n}": getattr(self.conv[i], n) for i in (0, 2, 3, 5, 6) for n in ("weight", "bias")}

    def stack(self, feats: Tensor, records: np.ndarray, ring: bool, out_rows: int, max_out: int) -> Tensor:
        """The convolution stack over ``records`` (SUB_STREAM) -> [out_rows, C*F3]."""
        w = self.conv_weights()
        dev, dt = w["conv.0.weight"].device, w["conv.0.weight"].dtype
        flat = torch.empty((max(out_rows, 1), self._conv_channels * self.final_freq_dim), dtype=dt, device=dev)
        if len(records) and max_out:
            hdr = torch.from_numpy(np.ascontiguousarray(records).view(np.uint8)).to(dev)
            ops.subsample(hdr, len(records), feats, ring, w, flat, max_out=max_out)
        return flat[:out_rows]

    def forward(self, x: Tensor, lengths: Tensor):
        """x: [B, T, feat_in]; lengths: [B].  Returns ([B, T3, hidden], lengths
        after the masks) as ConvSubsampling.forward does."""
        B, T, Fm = x.shape
        if Fm != self.feat_in:
            raise ValueError(f"x has {Fm} features, the module was built for {self.feat_in}")
        T3 = stack_len(T)
        lens = [min(int(v), T) for v in torch.as_tensor(lengths).reshape(-1).tolist()]
        rec = np.zeros(B, dtype=SUB_STREAM)
        rec["slot"] = np.arange(B)
        rec["rows"] = T
        rec["length"] = lens
        rec["n_out"] = T3
        rec["out_row"] = np.arange(B) * T3
        feats = x.to(torch.float32).contiguous()
        flat = self.stack(feats, rec, False, B * T3, T3)
        y = self.out(flat).view(B, T3, -1)
        out_len = torch.tensor([stack_len(v) for v in lens], dtype=torch.int64, device=x.device)
        return y, out_len


class StreamCounters:
    """Host bookkeeping of the front end for ``num_slots`` streams:
    FeatureExtractor.push / _trim_samples (feature_extractor.py:97-151) and the
    window / cache steps of _run_pre_encode (model_runner.py:198-234), vectorised
    over a batch.  Pure integer arithmetic; nothing here touches a device."""

    def __init__(self, num_slots: int, n_fft: int, win_length: int, hop: int, cache_size: int = 9, drop: int = 2,
                 ring_size: int = 8192, mel_rows: int = 64):
        S = int(num_slots)
        self.n_fft, self.win, self.hop = int(n_fft), int(win_length), int(hop)
        self.cache_size, self.drop = int(cache_size), int(drop)
        self.ring_size, self.mel_rows = int(ring_size), int(mel_rows)
        self.total = np.zeros(S, dtype=np.int64)
        self.emitted = np.zeros(S, dtype=np.int64)
        self.offset = np.zeros(S, dtype=np.int64)
        self.cached = np.zeros(S, dtype=np.int64)
        self.has_cache = np.zeros(S, dtype=bool)
        # window of each stream's last emitting push: (first global frame, rows)
        self.last_window = np.zeros((S, 2), dtype=np.int64)

    def reset(self, slot: int) -> None:
        self.total[slot] = self.emitted[slot] = self.offset[slot] = self.cached[slot] = 0
        self.has_cache[slot] = False

    def plan(self, slots: np.ndarray, n_new: np.ndarray, final: np.ndarray):
        """Advances the counters of ``slots`` by one push each.  Returns
        (samples before the push, first frame, frame count, cached frames in the
        window, window rows, dropped outputs, kept outputs, emitted?) per stream."""
        hop, pad = self.hop, self.n_fft // 2
        total0 = self.total[slots]
        active = n_new > 0
        total = total0 + n_new
        max_frame = np.where(final, total // hop, (total - pad) // hop)
        ok = active & (final | (total > pad))
        off = self.offset[slots]
        min_frame = np.where(off == 0, 0, (off + pad + hop - 1) // hop)
        start = np.maximum(self.emitted[slots], min_frame)
        emit = ok & (start <= max_frame)
        n_frames = np.where(emit, max_frame - start + 1, 0)
        # every sample a frame reads is in the ring and not overwritten by this push
        wl = (self.n_fft - self.win) // 2
        first_read = np.maximum(start * hop - pad + wl - 1, 0)
        need = np.where(emit, total - first_read, n_new)
        if (need > self.ring_size).any():
            raise RuntimeError(f"a push needs {int(need.max())} samples in the ring (ring_size {self.ring_size})")
        emitted = np.where(emit, max_frame + 1, self.emitted[slots])
        min_keep = np.maximum(0, emitted * hop - pad)
        aligned = (min_keep // hop) * hop
        off = np.where(emit & (min_keep > off) & (aligned > off), aligned, off)
        # pre-encode window: the cached frames, then the new ones
        c = np.where(emit, self.cached[slots], 0)
        W = c + n_frames
        if (W > self.mel_rows).any():
            raise RuntimeError(f"a window of {int(W.max())} frames exceeds the mel ring ({self.mel_rows} rows)")
        has = self.has_cache[slots]
        drop = np.where(has, self.drop, 0)
        L3 = ((W // 2 + 1) // 2 + 1) // 2 + 1
        n_out = np.where(emit, np.maximum(L3 - drop, 0), 0)
        self.total[slots] = total
        self.emitted[slots] = emitted
        self.offset[slots] = off
        if self.cache_size > 0:
            self.cached[slots] = np.where(emit, np.minimum(W, self.cache_size), self.cached[slots])
            self.has_cache[slots] = has | emit
        self.last_window[slots[emit]] = np.stack([start - c, W], axis=1)[emit]
        return total0, start, n_frames, c, W, drop, n_out, emit


class PreEncoder:
    """The pre-encode step of every stream of a batch (model_runner.py:181-252):
    pcm -> log-mel (FeatureExtractor.push) -> [cached frames ; new frames] ->
    ConvSubsampling -> drop of the leading rows once a cache exists -> rows for
    the stream's encoder buffer.

    Per slot on the device: the last ``ring_size`` samples (float32) and the last
    ``mel_rows`` mel frames; the pre-encode cache is the ring rows before a
    window's new frames, so nothing is copied.  Per slot on the host: samples
    pushed, frames emitted, the trim offset, cached frame count."""

    def __init__(
        self,
        feature_extractor: FeatureExtractor,
        subsampling: ConvSubsampling | None,
        num_slots: int,
        device=None,
        pre_encode_cache_size: int = 9,
        drop_extra_pre_encoded: int = 2,
        ring_size: int = 8192,
        mel_rows: int = 64,
        max_batch: int | None = None,
    ):
        fe = feature_extractor
        self.fe = fe
        self.sub = subsampling
        self.num_slots = S = int(num_slots)
        self.device = dev = torch.device(device) if device is not None else fe._device()
        self.cache_size = int(pre_encode_cache_size)
        self.drop = int(drop_extra_pre_encoded)
        if ring_size & (ring_size - 1) or mel_rows & (mel_rows - 1):
            raise ValueError("ring_size and mel_rows must be powers of two")
        self.ring_size, self.mel_rows = int(ring_size), int(mel_rows)
        self.tables = fe.tables(dev)
        self.sample_ring = torch.zeros((S, self.ring_size), dtype=torch.float32, device=dev)
        self.mel_ring = torch.zeros((S, self.mel_rows, fe.n_mels), dtype=torch.float32, device=dev)
        self.counters = StreamCounters(S, fe.n_fft, fe.win_length, fe.hop_length, self.cache_size, self.drop,
                                       self.ring_size, self.mel_rows)
        self.noise_id = np.arange(S, dtype=np.uint32)
        self._next_noise = S
        self.max_batch = int(max_batch or S)
        self.hdr = torch.zeros(64 * self.max_batch, dtype=torch.uint8, device=dev)
        self._stage = _Staging(64 * self.max_batch)

    @property
    def emitted(self) -> np.ndarray:
        return self.counters.emitted

    @property
    def offset(self) -> np.ndarray:
        return self.counters.offset

    @property
    def last_window(self) -> np.ndarray:
        return self.counters.last_window

    # ------------------------------------------------------------ slot life
    def reset_slot(self, slot: int) -> None:
        """A stream starts on ``slot`` (create_sequence, model_runner.py:65-98):
        counters to zero, a fresh dither stream.  The rings need no clearing: a
        stream reads only samples and frames it wrote itself."""
        s = int(slot)
        self.counters.reset(s)
        self.noise_id[s] = self._next_noise & 0xFFFFFFFF
        self._next_noise += 1

    # ------------------------------------------------------------ one step
    def _features(self, slots, samples, n_new, final):
        slots = np.ascontiguousarray(slots, dtype=np.int64)
        B = len(slots)
        if B > self.max_batch:
            raise ValueError(f"batch {B} exceeds max_batch {self.max_batch}")
        if len(np.unique(slots)) != B or (B and (slots.min() < 0 or slots.max() >= self.num_slots)):
            raise ValueError("slots must be distinct and in range")
        n_new = np.broadcast_to(np.asarray(n_new, dtype=np.int64), (B,)).copy()
        final = np.broadcast_to(np.asarray(final, dtype=bool), (B,)).copy()
        plan = self.counters.plan(slots, n_new, final)
        total0, start, n_frames, c, W, drop, n_out, emit = plan
        i, buf = self._stage.take()
        fe_rec = buf[: 32 * B].numpy().view(FE_STREAM)
        fe_rec["slot"] = slots
        fe_rec["n_new"] = n_new
        fe_rec["sample_base"] = total0
        fe_rec["frame0"] = np.where(emit, start, 0)
        fe_rec["n_frames"] = n_frames
        fe_rec["noise_id"] = self.noise_id[slots]
        fe_rec["reserved"] = 0
        sel = np.nonzero(n_out > 0)[0]
        sub_rec = buf[32 * B : 32 * (B + len(sel))].numpy().view(SUB_STREAM)
        out_row = np.zeros(B, dtype=np.int64)
        out_row[sel] = np.concatenate([[0], np.cumsum(n_out[sel])[:-1]]) if len(sel) else []
        sub_rec["slot"] = slots[sel]
        sub_rec["row0"] = (start - c)[sel]
        sub_rec["rows"] = W[sel]
        sub_rec["length"] = W[sel]
        sub_rec["drop"] = drop[sel]
        sub_rec["n_out"] = n_out[sel]
        sub_rec["out_row"] = out_row[sel]
        sub_rec["reserved"] = 0
        nbytes = 32 * (B + len(sel))
        self._stage.upload(i, self.hdr, nbytes)
        max_new = int(n_new.max()) if B else 0
        max_frames = int(n_frames.max()) if B else 0
        if B and (max_new or max_frames):
            ops.fe_step(self.hdr[: 32 * B], B, samples, self.sample_ring, self.mel_ring, self.tables,
                        dither=self.fe.dither, seed=self.fe.seed, max_new=max_new, max_frames=max_frames)
        return plan, sel, out_row

    def push_features(self, slot: int, samples, final: bool = False):
        """FeatureExtractor.push for one slot: [1, n_mels, n] or None."""
        x = torch.as_tensor(np.asarray(samples, dtype=np.float32)).to(self.device).reshape(1, -1)
        n = int(x.shape[1])
        plan, _, _ = self._features(np.array([slot]), x if n else None, n, final)
        _, start, n_frames, *_ = plan
        if not n_frames[0]:
            return None
        rows = (int(start[0]) + torch.arange(int(n_frames[0]), device=self.device)) & (self.mel_rows - 1)
        return self.mel_ring[int(slot)].index_select(0, rows).t().unsqueeze(0)

    def step(self, slots, samples: Tensor | None, n_new, final=False):
        """One pre-encode step for the streams on ``slots``.

        samples: [B, >= max(n_new)] int16 pcm (value / 32768, parakeet/server.py:442)
        or float32 on the device; n_new: samples per stream (int or [B]); final:
        the reference's is_final flag per stream.  Returns (rows [R, hidden] in
        the model dtype, counts [B], first row [B]) -- stream b's new encoder
        frames are rows[first[b] : first[b] + counts[b]]."""
        if self.sub is None:
            raise RuntimeError("this PreEncoder has no subsampling module")
        plan, sel, out_row = self._features(slots, samples, n_new, final)
        n_out = plan[6]
        R = int(n_out.sum())
        C, F3 = self.sub._conv_channels, self.sub.final_freq_dim
        w = self.sub.out.weight
        if R == 0:
            return torch.empty((0, w.shape[0]), dtype=w.dtype, device=self.device), n_out, out_row
        B = len(plan[0])
        flat = torch.empty((R, C * F3), dtype=w.dtype, device=self.device)
        ops.subsample(self.hdr[32 * B :], len(sel), self.mel_ring, True, self.sub.conv_weights(), flat,
                      max_out=int(n_out.max()))
        return F.linear(flat, w, self.sub.out.bias), n_out, out_row


__all__ = ["FeatureExtractor", "ConvSubsampling", "PreEncoder", "StreamCounters", "slaney_mel_filterbank", "stack_len"]
