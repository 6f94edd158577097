"""Batched RNNT greedy decoding on the GPU, the predictor state of every stream
kept on the device by slot.

* :class:`Predictor`, :class:`Joiner` -- the parameter structure of
  parakeet/modules/decoder.py:5-86 (same constructors and state-dict names), so
  a reference checkpoint loads.  Their per-call forwards are not the decoding
  path here: the greedy loop runs in :class:`GreedyDecoder`.
* :class:`GreedyDecoder` -- ModelRunner._decode_batch / _decode_frame_batch
  (parakeet/engine/model_runner.py:347-447) for a batch: one ``enc`` GEMM for the
  step's frames, then ``pk_rnnt_greedy_step`` issues the whole per-frame,
  per-symbol loop with no host synchronisation; the tokens come back in one copy.
  ``reset_slot`` is create_sequence's predictor start state (model_runner.py:70-77).

There is no CPU path: without the HIP library the calls raise.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import numpy as np
import torch
from torch import Tensor, nn
from torch.nn import functional as F

from .. import _lib, ops
from .._lib import RnntArgs, check, lib


class Predictor(nn.Module):
    """decoder.py:5-42: embedding (blank = padding row) and an LSTM."""

    def __init__(self, pred_dim: int, hidden_dim: int, num_layers: int, vocab_size: int):
        super().__init__()
        self.prediction = nn.ModuleDict(
            {
                "embed": nn.Embedding(vocab_size + 1, pred_dim, padding_idx=vocab_size),
                "dec_rnn": nn.LSTM(input_size=pred_dim, hidden_size=hidden_dim, num_layers=num_layers),
            }
        )
        self.pred_dim = pred_dim
        self.num_layers = num_layers

    def init_state(self, batch_size: int):
        p = next(self.parameters())
        z = torch.zeros(self.num_layers, batch_size, self.pred_dim, device=p.device, dtype=p.dtype)
        return (z, z.clone())


class Joiner(nn.Module):
    """decoder.py:53-80: enc / pred projections, ReLU, dropout, output layer."""

    def __init__(self, encoder_dim, pred_dim, joint_dim, dropout: float = 0.2, num_classes: int = 1024):
        super().__init__()
        self._vocab_size = num_classes
        self._num_classes = num_classes + 1
        self.encoder_dim, self.pred_dim, self.joint_dim, self.dropout = encoder_dim, pred_dim, joint_dim, dropout
        self.pred = nn.Linear(pred_dim, joint_dim)
        self.enc = nn.Linear(encoder_dim, joint_dim)
        self.joint_net = nn.Sequential(nn.ReLU(inplace=True), nn.Dropout(p=dropout), nn.Linear(joint_dim, num_classes + 1))


class GreedyDecoder:
    """Greedy RNNT decoding of many streams at once (model_runner.py:306-447).

    ``predictor`` / ``joiner``: modules with the reference's parameter names
    (this package's or the reference's own).  State per slot on ``device``: LSTM h
    and c [slots, layers, hidden] and the predictor's joint projection
    [slots, joint], in the modules' dtype."""

    def __init__(self, predictor: nn.Module, joiner: nn.Module, blank_id: int, num_slots: int, max_symbols: int = 5):
        self.pred, self.joiner = predictor, joiner
        self.blank, self.max_symbols = int(blank_id), int(max_symbols)
        # 0: the library compacts each iteration's updating streams from 1024
        # streams on; 1 / -1: always / never (the outputs are the same)
        self.compact = 0
        self.num_slots = S = int(num_slots)
        lstm = predictor.prediction["dec_rnn"]
        embed = predictor.prediction["embed"]
        self.layers, self.hidden = lstm.num_layers, lstm.hidden_size
        w = embed.weight
        self.device, self.dtype = w.device, w.dtype
        if self.device.type != "cuda":
            raise RuntimeError("GreedyDecoder runs on a HIP device (there is no CPU implementation)")
        self.vocab1 = int(w.shape[0])
        self.joint = int(joiner.pred.weight.shape[0])
        if not 0 <= self.blank < self.vocab1:
            raise ValueError(f"blank id {self.blank} outside the vocabulary of {self.vocab1}")
        self.refresh_weights()
        L, H, J = self.layers, self.hidden, self.joint
        self.h = torch.zeros((S, L, H), dtype=self.dtype, device=self.device)
        self.c = torch.zeros((S, L, H), dtype=self.dtype, device=self.device)
        self.pred_proj = torch.zeros((S, J), dtype=self.dtype, device=self.device)
        self._ws: dict[int, torch.Tensor] = {}
        self._graphs: dict[tuple[int, int, int], dict] = {}

    _WEIGHTS = ("w_ih", "w_hh", "b_ih", "b_hh", "embed", "w_pred", "b_pred", "w_enc", "b_enc", "w_out", "b_out")

    def refresh_weights(self) -> None:
        """Copies of the parameters in the layouts the kernels read (LSTM weights
        stacked over layers), owned by the decoder; call after loading new
        weights.  When the shapes are unchanged the new values are copied into
        the same buffers, so decode steps recorded earlier (graph=True) replay
        with the new weights; otherwise the recordings are dropped and made
        again on the next call."""
        lstm = self.pred.prediction["dec_rnn"]
        L = self.layers
        j = self.joiner
        out = j.joint_net[-1]
        with torch.no_grad():
            own = lambda t: t.detach().clone(memory_format=torch.contiguous_format)  # noqa: E731
            stack = lambda n: torch.stack([getattr(lstm, f"{n}_l{k}") for k in range(L)]).contiguous()  # noqa: E731
            new = {
                "w_ih": stack("weight_ih"), "w_hh": stack("weight_hh"), "b_ih": stack("bias_ih"), "b_hh": stack("bias_hh"),
                "embed": own(self.pred.prediction["embed"].weight),
                "w_pred": own(j.pred.weight), "b_pred": own(j.pred.bias),
                "w_enc": own(j.enc.weight), "b_enc": own(j.enc.bias),
                "w_out": own(out.weight), "b_out": own(out.bias),
            }
        if new["w_ih"].shape[2] != self.hidden:
            raise NotImplementedError("the predictor's embedding size must equal its hidden size (config.py:19)")
        for t in new.values():
            if t.dtype != self.dtype or t.device != self.device:
                raise ValueError("predictor and joiner parameters must share one dtype and device")
        cur = getattr(self, "w_ih", None)
        same = cur is not None and all(getattr(self, k).shape == v.shape for k, v in new.items())
        if same:
            with torch.no_grad():
                for k, v in new.items():
                    getattr(self, k).copy_(v)  # recorded steps keep reading these buffers
        else:
            for k, v in new.items():
                setattr(self, k, v)
            if getattr(self, "_graphs", None):
                self._graphs.clear()  # they hold the old buffers' addresses

    def _workspace(self, batch: int) -> torch.Tensor:
        n = int(lib().pk_rnnt_workspace_bytes(ops.dtype_code(self.dtype), batch, self.vocab1, self.layers, self.hidden))
        ws = self._ws.get(batch)
        if ws is None or ws.numel() < n:
            ws = torch.empty(max(n, 256), dtype=torch.uint8, device=self.device)
            self._ws[batch] = ws
        return ws

    def _args(self, slots: Tensor, prime: bool) -> RnntArgs:
        a = RnntArgs()
        a.dtype = ops.dtype_code(self.dtype)
        a.device = self.device.index if self.device.index is not None else torch.cuda.current_device()
        a.batch, a.slots, a.num_slots = int(slots.numel()), slots.data_ptr(), self.num_slots
        a.layers, a.hidden, a.joint, a.vocab1 = self.layers, self.hidden, self.joint, self.vocab1
        a.blank, a.max_symbols, a.prime = self.blank, self.max_symbols, int(prime)
        a.compact = int(self.compact)
        a.embed, a.w_ih, a.w_hh = self.embed.data_ptr(), self.w_ih.data_ptr(), self.w_hh.data_ptr()
        a.b_ih, a.b_hh = self.b_ih.data_ptr(), self.b_hh.data_ptr()
        a.w_pred, a.b_pred = self.w_pred.data_ptr(), self.b_pred.data_ptr()
        a.w_out, a.b_out = self.w_out.data_ptr(), self.b_out.data_ptr()
        a.h, a.c, a.pred_proj = self.h.data_ptr(), self.c.data_ptr(), self.pred_proj.data_ptr()
        a.workspace = self._workspace(a.batch).data_ptr()
        return a

    def _check_slots(self, slots) -> np.ndarray:
        s = np.ascontiguousarray(np.asarray(slots, dtype=np.int32).reshape(-1))
        if len(np.unique(s)) != len(s) or (len(s) and (s.min() < 0 or s.max() >= self.num_slots)):
            raise ValueError(f"slots must be distinct and in [0, {self.num_slots})")
        return s

    def _slots(self, slots) -> Tensor:
        return torch.from_numpy(self._check_slots(slots)).to(self.device)

    def reset_slot(self, slots) -> None:
        """A new stream on each of ``slots``: the predictor run on the blank start
        token from zero state (model_runner.py:70-77)."""
        st = self._slots(slots)
        if st.numel() == 0:
            return
        a = self._args(st, prime=True)
        check(lib().pk_rnnt_greedy_step(ctypes.byref(a), ops._stream(self.device)), "pk_rnnt_greedy_step")

    def _graph_for(self, B: int, T: int, D: int) -> dict:
        """A HIP graph of one decode step for B streams and T frames: the enc GEMM
        and every launch of pk_rnnt_greedy_step, over persistent input and output
        buffers (recorded once, replayed per step)."""
        key = (B, T, D, int(self.compact))  # a recording keeps the mode it was made with
        g = self._graphs.get(key)
        if g is not None:
            return g
        dev = self.device
        W = T * self.max_symbols + T  # per stream: tokens, then counts per frame
        meta = torch.zeros(2 * B, dtype=torch.int32, device=dev)  # slots | lengths
        out = torch.zeros((B, W), dtype=torch.int32, device=dev)
        g = {
            "meta": meta,
            # two pinned upload and two pinned result buffers, used in turn: a call
            # may return before its copies ran, so the next call fills the other
            # pair (each buffer is reused only after its event)
            "meta_h": [torch.zeros(2 * B, dtype=torch.int32, pin_memory=True) for _ in range(2)],
            "meta_ev": [None, None],
            "out_ev": [None, None],
            "pending": [None, None],
            "turn": 0,
            "slots": meta[:B],
            "lens": meta[B:],
            "enc": torch.zeros((B, T, D), dtype=self.dtype, device=dev),
            "e": torch.empty((B, T, self.joint), dtype=self.dtype, device=dev),
            "out": out,
            "out_h": [torch.zeros((B, W), dtype=torch.int32, pin_memory=True) for _ in range(2)],
            "tokens": out[:, : T * self.max_symbols],
            "counts": out[:, T * self.max_symbols :],
        }
        a = self._args(g["slots"], prime=False)
        a.enc_proj, a.enc_stride_b, a.enc_stride_t = g["e"].data_ptr(), g["e"].stride(0), g["e"].stride(1)
        a.lengths, a.max_frames = g["lens"].data_ptr(), T
        a.tokens, a.frame_counts = g["tokens"].data_ptr(), g["counts"].data_ptr()
        # rows of `out` hold T*max_symbols tokens then T counts: the kernels index
        # tokens with row length T*max_symbols and counts with row length T, so
        # they get their own buffers and the graph copies them into `out`
        g["tok_buf"] = torch.empty((B, T * self.max_symbols), dtype=torch.int32, device=dev)
        g["cnt_buf"] = torch.empty((B, T), dtype=torch.int32, device=dev)
        a.tokens, a.frame_counts = g["tok_buf"].data_ptr(), g["cnt_buf"].data_ptr()
        g["args"] = a

        def run():
            torch.addmm(self.b_enc, g["enc"].view(B * T, D), self.w_enc.t(), out=g["e"].view(B * T, self.joint))
            check(lib().pk_rnnt_greedy_step(ctypes.byref(a), ops._stream(dev)), "pk_rnnt_greedy_step")
            g["tokens"].copy_(g["tok_buf"])
            g["counts"].copy_(g["cnt_buf"])

        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            run()  # warm the GEMM outside the capture; every length is 0, so no state moves
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            run()
        torch.cuda.current_stream(dev).wait_stream(side)
        g["graph"] = graph
        self._graphs[key] = g
        return g

    def decode(
        self, slots, enc_out: Tensor, lengths=None, frame_tokens: bool = False, graph: bool = False, wait: bool = True
    ):
        """Greedy decoding of one step's encoder frames.

        enc_out: [B, T, D] encoder output (frames of stream b in enc_out[b, :lengths[b]]);
        lengths: frames per stream (None: all T).  Returns the emitted tokens of
        each stream (``frame_tokens=True``: a list per frame).  ``graph=True``
        replays a recorded step over persistent buffers: one upload of slots and
        lengths, one copy of the tokens back.  With ``graph=True, wait=False`` the
        call returns a :class:`PendingTokens` as soon as the step and the copy are
        issued; its ``result()`` waits for the copy and builds the lists, so a
        caller can split one step's tokens while the GPU runs the next step.  A
        pending result is built at the latest when its buffer comes round again,
        two calls of the same shape later."""
        sl = self._check_slots(slots)
        B = len(sl)
        if enc_out.dim() != 3 or enc_out.shape[0] != B:
            raise ValueError(f"enc_out must be [{B}, T, D]")
        T = int(enc_out.shape[1])
        if lengths is None:
            lens = np.full(B, T, dtype=np.int32)
        else:
            lens = np.asarray(torch.as_tensor(lengths).cpu(), dtype=np.int32).reshape(-1)
            if lens.shape != (B,) or (B and (lens.min() < 0 or lens.max() > T)):
                raise ValueError(f"lengths must be [{B}] in [0, {T}]")
        if B == 0 or T == 0:
            return [[] for _ in range(B)]
        if graph:
            g = self._graph_for(B, T, int(enc_out.shape[2]))
            i = g["turn"]
            g["turn"] = i ^ 1
            if g["meta_ev"][i] is not None:
                g["meta_ev"][i].synchronize()  # the upload that last read this buffer ran
            mh = g["meta_h"][i].numpy()
            mh[:B] = sl
            mh[B:] = lens
            g["meta"].copy_(g["meta_h"][i], non_blocking=True)
            g["meta_ev"][i] = torch.cuda.Event()
            g["meta_ev"][i].record()
            g["enc"].copy_(enc_out)
            g["graph"].replay()
            if g["pending"][i] is not None:
                g["pending"][i].result()  # its buffer is about to be overwritten
            g["out_h"][i].copy_(g["out"], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            res = PendingTokens(g["out_h"][i], ev, T * self.max_symbols, lens, frame_tokens)
            g["pending"][i] = res
            return res.result() if wait else res
        st = torch.from_numpy(sl).to(self.device)
        with torch.no_grad():
            e = F.linear(enc_out.to(self.dtype), self.w_enc, self.b_enc).contiguous()  # Joiner.enc (decoder.py:83)
        tokens = torch.empty((B, T * self.max_symbols), dtype=torch.int32, device=self.device)
        counts = torch.empty((B, T), dtype=torch.int32, device=self.device)
        lens_d = torch.from_numpy(lens).to(self.device)
        a = self._args(st, prime=False)
        a.enc_proj, a.enc_stride_b, a.enc_stride_t = e.data_ptr(), e.stride(0), e.stride(1)
        a.lengths, a.max_frames = lens_d.data_ptr(), T
        a.tokens, a.frame_counts = tokens.data_ptr(), counts.data_ptr()
        check(lib().pk_rnnt_greedy_step(ctypes.byref(a), ops._stream(self.device)), "pk_rnnt_greedy_step")
        return self._collect(tokens, counts, lens, frame_tokens)

    @staticmethod
    def _collect(tokens: Tensor, counts: Tensor, lens: np.ndarray, frame_tokens: bool):
        tok, cnt = tokens.cpu().numpy(), counts.cpu().numpy()  # the step's one synchronisation
        return GreedyDecoder._split(tok, cnt, lens, frame_tokens)

    @staticmethod
    def _split(tok: np.ndarray, cnt: np.ndarray, lens: np.ndarray, frame_tokens: bool):
        """Per-stream tokens from the step's [B, frames * max_symbols] tokens and
        [B, frames] counts (frames past a stream's length count nothing); the
        counts and offsets are computed for the whole batch at once.  Returns a
        StreamTokens (each stream's list built when it is read), or with
        ``frame_tokens`` a list per stream of a list per frame."""
        B = len(lens)
        if B == 0:
            return StreamTokens(np.zeros((0, 0), dtype=np.int32), np.zeros(0, dtype=np.int64)) if not frame_tokens else []
        T = cnt.shape[1]
        n = np.where(np.arange(T)[None, :] < np.asarray(lens)[:, None], cnt, 0).astype(np.int64)
        tot = n.sum(1)
        if not frame_tokens:
            return StreamTokens(tok, tot)
        # the emitted tokens only, stream after stream
        flat = tok[np.arange(tok.shape[1])[None, :] < tot[:, None]].tolist()
        off = np.concatenate([[0], np.cumsum(tot)])
        edges = (off[:-1, None] + np.concatenate([np.zeros((B, 1), dtype=np.int64), np.cumsum(n, axis=1)], axis=1)).tolist()
        return [[flat[e[i] : e[i + 1]] for i in range(int(l))] for e, l in zip(edges, lens)]


class StreamTokens(Sequence):
    """The tokens a decode step emitted for each stream of its batch, as the
    step left them: row b of ``rows`` [B, frames * max_symbols] holds stream b's
    tokens in its first ``counts()[b]`` entries.  Reads as a sequence of
    per-stream lists (``tokens[b]`` is stream b's list, built when read), so a
    caller that touches a few streams, or only the counts, pays nothing for the
    rest; ``flat()`` packs them stream after stream (the reference returns a
    list per stream, model_runner.py:347-447)."""

    __slots__ = ("rows", "_counts")

    def __init__(self, rows: np.ndarray, counts: np.ndarray):
        self.rows = rows
        self._counts = counts

    def __len__(self) -> int:
        return len(self._counts)

    def __getitem__(self, b):
        if isinstance(b, slice):
            return [self[i] for i in range(*b.indices(len(self)))]
        n = len(self)
        b = int(b)
        if b < 0:
            b += n
        if not 0 <= b < n:
            raise IndexError(f"stream {b} out of range for a batch of {n}")
        return self.rows[b, : self._counts[b]].tolist()

    def counts(self) -> np.ndarray:
        """Tokens per stream, [B]."""
        return self._counts

    def total(self) -> int:
        return int(self._counts.sum())

    def offsets(self) -> np.ndarray:
        """[B + 1] offsets of the streams' tokens in ``flat()``."""
        return np.concatenate([[0], np.cumsum(self._counts)])

    def flat(self) -> np.ndarray:
        """Every emitted token, stream after stream."""
        return self.rows[np.arange(self.rows.shape[1])[None, :] < self._counts[:, None]]

    def __eq__(self, other):
        if isinstance(other, StreamTokens):
            return np.array_equal(self._counts, other._counts) and np.array_equal(self.flat(), other.flat())
        if isinstance(other, Sequence) and not isinstance(other, (str, bytes)):
            return len(self) == len(other) and all(self[b] == list(other[b]) for b in range(len(self)))
        return NotImplemented

    def __repr__(self) -> str:
        return f"StreamTokens({[self[b] for b in range(min(len(self), 4))]}{' ...' if len(self) > 4 else ''})"


class PendingTokens:
    """The tokens of a decode step whose copy back may still be running:
    ``result()`` waits for it and returns the per-stream token lists (per frame
    with ``frame_tokens``), as ``GreedyDecoder.decode`` does with ``wait=True``."""

    def __init__(self, buf: Tensor, event, n_tok: int, lens: np.ndarray, frame_tokens: bool):
        self._buf, self._event, self._n_tok = buf, event, int(n_tok)
        self._lens, self._frame_tokens = np.array(lens, copy=True), frame_tokens
        self._out = None

    def result(self):
        if self._out is None:
            self._event.synchronize()
            o = self._buf.numpy()
            # the buffer is reused two calls later: the lazy result keeps its own copy
            self._out = GreedyDecoder._split(o[:, : self._n_tok].copy(), o[:, self._n_tok :], self._lens,
                                             self._frame_tokens)
            self._buf = None
        return self._out


__all__ = ["Predictor", "Joiner", "GreedyDecoder", "PendingTokens", "StreamTokens"]
