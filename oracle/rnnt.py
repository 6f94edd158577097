"""RNNT greedy decoding of the reference, restated.

Test infrastructure only.

* ``predictor_step``  Predictor.forward (parakeet/modules/decoder.py:44-50): the
  embedding of the previous token (padding row = blank), then nn.LSTM layers
  (gate order i, f, g, o; c' = f c + i g, h' = o tanh(c')), one time step.
* ``joint``           Joiner.forward (decoder.py:82-86): W_out relu(enc(e) +
  pred(p)) + b_out (dropout is the identity in eval).
* ``greedy_decode``   ModelRunner._decode_frame_batch / _decode_batch
  (parakeet/engine/model_runner.py:347-447) for one stream: per encoder frame,
  up to ``max_symbols`` argmax decisions; a blank ends the frame, a token is
  emitted and advances the predictor.  The reference evaluates a batch and
  stops when every stream's decision is blank; a stream whose decision was
  blank keeps its state and, its inputs unchanged, would decide blank again, so
  the batched loop equals this per-stream loop (pinned in the tests against the
  reference's batched operator sequence).
* ``replay``          the same loop following a given decision sequence, for
  parity checks of a decoder whose argmax may break near-ties differently.

``store_dtype`` rounds what the reference's tensors hold in that dtype: the
projections, their sum, the logits, h and c.  Arithmetic is float64.
"""

from __future__ import annotations

import numpy as np
import torch


def round_to(x, dtype):
    if dtype is None or dtype == torch.float64:
        return np.asarray(x, dtype=np.float64)
    return torch.from_numpy(np.asarray(x, dtype=np.float64)).to(dtype).double().numpy()


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


class RnntParams:
    """Float64 copies of the Predictor and Joiner parameters (state-dict names of
    decoder.py:10-19,71-80)."""

    def __init__(self, pred_sd: dict, joint_sd: dict, num_layers: int):
        f = lambda v: np.asarray(v.detach().double().cpu().numpy() if isinstance(v, torch.Tensor) else v, dtype=np.float64)
        self.embed = f(pred_sd["prediction.embed.weight"])
        self.layers = []
        for k in range(num_layers):
            p = f"prediction.dec_rnn."
            self.layers.append(
                (
                    f(pred_sd[p + f"weight_ih_l{k}"]),
                    f(pred_sd[p + f"weight_hh_l{k}"]),
                    f(pred_sd[p + f"bias_ih_l{k}"]) + 0.0,
                    f(pred_sd[p + f"bias_hh_l{k}"]) + 0.0,
                )
            )
        self.w_pred, self.b_pred = f(joint_sd["pred.weight"]), f(joint_sd["pred.bias"])
        self.w_enc, self.b_enc = f(joint_sd["enc.weight"]), f(joint_sd["enc.bias"])
        self.w_out, self.b_out = f(joint_sd["joint_net.2.weight"]), f(joint_sd["joint_net.2.bias"])


def predictor_step(P: RnntParams, token: int, h, c, dtype=None):
    """One Predictor.forward step for one stream.  h, c: [layers, H].  Returns
    (pred_out [H], h', c')."""
    x = P.embed[token]
    h2, c2 = np.empty_like(h), np.empty_like(c)
    for k, (wih, whh, bih, bhh) in enumerate(P.layers):
        g = wih @ x + bih + whh @ h[k] + bhh
        H = h.shape[1]
        i, f, gg, o = _sigmoid(g[:H]), _sigmoid(g[H : 2 * H]), np.tanh(g[2 * H : 3 * H]), _sigmoid(g[3 * H :])
        c2[k] = round_to(f * c[k] + i * gg, dtype)
        h2[k] = round_to(o * np.tanh(f * c[k] + i * gg), dtype)
        x = h2[k]
    return h2[-1].copy(), h2, c2


def enc_proj(P: RnntParams, frames, dtype=None):
    """Joiner.enc over encoder frames [..., D] (decoder.py:83)."""
    return round_to(np.asarray(frames, dtype=np.float64) @ P.w_enc.T + P.b_enc, dtype)


def pred_proj(P: RnntParams, pred_out, dtype=None):
    return round_to(np.asarray(pred_out, dtype=np.float64) @ P.w_pred.T + P.b_pred, dtype)


def joint_logits(P: RnntParams, e_proj, p_proj, dtype=None):
    """decoder.py:84-86 from the two projections: logits [V + 1]."""
    hid = np.maximum(round_to(e_proj + p_proj, dtype), 0.0)
    return round_to(hid @ P.w_out.T + P.b_out, dtype)


def init_state(P: RnntParams, blank: int, dtype=None):
    """create_sequence (model_runner.py:70-77): the predictor run once on the
    blank start token from zero state."""
    L = len(P.layers)
    H = P.layers[0][1].shape[1]
    z = np.zeros((L, H))
    return predictor_step(P, blank, z, z, dtype)


class StreamDecoder:
    """Greedy RNNT decoding of one stream across steps (the stream's pred_out /
    pred_state live between steps, model_runner.py:404-408)."""

    def __init__(self, P: RnntParams, blank: int, max_symbols: int = 5, dtype=None):
        self.P, self.blank, self.max_symbols, self.dtype = P, blank, max_symbols, dtype
        self.pred_out, self.h, self.c = init_state(P, blank, dtype)

    def decode(self, frames) -> list[int]:
        """frames: [T, D] encoder output of this step; returns the emitted tokens
        (``self.frame_tokens`` keeps them per frame)."""
        P, dt = self.P, self.dtype
        self.frame_tokens = []
        for e in enc_proj(P, frames, dt):
            toks = []
            for _ in range(self.max_symbols):
                logits = joint_logits(P, e, pred_proj(P, self.pred_out, dt), dt)
                k = int(np.argmax(logits))  # first maximum, as torch.argmax
                if k == self.blank:
                    break
                toks.append(k)
                self.pred_out, self.h, self.c = predictor_step(P, k, self.h, self.c, dt)
            self.frame_tokens.append(toks)
        return [k for toks in self.frame_tokens for k in toks]

    def replay(self, frames, frame_tokens, tol_fn):
        """Follows another decoder's decisions for ``frames``: ``frame_tokens[t]``
        are the tokens it emitted at frame t, so its decisions there were those
        tokens, then blank if fewer than max_symbols.  Every decision must have a
        logit within ``tol_fn(logits)`` of the maximum (near-ties may break
        either way); the state advances along the given tokens.  Returns
        (decisions, largest shortfall, decisions that differ from this argmax);
        raises AssertionError on a decision beyond the tolerance."""
        P, dt = self.P, self.dtype
        n, worst, differ = 0, 0.0, 0
        e_all = enc_proj(P, frames, dt)
        if len(frame_tokens) != len(e_all):
            raise AssertionError(f"{len(frame_tokens)} frames of tokens for {len(e_all)} frames")
        for e, toks in zip(e_all, frame_tokens):
            if len(toks) > self.max_symbols:
                raise AssertionError(f"{len(toks)} tokens in one frame > {self.max_symbols}")
            choices = list(toks) + ([self.blank] if len(toks) < self.max_symbols else [])
            for choice in choices:
                logits = joint_logits(P, e, pred_proj(P, self.pred_out, dt), dt)
                top = float(logits.max())
                short = top - float(logits[int(choice)])
                n += 1
                worst = max(worst, short)
                differ += int(int(np.argmax(logits)) != int(choice))
                if short > tol_fn(logits):
                    raise AssertionError(
                        f"decision {n}: chose {choice} (logit {logits[int(choice)]:.6f}), "
                        f"maximum {top:.6f} at {int(np.argmax(logits))}"
                    )
                if choice == self.blank:
                    break
                self.pred_out, self.h, self.c = predictor_step(P, int(choice), self.h, self.c, dt)
        return n, worst, differ
