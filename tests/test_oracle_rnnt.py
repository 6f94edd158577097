"""Pins for the RNNT greedy-decoding oracle (oracle/rnnt.py).

The reference ships no tests or fixtures for its decoder; the restatement is
checked against torch's own modules and the reference's batched algorithm:
* predictor_step against nn.Embedding + nn.LSTM (1 and 2 layers) in float64;
* joint_logits against nn.Linear / ReLU composed as Joiner.forward;
* the per-stream greedy loop against ModelRunner._decode_batch /
  _decode_frame_batch (model_runner.py:347-447) rewritten operator for operator
  in float64 torch over a batch of variable-length chunks (length sort, the
  all-blank break, the torch.where state selects);
* replay accepts the oracle's own decisions with no shortfall and rejects a
  planted wrong token.
"""

import numpy as np
import pytest
import torch
from torch import nn

from oracle import rnnt


def _modules(V, H, J, D, layers, seed):
    torch.manual_seed(seed)
    embed = nn.Embedding(V + 1, H, padding_idx=V)
    lstm = nn.LSTM(input_size=H, hidden_size=H, num_layers=layers)
    enc, pred = nn.Linear(D, J), nn.Linear(H, J)
    out = nn.Linear(J, V + 1)
    with torch.no_grad():  # a larger output scale so blanks and tokens both occur
        out.weight.mul_(6.0)
        out.bias[V] += 2.0
    mods = [m.double() for m in (embed, lstm, enc, pred, out)]
    pred_sd = {"prediction.embed.weight": embed.weight}
    pred_sd.update({f"prediction.dec_rnn.{k}": v for k, v in lstm.state_dict().items()})
    joint_sd = {"enc.weight": enc.weight, "enc.bias": enc.bias, "pred.weight": pred.weight, "pred.bias": pred.bias,
                "joint_net.2.weight": out.weight, "joint_net.2.bias": out.bias}
    return mods, rnnt.RnntParams(pred_sd, joint_sd, layers)


@pytest.mark.parametrize("layers", [1, 2])
def test_predictor_step_matches_torch_lstm(layers):
    V, H = 30, 24
    (embed, lstm, *_), P = _modules(V, H, 16, 20, layers, seed=layers)
    g = torch.Generator().manual_seed(0)
    h = torch.randn(layers, 1, H, generator=g, dtype=torch.float64)
    c = torch.randn(layers, 1, H, generator=g, dtype=torch.float64)
    for tok in (3, V, 0):
        with torch.no_grad():
            y = embed(torch.tensor([[tok]])).transpose(0, 1)  # decoder.py:45-47
            g_out, (h2, c2) = lstm(y, (h, c))
        po, hh, cc = rnnt.predictor_step(P, tok, h[:, 0].numpy(), c[:, 0].numpy())
        np.testing.assert_allclose(po, g_out[0, 0].numpy(), atol=1e-13)
        np.testing.assert_allclose(hh, h2[:, 0].numpy(), atol=1e-13)
        np.testing.assert_allclose(cc, c2[:, 0].numpy(), atol=1e-13)
        h, c = h2, c2
    assert not P.embed[V].any()  # padding_idx row: the blank start token embeds to zero


def test_joint_matches_joiner_composition():
    V, H, J, D = 30, 24, 16, 20
    (_, _, enc, pred, out), P = _modules(V, H, J, D, 1, seed=3)
    g = torch.Generator().manual_seed(1)
    e = torch.randn(4, 1, D, generator=g, dtype=torch.float64)
    p = torch.randn(4, H, generator=g, dtype=torch.float64)
    with torch.no_grad():  # decoder.py:82-86
        ref = out(torch.relu(enc(e) + pred(p).unsqueeze(1))).squeeze(1).numpy()
    got = np.stack([rnnt.joint_logits(P, rnnt.enc_proj(P, e[b, 0].numpy()), rnnt.pred_proj(P, p[b].numpy())) for b in range(4)])
    np.testing.assert_allclose(got, ref, atol=1e-12)


def _reference_batched(mods, blank, chunks, pred_outs, states, max_symbols=5):
    """model_runner.py:347-447 in float64 torch, operator for operator (the
    Predictor and Joiner forwards of decoder.py:44-50,82-86)."""
    embed, lstm, enc, pred, out = mods

    def decoder(ids, state):
        y = embed(ids.reshape(-1, 1)).transpose(0, 1)
        g, hidden = lstm(y, state)
        return g.transpose(0, 1)[:, -1, :], hidden

    def joiner(frame, pred_out):
        return out(torch.relu(enc(frame) + pred(pred_out).unsqueeze(1))).squeeze(1)

    lengths = [int(c.size(2)) for c in chunks]
    order = sorted(range(len(chunks)), key=lengths.__getitem__, reverse=True)
    s_chunks = [chunks[i] for i in order]
    s_len = [lengths[i] for i in order]
    s_po = [pred_outs[i] for i in order]
    s_st = [states[i] for i in order]
    toks_sorted = [[] for _ in order]
    batch = len(order)
    with torch.no_grad():
        for t in range(s_len[0]):
            while batch > 0 and t >= s_len[batch - 1]:
                batch -= 1
            if batch == 0:
                break
            frame = torch.cat([s_chunks[r][:, :, t].unsqueeze(1) for r in range(batch)])
            po = torch.cat(s_po[:batch])
            st = tuple(torch.cat([s[k] for s in s_st[:batch]], dim=1) for k in range(2))
            token_lists = [[] for _ in range(batch)]
            for _ in range(max_symbols):
                ids = joiner(frame, po).argmax(-1)
                blank_mask = ids == blank
                if bool(blank_mask.all()):
                    break
                for idx, tok in enumerate(ids.tolist()):
                    if tok != blank:
                        token_lists[idx].append(tok)
                new_po, new_st = decoder(ids, st)
                po = torch.where(blank_mask.unsqueeze(-1), po, new_po)
                st = tuple(torch.where(blank_mask.view(1, -1, 1), o, n) for o, n in zip(st, new_st))
            for r in range(batch):
                toks_sorted[r].extend(token_lists[r])
                s_po[r] = po[r : r + 1]
                s_st[r] = tuple(x[:, r : r + 1] for x in st)
    res = [None] * len(order)
    for si, oi in enumerate(order):
        res[oi] = toks_sorted[si]
    return res


@pytest.mark.parametrize("layers", [1, 2])
def test_per_stream_greedy_equals_the_reference_batched_loop(layers):
    V, H, J, D = 40, 24, 16, 20
    mods, P = _modules(V, H, J, D, layers, seed=10 + layers)
    blank = V
    g = torch.Generator().manual_seed(2)
    B = 6
    decs = [rnnt.StreamDecoder(P, blank) for _ in range(B)]
    pred_outs = [torch.from_numpy(d.pred_out)[None] for d in decs]
    states = [(torch.from_numpy(d.h)[:, None].clone(), torch.from_numpy(d.c)[:, None].clone()) for d in decs]
    total = 0
    for step in range(4):
        chunks = [torch.randn(1, D, int(T), generator=g, dtype=torch.float64) for T in (2, 1, 2, 3, 2, 1)]
        ref = _reference_batched(mods, blank, chunks, pred_outs, states)
        for b in range(B):
            got = decs[b].decode(chunks[b][0].t().numpy())
            assert got == ref[b], f"step {step} stream {b}"
            total += len(got)
            pred_outs[b] = torch.from_numpy(decs[b].pred_out)[None]
            states[b] = (torch.from_numpy(decs[b].h)[:, None].clone(), torch.from_numpy(decs[b].c)[:, None].clone())
    assert total > 10  # tokens were emitted, not only blanks


def test_replay_accepts_own_decisions_and_rejects_a_planted_token():
    V, H, J, D = 40, 24, 16, 20
    _, P = _modules(V, H, J, D, 1, seed=21)
    frames = np.random.default_rng(3).standard_normal((6, D))
    a = rnnt.StreamDecoder(P, V)
    a.decode(frames)
    ft = a.frame_tokens
    assert sum(len(t) for t in ft) > 0
    b = rnnt.StreamDecoder(P, V)
    n, worst, differ = b.replay(frames, ft, lambda lg: 0.0)
    assert worst == 0.0 and differ == 0 and n >= len(ft)
    bad = [list(t) for t in ft]
    k = next(i for i, t in enumerate(bad) if t)
    bad[k][0] = (bad[k][0] + 1) % V
    with pytest.raises(AssertionError):
        rnnt.StreamDecoder(P, V).replay(frames, bad, lambda lg: 1e-3)
