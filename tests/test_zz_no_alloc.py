"""pk_rnnt_greedy_step_static (the decode step on the library's static scratch,
no workspace argument, no allocation) against pk_rnnt_greedy_step with a
caller's workspace, through the C ABI: from the same predictor state, two calls
in a row, the second with a smaller batch, in both list modes; tokens, frame
counts and the updated state (h, c, joint projection) agree bit for bit.  The
static step recorded in a HIP graph (the callers it is for) replays the same
step, replay after replay.  Also the argument checks of the static entry
point."""

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from parakeet_amd import ops
from parakeet_amd._lib import PK_ERR_INVALID, PK_ERR_UNSUPPORTED, lib
from parakeet_amd.modules.decoder import GreedyDecoder, Joiner, Predictor

pytestmark = pytest.mark.gpu


def _decoder(cuda, seed=3, vocab=1026, enc_dim=512, slots=64):
    torch.manual_seed(seed)
    pred = Predictor(640, 640, 1, vocab)
    joint = Joiner(enc_dim, 640, 640, num_classes=vocab)
    with torch.no_grad():
        joint.joint_net[2].weight.mul_(4.0)
        joint.joint_net[2].bias[vocab] += 4.0  # a mix of tokens and blanks
    pred = pred.to(torch.float16).to(cuda).eval().requires_grad_(False)
    joint = joint.to(torch.float16).to(cuda).eval().requires_grad_(False)
    return GreedyDecoder(pred, joint, blank_id=vocab, num_slots=slots)


def _step(dec, slots, enc, static, compact):
    """One decode step through the C ABI; returns (tokens, counts)."""
    B, T, _ = enc.shape
    st = torch.from_numpy(slots.astype(np.int32)).to(dec.device)
    e = F.linear(enc, dec.w_enc, dec.b_enc).contiguous()
    lens = torch.full((B,), T, dtype=torch.int32, device=dec.device)
    tokens = torch.full((B, T * dec.max_symbols), -7, dtype=torch.int32, device=dec.device)
    counts = torch.full((B, T), -7, dtype=torch.int32, device=dec.device)
    dec.compact = compact
    a = dec._args(st, prime=False)
    a.enc_proj, a.enc_stride_b, a.enc_stride_t = e.data_ptr(), e.stride(0), e.stride(1)
    a.lengths, a.max_frames = lens.data_ptr(), T
    a.tokens, a.frame_counts = tokens.data_ptr(), counts.data_ptr()
    if static:
        a.workspace = None
        rc = lib().pk_rnnt_greedy_step_static(ctypes.byref(a), ops._stream(dec.device))
    else:
        rc = lib().pk_rnnt_greedy_step(ctypes.byref(a), ops._stream(dec.device))
    assert rc == 0, lib().pk_last_error()
    torch.cuda.synchronize()
    return tokens.cpu(), counts.cpu()


@pytest.mark.parametrize("compact", [1, -1], ids=["lists", "tiles"])
def test_static_scratch_step_matches_workspace_step(cuda, compact):
    print(f"\n[no-alloc decode] compact={compact}", flush=True)
    dec = _decoder(cuda)
    rng = np.random.default_rng(4)
    g = torch.Generator().manual_seed(5)
    dec.reset_slot(np.arange(64))
    for B in (48, 16):  # the second call smaller: stale scratch from the first must not matter
        slots = rng.permutation(64)[:B]
        enc = torch.randn(B, 3, 512, generator=g).to(torch.float16).to(cuda)
        state = [t.clone() for t in (dec.h, dec.c, dec.pred_proj)]
        tok_ws, cnt_ws = _step(dec, slots, enc, static=False, compact=compact)
        after_ws = [t.clone() for t in (dec.h, dec.c, dec.pred_proj)]
        for t, s in zip((dec.h, dec.c, dec.pred_proj), state):
            t.copy_(s)
        tok_st, cnt_st = _step(dec, slots, enc, static=True, compact=compact)
        print(f"  batch {B}: {int(cnt_ws.sum())} tokens", flush=True)
        assert 0 < int(cnt_ws.sum()) < B * 3 * dec.max_symbols and (cnt_ws >= 0).all()  # tokens and blanks
        assert torch.equal(tok_ws, tok_st) and torch.equal(cnt_ws, cnt_st), f"batch {B}"
        for got, want in zip((dec.h, dec.c, dec.pred_proj), after_ws):
            assert torch.equal(got, want), f"batch {B}: state differs"
    torch.cuda.synchronize()


def test_static_scratch_rejects_oversized_and_workspace(cuda):
    dec = _decoder(cuda, slots=8)
    st = torch.zeros(8, dtype=torch.int32, device=cuda)
    a = dec._args(st, prime=True)  # carries a workspace pointer: rejected
    assert lib().pk_rnnt_greedy_step_static(ctypes.byref(a), ops._stream(cuda)) == PK_ERR_INVALID
    a.workspace = None
    a.batch = 1 << 16  # 65536 streams need far more than the static scratch
    assert lib().pk_rnnt_greedy_step_static(ctypes.byref(a), ops._stream(cuda)) == PK_ERR_UNSUPPORTED
    assert b"static scratch" in lib().pk_last_error()


def test_static_scratch_step_replayed_from_a_graph(cuda):
    """One static step recorded in a HIP graph after an eager call on the device
    (which looks up the scratch address), replayed three times from the same
    predictor state with eager work between: every replay's tokens, frame
    counts and state equal the workspace step's, bit for bit."""
    print("\n[no-alloc decode] graph replay", flush=True)
    dec = _decoder(cuda, seed=7)
    dec.compact = 1
    rng = np.random.default_rng(8)
    g = torch.Generator().manual_seed(9)
    dec.reset_slot(np.arange(64))
    B, T = 40, 3
    slots = rng.permutation(64)[:B]
    enc = torch.randn(B, T, 512, generator=g).to(torch.float16).to(cuda)
    _step(dec, slots, enc, static=True, compact=1)  # eager: the address is looked up here
    state0 = [t.clone() for t in (dec.h, dec.c, dec.pred_proj)]
    tok_ref, cnt_ref = _step(dec, slots, enc, static=False, compact=1)
    after_ref = [t.clone() for t in (dec.h, dec.c, dec.pred_proj)]
    # fixed buffers for the recording
    st = torch.from_numpy(slots.astype(np.int32)).to(cuda)
    e = F.linear(enc, dec.w_enc, dec.b_enc).contiguous()
    lens = torch.full((B,), T, dtype=torch.int32, device=cuda)
    tokens = torch.full((B, T * dec.max_symbols), -7, dtype=torch.int32, device=cuda)
    counts = torch.full((B, T), -7, dtype=torch.int32, device=cuda)
    a = dec._args(st, prime=False)
    a.enc_proj, a.enc_stride_b, a.enc_stride_t = e.data_ptr(), e.stride(0), e.stride(1)
    a.lengths, a.max_frames = lens.data_ptr(), T
    a.tokens, a.frame_counts = tokens.data_ptr(), counts.data_ptr()
    a.workspace = None
    for t, s0 in zip((dec.h, dec.c, dec.pred_proj), state0):
        t.copy_(s0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.graph(graph, stream=side):
        rc = lib().pk_rnnt_greedy_step_static(ctypes.byref(a), ops._stream(cuda))
    torch.cuda.current_stream(cuda).wait_stream(side)
    assert rc == 0, lib().pk_last_error()
    for rep in range(3):
        for t, s0 in zip((dec.h, dec.c, dec.pred_proj), state0):
            t.copy_(s0)
        tokens.fill_(-7)
        counts.fill_(-7)
        _ = torch.randn(1024, 1024, device=cuda) @ torch.randn(1024, 1024, device=cuda)  # eager work between
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(tokens.cpu(), tok_ref) and torch.equal(counts.cpu(), cnt_ref), f"replay {rep}"
        for got, want in zip((dec.h, dec.c, dec.pred_proj), after_ref):
            assert torch.equal(got, want), f"replay {rep}: state differs"
    torch.cuda.synchronize()
