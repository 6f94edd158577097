"""GPU parity of the drop-in modules -- the reference's Python surfaces on the
paged cache -- against the oracle:

* ModelCache.update_attn_cache (parakeet/modules/cache.py:36-45): the returned
  windows equal the dense shift buffer bit for bit, step after step, through
  the full cache, prefix views (cache.py:65-77) and shuffled slot subsets (the
  batches Scheduler.pack_states forms), with slot resets (cache.py:60-63);
* ConformerAttention.forward (parakeet/modules/attention.py:85-125) with its
  own projections: the module's q/k/v and position projections feed the
  oracle's float64 rel-pos attention over the dense window, and linear_out is
  applied in float64; with a cache over several steps, and without a cache;
* ConformerEncoder (parakeet/modules/encoder.py:140-267): streaming steps of a
  random-init 2-layer stack on the GPU against the same weights in float64 on
  the CPU where every layer's attention is the oracle over a dense cache, every
  layer's convolution step is the oracle's (convolution.py:150-158 with its
  dense conv cache) and the masks are the oracle's loop (encoder.py:167-227);
  the state scalars advance as encoder.py:257-260.
"""

import copy

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import masks as om
from parakeet_amd.modules.attention import ConformerAttention, PositionalEncoding
from parakeet_amd.modules.cache import ModelCache, StreamingState
from parakeet_amd.modules.encoder import ConformerEncoder

from _dense_encoder import DenseCache as _DenseCache
from _dense_encoder import dense_shift as _dense_shift
from _dense_encoder import init_attention as _init_attention
from _dense_encoder import oracle_attention as _oracle_attention
from _dense_encoder import oracle_conv as _oracle_conv
from _dense_encoder import torch_residual_norm


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_model_cache_windows_match_dense(cuda, dtype):
    print(f"\n[model-cache] {dtype}", flush=True)
    left, right, D, Ly, N = 9, 1, 64, 2, 5
    T = right + 1
    L = left + T
    mc = ModelCache(Ly, (left, right), D, 9, batch_size=N, device=cuda, dtype=dtype, page_size=4)
    win_k = np.zeros((N, Ly, L, D))
    win_v = np.zeros((N, Ly, L, D))
    rng = np.random.default_rng(0)
    g = torch.Generator().manual_seed(0)
    for step in range(30):
        if step % 7 == 6:
            s = step % N
            mc.reset_slot(s)
            win_k[s] = 0
            win_v[s] = 0
        kind = step % 3
        if kind == 0:
            view, slots = mc, np.arange(N)
        elif kind == 1:
            view, slots = mc.view(3), np.arange(3)
        else:
            slots = rng.permutation(N)[:4]
            view = mc.batch(slots)
        B = len(slots)
        for layer in range(Ly):
            x = torch.randn(B, T, 3 * D, generator=g).to(dtype)
            _, k, v = x.to(cuda).chunk(3, dim=-1)  # strided views, as qkv.chunk(3)
            gk, gv = view.update_attn_cache(layer, k, v)
            kc, vc = k.cpu().double().numpy(), v.cpu().double().numpy()
            for b, s in enumerate(slots):
                _dense_shift(win_k, s, layer, left, kc[b])
                _dense_shift(win_v, s, layer, left, vc[b])
            assert torch.equal(gk.cpu(), torch.from_numpy(win_k[slots, layer]).to(dtype)), f"step {step} layer {layer}"
            assert torch.equal(gv.cpu(), torch.from_numpy(win_v[slots, layer]).to(dtype)), f"step {step} layer {layer}"
    torch.cuda.synchronize()


# fp32: the kernel's 1e-4; fp16: the kernel's 2e-3 plus linear_out's fp16
# rounding of its input and output (outputs are O(1)); bf16 the same rule on the
# kernel's 1e-2 (bf16 keeps 3 mantissa bits fewer than fp16)
ATT_TOL = {torch.float32: 1e-4, torch.float16: 6e-3, torch.bfloat16: 3e-2}


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_conformer_attention_matches_oracle(cuda, dtype):
    print(f"\n[conformer-attention] {dtype}", flush=True)
    H, dk, left, right, B = 8, 64, 20, 1, 3
    D, T = H * dk, right + 1
    L = left + T
    att = ConformerAttention(0, H, D)
    _init_attention(att, D, seed=1)
    att = att.to(device=cuda, dtype=dtype)
    pe = PositionalEncoding(D, 0.0, 128, 0.0)
    pe.extend_pe(128, device=cuda)
    mc = ModelCache(1, (left, right), D, 9, batch_size=B, device=cuda, dtype=dtype, page_size=16)
    win_k = np.zeros((B, 1, L, D))
    win_v = np.zeros((B, 1, L, D))
    proc = np.zeros(B, dtype=np.int64)
    g = torch.Generator().manual_seed(2)
    w_out = att.linear_out.weight.detach().double().cpu().numpy()
    bu = att.pos_bias_u.detach().double().cpu().numpy()
    bv = att.pos_bias_v.detach().double().cpu().numpy()
    worst = 0.0
    for step in range(14):
        x = torch.randn(B, T, D, generator=g).to(dtype).to(cuda)
        _, pos_emb = pe(x, cache_len=left)
        pos_emb = pos_emb.to(dtype)
        cl = np.minimum(proc, left)
        _, mask = om.create_streaming_masks(T, cl, proc, T, (left, right))
        with torch.no_grad():
            out = att(x, pos_emb, torch.from_numpy(mask).to(cuda), cache=mc)
            q, k, v = (t.double().cpu().numpy() for t in att.qkv(x).chunk(3, dim=-1))
            pos = att.linear_pos(pos_emb)[0].double().cpu().numpy()
        for b in range(B):
            _dense_shift(win_k, b, 0, left, k[b])
            _dense_shift(win_v, b, 0, left, v[b])
        core = oa.relpos_attention(q, win_k[:, 0], win_v[:, 0], pos, bu, bv, mask, H)
        ref = core @ w_out.T
        err = float(np.abs(out.double().cpu().numpy() - ref).max())
        worst = max(worst, err)
        assert err <= ATT_TOL[dtype], f"step {step}: max abs err {err:.3e}"
        proc += T
    print(f"  worst max-abs error {worst:.3e}", flush=True)
    # without a cache the keys are this chunk's frames only
    x = torch.randn(B, T, D, generator=g).to(dtype).to(cuda)
    _, pos_emb = pe(x, cache_len=0)
    pos_emb = pos_emb.to(dtype)
    with torch.no_grad():
        out = att(x, pos_emb, None, cache=None)
        q, k, v = (t.double().cpu().numpy() for t in att.qkv(x).chunk(3, dim=-1))
        pos = att.linear_pos(pos_emb)[0].double().cpu().numpy()
    ref = oa.relpos_attention(q, k, v, pos, bu, bv, None, H) @ w_out.T
    assert float(np.abs(out.double().cpu().numpy() - ref).max()) <= ATT_TOL[dtype]
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_conformer_attention_per_stream_position_tables(cuda, dtype):
    """pos_emb of batch B: every stream attends with its own position table, as
    the reference's broadcast of linear_pos(pos_emb) [B, P, H, dk] against the
    queries does (attention.py:102-113); each stream is checked against the
    oracle with its own table, through eviction."""
    print(f"\n[conformer-attention per-stream pos] {dtype}", flush=True)
    H, dk, left, right, B = 8, 64, 20, 1, 3
    D, T = H * dk, right + 1
    L = left + T
    att = ConformerAttention(0, H, D)
    _init_attention(att, D, seed=3)
    att = att.to(device=cuda, dtype=dtype)
    mc = ModelCache(1, (left, right), D, 9, batch_size=B, device=cuda, dtype=dtype, page_size=16)
    win_k = np.zeros((B, 1, L, D))
    win_v = np.zeros((B, 1, L, D))
    proc = np.zeros(B, dtype=np.int64)
    g = torch.Generator().manual_seed(4)
    w_out = att.linear_out.weight.detach().double().cpu().numpy()
    bu = att.pos_bias_u.detach().double().cpu().numpy()
    bv = att.pos_bias_v.detach().double().cpu().numpy()
    worst = 0.0
    for step in range(14):
        x = torch.randn(B, T, D, generator=g).to(dtype).to(cuda)
        pos_emb = torch.randn(B, 2 * L - 1, D, generator=g).to(dtype).to(cuda)  # a different table per stream
        cl = np.minimum(proc, left)
        _, mask = om.create_streaming_masks(T, cl, proc, T, (left, right))
        with torch.no_grad():
            out = att(x, pos_emb, torch.from_numpy(mask).to(cuda), cache=mc)
            q, k, v = (t.double().cpu().numpy() for t in att.qkv(x).chunk(3, dim=-1))
            pos = att.linear_pos(pos_emb).double().cpu().numpy()
        for b in range(B):
            _dense_shift(win_k, b, 0, left, k[b])
            _dense_shift(win_v, b, 0, left, v[b])
        for b in range(B):
            core = oa.relpos_attention(q[b : b + 1], win_k[b : b + 1, 0], win_v[b : b + 1, 0], pos[b], bu, bv,
                                       mask[b : b + 1], H)
            err = float(np.abs(out[b].double().cpu().numpy() - (core @ w_out.T)[0]).max())
            worst = max(worst, err)
            assert err <= ATT_TOL[dtype], f"step {step} stream {b}: max abs err {err:.3e}"
        proc += T
    print(f"  worst max-abs error {worst:.3e}", flush=True)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_encoder_streaming_matches_dense_reference(cuda):
    print("\n[encoder] 2 layers fp32 vs float64 dense reference", flush=True)
    left, right, D, H, Ly, B, K = 6, 1, 128, 2, 2, 3, 9
    T = right + 1
    torch.manual_seed(3)
    enc = ConformerEncoder(
        feat_in=80, hidden_size=D, ff_expansion_factor=2, num_layers=Ly, num_heads=H,
        subsampling_factor=8, pos_emb_max_len=64, conv_kernel_size=K, att_context_size=[left, right],
        subsampling_conv_channels=32, use_bias=False, page_size=4,
    )
    for layer in enc.layers:
        _init_attention(layer.self_attn, D, seed=10 + layer.layer_idx)
    ref = copy.deepcopy(enc).double()
    enc = enc.to(cuda)
    state = enc.init_streaming_state(batch_size=B, device=cuda, dtype=torch.float32)
    dense = _DenseCache(B, Ly, left, right, D, K)
    for layer in ref.layers:
        layer.self_attn.forward = _oracle_attention(layer.self_attn, left, H)
        layer.conv.forward = _oracle_conv(layer.conv)
        layer.residual_norm = torch_residual_norm
    proc = np.zeros(B, dtype=np.int64)
    cl = np.zeros(B, dtype=np.int64)

    def ref_masks(current_len, cache_lengths, processed_frames, device, lengths):
        pad, att = om.create_streaming_masks(
            current_len, cache_lengths.numpy(), processed_frames.numpy(), lengths.numpy(), (left, right)
        )
        return torch.from_numpy(pad), torch.from_numpy(att)

    ref._create_streaming_masks = ref_masks
    g = torch.Generator().manual_seed(4)
    worst = 0.0
    for step in range(12):
        x = torch.randn(B, T, D, generator=g)
        # the engine passes per-stream lengths as a tensor (model_runner.py:285-291)
        lengths = torch.full((B,), T, dtype=torch.int64)
        with torch.no_grad():
            out, state = enc(x.to(cuda), state, length=lengths.to(cuda))
            rstate = StreamingState(dense, torch.from_numpy(proc.copy()), torch.from_numpy(cl.copy()))
            rout, _ = ref(x.double(), rstate, length=lengths)
        err = float((out.double().cpu() - rout).abs().max())
        worst = max(worst, err)
        assert err <= 2e-4, f"step {step}: max abs err {err:.3e}"
        proc += T
        cl = np.minimum(cl + T, left)
        assert state.processed_frames.cpu().tolist() == proc.tolist()
        assert state.cache_lengths.cpu().tolist() == cl.tolist()
    print(f"  worst max-abs error {worst:.3e}", flush=True)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_encoder_step_graph_matches_eager_steps(cuda, dtype):
    """EncoderStepGraph (one recorded step replayed per call) against the eager
    forward on a second state with the same weights: outputs, state counters,
    conv state and the pages of every layer agree bit for bit, step after step
    (eviction included), with the eager path's launches between the replays.
    Halfway, every layer's linear_pos weight changes in place before a replay:
    the replay refreshes the kept position projections it reads."""
    print(f"\n[encoder graph] 2 layers {dtype} replay vs eager", flush=True)
    from parakeet_amd.modules.encoder import EncoderStepGraph

    left, right, D, H, Ly, B, K = 10, 1, 128, 2, 2, 5, 9
    T = right + 1
    torch.manual_seed(5)
    enc = ConformerEncoder(
        feat_in=80, hidden_size=D, ff_expansion_factor=2, num_layers=Ly, num_heads=H,
        subsampling_factor=8, pos_emb_max_len=64, conv_kernel_size=K, att_context_size=[left, right],
        subsampling_conv_channels=32, use_bias=False, page_size=4,
    )
    for layer in enc.layers:
        _init_attention(layer.self_attn, D, seed=20 + layer.layer_idx)
    enc = enc.to(cuda).to(dtype).eval().requires_grad_(False)
    eager = enc.init_streaming_state(batch_size=B, device=cuda, dtype=dtype)
    replay = enc.init_streaming_state(batch_size=B, device=cuda, dtype=dtype)
    length = torch.full((B,), T, dtype=torch.int64, device=cuda)
    graph = EncoderStepGraph(enc, replay, length)
    g = torch.Generator().manual_seed(6)
    with torch.no_grad():
        for step in range(12):  # the window fills after 5 steps; pages are evicted from then on
            x = torch.randn(B, T, D, generator=g).to(dtype).to(cuda)
            if step == 6:
                for layer in enc.layers:
                    layer.self_attn.linear_pos.weight.mul_(1.5)
            got = graph(x)
            ref, _ = enc(x, eager, length=length)
            assert torch.equal(got, ref), f"step {step}: max diff {(got.float() - ref.float()).abs().max():.3e}"
            assert torch.equal(replay.processed_frames, eager.processed_frames)
            assert torch.equal(replay.cache_lengths, eager.cache_lengths)
            assert torch.equal(replay.cache.conv_frames, eager.cache.conv_frames)
            for layer in range(Ly):
                kr, vr = replay.cache.window(layer)
                ke, ve = eager.cache.window(layer)
                assert torch.equal(kr, ke) and torch.equal(vr, ve), f"step {step} layer {layer}"
    assert graph.graph is not None
    assert replay.processed_frames.tolist() == [12 * T] * B
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_kept_position_projection_follows_its_inputs(cuda):
    """projected_pos keeps linear_pos(pos_emb) in one buffer and recomputes it
    after an in-place change of the weights or the table; with gradients
    enabled it keeps nothing (linear_pos stays trainable)."""
    from parakeet_amd.modules.attention import ConformerAttention

    att = ConformerAttention(layer_idx=0, num_heads=2, hidden_size=64).to(cuda)
    pe = torch.randn(1, 9, 64, device=cuda)
    with torch.no_grad():
        first = att.projected_pos(pe)
        kept = first.data_ptr()
        assert torch.equal(first, att.linear_pos(pe))
        before = first.clone()
        assert att.projected_pos(pe).data_ptr() == kept  # no recomputation
        att.linear_pos.weight.mul_(2.0)
        again = att.projected_pos(pe)
        assert again.data_ptr() == kept and torch.equal(again, att.linear_pos(pe))
        assert not torch.equal(again, before)
        pe.add_(1.0)
        assert torch.equal(att.projected_pos(pe), att.linear_pos(pe))
    y = att.projected_pos(pe)
    y.float().sum().backward()
    assert att.linear_pos.weight.grad is not None


@pytest.mark.gpu
@pytest.mark.parametrize("sync_each_step", [True, False])
def test_engine_loop_with_scheduler_matches_per_stream_reference(cuda, sync_each_step):
    """The reference's _encode_step call pattern (parakeet/engine/model_runner.py:
    254-304) on the drop-ins: Scheduler.init_state_pool, acquire_state_slot,
    pack_states -> encoder(batch, state, length) -> unpack_states,
    release_state_slot (scheduler.py:68-201), with streams arriving and leaving,
    batches of varying slot subsets in varying order, and slots reused by new
    streams.  Every stream's output of every step equals the float64 reference
    encoder (oracle attention over a dense shift cache, oracle conv step, oracle
    masks) run on that stream alone from its own start: streams are independent,
    so that is what the reference's batched pack / unpack computes.  Without a
    synchronisation per step, every release and re-acquire happens while earlier
    steps may still run on the GPU (the reference's "release while a chunk is in
    flight"); stream order keeps the reused pages and slots correct."""
    print("\n[engine loop] scheduler + paged encoder vs per-stream dense reference", flush=True)
    from parakeet_amd.engine.scheduler import Scheduler

    left, right, D, H, Ly, K, S = 6, 1, 128, 2, 2, 9, 4
    T = right + 1
    torch.manual_seed(7)
    enc = ConformerEncoder(
        feat_in=80, hidden_size=D, ff_expansion_factor=2, num_layers=Ly, num_heads=H,
        subsampling_factor=8, pos_emb_max_len=64, conv_kernel_size=K, att_context_size=[left, right],
        subsampling_conv_channels=32, use_bias=False, page_size=4,
    )
    for layer in enc.layers:
        _init_attention(layer.self_attn, D, seed=30 + layer.layer_idx)
    ref = copy.deepcopy(enc).double()
    for layer in ref.layers:
        layer.self_attn.forward = _oracle_attention(layer.self_attn, left, H)
        layer.conv.forward = _oracle_conv(layer.conv)
        layer.residual_norm = torch_residual_norm

    def ref_masks(current_len, cache_lengths, processed_frames, device, lengths):
        pad, att = om.create_streaming_masks(
            current_len, cache_lengths.numpy(), processed_frames.numpy(), lengths.numpy(), (left, right)
        )
        return torch.from_numpy(pad), torch.from_numpy(att)

    ref._create_streaming_masks = ref_masks
    enc = enc.to(cuda)
    sch = Scheduler(max_active=S)
    sch.init_state_pool(enc, cuda, torch.float32, pool_size=S, page_size=4)

    class Seq:
        def __init__(self, slot, steps):
            self.status = None
            self.encoder_state = slot
            self.steps = steps
            self.done = 0
            self.dense = _DenseCache(1, Ly, left, right, D, K)
            self.proc = 0
            self.cl = 0

    rng = np.random.default_rng(12)
    g = torch.Generator().manual_seed(13)
    live: list[Seq] = []
    deferred = []  # (GPU output, input, streams, their (proc, cache_len)) checked at the end
    slot_users: dict[int, int] = {}
    compared = worst = 0.0
    with torch.no_grad():
        for step in range(40):
            while rng.random() < 0.6:  # arrivals until the pool is full
                slot = sch.acquire_state_slot()
                if slot is None:
                    break
                live.append(Seq(slot, int(rng.integers(3, 12))))
                slot_users[slot] = slot_users.get(slot, 0) + 1
            ready = [s for s in live if rng.random() < 0.8]
            rng.shuffle(ready)
            if ready:
                B = len(ready)
                x = torch.randn(B, T, D, generator=g)
                state, index = sch.pack_states(ready)
                out, state = enc(x.to(cuda), state, length=torch.full((B,), T, dtype=torch.int64, device=cuda))
                sch.unpack_states(state, index)
                if not sync_each_step:
                    deferred.append((out.clone(), x, list(ready), [(s.proc, s.cl) for s in ready]))
                    for s in ready:
                        s.proc += T
                        s.cl = min(s.cl + T, left)
                        s.done += 1
                else:
                    out = out.double().cpu()
                    for b, s in enumerate(ready):
                        rstate = StreamingState(
                            s.dense, torch.tensor([s.proc], dtype=torch.int64), torch.tensor([s.cl], dtype=torch.int64)
                        )
                        rout, _ = ref(x[b : b + 1].double(), rstate, length=torch.full((1,), T, dtype=torch.int64))
                        err = float((out[b] - rout[0]).abs().max())
                        worst = max(worst, err)
                        assert err <= 2e-4, f"step {step} slot {s.encoder_state}: max abs err {err:.3e}"
                        s.proc += T
                        s.cl = min(s.cl + T, left)
                        s.done += 1
                        compared += 1
                    pf = sch.pool_state.processed_frames.cpu().tolist()
                    for s in live:
                        assert pf[s.encoder_state] == s.proc
            for s in [s for s in live if s.done >= s.steps]:  # departures
                sch.release_state_slot(s.encoder_state)
                live.remove(s)
        for out, x, streams, pre in deferred:  # the reference, in step order, per stream
            out = out.double().cpu()
            for b, (s, (proc, cl)) in enumerate(zip(streams, pre)):
                rstate = StreamingState(s.dense, torch.tensor([proc], dtype=torch.int64), torch.tensor([cl], dtype=torch.int64))
                rout, _ = ref(x[b : b + 1].double(), rstate, length=torch.full((1,), T, dtype=torch.int64))
                err = float((out[b] - rout[0]).abs().max())
                worst = max(worst, err)
                assert err <= 2e-4, f"deferred check, slot {s.encoder_state}: max abs err {err:.3e}"
                compared += 1
    assert compared >= 60, compared
    assert max(slot_users.values()) >= 2, "no slot was reused by a new stream"
    print(f"  {int(compared)} stream-steps, worst max-abs error {worst:.3e}", flush=True)
    torch.cuda.synchronize()
