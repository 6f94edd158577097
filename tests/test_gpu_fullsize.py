"""The paged path at full stream counts on the GPU, driven by the serving-loop
step (parakeet_amd.step.AttentionStep) with continuous arrivals and departures:

* large shape (d_model 1024, 8 heads x 128, bf16) with 256 stream slots at 90%
  steady occupancy, lifetimes U(2, 30) s (the 256-stream benchmark workload);
* fragmentation stress: small shape (d_model 512, 8 x 64, fp16), 1024 slots,
  the page pool pre-shuffled by a seeded permutation, lifetimes log-U(1, 60) s;
* the large shape at the large model's own chunk of 14 frames (att_context
  (70, 13), parakeet/config.py:29), 256 slots at 90% occupancy.

Four layers for the large shape and two for the fragmentation stress, over
enough steps that windows fill, pages are evicted and reused, and slots are
reused by new streams.  A launch's windows over all layers pass the host's
192 MiB streaming threshold in both (230 x 72 x 1024 x 2 bytes x K and V x 4
layers = 271 MB; 1024 x 72 x 512 x 2 x 2 x 2 = 302 MB), so the kernels read
with the streaming cache policy, as in the 24-layer benchmark.  Every step:
* the block-table rows the host pool hands the kernels equal the oracle's FIFO
  page-pool model (oracle/paging.py, scheduler.py:84,97,104) fed the same slot
  sequence, bit for bit;
* every live stream's window read back from the pages (pk_kv_gather), after the
  kernel's fused append, equals a dense shift buffer on the device updated with
  plain torch copies (the semantics of cache.py:36-45; a departed slot starts
  from zeros, scheduler.py:86-91), bit for bit; the pools start NaN-filled, so
  a read of a never-written row shows;
and every 20 steps four sampled streams' attention outputs of each layer are
compared with the float64 oracle (attention.py:94-121) over the dense window
with the reference's mask loop (encoder.py:167-227): max-abs 2e-3 (fp16),
1e-2 (bf16).
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import masks as om
from oracle import paging
from parakeet_amd import ops, synth
from parakeet_amd.pool import pages_per_slot
from parakeet_amd.step import AttentionStep

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}

CASES = {
    # shape, slots, occupancy, lifetimes, shuffled pool, seed, steps
    "large_256slots_bf16": (synth.Shape("large-4layer-bf16", 4, 1024, 8, dtype=torch.bfloat16), 256, 0.9,
                            ("uniform", 2.0, 30.0), False, 3, 220),
    "frag_1024slots_fp16": (synth.Shape("small-2layer-fp16", 2, 512, 8, dtype=torch.float16), 1024, 1.0,
                            ("loguniform", 1.0, 60.0), True, 4, 300),
    # the large model's own context (70, 13): 14 frames a step, 84-frame windows
    # (the whole-chunk kernel; 230 x 84 x 1024 x 2 x 2 x 4 = 317 MB a launch, streaming)
    "large_t14_256slots_bf16": (synth.Shape("large-4layer-bf16-t14", 4, 1024, 8, right=13, dtype=torch.bfloat16), 256,
                                0.9, ("uniform", 2.0, 30.0), False, 3, 80),
}


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("case", sorted(CASES))
def test_full_size_churn_pages_and_attention(cuda, case):
    shape, S, occ, durations, shuffle, seed, steps = CASES[case]
    print(f"\n[full size] {case}: {S} slots, {steps} steps", flush=True)
    T, D, Ly, L, left, H = shape.chunk, shape.d_model, shape.layers, shape.window, shape.left, shape.heads
    M = pages_per_slot(left, T, shape.page_size)
    order = np.random.default_rng(seed).permutation(S * M) if shuffle else None
    qkv = [torch.zeros(S, T, 3 * D, dtype=shape.dtype, device=cuda) for _ in range(Ly)]
    pos, _, _ = synth.relpos_inputs(shape, cuda, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    bu = [(torch.randn(H, shape.head_dim, generator=g) * 0.02).to(shape.dtype).to(cuda) for _ in range(Ly)]
    bv = [(torch.randn(H, shape.head_dim, generator=g) * 0.02).to(shape.dtype).to(cuda) for _ in range(Ly)]
    st = AttentionStep(shape, S, cuda, qkv, pos, bu, bv, page_order=order)
    st.k_pages.fill_(float("nan"))
    st.v_pages.fill_(float("nan"))
    model = paging.PagePoolModel(st.pool.num_pages, S, shape.page_size, left, T, page_order=order)
    churn = synth.Churn(num_slots=S, chunk=T, occupancy=occ, durations=durations, seed=seed)
    win_k = torch.zeros((S, Ly, L, D), dtype=shape.dtype, device=cuda)
    win_v = torch.zeros_like(win_k)
    proc = np.zeros(S, dtype=np.int64)
    cl = np.zeros(S, dtype=np.int64)
    gdev = torch.Generator(device=cuda).manual_seed(seed + 2)
    rng = np.random.default_rng(seed + 3)
    pos64 = pos.double().cpu().numpy()
    worst, departures, reused, checked = 0.0, 0, 0, 0
    used = np.zeros(S, dtype=bool)
    for step in range(steps):
        departed, arrived = churn.step()
        if departed:
            st.reset_slots(departed)
            for s in departed:
                model.reset_slot(s)
            d = torch.as_tensor(departed, dtype=torch.long, device=cuda)
            win_k[d] = 0
            win_v[d] = 0
            proc[departed] = 0
            cl[departed] = 0
            departures += len(departed)
        reused += int(used[arrived].sum()) if arrived else 0
        used[arrived] = True
        active = np.asarray(churn.active(), dtype=np.int32)
        B = len(active)
        for layer in range(Ly):
            qkv[layer][:B] = torch.randn((B, T, 3 * D), generator=gdev, device=cuda, dtype=torch.float32).to(shape.dtype)
        st.step(active)
        rows_ref = model.advance(active)
        assert np.array_equal(st.rows[:B].cpu().numpy(), rows_ref), f"step {step}: block-table rows differ from the model"
        idx = torch.from_numpy(active.astype(np.int64)).to(cuda)
        pages = ops.PagedKV(st.k_pages, st.v_pages, st.rows[:B], st.pool.max_pages)
        every = 20 if T <= 2 else 10
        sample = rng.choice(B, size=min(4, B), replace=False) if step % every == every - 1 else None
        if sample is not None:
            _, mask = om.create_streaming_masks(T, cl[active[sample]], proc[active[sample]], T, (left, shape.right))
        for layer in range(Ly):
            k = qkv[layer][:B, :, D : 2 * D]
            v = qkv[layer][:B, :, 2 * D :]
            for win, new in ((win_k, k), (win_v, v)):  # cache.py:37-44 per stream
                w = win[idx, layer]
                w[:, :left] = w[:, T:].clone()
                w[:, left:] = new
                win[idx, layer] = w
            gk, gv = ops.kv_gather(pages, layer, B, L, T)
            assert torch.equal(_bits(gk), _bits(win_k[idx, layer])), f"step {step} layer {layer}: K pages"
            assert torch.equal(_bits(gv), _bits(win_v[idx, layer])), f"step {step} layer {layer}: V pages"
            if sample is not None:
                q = qkv[layer][:B][sample, :, :D].double().cpu().numpy()
                ref = oa.relpos_attention(
                    q, win_k[idx[sample], layer].double().cpu().numpy(), win_v[idx[sample], layer].double().cpu().numpy(),
                    pos64, bu[layer].double().cpu().numpy(), bv[layer].double().cpu().numpy(), mask, H,
                )
                got = st.out[layer][:B][sample].double().cpu().numpy()
                err = float(np.abs(got - ref).max())
                worst = max(worst, err)
                assert err <= TOL[shape.dtype], f"step {step} layer {layer}: attention max-abs err {err:.3e}"
                checked += len(sample)
        proc[active] += T  # encoder.py:257-260
        cl[active] = np.minimum(cl[active] + T, left)
        if step % 50 == 0:
            print(f"  step {step}: {B} live, {departures} departures so far", flush=True)
    torch.cuda.synchronize()
    assert departures > S // 4 and reused > 0, (departures, reused)
    assert int(proc.max()) > L, "no window filled"
    print(f"  {departures} departures, {reused} slot reuses, {checked} stream-layers against the oracle, "
          f"worst attention error {worst:.3e}", flush=True)
