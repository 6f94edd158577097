"""GPU parity of the serving-loop step (parakeet_amd.step.AttentionStep): every
layer's paged attention output against the oracle, step after step, with stream
arrivals and departures (slot resets), batches that name a subset of the slots
in shuffled order, and a pre-shuffled page pool.

The oracle keeps one dense shift-buffer window per slot
(parakeet/modules/cache.py:36-45), the reference's per-stream mask loop
(parakeet/modules/encoder.py:167-227) over the batch's state scalars, and the
float64 rel-pos attention (attention.py:94-121).  Tolerance as in
test_gpu_attention.py; pages are also checked bit-exact through pk_kv_gather.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import masks as om
from parakeet_amd import ops, synth
from parakeet_amd.step import AttentionStep

TOL = {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _run(cuda, shape, slots, steps, seed, rows_per_lane=0, graph=False):
    print(f"\n[step] {shape.name} slots={slots} steps={steps} nr={rows_per_lane} graph={graph}", flush=True)
    T, D, Ly, L, left = shape.chunk, shape.d_model, shape.layers, shape.window, shape.left
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    qkv = [torch.zeros(slots, T, 3 * D, dtype=shape.dtype, device=cuda) for _ in range(Ly)]
    pos, _, _ = synth.relpos_inputs(shape, cuda, seed=seed)
    bu = [(torch.randn(shape.heads, shape.head_dim, generator=g) * 0.02).to(shape.dtype).to(cuda) for _ in range(Ly)]
    bv = [(torch.randn(shape.heads, shape.head_dim, generator=g) * 0.02).to(shape.dtype).to(cuda) for _ in range(Ly)]
    M = (L + shape.page_size - 2) // shape.page_size + 1
    order = rng.permutation(slots * M)
    st = AttentionStep(shape, slots, cuda, qkv, pos, bu, bv, page_order=order, rows_per_lane=rows_per_lane)
    # poison: a read of a never-written page row shows up as NaN
    st.k_pages.fill_(float("nan"))
    st.v_pages.fill_(float("nan"))

    win_k = np.zeros((slots, Ly, L, D))
    win_v = np.zeros((slots, Ly, L, D))
    proc = np.zeros(slots, dtype=np.int64)
    cl = np.zeros(slots, dtype=np.int64)
    pos64 = pos.double().cpu().numpy()
    worst = 0.0
    for step in range(steps):
        if step and step % 7 == 0:
            gone = rng.choice(slots, size=2, replace=False)
            st.reset_slots(gone)
            for s in gone:  # scheduler.py:86-91 zeroes a slot
                win_k[s] = 0
                win_v[s] = 0
                proc[s] = 0
                cl[s] = 0
        batch = rng.permutation(slots)[: max(1, slots - step % 3)]
        B = len(batch)
        frames = []
        for layer in range(Ly):
            x = torch.randn(B, T, 3 * D, generator=g).to(shape.dtype)
            qkv[layer][:B].copy_(x.to(cuda))
            frames.append(x.double().numpy())
        st.step(batch, graph=graph)
        _, mask = om.create_streaming_masks(T, cl[batch], proc[batch], T, (left, shape.right))
        for layer in range(Ly):
            q, k, v = np.split(frames[layer], 3, axis=-1)
            for b, s in enumerate(batch):  # cache.py:36-45 per slot
                for win, new in ((win_k, k[b]), (win_v, v[b])):
                    win[s, layer, :left] = win[s, layer, -left:].copy()
                    win[s, layer, left:] = new
            ref = oa.relpos_attention(
                q, win_k[batch, layer], win_v[batch, layer], pos64,
                bu[layer].double().cpu().numpy(), bv[layer].double().cpu().numpy(), mask, shape.heads,
            )
            got = st.out[layer][:B].double().cpu().numpy()
            err = float(np.abs(got - ref).max())
            worst = max(worst, err)
            assert err <= TOL[shape.dtype], f"step {step} layer {layer}: max abs err {err:.3e}"
            pages = ops.PagedKV(st.k_pages, st.v_pages, st.rows[:B], st.pool.max_pages)
            gk, gv = ops.kv_gather(pages, layer, B, L, T)
            ek = torch.from_numpy(win_k[batch, layer]).to(shape.dtype)
            ev = torch.from_numpy(win_v[batch, layer]).to(shape.dtype)
            assert torch.equal(gk.cpu(), ek) and torch.equal(gv.cpu(), ev), f"step {step} layer {layer}: pages"
        proc[batch] += T  # encoder.py:257-260
        cl[batch] = np.minimum(cl[batch] + T, left)
    torch.cuda.synchronize()
    print(f"  worst max-abs error {worst:.3e}", flush=True)


SMALL = synth.Shape("small-3layer-fp16", 3, 512, 8, dtype=torch.float16)
LARGE = synth.Shape("large-3layer-bf16", 3, 1024, 8, dtype=torch.bfloat16)
SMALL32 = synth.Shape("small-2layer-fp32", 2, 512, 8, dtype=torch.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [SMALL, LARGE, SMALL32], ids=lambda s: s.name)
def test_step_churn_matches_oracle(cuda, shape):
    _run(cuda, shape, slots=6, steps=45, seed=5)


@pytest.mark.gpu
def test_step_vector_kernel_path(cuda):
    """rows_per_lane forces the vector-ALU kernel for 16-bit types too."""
    _run(cuda, SMALL, slots=5, steps=30, seed=6, rows_per_lane=9)


@pytest.mark.gpu
def test_step_t14_chunks(cuda):
    """The real large model's att_context_size (70, 13): 14-frame chunks that
    straddle pages and several query groups per stream."""
    shape = synth.Shape("large-t14-bf16", 2, 1024, 8, right=13, dtype=torch.bfloat16)
    _run(cuda, shape, slots=4, steps=14, seed=7)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [SMALL, LARGE], ids=lambda s: s.name)
def test_step_graph_replays_match_oracle(cuda, shape):
    """All layers recorded once in a HIP graph and replayed every step for
    batches of changing size (the live count is read on the device); between
    replays the test's own eager work runs (uploads, gathers, copies back,
    synchronizations) and every replay is checked against the oracle."""
    _run(cuda, shape, slots=6, steps=30, seed=8, graph=True)
