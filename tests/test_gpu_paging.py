"""GPU parity: page append + gather through the C-ABI reproduce the reference's
dense shift-buffer window (parakeet/modules/cache.py:36-45) bit-for-bit, step
after step with sliding-window eviction, on identity and shuffled pools, with
slot resets and partial batches, for fp32 / fp16 / bf16."""

import numpy as np
import pytest
import torch

from _scenario import PagedScenario
from parakeet_amd import ops

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _check_window(sc, layer, dk, dv):
    gk, gv = ops.kv_gather(sc.pages, layer, sc.rows.shape[0], sc.L, sc.T)
    ek = torch.from_numpy(np.ascontiguousarray(dk)).to(sc.dtype)
    ev = torch.from_numpy(np.ascontiguousarray(dv)).to(sc.dtype)
    assert torch.equal(gk.cpu(), ek), f"K window differs at layer {layer}"
    assert torch.equal(gv.cpu(), ev), f"V window differs at layer {layer}"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("left,right,P,steps", [(70, 1, 16, 50), (70, 13, 16, 12), (5, 0, 4, 20), (9, 2, 2, 15)])
def test_append_gather_bit_exact(cuda, dtype, left, right, P, steps):
    print(f"\n[append/gather] dtype={dtype} left={left} right={right} P={P}", flush=True)
    sc = PagedScenario(cuda, dtype, B=4, layers=2, d_model=64, left=left, right=right, page_size=P, seed=1)
    for step in range(steps):
        sc.open_step()
        for layer in range(sc.Ly):
            _, (q, k, v) = sc.frames()
            ops.kv_append(sc.pages, layer, k, v)
            dk, dv = sc.dense_update(layer, k, v)
            _check_window(sc, layer, dk, dv)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_shuffled_pool_churn_resets(cuda, dtype):
    print(f"\n[churn] dtype={dtype}", flush=True)
    sc = PagedScenario(cuda, dtype, B=6, layers=3, d_model=128, left=70, right=1, page_size=16, seed=2, shuffle=True)
    rng = np.random.default_rng(0)
    for step in range(90):
        if step in (20, 55):
            for s in rng.choice(sc.B, size=2, replace=False):
                sc.reset(int(s))
        sc.open_step()
        for layer in range(sc.Ly):
            _, (q, k, v) = sc.frames()
            ops.kv_append(sc.pages, layer, k, v)
            dk, dv = sc.dense_update(layer, k, v)
            _check_window(sc, layer, dk, dv)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_partial_batch_subset_rows(cuda):
    """A batch that names a subset of slots in another order touches only them."""
    dtype = torch.float16
    sc = PagedScenario(cuda, dtype, B=5, layers=1, d_model=64, left=20, right=1, page_size=8, seed=3)
    hist = {s: [] for s in range(sc.B)}
    order_rng = np.random.default_rng(1)
    for step in range(40):
        slots = [int(s) for s in order_rng.permutation(sc.B)[: 2 + step % 3]]
        sc.open_step(slots)
        x = torch.randn(len(slots), sc.T, sc.D, generator=sc.gen).to(dtype).to(cuda)
        ops.kv_append(sc.pages, 0, x, x)
        for b, s in enumerate(slots):
            hist[s].extend(x[b].cpu().float().numpy())
        gk, _ = ops.kv_gather(sc.pages, 0, len(slots), sc.L, sc.T)
        for b, s in enumerate(slots):
            H = np.array(hist[s], dtype=np.float32)
            want = np.zeros((sc.L, sc.D), np.float32)
            n = len(H)
            for j in range(sc.L):
                p = n - sc.L + j
                if p >= 0:
                    want[j] = H[p]
            assert torch.equal(gk[b].cpu(), torch.from_numpy(want).to(dtype))
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_empty_batch_is_noop(cuda):
    sc = PagedScenario(cuda, torch.float16, B=2, layers=1, d_model=64, left=6, right=1, page_size=4)
    sc.open_step([])
    x = torch.empty(0, sc.T, sc.D, dtype=torch.float16, device=cuda)
    ops.kv_append(sc.pages, 0, x, x)
    k, v = ops.kv_gather(sc.pages, 0, 0, sc.L, sc.T)
    assert k.shape == (0, sc.L, sc.D)
    torch.cuda.synchronize()


def _poison_free_pages(sc):
    """NaN into every page of the free queue: a read of a page after it was
    freed (a stale window row) shows up as NaN."""
    free = torch.from_numpy(sc.pool.free_list().astype(np.int64)).to(sc.k_pages.device)
    if free.numel():
        sc.k_pages[:, free] = float("nan")
        sc.v_pages[:, free] = float("nan")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_freed_pages_are_never_read(cuda, dtype):
    """Use-after-free check: after every step's eviction and allocation, every
    free page is filled with NaN.  The windows the pages give stay equal to the
    dense shift buffer (cache.py:36-45) and the fused append + attention reads no
    NaN, over churn with slot resets on a shuffled pool (pages are reused by
    other streams soon after they are freed)."""
    print(f"\n[poisoned free pages] dtype={dtype}", flush=True)
    sc = PagedScenario(cuda, dtype, B=6, layers=2, d_model=128, left=70, right=1, page_size=16, seed=3, shuffle=True)
    H, dk = 2, 64
    g = torch.Generator().manual_seed(1)
    pos = torch.randn(sc.L + sc.T - 1, sc.D, generator=g).to(dtype).to(cuda)
    bu = (torch.randn(H, dk, generator=g) * 0.02).to(dtype).to(cuda)
    bv = (torch.randn(H, dk, generator=g) * 0.02).to(dtype).to(cuda)
    rng = np.random.default_rng(5)
    for step in range(80):
        if step in (15, 40, 41, 60):
            for s in rng.choice(sc.B, size=2, replace=False):
                sc.reset(int(s))
        sc.open_step()
        _poison_free_pages(sc)
        for layer in range(sc.Ly):
            _, (q, k, v) = sc.frames()
            if layer == 0:
                ops.kv_append(sc.pages, layer, k, v)
            else:  # the fused append inside the attention launch
                out = ops.paged_relpos_attn(q, k, v, pos, bu, bv, None, num_heads=H, left=sc.left, pages=sc.pages,
                                            layer=layer, append=True)
                assert torch.isfinite(out.float()).all(), f"step {step}: attention read a freed page"
            dk_, dv_ = sc.dense_update(layer, k, v)
            _check_window(sc, layer, dk_, dv_)
    torch.cuda.synchronize()
