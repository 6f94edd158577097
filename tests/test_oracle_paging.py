"""Pins oracle/dense_cache.py and oracle/paging.py.

* the dense shift buffer (cache.py:36-45) holds exactly the closed-form window
  (frame appended-L+j at row j, zeros before position 0) after every update;
* the page model's append + gather reproduces that window bit-for-bit over many
  steps with eviction, on identity and shuffled pools, with slot resets;
* the FIFO discipline: pages leave the queue in initial order followed by
  the order they were freed; no page is held twice; pages are conserved.
"""

import numpy as np
import pytest

from oracle import dense_cache, paging


def test_dense_cache_closed_form():
    rng = np.random.default_rng(0)
    left, right, D, B = 7, 1, 4, 3
    T = right + 1
    dc = dense_cache.DenseCache(1, left, right, D, B)
    hist = [np.zeros((0, D), np.float32) for _ in range(B)]
    for step in range(20):
        k = rng.standard_normal((B, T, D)).astype(np.float32)
        win, _ = dc.update_attn_cache(0, k, k)
        for b in range(B):
            hist[b] = np.concatenate([hist[b], k[b]])
            np.testing.assert_array_equal(win[b], dense_cache.window_closed_form(hist[b], (step + 1) * T, left + T))


def _run_paged_vs_dense(left, right, P, B, steps, order=None, resets=(), seed=0, layers=2):
    rng = np.random.default_rng(seed)
    T = right + 1
    D = 8
    M = paging.max_pages(left, T, P)
    num_pages = B * M
    pool = paging.PagePoolModel(num_pages, B, P, left, T, order)
    kp = np.full((layers, num_pages, P, D), np.nan, np.float32)  # poison: never-written pages
    vp = kp.copy()
    dc = dense_cache.DenseCache(layers, left, right, D, B)
    for step in range(steps):
        for s in resets_at(resets, step):
            pool.reset_slot(s)
            dc.reset_slot(s)
        rows = pool.advance(range(B))
        held = [p for b in range(B) for p in rows[b, 1:] if p >= 0]
        assert len(held) == len(set(held)), "a page is held twice"
        assert len(held) + len(pool.free) == num_pages, "pages not conserved"
        for layer in range(layers):
            k = rng.standard_normal((B, T, D)).astype(np.float32)
            v = rng.standard_normal((B, T, D)).astype(np.float32)
            dk, dv = dc.update_attn_cache(layer, k, v)
            paging.append(kp, vp, rows, layer, k, v, P, M)
            gk, gv = paging.gather(kp, vp, rows, layer, left + T, T, P, M)
            np.testing.assert_array_equal(gk, dk)
            np.testing.assert_array_equal(gv, dv)


def resets_at(resets, step):
    return [s for (st, s) in resets if st == step]


@pytest.mark.parametrize("left,right,P", [(70, 1, 16), (70, 13, 16), (5, 0, 4), (9, 2, 2), (3, 4, 8), (70, 1, 64)])
def test_paged_window_equals_dense(left, right, P):
    _run_paged_vs_dense(left, right, P, B=3, steps=60)


def test_paged_window_shuffled_pool_with_resets():
    left, right, P, B = 70, 1, 16, 4
    M = paging.max_pages(left, right + 1, P)
    order = np.random.default_rng(5).permutation(B * M)
    _run_paged_vs_dense(left, right, P, B, steps=80, order=order, resets=[(10, 1), (45, 3), (46, 1)], seed=3)


def _alloc_free_sequences(pool, schedule):
    """Runs the schedule (lists of slots, one list per step) and records, from
    the rings alone, the order in which pages were taken (new ring entries) and
    released (dropped ring entries); slots in call order, evictions before
    allocations, logical page order within each."""
    allocs, frees = [], []
    for slots in schedule:
        before = {s: (pool.lo[s], pool.hi[s], list(pool.ring[s])) for s in slots}
        pool.advance(slots)
        for s in slots:
            lo0, hi0, ring0 = before[s]
            frees.extend(ring0[k % pool.M] for k in range(lo0, min(pool.lo[s], hi0)))
            allocs.extend(pool.ring[s][k % pool.M] for k in range(max(hi0, pool.lo[s]), pool.hi[s]))
    return allocs, frees


def test_fifo_order():
    # allocations come out in initial order, then in the order pages were freed
    rng = np.random.default_rng(1)
    order = [int(x) for x in rng.permutation(2 * 3 + 4)]
    pool = paging.PagePoolModel(len(order), 2, 2, 3, 1, page_order=order)
    initial = list(order)
    schedule = [[0, 1]] * 5 + [[1]] * 4 + [[0]] * 9 + [[0, 1]] * 6
    allocs, frees = _alloc_free_sequences(pool, schedule)
    assert len(allocs) > len(initial)  # pages were recycled
    assert allocs == (initial + frees)[: len(allocs)]


def test_fifo_exact_trace():
    # window 4 frames (left 3, chunk 1), page size 2 -> max_pages 3
    pool = paging.PagePoolModel(6, 2, 2, 3, 1)
    assert pool.M == 3
    got = [pool.advance([0]).tolist()[0] for _ in range(7)]
    # A: 0..6; pages allocated at A=0 (p0), A=2 (p1), A=4 (p2), A=6 (p3);
    # page for positions 0-1 evicted when the window start (A+1-4) reaches 2 (A=5)
    assert [r[0] for r in got] == list(range(7))
    assert got[0][1:] == [0, -1, -1]
    assert got[2][1:] == [0, 1, -1]
    assert got[4][1:] == [0, 1, 2]
    assert got[5][1:] == [-1, 1, 2]
    assert got[6][1:] == [3, 1, 2]
    assert list(pool.free_list()) == [4, 5, 0]


def test_reset_returns_pages():
    pool = paging.PagePoolModel(12, 2, 4, 5, 2)
    for _ in range(4):
        pool.advance([0, 1])
    lo, hi = pool.lo[1], pool.hi[1]
    held_in_order = [pool.ring[1][k % pool.M] for k in range(lo, hi)]
    before = list(pool.free_list())
    pool.reset_slot(1)
    assert list(pool.free_list()) == before + held_in_order
    assert pool.slot_info(1)[0] == 0
    assert all(p == -1 for p in pool.ring[1])


def test_pool_too_small_rejected():
    with pytest.raises(ValueError):
        paging.PagePoolModel(5, 1, 16, 70, 2)
