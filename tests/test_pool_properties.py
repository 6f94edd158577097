"""Property tests of the C++ host page pool (pk_pool_*), driven by hypothesis:
random pool shapes (left context, chunk, page size, slots, spare pages, initial
order) and random operation sequences (steps over random slot subsets in random
order, slot resets, full resets, rejected steps).

Checked after every operation:
* the native pool equals the Python FIFO model of oracle/paging.py (rows, rings,
  A counters, free-queue order) -- the deque discipline of
  parakeet/engine/scheduler.py:84,97,104 applied to pages;
* invariants that hold whatever the model says:
  - conservation: every page is either free or held by exactly one slot;
  - a stream holds exactly the pages its window [A - (left + chunk), A) spans
    (eviction as soon as a page leaves the window, cache.py:37-42), and every
    position of that window maps to a held page;
  - a step returns the stream's A before the step and advances it by the chunk;
  - a reset slot holds nothing, and its pages went to the back of the queue;
  - a step naming a slot twice is rejected and changes nothing.
Host code only: runs without a GPU."""

import numpy as np
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import paging
from parakeet_amd.pool import PagePool, pages_per_slot


@st.composite
def pool_config(draw):
    left = draw(st.integers(0, 80))
    chunk = draw(st.integers(1, 16))
    P = draw(st.sampled_from([1, 2, 4, 8, 16, 32]))
    slots = draw(st.integers(1, 8))
    spare = draw(st.integers(0, 4))
    M = pages_per_slot(left, chunk, P)
    num_pages = slots * M + spare
    order = draw(st.permutations(list(range(num_pages)))) if draw(st.booleans()) else None
    return left, chunk, P, slots, num_pages, order


def op_strategy(slots):
    step = st.tuples(st.just("step"), st.lists(st.integers(0, slots - 1), unique=True, min_size=1, max_size=slots), st.randoms())
    reset = st.tuples(st.just("reset"), st.integers(0, slots - 1), st.none())
    dup = st.tuples(st.just("dup"), st.integers(0, slots - 1), st.none())
    return st.one_of(step, step, step, reset, dup, st.tuples(st.just("reset_all"), st.none(), st.none()))


def _held(pool, slots):
    rings = {}
    for s in range(slots):
        a, ring = pool.slot_info(s)
        rings[s] = (a, [int(x) for x in ring])
    return rings


def _check_invariants(native, num_pages, slots, left, chunk, P):
    M = native.max_pages
    window = left + chunk
    free = [int(x) for x in native.free_list()]
    held = _held(native, slots)
    owned = [pg for s in range(slots) for pg in held[s][1] if pg >= 0]
    assert sorted(free + owned) == list(range(num_pages)), "a page is lost or held twice"
    for s in range(slots):
        a, ring = held[s]
        n_held = sum(1 for pg in ring if pg >= 0)
        if a == 0:
            assert n_held == 0
            continue
        start = max(0, a - window)
        lo, hi = start // P, (a - 1) // P + 1
        assert n_held == hi - lo, f"slot {s}: holds {n_held} pages, window spans {hi - lo}"
        assert hi - lo <= M
        for pos in range(start, a):
            assert ring[(pos // P) % M] >= 0, f"slot {s}: window position {pos} has no page"


@settings(max_examples=120, deadline=None, suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])
@given(data=st.data(), cfg=pool_config())
def test_pool_properties_under_random_operations(data, cfg):
    left, chunk, P, slots, num_pages, order = cfg
    native = PagePool(slots, P, left, chunk, num_pages=num_pages, page_order=order)
    model = paging.PagePoolModel(num_pages, slots, P, left, chunk, order)
    assert native.max_pages == model.M
    ops = data.draw(st.lists(op_strategy(slots), min_size=1, max_size=60))
    for kind, arg, rnd in ops:
        if kind == "step":
            batch = list(arg)
            rnd.shuffle(batch)
            before = {s: native.slot_info(s)[0] for s in batch}
            rows_n = native.advance(np.array(batch, dtype=np.int32))
            rows_m = model.advance(batch)
            np.testing.assert_array_equal(rows_n, rows_m)
            for b, s in enumerate(batch):
                assert rows_n[b, 0] == before[s]
                assert native.slot_info(s)[0] == before[s] + chunk
        elif kind == "reset":
            a, ring = native.slot_info(arg)
            lo = (max(0, a - left - chunk) // P) if a else 0
            hi = ((a - 1) // P + 1) if a else 0
            expect_tail = [int(ring[k % native.max_pages]) for k in range(lo, hi)]
            native.reset_slot(arg)
            model.reset_slot(arg)
            free = [int(x) for x in native.free_list()]
            if expect_tail:
                assert free[-len(expect_tail):] == expect_tail
            a2, ring2 = native.slot_info(arg)
            assert a2 == 0 and (ring2 < 0).all()
        elif kind == "dup":
            snapshot = (native.free_list().copy(), _held(native, slots))
            try:
                native.advance(np.array([arg, arg], dtype=np.int32))
            except RuntimeError as e:
                assert "twice" in str(e)
            else:
                raise AssertionError("a step naming a slot twice was accepted")
            np.testing.assert_array_equal(native.free_list(), snapshot[0])
            assert _held(native, slots) == snapshot[1]
        else:
            native.reset_all()
            model.reset_all()
            assert native.free_pages() == num_pages
        np.testing.assert_array_equal(native.free_list(), model.free_list())
        for s in range(slots):
            a_n, ring_n = native.slot_info(s)
            a_m, ring_m = model.slot_info(s)
            assert a_n == a_m
            np.testing.assert_array_equal(ring_n, ring_m)
        _check_invariants(native, num_pages, slots, left, chunk, P)
    native.close()


def test_invariant_check_catches_a_planted_leak():
    """The invariant check itself fails on a pool state that lost a page (the
    mistake planted in the model, on the CPU)."""
    model = paging.PagePoolModel(12, 2, 4, 5, 2, None)
    model.advance([0, 1])
    model.free.popleft()  # a page vanishes from the queue

    class View:
        max_pages = model.M

        def free_list(self):
            return model.free_list()

        def slot_info(self, s):
            return model.slot_info(s)

    try:
        _check_invariants(View(), 12, 2, 5, 2, 4)
    except AssertionError:
        return
    raise AssertionError("the invariant check missed a lost page")
