"""The C++ host page pool (pk_pool_*) against the Python model in
oracle/paging.py: identical rows, rings, A counters and free-queue order after
every step of random churn (stream arrivals, departures with reset, partial
batches), identity and shuffled initial orders.  Also error paths and a
multi-thread smoke test.  Host code only: runs without a GPU."""

import threading

import numpy as np
import pytest

from oracle import paging
from parakeet_amd.pool import PagePool, pages_per_slot


def _compare(native, model, num_slots):
    np.testing.assert_array_equal(native.free_list(), model.free_list())
    for s in range(num_slots):
        a_n, ring_n = native.slot_info(s)
        a_m, ring_m = model.slot_info(s)
        assert a_n == a_m
        np.testing.assert_array_equal(ring_n, ring_m)


@pytest.mark.parametrize(
    "left,chunk,P,slots,shuffle",
    [(70, 2, 16, 8, False), (70, 2, 16, 16, True), (70, 14, 16, 6, True), (5, 1, 4, 5, False), (9, 3, 2, 7, True), (0, 2, 4, 3, False)],
)
def test_native_pool_matches_model_under_churn(left, chunk, P, slots, shuffle):
    rng = np.random.default_rng(left * 7 + chunk + P + slots)
    M = pages_per_slot(left, chunk, P)
    assert M == paging.max_pages(left, chunk, P)
    num_pages = slots * M + int(rng.integers(0, 5))
    order = rng.permutation(num_pages) if shuffle else None
    native = PagePool(slots, P, left, chunk, num_pages=num_pages, page_order=order)
    model = paging.PagePoolModel(num_pages, slots, P, left, chunk, order)
    active = []
    free_slots = list(range(slots))
    for step in range(400):
        # departures
        for s in list(active):
            if rng.random() < 0.03:
                active.remove(s)
                native.reset_slot(s)
                model.reset_slot(s)
                free_slots.append(s)
        # arrivals
        while free_slots and rng.random() < 0.3:
            active.append(free_slots.pop(0))
        if not active:
            continue
        batch = [s for s in active if rng.random() < 0.9]
        rng.shuffle(batch)
        rows_n = native.advance(np.array(batch, dtype=np.int32))
        rows_m = model.advance(batch)
        np.testing.assert_array_equal(rows_n, rows_m)
        if step % 37 == 0:
            _compare(native, model, slots)
    _compare(native, model, slots)
    native.reset_all()
    model.reset_all()
    _compare(native, model, slots)
    assert native.free_pages() == num_pages


def test_slot_twice_in_one_step_rejected():
    pool = PagePool(4, 16, 70, 2)
    with pytest.raises(RuntimeError, match="twice"):
        pool.advance(np.array([1, 2, 1], dtype=np.int32))
    # nothing changed
    assert pool.slot_info(1)[0] == 0 and pool.slot_info(2)[0] == 0


def test_bad_arguments_rejected():
    with pytest.raises(RuntimeError, match="power of two"):
        PagePool(2, 12, 70, 2)
    with pytest.raises(RuntimeError, match="cannot hold"):
        PagePool(2, 16, 70, 2, num_pages=11)
    with pytest.raises(RuntimeError, match="permutation"):
        PagePool(1, 16, 70, 2, num_pages=6, page_order=[0, 1, 2, 3, 4, 4])
    pool = PagePool(2, 16, 70, 2)
    with pytest.raises(RuntimeError, match="out of range"):
        pool.advance(np.array([2], dtype=np.int32))
    with pytest.raises(RuntimeError, match="out of range"):
        pool.reset_slot(-1)


def test_threads_share_the_pool():
    # admission/release threads reset slots while the "encode" thread advances
    slots = 32
    pool = PagePool(slots, 16, 70, 2)
    errors = []

    def encode():
        try:
            for _ in range(300):
                pool.advance(np.arange(0, slots // 2, dtype=np.int32))
        except Exception as e:  # pragma: no cover
            errors.append(e)

    def churn():
        try:
            for i in range(300):
                pool.reset_slot(slots // 2 + i % (slots // 2))
        except Exception as e:  # pragma: no cover
            errors.append(e)

    ts = [threading.Thread(target=encode), threading.Thread(target=churn)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    held = sum(int(np.sum(pool.slot_info(s)[1] >= 0)) for s in range(slots))
    assert held + pool.free_pages() == pool.num_pages
