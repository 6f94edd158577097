"""The drop-in Scheduler (parakeet/engine/scheduler.py:20-201) on a paged state
pool, host side only (the pool tensors live on the CPU here; no kernel runs):

* slots come from a FIFO deque: acquire pops the front, release appends at the
  back, an empty pool gives None (scheduler.py:84,92-104);
* acquire and release zero the slot's state scalars and return its pages to
  the page pool (scheduler.py:86-91 zeroes the dense slot);
* pack_states gathers the state scalars of the batch's slots in batch order
  and the batch cache view names those slots (scheduler.py:128-170 gathers
  the dense state); unpack_states scatters the scalars back (:172-201);
* admission keeps at most max_active sequences running and skips finished
  ones (scheduler.py:20-60).
"""

from enum import Enum, auto

import numpy as np
import pytest
import torch

from parakeet_amd.engine.scheduler import Scheduler
from parakeet_amd.modules.encoder import ConformerEncoder


class Status(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Seq:
    def __init__(self, slot=None):
        self.status = Status.WAITING
        self.encoder_state = slot


def _encoder(left=9, right=1, layers=2, d=64):
    return ConformerEncoder(
        feat_in=80, hidden_size=d, ff_expansion_factor=2, num_layers=layers, num_heads=2,
        subsampling_factor=8, pos_emb_max_len=64, conv_kernel_size=9, att_context_size=[left, right],
        subsampling_conv_channels=32, use_bias=False, page_size=4,
    )


def _scheduler(pool_size=4):
    sch = Scheduler(max_active=3)
    sch.init_state_pool(_encoder(), torch.device("cpu"), torch.float32, pool_size)
    return sch


def test_slots_fifo_and_exhaustion():
    sch = _scheduler(4)
    assert [sch.acquire_state_slot() for _ in range(4)] == [0, 1, 2, 3]
    assert sch.acquire_state_slot() is None
    sch.release_state_slot(2)
    sch.release_state_slot(0)
    assert sch.acquire_state_slot() == 2
    assert sch.acquire_state_slot() == 0
    assert sch.acquire_state_slot() is None


def test_release_zeroes_state_and_returns_pages():
    sch = _scheduler(3)
    pool = sch.pool_state
    cache = pool.cache
    free0 = cache.pool.free_pages()
    slots = [sch.acquire_state_slot() for _ in range(3)]
    # advance every stream a few steps: pages are taken from the pool
    for _ in range(5):
        view = cache.batch(slots)
        view._open_step()
    pool.processed_frames[:] = torch.tensor([10, 20, 30])
    pool.cache_lengths[:] = torch.tensor([9, 9, 9])
    assert cache.pool.free_pages() < free0
    held = free0 - cache.pool.free_pages()
    sch.release_state_slot(1)
    assert int(pool.processed_frames[1]) == 0 and int(pool.cache_lengths[1]) == 0
    assert cache.pool.free_pages() == free0 - held + held // 3
    appended, ring = cache.pool.slot_info(1)
    assert appended == 0 and (ring == -1).all()


def test_pack_unpack_scalars_in_batch_order():
    sch = _scheduler(5)
    for _ in range(5):
        sch.acquire_state_slot()
    pool = sch.pool_state
    pool.processed_frames[:] = torch.arange(5) * 10
    pool.cache_lengths[:] = torch.arange(5)
    seqs = [Seq(3), Seq(0), Seq(4)]
    state, index = sch.pack_states(seqs)
    assert index.tolist() == [3, 0, 4]
    assert state.processed_frames.tolist() == [30, 0, 40]
    assert state.cache_lengths.tolist() == [3, 0, 4]
    np.testing.assert_array_equal(state.cache.slots, [3, 0, 4])
    state.processed_frames += 2
    state.cache_lengths.fill_(7)
    sch.unpack_states(state, index)
    assert pool.processed_frames.tolist() == [2, 10, 20, 32, 42]
    assert pool.cache_lengths.tolist() == [7, 1, 2, 7, 7]


def test_pack_before_init_raises():
    with pytest.raises(RuntimeError, match="not initialized"):
        Scheduler().pack_states([Seq(0)])


def test_admission_limits_and_skips_finished():
    sch = Scheduler(max_active=2)
    a, b, c, d = Seq(), Seq(), Seq(), Seq()
    for s in (a, b, c, d):
        sch.add(s)
    assert list(sch.active_sequences()) == [a, b]
    assert c.status is Status.WAITING and d.status is Status.WAITING
    sch.release(a)
    c.status = Status.FINISHED
    assert sch.admit_ready() == [d]
    assert a.status is Status.FINISHED
    assert list(sch.active_sequences()) == [b, d]
