"""Pins oracle/masks.py: the loop restatement of _create_streaming_masks
(encoder.py:167-227) against an independent per-position statement over grids
of (proc, cache_len, length, chunk, left), against the engine-regime closed
form, and against the torch restatement used by the CPU baseline."""

import itertools

import numpy as np
import pytest
import torch

from oracle import dense_path, masks


def _grid(left, right, T):
    C = right + 1
    cases = []
    for proc in range(0, 3 * (left + T) + 1):
        for cl in sorted({0, min(proc, left), min(proc, left) // 2, max(min(proc, left) - 1, 0)}):
            if cl > proc or cl > left:
                continue
            for n in range(0, T + 1):
                cases.append((proc, cl, n))
    del C
    return cases


@pytest.mark.parametrize("left,right,T", [(70, 1, 2), (6, 1, 2), (7, 2, 3), (5, 0, 1), (9, 3, 4), (70, 13, 14), (4, 1, 3)])
def test_loop_equals_position_rule(left, right, T):
    cases = _grid(left, right, T)
    proc = np.array([c[0] for c in cases])
    cl = np.array([c[1] for c in cases])
    n = np.array([c[2] for c in cases])
    pad_a, att_a = masks.create_streaming_masks(T, cl, proc, n, (left, right))
    pad_b, att_b = masks.masks_by_position(T, cl, proc, n, (left, right))
    np.testing.assert_array_equal(pad_a, pad_b)
    np.testing.assert_array_equal(att_a, att_b)


@pytest.mark.parametrize("left,right", [(70, 1), (70, 13), (8, 1)])
def test_engine_regime_closed_form(left, right):
    # engine: length == T == right + 1, proc a multiple of T, cache_len = min(proc, left)
    T = right + 1
    for step in range(0, 3 * left // T + 3):
        proc = step * T
        cl = min(proc, left)
        _, att = masks.create_streaming_masks(T, [cl], [proc], [T], (left, right))
        j = np.arange(left + T)
        expected = np.broadcast_to(j < left - cl, (T, left + T))
        if left % T == 0:
            np.testing.assert_array_equal(att[0], expected)
        else:
            # the chunk rule can also hide the oldest cached frames
            assert np.all(att[0][expected])


def test_torch_restatement_matches():
    left, right, T = 10, 1, 2
    cases = _grid(left, right, T)
    proc = torch.tensor([c[0] for c in cases])
    cl = torch.tensor([c[1] for c in cases])
    n = torch.tensor([c[2] for c in cases])
    pad_t, att_t = dense_path.streaming_masks_torch(T, cl, proc, n, (left, right))
    pad_n, att_n = masks.create_streaming_masks(T, cl.numpy(), proc.numpy(), n.numpy(), (left, right))
    np.testing.assert_array_equal(pad_t.numpy(), pad_n)
    np.testing.assert_array_equal(att_t.numpy(), att_n)


def test_scalar_length_broadcasts():
    left, right, T = 6, 1, 2
    for proc, cl in itertools.product(range(0, 12), range(0, 7)):
        if cl > proc:
            continue
        a = masks.create_streaming_masks(T, [cl, cl], [proc, proc], 1, (left, right))
        b = masks.create_streaming_masks(T, [cl, cl], [proc, proc], [1, 1], (left, right))
        np.testing.assert_array_equal(a[1], b[1])
