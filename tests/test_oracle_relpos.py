"""Pins oracle/relpos.py: sinusoid table against per-element math.sin/cos, the
position slice against its row->position rule, and rel_shift against the
closed-form index shifted[i, j] = x[i, j + T - 1 - i] (brute force)."""

import math

import numpy as np
import pytest

from oracle import relpos


@pytest.mark.parametrize("length,d_model", [(5, 8), (80, 512), (143, 1024)])
def test_sinusoid_table_closed_form(length, d_model):
    pe = relpos.sinusoid_table(length, d_model)
    assert pe.shape == (2 * length - 1, d_model)
    rng = np.random.default_rng(0)
    rows = rng.integers(0, pe.shape[0], size=40)
    cols = rng.integers(0, d_model // 2, size=40)
    for r, k in zip(rows, cols):
        pos = (length - 1) - r
        w = math.exp(2 * k * -(math.log(10000.0) / d_model))
        # the reference forms w and pos*w in fp32: the angle carries a relative
        # error of a few fp32 ulps, so the bound grows with |angle|
        ang = pos * w
        tol = 1e-6 + 3e-7 * abs(ang)
        assert abs(pe[r, 2 * k] - math.sin(ang)) <= tol
        assert abs(pe[r, 2 * k + 1] - math.cos(ang)) <= tol
    # position 0 row: sin = 0, cos = 1
    zero_row = length - 1
    assert np.all(pe[zero_row, 0::2] == 0.0) and np.all(pe[zero_row, 1::2] == 1.0)


def test_sinusoid_table_matches_torch():
    torch = pytest.importorskip("torch")
    length, d = 50, 64
    positions = torch.arange(length - 1, -length, -1, dtype=torch.float32).unsqueeze(1)
    div = torch.exp(torch.arange(0, d, 2, dtype=torch.float32) * -(math.log(10000.0) / d))
    ref = torch.zeros(2 * length - 1, d)
    ref[:, 0::2] = torch.sin(positions * div)
    ref[:, 1::2] = torch.cos(positions * div)
    np.testing.assert_allclose(relpos.sinusoid_table(length, d), ref.numpy(), atol=3e-6, rtol=0)


@pytest.mark.parametrize("T,cache_len", [(2, 70), (14, 70), (1, 0), (3, 5)])
def test_pos_slice_rows(T, cache_len):
    length = 200
    pe = relpos.sinusoid_table(length, 16, dtype=np.float64)
    sl = relpos.pos_slice(pe, T, cache_len)
    L = T + cache_len
    assert sl.shape[0] == 2 * L - 1
    # row r holds relative position (L - 1) - r
    for r in range(sl.shape[0]):
        pos = (L - 1) - r
        np.testing.assert_array_equal(sl[r], pe[(length - 1) - pos])


@pytest.mark.parametrize("T,L", [(2, 72), (14, 84), (3, 8), (1, 5), (4, 4)])
def test_rel_shift_closed_form(T, L):
    rng = np.random.default_rng(T * 100 + L)
    P = 2 * L - 1
    x = rng.standard_normal((2, 3, T, P))
    y = relpos.rel_shift(x)[:, :, :, :L]
    for i in range(T):
        for j in range(L):
            np.testing.assert_array_equal(y[:, :, i, j], x[:, :, i, j + T - 1 - i])


def test_rel_shift_relative_position():
    # with the sinusoid slice, column j of query i sees relative position left + i - j
    left, T = 70, 2
    L = left + T
    rng = np.random.default_rng(1)
    rel_of_row = (L - 1) - np.arange(2 * L - 1)
    x = np.broadcast_to(rel_of_row.astype(np.float64), (1, 1, T, 2 * L - 1)).copy()
    y = relpos.rel_shift(x)[0, 0, :, :L]
    for i in range(T):
        for j in range(L):
            assert y[i, j] == left + i - j
    del rng


def test_rel_shift_catches_wrong_index():
    # a plausible mistake (dropping the T - 1 offset) must be caught by the closed form
    rng = np.random.default_rng(2)
    T, L = 3, 6
    x = rng.standard_normal((1, 1, T, 2 * L - 1))
    y = relpos.rel_shift(x)[0, 0, :, :L]
    wrong = np.array([[x[0, 0, i, j - i] if j - i >= 0 else 0.0 for j in range(L)] for i in range(T)])
    assert not np.allclose(y, wrong)
