"""The convolution-module oracle (oracle/conv.py) pinned on the CPU:
* against the reference's own operator composition (convolution.py:150-158:
  channel-major F.glu, masked_fill, cat with the [B, D, K-1] cache, grouped
  F.conv1d, LayerNorm, SiLU) in float64 torch;
* by the streaming invariant that defines the cache: a sequence fed chunk by
  chunk through the cache gives the same frames and the same final cache as the
  whole sequence in one step from a zero cache (cache.py:30-34 zero state);
* by a planted mistake (taps reversed) that both checks catch."""

import numpy as np
import pytest
import torch

from oracle import conv as oc


def _inputs(B, T, D, K, seed, bias=True):
    g = np.random.default_rng(seed)
    h = g.standard_normal((B, T, 2 * D))
    cache = g.standard_normal((B, K - 1, D))
    w = g.standard_normal((D, K)) / np.sqrt(K)
    b = g.standard_normal(D) * 0.1 if bias else None
    lw = 1.0 + 0.1 * g.standard_normal(D)
    lb = 0.1 * g.standard_normal(D)
    pad = g.random((B, T)) < 0.25
    return h, cache, w, b, lw, lb, pad


def _torch(h, cache, pad, w, b, lw, lb):
    t = lambda a: None if a is None else torch.from_numpy(np.asarray(a, dtype=np.float64))  # noqa: E731
    y, nxt = oc.conv_module_step_torch(
        t(h), t(cache).transpose(1, 2), None if pad is None else torch.from_numpy(pad), t(w), t(b), t(lw), t(lb)
    )
    return y.numpy(), nxt.transpose(1, 2).numpy()


@pytest.mark.parametrize("B,T,D,K", [(3, 2, 16, 9), (2, 14, 8, 9), (2, 1, 12, 3), (1, 5, 24, 5)])
@pytest.mark.parametrize("bias", [True, False])
def test_oracle_matches_reference_operator_order(B, T, D, K, bias):
    h, cache, w, b, lw, lb, pad = _inputs(B, T, D, K, seed=B * 100 + T, bias=bias)
    y, nxt = oc.conv_module_step(h, cache, pad, w, b, lw, lb)
    ry, rn = _torch(h, cache, pad, w, b, lw, lb)
    np.testing.assert_allclose(y, ry, rtol=0, atol=1e-12)
    np.testing.assert_allclose(nxt, rn, rtol=0, atol=1e-15)  # GLU frames: float64 rounding of sigmoid


def test_chunked_stream_equals_one_shot():
    B, D, K, steps, T = 2, 16, 9, 7, 2
    h, _, w, b, lw, lb, _ = _inputs(B, steps * T, D, K, seed=5)
    y_all, cache_all = oc.conv_module_step(h, np.zeros((B, K - 1, D)), None, w, b, lw, lb)
    cache = np.zeros((B, K - 1, D))
    ys = []
    for s in range(steps):
        y, cache = oc.conv_module_step(h[:, s * T : (s + 1) * T], cache, None, w, b, lw, lb)
        ys.append(y)
    np.testing.assert_allclose(np.concatenate(ys, axis=1), y_all, rtol=0, atol=1e-12)
    np.testing.assert_array_equal(cache, cache_all)


def test_cache_rows_are_the_last_frames():
    B, T, D, K = 2, 3, 8, 9
    h, cache, w, b, lw, lb, _ = _inputs(B, T, D, K, seed=11)
    _, nxt = oc.conv_module_step(h, cache, None, w, b, lw, lb)
    np.testing.assert_array_equal(nxt[:, : K - 1 - T], cache[:, T:])  # shifted, untouched
    np.testing.assert_array_equal(nxt[:, K - 1 - T :], oc.glu(h))  # this step's GLU frames
    # a chunk longer than the cache keeps only its own last K-1 frames
    h2 = np.random.default_rng(3).standard_normal((B, 12, 2 * D))
    _, nxt2 = oc.conv_module_step(h2, cache, None, w, b, lw, lb)
    np.testing.assert_array_equal(nxt2, oc.glu(h2)[:, -(K - 1) :])


def test_store_dtype_rounds_the_cached_frames():
    B, T, D, K = 1, 2, 8, 9
    h, cache, w, b, lw, lb, _ = _inputs(B, T, D, K, seed=2)
    cache = oc.round_to(cache, torch.float16)
    _, nxt = oc.conv_module_step(h, cache, None, w, b, lw, lb, store_dtype=torch.float16)
    assert np.array_equal(oc.round_to(nxt, torch.float16), nxt)


def test_planted_reversed_taps_is_caught():
    B, T, D, K = 2, 2, 16, 9
    h, cache, w, b, lw, lb, pad = _inputs(B, T, D, K, seed=7)
    ry, _ = _torch(h, cache, pad, w, b, lw, lb)
    bad, _ = oc.conv_module_step(h, cache, pad, w[:, ::-1], b, lw, lb)
    assert np.abs(bad - ry).max() > 1e-3
