"""Pins oracle/attention.py.

* the reference-order form (pad/view rel_shift) equals the per-score form with
  the closed-form relative row index (float64, tiny inputs, with masks);
* with pos = 0, u = v = 0 and no mask it reduces to plain softmax attention,
  checked against torch's scaled_dot_product_attention (a library routine);
* the torch CPU fp32 operator path (the CPU baseline) matches the float64 form;
* invariants: constant value rows are reproduced; a fully masked row except one
  key returns that key's value; swapping u and v changes the result (both
  biases are wired in).
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import relpos


def _inputs(B, T, left, H, dk, seed, masked=True):
    rng = np.random.default_rng(seed)
    D = H * dk
    L = left + T
    q = rng.standard_normal((B, T, D))
    k = rng.standard_normal((B, L, D))
    v = rng.standard_normal((B, L, D))
    pos = rng.standard_normal((2 * L - 1, D)) * 0.5
    bu = rng.standard_normal((H, dk)) * 0.02
    bv = rng.standard_normal((H, dk)) * 0.02
    mask = rng.random((B, T, L)) < 0.3 if masked else None
    if mask is not None:
        mask[:, :, -1] = False  # keep a key per row
    return q, k, v, pos, bu, bv, mask


@pytest.mark.parametrize("B,T,left,H,dk", [(2, 2, 5, 2, 4), (1, 3, 4, 3, 2), (2, 1, 6, 1, 8), (1, 4, 0, 2, 4)])
@pytest.mark.parametrize("masked", [False, True])
def test_padview_equals_direct_index(B, T, left, H, dk, masked):
    q, k, v, pos, bu, bv, mask = _inputs(B, T, left, H, dk, seed=B + T + left, masked=masked)
    a = oa.relpos_attention(q, k, v, pos, bu, bv, mask, H)
    b = oa.relpos_attention_direct(q, k, v, pos, bu, bv, mask, H)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_reduces_to_sdpa_without_relpos():
    B, T, left, H, dk = 3, 2, 9, 4, 8
    q, k, v, pos, bu, bv, _ = _inputs(B, T, left, H, dk, seed=7, masked=False)
    pos[:] = 0
    bu[:] = 0
    bv[:] = 0
    got = oa.relpos_attention(q, k, v, pos, bu, bv, None, H)
    D = H * dk
    L = left + T
    tq = torch.from_numpy(q).view(B, T, H, dk).transpose(1, 2)
    tk = torch.from_numpy(k).view(B, L, H, dk).transpose(1, 2)
    tv = torch.from_numpy(v).view(B, L, H, dk).transpose(1, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv).transpose(1, 2).reshape(B, T, D)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-12)


def test_torch_fp32_operator_path_matches():
    B, T, left, H, dk = 3, 2, 70, 8, 64
    q, k, v, pos, bu, bv, mask = _inputs(B, T, left, H, dk, seed=3)
    got = oa.relpos_attention_torch(*(torch.from_numpy(x).float() for x in (q, k, v, pos, bu, bv)), torch.from_numpy(mask), H)
    ref = oa.relpos_attention(q, k, v, pos, bu, bv, mask, H)
    np.testing.assert_allclose(got.numpy(), ref, atol=2e-5, rtol=0)


def test_constant_values_reproduced():
    B, T, left, H, dk = 2, 2, 10, 2, 4
    q, k, v, pos, bu, bv, mask = _inputs(B, T, left, H, dk, seed=11)
    v[:] = np.arange(H * dk, dtype=np.float64)
    out = oa.relpos_attention(q, k, v, pos, bu, bv, mask, H)
    np.testing.assert_allclose(out, np.broadcast_to(v[:, :T], out.shape), atol=1e-12)


def test_single_unmasked_key_selects_it():
    B, T, left, H, dk = 1, 2, 6, 2, 4
    q, k, v, pos, bu, bv, _ = _inputs(B, T, left, H, dk, seed=5, masked=False)
    L = left + T
    mask = np.ones((B, T, L), dtype=bool)
    mask[0, 0, 3] = False
    mask[0, 1, 7] = False
    out = oa.relpos_attention(q * 0.1, k * 0.1, v, pos, bu, bv, mask, H)
    np.testing.assert_allclose(out[0, 0], v[0, 3], atol=1e-12)
    np.testing.assert_allclose(out[0, 1], v[0, 7], atol=1e-12)


def test_both_biases_matter():
    B, T, left, H, dk = 1, 2, 5, 2, 4
    q, k, v, pos, bu, bv, mask = _inputs(B, T, left, H, dk, seed=9)
    bu = bu * 50
    bv = bv * 50
    a = oa.relpos_attention(q, k, v, pos, bu, bv, mask, H)
    b = oa.relpos_attention(q, k, v, pos, bv, bu, mask, H)
    assert not np.allclose(a, b)


def test_with_sinusoid_table_and_projection():
    # the bench/test workload: linear_pos of the sinusoid slice
    B, T, left, H, dk = 2, 2, 70, 8, 64
    D = H * dk
    pe = relpos.pos_slice(relpos.sinusoid_table(500, D), T, left)
    rng = np.random.default_rng(0)
    w = rng.standard_normal((D, D)) / np.sqrt(D)
    pos = pe.astype(np.float64) @ w.T
    q, k, v, _, bu, bv, mask = _inputs(B, T, left, H, dk, seed=4)
    a = oa.relpos_attention(q, k, v, pos, bu, bv, mask, H)
    assert np.all(np.isfinite(a))
