"""GPU parity: the device mask builder (pk_streaming_mask) against the oracle's
loop restatement of ConformerEncoder._create_streaming_masks
(parakeet/modules/encoder.py:167-227), bit-exact over grids of processed
frames, cache lengths and lengths, tensor and scalar lengths."""

import numpy as np
import pytest
import torch

from oracle import masks as om
from parakeet_amd import ops


def _grid(left, T):
    cases = []
    for proc in range(0, 3 * (left + T) + 1):
        for cl in sorted({0, min(proc, left), min(proc, left) // 2}):
            if cl > proc:
                continue
            for n in range(0, T + 1):
                cases.append((proc, cl, n))
    return cases


@pytest.mark.gpu
@pytest.mark.parametrize("left,right,T", [(70, 1, 2), (70, 13, 14), (7, 2, 3), (5, 0, 1), (9, 3, 4), (4, 1, 3)])
def test_mask_kernel_bit_exact(cuda, left, right, T):
    print(f"\n[mask] left={left} right={right} T={T}", flush=True)
    cases = _grid(left, T)
    proc = np.array([c[0] for c in cases], dtype=np.int64)
    cl = np.array([c[1] for c in cases], dtype=np.int64)
    n = np.array([c[2] for c in cases], dtype=np.int64)
    pad, att = ops.streaming_mask(
        torch.from_numpy(proc).to(cuda), torch.from_numpy(cl).to(cuda), torch.from_numpy(n).to(cuda),
        chunk=T, left=left, chunk_size=right + 1,
    )
    pad_r, att_r = om.create_streaming_masks(T, cl, proc, n, (left, right))
    np.testing.assert_array_equal(pad.cpu().numpy(), pad_r)
    np.testing.assert_array_equal(att.cpu().numpy(), att_r)


@pytest.mark.gpu
def test_mask_kernel_scalar_length(cuda):
    left, right, T = 70, 1, 2
    proc = np.arange(0, 200, 2, dtype=np.int64)
    cl = np.minimum(proc, left)
    pad, att = ops.streaming_mask(torch.from_numpy(proc).to(cuda), torch.from_numpy(cl).to(cuda), T, chunk=T, left=left, chunk_size=2)
    pad_r, att_r = om.create_streaming_masks(T, cl, proc, T, (left, right))
    np.testing.assert_array_equal(att.cpu().numpy(), att_r)
    np.testing.assert_array_equal(pad.cpu().numpy(), pad_r)
