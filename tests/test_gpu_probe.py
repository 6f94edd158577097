"""The HBM read probe the benchmark times beside each attention launch: it must
read every byte of its buffer exactly once.  XOR is associative, so the XOR of
the per-wave words it writes equals the XOR of all 16-byte words of the buffer."""

import numpy as np
import pytest
import torch

from parakeet_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,workgroups", [(16, 0), (65536 * 3 + 48, 0), (1 << 22, 0), ((1 << 22) + 16, 7)])
def test_read_probe_reads_every_word_once(cuda, nbytes, workgroups):
    print(f"\n[read probe] {nbytes} bytes, workgroups {workgroups}", flush=True)
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    src = torch.from_numpy(host.view(np.int32).copy()).to(cuda)
    wg = workgroups if workgroups else 8 * torch.cuda.get_device_properties(cuda).multi_processor_count
    out = torch.zeros(64 * wg, dtype=torch.uint8, device=cuda)
    ops.hbm_read_probe(src, out, workgroups)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32).reshape(-1, 4), axis=0)
    want = np.bitwise_xor.reduce(host.reshape(-1, 4), axis=0)
    assert np.array_equal(got, want)
