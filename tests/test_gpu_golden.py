"""GPU parity against the committed golden fixtures (tests/golden/):

* the device mask builder (pk_streaming_mask) against the streaming-mask grids,
  bit-exact (encoder.py:167-227);
* the fused append + paged rel-pos attention kernel against the rel-pos
  attention vectors (attention.py:94-121) in fp32, fp16 and bf16 -- the fixture
  inputs are bf16 values, exact in every dtype, so the tolerance is the
  kernel's own (fp32 1e-4, fp16 2e-3, bf16 1e-2 max-abs); the appended pages
  are checked bit-exact;
* page append + gather (pk_kv_append / pk_kv_gather) over the page-pool trace
  with the native pool producing the rows: every row matches the trace and
  every gathered window matches the dense window of the trace bit for bit
  (cache.py:36-45).
"""

import numpy as np
import pytest
import torch

from parakeet_amd import ops
from parakeet_amd.pool import PagePool, pages_per_slot
from test_golden import MASK_CONFIGS, golden_attention, golden_masks, golden_trace

TOL = {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 1e-2}


@pytest.mark.gpu
@pytest.mark.parametrize("left,right,T", MASK_CONFIGS)
def test_mask_kernel_matches_golden(cuda, left, right, T):
    print(f"\n[golden-mask] left={left} right={right} T={T}", flush=True)
    cases, pad_g, att_g = golden_masks(left, right, T)
    proc, cl, n = (torch.from_numpy(np.ascontiguousarray(cases[:, c])).to(cuda) for c in (0, 1, 2))
    pad, att = ops.streaming_mask(proc, cl, n, chunk=T, left=left, chunk_size=right + 1)
    np.testing.assert_array_equal(pad.cpu().numpy(), pad_g)
    np.testing.assert_array_equal(att.cpu().numpy(), att_g)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("name", ["gpu_b2_t2_l20_h2_d64", "gpu_b2_t3_l13_h1_d128"])
def test_attention_kernel_matches_golden(cuda, name, dtype):
    print(f"\n[golden-attn] {name} {dtype}", flush=True)
    d = golden_attention(name)
    B, T, left, H = d["B"], d["T"], d["left"], d["H"]
    L = left + T
    D = d["q"].shape[-1]
    P = 16
    M = pages_per_slot(left, T, P)
    # stream b: frames 0..L-1 = the fixture's window; the history (frames
    # 0..left-1) is in the pages, this step's frames are appended by the kernel
    kp = torch.full((1, B * M, P, D), float("nan"), dtype=dtype)
    vp = torch.full_like(kp, float("nan"))
    rows = np.full((B, 1 + M), -1, dtype=np.int32)
    for b in range(B):
        rows[b, 0] = left
        for lp in range((L + P - 1) // P):
            rows[b, 1 + lp % M] = b * M + lp
        kb, vb = ops.page_blocks(kp), ops.page_blocks(vp)
        nb = kb.shape[2]
        for pos in range(left):
            page = rows[b, 1 + (pos // P) % M]
            kb[0, page, :, pos % P] = torch.from_numpy(d["k"][b, pos]).to(dtype).view(nb, -1)
            vb[0, page, :, pos % P] = torch.from_numpy(d["v"][b, pos]).to(dtype).view(nb, -1)
    pages = ops.PagedKV(kp.to(cuda), vp.to(cuda), torch.from_numpy(rows).to(cuda), M)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(cuda)  # noqa: E731
    q, kn, vn = dev(d["q"]), dev(d["k"][:, left:]), dev(d["v"][:, left:])
    out = ops.paged_relpos_attn(
        q, kn, vn, dev(d["pos"]), dev(d["bu"]), dev(d["bv"]), torch.from_numpy(d["mask"]).to(cuda),
        num_heads=H, left=left, pages=pages, layer=0, append=True,
    )
    err = float(np.abs(out.double().cpu().numpy() - d["out"]).max())
    print(f"  max abs err {err:.3e}", flush=True)
    assert err <= TOL[dtype]
    gk, gv = ops.kv_gather(pages, 0, B, L, T)
    assert torch.equal(gk.cpu(), torch.from_numpy(d["k"]).to(dtype))
    assert torch.equal(gv.cpu(), torch.from_numpy(d["v"]).to(dtype))


@pytest.mark.gpu
def test_page_trace_matches_golden(cuda):
    print("\n[golden-trace]", flush=True)
    tr, win = golden_trace()
    p = tr["pool"]
    P, left, T = p["page_size"], p["left"], p["chunk"]
    L = left + T
    pool = PagePool(p["num_slots"], P, left, T, num_pages=p["num_pages"], page_order=tr["page_order"])
    M = pool.max_pages
    kp = torch.full((1, p["num_pages"], P, 4), float("nan"), device=cuda)
    vp = torch.full_like(kp, float("nan"))
    step = 0
    try:
        for i, rec in enumerate(tr["trace"]):
            if rec["op"] == "reset":
                pool.reset_slot(rec["slot"])
                continue
            if rec["op"] == "reset_all":
                pool.reset_all()
                continue
            rows = pool.advance(np.asarray(rec["slots"], dtype=np.int32))
            np.testing.assert_array_equal(rows, np.asarray(rec["rows"], dtype=np.int32), err_msg=f"op {i}")
            pages = ops.PagedKV(kp, vp, torch.from_numpy(np.ascontiguousarray(rows)).to(cuda), M)
            fr = torch.from_numpy(win[f"frames_{step:03d}"]).to(cuda)
            ops.kv_append(pages, 0, fr, -fr)
            gk, gv = ops.kv_gather(pages, 0, len(rec["slots"]), L, T)
            expect = torch.from_numpy(win[f"window_{step:03d}"])
            assert torch.equal(gk.cpu(), expect), f"op {i}"
            assert torch.equal(gv.cpu(), -expect), f"op {i}"
            step += 1
    finally:
        pool.close()
    torch.cuda.synchronize()
