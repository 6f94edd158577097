"""The oracle and the host page pool against the committed golden fixtures
(tests/golden/, written by tests/golden/make_golden.py from statements
independent of oracle/): streaming masks (encoder.py:167-227), the sinusoid
table (attention.py:33-49), rel-pos attention on tiny inputs
(attention.py:94-121), a page-pool trace (the FIFO deque discipline of
scheduler.py:84,97,104 at page granularity) and the dense windows of that
trace (cache.py:36-45).  CPU only."""

import json
import os

import numpy as np
import pytest

from oracle import attention as oa
from oracle import masks as om
from oracle import paging
from oracle import relpos
from parakeet_amd.pool import PagePool

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MASK_CONFIGS = [(70, 1, 2), (70, 13, 14), (9, 2, 3), (5, 0, 1), (4, 1, 3), (0, 1, 2)]
ATTN_CASES = [
    "b2_t2_l5_h2_d4", "b1_t3_l4_h3_d2", "b2_t2_l6_h2_d8_nomask", "b1_t1_l0_h2_d4",
    "gpu_b2_t2_l20_h2_d64", "gpu_b2_t3_l13_h1_d128",
]


def golden_masks(left, right, T):
    z = np.load(os.path.join(GOLDEN, "masks.npz"))
    k = f"l{left}_r{right}_t{T}"
    cases = z[k + "_cases"]
    att = np.unpackbits(z[k + "_att"], axis=-1, count=left + T).astype(bool)
    pad = np.unpackbits(z[k + "_pad"], axis=-1, count=T).astype(bool)
    return cases, pad, att


def golden_attention(name):
    z = np.load(os.path.join(GOLDEN, "relpos_attn.npz"))
    d = {key: z[f"{name}_{key}"] for key in ("q", "k", "v", "pos", "bu", "bv", "mask", "out")}
    B, T, left, H, dk, masked = (int(x) for x in z[f"{name}_dims"])
    d.update(B=B, T=T, left=left, H=H, dk=dk, masked=bool(masked))
    return d


def golden_trace():
    with open(os.path.join(GOLDEN, "pool_trace.json")) as f:
        tr = json.load(f)
    win = np.load(os.path.join(GOLDEN, "window_trace.npz"))
    return tr, win


@pytest.mark.parametrize("left,right,T", MASK_CONFIGS)
def test_masks_match_golden(left, right, T):
    cases, pad_g, att_g = golden_masks(left, right, T)
    proc, cl, n = cases[:, 0], cases[:, 1], cases[:, 2]
    pad, att = om.create_streaming_masks(T, cl, proc, n, (left, right))
    np.testing.assert_array_equal(pad, pad_g)
    np.testing.assert_array_equal(att, att_g)
    pad2, att2 = om.masks_by_position(T, cl, proc, n, (left, right))
    np.testing.assert_array_equal(att2, att_g)
    np.testing.assert_array_equal(pad2, pad_g)


def test_sinusoid_matches_golden():
    z = np.load(os.path.join(GOLDEN, "sinusoid.npz"))
    for length, d_model in ((9, 16), (143, 32)):
        g = z[f"len{length}_d{d_model}"]
        got = relpos.sinusoid_table(length, d_model)
        # numpy's and torch's float32 exp may differ by an ulp in a frequency
        # term w (< 2^-23 relative); the angle pos*w, |pos| <= length, carries
        # that times |pos|, so |d sin| <= length * 2^-23 plus the final roundings
        np.testing.assert_allclose(got, g, rtol=0, atol=length * 2.0 ** -23 + 2.0 ** -23)


@pytest.mark.parametrize("name", ATTN_CASES)
def test_attention_matches_golden(name):
    d = golden_attention(name)
    mask = d["mask"] if d["masked"] else None
    got = oa.relpos_attention(d["q"], d["k"], d["v"], d["pos"], d["bu"], d["bv"], mask, d["H"])
    np.testing.assert_allclose(got, d["out"], rtol=0, atol=1e-12)
    got2 = oa.relpos_attention_direct(d["q"], d["k"], d["v"], d["pos"], d["bu"], d["bv"], mask, d["H"])
    np.testing.assert_allclose(got2, d["out"], rtol=0, atol=1e-12)


def _replay_pool(pool, tr):
    """Replays the trace on a pool object (oracle model or native pool) and
    checks every block-table row and the free queue after every operation."""
    for i, rec in enumerate(tr["trace"]):
        if rec["op"] == "advance":
            rows = pool.advance(np.asarray(rec["slots"], dtype=np.int32))
            np.testing.assert_array_equal(np.asarray(rows), np.asarray(rec["rows"], dtype=np.int32), err_msg=f"op {i}")
        elif rec["op"] == "reset":
            pool.reset_slot(rec["slot"])
        else:
            pool.reset_all()
        np.testing.assert_array_equal(pool.free_list(), np.asarray(rec["free"], dtype=np.int32), err_msg=f"op {i}")


def test_pool_model_matches_golden_trace():
    tr, _ = golden_trace()
    p = tr["pool"]
    model = paging.PagePoolModel(p["num_pages"], p["num_slots"], p["page_size"], p["left"], p["chunk"], tr["page_order"])
    _replay_pool(model, tr)


def test_native_pool_matches_golden_trace():
    tr, _ = golden_trace()
    p = tr["pool"]
    pool = PagePool(p["num_slots"], p["page_size"], p["left"], p["chunk"], num_pages=p["num_pages"], page_order=tr["page_order"])
    try:
        _replay_pool(pool, tr)
    finally:
        pool.close()


def test_paged_windows_match_golden_trace():
    """oracle.paging append + gather over the trace's rows reproduce the dense
    window of every step, bit for bit."""
    tr, win = golden_trace()
    p = tr["pool"]
    P, left, T = p["page_size"], p["left"], p["chunk"]
    L = left + T
    M = paging.max_pages(left, T, P)
    D = 4
    kp = np.full((1, p["num_pages"], P, D), np.nan, dtype=np.float32)
    vp = np.full_like(kp, np.nan)
    step = 0
    for rec in tr["trace"]:
        if rec["op"] != "advance":
            continue
        rows = np.asarray(rec["rows"], dtype=np.int32)
        fr = win[f"frames_{step:03d}"]
        paging.append(kp, vp, rows, 0, fr, -fr, P, M)
        ok, ov = paging.gather(kp, vp, rows, 0, L, T, P, M)
        np.testing.assert_array_equal(ok, win[f"window_{step:03d}"])
        np.testing.assert_array_equal(ov, -win[f"window_{step:03d}"])
        step += 1
    assert step > 20
