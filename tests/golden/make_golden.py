"""Writes the golden fixtures of this directory.

odunola499/parakeet-streaming ships no tests, golden vectors or fixtures for the
paged-cache path, so these vectors are computed here from statements written
independently of ``oracle/`` (different formulations of the same rules), and
both the oracle and the library are checked against them:

* ``masks.npz`` -- streaming attention / padding masks of
  ConformerEncoder._create_streaming_masks (parakeet/modules/encoder.py:167-227)
  over grids of (processed_frames, cache_length, length), in an *interval*
  form: query i of a stream at frame proc may attend the absolute frames
  [max(proc - cache_len, (q_chunk - left_chunks) * C), min(proc + length,
  (q_chunk + 1) * C)) when i < length, with C = right + 1 and the window column
  j holding frame proc - left + j.
* ``sinusoid.npz`` -- PositionalEncoding's table (parakeet/modules/attention.py:
  33-49) with torch fp32 ops in the reference's order.
* ``relpos_attn.npz`` -- rel-pos attention (attention.py:94-121) on tiny inputs
  in float64 torch: the pad/view rel_shift of attention.py:79-83, the slice to
  the key length, 1/sqrt(dk), masked_fill(-1e5), then softmax and the value
  product written out (no SDPA call).
* ``pool_trace.json`` -- a page-pool trace (advance / reset operations, block
  table rows and free queue after each) from a dictionary simulation of the
  FIFO page discipline: a slot holds logical page k of its stream while
  [k*P, (k+1)*P) meets its window [end - window, end); pages leaving the window
  go to the back of the free queue in increasing k, missing pages come from its
  front in increasing k (the deque of parakeet/engine/scheduler.py:84,97,104 at
  page granularity); a reset returns the slot's pages in increasing k.
* ``window_trace.npz`` -- for the same trace with frame codes written at every
  step, the dense window each step must see (parakeet/modules/cache.py:36-45 in
  closed form: column r holds the frame at position end - window + r of the
  stream's current life, zero before its first frame).

Run ``python tests/golden/make_golden.py`` to regenerate; the output is
deterministic.
"""

from __future__ import annotations

import json
import math
import os
from collections import deque

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

MASK_CONFIGS = [(70, 1, 2), (70, 13, 14), (9, 2, 3), (5, 0, 1), (4, 1, 3), (0, 1, 2)]


def mask_cases(left, T):
    cases = []
    for proc in range(0, 2 * (left + T) + 3):
        for cl in sorted({0, min(proc, left), min(proc, left) // 2, max(min(proc, left) - 1, 0)}):
            for n in range(0, T + 1):
                cases.append((proc, cl, n))
    return np.array(cases, dtype=np.int64)


def masks_interval(left, right, T, cases):
    C = right + 1
    lc = left // C
    B = len(cases)
    att = np.ones((B, T, left + T), dtype=bool)
    pad = np.zeros((B, T), dtype=bool)
    for b, (proc, cl, n) in enumerate(cases):
        proc, cl, n = int(proc), int(cl), int(n)
        for i in range(T):
            pad[b, i] = i >= n
            if i >= n:
                continue
            qc = (proc + i) // C
            lo = max(proc - cl, (qc - lc) * C)
            hi = min(proc + n, (qc + 1) * C)
            for kp in range(lo, hi):
                j = kp - proc + left
                if 0 <= j < left + T:
                    att[b, i, j] = False
    return pad, att


def write_masks():
    out = {}
    for left, right, T in MASK_CONFIGS:
        cases = mask_cases(left, T)
        pad, att = masks_interval(left, right, T, cases)
        key = f"l{left}_r{right}_t{T}"
        out[f"{key}_cases"] = cases
        out[f"{key}_pad"] = np.packbits(pad, axis=-1)
        out[f"{key}_att"] = np.packbits(att, axis=-1)
    np.savez_compressed(os.path.join(HERE, "masks.npz"), **out)


def write_sinusoid():
    out = {}
    for length, d_model in ((9, 16), (143, 32)):
        positions = torch.arange(length - 1, -length, -1, dtype=torch.float32).unsqueeze(1)
        div_term = torch.exp(torch.arange(0, d_model, 2, dtype=torch.float32) * -(math.log(10000.0) / d_model))
        pe = torch.zeros(positions.size(0), d_model)
        pe[:, 0::2] = torch.sin(positions * div_term)
        pe[:, 1::2] = torch.cos(positions * div_term)
        out[f"len{length}_d{d_model}"] = pe.numpy()
    np.savez_compressed(os.path.join(HERE, "sinusoid.npz"), **out)


ATTN_CASES = [
    # name, B, T, left, H, dk, masked
    ("b2_t2_l5_h2_d4", 2, 2, 5, 2, 4, True),
    ("b1_t3_l4_h3_d2", 1, 3, 4, 3, 2, True),
    ("b2_t2_l6_h2_d8_nomask", 2, 2, 6, 2, 8, False),
    ("b1_t1_l0_h2_d4", 1, 1, 0, 2, 4, False),
    # head sizes the device kernels are built for; inputs rounded to bf16
    # values, which fp16 and fp32 hold exactly, so every kernel dtype sees
    # exactly these inputs
    ("gpu_b2_t2_l20_h2_d64", 2, 2, 20, 2, 64, True),
    ("gpu_b2_t3_l13_h1_d128", 2, 3, 13, 1, 128, True),
]


def bf16_exact(x):
    """Round to bf16 and flush magnitudes below 2^-12 to zero (exact in fp16)."""
    y = x.to(torch.bfloat16).to(torch.float64)
    return torch.where(y.abs() < 2.0 ** -12, torch.zeros_like(y), y)


def relpos_attn_reference_order(q, k, v, pos, bu, bv, mask, H):
    B, T, D = q.shape
    L = k.shape[1]
    dk = D // H
    query = q.view(B, T, H, dk)
    q_u = (query + bu).transpose(1, 2)
    q_v = (query + bv).transpose(1, 2)
    key = k.view(B, L, H, dk).transpose(1, 2)
    value = v.view(B, L, H, dk).transpose(1, 2)
    p = pos.view(1, -1, H, dk).transpose(1, 2)
    bd = torch.matmul(q_v, p.transpose(-2, -1))
    b_, h_, qlen, plen = bd.shape
    padded = torch.cat([torch.zeros(b_, h_, qlen, 1, dtype=bd.dtype), bd], dim=-1)
    bd = padded.view(b_, h_, plen + 1, qlen)[:, :, 1:].reshape(b_, h_, qlen, plen)
    bd = bd[:, :, :, :L] / math.sqrt(dk)
    if mask is not None:
        bd = bd.masked_fill(mask.unsqueeze(1), -1e5)
    scores = torch.matmul(q_u, key.transpose(-2, -1)) / math.sqrt(dk) + bd
    w = torch.softmax(scores, dim=-1)
    return torch.matmul(w, value).transpose(1, 2).reshape(B, T, D)


def write_relpos_attn():
    out = {}
    g = torch.Generator().manual_seed(20240611)
    for name, B, T, left, H, dk, masked in ATTN_CASES:
        D = H * dk
        L = left + T
        q = torch.randn(B, T, D, generator=g, dtype=torch.float64)
        k = torch.randn(B, L, D, generator=g, dtype=torch.float64)
        v = torch.randn(B, L, D, generator=g, dtype=torch.float64)
        pos = torch.randn(2 * L - 1, D, generator=g, dtype=torch.float64) * 0.5
        bu = torch.randn(H, dk, generator=g, dtype=torch.float64) * 0.02
        bv = torch.randn(H, dk, generator=g, dtype=torch.float64) * 0.02
        mask = None
        if masked:
            mask = torch.rand(B, T, L, generator=g) < 0.3
            mask[:, :, -1] = False
        if name.startswith("gpu_"):
            q, k, v, pos, bu, bv = (bf16_exact(t) for t in (q, k, v, pos, bu, bv))
        o = relpos_attn_reference_order(q, k, v, pos, bu, bv, mask, H)
        for key, val in (("q", q), ("k", k), ("v", v), ("pos", pos), ("bu", bu), ("bv", bv), ("out", o)):
            out[f"{name}_{key}"] = val.numpy()
        out[f"{name}_mask"] = (mask if mask is not None else torch.zeros(B, T, L, dtype=torch.bool)).numpy()
        out[f"{name}_dims"] = np.array([B, T, left, H, dk, int(masked)], dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "relpos_attn.npz"), **out)


# ------------------------------------------------------------------ pool trace
POOL = dict(num_slots=3, page_size=4, left=5, chunk=2, num_pages=11)


def pool_ops():
    rng = np.random.default_rng(7)
    ops = []
    for step in range(26):
        if step in (9, 17):
            ops.append({"op": "reset", "slot": int(step % 3)})
        n = 1 + step % 3
        slots = [int(s) for s in rng.permutation(3)[:n]]
        ops.append({"op": "advance", "slots": slots})
    ops.append({"op": "reset_all"})
    ops.append({"op": "advance", "slots": [2, 0]})
    return ops


class DictPool:
    def __init__(self, num_slots, page_size, left, chunk, num_pages, order):
        self.P, self.left, self.chunk = page_size, left, chunk
        self.window = left + chunk
        self.M = (self.window + page_size - 2) // page_size + 1
        self.free = deque(order)
        self.appended = [0] * num_slots
        self.held = [dict() for _ in range(num_slots)]  # logical page -> physical

    def advance(self, slots):
        rows = []
        for s in slots:
            end = self.appended[s] + self.chunk
            start = end - self.window
            first = max(start, 0) // self.P
            last = (end - 1) // self.P
            for k in sorted(self.held[s]):
                if k < first:
                    self.free.append(self.held[s].pop(k))
            for k in range(first, last + 1):
                if k not in self.held[s]:
                    self.held[s][k] = self.free.popleft()
            ring = [-1] * self.M
            for k, page in self.held[s].items():
                ring[k % self.M] = page
            rows.append([self.appended[s]] + ring)
            self.appended[s] = end
        return rows

    def reset(self, s):
        for k in sorted(self.held[s]):
            self.free.append(self.held[s].pop(k))
        self.appended[s] = 0


def write_pool_trace():
    order = [int(x) for x in np.random.default_rng(3).permutation(POOL["num_pages"])]
    pool = DictPool(POOL["num_slots"], POOL["page_size"], POOL["left"], POOL["chunk"], POOL["num_pages"], order)
    D = 4
    window = POOL["left"] + POOL["chunk"]
    life = [0] * POOL["num_slots"]  # incremented on every reset: a new stream on the slot
    trace = []
    windows = []
    frames = []
    for op in pool_ops():
        rec = dict(op)
        if op["op"] == "advance":
            rows = pool.advance(op["slots"])
            rec["rows"] = rows
            # frame code: slot, life, position; D values per frame
            fr = np.zeros((len(op["slots"]), POOL["chunk"], D), dtype=np.float32)
            win = np.zeros((len(op["slots"]), window, D), dtype=np.float32)
            for b, s in enumerate(op["slots"]):
                A = rows[b][0]
                code = lambda pos: 1 + s * 64 + (life[s] % 4) * 16 + (pos % 16)  # noqa: E731
                for t in range(POOL["chunk"]):
                    fr[b, t] = code(A + t) + np.arange(D) / 8.0
                for r in range(window):
                    pos = A + POOL["chunk"] - window + r
                    if pos >= 0:
                        win[b, r] = code(pos) + np.arange(D) / 8.0
            frames.append(fr)
            windows.append(win)
        elif op["op"] == "reset":
            pool.reset(op["slot"])
            life[op["slot"]] += 1
        else:
            for s in range(POOL["num_slots"]):
                pool.reset(s)
                life[s] += 1
        rec["free"] = list(pool.free)
        trace.append(rec)
    with open(os.path.join(HERE, "pool_trace.json"), "w") as f:
        json.dump({"pool": POOL, "page_order": order, "trace": trace}, f, indent=0)
    out = {}
    for i, (fr, win) in enumerate(zip(frames, windows)):
        out[f"frames_{i:03d}"] = fr
        out[f"window_{i:03d}"] = win
    np.savez_compressed(os.path.join(HERE, "window_trace.npz"), **out)


if __name__ == "__main__":
    write_masks()
    write_sinusoid()
    write_relpos_attn()
    write_pool_trace()
    for f in sorted(os.listdir(HERE)):
        print(f, os.path.getsize(os.path.join(HERE, f)))
