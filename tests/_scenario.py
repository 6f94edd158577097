"""Stepped scenario shared by the GPU parity tests: the HIP paged path and the
oracle's dense shift buffer see the same seeded frames, step after step."""

from __future__ import annotations

import numpy as np
import torch

from oracle import dense_cache
from parakeet_amd import ops
from parakeet_amd.pool import PagePool

NP_OF = {torch.float32: np.float32, torch.float16: np.float32, torch.bfloat16: np.float32}


class PagedScenario:
    def __init__(self, device, dtype, B, layers, d_model, left, right, page_size, seed=0, shuffle=False, extra_pages=0):
        self.device, self.dtype = device, dtype
        self.B, self.Ly, self.D = B, layers, d_model
        self.left, self.right = left, right
        self.T = right + 1
        self.L = left + self.T
        self.P = page_size
        self.gen = torch.Generator().manual_seed(seed)
        rng = np.random.default_rng(seed)
        M = (self.L + page_size - 2) // page_size + 1
        self.num_pages = B * M + extra_pages
        order = rng.permutation(self.num_pages) if shuffle else None
        self.pool = PagePool(B, page_size, left, self.T, num_pages=self.num_pages, page_order=order)
        self.M = self.pool.max_pages
        # poison: any read of a never-written page row shows up as NaN
        self.k_pages = torch.full((layers, self.num_pages, page_size, d_model), float("nan"), dtype=dtype, device=device)
        self.v_pages = torch.full_like(self.k_pages, float("nan"))
        self.dense = dense_cache.DenseCache(layers, left, right, d_model, B)
        self.rows = None
        self.pages = None

    def open_step(self, slots=None):
        slots = np.arange(self.B, dtype=np.int32) if slots is None else np.asarray(slots, dtype=np.int32)
        rows = self.pool.advance(slots)
        self.rows = torch.from_numpy(rows.copy()).to(self.device)
        self.pages = ops.PagedKV(self.k_pages, self.v_pages, self.rows, self.M)
        return rows

    def reset(self, slot):
        self.pool.reset_slot(slot)
        self.dense.reset_slot(slot)

    def frames(self):
        """qkv [B, T, 3D] in dtype on the device (views q/k/v like qkv.chunk)."""
        x = torch.randn(self.B, self.T, 3 * self.D, generator=self.gen).to(self.dtype).to(self.device)
        return x, x.chunk(3, dim=-1)

    def dense_update(self, layer, k, v):
        kk = k.float().cpu().numpy()
        vv = v.float().cpu().numpy()
        return self.dense.update_attn_cache(layer, kk, vv)


def to_np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)
