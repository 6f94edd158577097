"""Seeded synthetic workloads for the paged encoder-attention step.

There are no checkpoints offline, so inputs are random with the shapes of the
reference models (parakeet/config.py:5-31):

* Q/K/V frames ~ N(0, 1) as the qkv projection output [B, T, 3D] (q | k | v);
* pos_bias_u / pos_bias_v ~ N(0, 0.02^2);
* the position table is linear_pos (W ~ N(0, 1/D)) applied to the sinusoid
  slice of 2L-1 rows PositionalEncoding returns for cache_len = left;
* stream lifetimes for churn: each stream lives a drawn number of steps, and
  free slots are refilled to a target occupancy, FIFO over free slots like the
  reference's slot deque.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass(frozen=True)
class Shape:
    name: str
    layers: int
    d_model: int
    heads: int
    left: int = 70
    right: int = 1
    page_size: int = 16
    dtype: torch.dtype = torch.float16

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads

    @property
    def chunk(self) -> int:
        return self.right + 1

    @property
    def window(self) -> int:
        return self.left + self.chunk

    @property
    def elem_bytes(self) -> int:
        return torch.tensor([], dtype=self.dtype).element_size()


SMALL_FP32 = Shape("small-1layer-fp32", 1, 512, 8, dtype=torch.float32)
SMALL_FP16 = Shape("small-17layer-fp16", 17, 512, 8, dtype=torch.float16)
LARGE_BF16 = Shape("large-24layer-bf16", 24, 1024, 8, dtype=torch.bfloat16)
# the large model's own attention context (70, 13): 14 frames per step, an
# 84-frame window (parakeet/config.py:29, parakeet/modules/cache.py:22)
LARGE_BF16_T14 = Shape("large-24layer-bf16-t14", 24, 1024, 8, right=13, dtype=torch.bfloat16)


def sinusoid_slice(d_model: int, left: int, chunk: int, max_len: int = 5000) -> torch.Tensor:
    """[2L-1, D] fp32 rows for relative positions L-1 ... -(L-1), L = left+chunk,
    as PositionalEncoding.forward(x, cache_len=left) slices them."""
    L = left + chunk
    positions = torch.arange(L - 1, -L, -1, dtype=torch.float32).unsqueeze(1)
    freqs = torch.exp(torch.arange(0, d_model, 2, dtype=torch.float32) * -(math.log(10000.0) / d_model))
    pe = torch.zeros(2 * L - 1, d_model)
    pe[:, 0::2] = torch.sin(positions * freqs)
    pe[:, 1::2] = torch.cos(positions * freqs)
    del max_len
    return pe


def relpos_inputs(shape: Shape, device, seed: int = 0):
    """(pos [2L-1, D], bias_u [H, dk], bias_v [H, dk]) in shape.dtype on device."""
    g = torch.Generator().manual_seed(seed)
    D, H = shape.d_model, shape.heads
    w = torch.randn(D, D, generator=g, dtype=torch.float64) / math.sqrt(D)
    pos = (sinusoid_slice(D, shape.left, shape.chunk).double() @ w.T).to(shape.dtype)
    bu = (torch.randn(H, D // H, generator=g) * 0.02).to(shape.dtype)
    bv = (torch.randn(H, D // H, generator=g) * 0.02).to(shape.dtype)
    return pos.to(device), bu.to(device), bv.to(device)


def qkv_frames(batch: int, shape: Shape, device, seed: int) -> torch.Tensor:
    """[batch, T, 3D] ~ N(0, 1) in shape.dtype (the qkv projection output)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, shape.chunk, 3 * shape.d_model, generator=g)
    return x.to(shape.dtype).to(device)


@dataclass
class Churn:
    """Stream arrivals/departures over a slot pool.

    Each arriving stream lives ``lifetime`` steps drawn from ``durations``
    (seconds at 80 ms/frame, chunk frames per step).  ``occupancy`` of the pool
    is kept filled; freed slots are reused FIFO.  ``stagger`` gives the first
    streams random ages so the pool starts near steady state."""

    num_slots: int
    chunk: int
    occupancy: float = 0.9
    durations: tuple = ("uniform", 2.0, 30.0)
    seed: int = 0
    frame_s: float = 0.08
    rng: np.random.Generator = field(init=False)
    free: list = field(init=False)
    remaining: dict = field(init=False)

    def __post_init__(self):
        self.rng = np.random.default_rng(self.seed)
        self.free = list(range(self.num_slots))
        self.remaining = {}

    def _lifetime(self) -> int:
        kind, lo, hi = self.durations
        if kind == "uniform":
            sec = self.rng.uniform(lo, hi)
        elif kind == "loguniform":
            sec = math.exp(self.rng.uniform(math.log(lo), math.log(hi)))
        else:
            raise ValueError(kind)
        frames = max(1, int(round(sec / self.frame_s)))
        return max(1, -(-frames // self.chunk))

    def step(self) -> tuple[list[int], list[int]]:
        """Advances one step; returns (departed slots, arrived slots).  Streams
        whose lifetime ran out leave; free slots are filled up to occupancy."""
        departed = [s for s, r in self.remaining.items() if r <= 0]
        for s in departed:
            del self.remaining[s]
            self.free.append(s)
        target = int(round(self.occupancy * self.num_slots))
        arrived = []
        while self.free and len(self.remaining) < target:
            s = self.free.pop(0)
            self.remaining[s] = self._lifetime()
            arrived.append(s)
        for s in self.remaining:
            self.remaining[s] -= 1
        return departed, arrived

    def active(self) -> list[int]:
        return sorted(self.remaining)
