"""One encoder-attention step for a batch of streams, all layers, with the
launch arguments built once.

This is the hot path of ``_encode_step`` (parakeet/engine/model_runner.py:254-304)
reduced to its paged-cache work, for serving loops that drive the kernels
directly and for measurement:

  1. open the step on the host page pool (evict / allocate / rows upload),
  2. gather the batch's processed_frames / cache_lengths and build the
     streaming masks on the device (encoder.py:167-227),
  3. per layer: fused page append + paged rel-pos attention
     (attention.py:97-121),
  4. advance the state scalars (encoder.py:257-260).

The qkv projection output of every layer is an input ([slots, T, 3D] per
layer, q | k | v); the outputs land in per-layer [slots, T, D] buffers.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import ops
from ._lib import AttnArgs, MaskArgs, check, lib
from .pool import PagePool
from .synth import Shape


class AttentionStep:
    def __init__(
        self,
        shape: Shape,
        num_slots: int,
        device: torch.device,
        qkv: list[torch.Tensor],
        pos: torch.Tensor,
        bias_u: list[torch.Tensor],
        bias_v: list[torch.Tensor],
        page_order=None,
        num_pages: int | None = None,
        rows_per_lane: int = 0,
    ):
        self.shape = shape
        self.num_slots = int(num_slots)
        self.device = device
        T, D, Ly = shape.chunk, shape.d_model, shape.layers
        L = shape.window
        self.pool = PagePool(num_slots, shape.page_size, shape.left, T, num_pages=num_pages, page_order=page_order)
        M = self.pool.max_pages
        self.k_pages = torch.empty((Ly, self.pool.num_pages, shape.page_size, D), dtype=shape.dtype, device=device)
        self.v_pages = torch.empty_like(self.k_pages)
        self.proc = torch.zeros(num_slots, dtype=torch.int64, device=device)
        self.cache_len = torch.zeros(num_slots, dtype=torch.int64, device=device)
        self.rows = torch.zeros((num_slots, 1 + M), dtype=torch.int32, device=device)
        self.slot_idx = torch.zeros(num_slots, dtype=torch.int64, device=device)
        self.b_proc = torch.zeros(num_slots, dtype=torch.int64, device=device)
        self.b_cl = torch.zeros(num_slots, dtype=torch.int64, device=device)
        self.mask = torch.empty((num_slots, T, L), dtype=torch.bool, device=device)
        self.pad = torch.empty((num_slots, T), dtype=torch.bool, device=device)
        self.out = [torch.empty((num_slots, T, D), dtype=shape.dtype, device=device) for _ in range(Ly)]
        if len(qkv) != Ly or any(tuple(x.shape) != (num_slots, T, 3 * D) for x in qkv):
            raise ValueError(f"qkv must be {Ly} tensors of shape {(num_slots, T, 3 * D)}")
        self.qkv = qkv
        self.pos, self.bias_u, self.bias_v = pos, bias_u, bias_v
        # pinned staging for the per-step uploads (rows, slot ids), ring of 4
        self._stage_rows = [torch.empty((num_slots, 1 + M), dtype=torch.int32, pin_memory=True) for _ in range(4)]
        self._stage_idx = [torch.empty(num_slots, dtype=torch.int64, pin_memory=True) for _ in range(4)]
        self._stage_ev: list[torch.cuda.Event | None] = [None] * 4
        self._stage_i = 0
        self._args = [self._attn_args(layer, rows_per_lane) for layer in range(Ly)]
        self._mask_args = self._build_mask_args()
        self._stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        self.batch = 0

    # ------------------------------------------------------------ arg structs
    def _attn_args(self, layer: int, rows_per_lane: int) -> AttnArgs:
        sh = self.shape
        D = sh.d_model
        x = self.qkv[layer]
        q, k, v = x.chunk(3, dim=-1)
        pages = ops.PagedKV(self.k_pages, self.v_pages, self.rows, self.pool.max_pages)
        a = AttnArgs()
        a.dtype = ops.dtype_code(sh.dtype)
        a.device = self.device.index if self.device.index is not None else torch.cuda.current_device()
        a.pages = pages.layout()
        a.layer, a.batch, a.chunk = layer, 0, sh.chunk
        a.num_heads, a.head_dim, a.left, a.append = sh.heads, sh.head_dim, sh.left, 1
        a.query, a.query_stride_b, a.query_stride_t = q.data_ptr(), q.stride(0), q.stride(1)
        a.key, a.key_stride_b, a.key_stride_t = k.data_ptr(), k.stride(0), k.stride(1)
        a.value, a.value_stride_b, a.value_stride_t = v.data_ptr(), v.stride(0), v.stride(1)
        a.pos, a.pos_stride, a.pos_rows = self.pos.data_ptr(), self.pos.stride(0), self.pos.shape[0]
        bu, bv = self.bias_u[layer], self.bias_v[layer]
        if tuple(bu.shape) != (sh.heads, sh.head_dim) or not bu.is_contiguous() or not bv.is_contiguous():
            raise ValueError("bias_u / bias_v must be contiguous [H, dk]")
        a.bias_u, a.bias_v = bu.data_ptr(), bv.data_ptr()
        a.mask = self.mask.data_ptr()
        a.mask_stride_b, a.mask_stride_h, a.mask_stride_t = self.mask.stride(0), 0, self.mask.stride(1)
        o = self.out[layer]
        a.out, a.out_stride_b, a.out_stride_t = o.data_ptr(), o.stride(0), o.stride(1)
        a.rows_per_lane = rows_per_lane
        if D != self.k_pages.shape[3]:
            raise ValueError("d_model mismatch")
        return a

    def _build_mask_args(self) -> MaskArgs:
        sh = self.shape
        m = MaskArgs()
        m.device = self.device.index if self.device.index is not None else torch.cuda.current_device()
        m.batch, m.chunk, m.left, m.chunk_size = 0, sh.chunk, sh.left, sh.right + 1
        m.processed_frames = self.b_proc.data_ptr()
        m.cache_lengths = self.b_cl.data_ptr()
        m.lengths = None
        m.length_scalar = sh.chunk
        m.att_mask = self.mask.data_ptr()
        m.pad_mask = self.pad.data_ptr()
        return m

    # ------------------------------------------------------------ stream life
    def reset_slots(self, slots) -> None:
        """Streams leaving (or arriving on reused slots): free their pages and
        zero their state (parakeet/engine/scheduler.py:86-91)."""
        if len(slots) == 0:
            return
        for s in slots:
            self.pool.reset_slot(int(s))
        idx = torch.as_tensor(np.asarray(slots, dtype=np.int64)).to(self.device, non_blocking=False)
        self.proc.index_fill_(0, idx, 0)
        self.cache_len.index_fill_(0, idx, 0)

    # ------------------------------------------------------------ one step
    def open(self, slots: np.ndarray) -> int:
        """Host page work + uploads for the batch ``slots``; returns B."""
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        B = int(slots.shape[0])
        i = self._stage_i
        self._stage_i = (i + 1) % len(self._stage_rows)
        ev = self._stage_ev[i]
        if ev is not None:
            ev.synchronize()
        rows_h = self._stage_rows[i]
        self.pool.advance(slots, out=rows_h.numpy())
        idx_h = self._stage_idx[i]
        idx_h.numpy()[:B] = slots
        self.rows[:B].copy_(rows_h[:B], non_blocking=True)
        self.slot_idx[:B].copy_(idx_h[:B], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._stage_ev[i] = ev
        self.batch = B
        return B

    def run(self, events=None) -> None:
        """Masks, all layers' fused append + attention, state advance for the
        batch opened last.  ``events``: optional per-layer (start, stop) pairs
        timing each attention kernel."""
        B = self.batch
        if B == 0:
            return
        sh = self.shape
        L = lib()
        idx = self.slot_idx[:B]
        torch.index_select(self.proc, 0, idx, out=self.b_proc[:B])
        torch.index_select(self.cache_len, 0, idx, out=self.b_cl[:B])
        self._mask_args.batch = B
        check(L.pk_streaming_mask(ctypes.byref(self._mask_args), self._stream), "pk_streaming_mask")
        for layer, a in enumerate(self._args):
            a.batch = B
            if events is not None:
                a.start_event, a.stop_event = events[layer]
            else:
                a.start_event = a.stop_event = None
            check(L.pk_paged_relpos_attn(ctypes.byref(a), self._stream), "pk_paged_relpos_attn")
        # encoder.py:257-260 with length == chunk
        self.b_proc[:B] += sh.chunk
        self.b_cl[:B] += sh.chunk
        self.b_cl[:B].clamp_(max=sh.left)
        self.proc.index_copy_(0, idx, self.b_proc[:B])
        self.cache_len.index_copy_(0, idx, self.b_cl[:B])

    def step(self, slots: np.ndarray, events=None) -> None:
        self.open(slots)
        self.run(events)

    # ------------------------------------------------------------ accounting
    def bytes_per_stream(self) -> int:
        """Algorithmic HBM bytes per stream per layer: K/V window read (2L
        frames), K/V append write (2T), query read + output write (2T), and the
        block-table row (4 * max_pages)."""
        sh = self.shape
        s = sh.elem_bytes
        return s * sh.d_model * (2 * sh.window + 2 * sh.chunk + 2 * sh.chunk) + 4 * self.pool.max_pages

    def bytes_shared_per_launch(self) -> int:
        """Position-table rows the launch needs (left + 2T - 1) and both biases."""
        sh = self.shape
        s = sh.elem_bytes
        return s * sh.d_model * (sh.left + 2 * sh.chunk - 1) + 2 * s * sh.d_model
