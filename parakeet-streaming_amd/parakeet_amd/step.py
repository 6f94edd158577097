"""One encoder-attention step for a batch of streams, all layers, with the
launch arguments built once.

This is the hot path of ``_encode_step`` (parakeet/engine/model_runner.py:254-304)
reduced to its paged-cache work, for serving loops that drive the kernels
directly and for measurement:

  1. open the step on the host page pool (evict / allocate) and upload, in one
     asynchronous copy from pinned memory, the live stream count, the batch's
     processed_frames / cache_lengths and its block-table rows (the reference
     gathers the state per step with index_select, parakeet/engine/scheduler.py:
     128-170);
  2. per layer: one kernel -- fused page append + paged rel-pos attention with
     the streaming mask evaluated in the kernel from the stream state
     (attention.py:97-121, encoder.py:167-227);
  3. advance the state scalars (encoder.py:257-260) on the host mirror.

The engine always feeds whole chunks (parakeet/engine/sequence.py:137-146), so
``length`` is the chunk for every stream and the state advance is known on the
host without a device round trip.

Every device pointer the launches use is fixed for the life of the object (the
batch arrays are sized for all slots and the live count is read on the device),
so ``capture()`` can record all layers' launches once in a HIP graph and
``step(..., graph=True)`` replays it for a batch of any size.

The qkv projection output of every layer is an input ([slots, T, 3D] per
layer, q | k | v; batch row b reads row b); the outputs land in per-layer
[slots, T, D] buffers.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import ops
from ._lib import AttnArgs, check, lib
from .pool import PagePool
from .synth import Shape

_HDR = 16  # bytes before the state: the int32 live count, padded


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
        self.num_slots = S = int(num_slots)
        self.device = device
        T, D, Ly = shape.chunk, shape.d_model, shape.layers
        self.pool = PagePool(S, shape.page_size, shape.left, T, num_pages=num_pages, page_order=page_order)
        M = self.pool.max_pages
        self.k_pages = torch.empty((Ly, self.pool.num_pages, shape.page_size, D), dtype=shape.dtype, device=device)
        self.v_pages = torch.empty_like(self.k_pages)
        # one upload per step: [live count | pad][processed_frames[S] | cache_lengths[S]][rows[S][1+M]]
        self._state_off = _HDR
        self._rows_off = _HDR + 16 * S
        self._meta_bytes = self._rows_off + 4 * S * (1 + M)
        self.meta = torch.zeros(self._meta_bytes, dtype=torch.uint8, device=device)
        self.live, self.state, self.rows = self._views(self.meta)
        # per-slot streaming state, advanced on the host (length == chunk)
        self.h_proc = np.zeros(S, dtype=np.int64)
        self.h_cl = np.zeros(S, dtype=np.int64)
        self.out = [torch.empty((S, T, D), dtype=shape.dtype, device=device) for _ in range(Ly)]
        if len(qkv) != Ly or any(tuple(x.shape) != (S, T, 3 * D) for x in qkv):
            raise ValueError(f"qkv must be {Ly} tensors of shape {(S, T, 3 * D)}")
        self.qkv = qkv
        self.pos, self.bias_u, self.bias_v = pos, bias_u, bias_v
        # pinned staging, ring of 4: a buffer is reused only after the copy that
        # read it has completed
        depth = 4
        self._stage = [torch.zeros(self._meta_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(depth)]
        self._stage_ev = [torch.cuda.Event() for _ in range(depth)]
        self._stage_used = [False] * depth
        self._stage_i = 0
        self._args = [self._attn_args(layer, rows_per_lane) for layer in range(Ly)]
        self._stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        self.batch = 0
        self.graph: torch.cuda.CUDAGraph | None = None

    def _views(self, buf: torch.Tensor):
        S, M = self.num_slots, self.pool.max_pages
        live = buf[0:4].view(torch.int32)
        state = buf[self._state_off : self._rows_off].view(torch.int64)
        rows = buf[self._rows_off :].view(torch.int32).view(S, 1 + M)
        return live, state, rows

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
        # streaming mask from the stream state (encoder.py:167-227), length == chunk
        a.processed_frames = self.state.data_ptr()
        a.cache_lengths = self.state.data_ptr() + 8 * self.num_slots
        a.length_scalar = sh.chunk
        a.chunk_size = sh.right + 1
        o = self.out[layer]
        a.out, a.out_stride_b, a.out_stride_t = o.data_ptr(), o.stride(0), o.stride(1)
        a.rows_per_lane = rows_per_lane
        if D != self.k_pages.shape[3]:
            raise ValueError("d_model mismatch")
        return a

    # ------------------------------------------------------------ stream life
    def reset_slots(self, slots) -> None:
        """Streams leaving (or arriving on reused slots): free their pages and
        zero their state (parakeet/engine/scheduler.py:86-91)."""
        for s in slots:
            self.pool.reset_slot(int(s))
            self.h_proc[int(s)] = 0
            self.h_cl[int(s)] = 0

    # ------------------------------------------------------------ one step
    def open(self, slots: np.ndarray) -> int:
        """Host page work + the upload for the batch ``slots``; returns B."""
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        B = int(slots.shape[0])
        S = self.num_slots
        if B > S:
            raise ValueError(f"batch of {B} streams exceeds {S} slots")
        i = self._stage_i
        self._stage_i = (i + 1) % len(self._stage)
        if self._stage_used[i]:
            self._stage_ev[i].synchronize()
        buf = self._stage[i]
        live, state, rows = self._views(buf)
        live.fill_(B)
        st = state.numpy()
        st[:B] = self.h_proc[slots]
        st[S : S + B] = self.h_cl[slots]
        if B:
            self.pool.advance(slots, out=rows.numpy())
        n = self._rows_off + 4 * B * (1 + self.pool.max_pages)
        self.meta[:n].copy_(buf[:n], non_blocking=True)
        self._stage_ev[i].record()
        self._stage_used[i] = True
        # encoder.py:257-260 with length == chunk
        T = self.shape.chunk
        self.h_proc[slots] += T
        self.h_cl[slots] = np.minimum(self.h_cl[slots] + T, self.shape.left)
        self.batch = B
        return B

    def run(self, events=None) -> None:
        """All layers' fused append + attention for the batch opened last, one
        launch per layer sized to the batch.  ``events``: optional per-layer
        (start, stop) pairs timing each kernel."""
        B = self.batch
        if B == 0:
            return
        L = lib()
        for layer, a in enumerate(self._args):
            a.batch = B
            a.live_streams = None
            if events is not None:
                a.start_event, a.stop_event = events[layer]
            else:
                a.start_event = a.stop_event = None
            check(L.pk_paged_relpos_attn(ctypes.byref(a), self._stream), "pk_paged_relpos_attn")

    def capture(self) -> None:
        """Records every layer's launch in a HIP graph: the launches cover all
        slots and read the live count from the device, so one recording serves
        every batch size.  The recording holds no memset and no allocation."""
        L = lib()
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.graph(g, stream=side):
            stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
            for a in self._args:
                a.batch = self.num_slots
                a.live_streams = self.live.data_ptr()
                a.start_event = a.stop_event = None
                check(L.pk_paged_relpos_attn(ctypes.byref(a), stream), "pk_paged_relpos_attn")
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.graph = g

    def step(self, slots: np.ndarray, events=None, graph: bool = False) -> None:
        self.open(slots)
        if graph:
            if self.graph is None:
                self.capture()
            if self.batch:
                self.graph.replay()
        else:
            self.run(events)

    # ------------------------------------------------------------ accounting
    def bytes_per_stream(self) -> int:
        """Algorithmic HBM bytes per stream per layer: K/V window read (2L
        frames), K/V append write (2T), query read + output write (2T), the
        block-table row (4 * (1 + max_pages)) and the two state scalars (16)."""
        sh = self.shape
        s = sh.elem_bytes
        return s * sh.d_model * (2 * sh.window + 2 * sh.chunk + 2 * sh.chunk) + 4 * (1 + self.pool.max_pages) + 16

    def bytes_shared_per_launch(self) -> int:
        """Position-table rows the launch needs (left + 2T - 1) and both biases."""
        sh = self.shape
        s = sh.elem_bytes
        return s * sh.d_model * (sh.left + 2 * sh.chunk - 1) + 2 * s * sh.d_model
