"""Tensor-level entry points of the paged K/V-cache hot path.

Each function checks shapes, dtypes, devices and strides on the host, then makes
one call into ``libparakeet_paged.so`` on torch's current HIP stream.  Nothing
here computes on the CPU: without the library or a HIP device the call raises.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import AttnArgs, ConvArgs, FeArgs, KvAppendArgs, KvGatherArgs, MaskArgs, PagedLayout, ResNormArgs, SubArgs, check, lib

_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"paged K/V cache supports float32/float16/bfloat16, got {dtype}") from None


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"paged K/V cache kernels run on a HIP device; got a tensor on {dev} "
            "(there is no CPU implementation)"
        )
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _event_handle(ev) -> int:
    """hipEvent_t of a torch.cuda.Event (recorded once, so it exists) or a raw handle."""
    handle = getattr(ev, "cuda_event", ev)
    if not handle:
        raise ValueError("timing event has no handle yet: record it once before use")
    return int(handle)


def _rows3(t: torch.Tensor, name: str, B: int, T: int, D: int, dtype: torch.dtype) -> None:
    if t.dim() != 3 or tuple(t.shape) != (B, T, D):
        raise ValueError(f"{name}: expected shape {(B, T, D)}, got {tuple(t.shape)}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype} != {dtype}")
    if t.stride(2) != 1:
        raise ValueError(f"{name}: last dimension must be contiguous")


def page_column_block(d_model: int, element_size: int) -> int:
    """Columns per page column block: gcd(d_model, 64 bytes of elements)."""
    return math.gcd(d_model, 64 // element_size)


def page_blocks(pool: torch.Tensor) -> torch.Tensor:
    """The element order of a page pool: a [Ly, num_pages, P, D] pool tensor
    holds each page as column blocks of CB = page_column_block(D, element size)
    columns (64 bytes at the model shapes), so page row r, column c of
    (layer, page) is ``page_blocks(pool)[layer, page, c // CB, r, c % CB]``.
    Returns that [Ly, num_pages, D // CB, P, CB] view of the same memory (for
    filling or reading pages directly)."""
    Ly, N, P, D = pool.shape
    cb = page_column_block(D, pool.element_size())
    return pool.view(Ly, N, D // cb, P, cb)


@dataclass
class PagedKV:
    """Device view of a batch's pages: pools of Ly x num_pages pages of P frames
    x D columns (tensors [Ly, num_pages, P, D] whose pages are stored as 64-byte
    column blocks, see page_blocks) and the per-stream rows {A, ring[max_pages]}
    (int32 [B, 1 + max_pages])."""

    k_pool: torch.Tensor
    v_pool: torch.Tensor
    rows: torch.Tensor
    max_pages: int

    def layout(self) -> PagedLayout:
        kp, vp, rows = self.k_pool, self.v_pool, self.rows
        if kp.shape != vp.shape or kp.dim() != 4 or kp.dtype != vp.dtype:
            raise ValueError("k_pool and v_pool must be matching [Ly, num_pages, P, D] tensors")
        if not (kp.is_contiguous() and vp.is_contiguous()):
            raise ValueError("page pools must be contiguous")
        if rows.dtype != torch.int32 or rows.dim() != 2:
            raise ValueError("rows must be int32 [B, 1 + max_pages]")
        if rows.shape[1] < 1 + self.max_pages:
            raise ValueError(f"rows has {rows.shape[1]} columns, needs {1 + self.max_pages}")
        # an empty batch reads no row; torch gives empty tensors arbitrary strides
        empty = rows.shape[0] == 0
        if not empty and rows.stride(1) != 1:
            raise ValueError("rows must have unit inner stride")
        L = PagedLayout()
        L.k_pool = kp.data_ptr()
        L.v_pool = vp.data_ptr()
        L.num_layers, L.num_pages, L.page_size, L.d_model = (int(s) for s in kp.shape)
        L.rows = rows.data_ptr()
        L.rows_stride = 1 + self.max_pages if empty else rows.stride(0)
        L.max_pages = self.max_pages
        return L


def kv_append(pages: PagedKV, layer: int, key: torch.Tensor, value: torch.Tensor) -> None:
    """Writes key/value [B, T, D] into the pages at positions [A, A+T) of each
    row (parakeet/modules/cache.py:43-44)."""
    B, T, D = key.shape
    _rows3(key, "key", B, T, D, pages.k_pool.dtype)
    _rows3(value, "value", B, T, D, pages.k_pool.dtype)
    if pages.rows.shape[0] < B:
        raise ValueError(f"rows covers {pages.rows.shape[0]} streams, batch is {B}")
    dev = _require_device(key, value, pages.k_pool, pages.v_pool, pages.rows)
    a = KvAppendArgs()
    a.dtype = dtype_code(key.dtype)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.pages = pages.layout()
    a.layer, a.batch, a.chunk = int(layer), B, T
    a.key, a.key_stride_b, a.key_stride_t = key.data_ptr(), key.stride(0), key.stride(1)
    a.value, a.value_stride_b, a.value_stride_t = value.data_ptr(), value.stride(0), value.stride(1)
    check(lib().pk_kv_append(ctypes.byref(a), _stream(dev)), "pk_kv_append")


def kv_gather(
    pages: PagedKV,
    layer: int,
    batch: int,
    window: int,
    end_offset: int,
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense window [B, window, D] of positions [A + end_offset - window,
    A + end_offset), zeros before position 0 (parakeet/modules/cache.py:45)."""
    kp = pages.k_pool
    D = kp.shape[3]
    if out_k is None:
        out_k = torch.empty((batch, window, D), dtype=kp.dtype, device=kp.device)
    if out_v is None:
        out_v = torch.empty((batch, window, D), dtype=kp.dtype, device=kp.device)
    _rows3(out_k, "out_k", batch, window, D, kp.dtype)
    _rows3(out_v, "out_v", batch, window, D, kp.dtype)
    if pages.rows.shape[0] < batch:
        raise ValueError(f"rows covers {pages.rows.shape[0]} streams, batch is {batch}")
    dev = _require_device(out_k, out_v, kp, pages.v_pool, pages.rows)
    a = KvGatherArgs()
    a.dtype = dtype_code(kp.dtype)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.pages = pages.layout()
    a.layer, a.batch, a.window, a.end_offset = int(layer), int(batch), int(window), int(end_offset)
    a.out_k, a.out_k_stride_b, a.out_k_stride_t = out_k.data_ptr(), out_k.stride(0), out_k.stride(1)
    a.out_v, a.out_v_stride_b, a.out_v_stride_t = out_v.data_ptr(), out_v.stride(0), out_v.stride(1)
    check(lib().pk_kv_gather(ctypes.byref(a), _stream(dev)), "pk_kv_gather")
    return out_k, out_v


def _mask_strides(mask: torch.Tensor, B: int, H: int, T: int, Lk: int) -> tuple[torch.Tensor, int, int, int]:
    if mask.dtype not in (torch.bool, torch.uint8):
        raise TypeError(f"mask must be bool or uint8, got {mask.dtype}")
    if mask.dim() == 3:
        mask = mask.unsqueeze(1)
    if mask.dim() != 4:
        raise ValueError(f"mask must be [B, T, L] or [B, H, T, L], got {tuple(mask.shape)}")
    mb, mh, mt, ml = mask.shape
    if mb != B or mt != T or ml != Lk or mh not in (1, H):
        raise ValueError(f"mask shape {tuple(mask.shape)} does not broadcast to {(B, H, T, Lk)}")
    if mask.stride(3) != 1:
        mask = mask.contiguous()
    sh = 0 if mh == 1 else mask.stride(1)
    return mask, mask.stride(0), sh, mask.stride(2)


@dataclass
class StreamMaskState:
    """Per-stream streaming state from which the attention kernel evaluates the
    streaming mask of ConformerEncoder._create_streaming_masks
    (parakeet/modules/encoder.py:167-227) score by score, instead of reading a
    materialised [B, T, L] mask.  processed_frames / cache_lengths: int64 [B] on
    the device; lengths: int64 [B] or one int for every stream; chunk_size:
    att_context_size[1] + 1.  Needs 0 <= cache_lengths <= left and
    processed_frames < 2**31."""

    processed_frames: torch.Tensor
    cache_lengths: torch.Tensor
    lengths: torch.Tensor | int
    chunk_size: int

    def check(self, B: int, dev: torch.device) -> None:
        for name, t in (("processed_frames", self.processed_frames), ("cache_lengths", self.cache_lengths)):
            if t.dtype != torch.int64 or tuple(t.shape) != (B,) or not t.is_contiguous() or t.device != dev:
                raise ValueError(f"{name} must be contiguous int64 [{B}] on {dev}")
        if isinstance(self.lengths, torch.Tensor):
            t = self.lengths
            if t.dtype != torch.int64 or tuple(t.shape) != (B,) or not t.is_contiguous() or t.device != dev:
                raise ValueError(f"lengths must be contiguous int64 [{B}] on {dev}")
        if int(self.chunk_size) <= 0:
            raise ValueError("chunk_size must be > 0")


def paged_relpos_attn(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    pos: torch.Tensor,
    bias_u: torch.Tensor,
    bias_v: torch.Tensor,
    mask: torch.Tensor | None,
    *,
    num_heads: int,
    left: int,
    pages: PagedKV | None = None,
    layer: int = 0,
    append: bool = True,
    out: torch.Tensor | None = None,
    rows_per_lane: int = 0,
    mask_state: StreamMaskState | None = None,
    start_event=None,
    stop_event=None,
) -> torch.Tensor:
    """Relative-position MHA of the chunk's queries over each stream's window
    (``left`` cached frames from ``pages`` + this chunk's frames), appending the
    chunk's K/V to the pages when ``append``.  Restates
    parakeet/modules/attention.py:97-121; returns [B, T, D] before linear_out.

    query/key/value: [B, T, D] (views of the qkv projection are fine);
    pos: [>= L + T - 1, D] (linear_pos of the sinusoid slice, batch dim dropped),
    or [B, >= L + T - 1, D]: one table per stream (attention.py:102-106
    broadcasts a pos_emb of batch B the same way);
    bias_u/bias_v: [H, dk]; mask: [B, T, L] / [B, 1|H, T, L] bool, True = masked.
    With ``mask`` None and ``mask_state`` given, the kernel evaluates the
    streaming mask from the stream state instead.
    rows_per_lane: 0 lets the library pick the kernel; 4, 5, 9, 12 or 18 force
    the one-wave vector-ALU kernel with that many key rows per lane (automatic
    fp32 splits each window over 4 waves on small grids); for fp16/bf16, -1 forces
    the two-query matrix-core kernel and -2 the whole-chunk one (chunks of up to
    14 frames over windows of up to 96).
    """
    B, T, D = query.shape
    dt = query.dtype
    _rows3(query, "query", B, T, D, dt)
    _rows3(key, "key", B, T, D, dt)
    _rows3(value, "value", B, T, D, dt)
    H = int(num_heads)
    if D % H != 0:
        raise ValueError(f"d_model {D} not divisible by {H} heads")
    dk = D // H
    Lk = int(left) + T
    pos_sb = 0
    if pos.dim() == 3:
        if pos.shape[0] == 1:
            pos = pos[0]
        elif pos.shape[0] == B:
            pos_sb = pos.stride(0)  # 0 for an expanded table: one table shared by all
            pos = pos[0]
        else:
            raise ValueError(f"pos batch {pos.shape[0]} must be 1 or the query batch {B}")
    if pos.dim() != 2 or pos.shape[1] != D or pos.stride(1) != 1 or pos.dtype != dt:
        raise ValueError(f"pos must be [rows, {D}] or [B, rows, {D}] of {dt} with unit inner stride, "
                         f"got {tuple(pos.shape)} {pos.dtype}")
    for name, bias in (("bias_u", bias_u), ("bias_v", bias_v)):
        if tuple(bias.shape) != (H, dk) or bias.dtype != dt or not bias.is_contiguous():
            raise ValueError(f"{name} must be contiguous [{H}, {dk}] of {dt}")
    tensors = [query, key, value, pos, bias_u, bias_v]
    if pages is not None:
        if pages.k_pool.dtype != dt:
            raise TypeError(f"pages dtype {pages.k_pool.dtype} != {dt}")
        if pages.rows.shape[0] < B:
            raise ValueError(f"rows covers {pages.rows.shape[0]} streams, batch is {B}")
        tensors += [pages.k_pool, pages.v_pool, pages.rows]
    elif left != 0 or append:
        raise ValueError("left > 0 or append needs pages")
    dev = _require_device(*tensors)
    if out is None:
        out = torch.empty((B, T, D), dtype=dt, device=dev)
    _rows3(out, "out", B, T, D, dt)

    a = AttnArgs()
    a.dtype = dtype_code(dt)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    if pages is not None:
        a.pages = pages.layout()
    a.layer, a.batch, a.chunk = int(layer), B, T
    a.num_heads, a.head_dim, a.left, a.append = H, dk, int(left), 1 if append else 0
    a.query, a.query_stride_b, a.query_stride_t = query.data_ptr(), query.stride(0), query.stride(1)
    a.key, a.key_stride_b, a.key_stride_t = key.data_ptr(), key.stride(0), key.stride(1)
    a.value, a.value_stride_b, a.value_stride_t = value.data_ptr(), value.stride(0), value.stride(1)
    a.pos, a.pos_stride, a.pos_rows, a.pos_stride_b = pos.data_ptr(), pos.stride(0), pos.shape[0], pos_sb
    a.bias_u, a.bias_v = bias_u.data_ptr(), bias_v.data_ptr()
    if mask is not None:
        mask, sb, sh, st = _mask_strides(mask, B, H, T, Lk)
        if mask.device != dev:
            raise ValueError("mask on a different device")
        a.mask, a.mask_stride_b, a.mask_stride_h, a.mask_stride_t = mask.data_ptr(), sb, sh, st
    elif mask_state is not None:
        mask_state.check(B, dev)
        a.processed_frames = mask_state.processed_frames.data_ptr()
        a.cache_lengths = mask_state.cache_lengths.data_ptr()
        if isinstance(mask_state.lengths, torch.Tensor):
            a.lengths = mask_state.lengths.data_ptr()
        else:
            a.length_scalar = int(mask_state.lengths)
        a.chunk_size = int(mask_state.chunk_size)
    a.out, a.out_stride_b, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
    a.rows_per_lane = int(rows_per_lane)
    if start_event is not None:
        a.start_event = _event_handle(start_event)
    if stop_event is not None:
        a.stop_event = _event_handle(stop_event)
    check(lib().pk_paged_relpos_attn(ctypes.byref(a), _stream(dev)), "pk_paged_relpos_attn")
    return out


def streaming_mask(
    processed_frames: torch.Tensor,
    cache_lengths: torch.Tensor,
    lengths: torch.Tensor | int,
    *,
    chunk: int,
    left: int,
    chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(pad_mask [B, T], att_mask [B, T, left + T]) bool, as
    ConformerEncoder._create_streaming_masks (parakeet/modules/encoder.py:167-227)."""
    B = int(cache_lengths.shape[0])
    tensors = [processed_frames, cache_lengths]
    for name, t in (("processed_frames", processed_frames), ("cache_lengths", cache_lengths)):
        if t.dtype != torch.int64 or t.shape != (B,) or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous int64 [{B}]")
    if isinstance(lengths, torch.Tensor):
        if lengths.dtype != torch.int64 or lengths.shape != (B,) or not lengths.is_contiguous():
            raise ValueError(f"lengths must be contiguous int64 [{B}]")
        tensors.append(lengths)
    dev = _require_device(*tensors)
    att = torch.empty((B, chunk, left + chunk), dtype=torch.bool, device=dev)
    pad = torch.empty((B, chunk), dtype=torch.bool, device=dev)
    a = MaskArgs()
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.batch, a.chunk, a.left, a.chunk_size = B, int(chunk), int(left), int(chunk_size)
    a.processed_frames = processed_frames.data_ptr()
    a.cache_lengths = cache_lengths.data_ptr()
    if isinstance(lengths, torch.Tensor):
        a.lengths = lengths.data_ptr()
    else:
        a.length_scalar = int(lengths)
    a.att_mask = att.data_ptr()
    a.pad_mask = pad.data_ptr()
    check(lib().pk_streaming_mask(ctypes.byref(a), _stream(dev)), "pk_streaming_mask")
    return pad, att


def hbm_read_probe(src: torch.Tensor, out: torch.Tensor, workgroups: int = 0, start_event=None, stop_event=None) -> None:
    """One launch that reads all of ``src`` once (streaming policy) and writes a
    16-byte XOR per wave to ``out`` (uint8, >= 64 * workgroups bytes): the read
    ceiling of a launch moving that many bytes.  Measurement only."""
    dev = _require_device(src, out)
    if not src.is_contiguous() or not out.is_contiguous():
        raise ValueError("src and out must be contiguous")
    nbytes = src.numel() * src.element_size()
    wg = int(workgroups)
    need = 64 * (wg if wg > 0 else 8 * torch.cuda.get_device_properties(dev).multi_processor_count)
    if out.numel() * out.element_size() < need:
        raise ValueError(f"out holds {out.numel() * out.element_size()} bytes, needs {need}")
    a_ev = _event_handle(start_event) if start_event is not None else None
    b_ev = _event_handle(stop_event) if stop_event is not None else None
    check(lib().pk_hbm_read_probe(src.data_ptr(), nbytes, out.data_ptr(), wg, a_ev, b_ev, _stream(dev)),
          "pk_hbm_read_probe")


def conv_step(
    glu_in: torch.Tensor,
    cache: torch.Tensor,
    dw_weight: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    *,
    layer: int = 0,
    slots: torch.Tensor | None = None,
    pad_mask: torch.Tensor | None = None,
    lengths: torch.Tensor | int | None = None,
    dw_bias: torch.Tensor | None = None,
    eps: float = 1e-5,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One streaming step of the convolution module's middle for a batch:
    SiLU(LayerNorm(depthwise_conv([cache ; mask(GLU(glu_in))]))), with each
    stream's cache updated in place (parakeet/modules/convolution.py:37-47,
    152-157; parakeet/modules/cache.py:47-53).  Returns [B, T, D].

    glu_in: [B, T, 2D] pointwise-conv1 output (channels last, unit inner stride);
    cache: [num_slots, num_layers, K-1, D] contiguous, stream b in slot
    ``slots[b]`` (int32 [B] on the device, distinct values; None: slot b);
    pad_mask: [B, T] bool/uint8 (True = padded) or None, then frames t >=
    ``lengths`` (int64 [B] on the device, or one int; None: no padding) are padded;
    dw_weight: [D, 1, K] or [D, K]; ln_weight/ln_bias: [D]; dw_bias: [D] or None."""
    B, T, D2 = glu_in.shape
    if D2 % 2:
        raise ValueError(f"glu_in has {D2} channels; the GLU needs an even count")
    D = D2 // 2
    dt = glu_in.dtype
    if glu_in.stride(2) != 1:
        raise ValueError("glu_in: last dimension must be contiguous")
    if cache.dim() != 4 or cache.shape[3] != D or cache.dtype != dt or not cache.is_contiguous():
        raise ValueError(f"cache must be contiguous [slots, layers, K-1, {D}] of {dt}, got {tuple(cache.shape)} {cache.dtype}")
    S, Ly, R, _ = (int(x) for x in cache.shape)
    K = R + 1
    w = dw_weight.reshape(dw_weight.shape[0], -1) if dw_weight.dim() == 3 else dw_weight
    if tuple(w.shape) != (D, K) or w.dtype != dt or not w.is_contiguous():
        raise ValueError(f"dw_weight must be contiguous [{D}, 1, {K}] or [{D}, {K}] of {dt}")
    vecs = [("ln_weight", ln_weight), ("ln_bias", ln_bias)] + ([("dw_bias", dw_bias)] if dw_bias is not None else [])
    for name, v in vecs:
        if tuple(v.shape) != (D,) or v.dtype != dt or not v.is_contiguous():
            raise ValueError(f"{name} must be contiguous [{D}] of {dt}")
    tensors = [glu_in, cache, w, ln_weight, ln_bias] + ([dw_bias] if dw_bias is not None else [])
    if slots is not None:
        if slots.dtype != torch.int32 or tuple(slots.shape) != (B,) or not slots.is_contiguous():
            raise ValueError(f"slots must be contiguous int32 [{B}]")
        tensors.append(slots)
    elif B > S:
        raise ValueError(f"batch {B} exceeds {S} cache slots")
    if not 0 <= int(layer) < Ly:
        raise IndexError(f"layer {layer} out of range [0, {Ly})")
    dev = _require_device(*tensors)
    if out is None:
        out = torch.empty((B, T, D), dtype=dt, device=dev)
    _rows3(out, "out", B, T, D, dt)
    a = ConvArgs()
    a.dtype = dtype_code(dt)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.batch, a.chunk, a.d_model, a.kernel = B, T, D, K
    a.glu_in, a.glu_in_stride_b, a.glu_in_stride_t = glu_in.data_ptr(), glu_in.stride(0), glu_in.stride(1)
    a.cache, a.num_slots, a.num_layers, a.layer = cache.data_ptr(), S, Ly, int(layer)
    a.slots = slots.data_ptr() if slots is not None else None
    if pad_mask is not None:
        if pad_mask.dtype not in (torch.bool, torch.uint8) or tuple(pad_mask.shape) != (B, T):
            raise ValueError(f"pad_mask must be bool/uint8 [{B}, {T}]")
        pad_mask = pad_mask.contiguous()
        if pad_mask.device != dev:
            raise ValueError("pad_mask on a different device")
        a.pad_mask = pad_mask.data_ptr()
    elif isinstance(lengths, torch.Tensor):
        if lengths.dtype != torch.int64 or tuple(lengths.shape) != (B,) or not lengths.is_contiguous() or lengths.device != dev:
            raise ValueError(f"lengths must be contiguous int64 [{B}] on {dev}")
        a.lengths = lengths.data_ptr()
    else:
        a.length_scalar = T if lengths is None else int(lengths)
    a.dw_weight = w.data_ptr()
    a.dw_bias = dw_bias.data_ptr() if dw_bias is not None else None
    a.ln_weight, a.ln_bias, a.ln_eps = ln_weight.data_ptr(), ln_bias.data_ptr(), float(eps)
    a.out, a.out_stride_b, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
    check(lib().pk_conv_step(ctypes.byref(a), _stream(dev)), "pk_conv_step")
    return out


def residual_norm(
    residual: torch.Tensor,
    branch: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    *,
    alpha: float = 1.0,
    eps: float = 1e-5,
    in_place: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """A Conformer layer's residual update and the LayerNorm that reads it, in
    one launch (parakeet/modules/encoder.py:61-80): ``r = residual + alpha *
    branch`` (``alpha * branch`` rounded to the dtype first when alpha != 1, as
    ``residual += x * 0.5`` rounds it) and ``LayerNorm(r)`` with ``ln_weight``,
    ``ln_bias`` and ``eps``.  Returns ``(r, norm)``; ``r`` is ``residual``
    itself, updated, when ``in_place``.

    residual, branch: [..., D] of one dtype and shape (``residual`` contiguous
    when ``in_place``); ln_weight, ln_bias: [D] of the same dtype."""
    if residual.shape != branch.shape or residual.dtype != branch.dtype:
        raise ValueError(f"residual {tuple(residual.shape)} {residual.dtype} and branch "
                         f"{tuple(branch.shape)} {branch.dtype} must match")
    D = int(residual.shape[-1])
    dt = residual.dtype
    for name, v in (("ln_weight", ln_weight), ("ln_bias", ln_bias)):
        if tuple(v.shape) != (D,) or v.dtype != dt or not v.is_contiguous():
            raise ValueError(f"{name} must be contiguous [{D}] of {dt}")
    if in_place and not residual.is_contiguous():
        raise ValueError("residual must be contiguous to be updated in place")
    dev = _require_device(residual, branch, ln_weight, ln_bias)
    res = residual.contiguous()
    br = branch.contiguous()
    rout = res if in_place else torch.empty_like(res)
    nout = torch.empty_like(res)
    a = ResNormArgs()
    a.dtype = dtype_code(dt)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.rows = res.numel() // D if D else 0
    a.d_model = D
    a.alpha, a.ln_eps = float(alpha), float(eps)
    a.residual, a.residual_stride = res.data_ptr(), D
    a.branch, a.branch_stride = br.data_ptr(), D
    a.ln_weight, a.ln_bias = ln_weight.data_ptr(), ln_bias.data_ptr()
    a.residual_out, a.residual_out_stride = rout.data_ptr(), D
    a.norm_out, a.norm_out_stride = nout.data_ptr(), D
    check(lib().pk_residual_norm(ctypes.byref(a), _stream(dev)), "pk_residual_norm")
    return rout, nout


# ---------------------------------------------------------------------------
# pre-encode front end


@dataclass
class FeTables:
    """Device constants of one feature extractor (feature_extractor.py:11-57):
    the Hann window, the Slaney filterbank [n_mels, n_fft/2+1] and, per mel
    band, the bin range where its weights are not zero."""

    window: torch.Tensor  # float32 [win_length]
    fb: torch.Tensor  # float32 [n_mels, n_fft//2 + 1]
    fb_range: torch.Tensor  # int32 [n_mels, 2]
    n_fft: int
    hop: int
    preemph: float
    log_guard: float

    @property
    def n_mels(self) -> int:
        return int(self.fb.shape[0])


def _check_f32(t: torch.Tensor, name: str, dim: int) -> None:
    if t.dtype != torch.float32 or t.dim() != dim or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor with {dim} dimensions")


def fe_step(
    streams: torch.Tensor,
    batch: int,
    samples: torch.Tensor | None,
    sample_ring: torch.Tensor,
    mel_ring: torch.Tensor,
    tables: FeTables,
    *,
    dither: float,
    seed: int,
    max_new: int,
    max_frames: int,
) -> None:
    """Stores new samples and writes the log-mel frames of ``batch`` streams
    (pk_fe_step; feature_extractor.py:63-151).  ``streams``: device bytes
    holding ``batch`` pk_fe_stream records; ``samples``: [batch, >= max_new]
    int16 pcm or float32 (None when max_new == 0); rings: float32 [S, R] and
    [S, M, n_mels]."""
    _check_f32(sample_ring, "sample_ring", 2)
    _check_f32(mel_ring, "mel_ring", 3)
    S, R = (int(x) for x in sample_ring.shape)
    if mel_ring.shape[0] != S or mel_ring.shape[2] != tables.n_mels:
        raise ValueError(f"mel_ring must be [{S}, rows, {tables.n_mels}]")
    nb = tables.n_fft // 2 + 1
    if tables.fb.dtype != torch.float32 or tables.fb.dim() != 2 or tables.fb.shape[1] != nb or not tables.fb.is_contiguous():
        raise ValueError(f"fb must be contiguous float32 [n_mels, {nb}]")
    if tables.fb_range.dtype != torch.int32 or tuple(tables.fb_range.shape) != (tables.n_mels, 2) or not tables.fb_range.is_contiguous():
        raise ValueError(f"fb_range must be contiguous int32 [{tables.n_mels}, 2]")
    if tables.window.dtype != torch.float32 or tables.window.dim() != 1 or not tables.window.is_contiguous():
        raise ValueError("window must be a contiguous float32 vector")
    tensors = [streams, sample_ring, mel_ring, tables.window, tables.fb, tables.fb_range]
    a = FeArgs()
    if samples is not None:
        if samples.dim() != 2 or samples.stride(1) != 1 or samples.shape[0] < batch:
            raise ValueError("samples must be [batch, n] with unit inner stride")
        if samples.dtype == torch.int16:
            a.pcm_dtype = _lib.PCM_S16
        elif samples.dtype == torch.float32:
            a.pcm_dtype = _lib.PCM_F32
        else:
            raise TypeError(f"samples must be int16 pcm or float32, got {samples.dtype}")
        if samples.shape[1] < max_new:
            raise ValueError(f"samples has {samples.shape[1]} columns < max_new {max_new}")
        a.samples, a.samples_stride = samples.data_ptr(), samples.stride(0)
        tensors.append(samples)
    else:
        if max_new:
            raise ValueError("max_new > 0 needs samples")
        a.pcm_dtype, a.samples_stride = _lib.PCM_F32, 0
    if streams.dtype != torch.uint8 or streams.numel() < 32 * batch:
        raise ValueError("streams must hold batch x 32 bytes of pk_fe_stream records")
    dev = _require_device(*tensors)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.batch, a.streams = int(batch), streams.data_ptr()
    a.sample_ring, a.num_slots, a.ring_size = sample_ring.data_ptr(), S, R
    a.mel_ring, a.mel_ring_rows, a.n_mels = mel_ring.data_ptr(), int(mel_ring.shape[1]), tables.n_mels
    a.window, a.win_length = tables.window.data_ptr(), int(tables.window.shape[0])
    a.n_fft, a.hop = tables.n_fft, tables.hop
    a.fb, a.fb_range = tables.fb.data_ptr(), tables.fb_range.data_ptr()
    a.preemph, a.dither, a.seed, a.log_guard = tables.preemph, float(dither), int(seed) & (2**64 - 1), tables.log_guard
    a.max_new, a.max_frames = int(max_new), int(max_frames)
    check(lib().pk_fe_step(ctypes.byref(a), _stream(dev)), "pk_fe_step")


SUB_KEYS = ("conv.0", "conv.2", "conv.3", "conv.5", "conv.6")


def subsample(
    streams: torch.Tensor,
    batch: int,
    feats: torch.Tensor,
    ring: bool,
    weights: dict,
    out: torch.Tensor,
    *,
    max_out: int,
) -> torch.Tensor:
    """ConvSubsampling's convolution stack for ``batch`` windows (pk_subsample;
    subsample.py:30-57,140-152).  ``feats``: float32 [slots, rows, n_mels];
    ``weights``: {"conv.0.weight": [C,1,3,3], "conv.0.bias": [C] or None, ...}
    for conv.0/2/3/5/6 in the model dtype; ``out``: [rows_out, C * F3]."""
    _check_f32(feats, "feats", 3)
    w0 = weights["conv.0.weight"]
    dt, C = w0.dtype, int(w0.shape[0])
    F = int(feats.shape[2])
    F3 = ((F // 2 + 1) // 2 + 1) // 2 + 1
    shapes = {"conv.0": (C, 1, 3, 3), "conv.2": (C, 1, 3, 3), "conv.3": (C, C, 1, 1), "conv.5": (C, 1, 3, 3), "conv.6": (C, C, 1, 1)}
    a = SubArgs()
    tensors = [streams, feats, out]
    for key in SUB_KEYS:
        w, bias = weights[key + ".weight"], weights.get(key + ".bias")
        if tuple(w.shape) != shapes[key] or w.dtype != dt or not w.is_contiguous():
            raise ValueError(f"{key}.weight must be contiguous {shapes[key]} of {dt}")
        if bias is not None and (tuple(bias.shape) != (C,) or bias.dtype != dt or not bias.is_contiguous()):
            raise ValueError(f"{key}.bias must be contiguous [{C}] of {dt}")
        n = key.split(".")[1]
        setattr(a, "w" + n, w.data_ptr())
        setattr(a, "b" + n, bias.data_ptr() if bias is not None else None)
        tensors += [w] + ([bias] if bias is not None else [])
    if out.dim() != 2 or out.shape[1] != C * F3 or out.dtype != dt or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [rows, {C * F3}] of {dt}")
    if streams.dtype != torch.uint8 or streams.numel() < 32 * batch:
        raise ValueError("streams must hold batch x 32 bytes of pk_sub_stream records")
    dev = _require_device(*tensors)
    a.dtype = dtype_code(dt)
    a.device = dev.index if dev.index is not None else torch.cuda.current_device()
    a.batch, a.streams = int(batch), streams.data_ptr()
    a.feats, a.feat_slots, a.feat_rows, a.feat_ring = feats.data_ptr(), int(feats.shape[0]), int(feats.shape[1]), int(bool(ring))
    a.n_mels, a.channels = F, C
    a.out, a.out_rows, a.max_out = out.data_ptr(), int(out.shape[0]), int(max_out)
    check(lib().pk_subsample(ctypes.byref(a), _stream(dev)), "pk_subsample")
    return out
