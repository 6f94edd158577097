"""Drop-in for the streaming parts of ``parakeet.modules.encoder``
(parakeet/modules/encoder.py).

* ``init_streaming_state`` builds the paged :class:`ModelCache`
  (encoder.py:140-165);
* ``_create_streaming_masks`` is one HIP launch for the whole batch instead of
  a per-stream Python loop with two device->host syncs per stream
  (encoder.py:167-227);
* ``forward`` keeps the layer loop and the state advance (encoder.py:229-267);
  the attention of every layer runs on the paged cache;
* ``EncoderStepGraph`` replays a recorded step for a fixed batch: the about 20
  launches per layer that ``forward`` issues from Python become one HIP graph
  replay, with the host page work and one upload per step left outside it.

The convolution module's GLU / depthwise conv / LayerNorm / SiLU runs as one HIP
launch with each stream's conv state updated in place (convolution.py:107-162,
cache.py:47-53); the feed-forward blocks, layer norms and pointwise projections
are torch modules with the reference's parameter names (encoder.py:11-81,
feedforward.py:4-26).  ``pre_encode`` is the batched convolution subsampling of
``modules/frontend.py`` (one HIP launch for the 8x stack), built from the same
constructor arguments as the reference's (encoder.py:105-112), so a reference
checkpoint loads strictly and ``ModelRunner`` finds ``encoder.pre_encode``
(model_runner.py:44,221).
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from .. import ops
from .attention import ConformerAttention, PositionalEncoding
from .cache import ConvCacheRef, ModelCache, StreamingState
from .frontend import ConvSubsampling


class ConformerFeedForward(nn.Module):
    def __init__(self, hidden_size: int, d_ff: int, dropout: float, use_bias: bool = True):
        super().__init__()
        self.d_model = hidden_size
        self.d_ff = d_ff
        self.use_bias = use_bias
        self.linear1 = nn.Linear(hidden_size, d_ff, bias=use_bias)
        self.activation = nn.SiLU()
        self.linear2 = nn.Linear(d_ff, hidden_size, bias=use_bias)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: Tensor) -> Tensor:
        return self.linear2(self.dropout(self.activation(self.linear1(x))))


class CausalConv1d(nn.Conv1d):
    """Depthwise conv whose left context comes from a per-stream cache of
    kernel_size-1 frames (parakeet/modules/convolution.py:8-52); holds the
    parameters, the step itself runs in ConformerConvolution."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=(0, 0), dilation=1, groups=1, bias=True):
        self._left_padding = padding[0]
        self._right_padding = padding[1]
        super().__init__(in_channels, out_channels, kernel_size, stride=stride, padding=0, dilation=dilation, groups=groups, bias=bias)


class ConformerConvolution(nn.Module):
    """pointwise conv -> [GLU -> pad mask -> causal depthwise conv with the
    stream's cache -> LayerNorm -> SiLU] -> pointwise conv
    (parakeet/modules/convolution.py:107-162).  The bracket is one HIP launch
    (``pk_conv_step``); the pointwise convolutions (kernel size 1) are matrix
    products.  ``cache`` is the reference's [B, D, kernel-1] state (a new state is
    returned), None (zeros), or a ``ConvCacheRef`` from ``ModelCache.conv_ref``
    (the batch's state is updated in place and None is returned)."""

    def __init__(self, hidden_size, kernel_size, use_bias=False):
        super().__init__()
        self.d_model = hidden_size
        self.kernel_size = kernel_size
        self.pointwise_conv1 = nn.Conv1d(hidden_size, hidden_size * 2, kernel_size=1, bias=use_bias)
        self.depthwise_conv = CausalConv1d(
            hidden_size, hidden_size, kernel_size, groups=hidden_size, padding=(kernel_size - 1, 0), bias=use_bias
        )
        self.batch_norm = nn.LayerNorm(hidden_size)
        self.activation = nn.SiLU()
        self.pointwise_conv2 = nn.Conv1d(hidden_size, hidden_size, kernel_size=1, bias=use_bias)

    def _middle(self, h: Tensor, pad_mask: Tensor | None, frames: Tensor, layer: int = 0, slots=None) -> Tensor:
        dw = self.depthwise_conv
        return ops.conv_step(
            h,
            frames,
            dw.weight,
            self.batch_norm.weight,
            self.batch_norm.bias,
            layer=layer,
            slots=slots,
            pad_mask=pad_mask,
            dw_bias=dw.bias,
            eps=self.batch_norm.eps,
        )

    def forward(self, x: Tensor, pad_mask: Tensor, cache=None):
        h = F.linear(x, self.pointwise_conv1.weight.squeeze(-1), self.pointwise_conv1.bias)
        if isinstance(cache, ConvCacheRef):
            bn, dw = self.batch_norm, self.depthwise_conv
            y = cache.cache.conv_step(cache.layer_idx, h, pad_mask, dw.weight, dw.bias, bn.weight, bn.bias, bn.eps)
            new_cache = None
        else:
            B, K = x.shape[0], self.kernel_size
            if cache is None:
                frames = torch.zeros((B, 1, K - 1, self.d_model), dtype=x.dtype, device=x.device)
            else:
                frames = cache.transpose(1, 2).unsqueeze(1).contiguous()
            y = self._middle(h, pad_mask, frames)
            new_cache = frames[:, 0].transpose(1, 2)
        out = F.linear(y, self.pointwise_conv2.weight.squeeze(-1), self.pointwise_conv2.bias)
        return out, new_cache


class ConformerLayer(nn.Module):
    """FF/2 -> rel-pos MHA -> conv -> FF/2 -> LN (parakeet/modules/encoder.py:11-81)."""

    def __init__(self, layer_idx, hidden_size, d_ff, num_heads, dropout, conv_kernel_size, use_bias):
        super().__init__()
        self.layer_idx = layer_idx
        self.hidden_size = hidden_size
        self.norm_feed_forward1 = nn.LayerNorm(hidden_size)
        self.feed_forward1 = ConformerFeedForward(hidden_size, d_ff, dropout, use_bias)
        self.norm_conv = nn.LayerNorm(hidden_size)
        self.conv = ConformerConvolution(hidden_size, conv_kernel_size)
        self.norm_self_att = nn.LayerNorm(hidden_size)
        self.self_attn = ConformerAttention(layer_idx=layer_idx, hidden_size=hidden_size, num_heads=num_heads, use_bias=use_bias)
        self.norm_feed_forward2 = nn.LayerNorm(hidden_size)
        self.feed_forward2 = ConformerFeedForward(hidden_size, d_ff, dropout, use_bias)
        self.norm_out = nn.LayerNorm(hidden_size)

    def forward(self, x: Tensor, pos_emb: Tensor, pad_mask: Tensor, attn_mask: Tensor, cache: ModelCache):
        # each residual update and the LayerNorm that reads it are one step
        # (``residual_norm``); the layer's input is not modified
        residual, h = self.residual_norm(x, self.feed_forward1(self.norm_feed_forward1(x)), self.norm_self_att, 0.5)
        attn = self.self_attn(h, pos_emb, attn_mask=attn_mask, cache=cache)
        residual, h = self.residual_norm(residual, attn, self.norm_conv, 1.0, in_place=True)
        conv_out, conv_cache = self.conv(h, pad_mask=pad_mask, cache=cache.conv_ref(self.layer_idx))
        cache.update_conv_cache(self.layer_idx, conv_cache)
        residual, h = self.residual_norm(residual, conv_out, self.norm_feed_forward2, 1.0, in_place=True)
        _, out = self.residual_norm(residual, self.feed_forward2(h), self.norm_out, 0.5, in_place=True)
        return out

    @staticmethod
    def residual_norm(residual: Tensor, branch: Tensor, norm: nn.LayerNorm, alpha: float, in_place: bool = False):
        """``residual += alpha * branch`` and ``norm(residual)`` (encoder.py:61-80),
        one HIP launch: returns the updated residual (``residual`` itself when
        ``in_place``) and its norm."""
        return ops.residual_norm(residual, branch, norm.weight, norm.bias, alpha=alpha, eps=norm.eps, in_place=in_place)


class ConformerEncoder(nn.Module):
    """Streaming FastConformer encoder stack on the paged cache
    (parakeet/modules/encoder.py:84-267); same constructor arguments."""

    def __init__(
        self,
        feat_in: int,
        hidden_size,
        ff_expansion_factor: int,
        num_layers: int,
        num_heads: int,
        subsampling_factor: int,
        pos_emb_max_len: int,
        conv_kernel_size: int,
        att_context_size,
        subsampling_conv_channels: int,
        use_bias: bool,
        pre_encode_cache_size: list | tuple = (0, 9),
        drop_extra_pre_encoded: int = 2,
        page_size: int = 16,
    ):
        super().__init__()
        self.embed_dim = hidden_size
        self.feat_in = feat_in
        self.subsampling_factor = subsampling_factor
        self.pre_encode = ConvSubsampling(
            hidden_size=hidden_size,
            subsampling_conv_channels=subsampling_conv_channels,
            feat_in=feat_in,
            subsampling_factor=subsampling_factor,
            stride=2,
            kernel_size=3,
        )
        self.pos_enc = PositionalEncoding(hidden_size=hidden_size, dropout_rate_emb=0.0, max_len=pos_emb_max_len, dropout=0.0)
        self.layers = nn.ModuleList(
            ConformerLayer(i, hidden_size, hidden_size * ff_expansion_factor, num_heads, 0.0, conv_kernel_size, use_bias)
            for i in range(num_layers)
        )
        self.pos_enc.extend_pe(pos_emb_max_len, device=next(self.parameters()).device)
        self.att_context_size = list(att_context_size)
        self.conv_kernel_size = conv_kernel_size
        self.pre_encode_cache_size = pre_encode_cache_size
        self.drop_extra_pre_encoded = drop_extra_pre_encoded
        self.page_size = page_size

    def init_streaming_state(
        self,
        batch_size: int = 1,
        device: torch.device | None = None,
        dtype: torch.dtype | None = None,
        **cache_kwargs,
    ) -> StreamingState:
        if device is None:
            device = next(self.parameters()).device
        if dtype is None:
            dtype = next(self.parameters()).dtype
        cache_kwargs.setdefault("page_size", self.page_size)
        cache = ModelCache(
            num_layers=len(self.layers),
            attn_context_size=self.att_context_size,
            embed_dim=self.embed_dim,
            conv_kernel_size=self.conv_kernel_size,
            batch_size=batch_size,
            device=device,
            dtype=dtype,
            **cache_kwargs,
        )
        return StreamingState(
            cache=cache,
            processed_frames=torch.zeros(batch_size, dtype=torch.int64, device=device),
            cache_lengths=torch.zeros(batch_size, dtype=torch.int64, device=device),
        )

    def _create_streaming_masks(
        self,
        current_len: int,
        cache_lengths: Tensor,
        processed_frames: Tensor,
        device: torch.device,
        lengths: Tensor | int,
    ):
        """(pad_mask [B, T], att_mask [B, T, left+T]) from one kernel launch."""
        batch = cache_lengths.shape[0]

        def as_state(v):
            if isinstance(v, Tensor):
                return v.to(device=device, dtype=torch.int64).contiguous()
            return torch.full((batch,), int(v), dtype=torch.int64, device=device)

        if lengths is None:
            raise ValueError("lengths is required (the reference compares against it, encoder.py:204)")
        lengths = as_state(lengths) if isinstance(lengths, Tensor) else int(lengths)
        return ops.streaming_mask(
            as_state(processed_frames),
            as_state(cache_lengths),
            lengths,
            chunk=current_len,
            left=self.att_context_size[0],
            chunk_size=self.att_context_size[1] + 1,
        )

    def forward(self, x: Tensor, state: StreamingState, length: Tensor | None = None, bypass_pre_encode: bool = False):
        cache_lengths = state.cache_lengths
        if not isinstance(cache_lengths, Tensor):
            cache_lengths = torch.full((x.size(0),), int(cache_lengths), dtype=torch.int64, device=x.device)
        processed = state.processed_frames
        if not isinstance(processed, Tensor):
            processed = torch.full((x.size(0),), int(processed), dtype=torch.int64, device=x.device)
        x, pos_emb = self.pos_enc(x, cache_len=self.att_context_size[0])
        pad_mask, att_mask = self._create_streaming_masks(
            current_len=x.size(1),
            cache_lengths=cache_lengths,
            processed_frames=processed,
            device=x.device,
            lengths=length,
        )
        for layer in self.layers:
            x = layer(x, pos_emb=pos_emb, pad_mask=pad_mask, attn_mask=att_mask, cache=state.cache)
        if isinstance(length, Tensor):
            state.processed_frames.add_(length)
            state.cache_lengths.add_(length)
            state.cache_lengths.clamp_(max=self.att_context_size[0])
        else:
            state.processed_frames += x.size(1)
            state.cache_lengths = min(int(state.cache_lengths) + x.size(1), self.att_context_size[0])
        return x.transpose(1, 2), state


class EncoderStepGraph:
    """``encoder(x, state, length)`` for a fixed batch, recorded once in a HIP
    graph and replayed every step (the call ModelRunner._encode_step makes,
    parakeet/engine/model_runner.py:285-291, with whole chunks).

    Every launch of a step reads the same device memory each step: the page
    pools, the batch's block-table rows, the state counters, the conv state, the
    position table and the weights; only their contents change.  A call runs
    ``state.cache.open_step()`` (the host page work and the one upload of the
    batch's rows), copies ``x`` into a fixed input buffer and replays.  The first
    call runs the step eagerly -- its real work, which also initialises the
    libraries' handles -- and then records the step without running it.

    ``length`` is the per-stream frame count of every step ([B] int64; the engine
    feeds whole chunks, parakeet/engine/sequence.py:137-146).  The returned
    [B, D, T] tensor is a fixed buffer that the next call overwrites.
    """

    def __init__(self, encoder: ConformerEncoder, state: StreamingState, length: Tensor):
        cache = state.cache
        if not isinstance(cache, ModelCache):
            raise TypeError("state.cache must be the paged ModelCache")
        for name in ("processed_frames", "cache_lengths"):
            if not isinstance(getattr(state, name), Tensor):
                raise TypeError(f"state.{name} must be a device tensor (a recorded step advances it on the device)")
        B = cache.batch_size
        dev = cache.k_pages.device
        if not isinstance(length, Tensor) or tuple(length.shape) != (B,):
            raise ValueError(f"length must be a [{B}] tensor")
        self.encoder = encoder
        self.state = state
        self.length = length.to(device=dev, dtype=torch.int64).clone()
        self.shape = (B, cache.chunk, encoder.embed_dim)
        self.x: Tensor | None = None
        self.out: Tensor | None = None
        self.graph: torch.cuda.CUDAGraph | None = None

    def __call__(self, x: Tensor) -> Tensor:
        if tuple(x.shape) != self.shape:
            raise ValueError(f"x must be {self.shape}, got {tuple(x.shape)}")
        cache = self.state.cache
        cache.open_step()
        if self.graph is None:
            self.x = x.detach().clone()
            out, _ = self.encoder(self.x, self.state, length=self.length)
            graph = torch.cuda.CUDAGraph()
            with cache.recording(), torch.cuda.graph(graph):
                self.out, _ = self.encoder(self.x, self.state, length=self.length)
            self.graph = graph
            return out
        self.x.copy_(x)
        for layer in self.encoder.layers:  # the recording reads the kept position projections
            layer.self_attn.refresh_projected_pos()
        self.graph.replay()
        return self.out


__all__ = [
    "ConformerEncoder",
    "ConformerLayer",
    "ConformerConvolution",
    "ConformerFeedForward",
    "CausalConv1d",
    "EncoderStepGraph",
]
