/*
 * parakeet_paged.h -- C ABI of the MI355X (gfx950) paged KV-cache hot path for
 * cache-aware FastConformer streaming.
 *
 * Every entry point takes plain pointers, sizes and element strides; no torch
 * types cross this boundary.  Device pointers are raw HIP device addresses
 * (a torch tensor's data_ptr()), `stream` is a hipStream_t (torch's
 * current_stream().cuda_stream).  Calls return PK_OK (0) or a negative PK_ERR_*
 * code; pk_last_error() then holds a message for the calling thread.  No C++
 * exception crosses the ABI.  The library never allocates device memory and keeps
 * no device pointer past a call.
 *
 * Paged layout shared by the kernels (pk_paged_layout):
 *   k_pool, v_pool : num_layers x num_pages pages of page_size frames x d_model
 *                    elements of `dtype`, contiguous; inside a page the frames
 *                    are stored as column blocks [d_model / CB][page_size][CB],
 *                    CB = gcd(d_model, 64 / element size) (64-byte blocks for
 *                    any d_model of a multiple of 64 bytes), so element (layer,
 *                    page, row r, column c) is at
 *                    ((layer * num_pages + page) * page_size * d_model)
 *                      + (c / CB) * page_size * CB + r * CB + c % CB.
 *   rows           : int32 [batch][rows_stride], one row per stream of the batch:
 *                    rows[b][0]     = frames appended to stream b before this step (A)
 *                    rows[b][1 + r] = page id held in ring entry r, -1 if none,
 *                                     r in [0, max_pages)
 *   Frame position p of a stream (its p-th appended frame) lives in page
 *   rows[b][1 + (p / page_size) % max_pages] at row p % page_size.
 * The dense window a kernel sees for stream b after appending this step's
 * `chunk` frames is positions [A + chunk - window, A + chunk); positions < 0
 * read as zeros (the reference zeroes a slot before use).
 */
#ifndef PARAKEET_PAGED_H
#define PARAKEET_PAGED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_ABI_VERSION 9

enum pk_dtype { PK_DTYPE_F32 = 0, PK_DTYPE_F16 = 1, PK_DTYPE_BF16 = 2 };

#define PK_OK 0
#define PK_ERR_INVALID (-1)     /* bad argument: shape, stride, pointer, range */
#define PK_ERR_UNSUPPORTED (-2) /* valid but not built: e.g. head_dim not 64/128 */
#define PK_ERR_EXHAUSTED (-3)   /* page pool has no page for a reserved slot */
#define PK_ERR_HIP (-4)         /* a HIP runtime call failed */
#define PK_ERR_STATE (-5)       /* call out of order: e.g. a slot twice in one step */

typedef struct pk_paged_layout {
  void* k_pool;
  void* v_pool;
  int32_t num_layers;
  int32_t num_pages;
  int32_t page_size; /* frames per page, power of two */
  int32_t d_model;
  const int32_t* rows;
  int32_t rows_stride; /* int32 elements between consecutive rows */
  int32_t max_pages;   /* ring entries per stream */
} pk_paged_layout;

/* ---------------------------------------------------------------------------
 * pk_kv_append -- write this step's `chunk` new K and V frames of every stream
 * into its pages at positions [A, A + chunk).
 * Replaces ModelCache.update_attn_cache, the tail write
 *   parakeet/modules/cache.py:43-44  (attn_k[:, l, left:].copy_(key), same for V)
 * and, together with the host page pool, the window shift cache.py:37-42.
 * key/value: [batch][chunk][d_model] with element strides (stride_b, stride_t),
 * last dimension contiguous (the views qkv.chunk(3) makes, attention.py:94-95).
 */
typedef struct pk_kv_append_args {
  int32_t dtype;
  int32_t device;
  pk_paged_layout pages;
  int32_t layer;
  int32_t batch;
  int32_t chunk;
  const void* key;
  int64_t key_stride_b;
  int64_t key_stride_t;
  const void* value;
  int64_t value_stride_b;
  int64_t value_stride_t;
} pk_kv_append_args;
int pk_kv_append(const pk_kv_append_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * pk_kv_gather -- materialise the dense window [batch][window][d_model] of K
 * and V from the pages, positions [A + end_offset - window, A + end_offset),
 * zero for positions < 0.  Bit-exact copy of what the reference returns from
 *   parakeet/modules/cache.py:45  (attn_k[:, l], attn_v[:, l])
 * after update_attn_cache when end_offset == chunk.
 */
typedef struct pk_kv_gather_args {
  int32_t dtype;
  int32_t device;
  pk_paged_layout pages;
  int32_t layer;
  int32_t batch;
  int32_t window;
  int32_t end_offset;
  void* out_k;
  int64_t out_k_stride_b;
  int64_t out_k_stride_t;
  void* out_v;
  int64_t out_v_stride_b;
  int64_t out_v_stride_t;
} pk_kv_gather_args;
int pk_kv_gather(const pk_kv_gather_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * pk_paged_relpos_attn -- fused page append + relative-position multi-head
 * attention (Transformer-XL form with pos_bias_u / pos_bias_v) over each
 * stream's window read straight from its pages.
 * Replaces parakeet/modules/attention.py:97-121 (ConformerAttention.forward from
 * update_attn_cache through sdpa_attention_forward, incl. rel_shift :79-83,
 * masked_fill :115 and SDPA :9-20); the qkv / linear_pos / linear_out GEMMs stay
 * with the caller.
 * For query i (0..chunk-1) and window key j (0..window-1, window = left + chunk):
 *   s = ((q_i + u_h).k_j + (q_i + v_h).pos[j + chunk - 1 - i]) / sqrt(head_dim)
 *   s = (q_i + u_h).k_j / sqrt(head_dim) - 1e5          where mask[b,h,i,j] != 0
 *   out_i = sum_j softmax_j(s) v_j            (fp32 accumulation)
 * Keys j >= left are this step's frames, read from key/value; keys j < left come
 * from the pages.  With append != 0 the new frames are also written to the pages
 * (pk_kv_append fused).  left == 0 with k_pool == NULL attends over the chunk only
 * (cache=None in the reference).  Cache policy (no effect on results): when a
 * step's windows, batch * window * d_model * element size * 2 * pages.num_layers
 * bytes, exceed 192 MiB, the page rows are read, and the appends and out written,
 * with the streaming (non-temporal) policy, so a stream of windows larger than
 * the last-level cache does not displace what the step reuses.
 * query/key/value: [batch][chunk][num_heads*head_dim], strides (b, t), last dim
 * contiguous.  pos: [pos_rows][num_heads*head_dim], row stride pos_stride; needs
 * pos_rows >= window + chunk - 1; pos_stride_b != 0 gives every stream its own
 * table, stream b's at pos + b * pos_stride_b (a linear_pos(pos_emb) of batch
 * `batch`, which the reference broadcasts like a batch-1 table,
 * attention.py:102-106).  bias_u/bias_v: [num_heads][head_dim] contiguous.
 * out: [batch][chunk][d_model].
 * The mask comes from one of three sources:
 *   mask != NULL   uint8/bool [batch][heads][chunk][window] with element strides
 *                  (b, h, t) and unit stride along window (mask_stride_h 0
 *                  broadcasts a [batch][chunk][window] mask), 1 = masked -- the
 *                  attn_mask argument of ConformerAttention.forward;
 *   mask == NULL and processed_frames != NULL
 *                  the streaming mask of ConformerEncoder._create_streaming_masks
 *                  (parakeet/modules/encoder.py:167-227) evaluated per score from
 *                  processed_frames / cache_lengths / lengths (int64 [batch], lengths
 *                  NULL -> length_scalar for every stream) and chunk_size
 *                  (att_context_size[1] + 1); bit-identical to pk_streaming_mask for
 *                  0 <= cache_lengths <= left and processed_frames < 2^31;
 *   both NULL      no mask.
 * All floating tensors share `dtype`.  head_dim must be 64 or 128.
 * start_event/stop_event: optional hipEvent_t pair timing this kernel alone.
 * live_streams: optional int32 in device memory.  When set, `batch` is the row
 * count of every batch array (rows, query/key/value, out, mask, state) and only
 * streams 0 .. *live_streams - 1 are attended, appended and written; the count is
 * read when the kernel runs, so one launch recorded in a HIP graph serves a batch
 * whose size changes from step to step (the reference re-packs a batch of the
 * current size every step, scheduler.py:128-170).  NULL: all `batch` streams.
 */
typedef struct pk_attn_args {
  int32_t dtype;
  int32_t device;
  pk_paged_layout pages;
  int32_t layer;
  int32_t batch;
  int32_t chunk;
  int32_t num_heads;
  int32_t head_dim;
  int32_t left;
  int32_t append;
  const void* query;
  int64_t query_stride_b;
  int64_t query_stride_t;
  const void* key;
  int64_t key_stride_b;
  int64_t key_stride_t;
  const void* value;
  int64_t value_stride_b;
  int64_t value_stride_t;
  const void* pos;
  int64_t pos_stride;
  int32_t pos_rows;
  const void* bias_u;
  const void* bias_v;
  const uint8_t* mask;
  int64_t mask_stride_b;
  int64_t mask_stride_h;
  int64_t mask_stride_t;
  const int64_t* processed_frames;
  const int64_t* cache_lengths;
  const int64_t* lengths;
  int64_t length_scalar;
  int32_t chunk_size;
  void* out;
  int64_t out_stride_b;
  int64_t out_stride_t;
  int32_t rows_per_lane; /* kernel choice: 0 = automatic; 4, 5, 9, 12, 18 = the vector-ALU
                            kernel, one wave a workgroup, with that many key rows per
                            lane (automatic fp32 splits a window over 4 waves when the
                            grid is at most two workgroups a CU); fp16/bf16 only:
                            -1 = the two-query matrix-core kernel, -2 = the whole-chunk
                            matrix-core kernel (chunk <= 14, window <= 96; automatic for
                            chunks of 3..14 frames); fp32 ignores negative values */
  void* start_event;
  void* stop_event;
  const int32_t* live_streams;
  int64_t pos_stride_b; /* elements between streams' position tables; 0: one table for all */
} pk_attn_args;
int pk_paged_relpos_attn(const pk_attn_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * pk_streaming_mask -- device-side construction of the streaming attention and
 * padding masks for a batch, bit-exact with the reference's per-stream loop
 *   parakeet/modules/encoder.py:167-227 (ConformerEncoder._create_streaming_masks)
 * att_mask: uint8 [batch][chunk][left + chunk] (1 = masked); pad_mask: uint8
 * [batch][chunk] (1 = padded query).  processed_frames, cache_lengths, lengths:
 * int64 [batch] contiguous device arrays; lengths may be NULL, then every
 * stream uses length_scalar.  chunk_size is att_context_size[1] + 1 and
 * left_chunks = left / chunk_size.  Requires 0 <= cache_lengths <= left (the
 * reference clamps it, encoder.py:260).
 */
typedef struct pk_mask_args {
  int32_t device;
  int32_t batch;
  int32_t chunk;
  int32_t left;
  int32_t chunk_size;
  const int64_t* processed_frames;
  const int64_t* cache_lengths;
  const int64_t* lengths;
  int64_t length_scalar;
  uint8_t* att_mask;
  uint8_t* pad_mask;
} pk_mask_args;
int pk_streaming_mask(const pk_mask_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * pk_conv_step -- one streaming step of the middle of the Conformer convolution
 * module for a batch, with each stream's convolution cache read and written in
 * place:  GLU of the pointwise-conv1 output, padded frames set to zero, causal
 * depthwise convolution over [cache ; this step's frames], LayerNorm over the
 * channels, SiLU.  Replaces, per layer:
 *   parakeet/modules/convolution.py:152-158  (F.glu, masked_fill, depthwise_conv,
 *       batch_norm -- a LayerNorm --, activation);
 *   CausalConv1d.update_cache convolution.py:37-47 (cat of cache and frames; the
 *       next cache is the last kernel-1 frames);
 *   ModelCache.get_conv_cache / update_conv_cache parakeet/modules/cache.py:47-53;
 *   the conv rows of the per-step batch gather / scatter
 *       parakeet/engine/scheduler.py:157-168,193-201 (the cache is addressed
 *       through `slots` instead of being copied in and out of a batch buffer).
 * The two pointwise convolutions (kernel size 1) stay plain GEMMs.
 *
 * glu_in    : [batch][chunk][2*d_model] pointwise-conv1 output, frame-major, element
 *             strides (stride_b, stride_t), channels contiguous; output channel c is
 *             glu_in[..c] * sigmoid(glu_in[..d_model + c]).
 * cache     : [num_slots][num_layers][kernel - 1][d_model] of `dtype`, contiguous;
 *             row r of a stream-layer holds the frame kernel-1-r steps before the
 *             step's first frame (all zeros for a fresh stream, cache.py:30-34).
 *             Stream b uses slot slots[b] (slots NULL: slot b); the slots of one
 *             call must be distinct.
 * pad_mask  : uint8 [batch][chunk] (1 = padded frame), or NULL: then frame t of
 *             stream b is padded when t >= lengths[b] (lengths NULL: length_scalar).
 * dw_weight : [d_model][kernel] (Conv1d weight [d_model][1][kernel]); dw_bias
 *             [d_model] or NULL; ln_weight, ln_bias [d_model]; ln_eps.
 * out       : [batch][chunk][d_model], element strides (stride_b, stride_t).
 * One dtype for every tensor; fp32 arithmetic; the frames written to the cache
 * are the GLU outputs rounded to `dtype`, as the reference's cache holds them.
 * kernel in {3, 5, 7, 9} (the reference models use 9, config.py:13); d_model a
 * multiple of 8 (fp16/bf16) or 4 (fp32), at most 4096 (fp16/bf16) or 2048 (fp32).
 */
typedef struct pk_conv_args {
  int32_t dtype;
  int32_t device;
  int32_t batch;
  int32_t chunk;
  int32_t d_model;
  int32_t kernel;
  const void* glu_in;
  int64_t glu_in_stride_b;
  int64_t glu_in_stride_t;
  void* cache;
  int32_t num_slots;
  int32_t num_layers;
  int32_t layer;
  const int32_t* slots;
  const uint8_t* pad_mask;
  const int64_t* lengths;
  int64_t length_scalar;
  const void* dw_weight;
  const void* dw_bias;
  const void* ln_weight;
  const void* ln_bias;
  float ln_eps;
  void* out;
  int64_t out_stride_b;
  int64_t out_stride_t;
} pk_conv_args;
int pk_conv_step(const pk_conv_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * pk_residual_norm -- a Conformer layer's residual update and the LayerNorm that
 * reads it, for `rows` frames of d_model channels:
 *   residual_out = residual + alpha * branch   (alpha * branch rounded to
 *                  `dtype` first when alpha != 1, then the sum rounded: the two
 *                  roundings of the reference's `residual += x * 0.5`; one
 *                  rounding of `residual += x` when alpha == 1)
 *   norm_out     = LayerNorm(residual_out) * ln_weight + ln_bias  (biased
 *                  variance, fp32 two-pass statistics over the channels of the
 *                  rounded residual_out, each output rounded once)
 * Replaces, per layer, parakeet/modules/encoder.py:61,63,68,70,74,76,78,80: the
 * four `residual += ...` updates, the two `x * 0.5` scalings, and the LayerNorms
 * norm_self_att, norm_conv, norm_feed_forward2 and norm_out that read them.
 * residual, branch, residual_out, norm_out: [rows][d_model] of `dtype` with row
 * strides in elements (channels contiguous, 16-byte aligned rows);
 * residual_out may be residual (updated in place), norm_out may be branch; no
 * other overlap.  ln_weight, ln_bias: [d_model].  d_model a multiple of 8
 * (fp16/bf16) or 4 (fp32), at most 4096 (fp16/bf16) or 2048 (fp32).
 */
typedef struct pk_resnorm_args {
  int32_t dtype;
  int32_t device;
  int32_t rows;
  int32_t d_model;
  float alpha;
  float ln_eps;
  const void* residual;
  int64_t residual_stride;
  const void* branch;
  int64_t branch_stride;
  const void* ln_weight;
  const void* ln_bias;
  void* residual_out;
  int64_t residual_out_stride;
  void* norm_out;
  int64_t norm_out_stride;
} pk_resnorm_args;
int pk_residual_norm(const pk_resnorm_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Pre-encode front end: pcm -> log-mel (pk_fe_step) -> 8x convolution
 * subsampling (pk_subsample), batched over streams whose state lives in device
 * rings addressed by slot.
 *
 * pk_fe_step -- store each stream's new samples in its sample ring and compute
 * the log-mel features of frames [frame0, frame0 + n_frames) into its mel ring.
 * Replaces, per stream and push:
 *   FeatureExtractor.push / _trim_samples parakeet/modules/feature_extractor.py:97-151
 *       (the host keeps the frame counters; the ring replaces the trimmed buffer);
 *   FeatureExtractor._compute_features feature_extractor.py:63-88 (dither,
 *       pre-emphasis, centred STFT with constant padding, power, Slaney mel, log);
 *   the feature half of ModelRunner._run_pre_encode
 *       parakeet/engine/model_runner.py:193-196 and the pcm16 -> float conversion of
 *       parakeet/server.py:442.
 * Frame f of a stream is computed from its global samples as the reference's
 * centred STFT sees them: y[i] = xd[i] - preemph * xd[i-1] (xd[-1] = 0),
 * xd[i] = x[i] + dither * N(i); y[i] = 0 for i < 0 or i >= samples pushed so
 * far; frame f = y[f*hop - n_fft/2 + n] * w[n], the win_length window in the
 * middle of n_fft.  N(i) is a standard normal from Philox4x32-10 with counter
 * (i mod 2^32, i / 2^32, noise_id, 0) and key (seed mod 2^32, seed / 2^32),
 * Box-Muller on the first two words (the reference draws torch.randn per push).
 *
 * streams     : device array [batch] of pk_fe_stream.  The host guarantees for
 *               each stream that sample_base + n_new - (frame0*hop - n_fft/2 +
 *               (n_fft - win)/2 - 1) <= ring_size (every sample a frame reads is
 *               still in the ring and not overwritten by this call) and that
 *               n_frames <= mel_ring_rows; slots of one call are distinct.
 * samples     : new samples of stream b at samples + b*samples_stride, int16 pcm
 *               (value / 32768) or float32, by pcm_dtype.
 * sample_ring : float32 [num_slots][ring_size]; global sample i of a slot at
 *               i mod ring_size.  mel_ring: float32 [num_slots][mel_ring_rows]
 *               [n_mels]; frame f of a slot at row f mod mel_ring_rows.
 * window      : float32 [win_length]; fb: float32 [n_mels][n_fft/2 + 1]; fb_range:
 *               int32 [n_mels][2], the bins [first, end) where row m of fb is not 0.
 * n_fft = 512; win_length <= n_fft; ring_size, mel_ring_rows powers of two;
 * n_mels <= 128; max_new, max_frames bound n_new and n_frames over the batch
 * (they size the grid).  Entries out of these bounds are skipped by the kernel.
 */
enum pk_pcm { PK_PCM_S16 = 0, PK_PCM_F32 = 1 };

typedef struct pk_fe_stream {
  int32_t slot;
  int32_t n_new;
  int64_t sample_base; /* samples pushed to the slot before this call */
  int32_t frame0;
  int32_t n_frames;
  uint32_t noise_id;
  int32_t reserved;
} pk_fe_stream;

typedef struct pk_fe_args {
  int32_t device;
  int32_t batch;
  const pk_fe_stream* streams;
  int32_t pcm_dtype;
  const void* samples;
  int64_t samples_stride;
  float* sample_ring;
  int32_t num_slots;
  int32_t ring_size;
  float* mel_ring;
  int32_t mel_ring_rows;
  int32_t n_mels;
  const float* window;
  int32_t win_length;
  int32_t n_fft;
  int32_t hop;
  const float* fb;
  const int32_t* fb_range;
  float preemph;
  float dither;
  uint64_t seed;
  float log_guard;
  int32_t max_new;
  int32_t max_frames;
} pk_fe_args;
int pk_fe_step(const pk_fe_args* args, void* stream);

/* pk_subsample -- ConvSubsampling's convolution stack for a batch of feature
 * windows: CausalConv2D(1 -> C, 3x3, stride 2) + ReLU, then twice
 * [depthwise CausalConv2D(3x3, stride 2), pointwise 1x1 C -> C, ReLU], with the
 * time masks of MaskedConvSequential, flattened per output frame as
 * [channel][freq] (the input of ConvSubsampling.out).  Replaces
 *   ConvSubsampling.forward / conv_forward parakeet/modules/subsample.py:140-152,177-179
 *       up to `out` (which stays a plain GEMM);
 *   MaskedConvSequential.forward subsample.py:30-57;
 *   CausalConv2D.forward parakeet/modules/convolution.py:94-104;
 *   the window assembly and drop of ModelRunner._run_pre_encode
 *       parakeet/engine/model_runner.py:198-234 (the window is read in place from
 *       the mel ring; the cache is the ring's previous rows).
 * Stream b's window is feature rows row0 .. row0 + rows - 1 of block `slot`
 * (taken mod feat_rows when feat_ring is set); rows >= length are masked; output
 * frames drop .. drop + n_out - 1 of the stack go to rows out_row .. of `out`.
 *
 * feats : float32 [feat_slots][feat_rows][n_mels] (the mel ring, or plain
 *         features); values are rounded to `dtype` on entry.
 * w0,b0 : conv.0 [C][1][3][3], [C];  w2,b2 / w5,b5: depthwise [C][1][3][3], [C];
 * w3,b3 / w6,b6: pointwise [C][C][1][1], [C].  Biases may be NULL.  All of `dtype`.
 * out   : [out_rows][C * F3] of `dtype`, F3 = the frequency size after three
 *         stride-2 convolutions (n_mels -> n_mels/2 + 1, three times).
 * C in {64, 128, 256}; n_mels <= 128; fp32 accumulation, each layer's output
 * rounded to `dtype` as the reference's tensors hold them.
 */
typedef struct pk_sub_stream {
  int32_t slot;
  int32_t row0;
  int32_t rows;
  int32_t length;
  int32_t drop;
  int32_t n_out;
  int32_t out_row;
  int32_t reserved;
} pk_sub_stream;

typedef struct pk_sub_args {
  int32_t dtype;
  int32_t device;
  int32_t batch;
  const pk_sub_stream* streams;
  const float* feats;
  int32_t feat_slots;
  int32_t feat_rows;
  int32_t feat_ring;
  int32_t n_mels;
  int32_t channels;
  const void* w0;
  const void* b0;
  const void* w2;
  const void* b2;
  const void* w3;
  const void* b3;
  const void* w5;
  const void* b5;
  const void* w6;
  const void* b6;
  void* out;
  int32_t out_rows;
  int32_t max_out;
} pk_sub_args;
int pk_subsample(const pk_sub_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * pk_rnnt_greedy_step -- one greedy RNNT decoding step for a batch of streams
 * whose predictor state (LSTM h and c of every layer, and the predictor's joint
 * projection) lives on the device in slots.  For each encoder frame t <
 * lengths[b] and up to max_symbols decisions per frame:
 *   logits = W_out relu(enc_proj[b, t] + pred_proj[slot]) + b_out, each rounded
 *   to `dtype`; the decision is the first maximum.  A blank ends the frame; a
 *   token is appended to tokens[b] and advances the predictor: x = embed[token],
 *   per layer gates = W_ih x + W_hh h + b_ih + b_hh (i, f, g, o),
 *   c' = sig(f) c + sig(i) tanh(g), h' = sig(o) tanh(c') (h', c' rounded to
 *   `dtype`), then pred_proj = W_pred h'_top + b_pred.
 * The whole step is issued from the host with no synchronisation; workgroups
 * whose streams are done for the frame return at once.  Replaces
 *   ModelRunner._decode_batch / _decode_frame_batch / _stack_states /
 *       _unstack_states parakeet/engine/model_runner.py:347-484 (the per-symbol
 *       `.all()` and `.tolist()` synchronisations and the state copies);
 *   Predictor.forward parakeet/modules/decoder.py:44-50 and Joiner.forward
 *       decoder.py:82-86 (dropout is the identity at inference);
 *   with prime != 0: the predictor run on the blank start token from zero state
 *       in ModelRunner.create_sequence model_runner.py:70-77 (no frames are read).
 *
 * slots      : int32 [batch] device, distinct, < num_slots (a stream whose slot
 *              is out of range is treated as absent: no tokens, zero counts,
 *              no state read or written).
 * embed      : [vocab1][hidden] (nn.Embedding, vocab1 = vocabulary + blank).
 * w_ih, w_hh : [layers][4*hidden][hidden]; b_ih, b_hh: [layers][4*hidden]
 *              (nn.LSTM weight_ih_l*, ... stacked over layers).
 * w_pred, b_pred: [joint][hidden], [joint]; w_out, b_out: [vocab1][joint], [vocab1].
 * h, c       : [num_slots][layers][hidden]; pred_proj: [num_slots][joint].
 * enc_proj   : [batch][frames][joint] Joiner.enc of the step's encoder frames,
 *              element strides (stride_b, stride_t), rows 16-byte aligned.
 * lengths    : int32 [batch] frames of each stream (<= max_frames).
 * tokens     : int32 [batch][max_frames * max_symbols] out: the emitted tokens;
 *              frame_counts: int32 [batch][max_frames] out: tokens per frame.
 * compact    : 0 (by batch size: from 1024 streams), 1 or -1.  Compact mode
 *              keeps, per iteration, a device list of the streams that emitted a
 *              token: the next symbol's joint and the LSTM and projection
 *              launches run over that list instead of every 16-stream tile that
 *              holds one such stream (one more small launch per iteration, which
 *              decides and builds the list).  Outputs are the same either way.
 * workspace  : device bytes, at least pk_rnnt_workspace_bytes(...), 16-aligned.
 * One dtype for every floating tensor; fp32 accumulation.  hidden must be 640
 * (both reference models, config.py:19-21); joint a multiple of 64, <= 1024.
 */
typedef struct pk_rnnt_args {
  int32_t dtype;
  int32_t device;
  int32_t batch;
  const int32_t* slots;
  int32_t num_slots;
  int32_t layers;
  int32_t hidden;
  int32_t joint;
  int32_t vocab1;
  int32_t blank;
  int32_t max_symbols;
  int32_t prime;
  const void* embed;
  const void* w_ih;
  const void* w_hh;
  const void* b_ih;
  const void* b_hh;
  const void* w_pred;
  const void* b_pred;
  const void* w_out;
  const void* b_out;
  void* h;
  void* c;
  void* pred_proj;
  const void* enc_proj;
  int64_t enc_stride_b;
  int64_t enc_stride_t;
  const int32_t* lengths;
  int32_t max_frames;
  int32_t compact;  /* 0: by batch size, 1: always, -1: never (see below) */
  int32_t* tokens;
  int32_t* frame_counts;
  void* workspace;
} pk_rnnt_args;
int64_t pk_rnnt_workspace_bytes(int32_t dtype, int32_t batch, int32_t vocab1, int32_t layers, int32_t hidden);
int pk_rnnt_greedy_step(const pk_rnnt_args* args, void* stream);

/* pk_rnnt_greedy_step_static -- pk_rnnt_greedy_step without a workspace
 * argument and without allocating: the step's workspace is a static device
 * array of PK_RNNT_STATIC_SCRATCH_BYTES (8 MiB) that each GPU the library runs
 * on holds until the process ends.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  args->workspace must be NULL; every
 * other argument is pk_rnnt_greedy_step's.  A step whose
 * pk_rnnt_workspace_bytes(...) exceeds the array is rejected with
 * PK_ERR_UNSUPPORTED (at fp16 with one 640-unit LSTM layer, about 5,800
 * streams).  The kernels initialise every scratch word they read, so nothing
 * needs clearing between calls.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, different threads)
 * race and must be serialised by the caller.  The array's address is looked up
 * once per device, outside stream capture: by the first call of either entry
 * point on the device; a first call made under capture is refused
 * (PK_ERR_STATE), so make one eager call before recording steps in a graph. */
#define PK_RNNT_STATIC_SCRATCH_BYTES (8 << 20)
int pk_rnnt_greedy_step_static(const pk_rnnt_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Host page pool: FIFO free-page queue and per-slot page rings.  Thread safe
 * (one internal mutex, the counterpart of Scheduler._state_lock,
 * parakeet/engine/scheduler.py:26,94-97,103-104).  Host memory only.
 *
 * pk_pool_create   -- replaces the slot-pool construction
 *                     parakeet/engine/scheduler.py:68-84 and the dense buffers of
 *                     ModelCache.__init__ parakeet/modules/cache.py:8-34.  Pages are
 *                     handed out in `page_order` (NULL: 0..num_pages-1), freed pages
 *                     go to the back (deque discipline of scheduler.py:84,97,104).
 *                     Requires num_pages >= num_slots * max_pages, so every slot's
 *                     window can always be held (no allocation can fail mid-step).
 * pk_pool_advance  -- opens one step for `n` slots: frees the pages that fell out of
 *                     each window (sliding-window eviction, the shift of
 *                     cache.py:37-42), allocates pages for positions [A, A+chunk),
 *                     writes rows_out[b] = {A, ring[0..max_pages-1]} and advances A by
 *                     chunk.  Slots are processed in the given order.  Replaces the
 *                     per-step batch gather of Scheduler.pack_states
 *                     scheduler.py:128-170 (a block-table row replaces the dense
 *                     state copy).
 * pk_pool_reset_slot / pk_pool_reset_all -- free every page of a slot and set A = 0:
 *                     replaces ModelCache.reset_slot / reset cache.py:55-63 as used
 *                     by Scheduler._reset_state scheduler.py:86-91.
 * pk_pool_slot_info, pk_pool_free_list, pk_pool_free_pages -- inspection for
 *                     parity tests (free queue in FIFO order).
 */
typedef struct pk_pool pk_pool;
int pk_pool_create(int32_t num_pages, int32_t num_slots, int32_t page_size, int32_t left,
                   int32_t chunk, const int32_t* page_order, pk_pool** out);
void pk_pool_destroy(pk_pool* pool);
int pk_pool_max_pages(const pk_pool* pool);
int pk_pool_advance(pk_pool* pool, int32_t n, const int32_t* slots, int32_t* rows_out,
                    int32_t rows_stride);
int pk_pool_reset_slot(pk_pool* pool, int32_t slot);
int pk_pool_reset_all(pk_pool* pool);
int pk_pool_free_pages(const pk_pool* pool);
int pk_pool_slot_info(const pk_pool* pool, int32_t slot, int64_t* appended, int32_t* ring_out);
int pk_pool_free_list(const pk_pool* pool, int32_t* out, int32_t capacity);

/* ---------------------------------------------------------------------------
 * pk_hbm_read_probe -- measurement only; it has no counterpart in the reference.
 * Reads `bytes` (a positive multiple of 16) from the device buffer `src` once,
 * 16 bytes a lane with the streaming cache policy, and writes to out[4 w + x]
 * (16 bytes each, device memory of workgroups * 64 bytes) the XOR of what wave x of
 * workgroup w read, so no read can be dropped.  workgroups: the grid (4 waves of 64
 * lanes each); 0 = 8 per CU.
 * start_event/stop_event: optional hipEvent_t pair timing the launch alone.
 * For a benchmark: the read ceiling of one launch that moves a kernel's bytes.
 */
int pk_hbm_read_probe(const void* src, int64_t bytes, void* out, int32_t workgroups, void* start_event,
                      void* stop_event, void* stream);

/* Message for the last failed call on this thread ("" if none). */
const char* pk_last_error(void);
int pk_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PARAKEET_PAGED_H */
