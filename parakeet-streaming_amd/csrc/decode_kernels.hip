// gfx950 kernels of batched RNNT greedy decoding with the predictor state of
// every stream on the device (parakeet/engine/model_runner.py:306-447,
// parakeet/modules/decoder.py:5-86).
//
// One decode step for a batch runs, for each encoder frame t and each symbol
// s < max_symbols, 2 + layers launches with no host synchronisation:
//   joint_kernel     hid = relu(enc_proj[b, t] + pred_proj[slot]) (rounded to the
//                    storage type), logits = W_out hid + b_out (rounded), and the
//                    first maximum over a tile of 64 vocabulary rows: MFMA with
//                    the weight rows as A and the 16 streams as B columns.
//                    Workgroups whose streams are all done for the frame return
//                    at once -- the reference's "every decision blank" break.
//   lstm_kernel      layer 0 first takes the first maximum over the tiles (the
//                    decision; column 0 of the grid records it: a blank ends the
//                    stream's frame, a token is appended); per layer: gates =
//                    W_ih x + W_hh h + b_ih + b_hh as MFMA over K = [x ; h] (x =
//                    embedding of the token, or the layer below), then c' = sig(f)
//                    c + sig(i) tanh(g), h' = sig(o) tanh(c') for 16 hidden units x
//                    SPW streams per workgroup; other streams keep their state.
//                    Every workgroup reads all of a stream's h, so h' goes to a
//                    per-batch scratch; c is owned by one thread per element.
//   pred_kernel      pred_proj[slot] = W_pred h'_top + b_pred for the updated
//                    streams, and h' copied from the scratch into the slot state,
//                    a share by every workgroup (this launch runs after every
//                    read of the old h).
// In compact mode (large batches) a select_kernel launch after the joint takes
// every stream's decision, records it and lists the streams that emitted a
// token; the LSTM and pred launches, and the next symbol's joint, then tile over
// that list instead of the whole batch.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "pk_common.h"
#include "pk_device.h"

namespace pk {

template <typename ST>
struct MmaR;
template <>
struct MmaR<_Float16> {
  typedef _Float16 H8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4_t step(u32x4 a, u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(H8, a), __builtin_bit_cast(H8, b), c, 0,
                                                  0, 0);
  }
};
template <>
struct MmaR<bf16_t> {
  typedef __bf16 H8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4_t step(u32x4 a, u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(H8, a), __builtin_bit_cast(H8, b), c, 0,
                                                   0, 0);
  }
};
template <>
struct MmaR<float> {
  __device__ static inline f32x4_t step(u32x4 a, u32x4 b, f32x4_t c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    return c;
  }
};

// Workgroup sizes of the joint and pred launches: more, smaller workgroups
// than one per 128 rows, so that a launch spreads its weight reads over more
// CUs (at 128 streams the joint then takes 136 workgroups, the pred 160).
constexpr int kVT = 64;                // vocabulary rows per joint workgroup
constexpr int kJointWaves = kVT / 16;  // a wave per 16 rows
constexpr int kPredWaves = 2;          // pred_proj columns per workgroup: 16 a wave
constexpr int kCompactMinBatch = 1024;  // compact mode by default from this batch
constexpr int kMaxDim = 1024;  // hidden / joint sizes held in LDS
// per-stream words of the step workspace: flag, token, emitted count, pad
constexpr int kWsHead = 4;

struct DecK {
  int32_t batch, num_slots, layers, H, J, V1, blank, max_symbols, t, s, vtiles, max_frames;
  const int32_t* slots;
  const int32_t* lengths;
  const void* embed;
  const void *w_ih, *w_hh, *b_ih, *b_hh;
  const void *w_pred, *b_pred, *w_out, *b_out;
  void* h;   // [num_slots][layers][H]
  void* hn;  // [batch][layers][H] scratch: this iteration's new h
  void* c;
  void* pred_proj;  // [num_slots][J]
  const void* enc;  // [batch][.. frames][J] enc projections
  int64_t enc_sb, enc_st;
  int32_t* tokens;        // [batch][max_frames * max_symbols]
  int32_t* frame_counts;  // [batch][max_frames]
  int32_t* ws;            // [batch][kWsHead + 2 * vtiles]
  int32_t layer;
  int32_t prime;
  // compact mode: list[i & 1] holds the streams that emitted a token in
  // iteration i = t * max_symbols + s, count[i & 1] their number
  int32_t* alist;   // [2][batch]
  int32_t* acount;  // [2]
  int32_t compact;
  int32_t it;
};

// stream state words in the workspace
__device__ static inline int32_t* ws_of(const DecK& p, int b) { return p.ws + (int64_t)b * (kWsHead + 2 * p.vtiles); }

// Stream b is in the batch and its slot addresses the state arrays.  A slot
// outside them is a caller error the host wrapper rejects; the kernels treat such
// a stream as absent (no tokens, no state read or written) rather than address
// outside the state.
__device__ static inline bool stream_ok(const DecK& p, int b) {
  return b < p.batch && (uint32_t)p.slots[b] < (uint32_t)p.num_slots;
}


// Entry e of a launch's stream set: the batch itself (list < 0), or list
// `list` of the streams that emitted a token; -1 past the set.
__device__ static inline int listed_stream(const DecK& p, int list, int e) {
  if (e >= p.batch) return -1;
  if (list < 0) return e;
  if (e >= min(p.acount[list], p.batch)) return -1;
  const int b = p.alist[(int64_t)list * p.batch + e];
  return (uint32_t)b < (uint32_t)p.batch ? b : -1;
}

// Weight chunks loaded ahead of their MFMAs: 10 k-steps per round trip.  A
// workgroup of 4-8 waves then has 40-80 KB of weights in flight; with twice
// that in flight a round trip took about four times as long.
template <typename ST>
struct KChunk {
  static constexpr int CH = 10;
};

// The wave's 16 weight rows (A, from global memory) against 16 columns held in
// LDS (B), over nk k-steps of 4*VEC elements.  Rows are read from `wa` for
// k-steps [0, ka) and from `wb` (at k-step - ka) after it; the LDS column runs
// contiguously over all nk k-steps.  Weights move in chunks of CH k-steps whose
// loads are all issued before the chunk's first MFMA (the index clamped, so
// every load is valid): a wave waits for one L2 round trip per CH k-steps rather
// than one per k-step.  The k-steps accumulate in order, as a plain loop would.
template <typename ST, int CH>
__device__ static inline void load_chunk(u32x4 (&w)[CH], const ST* wa, const ST* wb, int ka, int nk, int k0, int lg) {
  constexpr int VEC = 16 / sizeof(ST);
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int kk = min(k0 + u, nk - 1);
    const ST* src = kk < ka ? wa + kk * 4 * VEC : wb + (kk - ka) * 4 * VEC;
    w[u] = ld16(src + VEC * lg);
  }
}

template <typename ST, int CH>
__device__ static inline f32x4_t mma_chunk(const u32x4 (&w)[CH], const ST* col, int k0, int nk, int lg, f32x4_t d) {
  constexpr int VEC = 16 / sizeof(ST);
#pragma unroll
  for (int u = 0; u < CH; ++u)
    if (k0 + u < nk) d = MmaR<ST>::step(w[u], *reinterpret_cast<const u32x4*>(col + (k0 + u) * 4 * VEC + VEC * lg), d);
  return d;
}

// d += the product, with the first chunk's weights already loaded into w0 (its
// loads issued early, so their round trip overlaps the caller's other loads).
template <typename ST, int CH>
__device__ static inline f32x4_t mma_rows(const u32x4 (&w0)[CH], const ST* wa, const ST* wb, int ka, int nk,
                                          const ST* col, int lg, f32x4_t d) {
  d = mma_chunk<ST>(w0, col, 0, nk, lg, d);
  for (int k0 = CH; k0 < nk; k0 += CH) {
    u32x4 w[CH];
    load_chunk<ST>(w, wa, wb, ka, nk, k0, lg);
    __builtin_amdgcn_sched_barrier(0);  // the chunk's loads all issue before its first MFMA
    d = mma_chunk<ST>(w, col, k0, nk, lg, d);
  }
  return d;
}

// The same with the first two chunks already loaded (w1: k-steps CH .. 2 CH).
template <typename ST, int CH>
__device__ static inline f32x4_t mma_rows2(const u32x4 (&w0)[CH], const u32x4 (&w1)[CH], const ST* wa,
                                           const ST* wb, int ka, int nk, const ST* col, int lg, f32x4_t d) {
  d = mma_chunk<ST>(w0, col, 0, nk, lg, d);
  d = mma_chunk<ST>(w1, col, CH, nk, lg, d);
  for (int k0 = 2 * CH; k0 < nk; k0 += CH) {
    u32x4 w[CH];
    load_chunk<ST>(w, wa, wb, ka, nk, k0, lg);
    __builtin_amdgcn_sched_barrier(0);
    d = mma_chunk<ST>(w, col, k0, nk, lg, d);
  }
  return d;
}

// ---------------------------------------------------------------------------
// The words a stream's activity test reads, loaded in one round (b < batch).
struct StreamWords {
  int32_t slot, len, blank_seen;
};
__device__ static inline StreamWords stream_words(const DecK& p, int b) {
  return StreamWords{p.slots[b], p.lengths[b], ws_of(p, b)[0]};
}
// A stream decides at (t, s) while its slot is valid, t is one of its frames
// and it has not yet decided blank in frame t (word 0 of its workspace: 1 =
// blank seen).
__device__ static inline bool active_from(const DecK& p, const StreamWords& w) {
  return (uint32_t)w.slot < (uint32_t)p.num_slots && p.t < w.len && (p.s == 0 || w.blank_seen == 0);
}

template <typename ST>
__global__ void __launch_bounds__(kJointWaves * 64) joint_kernel(const DecK p) {
  constexpr int VEC = 16 / sizeof(ST), W = kJointWaves;
  constexpr int CPT = kMaxDim / VEC / 16;  // a thread's 16-byte chunks of a hid row, at most
  static_assert(W * 64 == 16 * 16, "hid staging: 16 threads a stream");
  __shared__ __align__(16) ST hid[16][kMaxDim + 8];
  __shared__ float bv[W][16];
  __shared__ int bi[W][16];
  __shared__ int32_t bid_s[16];
  const int vt = blockIdx.x, b0 = blockIdx.y * 16;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  // this iteration's list starts empty (its other half, read below, is the
  // previous iteration's)
  if (p.compact && vt == 0 && blockIdx.y == 0 && tid == 0) p.acount[p.it & 1] = 0;
  // the tile's streams: the batch, or after a frame's first symbol (compact
  // mode) the streams that emitted a token in the previous iteration; a
  // workgroup past that list loads nothing
  const int list = p.compact && p.s > 0 ? (p.it - 1) & 1 : -1;
  if (list >= 0 && b0 >= min(p.acount[list], p.batch)) return;
  // lane c of every 16-lane group reads entry c's stream words, so each wave
  // holds the activity of all 16 entries: a tile with none deciding returns
  // before any weight or row load, with no barrier (every wave sees the same
  // words).  Thread -> (stream entry k, chunks c + 16 j of its hid row); entry
  // k's words come from lane k of the thread's group.
  const int k = tid >> 4, c = tid & 15;
  const int bc = listed_stream(p, list, b0 + c);
  StreamWords swc{0, 0, 1};
  if (bc >= 0) swc = stream_words(p, bc);
  const bool ac = bc >= 0 && active_from(p, swc);
  if (__ballot(ac) == 0) return;
  const int src = (lane & 48) | k;
  const int b = __shfl(bc, src);
  const bool act = __shfl((int)ac, src) != 0;
  const int sk = __shfl(swc.slot, src);  // every lane takes part in the shuffles
  const int slot = act ? sk : 0;
  // the weight rows' first chunk and the biases of the lane's 4 rows, then the
  // hid row of the entry (zero for a stream not deciding: every load from an
  // address valid for any entry, then masked), the second weight chunk behind
  const int J = p.J, nch = J / VEC, ks = J / (4 * VEC);
  const int r0 = vt * kVT + wave * 16;
  const ST* wrow = (const ST*)p.w_out + (int64_t)min(r0 + lr, p.V1 - 1) * J;
  u32x4 w0[KChunk<ST>::CH], w1[KChunk<ST>::CH];
  load_chunk<ST>(w0, wrow, wrow, ks, ks, 0, lg);
  float bias[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bias[i] = from_st(((const ST*)p.b_out)[min(r0 + 4 * lg + i, p.V1 - 1)]);
  const ST* er_src = (const ST*)p.enc + max(b, 0) * p.enc_sb + (int64_t)p.t * p.enc_st;
  const ST* qr_src = (const ST*)p.pred_proj + (int64_t)slot * J;
  u32x4 er[CPT], qr[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    if (16 * j < nch) {  // uniform
      const int cc = min(c + 16 * j, nch - 1) * VEC;
      er[j] = ld16(er_src + cc);
      qr[j] = ld16(qr_src + cc);
    }
  }
  load_chunk<ST>(w1, wrow, wrow, ks, ks, KChunk<ST>::CH, lg);
  if (c == 0) bid_s[k] = b;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    if (c + 16 * j < nch) {
      float out[VEC];
      if (act) {
        float e[VEC], q[VEC];
        Tr<ST>::unpack(er[j], e);
        Tr<ST>::unpack(qr[j], q);
#pragma unroll
        for (int u = 0; u < VEC; ++u) out[u] = fmaxf(round_to<ST>(e[u] + q[u]), 0.f);
      } else {
#pragma unroll
        for (int u = 0; u < VEC; ++u) out[u] = 0.f;
      }
      *reinterpret_cast<u32x4*>(&hid[k][(c + 16 * j) * VEC]) = Tr<ST>::pack(out);
    }
  }
  __syncthreads();
  // logits of rows r0 .. r0 + 15 for the 16 streams
  const f32x4_t d = mma_rows2<ST>(w0, w1, wrow, wrow, ks, ks, &hid[lr][0], lg, f32x4_t{0.f, 0.f, 0.f, 0.f});
  // lane holds rows 4*lg + i (of the wave's 16) for stream lr
  float best = -INFINITY;
  int bidx = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = r0 + 4 * lg + i;
    if (row < p.V1) {
      const float v = round_to<ST>(d[i] + bias[i]);
      if (v > best) {  // rows ascend: the first maximum wins ties
        best = v;
        bidx = row;
      }
    }
  }
#pragma unroll
  for (int m = 16; m < 64; m <<= 1) {
    const float ov = __shfl_xor(best, m);
    const int oi = __shfl_xor(bidx, m);
    if (ov > best || (ov == best && oi < bidx)) {
      best = ov;
      bidx = oi;
    }
  }
  if (W == 1) {
    if (lg == 0 && bid_s[lr] >= 0) {
      int32_t* ws = ws_of(p, bid_s[lr]);
      ws[kWsHead + 2 * vt] = __float_as_int(best);
      ws[kWsHead + 2 * vt + 1] = bidx;
    }
    return;
  }
  if (lg == 0) {
    bv[wave][lr] = best;
    bi[wave][lr] = bidx;
  }
  __syncthreads();
  if (tid < 16 && bid_s[tid] >= 0) {
    float v = bv[0][tid];
    int ix = bi[0][tid];
    for (int w = 1; w < W; ++w)
      if (bv[w][tid] > v || (bv[w][tid] == v && bi[w][tid] < ix)) {
        v = bv[w][tid];
        ix = bi[w][tid];
      }
    int32_t* ws = ws_of(p, bid_s[tid]);
    ws[kWsHead + 2 * vt] = __float_as_int(v);
    ws[kWsHead + 2 * vt + 1] = ix;
  }
}

// ---------------------------------------------------------------------------
// Stream b's decision at (t, s): the first maximum over the vocabulary tiles'
// partial maxima; -1 when the stream is not deciding or decides blank.  Taken
// by the N lanes c = 0 .. N - 1 of an aligned lane group, every lane with the
// same b (every lane gets the result): lane c reads tiles c, c + N, ... and
// the lanes combine.  The (value, index) pairs are ordered by value, then by
// the lower index, a total order over the pairs the joint writes (never NaN),
// so any combining order gives the sequential scan's first maximum.  The
// stream words and the first 64 tiles are loaded in one round.
// Workspace words: 0 = blank seen in the current frame, 1 = token that updates
// the predictor this iteration (-1: none), 2 = tokens emitted this step.
// The loads of a decision taken by N lanes (N = 4 or 16): the stream words and
// the lane's first 64 / N tiles (the first 64 tiles of the group), issued
// together.
template <int N>
struct DecideLoads {
  StreamWords sw;
  int2 m[64 / N];
};
template <int N>
__device__ static inline DecideLoads<N> decide_load(const DecK& p, int b, int c) {
  const int32_t* ws = ws_of(p, b);
  DecideLoads<N> d;
  d.sw = stream_words(p, b);
#pragma unroll
  for (int u = 0; u < 64 / N; ++u)
    d.m[u] = *reinterpret_cast<const int2*>(ws + kWsHead + 2 * min(c + N * u, p.vtiles - 1));
  return d;
}
__device__ static inline void decide_take(float ov, int oi, float& v, int& ix) {
  if (ov > v || (ov == v && oi < ix)) {
    v = ov;
    ix = oi;
  }
}
template <int N>
__device__ static inline int decide_finish(const DecK& p, int b, int c, const DecideLoads<N>& d, bool* act_out) {
  float v = -INFINITY;
  int ix = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < 64 / N; ++u)
    if (c + N * u < p.vtiles) decide_take(__int_as_float(d.m[u].x), d.m[u].y, v, ix);
  const int32_t* ws = ws_of(p, b);
  for (int k0 = 64; k0 < p.vtiles; k0 += N) {  // tiles past the first 64 (vocabularies past 4,096 rows)
    const int t = k0 + c;
    if (t < p.vtiles) {
      const int2 m = *reinterpret_cast<const int2*>(ws + kWsHead + 2 * t);
      decide_take(__int_as_float(m.x), m.y, v, ix);
    }
  }
#pragma unroll
  for (int m = 1; m < N; m <<= 1) decide_take(__shfl_xor(v, m), __shfl_xor(ix, m), v, ix);
  const bool act = active_from(p, d.sw);
  *act_out = act;
  if (!act) return -1;
  return (ix == p.blank || ix < 0 || ix >= p.V1) ? -1 : ix;
}

// The record of stream b's decision (one writer per stream).  Other
// workgroups of the same launch may read word 0 before or after this write:
// an update needs a token, and a stream that just decided blank has none
// either way.
__device__ static inline void record(const DecK& p, int b, bool act, int tok) {
  int32_t* ws = ws_of(p, b);
  if (p.t == 0 && p.s == 0) ws[2] = 0;
  if (p.s == 0) {
    ws[0] = 0;
    if (p.t < p.max_frames) p.frame_counts[(int64_t)b * p.max_frames + p.t] = 0;
  }
  ws[1] = tok;
  if (!act) return;
  if (tok < 0) {
    ws[0] = 1;
    return;
  }
  const int n = ws[2];
  p.tokens[(int64_t)b * p.max_frames * p.max_symbols + n] = tok;
  ws[2] = n + 1;
  p.frame_counts[(int64_t)b * p.max_frames + p.t] += 1;
}

// Compact mode: every stream's decision and record for iteration `it`, and
// the list of the streams that emitted a token (their order in the list is
// the order of the atomic appends; every later launch treats each stream on
// its own, so the order does not change any result).
__global__ void __launch_bounds__(256) select_kernel(const DecK p) {
  const int c = threadIdx.x & 3, b = blockIdx.x * 64 + (threadIdx.x >> 2);  // 4 lanes a stream
  if (b >= p.batch) return;  // uniform per lane group
  bool act;
  const int tk = decide_finish<4>(p, b, c, decide_load<4>(p, b, c), &act);
  if (c != 0) return;
  record(p, b, act, tk);
  if (tk >= 0) {
    const int cur = p.it & 1;
    const int pos = atomicAdd(&p.acount[cur], 1);
    p.alist[(int64_t)cur * p.batch + pos] = b;
  }
}

// ---------------------------------------------------------------------------
// SPW streams per workgroup (16 or 32; the host takes 32 in compact mode, and
// when every stream may update and that keeps every workgroup on a CU of its
// own), 8 waves: 4 gates x {input part, recurrent part}.
template <typename ST, int SPW>
struct LstmCfg {
  static constexpr int WAVES = 8;
  static constexpr int NE = SPW / 16;  // stream entries a thread: k + 16 e
  static constexpr int CH = 10;        // k-steps of a weight chunk
};

// Waves 0-3 (the input part) take gate gi's W_ih x, waves 4-7 (the recurrent
// part) W_hh h.  The recurrent part's loads (its weight rows, the slots' h and
// c, the biases) do not depend on this iteration's decision, so they are in
// flight beside the decision and the embedding rows of the input part.  The
// recurrent part continues each gate's MFMA chain from the input part's sums,
// so the k-steps run in the order of one chain over K = [x ; h].
template <typename ST, int SPW>
__global__ void __launch_bounds__(512) lstm_kernel(const DecK p) {  // LstmCfg::WAVES x 64
#pragma clang fp contract(off)
  typedef LstmCfg<ST, SPW> Cfg;
  constexpr int VEC = 16 / sizeof(ST), NE = Cfg::NE, CH = Cfg::CH;
  constexpr int H = 640;                 // the hidden size the host accepts
  constexpr int RS = H + VEC;            // x or h row of one stream in LDS
  constexpr int NCH = H / VEC, CPT = NCH / 16;  // 16-byte chunks of a row; a thread's share
  static_assert(NCH % 16 == 0 && (NE == 1 || NE == 2) && Cfg::WAVES * 64 == 512, "a part's 256 threads: 16 a stream entry");
  __shared__ __align__(16) ST xs[SPW][RS];
  __shared__ __align__(16) ST hs[SPW][RS];
  __shared__ float gsm[4][SPW][17];
  __shared__ int32_t tok_s[SPW];
  const int L = p.layers, layer = p.layer;
  const int u0 = blockIdx.x * 16, b0 = blockIdx.y * SPW;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int part = wave >> 2, gi = wave & 3;
  // compact mode: a workgroup past the list's entries loads nothing
  const bool listed = p.compact && !p.prime;
  if (listed && b0 >= min(p.acount[p.it & 1], p.batch)) return;
  // thread -> stream entries k + 16 e and chunks c + 16 j of their rows; the 16
  // threads of an entry are lanes of one wave.  Layer 0 decides (prime: every
  // stream, token blank); the layers above and compact mode read the recorded
  // token.  Every thread of an entry takes the decision; lane c == 0 of column
  // 0 records it.
  const int pt = tid & 255, k = pt >> 4, c = pt & 15;
  const bool deciding = layer == 0 && !p.compact && !p.prime;
  int tk[NE];
  bool act[NE];
  DecideLoads<16> dl[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    tk[e] = -1;
    act[e] = false;
    if (deciding && part == 0) dl[e] = decide_load<16>(p, min(b0 + k + 16 * e, p.batch - 1), c);
  }
  // lane c of every 16-lane group reads whether entries c + 16 e may update
  // (deciding: they are active), so each wave holds all entries: a tile with
  // none returns before any weight or row load, with no barrier (every wave
  // sees the same words); entry k + 16 e's stream, token and slot come from
  // lane k of the thread's group
  int bq[NE], tq[NE], sq[NE];
  bool may = false;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int q = b0 + (lane & 15) + 16 * e;
    bq[e] = listed ? listed_stream(p, p.it & 1, q) : (q < p.batch ? q : -1);
    tq[e] = -1;  // deciding: 0 if active
    sq[e] = 0;
    if (bq[e] >= 0) {
      const StreamWords w = stream_words(p, bq[e]);
      const bool sok = (uint32_t)w.slot < (uint32_t)p.num_slots;
      sq[e] = sok ? w.slot : 0;
      if (deciding) tq[e] = active_from(p, w) ? 0 : -1;
      else if (p.prime) tq[e] = sok ? p.blank : -1;
      else tq[e] = ws_of(p, bq[e])[1];
    }
    may |= tq[e] >= 0;
  }
  const int kl = (lane & 48) | k;  // the lane holding entry k; every lane takes part in the shuffles
  int b[NE], slot[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    b[e] = __shfl(bq[e], kl);
    slot[e] = __shfl(sq[e], kl);
    const int t = __shfl(tq[e], kl);
    if (!deciding) tk[e] = t;
  }
  if (deciding && part == 0) {
#pragma unroll
    for (int e = 0; e < NE; ++e)
      if (b[e] >= 0) tk[e] = decide_finish<16>(p, b[e], c, dl[e], &act[e]);
  }
  const bool rec = deciding && part == 0 && blockIdx.x == 0 && c == 0;
  if (__ballot(may) == 0) {
    // no stream of the tile is active: column 0 still records every decision
    // (no token, and the frame's counters at its first symbol)
    if (rec) {
#pragma unroll
      for (int e = 0; e < NE; ++e)
        if (b[e] >= 0) record(p, b[e], act[e], tk[e]);
    }
    return;
  }
  // the wave's weight rows: gate gi, units u0 .. u0 + 15, first chunk
  const int64_t row = (int64_t)layer * 4 * H + gi * H + u0 + lr;
  constexpr int ks = H / (4 * VEC);
  const ST* wrow = (const ST*)(part ? p.w_hh : p.w_ih) + row * H;
  u32x4 w0[CH];
  load_chunk<ST>(w0, wrow, wrow, ks, ks, 0, lg);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 v[NE][CPT];
  u32x4 w1[CH];   // the second weight chunk
  float cb[8];    // recurrent part: the 8 biases of unit u0 + c
  float c0[NE];   // recurrent part: c of (entry k + 16 e, unit u0 + c)
  if (part == 0) {
    if (c == 0) {
#pragma unroll
      for (int e = 0; e < NE; ++e) tok_s[k + 16 * e] = tk[e];
    }
    // the second weight chunk, then x: the embedding row of the token (layer 0)
    // or the layer below's new h; loads from addresses valid for any entry,
    // then masked
    load_chunk<ST>(w1, wrow, wrow, ks, ks, CH, lg);
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const ST* src = layer == 0 ? (const ST*)p.embed + (int64_t)max(tk[e], 0) * H
                                 : (const ST*)p.hn + ((int64_t)max(b[e], 0) * L + layer - 1) * H;
#pragma unroll
      for (int j = 0; j < CPT; ++j) v[e][j] = ld16(src + (c + 16 * j) * VEC);
    }
    if (rec) {  // its reads queue behind the row loads
#pragma unroll
      for (int e = 0; e < NE; ++e)
        if (b[e] >= 0) record(p, b[e], act[e], tk[e]);
    }
#pragma unroll
    for (int e = 0; e < NE; ++e)
#pragma unroll
      for (int j = 0; j < CPT; ++j)
        *reinterpret_cast<u32x4*>(&xs[k + 16 * e][(c + 16 * j) * VEC]) = tk[e] >= 0 ? v[e][j] : u32x4{0u, 0u, 0u, 0u};
  } else {
    // h of the entries' slots (zero on a stream's first step), and for the cell
    // update of unit u0 + c: its c and biases.  An entry that does not update
    // reads slot 0's finite values; its MFMA column and cell are never used.
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const ST* src = (const ST*)p.h + ((int64_t)slot[e] * L + layer) * H;
#pragma unroll
      for (int j = 0; j < CPT; ++j) v[e][j] = ld16(src + (c + 16 * j) * VEC);
    }
    const int64_t bo = (int64_t)layer * 4 * H + u0 + c;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      cb[q] = from_st(((const ST*)p.b_ih)[bo + q * H]);
      cb[4 + q] = from_st(((const ST*)p.b_hh)[bo + q * H]);
    }
#pragma unroll
    for (int e = 0; e < NE; ++e) c0[e] = from_st(((const ST*)p.c)[((int64_t)slot[e] * L + layer) * H + u0 + c]);
#pragma unroll
    for (int e = 0; e < NE; ++e)
#pragma unroll
      for (int j = 0; j < CPT; ++j)
        *reinterpret_cast<u32x4*>(&hs[k + 16 * e][(c + 16 * j) * VEC]) = p.prime ? u32x4{0u, 0u, 0u, 0u} : v[e][j];
  }
  __syncthreads();
  bool any = false;
  for (int e = 0; e < SPW; ++e) any |= tok_s[e] >= 0;
  if (!any) return;  // uniform: no stream of the tile updates
  // gate gi rows for the streams, 16 a column tile: the input part's k-steps,
  // then the recurrent part's from those sums (its second chunk loading
  // meanwhile); lane: units u0 + 4 lg + i, stream 16 ct + lr
  if (part == 1) load_chunk<ST>(w1, wrow, wrow, ks, ks, CH, lg);
  if (part == 0) {
#pragma unroll
    for (int ct = 0; ct < NE; ++ct) {
      const f32x4_t d =
          mma_rows2<ST>(w0, w1, wrow, wrow, ks, ks, &xs[16 * ct + lr][0], lg, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int i = 0; i < 4; ++i) gsm[gi][16 * ct + lr][4 * lg + i] = d[i];
    }
  }
  __syncthreads();
  if (part == 1) {
#pragma unroll
    for (int ct = 0; ct < NE; ++ct) {
      f32x4_t d;
#pragma unroll
      for (int i = 0; i < 4; ++i) d[i] = gsm[gi][16 * ct + lr][4 * lg + i];
      d = mma_rows2<ST>(w0, w1, wrow, wrow, ks, ks, &hs[16 * ct + lr][0], lg, d);
#pragma unroll
      for (int i = 0; i < 4; ++i) gsm[gi][16 * ct + lr][4 * lg + i] = d[i];
    }
  }
  __syncthreads();
  // cell update: recurrent-part thread -> (stream entries k + 16 e, unit u0 + c)
  if (part == 1) {
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int ke = k + 16 * e;
      if (tok_s[ke] < 0) continue;  // a stream that updates has a valid slot
      float g4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) g4[q] = gsm[q][ke][c] + cb[q] + cb[4 + q];
      const float ig = 1.f / (1.f + __expf(-g4[0])), fg = 1.f / (1.f + __expf(-g4[1]));
      const float gg = tanhf(g4[2]), og = 1.f / (1.f + __expf(-g4[3]));
      const float cp = p.prime ? 0.f : c0[e];
      // one rounding order whatever the surrounding code: the input gate's
      // product fused, the forget gate's rounded first
      const float c1 = fmaf(ig, gg, fg * cp);
      ((ST*)p.c)[((int64_t)slot[e] * L + layer) * H + u0 + c] = to_st<ST>(c1);
      ((ST*)p.hn)[((int64_t)b[e] * L + layer) * H + u0 + c] = to_st<ST>(og * tanhf(c1));
    }
  }
}

// ---------------------------------------------------------------------------
template <typename ST>
__global__ void __launch_bounds__(kPredWaves * 64) pred_kernel(const DecK p) {
  constexpr int VEC = 16 / sizeof(ST), W = kPredWaves, NTH = W * 64, TPS = NTH / 16;
  constexpr int H = 640;                        // the hidden size the host accepts
  constexpr int NCH = H / VEC, CPT = NCH / TPS;  // 16-byte chunks of an h row; a thread's share
  static_assert(NCH % TPS == 0, "h row chunks over a stream's threads");
  __shared__ __align__(16) ST hs[16][H + VEC];
  __shared__ int32_t tok_s[16], slot_s[16];
  const int J = p.J, L = p.layers;
  const int j0 = blockIdx.x * (16 * W), b0 = blockIdx.y * 16;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  // the streams that updated: the batch's (prime: every stream's), or in compact
  // mode the list of this iteration's token emitters; a workgroup past that
  // list loads nothing
  const int list = p.compact && !p.prime ? p.it & 1 : -1;
  if (list >= 0 && b0 >= min(p.acount[list], p.batch)) return;
  // lane c of every 16-lane group reads entry c's token and slot, so each wave
  // holds all 16: a tile with no update returns before any weight or row
  // load, with no barrier (every wave sees the same words).  Thread ->
  // (stream entry k, chunks c + TPS j of a row); entry k's words come from
  // lane k of the thread's group.
  const int k = tid / TPS, c = tid % TPS;
  const int bq = listed_stream(p, list, b0 + (lane & 15));
  int sq = 0, tq = -1;
  if (bq >= 0) {
    sq = p.slots[bq];
    if ((uint32_t)sq < (uint32_t)p.num_slots) tq = p.prime ? 0 : ws_of(p, bq)[1];
  }
  if (__ballot(tq >= 0) == 0) return;
  const int src = (lane & 48) | k;
  const int b = __shfl(bq, src), tk = __shfl(tq, src);
  const int sk = __shfl(sq, src);  // every lane takes part in the shuffles
  const int slot = tk >= 0 ? sk : 0;
  // this wave's weight rows (first chunk) and its lanes' biases; a wave past
  // the joint size keeps its lanes but reads row J - 1
  constexpr int ks = H / (4 * VEC);
  const int jw = j0 + wave * 16;
  const bool wave_live = jw < J;  // uniform per wave
  const ST* wrow = (const ST*)p.w_pred + (int64_t)min(jw + lr, J - 1) * H;
  u32x4 w0[KChunk<ST>::CH], w1[KChunk<ST>::CH];
  load_chunk<ST>(w0, wrow, wrow, ks, ks, 0, lg);
  float bias[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bias[i] = from_st(((const ST*)p.b_pred)[min(jw + 4 * lg + i, J - 1)]);
  // the top layer's new h of the entry, loads first (valid addresses for any
  // entry), then masked into LDS
  const ST* top = (const ST*)p.hn + ((int64_t)max(b, 0) * L + L - 1) * H;
  u32x4 hr[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) hr[j] = ld16(top + (c + TPS * j) * VEC);
  // the new h of every layer into the slot state: this workgroup's share,
  // chunks q = blockIdx.x + gridDim.x (c + TPS m) of the entry's L rows
  const int nq = L * NCH, qs = gridDim.x * TPS;
  const ST* hn_b = (const ST*)p.hn + (int64_t)max(b, 0) * L * H;
  ST* h_s = (ST*)p.h + (int64_t)slot * L * H;
  load_chunk<ST>(w1, wrow, wrow, ks, ks, KChunk<ST>::CH, lg);
  if (c == 0) {
    tok_s[k] = tk;
    slot_s[k] = slot;
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j)
    *reinterpret_cast<u32x4*>(&hs[k][(c + TPS * j) * VEC]) = tk >= 0 ? hr[j] : u32x4{0u, 0u, 0u, 0u};
  for (int q = blockIdx.x + gridDim.x * c; q < nq; q += qs) {
    const u32x4 v = ld16(hn_b + (q / NCH) * H + (q % NCH) * VEC);
    if (tk >= 0) st16(h_s + (q / NCH) * H + (q % NCH) * VEC, v);
  }
  __syncthreads();
  if (!wave_live) return;  // uniform per wave; no barrier below
  const f32x4_t d = mma_rows2<ST>(w0, w1, wrow, wrow, ks, ks, &hs[lr][0], lg, f32x4_t{0.f, 0.f, 0.f, 0.f});
  // lane: outputs jw + 4 lg + i for stream lr
  if (tok_s[lr] >= 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jj = jw + 4 * lg + i;
      ((ST*)p.pred_proj)[(int64_t)slot_s[lr] * J + jj] = to_st<ST>(d[i] + bias[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// int32 words: the per-stream words, then the two stream lists and their two
// counts (compact mode), rounded up to 256 bytes
static int64_t ws_int_bytes(int batch, int vocab1) {
  const int64_t w = (int64_t)batch * (kWsHead + 2 * ((vocab1 + kVT - 1) / kVT)) + 2 * (int64_t)batch + 4;
  return (w * 4 + 255) / 256 * 256;
}

template <typename ST>
static int run_step(const pk_rnnt_args* a, hipStream_t st) {
  DecK k{};
  k.batch = a->batch;
  k.num_slots = a->num_slots;
  k.layers = a->layers;
  k.H = a->hidden;
  k.J = a->joint;
  k.V1 = a->vocab1;
  k.blank = a->blank;
  k.max_symbols = a->max_symbols;
  k.vtiles = (a->vocab1 + kVT - 1) / kVT;
  k.max_frames = a->max_frames;
  k.slots = a->slots;
  k.lengths = a->lengths;
  k.embed = a->embed;
  k.w_ih = a->w_ih;
  k.w_hh = a->w_hh;
  k.b_ih = a->b_ih;
  k.b_hh = a->b_hh;
  k.w_pred = a->w_pred;
  k.b_pred = a->b_pred;
  k.w_out = a->w_out;
  k.b_out = a->b_out;
  k.c = a->c;
  k.pred_proj = a->pred_proj;
  k.enc = a->enc_proj;
  k.enc_sb = a->enc_stride_b;
  k.enc_st = a->enc_stride_t;
  k.tokens = a->tokens;
  k.frame_counts = a->frame_counts;
  k.ws = (int32_t*)a->workspace;
  k.hn = (char*)a->workspace + ws_int_bytes(a->batch, a->vocab1);
  const int64_t words = (int64_t)a->batch * (kWsHead + 2 * k.vtiles);
  k.alist = (int32_t*)a->workspace + words;
  k.acount = k.alist + 2 * (int64_t)a->batch;
  k.compact = !a->prime && (a->compact > 0 || (a->compact == 0 && a->batch >= kCompactMinBatch));
  k.h = a->h;
  k.prime = a->prime;
  const dim3 gj(k.vtiles, (a->batch + 15) / 16);
  // 32 streams a LSTM workgroup (16-bit types only: the fp32 rows of 32 streams
  // do not fit in LDS) in compact mode, where the tiles hold only streams that
  // update and 32 of them read the weights half as often, and otherwise when
  // every stream may update (a frame's first symbol, or priming) and that
  // leaves no CU with two workgroups; else 16: at later symbols the smaller
  // tiles more often have no update and return early
  const int cus = cu_count();
  const bool wide_fits = sizeof(ST) == 2 && !k.compact &&
                         (int64_t)(a->hidden / 16) * ((a->batch + 15) / 16) > cus &&
                         (int64_t)(a->hidden / 16) * ((a->batch + 31) / 32) <= cus;
  const dim3 gl16(a->hidden / 16, (a->batch + 15) / 16), gl32(a->hidden / 16, (a->batch + 31) / 32);
  const dim3 gp((a->joint + 16 * kPredWaves - 1) / (16 * kPredWaves), (a->batch + 15) / 16);
  auto lstm = [&]() {
    for (int l = 0; l < a->layers; ++l) {
      k.layer = l;
      if constexpr (sizeof(ST) == 2) {
        if (k.compact || (wide_fits && (k.prime || k.s == 0))) {
          hipLaunchKernelGGL((lstm_kernel<ST, 32>), gl32, dim3(LstmCfg<ST, 32>::WAVES * 64), 0, st, k);
          continue;
        }
      }
      hipLaunchKernelGGL((lstm_kernel<ST, 16>), gl16, dim3(LstmCfg<ST, 16>::WAVES * 64), 0, st, k);
    }
  };
  auto pred = [&]() { hipLaunchKernelGGL(pred_kernel<ST>, gp, dim3(kPredWaves * 64), 0, st, k); };
  k.t = k.s = 0;
  if (!a->prime) {
    for (int t = 0; t < a->max_frames; ++t)
      for (int s = 0; s < a->max_symbols; ++s) {
        k.t = t;
        k.s = s;
        k.it = t * a->max_symbols + s;
        hipLaunchKernelGGL(joint_kernel<ST>, gj, dim3(kJointWaves * 64), 0, st, k);
        if (k.compact) hipLaunchKernelGGL(select_kernel, dim3((a->batch + 63) / 64), dim3(256), 0, st, k);
        lstm();
        pred();
      }
  } else {
    lstm();
    pred();
  }
  return check_launch("pk_rnnt_greedy_step");
}

}  // namespace pk

using namespace pk;

extern "C" int64_t pk_rnnt_workspace_bytes(int32_t dtype, int32_t batch, int32_t vocab1, int32_t layers,
                                           int32_t hidden) {
  if (batch < 0 || vocab1 < 1 || layers < 1 || hidden < 1) return -1;
  const int es = dtype == PK_DTYPE_F32 ? 4 : 2;
  return ws_int_bytes(batch, vocab1) + (int64_t)batch * layers * hidden * es;
}

// ---------------------------------------------------------------------------
// Allocation-free decode step: the step's workspace is a static device array,
// one per GPU, held until the process ends.  Its device address is looked up
// once per device (with that device current) and passed to the kernels like a
// caller's workspace; the array's name is never used as an address on the host.

static __device__ __align__(256) uint8_t scratch[PK_RNNT_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's scratch address; the device must be current.  The lookup
// (which may load the code object) runs once per device and never under stream
// capture: a first call made while `stream` is capturing is refused, and the
// workspace entry point looks the address up on its first call on a device, so
// a decoder that has run one eager step can record static steps in a graph.
int scratch_address(void** out, hipStream_t stream, bool quiet = false) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return quiet ? PK_ERR_HIP : fail(PK_ERR_HIP, "pk_rnnt_greedy_step_static: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
      return quiet ? PK_ERR_STATE : fail(PK_ERR_STATE,
                  "pk_rnnt_greedy_step_static: first call on device %d is under stream capture; make one call "
                  "(or one pk_rnnt_greedy_step call) outside capture first, which looks up the static scratch",
                  dev);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return quiet ? PK_ERR_HIP : fail(PK_ERR_HIP, "pk_rnnt_greedy_step_static: hipGetSymbolAddress on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PK_OK;
}

}  // namespace

extern "C" int pk_rnnt_greedy_step(const pk_rnnt_args* a, void* stream) {
  clear_error();
  if (!a) return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: args is NULL");
  if (a->dtype != PK_DTYPE_F32 && a->dtype != PK_DTYPE_F16 && a->dtype != PK_DTYPE_BF16)
    return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: dtype %d", a->dtype);
  if (a->batch < 0 || a->max_frames < 0 || a->max_symbols < 1 || a->layers < 1 || a->num_slots < 1)
    return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: bad batch/max_frames/max_symbols/layers/num_slots");
  if (a->hidden != 640 || a->joint < 64 || a->joint > kMaxDim || a->joint % 64)
    return fail(PK_ERR_UNSUPPORTED, "pk_rnnt_greedy_step: hidden %d (built: 640), joint %d (multiple of 64, <= %d)",
                a->hidden, a->joint, kMaxDim);
  if (a->vocab1 < 2 || a->blank < 0 || a->blank >= a->vocab1)
    return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: vocab1 %d, blank %d", a->vocab1, a->blank);
  if (a->batch == 0 || (!a->prime && a->max_frames == 0)) return PK_OK;
  if (a->batch > 65535 * 16) return fail(PK_ERR_UNSUPPORTED, "pk_rnnt_greedy_step: batch %d", a->batch);
  if (!a->slots || !a->embed || !a->w_ih || !a->w_hh || !a->b_ih || !a->b_hh || !a->w_pred || !a->b_pred ||
      !a->w_out || !a->b_out || !a->h || !a->c || !a->pred_proj || !a->workspace ||
      (!a->prime && (!a->enc_proj || !a->lengths || !a->tokens || !a->frame_counts)))
    return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: NULL pointer");
  const void* vecs[] = {a->embed, a->w_ih, a->w_hh, a->w_pred, a->w_out, a->h, a->c, a->pred_proj, a->enc_proj};
  for (const void* v : vecs)
    if (v && !aligned16(v)) return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: weights and state must be 16-byte aligned");
  if (!aligned16(a->workspace)) return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: workspace must be 16-byte aligned");
  if (!a->prime && (a->enc_stride_b % 8 || a->enc_stride_t % 8))
    return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step: enc_proj strides must keep 16-byte rows");
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "pk_rnnt_greedy_step: cannot select device %d", a->device);
  {  // the static entry point's scratch, looked up on this device's first call (outside capture)
    void* unused = nullptr;
    (void)scratch_address(&unused, (hipStream_t)stream, true);
  }
  switch (a->dtype) {
    case PK_DTYPE_F16:
      return run_step<_Float16>(a, (hipStream_t)stream);
    case PK_DTYPE_BF16:
      return run_step<bf16_t>(a, (hipStream_t)stream);
    default:
      return run_step<float>(a, (hipStream_t)stream);
  }
}


extern "C" int pk_rnnt_greedy_step_static(const pk_rnnt_args* a, void* stream) {
  clear_error();
  if (!a) return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step_static: args is NULL");
  if (a->workspace)
    return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step_static: workspace must be NULL (the static scratch is used)");
  const int64_t need = pk_rnnt_workspace_bytes(a->dtype, a->batch, a->vocab1, a->layers, a->hidden);
  if (need < 0) return fail(PK_ERR_INVALID, "pk_rnnt_greedy_step_static: bad batch/vocab1/layers/hidden");
  if (need > (int64_t)PK_RNNT_STATIC_SCRATCH_BYTES)
    return fail(PK_ERR_UNSUPPORTED,
                "pk_rnnt_greedy_step_static: batch %d needs %lld bytes of workspace, the static scratch holds %lld "
                "(use pk_rnnt_greedy_step with a workspace)",
                a->batch, (long long)need, (long long)PK_RNNT_STATIC_SCRATCH_BYTES);
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "pk_rnnt_greedy_step_static: cannot select device %d", a->device);
  void* ptr = nullptr;
  const int rc = scratch_address(&ptr, (hipStream_t)stream);
  if (rc != PK_OK) return rc;
  pk_rnnt_args b = *a;
  b.workspace = ptr;
  return pk_rnnt_greedy_step(&b, stream);
}
