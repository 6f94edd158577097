// gfx950 kernel of the Conformer convolution module's streaming step, with each
// stream's convolution cache read and written in place
// (parakeet/modules/convolution.py:37-47,150-158; parakeet/modules/cache.py:47-53).
//
//   conv_step_kernel  GLU -> padded frames zeroed -> causal depthwise conv over
//                     [cache ; frames] -> LayerNorm over channels -> SiLU; the
//                     next cache is written back in place
//   conv_chunk_kernel the same step with a chunk's frames in parallel (chunks of
//                     3 or more frames at small batches); same bits
//   resnorm_kernel    a Conformer layer's residual update and the LayerNorm
//                     that reads it (parakeet/modules/encoder.py:58-81)
//
// conv_step_kernel: one workgroup per stream.  Lane l of the workgroup owns the channels
// [l*VEC, (l+1)*VEC) -- one 16-byte chunk, 8 fp16/bf16 or 4 fp32 channels -- so
// every frame row (cache, GLU input, output) is read and written as whole
// 16-byte lanes.  A lane keeps a window of `kernel` frames of its channels in
// registers: the cache rows first, then each new frame's GLU output rounded to
// the storage type (the value the reference's concatenated tensor holds).  After
// the last frame the window holds exactly the next cache; each lane owns its
// channels, so the rows go back to the cache with no ordering hazard and no
// separate shift.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "pk_common.h"
#include "pk_device.h"

namespace pk {

template <typename ST>
struct ConvK {
  const ST* h;  // [B][T][2D] pointwise-conv1 output
  int64_t h_sb, h_st;
  ST* cache;  // [slots][layers][K-1][D]
  int32_t num_slots, num_layers, layer;
  const int32_t* slots;
  const uint8_t* pad;  // [B][T], 1 = padded
  const int64_t* lengths;
  int64_t len_scalar;
  const ST* w;     // [D][K]
  const ST* bias;  // [D] or nullptr
  const ST* lnw;   // [D]
  const ST* lnb;   // [D]
  float eps;
  ST* out;  // [B][T][D]
  int64_t o_sb, o_st;
  int32_t T, D;
};

// Sum over the workgroup's waves, in every thread.  Every thread of the
// workgroup calls it the same number of times (the frame loop is uniform).
__device__ static inline float block_sum(float v, float* red, int nw) {
  v = group_sum<64>(v);
  if (nw == 1) return v;
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += red[i];
  __syncthreads();  // `red` is rewritten by the next call
  return s;
}

constexpr int kConvMaxWaves = 8;

// STREAM (host-chosen when the conv caches of a step outgrow the last-level
// cache): the cache rows and the GLU input, each read once a step, move with
// the streaming (non-temporal) policy, so they do not displace what the
// step's other kernels reuse
template <typename ST, int K, bool STREAM>
__global__ void __launch_bounds__(64 * kConvMaxWaves) conv_step_kernel(const ConvK<ST> p) {
  // every product and sum rounds as written (fused only where fmaf says so),
  // so both forms of the step give the same bits
#pragma clang fp contract(off)
  constexpr int VEC = Tr<ST>::VEC;
  constexpr int R = K - 1;  // cache rows
  __shared__ float red[kConvMaxWaves];

  const int b = blockIdx.x;
  const int nw = blockDim.x >> 6;
  const int nchunk = p.D / VEC;
  const bool own = (int)threadIdx.x < nchunk;  // lanes past d_model hold no channels
  const int c0 = min((int)threadIdx.x, nchunk - 1) * VEC;
  const int slot = p.slots ? p.slots[b] : b;
  // a slot outside the cache is a caller error the host wrapper rejects; the
  // kernel leaves such a stream untouched rather than address outside the cache
  if (slot < 0 || slot >= p.num_slots) return;  // workgroup-uniform
  ST* const crow = p.cache + ((int64_t)slot * p.num_layers + p.layer) * R * p.D + c0;
  const ST* const hb = p.h + b * p.h_sb + c0;
  ST* const ob = p.out + b * p.o_sb + c0;

  // depthwise taps of the lane's channels: the [VEC][K] block of the [D][K]
  // weight is VEC*K contiguous elements, K chunks of VEC
  float w[VEC][K];
  {
    const ST* wp = p.w + (int64_t)c0 * K;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      float f[VEC];
      Tr<ST>::unpack(ld16(wp + i * VEC), f);
#pragma unroll
      for (int e = 0; e < VEC; ++e) w[(i * VEC + e) / K][(i * VEC + e) % K] = f[e];
    }
  }
  float bias[VEC], lw[VEC], lb[VEC];
  if (p.bias) {
    Tr<ST>::unpack(ld16(p.bias + c0), bias);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) bias[e] = 0.f;
  }
  Tr<ST>::unpack(ld16(p.lnw + c0), lw);
  Tr<ST>::unpack(ld16(p.lnb + c0), lb);

  // window rows 0..R-1: the cache (the R frames before this step's first)
  float win[K][VEC];
#pragma unroll
  for (int r = 0; r < R; ++r)
    Tr<ST>::unpack(STREAM ? ld16_stream(crow + (int64_t)r * p.D) : ld16(crow + (int64_t)r * p.D), win[r]);

  const uint8_t* padb = p.pad ? p.pad + (int64_t)b * p.T : nullptr;
  const int64_t len = p.lengths ? p.lengths[b] : p.len_scalar;
  const float inv_d = 1.f / (float)p.D;

  for (int t = 0; t < p.T; ++t) {
    // this frame's GLU output (convolution.py:152-155), zero where padded
    float a[VEC], g[VEC];
    Tr<ST>::unpack(STREAM ? ld16_stream(hb + t * p.h_st) : ld16(hb + t * p.h_st), a);
    Tr<ST>::unpack(STREAM ? ld16_stream(hb + t * p.h_st + p.D) : ld16(hb + t * p.h_st + p.D), g);
    const bool valid = padb ? padb[t] == 0 : (int64_t)t < len;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float v = a[e] / (1.f + __expf(-g[e]));
      win[R][e] = valid ? round_to<ST>(v) : 0.f;
    }
    // causal depthwise conv: output t sees window rows 0..R = frames t..t+R of
    // [cache ; frames] (convolution.py:43-46, Conv1d cross-correlation)
    float y[VEC];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float acc = bias[e];
#pragma unroll
      for (int k = 0; k < K; ++k) acc = fmaf(w[e][k], win[k][e], acc);
      y[e] = acc;
      s += acc;
    }
    // LayerNorm over d_model (convolution.py:156), two-pass mean / variance
    const float mean = block_sum(own ? s : 0.f, red, nw) * inv_d;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float d = y[e] - mean;
      q = fmaf(d, d, q);
    }
    const float var = block_sum(own ? q : 0.f, red, nw) * inv_d;
    const float rstd = rsqrtf(var + p.eps);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float z = fmaf((y[e] - mean) * rstd, lw[e], lb[e]);
      y[e] = z / (1.f + __expf(-z));  // SiLU (convolution.py:157)
    }
    if (own) st16(ob + t * p.o_st, Tr<ST>::pack(y));
#pragma unroll
    for (int k = 0; k < R; ++k) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) win[k][e] = win[k + 1][e];
    }
  }
  // the window now holds the last R frames of [cache ; frames]: the next cache
  // (convolution.py:46, next_cache = new_x[:, :, -(K-1):])
  if (own) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (STREAM)
        st16_stream(crow + (int64_t)r * p.D, Tr<ST>::pack(win[r]));
      else
        st16(crow + (int64_t)r * p.D, Tr<ST>::pack(win[r]));
    }
  }
}

// The same step with the chunk's frames in parallel, for chunks of several
// frames (the frames of a chunk depend on each other only through the window,
// not through any recurrence).  One workgroup per stream of FG groups of nw
// waves (a group's lanes own the channels as above):
//   1. every thread: the window [cache ; GLU(frames)] into LDS as the storage
//      type ([R + T][D]; every global load of the stream issued at once), then
//      its last R rows back to the cache (every read of the old cache is
//      behind the barrier);
//   2. group g takes frames g, g + FG, ...: the depthwise conv over its window
//      rows in LDS, LayerNorm summed over the group's waves, SiLU.
// Every sum is the sequential kernel's, in the same order (a lane's channels,
// then the wave, then the group's waves in order), so the two give the same
// bits.  The reductions are workgroup barriers, so every group runs the same
// number of frame iterations (a group past the chunk's end sums zeros).
template <typename ST, int K, bool STREAM>
__global__ void __launch_bounds__(64 * kConvMaxWaves) conv_chunk_kernel(const ConvK<ST> p, int FG) {
#pragma clang fp contract(off)
  constexpr int VEC = Tr<ST>::VEC;
  constexpr int R = K - 1;
  extern __shared__ __align__(16) unsigned char conv_smem[];

  const int b = blockIdx.x;
  const int nchunk = p.D / VEC;
  const int nw = (nchunk + 63) >> 6;  // waves of a group
  const int fg = threadIdx.x / (64 * nw), gt = threadIdx.x - fg * 64 * nw;
  const int gwave = gt >> 6;
  const bool own = gt < nchunk;
  const int c0 = min(gt, nchunk - 1) * VEC;
  const int slot = p.slots ? p.slots[b] : b;
  if (slot < 0 || slot >= p.num_slots) return;  // workgroup-uniform
  const int rows = R + p.T;
  ST* const win = reinterpret_cast<ST*>(conv_smem);                               // [rows][D]
  float* const red = reinterpret_cast<float*>(conv_smem + (size_t)rows * p.D * sizeof(ST)) + fg * nw;  // [FG][nw]
  ST* const crow0 = p.cache + ((int64_t)slot * p.num_layers + p.layer) * R * p.D;
  const uint8_t* padb = p.pad ? p.pad + (int64_t)b * p.T : nullptr;
  const int64_t len = p.lengths ? p.lengths[b] : p.len_scalar;

  // 1. the window: cache rows, then each frame's GLU output (convolution.py:152-155)
  //    rounded to the storage type, zero where padded
  for (int i = threadIdx.x; i < rows * nchunk; i += blockDim.x) {
    const int r = i / nchunk, c = (i - r * nchunk) * VEC;
    u32x4 v;
    if (r < R) {
      const ST* q = crow0 + (int64_t)r * p.D + c;
      v = STREAM ? ld16_stream(q) : ld16(q);
    } else {
      const int t = r - R;
      const ST* q = p.h + b * p.h_sb + t * p.h_st + c;
      float a[VEC], g[VEC], o[VEC];
      Tr<ST>::unpack(STREAM ? ld16_stream(q) : ld16(q), a);
      Tr<ST>::unpack(STREAM ? ld16_stream(q + p.D) : ld16(q + p.D), g);
      const bool valid = padb ? padb[t] == 0 : (int64_t)t < len;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = valid ? a[e] / (1.f + __expf(-g[e])) : 0.f;
      v = Tr<ST>::pack(o);
    }
    *reinterpret_cast<u32x4*>(win + (size_t)r * p.D + c) = v;
  }
  __syncthreads();
  // the next cache: the window's last R rows (convolution.py:46)
  for (int i = threadIdx.x; i < R * nchunk; i += blockDim.x) {
    const int r = i / nchunk, c = (i - r * nchunk) * VEC;
    const u32x4 v = *reinterpret_cast<const u32x4*>(win + (size_t)(p.T + r) * p.D + c);
    if constexpr (STREAM)
      st16_stream(crow0 + (int64_t)r * p.D + c, v);
    else
      st16(crow0 + (int64_t)r * p.D + c, v);
  }

  // 2. the lane's taps, bias and LayerNorm parameters
  float w[VEC][K];
  {
    const ST* wp = p.w + (int64_t)c0 * K;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      float f[VEC];
      Tr<ST>::unpack(ld16(wp + i * VEC), f);
#pragma unroll
      for (int e = 0; e < VEC; ++e) w[(i * VEC + e) / K][(i * VEC + e) % K] = f[e];
    }
  }
  float bias[VEC], lw[VEC], lb[VEC];
  if (p.bias) {
    Tr<ST>::unpack(ld16(p.bias + c0), bias);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) bias[e] = 0.f;
  }
  Tr<ST>::unpack(ld16(p.lnw + c0), lw);
  Tr<ST>::unpack(ld16(p.lnb + c0), lb);
  const float inv_d = 1.f / (float)p.D;
  // the group's sum of a value over its waves, in wave order, in every lane
  auto gsum = [&](float v) {
    v = group_sum<64>(v);
    if (nw == 1) return v;
    if ((gt & 63) == 0) red[gwave] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < nw; ++i) s += red[i];
    __syncthreads();  // `red` is rewritten by the next call
    return s;
  };

  const int iters = (p.T + FG - 1) / FG;
  for (int it = 0; it < iters; ++it) {
    const int t = fg + it * FG;
    const bool act = t < p.T && own;
    // causal depthwise conv: output t sees window rows t .. t + R
    float y[VEC];
    float s = 0.f;
    if (act) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) y[e] = bias[e];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        float x[VEC];
        Tr<ST>::unpack(*reinterpret_cast<const u32x4*>(win + (size_t)(t + k) * p.D + c0), x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) y[e] = fmaf(w[e][k], x[e], y[e]);
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += y[e];
    }
    // LayerNorm over d_model (convolution.py:156), two-pass mean / variance
    const float mean = gsum(act ? s : 0.f) * inv_d;
    float q = 0.f;
    if (act) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = y[e] - mean;
        q = fmaf(d, d, q);
      }
    }
    const float var = gsum(act ? q : 0.f) * inv_d;
    const float rstd = rsqrtf(var + p.eps);
    if (act) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float z = fmaf((y[e] - mean) * rstd, lw[e], lb[e]);
        y[e] = z / (1.f + __expf(-z));  // SiLU (convolution.py:157)
      }
      st16(p.out + b * p.o_sb + t * p.o_st + c0, Tr<ST>::pack(y));
    }
  }
}

// ---------------------------------------------------------------------------
// Residual update + LayerNorm (parakeet/modules/encoder.py:58-81): per row,
//   r = residual + alpha * branch  (alpha * branch rounded to the storage type
//       first when alpha != 1, then the sum rounded: `residual += x * 0.5`)
//   n = LayerNorm(r) * w + b       (fp32 two-pass statistics of the rounded r)
// One wave per row; lane l owns the 16-byte chunks l, l + 64, ... (NV of them)
// and reads each before writing it, so r may overwrite residual in place.
template <typename ST>
struct ResNormK {
  const ST* res;
  int64_t res_s;
  const ST* br;
  int64_t br_s;
  const ST* lnw;
  const ST* lnb;
  ST* rout;
  int64_t rout_s;
  ST* nout;
  int64_t nout_s;
  float alpha, eps;
  int32_t rows, D;
};

constexpr int kResNormRows = 4;  // rows (waves) a workgroup

template <typename ST, int NV>
__global__ void __launch_bounds__(64 * kResNormRows) resnorm_kernel(const ResNormK<ST> p) {
#pragma clang fp contract(off)
  constexpr int VEC = Tr<ST>::VEC;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kResNormRows + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // the whole wave: the kernel has no barrier
  const float inv_d = 1.f / (float)p.D;
  const bool scaled = p.alpha != 1.f;
  u32x4 rv[NV], bv[NV], wv[NV], cv[NV];
  bool own[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (lane + 64 * v) * VEC;
    own[v] = c < p.D;
    const int cc = own[v] ? c : 0;  // a valid address for every lane
    rv[v] = ld16(p.res + row * p.res_s + cc);
    bv[v] = ld16(p.br + row * p.br_s + cc);
    wv[v] = ld16(p.lnw + cc);
    cv[v] = ld16(p.lnb + cc);
  }
  float x[NV][VEC];
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float r[VEC], b[VEC];
    Tr<ST>::unpack(rv[v], r);
    Tr<ST>::unpack(bv[v], b);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = scaled ? round_to<ST>(p.alpha * b[e]) : b[e];
      x[v][e] = round_to<ST>(r[e] + t);
      s += own[v] ? x[v][e] : 0.f;
    }
  }
  const float mean = group_sum<64>(s) * inv_d;
  float q = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float d = x[v][e] - mean;
      q += own[v] ? d * d : 0.f;
    }
  const float var = group_sum<64>(q) * inv_d;
  const float rstd = rsqrtf(var + p.eps);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (!own[v]) continue;
    const int c = (lane + 64 * v) * VEC;
    float w[VEC], bb[VEC], z[VEC];
    Tr<ST>::unpack(wv[v], w);
    Tr<ST>::unpack(cv[v], bb);
#pragma unroll
    for (int e = 0; e < VEC; ++e) z[e] = fmaf((x[v][e] - mean) * rstd, w[e], bb[e]);
    st16(p.rout + row * p.rout_s + c, Tr<ST>::pack(x[v]));
    st16(p.nout + row * p.nout_s + c, Tr<ST>::pack(z));
  }
}

namespace {

// a step's conv caches (every layer's rows of the batch) above this share of
// the 256 MB last-level cache take the streaming policy
constexpr int64_t kConvStreamingBytes = 192ll << 20;
// chunks of at least this many frames take the frames-in-parallel kernel when
// the stream's window fits its LDS budget and the frame-by-frame kernel would
// have fewer than kConvChunkWavesPerCu waves a CU (measured crossover at 14
// frames: about 700 streams at d_model 1024 bf16, 1,500 at 512 fp16; past it
// the frame-by-frame kernel's many streams hide its per-frame latency better)
constexpr int kConvChunkMinT = 3;
constexpr size_t kConvChunkLds = 64 * 1024;
constexpr int kConvChunkWavesPerCu = 6;

template <typename ST, int K>
int launch_conv(const ConvK<ST>& k, int batch, hipStream_t s) {
  constexpr int VEC = Tr<ST>::VEC;
  const int nchunk = k.D / VEC;
  const int nw = (nchunk + 63) / 64;
  const int64_t cache_bytes = (int64_t)batch * k.num_layers * (K - 1) * k.D * (int64_t)sizeof(ST);
  const size_t win_bytes = (size_t)(K - 1 + k.T) * k.D * sizeof(ST);
  if (k.T >= kConvChunkMinT && win_bytes + kConvMaxWaves * sizeof(float) <= kConvChunkLds &&
      (int64_t)batch * nw < (int64_t)kConvChunkWavesPerCu * cu_count()) {
    // as many groups of nw waves as the frames and the workgroup's waves allow
    const int fgroups = std::min(k.T, kConvMaxWaves / nw);
    const size_t lds = win_bytes + (size_t)fgroups * nw * sizeof(float);
    const dim3 grid((unsigned)batch), block(64u * nw * fgroups);
    if (cache_bytes > kConvStreamingBytes)
      hipLaunchKernelGGL((conv_chunk_kernel<ST, K, true>), grid, block, lds, s, k, fgroups);
    else
      hipLaunchKernelGGL((conv_chunk_kernel<ST, K, false>), grid, block, lds, s, k, fgroups);
    return check_launch("pk_conv_step");
  }
  if (cache_bytes > kConvStreamingBytes)
    hipLaunchKernelGGL((conv_step_kernel<ST, K, true>), dim3((unsigned)batch), dim3(64u * nw), 0, s, k);
  else
    hipLaunchKernelGGL((conv_step_kernel<ST, K, false>), dim3((unsigned)batch), dim3(64u * nw), 0, s, k);
  return check_launch("pk_conv_step");
}

template <typename ST>
int conv_typed(const pk_conv_args* a, hipStream_t s) {
  constexpr int VEC = Tr<ST>::VEC;
  const char* what = "pk_conv_step";
  if (a->batch < 0 || a->chunk <= 0)
    return fail(PK_ERR_INVALID, "%s: need batch >= 0 and chunk > 0", what);
  if (a->d_model <= 0 || a->d_model % VEC != 0 || a->d_model > 64 * kConvMaxWaves * VEC)
    return fail(PK_ERR_INVALID, "%s: d_model %d must be a positive multiple of %d, at most %d",
                what, a->d_model, VEC, 64 * kConvMaxWaves * VEC);
  if (a->num_slots <= 0 || a->num_layers <= 0 || a->layer < 0 || a->layer >= a->num_layers)
    return fail(PK_ERR_INVALID, "%s: layer %d / layers %d / slots %d out of range", what,
                a->layer, a->num_layers, a->num_slots);
  if (!a->slots && a->batch > a->num_slots)
    return fail(PK_ERR_INVALID, "%s: batch %d exceeds %d slots", what, a->batch, a->num_slots);
  if (a->batch == 0) return PK_OK;
  if (!a->glu_in || !a->cache || !a->dw_weight || !a->ln_weight || !a->ln_bias || !a->out)
    return fail(PK_ERR_INVALID, "%s: a tensor pointer is NULL", what);
  const void* ptrs[7] = {a->glu_in, a->cache, a->dw_weight, a->ln_weight, a->ln_bias, a->out,
                         a->dw_bias ? a->dw_bias : a->ln_bias};
  for (const void* q : ptrs)
    if (!aligned16(q)) return fail(PK_ERR_INVALID, "%s: tensors must be 16-byte aligned", what);
  const int64_t strides[4] = {a->glu_in_stride_b, a->glu_in_stride_t, a->out_stride_b,
                              a->out_stride_t};
  for (int64_t st : strides)
    if (st < 0 || st % VEC != 0)
      return fail(PK_ERR_INVALID, "%s: strides must be non-negative multiples of %d elements",
                  what, VEC);
  if (a->chunk > 1 && (a->glu_in_stride_t < 2 * (int64_t)a->d_model ||
                       a->out_stride_t < (int64_t)a->d_model))
    return fail(PK_ERR_INVALID, "%s: frame strides overlap a frame's channels", what);
  if (!(a->ln_eps >= 0.f)) return fail(PK_ERR_INVALID, "%s: ln_eps must be >= 0", what);

  ConvK<ST> k{};
  k.h = static_cast<const ST*>(a->glu_in);
  k.h_sb = a->glu_in_stride_b;
  k.h_st = a->glu_in_stride_t;
  k.cache = static_cast<ST*>(a->cache);
  k.num_slots = a->num_slots;
  k.num_layers = a->num_layers;
  k.layer = a->layer;
  k.slots = a->slots;
  k.pad = a->pad_mask;
  k.lengths = a->lengths;
  k.len_scalar = a->length_scalar;
  k.w = static_cast<const ST*>(a->dw_weight);
  k.bias = static_cast<const ST*>(a->dw_bias);
  k.lnw = static_cast<const ST*>(a->ln_weight);
  k.lnb = static_cast<const ST*>(a->ln_bias);
  k.eps = a->ln_eps;
  k.out = static_cast<ST*>(a->out);
  k.o_sb = a->out_stride_b;
  k.o_st = a->out_stride_t;
  k.T = a->chunk;
  k.D = a->d_model;
  if (a->kernel != 3 && a->kernel != 5 && a->kernel != 7 && a->kernel != 9)
    return fail(PK_ERR_UNSUPPORTED, "%s: kernel size %d not built (3, 5, 7, 9)", what, a->kernel);
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "%s: cannot select device %d", what, a->device);
  switch (a->kernel) {
    case 3: return launch_conv<ST, 3>(k, a->batch, s);
    case 5: return launch_conv<ST, 5>(k, a->batch, s);
    case 7: return launch_conv<ST, 7>(k, a->batch, s);
    case 9: return launch_conv<ST, 9>(k, a->batch, s);
    default:
      return fail(PK_ERR_UNSUPPORTED, "%s: kernel size %d not built (3, 5, 7, 9)", what, a->kernel);
  }
}

constexpr int kResNormMaxNV = 8;  // 16-byte chunks a lane: d_model up to 512 chunks

template <typename ST, int NV>
int launch_resnorm(const ResNormK<ST>& k, hipStream_t s) {
  const dim3 grid((unsigned)((k.rows + kResNormRows - 1) / kResNormRows)), block(64u * kResNormRows);
  hipLaunchKernelGGL((resnorm_kernel<ST, NV>), grid, block, 0, s, k);
  return check_launch("pk_residual_norm");
}

template <typename ST>
int resnorm_typed(const pk_resnorm_args* a, hipStream_t s) {
  constexpr int VEC = Tr<ST>::VEC;
  const char* what = "pk_residual_norm";
  if (a->rows < 0) return fail(PK_ERR_INVALID, "%s: rows %d < 0", what, a->rows);
  if (a->d_model <= 0 || a->d_model % VEC != 0 || a->d_model > 64 * kResNormMaxNV * VEC)
    return fail(PK_ERR_INVALID, "%s: d_model %d must be a positive multiple of %d, at most %d", what,
                a->d_model, VEC, 64 * kResNormMaxNV * VEC);
  if (!(a->ln_eps >= 0.f)) return fail(PK_ERR_INVALID, "%s: ln_eps must be >= 0", what);
  if (!(a->alpha == a->alpha) || a->alpha == INFINITY || a->alpha == -INFINITY)
    return fail(PK_ERR_INVALID, "%s: alpha must be finite", what);
  if (a->rows == 0) return PK_OK;
  const void* ptrs[6] = {a->residual, a->branch, a->ln_weight, a->ln_bias, a->residual_out, a->norm_out};
  for (const void* q : ptrs) {
    if (!q) return fail(PK_ERR_INVALID, "%s: a tensor pointer is NULL", what);
    if (!aligned16(q)) return fail(PK_ERR_INVALID, "%s: tensors must be 16-byte aligned", what);
  }
  const int64_t strides[4] = {a->residual_stride, a->branch_stride, a->residual_out_stride, a->norm_out_stride};
  for (int64_t st : strides)
    if (st % VEC != 0 || (a->rows > 1 && st < a->d_model))
      return fail(PK_ERR_INVALID, "%s: row strides must be multiples of %d elements, at least d_model", what, VEC);
  ResNormK<ST> k{};
  k.res = static_cast<const ST*>(a->residual);
  k.res_s = a->residual_stride;
  k.br = static_cast<const ST*>(a->branch);
  k.br_s = a->branch_stride;
  k.lnw = static_cast<const ST*>(a->ln_weight);
  k.lnb = static_cast<const ST*>(a->ln_bias);
  k.rout = static_cast<ST*>(a->residual_out);
  k.rout_s = a->residual_out_stride;
  k.nout = static_cast<ST*>(a->norm_out);
  k.nout_s = a->norm_out_stride;
  k.alpha = a->alpha;
  k.eps = a->ln_eps;
  k.rows = a->rows;
  k.D = a->d_model;
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "%s: cannot select device %d", what, a->device);
  const int nv = (a->d_model / VEC + 63) / 64;
  if (nv <= 1) return launch_resnorm<ST, 1>(k, s);
  if (nv <= 2) return launch_resnorm<ST, 2>(k, s);
  if (nv <= 4) return launch_resnorm<ST, 4>(k, s);
  return launch_resnorm<ST, kResNormMaxNV>(k, s);
}

}  // namespace
}  // namespace pk

extern "C" int pk_residual_norm(const pk_resnorm_args* a, void* stream) {
  pk::clear_error();
  if (!a) return pk::fail(PK_ERR_INVALID, "pk_residual_norm: args is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case PK_DTYPE_F32: return pk::resnorm_typed<float>(a, s);
    case PK_DTYPE_F16: return pk::resnorm_typed<_Float16>(a, s);
    case PK_DTYPE_BF16: return pk::resnorm_typed<pk::bf16_t>(a, s);
    default: return pk::fail(PK_ERR_INVALID, "pk_residual_norm: unknown dtype %d", a->dtype);
  }
}

extern "C" int pk_conv_step(const pk_conv_args* a, void* stream) {
  pk::clear_error();
  if (!a) return pk::fail(PK_ERR_INVALID, "pk_conv_step: args is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case PK_DTYPE_F32: return pk::conv_typed<float>(a, s);
    case PK_DTYPE_F16: return pk::conv_typed<_Float16>(a, s);
    case PK_DTYPE_BF16: return pk::conv_typed<pk::bf16_t>(a, s);
    default: return pk::fail(PK_ERR_INVALID, "pk_conv_step: unknown dtype %d", a->dtype);
  }
}
