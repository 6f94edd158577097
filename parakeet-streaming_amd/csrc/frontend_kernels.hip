// gfx950 kernels of the streaming pre-encode front end, batched over streams
// (parakeet/modules/feature_extractor.py:63-151, parakeet/modules/subsample.py:30-179,
// parakeet/engine/model_runner.py:181-252).
//
//   fe_kernel         new samples -> each stream's sample ring; for every frame to
//                     emit: dither, pre-emphasis, Hann window, 512-point real FFT,
//                     power, Slaney mel, log -> the stream's mel ring.  One wave per
//                     frame: the real FFT is a 256-point complex FFT (even samples
//                     real, odd imaginary) as four radix-4 Stockham passes through a
//                     wave-private LDS buffer, then the split into the 257 real-input
//                     bins.  Twiddles come from sincospi into LDS once per workgroup.
//   subsample_kernel  the convolution stack of ConvSubsampling for one output frame
//                     and a tile of QT output frequency columns per workgroup, every
//                     intermediate in LDS: conv.0 (1 -> C, 3x3/2) as an MFMA over
//                     the 9 taps, ReLU, depthwise 3x3/2 on the vector ALUs, one
//                     64-channel group at a time; pointwise C x C as MFMA with the
//                     weight rows read as the module holds them; ReLU; depthwise
//                     3x3/2; pointwise + ReLU; the tile is written to the flattened
//                     [channel][freq] output row.  Only the rows and columns the
//                     tile's outputs depend on are computed: 15 input rows, 7 rows
//                     after conv.0, 3 after the first depthwise conv.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pk_common.h"
#include "pk_device.h"

namespace pk {

// ===========================================================================
// log-mel features

constexpr int kNfft = 512;
constexpr int kCplx = kNfft / 2;  // complex FFT points
constexpr int kBins = kNfft / 2 + 1;
constexpr int kFeWaves = 4;  // frames per workgroup
constexpr int kMaxMels = 128;

struct FeK {
  const pk_fe_stream* streams;
  const void* samples;
  int64_t s_stride;
  float* ring;
  float* mel;
  const float* window;
  const float* fb;
  const int32_t* fb_range;
  int32_t pcm, num_slots, ring_size, mel_rows, n_mels, win, hop, max_new, max_frames;
  float preemph, dither, guard;
  uint32_t seed_lo, seed_hi;
};

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): 10 rounds of two 32x32->64
// multiplies, Weyl key schedule.
__device__ static inline void philox4x32_10(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3,
                                            uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
}

// Standard normal for global sample i of one stream: Box-Muller on the first two
// Philox words, u1 = (r0 + 1) 2^-32, u2 = r1 2^-32.  v_cos_f32 takes revolutions.
__device__ static inline float dither_normal(int64_t i, uint32_t noise_id, uint32_t k0, uint32_t k1) {
  uint32_t c0 = (uint32_t)i, c1 = (uint32_t)((uint64_t)i >> 32), c2 = noise_id, c3 = 0u;
  philox4x32_10(c0, c1, c2, c3, k0, k1);
  const float u1 = ((float)c0 + 1.0f) * 2.3283064365386963e-10f;
  const float u2 = (float)c1 * 2.3283064365386963e-10f;
  return sqrtf(-2.0f * __logf(u1)) * __builtin_amdgcn_cosf(u2);
}

__device__ static inline float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// 4-point forward DFT in place.
__device__ static inline void dft4(float2* v) {
  const float2 t0 = make_float2(v[0].x + v[2].x, v[0].y + v[2].y);
  const float2 t1 = make_float2(v[0].x - v[2].x, v[0].y - v[2].y);
  const float2 t2 = make_float2(v[1].x + v[3].x, v[1].y + v[3].y);
  const float2 t3 = make_float2(v[1].x - v[3].x, v[1].y - v[3].y);
  v[0] = make_float2(t0.x + t2.x, t0.y + t2.y);
  v[2] = make_float2(t0.x - t2.x, t0.y - t2.y);
  v[1] = make_float2(t1.x + t3.y, t1.y - t3.x);  // t1 - i t3
  v[3] = make_float2(t1.x - t3.y, t1.y + t3.x);  // t1 + i t3
}

constexpr int kMaxWin = kNfft;
constexpr int kMaxHop = kNfft;
constexpr int kSpanMax = (kFeWaves - 1) * kMaxHop + kMaxWin + 1;  // samples the frames of a workgroup read
constexpr int kBand = 32;  // filterbank weights per band staged in LDS

template <int PCM>
__global__ void __launch_bounds__(64 * kFeWaves) fe_kernel(const FeK p) {
  __shared__ float2 tw[kCplx];   // e^{-2 pi i m / 256}
  __shared__ float2 tw2[kBins];  // e^{-2 pi i k / 512}, k <= 256
  __shared__ float2 buf[kFeWaves][kCplx];
  __shared__ float pw[kFeWaves][kBins + 3];
  __shared__ float xs[kSpanMax + 3];  // dithered samples of the workgroup's frames
  __shared__ float win_s[kMaxWin];
  __shared__ float fbw[kMaxMels][kBand];  // band m's weights from its first bin on

  const int b = blockIdx.y;
  const pk_fe_stream s = p.streams[b];
  if (s.slot < 0 || s.slot >= p.num_slots || s.n_new < 0 || s.n_new > p.max_new || s.n_frames < 0 ||
      s.n_frames > p.max_frames || s.frame0 < 0 || s.sample_base < 0)
    return;  // uniform over the workgroup
  const int64_t total = s.sample_base + s.n_new;
  const int rmask = p.ring_size - 1;
  float* ring = p.ring + (int64_t)s.slot * p.ring_size;
  const int tid = threadIdx.x;

  // (with no new samples the input may be NULL: read the ring instead, discarded)
  const void* smp = p.samples ? p.samples : (const void*)p.ring;
  const int64_t sst = p.samples ? b * p.s_stride : 0;
  auto sample_in = [&](int64_t o) -> float {
    if constexpr (PCM == PK_PCM_S16)
      return (float)((const int16_t*)smp)[sst + o] * (1.0f / 32768.0f);
    else
      return ((const float*)smp)[sst + o];
  };
  // new samples -> ring (this call reads only ring entries of older samples);
  // four loads per thread in flight before their stores
  constexpr int kCopy = 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + tid; i0 < s.n_new; i0 += kCopy * stride) {
    float x[kCopy];
#pragma unroll
    for (int u = 0; u < kCopy; ++u) x[u] = sample_in(min(i0 + u * stride, (int64_t)s.n_new - 1));
#pragma unroll
    for (int u = 0; u < kCopy; ++u)
      if (i0 + u * stride < s.n_new) ring[(s.sample_base + i0 + u * stride) & rmask] = x[u];
  }
  const int j0 = blockIdx.x * kFeWaves;
  if (j0 >= s.n_frames) return;  // no frame for this workgroup
  const int nf = min(kFeWaves, s.n_frames - j0);
  const int wl = (kNfft - p.win) / 2;
  const int64_t f0 = (int64_t)s.frame0 + j0;
  const int64_t span0 = f0 * p.hop - kNfft / 2 + wl - 1;  // global index of xs[0]
  const int span = (nf - 1) * p.hop + p.win + 1;

  // staging, one global round trip per phase: every load of a phase is issued
  // into registers before any of them is stored
  __shared__ int2 rng_s[kMaxMels];
  constexpr int kXsPer = (kSpanMax + 64 * kFeWaves - 1) / (64 * kFeWaves);
  constexpr int kFbPer = kMaxMels * kBand / (64 * kFeWaves);
  constexpr int kWinPer = kMaxWin / (64 * kFeWaves);
  float xr[kXsPer], wr[kWinPer];
  const int mc = min(tid, p.n_mels - 1);
  const int2 rr = make_int2(p.fb_range[2 * mc], p.fb_range[2 * mc + 1]);
#pragma unroll
  for (int u = 0; u < kWinPer; ++u) wr[u] = p.window[min(tid + u * 64 * kFeWaves, p.win - 1)];
  // raw sample i from this call's input or the ring (0 outside [0, total)):
  // unconditional loads from clamped addresses
#pragma unroll
  for (int u = 0; u < kXsPer; ++u) {
    const int i = tid + u * 64 * kFeWaves;
    const int64_t g = span0 + i;
    const bool ok = i < span && g >= 0 && g < total;
    const bool fresh = g >= s.sample_base;
    const float xn = sample_in(ok && fresh ? g - s.sample_base : 0);
    const float xo = ring[ok && !fresh ? (g & rmask) : 0];
    const float x = fresh ? xn : xo;
    xr[u] = ok ? x : 0.f;
  }
  if (tid < p.n_mels) rng_s[tid] = make_int2(max(rr.x, 0), min(rr.y, kBins));
#pragma unroll
  for (int u = 0; u < kWinPer; ++u) {
    const int i = tid + u * 64 * kFeWaves;
    if (i < p.win) win_s[i] = wr[u];
  }
#pragma unroll
  for (int u = 0; u < kXsPer; ++u) {
    const int i = tid + u * 64 * kFeWaves;
    const int64_t g = span0 + i;
    float x = xr[u];
    if (p.dither != 0.f && g >= 0 && g < total) x += p.dither * dither_normal(g, s.noise_id, p.seed_lo, p.seed_hi);
    if (i < span) xs[i] = x;
  }
  __syncthreads();
  // band m's weights from its first bin (the bins past kBand are read from fb)
  float fr[kFbPer];
#pragma unroll
  for (int u = 0; u < kFbPer; ++u) {
    const int i = tid + u * 64 * kFeWaves;
    const int m = i / kBand, k = rng_s[m].x + i % kBand;
    fr[u] = (m < p.n_mels && k < rng_s[m].y) ? p.fb[(int64_t)m * kBins + k] : 0.f;
  }
  for (int m = tid; m < kBins; m += blockDim.x) {
    float sn, cs;
    if (m < kCplx) {
      sincospif((float)m / 128.0f, &sn, &cs);
      tw[m] = make_float2(cs, -sn);
    }
    sincospif((float)m / 256.0f, &sn, &cs);
    tw2[m] = make_float2(cs, -sn);
  }
#pragma unroll
  for (int u = 0; u < kFbPer; ++u) {
    const int i = tid + u * 64 * kFeWaves;
    fbw[i / kBand][i % kBand] = fr[u];
  }
  __syncthreads();

  const int wave = tid >> 6, lane = tid & 63;
  if (wave >= nf) return;  // no barrier below this point
  const int64_t f = f0 + wave;
  const int64_t base = f * p.hop - kNfft / 2;
  const int off = wave * p.hop - wl + 1;  // xs index of frame sample n is off + n
  // windowed, pre-emphasised frame sample n (0 <= n < 512)
  auto frame_val = [&](int n) -> float {
    if (n < wl || n >= wl + p.win) return 0.f;
    const int64_t i = base + n;
    if (i < 0 || i >= total) return 0.f;
    return (xs[off + n] - p.preemph * xs[off + n - 1]) * win_s[n - wl];
  };

  // z[n] = v[2n] + i v[2n+1]; lane holds z[lane + 64 r]
  float2 v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int n = 2 * (lane + 64 * r);
    v[r] = make_float2(frame_val(n), frame_val(n + 1));
  }
  float2* bw = buf[wave];
  // radix-4 Stockham passes: span Ns = 1, 4, 16, 64
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int Ns = 1 << (2 * pass);
    const int k = lane & (Ns - 1);
    if (pass) {
#pragma unroll
      for (int r = 1; r < 4; ++r) v[r] = cmul(v[r], tw[(r * k * 64) >> (2 * pass)]);
    }
    dft4(v);
    const int d = ((lane >> (2 * pass)) << (2 * pass + 2)) + k;
    wave_lds_sync();  // the previous pass's reads of bw are done
#pragma unroll
    for (int r = 0; r < 4; ++r) bw[d + r * Ns] = v[r];
    wave_lds_sync();
    if (pass < 3) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = bw[lane + 64 * r];
    }
  }
  // real-input bins: X[k] = E[k] + W^k O[k], E/O from Z[k] and conj(Z[256-k])
  float* pwv = pw[wave];
  for (int kk = lane; kk < kBins; kk += 64) {
    const float2 zk = bw[kk & (kCplx - 1)], zm = bw[(kCplx - kk) & (kCplx - 1)];
    const float er = 0.5f * (zk.x + zm.x), ei = 0.5f * (zk.y - zm.y);
    const float orr = 0.5f * (zk.y + zm.y), oi = -0.5f * (zk.x - zm.x);
    const float2 w = tw2[kk];
    const float xr = er + (w.x * orr - w.y * oi), xi = ei + (w.x * oi + w.y * orr);
    pwv[kk] = xr * xr + xi * xi;
  }
  wave_lds_sync();
  float* mrow = p.mel + ((int64_t)s.slot * p.mel_rows + (f & (p.mel_rows - 1))) * p.n_mels;
  for (int m = lane; m < p.n_mels; m += 64) {
    const int lo = rng_s[m].x, hi = rng_s[m].y;
    float acc = 0.f;
    for (int kk = lo; kk < hi; ++kk)
      acc += (kk - lo < kBand ? fbw[m][kk - lo] : p.fb[(int64_t)m * kBins + kk]) * pwv[kk];
    mrow[m] = logf(acc + p.guard);
  }
}

// ===========================================================================
// convolution subsampling

// One MFMA step over a 16-byte K chunk per lane:
//   lane l holds A[l%16][VEC*(l/16) + e] and B[VEC*(l/16) + e][l%16], e < VEC;
//   D: lane l holds D[4*(l/16) + i][l%16], i < 4.
// fp16/bf16: one 16x16x32 instruction; fp32: four 16x16x4 (K element e of every
// lane group in instruction e).
template <typename ST>
struct MmaK;
template <>
struct MmaK<_Float16> {
  typedef _Float16 H8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4_t step(u32x4 a, u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(H8, a), __builtin_bit_cast(H8, b), c, 0,
                                                  0, 0);
  }
};
template <>
struct MmaK<bf16_t> {
  typedef __bf16 H8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4_t step(u32x4 a, u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(H8, a), __builtin_bit_cast(H8, b), c, 0,
                                                   0, 0);
  }
};
template <>
struct MmaK<float> {
  __device__ static inline f32x4_t step(u32x4 a, u32x4 b, f32x4_t c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    return c;
  }
};

template <typename ST>
struct Chunk {
  static constexpr int VEC = 16 / sizeof(ST);
  ST v[VEC];
};

template <typename ST>
struct SubK {
  const pk_sub_stream* streams;
  const float* in;
  const ST *w0, *b0, *w2, *b2, *w3, *b3, *w5, *b5, *w6, *b6;
  ST* out;
  int32_t in_slots, in_rows, in_ring, F, C, out_rows, max_out;
};

constexpr int kSubWaves = 8;
constexpr int kSubThreads = 64 * kSubWaves;
constexpr int kCG = 64;  // channels per conv.0 / first depthwise group

// output length of a 3x3 stride-2 conv padded (2, 1): (n + 2 + 1 - 3) / 2 + 1
__host__ __device__ static inline int half_up(int n) { return n / 2 + 1; }

template <int A, int B>
struct cmax {
  static constexpr int v = A > B ? A : B;
};

template <typename ST, int QT, int C>
struct SubGeom {
  static constexpr int VEC = 16 / sizeof(ST);
  static constexpr int XR = 15, XC = 8 * QT + 7;  // input rows / cols of the tile
  static constexpr int A1R = 7, A1C = 4 * QT + 3;  // after conv.0
  static constexpr int A2R = 3, A2C = 2 * QT + 1;  // after the first depthwise conv
  static constexpr int M1 = A1R * A1C, T1 = (M1 + 15) / 16;
  static constexpr int M2 = A2R * A2C, T2 = (M2 + 15) / 16;
  // LDS rows of per-position channel vectors are padded by one 16-byte chunk so
  // the 16 positions of an MFMA fragment fall on distinct banks
  static constexpr int RS = C + VEC;    // a2 (before and after the pointwise conv), a3
  static constexpr int A1S = kCG + VEC;  // a1 (one channel group)
  // regA: a1 [T1*16][A1S] -> a2 [T2*16][RS] -> output tile [C][QT]
  static constexpr int REG_A = cmax<cmax<T1 * 16 * A1S, T2 * 16 * RS>::v, C * QT>::v;
  // regB: a2 before the pointwise conv [T2*16][RS] -> a3 before it [16][RS]
  static constexpr int REG_B = cmax<T2, 1>::v * 16 * RS;
  static constexpr int T1W = (T1 + kSubWaves - 1) / kSubWaves;  // conv.0 position tiles per wave
  static constexpr int KS = C / (4 * VEC);                      // K steps of a pointwise conv
  static constexpr int NT = C / 16;                             // channel tiles of a pointwise conv
  static constexpr int NPW = (NT + kSubWaves - 1) / kSubWaves;  // channel tiles per wave
  static constexpr int CH = C / VEC;                            // 16-byte channel chunks
  static constexpr int KP = 4 * VEC;                            // conv.0 taps padded to one K step
};

// Weight rows W[n][k] of a pointwise conv ([C out][C in], as the module holds
// them) for the wave's channel tiles: the MFMA A operand, lane l holding
// W[tile*16 + l%16][kstep*4*VEC + VEC*(l/16) + e].
template <int NPW, int KS, int C, typename ST>
__device__ static inline void load_pw(u32x4 (&b)[NPW][KS], const ST* w, int wave, int lr, int lg) {
  constexpr int VEC = 16 / sizeof(ST);
#pragma unroll
  for (int h = 0; h < NPW; ++h) {
    const int n = (wave * NPW + h) * 16 + lr;
    if (n >= C) continue;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) b[h][kk] = ld16(w + (int64_t)n * C + kk * 4 * VEC + VEC * lg);
  }
}

// four consecutive elements from fp32
template <typename ST>
__device__ static inline void store4(ST* dst, const float* v) {
  if constexpr (sizeof(ST) == 4) {
    *reinterpret_cast<u32x4*>(dst) = Tr<ST>::pack(v);
  } else {
    Chunk<ST> c;
#pragma unroll
    for (int e = 0; e < 4; ++e) c.v[e] = to_st<ST>(v[e]);
    const u32x4 w = __builtin_bit_cast(u32x4, c);
    *reinterpret_cast<uint2*>(dst) = make_uint2(w.x, w.y);
  }
}

// One output frame t of the stack for output columns [p0, p0 + QT) per
// workgroup.  MFMA operands: the weights are A (rows = output channels), the
// activations B (columns = positions), so lane l holds 4 consecutive channels
// 4*(l/16) .. of position l%16 and writes them as one 8- or 16-byte chunk.
// Depthwise convs run on 16-byte channel chunks per thread.
template <typename ST, int QT, int C>
__global__ void __launch_bounds__(kSubThreads) subsample_kernel(const SubK<ST> p) {
  typedef SubGeom<ST, QT, C> G;
  constexpr int VEC = G::VEC;
  static_assert(C <= kSubThreads && C % kCG == 0, "one bias per thread, whole channel groups");
  __shared__ __align__(16) ST xin[G::XR * G::XC];
  __shared__ __align__(16) ST regA[G::REG_A];
  __shared__ __align__(16) ST regB[G::REG_B];
  __shared__ __align__(16) ST w0p[C * G::KP];  // conv.0 weights [C][KP], taps 9.. zero
  __shared__ __align__(16) ST w2t[9 * C];   // depthwise weights tap-major [tap][C]
  __shared__ __align__(16) ST w5t[9 * C];
  __shared__ __align__(16) float bsm[5][C];  // biases of conv.0/2/3/5/6, 0 where absent

  const int b = blockIdx.z;
  const pk_sub_stream s = p.streams[b];
  const int j = blockIdx.x;
  if (j >= s.n_out || j >= p.max_out || s.slot < 0 || s.slot >= p.in_slots || s.rows < 0 || s.length < 0 ||
      s.length > s.rows || s.drop < 0 || s.out_row < 0 || s.out_row + s.n_out > p.out_rows)
    return;
  if (!p.in_ring && (s.row0 < 0 || (int64_t)s.row0 + s.rows > p.in_rows)) return;
  const int t = s.drop + j;  // output frame of the stack
  const int L3 = half_up(half_up(half_up(s.rows)));
  if (t >= L3) return;
  const int F = p.F;
  const int F1 = half_up(F), F2 = half_up(F1), F3 = half_up(F2);
  const int p0 = blockIdx.y * QT;  // first output column of the tile
  if (p0 >= F3) return;
  const int qv = min(QT, F3 - p0);  // valid output columns
  const int len1 = half_up(s.length), len2 = half_up(len1), len3 = half_up(len2);
  ST* orow = p.out + (int64_t)(s.out_row + j) * C * F3;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  if (t >= len3) {  // masked output frame (subsample.py:47)
    for (int i = tid; i < C * qv; i += kSubThreads) orow[(i / qv) * F3 + p0 + i % qv] = to_st<ST>(0.f);
    return;
  }

  // every global load before the convolutions is issued into registers first
  // (one round trip): the small weights, biases and the input tile (stored to
  // LDS), then the first pointwise conv's weights (kept in registers).  The
  // loads are unconditional, from clamped addresses, so none waits in a branch.
  constexpr int kWPer = (C * 9 + kSubThreads - 1) / kSubThreads;
  constexpr int kXPer = (G::XR * G::XC + kSubThreads - 1) / kSubThreads;
  ST w0r[kWPer], w2r[kWPer], w5r[kWPer], brs0[kWPer];
#pragma unroll
  for (int u = 0; u < kWPer; ++u) {
    const int i = min(tid + u * kSubThreads, C * 9 - 1);
    w0r[u] = p.w0[i];
    w2r[u] = p.w2[i];
    w5r[u] = p.w5[i];
    brs0[u] = (p.b0 ? p.b0 : p.w0)[i / 9];  // conv.0 bias of the channel whose tap 0 this is
  }
  ST brs[5];
  {
    const int c = min(tid, C - 1);
    brs[0] = (p.b0 ? p.b0 : p.w0)[c];
    brs[1] = (p.b2 ? p.b2 : p.w0)[c];
    brs[2] = (p.b3 ? p.b3 : p.w0)[c];
    brs[3] = (p.b5 ? p.b5 : p.w0)[c];
    brs[4] = (p.b6 ? p.b6 : p.w0)[c];
  }
  // input tile: rows 8t-14 .., cols 8p0-14 .., masked by length
  float xr[kXPer];
  {
    const int r0 = 8 * t - 14, c0 = 8 * p0 - 14;
    const float* inb = p.in + (int64_t)s.slot * p.in_rows * F;
    const int rmask = p.in_rows - 1;
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
      const int i = tid + u * kSubThreads;
      const int rr = i / G::XC, cc = i - rr * G::XC;
      const int gr = r0 + rr, gc = c0 + cc;
      const bool ok = i < G::XR * G::XC && gr >= 0 && gr < s.length && gc >= 0 && gc < F;
      const int row = p.in_ring ? ((s.row0 + gr) & rmask) : s.row0 + gr;
      const float v = inb[ok ? (int64_t)row * F + gc : 0];
      xr[u] = ok ? v : 0.f;
    }
  }
  u32x4 bq[G::NPW][G::KS];
  load_pw<G::NPW, G::KS, C>(bq, p.w3, wave, lr, lg);
  const float br[5] = {p.b0 ? from_st(brs[0]) : 0.f, p.b2 ? from_st(brs[1]) : 0.f, p.b3 ? from_st(brs[2]) : 0.f,
                       p.b5 ? from_st(brs[3]) : 0.f, p.b6 ? from_st(brs[4]) : 0.f};
  for (int i = tid; i < C * G::KP; i += kSubThreads) w0p[i] = to_st<ST>(0.f);  // tap padding
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kWPer; ++u) {
    const int i = tid + u * kSubThreads;
    if (i < C * 9) {
      const int c = i / 9, k = i - c * 9;
      w0p[c * G::KP + k] = w0r[u];
      if (k == 0) w0p[c * G::KP + 9] = p.b0 ? brs0[u] : to_st<ST>(0.f);  // bias against the im2col's 1
      w2t[k * C + c] = w2r[u];
      w5t[k * C + c] = w5r[u];
    }
  }
  if (tid < C) {
#pragma unroll
    for (int k = 0; k < 5; ++k) bsm[k][tid] = br[k];
  }
#pragma unroll
  for (int u = 0; u < kXPer; ++u) {
    const int i = tid + u * kSubThreads;
    if (i < G::XR * G::XC) xin[i] = to_st<ST>(xr[u]);
  }
  __syncthreads();

  // conv.0 B operand: the 9 taps of each position (one K chunk), per wave its
  // position tiles wave + 8 u
  u32x4 a0[G::T1W];
#pragma unroll
  for (int u = 0; u < G::T1W; ++u) {
    const int m = (wave + kSubWaves * u) * 16 + lr;
    const int mm = min(m, G::M1 - 1);
    const int i = mm / G::A1C, q = mm - i * G::A1C;
    Chunk<ST> ch;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int tap = VEC * lg + e;
      const int tc = min(tap, 8);
      const ST v = xin[(2 * i + tc / 3) * G::XC + 2 * q + tc % 3];
      ch.v[e] = (tap < 9 && m < G::M1) ? v : to_st<ST>(tap == 9 ? 1.f : 0.f);
    }
    a0[u] = __builtin_bit_cast(u32x4, ch);
  }
  // validity of the wave's conv.0 positions (rows 4t-6 .., cols 4p0-6 ..)
  bool ok1[G::T1W];
#pragma unroll
  for (int u = 0; u < G::T1W; ++u) {
    const int m = (wave + kSubWaves * u) * 16 + lr;
    const int i = m / G::A1C, q = m - i * G::A1C;
    const int gr = 4 * t - 6 + i, gq = 4 * p0 - 6 + q;
    ok1[u] = m < G::M1 && gr >= 0 && gr < len1 && gq >= 0 && gq < F1;
  }

  ST* a1 = regA;
  ST* a2p = regB;
#pragma unroll 1
  for (int cg = 0; cg < C; cg += kCG) {
    // conv.0 for channels cg .. cg+63 -> bias, mask, ReLU -> a1 [T1*16][A1S]
    u32x4 aw[kCG / 16];
#pragma unroll
    for (int nt = 0; nt < kCG / 16; ++nt)
      aw[nt] = *reinterpret_cast<const u32x4*>(&w0p[(cg + nt * 16 + lr) * G::KP + VEC * lg]);
    f32x4_t d[G::T1W][kCG / 16];
#pragma unroll
    for (int u = 0; u < G::T1W; ++u)
#pragma unroll
      for (int nt = 0; nt < kCG / 16; ++nt)
        d[u][nt] = wave + kSubWaves * u < G::T1 ? MmaK<ST>::step(aw[nt], a0[u], f32x4_t{0.f, 0.f, 0.f, 0.f})
                                                 : f32x4_t{0.f, 0.f, 0.f, 0.f};
    // the bias came in through tap 9; ReLU before the one rounding to the
    // storage type is the same as after it
#pragma unroll
    for (int u = 0; u < G::T1W; ++u) {
      const int mt = wave + kSubWaves * u;
      if (mt < G::T1) {
#pragma unroll
        for (int nt = 0; nt < kCG / 16; ++nt) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = ok1[u] ? fmaxf(d[u][nt][e], 0.f) : 0.f;
          store4<ST>(&a1[(mt * 16 + lr) * G::A1S + nt * 16 + 4 * lg], v);
        }
      }
    }
    __syncthreads();
    // first depthwise conv for the group -> a2p [M2][RS]: a thread owns one
    // 16-byte chunk of channels (weights held in registers) and positions
    // m, m + kPS, ...
    {
      constexpr int kGC = kCG / VEC;              // chunks per group
      constexpr int kPS = kSubThreads / kGC;      // positions per sweep
      const int cc = (tid % kGC) * VEC;
      float w[9][VEC], bias[VEC];
#pragma unroll
      for (int k = 0; k < 9; ++k) Tr<ST>::unpack(*reinterpret_cast<const u32x4*>(&w2t[k * C + cg + cc]), w[k]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) bias[e] = bsm[1][cg + cc + e];
#pragma unroll
      for (int m0 = 0; m0 < G::M2; m0 += kPS) {
        const int m = m0 + tid / kGC;
        if (m < G::M2) {
          const int si = m / G::A2C, pp = m - si * G::A2C;
          float acc[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] = bias[e];
#pragma unroll
          for (int kt = 0; kt < 3; ++kt)
#pragma unroll
            for (int kf = 0; kf < 3; ++kf) {
              float a[VEC];
              Tr<ST>::unpack(
                  *reinterpret_cast<const u32x4*>(&a1[((2 * si + kt) * G::A1C + 2 * pp + kf) * G::A1S + cc]), a);
#pragma unroll
              for (int e = 0; e < VEC; ++e) acc[e] += w[kt * 3 + kf][e] * a[e];
            }
          *reinterpret_cast<u32x4*>(&a2p[m * G::RS + cg + cc]) = Tr<ST>::pack(acc);
        }
      }
    }
    __syncthreads();
  }

  // pointwise conv.3 (C x C): wave owns channel tiles wave*NPW .. -> bias, mask,
  // ReLU -> a2 [T2*16][RS] (rows past M2 are scratch)
  ST* a2 = regA;
  const bool pw_active = wave * G::NPW < G::NT;
  {
    f32x4_t acc[G::T2][G::NPW];
#pragma unroll
    for (int mt = 0; mt < G::T2; ++mt)
#pragma unroll
      for (int h = 0; h < G::NPW; ++h) acc[mt][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (pw_active) {
#pragma unroll
      for (int kk = 0; kk < G::KS; ++kk) {
        const int k = kk * 4 * VEC + VEC * lg;
#pragma unroll
        for (int mt = 0; mt < G::T2; ++mt) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(a2p + (mt * 16 + lr) * G::RS + k);
#pragma unroll
          for (int h = 0; h < G::NPW; ++h) acc[mt][h] = MmaK<ST>::step(bq[h][kk], x, acc[mt][h]);
        }
      }
    }
    // the second pointwise conv's weights load while this epilogue and the
    // second depthwise conv run
    load_pw<G::NPW, G::KS, C>(bq, p.w6, wave, lr, lg);
    if (pw_active) {
#pragma unroll
      for (int mt = 0; mt < G::T2; ++mt) {
        const int m = mt * 16 + lr;
        const int si = m / G::A2C, pp = m - si * G::A2C;
        const int gs = 2 * t - 2 + si, gp = 2 * p0 - 2 + pp;
        const bool ok = m < G::M2 && gs >= 0 && gs < len2 && gp >= 0 && gp < F2;
#pragma unroll
        for (int h = 0; h < G::NPW; ++h) {
          const int c0 = (wave * G::NPW + h) * 16 + 4 * lg;
          const float4 bias = *reinterpret_cast<const float4*>(&bsm[2][c0]);
          float v[4] = {acc[mt][h][0] + bias.x, acc[mt][h][1] + bias.y, acc[mt][h][2] + bias.z,
                        acc[mt][h][3] + bias.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = ok ? fmaxf(v[e], 0.f) : 0.f;
          store4<ST>(&a2[m * G::RS + c0], v);
        }
      }
    }
  }
  __syncthreads();

  // second depthwise conv -> a3p [QT][RS]
  ST* a3p = regB;
  for (int it = tid; it < QT * G::CH; it += kSubThreads) {
    const int q = it / G::CH, cc = (it - q * G::CH) * VEC;
    float acc[VEC];
    {
      const float4* bb = reinterpret_cast<const float4*>(&bsm[3][cc]);
#pragma unroll
      for (int e = 0; e < VEC; e += 4) {
        const float4 x = bb[e / 4];
        acc[e] = x.x;
        acc[e + 1] = x.y;
        acc[e + 2] = x.z;
        acc[e + 3] = x.w;
      }
    }
#pragma unroll
    for (int kt = 0; kt < 3; ++kt)
#pragma unroll
      for (int kf = 0; kf < 3; ++kf) {
        float a[VEC], w[VEC];
        Tr<ST>::unpack(*reinterpret_cast<const u32x4*>(&a2[(kt * G::A2C + 2 * q + kf) * G::RS + cc]), a);
        Tr<ST>::unpack(*reinterpret_cast<const u32x4*>(&w5t[(kt * 3 + kf) * C + cc]), w);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += w[e] * a[e];
      }
    *reinterpret_cast<u32x4*>(&a3p[q * G::RS + cc]) = Tr<ST>::pack(acc);
  }
  __syncthreads();

  // pointwise conv.6 + ReLU -> flattened tile [C][QT] in regA
  ST* ot = regA;
  if (pw_active) {
    f32x4_t acc[G::NPW];
#pragma unroll
    for (int h = 0; h < G::NPW; ++h) acc[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < G::KS; ++kk) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(a3p + lr * G::RS + kk * 4 * VEC + VEC * lg);
#pragma unroll
      for (int h = 0; h < G::NPW; ++h) acc[h] = MmaK<ST>::step(bq[h][kk], x, acc[h]);
    }
    if (lr < QT) {
#pragma unroll
      for (int h = 0; h < G::NPW; ++h) {
        const int c0 = (wave * G::NPW + h) * 16 + 4 * lg;
        const float4 bias = *reinterpret_cast<const float4*>(&bsm[4][c0]);
        const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) ot[(c0 + e) * QT + lr] = to_st<ST>(fmaxf(acc[h][e] + bv[e], 0.f));
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < C * qv; i += kSubThreads) {
    const int c = i / qv, q = i - c * qv;
    orow[c * F3 + p0 + q] = ot[c * QT + q];
  }
}

// ===========================================================================
// host side

static bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

template <typename ST, int QT, int C>
static int launch_sub(const pk_sub_args* a, hipStream_t st) {
  SubK<ST> k;
  k.streams = a->streams;
  k.in = a->feats;
  k.w0 = (const ST*)a->w0;
  k.b0 = (const ST*)a->b0;
  k.w2 = (const ST*)a->w2;
  k.b2 = (const ST*)a->b2;
  k.w3 = (const ST*)a->w3;
  k.b3 = (const ST*)a->b3;
  k.w5 = (const ST*)a->w5;
  k.b5 = (const ST*)a->b5;
  k.w6 = (const ST*)a->w6;
  k.b6 = (const ST*)a->b6;
  k.out = (ST*)a->out;
  k.in_slots = a->feat_slots;
  k.in_rows = a->feat_rows;
  k.in_ring = a->feat_ring;
  k.F = a->n_mels;
  k.C = C;
  k.out_rows = a->out_rows;
  k.max_out = a->max_out;
  const int F3 = half_up(half_up(half_up(a->n_mels)));
  const dim3 grid(a->max_out, (F3 + QT - 1) / QT, a->batch);
  hipLaunchKernelGGL((subsample_kernel<ST, QT, C>), grid, dim3(kSubThreads), 0, st, k);
  return check_launch("pk_subsample");
}

template <typename ST, int QT>
static int launch_sub_c(const pk_sub_args* a, hipStream_t st) {
  switch (a->channels) {
    case 64:
      return launch_sub<ST, QT, 64>(a, st);
    case 128:
      return launch_sub<ST, QT, 128>(a, st);
    default:
      return launch_sub<ST, QT, 256>(a, st);
  }
}

}  // namespace pk

using namespace pk;

extern "C" int pk_fe_step(const pk_fe_args* a, void* stream) {
  clear_error();
  if (!a) return fail(PK_ERR_INVALID, "pk_fe_step: args is NULL");
  if (a->batch < 0 || a->max_new < 0 || a->max_frames < 0)
    return fail(PK_ERR_INVALID, "pk_fe_step: negative batch/max_new/max_frames");
  if (a->n_fft != kNfft) return fail(PK_ERR_UNSUPPORTED, "pk_fe_step: n_fft %d (only 512 is built)", a->n_fft);
  if (a->win_length < 1 || a->win_length > a->n_fft || (a->n_fft - a->win_length) % 2)
    return fail(PK_ERR_INVALID, "pk_fe_step: win_length %d must be in [1, n_fft] with n_fft - win even",
                a->win_length);
  if (a->hop < 1 || a->hop > kMaxHop) return fail(PK_ERR_INVALID, "pk_fe_step: hop %d not in [1, %d]", a->hop, kMaxHop);
  if (a->n_mels < 1 || a->n_mels > kMaxMels)
    return fail(PK_ERR_UNSUPPORTED, "pk_fe_step: n_mels %d not in [1, %d]", a->n_mels, kMaxMels);
  if (!pow2(a->ring_size) || !pow2(a->mel_ring_rows))
    return fail(PK_ERR_INVALID, "pk_fe_step: ring_size %d and mel_ring_rows %d must be powers of two",
                a->ring_size, a->mel_ring_rows);
  if (a->max_frames > a->mel_ring_rows)
    return fail(PK_ERR_INVALID, "pk_fe_step: max_frames %d exceeds the mel ring (%d rows)", a->max_frames,
                a->mel_ring_rows);
  if (a->max_new > a->ring_size)
    return fail(PK_ERR_INVALID, "pk_fe_step: max_new %d exceeds the sample ring (%d)", a->max_new, a->ring_size);
  if (a->pcm_dtype != PK_PCM_S16 && a->pcm_dtype != PK_PCM_F32)
    return fail(PK_ERR_INVALID, "pk_fe_step: pcm_dtype %d", a->pcm_dtype);
  if (a->num_slots < 1) return fail(PK_ERR_INVALID, "pk_fe_step: num_slots %d", a->num_slots);
  if (a->samples_stride < a->max_new) return fail(PK_ERR_INVALID, "pk_fe_step: samples_stride < max_new");
  if (a->batch > 65535) return fail(PK_ERR_UNSUPPORTED, "pk_fe_step: batch %d > 65535", a->batch);
  if (a->batch == 0 || (a->max_new == 0 && a->max_frames == 0)) return PK_OK;
  if (!a->streams || !a->sample_ring || !a->mel_ring || !a->window || !a->fb || !a->fb_range ||
      (a->max_new > 0 && !a->samples))
    return fail(PK_ERR_INVALID, "pk_fe_step: NULL pointer");
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "pk_fe_step: cannot select device %d", a->device);
  FeK k;
  k.streams = a->streams;
  k.samples = a->samples;
  k.s_stride = a->samples_stride;
  k.ring = a->sample_ring;
  k.mel = a->mel_ring;
  k.window = a->window;
  k.fb = a->fb;
  k.fb_range = a->fb_range;
  k.pcm = a->pcm_dtype;
  k.num_slots = a->num_slots;
  k.ring_size = a->ring_size;
  k.mel_rows = a->mel_ring_rows;
  k.n_mels = a->n_mels;
  k.win = a->win_length;
  k.hop = a->hop;
  k.max_new = a->max_new;
  k.max_frames = a->max_frames;
  k.preemph = a->preemph;
  k.dither = a->dither;
  k.guard = a->log_guard;
  k.seed_lo = (uint32_t)a->seed;
  k.seed_hi = (uint32_t)(a->seed >> 32);
  const int gx = a->max_frames > 0 ? (a->max_frames + kFeWaves - 1) / kFeWaves : 1;
  if (a->pcm_dtype == PK_PCM_S16)
    hipLaunchKernelGGL(fe_kernel<PK_PCM_S16>, dim3(gx, a->batch), dim3(64 * kFeWaves), 0, (hipStream_t)stream, k);
  else
    hipLaunchKernelGGL(fe_kernel<PK_PCM_F32>, dim3(gx, a->batch), dim3(64 * kFeWaves), 0, (hipStream_t)stream, k);
  return check_launch("pk_fe_step");
}

extern "C" int pk_subsample(const pk_sub_args* a, void* stream) {
  clear_error();
  if (!a) return fail(PK_ERR_INVALID, "pk_subsample: args is NULL");
  if (a->batch < 0 || a->max_out < 0 || a->out_rows < 0)
    return fail(PK_ERR_INVALID, "pk_subsample: negative batch/max_out/out_rows");
  if (a->dtype != PK_DTYPE_F32 && a->dtype != PK_DTYPE_F16 && a->dtype != PK_DTYPE_BF16)
    return fail(PK_ERR_INVALID, "pk_subsample: dtype %d", a->dtype);
  if (a->channels != 64 && a->channels != 128 && a->channels != 256)
    return fail(PK_ERR_UNSUPPORTED, "pk_subsample: channels %d (built: 64, 128, 256)", a->channels);
  if (a->n_mels < 1 || a->n_mels > kMaxMels)
    return fail(PK_ERR_UNSUPPORTED, "pk_subsample: n_mels %d not in [1, %d]", a->n_mels, kMaxMels);
  if (a->feat_slots < 1 || a->feat_rows < 1) return fail(PK_ERR_INVALID, "pk_subsample: empty features");
  if (a->feat_ring && !pow2(a->feat_rows))
    return fail(PK_ERR_INVALID, "pk_subsample: feat_rows %d must be a power of two for a ring", a->feat_rows);
  if (a->batch == 0 || a->max_out == 0) return PK_OK;
  if (!a->streams || !a->feats || !a->w0 || !a->w2 || !a->w3 || !a->w5 || !a->w6 || !a->out)
    return fail(PK_ERR_INVALID, "pk_subsample: NULL pointer");
  if (!aligned16(a->w3) || !aligned16(a->w6))
    return fail(PK_ERR_INVALID, "pk_subsample: pointwise weights must be 16-byte aligned");
  if (a->batch > 65535) return fail(PK_ERR_UNSUPPORTED, "pk_subsample: batch %d > 65535", a->batch);
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "pk_subsample: cannot select device %d", a->device);
  const hipStream_t st = (hipStream_t)stream;
  const int F3 = half_up(half_up(half_up(a->n_mels)));
  switch (a->dtype) {
    case PK_DTYPE_F16:
      return F3 <= 11 ? launch_sub_c<_Float16, 11>(a, st) : launch_sub_c<_Float16, 9>(a, st);
    case PK_DTYPE_BF16:
      return F3 <= 11 ? launch_sub_c<bf16_t, 11>(a, st) : launch_sub_c<bf16_t, 9>(a, st);
    default:
      return launch_sub_c<float, 6>(a, st);
  }
}
