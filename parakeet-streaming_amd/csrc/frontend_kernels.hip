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
constexpr int kMaxGridYZ = 65535;  // largest y or z extent of a launch grid
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
    // each 32x32 -> 64-bit product as one multiply (both halves at once)
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
}

// Standard normals for global samples 4j .. 4j + 3 of one stream, from one
// Philox draw (counter j): Box-Muller on the word pairs (r0, r1) -> cos, sin
// for 4j, 4j + 1 and (r2, r3) -> cos, sin for 4j + 2, 4j + 3, with
// u1 = (ra + 1) 2^-32 and u2 = rb 2^-32.  v_cos_f32 / v_sin_f32 take revolutions.
__device__ static inline void dither_normal4(int64_t j, uint32_t noise_id, uint32_t k0, uint32_t k1, float* z) {
  uint32_t c0 = (uint32_t)j, c1 = (uint32_t)((uint64_t)j >> 32), c2 = noise_id, c3 = 0u;
  philox4x32_10(c0, c1, c2, c3, k0, k1);
  const float ra = sqrtf(-2.0f * __logf(((float)c0 + 1.0f) * 2.3283064365386963e-10f));
  const float rb = sqrtf(-2.0f * __logf(((float)c2 + 1.0f) * 2.3283064365386963e-10f));
  const float va = (float)c1 * 2.3283064365386963e-10f, vb = (float)c3 * 2.3283064365386963e-10f;
  z[0] = ra * __builtin_amdgcn_cosf(va);
  z[1] = ra * __builtin_amdgcn_sinf(va);
  z[2] = rb * __builtin_amdgcn_cosf(vb);
  z[3] = rb * __builtin_amdgcn_sinf(vb);
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
constexpr int kBand = 32;  // filterbank weights per band staged in LDS
// FPW frames a wave: 1, or 4 at large batches (the workgroup's staging of
// twiddles, window and filterbank then serves 16 frames), which stages the
// samples of 16 frames and so takes hops up to kFeHopWide
constexpr int kFeHopWide = 192;
constexpr int kFeWideRounds = 8;  // workgroups a CU from which the 4-frames-a-wave form is used
template <int FPW>
struct FeGeom {
  static constexpr int HOP = FPW == 1 ? kMaxHop : kFeHopWide;
  static constexpr int SPAN = (kFeWaves * FPW - 1) * HOP + kMaxWin + 1;  // samples the frames of a workgroup read
};

template <int PCM, int FPW>
__global__ void __launch_bounds__(64 * kFeWaves) fe_kernel(const FeK p) {
  constexpr int kSpanMax = FeGeom<FPW>::SPAN;
  __shared__ float2 tw[kCplx];   // e^{-2 pi i m / 256}
  __shared__ float2 tw2[kBins];  // e^{-2 pi i k / 512}, k <= 256
  __shared__ float2 buf[kFeWaves][kCplx];
  __shared__ float pw[kFeWaves][kBins + 3];
  __shared__ float xs[kSpanMax + 3];  // dithered samples of the workgroup's frames
  __shared__ float win_s[kMaxWin];
  __shared__ float fbw[kMaxMels][kBand + 1];  // band m's weights from its first bin on (rows padded:
                                              // lane m reads row m, so the rows fall on distinct banks)

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
  const int j0 = blockIdx.x * kFeWaves * FPW;
  if (j0 >= s.n_frames) return;  // no frame for this workgroup
  const int nf = min(kFeWaves * FPW, s.n_frames - j0);
  const int wl = (kNfft - p.win) / 2;
  const int64_t f0 = (int64_t)s.frame0 + j0;
  const int64_t span0 = f0 * p.hop - kNfft / 2 + wl - 1;  // global index of xs[0]
  const int span = (nf - 1) * p.hop + p.win + 1;

  // staging, one global round trip per phase: every load of a phase is issued
  // into registers before any of them is stored
  __shared__ int2 rng_s[kMaxMels];
  // the span in groups of 4 consecutive global samples (one dither draw a
  // group): group q holds samples 4 (g0 + q) .. + 3, g0 = floor(span0 / 4)
  constexpr int kGroups = (kSpanMax + 3) / 4 + 1;
  constexpr int kXsPer = (kGroups + 64 * kFeWaves - 1) / (64 * kFeWaves);
  constexpr int kFbPer = kMaxMels * kBand / (64 * kFeWaves);
  constexpr int kWinPer = kMaxWin / (64 * kFeWaves);
  float xr[kXsPer][4], wr[kWinPer];
  const int mc = min(tid, p.n_mels - 1);
  const int2 rr = make_int2(p.fb_range[2 * mc], p.fb_range[2 * mc + 1]);
#pragma unroll
  for (int u = 0; u < kWinPer; ++u) wr[u] = p.window[min(tid + u * 64 * kFeWaves, p.win - 1)];
  // raw samples from this call's input or the ring (0 outside [0, total)):
  // unconditional loads from clamped addresses
  const int64_t g0 = span0 >> 2;  // floor, span0 may be negative
#pragma unroll
  for (int u = 0; u < kXsPer; ++u) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t g = 4 * (g0 + tid + u * 64 * kFeWaves) + e;
      const int64_t i = g - span0;
      const bool ok = i >= 0 && i < span && g >= 0 && g < total;
      const bool fresh = g >= s.sample_base;
      const float xn = sample_in(ok && fresh ? g - s.sample_base : 0);
      const float xo = ring[ok && !fresh ? (g & rmask) : 0];
      const float x = fresh ? xn : xo;
      xr[u][e] = ok ? x : 0.f;
    }
  }
  if (tid < p.n_mels) rng_s[tid] = make_int2(max(rr.x, 0), min(rr.y, kBins));
#pragma unroll
  for (int u = 0; u < kWinPer; ++u) {
    const int i = tid + u * 64 * kFeWaves;
    if (i < p.win) win_s[i] = wr[u];
  }
#pragma unroll
  for (int u = 0; u < kXsPer; ++u) {
    const int64_t j = g0 + tid + u * 64 * kFeWaves;
    const int64_t i0 = 4 * j - span0;  // xs index of the group's first sample
    // the span is the frames' reach, usually well under the staging's size
    if (i0 + 3 >= 0 && i0 < span) {
      float z[4] = {0.f, 0.f, 0.f, 0.f};
      if (p.dither != 0.f && 4 * j + 3 >= 0 && 4 * j < total) dither_normal4(j, s.noise_id, p.seed_lo, p.seed_hi, z);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e, g = 4 * j + e;
        if (i >= 0 && i < span) xs[i] = g >= 0 && g < total ? xr[u][e] + p.dither * z[e] : xr[u][e];
      }
    }
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
  // the wave's frames fw = wave + kFeWaves r of the workgroup's nf; no barrier
  // below this point
#pragma unroll 1
  for (int fw = wave; fw < nf; fw += kFeWaves) {
    const int64_t f = f0 + fw;
    const int64_t base = f * p.hop - kNfft / 2;
    const int off = fw * p.hop - wl + 1;  // xs index of frame sample n is off + n
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
    // real-input bins: X[k] = E[k] + W^k O[k], E/O from Z[k] and conj(Z[256-k]);
    // bins lane + 64 r in one unrolled pass, the Nyquist bin 256 by lane 0.
    // The products are fused as written (one rounding order whatever the
    // surrounding code)
    float* pwv = pw[wave];
    auto bin = [&](int kk) {
#pragma clang fp contract(off)
      const float2 zk = bw[kk & (kCplx - 1)], zm = bw[(kCplx - kk) & (kCplx - 1)];
      const float er = 0.5f * (zk.x + zm.x), ei = 0.5f * (zk.y - zm.y);
      const float orr = 0.5f * (zk.y + zm.y), oi = -0.5f * (zk.x - zm.x);
      const float2 w = tw2[kk];
      const float xr = er + fmaf(w.x, orr, -(w.y * oi)), xi = ei + fmaf(w.x, oi, w.y * orr);
      pwv[kk] = fmaf(xr, xr, xi * xi);
    };
#pragma unroll
    for (int r = 0; r < kCplx / 64; ++r) bin(lane + 64 * r);
    if (lane == 0) bin(kCplx);
    wave_lds_sync();
    float* mrow = p.mel + ((int64_t)s.slot * p.mel_rows + (f & (p.mel_rows - 1))) * p.n_mels;
    for (int m = lane; m < p.n_mels; m += 64) {
      const int lo = rng_s[m].x, hi = rng_s[m].y, mid = min(hi, lo + kBand);
      // the band's first kBand weights from LDS, the rest (wider bands) from
      // global memory: two loops, so the LDS one reads through LDS
      // instructions (one select between the two spaces made every read a
      // generic load that waited for memory); the sum runs over the bins in
      // order either way; four bins' reads are issued before their sums
      const float* const wl = &fbw[m][0];
      const float* const pl = pwv + lo;
      const int nl = mid - lo;
      float acc = 0.f;
      int j = 0;
      for (; j + 4 <= nl; j += 4) {
        float w[4], q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          w[e] = wl[j + e];
          q[e] = pl[j + e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += w[e] * q[e];
      }
      for (; j < nl; ++j) acc += wl[j] * pl[j];
      for (int kk = mid; kk < hi; ++kk) acc += p.fb[(int64_t)m * kBins + kk] * pwv[kk];
      mrow[m] = logf(acc + p.guard);
    }
    wave_lds_sync();  // this frame's reads of bw and pwv before the next frame's writes
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

// ---------------------------------------------------------------------------
// Convolution stack for the 16-bit types: NF output frames x QT output columns
// of one stream per workgroup of 16 waves, so the frames of a stream share the
// rows their receptive fields overlap in and each pointwise weight matrix is
// read once per tile.  The channels run in groups of 32:
//   conv.0 (1 -> 32 channels) on 16x16x16 MFMAs (taps 0..8 of each position
//     with the bias on tap 9; a position outside the map has all-zero
//     operands, so it comes out 0) -> ReLU -> a1g;
//   the first depthwise conv of the group on dot2 instructions -> a2g;
//   conv.3's product accumulated over the groups: one 16x16x32 k-step per
//     group on the group's 32 input channels, the fp32 sums (started at the
//     bias) held in the waves' accumulators (wave w: output channels
//     16 (w mod C/16) ..);
// then conv.3's mask, ReLU -> a2out (which zeroes every position outside the
// map, so the first depthwise conv needs no mask of its own); the second
// depthwise conv -> a3; conv.6 + bias, ReLU -> the output tile
// [frame][channel][column].  Every layer's output is rounded to the storage
// type (to nearest even), as in the stack above.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

template <typename ST>
struct Mma16;
template <>
struct Mma16<_Float16> {
  typedef _Float16 H4 __attribute__((ext_vector_type(4)));
  __device__ static inline f32x4_t k16(s16x4_t a, s16x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(H4, a), __builtin_bit_cast(H4, b), c, 0, 0, 0);
  }
};
template <>
struct Mma16<bf16_t> {
  __device__ static inline f32x4_t k16(s16x4_t a, s16x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};

typedef _Float16 h2x __attribute__((ext_vector_type(2)));
typedef __bf16 b2x __attribute__((ext_vector_type(2)));
// acc + a.lo * w.lo + a.hi * w.hi, two 16-bit pairs, fp32 accumulation
template <typename ST>
__device__ static inline float dot2(uint32_t a, uint32_t w, float acc);
template <>
__device__ inline float dot2<_Float16>(uint32_t a, uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2x, a), __builtin_bit_cast(h2x, w), acc, false);
}
template <>
__device__ inline float dot2<bf16_t>(uint32_t a, uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2x, a), __builtin_bit_cast(b2x, w), acc, false);
}
// two fp32 values as two storage elements in one dword (lo = a), rounded to
// nearest even by the packed conversion instructions
template <typename ST>
__device__ static inline uint32_t cvt2(float a, float b);
template <>
__device__ inline uint32_t cvt2<_Float16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, h2x));
}
template <>
__device__ inline uint32_t cvt2<bf16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, b2x));
}
// ReLU of two packed fp16 or bf16 values: an element with its sign bit set is
// a negative int16, so an int16 max with 0 clears it (-0 included)
__device__ static inline uint32_t relu2(uint32_t v) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(s16x2_t, v), (s16x2_t){0, 0}));
}
// x.lo | y.lo << 16, and x.hi | y.hi << 16 (v_perm_b32 byte selects)
__device__ static inline uint32_t lo2(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x05040100u); }
__device__ static inline uint32_t hi2(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x07060302u); }

constexpr int kSub2CG = 32;  // channels per group: one k-step of conv.3

// conv.0 weights in LDS as the MFMA B operand: tap k of channel c at lane
// (c mod 16, k / 4) of channel tile c / 16, 4 taps a lane, so the 16 lanes of
// one LDS pass read consecutive 8-byte runs
__device__ static inline int w0_index(int c, int k) {
  return (((c >> 4) * 4 + (k >> 2)) * 16 + (c & 15)) * 4 + (k & 3);
}

// second depthwise conv weights in LDS: tap pair pp = (2 pp, 2 pp + 1) of
// channel c as one dword (tap 9 is 0); channels c .. c + 3 of an 8-channel
// chunk sit in one 16-byte run and c + 4 .. c + 7 in another, half a row on
template <int C>
__device__ static inline int w5_index(int pp, int c) {
  return pp * C + ((c >> 2) & 1) * (C / 2) + (c >> 3) * 4 + (c & 3);
}

// Position (within a wave's 16 T1W conv.0 positions) of row r of the wave's
// conv.0 tile u: tiles 2v and 2v + 1 map row 4a + e to 32 v + 8 a + 4 (u & 1)
// + e, so D fragments of the pair in one lane are 8 consecutive positions; a
// last unpaired tile maps row r to 32 (T1W / 2) + r
__device__ static inline int sub2_pos(int u, int r, int T1W) {
  return u < (T1W & ~1) ? 32 * (u >> 1) + 8 * (r >> 2) + 4 * (u & 1) + (r & 3) : 32 * (T1W >> 1) + r;
}

// W waves a workgroup: 16 (one workgroup a CU), or 8 with the second stage
// run over channel halves (NH = 2) so that two workgroups share a CU and one's
// depthwise (VALU) work overlaps the other's pointwise (MFMA) work
template <typename ST, int NF, int QT, int C, int W>
struct Sub2Geom {
  static constexpr int NTH = 64 * W;                                // threads
  static constexpr int VEC = 8;                                     // 16-bit elements per 16 bytes
  static constexpr int XR = 8 * NF + 7, XC = 8 * QT + 7;             // input rows / cols of the tile
  static constexpr int XN = (XR * XC + 7) / 8 * 8;
  static constexpr int R2 = 2 * NF + 1, C2 = 2 * QT + 1;  // after dw 1
  static constexpr int JG = (C2 + 3) / 4;   // first depthwise conv: groups of 4 output columns
  // after dw 1 and conv.3, positions i2 C2P + q2: rows padded to whole 4-column
  // groups, so every group's 4 stores land in its own row (the padding
  // columns are never read as taps of the second depthwise conv)
  static constexpr int C2P = 4 * JG, M2 = R2 * C2P, T2 = (M2 + 15) / 16;
  // after conv.0: rows of C1 columns stored C1P apart, so a row's 4-output group
  // reads 9 columns from one 16-byte aligned chunk and the next dword
  static constexpr int R1 = 4 * NF + 3, C1 = 4 * QT + 3, C1P = 8 * JG + 8;
  static constexpr int M1 = R1 * C1P, T1 = (M1 + 15) / 16;
  static constexpr int T1W = (T1 + W - 1) / W;  // conv.0 position tiles a wave (wave + W u)
  static constexpr int T1P = T1W * W;           // tiles stored: every wave's last tile, zeros past M1
  static constexpr int M1S = ((T1P * 2) | 1) * 8;  // a1g channel stride: 8 x odd elements (distinct banks)
  static constexpr int M3 = NF * QT, T3 = (M3 + 15) / 16;                                   // after dw 2
  static constexpr int GS = kSub2CG + VEC;  // a2g position stride (padded by 16 bytes)
  static constexpr int NH = W < 16 ? 2 : 1;  // channel parts of the second depthwise conv and conv.6
  static constexpr int CH = C / NH;          // channels of a part
  static constexpr int RS = CH + VEC;        // a2out / a3 position stride
  static constexpr int NTL = C / 16;        // channel tiles of a pointwise conv
  // conv.6: a wave takes CPW channel tiles (consecutive) and position tiles pg + PG u
  static constexpr int CPW = NTL > W ? NTL / W : 1, NTW = NTL / CPW, PG = W / NTW;
  // conv.3: a wave takes channel tiles 2 (w mod NP), 2 (w mod NP) + 1 and
  // position tiles w / NP + P3 u, so each wave reads 1 / P3 of the positions' rows
  static constexpr int NP = C / 32, P3 = W / NP, T2W = (T2 + P3 - 1) / P3;
  static constexpr int T3W = (T3 + PG - 1) / PG;
  static constexpr int KS = C / 32;         // k-steps of a pointwise conv
  static constexpr int KSH = KS / NH;       // conv.6 k-steps of a channel part
  static constexpr int A1N = kSub2CG * M1S, A2N = T2 * 16 * GS;  // the a1g / a2g buffers
  static constexpr int P1 = XN + A1N + A2N;                        // xin | a1g | a2g
  static constexpr int P2 = T2 * 16 * RS + T3 * 16 * RS;       // a2out (output tile) | a3
  static constexpr int REG = cmax<P1, P2>::v;
  // LDS of the kernel: reg, w0p, w2p, w5p, bsm
  static constexpr int LDS_BYTES = REG * 2 + C * 16 * 2 + C * 32 + 5 * C * 4 + 4 * C * 4;
  static constexpr bool FITS = LDS_BYTES <= (W < 16 ? 80 : 160) * 1024;  // W < 16: two a CU
  static_assert(W == 8 || W == 16, "waves");
  static_assert(W % NP == 0 && (NTL % W == 0 || W % NTL == 0), "channel tiles over waves");
  static_assert(CH % kSub2CG == 0 && KS % NH == 0, "channel parts");
  static_assert(NF * C * QT <= T2 * 16 * RS, "output tile fits over a2out");
};

// four waves a SIMD (at most 128 registers a lane): one workgroup of 16 waves,
// or two of 8, a CU
template <typename ST, int NF, int QT, int C, int W>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4))) subsample2_kernel(const SubK<ST> p) {
  typedef Sub2Geom<ST, NF, QT, C, W> G;
  constexpr int VEC = G::VEC, NTH = G::NTH;
  static_assert(C % 64 == 0, "channels");
  __shared__ __align__(16) ST reg[G::REG];
  __shared__ __align__(16) ST w0p[C * 16];  // conv.0 (w0_index): taps 0..8, bias at 9, zeros
  // first depthwise conv: dword d of channel c at [d / 4][c][d % 4], rows kt as
  // dwords 2 kt (w0 w1) and 2 kt + 1 (w2 0)
  __shared__ __align__(16) uint32_t w2p[2][C][4];
  __shared__ __align__(16) uint32_t w5p[5 * C];  // second depthwise conv by tap pairs (w5_index)
  __shared__ __align__(16) float bsm[4][C];  // biases of conv.2/3/5/6, 0 where absent
  ST* const xin = reg;
  ST* const a1g = reg + G::XN;
  ST* const a2g = a1g + G::A1N;
  ST* const a2o = reg;  // after the group loop
  ST* const a3 = reg + G::T2 * 16 * G::RS;
  ST* const ot = reg;   // after the second depthwise conv: [frame][C][qv]

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  // the wave's first conv.6 channel tile and its position group (0 when one
  // group takes every position tile)
  const int nt = (wave % G::NTW) * G::CPW, pg = G::PG == 1 ? 0 : wave / G::NTW;
  // the wave's conv.3 channel tile pair and position group (0 when one group
  // takes every position tile, which the compiler then sees)
  const int np = wave % G::NP, pg3 = G::P3 == 1 ? 0 : wave / G::NP;
  const int F = p.F;
  const int F1 = half_up(F), F2 = half_up(F1), F3 = half_up(F2);

  // ---- the workgroup's tile: output frames blockIdx.x, columns blockIdx.y, stream blockIdx.z
  const int b = blockIdx.z;
  const pk_sub_stream s = p.streams[b];
  const int j0 = blockIdx.x * NF;  // first output frame of the tile (of the kept frames)
  const int n_keep = min(s.n_out, p.max_out);
  if (j0 >= n_keep || s.slot < 0 || s.slot >= p.in_slots || s.rows < 0 || s.length < 0 || s.length > s.rows ||
      s.drop < 0 || s.out_row < 0 || s.out_row + s.n_out > p.out_rows)
    return;
  if (!p.in_ring && (s.row0 < 0 || (int64_t)s.row0 + s.rows > p.in_rows)) return;
  const int t0 = s.drop + j0;  // its frame of the stack
  const int L3 = half_up(half_up(half_up(s.rows)));
  const int nf = min(NF, min(n_keep - j0, L3 - t0));  // frames the tile writes
  if (nf <= 0) return;
  const int p0 = blockIdx.y * QT;
  if (p0 >= F3) return;
  const int qv = min(QT, F3 - p0);
  const int len1 = half_up(s.length), len2 = half_up(len1), len3 = half_up(len2);

  // ---- weights, biases and the input tile, every global load issued before
  //      the first LDS store (one round trip): thread c < C reads channel c's
  //      9 taps of each 3x3 conv and its biases (as 16-bit words) and stores
  //      them in the layouts above with dword or wider stores; the input rows
  //      >= length and the padding as zeros
  constexpr int kXPer = (G::XN + NTH - 1) / NTH;
  uint16_t k0[9], k2[9], k5[9], b0 = 0;
  float bias[4] = {0.f, 0.f, 0.f, 0.f};  // conv.2/3/5/6 of channel tid
  if (tid < C) {
    const uint16_t* const q0 = reinterpret_cast<const uint16_t*>(p.w0) + 9 * tid;
    const uint16_t* const q2 = reinterpret_cast<const uint16_t*>(p.w2) + 9 * tid;
    const uint16_t* const q5 = reinterpret_cast<const uint16_t*>(p.w5) + 9 * tid;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      k0[k] = q0[k];
      k2[k] = q2[k];
      k5[k] = q5[k];
    }
    if (p.b0) b0 = reinterpret_cast<const uint16_t*>(p.b0)[tid];
    const ST* bp[4] = {p.b2, p.b3, p.b5, p.b6};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (bp[k]) bias[k] = from_st(bp[k][tid]);
  }
  // the input tile: rows >= length and the padding as zeros
  float xr[kXPer];
  {
    const int r0 = 8 * t0 - 14, c0 = 8 * p0 - 14;
    const float* inb = p.in + (int64_t)s.slot * p.in_rows * F;
    const int rmask = p.in_rows - 1;
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
      const int i = tid + u * NTH;
      const int rr = i / G::XC, cc = i - rr * G::XC;
      const int gr = r0 + rr, gc = c0 + cc;
      const bool ok = i < G::XR * G::XC && gr >= 0 && gr < s.length && gc >= 0 && gc < F;
      const int row = p.in_ring ? ((s.row0 + gr) & rmask) : s.row0 + gr;
      const float v = inb[ok ? (int64_t)row * F + gc : 0];
      xr[u] = ok ? v : 0.f;
    }
  }
  if (tid < C) {
    auto pk = [](uint32_t lo, uint32_t hi) { return lo | hi << 16; };
    // conv.0: taps 0..8, the bias at 9 (it rides on a tap that reads 1), zeros
    *reinterpret_cast<uint2*>(&w0p[w0_index(tid, 0)]) = make_uint2(pk(k0[0], k0[1]), pk(k0[2], k0[3]));
    *reinterpret_cast<uint2*>(&w0p[w0_index(tid, 4)]) = make_uint2(pk(k0[4], k0[5]), pk(k0[6], k0[7]));
    *reinterpret_cast<uint2*>(&w0p[w0_index(tid, 8)]) = make_uint2(pk(k0[8], b0), 0u);
    *reinterpret_cast<uint2*>(&w0p[w0_index(tid, 12)]) = make_uint2(0u, 0u);
    // first depthwise conv: rows kt as (w0 w1) and (w2 0)
    *reinterpret_cast<u32x4*>(&w2p[0][tid][0]) = u32x4{pk(k2[0], k2[1]), k2[2], pk(k2[3], k2[4]), k2[5]};
    *reinterpret_cast<u32x4*>(&w2p[1][tid][0]) = u32x4{pk(k2[6], k2[7]), k2[8], 0u, 0u};
    // second depthwise conv: tap pairs, tap 9 is 0
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) w5p[w5_index<C>(pp, tid)] = pk(k5[2 * pp], k5[2 * pp + 1]);
    w5p[w5_index<C>(4, tid)] = k5[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) bsm[k][tid] = bias[k];
  }
  // conv.3's weight rows of the wave's channel tiles: lane holds W3[n][g + 8 lg ..];
  // the first group's k-step loads now, each next one during the group before
  const ST* w3row[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) w3row[h] = p.w3 + (int64_t)((2 * np + h) * 16 + lr) * C + VEC * lg;

  u32x4 wk[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) wk[h] = ld16(w3row[h]);
#pragma unroll
  for (int u = 0; u < kXPer; ++u) {
    const int i = tid + u * NTH;
    if (i < G::XN) xin[i] = to_st<ST>(xr[u]);
  }
  __syncthreads();

  // ---- conv.0 A operands: the wave's T1W tiles cover its 16 T1W positions
  //      from 16 T1W wave on (sub2_pos); lane (lr, lg) holds taps 4 lg ..
  //      4 lg + 3 of the position of row lr (tap 9 reads 1, taps 10.. read 0),
  //      all zero for a position outside the map
  int toff[4];
  short tval[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int tap = 4 * lg + e;
    toff[e] = tap < 9 ? (tap / 3) * G::XC + tap % 3 : 0;
    tval[e] = tap < 9 ? -1 : __builtin_bit_cast(short, to_st<ST>(tap == 9 ? 1.f : 0.f));
  }
  s16x4_t xop[G::T1W];
#pragma unroll
  for (int u = 0; u < G::T1W; ++u) {
    const int m = 16 * G::T1W * wave + sub2_pos(u, lr, G::T1W);
    const int mm = min(m, G::M1 - 1);
    const int i1 = mm / G::C1P, qr = mm - i1 * G::C1P, q1 = min(qr, G::C1 - 1);
    const int r1 = 4 * t0 - 6 + i1, c1 = 4 * p0 - 6 + qr;
    const bool ok = m < G::M1 && qr < G::C1 && r1 >= 0 && r1 < len1 && c1 >= 0 && c1 < F1;
    const ST* const x = &xin[2 * i1 * G::XC + 2 * q1];  // in the tile for every lane
    // masked with an and rather than a select, so the reads are not moved
    // under a branch (one LDS round trip for all of them)
    const short okm = ok ? short(-1) : short(0);
    short v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const short t = __builtin_bit_cast(short, x[toff[e]]);
      v[e] = (4 * lg + e < 9 ? t : tval[e]) & okm;
    }
    xop[u] = s16x4_t{v[0], v[1], v[2], v[3]};
  }

  f32x4_t acc[G::T2W][2];  // conv.3 sums, started at the bias
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float4 b3 = *reinterpret_cast<const float4*>(&bsm[1][(2 * np + h) * 16 + 4 * lg]);
#pragma unroll
    for (int u = 0; u < G::T2W; ++u) acc[u][h] = f32x4_t{b3.x, b3.y, b3.z, b3.w};
  }

  // conv.0 for channels g .. g + 31 -> a1 [channel][position]: D rows are
  // positions, so a lane holds 4 positions of one channel per tile, and 8
  // consecutive ones over a pair of tiles (sub2_pos): one 16-byte store, which
  // 16 channels' rows at this stride take without bank conflicts.  Every wave
  // stores T1W tiles (the tiles past the map are zeros), so the products carry
  // no branch and the compiler interleaves them with the stores.
  auto conv0 = [&](int g, ST* a1) {
    s16x4_t wop[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) wop[ct] = *reinterpret_cast<const s16x4_t*>(&w0p[w0_index(g + ct * 16 + lr, 4 * lg)]);
    ST* const a1w = a1 + 16 * G::T1W * wave;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      ST* const row = a1w + (ct * 16 + lr) * G::M1S;
#pragma unroll
      for (int v = 0; v < G::T1W / 2; ++v) {
        const f32x4_t d0 = Mma16<ST>::k16(xop[2 * v], wop[ct], f32x4_t{0.f, 0.f, 0.f, 0.f});
        const f32x4_t d1 = Mma16<ST>::k16(xop[2 * v + 1], wop[ct], f32x4_t{0.f, 0.f, 0.f, 0.f});
        *reinterpret_cast<u32x4*>(&row[32 * v + 8 * lg]) =
            u32x4{relu2(cvt2<ST>(d0[0], d0[1])), relu2(cvt2<ST>(d0[2], d0[3])), relu2(cvt2<ST>(d1[0], d1[1])),
                  relu2(cvt2<ST>(d1[2], d1[3]))};
      }
      if constexpr (G::T1W % 2) {
        const f32x4_t d = Mma16<ST>::k16(xop[G::T1W - 1], wop[ct], f32x4_t{0.f, 0.f, 0.f, 0.f});
        *reinterpret_cast<uint2*>(&row[32 * (G::T1W / 2) + 4 * lg]) =
            make_uint2(relu2(cvt2<ST>(d[0], d[1])), relu2(cvt2<ST>(d[2], d[3])));
      }
    }
  };
  // first depthwise conv of channels g .. g + 31 -> a2 [position][32]: a
  // thread takes one channel (tid mod 32, the same in every group) and 4
  // adjacent output columns of one output row, at most D1N such items, whose
  // a1 / a2 offsets are worked out once (d1off: a1 offset | a2 offset << 16,
  // all ones past the items); per input row, 9 columns come from a 16-byte
  // chunk and the next one's first dword (that chunk read whole: a 16-byte
  // LDS read of 16 channels' rows is conflict free, a 4-byte one at this
  // stride is not), and each tap pair is one fp32-accumulating dot2
  // (w0 w1 | w2 0)
  constexpr int kD1Items = kSub2CG * G::R2 * G::JG, D1N = (kD1Items + NTH - 1) / NTH;
  static_assert(NTH % kSub2CG == 0, "a thread keeps its channel");
  static_assert(kSub2CG * G::M1S <= 65536 && G::T2 * 16 * G::GS <= 65536, "16-bit offsets");
  const int dc = tid % kSub2CG;
  uint32_t d1off[D1N];
#pragma unroll
  for (int u = 0; u < D1N; ++u) {
    const int rest = tid / kSub2CG + u * (NTH / kSub2CG);
    const int i2 = rest % G::R2, jg = rest / G::R2;
    d1off[u] = rest < G::R2 * G::JG
                   ? (uint32_t)(dc * G::M1S + 2 * i2 * G::C1P + 8 * jg) |
                         ((uint32_t)((i2 * G::C2P + 4 * jg) * G::GS + dc) << 16)
                   : ~0u;
  }
  auto dwconv1 = [&](int g, const ST* a1, ST* a2) {
    const u32x4 wa = *reinterpret_cast<const u32x4*>(&w2p[0][g + dc][0]);
    const u32x4 wb = *reinterpret_cast<const u32x4*>(&w2p[1][g + dc][0]);
    const uint32_t wr[6] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y};
    const float bv = bsm[0][g + dc];
#pragma unroll
    for (int u = 0; u < D1N; ++u) {
      if (d1off[u] == ~0u) continue;
      float o[4] = {bv, bv, bv, bv};
#pragma unroll
      for (int kt = 0; kt < 3; ++kt) {
        const ST* row = &a1[(d1off[u] & 0xffffu) + kt * G::C1P];
        const u32x4 q = *reinterpret_cast<const u32x4*>(row);
        const u32x4 q2 = *reinterpret_cast<const u32x4*>(row + 8);
        asm volatile("" ::"v"(q2.y), "v"(q2.z), "v"(q2.w));  // keep the read 16 bytes wide
        const uint32_t d4 = q2.x;
        const uint32_t d[5] = {q.x, q.y, q.z, q.w, d4};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) o[jj] = dot2<ST>(d[jj + 1], wr[2 * kt + 1], dot2<ST>(d[jj], wr[2 * kt], o[jj]));
      }
      const uint32_t p01 = cvt2<ST>(o[0], o[1]), p23 = cvt2<ST>(o[2], o[3]);
      const uint16_t h[4] = {(uint16_t)p01, (uint16_t)(p01 >> 16), (uint16_t)p23, (uint16_t)(p23 >> 16)};
      uint16_t* const dst = reinterpret_cast<uint16_t*>(&a2[d1off[u] >> 16]);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dst[jj * G::GS] = h[jj];
    }
  };
  // conv.3: one k-step over a group's 32 input channels (weights in wk) for
  // the wave's two channel tiles and its position tiles
  auto pw3 = [&](const ST* a2) {
#pragma unroll
    for (int u = 0; u < G::T2W; ++u) {
      const int mt = pg3 + G::P3 * u;
      if (mt < G::T2) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(&a2[(mt * 16 + lr) * G::GS + VEC * lg]);
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[u][h] = MmaK<ST>::step(wk[h], x, acc[u][h]);
      }
    }
  };
  // Two barriers a group: conv.0 (a1g) | the depthwise conv (a1g -> a2g) |
  // conv.3 (a2g) with the next group's conv.0 (a1g, whose last reader is
  // behind the second barrier); the next depthwise conv rewrites a2g only
  // after the next first barrier, which every wave reaches after its conv.3.
  conv0(0, a1g);
#pragma unroll 1
  for (int g = 0; g < C; g += kSub2CG) {
    __syncthreads();
    dwconv1(g, a1g, a2g);
    __syncthreads();
    pw3(a2g);
    if (g + kSub2CG < C) {  // the next group's k-step loads during its conv.0 and depthwise conv
#pragma unroll
      for (int h = 0; h < 2; ++h) wk[h] = ld16(w3row[h] + g + kSub2CG);
      conv0(g + kSub2CG, a1g);
    }
  }
  __syncthreads();  // the second stage rewrites the group buffers

  // ---- second stage, NH channel parts of CH channels one after the other:
  //      conv.3's mask and ReLU -> a2out [position][CH] (over the group
  //      buffers), the second depthwise conv -> a3 [frame * QT + column][CH],
  //      and conv.6's k-steps over the part's channels, summed in d

  // conv.3's outputs as 16-bit pairs (half the registers of the sums), zero
  // outside the map
  uint2 c3v[G::T2W][2];
#pragma unroll
  for (int u = 0; u < G::T2W; ++u) {
    const int m = (pg3 + G::P3 * u) * 16 + lr;
    const int i2 = m / G::C2P, q2 = m - i2 * G::C2P;
    const int r2 = 2 * t0 - 2 + i2, c2 = 2 * p0 - 2 + q2;
    const bool ok = m < G::M2 && r2 >= 0 && r2 < len2 && c2 >= 0 && c2 < F2;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4_t& a = acc[u][h];
      c3v[u][h] = ok ? make_uint2(relu2(cvt2<ST>(a[0], a[1])), relu2(cvt2<ST>(a[2], a[3]))) : make_uint2(0u, 0u);
    }
  }
  f32x4_t d[G::T3W][G::CPW];
#pragma unroll
  for (int i = 0; i < G::CPW; ++i) {
    const f32x4_t b6 = *reinterpret_cast<const f32x4_t*>(&bsm[3][(nt + i) * 16 + 4 * lg]);
#pragma unroll
    for (int u = 0; u < G::T3W; ++u) d[u][i] = b6;
  }
#pragma unroll
  for (int hh = 0; hh < G::NH; ++hh) {
    if (np / (G::NP / G::NH) == hh) {  // the wave's conv.3 channels lie in this part
#pragma unroll
      for (int u = 0; u < G::T2W; ++u) {
        const int mt = pg3 + G::P3 * u;
        if (mt < G::T2) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            *reinterpret_cast<uint2*>(&a2o[(mt * 16 + lr) * G::RS + (2 * np + h) * 16 - hh * G::CH + 4 * lg]) =
                c3v[u][h];
        }
      }
    }
    // conv.6's weights for the wave's channel tiles and this part's k-steps
    // load while the second depthwise conv runs
    u32x4 w6q[G::CPW][G::KSH];
    auto load_w6 = [&]() {
#pragma unroll
      for (int i = 0; i < G::CPW; ++i)
#pragma unroll
        for (int kk = 0; kk < G::KSH; ++kk)
          w6q[i][kk] = ld16(p.w6 + (int64_t)((nt + i) * 16 + lr) * C + VEC * lg + (hh * G::KSH + kk) * 32);
    };
    load_w6();
    __syncthreads();

    // second depthwise conv, masked: a thread takes 8 channels of one
    // position; per tap pair, the two taps' values of a channel are gathered
    // into one dword (v_perm) for a dot2
    for (int it = tid; it < G::T3 * 16 * (G::CH / VEC); it += NTH) {
      const int m3 = it / (G::CH / VEC), cc = (it - m3 * (G::CH / VEC)) * VEC;
      const int cw = hh * G::CH + cc;  // channel of the weights and bias
      const int f = min(m3 / QT, NF - 1), q = m3 - (m3 / QT) * QT;
      float sum[VEC];
      {
        const float4 x = *reinterpret_cast<const float4*>(&bsm[2][cw]);
        const float4 y = *reinterpret_cast<const float4*>(&bsm[2][cw + 4]);
        sum[0] = x.x, sum[1] = x.y, sum[2] = x.z, sum[3] = x.w;
        sum[4] = y.x, sum[5] = y.y, sum[6] = y.z, sum[7] = y.w;
      }
      const ST* const src = &a2o[(2 * f * G::C2P + 2 * q) * G::RS + cc];
#pragma unroll
      for (int pp = 0; pp < 5; ++pp) {
        const int ta = 2 * pp, tb = 2 * pp + 1;
        const u32x4 A = ld16(src + ((ta / 3) * G::C2P + ta % 3) * G::RS);
        const u32x4 B = tb < 9 ? ld16(src + ((tb / 3) * G::C2P + tb % 3) * G::RS) : u32x4{0u, 0u, 0u, 0u};
        const u32x4 W0 = *reinterpret_cast<const u32x4*>(&w5p[w5_index<C>(pp, cw)]);
        const u32x4 W1 = *reinterpret_cast<const u32x4*>(&w5p[w5_index<C>(pp, cw + 4)]);
        const uint32_t a[4] = {A.x, A.y, A.z, A.w}, bb[4] = {B.x, B.y, B.z, B.w};
        const uint32_t w[8] = {W0.x, W0.y, W0.z, W0.w, W1.x, W1.y, W1.z, W1.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum[2 * e] = dot2<ST>(lo2(a[e], bb[e]), w[2 * e], sum[2 * e]);
          sum[2 * e + 1] = dot2<ST>(hi2(a[e], bb[e]), w[2 * e + 1], sum[2 * e + 1]);
        }
      }
      const bool ok = m3 < G::M3 && t0 + f < len3;
      const u32x4 o = {cvt2<ST>(sum[0], sum[1]), cvt2<ST>(sum[2], sum[3]), cvt2<ST>(sum[4], sum[5]),
                       cvt2<ST>(sum[6], sum[7])};
      *reinterpret_cast<u32x4*>(&a3[m3 * G::RS + cc]) = ok ? o : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    // conv.6 k-steps over the part's channels
#pragma unroll
    for (int u = 0; u < G::T3W; ++u) {
      const int mt = pg + G::PG * u;
      if (mt < G::T3) {
#pragma unroll
        for (int kk = 0; kk < G::KSH; ++kk) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(&a3[(mt * 16 + lr) * G::RS + kk * 32 + VEC * lg]);
#pragma unroll
          for (int i = 0; i < G::CPW; ++i) d[u][i] = MmaK<ST>::step(w6q[i][kk], x, d[u][i]);
        }
      }
    }
  }

  // ---- conv.6 ReLU and mask -> output tile [frame][channel][qv columns],
  //      over a2out (no wave reads it after the last barrier)
#pragma unroll
  for (int u = 0; u < G::T3W; ++u) {
    const int mt = pg + G::PG * u;
    if (mt < G::T3) {
      const int m3 = mt * 16 + lr;
      const int f = m3 / QT, q = m3 - f * QT;
      if (m3 < G::M3 && q < qv) {
        const bool ok = t0 + f < len3;
#pragma unroll
        for (int i = 0; i < G::CPW; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            ot[(f * C + (nt + i) * 16 + 4 * lg + e) * qv + q] = to_st<ST>(ok ? fmaxf(d[u][i][e], 0.f) : 0.f);
      }
    }
  }
  __syncthreads();
  ST* const out = p.out + (int64_t)(s.out_row + j0) * C * F3;
  if (qv == F3 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0) {
    // the tile spans every column: its nf frames of [C][F3] are one run
    for (int i = tid * VEC; i < nf * C * F3; i += NTH * VEC) st16(out + i, ld16(ot + i));
  } else {
    for (int f = 0; f < nf; ++f)
      for (int i = tid; i < C * qv; i += NTH) {
        const int c = i / qv, q = i - c * qv;
        out[(int64_t)f * C * F3 + c * F3 + p0 + q] = ot[f * C * qv + i];
      }
  }
}

// ===========================================================================
// host side

static bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

template <typename ST>
static SubK<ST> sub_args(const pk_sub_args* a, int C) {
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
  return k;
}

// fp32: one output frame x QT columns per workgroup
template <typename ST, int QT, int C>
static int launch_sub(const pk_sub_args* a, hipStream_t st) {
  const SubK<ST> k = sub_args<ST>(a, C);
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


// fp16 / bf16: one tile of NF output frames x QT columns a workgroup of W
// waves (one workgroup a CU for W 16, two for W 8)
template <typename ST, int NF, int QT, int C, int W>
static int launch_sub2(const pk_sub_args* a, hipStream_t st) {
  const SubK<ST> k = sub_args<ST>(a, C);
  const int F3 = half_up(half_up(half_up(a->n_mels)));
  const dim3 grid((a->max_out + NF - 1) / NF, (F3 + QT - 1) / QT, a->batch);
  hipLaunchKernelGGL((subsample2_kernel<ST, NF, QT, C, W>), grid, dim3(64 * W), 0, st, k);
  return check_launch("pk_subsample");
}

// two-frame tiles a CU (of 8 waves each) from which the paired form is used
constexpr int kSub2PairTiles = 2;

// Two frames a tile share the conv.0 / first depthwise rows their receptive
// fields overlap in (about 0.6 of the one-frame tile's work per frame), but
// when one-frame tiles fit on the CUs in one round they finish sooner, and
// wide tiles (QT 17) of two frames do not fit in LDS with C of 128 or more.
// With several two-frame tiles a CU to run, workgroups of 8 waves that fit
// two a CU overlap one tile's depthwise convs with the other's pointwise ones.
template <typename ST, int QT, int C>
static int launch_sub2_nf(const pk_sub_args* a, hipStream_t st) {
  const int F3 = half_up(half_up(half_up(a->n_mels)));
  const int64_t yt = (F3 + QT - 1) / QT;
  const int64_t tiles1 = (int64_t)a->max_out * yt * a->batch;
  const int64_t tiles2 = (int64_t)((a->max_out + 1) / 2) * yt * a->batch;
  if constexpr (Sub2Geom<ST, 2, QT, C, 16>::FITS) {
    if (tiles1 > cu_count()) {
      if constexpr (C == 256 && Sub2Geom<ST, 2, QT, C, 8>::FITS) {  // the models' channel count
        if (tiles2 >= (int64_t)kSub2PairTiles * cu_count()) return launch_sub2<ST, 2, QT, C, 8>(a, st);
      }
      return launch_sub2<ST, 2, QT, C, 16>(a, st);
    }
  }
  return launch_sub2<ST, 1, QT, C, 16>(a, st);
}

template <typename ST, int QT>
static int launch_sub2_c(const pk_sub_args* a, hipStream_t st) {
  switch (a->channels) {
    case 64:
      return launch_sub2_nf<ST, QT, 64>(a, st);
    case 128:
      return launch_sub2_nf<ST, QT, 128>(a, st);
    default:
      return launch_sub2_nf<ST, QT, 256>(a, st);
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
  // four frames a wave when the batch fills the CUs several times over with
  // such workgroups (and the hop fits their sample staging), one otherwise
  const int wide_frames = 4 * kFeWaves;
  const int64_t gx4 = a->max_frames > 0 ? (a->max_frames + wide_frames - 1) / wide_frames : 1;
  const bool wide = a->hop <= kFeHopWide && gx4 * a->batch >= (int64_t)kFeWideRounds * cu_count();
  const int gx = a->max_frames > 0 ? (a->max_frames + (wide ? wide_frames : kFeWaves) - 1) / (wide ? wide_frames : kFeWaves) : 1;
  // the streams in launches of at most kMaxGridYZ (the grid's y extent)
  const size_t pcm_bytes = a->pcm_dtype == PK_PCM_S16 ? 2 : 4;
  for (int b0 = 0; b0 < a->batch; b0 += kMaxGridYZ) {
    const int nb = a->batch - b0 < kMaxGridYZ ? a->batch - b0 : kMaxGridYZ;
    k.streams = a->streams + b0;
    k.samples = a->samples ? (const char*)a->samples + (size_t)b0 * (size_t)a->samples_stride * pcm_bytes : nullptr;
    const dim3 grid(gx, nb), block(64 * kFeWaves);
    const hipStream_t st = (hipStream_t)stream;
    if (a->pcm_dtype == PK_PCM_S16) {
      if (wide)
        hipLaunchKernelGGL((fe_kernel<PK_PCM_S16, 4>), grid, block, 0, st, k);
      else
        hipLaunchKernelGGL((fe_kernel<PK_PCM_S16, 1>), grid, block, 0, st, k);
    } else {
      if (wide)
        hipLaunchKernelGGL((fe_kernel<PK_PCM_F32, 4>), grid, block, 0, st, k);
      else
        hipLaunchKernelGGL((fe_kernel<PK_PCM_F32, 1>), grid, block, 0, st, k);
    }
    const int rc = check_launch("pk_fe_step");
    if (rc != PK_OK) return rc;
  }
  return PK_OK;
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
  DeviceGuard dg(a->device);
  if (!dg.ok) return fail(PK_ERR_HIP, "pk_subsample: cannot select device %d", a->device);
  const hipStream_t st = (hipStream_t)stream;
  const int F3 = half_up(half_up(half_up(a->n_mels)));
  // the stream records in launches of at most kMaxGridYZ (the grid's z extent);
  // every output row is addressed through its record
  pk_sub_args part = *a;
  for (int b0 = 0; b0 < a->batch; b0 += kMaxGridYZ) {
    part.streams = a->streams + b0;
    part.batch = a->batch - b0 < kMaxGridYZ ? a->batch - b0 : kMaxGridYZ;
    int rc;
    switch (a->dtype) {
      case PK_DTYPE_F16:
        rc = F3 <= 11 ? launch_sub2_c<_Float16, 11>(&part, st) : launch_sub2_c<_Float16, 17>(&part, st);
        break;
      case PK_DTYPE_BF16:
        rc = F3 <= 11 ? launch_sub2_c<bf16_t, 11>(&part, st) : launch_sub2_c<bf16_t, 17>(&part, st);
        break;
      default:
        rc = launch_sub_c<float, 6>(&part, st);
    }
    if (rc != PK_OK) return rc;
  }
  return PK_OK;
}
