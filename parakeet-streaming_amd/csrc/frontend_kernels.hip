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

__global__ void __launch_bounds__(64 * kFeWaves) fe_kernel(const FeK p) {
  __shared__ float2 tw[kCplx];        // e^{-2 pi i m / 256}
  __shared__ float2 tw2[kBins];       // e^{-2 pi i k / 512}, k <= 256
  __shared__ float2 buf[kFeWaves][kCplx];
  __shared__ float pw[kFeWaves][kBins + 3];

  const int b = blockIdx.y;
  const pk_fe_stream s = p.streams[b];
  if (s.slot < 0 || s.slot >= p.num_slots || s.n_new < 0 || s.n_new > p.max_new || s.n_frames < 0 ||
      s.n_frames > p.max_frames || s.frame0 < 0 || s.sample_base < 0)
    return;  // uniform over the workgroup
  const int64_t total = s.sample_base + s.n_new;
  const int rmask = p.ring_size - 1;
  float* ring = p.ring + (int64_t)s.slot * p.ring_size;

  // new samples -> ring (this call reads only ring entries of older samples)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < s.n_new;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float x = p.pcm == PK_PCM_S16
                        ? (float)((const int16_t*)p.samples)[b * p.s_stride + i] * (1.0f / 32768.0f)
                        : ((const float*)p.samples)[b * p.s_stride + i];
    ring[(s.sample_base + i) & rmask] = x;
  }
  if ((int)blockIdx.x * kFeWaves >= s.n_frames) return;  // no frame for this workgroup

  for (int m = threadIdx.x; m < kBins; m += blockDim.x) {
    float sn, cs;
    if (m < kCplx) {
      sincospif((float)m / 128.0f, &sn, &cs);
      tw[m] = make_float2(cs, -sn);
    }
    sincospif((float)m / 256.0f, &sn, &cs);
    tw2[m] = make_float2(cs, -sn);
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int j = blockIdx.x * kFeWaves + wave;
  if (j >= s.n_frames) return;  // no barrier below this point
  const int f = s.frame0 + j;
  const int64_t base = (int64_t)f * p.hop - kNfft / 2;
  const int wl = (kNfft - p.win) / 2;
  const uint32_t k0 = p.seed_lo, k1 = p.seed_hi;

  // raw sample i (0 <= i < total) from this call's input or the ring, dithered
  auto xd = [&](int64_t i) -> float {
    float x;
    if (i >= s.sample_base) {
      const int64_t o = i - s.sample_base;
      x = p.pcm == PK_PCM_S16 ? (float)((const int16_t*)p.samples)[b * p.s_stride + o] * (1.0f / 32768.0f)
                              : ((const float*)p.samples)[b * p.s_stride + o];
    } else {
      x = ring[i & rmask];
    }
    if (p.dither != 0.f) x += p.dither * dither_normal(i, s.noise_id, k0, k1);
    return x;
  };
  // windowed, pre-emphasised frame sample n (0 <= n < 512)
  auto frame_val = [&](int n) -> float {
    if (n < wl || n >= wl + p.win) return 0.f;
    const int64_t i = base + n;
    if (i < 0 || i >= total) return 0.f;
    const float cur = xd(i);
    const float prev = i >= 1 ? xd(i - 1) : 0.f;
    return (cur - p.preemph * prev) * p.window[n - wl];
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
    const int lo = p.fb_range[2 * m], hi = p.fb_range[2 * m + 1];
    const float* w = p.fb + (int64_t)m * kBins;
    float acc = 0.f;
    for (int kk = max(lo, 0); kk < min(hi, kBins); ++kk) acc += w[kk] * pwv[kk];
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
constexpr int kMaxC = 256;
constexpr int kCG = 64;  // channels per conv.0 / first depthwise group

// output length of a 3x3 stride-2 conv padded (2, 1): (n + 2 + 1 - 3) / 2 + 1
__host__ __device__ static inline int half_up(int n) { return n / 2 + 1; }

template <typename ST, int QT>
struct SubGeom {
  static constexpr int VEC = 16 / sizeof(ST);
  static constexpr int XR = 15, XC = 8 * QT + 7;  // input rows / cols of the tile
  static constexpr int A1R = 7, A1C = 4 * QT + 3;  // after conv.0
  static constexpr int A2R = 3, A2C = 2 * QT + 1;  // after the first depthwise conv
  static constexpr int M1 = A1R * A1C, T1 = (M1 + 15) / 16;
  static constexpr int M2 = A2R * A2C, T2 = (M2 + 15) / 16;
  static constexpr int RS = kMaxC + VEC;  // padded LDS row (elements) of MFMA A operands
  static constexpr int REG_A = (A1R * A1C * kCG > M2 * kMaxC ? A1R * A1C * kCG : M2 * kMaxC) > kMaxC * QT
                                   ? (A1R * A1C * kCG > M2 * kMaxC ? A1R * A1C * kCG : M2 * kMaxC)
                                   : kMaxC * QT;
  static constexpr int REG_B = (T2 > 1 ? T2 : 1) * 16 * RS;
  static constexpr int T1W = (T1 + kSubWaves - 1) / kSubWaves;  // conv.0 M tiles per wave
};

template <typename ST, int QT>
__global__ void __launch_bounds__(kSubThreads) subsample_kernel(const SubK<ST> p) {
  typedef SubGeom<ST, QT> G;
  constexpr int VEC = G::VEC;
  __shared__ __align__(16) ST xin[G::XR * G::XC];
  __shared__ __align__(16) ST regA[G::REG_A];  // a1 (one group) -> a2 -> flattened output tile
  __shared__ __align__(16) ST regB[G::REG_B];  // a2 before pw (all channels) -> a3 before pw

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
  const int F = p.F, C = p.C;
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

  // ---- input tile: rows 8t-14 .., cols 8p0-14 .., masked by length, rounded
  {
    const int r0 = 8 * t - 14, c0 = 8 * p0 - 14;
    const float* inb = p.in + (int64_t)s.slot * p.in_rows * F;
    const int rmask = p.in_rows - 1;
    for (int i = tid; i < G::XR * G::XC; i += kSubThreads) {
      const int rr = i / G::XC, cc = i - rr * G::XC;
      const int gr = r0 + rr, gc = c0 + cc;
      float v = 0.f;
      if (gr >= 0 && gr < s.length && gc >= 0 && gc < F) {
        const int row = p.in_ring ? ((s.row0 + gr) & rmask) : s.row0 + gr;
        v = inb[(int64_t)row * F + gc];
      }
      xin[i] = to_st<ST>(v);
    }
  }
  __syncthreads();

  // ---- conv.0 operands: A = the 9 taps of each position (one K chunk), per wave
  // its M tiles m = wave + 8 u
  u32x4 a0[G::T1W];
#pragma unroll
  for (int u = 0; u < G::T1W; ++u) {
    const int m = (wave + kSubWaves * u) * 16 + lr;
    Chunk<ST> ch;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int tap = VEC * lg + e;
      float v = 0.f;
      if (tap < 9 && m < G::M1) {
        const int i = m / G::A1C, q = m - i * G::A1C;
        v = from_st(xin[(2 * i + tap / 3) * G::XC + 2 * q + tap % 3]);
      }
      ch.v[e] = to_st<ST>(v);
    }
    a0[u] = __builtin_bit_cast(u32x4, ch);
  }

  ST* a1 = regA;
  ST* a2p = regB;
  for (int cg = 0; cg < C; cg += kCG) {
    // conv.0 for channels cg .. cg+63 -> bias, mask, ReLU -> a1 [7][A1C][64]
    u32x4 bw[kCG / 16];
#pragma unroll
    for (int nt = 0; nt < kCG / 16; ++nt) {
      const int c = cg + nt * 16 + lr;
      Chunk<ST> ch;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int tap = VEC * lg + e;
        ch.v[e] = tap < 9 ? p.w0[c * 9 + tap] : to_st<ST>(0.f);
      }
      bw[nt] = __builtin_bit_cast(u32x4, ch);
    }
#pragma unroll
    for (int u = 0; u < G::T1W; ++u) {
      const int mt = wave + kSubWaves * u;
      if (mt >= G::T1) break;
#pragma unroll
      for (int nt = 0; nt < kCG / 16; ++nt) {
        const int c = cg + nt * 16 + lr;
        const float bias = p.b0 ? from_st(p.b0[c]) : 0.f;
        f32x4_t d = MmaK<ST>::step(a0[u], bw[nt], f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int m = mt * 16 + 4 * lg + ii;
          if (m >= G::M1) continue;
          const int i = m / G::A1C, q = m - i * G::A1C;
          const int gr = 4 * t - 6 + i, gq = 4 * p0 - 6 + q;
          const bool ok = gr >= 0 && gr < len1 && gq >= 0 && gq < F1;
          a1[m * kCG + nt * 16 + lr] = to_st<ST>(ok ? fmaxf(round_to<ST>(d[ii] + bias), 0.f) : 0.f);
        }
      }
    }
    __syncthreads();
    // first depthwise conv for the group -> a2p [M2][RS] (before the pointwise conv)
    {
      const int c = cg + lane;
      float w[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) w[k] = from_st(p.w2[c * 9 + k]);
      const float bias = p.b2 ? from_st(p.b2[c]) : 0.f;
      for (int m = wave; m < G::M2; m += kSubWaves) {
        const int si = m / G::A2C, pp = m - si * G::A2C;
        float acc = bias;
#pragma unroll
        for (int kt = 0; kt < 3; ++kt)
#pragma unroll
          for (int kf = 0; kf < 3; ++kf)
            acc += w[kt * 3 + kf] * from_st(a1[((2 * si + kt) * G::A1C + 2 * pp + kf) * kCG + lane]);
        a2p[m * G::RS + c] = to_st<ST>(acc);
      }
    }
    __syncthreads();
  }

  // ---- pointwise conv.3 (C x C): wave owns N tiles 2w, 2w+1 -> bias, mask, ReLU -> a2
  ST* a2 = regA;
  const int ntiles = C / 16;
  const int ksteps = C / (4 * VEC);
  {
    f32x4_t acc[G::T2][2];
#pragma unroll
    for (int mt = 0; mt < G::T2; ++mt) acc[mt][0] = acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int n0 = 2 * wave;
    if (n0 < ntiles) {
      for (int kk = 0; kk < ksteps; ++kk) {
        const int k = kk * 4 * VEC + VEC * lg;
        const u32x4 b0 = ld16(p.w3 + (int64_t)(n0 * 16 + lr) * C + k);
        const u32x4 b1 = ld16(p.w3 + (int64_t)((n0 + 1) * 16 + lr) * C + k);
#pragma unroll
        for (int mt = 0; mt < G::T2; ++mt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(a2p + (mt * 16 + lr) * G::RS + k);
          acc[mt][0] = MmaK<ST>::step(a, b0, acc[mt][0]);
          acc[mt][1] = MmaK<ST>::step(a, b1, acc[mt][1]);
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = (n0 + h) * 16 + lr;
        const float bias = p.b3 ? from_st(p.b3[c]) : 0.f;
#pragma unroll
        for (int mt = 0; mt < G::T2; ++mt)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int m = mt * 16 + 4 * lg + ii;
            if (m >= G::M2) continue;
            const int si = m / G::A2C, pp = m - si * G::A2C;
            const int gs = 2 * t - 2 + si, gp = 2 * p0 - 2 + pp;
            const bool ok = gs >= 0 && gs < len2 && gp >= 0 && gp < F2;
            a2[m * kMaxC + c] = to_st<ST>(ok ? fmaxf(round_to<ST>(acc[mt][h][ii] + bias), 0.f) : 0.f);
          }
      }
    }
  }
  __syncthreads();

  // ---- second depthwise conv -> a3p [QT][RS]
  ST* a3p = regB;
  for (int c = lane; c < C; c += 64) {
    float w[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) w[k] = from_st(p.w5[c * 9 + k]);
    const float bias = p.b5 ? from_st(p.b5[c]) : 0.f;
    for (int q = wave; q < QT; q += kSubWaves) {
      float acc = bias;
#pragma unroll
      for (int kt = 0; kt < 3; ++kt)
#pragma unroll
        for (int kf = 0; kf < 3; ++kf)
          acc += w[kt * 3 + kf] * from_st(a2[(kt * G::A2C + 2 * q + kf) * kMaxC + c]);
      a3p[q * G::RS + c] = to_st<ST>(acc);
    }
  }
  __syncthreads();

  // ---- pointwise conv.6 + ReLU -> flattened tile [C][QT] in regA
  ST* ot = regA;
  {
    const int n0 = 2 * wave;
    if (n0 < ntiles) {
      f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
      for (int kk = 0; kk < ksteps; ++kk) {
        const int k = kk * 4 * VEC + VEC * lg;
        const u32x4 b0 = ld16(p.w6 + (int64_t)(n0 * 16 + lr) * C + k);
        const u32x4 b1 = ld16(p.w6 + (int64_t)((n0 + 1) * 16 + lr) * C + k);
        const u32x4 a = *reinterpret_cast<const u32x4*>(a3p + lr * G::RS + k);
        acc0 = MmaK<ST>::step(a, b0, acc0);
        acc1 = MmaK<ST>::step(a, b1, acc1);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = (n0 + h) * 16 + lr;
        const float bias = p.b6 ? from_st(p.b6[c]) : 0.f;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int q = 4 * lg + ii;
          if (q >= QT) continue;
          const float v = (h ? acc1 : acc0)[ii];
          ot[c * QT + q] = to_st<ST>(fmaxf(round_to<ST>(v + bias), 0.f));
        }
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

template <typename ST, int QT>
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
  k.C = a->channels;
  k.out_rows = a->out_rows;
  k.max_out = a->max_out;
  const int F3 = half_up(half_up(half_up(a->n_mels)));
  const dim3 grid(a->max_out, (F3 + QT - 1) / QT, a->batch);
  hipLaunchKernelGGL((subsample_kernel<ST, QT>), grid, dim3(kSubThreads), 0, st, k);
  return check_launch("pk_subsample");
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
  if (a->hop < 1) return fail(PK_ERR_INVALID, "pk_fe_step: hop %d", a->hop);
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
  hipLaunchKernelGGL(fe_kernel, dim3(gx, a->batch), dim3(64 * kFeWaves), 0, (hipStream_t)stream, k);
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
      return F3 <= 11 ? launch_sub<_Float16, 11>(a, st) : launch_sub<_Float16, 9>(a, st);
    case PK_DTYPE_BF16:
      return F3 <= 11 ? launch_sub<bf16_t, 11>(a, st) : launch_sub<bf16_t, 9>(a, st);
    default:
      return launch_sub<float, 6>(a, st);
  }
}
