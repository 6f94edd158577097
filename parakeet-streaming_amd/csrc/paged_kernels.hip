// gfx950 kernels of the paged K/V-cache hot path.
//
//   relpos_attn_kernel  fused page append + relative-position MHA over each
//                       stream's window read from its pages
//                       (parakeet/modules/attention.py:97-121)
//   kv_append_kernel    new K/V frames -> pages (cache.py:43-44)
//   kv_gather_kernel    pages -> dense window (cache.py:45), bit-exact
//   stream_mask_kernel  streaming attention / padding masks (encoder.py:167-227)
//
// All loads and stores of K/V/Q/pos/out are 16 bytes per lane: a lane owns VEC
// consecutive elements (8 for fp16/bf16, 4 for fp32) of one head's slice of one
// frame, G = head_dim / VEC lanes cover one head-row, so every row segment a
// wave touches is a whole number of 128-byte lines.

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstdint>

#include "pk_common.h"

namespace pk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// element traits: 16-byte chunk <-> fp32 registers

template <typename ST>
struct Tr;

template <>
struct Tr<float> {
  static constexpr int VEC = 4;
  __device__ static inline void unpack(const u32x4 v, float* f) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
    v.x = __float_as_uint(f[0]);
    v.y = __float_as_uint(f[1]);
    v.z = __float_as_uint(f[2]);
    v.w = __float_as_uint(f[3]);
    return v;
  }
};

template <>
struct Tr<_Float16> {
  static constexpr int VEC = 8;
  __device__ static inline void two(uint32_t w, float* f) {
    const h2 x = __builtin_bit_cast(h2, w);
    f[0] = (float)x.x;
    f[1] = (float)x.y;
  }
  __device__ static inline uint32_t two(const float* f) {
    h2 x;
    x.x = (_Float16)f[0];
    x.y = (_Float16)f[1];
    return __builtin_bit_cast(uint32_t, x);
  }
  __device__ static inline void unpack(const u32x4 v, float* f) {
    two(v.x, f);
    two(v.y, f + 2);
    two(v.z, f + 4);
    two(v.w, f + 6);
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
    v.x = two(f);
    v.y = two(f + 2);
    v.z = two(f + 4);
    v.w = two(f + 6);
    return v;
  }
};

// bfloat16 is carried as raw 16-bit patterns; fp32 -> bf16 rounds to nearest even.
struct bf16_t {
  uint16_t bits;
};

__device__ static inline uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

template <>
struct Tr<bf16_t> {
  static constexpr int VEC = 8;
  __device__ static inline void unpack(const u32x4 v, float* f) {
    f[0] = __uint_as_float(v.x << 16);
    f[1] = __uint_as_float(v.x & 0xffff0000u);
    f[2] = __uint_as_float(v.y << 16);
    f[3] = __uint_as_float(v.y & 0xffff0000u);
    f[4] = __uint_as_float(v.z << 16);
    f[5] = __uint_as_float(v.z & 0xffff0000u);
    f[6] = __uint_as_float(v.w << 16);
    f[7] = __uint_as_float(v.w & 0xffff0000u);
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
    v.x = f32_to_bf16_bits(f[0]) | (f32_to_bf16_bits(f[1]) << 16);
    v.y = f32_to_bf16_bits(f[2]) | (f32_to_bf16_bits(f[3]) << 16);
    v.z = f32_to_bf16_bits(f[4]) | (f32_to_bf16_bits(f[5]) << 16);
    v.w = f32_to_bf16_bits(f[6]) | (f32_to_bf16_bits(f[7]) << 16);
    return v;
  }
};

template <typename ST>
__device__ static inline u32x4 ld16(const ST* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// K/V page rows are read once per step: stream them past the caches.
template <typename ST>
__device__ static inline u32x4 ld16_stream(const ST* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

template <typename ST>
__device__ static inline void st16(ST* p, const u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// ---------------------------------------------------------------------------
// lane-group all-reduce (sum) over G consecutive lanes with DPP row ops:
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror, then
// cross-row shuffles for groups wider than a DPP row.

template <int CTRL>
__device__ static inline float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

template <int G>
__device__ static inline float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_f<0xB1>(v);
  if constexpr (G >= 4) v += dpp_f<0x4E>(v);
  if constexpr (G >= 8) v += dpp_f<0x141>(v);
  if constexpr (G >= 16) v += dpp_f<0x140>(v);
  if constexpr (G >= 32) v += __shfl_xor(v, 16);
  if constexpr (G >= 64) v += __shfl_xor(v, 32);
  return v;
}

// Orders this wave's LDS writes before its later LDS reads (LDS instructions of
// one wave execute in issue order; this stops the compiler from reordering).
__device__ static inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// paged layout, device view

struct PagesK {
  const int32_t* rows;
  int32_t rows_stride;
  int32_t max_pages;
  int32_t page_shift;
  int32_t num_pages;
  int64_t page_elems;  // page_size * d_model
  int32_t D;
};

// Element offset of frame `pos` (>= 0) of stream `ring` in a layer's pool slab,
// or -1 when the ring holds no valid page for it.
__device__ static inline int64_t page_offset(const PagesK& pg, const int32_t* ring, int64_t pos) {
  const int32_t page = ring[(int32_t)((pos >> pg.page_shift) % pg.max_pages)];
  if (page < 0 || page >= pg.num_pages) return -1;
  return (int64_t)page * pg.page_elems + (pos & ((1 << pg.page_shift) - 1)) * (int64_t)pg.D;
}

// ---------------------------------------------------------------------------
// fused append + paged relative-position attention

template <typename ST>
struct AttnK {
  const ST* q;
  const ST* kn;
  const ST* vn;
  int64_t q_sb, q_st, k_sb, k_st, v_sb, v_st;
  ST* kp;  // this layer's K slab of the pool (nullptr without pages)
  ST* vp;
  PagesK pg;
  const ST* pos;
  int64_t pos_sr;
  int32_t pos_rows;
  const ST* bu;
  const ST* bv;
  const uint8_t* mask;
  int64_t m_sb, m_sh, m_st;
  ST* out;
  int64_t o_sb, o_st;
  int32_t T, H, left, Lk, append, tiles;
  float scale;  // log2(e) / sqrt(head_dim)
};

// One workgroup per (stream b, head h, query group of TQ queries); W waves.
// Wave w of tile t owns the contiguous window rows jb = (t*W + w)*BLK ...
// jb + BLK - 1; inside the wave, lane group rl (G lanes) owns rows
// jb + n*RLW + rl, n < NR.  Each wave computes its own (q+v).pos terms for the
// BLK + TQ - 1 position rows its keys need into a wave-private LDS strip, so no
// workgroup barrier stalls the K/V loads in flight; the only barrier is the
// final cross-wave softmax combine.
template <typename ST, int DK, int TQ, int NR>
__global__ void __launch_bounds__(512) relpos_attn_kernel(const AttnK<ST> p) {
  constexpr int VEC = Tr<ST>::VEC;
  constexpr int G = DK / VEC;
  static_assert(G >= 1 && 64 % G == 0, "head_dim / VEC must divide 64");
  constexpr int RLW = 64 / G;
  constexpr int BLK = RLW * NR;
  constexpr int CROWS = BLK + TQ - 1;
  constexpr int NP = (CROWS + RLW - 1) / RLW;
  constexpr float NEG = -1e30f;
  constexpr float MASKED = -1e5f * 1.4426950408889634f;  // -1e5 in log2 units

  extern __shared__ float smem[];
  const int W = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane % G;
  const int rl = lane / G;
  const int b = blockIdx.x / p.H;
  const int h = blockIdx.x - b * p.H;
  const int i0 = blockIdx.y * TQ;
  const int nq = min(TQ, p.T - i0);
  const int col = h * DK + g * VEC;
  float* cbuf = smem + wave * (TQ * CROWS);

  int64_t A = 0;
  const int32_t* ring = nullptr;
  if (p.pg.rows) {
    const int32_t* row = p.pg.rows + (int64_t)b * p.pg.rows_stride;
    A = row[0];
    ring = row + 1;
  }

  float qu[TQ][VEC], qv[TQ][VEC];
  {
    float bu[VEC], bv[VEC];
    Tr<ST>::unpack(ld16(p.bu + col), bu);
    Tr<ST>::unpack(ld16(p.bv + col), bv);
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) {
      float qf[VEC];
      if (ii < nq) {
        Tr<ST>::unpack(ld16(p.q + b * p.q_sb + (int64_t)(i0 + ii) * p.q_st + col), qf);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) qf[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        qu[ii][e] = qf[e] + bu[e];
        qv[ii][e] = qf[e] + bv[e];
      }
    }
  }

  float m[TQ], l[TQ], acc[TQ][VEC];
#pragma unroll
  for (int ii = 0; ii < TQ; ++ii) {
    m[ii] = NEG;
    l[ii] = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[ii][e] = 0.f;
  }

  for (int tile = 0; tile < p.tiles; ++tile) {
    const int jb = (tile * W + wave) * BLK;
    if (jb >= p.Lk) break;  // uniform per wave

    // position-table rows rb .. rb + CROWS - 1 (L2-resident, shared by all streams)
    const int rb = jb + p.T - i0 - TQ;
    u32x4 pr[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int mm = rl + k * RLW;
      const int r = rb + mm;
      if (mm < CROWS && r >= 0 && r < p.pos_rows)
        pr[k] = ld16(p.pos + r * p.pos_sr + col);
      else
        pr[k] = u32x4{0u, 0u, 0u, 0u};
    }
    // mask bytes
    uint8_t mk[NR][TQ];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      const int j = jb + n * RLW + rl;
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii)
        mk[n][ii] = (p.mask && j < p.Lk && ii < nq)
                        ? p.mask[b * p.m_sb + h * p.m_sh + (int64_t)(i0 + ii) * p.m_st + j]
                        : (uint8_t)0;
    }
    // K/V rows: this step's frames from the projection output, older ones from pages
    u32x4 kr[NR], vr[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      const int j = jb + n * RLW + rl;
      kr[n] = u32x4{0u, 0u, 0u, 0u};
      vr[n] = u32x4{0u, 0u, 0u, 0u};
      if (j < p.Lk) {
        if (j >= p.left) {
          const int t = j - p.left;
          kr[n] = ld16(p.kn + b * p.k_sb + (int64_t)t * p.k_st + col);
          vr[n] = ld16(p.vn + b * p.v_sb + (int64_t)t * p.v_st + col);
        } else {
          const int64_t pos = A - p.left + j;
          if (pos >= 0) {
            const int64_t off = page_offset(p.pg, ring, pos);
            if (off >= 0) {
              kr[n] = ld16_stream(p.kp + off + col);
              vr[n] = ld16_stream(p.vp + off + col);
            }
          }
        }
      }
    }

    // bd terms c[ii][mm] = (q_ii + v) . pos[rb + mm], into this wave's LDS strip
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      float pf[VEC];
      Tr<ST>::unpack(pr[k], pf);
      const int mm = rl + k * RLW;
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) d = fmaf(qv[ii][e], pf[e], d);
        d = group_sum<G>(d);
        if (g == 0 && mm < CROWS) cbuf[ii * CROWS + mm] = d;
      }
    }
    wave_lds_sync();

    // scores in log2 units
    float s[TQ][NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      const int j = jb + n * RLW + rl;
      float kf[VEC];
      Tr<ST>::unpack(kr[n], kf);
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        float ac = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) ac = fmaf(qu[ii][e], kf[e], ac);
        ac = group_sum<G>(ac);
        float sc = NEG;
        if (j < p.Lk && ii < nq) {
          if (mk[n][ii])
            sc = fmaf(ac, p.scale, MASKED);
          else
            sc = (ac + cbuf[ii * CROWS + n * RLW + rl + TQ - 1 - ii]) * p.scale;
        }
        s[ii][n] = sc;
      }
    }

    // online softmax update over this lane group's rows
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) {
      float tmax = NEG;
#pragma unroll
      for (int n = 0; n < NR; ++n) tmax = fmaxf(tmax, s[ii][n]);
      const float mnew = fmaxf(m[ii], tmax);
      const float corr = __builtin_amdgcn_exp2f(m[ii] - mnew);
      l[ii] *= corr;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[ii][e] *= corr;
      m[ii] = mnew;
    }
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      float vf[VEC];
      Tr<ST>::unpack(vr[n], vf);
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        const float e = s[ii][n] > 0.5f * NEG ? __builtin_amdgcn_exp2f(s[ii][n] - m[ii]) : 0.f;
        l[ii] += e;
#pragma unroll
        for (int x = 0; x < VEC; ++x) acc[ii][x] = fmaf(e, vf[x], acc[ii][x]);
      }
    }

    // append this step's frames to the pages (query group 0 only)
    if (p.append && blockIdx.y == 0) {
#pragma unroll
      for (int n = 0; n < NR; ++n) {
        const int j = jb + n * RLW + rl;
        if (j < p.Lk && j >= p.left) {
          const int64_t off = page_offset(p.pg, ring, A + (j - p.left));
          if (off >= 0) {
            st16(p.kp + off + col, kr[n]);
            st16(p.vp + off + col, vr[n]);
          }
        }
      }
    }
    wave_lds_sync();  // the next tile rewrites cbuf
  }

  // combine the RLW lane groups of the wave
#pragma unroll
  for (int ii = 0; ii < TQ; ++ii) {
#pragma unroll
    for (int off = G; off < 64; off <<= 1) {
      const float m2 = __shfl_xor(m[ii], off);
      const float l2 = __shfl_xor(l[ii], off);
      const float mx = fmaxf(m[ii], m2);
      const float c1 = __builtin_amdgcn_exp2f(m[ii] - mx);
      const float c2 = __builtin_amdgcn_exp2f(m2 - mx);
      l[ii] = l[ii] * c1 + l2 * c2;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float a2 = __shfl_xor(acc[ii][e], off);
        acc[ii][e] = acc[ii][e] * c1 + a2 * c2;
      }
      m[ii] = mx;
    }
  }

  // combine the W waves through LDS and write [b, i, h*DK ...]
  float* comb = smem + W * TQ * CROWS;  // [W][TQ][2 + DK]
  if (rl == 0) {
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) {
      float* c = comb + (wave * TQ + ii) * (2 + DK);
      if (g == 0) {
        c[0] = m[ii];
        c[1] = l[ii];
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) c[2 + g * VEC + e] = acc[ii][e];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < TQ * G; idx += blockDim.x) {
    const int ii = idx / G;
    const int gg = idx - ii * G;
    if (ii >= nq) continue;
    float mx = NEG;
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, comb[(w * TQ + ii) * (2 + DK)]);
    float L = 0.f, o[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = 0.f;
    for (int w = 0; w < W; ++w) {
      const float* c = comb + (w * TQ + ii) * (2 + DK);
      const float f = __builtin_amdgcn_exp2f(c[0] - mx);
      L = fmaf(c[1], f, L);
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = fmaf(c[2 + gg * VEC + e], f, o[e]);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] *= inv;
    st16(p.out + b * p.o_sb + (int64_t)(i0 + ii) * p.o_st + h * DK + gg * VEC, Tr<ST>::pack(o));
  }
}

// ---------------------------------------------------------------------------
// append / gather

template <typename ST>
struct CopyK {
  ST* kp;  // layer slab
  ST* vp;
  PagesK pg;
  const ST* k;  // append: source; gather: destination
  const ST* v;
  ST* ko;
  ST* vo;
  int64_t k_sb, k_st, v_sb, v_st;
  int32_t B, rows, nchunk;  // rows: chunk (append) or window (gather)
  int32_t end_offset;       // gather: window ends at A + end_offset
};

template <typename ST>
__global__ void __launch_bounds__(256) kv_append_kernel(const CopyK<ST> p) {
  constexpr int VEC = Tr<ST>::VEC;
  const int64_t total = (int64_t)p.B * p.rows * p.nchunk;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % p.nchunk);
    const int64_t bt = idx / p.nchunk;
    const int t = (int)(bt % p.rows);
    const int b = (int)(bt / p.rows);
    const int32_t* row = p.pg.rows + (int64_t)b * p.pg.rows_stride;
    const int64_t off = page_offset(p.pg, row + 1, (int64_t)row[0] + t);
    if (off < 0) continue;
    const int64_t e = off + (int64_t)c * VEC;
    st16(p.kp + e, ld16(p.k + b * p.k_sb + (int64_t)t * p.k_st + c * VEC));
    st16(p.vp + e, ld16(p.v + b * p.v_sb + (int64_t)t * p.v_st + c * VEC));
  }
}

template <typename ST>
__global__ void __launch_bounds__(256) kv_gather_kernel(const CopyK<ST> p) {
  constexpr int VEC = Tr<ST>::VEC;
  const int64_t total = (int64_t)p.B * p.rows * p.nchunk;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % p.nchunk);
    const int64_t br = idx / p.nchunk;
    const int r = (int)(br % p.rows);
    const int b = (int)(br / p.rows);
    const int32_t* row = p.pg.rows + (int64_t)b * p.pg.rows_stride;
    const int64_t pos = (int64_t)row[0] + p.end_offset - p.rows + r;
    u32x4 kv = u32x4{0u, 0u, 0u, 0u}, vv = u32x4{0u, 0u, 0u, 0u};
    if (pos >= 0) {
      const int64_t off = page_offset(p.pg, row + 1, pos);
      if (off >= 0) {
        kv = ld16(p.kp + off + (int64_t)c * VEC);
        vv = ld16(p.vp + off + (int64_t)c * VEC);
      }
    }
    st16(p.ko + b * p.k_sb + (int64_t)r * p.k_st + c * VEC, kv);
    st16(p.vo + b * p.v_sb + (int64_t)r * p.v_st + c * VEC, vv);
  }
}

// ---------------------------------------------------------------------------
// streaming masks

struct MaskK {
  const int64_t* proc;
  const int64_t* cache_len;
  const int64_t* lengths;
  int64_t length_scalar;
  uint8_t* att;
  uint8_t* pad;
  int32_t B, T, left, C, left_chunks;
};

__global__ void __launch_bounds__(256) stream_mask_kernel(const MaskK p) {
  const int Lk = p.left + p.T;
  const int64_t total = (int64_t)p.B * p.T * Lk;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int j = (int)(idx % Lk);
    const int64_t bi = idx / Lk;
    const int i = (int)(bi % p.T);
    const int b = (int)(bi / p.T);
    const int64_t cl = p.cache_len[b];
    const int64_t pr = p.proc[b];
    const int64_t len = p.lengths ? p.lengths[b] : p.length_scalar;
    const int64_t key_start = pr - cl > 0 ? pr - cl : 0;
    const int64_t offset = p.left - cl;
    const bool valid_q = i < len;
    bool allow = false;
    if (j >= offset) {
      const int64_t kidx = j - offset;
      const int64_t kp = key_start + kidx;
      const int64_t qp = key_start + cl + i;
      const int64_t diff = qp / p.C - kp / p.C;
      const bool allowed = diff >= 0 && diff <= p.left_chunks;
      const bool valid_k = kidx < cl || (kidx - cl) < len;
      allow = allowed && valid_q && valid_k;
    }
    p.att[idx] = allow ? 0 : 1;
    if (j == 0 && p.pad) p.pad[bi] = valid_q ? 0 : 1;
  }
}

// ---------------------------------------------------------------------------
// host side

namespace {

struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) {
      ok = false;
      return;
    }
    if (dev >= 0 && dev != prev && hipSetDevice(dev) != hipSuccess) ok = false;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

int elem_size(int dtype) {
  switch (dtype) {
    case PK_DTYPE_F32: return 4;
    case PK_DTYPE_F16: return 2;
    case PK_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int log2_exact(int x) {
  int s = 0;
  while ((1 << s) < x) ++s;
  return (1 << s) == x ? s : -1;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PK_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PK_OK;
}

// Validates the paged layout for `batch` rows; fills the device view.
int pages_view(const pk_paged_layout& L, int layer, int vec, const char* what, PagesK* out) {
  if (!L.k_pool || !L.v_pool || !L.rows)
    return fail(PK_ERR_INVALID, "%s: k_pool, v_pool and rows must be set", what);
  if (!aligned16(L.k_pool) || !aligned16(L.v_pool))
    return fail(PK_ERR_INVALID, "%s: pools must be 16-byte aligned", what);
  if (L.num_layers <= 0 || layer < 0 || layer >= L.num_layers)
    return fail(PK_ERR_INVALID, "%s: layer %d out of range [0, %d)", what, layer, L.num_layers);
  if (L.num_pages <= 0) return fail(PK_ERR_INVALID, "%s: num_pages must be > 0", what);
  const int ps = log2_exact(L.page_size);
  if (L.page_size <= 0 || ps < 0)
    return fail(PK_ERR_INVALID, "%s: page_size %d is not a power of two", what, L.page_size);
  if (L.max_pages <= 0 || L.rows_stride < 1 + L.max_pages)
    return fail(PK_ERR_INVALID, "%s: need max_pages > 0 and rows_stride >= 1 + max_pages", what);
  if (L.d_model <= 0 || L.d_model % vec != 0)
    return fail(PK_ERR_INVALID, "%s: d_model %d must be a positive multiple of %d", what,
                L.d_model, vec);
  out->rows = L.rows;
  out->rows_stride = L.rows_stride;
  out->max_pages = L.max_pages;
  out->page_shift = ps;
  out->num_pages = L.num_pages;
  out->page_elems = (int64_t)L.page_size * L.d_model;
  out->D = L.d_model;
  return PK_OK;
}

int64_t layer_offset(const pk_paged_layout& L, int layer) {
  return (int64_t)layer * L.num_pages * L.page_size * L.d_model;
}

unsigned grid_for(int64_t total, int block) {
  int64_t g = (total + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (unsigned)g;
}

// ---- attention dispatch

template <typename ST, int DK, int TQ, int NR>
int launch_attn_t(const pk_attn_args* a, const AttnK<ST>& k, int W, hipStream_t s) {
  constexpr int VEC = Tr<ST>::VEC;
  constexpr int G = DK / VEC;
  constexpr int RLW = 64 / G;
  constexpr int CROWS = RLW * NR + TQ - 1;
  dim3 grid((unsigned)(a->batch * a->num_heads), (unsigned)((a->chunk + TQ - 1) / TQ));
  dim3 block((unsigned)(64 * W));
  const size_t smem = sizeof(float) * ((size_t)W * TQ * CROWS + (size_t)W * TQ * (2 + DK));
  if (a->start_event || a->stop_event) {
    hipExtLaunchKernelGGL(relpos_attn_kernel<ST, DK, TQ, NR>, grid, block, (uint32_t)smem, s,
                          (hipEvent_t)a->start_event, (hipEvent_t)a->stop_event, 0u, k);
  } else {
    hipLaunchKernelGGL((relpos_attn_kernel<ST, DK, TQ, NR>), grid, block, smem, s, k);
  }
  return check_launch("pk_paged_relpos_attn");
}

template <typename ST, int DK, int TQ>
int launch_attn_nr(const pk_attn_args* a, const AttnK<ST>& k, int NR, int W, hipStream_t s) {
  switch (NR) {
    case 2: return launch_attn_t<ST, DK, TQ, 2>(a, k, W, s);
    case 3: return launch_attn_t<ST, DK, TQ, 3>(a, k, W, s);
    case 4: return launch_attn_t<ST, DK, TQ, 4>(a, k, W, s);
    case 6: return launch_attn_t<ST, DK, TQ, 6>(a, k, W, s);
    default: return fail(PK_ERR_UNSUPPORTED, "pk_paged_relpos_attn: rows_per_lane %d not built", NR);
  }
}

template <typename ST, int DK>
int launch_attn_tq(const pk_attn_args* a, const AttnK<ST>& k, int TQ, int NR, int W,
                   hipStream_t s) {
  switch (TQ) {
    case 1: return launch_attn_nr<ST, DK, 1>(a, k, NR, W, s);
    case 2: return launch_attn_nr<ST, DK, 2>(a, k, NR, W, s);
    case 4: return launch_attn_nr<ST, DK, 4>(a, k, NR, W, s);
    default: return fail(PK_ERR_UNSUPPORTED, "pk_paged_relpos_attn: query group %d not built", TQ);
  }
}

// Queries per workgroup: 1, 2 or 4 for chunks up to 4 frames, else groups of 2.
int pick_tq(int T) {
  if (T <= 1) return 1;
  if (T == 2) return 2;
  if (T <= 4) return 4;
  return 2;
}

// Rows per lane NR and waves per workgroup W for a window of Lk keys: prefer a
// single tile, then the least padding, then NR close to 4.
void pick_tiling(int Lk, int rlw, int hint, int* NR, int* W, int* tiles) {
  static const int cand[4] = {2, 3, 4, 6};
  int best_nr = 0, best_w = 0, best_t = 0;
  long best_score = -1;
  for (int c : cand) {
    if (hint > 0 && c != hint) continue;
    const int per_wave = rlw * c;
    int w = (Lk + per_wave - 1) / per_wave;
    if (w > 8) w = 8;
    if (w < 1) w = 1;
    const int t = (Lk + w * per_wave - 1) / (w * per_wave);
    const int waste = t * w * per_wave - Lk;
    const int dist = c > 4 ? c - 4 : 4 - c;
    const long score = (long)t * 1000000L + (long)waste * 100L + dist;
    if (best_score < 0 || score < best_score) {
      best_score = score;
      best_nr = c;
      best_w = w;
      best_t = t;
    }
  }
  *NR = best_nr;
  *W = best_w;
  *tiles = best_t;
}

template <typename ST>
int attn_typed(const pk_attn_args* a, hipStream_t s) {
  constexpr int VEC = Tr<ST>::VEC;
  const char* what = "pk_paged_relpos_attn";
  const int DK = a->head_dim;
  if (DK != 64 && DK != 128)
    return fail(PK_ERR_UNSUPPORTED, "%s: head_dim %d not built (64 or 128)", what, DK);
  if (a->num_heads <= 0) return fail(PK_ERR_INVALID, "%s: num_heads must be > 0", what);
  const int D = a->num_heads * DK;
  if (a->chunk <= 0 || a->left < 0)
    return fail(PK_ERR_INVALID, "%s: need chunk > 0 and left >= 0", what);
  const int Lk = a->left + a->chunk;
  if (a->batch < 0) return fail(PK_ERR_INVALID, "%s: batch must be >= 0", what);
  if (a->batch == 0) return PK_OK;
  if (a->pos_rows < Lk + a->chunk - 1)
    return fail(PK_ERR_INVALID, "%s: pos has %d rows, needs >= window + chunk - 1 = %d", what,
                a->pos_rows, Lk + a->chunk - 1);
  if (!a->query || !a->key || !a->value || !a->pos || !a->bias_u || !a->bias_v || !a->out)
    return fail(PK_ERR_INVALID, "%s: a tensor pointer is NULL", what);
  const void* ptrs[7] = {a->query, a->key, a->value, a->pos, a->bias_u, a->bias_v, a->out};
  for (const void* q : ptrs)
    if (!aligned16(q)) return fail(PK_ERR_INVALID, "%s: tensors must be 16-byte aligned", what);
  const int64_t strides[9] = {a->query_stride_b, a->query_stride_t, a->key_stride_b,
                              a->key_stride_t,   a->value_stride_b, a->value_stride_t,
                              a->pos_stride,     a->out_stride_b,   a->out_stride_t};
  for (int64_t st : strides)
    if (st < 0 || st % VEC != 0)
      return fail(PK_ERR_INVALID, "%s: strides must be non-negative multiples of %d elements",
                  what, VEC);
  if ((int64_t)a->batch * a->num_heads > 0x7fffffffLL)
    return fail(PK_ERR_INVALID, "%s: batch * heads too large", what);

  AttnK<ST> k{};
  k.q = static_cast<const ST*>(a->query);
  k.kn = static_cast<const ST*>(a->key);
  k.vn = static_cast<const ST*>(a->value);
  k.q_sb = a->query_stride_b;
  k.q_st = a->query_stride_t;
  k.k_sb = a->key_stride_b;
  k.k_st = a->key_stride_t;
  k.v_sb = a->value_stride_b;
  k.v_st = a->value_stride_t;
  const bool need_pages = a->left > 0 || a->append;
  if (need_pages) {
    const int rc = pages_view(a->pages, a->layer, VEC, what, &k.pg);
    if (rc != PK_OK) return rc;
    if (a->pages.d_model != D)
      return fail(PK_ERR_INVALID, "%s: pages.d_model %d != heads*head_dim %d", what,
                  a->pages.d_model, D);
    const int64_t lo = layer_offset(a->pages, a->layer);
    k.kp = static_cast<ST*>(a->pages.k_pool) + lo;
    k.vp = static_cast<ST*>(a->pages.v_pool) + lo;
  }
  k.pos = static_cast<const ST*>(a->pos);
  k.pos_sr = a->pos_stride;
  k.pos_rows = a->pos_rows;
  k.bu = static_cast<const ST*>(a->bias_u);
  k.bv = static_cast<const ST*>(a->bias_v);
  k.mask = a->mask;
  k.m_sb = a->mask_stride_b;
  k.m_sh = a->mask_stride_h;
  k.m_st = a->mask_stride_t;
  k.out = static_cast<ST*>(a->out);
  k.o_sb = a->out_stride_b;
  k.o_st = a->out_stride_t;
  k.T = a->chunk;
  k.H = a->num_heads;
  k.left = a->left;
  k.Lk = Lk;
  k.append = a->append ? 1 : 0;
  k.scale = 1.4426950408889634f / sqrtf((float)DK);

  const int G = DK / VEC;
  const int rlw = 64 / G;
  const int TQ = pick_tq(a->chunk);
  int NR = 0, W = 0, tiles = 0;
  pick_tiling(Lk, rlw, a->rows_per_lane, &NR, &W, &tiles);
  if (NR == 0)
    return fail(PK_ERR_UNSUPPORTED, "%s: rows_per_lane %d not built (2, 3, 4, 6)", what,
                a->rows_per_lane);
  k.tiles = tiles;
  if (DK == 64) return launch_attn_tq<ST, 64>(a, k, TQ, NR, W, s);
  return launch_attn_tq<ST, 128>(a, k, TQ, NR, W, s);
}

template <typename ST>
int copy_typed(bool gather, const pk_paged_layout& L, int layer, int B, int rows, int end_offset,
               const void* k, int64_t k_sb, int64_t k_st, const void* v, int64_t v_sb,
               int64_t v_st, hipStream_t s, const char* what) {
  constexpr int VEC = Tr<ST>::VEC;
  CopyK<ST> p{};
  if (B == 0) return PK_OK;
  int rc = pages_view(L, layer, VEC, what, &p.pg);
  if (rc != PK_OK) return rc;
  if (!k || !v || !aligned16(k) || !aligned16(v))
    return fail(PK_ERR_INVALID, "%s: K/V tensors must be non-NULL and 16-byte aligned", what);
  const int64_t strides[4] = {k_sb, k_st, v_sb, v_st};
  for (int64_t st : strides)
    if (st < 0 || st % VEC != 0)
      return fail(PK_ERR_INVALID, "%s: strides must be non-negative multiples of %d elements",
                  what, VEC);
  if (B < 0 || rows <= 0) return fail(PK_ERR_INVALID, "%s: need batch >= 0 and rows > 0", what);
  if (B == 0) return PK_OK;
  const int64_t lo = layer_offset(L, layer);
  p.kp = static_cast<ST*>(L.k_pool) + lo;
  p.vp = static_cast<ST*>(L.v_pool) + lo;
  p.k = static_cast<const ST*>(k);
  p.v = static_cast<const ST*>(v);
  p.ko = const_cast<ST*>(p.k);
  p.vo = const_cast<ST*>(p.v);
  p.k_sb = k_sb;
  p.k_st = k_st;
  p.v_sb = v_sb;
  p.v_st = v_st;
  p.B = B;
  p.rows = rows;
  p.nchunk = L.d_model / VEC;
  p.end_offset = end_offset;
  const int64_t total = (int64_t)B * rows * p.nchunk;
  if (gather)
    hipLaunchKernelGGL(kv_gather_kernel<ST>, dim3(grid_for(total, 256)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(kv_append_kernel<ST>, dim3(grid_for(total, 256)), dim3(256), 0, s, p);
  return check_launch(what);
}

}  // namespace
}  // namespace pk

extern "C" {

int pk_paged_relpos_attn(const pk_attn_args* a, void* stream) {
  pk::clear_error();
  if (!a) return pk::fail(PK_ERR_INVALID, "pk_paged_relpos_attn: args is NULL");
  pk::DeviceGuard dg(a->device);
  if (!dg.ok) return pk::fail(PK_ERR_HIP, "pk_paged_relpos_attn: cannot select device %d", a->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case PK_DTYPE_F32: return pk::attn_typed<float>(a, s);
    case PK_DTYPE_F16: return pk::attn_typed<_Float16>(a, s);
    case PK_DTYPE_BF16: return pk::attn_typed<pk::bf16_t>(a, s);
    default: return pk::fail(PK_ERR_INVALID, "pk_paged_relpos_attn: unknown dtype %d", a->dtype);
  }
}

int pk_kv_append(const pk_kv_append_args* a, void* stream) {
  pk::clear_error();
  if (!a) return pk::fail(PK_ERR_INVALID, "pk_kv_append: args is NULL");
  pk::DeviceGuard dg(a->device);
  if (!dg.ok) return pk::fail(PK_ERR_HIP, "pk_kv_append: cannot select device %d", a->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* what = "pk_kv_append";
  switch (a->dtype) {
    case PK_DTYPE_F32:
      return pk::copy_typed<float>(false, a->pages, a->layer, a->batch, a->chunk, 0, a->key,
                                   a->key_stride_b, a->key_stride_t, a->value, a->value_stride_b,
                                   a->value_stride_t, s, what);
    case PK_DTYPE_F16:
      return pk::copy_typed<_Float16>(false, a->pages, a->layer, a->batch, a->chunk, 0, a->key,
                                      a->key_stride_b, a->key_stride_t, a->value,
                                      a->value_stride_b, a->value_stride_t, s, what);
    case PK_DTYPE_BF16:
      return pk::copy_typed<pk::bf16_t>(false, a->pages, a->layer, a->batch, a->chunk, 0, a->key,
                                        a->key_stride_b, a->key_stride_t, a->value,
                                        a->value_stride_b, a->value_stride_t, s, what);
    default: return pk::fail(PK_ERR_INVALID, "pk_kv_append: unknown dtype %d", a->dtype);
  }
}

int pk_kv_gather(const pk_kv_gather_args* a, void* stream) {
  pk::clear_error();
  if (!a) return pk::fail(PK_ERR_INVALID, "pk_kv_gather: args is NULL");
  pk::DeviceGuard dg(a->device);
  if (!dg.ok) return pk::fail(PK_ERR_HIP, "pk_kv_gather: cannot select device %d", a->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* what = "pk_kv_gather";
  switch (a->dtype) {
    case PK_DTYPE_F32:
      return pk::copy_typed<float>(true, a->pages, a->layer, a->batch, a->window, a->end_offset,
                                   a->out_k, a->out_k_stride_b, a->out_k_stride_t, a->out_v,
                                   a->out_v_stride_b, a->out_v_stride_t, s, what);
    case PK_DTYPE_F16:
      return pk::copy_typed<_Float16>(true, a->pages, a->layer, a->batch, a->window,
                                      a->end_offset, a->out_k, a->out_k_stride_b,
                                      a->out_k_stride_t, a->out_v, a->out_v_stride_b,
                                      a->out_v_stride_t, s, what);
    case PK_DTYPE_BF16:
      return pk::copy_typed<pk::bf16_t>(true, a->pages, a->layer, a->batch, a->window,
                                        a->end_offset, a->out_k, a->out_k_stride_b,
                                        a->out_k_stride_t, a->out_v, a->out_v_stride_b,
                                        a->out_v_stride_t, s, what);
    default: return pk::fail(PK_ERR_INVALID, "pk_kv_gather: unknown dtype %d", a->dtype);
  }
}

int pk_streaming_mask(const pk_mask_args* a, void* stream) {
  pk::clear_error();
  if (!a) return pk::fail(PK_ERR_INVALID, "pk_streaming_mask: args is NULL");
  if (a->batch < 0 || a->chunk <= 0 || a->left < 0 || a->chunk_size <= 0)
    return pk::fail(PK_ERR_INVALID,
                    "pk_streaming_mask: need batch >= 0, chunk > 0, left >= 0, chunk_size > 0");
  if (a->batch == 0) return PK_OK;
  if (!a->processed_frames || !a->cache_lengths || !a->att_mask)
    return pk::fail(PK_ERR_INVALID, "pk_streaming_mask: state and att_mask must be set");
  pk::DeviceGuard dg(a->device);
  if (!dg.ok) return pk::fail(PK_ERR_HIP, "pk_streaming_mask: cannot select device %d", a->device);
  pk::MaskK p{};
  p.proc = a->processed_frames;
  p.cache_len = a->cache_lengths;
  p.lengths = a->lengths;
  p.length_scalar = a->length_scalar;
  p.att = a->att_mask;
  p.pad = a->pad_mask;
  p.B = a->batch;
  p.T = a->chunk;
  p.left = a->left;
  p.C = a->chunk_size;
  p.left_chunks = a->left / a->chunk_size;
  const int64_t total = (int64_t)a->batch * a->chunk * (a->left + a->chunk);
  hipLaunchKernelGGL(pk::stream_mask_kernel, dim3(pk::grid_for(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p);
  return pk::check_launch("pk_streaming_mask");
}

}  // extern "C"
