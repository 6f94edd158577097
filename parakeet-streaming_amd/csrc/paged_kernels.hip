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
#include <type_traits>

#include "pk_common.h"
#include "pk_device.h"

namespace pk {

// ---------------------------------------------------------------------------
// paged layout, device view

// A page holds its page_size frames as column blocks: element (page, row r,
// column c) of a layer's slab is at
//   page * page_size * D + (c / CB) * page_size * CB + r * CB + c % CB,
// CB = gcd(D, 64 / element size): 64-byte blocks at the model shapes (32
// fp16/bf16 elements, 16 fp32), so one block of 16 consecutive frames is 1 KB
// of contiguous memory; rows narrower than 64 bytes are one block.
struct PagesK {
  const int32_t* rows;
  int32_t rows_stride;
  int32_t max_pages;
  int32_t page_shift;
  int32_t num_pages;
  int64_t page_elems;  // page_size * d_model
  int32_t D;
  int32_t cb_shift;    // log2(CB)
};

// Element offset of frame `pos` (0 <= pos < 2^31, the int32 range of the
// rows' frame counter) of stream `ring` in a layer's pool slab, without the
// column part (page_col), or -1 when the ring holds no valid page for it.
// 32-bit index arithmetic.
__device__ static inline int64_t page_offset(const PagesK& pg, const int32_t* ring, int64_t pos) {
  const uint32_t p32 = (uint32_t)pos;
  const int32_t page = ring[(p32 >> pg.page_shift) % (uint32_t)pg.max_pages];
  if (page < 0 || page >= pg.num_pages) return -1;
  return (int64_t)page * pg.page_elems + ((int64_t)(p32 & ((1u << pg.page_shift) - 1u)) << pg.cb_shift);
}

// Column part of a page element offset: column c (a 16-byte chunk never
// crosses a block).
__device__ static inline int64_t page_col(const PagesK& pg, int c) {
  return ((int64_t)(c >> pg.cb_shift) << (pg.page_shift + pg.cb_shift)) + (c & ((1 << pg.cb_shift) - 1));
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
  int64_t pos_sb;  // per-stream tables (vector-ALU kernel only); 0: one shared table
  int32_t pos_rows;
  const ST* bu;
  const ST* bv;
  const uint8_t* mask;
  int64_t m_sb, m_sh, m_st;
  const int64_t* st_proc;  // state-derived mask (mask == nullptr)
  const int64_t* st_cl;
  const int64_t* st_len;
  int64_t len_scalar;
  int32_t chunk_size, left_chunks;
  uint32_t c_magic;
  ST* out;
  int64_t o_sb, o_st;
  int32_t B, T, H, left, Lk, append, tiles;  // B: rows of the batch arrays
  const int32_t* nact;  // streams 0..*nact-1 are live (nullptr: all B)
  float scale;          // log2(e) / sqrt(head_dim)
};

// Streaming-mask state of one stream (encoder.py:186-212), 32-bit.  The key and
// query chunk indices are floor((key_start + x) / C) = ks_q + (ks_r + x) / C with
// key_start = ks_q * C + ks_r, so only small non-negative values are divided.
struct StreamMask {
  int cl, len, offset, ks_q, ks_r, C, left_chunks;
  uint32_t magic;  // floor(2^32 / C) + 1 for C >= 2: x / C == umulhi(x, magic), x < 2^32 / C
                   // (the small per-score arguments, bounded on the host)

  __device__ inline int div_c(uint32_t x) const {
    return C == 1 ? (int)x : (int)__umulhi(x, magic);
  }
  __device__ inline void set(int64_t pr, int64_t c, int64_t n, int left, int C_, int lc,
                             uint32_t magic_) {
    n = n < -1 ? -1 : (n > 0x7fffffff ? 0x7fffffff : n);
    const int64_t ks = pr - c > 0 ? pr - c : 0;  // encoder.py:189
    cl = (int)c;
    len = (int)n;
    offset = left - cl;  // encoder.py:214
    C = C_;
    left_chunks = lc;
    magic = magic_;
    ks_q = (int)((uint32_t)ks / (uint32_t)C);  // once per stream: exact for any ks < 2^32
    ks_r = (int)ks - ks_q * C;
  }
  // chunk index of query i (its frame is key_start + cl + i)
  __device__ inline int query_chunk(int i) const { return ks_q + div_c((uint32_t)(ks_r + cl + i)); }
  // true where the reference's att_mask is set (encoder.py:199-225)
  __device__ inline bool masked(int i, int qchunk, int j) const {
    if (j < offset || i >= len) return true;
    const int kidx = j - offset;
    const int kc = ks_q + div_c((uint32_t)(ks_r + kidx));
    const int diff = qchunk - kc;
    const bool allowed = diff >= 0 && diff <= left_chunks;
    const bool valid_k = kidx < cl || kidx - cl < len;
    return !(allowed && valid_k);
  }
};

// One workgroup of WAVES waves per (stream b, head h, query group of TQ
// queries); wave w takes the tiles w, w + WAVES, ... of BLK = RLW*NR window
// rows, and its lane group rl (G lanes, VEC columns each) the rows jb + n*RLW
// + rl, n < NR, of each.  Per tile:
//   1. the position rows of the tile (L2-resident, shared by all streams) are
//      loaded in the same round trip as the stream's page header, the queries
//      and the biases, and reduced to the (q+v).pos terms in a wave-private LDS
//      strip before any K/V load is issued (vector loads complete in issue
//      order, so position loads queued behind K/V would wait for all of them);
//   2. page ids come from the ring held one entry per lane (ds_bpermute), and
//      all NR K rows and NR V rows of the lane are issued back to back;
//   3. scores, an online softmax over the lane group's rows and the value sum.
// The lane groups are combined with cross-lane shuffles at the end, then
// (WAVES > 1) the waves' states through LDS in wave order, one barrier: one
// wave holds a whole window in flight, or WAVES waves a quarter of it each
// (small batches, where a single wave's latency is the launch's).
template <typename ST, int DK, int TQ, int NR, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) relpos_attn_kernel(const AttnK<ST> p) {
  constexpr int VEC = Tr<ST>::VEC;
  constexpr int G = DK / VEC;
  static_assert(G >= 1 && 64 % G == 0, "head_dim / VEC must divide 64");
  constexpr int RLW = 64 / G;
  constexpr int BLK = RLW * NR;
  constexpr int CROWS = BLK + TQ - 1;
  constexpr int NP = (CROWS + RLW - 1) / RLW;
  constexpr float NEG = -1e30f;
  constexpr float MASKED = -1e5f * 1.4426950408889634f;  // -1e5 in log2 units

  __shared__ float cbuf[WAVES][TQ][NP * RLW];  // (q+v).pos terms of the wave's tile
  __shared__ uint8_t mbuf[WAVES][TQ][BLK];     // mask bytes of the wave's tile (pointer mask)

  const int lane = threadIdx.x & 63;
  const int wave = WAVES == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float(*const cb)[NP * RLW] = cbuf[wave];
  uint8_t(*const mb)[BLK] = mbuf[wave];
  const int g = lane % G;
  const int rl = lane / G;
  const int b = blockIdx.x / p.H;
  const int h = blockIdx.x - b * p.H;
  if (p.nact && b >= *p.nact) return;  // the workgroup's stream is not live this step
  const int i0 = blockIdx.y * TQ;
  const int nq = min(TQ, p.T - i0);
  const int col = h * DK + g * VEC;
  const int64_t pcol = page_col(p.pg, col);  // the lane's columns in a page row

  // page header of the stream: frames appended before this step and the ring,
  // one ring entry per lane
  int A = 0;
  int ring_lane = -1;
  const int32_t* ring = nullptr;
  const int M = p.pg.max_pages;
  if (p.pg.rows) {
    const int32_t* row = p.pg.rows + (int64_t)b * p.pg.rows_stride;
    A = row[0];
    ring = row + 1;
    ring_lane = ring[min(lane, M - 1)];
  }
  const int mask_mode = p.mask ? 1 : (p.st_proc ? 2 : 0);
  StreamMask sm{};
  int qchunk[TQ];
  if (mask_mode == 2) {
    sm.set(p.st_proc[b], p.st_cl[b], p.st_len ? p.st_len[b] : p.len_scalar, p.left, p.chunk_size,
           p.left_chunks, p.c_magic);
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) qchunk[ii] = sm.query_chunk(i0 + ii);
  }

  u32x4 qraw[TQ];
#pragma unroll
  for (int ii = 0; ii < TQ; ++ii) {
    const int ic = min(i0 + ii, p.T - 1);
    qraw[ii] = ld16(p.q + b * p.q_sb + (int64_t)ic * p.q_st + col);
  }
  const u32x4 buraw = ld16(p.bu + col);
  const u32x4 bvraw = ld16(p.bv + col);

  float m[TQ], l[TQ], acc[TQ][VEC];
#pragma unroll
  for (int ii = 0; ii < TQ; ++ii) {
    m[ii] = NEG;
    l[ii] = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[ii][e] = 0.f;
  }

  const uint32_t pmask = (1u << p.pg.page_shift) - 1u;
  const ST* kn_b = p.kn + b * p.k_sb;
  const ST* vn_b = p.vn + b * p.v_sb;

  for (int tile = wave; tile < p.tiles; tile += WAVES) {
    const int jb = tile * BLK;

    // (1) position rows rb .. rb + CROWS - 1 and mask bytes of the tile
    const int rb = jb + p.T - i0 - TQ;
    u32x4 pr[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int r = min(max(rb + rl + k * RLW, 0), p.pos_rows - 1);
      pr[k] = ld16(p.pos + b * p.pos_sb + r * p.pos_sr + col);
    }
    if (mask_mode == 1) {
      for (int x = lane; x < TQ * BLK; x += 64) {
        const int ii = x / BLK;
        const int jj = x - ii * BLK;
        const int ic = min(i0 + ii, p.T - 1);
        const int jcl = min(jb + jj, p.Lk - 1);
        mb[ii][jj] = p.mask[b * p.m_sb + h * p.m_sh + (int64_t)ic * p.m_st + jcl];
      }
    }
    float qu[TQ][VEC];
    {
      float bu[VEC], bv[VEC];
      Tr<ST>::unpack(buraw, bu);
      Tr<ST>::unpack(bvraw, bv);
      float qv[TQ][VEC];
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        float qf[VEC];
        Tr<ST>::unpack(qraw[ii], qf);
        const bool live = ii < nq;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float x = live ? qf[e] : 0.f;
          qu[ii][e] = x + bu[e];
          qv[ii][e] = x + bv[e];
        }
      }
      // bd terms cb[ii][mm] = (q_ii + v) . pos[rb + mm]
#pragma unroll
      for (int k = 0; k < NP; ++k) {
        float pf[VEC];
        Tr<ST>::unpack(pr[k], pf);
        const int mm = rl + k * RLW;
        const int r = rb + mm;
        const bool live = r >= 0 && r < p.pos_rows;
#pragma unroll
        for (int ii = 0; ii < TQ; ++ii) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) d = fmaf(qv[ii][e], pf[e], d);
          d = group_sum<G>(d);
          if (g == 0) cb[ii][mm] = live ? d : 0.f;
        }
      }
    }

    // (2) page ids and K/V rows: this step's frames from the projection
    //     output, older ones from the pages
    u32x4 kr[NR], vr[NR];
    bool ok[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      const int j = jb + n * RLW + rl;
      const int jc = min(j, p.Lk - 1);
      const int pos = A - p.left + jc;
      const bool fresh = jc >= p.left;
      int page = -1;
      if (ring) {
        const uint32_t ridx = ((uint32_t)max(pos, 0) >> p.pg.page_shift) % (uint32_t)M;
        page = __shfl(ring_lane, (int)ridx);
      }
      const bool paged_ok = pos >= 0 && page >= 0 && page < p.pg.num_pages;
      ok[n] = j < p.Lk && (fresh || paged_ok);
      const int t = fresh ? jc - p.left : 0;
      const int64_t poff = (int64_t)(paged_ok ? page : 0) * p.pg.page_elems +
                           ((int64_t)((uint32_t)max(pos, 0) & pmask) << p.pg.cb_shift);
      const bool from_new = fresh || !paged_ok;
      const ST* ka = from_new ? kn_b + (int64_t)t * p.k_st + col : p.kp + poff + pcol;
      const ST* va = from_new ? vn_b + (int64_t)t * p.v_st + col : p.vp + poff + pcol;
      kr[n] = ld16(ka);
      vr[n] = ld16(va);
    }
    wave_lds_sync();

    // (3) scores in log2 units
    float s[TQ][NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) {
      const int j = jb + n * RLW + rl;
      const int jc = min(j, p.Lk - 1);
      float kf[VEC];
      Tr<ST>::unpack(kr[n], kf);
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        float ac = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) ac = fmaf(qu[ii][e], kf[e], ac);
        ac = group_sum<G>(ac);
        if (!ok[n]) ac = 0.f;  // a key outside the stream's history reads as zeros
        bool msk = false;
        if (mask_mode == 1) msk = mb[ii][n * RLW + rl] != 0;
        if (mask_mode == 2) msk = sm.masked(i0 + ii, qchunk[ii], jc);
        float sc;
        if (msk)
          sc = fmaf(ac, p.scale, MASKED);
        else
          sc = (ac + cb[ii][n * RLW + rl + TQ - 1 - ii]) * p.scale;
        s[ii][n] = (j < p.Lk && ii < nq) ? sc : NEG;
      }
    }

    // online softmax over the lane group's rows, then the value sum
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
      if (!ok[n]) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) vf[e] = 0.f;
      }
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
            st16(p.kp + off + pcol, kr[n]);
            st16(p.vp + off + pcol, vr[n]);
          }
        }
      }
    }
    wave_lds_sync();  // the wave's next tile rewrites its cbuf / mbuf
  }

  // combine the RLW lane groups and write [b, i, h*DK + ...]
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
  if constexpr (WAVES > 1) {
    // every lane holds its wave's state; lane group 0 of each wave stores it
    // and wave 0 folds in waves 1 .. WAVES-1 in order (an empty wave: m = NEG,
    // l = 0, adds nothing)
    __shared__ float part[WAVES][TQ][2 + VEC][G];
    if (rl == 0) {
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        part[wave][ii][0][g] = m[ii];
        part[wave][ii][1][g] = l[ii];
#pragma unroll
        for (int e = 0; e < VEC; ++e) part[wave][ii][2 + e][g] = acc[ii][e];
      }
    }
    __syncthreads();
    if (wave != 0) return;
    if (rl == 0) {
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        for (int w = 1; w < WAVES; ++w) {
          const float m2 = part[w][ii][0][g];
          const float l2 = part[w][ii][1][g];
          const float mx = fmaxf(m[ii], m2);
          const float c1 = __builtin_amdgcn_exp2f(m[ii] - mx);
          const float c2 = __builtin_amdgcn_exp2f(m2 - mx);
          l[ii] = l[ii] * c1 + l2 * c2;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[ii][e] = acc[ii][e] * c1 + part[w][ii][2 + e][g] * c2;
          m[ii] = mx;
        }
      }
    }
  }
  if (rl == 0) {
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) {
      if (ii >= nq) continue;
      const float inv = l[ii] > 0.f ? 1.f / l[ii] : 0.f;
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = acc[ii][e] * inv;
      st16(p.out + b * p.o_sb + (int64_t)(i0 + ii) * p.o_st + col, Tr<ST>::pack(o));
    }
  }
}

// ---------------------------------------------------------------------------
// fused append + paged relative-position attention on the matrix cores
// (fp16 / bf16)

typedef short i16x4_t __attribute__((ext_vector_type(4)));

// 16-bit operand type of the matrix-core path, with the two MFMA shapes used:
//   16x16x32: lane l holds A[l%16][8*(l/16)+e], B[8*(l/16)+e][l%16], e < 8
//   16x16x16: lane l holds A[l%16][4*(l/16)+e], B[4*(l/16)+e][l%16], e < 4
//   both:     lane l holds D[4*(l/16)+i][l%16], i < 4
template <typename ST>
struct Mma;

template <>
struct Mma<bf16_t> {
  typedef __bf16 H;
  typedef __bf16 H8 __attribute__((ext_vector_type(8)));
  typedef __bf16 H4 __attribute__((ext_vector_type(4)));
  __device__ static inline f32x4_t k32(const u32x4 a, const u32x4 b, const f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(H8, a),
                                                   __builtin_bit_cast(H8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4_t k16(const i16x4_t a, const i16x4_t b, const f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mma<_Float16> {
  typedef _Float16 H;
  typedef _Float16 H8 __attribute__((ext_vector_type(8)));
  typedef _Float16 H4 __attribute__((ext_vector_type(4)));
  __device__ static inline f32x4_t k32(const u32x4 a, const u32x4 b, const f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(H8, a),
                                                  __builtin_bit_cast(H8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4_t k16(const i16x4_t a, const i16x4_t b, const f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(H4, a),
                                                 __builtin_bit_cast(H4, b), c, 0, 0, 0);
  }
};

// x = hi + lo with hi, lo in the 16-bit operand type (x to ~2^-17 for bf16,
// ~2^-22 for fp16): the high or the low part of each element.
template <typename ST, int N, typename V>
__device__ static inline V split16(const float* x, bool low) {
  typedef typename Mma<ST>::H H;
  typedef H HN __attribute__((ext_vector_type(N)));
  HN out;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const H hi = (H)x[e];
    out[e] = low ? (H)(x[e] - (float)hi) : hi;
  }
  return __builtin_bit_cast(V, out);
}

__device__ static inline float lane_at(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Max / sum over all 64 lanes as a wave-uniform value: within each row of 16
// lanes by DPP, then the rows' lanes 0, 16, 32 and 48 read as scalars (no LDS
// round trip); the sum adds (row 0 + row 1) + (row 2 + row 3).
__device__ static inline float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(lane_at(v, 0), lane_at(v, 16)), fmaxf(lane_at(v, 32), lane_at(v, 48)));
}
__device__ static inline float wave_sum(float v) {
  v = group_sum<16>(v);
  return (lane_at(v, 0) + lane_at(v, 16)) + (lane_at(v, 32) + lane_at(v, 48));
}

// Index-mode buffer access: a resource describes `nrows` rows of `stride`
// bytes; a row index >= nrows reads zeros and drops stores (the hardware range
// check), which is how absent rows -- positions before a stream's first frame,
// pages a stream does not hold, keys past the window -- come out as the zeros
// the reference's dense window holds there.
extern "C" __device__ u32x4 pk_buffer_load_x4(__amdgpu_buffer_rsrc_t rsrc, int vindex, int voffset,
                                              int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");
extern "C" __device__ void pk_buffer_store_x4(u32x4 data, __amdgpu_buffer_rsrc_t rsrc, int vindex,
                                              int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.store.v4i32");

constexpr uint32_t kNoRow = 0xffffffffu;  // a row index every resource rejects
constexpr int kMaxBufferStride = 16383;   // bytes, stride field of the resource

__device__ static inline __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int stride_bytes,
                                                          uint32_t nrows) {
  // word 3 0x00020000: 32-bit data format, the setting untyped loads need on CDNA
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)stride_bytes,
                                           (int)nrows, 0x00020000);
}

// Workgroup of NW waves (4, or 2 when a 4-wave grid would leave CUs idle):
// NW / SPLIT streams of one head h and one query pair, each stream's head
// split over SPLIT = head_dim / 64 waves of 64 columns.
// Score slots are window columns: per pass, NT tiles of 16 slots hold columns
// jb .. jb + 16*NT - 1; column j is cached history (j < left, read from the
// pages), one of this step's frames (left <= j < left + chunk, read from the
// projection output) or past the window.  Absent rows (positions before the
// stream's first frame, pages the stream does not hold, columns past the
// window) read zeros through the buffer range check.
// Per pass:
//   * the position rows the pass needs (shared by the workgroup's streams) are
//     staged once in LDS, rows padded by 16 bytes so the 16 lanes of an MFMA
//     operand read hit distinct banks; only the tiles that hold a row some
//     valid slot reads are staged and multiplied;
//   * (q+u).k and (q+v).pos on 16x16x32 MFMAs: A rows 0..7 hold (q+u) and
//     (q+v) of both queries split into high and low 16-bit parts, so the
//     16-bit operands lose nothing against the fp32 query + bias sums; B is a
//     tile of 16 K rows (lane = key, 8 columns per k-step) or 16 staged
//     position rows; the SPLIT waves' partial sums meet in LDS;
//   * scores and the online softmax spread over the 64 lanes (slot = lane,
//     lane + 64);
//   * P.V on 16x16x16 MFMAs: A = the probabilities (high and low 16-bit
//     parts), B = 16 V rows x 16 columns transposed on the way out of LDS by
//     ds_read_b64_tr_b16 (the wave writes its V tile row-major and each 16-lane
//     group reads 4 rows x 16 columns back transposed);
//   * the fused append stores this step's frame rows into their pages (query
//     group 0): a lane holds at most one frame column a pass (chunks of at
//     most 16 frames), loaded once and selected into the tile that holds it,
//     so every load and store is branch-free; the stores are the wave's last
//     instructions.
//   * STREAM (host-chosen when a step's windows outgrow the last-level
//     cache): page rows, appends and the output with the streaming cache
//     policy.
// Pages hold 64-byte column blocks ([page][block][page_size][32 elements]),
// so one k-step load of a 16-slot tile reads 16 rows x 64 bytes of one block:
// 1 KB of contiguous memory when the 16 slots share a page.
template <typename ST, int DK, int NT, int MODE, bool MULTI, bool STREAM, int NW>
__global__ void __launch_bounds__(64 * NW) relpos_attn_mfma_kernel(const AttnK<ST> p) {
  constexpr int SPLIT = DK / 64;
  static_assert(NW == 4 || NW == 2, "waves a workgroup");
  constexpr int SPW = NW / SPLIT;  // streams per workgroup
  constexpr int NTH = 64 * NW;
  constexpr int TQ = 2;
  constexpr int KS = 2;            // 16x16x32 k-steps over the wave's 64 columns
  constexpr int KT = 16 * NT;      // slots (window columns) per pass
  constexpr int CHR = DK / 8;                   // 16-byte chunks per staged position row
  // position-row tiles: slot s of query ii reads row s + TQ-1-ii.  A single
  // pass holds at most KT - 1 keys (the host takes the multi-pass form for
  // more), so its rows stay below KT, which at head_dim 128 are whole staging
  // instructions: one tile fewer to stage ahead of the K rows
  constexpr int NPT = (!MULTI && (16 * NT * CHR) % (64 * NW) == 0) ? NT : NT + 1;
  constexpr int PROWS = 16 * NPT;
  constexpr int PSTRIDE = CHR * 16;             // bytes per staged position row (unpadded)
  constexpr int RPB = 16 / CHR;                 // staged rows per 256 bytes (all 64 banks)
  constexpr int PCH = (PROWS * CHR + NTH - 1) / NTH;  // staged chunks per thread
  constexpr int VSTRIDE = 64 * 2 + 16;          // bytes per staged V row
  constexpr int SK = (KT + 63) / 64;            // slots per lane per query
  constexpr float NEG = -1e30f;
  constexpr float MASKED = -1e5f * 1.4426950408889634f;  // -1e5 in log2 units
  constexpr int mask_mode = MODE;  // 0 none, 1 mask bytes, 2 stream state
  constexpr int ES = 2;            // bytes per element
  constexpr int BLK = 64;          // bytes per page row in a column block
  typedef typename Mma<ST>::H H;

  // The staged position rows are dead once the dot products are in LDS (the
  // second barrier of a pass, when a stream's waves exchange their partial
  // dot products); there the P.V staging (V tiles and the 16-bit high and low
  // parts of the probabilities, [hi|lo][query][slot]) reuses their space.
  // With one wave a stream (head_dim 64) the waves of a workgroup share only
  // the position rows, so the P.V staging gets its own space and the waves go
  // on without that barrier.
  constexpr int POS_BYTES = PROWS * PSTRIDE;
  constexpr int PV_BYTES = NW * 16 * VSTRIDE + NW * 2 * TQ * KT * 2;
  constexpr bool PV_OWN = SPLIT == 1;
  constexpr int PV_OFF = PV_OWN ? POS_BYTES : 0;
  constexpr int STAGE_BYTES = PV_OWN ? POS_BYTES + PV_BYTES : (POS_BYTES > PV_BYTES ? POS_BYTES : PV_BYTES);
  __shared__ __attribute__((aligned(16))) uint8_t stage_lds[STAGE_BYTES];
  __shared__ float bd_lds[NW][TQ][PROWS];
  __shared__ float ac_lds[NW][TQ][KT];
  uint8_t* const pos_lds = stage_lds;
  uint8_t (*const v_lds)[16 * VSTRIDE] = reinterpret_cast<uint8_t (*)[16 * VSTRIDE]>(stage_lds + PV_OFF);
  uint16_t (*const p_lds)[2][TQ][KT] =
      reinterpret_cast<uint16_t (*)[2][TQ][KT]>(stage_lds + PV_OFF + NW * 16 * VSTRIDE);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q16 = lane & 15;
  const int kg = lane >> 4;
  const int sw = wave / SPLIT;  // stream slot in the workgroup
  const int hf = wave % SPLIT;  // 64-column part of the head
  const int w0 = sw * SPLIT;    // first wave of this stream
  const int sb = blockIdx.x;  // stream block
  const int h = blockIdx.y;
  const int i0 = blockIdx.z * TQ;
  const int nq = min(TQ, p.T - i0);
  const int b_raw = sb * SPW + sw;
  const int b = min(b_raw, p.B - 1);  // loads stay inside the batch arrays
  const int hcol = h * DK + hf * 64;       // first column of the wave
  // k-step ks of the wave's 64 columns covers columns ks*32 .. ks*32 + 31 (one
  // 64-byte page block); the lane holds 8 of them, ks*32 + kg*8 ..
  const int cbyte = (hcol + kg * 8) * ES;  // byte offset of the lane's k-step 0 columns in a row
  constexpr int KSB = 32 * ES;             // bytes between a lane's k-steps
  const int M = p.pg.max_pages;
  const bool paged = p.pg.rows != nullptr;
  const int nblk = p.pg.D >> 5;            // column blocks per page row
  // byte offset of the wave's k-step ks block in a page, added as soffset
  const int blk_soff = (hcol >> 5) << (p.pg.page_shift + 6);
  const int blk_step = 1 << (p.pg.page_shift + 6);

  // Every resource has a valid base and a non-zero row stride (the range check
  // that turns absent rows into zeros is index-based); a zero stride can only
  // come with a single row, where any stride addresses it.  The pool resources
  // address 64-byte block rows: index page*page_size*nblk + row, so a page row
  // index never reaches past the layer slab.  Without pages the pool resources
  // are never read or written.
  const int dmodel = p.H * DK;
  const int st_k = (int)(p.k_st > 0 ? p.k_st : dmodel) * ES;
  const int st_v = (int)(p.v_st > 0 ? p.v_st : dmodel) * ES;
  const int st_p = (int)(p.pos_sr > 0 ? p.pos_sr : dmodel) * ES;
  const uint32_t pool_rows = paged ? ((uint32_t)p.pg.num_pages << p.pg.page_shift) * (uint32_t)nblk : 0u;
  const __amdgpu_buffer_rsrc_t r_kp = rows_rsrc(paged ? (const void*)p.kp : (const void*)p.kn, BLK, pool_rows);
  const __amdgpu_buffer_rsrc_t r_vp = rows_rsrc(paged ? (const void*)p.vp : (const void*)p.vn, BLK, pool_rows);
  const __amdgpu_buffer_rsrc_t r_kn = rows_rsrc(p.kn + b * p.k_sb, st_k, (uint32_t)p.T);
  const __amdgpu_buffer_rsrc_t r_vn = rows_rsrc(p.vn + b * p.v_sb, st_v, (uint32_t)p.T);
  const __amdgpu_buffer_rsrc_t r_pos = rows_rsrc(p.pos, st_p, (uint32_t)p.pos_rows);

  // ---------------- prologue: every load independent of the page table,
  //                  issued branch-free (absent inputs read a valid stand-in
  //                  address and are replaced afterwards)
  // A operand source: row m = q16 is (q+u)_hi, (q+u)_lo, (q+v)_hi, (q+v)_lo of
  // query m & 1 for m < 8, zero above; element e of k-step ks is column
  // ks*32 + kg*8 + e of the wave's 64.  The wave needs 256 bytes of q (its 64
  // columns of two query rows) and 256 of the biases (u and v).
  //  * Q_GATHER (head_dim 128, or a streaming launch: the launches that queue
  //    on the CUs' load path):
  //    one dword a lane of each, lane l holding dword l & 31 of row l >> 5,
  //    loaded after the block table's ring entries (which the K rows'
  //    addresses need first) and gathered into the operand layout across lanes
  //    after the K rows are issued, while they are in flight.  Four 16-byte
  //    loads a lane read each byte eight times over, all queued ahead of the K
  //    rows on the CU.
  //  * otherwise (head_dim 64 below the streaming size, latency-bound
  //    launches, where the gather's LDS round trips cost more than the loads,
  //    8,430 against 8,313-8,377 steps/s at 64 streams): each lane loads its own 16-byte
  //    operand chunks first, ahead of the header, and the operand is built
  //    before the K rows are issued (after them it would hold the 16 registers
  //    of the raw rows through the K loads).
  constexpr bool Q_GATHER = DK == 128 || STREAM;
  const int a_ii = q16 & 1;
  const int a_kind = q16 >> 1;  // 0 u-hi, 1 u-lo, 2 v-hi, 3 v-lo, >= 4 zero
  u32x4 qraw[KS], braw[KS];
  if constexpr (!Q_GATHER) {
    const int ic = min(i0 + a_ii, p.T - 1);
    const ST* qrow = p.q + b * p.q_sb + (int64_t)ic * p.q_st + hcol + kg * 8;
    const ST* brow = (a_kind < 2 ? p.bu : p.bv) + hcol + kg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qraw[ks] = ld16(qrow + ks * 32);
      braw[ks] = ld16(brow + ks * 32);
    }
  }
  // (branch-free, so the row stride loads with the other kernel arguments
  // rather than in a second round trip before the header's address is known)
  const int64_t hdr_off = (int64_t)b * p.pg.rows_stride;
  const int32_t* hdr = paged ? p.pg.rows + hdr_off : reinterpret_cast<const int32_t*>(p.q);
  const int hdr_a = hdr[0];
  int ring_lane = hdr[paged ? 1 + min(lane, M - 1) : 0];
  uint32_t q_dw = 0u, b_dw = 0u;
  if constexpr (Q_GATHER) {
    const int rr = lane >> 5, cd = lane & 31;
    const int ic = min(i0 + rr, p.T - 1);
    q_dw = reinterpret_cast<const uint32_t*>(p.q + b * p.q_sb + (int64_t)ic * p.q_st + hcol)[cd];
    b_dw = reinterpret_cast<const uint32_t*>((rr ? p.bv : p.bu) + hcol)[cd];
  }
  const int64_t* stp = mask_mode == 2 ? p.st_proc + b : reinterpret_cast<const int64_t*>(p.q);
  const int64_t* stc = mask_mode == 2 ? p.st_cl + b : stp;
  const int64_t* stn = (mask_mode == 2 && p.st_len) ? p.st_len + b : stp;
  const int64_t st_pr_v = *stp, st_cl_v = *stc, st_n_v = *stn;
  const int32_t nact_v = p.nact ? *p.nact : p.B;
  // the last slot any query of the pass at jb reads, and the position-row
  // tiles it needs (slot s of query ii reads staged row s + TQ - 1 - ii)
  auto pass_tiles = [&](int jb) {
    const int s_max = min(KT, p.Lk - jb) - 1;
    return min(NPT, (s_max + TQ - 1) / 16 + 1);
  };
  // position rows (rows outside the table read zeros) and mask bytes of a pass
  // staged position rows: chunk c of row r sits at chunk c ^ pkey(r) of the
  // unpadded row, so the 16 rows an MFMA operand read takes (one chunk each)
  // fall on distinct banks
  auto pkey = [&](int row) { return (row / RPB) & (CHR - 1); };
  uint8_t mk[SK][TQ];
  auto load_pass_shared = [&](int jb) {
    // the position rows of the pass go straight to LDS (buffer loads to LDS:
    // no registers, so the K rows can be issued before they are in); each
    // wave's instruction c fills 64 consecutive chunks, lane = chunk, reading
    // the chunk that belongs at its swizzled place.  All PROWS rows, with
    // every lane active (no branch: the compiler then counts these loads
    // exactly when it places its waits); rows past the table read zeros.
    static_assert(PROWS * CHR % NTH == 0, "whole instructions");
    const int rb = jb + p.T - i0 - TQ;
#pragma unroll
    for (int c = 0; c < PCH; ++c) {
      const int base = c * NTH + wave * 64;  // wave-uniform
      const int idx = base + lane;
      const int row = idx / CHR, cc = (idx % CHR) ^ pkey(row);
      __builtin_amdgcn_struct_ptr_buffer_load_lds(r_pos, (__attribute__((address_space(3))) void*)(pos_lds + base * 16), 16,
                                                  rb + row, (h * DK + cc * 8) * ES, 0, 0, 0);
    }
    if (mask_mode == 1) {
#pragma unroll
      for (int r = 0; r < SK; ++r)
#pragma unroll
        for (int ii = 0; ii < TQ; ++ii) {
          const int ic = min(i0 + ii, p.T - 1);
          const int jc = min(jb + min(lane + 64 * r, KT - 1), p.Lk - 1);
          mk[r][ii] = p.mask[b * p.m_sb + h * p.m_sh + (int64_t)ic * p.m_st + jc];
        }
    }
  };
  load_pass_shared(0);
  __builtin_amdgcn_sched_barrier(0);  // all of the above in flight before any use

  // ---------------- live streams: a launch recorded once for a batch that
  //                  changes reads the live count from the device; workgroups
  //                  past it end here (workgroup-uniform, so no barrier is left
  //                  waiting)
  const int nact = min(__builtin_amdgcn_readfirstlane(nact_v), p.B);
  if (sb * SPW >= nact) return;
  const bool active = b_raw < nact;  // uniform per wave

  // ---------------- per-stream scalars
  const int A = paged ? __builtin_amdgcn_readfirstlane(hdr_a) : 0;
  if (!paged) ring_lane = -1;
  // ring entry of the first page that holds a window position
  const int win0 = A - p.left;
  const uint32_t lp0 = (uint32_t)max(win0, 0) >> p.pg.page_shift;
  const int r0 = paged ? (int)(lp0 % (uint32_t)M) : 0;
  const uint32_t pmask = (1u << p.pg.page_shift) - 1u;
  const uint32_t page_blk_rows = (uint32_t)nblk << p.pg.page_shift;  // block rows per page
  // block-row index of window column j (a frame position of the stream), kNoRow
  // if the stream holds none; every lane must be active (ds_bpermute)
  auto page_row = [&](int j) {
    const int pos = win0 + j;
    int ridx = r0 + (int)(((uint32_t)max(pos, 0) >> p.pg.page_shift) - lp0);
    ridx = ridx >= M ? ridx - M : ridx;
    const int page = __shfl(ring_lane, ridx);
    return (paged && pos >= 0 && page >= 0) ? (uint32_t)page * page_blk_rows + ((uint32_t)pos & pmask)
                                            : kNoRow;
  };
  StreamMask sm{};
  int qchunk[TQ];
  if (mask_mode == 2) {
    auto u64 = [](int64_t v) {
      const int lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)v);
      const int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
      return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
    };
    const int64_t n = p.st_len ? u64(st_n_v) : p.len_scalar;
    sm.set(u64(st_pr_v), u64(st_cl_v), n, p.left, p.chunk_size, p.left_chunks, p.c_magic);
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) qchunk[ii] = sm.query_chunk(i0 + ii);
  }

  // ---------------- A operand (high / low parts of the fp32 sums)
  u32x4 aop[KS];
  auto build_aop = [&]() {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (Q_GATHER) {
        // the lane's 8 columns ks*32 + kg*8 .. are dwords ks*16 + kg*4 .. + 3
        // of its query row (lanes 32 a_ii ..) and of its bias row (u: lanes
        // 0 .., v: lanes 32 ..); every lane is active here
        const int dw0 = ks * 16 + kg * 4;
        const int bsel = a_kind >= 2 ? 32 : 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qraw[ks][e] = (uint32_t)__builtin_amdgcn_ds_bpermute((a_ii * 32 + dw0 + e) * 4, (int)q_dw);
          braw[ks][e] = (uint32_t)__builtin_amdgcn_ds_bpermute((bsel + dw0 + e) * 4, (int)b_dw);
        }
      }
      float qf[8], bf[8], x[8];
      Tr<ST>::unpack(qraw[ks], qf);
      Tr<ST>::unpack(braw[ks], bf);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (a_ii < nq ? qf[e] : 0.f) + bf[e];
      aop[ks] = split16<ST, 8, u32x4>(x, a_kind & 1);
      if (a_kind >= 4) aop[ks] = u32x4{0u, 0u, 0u, 0u};
      asm volatile("" ::"v"(aop[ks]));  // built where it is called
    }
  };
  // otherwise built here, before the K rows are issued: q and the biases are
  // in by now (they were loaded ahead of the header's wait)
  if constexpr (!Q_GATHER) build_aop();

  f32x4_t oacc[4];  // P.V: D rows (hi q0, hi q1, lo q0, lo q1), 4 column tiles of 16
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) oacc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[TQ], l_run[TQ];
#pragma unroll
  for (int ii = 0; ii < TQ; ++ii) {
    m_run[ii] = NEG;
    l_run[ii] = 0.f;
  }
  uint8_t* vl = v_lds[wave];
  const bool do_append = p.append && blockIdx.z == 0 && active && paged;

  // MULTI: windows longer than one pass (the single-pass form is straight-line
  // code, with nothing carried around a loop)
  const int npass = MULTI ? p.tiles : 1;
  // The fused append stores this step's frame rows as the wave's last
  // instructions (the multi-pass form after each pass): scattered 128-byte
  // writes into the page blocks the launch streams its reads from cost 4% of
  // the launch at 230 streams more when issued mid-wave and cached.  The page
  // rows' loads, the appends and the output take the streaming cache policy
  // (nt) when the step's windows outgrow the last-level cache (STREAM, chosen
  // by the host), so they do not displace what the step reuses; below that
  // the windows stay cached from one step to the next.
  constexpr int kPagePolicy = STREAM ? 2 : 0;
  constexpr int kAppendPolicy = kPagePolicy;
  u32x4 app_rows[2 * KS];           // K then V frame rows of the single pass
  uint32_t app_row = kNoRow;
  for (int pass = 0; pass < npass; ++pass) {
    const int jb = pass * KT;
    const int npt = pass_tiles(jb);
    if (MULTI && pass > 0) load_pass_shared(jb);

    // ---- K and V rows, lane = slot 16*kt + q16 (window column jb + slot),
    //      columns ks*32 + kg*8 .. + 7 of the wave's 64.  Cached columns
    //      (j < left) load from the pages, this step's frames (left <= j < Lk,
    //      at most 16 of them) from the projection output.  With at most 16
    //      frames a lane holds at most one frame column in a pass, the one
    //      congruent to its slot mod 16: its frame row is a single load per
    //      k-step, selected in when its tile is consumed (the select reads it
    //      for every tile, so it is issued ahead of the page rows).  Every
    //      load is unconditional (absent rows read zeros), so the compiler
    //      counts them exactly when it places its waits: a load under a
    //      branch would have it wait for every outstanding load at the first
    //      use of any of them.
    uint32_t prow[NT];
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      const int j = jb + 16 * kt + q16;
      const uint32_t r = page_row(j);
      prow[kt] = j < p.left ? r : kNoRow;
    }
    const int fbase = max(p.left, jb);
    const int jf = fbase + ((jb + q16 - fbase) & 15);  // the lane's frame column
    const bool fvalid = jf < p.Lk && jf < jb + KT;
    const int ftile = fvalid ? (jf - jb) >> 4 : -1;  // tile that holds it
    const uint32_t frow = fvalid ? (uint32_t)(jf - p.left) : kNoRow;
    const uint32_t arow_f = page_row(jf);
    const uint32_t arow = fvalid && do_append ? arow_f : kNoRow;  // its append target
    // tile kt holds a frame of this step (workgroup-uniform)
    auto has_frames = [&](int kt) { return jb + 16 * kt + 15 >= p.left && jb + 16 * kt < p.Lk; };
    // the operand rows of tile kt: page rows, with the lane's frame row in
    // place of the (zero) page row where the tile holds it
    auto with_frame = [&](int kt, u32x4 v, u32x4 f) {
      if (has_frames(kt) && ftile == kt) v = f;
      return v;
    };
    u32x4 kr[NT][KS], vr[NT][KS], kf[KS], vf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = pk_buffer_load_x4(r_kn, frow, cbyte + ks * KSB, 0, 0);
#pragma unroll
    for (int kt = 0; kt < NT; ++kt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kr[kt][ks] = pk_buffer_load_x4(r_kp, prow[kt], kg * 16, blk_soff + ks * blk_step, kPagePolicy);
    // which scores of the pass take no value (a slot past the window or the
    // pass, a query past the chunk: bit r * TQ + ii of neg_bits) or the mask's
    // -1e5 term (the streaming rule: msk_bits), for slot lane + 64 r of query
    // ii: none of it waits for the K rows, so it is done while they are in flight
    static_assert(SK * TQ <= 32, "score bits");
    uint32_t neg_bits = 0u, msk_bits = 0u;
#pragma unroll
    for (int r = 0; r < SK; ++r) {
      const int sl = lane + 64 * r;
      const int j = jb + min(sl, KT - 1);
      const bool valid = sl < KT && j < p.Lk;
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        const uint32_t bit = 1u << (r * TQ + ii);
        if (!(valid && ii < nq)) neg_bits |= bit;
        if (mask_mode == 2 && sm.masked(i0 + ii, qchunk[ii], j)) msk_bits |= bit;
      }
    }
    asm volatile("" ::"v"(neg_bits), "v"(msk_bits));
    // Q_GATHER: the A operand is built once the first pass's K rows are
    // issued (waits are counted exactly, so this waits for q and the biases
    // only, not for the K rows)
    if (Q_GATHER && pass == 0) build_aop();
    // the wave's position-row loads (issued before any K row, and exactly
    // (NT + 1)*KS vector loads ago) are in LDS: wait for them, not for the K
    // rows, before the barrier that makes every wave's part visible
    static_assert((NT + 1) * KS <= 15, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0f70 | ((NT + 1) * KS));
    __syncthreads();  // position rows in LDS

    // ---- (q+v).pos over the wave's columns: D rows 4..7 (lanes 16..31)
#pragma unroll
    for (int pt = 0; pt < NPT; ++pt) {
      if (pt >= npt) break;
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
      const int prow_l = pt * 16 + q16;
      const uint8_t* src = pos_lds + prow_l * PSTRIDE;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int chunk = hf * 8 + ks * (KSB / 16) + kg;  // columns hf*64 + ks*32 + kg*8 ..
        d = Mma<ST>::k32(aop[ks], *reinterpret_cast<const u32x4*>(src + ((chunk ^ pkey(prow_l)) * 16)), d);
      }
      if (kg == 1) {
        bd_lds[wave][0][pt * 16 + q16] = d[0] + d[2];
        bd_lds[wave][1][pt * 16 + q16] = d[1] + d[3];
      }
    }
    // ---- (q+u).k over the wave's columns, D rows 0..3 (lanes 0..15), tile by
    //      tile.  Once a tile's K rows are consumed, the tile's V page rows are
    //      issued into the registers it frees: no more registers in flight
    //      than the K rows alone, and the V round trip overlaps the rest of the
    //      K phase, the scores and the softmax (the frames' V rows go first,
    //      ahead of tile 0's).  The frames' K rows go to their pages later
    //      (query group 0 only: the row index is valid only for the frames'
    //      lanes).
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) d = Mma<ST>::k32(aop[ks], with_frame(kt, kr[kt][ks], kf[ks]), d);
      if (kg == 0) {
        ac_lds[wave][0][16 * kt + q16] = d[0] + d[2];
        ac_lds[wave][1][16 * kt + q16] = d[1] + d[3];
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kt == 0) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) vf[ks] = pk_buffer_load_x4(r_vn, frow, cbyte + ks * KSB, 0, 0);
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        vr[kt][ks] = pk_buffer_load_x4(r_vp, prow[kt], kg * 16, blk_soff + ks * blk_step, kPagePolicy);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MULTI) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        pk_buffer_store_x4(kf[ks], r_kp, arow, kg * 16, blk_soff + ks * blk_step, kAppendPolicy);
    }
    if constexpr (PV_OWN)
      wave_lds_sync();  // the wave's own dot products in LDS
    else
      __syncthreads();  // partial dot products of the stream's waves in LDS

    // ---- scores: lane handles slots lane + 64*r; online softmax.  Every LDS
    //      read of the partial products is issued first, then selects (the
    //      conditions are the bits computed above), so no read waits behind a
    //      branch; the queries' reductions run side by side
    float acv[SK][TQ], bdv[SK][TQ];
#pragma unroll
    for (int r = 0; r < SK; ++r) {
      const int slc = min(lane + 64 * r, KT - 1);
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        // (q+v).pos row of column jb + slc for query i0 + ii, relative to the staged rows
        const int prw = min(slc + TQ - 1 - ii, PROWS - 1);
        float ac = 0.f, bd = 0.f;
#pragma unroll
        for (int x = 0; x < SPLIT; ++x) {
          ac += ac_lds[w0 + x][ii][slc];
          bd += bd_lds[w0 + x][ii][prw];
        }
        acv[r][ii] = ac;
        bdv[r][ii] = bd;
      }
    }
    float s[SK][TQ];
#pragma unroll
    for (int r = 0; r < SK; ++r)
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        const uint32_t bit = 1u << (r * TQ + ii);
        const bool msk = mask_mode == 1 ? mk[r][ii] != 0 : (msk_bits & bit) != 0u;
        const float sc = msk ? fmaf(acv[r][ii], p.scale, MASKED) : (acv[r][ii] + bdv[r][ii]) * p.scale;
        s[r][ii] = (neg_bits & bit) != 0u ? NEG : sc;
      }
    float corr[TQ], mnew[TQ], lsum[TQ];
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) {
      float tmax = NEG;
#pragma unroll
      for (int r = 0; r < SK; ++r) tmax = fmaxf(tmax, s[r][ii]);
      mnew[ii] = tmax;
    }
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) mnew[ii] = fmaxf(m_run[ii], wave_max(mnew[ii]));
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) {
      corr[ii] = __builtin_amdgcn_exp2f(m_run[ii] - mnew[ii]);
      m_run[ii] = mnew[ii];
      lsum[ii] = 0.f;
#pragma unroll
      for (int r = 0; r < SK; ++r) {
        const int sl = lane + 64 * r;
        const float e = s[r][ii] > 0.5f * NEG ? __builtin_amdgcn_exp2f(s[r][ii] - mnew[ii]) : 0.f;
        lsum[ii] += e;
        if (sl < KT) {  // e = hi + lo in the operand type, exact to ~2^-17
          const H hi = (H)e;
          const H lo = (H)(e - (float)hi);
          p_lds[wave][0][ii][sl] = __builtin_bit_cast(uint16_t, hi);
          p_lds[wave][1][ii][sl] = __builtin_bit_cast(uint16_t, lo);
        }
      }
    }
#pragma unroll
    for (int ii = 0; ii < TQ; ++ii) l_run[ii] = l_run[ii] * corr[ii] + wave_sum(lsum[ii]);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      oacc[nt][0] *= corr[0];
      oacc[nt][1] *= corr[1];
      oacc[nt][2] *= corr[0];
      oacc[nt][3] *= corr[1];
    }
    wave_lds_sync();


    // ---- P.V, 16 slots at a time: stage the V rows, read them back
    //      transposed; A row m = q16 & 3 holds the high (m < 2) or low part of
    //      query m & 1's probabilities, so D[q] + D[2 + q] is the product with
    //      p = hi + lo; rows 4..15 repeat rows 0..3 and feed only D rows that
    //      are never read
    const uint16_t* p_arow = &p_lds[wave][(q16 >> 1) & 1][q16 & 1][0];
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      uint8_t* vrow = vl + q16 * VSTRIDE + kg * 16;
      *reinterpret_cast<u32x4*>(vrow) = with_frame(kt, vr[kt][0], vf[0]);
      *reinterpret_cast<u32x4*>(vrow + KSB) = with_frame(kt, vr[kt][1], vf[1]);
      const i16x4_t pop = *reinterpret_cast<const i16x4_t*>(p_arow + 16 * kt + 4 * kg);
      wave_lds_sync();
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint8_t* src = vl + (4 * kg + (q16 >> 2)) * VSTRIDE + (nt * 16 + 4 * (q16 & 3)) * 2;
        const i16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)src);
        oacc[nt] = Mma<ST>::k16(pop, vt, oacc[nt]);
      }
      wave_lds_sync();  // the next 16 rows overwrite the staging rows
    }
    // ---- the frames' V rows to their pages
    if constexpr (MULTI) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        pk_buffer_store_x4(vf[ks], r_vp, arow, kg * 16, blk_soff + ks * blk_step, kAppendPolicy);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        app_rows[ks] = kf[ks];
        app_rows[KS + ks] = vf[ks];
      }
      app_row = arow;
    }
    if (MULTI) __syncthreads();  // the next pass restages pos_lds and rewrites bd / ac
  }

  // ---- write: lanes 0..15 hold column nt*16 + q16 of both queries; the wave's
  //      two 128-byte output rows go through its V staging rows so that 16
  //      lanes store them 16 bytes each
  if (active) {
    if (kg == 0) {
#pragma unroll
      for (int ii = 0; ii < TQ; ++ii) {
        const float inv = l_run[ii] > 0.f ? __builtin_amdgcn_rcpf(l_run[ii]) : 0.f;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          *reinterpret_cast<H*>(vl + ii * VSTRIDE + (nt * 16 + q16) * 2) = (H)((oacc[nt][ii] + oacc[nt][2 + ii]) * inv);
      }
    }
    wave_lds_sync();
    const int oi = lane >> 3;  // query of the lane's 16 bytes
    if (lane < 16 && oi < nq) {
      const u32x4 o = *reinterpret_cast<const u32x4*>(vl + oi * VSTRIDE + (lane & 7) * 16);
      u32x4* const dst =
          reinterpret_cast<u32x4*>(p.out + b * p.o_sb + (int64_t)(i0 + oi) * p.o_st + hcol + (lane & 7) * 8);
      if constexpr (STREAM)
        __builtin_nontemporal_store(o, dst);
      else
        *dst = o;
    }
  }
  // ---- the single pass's fused append (row kNoRow where there is nothing to store)
  if constexpr (!MULTI) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      pk_buffer_store_x4(app_rows[ks], r_kp, app_row, kg * 16, blk_soff + ks * blk_step, kAppendPolicy);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      pk_buffer_store_x4(app_rows[KS + ks], r_vp, app_row, kg * 16, blk_soff + ks * blk_step, kAppendPolicy);
  }
}

// s_waitcnt that waits until at most n vector memory operations of the wave are
// outstanding (vmcnt is 6 bits: [3:0] and [15:14]; expcnt and lgkmcnt left
// at their no-wait maxima)
#define PK_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0f70 | ((n) & 15) | (((n) & 0x30) << 10))

// DPP row_newbcast: every lane of a row of 16 reads lane `src` of its row
template <int SRC>
__device__ static inline float row_bcast(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + SRC, 0xF, 0xF, false));
}

// ---------------------------------------------------------------------------
// A whole chunk of queries (up to 14 frames a step, the large model's (70, 13)
// context, parakeet/config.py:29) over one pass of the window.
//
// Workgroup of 4 waves: 2 streams of head h, each stream's window split by key
// between 2 waves (wave kh takes window columns 48 kh .. 48 kh + 47), so every
// K and V row of the window is read from HBM once for all of the chunk's
// queries.  Each wave works on the whole head (head_dim columns).
//
// The matrix products are taken transposed, keys (or position rows) as the 16
// M rows and queries as the 16 N columns, with one 16-bit operand for all of
// them: row n < 14 of the query operand is q_n, row 14 is pos_bias_u, row 15 is
// pos_bias_v.  So
//   D = K_tile . Qop^T:    D[j][i] = q_i.k_j,   D[j][14] = u.k_j
//   D = Pos_tile . Qop^T:  D[m][i] = q_i.pos_m, D[m][15] = v.pos_m
// and (q_i + u).k_j = D[j][i] + D[j][14] exactly as the fp32 sum of products of
// the stored 16-bit values, without splitting q + u into high and low parts.
// The product's layout (lane = query column, registers = 4 consecutive keys) is
// the A operand layout of the 16x16x16 P.V product: the probabilities go from
// the softmax into P.V without a transpose.
//   * position rows (shared by the workgroup's streams; slot j of query i reads
//     row j + T - 1 - i) and this step's K frame rows go straight to LDS
//     (buffer loads to LDS: no registers held); each wave multiplies the 4
//     position tiles its keys read (rows 48 kh ..), adds v.pos with a row
//     broadcast and leaves them in its LDS strip (after a workgroup barrier:
//     the strips reuse the staging space), where the scores read them along
//     the relative-position diagonal;
//   * K rows as the A operand, from the pages (64-byte column blocks, one
//     k-step of a tile is 16 rows x 64 bytes of one block, absent rows read
//     zeros through the buffer range check) or, for this step's frames, from
//     the staged frame rows; the V rows of a tile are issued into the
//     registers its K rows free, with the lane's V frame row (one at most);
//   * a softmax over the wave's keys (max and sum over the 4 lanes of a query
//     column with two cross-row shuffles), probabilities split into high and
//     low 16-bit parts, P.V on 16x16x16 MFMAs with V read back transposed from
//     LDS (ds_read_b64_tr_b16), in two halves of the head's columns so the
//     first half's V registers are free before the second's accumulators;
//   * the two key halves meet in LDS once, flash-style: each wave's max and
//     sum per query, and the column half the other wave writes out;
//   * the fused append stores the frame rows into their pages (K after the K
//     products, V after P.V).
// 4 waves a SIMD: at most 128 registers a lane and 40 KB of LDS a workgroup.
template <typename ST, int DK, int MODE, bool STREAM>
__global__ void __launch_bounds__(256, 4) relpos_attn_chunk_kernel(const AttnK<ST> p) {
  constexpr int NW = 4;
  constexpr int NTH = 64 * NW;
  constexpr int KS = DK / 32;       // 16x16x32 k-steps over the head
  constexpr int KSH = KS / 2;       // k-steps (64-byte column blocks) per column half
  constexpr int NTW = 3;            // key tiles of 16 per wave
  constexpr int KW = 16 * NTW;      // window columns per wave
  constexpr int NPW = NTW + 1;      // position-row tiles per wave (rows KW*kh .. + 16*NPW - 1)
  constexpr int CHR = DK / 8;       // 16-byte chunks per row
  constexpr int RPB = 16 / CHR;     // staged rows per 256 bytes (all 64 banks)
  constexpr int RSTRIDE = DK * 2;   // bytes per staged row (unpadded, swizzled)
  constexpr int PROWS_MIN = KW + 16 * NPW;  // rows the second wave's tiles reach
  constexpr int PROWS = ((PROWS_MIN * CHR + NTH - 1) / NTH) * NTH / CHR;  // whole staging instructions
  constexpr int PCH = PROWS * CHR / NTH;
  constexpr int FCH = CHR / 8;      // frame staging instructions per wave (16 rows of its stream, 2 waves)
  constexpr int BDS = 20;           // floats per LDS row of a wave's position products (bank-conflict free)
  constexpr int BD_BYTES = 16 * NPW * BDS * 4;
  constexpr int HC = DK / 2;        // columns per half
  constexpr int VSTRIDE = HC * 2 + 16;  // bytes per staged V row (one column half)
  constexpr int WAVE_BYTES = BD_BYTES + 16 * VSTRIDE;
  constexpr int NOH = HC / 16;      // P.V output column tiles per half
  constexpr float NEG = -1e30f;
  constexpr float MASKED = -1e5f * 1.4426950408889634f;  // -1e5 in log2 units
  constexpr int ES = 2;
  constexpr int BLK = 64;
  constexpr int kPolicy = STREAM ? 2 : 0;
  static_assert(PROWS * CHR % NTH == 0 && PROWS >= PROWS_MIN, "whole staging instructions");
  static_assert(NOH * 4 * 64 * 4 <= BD_BYTES, "output exchange fits the position strip");
  static_assert(16 * HC * 2 <= 16 * VSTRIDE, "output staging fits the V strip");
  static_assert(FCH >= 1 && 16 * CHR == 2 * 64 * FCH, "a stream's 16 frame rows in 2 waves x FCH instructions");
  typedef typename Mma<ST>::H H;

  constexpr int POS_BYTES = PROWS * RSTRIDE;
  constexpr int STAGE_BYTES = POS_BYTES > NW * WAVE_BYTES ? POS_BYTES : NW * WAVE_BYTES;
  constexpr int KFR_BYTES = 16 * RSTRIDE;  // a stream's frame rows 0..15 (rows >= T read zeros)
  __shared__ __attribute__((aligned(16))) uint8_t stage_lds[STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t kfr_lds[2 * KFR_BYTES];
  __shared__ float ml_lds[NW][2][16];
  uint8_t* const pos_lds = stage_lds;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int q16 = lane & 15;
  const int kg = lane >> 4;
  const int sw = wave >> 1;  // stream slot in the workgroup
  const int kh = wave & 1;   // key half
  const int h = blockIdx.y;
  const int b_raw = blockIdx.x * 2 + sw;
  const int b = min(b_raw, p.B - 1);  // loads stay inside the batch arrays
  const int hcol = h * DK;
  const int jlo = KW * kh;            // first window column of the wave
  const int M = p.pg.max_pages;
  const bool paged = p.pg.rows != nullptr;
  const int nblk = p.pg.D >> 5;
  const int blk_soff = (hcol >> 5) << (p.pg.page_shift + 6);  // the head's first column block in a page
  const int blk_step = 1 << (p.pg.page_shift + 6);
  float* const bdl = reinterpret_cast<float*>(stage_lds + wave * WAVE_BYTES);
  uint8_t* const vst = stage_lds + wave * WAVE_BYTES + BD_BYTES;
  uint8_t* const kfr = kfr_lds + sw * KFR_BYTES;

  const int dmodel = p.H * DK;
  const int st_q = (int)(p.q_st > 0 ? p.q_st : dmodel) * ES;
  const int st_k = (int)(p.k_st > 0 ? p.k_st : dmodel) * ES;
  const int st_v = (int)(p.v_st > 0 ? p.v_st : dmodel) * ES;
  const int st_p = (int)(p.pos_sr > 0 ? p.pos_sr : dmodel) * ES;
  const uint32_t pool_rows = paged ? ((uint32_t)p.pg.num_pages << p.pg.page_shift) * (uint32_t)nblk : 0u;
  const __amdgpu_buffer_rsrc_t r_kp = rows_rsrc(paged ? (const void*)p.kp : (const void*)p.kn, BLK, pool_rows);
  const __amdgpu_buffer_rsrc_t r_vp = rows_rsrc(paged ? (const void*)p.vp : (const void*)p.vn, BLK, pool_rows);
  const __amdgpu_buffer_rsrc_t r_kn = rows_rsrc(p.kn + b * p.k_sb, st_k, (uint32_t)p.T);
  const __amdgpu_buffer_rsrc_t r_vn = rows_rsrc(p.vn + b * p.v_sb, st_v, (uint32_t)p.T);
  const __amdgpu_buffer_rsrc_t r_q = rows_rsrc(p.q + b * p.q_sb, st_q, (uint32_t)min(p.T, 14));
  // the position rows any score reads: 0 .. window + chunk - 2 (the staging's
  // rows past them read zeros without a memory request)
  const __amdgpu_buffer_rsrc_t r_pos = rows_rsrc(p.pos, st_p, (uint32_t)min(p.pos_rows, p.Lk + p.T - 1));

  // ---------------- prologue: every load independent of the page table
  // query operand: lane (kg, q16) holds row q16's columns ks*32 + kg*8 .. + 7
  // (rows of queries past the chunk read zeros)
  u32x4 qraw[KS], braw[KS];
  {
    const uint32_t qrow = q16 < 14 ? (uint32_t)q16 : kNoRow;
    const ST* brow = (q16 == 15 ? p.bv : p.bu) + hcol + kg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qraw[ks] = pk_buffer_load_x4(r_q, qrow, (hcol + ks * 32 + kg * 8) * ES, 0, 0);
      braw[ks] = ld16(brow + ks * 32);
    }
  }
  const int64_t hdr_off = (int64_t)b * p.pg.rows_stride;
  const int32_t* hdr = paged ? p.pg.rows + hdr_off : reinterpret_cast<const int32_t*>(p.q);
  const int hdr_a = hdr[0];
  int ring_lane = hdr[paged ? 1 + min(lane, M - 1) : 0];
  const int64_t* stp = MODE == 2 ? p.st_proc + b : reinterpret_cast<const int64_t*>(p.q);
  const int64_t* stc = MODE == 2 ? p.st_cl + b : stp;
  const int64_t* stn = (MODE == 2 && p.st_len) ? p.st_len + b : stp;
  const int64_t st_pr_v = *stp, st_cl_v = *stc, st_n_v = *stn;
  const int32_t nact_v = p.nact ? *p.nact : p.B;
  // mask bytes of the lane's scores: query q16, window columns jlo + 16 kt + 4 kg + r
  uint8_t mk[NTW][4];
  if constexpr (MODE == 1) {
    const int ic = min(q16, p.T - 1);
#pragma unroll
    for (int kt = 0; kt < NTW; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int jc = min(jlo + 16 * kt + 4 * kg + r, p.Lk - 1);
        mk[kt][r] = p.mask[b * p.m_sb + h * p.m_sh + (int64_t)ic * p.m_st + jc];
      }
  }
  // position rows 0 .. PROWS - 1 and the stream's K frame rows 0 .. 15 straight
  // to LDS; chunk c of row r sits at chunk c ^ pkey(r), so the 16 rows of an
  // operand read fall on distinct banks
  auto pkey = [&](int row) { return (row / RPB) & (CHR - 1); };
#pragma unroll
  for (int c = 0; c < PCH; ++c) {
    const int base = c * NTH + wave * 64;  // wave-uniform
    const int idx = base + lane;
    const int row = idx / CHR, cc = (idx % CHR) ^ pkey(row);
    __builtin_amdgcn_struct_ptr_buffer_load_lds(r_pos, (__attribute__((address_space(3))) void*)(pos_lds + base * 16), 16,
                                                row, (hcol + cc * 8) * ES, 0, 0, 0);
  }
#pragma unroll
  for (int c = 0; c < FCH; ++c) {
    const int base = (kh * FCH + c) * 64;  // wave-uniform chunk of the stream's frame rows
    const int idx = base + lane;
    const int row = idx / CHR, cc = (idx % CHR) ^ pkey(row);
    __builtin_amdgcn_struct_ptr_buffer_load_lds(r_kn, (__attribute__((address_space(3))) void*)(kfr + base * 16), 16,
                                                row, (hcol + cc * 8) * ES, 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);  // all of the above in flight before any use

  // ---------------- live streams (workgroup-uniform exit; the staging into
  //                  LDS completes before the workgroup leaves)
  const int nact = min(__builtin_amdgcn_readfirstlane(nact_v), p.B);
  if (blockIdx.x * 2 >= nact) {
    PK_WAIT_VMCNT(0);
    return;
  }
  const bool active = b_raw < nact;  // uniform per wave

  // query operand: q rows, u (row 14), v (row 15) as loaded (they were issued
  // ahead of the block-table ring, which the page rows wait for anyway)
  u32x4 qop[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qop[ks] = q16 < 14 ? qraw[ks] : braw[ks];
  asm volatile("" ::"v"(qop[0]));  // selected here, not where first used

  // ---------------- per-stream scalars and the lane's page rows
  const int A = paged ? __builtin_amdgcn_readfirstlane(hdr_a) : 0;
  if (!paged) ring_lane = -1;
  const int win0 = A - p.left;
  const uint32_t lp0 = (uint32_t)max(win0, 0) >> p.pg.page_shift;
  const int r0 = paged ? (int)(lp0 % (uint32_t)M) : 0;
  const uint32_t pmask = (1u << p.pg.page_shift) - 1u;
  const uint32_t page_blk_rows = (uint32_t)nblk << p.pg.page_shift;
  auto page_row = [&](int j) {  // every lane active (ds_bpermute)
    const int pos = win0 + j;
    int ridx = r0 + (int)(((uint32_t)max(pos, 0) >> p.pg.page_shift) - lp0);
    ridx = ridx >= M ? ridx - M : ridx;
    const int page = __shfl(ring_lane, ridx);
    return (paged && pos >= 0 && page >= 0) ? (uint32_t)page * page_blk_rows + ((uint32_t)pos & pmask) : kNoRow;
  };
  uint32_t prow[NTW];
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt) {
    const int j = jlo + 16 * kt + q16;
    const uint32_t r = page_row(j);
    prow[kt] = j < p.left ? r : kNoRow;
  }
  // the lane's frame column in the wave's range (the one congruent to its slot
  // mod 16: chunks of at most 14 frames hold one), its tile and its page row
  const bool do_append = p.append && active && paged;
  const int fbase = max(p.left, jlo);
  const int jf = fbase + ((jlo + q16 - fbase) & 15);
  const bool fvalid = jf < p.Lk && jf < jlo + KW;
  const int ftile = fvalid ? (jf - jlo) >> 4 : -1;
  const int ft = fvalid ? jf - p.left : 0;  // its frame (row of the staged frames)
  const uint32_t frow = fvalid ? (uint32_t)ft : kNoRow;
  const uint32_t arow_f = page_row(jf);
  const uint32_t arow = fvalid && do_append ? arow_f : kNoRow;
  auto has_frames = [&](int kt) { return jlo + 16 * kt + 15 >= p.left && jlo + 16 * kt < p.Lk; };
  // the lane's staged K frame row, 16 bytes of k-step ks
  auto kframe = [&](int ks) {
    return *reinterpret_cast<const u32x4*>(kfr + ft * RSTRIDE + (((ks * 4 + kg) ^ pkey(ft)) * 16));
  };

  // ---------------- K rows
  u32x4 kr[NTW][KS], vr[NTW][KS], vf[KS];
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kr[kt][ks] = pk_buffer_load_x4(r_kp, prow[kt], kg * 16, blk_soff + ks * blk_step, kPolicy);
  __builtin_amdgcn_sched_barrier(0);  // exactly NTW * KS loads after the staging

  // score conditions while the K rows are in flight: bit kt*4 + r for window
  // column jlo + 16 kt + 4 kg + r of query q16 (no value: past the window or
  // the chunk; the mask's -1e5 term: the streaming rule)
  StreamMask sm{};
  uint32_t neg_bits = 0u, msk_bits = 0u;
  if (MODE == 2) {
    auto u64 = [](int64_t v) {
      const int lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)v);
      const int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
      return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
    };
    const int64_t n = p.st_len ? u64(st_n_v) : p.len_scalar;
    sm.set(u64(st_pr_v), u64(st_cl_v), n, p.left, p.chunk_size, p.left_chunks, p.c_magic);
  }
  const int qchunk = MODE == 2 ? sm.query_chunk(q16) : 0;
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = jlo + 16 * kt + 4 * kg + r;
      const uint32_t bit = 1u << (kt * 4 + r);
      if (!(j < p.Lk && q16 < p.T)) neg_bits |= bit;
      if (MODE == 2 && sm.masked(q16, qchunk, j)) msk_bits |= bit;
      if (MODE == 1 && mk[kt][r] != 0) msk_bits |= bit;
    }
  // one register each from here on (not their partial products)
  asm volatile("" : "+v"(neg_bits), "+v"(msk_bits));

  // the position rows and frame rows (issued before every K row) are in LDS
  PK_WAIT_VMCNT(NTW * KS);
  __syncthreads();

  // ---- (q + v).pos: D[m][i] = q_i.pos_m, + v.pos_m from column 15
  f32x4_t bdd[NPW];
#pragma unroll
  for (int pt = 0; pt < NPW; ++pt) {
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
    const int prw = jlo + 16 * pt + q16;
    const uint8_t* src = pos_lds + prw * RSTRIDE;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int chunk = ks * 4 + kg;
      d = Mma<ST>::k32(*reinterpret_cast<const u32x4*>(src + ((chunk ^ pkey(prw)) * 16)), qop[ks], d);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) d[r] += row_bcast<15>(d[r]);
    bdd[pt] = d;
  }
  __syncthreads();  // every wave is done with the staged rows: the strips reuse them
#pragma unroll
  for (int pt = 0; pt < NPW; ++pt)
#pragma unroll
    for (int r = 0; r < 4; ++r) bdl[(16 * pt + 4 * kg + r) * BDS + q16] = bdd[pt][r];

  // ---- (q + u).k: D[j][i] = q_i.k_j, + u.k_j from column 14; the frame rows
  //      (staged) in place of the page rows (zeros) where the tile holds
  //      them; the V rows of a tile go into the registers its K rows free
  f32x4_t acd[NTW];
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt) {
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
    if (has_frames(kt)) {  // wave-uniform
      const bool mine = ftile == kt;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 f = kframe(ks);
        d = Mma<ST>::k32(mine ? f : kr[kt][ks], qop[ks], d);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) d = Mma<ST>::k32(kr[kt][ks], qop[ks], d);
    }
    acd[kt] = d;
    __builtin_amdgcn_sched_barrier(0);
    if (kt == 0) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) vf[ks] = pk_buffer_load_x4(r_vn, frow, (hcol + ks * 32 + kg * 8) * ES, 0, 0);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      vr[kt][ks] = pk_buffer_load_x4(r_vp, prow[kt], kg * 16, blk_soff + ks * blk_step, kPolicy);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the frames' K rows to their pages (row kNoRow where the lane holds no frame)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) pk_buffer_store_x4(kframe(ks), r_kp, arow, kg * 16, blk_soff + ks * blk_step, kPolicy);
  wave_lds_sync();  // the wave's position products in its strip

  // ---- scores (window column j = jlo + 16 kt + 4 kg + r, query i = q16): the
  //      position term of row j + T - 1 - i, local row 16 kt + 4 kg + r + T - 1 - i
  float s[NTW][4];
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ml = min(max(16 * kt + 4 * kg + r + p.T - 1 - q16, 0), 16 * NPW - 1);
      const float bd = bdl[ml * BDS + q16];
      const float ac = acd[kt][r] + row_bcast<14>(acd[kt][r]);
      const uint32_t bit = 1u << (kt * 4 + r);
      const float sc = (msk_bits & bit) ? fmaf(ac, p.scale, MASKED) : (ac + bd) * p.scale;
      s[kt][r] = (neg_bits & bit) ? NEG : sc;
    }
  // softmax over the wave's keys: a query's scores sit in the 4 lanes q16 + 16 kg
  float mx = NEG;
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kt][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float lsum = 0.f;
  i16x4_t phi[NTW], plo[NTW];
#pragma unroll
  for (int kt = 0; kt < NTW; ++kt) {
    H hv[4], lv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = s[kt][r] > 0.5f * NEG ? __builtin_amdgcn_exp2f(s[kt][r] - mx) : 0.f;
      lsum += e;
      hv[r] = (H)e;
      lv[r] = (H)(e - (float)hv[r]);
    }
    phi[kt] = i16x4_t{__builtin_bit_cast(short, hv[0]), __builtin_bit_cast(short, hv[1]),
                      __builtin_bit_cast(short, hv[2]), __builtin_bit_cast(short, hv[3])};
    plo[kt] = i16x4_t{__builtin_bit_cast(short, lv[0]), __builtin_bit_cast(short, lv[1]),
                      __builtin_bit_cast(short, lv[2]), __builtin_bit_cast(short, lv[3])};
  }
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  if (kg == 0) {
    ml_lds[wave][0][q16] = mx;
    ml_lds[wave][1][q16] = lsum;
  }

  // ---- P.V in two column halves: D[i][c] over 16 keys a tile, V staged
  //      row-major (the half's columns) and read back transposed; p = hi + lo.
  //      Wave kh writes column half kh out; it leaves the other half's
  //      partial sums for the other wave in its (dead) position strip.
  float* const xo_own = bdl;
  f32x4_t keep[NOH];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    f32x4_t oacc[NOH];
#pragma unroll
    for (int n = 0; n < NOH; ++n) oacc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < NTW; ++kt) {
      uint8_t* vrow = vst + q16 * VSTRIDE + kg * 16;
      const bool mine = has_frames(kt) && ftile == kt;
#pragma unroll
      for (int x = 0; x < KSH; ++x) {
        const int ks = half * KSH + x;
        *reinterpret_cast<u32x4*>(vrow + x * 64) = mine ? vf[ks] : vr[kt][ks];
      }
      wave_lds_sync();
#pragma unroll
      for (int n = 0; n < NOH; ++n) {
        const uint8_t* src = vst + (4 * kg + (q16 >> 2)) * VSTRIDE + (n * 16 + 4 * (q16 & 3)) * 2;
        const i16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)src);
        oacc[n] = Mma<ST>::k16(phi[kt], vt, oacc[n]);
        oacc[n] = Mma<ST>::k16(plo[kt], vt, oacc[n]);
      }
      wave_lds_sync();  // the next tile overwrites the staging rows
    }
    if (half == kh) {  // wave-uniform
#pragma unroll
      for (int n = 0; n < NOH; ++n) keep[n] = oacc[n];
    } else {
#pragma unroll
      for (int n = 0; n < NOH; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) xo_own[(n * 4 + r) * 64 + lane] = oacc[n][r];
    }
  }
  // the frames' V rows to their pages
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) pk_buffer_store_x4(vf[ks], r_vp, arow, kg * 16, blk_soff + ks * blk_step, kPolicy);
  __syncthreads();

  // ---- the key halves meet: lane (kg, q16) holds output rows (queries)
  //      4 kg + r, column 16 n + q16 of the wave's half
  const float* const xo_other = reinterpret_cast<const float*>(stage_lds + (wave ^ 1) * WAVE_BYTES);
  H* const ost = reinterpret_cast<H*>(vst);  // [16 queries][HC columns]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int qi = 4 * kg + r;
    const float m0 = ml_lds[wave][0][qi], l0 = ml_lds[wave][1][qi];
    const float m1 = ml_lds[wave ^ 1][0][qi], l1 = ml_lds[wave ^ 1][1][qi];
    const float mm = fmaxf(m0, m1);
    const float c0 = __builtin_amdgcn_exp2f(m0 - mm), c1 = __builtin_amdgcn_exp2f(m1 - mm);
    const float den = c0 * l0 + c1 * l1;
    const float inv = den > 0.f ? __builtin_amdgcn_rcpf(den) : 0.f;
#pragma unroll
    for (int n = 0; n < NOH; ++n) {
      const float o = (c0 * keep[n][r] + c1 * xo_other[(n * 4 + r) * 64 + lane]) * inv;
      ost[qi * HC + n * 16 + q16] = (H)o;
    }
  }
  wave_lds_sync();
  if (active) {
    constexpr int CPR = HC * 2 / 16;  // 16-byte chunks per output half-row
#pragma unroll
    for (int c = 0; c < DK / 64; ++c) {
      const int idx = c * 64 + lane;
      const int qi = idx / CPR, ch = idx % CPR;
      if (qi < p.T) {
        const u32x4 o = *reinterpret_cast<const u32x4*>(vst + qi * (HC * 2) + ch * 16);
        u32x4* const dst = reinterpret_cast<u32x4*>(p.out + b * p.o_sb + (int64_t)qi * p.o_st + hcol + kh * HC + ch * 8);
        if constexpr (STREAM)
          __builtin_nontemporal_store(o, dst);
        else
          *dst = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// read probe: one pass over a buffer, the read ceiling of a launch of its size

__global__ void __launch_bounds__(256) read_probe_kernel(const u32x4* src, int64_t n16, u32x4* out) {
  constexpr int U = 8;  // loads in flight per lane
  u32x4 acc = {0u, 0u, 0u, 0u};
  // workgroup w reads blocks of 32 KB: w, w + grid, ...; within a block, load u
  // of the workgroup reads 4 KB at u * 4 KB (lane = 16 bytes).  Of the forms
  // measured for one launch of 72 MB to 1 GB (grid-stride or blocked, 4 to 16
  // loads a lane, cached or streaming, 512 to 16,384 workgroups) this one, at 8
  // workgroups a CU, read fastest at every size.
  for (int64_t blk = blockIdx.x; blk * (256 * U) < n16; blk += gridDim.x) {
    const int64_t base = blk * (256 * U) + threadIdx.x;
    if (base + (U - 1) * 256 < n16) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + base + u * 256);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u];
    } else {
      for (int u = 0; u < U; ++u)
        if (base + u * 256 < n16) acc ^= __builtin_nontemporal_load(src + base + u * 256);
    }
  }
  // XOR over the wave, lane 0 writes the wave's 16 bytes
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    acc.x ^= (uint32_t)__shfl_xor((int)acc.x, off);
    acc.y ^= (uint32_t)__shfl_xor((int)acc.y, off);
    acc.z ^= (uint32_t)__shfl_xor((int)acc.z, off);
    acc.w ^= (uint32_t)__shfl_xor((int)acc.w, off);
  }
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
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
    const int64_t e = off + page_col(p.pg, c * VEC);
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
        kv = ld16(p.kp + off + page_col(p.pg, c * VEC));
        vv = ld16(p.vp + off + page_col(p.pg, c * VEC));
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

int elem_size(int dtype) {
  switch (dtype) {
    case PK_DTYPE_F32: return 4;
    case PK_DTYPE_F16: return 2;
    case PK_DTYPE_BF16: return 2;
    default: return 0;
  }
}

int log2_exact(int x) {
  int s = 0;
  while ((1 << s) < x) ++s;
  return (1 << s) == x ? s : -1;
}

// Validates the paged layout for `batch` rows; fills the device view.
int pages_view(const pk_paged_layout& L, int layer, int vec, int elem_bytes, const char* what,
               PagesK* out) {
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
  int cb = 64 / elem_bytes;  // column block: gcd(d_model, 64 bytes of elements)
  while (L.d_model % cb != 0) cb >>= 1;
  if ((int64_t)L.num_pages * L.page_size * (L.d_model / cb) >= (1LL << 32))
    return fail(PK_ERR_INVALID, "%s: a layer slab of %d pages exceeds 2^32 block rows", what,
                L.num_pages);
  out->rows = L.rows;
  out->rows_stride = L.rows_stride;
  out->max_pages = L.max_pages;
  out->page_shift = ps;
  out->num_pages = L.num_pages;
  out->page_elems = (int64_t)L.page_size * L.d_model;
  out->D = L.d_model;
  out->cb_shift = log2_exact(cb);
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

template <typename ST, int DK, int TQ, int NR, int WAVES>
int launch_attn_t(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  dim3 grid((unsigned)(a->batch * a->num_heads), (unsigned)((a->chunk + TQ - 1) / TQ));
  dim3 block(64u * WAVES);
  if (a->start_event || a->stop_event) {
    hipExtLaunchKernelGGL(relpos_attn_kernel<ST, DK, TQ, NR, WAVES>, grid, block, 0u, s,
                          (hipEvent_t)a->start_event, (hipEvent_t)a->stop_event, 0u, k);
  } else {
    hipLaunchKernelGGL((relpos_attn_kernel<ST, DK, TQ, NR, WAVES>), grid, block, 0, s, k);
  }
  return check_launch("pk_paged_relpos_attn");
}

// Rows per lane a kernel is built for.
constexpr int kRowsPerLane[5] = {4, 5, 9, 12, 18};
// Waves a workgroup of the fp32 kernel when the window is split (small grids)
constexpr int kSplitWaves = 4;

template <typename ST, int DK, int TQ, int NR>
int launch_attn_w(const pk_attn_args* a, const AttnK<ST>& k, int waves, hipStream_t s) {
  if constexpr (std::is_same<ST, float>::value) {
    if (waves == kSplitWaves) return launch_attn_t<ST, DK, TQ, NR, kSplitWaves>(a, k, s);
  }
  if (waves != 1) return fail(PK_ERR_UNSUPPORTED, "pk_paged_relpos_attn: %d waves a workgroup not built", waves);
  return launch_attn_t<ST, DK, TQ, NR, 1>(a, k, s);
}

template <typename ST, int DK, int TQ>
int launch_attn_nr(const pk_attn_args* a, const AttnK<ST>& k, int NR, int waves, hipStream_t s) {
  switch (NR) {
    case 4: return launch_attn_w<ST, DK, TQ, 4>(a, k, waves, s);
    case 5: return launch_attn_w<ST, DK, TQ, 5>(a, k, waves, s);
    case 9: return launch_attn_w<ST, DK, TQ, 9>(a, k, waves, s);
    case 12: return launch_attn_w<ST, DK, TQ, 12>(a, k, waves, s);
    case 18: return launch_attn_w<ST, DK, TQ, 18>(a, k, waves, s);
    default: return fail(PK_ERR_UNSUPPORTED, "pk_paged_relpos_attn: rows_per_lane %d not built", NR);
  }
}

template <typename ST, int DK>
int launch_attn_tq(const pk_attn_args* a, const AttnK<ST>& k, int TQ, int NR, int waves, hipStream_t s) {
  switch (TQ) {
    case 1: return launch_attn_nr<ST, DK, 1>(a, k, NR, waves, s);
    case 2: return launch_attn_nr<ST, DK, 2>(a, k, NR, waves, s);
    default: return fail(PK_ERR_UNSUPPORTED, "pk_paged_relpos_attn: query group %d not built", TQ);
  }
}

// Queries per workgroup: one chunk frame alone, otherwise groups of two.
int pick_tq(int T) { return T <= 1 ? 1 : 2; }

// Rows per lane NR for a window of Lk keys with rlw rows per wave load and
// `waves` waves sharing the tiles: the fewest tiles a wave, then the fewest
// rows a lane, then the least padding (one wave: the fewest tiles, then the
// least padding; hint > 0 forces NR).
void pick_tiling(int Lk, int rlw, int hint, int waves, int* NR, int* tiles) {
  int best_nr = 0, best_t = 0;
  long best_score = -1;
  for (int c : kRowsPerLane) {
    if (hint > 0 && c != hint) continue;
    const int per_tile = rlw * c;
    const int t = (Lk + per_tile - 1) / per_tile;
    const int waste = t * per_tile - Lk;
    const long rounds = (t + waves - 1) / waves;
    const long score = waves == 1 ? (long)t * 1000000L + waste : (rounds * 1000L + c) * 1000000L + waste;
    if (best_score < 0 || score < best_score) {
      best_score = score;
      best_nr = c;
      best_t = t;
    }
  }
  *NR = best_nr;
  *tiles = best_t;
}

// Matrix-core path (fp16 / bf16): workgroups of NW waves = NW / (head_dim /
// 64) streams x one head x one pair of queries, key tiles of 16 * kMfmaTiles
// rows.
constexpr int kMfmaTiles = 5;

template <typename ST, int DK, int MODE, bool MULTI, bool STREAM, int NW>
int launch_attn_mfma_t(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  constexpr int SPW = NW / (DK / 64);  // streams per workgroup
  dim3 grid((unsigned)((a->batch + SPW - 1) / SPW), (unsigned)a->num_heads,
            (unsigned)((a->chunk + 1) / 2));
  dim3 block(64u * NW);
  if (a->start_event || a->stop_event) {
    hipExtLaunchKernelGGL(relpos_attn_mfma_kernel<ST, DK, kMfmaTiles, MODE, MULTI, STREAM, NW>, grid, block,
                          0u, s, (hipEvent_t)a->start_event, (hipEvent_t)a->stop_event, 0u, k);
  } else {
    hipLaunchKernelGGL((relpos_attn_mfma_kernel<ST, DK, kMfmaTiles, MODE, MULTI, STREAM, NW>), grid, block, 0,
                       s, k);
  }
  return check_launch("pk_paged_relpos_attn");
}

// 2-wave workgroups (half the streams a workgroup, twice the workgroups) when
// the 4-wave grid has fewer workgroups than the chip has CUs: at 64 streams of
// the small model (128 workgroups of 4 waves) 6.3-6.5 -> 5.9-6.0 us a launch;
// with a CU's worth or more they are slower (230 streams of the large model:
// 13.6-14.1 -> 14.7-15.0 us), and small grids never take the streaming policy
template <typename ST, int DK, int MODE, bool MULTI, bool STREAM>
int launch_attn_mfma_nw(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  if constexpr (!STREAM) {
    const int64_t wgs4 = (int64_t)((a->batch + 4 / (DK / 64) - 1) / (4 / (DK / 64))) * a->num_heads *
                         ((a->chunk + 1) / 2);
    if (wgs4 < cu_count()) return launch_attn_mfma_t<ST, DK, MODE, MULTI, STREAM, 2>(a, k, s);
  }
  return launch_attn_mfma_t<ST, DK, MODE, MULTI, STREAM, 4>(a, k, s);
}

// Page rows are read with the streaming cache policy once a step's windows
// (every layer's K and V rows of the batch) outgrow this share of the 256 MB
// last-level cache: below it the windows stay cached from one step to the
// next and the cached policy reads them faster (64 streams of the small model,
// 160 MB: 8,430 against 8,220 steps/s); above it cached reads only displace
// what is reused (230 streams of the large model, 1.6 GB: 2,906 against
// 2,641 steps/s; 1,024 streams of the small model: 1,903 against 1,742)
constexpr int64_t kStreamingBytes = 192ll << 20;

template <typename ST, int DK, int MODE, bool STREAM>
int launch_attn_mfma_ms(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  // the single-pass form holds at most 16 * kMfmaTiles - 1 keys (its staged
  // position rows stop at 16 * kMfmaTiles)
  if (k.tiles > 1 || k.Lk > 16 * kMfmaTiles - 1) return launch_attn_mfma_nw<ST, DK, MODE, true, STREAM>(a, k, s);
  return launch_attn_mfma_nw<ST, DK, MODE, false, STREAM>(a, k, s);
}

template <typename ST, int DK, int MODE>
int launch_attn_mfma_mode(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  const int64_t layers = a->pages.num_layers > 1 ? a->pages.num_layers : 1;
  const int64_t window_bytes = (int64_t)a->batch * k.Lk * a->num_heads * DK * (int64_t)sizeof(ST) * 2 * layers;
  const bool stream = k.pg.rows != nullptr && window_bytes > kStreamingBytes;
  if (stream) return launch_attn_mfma_ms<ST, DK, MODE, true>(a, k, s);
  return launch_attn_mfma_ms<ST, DK, MODE, false>(a, k, s);
}

template <typename ST, int DK>
int launch_attn_mfma(const pk_attn_args* a, AttnK<ST>& k, hipStream_t s) {
  constexpr int KT = 16 * kMfmaTiles;  // window columns per pass
  k.tiles = (k.Lk + KT - 1) / KT;
  if (k.mask) return launch_attn_mfma_mode<ST, DK, 1>(a, k, s);
  if (k.st_proc) return launch_attn_mfma_mode<ST, DK, 2>(a, k, s);
  return launch_attn_mfma_mode<ST, DK, 0>(a, k, s);
}

// Whole-chunk matrix-core path: workgroups of 2 streams x one head, the
// window split by key between a stream's two waves (48 columns each).
constexpr int kChunkMaxT = 14;      // query operand rows 0..13 (14: u, 15: v)
constexpr int kChunkMaxWindow = 96;  // 2 waves x 3 tiles of 16 window columns

template <typename ST, int DK, int MODE, bool STREAM>
int launch_attn_chunk_t(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  dim3 grid((unsigned)((a->batch + 1) / 2), (unsigned)a->num_heads);
  dim3 block(256u);
  if (a->start_event || a->stop_event) {
    hipExtLaunchKernelGGL(relpos_attn_chunk_kernel<ST, DK, MODE, STREAM>, grid, block, 0u, s,
                          (hipEvent_t)a->start_event, (hipEvent_t)a->stop_event, 0u, k);
  } else {
    hipLaunchKernelGGL((relpos_attn_chunk_kernel<ST, DK, MODE, STREAM>), grid, block, 0, s, k);
  }
  return check_launch("pk_paged_relpos_attn");
}

template <typename ST, int DK, int MODE>
int launch_attn_chunk_mode(const pk_attn_args* a, const AttnK<ST>& k, hipStream_t s) {
  const int64_t layers = a->pages.num_layers > 1 ? a->pages.num_layers : 1;
  const int64_t window_bytes = (int64_t)a->batch * k.Lk * a->num_heads * DK * (int64_t)sizeof(ST) * 2 * layers;
  if (k.pg.rows != nullptr && window_bytes > kStreamingBytes) return launch_attn_chunk_t<ST, DK, MODE, true>(a, k, s);
  return launch_attn_chunk_t<ST, DK, MODE, false>(a, k, s);
}

template <typename ST, int DK>
int launch_attn_chunk(const pk_attn_args* a, AttnK<ST>& k, hipStream_t s) {
  k.tiles = 1;
  if (k.mask) return launch_attn_chunk_mode<ST, DK, 1>(a, k, s);
  if (k.st_proc) return launch_attn_chunk_mode<ST, DK, 2>(a, k, s);
  return launch_attn_chunk_mode<ST, DK, 0>(a, k, s);
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
  const int64_t strides[10] = {a->query_stride_b, a->query_stride_t, a->key_stride_b,
                               a->key_stride_t,   a->value_stride_b, a->value_stride_t,
                               a->pos_stride,     a->out_stride_b,   a->out_stride_t,
                               a->pos_stride_b};
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
    const int rc = pages_view(a->pages, a->layer, VEC, (int)sizeof(ST), what, &k.pg);
    if (rc != PK_OK) return rc;
    if (a->pages.d_model != D)
      return fail(PK_ERR_INVALID, "%s: pages.d_model %d != heads*head_dim %d", what,
                  a->pages.d_model, D);
    if (a->pages.max_pages > 64)
      return fail(PK_ERR_UNSUPPORTED, "%s: max_pages %d > 64 (window longer than 64 pages)", what,
                  a->pages.max_pages);
    const int64_t lo = layer_offset(a->pages, a->layer);
    k.kp = static_cast<ST*>(a->pages.k_pool) + lo;
    k.vp = static_cast<ST*>(a->pages.v_pool) + lo;
  }
  k.pos = static_cast<const ST*>(a->pos);
  k.pos_sr = a->pos_stride;
  k.pos_sb = a->pos_stride_b;
  k.pos_rows = a->pos_rows;
  k.bu = static_cast<const ST*>(a->bias_u);
  k.bv = static_cast<const ST*>(a->bias_v);
  k.mask = a->mask;
  k.m_sb = a->mask_stride_b;
  k.m_sh = a->mask_stride_h;
  k.m_st = a->mask_stride_t;
  if (!a->mask && a->processed_frames) {
    if (!a->cache_lengths)
      return fail(PK_ERR_INVALID, "%s: processed_frames needs cache_lengths", what);
    if (a->chunk_size <= 0)
      return fail(PK_ERR_INVALID, "%s: chunk_size %d must be > 0 for the streaming mask", what,
                  a->chunk_size);
    k.st_proc = a->processed_frames;
    k.st_cl = a->cache_lengths;
    k.st_len = a->lengths;
    k.len_scalar = a->length_scalar;
    k.chunk_size = a->chunk_size;
    k.left_chunks = a->left / a->chunk_size;
    // chunk indices are floor((key_start % C + x) / C) with x < C + window + chunk
    if ((int64_t)(2 * a->chunk_size + a->left + 2 * a->chunk) * a->chunk_size >= (1LL << 31))
      return fail(PK_ERR_UNSUPPORTED, "%s: chunk_size %d too large for the in-kernel mask", what,
                  a->chunk_size);
    k.c_magic = a->chunk_size == 1 ? 0u
                                   : (uint32_t)((1ULL << 32) / (uint64_t)a->chunk_size + 1ULL);
  }
  k.out = static_cast<ST*>(a->out);
  k.o_sb = a->out_stride_b;
  k.o_st = a->out_stride_t;
  k.B = a->batch;
  k.nact = a->live_streams;
  k.T = a->chunk;
  k.H = a->num_heads;
  k.left = a->left;
  k.Lk = Lk;
  k.append = a->append ? 1 : 0;
  k.scale = 1.4426950408889634f / sqrtf((float)DK);

  if (a->num_heads > 65535 || a->chunk > 2 * 65535)
    return fail(PK_ERR_INVALID, "%s: num_heads or chunk exceeds the launch grid", what);
  if constexpr (!std::is_same<ST, float>::value) {
    // the matrix-core kernel addresses rows through buffer resources: row
    // strides up to kMaxBufferStride bytes and fewer than 2^32 pool rows
    const int64_t es = (int64_t)sizeof(ST);
    auto row_bytes = [&](int64_t st) { return (st > 0 ? st : (int64_t)D) * es; };
    const bool fits = (int64_t)D * es <= kMaxBufferStride &&
                      row_bytes(a->key_stride_t) <= kMaxBufferStride &&
                      row_bytes(a->value_stride_t) <= kMaxBufferStride &&
                      row_bytes(a->pos_stride) <= kMaxBufferStride &&
                      (!need_pages || k.pg.cb_shift == 5);  // 64-byte page column blocks
    // per-stream position tables take the vector-ALU kernel: the matrix-core
    // kernels stage one table per workgroup for all of its streams
    const bool mfma_ok = fits && a->pos_stride_b == 0;
    // whole-chunk kernel: chunks of 3..14 frames over a window of at most 96
    // (the query operand's row stride is a buffer stride too); rows_per_lane
    // -2 asks for it at any chunk it supports, -1 for the two-query kernel
    const bool chunk_ok = mfma_ok && a->chunk <= kChunkMaxT && Lk <= kChunkMaxWindow &&
                          row_bytes(a->query_stride_t) <= kMaxBufferStride;
    if (a->rows_per_lane == -2) {
      if (!chunk_ok)
        return fail(PK_ERR_UNSUPPORTED, "%s: the whole-chunk kernel needs chunk <= %d, window <= %d, one position table",
                    what, kChunkMaxT, kChunkMaxWindow);
      if (DK == 64) return launch_attn_chunk<ST, 64>(a, k, s);
      return launch_attn_chunk<ST, 128>(a, k, s);
    }
    if (a->rows_per_lane == 0 && chunk_ok && a->chunk >= 3) {
      if (DK == 64) return launch_attn_chunk<ST, 64>(a, k, s);
      return launch_attn_chunk<ST, 128>(a, k, s);
    }
    if ((a->rows_per_lane == 0 || a->rows_per_lane == -1) && mfma_ok && a->chunk <= 16) {
      if (DK == 64) return launch_attn_mfma<ST, 64>(a, k, s);
      return launch_attn_mfma<ST, 128>(a, k, s);
    }
    if (a->rows_per_lane < 0)
      return fail(PK_ERR_UNSUPPORTED, "%s: rows_per_lane %d asks for a matrix-core kernel this call cannot take", what,
                  a->rows_per_lane);
  }
  const int G = DK / VEC;
  const int rlw = 64 / G;
  const int TQ = pick_tq(a->chunk);
  // fp32, automatic choice: a grid of at most two workgroups a CU splits each
  // window over kSplitWaves waves (one wave's latency would be the launch's)
  const int64_t wgs = (int64_t)a->batch * a->num_heads * ((a->chunk + TQ - 1) / TQ);
  const int waves =
      std::is_same<ST, float>::value && a->rows_per_lane == 0 && wgs <= 2 * (int64_t)cu_count() ? kSplitWaves : 1;
  int NR = 0, tiles = 0;
  pick_tiling(Lk, rlw, a->rows_per_lane, waves, &NR, &tiles);
  if (NR == 0)
    return fail(PK_ERR_UNSUPPORTED, "%s: rows_per_lane %d not built (4, 5, 9, 12, 18)", what,
                a->rows_per_lane);
  k.tiles = tiles;
  if (DK == 64) return launch_attn_tq<ST, 64>(a, k, TQ, NR, waves, s);
  return launch_attn_tq<ST, 128>(a, k, TQ, NR, waves, s);
}

template <typename ST>
int copy_typed(bool gather, const pk_paged_layout& L, int layer, int B, int rows, int end_offset,
               const void* k, int64_t k_sb, int64_t k_st, const void* v, int64_t v_sb,
               int64_t v_st, hipStream_t s, const char* what) {
  constexpr int VEC = Tr<ST>::VEC;
  CopyK<ST> p{};
  if (B == 0) return PK_OK;
  int rc = pages_view(L, layer, VEC, (int)sizeof(ST), what, &p.pg);
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

int pk_hbm_read_probe(const void* src, int64_t bytes, void* out, int32_t workgroups, void* start_event,
                      void* stop_event, void* stream) {
  pk::clear_error();
  if (!src || !out || !pk::aligned16(src) || !pk::aligned16(out))
    return pk::fail(PK_ERR_INVALID, "pk_hbm_read_probe: src and out must be non-NULL and 16-byte aligned");
  if (bytes <= 0 || bytes % 16 != 0)
    return pk::fail(PK_ERR_INVALID, "pk_hbm_read_probe: bytes must be a positive multiple of 16");
  if (workgroups < 0) return pk::fail(PK_ERR_INVALID, "pk_hbm_read_probe: workgroups must be >= 0");
  const int wg = workgroups > 0 ? workgroups : 8 * pk::cu_count();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const pk::u32x4* in = static_cast<const pk::u32x4*>(src);
  pk::u32x4* o = static_cast<pk::u32x4*>(out);
  if (start_event || stop_event) {
    hipExtLaunchKernelGGL(pk::read_probe_kernel, dim3(wg), dim3(256), 0u, s, (hipEvent_t)start_event,
                          (hipEvent_t)stop_event, 0u, in, bytes / 16, o);
  } else {
    hipLaunchKernelGGL(pk::read_probe_kernel, dim3(wg), dim3(256), 0, s, in, bytes / 16, o);
  }
  return pk::check_launch("pk_hbm_read_probe");
}

}  // extern "C"
