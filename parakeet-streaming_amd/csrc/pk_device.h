// Device helpers shared by the gfx950 kernels of the paged K/V-cache library:
// 16-byte element chunks <-> fp32 registers, bfloat16 rounding, DPP lane-group
// reductions, wave-local LDS ordering.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pk_common.h"

namespace pk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

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

// bfloat16 is carried as raw 16-bit patterns; fp32 -> bf16 rounds to nearest
// even with gfx950's v_cvt_pk_bf16_f32, two values an instruction.  For every
// fp32 input it gives the bits of the integer rounding (u + 0x7fff + ((u >> 16)
// & 1)) >> 16, and for a NaN (u >> 16) | 0x40 (sign and high payload kept,
// quieted): tests/native/bf16_rounding_check.hip runs all 2^32 inputs.
struct bf16_t {
  uint16_t bits;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// lo in bits 0-15, hi in bits 16-31
__device__ static inline uint32_t bf16_pair_bits(float lo, float hi) {
  bf16x2_t v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ static inline uint32_t f32_to_bf16_bits(float f) { return bf16_pair_bits(f, 0.f) & 0xffffu; }

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
    v.x = bf16_pair_bits(f[0], f[1]);
    v.y = bf16_pair_bits(f[2], f[3]);
    v.z = bf16_pair_bits(f[4], f[5]);
    v.w = bf16_pair_bits(f[6], f[7]);
    return v;
  }
};

// x rounded to the storage type and back.
template <typename ST>
__device__ static inline float round_to(float x);
template <>
__device__ inline float round_to<float>(float x) {
  return x;
}
template <>
__device__ inline float round_to<_Float16>(float x) {
  return (float)(_Float16)x;
}
template <>
__device__ inline float round_to<bf16_t>(float x) {
  return __uint_as_float(f32_to_bf16_bits(x) << 16);
}

// one element: fp32 <-> storage type
template <typename ST>
__device__ static inline ST to_st(float x);
template <>
__device__ inline float to_st<float>(float x) {
  return x;
}
template <>
__device__ inline _Float16 to_st<_Float16>(float x) {
  return (_Float16)x;
}
template <>
__device__ inline bf16_t to_st<bf16_t>(float x) {
  return bf16_t{(uint16_t)f32_to_bf16_bits(x)};
}
__device__ static inline float from_st(float v) { return v; }
__device__ static inline float from_st(_Float16 v) { return (float)v; }
__device__ static inline float from_st(bf16_t v) { return __uint_as_float((uint32_t)v.bits << 16); }

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

template <typename ST>
__device__ static inline void st16_stream(ST* p, const u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
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
// host-side launch helpers

// Makes `dev` current for the scope of a call (dev < 0: keep the current one).
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

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PK_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PK_OK;
}

// ---------------------------------------------------------------------------
// CUs of the current device, read once per device
static inline int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace pk
