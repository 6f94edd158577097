// Exhaustive check of the library's fp32 -> bf16 rounding (pk::f32_to_bf16_bits and
// the paired conversion behind Tr<bf16_t>::pack, pk_device.h), which uses gfx950's
// packed conversion instruction.  Every one of the 2^32 fp32 bit patterns is rounded
// by it and by the integer round-to-nearest-even the library used before,
//   (u + 0x7fff + ((u >> 16) & 1)) >> 16, and for a NaN (u >> 16) | 0x40,
// and the mismatches are counted.  Prints "mismatches N first X" and exits 0 only
// when N == 0.  Built by parakeet-streaming_amd/build.py; run by
// tests/test_gpu_bf16_rounding.py.
#include <hip/hip_runtime.h>

#include <cstdio>

#include "pk_device.h"

namespace {

__device__ unsigned integer_rne(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// thread: 256 consecutive bit patterns, as 128 pairs through both entry points
__global__ void __launch_bounds__(256) check(unsigned long long* count, unsigned* first) {
  const unsigned long long base = ((unsigned long long)blockIdx.x * 256 + threadIdx.x) * 256ull;
  unsigned bad = 0;
  for (unsigned i = 0; i < 256; i += 2) {
    const unsigned u0 = (unsigned)(base + i), u1 = u0 + 1;
    const float f0 = __uint_as_float(u0), f1 = __uint_as_float(u1);
    const unsigned pair = pk::bf16_pair_bits(f0, f1);
    const unsigned one0 = pk::f32_to_bf16_bits(f0), one1 = pk::f32_to_bf16_bits(f1);
    const unsigned r0 = integer_rne(f0), r1 = integer_rne(f1);
    if ((pair & 0xffffu) != r0 || one0 != r0) {
      ++bad;
      atomicMin(first, u0);
    }
    if ((pair >> 16) != r1 || one1 != r1) {
      ++bad;
      atomicMin(first, u1);
    }
  }
  if (bad) atomicAdd(count, (unsigned long long)bad);
}

}  // namespace

int main() {
  unsigned long long* count = nullptr;
  unsigned* first = nullptr;
  if (hipMalloc(&count, sizeof(*count)) != hipSuccess || hipMalloc(&first, sizeof(*first)) != hipSuccess) {
    printf("hipMalloc failed\n");
    return 2;
  }
  if (hipMemset(count, 0, sizeof(*count)) != hipSuccess || hipMemset(first, 0xff, sizeof(*first)) != hipSuccess) {
    printf("hipMemset failed\n");
    return 2;
  }
  hipLaunchKernelGGL(check, dim3(65536), dim3(256), 0, 0, count, first);  // 65536 x 256 x 256 = 2^32
  unsigned long long n = 0;
  unsigned f = 0;
  if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(&n, count, sizeof(n), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&f, first, sizeof(f), hipMemcpyDeviceToHost) != hipSuccess) {
    printf("kernel or copy failed\n");
    return 2;
  }
  printf("mismatches %llu first 0x%08x\n", n, f);
  (void)hipFree(count);
  (void)hipFree(first);
  return n == 0 ? 0 : 1;
}
