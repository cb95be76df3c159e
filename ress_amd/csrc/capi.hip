// C-ABI support: thread-local error string and version.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_err[512] = "";

void ress_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

RESS_API const char* ress_last_error(void) { return g_err; }

RESS_API int ress_abi_version(void) { return 5; }

// The bf16 rounding every kernel uses (round_bf16: the device's __bf16 conversion) against
// the round-to-nearest-even bit formula it stands for, over the fp32 bit patterns
// first .. first + count - 1 (mod 2^32): out[0] += the number of patterns that differ,
// out[1] = min(out[1], the lowest such pattern). Grid-stride; every access is in bounds.
__global__ void k_bf16_selfcheck(uint32_t first, unsigned long long count, unsigned long long* out) {
  const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
  unsigned long long bad = 0, low = ~0ull;
  for (unsigned long long i = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint32_t u = first + (uint32_t)i;
    const uint32_t want = (u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    if (f32_to_bf16_bits(__uint_as_float(u)) != want) {
      ++bad;
      low = min(low, (unsigned long long)u);
    }
  }
  if (bad) {
    atomicAdd(&out[0], bad);
    atomicMin(&out[1], low);
  }
}

RESS_API int ress_bf16_selfcheck(unsigned int first, unsigned long long count, void* out, hipStream_t stream) {
  RESS_REQUIRE(out && count <= (1ull << 32), "ress_bf16_selfcheck: null output or count above 2^32");
  if (count == 0) return 0;
  hipLaunchKernelGGL(k_bf16_selfcheck, dim3(2048), dim3(256), 0, stream, (uint32_t)first, count,
                     (unsigned long long*)out);
  RESS_LAUNCHED("k_bf16_selfcheck");
  return 0;
}
