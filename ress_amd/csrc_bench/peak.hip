// Measured-peak microbenchmark for bench.py (not part of libress_hip): dense MFMA
// throughput on this GPU, to report the attention kernel against a measured peak as
// well as the published one.
//
// Every wave runs `iters` rounds of four independent accumulator chains of one MFMA
// (bf16 v_mfma_f32_32x32x16_bf16: 32768 FLOP each; int8 v_mfma_i32_32x32x32_i8: 65536
// OP each), so the matrix cores never wait on a dependency. Operands are registers
// only; each lane writes one word of the result so nothing is optimised away.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void k_peak_bf16(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const uint4 a = make_uint4(lane, lane * 3u, lane * 5u, lane * 7u), b = make_uint4(lane * 11u, 13u, 1u, 2u);
  v16f c0, c1, c2, c3;
  for (int r = 0; r < 16; ++r) c0[r] = c1[r] = c2[r] = c3[r] = 0.0f;
  const v8bf A = __builtin_bit_cast(v8bf, a), B = __builtin_bit_cast(v8bf, b);
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(B, A, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, A, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(B, B, c3, 0, 0, 0);
  }
  float s = 0.0f;
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_peak_i8(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const v4i a = {lane, lane * 3, lane * 5, lane * 7}, b = {lane * 11, 13, 1, 2};
  v16i c0, c1, c2, c3;
  for (int r = 0; r < 16; ++r) c0[r] = c1[r] = c2[r] = c3[r] = 0;
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
  }
  int s = 0;
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  out[blockIdx.x * 256 + threadIdx.x] = (float)s;
}

// kind 0 = bf16, 1 = int8; `wgs` workgroups of 256 threads; out holds wgs*256 floats.
// Returns 0, or -1 on a bad argument / -2 on a launch failure.
extern "C" __attribute__((visibility("default"))) int ress_peak_mfma(int kind, int iters, int wgs, void* out,
                                                                       hipStream_t stream) {
  if (iters <= 0 || wgs <= 0 || !out || kind < 0 || kind > 1) return -1;
  if (kind == 0)
    hipLaunchKernelGGL(k_peak_bf16, dim3(wgs), dim3(256), 0, stream, iters, (float*)out);
  else
    hipLaunchKernelGGL(k_peak_i8, dim3(wgs), dim3(256), 0, stream, iters, (float*)out);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
