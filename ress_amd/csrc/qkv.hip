// Fused q/k normalisation and 2D rotary embedding of a QKV projection, writing q, k, v in
// the head-major layout the attention path reads.
//
// Replaces, for a VGGT-family attention module (reference src/ress/models/qkv.py:60-68,
// compute_patch_qkv before its patch/special split): qkv.reshape(B, N, 3, nh, hd)
// .permute(2, 0, 3, 1, 4), q_norm / k_norm (LayerNorm over the 64 head dims, affine), and
// the 2D RoPE of q and k (the first 32 head dims rotate with the row position, the last
// 32 with the column, rotate-half pairs (j, j+16) at frequencies base^(-2i/32)), with the
// same rounding points as the torch modules: LayerNorm output rounded to the activation
// dtype (bf16), the rotation in fp32 (x*cos + rot(x)*sin, no contraction), rounded again.
// cos/sin are the hardware functions (not the library's), so a small fraction of q/k
// values differ from the modules' by one bf16 rounding.
//
// One workgroup per QKN_TOKENS consecutive tokens, nh*16 threads: thread t owns dims
// 4(t%16)..+3 of head t/16 for q, k and v. Its four rotation frequencies are computed once
// for all of the workgroup's tokens, and q and k share each token's cos/sin. LayerNorm
// statistics reduce over the head's 16 threads (xor 1..8); the rotation partner dims
// j +- 16 sit 4 threads away (xor 4).
#include "common.h"

namespace {

__device__ __forceinline__ float4 ld_bf16x4(const uint16_t* p) {
  const uint2 r = *reinterpret_cast<const uint2*>(p);
  return make_float4(bf16_lo(r.x), bf16_hi(r.x), bf16_lo(r.y), bf16_hi(r.y));
}
__device__ __forceinline__ void st_bf16x4(uint16_t* p, float a, float b, float c, float d) {
  *reinterpret_cast<uint2*>(p) =
      make_uint2(f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16), f32_to_bf16_bits(c) | (f32_to_bf16_bits(d) << 16));
}
__device__ __forceinline__ float sum16(float v) {
  v = v + xor_lane_f<1>(v);
  v = v + xor_lane_f<2>(v);
  v = v + xor_lane_f<4>(v);
  v = v + xor_lane_f<8>(v);
  return v;
}

// LayerNorm of one head's 64 values (4 per thread) -> bf16-rounded fp32
__device__ __forceinline__ float4 head_norm(float4 x, const uint16_t* w, const uint16_t* b, int d0, float eps) {
  const float mean = sum16(((x.x + x.y) + (x.z + x.w))) * (1.0f / 64.0f);
  const float4 c = make_float4(x.x - mean, x.y - mean, x.z - mean, x.w - mean);
  const float var = sum16(((c.x * c.x + c.y * c.y) + (c.z * c.z + c.w * c.w))) * (1.0f / 64.0f);
  const float rstd = 1.0f / sqrtf(var + eps);
  const float4 gw = ld_bf16x4(w + d0), gb = ld_bf16x4(b + d0);
  return make_float4(round_bf16(c.x * rstd * gw.x + gb.x), round_bf16(c.y * rstd * gw.y + gb.y),
                     round_bf16(c.z * rstd * gw.z + gb.z), round_bf16(c.w * rstd * gw.w + gb.w));
}

#define QKN_TOKENS 16

// rotate-half RoPE of dims d0..d0+3 within a 32-dim half, given cos/sin of their angles
__device__ __forceinline__ float4 rope4(float4 y, int d0, const float (&cs)[4], const float (&sn)[4]) {
  const float4 o = make_float4(xor_lane_f<4>(y.x), xor_lane_f<4>(y.y), xor_lane_f<4>(y.z),
                               xor_lane_f<4>(y.w));  // dims d0 +- 16
  const bool lo = (d0 & 31) < 16;
  float r[4];
  const float yy[4] = {y.x, y.y, y.z, y.w}, oo[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float rot = lo ? -oo[u] : oo[u];
    const float a = yy[u] * cs[u], bb = rot * sn[u];
    r[u] = round_bf16(a + bb);
  }
  return make_float4(r[0], r[1], r[2], r[3]);
}

__global__ __launch_bounds__(1024) void k_qk_norm_rope(const uint16_t* __restrict__ qkv, int T, int nh,
                                                       const uint16_t* __restrict__ qw, const uint16_t* __restrict__ qb,
                                                       const uint16_t* __restrict__ kw, const uint16_t* __restrict__ kb,
                                                       float eps, const long long* __restrict__ pos, float base,
                                                       uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
                                                       uint16_t* __restrict__ v_out) {
  const int b = blockIdx.y, t = threadIdx.x, h = t >> 4, d0 = (t & 15) * 4;
  const int C = nh * 64;
  // frequencies base^(-2i/32) of this thread's dims (i = (d0 % 32) % 16 + u)
  float inv[4];
  const int i0 = (d0 & 31) & 15;
#pragma unroll
  for (int u = 0; u < 4; ++u) inv[u] = 1.0f / powf(base, (float)(2 * (i0 + u)) / 32.0f);
  const int tok1 = min(T, (int)(blockIdx.x + 1) * QKN_TOKENS);
  for (int tok = blockIdx.x * QKN_TOKENS; tok < tok1; ++tok) {
    const uint16_t* src = qkv + ((long long)b * T + tok) * 3 * C + h * 64 + d0;
    const float4 q = ld_bf16x4(src), k = ld_bf16x4(src + C);
    const uint2 v = *reinterpret_cast<const uint2*>(src + 2 * C);
    const long long o = (((long long)b * nh + h) * T + tok) * 64 + d0;
    *reinterpret_cast<uint2*>(v_out + o) = v;
    float4 qn = head_norm(q, qw, qb, d0, eps), kn = head_norm(k, kw, kb, d0, eps);
    if (pos) {
      const float p = (float)pos[((long long)b * T + tok) * 2 + (d0 >> 5)];
      float cs[4], sn[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float ang = p * inv[u];
        // the hardware sine/cosine for patch-grid positions (|angle| <= |p| <= 256 rad): their
        // absolute error (~1e-6 at a few tens of radians) moves about one output in a thousand
        // by one bf16 rounding against the library's cosf/sinf, at a fraction of the cost;
        // larger positions take the library functions
        if (fabsf(p) <= 256.0f) {
          cs[u] = __cosf(ang);
          sn[u] = __sinf(ang);
        } else {
          cs[u] = cosf(ang);
          sn[u] = sinf(ang);
        }
      }
      qn = rope4(qn, d0, cs, sn);
      kn = rope4(kn, d0, cs, sn);
    }
    st_bf16x4(q_out + o, qn.x, qn.y, qn.z, qn.w);
    st_bf16x4(k_out + o, kn.x, kn.y, kn.z, kn.w);
  }
}

}  // namespace

// qkv (B, T, 3*nh*64) bf16 contiguous (the qkv Linear's output); q_norm / k_norm affine
// weights and biases [64] bf16; pos (B, T, 2) int64 (row, column) or NULL (no rotation);
// outputs q, k, v (B, nh, T, 64) bf16 contiguous.
RESS_API int ress_qk_norm_rope(const void* qkv, int B, int T, int nh, const void* q_weight, const void* q_bias,
                               const void* k_weight, const void* k_bias, float eps, const void* pos, float rope_base,
                               void* q_out, void* k_out, void* v_out, hipStream_t stream) {
  RESS_REQUIRE(B > 0 && T >= 0 && nh > 0 && nh <= 64, "ress_qk_norm_rope: bad geometry B=%d T=%d nh=%d", B, T, nh);
  RESS_REQUIRE(qkv && q_weight && q_bias && k_weight && k_bias && q_out && k_out && v_out,
               "ress_qk_norm_rope: null pointer");
  RESS_REQUIRE(((uintptr_t)qkv & 7u) == 0 && ((uintptr_t)q_out & 7u) == 0 && ((uintptr_t)k_out & 7u) == 0 &&
                   ((uintptr_t)v_out & 7u) == 0 && ((uintptr_t)q_weight & 7u) == 0 && ((uintptr_t)q_bias & 7u) == 0 &&
                   ((uintptr_t)k_weight & 7u) == 0 && ((uintptr_t)k_bias & 7u) == 0,
               "ress_qk_norm_rope: buffers must be 8-byte aligned");
  if (T == 0) return 0;
  hipLaunchKernelGGL(k_qk_norm_rope, dim3(cdiv(T, QKN_TOKENS), B), dim3(nh * 16), 0, stream, (const uint16_t*)qkv, T, nh,
                     (const uint16_t*)q_weight, (const uint16_t*)q_bias, (const uint16_t*)k_weight,
                     (const uint16_t*)k_bias, eps, (const long long*)pos, rope_base, (uint16_t*)q_out,
                     (uint16_t*)k_out, (uint16_t*)v_out);
  RESS_LAUNCHED("k_qk_norm_rope");
  return 0;
}
