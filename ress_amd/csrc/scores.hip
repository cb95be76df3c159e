// Pooled block-attention map.
//
// Replaces predict_attention's pooled GEMM + softmax (reference
// src/ress/models/attention.py:98-100) and the patch-conditional renormalisation
// attn_cond = attn_pooled / clamp(rowsum, 1e-6) (attention.py:457,473).
//
// One wave per (q-block row, batch*head). Scores s[kb] = DOT64(pq, pk[kb]) * 0.125
// (1/sqrt(64), exact); softmax with ress_expf and SUM64 denominators; outputs
//   attn_full [BH][q_blk][kb_p]   softmax over all kb_p pooled key blocks
//   attn_cond [BH][q_blk][n_cand] the first n_cand renormalised to sum 1
#include "common.h"

__global__ __launch_bounds__(64) void k_pooled_scores(const float* __restrict__ pooled_q,
                                                      const float* __restrict__ pooled_k, int q_blk, int kb_p,
                                                      int n_cand, float scale, float* __restrict__ attn_full,
                                                      float* __restrict__ attn_cond) {
  extern __shared__ float e[];  // kb_p floats
  __shared__ float pq[64];
  const int qb = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  pq[lane] = pooled_q[((long long)bh * q_blk + qb) * 64 + lane];
  __syncthreads();
  const float4* pk = reinterpret_cast<const float4*>(pooled_k + (long long)bh * kb_p * 64);

  float lmax = -__builtin_huge_valf();
  for (int kb = lane; kb < kb_p; kb += 64) {
    float acc = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < 16; ++d4) {
      const float4 b = pk[kb * 16 + d4];
      acc = fmaf(pq[4 * d4 + 0], b.x, acc);
      acc = fmaf(pq[4 * d4 + 1], b.y, acc);
      acc = fmaf(pq[4 * d4 + 2], b.z, acc);
      acc = fmaf(pq[4 * d4 + 3], b.w, acc);
    }
    const float s = acc * scale;
    e[kb] = s;
    lmax = fmaxf(lmax, s);
  }
  const float m = wave_max(lmax);
  float part = 0.0f;
  for (int kb = lane; kb < kb_p; kb += 64) {
    const float x = ress_expf(e[kb] - m);
    e[kb] = x;
    part = part + x;
  }
  const float total = sum64_tree(part);
  float* full = attn_full + ((long long)bh * q_blk + qb) * kb_p;
  float cpart = 0.0f;
  for (int kb = lane; kb < kb_p; kb += 64) {
    const float p = e[kb] / total;
    full[kb] = p;
    if (kb < n_cand) cpart = cpart + p;
  }
  float rs = sum64_tree(cpart);
  rs = fmaxf(rs, 0x1.0c6f7ap-20f);  // clamp(min=1e-6)
  float* cond = attn_cond + ((long long)bh * q_blk + qb) * n_cand;
  for (int kb = lane; kb < n_cand; kb += 64) cond[kb] = (e[kb] / total) / rs;
}

// attn_full / attn_cond from pooled Q [BH][q_blk][64] and pooled K [BH][kb_p][64].
// n_cand <= kb_p leading blocks are the droppable candidates
// (reference attention.py:453-457).
RESS_API int ress_pooled_scores(const void* pooled_q, const void* pooled_k, int BH, int q_blk, int kb_p, int n_cand,
                                float scale, void* attn_full, void* attn_cond, hipStream_t stream) {
  RESS_REQUIRE(BH > 0 && q_blk > 0 && kb_p > 0 && n_cand >= 0 && n_cand <= kb_p,
               "ress_pooled_scores: bad geometry BH=%d q_blk=%d kb_p=%d n_cand=%d", BH, q_blk, kb_p, n_cand);
  RESS_REQUIRE(kb_p <= 16384, "ress_pooled_scores: kb_p=%d exceeds the LDS row limit 16384", kb_p);
  RESS_REQUIRE(pooled_q && pooled_k && attn_full && attn_cond, "ress_pooled_scores: null pointer");
  RESS_REQUIRE(((uintptr_t)pooled_k & 15u) == 0, "ress_pooled_scores: pooled_k must be 16-byte aligned");
  hipLaunchKernelGGL(k_pooled_scores, dim3(q_blk, BH), dim3(64), kb_p * sizeof(float), stream,
                     (const float*)pooled_q, (const float*)pooled_k, q_blk, kb_p, n_cand, scale, (float*)attn_full,
                     (float*)attn_cond);
  RESS_LAUNCHED("k_pooled_scores");
  return 0;
}
