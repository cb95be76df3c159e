// Pooled block-attention map.
//
// Replaces predict_attention's pooled GEMM + softmax (reference
// src/ress/models/attention.py:98-100) and the patch-conditional renormalisation
// attn_cond = attn_pooled / clamp(rowsum, 1e-6) (attention.py:457,473).
//
// Scores s[kb] = DOT64(pq, pk[kb]) * 0.125 (1/sqrt(64), exact); softmax with ress_expf
// and SUM64 denominators; outputs
//   attn_full [BH][q_blk][kb_p]   softmax over all kb_p pooled key blocks
//   attn_cond [BH][q_blk][n_cand] the first n_cand renormalised to sum 1
// k_pooled_scores_tiled (kb_p <= 2048): four q-block rows of one head per workgroup, one
// wave per row; pooled K goes through LDS in coalesced 64-block tiles that the four rows
// share (tile t+1 is loaded into registers while tile t is used), and lane l owns the
// columns kb = 64t + l, which is also the SUM64 partial order. k_pooled_scores: one wave
// per row for longer rows, pooled K staged through a small LDS chunk per 64 columns.
#include "common.h"

namespace {
constexpr int PS_TILED_MAX = 2048;
constexpr int PS_LDK = 65;  // tile row stride (floats): conflict-free column reads
constexpr int PS_CH_LD = 17;  // k_pooled_scores chunk row stride (floats)

__global__ __launch_bounds__(256) void k_pooled_scores_tiled(const float* __restrict__ pooled_q,
                                                             const float* __restrict__ pooled_k, int q_blk,
                                                             int kb_p, int n_cand, float scale,
                                                             float* __restrict__ attn_full,
                                                             float* __restrict__ attn_cond) {
  extern __shared__ float ps_dyn[];  // [4][kb_p] scores, then exponentials, per wave
  __shared__ float pk_l[64 * PS_LDK];
  __shared__ __align__(16) float pq_l[4][64];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.y, qb = blockIdx.x * 4 + w;
  const bool in_range = qb < q_blk;
  const long long row = (long long)bh * q_blk + qb;
  float* e = ps_dyn + w * kb_p;
  if (in_range) pq_l[w][lane] = pooled_q[row * 64 + lane];
  const float* pkh = pooled_k + (long long)bh * kb_p * 64;
  const int tiles = cdiv(kb_p, 64);
  float4 nxt[4];
  auto load_tile = [&](int t) {
    const int cols = min(64, kb_p - 64 * t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f4 = tid + 256 * i, col = f4 >> 4;
      nxt[i] = col < cols ? reinterpret_cast<const float4*>(pkh + (long long)(64 * t + col) * 64)[f4 & 15]
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  load_tile(0);
  float lmax = -__builtin_huge_valf();
#pragma unroll 1
  for (int t = 0; t < tiles; ++t) {
    __syncthreads();  // previous tile consumed (and pq_l written, first time)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f4 = tid + 256 * i;
      float* dst = pk_l + (f4 >> 4) * PS_LDK + (f4 & 15) * 4;
      dst[0] = nxt[i].x;
      dst[1] = nxt[i].y;
      dst[2] = nxt[i].z;
      dst[3] = nxt[i].w;
    }
    __syncthreads();
    if (t + 1 < tiles) load_tile(t + 1);
    const int kb = 64 * t + lane;
    if (in_range && kb < kb_p) {
      const float4* qv = reinterpret_cast<const float4*>(pq_l[w]);
      const float* kc = pk_l + lane * PS_LDK;
      float acc = 0.0f;
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        const float4 qq = qv[d4];
        acc = fmaf(qq.x, kc[4 * d4 + 0], acc);
        acc = fmaf(qq.y, kc[4 * d4 + 1], acc);
        acc = fmaf(qq.z, kc[4 * d4 + 2], acc);
        acc = fmaf(qq.w, kc[4 * d4 + 3], acc);
      }
      const float s = acc * scale;
      e[kb] = s;
      lmax = fmaxf(lmax, s);
    }
  }
  if (!in_range) return;
  // from here each lane reads back only its own columns: no further synchronisation
  const float m = wave_max(lmax);
  float part = 0.0f;
  for (int kb = lane; kb < kb_p; kb += 64) {
    const float x = ress_expf(e[kb] - m);
    e[kb] = x;
    part = part + x;
  }
  const float total = sum64_tree(part);
  float* full = attn_full + row * kb_p;
  float cpart = 0.0f;
  for (int kb = lane; kb < kb_p; kb += 64) {
    const float p = e[kb] / total;
    full[kb] = p;
    if (kb < n_cand) cpart = cpart + p;
  }
  float rs = sum64_tree(cpart);
  rs = fmaxf(rs, 0x1.0c6f7ap-20f);  // clamp(min=1e-6)
  float* cond = attn_cond + row * n_cand;
  for (int kb = lane; kb < n_cand; kb += 64) cond[kb] = (e[kb] / total) / rs;
}
}  // namespace

__global__ __launch_bounds__(64) void k_pooled_scores(const float* __restrict__ pooled_q,
                                                      const float* __restrict__ pooled_k, int q_blk, int kb_p,
                                                      int n_cand, float scale, float* __restrict__ attn_full,
                                                      float* __restrict__ attn_cond) {
  extern __shared__ float e[];  // kb_p floats
  __shared__ float pq[64];
  __shared__ float chunk[64 * PS_CH_LD];  // 64 columns x 16 dims of pooled K
  const int qb = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  pq[lane] = pooled_q[((long long)bh * q_blk + qb) * 64 + lane];
  __syncthreads();
  const float* pkh = pooled_k + (long long)bh * kb_p * 64;

  // 64 columns per step (lane = column): their pooled K goes through LDS 16 dims at a
  // time with coalesced loads (the next chunk in flight while one is used); the DOT64
  // chain runs over d = 0..63 in order
  float lmax = -__builtin_huge_valf();
  for (int c0 = 0; c0 < kb_p; c0 += 64) {
    float4 ld[4];
    auto load_chunk = [&](int q) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int f = 64 * t + lane, col = c0 + (f >> 2);
        ld[t] = col < kb_p ? *reinterpret_cast<const float4*>(pkh + (long long)col * 64 + 16 * q + 4 * (f & 3))
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    };
    load_chunk(0);
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int f = 64 * t + lane;
        float* dst = chunk + (f >> 2) * PS_CH_LD + 4 * (f & 3);
        dst[0] = ld[t].x;
        dst[1] = ld[t].y;
        dst[2] = ld[t].z;
        dst[3] = ld[t].w;
      }
      __builtin_amdgcn_wave_barrier();
      if (q + 1 < 4) load_chunk(q + 1);
      const float* kc = chunk + lane * PS_CH_LD;
#pragma unroll
      for (int d = 0; d < 16; ++d) acc = fmaf(pq[16 * q + d], kc[d], acc);
      __builtin_amdgcn_wave_barrier();  // every lane has read the chunk before it is overwritten
    }
    const int kb = c0 + lane;
    if (kb < kb_p) {
      const float s = acc * scale;
      e[kb] = s;
      lmax = fmaxf(lmax, s);
    }
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
  if (kb_p <= PS_TILED_MAX) {
    hipLaunchKernelGGL(k_pooled_scores_tiled, dim3(cdiv(q_blk, 4), BH), dim3(256), 4 * kb_p * sizeof(float), stream,
                       (const float*)pooled_q, (const float*)pooled_k, q_blk, kb_p, n_cand, scale, (float*)attn_full,
                       (float*)attn_cond);
  } else {
    hipLaunchKernelGGL(k_pooled_scores, dim3(q_blk, BH), dim3(64), kb_p * sizeof(float), stream,
                       (const float*)pooled_q, (const float*)pooled_k, q_blk, kb_p, n_cand, scale, (float*)attn_full,
                       (float*)attn_cond);
  }
  RESS_LAUNCHED("k_pooled_scores");
  return 0;
}
