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
// k_pooled_scores_tiled (kb_p <= 1024): 4*PS_TW q-block rows of one head per workgroup,
// PS_TW per wave (independent DOT64 chains per lane; two when that still leaves 512
// workgroups, else one), scores in LDS; pooled K goes through LDS in coalesced 64-block
// tiles that the rows share (tile t+1 is loaded into registers while tile t is used), and
// lane l owns the columns kb = 64t + l, which is also the SUM64 partial order.
// Longer rows: the scores as one matrix-core GEMM into attn_full (k_gemm64, DOT64
// exactly), then k_pooled_softmax_rows; k_pooled_scores_rows beyond 64*PS_E_MAX blocks.
#include <type_traits>

#include "common.h"
#include "mfma_gemm.h"

namespace {
constexpr int PS_TILED_MAX = 1024;
constexpr int PS_LDK = 65;  // tile row stride (floats): conflict-free column reads

template <int PS_TW>  // rows per wave
__global__ __launch_bounds__(256) void k_pooled_scores_tiled(const float* __restrict__ pooled_q,
                                                             const float* __restrict__ pooled_k, int q_blk,
                                                             int kb_p, int n_cand, float scale,
                                                             float* __restrict__ attn_full,
                                                             float* __restrict__ attn_cond) {
  extern __shared__ float ps_dyn[];  // [4*PS_TW][kb_p] scores, then exponentials, per row
  __shared__ float pk_l[64 * PS_LDK];
  __shared__ __align__(16) float pq_l[4 * PS_TW][64];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.y, qb_wg = blockIdx.x * 4 * PS_TW, qb0 = qb_wg + w * PS_TW;
  for (int i = tid; i < 4 * PS_TW * 64; i += 256) {
    const int qb = qb_wg + (i >> 6);
    pq_l[i >> 6][i & 63] = qb < q_blk ? pooled_q[((long long)bh * q_blk + qb) * 64 + (i & 63)] : 0.0f;
  }
  const int nrow = max(0, min(PS_TW, q_blk - qb0));  // this wave's valid rows (wave-uniform)
  float* e0 = ps_dyn + w * PS_TW * kb_p;
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
  float lmax[PS_TW];
#pragma unroll
  for (int r = 0; r < PS_TW; ++r) lmax[r] = -__builtin_huge_valf();
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
    if (nrow > 0 && kb < kb_p) {
      const float* kc = pk_l + lane * PS_LDK;
      float acc[PS_TW];
#pragma unroll
      for (int r = 0; r < PS_TW; ++r) acc[r] = 0.0f;
#pragma unroll 4
      for (int d4 = 0; d4 < 16; ++d4) {
        const float k0 = kc[4 * d4], k1 = kc[4 * d4 + 1], k2 = kc[4 * d4 + 2], k3 = kc[4 * d4 + 3];
#pragma unroll
        for (int r = 0; r < PS_TW; ++r) {
          const float4 qq = reinterpret_cast<const float4*>(pq_l[w * PS_TW + r])[d4];
          acc[r] = fmaf(qq.x, k0, acc[r]);
          acc[r] = fmaf(qq.y, k1, acc[r]);
          acc[r] = fmaf(qq.z, k2, acc[r]);
          acc[r] = fmaf(qq.w, k3, acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < PS_TW; ++r) {
        const float sc = acc[r] * scale;
        e0[r * kb_p + kb] = sc;
        lmax[r] = fmaxf(lmax[r], sc);
      }
    }
  }
  // from here each lane reads back only its own columns: no further synchronisation
  for (int r = 0; r < nrow; ++r) {
    float* e = e0 + r * kb_p;
    const long long row = (long long)bh * q_blk + qb0 + r;
    const float m = wave_max(lmax[r]);
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
}
// The softmax of rows whose raw scores are already in attn_full, one wave per row (four
// rows per workgroup): lane l holds columns kb = 64e + l (e < E) in registers, the SUM64
// partial order; the same outputs as k_pooled_scores_tiled.
template <int E>
__global__ __launch_bounds__(256) void k_pooled_softmax_rows(int q_blk, int kb_p, int n_cand, int qb_begin,
                                                             int qb_end, float* __restrict__ attn_full,
                                                             float* __restrict__ attn_cond) {
  const int lane = threadIdx.x & 63;
  const int qb = qb_begin + blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (qb >= qb_end) return;  // wave-uniform
  const long long row = (long long)blockIdx.y * q_blk + qb;
  float* full = attn_full + row * kb_p;
  float* cond = attn_cond + row * n_cand;
  // slots e < fk hold a column on every lane; slot fk on lanes below kb_p % 64 (the
  // bounds are wave-uniform, so the slot tests are scalar)
  const int fk = kb_p >> 6, rk = kb_p & 63, fc = n_cand >> 6, rc = n_cand & 63;
  float x[E];
  float m = -__builtin_huge_valf();
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = -__builtin_huge_valf();
    if (e < fk || (e == fk && lane < rk)) x[e] = full[64 * e + lane];
    m = fmaxf(m, x[e]);
  }
  m = wave_max(m);
  float part = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (e < fk || (e == fk && lane < rk)) {
      x[e] = ress_expf(x[e] - m);
      part = part + x[e];
    }
  const float total = sum64_tree(part);
  float cpart = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (e < fk || (e == fk && lane < rk)) {
      x[e] = x[e] / total;
      full[64 * e + lane] = x[e];
      if (e < fc || (e == fc && lane < rc)) cpart = cpart + x[e];
    }
  float rs = sum64_tree(cpart);
  rs = fmaxf(rs, 0x1.0c6f7ap-20f);  // clamp(min=1e-6)
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (e < fc || (e == fc && lane < rc)) cond[64 * e + lane] = x[e] / rs;
}
constexpr int PS_E_MAX = 128;  // k_pooled_softmax_rows: rows of up to 64*PS_E_MAX blocks
}  // namespace

int scores_gemm(const float* a, const float* b, int BH, int na, int nb, int r_begin, int r_end, float scale,
                float* S, hipStream_t stream) {
  hipLaunchKernelGGL(k_gemm64<G64Store<>>, g64_grid(BH, nb, r_begin, r_end, G64Store<>::kWalk), dim3(256), 0, stream,
                     a, b, na, nb,
                     64ll * nb, r_begin, r_end, G64Store<>{S, scale});
  RESS_LAUNCHED("k_gemm64<G64Store<>>");
  return 0;
}

// Rows longer than PS_TILED_MAX: PS_RW rows per wave (two measured fastest: more rows per
// wave do not pay on 4294-block rows), four waves, so a workgroup covers
// 4*PS_RW consecutive q-block rows of one head. Pooled K goes through LDS in the same
// coalesced 64-column tiles as the tiled kernel, shared by all of the workgroup's rows,
// and lane l computes column 64t + l for each of its wave's rows: PS_RW independent DOT64
// chains per lane. The raw scores are written to attn_full; the softmax passes then read
// back, lane by lane, the columns the same lane wrote (SUM64 order), recomputing the
// exponentials in the last pass rather than storing them.
constexpr int PS_RW = 2;
__global__ __launch_bounds__(256) void k_pooled_scores_rows(const float* __restrict__ pooled_q,
                                                            const float* __restrict__ pooled_k, int q_blk, int kb_p,
                                                            int n_cand, float scale, float* __restrict__ attn_full,
                                                            float* __restrict__ attn_cond) {
  __shared__ float pk_l[64 * PS_LDK];
  __shared__ __align__(16) float pq_l[4 * PS_RW][64];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.y, qb_wg = blockIdx.x * 4 * PS_RW, qb0 = qb_wg + w * PS_RW;
  for (int i = tid; i < 4 * PS_RW * 64; i += 256) {
    const int qb = qb_wg + (i >> 6);
    pq_l[i >> 6][i & 63] = qb < q_blk ? pooled_q[((long long)bh * q_blk + qb) * 64 + (i & 63)] : 0.0f;
  }
  const int nrow = max(0, min(PS_RW, q_blk - qb0));  // this wave's valid rows (wave-uniform)
  const float* pkh = pooled_k + (long long)bh * kb_p * 64;
  float* full0 = attn_full + ((long long)bh * q_blk + qb0) * kb_p;
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
  float lmax[PS_RW];
#pragma unroll
  for (int r = 0; r < PS_RW; ++r) lmax[r] = -__builtin_huge_valf();
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
    if (nrow > 0 && kb < kb_p) {
      const float* kc = pk_l + lane * PS_LDK;
      float acc[PS_RW];
#pragma unroll
      for (int r = 0; r < PS_RW; ++r) acc[r] = 0.0f;
#pragma unroll 4  // fully unrolled, the compiler issues every Q and K read up front (300 VGPRs)
      for (int d4 = 0; d4 < 16; ++d4) {
        const float k0 = kc[4 * d4], k1 = kc[4 * d4 + 1], k2 = kc[4 * d4 + 2], k3 = kc[4 * d4 + 3];
#pragma unroll
        for (int r = 0; r < PS_RW; ++r) {
          const float4 qq = reinterpret_cast<const float4*>(pq_l[w * PS_RW + r])[d4];
          acc[r] = fmaf(qq.x, k0, acc[r]);
          acc[r] = fmaf(qq.y, k1, acc[r]);
          acc[r] = fmaf(qq.z, k2, acc[r]);
          acc[r] = fmaf(qq.w, k3, acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < PS_RW; ++r)
        if (r < nrow) {
          const float sc = acc[r] * scale;
          full0[(long long)r * kb_p + kb] = sc;
          lmax[r] = fmaxf(lmax[r], sc);
        }
    }
  }
  // softmax of each row, by this wave alone (each lane reads back only the columns it wrote)
  for (int r = 0; r < nrow; ++r) {
    float* full = full0 + (long long)r * kb_p;
    const float m = wave_max(lmax[r]);
    float part = 0.0f;
    for (int kb = lane; kb < kb_p; kb += 64) part = part + ress_expf(full[kb] - m);
    const float total = sum64_tree(part);
    float cpart = 0.0f;
    float* cond = attn_cond + ((long long)bh * q_blk + qb0 + r) * n_cand;
    for (int kb = lane; kb < kb_p; kb += 64) {
      const float x = ress_expf(full[kb] - m);
      const float p = x / total;
      full[kb] = p;
      if (kb < n_cand) {
        cpart = cpart + p;
        cond[kb] = x;  // exponential for now; divided below once rs is known
      }
    }
    float rs = sum64_tree(cpart);
    rs = fmaxf(rs, 0x1.0c6f7ap-20f);  // clamp(min=1e-6)
    for (int kb = lane; kb < n_cand; kb += 64) cond[kb] = (cond[kb] / total) / rs;
  }
}

// attn_full / attn_cond from pooled Q [BH][q_blk][64] and pooled K [BH][kb_p][64].
// n_cand <= kb_p leading blocks are the droppable candidates
// (reference attention.py:453-457).
RESS_API int ress_pooled_scores(const void* pooled_q, const void* pooled_k, int BH, int q_blk, int kb_p, int n_cand,
                                float scale, void* attn_full, void* attn_cond, hipStream_t stream) {
  RESS_REQUIRE(BH > 0 && q_blk > 0 && kb_p > 0 && n_cand >= 0 && n_cand <= kb_p,
               "ress_pooled_scores: bad geometry BH=%d q_blk=%d kb_p=%d n_cand=%d", BH, q_blk, kb_p, n_cand);
  RESS_REQUIRE(pooled_q && pooled_k && attn_full && attn_cond, "ress_pooled_scores: null pointer");
  RESS_REQUIRE(((uintptr_t)pooled_k & 15u) == 0, "ress_pooled_scores: pooled_k must be 16-byte aligned");
  if (kb_p <= PS_TILED_MAX) {
    auto go = [&](auto tw) {
      constexpr int TW = decltype(tw)::value;
      hipLaunchKernelGGL(k_pooled_scores_tiled<TW>, dim3(cdiv(q_blk, 4 * TW), BH), dim3(256),
                         4 * TW * kb_p * sizeof(float), stream, (const float*)pooled_q, (const float*)pooled_k, q_blk,
                         kb_p, n_cand, scale, (float*)attn_full, (float*)attn_cond);
    };
    if ((long long)cdiv(q_blk, 8) * BH >= 512) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 1>{});
  } else if (kb_p <= 64 * PS_E_MAX) {
    RESS_REQUIRE(((uintptr_t)pooled_q & 15u) == 0, "ress_pooled_scores: pooled_q must be 16-byte aligned");
    const int rc = scores_gemm((const float*)pooled_q, (const float*)pooled_k, BH, q_blk, kb_p, 0, q_blk, scale,
                               (float*)attn_full, stream);
    if (rc) return rc;
    auto go = [&](auto ee) {
      constexpr int EE = decltype(ee)::value;
      hipLaunchKernelGGL(k_pooled_softmax_rows<EE>, dim3(cdiv(q_blk, 4), BH), dim3(256), 0, stream, q_blk, kb_p,
                         n_cand, 0, q_blk, (float*)attn_full, (float*)attn_cond);
    };
    const int e = cdiv(kb_p, 64);
    if (e <= 24) go(std::integral_constant<int, 24>{});
    else if (e <= 32) go(std::integral_constant<int, 32>{});
    else if (e <= 48) go(std::integral_constant<int, 48>{});
    else if (e <= 64) go(std::integral_constant<int, 64>{});
    else if (e <= 80) go(std::integral_constant<int, 80>{});
    else if (e <= 96) go(std::integral_constant<int, 96>{});
    else go(std::integral_constant<int, PS_E_MAX>{});
  } else {
    hipLaunchKernelGGL(k_pooled_scores_rows, dim3(cdiv(q_blk, 4 * PS_RW), BH), dim3(256), 0, stream,
                       (const float*)pooled_q, (const float*)pooled_k, q_blk, kb_p, n_cand, scale, (float*)attn_full,
                       (float*)attn_cond);
  }
  RESS_LAUNCHED("k_pooled_scores");
  return 0;
}
