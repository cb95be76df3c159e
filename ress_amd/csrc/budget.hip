// Per-(head, query-block) key-block budgets.
//
// Replaces:
//   compute_baseline_num_to_select  (reference src/ress/models/attention.py:268-293)
//     cdf:  sort desc, cumsum, searchsorted(cdf, fp32(tau) + 1e-5, right=True)
//     sr:   topk = int(k_blk * (1 - sr)) (host double arithmetic), max(cdf_count, topk)
//   adjust_attention_selection      (reference src/ress/budget/_proportional.py:49-115)
//     HeSS cap-and-redistribute across heads per query-block column, fp32
//   the MIN_NUM_TO_SELECT floor     (attention.py:525)
//
// The CDF prefix sum is sequential (SEQ) over the descending-sorted row, so it
// does not depend on how ties are ordered.
#include "common.h"

// One workgroup of 256 threads per row; bitonic sort (descending) in LDS.
__global__ __launch_bounds__(256) void k_cdf_count(const float* __restrict__ attn_cond, int n, int npow2,
                                                   float thr, int topk, int* __restrict__ out) {
  extern __shared__ float v[];  // npow2
  const long long row = blockIdx.x;
  const float* src = attn_cond + row * n;
  for (int i = threadIdx.x; i < npow2; i += 256) v[i] = i < n ? src[i] : -__builtin_huge_valf();
  __syncthreads();
  for (int size = 2; size <= npow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < (npow2 >> 1); t += 256) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const float a = v[lo], b = v[hi];
        // descending sub-sequence when desc: larger first
        if ((a < b) == desc) {
          v[lo] = b;
          v[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  if (threadIdx.x == 0) {
    float c = 0.0f;
    int count = n;
    for (int i = 0; i < n; ++i) {
      c = c + v[i];
      if (c > thr) {
        count = i;
        break;
      }
    }
    out[row] = count > topk ? count : topk;
  }
}

__global__ __launch_bounds__(64) void k_fill_int(int* __restrict__ out, long long n, int value) {
  const long long i = (long long)blockIdx.x * 64 + threadIdx.x;
  if (i < n) out[i] = value;
}

#define RESS_MAX_HEADS 64

// One thread per (batch, q-block) column over H heads. baseline/out are
// [B][H][q_blk] int32 (out may alias baseline). scores_norm [H] fp32 (already
// normalised, or null for the uniform budget). iters_out [B][q_blk] receives the
// number of cap-redistribute iterations, or -1 if max_iters was reached.
// HB >= H is a compile-time bound: the per-head loops unroll over HB with an h < H
// guard, so the head arrays stay in registers and the sums keep their order h = 0..H-1.
template <int HB>
__global__ __launch_bounds__(64) void k_head_budget(const int* baseline, int B, int H, int q_blk,
                                                    const float* __restrict__ scores_norm, float one_minus_beta,
                                                    float beta, int max_val, int max_iters, int min_select,
                                                    int* out, int* __restrict__ iters_out) {
  const int col = blockIdx.x * 64 + threadIdx.x;
  if (col >= B * q_blk) return;
  const int b = col / q_blk, qb = col - b * q_blk;
  const int* base = baseline + (long long)b * H * q_blk + qb;
  int* dst = out + (long long)b * H * q_blk + qb;
  if (scores_norm == nullptr) {
    for (int h = 0; h < H; ++h) {
      const int c = base[(long long)h * q_blk];
      dst[(long long)h * q_blk] = c < min_select ? min_select : c;
    }
    if (iters_out) iters_out[col] = 0;
    return;
  }
  float adj[HB], w[HB];
  int bv[HB];
  long long total = 0;
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    bv[h] = h < H ? base[(long long)h * q_blk] : 0;
    total += bv[h];
  }
  const float total_f = (float)total;
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    const float ideal = h < H ? scores_norm[h] * total_f : 0.0f;
    adj[h] = one_minus_beta * (float)bv[h] + beta * ideal;
  }
  const float maxv = (float)max_val;
  int it = 0;
  for (; it < max_iters; ++it) {
    float esum = 0.0f;
    bool finite = true;
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      if (h < H) {
        const float d = adj[h] - maxv;
        const float ex = d < 0.0f ? 0.0f : d;  // clamp(min=0), NaN kept
        finite = finite && (ex - ex == 0.0f);
        esum = esum + ex;
      }
    }
    if (!finite || !(esum > 0.0f)) break;
    float wsum = 0.0f;
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      if (h < H) {
        adj[h] = adj[h] > maxv ? maxv : adj[h];
        w[h] = adj[h] * (adj[h] < maxv ? 1.0f : 0.0f);
        wsum = wsum + w[h];
      }
    }
    const float den = wsum + 0x1.12e0bep-30f;  // + 1e-9
#pragma unroll
    for (int h = 0; h < HB; ++h)
      if (h < H) adj[h] = adj[h] + (w[h] / den) * esum;
  }
  if (iters_out) iters_out[col] = it < max_iters ? it : -1;
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    if (h < H) {
      const float a = adj[h] > maxv ? maxv : adj[h];
      int c = (int)floorf(a);
      dst[(long long)h * q_blk] = c < min_select ? min_select : c;
    }
  }
}

// Baseline budget for rows [rows][n]: cdf_threshold < 0 disables the CDF cut;
// topk < 0 disables the sparse-ratio floor (at least one must be enabled).
RESS_API int ress_baseline_budget(const void* attn_cond, long long rows, int n, float cdf_threshold, int topk,
                                  void* out_counts, hipStream_t stream) {
  RESS_REQUIRE(rows >= 0 && n > 0, "ress_baseline_budget: bad geometry rows=%lld n=%d", rows, n);
  RESS_REQUIRE(cdf_threshold >= 0.0f || topk >= 0,
               "ress_baseline_budget: at least one of sparse_ratio/cdf_threshold required");
  RESS_REQUIRE(attn_cond && out_counts, "ress_baseline_budget: null pointer");
  if (rows == 0) return 0;
  if (cdf_threshold < 0.0f) {
    hipLaunchKernelGGL(k_fill_int, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, stream, (int*)out_counts, rows,
                       topk);
    RESS_LAUNCHED("k_fill_int");
    return 0;
  }
  int npow2 = 1;
  while (npow2 < n) npow2 <<= 1;
  RESS_REQUIRE(npow2 <= 16384, "ress_baseline_budget: row length %d exceeds 16384", n);
  const float thr = cdf_threshold + 0x1.4f8b58p-17f;  // fp32(tau) + 1e-5
  hipLaunchKernelGGL(k_cdf_count, dim3((unsigned)rows), dim3(256), npow2 * sizeof(float), stream,
                     (const float*)attn_cond, n, npow2, thr, topk, (int*)out_counts);
  RESS_LAUNCHED("k_cdf_count");
  return 0;
}

// HeSS head reallocation + floor. scores_norm null = uniform budget (floor only).
RESS_API int ress_head_budget(const void* baseline, int B, int H, int q_blk, const void* scores_norm, double beta,
                              int max_val, int max_iters, int min_select, void* out_counts, void* iters_out,
                              hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && q_blk > 0, "ress_head_budget: bad geometry");
  RESS_REQUIRE(H <= RESS_MAX_HEADS, "ress_head_budget: H=%d exceeds %d", H, RESS_MAX_HEADS);
  RESS_REQUIRE(baseline && out_counts, "ress_head_budget: null pointer");
  RESS_REQUIRE(max_iters > 0, "ress_head_budget: max_iters must be positive");
  const int cols = B * q_blk;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((cols + 63) / 64), dim3(64), 0, stream, (const int*)baseline, B, H, q_blk,
                       (const float*)scores_norm, (float)(1.0 - beta), (float)beta, max_val, max_iters, min_select,
                       (int*)out_counts, (int*)iters_out);
  };
  if (H <= 8) go(k_head_budget<8>);
  else if (H <= 16) go(k_head_budget<16>);
  else if (H <= 32) go(k_head_budget<32>);
  else go(k_head_budget<RESS_MAX_HEADS>);
  RESS_LAUNCHED("k_head_budget");
  return 0;
}
