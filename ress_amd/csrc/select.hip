// Block selection: per-row top-n mask, sink columns, and the kept-block list (LUT)
// the attention kernel walks.
//
// Replaces build_block_mask (reference src/ress/models/attention.py:147-174: sort desc,
// fill_block_map_triton, append sink_blocks all-True columns), SpargeAttn's
// block_map_lut_triton (attention.py:224) and the leading attention_sink forcing of
// external/patches/spargeattn.patch:61-65.
//
// Selection order is (value descending, index ascending): the kept set of a row is
// the n largest keys, ties at the threshold going to the lowest column index, the
// rule of the reference's top-m kernel (src/ress/scoring/fused_topm.py:74-79).
// The n-th largest key is found exactly by an MSB-first radix select (four 8-bit
// digits) over the order-preserving uint32 image of the fp32 key.
#include <type_traits>

#include "common.h"

// Kept columns of one row -> LUT (ascending) + count, one wave. keep(c) is evaluated
// by the caller-provided functor for c in [0, ncol).
template <typename F>
__device__ __forceinline__ int write_lut(F keep, int ncol, int* __restrict__ lut) {
  const int lane = threadIdx.x;
  int pos = 0;
  for (int c0 = 0; c0 < ncol; c0 += 64) {
    const int c = c0 + lane;
    const bool k = c < ncol && keep(c);
    const unsigned long long mask = __ballot(k);
    if (k) lut[pos + __popcll(mask & ((1ull << lane) - 1ull))] = c;
    pos += __popcll(mask);
  }
  return pos;
}

// grid (q_blk_total, BH), SEL_WAVES waves per row (four from 1024 candidates, else one). Rows qb < q_blk_sel select from
// rank_key [BH][q_blk_sel][n_cand] the top max(counts, min_select) (at most n_cand)
// entries, counts [BH][q_blk_sel] int32; rows past q_blk_sel are dense (every column
// kept). Column c of the kernel key grid (kb_tot columns) is kept if
//   c <  n_cand: selected, or c < sink_lead
//   c >= n_cand: always (trailing sink / special blocks)
// map [BH][q_blk_sel][kb_tot] uint8 (may be null), lut [BH][q_blk_total][kb_tot],
// nvalid [BH][q_blk_total]. The row's keys are shared by the workgroup's waves: each
// histogram pass and the count of keys above the threshold split the keys over all
// threads; ties are taken in index order with each wave owning a contiguous run of
// 64-key chunks and starting from the tie count of the waves before it.
template <int SEL_WAVES>
__global__ __launch_bounds__(64 * SEL_WAVES) void k_select(const float* __restrict__ rank_key,
                                                           const int* __restrict__ counts, int q_blk_sel,
                                                           int q_blk_total, int n_cand, int kb_tot, int sink_lead,
                                                           int min_select, uint8_t* __restrict__ map,
                                                           int* __restrict__ lut, int* __restrict__ nvalid) {
  extern __shared__ uint32_t key[];  // n_cand order keys, then reused for the kept flags
  __shared__ int hist[256];
  __shared__ int pick[3];
  __shared__ int wcnt[2][SEL_WAVES];
  const int qb = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int NT = 64 * SEL_WAVES;
  const long long lrow = (long long)bh * q_blk_total + qb;
  int* lrow_p = lut + lrow * kb_tot;
  if (qb >= q_blk_sel) {
    if (w == 0) {
      const int n = write_lut([](int) { return true; }, kb_tot, lrow_p);
      if (lane == 0) nvalid[lrow] = n;
    }
    return;
  }
  const long long srow = (long long)bh * q_blk_sel + qb;
  const float* src = rank_key + srow * n_cand;
  for (int i = tid; i < n_cand; i += NT) key[i] = order_key(src[i]);
  int n = counts[srow];
  n = n < min_select ? min_select : n;  // clamp(min=min(2, n_cand)), attention.py:525
  n = n < 0 ? 0 : (n > n_cand ? n_cand : n);
  __syncthreads();
  // thr = the n-th largest key (n = 0: all ones, nothing above it). MSB-first radix
  // select: among the keys matching the digits fixed so far, an 8-bit histogram of the
  // next digit; the digit holding the rank-th largest (rank counted from the top) is
  // fixed and the keys above it leave the count.
  uint32_t thr = ~0u;
  if (n > 0) {
    uint32_t prefix = 0u, pmask = 0u;
    int rank = n;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int bin = tid; bin < 256; bin += NT) hist[bin] = 0;
      __syncthreads();
      for (int i = tid; i < n_cand; i += NT) {
        const uint32_t kv = key[i];
        if ((kv & pmask) == prefix) atomicAdd(&hist[(kv >> shift) & 255u], 1);
      }
      __syncthreads();
      if (w == 0) {
        // lane l owns bins 4l..4l+3; above = matching keys in bins > 4l+3
        const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
        const int own = h0 + h1 + h2 + h3;
        const int incl = wave_scan_sum_i(own);
        const int total = (int)lane63((uint32_t)incl);
        int above = total - incl;
        const int hv[4] = {h0, h1, h2, h3};
#pragma unroll
        for (int t = 3; t >= 0; --t) {
          if (above < rank && above + hv[t] >= rank) {
            pick[0] = 4 * lane + t;
            pick[1] = rank - above;
            pick[2] = rank - above == hv[t];  // the whole bin is taken
          }
          above += hv[t];
        }
      }
      __syncthreads();
      prefix |= (uint32_t)pick[0] << shift;
      pmask |= 255u << shift;
      rank = pick[1];
      // every key of the bin is taken: with the lower digits left zero, the keys above
      // thr plus the ties at thr are exactly the bin's keys and those above it, the set
      // the remaining digits would select, so they are skipped
      if (pick[2]) break;
    }
    thr = prefix;
  }
  // keys above thr, and ties per wave run, over the workgroup
  const int nchunk = cdiv(n_cand, 64), per = cdiv(nchunk, SEL_WAVES);
  const int c_lo = 64 * per * w, c_hi = min(n_cand, 64 * per * (w + 1));
  int ngt = 0, neq = 0;
  for (int i = c_lo + lane; i < c_hi; i += 64) {
    const uint32_t kv = key[i];
    ngt += kv > thr ? 1 : 0;
    neq += kv == thr ? 1 : 0;
  }
  ngt = wave_sum_i(ngt);
  neq = wave_sum_i(neq);
  if (lane == 0) {
    wcnt[0][w] = ngt;
    wcnt[1][w] = neq;
  }
  __syncthreads();
  int n_gt = 0, eq_before = 0;
#pragma unroll
  for (int v = 0; v < SEL_WAVES; ++v) {
    n_gt += wcnt[0][v];
    eq_before += v < w ? wcnt[1][v] : 0;
  }
  int need = n - n_gt - eq_before;  // ties this wave may still take, lowest index first
  for (int c0 = c_lo; c0 < c_hi; c0 += 64) {
    const int i = c0 + lane;
    const bool valid = i < c_hi;
    const uint32_t kv = valid ? key[i] : 0u;
    const bool eq = valid && kv == thr;
    const unsigned long long em = __ballot(eq);
    const int r = __popcll(em & ((1ull << lane) - 1ull));
    if (valid) key[i] = (kv > thr || (eq && r < need)) ? 1u : 0u;
    need -= __popcll(em);
  }
  __syncthreads();
  auto keepf = [&](int c) { return c >= n_cand || c < sink_lead || key[c] != 0u; };
  if (map) {
    uint8_t* mrow = map + srow * kb_tot;
    for (int c = tid; c < kb_tot; c += NT) mrow[c] = keepf(c) ? 1 : 0;
  }
  if (w == 0) {
    const int nv = write_lut(keepf, kb_tot, lrow_p);
    if (lane == 0) nvalid[lrow] = nv;
  }
}

// map[row, sorted_idx[row, :n[row]]] = 1 (SpargeAttn fill_block_map_triton,
// reference attention.py:168). map [rows][k] uint8 (pre-zeroed by the caller),
// sorted_idx [rows][k] int64, counts [rows] int64.
__global__ __launch_bounds__(64) void k_fill_block_map(uint8_t* __restrict__ map, const long long* __restrict__ counts,
                                                       const long long* __restrict__ sorted_idx, int k) {
  const long long row = blockIdx.x;
  long long n = counts[row];
  n = n < 0 ? 0 : (n > k ? k : n);
  for (int i = threadIdx.x; i < n; i += 64) {
    const long long c = sorted_idx[row * k + i];
    if (c >= 0 && c < k) map[row * k + c] = 1;
  }
}

// map [rows][k] uint8 -> lut [rows][k] int32 (ascending kept columns) + nvalid [rows]
__global__ __launch_bounds__(64) void k_map_to_lut(const uint8_t* __restrict__ map, int k, int* __restrict__ lut,
                                                   int* __restrict__ nvalid) {
  const long long row = blockIdx.x;
  const uint8_t* m = map + row * k;
  const int n = write_lut([&](int c) { return m[c] != 0; }, k, lut + row * k);
  if (threadIdx.x == 0) nvalid[row] = n;
}

RESS_API int ress_select_blocks(const void* rank_key, const void* counts, int BH, int q_blk_sel, int q_blk_total,
                                int n_cand, int kb_tot, int sink_lead, int min_select, void* map, void* lut,
                                void* nvalid, hipStream_t stream) {
  RESS_REQUIRE(BH > 0 && q_blk_sel >= 0 && q_blk_total >= q_blk_sel && q_blk_total > 0,
               "ress_select_blocks: bad row geometry");
  RESS_REQUIRE(n_cand >= 0 && kb_tot >= n_cand && kb_tot > 0 && sink_lead >= 0,
               "ress_select_blocks: bad column geometry n_cand=%d kb_tot=%d", n_cand, kb_tot);
  RESS_REQUIRE(kb_tot <= 16384, "ress_select_blocks: kb_tot=%d exceeds 16384", kb_tot);
  RESS_REQUIRE(lut && nvalid && (q_blk_sel == 0 || (rank_key && counts)), "ress_select_blocks: null pointer");
  auto go = [&](auto waves) {
    constexpr int W = decltype(waves)::value;
    hipLaunchKernelGGL(k_select<W>, dim3(q_blk_total, BH), dim3(64 * W), (n_cand > 0 ? n_cand : 1) * sizeof(uint32_t),
                       stream, (const float*)rank_key, (const int*)counts, q_blk_sel, q_blk_total, n_cand, kb_tot,
                       sink_lead, min_select, (uint8_t*)map, (int*)lut, (int*)nvalid);
  };
  if (n_cand >= 1024) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, 1>{});
  RESS_LAUNCHED("k_select");
  return 0;
}

RESS_API int ress_fill_block_map(void* map, const void* counts, const void* sorted_idx, long long rows, int k,
                                 hipStream_t stream) {
  RESS_REQUIRE(rows >= 0 && k > 0, "ress_fill_block_map: bad geometry");
  RESS_REQUIRE(map && counts && sorted_idx, "ress_fill_block_map: null pointer");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_fill_block_map, dim3((unsigned)rows), dim3(64), 0, stream, (uint8_t*)map,
                     (const long long*)counts, (const long long*)sorted_idx, k);
  RESS_LAUNCHED("k_fill_block_map");
  return 0;
}

RESS_API int ress_block_map_lut(const void* map, long long rows, int k, void* lut, void* nvalid, hipStream_t stream) {
  RESS_REQUIRE(rows >= 0 && k > 0, "ress_block_map_lut: bad geometry");
  RESS_REQUIRE(map && lut && nvalid, "ress_block_map_lut: null pointer");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_map_to_lut, dim3((unsigned)rows), dim3(64), 0, stream, (const uint8_t*)map, k, (int*)lut,
                     (int*)nvalid);
  RESS_LAUNCHED("k_map_to_lut");
  return 0;
}
