// SpargeAttn-convention block map ("meansim"): fused per-block pooling, intra-block
// cosine similarity and INT8 quantisation, then the pooled softmax, CDF budget and map.
//
// Replaces get_block_map_meansim_fuse_quant (SpargeAttn spas_sage_attn/utils.py as the
// reference patches it, external/patches/spargeattn.patch:50-67): attention_sink is a
// count of leading tokens and forces the ceil(sink/64) leading key blocks of every row
// (:63-65); Q is quantised with sm_scale = 1 (:38-41). SpargeAttn is not part of the
// reference, so the orders below are this library's own, written out so that every
// output is a pure function of the inputs:
//
//   per block of n tokens (Q 128, K 64; K minus km when km is given), x_t in fp32:
//     n2_t    = tree8 over dim groups g of fmaf(x, x) chains over dims 8g..8g+7
//     xh_t    = x_t * (n2_t > 0 ? 1/sqrt(n2_t) : 0)
//     pooled  = TSUM(x) / n,  ssum = TSUM(xh), where per dim TSUM over the block's
//               padded token rows (zeros past the sequence end) is: a[r] = the sum of
//               tokens r, r+32, r+64, r+96 in that order (r < 32; Q has 4 terms, K 2),
//               W[w] = tree8(a[8w..8w+7]), TSUM = (W[0] + W[1]) + (W[2] + W[3])
//     sim     = tree8 over g of fmaf chains of ssum^2  /  (n*n)   (the mean pairwise
//               cosine similarity, self pairs included); similar = sim > simthreshd1[h]
//     codes   = the per-block quantiser, scale = amax/127
//   per (head, q-block) row, over the nk key blocks:
//     s_c = DOT64(pooled_q, pooled_k[c]) * 0.125 for similar c, -inf otherwise
//     p_c = ress_expf(s_c - max) / SUM64(e)
//     n   = #{k : S_k <= T}, S_k = the exact (uint64) sum of the k largest q(p_c) =
//           floor(p_c * 2^50), T = floor(min(cdfthreshd[h], 8192) * 2^50); n = 0 when
//           cdfthreshd[h] < 0 (the prefix sums of the sorted p, evaluated exactly at 2^-50
//           resolution, so the count depends on the values alone, not on a summation order)
//     map = the first n of the (p desc, index asc) order | non-similar c | every c of a
//           non-similar row | c < ceil(attention_sink/64)
//
// k_ms_stats: one 256-thread workgroup per (block, batch*head), Q's and K's blocks in one
// launch. Thread (token lane tid>>3, dim group tid&7) loads 8 bf16 per token pass (BS/32
// passes) and keeps them in registers for the sums and the codes; the token-lane sums are
// lane butterflies, and only the 4 waves' partial sums go through LDS.
// k_ms_map_wave (nk <= 1024): one wave per (q-block, batch*head) row, four rows per
// workgroup; details at the kernel.
// k_ms_map_long (nk > 1024): one 256-thread workgroup per row; with a workspace the
// scores come from one matrix-core GEMM over all rows (scores_gemm, DOT64 exactly), else
// each row computes its own.
// Both find n without sorting: an MSB-first radix descent over the bits of p (8-bit
// digits from the highest bit where the row's keys differ) with per-digit counts and
// uint64 sums of q, and the tie rank by index.
#include "common.h"

namespace {

constexpr int MS_MAX_NK = 6144;    // key blocks per row of the map kernels (24 KiB of p, 6 KiB of flags in LDS)
constexpr int MS_CH_LD = 17;       // k_ms_map_long score chunks: 64 columns x 16 dims, odd row stride
constexpr float MS_Q_SCALE = 1125899906842624.0f;  // 2^50: q(p) = floor(p * 2^50)
// One 64-bit histogram word per bin: count << 51 | sum of q. A row's p sum to 1 within
// nk rounding errors (< 1.001 for nk <= MS_MAX_NK), so any bin's q sum stays below 2^51,
// and its count (<= MS_MAX_NK) fits the 13 bits above.
constexpr int MS_PACK_SHIFT = 51;
static_assert(MS_MAX_NK < (1 << (64 - MS_PACK_SHIFT)), "a bin's count fits above its q sum");
// front LDS region of k_ms_map_long: the four waves' score chunks
constexpr size_t MS_LONG_FRONT_BYTES = 4 * 64 * MS_CH_LD * 4;

// the value of lane ^ J (J < 64) for the stats kernel: DPP quad permutes for 1 and 2, a
// bit-mode ds_swizzle (source lane ((l & 31) ^ J) within each 32-lane half) for 4..16, the
// half swap for 32. The stats kernel's VALU is its busiest unit, so its middle exchanges
// stay on the LDS unit (ds_swizzle) rather than in VALU moves (common.h xor_lane).
template <int J>
__device__ __forceinline__ uint32_t ms_xor_lane(uint32_t a, int lane) {
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  } else if constexpr (J < 32) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)a, 0x1F | (J << 10));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);  // {lo,lo}, {hi,hi}
    return lane < 32 ? (uint32_t)r[1] : (uint32_t)r[0];
  }
}

// One butterfly step of the token-lane sums: lanes that differ in bit J of the lane id
// each send the half of their N partial sums that the other keeps, and keep the pairwise
// sums of their own half (the lane with bit J clear keeps the lower half).
template <int J, int N>
__device__ __forceinline__ void ms_halve(float (&v)[N], int lane) {
  const bool hi = (lane & J) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = hi ? v[i] : v[N / 2 + i];
    const float keep = hi ? v[N / 2 + i] : v[i];
    v[i] = keep + __uint_as_float(ms_xor_lane<J>(__float_as_uint(send), lane));
  }
}

// Statistics and codes of one block (BS = 128 query or 64 key tokens) by a 256-thread
// workgroup. Thread (token lane tr = tid>>3, dim group g = tid&7) holds dims 8g..8g+7 of
// tokens tr + 32p (p < BS/32; zeros past the sequence end) in registers. Per dim, the
// sums over tokens are: each thread adds its tokens in p order, the 8 token lanes of a
// wave combine as tree8 (lane bits 3, 4, 5: a reduce-scatter, so each lane ends with 2 of
// the wave's 128 sums), and the 4 waves as (w0 + w1) + (w2 + w3) through LDS.
template <int BS>
__device__ __forceinline__ void ms_stats_block(const uint16_t* __restrict__ x, const Strides& sx, int T,
                                               const float* __restrict__ km, const float* __restrict__ simth, int nb,
                                               int blk, int bh, int8_t* __restrict__ codes, float* __restrict__ scale,
                                               float* __restrict__ pooled, uint8_t* __restrict__ sim,
                                               float (&part_l)[4][2][64], float (&ssum_l)[64], float (&amax_l)[4]) {
  constexpr int PASSES = BS / 32;
  const int tid = threadIdx.x, g = tid & 7, tr = tid >> 3, lane = tid & 63, w = tid >> 6;
  const int base = blk * BS, cnt = min(BS, T - base);
  const uint16_t* xb = x + bh_offset(bh, sx);

  float kmv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) kmv[c] = km ? km[(long long)bh * 64 + 8 * g + c] : 0.0f;
  // every pass's row is loaded before any is used (tokens past the sequence end read the
  // last token's row and become zeros), so the loads are in flight together
  uint4 raw[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
    raw[p] = *reinterpret_cast<const uint4*>(xb + (long long)(base + min(tr + 32 * p, cnt - 1)) * sx.t + 8 * g);
  float xv[PASSES][8];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const bool in = tr + 32 * p < cnt;
    unpack_bf16x8(raw[p], xv[p]);
#pragma unroll
    for (int c = 0; c < 8; ++c) xv[p][c] = in ? xv[p][c] - kmv[c] : 0.0f;
  }
  // token norms (fmaf chain per dim group, tree8 across the token's 8 lanes, which all end
  // with the same sum), then the per-thread sums of x and of x/||x|| in p order
  float acc[16], amax = 0.0f, n2v[PASSES];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    float n2 = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      n2 = fmaf(xv[p][c], xv[p][c], n2);
      amax = fmaxf(amax, fabsf(xv[p][c]));
    }
    n2 = n2 + __uint_as_float(ms_xor_lane<1>(__float_as_uint(n2), lane));
    n2 = n2 + __uint_as_float(ms_xor_lane<2>(__float_as_uint(n2), lane));
    n2v[p] = n2 + __uint_as_float(ms_xor_lane<4>(__float_as_uint(n2), lane));
  }
  // 1/||x|| once per token: lane g of the token's 8 lanes computes it for pass g (g <
  // PASSES), and every pass takes it from there
  float n2own = n2v[0];
#pragma unroll
  for (int p = 1; p < PASSES; ++p)
    if (g == p) n2own = n2v[p];
  const float inv_own = n2own > 0.0f ? 1.0f / sqrtf(n2own) : 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const float inv = __shfl(inv_own, (lane & ~7) | p, 64);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      acc[c] = acc[c] + xv[p][c];
      acc[8 + c] = acc[8 + c] + xv[p][c] * inv;
    }
  }
  ms_halve<8, 16>(acc, lane);
  ms_halve<16, 8>(reinterpret_cast<float(&)[8]>(acc), lane);
  ms_halve<32, 4>(reinterpret_cast<float(&)[4]>(acc), lane);
  {  // acc[0..1]: sums (x if lane bit 3 is clear, else x/||x||) of dims 8g + 4*bit4 + 2*bit5 + {0, 1}
    const int d = 8 * g + 4 * ((lane >> 4) & 1) + 2 * ((lane >> 5) & 1);
    *reinterpret_cast<float2*>(&part_l[w][(lane >> 3) & 1][d]) = make_float2(acc[0], acc[1]);
  }
  amax = wave_max(amax);
  if (lane == 0) amax_l[w] = amax;
  __syncthreads();
  const float bamax = fmaxf(fmaxf(amax_l[0], amax_l[1]), fmaxf(amax_l[2], amax_l[3]));
  const float sc = bamax / 127.0f;
  if (w < 2) {  // wave 0: the pooled mean of dim `lane`; wave 1: the sum of x/||x|| of dim `lane`
    const float s = (part_l[0][w][lane] + part_l[1][w][lane]) + (part_l[2][w][lane] + part_l[3][w][lane]);
    if (w == 0) {
      pooled[((long long)bh * nb + blk) * 64 + lane] = s / (float)cnt;
    } else {
      ssum_l[lane] = s;
      const int gg = lane & 7;
      float q = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) q = fmaf(ssum_l[8 * gg + c], ssum_l[8 * gg + c], q);
      q = q + __shfl_xor(q, 1, 64);
      q = q + __shfl_xor(q, 2, 64);
      q = q + __shfl_xor(q, 4, 64);
      if (lane == 0) {
        const float si = q / ((float)cnt * (float)cnt);
        sim[(long long)bh * nb + blk] = si > simth[bh % sx.H] ? 1 : 0;
        scale[(long long)bh * nb + blk] = sc;
      }
    }
  }
  // codes of the whole padded block (rows past the sequence end hold exact zeros: code 0)
  const float rc = sc != 0.0f ? 1.0f / sc : 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int t = tr + 32 * p;
    int c8[8];
    quant_i8x8_rcp(xv[p], sc, rc, c8);
    *reinterpret_cast<uint2*>(codes + ((long long)bh * nb * BS + base + t) * 64 + 8 * g) = pack_i8x8(c8);
  }
}

// Both operands' blocks in one launch: x = 0..nq-1 are Q's 128-token blocks, nq..nq+nk-1
// K's 64-token blocks (K minus km when km is given).
__global__ __launch_bounds__(256) void k_ms_stats(const uint16_t* __restrict__ q, Strides sq, int Tq,
                                                  const uint16_t* __restrict__ k, Strides sk, int Tk,
                                                  const float* __restrict__ km, const float* __restrict__ simth,
                                                  int nq, int nk, int8_t* __restrict__ q_i8,
                                                  float* __restrict__ q_scale, float* __restrict__ pooled_q,
                                                  uint8_t* __restrict__ sim_q, int8_t* __restrict__ k_i8,
                                                  float* __restrict__ k_scale, float* __restrict__ pooled_k,
                                                  uint8_t* __restrict__ sim_k) {
  __shared__ __align__(16) float part_l[4][2][64];
  __shared__ float ssum_l[64];
  __shared__ float amax_l[4];
  const int bx = blockIdx.x, bh = blockIdx.y;
  if (bx < nq)
    ms_stats_block<128>(q, sq, Tq, nullptr, simth, nq, bx, bh, q_i8, q_scale, pooled_q, sim_q, part_l, ssum_l, amax_l);
  else
    ms_stats_block<64>(k, sk, Tk, km, simth, nk, bx - nq, bh, k_i8, k_scale, pooled_k, sim_k, part_l, ssum_l, amax_l);
}

// One digit of the CDF radix descent, by one wave over the 256 bins (hc counts, hs uint64
// sums of q) of the keys in the current range: bins are taken from the highest down while
// the running total stays <= T. Returns false if every bin fits (above, n_above then
// include them all); otherwise the crossing bin with its count and sum, and above /
// n_above advanced over the bins before it. Every lane gets the same results.
// PACKED: hs[bin] holds count << MS_PACK_SHIFT | sum of q (hc unused).
template <bool PACKED = false>
__device__ __forceinline__ bool ms_cdf_digit(const int* hc, const unsigned long long* hs, unsigned long long T,
                                             unsigned long long& above, int& n_above, int lane, int& bin,
                                             int& bcnt, unsigned long long& bsum) {
  int c4[4];
  unsigned long long s4[4], ls = 0ull;
  int lc = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // lane l: bins 255-4l down to 252-4l
    if constexpr (PACKED) {
      const unsigned long long v = hs[255 - 4 * lane - j];
      c4[j] = (int)(v >> MS_PACK_SHIFT);
      s4[j] = v & ((1ull << MS_PACK_SHIFT) - 1ull);
    } else {
      c4[j] = hc[255 - 4 * lane - j];
      s4[j] = hs[255 - 4 * lane - j];
    }
    ls += s4[j];
    lc += c4[j];
  }
  // inclusive scans over lanes (lane 0 = highest bins)
  const unsigned long long in = wave_scan_sum_u64(ls);
  const int inc = wave_scan_sum_i(lc);
  unsigned long long base = above + (in - ls);
  int basec = n_above + (inc - lc), jx = 4, cx = 0;
  unsigned long long sx = 0ull;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (jx == 4) {
      if (base + s4[j] > T) {
        jx = j;
        cx = c4[j];
        sx = s4[j];
      } else {
        base += s4[j];
        basec += c4[j];
      }
    }
  }
  const unsigned long long has = __ballot(jx < 4);
  if (has == 0ull) {
    above = lane63_u64(base);
    n_above = (int)lane63((uint32_t)basec);
    return false;
  }
  const int src = __ffsll((long long)has) - 1;  // uniform
  bin = 255 - 4 * src - __builtin_amdgcn_readlane(jx, src);
  above = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(base >> 32), src) << 32) |
          (uint32_t)__builtin_amdgcn_readlane((int)base, src);
  n_above = __builtin_amdgcn_readlane(basec, src);
  bcnt = __builtin_amdgcn_readlane(cx, src);
  bsum = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(sx >> 32), src) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)sx, src);
  return true;
}

// The row's CDF cut by one wave: key[e] = bits of p at column 64e + lane (p >= +0, so the
// bits order like the values). Returns n and the n-th largest key (vbits, for n > 0).
// hc / hs: this wave's 256-bin LDS histogram.
template <int E>
__device__ __forceinline__ int ms_cdf_wave(const uint32_t (&key)[E], int nk, float th, int lane, int* hc,
                                           unsigned long long* hs, uint32_t& vbits) {
  vbits = 0u;
  if (!(th >= 0.0f)) return 0;
  const unsigned long long T = (unsigned long long)(fminf(th, 8192.0f) * MS_Q_SCALE);
  unsigned long long q[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    q[e] = 64 * e + lane < nk ? (unsigned long long)(__uint_as_float(key[e]) * MS_Q_SCALE) : 0ull;
  // digits every valid key shares need no histogram: start at the first one that differs
  uint32_t kor = 0u, kand = 0xFFFFFFFFu;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (64 * e + lane < nk) {
      kor |= key[e];
      kand &= key[e];
    }
  kor = wave_or_u32(kor);
  kand = wave_and_u32(kand);
  // The digits start at the highest bit where the keys differ and take 8 bits at a time
  // downward (the last one what is left): a digit aligned to the bytes of the key would
  // put most keys of a row into the few bins of its exponent, and the histogram atomics
  // of one bin serialise.
  const uint32_t diff = kor ^ kand;
  int hi = diff == 0u ? 7 : 31 - __clz((int)diff);  // the next digit's highest bit
  uint32_t pmask = hi >= 31 ? 0u : 0xFFFFFFFFu << (hi + 1);
  uint32_t prefix = kand & pmask;
  unsigned long long above = 0ull, bsum = 0ull;
  int n_above = 0, bcnt = 0;
  bool crossed = true;
  while (hi >= 0) {
    const int shift = max(hi - 7, 0);
    const uint32_t dmask = (2u << (hi - shift)) - 1u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hc[64 * j + lane] = 0;
      hs[64 * j + lane] = 0ull;
    }
    asm volatile("" ::: "memory");  // this wave's LDS accesses stay in program order
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (64 * e + lane < nk && (key[e] & pmask) == prefix) {
        const int b = (key[e] >> shift) & dmask;
        atomicAdd(&hc[b], 1);
        atomicAdd(&hs[b], q[e]);
      }
    }
    asm volatile("" ::: "memory");
    int bin = 0;
    if (!ms_cdf_digit(hc, hs, T, above, n_above, lane, bin, bcnt, bsum)) {
      crossed = false;
      break;
    }
    prefix |= (uint32_t)bin << shift;
    pmask |= dmask << shift;
    hi = shift - 1;
    asm volatile("" ::: "memory");
    if (bcnt == 1) break;  // one key in the crossing bin: it does not fit, and nothing below it
  }
  // every key fits: n = all of them, the n-th largest the smallest; a lone crossing key
  // fits 0 times; otherwise the crossing key's ties (equal p, equal q) fit
  // floor((T - above) / q) times
  const int m = crossed && bcnt > 1 ? (int)((T - above) / (bsum / (unsigned long long)bcnt)) : 0;
  const int n = n_above + m;
  if (crossed && m > 0) {
    vbits = prefix;
  } else {  // the smallest key (all fit), or the smallest above the crossing key's range
    const uint32_t top = prefix | ~pmask;
    uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (64 * e + lane < nk && (!crossed || key[e] > top)) mn = min(mn, key[e]);
    vbits = wave_min_u32(mn);
  }
  return n;
}

// One 256-thread workgroup per (head, q-block) row for nk > 1024:
//  scores  PRE: read from S (the scores_gemm output, [BH][nq][nk], already * 0.125);
//          otherwise wave w scores columns c = 256i + 64w + lane, each lane reading its
//          column's pooled K through the wave's LDS chunk (DOT64 chain, pooled Q in registers).
//  cut     the CDF radix descent over p in LDS (column order): a workgroup histogram per
//          digit, scanned by wave 0 (ms_cdf_digit).
//  select  contiguous column chunks per thread and a workgroup scan for the tie rank.
template <bool PRE>
__global__ __launch_bounds__(256) void k_ms_map_long(const float* __restrict__ pooled_q,
                                                     const float* __restrict__ pooled_k,
                                                     const uint8_t* __restrict__ sim_q,
                                                     const uint8_t* __restrict__ sim_k, int H, int nq, int nk,
                                                     const float* __restrict__ cdfth, int n_sink,
                                                     const float* __restrict__ S, uint8_t* __restrict__ map) {
  extern __shared__ __align__(16) unsigned char ms_dyn[];
  // front region (MS_LONG_FRONT_BYTES, without PRE): the waves' score chunks
  float* scw = reinterpret_cast<float*>(ms_dyn) + (threadIdx.x >> 6) * (64 * MS_CH_LD);  // [64][MS_CH_LD]
  float* p = reinterpret_cast<float*>(ms_dyn + (PRE ? 0 : MS_LONG_FRONT_BYTES));  // [nk] scores -> p, column order
  uint8_t* skl = reinterpret_cast<uint8_t*>(p + nk);  // [nk] the columns' similarity flags, then the map row
  __shared__ float red[4];
  __shared__ int ired[4];
  __shared__ unsigned long long hs[256];  // packed histogram (MS_PACK_SHIFT)
  __shared__ unsigned long long cut_l[2];  // the digit's result: above, then bsum
  __shared__ int cut_i[4];                 // crossed, bin, n_above, bcnt
  __shared__ uint32_t vmin_l;
  __shared__ uint32_t kred[8];  // the waves' OR, then AND, of the keys
  const int r = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint8_t* row = map + ((long long)bh * nq + r) * nk;
  const uint8_t* sk = sim_k + (long long)bh * nk;
  if (!sim_q[(long long)bh * nq + r]) {  // a non-similar query block attends to every key block
    for (int c = tid; c < nk; c += 256) row[c] = 1;
    return;
  }
  float mx = -__builtin_huge_valf();
  if constexpr (PRE) {
    // every load of a batch of eight columns per thread is issued before any is used
    // (columns past nk read column nk - 1 and are dropped)
    const float* srow = S + ((long long)bh * nq + r) * nk;
    for (int cb = 0; cb < nk; cb += 256 * 8) {
      float sv[8];
      uint8_t kv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = min(cb + 256 * u + tid, nk - 1);
        sv[u] = srow[c];
        kv[u] = sk[c];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = cb + 256 * u + tid;
        if (c < nk) {
          if (kv[u]) mx = fmaxf(mx, sv[u]);
          p[c] = kv[u] ? sv[u] : -__builtin_huge_valf();
          skl[c] = kv[u];
        }
      }
    }
  } else {
  float pq[64];
  {
    const float4* q4 = reinterpret_cast<const float4*>(pooled_q + ((long long)bh * nq + r) * 64);
#pragma unroll
    for (int d4 = 0; d4 < 16; ++d4) {
      const float4 x = q4[d4];
      pq[4 * d4] = x.x;
      pq[4 * d4 + 1] = x.y;
      pq[4 * d4 + 2] = x.z;
      pq[4 * d4 + 3] = x.w;
    }
  }
  const float* pkh = pooled_k + (long long)bh * nk * 64;
  // wave w scores columns c0..c0+63 (c0 = 256i + 64w), lane = column: the columns' pooled
  // K goes through the wave's LDS chunk 16 dims at a time (coalesced loads, the next
  // chunk in flight while one is used), and the DOT64 chain runs over d = 0..63 in order
  for (int c0 = 64 * w; c0 < nk; c0 += 256) {
    const int c = c0 + lane;
    const bool live = c < nk && sk[c];
    float4 ld[4];
    auto load_chunk = [&](int q) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int f = 64 * t + lane, col = c0 + (f >> 2);
        ld[t] = col < nk ? *reinterpret_cast<const float4*>(pkh + (long long)col * 64 + 16 * q + 4 * (f & 3))
                         : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    };
    load_chunk(0);
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int f = 64 * t + lane;
        float* dst = scw + (f >> 2) * MS_CH_LD + 4 * (f & 3);
        dst[0] = ld[t].x;
        dst[1] = ld[t].y;
        dst[2] = ld[t].z;
        dst[3] = ld[t].w;
      }
      __builtin_amdgcn_wave_barrier();
      if (q + 1 < 4) load_chunk(q + 1);
      const float* kc = scw + lane * MS_CH_LD;
#pragma unroll
      for (int d = 0; d < 16; ++d) a = fmaf(pq[16 * q + d], kc[d], a);
      __builtin_amdgcn_wave_barrier();  // every lane has read the chunk before it is overwritten
    }
    if (c < nk) {
      float s = -__builtin_huge_valf();
      if (live) {
        s = a * 0.125f;
        mx = fmaxf(mx, s);
      }
      p[c] = s;
      skl[c] = live ? 1 : 0;
    }
  }
  }  // PRE
  mx = wave_max(mx);
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (!(mx > -__builtin_huge_valf())) {  // no similar key block: every block is forced on
    for (int c = tid; c < nk; c += 256) row[c] = 1;
    return;
  }
  for (int c = tid; c < nk; c += 256) p[c] = skl[c] ? ress_expf(p[c] - mx) : 0.0f;
  __syncthreads();
  if (w == 0) {  // lane l adds columns l, l + 64, ... in order; eight reads in flight
    float a = 0.0f;
    int i = lane;
    for (; i + 448 < nk; i += 512) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p[i + 64 * u];
#pragma unroll
      for (int u = 0; u < 8; ++u) a = a + v[u];
    }
    for (; i < nk; i += 64) a = a + p[i];
    a = sum64_tree(a);
    if (lane == 0) red[0] = a;
  }
  __syncthreads();
  const float tot = red[0];
  for (int c = tid; c < nk; c += 256) p[c] = p[c] / tot;
  __syncthreads();
  // the CDF cut: p >= +0, so its bits order like the value (ms_cdf_wave has the steps)
  int n = 0;
  uint32_t vbits = 0u;
  const float th = cdfth[bh % H];
  if (th >= 0.0f) {
    const unsigned long long T = (unsigned long long)(fminf(th, 8192.0f) * MS_Q_SCALE);
    // the digits start at the highest bit where the row's keys differ and take 8 bits at a
    // time downward (as in ms_cdf_wave)
    uint32_t kor = 0u, kand = 0xFFFFFFFFu;
    for (int c = tid; c < nk; c += 256) {
      const uint32_t b = __float_as_uint(p[c]);
      kor |= b;
      kand &= b;
    }
    kor = wave_or_u32(kor);
    kand = wave_and_u32(kand);
    if (lane == 0) {
      kred[w] = kor;
      kred[4 + w] = kand;
    }
    __syncthreads();
    kor = (kred[0] | kred[1]) | (kred[2] | kred[3]);
    kand = (kred[4] & kred[5]) & (kred[6] & kred[7]);
    const uint32_t diff = kor ^ kand;
    int hi = diff == 0u ? 7 : 31 - __clz((int)diff);  // the next digit's highest bit
    uint32_t pmask = hi >= 31 ? 0u : 0xFFFFFFFFu << (hi + 1);
    uint32_t prefix = kand & pmask;
    unsigned long long above = 0ull, bsum = 0ull;
    int n_above = 0, bcnt = 0;
    bool crossed = true;
    while (hi >= 0) {
      const int shift = max(hi - 7, 0);
      const uint32_t dmask = (2u << (hi - shift)) - 1u;
      hs[tid] = 0ull;
      __syncthreads();
      for (int c = tid; c < nk; c += 256) {
        const uint32_t b = __float_as_uint(p[c]);
        if ((b & pmask) == prefix)
          atomicAdd(&hs[(b >> shift) & dmask],
                    (1ull << MS_PACK_SHIFT) | (unsigned long long)(__uint_as_float(b) * MS_Q_SCALE));
      }
      __syncthreads();
      if (w == 0) {
        int bin = 0;
        const bool x = ms_cdf_digit<true>(nullptr, hs, T, above, n_above, lane, bin, bcnt, bsum);
        if (lane == 0) {
          cut_i[0] = x;
          cut_i[1] = bin;
          cut_i[2] = n_above;
          cut_i[3] = bcnt;
          cut_l[0] = above;
          cut_l[1] = bsum;
        }
      }
      __syncthreads();
      crossed = cut_i[0] != 0;
      n_above = cut_i[2];
      bcnt = cut_i[3];
      above = cut_l[0];
      bsum = cut_l[1];
      if (!crossed) break;
      prefix |= (uint32_t)cut_i[1] << shift;
      pmask |= dmask << shift;
      hi = shift - 1;
      if (bcnt == 1) break;  // one key in the crossing bin: it does not fit, and nothing below it
    }
    const int m = crossed && bcnt > 1 ? (int)((T - above) / (bsum / (unsigned long long)bcnt)) : 0;
    n = n_above + m;
    if (crossed && m > 0) {
      vbits = prefix;
    } else {  // the smallest key (every key fits) or the smallest above the crossing key's range
      if (tid == 0) vmin_l = 0xFFFFFFFFu;
      const uint32_t top = prefix | ~pmask;
      uint32_t mn = 0xFFFFFFFFu;
      for (int c = tid; c < nk; c += 256) {
        const uint32_t b = __float_as_uint(p[c]);
        if (!crossed || b > top) mn = min(mn, b);
      }
      mn = wave_min_u32(mn);
      __syncthreads();
      if (lane == 0) atomicMin(&vmin_l, mn);
      __syncthreads();
      vbits = vmin_l;
    }
  }
  // contiguous column chunks: p > v is kept; of the p == v columns, the lowest-indexed
  // n - #{p > v} (an exclusive scan of the per-chunk counts gives each one's rank)
  const int chunk = cdiv(nk, 256), c0 = min(nk, tid * chunk), c1 = min(nk, c0 + chunk);
  int gt = 0, eq = 0;
  for (int c = c0; c < c1; ++c) {
    const uint32_t b = __float_as_uint(p[c]);
    gt += b > vbits ? 1 : 0;
    eq += b == vbits ? 1 : 0;
  }
  const int incl = wave_scan_sum_i(eq);  // inclusive scan of eq over the wave, in thread order
  const int gsum = wave_sum_i(gt);
  if (lane == 63) ired[w] = incl;
  if (lane == 0) red[w] = __int_as_float(gsum);
  __syncthreads();
  int before = 0, n_gt = 0;
  for (int i = 0; i < 4; ++i) {
    if (i < w) before += ired[i];
    n_gt += __float_as_int(red[i]);
  }
  int rank_eq = before + incl - eq;
  const int take_eq = n - n_gt;
  for (int c = c0; c < c1; ++c) {
    const uint32_t b = __float_as_uint(p[c]);
    bool sel = false;
    if (n > 0) {
      if (b > vbits) {
        sel = true;
      } else if (b == vbits) {
        sel = rank_eq < take_eq;
        ++rank_eq;
      }
    }
    skl[c] = (sel || !skl[c] || c < n_sink) ? 1 : 0;  // column c is this thread's alone
  }
  __syncthreads();
  for (int c = tid; c < nk; c += 256) row[c] = skl[c];  // coalesced
}

// One wave per (head, q-block) row, E = 64-key-block columns per lane (nk <= 64E), four
// rows of one head per workgroup.
//  scores  pooled K goes through LDS in coalesced 64-block tiles that the four rows
//          share; lane l keeps the scores of columns c = 64e + l (also the SUM64 order).
//  cut     n and the n-th largest p by the CDF radix descent (ms_cdf_wave), each wave on
//          its own LDS histogram: no sort, no cross-wave step after the scores.
//  select  with v the n-th largest probability: every column with p > v, and of those
//          with p == v the lowest-indexed ones up to n (a ballot prefix count).
template <int E>
__global__ __launch_bounds__(256) void k_ms_map_wave(const float* __restrict__ pooled_q,
                                                     const float* __restrict__ pooled_k,
                                                     const uint8_t* __restrict__ sim_q,
                                                     const uint8_t* __restrict__ sim_k, int H, int nq, int nk,
                                                     const float* __restrict__ cdfth, int n_sink,
                                                     uint8_t* __restrict__ map) {
  constexpr int LDK = 68;  // row stride of a pooled-K tile: 16-byte rows, 8 consecutive columns in distinct banks
  constexpr int LDQ = 68;  // row stride of the pooled-Q rows
  constexpr int TB = 64 * LDK;
  // two pooled-K tiles; once the scores are done the same LDS holds the per-wave CDF digit
  // histograms (counts, then uint64 sums)
  __shared__ __align__(16) float pk_l[2 * TB];
  __shared__ __align__(16) float pq_l[4 * LDQ];
  __shared__ float sc_l[4][128];  // one pass's scores, row-major
  int(*hc_l)[256] = reinterpret_cast<int(*)[256]>(pk_l);
  unsigned long long(*hs_l)[256] = reinterpret_cast<unsigned long long(*)[256]>(pk_l + 4 * 256);
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.y, r = blockIdx.x * 4 + w;
  const long long row_id = (long long)bh * nq + r;
  const bool in_range = r < nq;
  const bool active = in_range && sim_q[row_id];
  const float pq = in_range ? pooled_q[row_id * 64 + lane] : 0.0f;
  const float* pkh = pooled_k + (long long)bh * nk * 64;
  const uint8_t* sk = sim_k + (long long)bh * nk;
  // the similarity flags of the lane's columns (0 past nk) and the row's threshold, loaded
  // now so that their latency overlaps the scores
  uint8_t skc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) skc[e] = 64 * e + lane < nk ? sk[64 * e + lane] : 0;
  const float th = cdfth[bh % H];

  // Passes of two 64-key-block tiles; pass p+1 is loaded into registers while pass p is
  // computed. Lane l of wave w scores row l/16 of the workgroup against column 16w + l%16
  // of both tiles (two independent DOT64 chains, each over d = 0..63 in order), so the
  // four rows share every pooled-K read; sc_l turns the scores back to one row per wave,
  // one column per lane.
  const int srow = lane >> 4, scol = 16 * w + (lane & 15);
  float s[E];
#pragma unroll
  for (int e = 0; e < E; ++e) s[e] = 0.0f;
  const int passes = cdiv(cdiv(nk, 64), 2);
  float4 nxt[8];
  auto load_pass = [&](int pp) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = 2 * pp + (i >> 2), cols = min(64, nk - 64 * t);  // cols <= 0: no such tile
      const int f4 = tid + 256 * (i & 3), col = f4 >> 4;
      nxt[i] = col < cols ? reinterpret_cast<const float4*>(pkh + (long long)(64 * t + col) * 64)[f4 & 15]
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  load_pass(0);  // in flight together with the loads above
  pq_l[w * LDQ + lane] = pq;
#pragma unroll 1
  for (int pp = 0; pp < passes; ++pp) {
    __syncthreads();  // previous pass consumed (and pq_l written, first time)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f4 = tid + 256 * (i & 3);
      *reinterpret_cast<float4*>(pk_l + (i >> 2) * TB + (f4 >> 4) * LDK + (f4 & 15) * 4) = nxt[i];
    }
    __syncthreads();
    if (pp + 1 < passes) load_pass(pp + 1);
    {
      const float4* qv = reinterpret_cast<const float4*>(pq_l + srow * LDQ);
      const float4* k0 = reinterpret_cast<const float4*>(pk_l + scol * LDK);
      const float4* k1 = reinterpret_cast<const float4*>(pk_l + TB + scol * LDK);
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        const float4 qq = qv[d4], x0 = k0[d4], x1 = k1[d4];
        a0 = fmaf(qq.x, x0.x, a0);
        a1 = fmaf(qq.x, x1.x, a1);
        a0 = fmaf(qq.y, x0.y, a0);
        a1 = fmaf(qq.y, x1.y, a1);
        a0 = fmaf(qq.z, x0.z, a0);
        a1 = fmaf(qq.z, x1.z, a1);
        a0 = fmaf(qq.w, x0.w, a0);
        a1 = fmaf(qq.w, x1.w, a1);
      }
      sc_l[srow][scol] = a0;
      sc_l[srow][64 + scol] = a1;
    }
    __syncthreads();
    const float b0 = sc_l[w][lane], b1 = sc_l[w][64 + lane];
    if (active) {
#pragma unroll
      for (int e2 = 0; e2 < E; ++e2) {
        if (64 * e2 + lane < nk && e2 == 2 * pp) s[e2] = b0;
        if (64 * e2 + lane < nk && e2 == 2 * pp + 1) s[e2] = b1;
      }
    }
  }

  bool simc[E];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int e = 0; e < E; ++e) {
    simc[e] = skc[e] != 0;
    s[e] = s[e] * 0.125f;
    if (simc[e]) mx = fmaxf(mx, s[e]);
  }
  mx = wave_max(mx);
  // the CDF path runs for a similar row with at least one similar key block; otherwise
  // every block of the row is on
  const bool go = active && mx > -__builtin_huge_valf();
  if (!in_range) return;
  uint8_t* row = map + row_id * nk;
  if (!go) {
    for (int c = lane; c < nk; c += 64) row[c] = 1;
    return;
  }
  float part = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    s[e] = simc[e] ? ress_expf(s[e] - mx) : 0.0f;
    if (64 * e + lane < nk) part = part + s[e];
  }
  const float tot = sum64_tree(part);
  uint32_t pb[E];  // bits of p at the lane's own columns (p >= +0: bits order like values)
#pragma unroll
  for (int e = 0; e < E; ++e) pb[e] = __float_as_uint(s[e] / tot);
  uint32_t vbits;
  const int n = ms_cdf_wave<E>(pb, nk, th, lane, hc_l[w], hs_l[w], vbits);
  int n_gt = 0;
  if (n > 0) {
    int gt = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) gt += (64 * e + lane < nk && pb[e] > vbits) ? 1 : 0;
    n_gt = wave_sum_i(gt);
  }
  int eq_before = 0;  // equal-to-v columns at lower indices, accumulated over slots
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = 64 * e + lane;
    const bool eq = n > 0 && c < nk && pb[e] == vbits;
    const unsigned long long m = __ballot(eq);
    const int rank_eq = eq_before + __popcll(m & lt_mask);
    eq_before += __popcll(m);
    const bool sel = n > 0 && c < nk && (pb[e] > vbits || (eq && rank_eq < n - n_gt));
    if (c < nk) row[c] = (sel || !skc[e] || c < n_sink) ? 1 : 0;
  }
}

}  // namespace

// Bytes of the optional workspace of ress_meansim_block_map: the fp32 scores of every row
// when rows are long (nk > 1024), else 0 (the short-row kernel keeps them on chip).
RESS_API long long ress_meansim_workspace_size(int B, int H, int Tq, int Tk) {
  const long long nq = cdiv(Tq, 128), nk = cdiv(Tk, 64);
  return B > 0 && H > 0 && nk > 1024 ? (long long)B * H * nq * nk * 4 : 0;
}

// get_block_map_meansim_fuse_quant (patched SpargeAttn, external/patches/spargeattn.patch:50-67)
RESS_API int ress_meansim_block_map(const void* q, const void* k, const void* km, int B, int H, int Tq, int Tk,
                                    long long sqB, long long sqH, long long sqT, long long skB, long long skH,
                                    long long skT, const void* simthreshd1, const void* cdfthreshd,
                                    int attention_sink, void* map, void* q_i8, void* q_scale, void* k_i8,
                                    void* k_scale, void* pooled_q, void* pooled_k, void* sim_q, void* sim_k,
                                    void* workspace, long long workspace_bytes, hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && Tq > 0 && Tk > 0, "ress_meansim_block_map: bad geometry B=%d H=%d Tq=%d Tk=%d", B,
               H, Tq, Tk);
  RESS_REQUIRE(attention_sink >= 0, "ress_meansim_block_map: attention_sink=%d < 0", attention_sink);
  RESS_REQUIRE(q && k && simthreshd1 && cdfthreshd && map && q_i8 && q_scale && k_i8 && k_scale && pooled_q &&
                   pooled_k && sim_q && sim_k,
               "ress_meansim_block_map: null pointer");
  RESS_REQUIRE(((uintptr_t)q & 15u) == 0 && ((uintptr_t)k & 15u) == 0 && sqT % 8 == 0 && skT % 8 == 0 &&
                   sqB % 8 == 0 && sqH % 8 == 0 && skB % 8 == 0 && skH % 8 == 0,
               "ress_meansim_block_map: q/k rows must be 16-byte aligned with unit stride over the 64 dims");
  RESS_REQUIRE(((uintptr_t)pooled_q & 15u) == 0 && ((uintptr_t)pooled_k & 15u) == 0 && ((uintptr_t)q_i8 & 7u) == 0 &&
                   ((uintptr_t)k_i8 & 7u) == 0,
               "ress_meansim_block_map: pooled buffers must be 16-byte and code buffers 8-byte aligned");
  const int nq = cdiv(Tq, 128), nk = cdiv(Tk, 64), BH = B * H;
  RESS_REQUIRE(nk <= MS_MAX_NK, "ress_meansim_block_map: %d key blocks exceed %d", nk, MS_MAX_NK);
  RESS_REQUIRE(!workspace || (workspace_bytes >= ress_meansim_workspace_size(B, H, Tq, Tk) &&
                              ((uintptr_t)workspace & 15u) == 0),
               "ress_meansim_block_map: workspace of %lld bytes is smaller than %lld or not 16-byte aligned",
               workspace_bytes, ress_meansim_workspace_size(B, H, Tq, Tk));
  const Strides sq{sqB, sqH, sqT, H}, sk{skB, skH, skT, H};
  hipLaunchKernelGGL(k_ms_stats, dim3(nq + nk, BH), dim3(256), 0, stream, (const uint16_t*)q, sq, Tq,
                     (const uint16_t*)k, sk, Tk, (const float*)km, (const float*)simthreshd1, nq, nk, (int8_t*)q_i8,
                     (float*)q_scale, (float*)pooled_q, (uint8_t*)sim_q, (int8_t*)k_i8, (float*)k_scale,
                     (float*)pooled_k, (uint8_t*)sim_k);
  RESS_LAUNCHED("k_ms_stats");
  const int n_sink = attention_sink > 0 ? cdiv(attention_sink, 64) : 0;
  const dim3 wgrid(cdiv(nq, 4), BH);
  const float* pq = (const float*)pooled_q;
  const float* pk = (const float*)pooled_k;
  const uint8_t *sq8 = (const uint8_t*)sim_q, *sk8 = (const uint8_t*)sim_k;
  const float* cd = (const float*)cdfthreshd;
  uint8_t* m8 = (uint8_t*)map;
  if (nk <= 64) {
    hipLaunchKernelGGL(k_ms_map_wave<1>, wgrid, dim3(256), 0, stream, pq, pk, sq8, sk8, H, nq, nk, cd, n_sink, m8);
  } else if (nk <= 128) {
    hipLaunchKernelGGL(k_ms_map_wave<2>, wgrid, dim3(256), 0, stream, pq, pk, sq8, sk8, H, nq, nk, cd, n_sink, m8);
  } else if (nk <= 256) {
    hipLaunchKernelGGL(k_ms_map_wave<4>, wgrid, dim3(256), 0, stream, pq, pk, sq8, sk8, H, nq, nk, cd, n_sink, m8);
  } else if (nk <= 512) {
    hipLaunchKernelGGL(k_ms_map_wave<8>, wgrid, dim3(256), 0, stream, pq, pk, sq8, sk8, H, nq, nk, cd, n_sink, m8);
  } else if (nk <= 1024) {
    hipLaunchKernelGGL(k_ms_map_wave<16>, wgrid, dim3(256), 0, stream, pq, pk, sq8, sk8, H, nq, nk, cd, n_sink, m8);
  } else {
    if (workspace) {
      const int rc = scores_gemm(pq, pk, BH, nq, nk, 0, nq, 0.125f, (float*)workspace, stream);
      if (rc) return rc;
      hipLaunchKernelGGL(k_ms_map_long<true>, dim3(nq, BH), dim3(256), (size_t)nk * 5, stream, pq, pk, sq8, sk8, H,
                         nq, nk, cd, n_sink, (const float*)workspace, m8);
    } else {
      hipLaunchKernelGGL(k_ms_map_long<false>, dim3(nq, BH), dim3(256), MS_LONG_FRONT_BYTES + (size_t)nk * 5, stream,
                         pq, pk, sq8, sk8, H, nq, nk, cd, n_sink, (const float*)nullptr, m8);
    }
  }
  RESS_LAUNCHED("k_ms_map");
  return 0;
}
