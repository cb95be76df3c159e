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
//     n   = #{prefix sums (SEQ) of p in (p desc, index asc) order that are <= cdfthreshd[h]}
//     map = the first n of that order | non-similar c | every c of a non-similar row
//           | c < ceil(attention_sink/64)
//
// k_ms_stats: one 256-thread workgroup per (block, batch*head), Q's and K's blocks in one
// launch. Thread (token lane tid>>3, dim group tid&7) loads 8 bf16 per token pass (BS/32
// passes) and keeps them in registers for the sums and the codes; the token-lane sums are
// lane butterflies, and only the 4 waves' partial sums go through LDS.
// k_ms_map_wave (nk <= 1024): one wave per (q-block, batch*head) row, four rows per
// workgroup; details at the kernel.
// k_ms_map_long (nk > 1024): one 256-thread workgroup per row: the same value sort with
// the keys in registers (cross-wave stages through LDS), one lane's CDF chain, and the
// tie rank by a workgroup scan.
#include "common.h"

namespace {

constexpr int MS_MAX_NK = 6144;    // key blocks per row of the map kernels (<= 32 KiB keys + 24 KiB p in LDS)
constexpr int MS_CH_LD = 17;       // k_ms_map_long score chunks: 64 columns x 16 dims, odd row stride
// front LDS region of k_ms_map_long: the NP2 sort keys, or the four waves' score chunks
__host__ __device__ constexpr size_t ms_long_front_bytes(int np2) {
  return (size_t)np2 * 4 > 4 * 64 * MS_CH_LD * 4 ? (size_t)np2 * 4 : 4 * 64 * MS_CH_LD * 4;
}

// Bitonic network of k_ms_map_long over sort positions i = 64E*w + 64e + lane (lane
// (w, lane) holds u[e]), stages as compile-time (K, J) so every register index is static:
// J >= 64E pairs positions of two waves (through LDS), 64 <= J < 64E two registers of a
// lane, J < 64 two lanes (shuffle).
// the value of lane ^ J (J < 64): DPP quad permutes for 1 and 2, a bit-mode ds_swizzle
// (source lane ((l & 31) ^ J) within each 32-lane half) for 4..16, the half swap for 32
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
  float xv[PASSES][8];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int t = tr + 32 * p;
    uint4 r = make_uint4(0u, 0u, 0u, 0u);
    if (t < cnt) r = *reinterpret_cast<const uint4*>(xb + (long long)(base + t) * sx.t + 8 * g);
    unpack_bf16x8(r, xv[p]);
    if (t < cnt) {
#pragma unroll
      for (int c = 0; c < 8; ++c) xv[p][c] = xv[p][c] - kmv[c];
    }
  }
  // token norms (fmaf chain per dim group, tree8 across the token's 8 lanes), then the
  // per-thread sums of x and of x/||x|| in p order
  float acc[16], amax = 0.0f;
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
    n2 = n2 + __shfl_xor(n2, 1, 64);
    n2 = n2 + __shfl_xor(n2, 2, 64);
    n2 = n2 + __shfl_xor(n2, 4, 64);
    const float inv = n2 > 0.0f ? 1.0f / sqrtf(n2) : 0.0f;
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
  // codes of the whole padded block (rows past the sequence end are zero)
  const float rc = sc != 0.0f ? 1.0f / sc : 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int t = tr + 32 * p;
    int c8[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) c8[c] = t < cnt ? quant_i8_rcp(xv[p][c], sc, rc) : 0;
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

template <int E, int K, int J>
__device__ __forceinline__ void ms_bstage(uint32_t (&u)[E], uint32_t* kx, int w, int lane) {
  constexpr int NW = 64 * E;
  if constexpr (J >= NW) {
#pragma unroll
    for (int e = 0; e < E; ++e) kx[NW * w + 64 * e + lane] = u[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = NW * w + 64 * e + lane;
      const uint32_t b = kx[i ^ J];
      const bool asc = (i & K) == 0, lower = (i & J) == 0;
      u[e] = (lower == asc) ? min(u[e], b) : max(u[e], b);
    }
    __syncthreads();  // every wave has read before the next exchange overwrites
  } else if constexpr (J >= 64) {
    constexpr int EJ = J / 64;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (e & EJ) continue;
      const uint32_t a = u[e], b = u[e | EJ];
      const bool asc = ((NW * w + 64 * e) & K) == 0;
      u[e] = asc ? min(a, b) : max(a, b);
      u[e | EJ] = asc ? max(a, b) : min(a, b);
    }
  } else {
    const bool lower = (lane & J) == 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = NW * w + 64 * e + lane;
      const bool asc = (i & K) == 0;
      const uint32_t a = u[e];
      const uint32_t b = ms_xor_lane<J>(a, lane);
      u[e] = (lower == asc) ? min(a, b) : max(a, b);
    }
  }
}
template <int E, int K, int J>
__device__ __forceinline__ void ms_bmerge(uint32_t (&u)[E], uint32_t* kx, int w, int lane) {
  ms_bstage<E, K, J>(u, kx, w, lane);
  if constexpr (J > 1) ms_bmerge<E, K, J / 2>(u, kx, w, lane);
}
template <int E, int K>
__device__ __forceinline__ void ms_bsort(uint32_t (&u)[E], uint32_t* kx, int w, int lane) {
  ms_bmerge<E, K, K / 2>(u, kx, w, lane);
  if constexpr (K < 256 * E) ms_bsort<E, K * 2>(u, kx, w, lane);
}
// The same network over one wave's 64E positions i = 64e + lane (no cross-wave stage).
template <int E, int K>
__device__ __forceinline__ void ms_bsort_wave(uint32_t (&u)[E], int lane) {
  ms_bmerge<E, K, K / 2>(u, nullptr, 0, lane);
  if constexpr (K < 64 * E) ms_bsort_wave<E, K * 2>(u, lane);
}

// One 256-thread workgroup per (head, q-block) row for nk > 1024, E keys per lane
// (NP2 = 256E sort positions):
//  scores  wave w scores columns c = 256i + 64w + lane, each lane reading its column's
//          pooled K (64 floats) straight from L2 (DOT64 chain, pooled Q in registers).
//  sort    lane (w, lane) holds sort positions i = 64Ew + 64e + lane in registers; a
//          bitonic network over i: partners 64 positions or more apart and in the same
//          wave are another register of the lane, closer ones one shuffle away, and only
//          the 3 stages whose partner is in another wave go through LDS.
//  prefix  the sequential CDF chain over the sorted values in one lane, as in k_ms_map_wave.
//  select  contiguous column chunks per thread and a workgroup scan for the tie rank.
template <int E>
__global__ __launch_bounds__(256) void k_ms_map_long(const float* __restrict__ pooled_q,
                                                     const float* __restrict__ pooled_k,
                                                     const uint8_t* __restrict__ sim_q,
                                                     const uint8_t* __restrict__ sim_k, int H, int nq, int nk,
                                                     const float* __restrict__ cdfth, int n_sink,
                                                     uint8_t* __restrict__ map) {
  constexpr int NW = 64 * E, NP2 = 4 * NW;
  extern __shared__ __align__(16) unsigned char ms_dyn[];
  // front region (ms_long_front_bytes): the waves' score chunks, later the sort exchange
  uint32_t* kx = reinterpret_cast<uint32_t*>(ms_dyn);  // [NP2] exchange, then the sorted keys
  float* scw = reinterpret_cast<float*>(ms_dyn) + (threadIdx.x >> 6) * (64 * MS_CH_LD);  // [64][MS_CH_LD]
  float* p = reinterpret_cast<float*>(ms_dyn + ms_long_front_bytes(NP2));  // [nk] scores -> p, column order
  __shared__ float red[4];
  __shared__ int ired[4];
  __shared__ int n_sel;
  const int r = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint8_t* row = map + ((long long)bh * nq + r) * nk;
  const uint8_t* sk = sim_k + (long long)bh * nk;
  if (!sim_q[(long long)bh * nq + r]) {  // a non-similar query block attends to every key block
    for (int c = tid; c < nk; c += 256) row[c] = 1;
    return;
  }
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
  float mx = -__builtin_huge_valf();
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
    }
  }
  mx = wave_max(mx);
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (!(mx > -__builtin_huge_valf())) {  // no similar key block: every block is forced on
    for (int c = tid; c < nk; c += 256) row[c] = 1;
    return;
  }
  for (int c = tid; c < nk; c += 256) p[c] = sk[c] ? ress_expf(p[c] - mx) : 0.0f;
  __syncthreads();
  if (w == 0) {
    float a = 0.0f;
    for (int i = lane; i < nk; i += 64) a = a + p[i];
    a = sum64_tree(a);
    if (lane == 0) red[0] = a;
  }
  __syncthreads();
  const float tot = red[0];
  for (int c = tid; c < nk; c += 256) p[c] = p[c] / tot;
  __syncthreads();
  // every p is >= +0, so its bit pattern orders like the value; only the values are
  // sorted (equal values are interchangeable in the prefix sums). Ascending keys ~bits(p):
  // descending p, padding (~0) last.
  uint32_t u[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = NW * w + 64 * e + lane;
    u[e] = i < nk ? ~__float_as_uint(p[i]) : ~0u;
  }
  ms_bsort<E, 2>(u, kx, w, lane);
#pragma unroll
  for (int e = 0; e < E; ++e) kx[NW * w + 64 * e + lane] = ~u[e];  // the sorted p (descending), as bits
  __syncthreads();
  if (tid == 0) {  // n = #{sequential prefix sums of the sorted p that are <= th}
    // p >= 0, so the sums only grow: n is the position of the first sum above th (nk if
    // none). One add per key; the batch that crosses th is searched once; the next 16
    // keys are read while a batch is summed. Keys past nk are p = 0 (padding).
    const float th = cdfth[bh % H];
    const float4* v4 = reinterpret_cast<const float4*>(kx);
    float cum = 0.0f;
    int n = nk;
    // 16 values a batch, the next two batches' reads in flight (v4[4b .. 4b+3] is batch b;
    // batches up to NP2/16 exist, NP2 >= 2048)
    float4 x[4], y[4], z[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      x[g] = v4[g];
      y[g] = v4[4 + g];
    }
    for (int i = 0; i < nk; i += 16) {
      if (i + 32 < nk) {
#pragma unroll
        for (int g = 0; g < 4; ++g) z[g] = v4[(i + 32) / 4 + g];  // i + 48 <= NP2
      }
      float cv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        cum = cum + x[g].x;
        cv[4 * g] = cum;
        cum = cum + x[g].y;
        cv[4 * g + 1] = cum;
        cum = cum + x[g].z;
        cv[4 * g + 2] = cum;
        cum = cum + x[g].w;
        cv[4 * g + 3] = cum;
      }
      if (!(cum <= th)) {
        int first = 15;
#pragma unroll
        for (int m = 14; m >= 0; --m) first = cv[m] <= th ? first : m;
        n = min(nk, i + first);
        break;
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        x[g] = y[g];
        y[g] = z[g];
      }
    }
    n_sel = n;
  }
  __syncthreads();
  const int n = n_sel;
  const uint32_t vbits = n > 0 ? kx[n - 1] : 0u;  // the n-th largest p
  // contiguous column chunks: p > v is kept; of the p == v columns, the lowest-indexed
  // n - #{p > v} (an exclusive scan of the per-chunk counts gives each one's rank)
  const int chunk = cdiv(nk, 256), c0 = min(nk, tid * chunk), c1 = min(nk, c0 + chunk);
  int gt = 0, eq = 0;
  for (int c = c0; c < c1; ++c) {
    const uint32_t b = __float_as_uint(p[c]);
    gt += b > vbits ? 1 : 0;
    eq += b == vbits ? 1 : 0;
  }
  int incl = eq;  // inclusive scan of eq over the workgroup, in thread order
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
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
    row[c] = (sel || !sk[c] || c < n_sink) ? 1 : 0;
  }
}

// One wave per (head, q-block) row, E = 64-key-block columns per lane (nk <= 64E), four
// rows of one head per workgroup.
//  scores  pooled K goes through LDS in coalesced 64-block tiles that the four rows
//          share; lane l keeps the scores of columns c = 64e + l (also the SUM64 order).
//  sort    only the probabilities are sorted (equal values are interchangeable in the
//          prefix sums): a bitonic network over 32-bit keys in registers, partners 64
//          positions or more apart in the same lane, closer ones one shuffle away.
//  prefix  the sequential CDF chain of each row runs in one lane of wave 0 over the
//          sorted values in LDS (the four rows' chains side by side) up to the batch of 16
//          where it first exceeds th; that position is the row's count.
//  select  with v the n-th largest probability: every column with p > v, and of those
//          with p == v the lowest-indexed ones up to n (a ballot prefix count).
template <int E>
__global__ __launch_bounds__(256) void k_ms_map_wave(const float* __restrict__ pooled_q,
                                                     const float* __restrict__ pooled_k,
                                                     const uint8_t* __restrict__ sim_q,
                                                     const uint8_t* __restrict__ sim_k, int H, int nq, int nk,
                                                     const float* __restrict__ cdfth, int n_sink,
                                                     uint8_t* __restrict__ map) {
  constexpr int NP = 64 * E, LDK = 65, LDS_ROW = NP + 4;  // LDK / LDS_ROW: padded strides
  __shared__ float pk_l[64 * LDK];
  __shared__ __align__(16) float pq_l[4][64];
  __shared__ __align__(16) float sv_l[4][LDS_ROW];
  __shared__ int go_l[4];
  __shared__ int n_l[4];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.y, r = blockIdx.x * 4 + w;
  const long long row_id = (long long)bh * nq + r;
  const bool in_range = r < nq;
  const bool active = in_range && sim_q[row_id];
  if (in_range) pq_l[w][lane] = pooled_q[row_id * 64 + lane];
  const float* pkh = pooled_k + (long long)bh * nk * 64;
  const uint8_t* sk = sim_k + (long long)bh * nk;

  // tiles of 64 key blocks: tile e+1 is loaded into registers while tile e is computed
  float s[E];
#pragma unroll
  for (int e = 0; e < E; ++e) s[e] = 0.0f;
  const int tiles = cdiv(nk, 64);
  float4 nxt[4];
  auto load_tile = [&](int t) {
    const int cols = min(64, nk - 64 * t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f4 = tid + 256 * i, col = f4 >> 4;
      nxt[i] = col < cols ? reinterpret_cast<const float4*>(pkh + (long long)(64 * t + col) * 64)[f4 & 15]
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  load_tile(0);
#pragma unroll 1
  for (int e = 0; e < tiles; ++e) {
    __syncthreads();  // previous tile consumed (and pq_l written, first time)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f4 = tid + 256 * i;
      float* dst = pk_l + (f4 >> 4) * LDK + (f4 & 15) * 4;
      dst[0] = nxt[i].x;
      dst[1] = nxt[i].y;
      dst[2] = nxt[i].z;
      dst[3] = nxt[i].w;
    }
    __syncthreads();
    if (e + 1 < tiles) load_tile(e + 1);
    if (active && 64 * e + lane < nk) {
      const float4* qv = reinterpret_cast<const float4*>(pq_l[w]);
      const float* kc = pk_l + lane * LDK;
      float a = 0.0f;
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        const float4 qq = qv[d4];
        a = fmaf(qq.x, kc[4 * d4 + 0], a);
        a = fmaf(qq.y, kc[4 * d4 + 1], a);
        a = fmaf(qq.z, kc[4 * d4 + 2], a);
        a = fmaf(qq.w, kc[4 * d4 + 3], a);
      }
#pragma unroll
      for (int e2 = 0; e2 < E; ++e2)
        if (e2 == e) s[e2] = a;
    }
  }

  bool simc[E];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = 64 * e + lane;
    simc[e] = c < nk && sk[c];
    s[e] = s[e] * 0.125f;
    if (simc[e]) mx = fmaxf(mx, s[e]);
  }
  mx = wave_max(mx);
  // the CDF path runs for a similar row with at least one similar key block; otherwise
  // every block of the row is on
  const bool go = active && mx > -__builtin_huge_valf();
  uint32_t pb[E];  // bits of p at the lane's own columns (p >= +0: bits order like values)
#pragma unroll
  for (int e = 0; e < E; ++e) pb[e] = 0;
  if (go) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      s[e] = simc[e] ? ress_expf(s[e] - mx) : 0.0f;
      if (64 * e + lane < nk) part = part + s[e];
    }
    const float tot = sum64_tree(part);
    uint32_t u[E];  // ascending sort keys ~bits(p): descending p; padding (~0) last
#pragma unroll
    for (int e = 0; e < E; ++e) {
      pb[e] = __float_as_uint(s[e] / tot);
      u[e] = 64 * e + lane < nk ? ~pb[e] : ~0u;
    }
    // bitonic network over positions 64e + lane: partners 64 or more apart are another
    // register of the lane, closer ones one DPP / swizzle / half-swap permute away
    ms_bsort_wave<E, 2>(u, lane);
#pragma unroll
    for (int e = 0; e < E; ++e) sv_l[w][64 * e + lane] = __uint_as_float(~u[e]);
    if (lane == 0) go_l[w] = 1;
    // s[] now holds the sorted values (position 64e + lane): the chain overwrites sv_l
#pragma unroll
    for (int e = 0; e < E; ++e) s[e] = __uint_as_float(~u[e]);
  } else if (lane == 0) {
    go_l[w] = 0;
  }
  __syncthreads();
  if (w == 0 && lane < 4 && go_l[lane]) {  // the four rows' sequential chains, side by side
    // n = #{sequential prefix sums of the sorted p that are <= th}; p >= 0, so the sums
    // only grow and n is the position of the first sum above th (nk if none): the chain
    // stops at the batch that crosses th
    const float th = cdfth[bh % H];
    const float* v = sv_l[lane];
    float cum = 0.0f;
    int n = nk, i = 0;
    bool crossed = false;
    for (; i + 16 <= nk; i += 16) {  // 16 values per LDS round trip
      float4 x[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) x[g] = reinterpret_cast<const float4*>(v + i)[g];
      float cv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        cum = cum + x[g].x;
        cv[4 * g] = cum;
        cum = cum + x[g].y;
        cv[4 * g + 1] = cum;
        cum = cum + x[g].z;
        cv[4 * g + 2] = cum;
        cum = cum + x[g].w;
        cv[4 * g + 3] = cum;
      }
      if (!(cum <= th)) {
        int first = 15;
#pragma unroll
        for (int m = 14; m >= 0; --m) first = cv[m] <= th ? first : m;
        n = i + first;
        crossed = true;
        break;
      }
    }
    if (!crossed) {
      for (; i < nk; ++i) {
        cum = cum + v[i];
        if (!(cum <= th)) {
          n = i;
          break;
        }
      }
    }
    n_l[lane] = n;
  }
  __syncthreads();
  if (!in_range) return;
  uint8_t* row = map + row_id * nk;
  if (!go) {
    for (int c = lane; c < nk; c += 64) row[c] = 1;
    return;
  }
  const int n = n_l[w];
  uint32_t vbits = 0;
  int n_gt = 0;
  if (n > 0) {  // v = the n-th largest p (sorted position n-1; s[] holds the sorted values)
    const int pos = n - 1, slot = pos >> 6;
    float sel = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) sel = e == slot ? s[e] : sel;
    vbits = __float_as_uint(__shfl(sel, pos & 63, 64));
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
    if (c < nk) row[c] = (sel || !sk[c] || c < n_sink) ? 1 : 0;
  }
}

}  // namespace

// get_block_map_meansim_fuse_quant (patched SpargeAttn, external/patches/spargeattn.patch:50-67)
RESS_API int ress_meansim_block_map(const void* q, const void* k, const void* km, int B, int H, int Tq, int Tk,
                                    long long sqB, long long sqH, long long sqT, long long skB, long long skH,
                                    long long skT, const void* simthreshd1, const void* cdfthreshd,
                                    int attention_sink, void* map, void* q_i8, void* q_scale, void* k_i8,
                                    void* k_scale, void* pooled_q, void* pooled_k, void* sim_q, void* sim_k,
                                    hipStream_t stream) {
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
    const size_t lds4 = (size_t)nk * 4;
    if (nk <= 2048)
      hipLaunchKernelGGL(k_ms_map_long<8>, dim3(nq, BH), dim3(256), ms_long_front_bytes(2048) + lds4, stream, pq, pk, sq8, sk8, H, nq,
                         nk, cd, n_sink, m8);
    else if (nk <= 4096)
      hipLaunchKernelGGL(k_ms_map_long<16>, dim3(nq, BH), dim3(256), ms_long_front_bytes(4096) + lds4, stream, pq, pk, sq8, sk8, H, nq,
                         nk, cd, n_sink, m8);
    else
      hipLaunchKernelGGL(k_ms_map_long<32>, dim3(nq, BH), dim3(256), ms_long_front_bytes(8192) + lds4, stream, pq, pk, sq8, sk8, H, nq,
                         nk, cd, n_sink, m8);
  }
  RESS_LAUNCHED("k_ms_map");
  return 0;
}
