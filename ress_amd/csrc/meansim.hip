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
//     pooled  = SUM8x(x) / n,  ssum = SUM8x(xh)
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
// k_ms_stats: one 256-thread workgroup per (block, batch*head). Thread (token lane
// tid>>3, dim group tid&7) loads 8 bf16 per token pass (BS/32 passes), keeps them in
// registers for the codes, and stages fp32 copies in LDS for the per-dim column pass.
// k_ms_map: one 256-thread workgroup per (q-block, batch*head); scores, softmax and
// the ranks (by counting, against LDS-resident probabilities) are parallel, the CDF
// prefix is one lane's sequential chain.
#include "common.h"

namespace {

constexpr int MS_LD = 68;          // LDS row stride (floats) of the staged block: 16-byte rows, offset banks
constexpr int MS_MAX_NK = 4096;    // key blocks per row the map kernel holds in LDS (2 x 16 KiB)

template <int BS>
__global__ __launch_bounds__(256) void k_ms_stats(const uint16_t* __restrict__ x, Strides sx, int T,
                                                  const float* __restrict__ km, const float* __restrict__ simth,
                                                  int nb, int8_t* __restrict__ codes, float* __restrict__ scale,
                                                  float* __restrict__ pooled, uint8_t* __restrict__ sim) {
  constexpr int PASSES = BS / 32;
  __shared__ __align__(16) float xs_l[BS * MS_LD];
  __shared__ float inv_l[BS];
  __shared__ float ssum_l[64];
  __shared__ float amax_l[4];
  const int blk = blockIdx.x, bh = blockIdx.y;
  const int tid = threadIdx.x, g = tid & 7, tr = tid >> 3, lane = tid & 63, w = tid >> 6;
  const int base = blk * BS, cnt = min(BS, T - base);
  const uint16_t* xb = x + bh_offset(bh, sx);

  float kmv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) kmv[c] = km ? km[(long long)bh * 64 + 8 * g + c] : 0.0f;

  // token pass: values, squared norm (fmaf chain per dim group, tree8 across the 8 lanes of a token)
  float xv[PASSES][8];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int t = tr + 32 * p;
    if (t < cnt) {
      const uint4 r = *reinterpret_cast<const uint4*>(xb + (long long)(base + t) * sx.t + 8 * g);
      unpack_bf16x8(r, xv[p]);
#pragma unroll
      for (int c = 0; c < 8; ++c) xv[p][c] = xv[p][c] - kmv[c];
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) xv[p][c] = 0.0f;
    }
    float part = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      part = fmaf(xv[p][c], xv[p][c], part);
      amax = fmaxf(amax, fabsf(xv[p][c]));
    }
    part = part + __shfl_xor(part, 1, 64);
    part = part + __shfl_xor(part, 2, 64);
    part = part + __shfl_xor(part, 4, 64);
    if (t < cnt) {
      float4* dst = reinterpret_cast<float4*>(xs_l + t * MS_LD + 8 * g);
      dst[0] = make_float4(xv[p][0], xv[p][1], xv[p][2], xv[p][3]);
      dst[1] = make_float4(xv[p][4], xv[p][5], xv[p][6], xv[p][7]);
      if (g == 0) inv_l[t] = part > 0.0f ? 1.0f / sqrtf(part) : 0.0f;
    }
  }
  amax = wave_max(amax);
  if (lane == 0) amax_l[w] = amax;
  __syncthreads();

  // column pass: lane (j = lane>>3, dims d0, d0+1); SUM8x over token lanes j
  {
    const int j = lane >> 3, d0 = w * 16 + (lane & 7) * 2;
    float pp0 = 0.0f, pp1 = 0.0f, ph0 = 0.0f, ph1 = 0.0f;
    for (int t = j; t < cnt; t += 8) {
      const float2 v = *reinterpret_cast<const float2*>(xs_l + t * MS_LD + d0);
      const float iv = inv_l[t];
      pp0 = pp0 + v.x;
      pp1 = pp1 + v.y;
      ph0 = ph0 + v.x * iv;
      ph1 = ph1 + v.y * iv;
    }
    pp0 = sum8_tree(pp0);
    pp1 = sum8_tree(pp1);
    ph0 = sum8_tree(ph0);
    ph1 = sum8_tree(ph1);
    if (j == 0) {
      float* pd = pooled + ((long long)bh * nb + blk) * 64 + d0;
      pd[0] = pp0 / (float)cnt;
      pd[1] = pp1 / (float)cnt;
      ssum_l[d0] = ph0;
      ssum_l[d0 + 1] = ph1;
    }
  }
  const float bamax = fmaxf(fmaxf(amax_l[0], amax_l[1]), fmaxf(amax_l[2], amax_l[3]));
  const float sc = bamax / 127.0f;
  __syncthreads();

  if (w == 0) {
    const int gg = lane & 7;
    float part = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) part = fmaf(ssum_l[8 * gg + c], ssum_l[8 * gg + c], part);
    part = part + __shfl_xor(part, 1, 64);
    part = part + __shfl_xor(part, 2, 64);
    part = part + __shfl_xor(part, 4, 64);
    if (lane == 0) {
      const float s = part / ((float)cnt * (float)cnt);
      sim[(long long)bh * nb + blk] = s > simth[bh % sx.H] ? 1 : 0;
      scale[(long long)bh * nb + blk] = sc;
    }
  }

  // codes of the whole padded block (rows past the sequence end are zero)
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int t = tr + 32 * p;
    int c8[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) c8[c] = t < cnt ? quant_i8(xv[p][c], sc) : 0;
    *reinterpret_cast<uint2*>(codes + ((long long)bh * nb * BS + base + t) * 64 + 8 * g) = pack_i8x8(c8);
  }
}

__global__ __launch_bounds__(256) void k_ms_map(const float* __restrict__ pooled_q, const float* __restrict__ pooled_k,
                                                const uint8_t* __restrict__ sim_q, const uint8_t* __restrict__ sim_k,
                                                int H, int nq, int nk, const float* __restrict__ cdfth, int n_sink,
                                                uint8_t* __restrict__ map) {
  extern __shared__ __align__(16) float ms_dyn[];
  float* p = ms_dyn;                 // [nk] scores -> exp -> probabilities
  float* sorted = ms_dyn + nk;       // [nk] probabilities in selection order
  __shared__ __align__(16) float pq[64];
  __shared__ float red[4];
  __shared__ int n_sel;
  const int r = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint8_t* row = map + ((long long)bh * nq + r) * nk;
  const uint8_t* sk = sim_k + (long long)bh * nk;

  if (!sim_q[(long long)bh * nq + r]) {  // a non-similar query block attends to every key block
    for (int c = tid; c < nk; c += 256) row[c] = 1;
    return;
  }
  if (tid < 64) pq[tid] = pooled_q[((long long)bh * nq + r) * 64 + tid];
  __syncthreads();

  float mx = -__builtin_huge_valf();
  for (int c = tid; c < nk; c += 256) {
    float s = -__builtin_huge_valf();
    if (sk[c]) {
      const float4* kv = reinterpret_cast<const float4*>(pooled_k + ((long long)bh * nk + c) * 64);
      const float4* qv = reinterpret_cast<const float4*>(pq);
      float a = 0.0f;
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        const float4 kk = kv[d4], qq = qv[d4];
        a = fmaf(qq.x, kk.x, a);
        a = fmaf(qq.y, kk.y, a);
        a = fmaf(qq.z, kk.z, a);
        a = fmaf(qq.w, kk.w, a);
      }
      s = a * 0.125f;
      mx = fmaxf(mx, s);
    }
    p[c] = s;
  }
  mx = wave_max(mx);
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int n = 0;
  if (mx > -__builtin_huge_valf()) {
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
    // rank = #{c' : p[c'] > p[c] or (p[c'] == p[c] and c' < c)}; every p is >= +0, so
    // its bit pattern orders like the value
    for (int c = tid; c < nk; c += 256) {
      const uint32_t key = __float_as_uint(p[c]);
      int rank = 0;
      for (int i = 0; i < nk; ++i) {
        const uint32_t ki = __float_as_uint(p[i]);
        rank += (ki > key) | ((ki == key) & (i < c));
      }
      sorted[rank] = p[c];
    }
    __syncthreads();
    if (tid == 0) {
      const float th = cdfth[bh % H];
      float cum = 0.0f;
      int i = 0;
      for (; i < nk; ++i) {
        cum = cum + sorted[i];
        if (!(cum <= th)) break;
      }
      n_sel = i;
    }
    __syncthreads();
    n = n_sel;
  }
  for (int c = tid; c < nk; c += 256) {
    bool keep = !sk[c] || c < n_sink;
    if (!keep && n > 0) {
      const uint32_t key = __float_as_uint(p[c]);
      int rank = 0;
      for (int i = 0; i < nk && rank < n; ++i) {
        const uint32_t ki = __float_as_uint(p[i]);
        rank += (ki > key) | ((ki == key) & (i < c));
      }
      keep = rank < n;
    }
    row[c] = keep ? 1 : 0;
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
  hipLaunchKernelGGL(k_ms_stats<128>, dim3(nq, BH), dim3(256), 0, stream, (const uint16_t*)q, sq, Tq,
                     (const float*)nullptr, (const float*)simthreshd1, nq, (int8_t*)q_i8, (float*)q_scale,
                     (float*)pooled_q, (uint8_t*)sim_q);
  RESS_LAUNCHED("k_ms_stats<128>");
  hipLaunchKernelGGL(k_ms_stats<64>, dim3(nk, BH), dim3(256), 0, stream, (const uint16_t*)k, sk, Tk,
                     (const float*)km, (const float*)simthreshd1, nk, (int8_t*)k_i8, (float*)k_scale,
                     (float*)pooled_k, (uint8_t*)sim_k);
  RESS_LAUNCHED("k_ms_stats<64>");
  const int n_sink = attention_sink > 0 ? cdiv(attention_sink, 64) : 0;
  hipLaunchKernelGGL(k_ms_map, dim3(nq, BH), dim3(256), (size_t)2 * nk * sizeof(float), stream,
                     (const float*)pooled_q, (const float*)pooled_k, (const uint8_t*)sim_q, (const uint8_t*)sim_k, H,
                     nq, nk, (const float*)cdfthreshd, n_sink, (uint8_t*)map);
  RESS_LAUNCHED("k_ms_map");
  return 0;
}
