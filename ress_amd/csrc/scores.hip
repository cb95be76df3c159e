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
// Longer rows: the scores as one matrix-core GEMM into attn_full (k_scores_gemm, DOT64
// exactly), then k_pooled_softmax_rows; k_pooled_scores_rows beyond 64*PS_E_MAX blocks.
#include <type_traits>

#include "common.h"

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
// ---- the score GEMM on the matrix cores ------------------------------------------------
// A workgroup of 4 waves takes a 128-row tile of S and walks column tiles of 128 (tiles
// blockIdx.x, blockIdx.x + gridDim.x, ...). Wave w holds rows 32w..32w+31 of the A operand
// in registers for the whole walk and computes them against all 128 columns of each tile
// (4 column sub-tiles of 32). Step s of v_mfma_f32_32x32x2_f32 takes dim 2s + l/32 of row
// l%32 from lane l, so B tiles sit in LDS with each row's 64 dims split into the even dims
// (floats 0..31) and the odd dims (32..63): a lane's 32 values are one contiguous run, read
// as 8 float4s; the 68-float row stride puts 16 consecutive rows' float4 reads in distinct
// banks. B tiles are double-buffered: the next tile's loads are in flight during the MFMAs.
constexpr int SG_T = 128;
constexpr int SG_LD = 68;
constexpr int SG_WALK = 4;  // column tiles per workgroup (at most)
typedef float sg_f16v __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void k_scores_gemm(const float* __restrict__ a, const float* __restrict__ b,
                                                     int na, int nb, int r_begin, int r_end, float scale,
                                                     float* __restrict__ S) {
  __shared__ __align__(16) float bl[2][SG_T * SG_LD];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = r_begin + blockIdx.y * SG_T, bh = blockIdx.z, h = lane >> 5, rl = lane & 31;
  const int ntile = cdiv(nb, SG_T);
  const float* bhd = b + (long long)bh * nb * 64;
  // B tile loads: 2048 float4 chunks, chunk f = row f/16, dims 4(f%16)..+3; rows past the
  // matrix read its last row (zeroed when written to LDS; their outputs are not stored)
  float4 ys[8];
  auto load_b = [&](int t) {
    const int c0 = t * SG_T;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i;
      ys[i] = reinterpret_cast<const float4*>(bhd + (long long)min(c0 + (f >> 4), nb - 1) * 64)[f & 15];
    }
  };
  auto store_b = [&](int t, float* dst) {
    const int c0 = t * SG_T;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i, r = f >> 4, q = f & 15;
      const float4 y = c0 + r < nb ? ys[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      // dims 4q and 4q+2 go to even positions 2q, 2q+1; dims 4q+1 and 4q+3 to the odd half
      *reinterpret_cast<float2*>(dst + r * SG_LD + 2 * q) = make_float2(y.x, y.z);
      *reinterpret_cast<float2*>(dst + r * SG_LD + 32 + 2 * q) = make_float2(y.y, y.w);
    }
  };
  int t = blockIdx.x;
  if (t >= ntile) return;  // workgroup-uniform
  load_b(t);
  // the wave's A operand: dim 2s + h of row r0 + 32w + rl for s = 0..31 (zero past the matrix)
  float av[32];
  {
    const int ra = r0 + 32 * w + rl;
    const float4* ap = reinterpret_cast<const float4*>(a + ((long long)bh * na + min(ra, r_end - 1)) * 64);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const float4 x = ap[q];
      av[2 * q] = ra < r_end ? (h ? x.y : x.x) : 0.0f;
      av[2 * q + 1] = ra < r_end ? (h ? x.w : x.z) : 0.0f;
    }
  }
  store_b(t, bl[0]);
  __syncthreads();
  const int lrow = 32 * w + 4 * h;
  char* trow = reinterpret_cast<char*>(S + ((long long)bh * na + r0) * nb);  // the row tile's origin
  constexpr int BCT = 32 * SG_LD / 4;            // float4s between column sub-tiles
#pragma unroll 1
  for (int it = 0;; ++it) {
    const int tn = t + (int)gridDim.x;
    const bool more = it + 1 < SG_WALK && tn < ntile;  // uniform
    if (more) load_b(tn);
    const float4* bp = reinterpret_cast<const float4*>(bl[it & 1] + rl * SG_LD + 32 * h);
    sg_f16v acc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[ct][j] = 0.0f;
    // every accumulator takes steps s = 0..31 in order: DOT64 over d = 0..63. The B
    // operands of steps 4(j+1).. are read from LDS before the MFMAs of steps 4j.. issue.
    float4 bv[4], bn[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) bv[ct] = bp[ct * BCT];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j + 1 < 8) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) bn[ct] = bp[ct * BCT + j + 1];
      }
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        acc[ct] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * j], bv[ct].x, acc[ct], 0, 0, 0);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        acc[ct] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * j + 1], bv[ct].y, acc[ct], 0, 0, 0);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        acc[ct] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * j + 2], bv[ct].z, acc[ct], 0, 0, 0);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        acc[ct] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * j + 3], bv[ct].w, acc[ct], 0, 0, 0);
      if (j + 1 < 8) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) bv[ct] = bn[ct];
      }
    }
    // accumulator element j of lane l is row 8(j/4) + 4(l/32) + j%4, column l%32 of its
    // sub-tile; offsets from the (uniform) tile origin fit 32 bits
    const int c0 = t * SG_T;
    char* tile = trow + 4ll * c0;
    // byte offsets from the uniform tile origin (below 2^31: 128 rows of at most 2^21
    // floats), unsigned so that the stores take the scalar-base + 32-bit offset form
    if (r0 + SG_T <= r_end && c0 + SG_T <= nb) {  // whole tile (uniform): no per-store test
      unsigned lofs = 4u * (unsigned)(lrow * nb + rl);
      // kept opaque so the 64 store offsets are formed per tile, not hoisted out of the
      // walk into 64 live registers
      asm volatile("" : "+v"(lofs));
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          *reinterpret_cast<float*>(tile + (lofs + 4u * (unsigned)((8 * (j >> 2) + (j & 3)) * nb + 32 * ct))) =
              acc[ct][j] * scale;
    } else {
      // rows and columns this lane may still store (opaque for the same reason as above)
      int rlim = r_end - r0 - lrow, clim = nb - c0 - rl;
      unsigned lofs = 4u * (unsigned)(lrow * nb + rl);
      asm volatile("" : "+v"(rlim), "+v"(clim), "+v"(lofs));
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int dr = 8 * (j >> 2) + (j & 3);
          if (dr < rlim && 32 * ct < clim)
            *reinterpret_cast<float*>(tile + (lofs + 4u * (unsigned)(dr * nb + 32 * ct))) = acc[ct][j] * scale;
        }
    }
    if (!more) break;
    // buffer (it+1)&1 was last read in the previous iteration, which every wave finished
    // before the barrier that ended it
    store_b(tn, bl[(it + 1) & 1]);
    __syncthreads();
    t = tn;
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
  // column tiles t = x, x + gx, ... per workgroup, at most SG_WALK of them
  const int gx = cdiv(cdiv(nb, SG_T), SG_WALK);
  hipLaunchKernelGGL(k_scores_gemm, dim3(gx, cdiv(r_end - r_begin, SG_T), BH), dim3(256), 0, stream, a, b, na, nb,
                     r_begin, r_end, scale, S);
  RESS_LAUNCHED("k_scores_gemm");
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
