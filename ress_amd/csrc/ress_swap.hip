// ReSS restore-swap block ranking for gfx950.
//
// Replaces restore_swap_rank_by (reference src/ress/scoring/projected.py:395-1058) with
// the round body of scoring/fused_round.py (kept-mass-normalised objective
// J = ||g||^2_M / K^2, drift compensate, geometric schedule, >=1 floor on beneficial
// rows, track-best) and fused_topm's exact top-m (ties to the lowest index). Every
// (batch*head, query-block) row is independent. A row runs on W waves (1, 2 or 4, by
// row length); a 1024-thread workgroup holds 16/W rows of one head, in lockstep, and V
// streams through LDS tiles that all of them share.
//
// Numerics (the same operation order as oracle/ress_oracle.c, whatever W is):
//  * With `big` (the recipe's _bf16) every value the reference keeps in bf16 is rounded
//    at the reference's points (quadratic_deviation projected.py:259-288,
//    dense_reference :313-356, the round :903-947, fused_round.py:176-226).
//  * SUMK (the sums over key blocks: P @ v_bar and sum P of the dense reference, the
//    dropped mass sum_Pd and Pd @ v_bar of the objective): 16 interleaved classes
//    k mod 16, each a sequential fp32 chain over increasing k (fmaf for products), the
//    16 class sums combined by the balanced pairwise tree over classes 0..15. Wave w of a
//    row's W waves owns the classes of one subtree.
//  * DOT4x16 (the per-candidate products v_k . Mvq and v_k . big(Mg)): four sequential
//    fmaf chains over dims 16c..16c+15, combined as (c0 + c1) + (c2 + c3).
//  * The objective after the initial cut is carried from round to round: each round adds
//    to the unrounded sum_Pd and Pd @ v_bar the change of the round, summed over the
//    restored (pd = -P) and compensated (pd = +P) candidates in four classes k mod 4, each
//    a sequential chain over increasing k (fmaf for the products), combined as
//    (d0 + d1) + (d2 + d3).
//  * The 64-term products and sums of M (M v_bar_query, M g, ||g||^2_M, the term_q sums,
//    and term_k once per head) are sequential fp32 chains in index order.
#include <type_traits>

#include "common.h"

#define RS_BF16 1
#define RS_TRACK_BEST 2
#define RS_MAXIMIZE 4
#define RS_INVERT_CUT 8
#define RS_NO_RENORM 16
#define RS_MAX_KBP 2048  // key blocks per row handled
// one workgroup: TPB/64 waves = TPB/64/W rows of W waves; TPB = 1024 with bf16 V tiles,
// 512 with fp32 ones (whose tiles take twice the LDS)
template <bool B16>
struct RsShape {
  static constexpr int TPB = B16 ? 1024 : 512;
  static constexpr int WAVES = TPB / 64;
};

__device__ __forceinline__ float rs_bf(float x, bool big) {
  if (!big) return x;
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(((u >> 16) | 0x40u) << 16);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float((u >> 16) << 16);
}
// fused_topm's order key: non-negatives get the sign bit set, negatives are complemented
__device__ __forceinline__ uint32_t rs_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// kept_mass_norm_quality (projected.py:191-211), grouping ((G*u)*(2K+u))/(K*K) - dG, / Kn^2
__device__ __forceinline__ float rs_knorm(float G, float K, float dG, float u) {
  float Kn = K + u;
  Kn = Kn < 1e-6f ? 1e-6f : Kn;
  const float a = G * u;
  const float b = 2.0f * K + u;
  return (a * b / (K * K) - dG) / (Kn * Kn);
}
// balanced pairwise tree over x[0..N-1] (N a power of two)
template <int N>
__device__ __forceinline__ float rs_tree(const float* x) {
  if constexpr (N == 1) return x[0];
  else return rs_tree<N / 2>(x) + rs_tree<N / 2>(x + N / 2);
}

// Sequential fmaf chain over j = 0..63 of lane i's column of an LDS matrix (col[64*j],
// big-rounded when BF) and the broadcast vec[j]; sequential sum of a broadcast vector.
template <bool BF>
__device__ __forceinline__ float rs_dot_col(const float* col, const float* vec, bool big) {
  float acc = 0.0f;
#pragma unroll 8
  for (int j = 0; j < 64; ++j) {
    float m = col[j * 64];
    if constexpr (BF) m = rs_bf(m, big);
    acc = fmaf(m, vec[j], acc);
  }
  return acc;
}
__device__ __forceinline__ float rs_sum64(const float* vec) {
  float acc = 0.0f;
  for (int i = 0; i < 64; i += 4) {
    const float4 x = *reinterpret_cast<const float4*>(vec + i);
    acc = acc + x.x;
    acc = acc + x.y;
    acc = acc + x.z;
    acc = acc + x.w;
  }
  return acc;
}

// Per-head preparation, 64 key blocks per workgroup: Vp = big(V) [kb_p][64] (bf16 bits when
// big, whose values are bf16-exact, else fp32) and the key side of quadratic_deviation,
// termk[k] = big(sum_i big(big(Mb v_k)_i * v_ki)) with the product and the sum sequential
// in index order (the block goes through an LDS tile).
__global__ __launch_bounds__(256) void k_rs_head(const float* __restrict__ V, const float* __restrict__ M, int H,
                                                 int kb_p, int n_cand, int big, void* __restrict__ Vp,
                                                 float* __restrict__ termk) {
  __shared__ float MbT[64 * 64];     // MbT[j*64 + i] = big(M[i][j])
  __shared__ float tile[64][65];     // [key][dim], padded
  __shared__ float prod[4][64];      // one key's rounded products per wave
  const int k0 = blockIdx.x * 64, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float* Mh = M + (long long)(bh % H) * 4096;
  for (int e = tid; e < 4096; e += 256) MbT[(e & 63) * 64 + (e >> 6)] = rs_bf(Mh[e], big);
  for (int r = w; r < 64; r += 4) {  // rows of V: lane = dim
    const int k = k0 + r;
    float x = 0.0f;
    if (k < kb_p) {
      x = rs_bf(V[((long long)bh * kb_p + k) * 64 + lane], big);
      const long long o = ((long long)bh * kb_p + k) * 64 + lane;
      if (big) reinterpret_cast<uint16_t*>(Vp)[o] = (uint16_t)(__float_as_uint(x) >> 16);
      else reinterpret_cast<float*>(Vp)[o] = x;
    }
    tile[r][lane] = x;
  }
  __syncthreads();
  for (int r = w; r < 64; r += 4) {  // termk: wave per key, lane = output dim i
    const int k = k0 + r;
    if (k >= n_cand) break;
    float acc = 0.0f;
    for (int j = 0; j < 64; ++j) acc = fmaf(MbT[j * 64 + lane], tile[r][j], acc);
    prod[w][lane] = rs_bf(rs_bf(acc, big) * tile[r][lane], big);
    __builtin_amdgcn_wave_barrier();
    float t = 0.0f;
    for (int i = 0; i < 64; ++i) t = t + prod[w][i];
    if (lane == 0) termk[(long long)bh * n_cand + k] = rs_bf(t, big);
    __builtin_amdgcn_wave_barrier();
  }
}

struct RsArgs {
  const float* A;   // [BH][q_blk][kb_p]
  const float* M;   // [H][64][64]
  const int* nts;   // [BH][q_blk]
  const void* Vp;   // [BH][kb_p][64] bf16 bits (big) or fp32
  const float* termk;
  float* rank_key;  // [BH][q_blk][n_cand]: 1 = kept, 0 = dropped
  float* obj;       // [BH][q_blk] or null: J of the returned set
  float* s_out;     // [BH][q_blk][n_cand] or null: s = P*sqrt(d^T M d)
  int H, q_blk, kb_p, n_cand, n_iters, flags;
  double restore_frac, decay;  // geometric schedule (projected.py:775-790)
};

// Dynamic LDS of one workgroup (byte offsets): M^T, then per wave five 64-float vectors,
// then per row its P, histograms, counters, cross-wave partials and block masks.
struct RsLds {
  int m32, waves, wave_stride, rows, row_stride;
  int pb, hist, ints, chain, dpart, prod, eq, dmask, rmask, cmask;
  int total;
};
__host__ __device__ __forceinline__ RsLds rs_lds(int kb_p, int n_cand, int W, int waves) {
  RsLds L;
  const int G = cdiv(n_cand, 64), Td = cdiv(kb_p, 64);
  L.m32 = 0;
  L.waves = 4096 * 4;
  L.wave_stride = 5 * 64 * 4;
  L.rows = L.waves + waves * L.wave_stride;
  int o = 0;
  L.pb = o;        o += Td * 64 * 4;
  L.hist = o;      o += 2 * 256 * 4;
  L.ints = o;      o += 16 * 4;
  L.chain = o;     o += ((W * 65 * 4) + 15) & ~15;
  L.dpart = o;     o += ((4 * 65 * 4) + 15) & ~15;
  L.prod = o;      o += 2 * W * 64 * 4;
  L.eq = o;        o += ((G * 4) + 15) & ~15;
  L.dmask = o;     o += ((G * 8) + 15) & ~15;
  L.rmask = o;     o += ((G * 8) + 15) & ~15;
  L.cmask = o;     o += ((G * 8) + 15) & ~15;
  L.row_stride = o;
  L.total = L.rows + (waves / W) * L.row_stride;
  return L;
}

__device__ __forceinline__ void rs_gl_lds16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)src,
                                   (void __attribute__((address_space(3)))*)lds_base, 16, 0, 0);
}
template <int N>
__device__ __forceinline__ void rs_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// workgroup barrier that does not wait for the DMA in flight (__syncthreads would):
// this wave's LDS accesses complete, then s_barrier; the empty asm keeps memory
// accesses from moving across it
__device__ __forceinline__ void rs_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The rows of one head: TPB/64/W rows of W waves each, in lockstep (every barrier below is
// reached by all the workgroup's waves the same number of times). NS: candidate slots per lane of a
// wave; slot i of wave w holds candidate 64*(W*i + w) + lane, i.e. 64-candidate group
// g = W*i + w. B16: V is bf16 (big mode).
template <int NS, int W, bool B16>
__global__ __launch_bounds__(RsShape<B16>::TPB) void k_restore_swap(RsArgs a) {
  constexpr int TPB = RsShape<B16>::TPB;
  constexpr int R = RsShape<B16>::WAVES / W;  // rows per workgroup
  constexpr int C = 16 / W;         // SUMK classes per wave
  constexpr int CH = 4 / W;         // DOT4x16 dim chunks per wave
  constexpr int CPR = B16 ? 8 : 16; // 16-byte chunks per V row
  constexpr int TB = 64 * CPR;      // 16-byte chunks per tile of 64 V rows
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ __align__(16) float4 tb0[TB];
  __shared__ __align__(16) float4 tb1[TB];
  __shared__ __align__(16) float4 tb2[TB];
  __shared__ int rowflag[2][RsShape<B16>::WAVES];

  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rloc = wid / W, w = wid - rloc * W;
  const int kb_p = a.kb_p, n_cand = a.n_cand;
  const int G = cdiv(n_cand, 64), Td = cdiv(kb_p, 64);
  const RsLds L = rs_lds(kb_p, n_cand, W, RsShape<B16>::WAVES);
  float* M32T = reinterpret_cast<float*>(lds + L.m32);  // M32T[j*64 + i] = M[i][j]
  float* wv = reinterpret_cast<float*>(lds + L.waves + wid * L.wave_stride);
  float* vqs = wv;                  // [64] v_bar_query (big-rounded)
  float* t0 = wv + 64;              // [64] the products' vector (big(M vq), then big(Mg))
  float* t1 = t0 + 64;              // [64] scratch vectors
  float* t2 = t1 + 64;
  float* t3 = t2 + 64;              // [64] Mg of the current state
  unsigned char* rb = lds + L.rows + rloc * L.row_stride;
  float* PbL = reinterpret_cast<float*>(rb + L.pb);       // [Td*64] big(P) of the row, 0 past kb_p
  int* hist2 = reinterpret_cast<int*>(rb + L.hist);       // [2][256]
  int* ints = reinterpret_cast<int*>(rb + L.ints);        // [4][4] per-wave counters
  float* chain = reinterpret_cast<float*>(rb + L.chain);  // [W][65] SUMK partials
  float* dpart = reinterpret_cast<float*>(rb + L.dpart);  // [4][65] a round's change per class
  float* prod = reinterpret_cast<float*>(rb + L.prod);    // [2][W][64] DOT4x16 partials
  int* eqcnt = reinterpret_cast<int*>(rb + L.eq);         // [G] ties per candidate group
  unsigned long long* dmask = reinterpret_cast<unsigned long long*>(rb + L.dmask);  // [G]
  unsigned long long* rmask = reinterpret_cast<unsigned long long*>(rb + L.rmask);  // [G]
  unsigned long long* cmask = reinterpret_cast<unsigned long long*>(rb + L.cmask);  // [G]

  // Workgroup gl = x + gx*y runs on XCD gl % 8. With a multiple of 8 heads, XCD x takes
  // heads x, x+8, ... whole (every row group of each), so each XCD's L2 holds the V and A
  // rows of its own heads only.
  const int gx = gridDim.x, gl = blockIdx.x + gx * blockIdx.y;
  const bool xmap = (gridDim.y & 7) == 0;
  const int bh = xmap ? (gl & 7) + 8 * ((gl >> 3) / gx) : blockIdx.y;
  const int bgrp = xmap ? (gl >> 3) % gx : blockIdx.x;
  const int q_raw = bgrp * R + rloc;
  const bool own = q_raw < a.q_blk;  // rows past q_blk repeat the last row and write nothing
  const long long row = (long long)bh * a.q_blk + (own ? q_raw : a.q_blk - 1);
  const bool big = a.flags & RS_BF16, track = a.flags & RS_TRACK_BEST;
  const bool maxim = a.flags & RS_MAXIMIZE, inv = a.flags & RS_INVERT_CUT;
  const bool renorm = !(a.flags & RS_NO_RENORM);

  const float* Mh = a.M + (long long)(bh % a.H) * 4096;
  for (int e = threadIdx.x; e < 4096; e += TPB) M32T[(e & 63) * 64 + (e >> 6)] = Mh[e];
  const float* Arow = a.A + row * kb_p;
  for (int k = w * 64 + lane; k < Td * 64; k += W * 64) PbL[k] = k < kb_p ? rs_bf(Arow[k], big) : 0.0f;
  for (int e = w * 64 + lane; e < 512; e += W * 64) hist2[e] = 0;
  __syncthreads();

  // ---- V tiles: rows 64t..64t+63 of the head (rows past kb_p repeat the last one), 16-byte
  // chunk c of row r at chunk position c ^ (r & (CPR-1)): lanes over the dims of one row
  // and lanes over the rows reading one chunk (ds_read_b128) are both conflict-free
  const unsigned char* Vh = reinterpret_cast<const unsigned char*>(a.Vp) + (long long)bh * kb_p * (CPR * 16);
  auto tile_dma = [&](float4* buf, int t) {
    // t through an empty asm: the addresses are then formed here, each call, instead of
    // being hoisted out of the round loop and kept live for every tile
    asm volatile("" : "+s"(t));
    // the tile's TB 16-byte chunks: chunk jj*TPB + thread (the whole waves below TB)
#pragma unroll
    for (int jj = 0; jj < (TB + TPB - 1) / TPB; ++jj) {
      if (jj * TPB + wid * 64 < TB) {
        const int s = jj * TPB + threadIdx.x, r = s / CPR, c = (s % CPR) ^ (r & (CPR - 1));
        const int vrow = min(64 * t + r, kb_p - 1);
        rs_gl_lds16(Vh + (long long)vrow * (CPR * 16) + 16 * c, buf + jj * TPB + wid * 64);
      }
    }
  };
  // V[r][d] of a tile for d = lane (the chains): the lane's word within row r0 = r % 16,
  // the same for r0 + 16j (the swizzle uses the low bits of r only)
  auto vword = [&](int r0) -> int {
    return B16 ? r0 * 32 + (((lane >> 3) ^ (r0 & 7)) << 2) + ((lane >> 1) & 3)
               : r0 * 64 + (((lane >> 2) ^ (r0 & 15)) << 2) + (lane & 3);
  };
  const uint32_t vsel = (lane & 1) ? 0x03020c0cu : 0x01000c0cu;  // B16: this lane's half as fp32
  auto vdim = [&](uint32_t word) -> float { return __uint_as_float(__builtin_amdgcn_perm(0u, word, vsel)); };
  // Collective pass over T tiles, three buffers (tile t in buffer t % 3), the DMA two tiles
  // ahead. Step t: wait for tile t (tile t+1 may stay in flight), barrier, pre(t) -- every
  // access to dynamic LDS of the step --, the DMA of tile t+2 into the buffer of tile t-1,
  // then body(tile, t), which reads the static tile buffer only: the compiler keeps an LDS
  // access it cannot tell apart from an LDS-DMA target behind a wait for that DMA.
  constexpr int DPT = (TB + TPB - 1) / TPB;  // DMA instructions per tile per wave (at most)
  auto step3 = [&](int T, int t, const float4* cur, float4* ahead, auto&& pre, auto&& body) {
    if (t + 1 < T) rs_wait_vmcnt<DPT>();
    else rs_wait_vmcnt<0>();
    rs_barrier();
    pre(t);
    if (t + 2 < T) tile_dma(ahead, t + 2);
    body(cur, t);
  };
  auto stream_begin = [&](int T) {
    rs_wait_vmcnt<0>();  // no other vector-memory operation of the wave is outstanding
    rs_barrier();        // every wave is done with the tile buffers of the previous collective
    tile_dma(tb0, 0);
    if (T > 1) tile_dma(tb1, 1);
  };

  // ---- SUMK over keys 0..64*T-1 of tile-streamed V: returns (dot = sum_k pd_k V[k][lane],
  // sum = sum_k pd_k), pd_k = PbL[k] (masked by the 64-bit word mask(t) of tile t when MASKED).
  // Collective: every wave of the workgroup calls it with the same T.
  auto sumk = [&](int T, auto masked_tag, const unsigned long long* mask, float& dot, float& sum) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    int voff[C];
#pragma unroll
    for (int cc = 0; cc < C; ++cc) voff[cc] = vword(C * w + cc);
    float acc[C], sps[C];
#pragma unroll
    for (int cc = 0; cc < C; ++cc) acc[cc] = sps[cc] = 0.0f;
    // W = 4: this wave's pd of the tile (rows 16j + C*w + cc) read in pre(); wider waves (more
    // classes each) read them in the body, as registers would not hold them
    constexpr bool PRE = W == 4;
    float pt[PRE ? 4 * C : 1];
    auto pre = [&](int t) {
      if constexpr (!PRE) return;
      unsigned long long mw = 0;
      if constexpr (MASKED) mw = mask[t];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int cc = 0; cc < C; cc += 4) {
          const float4 p4 = *reinterpret_cast<const float4*>(PbL + 64 * t + 16 * j + C * w + cc);
          pt[C * j + cc] = p4.x;
          pt[C * j + cc + 1] = p4.y;
          pt[C * j + cc + 2] = p4.z;
          pt[C * j + cc + 3] = p4.w;
        }
        if constexpr (MASKED) {
          // the drop bits of the wave's 16 rows of group j, in a uniform register
          const uint32_t half = __builtin_amdgcn_readfirstlane(j < 2 ? (uint32_t)mw : (uint32_t)(mw >> 32));
          const uint32_t bits = half >> (16 * (j & 1) + C * w);
#pragma unroll
          for (int cc = 0; cc < C; ++cc) pt[C * j + cc] = ((bits >> cc) & 1u) ? pt[C * j + cc] : 0.0f;
        }
      }
    };
    auto body = [&](const float4* tile, int t) {
      const float* tf = reinterpret_cast<const float*>(tile);
      const uint32_t* tw = reinterpret_cast<const uint32_t*>(tile);
      unsigned long long mw = 0;
      if constexpr (MASKED && !PRE) mw = mask[t];
      // with 8 or 16 classes per wave the four 16-row groups run as a loop: unrolled, their
      // loads would be paired across groups and all issued ahead of the arithmetic
#pragma unroll(C > 4 ? 1 : 4)
      for (int j = 0; j < 4; ++j) {
        float pv[C], vv[C];
        if constexpr (PRE) {
#pragma unroll
          for (int cc = 0; cc < C; ++cc) pv[cc] = pt[(C * j + cc) % (PRE ? 4 * C : 1)];
        } else {
#pragma unroll
          for (int cc = 0; cc < C; cc += 4) {
            const float4 p4 = *reinterpret_cast<const float4*>(PbL + 64 * t + 16 * j + C * w + cc);
            pv[cc] = p4.x;
            pv[cc + 1] = p4.y;
            pv[cc + 2] = p4.z;
            pv[cc + 3] = p4.w;
          }
          if constexpr (MASKED) {
            const uint32_t half = __builtin_amdgcn_readfirstlane(j < 2 ? (uint32_t)mw : (uint32_t)(mw >> 32));
            const uint32_t bits = half >> (16 * (j & 1) + C * w);
#pragma unroll
            for (int cc = 0; cc < C; ++cc) pv[cc] = ((bits >> cc) & 1u) ? pv[cc] : 0.0f;
          }
        }
#pragma unroll
        for (int cc = 0; cc < C; ++cc) vv[cc] = B16 ? vdim(tw[voff[cc] + 512 * j]) : tf[voff[cc] + 1024 * j];
#pragma unroll
        for (int cc = 0; cc < C; ++cc) {
          acc[cc] = fmaf(pv[cc], vv[cc], acc[cc]);
          sps[cc] = sps[cc] + pv[cc];
        }
      }
    };
    stream_begin(T);
    int t = 0;
    for (; t + 3 <= T; t += 3) {
      step3(T, t, tb0, tb2, pre, body);
      step3(T, t + 1, tb1, tb0, pre, body);
      step3(T, t + 2, tb2, tb1, pre, body);
    }
    if (t < T) step3(T, t, tb0, tb2, pre, body);
    if (t + 1 < T) step3(T, t + 1, tb1, tb0, pre, body);
    // the wave's subtree of classes, then the W subtrees
    chain[w * 65 + lane] = rs_tree<C>(acc);
    if (lane == 0) chain[w * 65 + 64] = rs_tree<C>(sps);
    rs_barrier();
    float pa[W], ps[W];
#pragma unroll
    for (int u = 0; u < W; ++u) {
      pa[u] = chain[u * 65 + lane];
      ps[u] = chain[u * 65 + 64];
    }
    dot = rs_tree<W>(pa);
    sum = rs_tree<W>(ps);
  };

  // ---- DOT4x16 of every candidate with vec (this wave's vector in LDS): out[i] for slot i.
  // Per tile (64 candidates), each wave of a row takes CH of the four 16-dim chunks for all
  // 64 candidates (lane = candidate); the owner wave of the tile (t % W) combines the W
  // partials one step later. Collective.
  auto products = [&](const float* vec, float (&out)[NS]) {
#pragma unroll
    for (int i = 0; i < NS; ++i) out[i] = 0.0f;
    // W = 4: this wave's chunk of vec in registers (read before any DMA of the pass); wider
    // waves read their chunks per tile
    constexpr bool VREG = W == 4;
    float vr[16];
    if constexpr (VREG) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 v4 = *reinterpret_cast<const float4*>(vec + 16 * w + 4 * q4);
        vr[4 * q4] = v4.x;
        vr[4 * q4 + 1] = v4.y;
        vr[4 * q4 + 2] = v4.z;
        vr[4 * q4 + 3] = v4.w;
      }
    }
    auto combine = [&](int t) -> float {
      float p[W];
#pragma unroll
      for (int u = 0; u < W; ++u) p[u] = prod[((t & 1) * W + u) * 64 + lane];
      return rs_tree<W>(p);
    };
    // the partial of tile t is held in a register, written to prod[t & 1] at step t+1 and
    // combined by the owner wave (t % W) at step t+2
    float held = 0.0f;
    stream_begin(G);
#pragma unroll
    for (int t = 0; t < NS * W; ++t) {
      if (t < G) {
        const float4* cur = t % 3 == 0 ? tb0 : (t % 3 == 1 ? tb1 : tb2);
        float4* ahead = t % 3 == 0 ? tb2 : (t % 3 == 1 ? tb0 : tb1);
        auto pre = [&](int) {
          if (t >= 1) prod[(((t - 1) & 1) * W + w) * 64 + lane] = held;
          if (t >= 2 && w == (t - 2) % W) out[(t - 2) / W] = combine(t - 2);
        };
        auto body = [&](const float4* tile, int) {
          float part[CH];
#pragma unroll
          for (int ch = 0; ch < CH; ++ch) {
            const int c = CH * w + ch;  // dims 16c..16c+15 of candidate 64t + lane
            float vc[16];
            if constexpr (VREG) {
#pragma unroll
              for (int u = 0; u < 16; ++u) vc[u] = vr[u];
            } else {
#pragma unroll
              for (int q4 = 0; q4 < 4; ++q4) {
                const float4 v4 = *reinterpret_cast<const float4*>(vec + 16 * c + 4 * q4);
                vc[4 * q4] = v4.x;
                vc[4 * q4 + 1] = v4.y;
                vc[4 * q4 + 2] = v4.z;
                vc[4 * q4 + 3] = v4.w;
              }
            }
            float sacc = 0.0f;
            if constexpr (B16) {
              uint4 q[2];
#pragma unroll
              for (int e = 0; e < 2; ++e)
                q[e] = *reinterpret_cast<const uint4*>(tile + lane * 8 + ((2 * c + e) ^ (lane & 7)));
#pragma unroll
              for (int e = 0; e < 2; ++e) {
                float x[8];
                unpack_bf16x8(q[e], x);
#pragma unroll
                for (int u = 0; u < 8; ++u) sacc = fmaf(x[u], vc[8 * e + u], sacc);
              }
            } else {
              float4 q[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) q[e] = tile[lane * 16 + ((4 * c + e) ^ (lane & 15))];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                sacc = fmaf(q[e].x, vc[4 * e], sacc);
                sacc = fmaf(q[e].y, vc[4 * e + 1], sacc);
                sacc = fmaf(q[e].z, vc[4 * e + 2], sacc);
                sacc = fmaf(q[e].w, vc[4 * e + 3], sacc);
              }
            }
            part[ch] = sacc;
            if constexpr (CH > 1) __builtin_amdgcn_sched_barrier(0);
          }
          held = rs_tree<CH>(part);
        };
        step3(G, t, cur, ahead, pre, body);
      }
    }
    // the last tile's partial, then the last two tiles' combines
#pragma unroll
    for (int t = 0; t < NS * W; ++t)
      if (t == G - 1) prod[((t & 1) * W + w) * 64 + lane] = held;
    rs_barrier();
#pragma unroll
    for (int t = 0; t < NS * W; ++t)
      if (t >= G - 2 && t < G && w == t % W) out[t / W] = combine(t);
  };

  // ---- sum of a wave-uniform count over the row's W waves (counter slot `slot`); one barrier
  auto row_sum = [&](int v, int slot) -> int {
    if (lane == 0) ints[4 * slot + w] = v;
    rs_barrier();
    int s = 0;
#pragma unroll
    for (int u = 0; u < W; ++u) s += ints[4 * slot + u];
    return s;
  };

  // ---- exact top-m of the row's `valid` candidates by order key, ties to the lowest index:
  // MSB-first radix select, one 256-bin histogram per 8-bit digit shared by the row's W
  // waves (double-buffered), then the ties at the threshold ranked across the candidate
  // groups in index order. Collective: the digit loop runs until no row of the workgroup
  // needs another digit.
  auto top_m = [&](const uint32_t (&key)[NS], uint32_t valid, int m) -> uint32_t {
    int c = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) c += __popcll(__ballot((valid >> i) & 1u));
    const int n_valid = row_sum(c, 0);
    const bool sel_all = n_valid <= m;  // includes m >= n_valid; m <= 0 selects nothing
    bool active = m > 0 && !sel_all;
    const bool searched = active;
    uint32_t prefix = 0u, pmask = 0u;
    int need = m;
    for (int dg = 0; dg < 4; ++dg) {
      const int shift = 24 - 8 * dg;
      int* hist = hist2 + 256 * (dg & 1);
      if (active) {
#pragma unroll
        for (int i = 0; i < NS; ++i)
          if (((valid >> i) & 1u) && (key[i] & pmask) == prefix) atomicAdd(&hist[(key[i] >> shift) & 255u], 1);
      }
      rs_barrier();
      if (active) {
        // lane l owns bins 4l..4l+3; suffix counts S(t) = #{digit >= t}
        const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
        const int incl = wave_scan_sum_i(h0 + h1 + h2 + h3);
        const int above = (int)lane63((uint32_t)incl) - incl;
        const int s3 = above + h3, s2 = s3 + h2, s1 = s2 + h1, s0 = s1 + h0;
        int t = -1, gt = 0, inbin = 0;
        if (s3 >= need && above < need) t = 3, gt = above, inbin = h3;
        else if (s2 >= need && s3 < need) t = 2, gt = s3, inbin = h2;
        else if (s1 >= need && s2 < need) t = 1, gt = s2, inbin = h1;
        else if (s0 >= need && s1 < need) t = 0, gt = s1, inbin = h0;
        const unsigned long long hit = __ballot(t >= 0);
        const int src = hit ? __ffsll((long long)hit) - 1 : 63;  // uniform
        const int digit = __builtin_amdgcn_readlane(4 * lane + t, src), n_gt = __builtin_amdgcn_readlane(gt, src),
                  n_in = __builtin_amdgcn_readlane(inbin, src);
        need -= n_gt;
        prefix |= (uint32_t)digit << shift;
        pmask |= 255u << shift;
        // every key of the threshold bin is taken: the keys above prefix (lower digits
        // zero) and the need >= (keys equal to prefix) ties below select exactly the set of
        // the full descent, so the remaining digits are skipped
        if (n_in == need) active = false;
      }
      // the other histogram (last read by the previous digit's scan) is cleared for the next
      int* nxt = hist2 + 256 * ((dg + 1) & 1);
      for (int e = w * 64 + lane; e < 256; e += W * 64) nxt[e] = 0;
      if (w == 0 && lane == 0) rowflag[dg & 1][rloc] = active ? 1 : 0;
      rs_barrier();
      int any = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) any |= rowflag[dg & 1][r];
      if (!any) break;
    }
    // a histogram of the next top_m starts clear: clear the one the loop may have left set
    for (int e = w * 64 + lane; e < 512; e += W * 64) hist2[e] = 0;
    // ties at the threshold: ranked by candidate index across the groups g = W*i + w
    const uint32_t thr = prefix;
    unsigned long long be[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      be[i] = __ballot(searched && ((valid >> i) & 1u) && key[i] == thr);
      if (lane == 0 && W * i + w < G) eqcnt[W * i + w] = __popcll(be[i]);
    }
    rs_barrier();
    const int ec = lane < G ? eqcnt[lane] : 0;
    const int pre = wave_scan_sum_i(ec) - ec;  // ties in the groups before group `lane`
    const unsigned long long lower = lane ? (~0ull >> (64 - lane)) : 0ull;
    uint32_t sel = 0u;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const bool v = (valid >> i) & 1u;
      const int rank = __builtin_amdgcn_readlane(pre, min(W * i + w, 63)) + __popcll(be[i] & lower);
      if (v && (key[i] > thr || (key[i] == thr && rank < need))) sel |= 1u << i;
    }
    if (!searched) sel = (sel_all && m > 0) ? valid : 0u;
    return sel;
  };

  // ---- the row's candidates ------------------------------------------------------
  const int n_valid_groups = G;
  uint32_t cand_bits = 0u;
  float Pb[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int k = 64 * (W * i + w) + lane;
    const bool c = W * i + w < n_valid_groups && k < n_cand;
    if (c) cand_bits |= 1u << i;
    Pb[i] = c ? PbL[k] : 0.0f;
  }

  // ---- dense reference: v_bar_query = big(P @ v_bar), total mass big(sum P) ----------
  float vq, tm;
  {
    float d, s;
    sumk(Td, std::false_type{}, nullptr, d, s);
    vq = rs_bf(d, big);
    tm = rs_bf(s, big);
  }
  vqs[lane] = vq;
  __builtin_amdgcn_wave_barrier();
  // quadratic_deviation's query side: Mvq = big(Mb vq), term_q = big(sum big(Mvq*vq))
  const float mvq = rs_bf(rs_dot_col<true>(M32T + lane, vqs, big), big);
  t0[lane] = mvq;
  t1[lane] = rs_bf(mvq * vq, big);
  __builtin_amdgcn_wave_barrier();
  const float tq = rs_bf(rs_sum64(t1), big);
  // s, s_cut, s^2 per candidate
  float ssq[NS];
  uint32_t key[NS];
  {
    float cr[NS];
    products(t0, cr);  // cross = Mvq . v_k
    const float* tkey = a.termk + (long long)bh * n_cand;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int k = 64 * (W * i + w) + lane;
      float sc = 0.0f;
      ssq[i] = 0.0f;
      if ((cand_bits >> i) & 1u) {
        const float c2 = rs_bf(2.0f * rs_bf(cr[i], big), big);
        float qd = rs_bf(rs_bf(tq - c2, big) + tkey[k], big);
        qd = qd < 0.0f ? 0.0f : qd;
        const float sq = rs_bf(sqrtf(qd), big);
        const float s = rs_bf(Pb[i] * sq, big);
        float om = rs_bf(1.0f - Pb[i], big);
        om = rs_bf(om < 1e-4f ? 1e-4f : om, big);
        sc = renorm ? rs_bf(s / om, big) : s;
        ssq[i] = rs_bf(s * s, big);
        if (a.s_out && own) a.s_out[row * n_cand + k] = s;
      }
      key[i] = rs_key(inv ? -sc : sc);
    }
  }
  const int nts = a.nts[row];
  const int nkeep = nts < 0 ? 0 : (nts > n_cand ? n_cand : nts);
  uint32_t drop = cand_bits & ~top_m(key, cand_bits, nkeep);

  // ---- the objective of the initial cut: sum_Pd and Pd @ v_bar over the dropped candidates
  // (SUMK), carried through the rounds afterwards
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const unsigned long long b = __ballot((drop >> i) & 1u);
    if (lane == 0 && W * i + w < G) dmask[W * i + w] = b;
  }
  float sp_raw, mv_raw;
  sumk(G, std::true_type{}, dmask, mv_raw, sp_raw);
  // J, ||g||^2_M and K of the carried state; leaves Mg in t3 (projected.py:859-868, 903-918)
  float gn = 0.0f, Kk = 1.0f;
  auto objective = [&]() -> float {
    const float sp = rs_bf(sp_raw, big);
    const float g = sp * vq - rs_bf(mv_raw, big);
    __builtin_amdgcn_wave_barrier();
    t1[lane] = g;
    __builtin_amdgcn_wave_barrier();
    const float mg = rs_dot_col<false>(M32T + lane, t1, big);
    t2[lane] = g * mg;  // products of ||g||^2_M
    t3[lane] = mg;
    __builtin_amdgcn_wave_barrier();
    const float n2 = rs_sum64(t2);
    float K = tm - sp;
    K = K < 1e-6f ? 1e-6f : K;
    gn = n2;
    Kk = K;
    return n2 / (K * K);
  };
  // the carried state moves by the round's change: the restored (pd = -P) and compensated
  // (pd = +P) candidates summed in four classes k mod 4, class c by wave c % W as a
  // sequential chain over increasing k; the class sums are combined as (d0 + d1) + (d2 + d3)
  // and added. Every wave of the row adds the same change. Collective.
  auto carry = [&]() {
    constexpr int CW = 4 / W;  // classes per wave
    int* wl = reinterpret_cast<int*>(t2);  // this wave's pending candidates (64 entries)
#pragma unroll
    for (int ci = 0; ci < CW; ++ci) {
      const int c = w + W * ci;
      const unsigned long long cls = 0x1111111111111111ull << c;
      float am = 0.0f, as = 0.0f;
      int g = 0;
      unsigned long long m = 0ull, mc = 0ull;
      for (;;) {
        // the next (up to) 64 changed candidates of the class, in index order; bit 30 = compensated
        int n = 0;
        while (n < 64) {
          if (!m) {
            if (g >= G) break;
            m = (rmask[g] | cmask[g]) & cls;
            mc = cmask[g];
            ++g;
            continue;
          }
          const int j = __builtin_ctzll(m);
          m &= m - 1;
          if (lane == 0) wl[n] = (64 * (g - 1) + j) | (((mc >> j) & 1ull) ? 0x40000000 : 0);
          ++n;
        }
        if (n == 0) break;
        __builtin_amdgcn_wave_barrier();
        for (int e0 = 0; e0 < n; e0 += 16) {
          int code[16];
          float vv[16], pp[16];
#pragma unroll
          for (int b = 0; b < 16; ++b) {
            code[b] = e0 + b < n ? wl[e0 + b] : 0;
            const int k = code[b] & 0x3fffffff;
            const long long o = ((long long)bh * kb_p + k) * 64 + lane;
            vv[b] = B16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(a.Vp)[o] << 16)
                        : reinterpret_cast<const float*>(a.Vp)[o];
            pp[b] = PbL[k];
          }
#pragma unroll
          for (int b = 0; b < 16; ++b) {
            if (e0 + b < n) {
              const float pd = (code[b] & 0x40000000) ? pp[b] : -pp[b];
              as = as + pd;
              am = fmaf(pd, vv[b], am);
            }
          }
        }
        __builtin_amdgcn_wave_barrier();
        if (n < 64) break;
      }
      dpart[c * 65 + lane] = am;
      if (lane == 0) dpart[c * 65 + 64] = as;
    }
    rs_barrier();
    mv_raw = mv_raw + ((dpart[lane] + dpart[65 + lane]) + (dpart[130 + lane] + dpart[195 + lane]));
    sp_raw = sp_raw + ((dpart[64] + dpart[129]) + (dpart[194] + dpart[259]));
  };

  float J = objective();
  uint32_t best = drop;
  float best_obj = J;
  double remaining = a.restore_frac;  // the reference forms the round fractions in double
  for (int it = 0; it < a.n_iters; ++it) {
    const double frac = remaining * a.decay;
    remaining -= frac;
    const int pic0 = (int)rintf((float)frac * (float)nts);
    if (track && (maxim ? J > best_obj : J < best_obj)) {
      best_obj = J;
      best = drop;
    }
    // term_q of the round, big(Mg)
    __builtin_amdgcn_wave_barrier();
    t2[lane] = vq * t3[lane];
    t0[lane] = rs_bf(t3[lane], big);
    __builtin_amdgcn_wave_barrier();
    const float tqb = rs_bf(rs_sum64(t2), big);
    float tk[NS];
    products(t0, tk);  // term_k = v_k . big(Mg)
    // restore quality of the dropped (higher is better), then the compensation quality of
    // the kept, one key array at a time
    auto quality = [&](int i, bool restore_side) -> float {
      const float raw = rs_bf(Pb[i] * rs_bf(rs_bf(tk[i], big) - tqb, big), big);
      const float q = restore_side ? rs_knorm(gn, Kk, 2.0f * raw + ssq[i], Pb[i])
                                   : rs_knorm(gn, Kk, ssq[i] - 2.0f * raw, -Pb[i]);
      return maxim ? -q : q;
    };
    uint32_t qkey[NS];
    bool ben = false;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const float r = quality(i, true);
      if ((drop >> i) & 1u) ben |= r > 0.0f;
      qkey[i] = rs_key(r);
    }
    // beneficial iff some drop candidate has quality > 0
    int nd = 0, nk = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      nd += __popcll(__ballot((drop >> i) & 1u));
      nk += __popcll(__ballot(((cand_bits & ~drop) >> i) & 1u));
    }
    const bool beneficial = row_sum(__ballot(ben) != 0ull ? 1 : 0, 1) > 0;
    const int n_drop = row_sum(nd, 2), n_kept = row_sum(nk, 3);
    int pic = pic0;
    if (beneficial && pic < 1) pic = 1;
    int cnt = pic < n_drop ? pic : n_drop;
    cnt = cnt < n_kept ? cnt : n_kept;
    if (!beneficial) cnt = 0;
    const uint32_t restore = top_m(qkey, drop, cnt);
#pragma unroll
    for (int i = 0; i < NS; ++i) qkey[i] = rs_key(quality(i, false));
    const uint32_t comp = top_m(qkey, cand_bits & ~drop, cnt);
    drop = (drop & ~restore) | comp;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const unsigned long long br = __ballot((restore >> i) & 1u), bc = __ballot((comp >> i) & 1u);
      if (lane == 0 && W * i + w < G) {
        rmask[W * i + w] = br;
        cmask[W * i + w] = bc;
      }
    }
    rs_barrier();
    carry();
    J = objective();
  }
  float fin = J;
  if (track && !(maxim ? fin > best_obj : fin < best_obj)) {
    drop = best;
    fin = best_obj;
  }
  if (a.obj && lane == 0 && w == 0 && own) a.obj[row] = fin;
  float* out = a.rank_key + row * n_cand;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int k = 64 * (W * i + w) + lane;
    if (((cand_bits >> i) & 1u) && own) out[k] = ((drop >> i) & 1u) ? 0.0f : 1.0f;
  }
}

// ---- short bf16 rows: one wave per row, the head's V resident in LDS -----------------
// When a head's V (bf16, big mode) fits in LDS next to the rows' scratch, the row kernel
// runs each row on one wave with no barriers at all: V is read from LDS by every pass,
// and the selections are wave-local. Same operation order as k_restore_swap (the
// numerics contract at the top of this file), so both kernels return the same bits.
// V in LDS: bf16 pairs, word w of row k at k*33 + w (one pad word per row): lanes over the
// 64 dims of one key block read 32 consecutive words, lanes over 32 consecutive key blocks
// at one dim pair hit 32 distinct banks, and a batch of consecutive rows is one lane base
// plus immediate offsets.
#define RS_VROW 33
#define RSR_WAVES 8
#define RSR_LDS_BYTES 163840
// LDS words of the resident V, rounded up so that the per-wave scratch after it stays
// 16-byte aligned
__host__ __device__ __forceinline__ int rs_vw_words(int kb_p) { return (kb_p * RS_VROW + 3) & ~3; }
// floats of one wave's scratch: P [kb4], five 64-float vectors, the drop mask [NPL] u64
// (rounded to 16 bytes)
__host__ __device__ __forceinline__ int rsr_wave_floats(int kb_p, int npl) {
  return ((kb_p + 3) & ~3) + 5 * 64 + ((2 * npl + 3) & ~3);
}
__host__ __device__ __forceinline__ long long rsr_lds_bytes(int kb_p, int npl) {
  return 4LL * (4096 + rs_vw_words(kb_p) + RSR_WAVES * rsr_wave_floats(kb_p, npl));
}

// Exact top-m among `valid` lane elements of one wave by MSB-first radix select over the
// order keys (four 8-bit digits, a 256-bin histogram in the wave's LDS per digit), then
// ties at the threshold taken in candidate-index order.
template <int NPL>
__device__ __forceinline__ uint32_t rs_top_m_wave(const uint32_t (&key)[NPL], uint32_t valid, int m, int lane,
                                                  int* hist) {
  if (m <= 0) return 0u;
  int n_valid = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) n_valid += __popcll(__ballot((valid >> i) & 1u));
  if (n_valid <= m) return valid;
  uint32_t prefix = 0u, pmask = 0u;
  int need = m;  // still to take among the keys matching the fixed high digits
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[lane] = hist[lane + 64] = hist[lane + 128] = hist[lane + 192] = 0;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (((valid >> i) & 1u) && (key[i] & pmask) == prefix) atomicAdd(&hist[(key[i] >> shift) & 255u], 1);
    __builtin_amdgcn_wave_barrier();
    const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
    const int incl = wave_scan_sum_i(h0 + h1 + h2 + h3);
    const int above = (int)lane63((uint32_t)incl) - incl;
    const int s3 = above + h3, s2 = s3 + h2, s1 = s2 + h1, s0 = s1 + h0;
    int t = -1, gt = 0, inbin = 0;
    if (s3 >= need && above < need) t = 3, gt = above, inbin = h3;
    else if (s2 >= need && s3 < need) t = 2, gt = s3, inbin = h2;
    else if (s1 >= need && s2 < need) t = 1, gt = s2, inbin = h1;
    else if (s0 >= need && s1 < need) t = 0, gt = s1, inbin = h0;
    const unsigned long long hit = __ballot(t >= 0);
    const int src = hit ? __ffsll((long long)hit) - 1 : 63;  // uniform
    const int digit = __builtin_amdgcn_readlane(4 * lane + t, src), n_gt = __builtin_amdgcn_readlane(gt, src),
              n_in = __builtin_amdgcn_readlane(inbin, src);
    need -= n_gt;
    prefix |= (uint32_t)digit << shift;
    pmask |= 255u << shift;
    __builtin_amdgcn_wave_barrier();
    if (n_in == need) break;  // the threshold bin is taken whole: the same set as the full descent
  }
  const uint32_t thr = prefix;
  uint32_t sel = 0u;
  int before = 0;
  const unsigned long long lower = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool v = (valid >> i) & 1u;
    const bool eq = v && key[i] == thr;
    const unsigned long long be = __ballot(eq);
    const int rank = before + __popcll(be & lower);
    if ((v && key[i] > thr) || (eq && rank < need)) sel |= 1u << i;
    before += __popcll(be);
  }
  return sel;
}

// The rows of one head, RSR_WAVES rows per workgroup at a time, one wave each; candidate
// k = lane + 64*i in slot i (NPL slots, n_cand <= 64*NPL).
template <int NPL>
__global__ __launch_bounds__(64 * RSR_WAVES) void k_restore_swap_row(RsArgs a, int rows_per_wg) {
  extern __shared__ __align__(16) float sh[];
  float* M32T = sh;                                          // [64][64] M^T (fp32)
  uint32_t* vw = reinterpret_cast<uint32_t*>(sh + 4096);     // [kb_p][RS_VROW] bf16 pairs
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kb_p = a.kb_p, n_cand = a.n_cand;
  const int kb4 = (kb_p + 3) & ~3;
  float* wsh = sh + 4096 + rs_vw_words(kb_p) + w * rsr_wave_floats(kb_p, NPL);
  float* Pw = wsh;                  // [kb_p] big(P) of the row
  float* vqs = wsh + kb4;           // [64]
  float* t0 = vqs + 64;             // [64] scratch vectors; t0..t3 double as the
  float* t1 = t0 + 64;              //      256-bin selection histogram
  float* t2 = t1 + 64;
  float* t3 = t2 + 64;
  int* hist = reinterpret_cast<int*>(t0);
  unsigned long long* dmask = reinterpret_cast<unsigned long long*>(t3 + 64);  // [NPL]
  const int gx = gridDim.x, gl = blockIdx.x + gx * blockIdx.y;
  const bool xmap = (gridDim.y & 7) == 0;
  const int bh = xmap ? (gl & 7) + 8 * ((gl >> 3) / gx) : blockIdx.y;
  const int bgrp = xmap ? (gl >> 3) % gx : blockIdx.x;
  const bool track = a.flags & RS_TRACK_BEST, maxim = a.flags & RS_MAXIMIZE, inv = a.flags & RS_INVERT_CUT;
  const bool renorm = !(a.flags & RS_NO_RENORM);
  constexpr bool big = true;
  const float* Mh = a.M + (long long)(bh % a.H) * 4096;
  for (int e = threadIdx.x; e < 4096; e += 64 * RSR_WAVES) M32T[(e & 63) * 64 + (e >> 6)] = Mh[e];
  const uint32_t* Vp32 = reinterpret_cast<const uint32_t*>(a.Vp) + (long long)bh * kb_p * 32;  // bf16 pairs
  for (int e = threadIdx.x; e < kb_p * 32; e += 64 * RSR_WAVES) vw[(e >> 5) * RS_VROW + (e & 31)] = Vp32[e];
  __syncthreads();
  const uint32_t vsel = (lane & 1) ? 0x03020c0cu : 0x01000c0cu;
  auto vdim = [&](uint32_t word) -> float { return __uint_as_float(__builtin_amdgcn_perm(0u, word, vsel)); };
  auto vrow = [&](int k) -> float { return vdim(vw[k * RS_VROW + (lane >> 1)]); };
  const float* tkey = a.termk + (long long)bh * n_cand;
  const int nel = (n_cand + 63) >> 6;
  uint32_t cand_bits = 0u;
#pragma unroll
  for (int i = 0; i < NPL; ++i)
    if (lane + 64 * i < n_cand) cand_bits |= 1u << i;

  // SUMK over k < n of pd_k = Pw[k] (times the drop bit of k when MASKED): sixteen class
  // chains, one per row of a 16-row batch, all of a batch's LDS reads issued first
  auto sumk = [&](int n, auto masked_tag, float& sum, float& dot) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    float acc[16], sps[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) acc[u] = sps[u] = 0.0f;
    auto bits_of = [&](int k0) -> uint32_t {  // drop bits of keys k0..k0+15 (k0 % 16 == 0)
      if constexpr (!MASKED) return 0xffffu;
      const unsigned long long mw = dmask[k0 >> 6];
      const uint32_t half = (k0 & 32) ? (uint32_t)(mw >> 32) : (uint32_t)mw;
      return (__builtin_amdgcn_readfirstlane(half) >> (k0 & 16)) & 0xffffu;
    };
    const int n16 = n & ~15;
    for (int k0 = 0; k0 < n16; k0 += 16) {
      const uint32_t* vb = vw + k0 * RS_VROW + (lane >> 1);
      uint32_t wv[16];
      float pv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) wv[u] = vb[u * RS_VROW];
#pragma unroll
      for (int u = 0; u < 16; u += 4) {
        const float4 p4 = *reinterpret_cast<const float4*>(Pw + k0 + u);
        pv[u] = p4.x;
        pv[u + 1] = p4.y;
        pv[u + 2] = p4.z;
        pv[u + 3] = p4.w;
      }
      const uint32_t bits = bits_of(k0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float pd = ((bits >> u) & 1u) ? pv[u] : 0.0f;
        acc[u] = fmaf(pd, vdim(wv[u]), acc[u]);
        sps[u] = sps[u] + pd;
      }
    }
    if (n16 < n) {
      const uint32_t bits = bits_of(n16);
#pragma unroll
      for (int u = 0; u < 15; ++u) {
        if (n16 + u < n) {
          const float pd = ((bits >> u) & 1u) ? Pw[n16 + u] : 0.0f;
          acc[u] = fmaf(pd, vrow(n16 + u), acc[u]);
          sps[u] = sps[u] + pd;
        }
      }
    }
    dot = rs_tree<16>(acc);
    sum = rs_tree<16>(sps);
  };
  // DOT4x16 of every candidate with vec (LDS, broadcast): NS = nel rounded up to a multiple
  // of 4 slots is a compile-time count (one instance per value), so no slot carries a
  // runtime guard; the last four slots read rows clamped to n_cand - 1 (their products
  // are never used). The words of dim pair p+1 are read while pair p is accumulated.
  auto products = [&](const float* vec, float (&out)[NPL]) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) out[i] = 0.0f;
    auto run = [&](auto ns_tag) {
      constexpr int NS = decltype(ns_tag)::value;
      const uint32_t* vl = vw + lane * RS_VROW;
      const uint32_t* vlast[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vlast[j] = vw + min(lane + 64 * (NS - 4 + j), n_cand - 1) * RS_VROW;
      uint32_t wa[NS], wb[NS];
      float acc[NS], s01[NS], s2[NS];
      auto load_pair = [&](int p, uint32_t(&wv)[NS]) {
#pragma unroll
        for (int i = 0; i < NS - 4; ++i) wv[i] = vl[64 * RS_VROW * i + p];
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[NS - 4 + j] = vlast[j][p];
      };
      auto use_pair = [&](int p, const uint32_t(&wv)[NS]) {
        const float m0 = vec[2 * p], m1 = vec[2 * p + 1];
#pragma unroll
        for (int i = 0; i < NS; ++i)
          acc[i] = fmaf(m1, __uint_as_float(wv[i] & 0xffff0000u), fmaf(m0, __uint_as_float(wv[i] << 16), acc[i]));
      };
      load_pair(0, wa);
#pragma unroll
      for (int c = 0; c < 4; ++c) {  // dims 16c..16c+15 = pairs 8c..8c+7
#pragma unroll
        for (int i = 0; i < NS; ++i) acc[i] = 0.0f;
        for (int p = 8 * c; p < 8 * c + 8; p += 2) {
          load_pair(p + 1, wb);
          __builtin_amdgcn_sched_barrier(0);
          use_pair(p, wa);
          if (p + 2 < 32) load_pair(p + 2, wa);
          __builtin_amdgcn_sched_barrier(0);
          use_pair(p + 1, wb);
        }
#pragma unroll
        for (int i = 0; i < NS; ++i) {
          if (c == 0) s01[i] = acc[i];
          else if (c == 1) s01[i] = s01[i] + acc[i];
          else if (c == 2) s2[i] = acc[i];
          else out[i] = s01[i] + (s2[i] + acc[i]);
        }
      }
    };
    const int ng = (nel + 3) >> 2;  // wave-uniform
    if (ng <= 1) run(std::integral_constant<int, 4>{});
    if constexpr (NPL >= 8) {
      if (ng == 2) run(std::integral_constant<int, 8>{});
    }
    if constexpr (NPL >= 12) {
      if (ng == 3) run(std::integral_constant<int, 12>{});
    }
  };

  const int q_begin = bgrp * rows_per_wg, q_end = min(a.q_blk, (bgrp + 1) * rows_per_wg);
  for (int q = q_begin + w; q < q_end; q += RSR_WAVES) {
    const long long row = (long long)bh * a.q_blk + q;
    const float* Arow = a.A + row * kb_p;
    for (int k = lane; k < kb_p; k += 64) Pw[k] = rs_bf(Arow[k], big);
    float Pb[NPL], ssq[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int k = lane + 64 * i;
      Pb[i] = k < n_cand ? rs_bf(Arow[k], big) : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();
    float vq, tm;
    {
      float d, sm;
      sumk(kb_p, std::false_type{}, sm, d);
      vq = rs_bf(d, big);
      tm = rs_bf(sm, big);
    }
    vqs[lane] = vq;
    __builtin_amdgcn_wave_barrier();
    const float mvq = rs_bf(rs_dot_col<true>(M32T + lane, vqs, big), big);
    t0[lane] = mvq;
    t1[lane] = rs_bf(mvq * vq, big);
    __builtin_amdgcn_wave_barrier();
    const float tq = rs_bf(rs_sum64(t1), big);
    uint32_t key[NPL];
    {
      float cr[NPL];
      products(t0, cr);  // cross = Mvq . v_k
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const int k = lane + 64 * i;
        float sc = 0.0f;
        ssq[i] = 0.0f;
        if (i < nel && k < n_cand) {
          const float c2 = rs_bf(2.0f * rs_bf(cr[i], big), big);
          float qd = rs_bf(rs_bf(tq - c2, big) + tkey[k], big);
          qd = qd < 0.0f ? 0.0f : qd;
          const float sq = rs_bf(sqrtf(qd), big);
          const float sv = rs_bf(Pb[i] * sq, big);
          float om = rs_bf(1.0f - Pb[i], big);
          om = rs_bf(om < 1e-4f ? 1e-4f : om, big);
          sc = renorm ? rs_bf(sv / om, big) : sv;
          ssq[i] = rs_bf(sv * sv, big);
          if (a.s_out) a.s_out[row * n_cand + k] = sv;
        }
        key[i] = rs_key(inv ? -sc : sc);
      }
    }
    const int nts = a.nts[row];
    const int nkeep = nts < 0 ? 0 : (nts > n_cand ? n_cand : nts);
    __builtin_amdgcn_wave_barrier();
    uint32_t drop = cand_bits & ~rs_top_m_wave<NPL>(key, cand_bits, nkeep, lane, hist);
    // the objective of the initial cut (SUMK over the dropped candidates), then carried
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const unsigned long long b = __ballot((drop >> i) & 1u);
      if (lane == 0) dmask[i] = b;
    }
    __builtin_amdgcn_wave_barrier();
    float sp_raw, mv_raw;
    sumk(n_cand, std::true_type{}, sp_raw, mv_raw);
    float gn = 0.0f, Kk = 1.0f;
    auto objective = [&]() -> float {
      const float sp = rs_bf(sp_raw, big);
      const float g = sp * vq - rs_bf(mv_raw, big);
      __builtin_amdgcn_wave_barrier();
      t1[lane] = g;
      __builtin_amdgcn_wave_barrier();
      const float mg = rs_dot_col<false>(M32T + lane, t1, big);
      t2[lane] = g * mg;
      t3[lane] = mg;
      __builtin_amdgcn_wave_barrier();
      const float n2 = rs_sum64(t2);
      float K = tm - sp;
      K = K < 1e-6f ? 1e-6f : K;
      gn = n2;
      Kk = K;
      return n2 / (K * K);
    };
    float J = objective();
    uint32_t best = drop;
    float best_obj = J;
    double remaining = a.restore_frac;
    for (int it = 0; it < a.n_iters; ++it) {
      const double frac = remaining * a.decay;
      remaining -= frac;
      const int pic0 = (int)rintf((float)frac * (float)nts);
      if (track && (maxim ? J > best_obj : J < best_obj)) {
        best_obj = J;
        best = drop;
      }
      __builtin_amdgcn_wave_barrier();
      t2[lane] = vq * t3[lane];
      t0[lane] = rs_bf(t3[lane], big);
      __builtin_amdgcn_wave_barrier();
      const float tqb = rs_bf(rs_sum64(t2), big);
      float tk[NPL];
      products(t0, tk);  // term_k = v_k . big(Mg)
      auto quality = [&](int i, bool restore_side) -> float {
        const float raw = rs_bf(Pb[i] * rs_bf(rs_bf(tk[i], big) - tqb, big), big);
        const float qv = restore_side ? rs_knorm(gn, Kk, 2.0f * raw + ssq[i], Pb[i])
                                      : rs_knorm(gn, Kk, ssq[i] - 2.0f * raw, -Pb[i]);
        return maxim ? -qv : qv;
      };
      uint32_t qkey[NPL];
      float rmax = -__builtin_huge_valf();
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        qkey[i] = 0u;
        if (i < nel) {
          const float r = quality(i, true);
          if ((drop >> i) & 1u) rmax = fmaxf(rmax, r);
          qkey[i] = rs_key(r);
        }
      }
      const bool beneficial = __ballot(rmax > 0.0f) != 0ull;
      int n_drop = 0, n_kept = 0;
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        n_drop += __popcll(__ballot((drop >> i) & 1u));
        n_kept += __popcll(__ballot(((cand_bits & ~drop) >> i) & 1u));
      }
      int pic = pic0;
      if (beneficial && pic < 1) pic = 1;
      int cnt = pic < n_drop ? pic : n_drop;
      cnt = cnt < n_kept ? cnt : n_kept;
      if (!beneficial) cnt = 0;
      __builtin_amdgcn_wave_barrier();
      const uint32_t restore = rs_top_m_wave<NPL>(qkey, drop, cnt, lane, hist);
#pragma unroll
      for (int i = 0; i < NPL; ++i) qkey[i] = i < nel ? rs_key(quality(i, false)) : 0u;
      __builtin_amdgcn_wave_barrier();
      const uint32_t comp = rs_top_m_wave<NPL>(qkey, cand_bits & ~drop, cnt, lane, hist);
      drop = (drop & ~restore) | comp;
      // the carry: the change summed in four classes k mod 4, increasing k within a class
      float am[4], as[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        am[c] = 0.0f;
        as[c] = 0.0f;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
          const unsigned long long rb = __ballot((restore >> i) & 1u), cb = __ballot((comp >> i) & 1u);
          unsigned long long m = (rb | cb) & (0x1111111111111111ull << c);
          while (m) {
            const int j = __builtin_ctzll(m);
            m &= m - 1;
            const int k = 64 * i + j;
            const float pd = ((cb >> j) & 1ull) ? Pw[k] : -Pw[k];
            as[c] = as[c] + pd;
            am[c] = fmaf(pd, vrow(k), am[c]);
          }
        }
      }
      mv_raw = mv_raw + ((am[0] + am[1]) + (am[2] + am[3]));
      sp_raw = sp_raw + ((as[0] + as[1]) + (as[2] + as[3]));
      J = objective();
    }
    float fin = J;
    if (track && !(maxim ? fin > best_obj : fin < best_obj)) {
      drop = best;
      fin = best_obj;
    }
    if (a.obj && lane == 0) a.obj[row] = fin;
    float* out = a.rank_key + row * n_cand;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int k = lane + 64 * i;
      if (k < n_cand) out[k] = ((drop >> i) & 1u) ? 0.0f : 1.0f;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ============================================================================
// C ABI
// ============================================================================
template <int NS, int W, bool B16>
static int launch_rs(int BH, hipStream_t stream, const RsArgs& a) {
  const RsLds L = rs_lds(a.kb_p, a.n_cand, W, RsShape<B16>::WAVES);
  const size_t lds = (size_t)L.total;
  RESS_REQUIRE(hipFuncSetAttribute((const void*)k_restore_swap<NS, W, B16>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess,
               "ress_restore_swap: cannot reserve %zu bytes of LDS", lds);
  constexpr int R = RsShape<B16>::WAVES / W;
  hipLaunchKernelGGL((k_restore_swap<NS, W, B16>), dim3(cdiv(a.q_blk, R), BH), dim3(RsShape<B16>::TPB), lds, stream,
                     a);
  RESS_LAUNCHED("k_restore_swap");
  return 0;
}

// Waves per row by row length (64-candidate groups G): W = 1 up to RS_W1_MAX groups, 2 up
// to RS_W2_MAX, 4 above (up to 32 groups: 2048 candidates).
#ifndef RS_W1_MAX
#define RS_W1_MAX 8
#endif
#ifndef RS_W2_MAX
#define RS_W2_MAX 16
#endif
template <int W, bool B16>
static int launch_rs_w(int BH, hipStream_t stream, const RsArgs& a) {
  constexpr int LO = W == 1 ? 0 : (W == 2 ? RS_W1_MAX : RS_W2_MAX);  // groups below this run narrower
  constexpr int HI = W == 1 ? RS_W1_MAX : (W == 2 ? RS_W2_MAX : 32);
  const int ns = cdiv(cdiv(a.n_cand, 64), W);
  if constexpr (cdiv(LO + 1, W) <= 2) if (ns <= 2) return launch_rs<2, W, B16>(BH, stream, a);
  if constexpr (cdiv(LO + 1, W) <= 4 && cdiv(HI, W) > 2) if (ns <= 4) return launch_rs<4, W, B16>(BH, stream, a);
  if constexpr (cdiv(LO + 1, W) <= 6 && cdiv(HI, W) > 4) if (ns <= 6) return launch_rs<6, W, B16>(BH, stream, a);
  if constexpr (cdiv(LO + 1, W) <= 8 && cdiv(HI, W) > 6) if (ns <= 8) return launch_rs<8, W, B16>(BH, stream, a);
  if constexpr (cdiv(HI, W) > 8) if (ns <= 12) return launch_rs<12, W, B16>(BH, stream, a);
  if constexpr (cdiv(HI, W) > 12) return launch_rs<16, W, B16>(BH, stream, a);
  RESS_REQUIRE(false, "ress_restore_swap: no kernel for %d candidate slots", ns);
}
template <bool B16>
static int launch_rs_b(int BH, hipStream_t stream, const RsArgs& a) {
  const int G = cdiv(a.n_cand, 64);
  if (G <= RS_W1_MAX) return launch_rs_w<1, B16>(BH, stream, a);
  if (G <= RS_W2_MAX) return launch_rs_w<2, B16>(BH, stream, a);
  return launch_rs_w<4, B16>(BH, stream, a);
}

template <int NPL>
static int launch_rs_row(int BH, hipStream_t stream, const RsArgs& a) {
  const size_t lds = (size_t)rsr_lds_bytes(a.kb_p, NPL);
  RESS_REQUIRE(hipFuncSetAttribute((const void*)k_restore_swap_row<NPL>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)lds) == hipSuccess,
               "ress_restore_swap: cannot reserve %zu bytes of LDS", lds);
  // one head's rows split over enough workgroups to give every CU about one
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  const int per_head = max(1, min(cdiv(a.q_blk, RSR_WAVES), cdiv(cus, BH)));
  const int rows_per_wg = cdiv(a.q_blk, per_head);
  hipLaunchKernelGGL((k_restore_swap_row<NPL>), dim3(cdiv(a.q_blk, rows_per_wg), BH), dim3(64 * RSR_WAVES), lds,
                     stream, a, rows_per_wg);
  RESS_LAUNCHED("k_restore_swap_row");
  return 0;
}

RESS_API long long ress_restore_swap_workspace_size(int BH, int kb_p, int n_cand) {
  return (long long)BH * kb_p * 64 * 4 + (long long)BH * n_cand * 4;  // Vp (fp32 at most), termk
}

// restore_swap_rank_by (src/ress/scoring/projected.py:395-1058) for every (batch*head,
// query-block) row: A [BH][q_blk][kb_p] the pooled map over the patch key blocks
// (attn_full), V [BH][kb_p][64] the block means (v_bar_full), M [H][64][64] (head h =
// bh % H; identity for the _nowo recipes), nts [BH][q_blk] the kept budgets (after the
// min-2 floor). Writes rank_key [BH][q_blk][n_cand] = 1 for kept candidates, 0 for
// dropped: top-nts of it is the restore-swap keep set, which is what build_block_mask
// selects from the reference's rank_by (where(drop, s, s + max|s| + 1)). obj [BH][q_blk]
// (optional) receives J = ||g||^2_M / K^2 of the returned set, s_out [BH][q_blk][n_cand]
// (optional) the scores s = P*sqrt(d^T M d) that rank_by is built from. flags: 1 bf16
// k-wide tensors (_bf16), 2 track_best, 4 maximize (_antiswap), 8 invert_cut (_anti),
// 16 renormalize off (the cut ranks s instead of s/(1-P)).
// Round i moves round(float(f_i) * nts) blocks (at least 1 on rows with a beneficial
// candidate), f_i = restore_frac * decay * (1 - decay)^i formed in double as the
// reference does. workspace: ress_restore_swap_workspace_size bytes.
RESS_API int ress_restore_swap(const void* A, const void* V, const void* M, const void* nts, int BH, int H, int q_blk,
                               int kb_p, int n_cand, int n_iters, double restore_frac, double decay, int flags,
                               void* rank_key, void* obj, void* s_out, void* workspace, long long workspace_bytes,
                               hipStream_t stream) {
  RESS_REQUIRE(BH > 0 && H > 0 && BH % H == 0 && q_blk >= 0 && kb_p > 0 && n_cand > 0 && n_cand <= kb_p,
               "ress_restore_swap: bad geometry BH=%d H=%d q_blk=%d kb_p=%d n_cand=%d", BH, H, q_blk, kb_p, n_cand);
  RESS_REQUIRE(n_cand <= RS_MAX_KBP && kb_p <= RS_MAX_KBP,
               "ress_restore_swap: rows of more than %d key blocks are not supported (kb_p=%d)", RS_MAX_KBP, kb_p);
  RESS_REQUIRE(n_iters >= 0 && n_iters <= 16, "ress_restore_swap: n_iters must be in [0, 16]");
  RESS_REQUIRE(A && V && M && nts && rank_key && workspace, "ress_restore_swap: null pointer");
  RESS_REQUIRE(workspace_bytes >= ress_restore_swap_workspace_size(BH, kb_p, n_cand),
               "ress_restore_swap: workspace of %lld bytes required", ress_restore_swap_workspace_size(BH, kb_p, n_cand));
  if (q_blk == 0) return 0;
  float* termk = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + (long long)BH * kb_p * 64 * 4);
  void* Vp = workspace;
  const int big = (flags & RS_BF16) ? 1 : 0;
  hipLaunchKernelGGL(k_rs_head, dim3(cdiv(kb_p, 64), BH), dim3(256), 0, stream, (const float*)V, (const float*)M, H,
                     kb_p, n_cand, big, Vp, termk);
  RESS_LAUNCHED("k_rs_head");
  RsArgs a;
  a.A = (const float*)A;
  a.M = (const float*)M;
  a.nts = (const int*)nts;
  a.Vp = Vp;
  a.termk = termk;
  a.rank_key = (float*)rank_key;
  a.obj = (float*)obj;
  a.s_out = (float*)s_out;
  a.H = H;
  a.q_blk = q_blk;
  a.kb_p = kb_p;
  a.n_cand = n_cand;
  a.n_iters = n_iters;
  a.flags = flags;
  a.restore_frac = restore_frac;
  a.decay = decay;
  if (big) {
    // the row kernel when the head's V fits in LDS (up to about 735 key blocks: 12 slots)
    const int npl = cdiv(n_cand, 64);
    const int nplr = npl <= 4 ? 4 : (npl <= 8 ? 8 : 12);
    if (npl <= 12 && rsr_lds_bytes(kb_p, nplr) <= RSR_LDS_BYTES) {
      if (nplr == 4) return launch_rs_row<4>(BH, stream, a);
      if (nplr == 8) return launch_rs_row<8>(BH, stream, a);
      return launch_rs_row<12>(BH, stream, a);
    }
    return launch_rs_b<true>(BH, stream, a);
  }
  return launch_rs_b<false>(BH, stream, a);
}
