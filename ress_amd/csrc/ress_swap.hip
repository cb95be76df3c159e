// ReSS restore-swap block ranking for gfx950.
//
// Replaces restore_swap_rank_by (reference src/ress/scoring/projected.py:395-1058) with
// the round body of scoring/fused_round.py (kept-mass-normalised objective
// J = ||g||^2_M / K^2, drift compensate, geometric schedule, >=1 floor on beneficial
// rows, track-best) and fused_topm's exact top-m (ties to the lowest index). Every
// (batch*head, query-block) row is independent, so one wave owns one row for the whole
// algorithm -- initial cut, n_iters rounds, track-best -- with no grid-wide sync.
//
// Numerics. With `big` (the recipe's _bf16) every value the reference keeps in bf16 is
// rounded at the reference's points (quadratic_deviation projected.py:259-288,
// dense_reference :313-356, the round :903-947, fused_round.py:176-226). Dot products
// and sums are sequential fp32 chains in index order (fmaf for products, plain adds for
// sums of rounded terms): lane-parallel over the independent outputs, never split.
//
// Work: per row, O(kb_p * 64) for the dense reference, O(n_cand * 64) per round for the
// masked sums and term_k; selections are 4-digit radix selects over the order keys with
// a per-wave LDS histogram.
#include <type_traits>

#include "common.h"

#define RS_BF16 1
#define RS_TRACK_BEST 2
#define RS_MAXIMIZE 4
#define RS_INVERT_CUT 8
#define RS_NO_RENORM 16
#define RS_MAX_KBP 2048  // candidates per row handled (32 per lane)

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

// Per-head preparation, 64 key blocks per workgroup: Vr = big(V) [kb_p][64] and the key
// side of quadratic_deviation, termk[k] = big(sum_i big(big(Mb v_k)_i * v_ki)) with the
// product and the sum sequential in index order (the block goes through an LDS tile).
__global__ __launch_bounds__(256) void k_rs_head(const float* __restrict__ V, const float* __restrict__ M, int H,
                                                 int kb_p, int n_cand, int big, float* __restrict__ Vr,
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
      Vr[((long long)bh * kb_p + k) * 64 + lane] = x;
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
  const float* A;  // [BH][q_blk][kb_p]
  const float* M;  // [H][64][64]
  const int* nts;  // [BH][q_blk]
  const float* Vr;
  const float* termk;
  float* rank_key;  // [BH][q_blk][n_cand]: 1 = kept, 0 = dropped
  float* obj;       // [BH][q_blk] or null: J of the returned set
  float* s_out;     // [BH][q_blk][n_cand] or null: s = P*sqrt(d^T M d)
  int H, q_blk, kb_p, n_cand, n_iters, flags;
  double restore_frac, decay;  // geometric schedule (projected.py:775-790)
};

// Exact top-m among `valid` lane elements by MSB-first radix select over the order keys
// (four 8-bit digits, a 256-bin histogram in LDS per digit), then ties at the threshold
// taken in candidate-index order. hist: 256 ints of this wave's LDS.
template <int NPL>
__device__ __forceinline__ uint32_t rs_top_m(const uint32_t (&key)[NPL], uint32_t valid, int m, int lane,
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
    // lane l owns bins 4l..4l+3; suffix counts S(t) = #{digit >= t}
    const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
    const int own = h0 + h1 + h2 + h3;
    // keys in bins of higher lanes: the total minus the inclusive prefix over lanes <= l
    const int incl = wave_scan_sum_i(own);
    const int above = (int)lane63((uint32_t)incl) - incl;
    const int s3 = above + h3, s2 = s3 + h2, s1 = s2 + h1, s0 = s1 + h0;
    // the digit t with S(t) >= need > S(t+1) is unique
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
    // every key of the threshold bin is taken: the keys above prefix (lower digits zero)
    // and the n_in >= (keys equal to prefix) ties below select exactly the same set as
    // the full descent, so the remaining digits are skipped
    if (n_in == need) break;
  }
  const uint32_t thr = prefix;  // the m-th largest key's high digits; `need` of the ties at thr are taken
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

// V of the head in LDS (VLDS, bf16 mode when it fits): bf16 pairs, word w of row k at
// k*33 + w (one pad word per row). Lanes over the 64 dims of one key block read 32
// consecutive words, lanes over 32 consecutive key blocks at one dim pair hit 32 distinct
// banks, and a batch of consecutive rows is one lane base plus immediate offsets (no
// per-row address arithmetic). Otherwise V is streamed from Vr (below).
#define RS_LDS_KBP 1024
#define RS_VROW 33
// LDS words of the resident V, rounded up so that the per-wave scratch after it stays
// 16-byte aligned
__host__ __device__ __forceinline__ int rs_vw_words(int kb_p) { return (kb_p * RS_VROW + 3) & ~3; }

// Streamed V (STREAM = !VLDS: rows whose V does not fit in LDS, or fp32 V): the workgroup's
// waves run their rows in lockstep -- every row makes the same sequence of P.V chains and
// per-candidate products, and only those synchronise -- and V goes through LDS in tiles
// of 64 key blocks x 64 dims (fp32, 16 KiB), two buffers filled by LDS-DMA one tile
// ahead, so each tile is fetched from L2 once for all of the workgroup's rows. In a tile,
// 16-byte chunk c of row r sits at chunk position c ^ (r & 15): lanes over the dims of one
// row and lanes over rows reading one chunk (ds_read_b128) are both conflict-free.
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

// The rows of one head: WAVES waves, each its own row at a time.
template <int NPL, bool VLDS, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_restore_swap(RsArgs a, int rows_per_wg) {
  constexpr bool STREAM = !VLDS;
  extern __shared__ float sh[];
  float* M32T = sh;                 // [64][64] M^T (fp32)
  float* MbT = sh + 4096;           // [64][64] big(M)^T
  uint32_t* vw = reinterpret_cast<uint32_t*>(sh + 8192);  // VLDS: [kb_p][RS_VROW] bf16 pairs
  // STREAM: the two V tile buffers (distinct objects, so the compiler can see that a
  // DMA into one never aliases reads of the other)
  __shared__ __align__(16) float4 tb0[STREAM ? 1024 : 1];
  __shared__ __align__(16) float4 tb1[STREAM ? 1024 : 1];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kb4 = (a.kb_p + 3) & ~3;
  constexpr int OUTL = STREAM ? NPL * 64 : 0;  // STREAM: per-wave slots of the candidate products
  float* wsh = sh + 8192 + (VLDS ? rs_vw_words(a.kb_p) : 0) + w * (kb4 + 5 * 64 + OUTL);
  float* Pw = wsh;                  // [kb_p] big(P) of the row, then P*drop (16-byte aligned)
  float* vqs = wsh + kb4;           // [64]
  float* t0 = vqs + 64;             // [64] scratch vectors; t0..t3 double as the
  float* t1 = t0 + 64;              //      256-bin selection histogram
  float* t2 = t1 + 64;
  float* t3 = t2 + 64;
  int* hist = reinterpret_cast<int*>(t0);
  float* outl = t3 + 64;            // STREAM: [NPL][64] candidate products, slot-major
  // Workgroup gl = x + gx*y runs on XCD gl % 8. With a multiple of 8 heads, XCD x takes
  // heads x, x+8, ... whole (every row group of each), so each XCD's L2 holds the V and A
  // rows of its own heads only: at kb_p = 1369 the 16 heads' V (5.6 MB in fp32) no longer
  // all pass through every XCD's 4 MB L2.
  const int gx = gridDim.x, gl = blockIdx.x + gx * blockIdx.y;
  const bool xmap = (gridDim.y & 7) == 0;
  const int bh = xmap ? (gl & 7) + 8 * ((gl >> 3) / gx) : blockIdx.y;
  const int bgrp = xmap ? (gl >> 3) % gx : blockIdx.x;  // this workgroup's row group of head bh
  const bool big = a.flags & RS_BF16, track = a.flags & RS_TRACK_BEST;
  const bool maxim = a.flags & RS_MAXIMIZE, inv = a.flags & RS_INVERT_CUT;
  const bool renorm = !(a.flags & RS_NO_RENORM);
  const float* Mh = a.M + (long long)(bh % a.H) * 4096;
  for (int e = threadIdx.x; e < 4096; e += 64 * WAVES) {
    const float m = Mh[e];
    M32T[(e & 63) * 64 + (e >> 6)] = m;
    MbT[(e & 63) * 64 + (e >> 6)] = rs_bf(m, big);
  }
  const float* Vr = a.Vr + (long long)bh * a.kb_p * 64;
  if constexpr (VLDS) {
    for (int e = threadIdx.x; e < a.kb_p * 32; e += 64 * WAVES) {
      const int k = e >> 5, wd = e & 31;
      const uint32_t lo = __float_as_uint(Vr[(long long)k * 64 + 2 * wd]) >> 16;
      const uint32_t hi = __float_as_uint(Vr[(long long)k * 64 + 2 * wd + 1]) & 0xffff0000u;
      vw[k * RS_VROW + wd] = hi | lo;  // Vr holds bf16-exact values in this mode
    }
  }
  __syncthreads();
  // VLDS: this lane's dim of a pair word as fp32 in one byte permute: the word's low half
  // (even dim) or high half (odd dim) moved to the upper 16 bits, zeros below
  const uint32_t vsel = (lane & 1) ? 0x03020c0cu : 0x01000c0cu;
  auto vdim = [&](uint32_t word) -> float { return __uint_as_float(__builtin_amdgcn_perm(0u, word, vsel)); };
  // VLDS: V[k][lane] (lanes over dims)
  auto vrow = [&](int k) -> float { return vdim(vw[k * RS_VROW + (lane >> 1)]); };
  // STREAM: tile t = V rows 64t..64t+63 (rows past kb_p repeat the last one; their
  // results are never used). Each wave DMAs four of the tile's sixteen 1 KiB slices.
  auto tile_dma = [&](float4* buf, int t) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 4 * w + jj, sl = 64 * j + lane, r = sl >> 4, c = (sl & 15) ^ (r & 15);
      const int row = min(64 * t + r, a.kb_p - 1);
      rs_gl_lds16(Vr + (long long)row * 64 + 4 * c, buf + 64 * j);
    }
  };
  // collective over T tiles: body(tile, t) runs once the tile is in LDS for every wave;
  // tile t+1 is in flight meanwhile (two buffers, unrolled by two so that each DMA's
  // target is a different object from the buffer being read)
  auto stream_tiles = [&](int T, auto&& body) {
    rs_barrier();  // every wave is done with the buffers of the previous collective
    tile_dma(tb0, 0);
    auto step = [&](const float4* cur, float4* other, int t) {
      rs_wait_vmcnt<0>();  // this wave's slices of tile t
      rs_barrier();        // ... and every other wave's; tile t-1 (in `other`) is done
      if (t + 1 < T) tile_dma(other, t + 1);
      body(cur, t);
    };
    int t = 0;
    for (; t + 2 <= T; t += 2) {
      step(tb0, tb1, t);
      step(tb1, tb0, t + 1);
    }
    if (t < T) step(tb0, tb1, t);
  };
  const float* tkey = a.termk + (long long)bh * a.n_cand;
  const int n_cand = a.n_cand, kb_p = a.kb_p;
  const int nel = (n_cand + 63) >> 6;  // lane elements holding candidates (wave-uniform)
  uint32_t cand_bits = 0u;             // lane elements that are candidates
#pragma unroll
  for (int i = 0; i < NPL; ++i)
    if (lane + 64 * i < n_cand) cand_bits |= 1u << i;
  // sequential sum + dot over k < n of Pw[k] and V[k][lane] (4 P values per LDS read)
  auto pv_chain = [&](int n, float& sum, float& dot) {
    float sp = 0.0f, acc = 0.0f;
    if constexpr (STREAM) {  // collective: every wave of the workgroup calls it with the same n
      const int dhi = lane >> 2, dlo = lane & 3;
      // this lane's word of row u of a 16-row group (the tile swizzle): computed once, so
      // a batch's reads are these offsets plus an immediate (tile, batch)
      int roff[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) roff[u] = u * 64 + ((dhi ^ u) << 2) + dlo;
      stream_tiles((n + 63) >> 6, [&](const float4* tile, int t) {
        const float* tf = reinterpret_cast<const float*>(tile);
        const int m = min(64, n - 64 * t);
        const float* pc = Pw + 64 * t;
        auto batch = [&](int kk) {  // rows kk..kk+15 (kk % 16 == 0), all sixteen reads in flight
          float v[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] = tf[kk * 64 + roff[u]];
#pragma unroll
          for (int u = 0; u < 16; u += 4) {
            const float4 p4 = *reinterpret_cast<const float4*>(pc + kk + u);
            sp = sp + p4.x;
            acc = fmaf(p4.x, v[u], acc);
            sp = sp + p4.y;
            acc = fmaf(p4.y, v[u + 1], acc);
            sp = sp + p4.z;
            acc = fmaf(p4.z, v[u + 2], acc);
            sp = sp + p4.w;
            acc = fmaf(p4.w, v[u + 3], acc);
          }
        };
        int kk = 0;
        if (m == 64) {  // full tile: batch offsets are compile-time
          batch(0);
          batch(16);
          batch(32);
          batch(48);
          kk = 64;
        } else {
          for (; kk + 16 <= m; kk += 16) batch(kk);
        }
        for (; kk < m; ++kk) {
          const float p = pc[kk];
          sp = sp + p;
          acc = fmaf(p, tf[kk * 64 + ((dhi ^ (kk & 15)) << 2) + dlo], acc);
        }
      });
      sum = sp;
      dot = acc;
      return;
    }
    // VLDS: sixteen rows per batch, all of the batch's LDS reads issued before its chain
    // steps, so the chain waits on LDS once per batch
    const int n16 = n & ~15;
    uint32_t wa[16];
    float4 pa[4];
    auto load16 = [&](int k, uint32_t(&wv)[16], float4(&pv)[4]) {
      const uint32_t* vb = vw + k * RS_VROW + (lane >> 1);
#pragma unroll
      for (int u = 0; u < 16; ++u) wv[u] = vb[u * RS_VROW];
#pragma unroll
      for (int u = 0; u < 4; ++u) pv[u] = *reinterpret_cast<const float4*>(Pw + k + 4 * u);
    };
    auto chain16 = [&](const uint32_t(&wv)[16], const float4(&pv)[4]) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        sp = sp + pv[u].x;
        acc = fmaf(pv[u].x, vdim(wv[4 * u]), acc);
        sp = sp + pv[u].y;
        acc = fmaf(pv[u].y, vdim(wv[4 * u + 1]), acc);
        sp = sp + pv[u].z;
        acc = fmaf(pv[u].z, vdim(wv[4 * u + 2]), acc);
        sp = sp + pv[u].w;
        acc = fmaf(pv[u].w, vdim(wv[4 * u + 3]), acc);
      }
    };
    int k = 0;
    for (; k < n16; k += 16) {
      load16(k, wa, pa);
      __builtin_amdgcn_sched_barrier(0);
      chain16(wa, pa);
    }
    for (; k < n; ++k) {
      const float p = Pw[k];
      sp = sp + p;
      acc = fmaf(p, vrow(k), acc);
    }
    sum = sp;
    dot = acc;
  };
  // out[i] = sequential dot over d of vec[d] (LDS, broadcast) and V[k_i][d]
  auto vdot_cols = [&](const float* vec, float (&out)[NPL]) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) out[i] = 0.0f;
    if constexpr (STREAM) {  // collective: tile i holds the candidates of lane slot i
      // vec (the same for every tile) in registers, and all sixteen of a tile's reads
      // issued before its chain: one wave per SIMD leaves nothing else to cover LDS
      // latency between the chain's steps
      float4 vc[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) vc[q] = *reinterpret_cast<const float4*>(vec + 4 * q);
      stream_tiles(nel, [&](const float4* tile, int i) {
        const float4* vk = tile + lane * 16;
        float4 v[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = vk[q ^ (lane & 15)];
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; ++q) {  // dims 4q..4q+3 in order
          o = fmaf(vc[q].y, v[q].y, fmaf(vc[q].x, v[q].x, o));
          o = fmaf(vc[q].w, v[q].w, fmaf(vc[q].z, v[q].z, o));
        }
        outl[i * 64 + lane] = o;
      });
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int e = 0; e < NPL; ++e) out[e] = e < nel ? outl[e * 64 + lane] : 0.0f;
      return;
    }
    // VLDS: NS = nel rounded up to a multiple of 4 slots is a compile-time count (one
    // instance per value), so no slot carries a runtime guard. Slots below NS - 4 hold
    // candidates lane + 64i < n_cand and read one lane base plus immediate offsets; the
    // last four read rows clamped to n_cand - 1 (the products of slots >= nel are never
    // used). The words of dim pair p+1 are read while pair p is accumulated (two register
    // buffers), so the products wait on LDS once per pair at most.
    auto products = [&](auto ns_tag) {
      constexpr int NS = decltype(ns_tag)::value;
      const uint32_t* vl = vw + lane * RS_VROW;
      const uint32_t* vlast[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vlast[j] = vw + min(lane + 64 * (NS - 4 + j), n_cand - 1) * RS_VROW;
      uint32_t wa[NS], wb[NS];
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
          out[i] = fmaf(m1, __uint_as_float(wv[i] & 0xffff0000u), fmaf(m0, __uint_as_float(wv[i] << 16), out[i]));
      };
      load_pair(0, wa);
      for (int p = 0; p < 32; p += 2) {
        load_pair(p + 1, wb);
        __builtin_amdgcn_sched_barrier(0);
        use_pair(p, wa);
        if (p + 2 < 32) load_pair(p + 2, wa);
        __builtin_amdgcn_sched_barrier(0);
        use_pair(p + 1, wb);
      }
    };
    const int ng = (nel + 3) >> 2;  // wave-uniform
    if (ng <= 1) products(std::integral_constant<int, 4>{});
    if constexpr (NPL >= 8) {
      if (ng == 2) products(std::integral_constant<int, 8>{});
    }
    if constexpr (NPL >= 16) {
      if (ng == 3) products(std::integral_constant<int, 12>{});
      if (ng == 4) products(std::integral_constant<int, 16>{});
    }
  };

  // sequential fmaf over j = 0..63 of this lane's column col[64 j] and the broadcast vec[j]
  // (vec 16-byte aligned); each batch's LDS reads are issued before its chain steps
  auto dot64 = [&](const float* col, const float* vec) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 64; j += 8) {
      float c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = col[(j + u) * 64];
      const float4 va = *reinterpret_cast<const float4*>(vec + j);
      const float4 vb = *reinterpret_cast<const float4*>(vec + j + 4);
      __builtin_amdgcn_sched_barrier(0);
      acc = fmaf(c[0], va.x, acc);
      acc = fmaf(c[1], va.y, acc);
      acc = fmaf(c[2], va.z, acc);
      acc = fmaf(c[3], va.w, acc);
      acc = fmaf(c[4], vb.x, acc);
      acc = fmaf(c[5], vb.y, acc);
      acc = fmaf(c[6], vb.z, acc);
      acc = fmaf(c[7], vb.w, acc);
    }
    return acc;
  };
  // sequential sum of the 64 broadcast values vec[0..63] (16-byte aligned), sixteen reads
  // in flight per batch
  auto sum64 = [&](const float* vec) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; i += 16) {
      float4 v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const float4*>(vec + i + 4 * q);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc = acc + v[q].x;
        acc = acc + v[q].y;
        acc = acc + v[q].z;
        acc = acc + v[q].w;
      }
    }
    return acc;
  };

  const int q_begin = bgrp * rows_per_wg, q_end = min(a.q_blk, (bgrp + 1) * rows_per_wg);
  // STREAM: every wave makes the same number of passes (a wave without a row of its own
  // repeats the last one and writes nothing), so the collective calls line up
  const int passes = STREAM ? (q_end - q_begin + WAVES - 1) / WAVES : 0x7fffffff;
  for (int pass = 0, q = q_begin + w; STREAM ? pass < passes : q < q_end; ++pass, q += WAVES) {
    const bool own = q < q_end;
    const long long row = (long long)bh * a.q_blk + (own ? q : q_end - 1);

    // ---- row inputs and the dense reference -------------------------------------
    const float* Arow = a.A + row * kb_p;
    for (int k = lane; k < kb_p; k += 64) Pw[k] = rs_bf(Arow[k], big);
    float Pb[NPL], ssq[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int k = lane + 64 * i;
      Pb[i] = k < n_cand ? rs_bf(Arow[k], big) : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();
    float vq, tm;  // v_bar_query[lane] = big(P @ v_bar), total mass big(sum P) (all lanes)
    {
      float acc;
      pv_chain(kb_p, tm, acc);
      vq = rs_bf(acc, big);
      tm = rs_bf(tm, big);
    }
    vqs[lane] = vq;
    __builtin_amdgcn_wave_barrier();
    // quadratic_deviation's query side: Mvq = big(Mb vq), term_q = big(sum big(Mvq*vq))
    float mvq;
    {
      mvq = rs_bf(dot64(MbT + lane, vqs), big);
    }
    t0[lane] = mvq;
    t1[lane] = rs_bf(mvq * vq, big);
    __builtin_amdgcn_wave_barrier();
    const float tq = rs_bf(sum64(t1), big);
    // s, s_cut, s^2 per candidate
    uint32_t key[NPL];
    {
      float cr[NPL];
      vdot_cols(t0, cr);  // cross = Mvq . v_k
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
    __builtin_amdgcn_wave_barrier();
    uint32_t drop = cand_bits & ~rs_top_m<NPL>(key, cand_bits, nkeep, lane, hist);

    // J, and g / Mg (left in t3) / ||g||^2_M / K of a drop set (projected.py:859-868, 903-918)
    float gn = 0.0f, Kk = 1.0f;
    auto objective = [&](uint32_t dr) -> float {
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const int k = lane + 64 * i;
        if (i < nel && k < n_cand) Pw[k] = ((dr >> i) & 1u) ? Pb[i] : 0.0f;
      }
      __builtin_amdgcn_wave_barrier();
      float sp, acc;
      pv_chain(n_cand, sp, acc);
      sp = rs_bf(sp, big);
      const float g = sp * vq - rs_bf(acc, big);
      t1[lane] = g;
      __builtin_amdgcn_wave_barrier();
      const float mg = dot64(M32T + lane, t1);
      t2[lane] = g * mg;  // products of ||g||^2_M
      t3[lane] = mg;
      __builtin_amdgcn_wave_barrier();
      const float n2 = sum64(t2);
      float K = tm - sp;
      K = K < 1e-6f ? 1e-6f : K;
      gn = n2;
      Kk = K;
      return n2 / (K * K);
    };

    uint32_t best = drop;
    float best_obj = track ? objective(drop) : 0.0f;
    double remaining = a.restore_frac;  // the reference forms the round fractions in double
    for (int it = 0; it < a.n_iters; ++it) {
      const double frac = remaining * a.decay;
      remaining -= frac;
      const int pic0 = (int)rintf((float)frac * (float)nts);
      const float J = objective(drop);  // leaves Mg in t3
      if (track && (maxim ? J > best_obj : J < best_obj)) {
        best_obj = J;
        best = drop;
      }
      // term_q of the round, big(Mg)
      __builtin_amdgcn_wave_barrier();
      t2[lane] = vq * t3[lane];
      t0[lane] = rs_bf(t3[lane], big);
      __builtin_amdgcn_wave_barrier();
      const float tqb = rs_bf(sum64(t2), big);
      float tk[NPL];
      vdot_cols(t0, tk);  // term_k = v_k . big(Mg)
      // restore quality of the dropped (higher is better), then the compensation quality
      // of the kept, one key array at a time
      auto quality = [&](int i, bool restore_side) -> float {
        const float raw = rs_bf(Pb[i] * rs_bf(rs_bf(tk[i], big) - tqb, big), big);
        const float q = restore_side ? rs_knorm(gn, Kk, 2.0f * raw + ssq[i], Pb[i])
                                     : rs_knorm(gn, Kk, ssq[i] - 2.0f * raw, -Pb[i]);
        return maxim ? -q : q;
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
      // beneficial iff some drop candidate has quality > 0
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
      const uint32_t restore = rs_top_m<NPL>(qkey, drop, cnt, lane, hist);
#pragma unroll
      for (int i = 0; i < NPL; ++i) qkey[i] = i < nel ? rs_key(quality(i, false)) : 0u;
      __builtin_amdgcn_wave_barrier();
      const uint32_t comp = rs_top_m<NPL>(qkey, cand_bits & ~drop, cnt, lane, hist);
      drop = (drop & ~restore) | comp;
    }
    float fin = 0.0f;
    if (track || a.obj) fin = objective(drop);
    if (track && !(maxim ? fin > best_obj : fin < best_obj)) {
      drop = best;
      fin = best_obj;
    }
    if (a.obj && lane == 0 && own) a.obj[row] = fin;
    float* out = a.rank_key + row * n_cand;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int k = lane + 64 * i;
      if (k < n_cand && own) out[k] = ((drop >> i) & 1u) ? 0.0f : 1.0f;
    }
    __builtin_amdgcn_wave_barrier();
  }  // rows of this wave
}

// ============================================================================
// C ABI
// ============================================================================
template <int NPL, bool VLDS, int WAVES>
static int launch_rs(int BH, size_t lds, hipStream_t stream, const RsArgs& a) {
  // the LDS-resident V needs more than the default 64 KiB of dynamic LDS
  RESS_REQUIRE(hipFuncSetAttribute((const void*)k_restore_swap<NPL, VLDS, WAVES>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess,
               "ress_restore_swap: cannot reserve %zu bytes of LDS", lds);
  // one head's rows split over enough workgroups to give every CU about one
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    cus = 256;
  const int per_head = max(1, min(cdiv(a.q_blk, WAVES), cdiv(cus, BH)));
  const int rows_per_wg = cdiv(a.q_blk, per_head);
  hipLaunchKernelGGL((k_restore_swap<NPL, VLDS, WAVES>), dim3(cdiv(a.q_blk, rows_per_wg), BH), dim3(64 * WAVES),
                     lds, stream, a, rows_per_wg);
  RESS_LAUNCHED("k_restore_swap");
  return 0;
}

// V resident in LDS (bf16 pairs, eight rows at a time) when it fits next to the M
// tables and the rows' scratch; otherwise streamed through one shared tile.
#define RS_LDS_BYTES 163840
template <int NPL>
static int launch_rs_npl(int BH, int kb_p, bool big, hipStream_t stream, const RsArgs& a) {
  const size_t scratch = ((size_t)((kb_p + 3) & ~3) + 5 * 64);
  if constexpr (NPL * 64 <= RS_LDS_KBP) {
    const size_t lds = sizeof(float) * (8192 + (size_t)rs_vw_words(kb_p) + 8 * scratch);
    if (big && lds <= RS_LDS_BYTES) return launch_rs<NPL, true, 8>(BH, lds, stream, a);
  }
  const size_t lds = sizeof(float) * (8192 + 4 * (scratch + NPL * 64));  // + the two 16 KiB static tiles
  return launch_rs<NPL, false, 4>(BH, lds, stream, a);
}

RESS_API long long ress_restore_swap_workspace_size(int BH, int kb_p, int n_cand) {
  return (long long)BH * kb_p * 64 * 4 + (long long)BH * n_cand * 4;  // Vr, termk
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
  float* Vr = (float*)workspace;
  float* termk = Vr + (long long)BH * kb_p * 64;
  const int big = (flags & RS_BF16) ? 1 : 0;
  hipLaunchKernelGGL(k_rs_head, dim3(cdiv(kb_p, 64), BH), dim3(256), 0, stream, (const float*)V, (const float*)M, H,
                     kb_p, n_cand, big, Vr, termk);
  RESS_LAUNCHED("k_rs_head");
  RsArgs a;
  a.A = (const float*)A;
  a.M = (const float*)M;
  a.nts = (const int*)nts;
  a.Vr = Vr;
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
  const int npl = cdiv(n_cand, 64);
  if (npl <= 4) return launch_rs_npl<4>(BH, kb_p, big, stream, a);
  if (npl <= 8) return launch_rs_npl<8>(BH, kb_p, big, stream, a);
  if (npl <= 16) return launch_rs_npl<16>(BH, kb_p, big, stream, a);
  return launch_rs_npl<32>(BH, kb_p, big, stream, a);
}
