// ReSS restore-swap block ranking for gfx950.
//
// Replaces restore_swap_rank_by (reference src/ress/scoring/projected.py:395-1058) with
// the round body of scoring/fused_round.py (kept-mass-normalised objective
// J = ||g||^2_M / K^2, drift compensate, geometric schedule, >=1 floor on beneficial
// rows, track-best) and fused_topm's exact top-m (ties to the lowest index). Every
// (batch*head, query-block) row is independent; the rows advance together, round by
// round, as the reference's batched tensors do, and each round is two kernels:
//   k_rs_pv      the drop set's sum_Pd and Pd @ v_bar for 32 rows per workgroup (the
//                matrix cores for Pd @ v_bar, one wave's VALU for sum_Pd), then per row g,
//                M g, ||g||^2_M, K and J (and track-best), then the candidate products
//                v_k . big(M g) of its rows on the matrix cores (rs_pv_products);
//   k_rs_select  one wave per row: the restore / compensate qualities from the products,
//                the round's counts and the two exact top-m selections in one radix pass.
// The setup is the same pair with the dense reference (P @ v_bar, M v_bar_query, the cut
// key s/(1-P)) and the initial cut; the last k_rs_pv applies track-best, k_rs_keep writes
// the keep set.
//
// Numerics (the same operation order as oracle/ress_oracle.c):
//  * With `big` (the recipe's _bf16) every value the reference keeps in bf16 is rounded
//    at the reference's points (quadratic_deviation projected.py:259-288,
//    dense_reference :313-356, the round :903-947, fused_round.py:176-226).
//  * SEQK (P @ v_bar and sum P of the dense reference, Pd @ v_bar and sum_Pd of a drop
//    set): one sequential fp32 chain over increasing k, fmaf(w_k, v_k[d], acc) with
//    w_k = big(P_k), or 0 outside the drop set, and the weight sum as fmaf(w_k, 1, acc).
//    v_mfma_f32_16x16x4_f32 adds its four k terms to the accumulator one fmaf at a time,
//    in k order, on gfx950 (IEEE, subnormals kept), so chained steps over k = 0..3,
//    4..7, ... are the chain; fmaf(w, 1, acc) is the rounded sum acc + w, so the weight
//    sum is a chain of adds. An accumulator that starts at +0 never holds -0, so the zero
//    terms (masked and padding blocks) leave it bit for bit unchanged.
//  * DOT64 (v_k . Mvq and v_k . big(Mg)): one sequential fmaf chain over d = 0..63
//    (v_mfma_f32_32x32x2_f32 steps over d = (0,1), (2,3), ..., as in mfma_gemm.h).
//  * The drop set's sums are formed afresh for every objective, as the reference
//    recomputes Pd @ v_bar each round (projected.py:903-907).
//  * The 64-term products and sums of M (M v_bar_query, M g, ||g||^2_M, the term_q sums,
//    and term_k once per head) are sequential fp32 chains in index order.
#include <type_traits>

#include "common.h"
#include "mfma_gemm.h"

#define RS_BF16 1
#define RS_TRACK_BEST 2
#define RS_MAXIMIZE 4
#define RS_INVERT_CUT 8
#define RS_NO_RENORM 16
#define RS_MAX_KBP 2048  // key blocks per row handled

namespace {

typedef float rs_f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float rs_bf(float x, bool big) { return big ? round_bf16(x) : x; }
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

// Drop and best sets: one byte per candidate, rows of rs_dstride(n_cand) bytes (a multiple
// of 64, so a thread's 8 bytes of a 64-block chunk are one aligned 8-byte load).
__host__ __device__ __forceinline__ int rs_dstride(int n_cand) { return (n_cand + 63) & ~63; }

// Per-row scalars of the workspace (RS_NSCAL floats per row).
// RSV_FLAG: after a round's objective, 1 when the round's set becomes the best so far;
// after the final objective, 1 when the best round's set is returned.
enum { RSV_TM = 0, RSV_TQ, RSV_TQB, RSV_GN, RSV_K, RSV_J, RSV_BEST, RSV_FLAG, RS_NSCAL = 8 };

// Per-head preparation, 64 key blocks per workgroup: Vb = big(V) [kb64][64] fp32 with each
// row's even dims first, then its odd dims (the products' B operand; rows past kb_p zero),
// the same values per 64-block chunk in the sums' operand order Vt (key 4s + j at position
// 16j + s) and the key side of quadratic_deviation, termk[k] =
// big(sum_i big(big(Mb v_k)_i * v_ki)) with the product and the sum sequential in index
// order (the block goes through an LDS tile).
__global__ __launch_bounds__(256) void k_rs_head(const float* __restrict__ V, const float* __restrict__ M, int H,
                                                 int kb_p, int kb64, int n_cand, int big, float* __restrict__ Vb,
                                                 float* __restrict__ Vt, float* __restrict__ termk) {
  __shared__ float MbT[64 * 64];  // MbT[j*64 + i] = big(M[i][j])
  __shared__ float tile[64][65];  // [key][dim], padded
  __shared__ float prod[4][64];   // one key's rounded products per wave
  const int k0 = blockIdx.x * 64, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float* Mh = M + (long long)(bh % H) * 4096;
  for (int e = tid; e < 4096; e += 256) MbT[(e & 63) * 64 + (e >> 6)] = rs_bf(Mh[e], big);
  for (int r = w; r < 64; r += 4) {  // rows of V: lane = dim; the grid covers kb64 rows exactly
    const int k = k0 + r;
    const float x = k < kb_p ? rs_bf(V[((long long)bh * kb_p + k) * 64 + lane], big) : 0.0f;
    Vb[((long long)bh * kb64 + k) * 64 + (lane >> 1) + 32 * (lane & 1)] = x;  // evens, then odds
    tile[r][lane] = x;
  }
  __syncthreads();
  {  // Vt[bh][chunk][dim][pos]: key 4s + j of the chunk at pos 16j + s
    float* dst = Vt + ((long long)bh * kb64 + k0) * 64;
    for (int e = tid; e < 4096; e += 256) {
      const int pos = e & 63;
      dst[e] = tile[4 * (pos & 15) + (pos >> 4)][e >> 6];
    }
  }
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

struct RsPvArgs {
  const float* A;   // [BH][q_blk][kb_p] pooled map
  const float* M;   // [H][64][64]
  const float* Vt;  // [BH][kb64/64][64 dims][64] big(V) per chunk in operand order, zero past kb_p
  const float* Vb;  // [BH][kb64][64] big(V), zero rows past kb_p; each row's even dims, then its odd dims
  uint8_t* drop;    // [BH][q_blk][n_cand] 1 = dropped
  uint8_t* best;    // [BH][q_blk][n_cand] the track-best set
  float* vq;        // [BH][q_blk][64] big(v_bar_query)
  float* T;         // [BH][q_blk][n_cand] setup: v_k . big(Mb vq); rounds: v_k . big(M g)
  float* rsv;       // [BH][q_blk][RS_NSCAL]
  float* rank_key;  // [BH][q_blk][n_cand] final: 1 kept, 0 dropped
  float* obj;       // [BH][q_blk] final (optional): J of the returned set
  int H, q_blk, kb_p, kb64, n_cand, flags, first;
};

enum { RS_PV_SETUP = 0, RS_PV_OBJ = 1, RS_PV_FINAL = 2 };
constexpr int PV_ROWS = 32;  // rows per workgroup: two 16-row MFMA tiles per wave
constexpr int PV_KC = 64;    // key blocks per chunk
// Operand order of a chunk: key 4s + j (s < 16, j < 4) at position 16j + s, so the lane
// that supplies key 4s + j to MFMA step s (j = lane / 16) reads its 16 steps' values as
// four 16-byte LDS reads.
constexpr int PV_LDA = 68;   // A chunk row stride (rows of 64 positions; 16-lane groups of
                             // 16-byte reads at this stride hit 64 distinct banks)
constexpr int PV_LDV = 68;   // V chunk stride per dim (64 positions each)
constexpr int PV_LDM = 65;   // M row stride
constexpr int PV_LDC = 68;
constexpr int PV_NBUF = 2;   // chunk buffers (double-buffered LDS)

// float offset of V chunk float4 f (dim f/16, positions 4(f%16)..+3)
__device__ __forceinline__ int pv_vofs(int f) { return (f >> 4) * PV_LDV + 4 * (f & 15); }

// The products of a workgroup's rows, T[r][k] = X_r . big(V_k) for k < n_cand (DOT64 on the
// matrix cores, the chain k_gemm64 runs: v_mfma_f32_32x32x2_f32 steps over d = (0,1), (2,3),
// ...), with X_r row r of Cl (rounded to big here when ROUND: the rounds' M g). The
// candidates are taken in blocks of 32, block b by wave b % 4 (waves 0..3, one per SIMD; a
// fifth wave would share SIMD 0's matrix core), each wave on its own (no barrier): lane l
// supplies A = X[l%32][2s + l/32] and B = V[32b + l%32][2s + l/32], which is
// one contiguous run of 32 floats of Vbe (a row's even dims, then its odd dims), loaded as
// eight 16-byte loads a block ahead. Candidate rows past kb64 read row kb64 - 1 (their
// products are not stored).
template <bool ROUND>
__device__ __forceinline__ void rs_pv_products(const float* Cl, const float* __restrict__ Vbe, int kb64, int n_cand,
                                               int nrow, float* __restrict__ Tg, bool big, int w, int lane) {
  const int rl = lane & 31, h = lane >> 5;
  float av[32];
#pragma unroll
  for (int s = 0; s < 32; ++s) {
    const float x = Cl[rl * PV_LDC + 2 * s + h];
    av[s] = ROUND ? rs_bf(x, big) : x;
  }
  const int nblk = cdiv(n_cand, 32);
  if (w >= 4) return;  // wave-uniform; no barrier follows
  // block loads into two register sets used in turn (no copies between them); every load
  // is issued (past the last block it repeats the last block), so each compute step waits
  // only for its own set
  auto load = [&](int blk, float4 (&y)[8]) {
    const float4* src = reinterpret_cast<const float4*>(
        Vbe + (long long)min(32 * min(blk, nblk - 1) + rl, kb64 - 1) * 64 + 32 * h);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = src[i];
  };
  auto compute = [&](int blk, const float4 (&y)[8]) {
    g64_f16v acc;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * i], y[i].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * i + 1], y[i].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * i + 2], y[i].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[4 * i + 3], y[i].w, acc, 0, 0, 0);
    }
    // element j: row 8(j/4) + 4h + j%4, column 32 blk + l%32
    const int col = 32 * blk + rl;
    float* dst = Tg + col;
    if (nrow == PV_ROWS && 32 * blk + 32 <= n_cand) {  // uniform: the whole block is stored
#pragma unroll
      for (int j = 0; j < 16; ++j) dst[(long long)(8 * (j >> 2) + 4 * h + (j & 3)) * n_cand] = acc[j];
    } else if (col < n_cand) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = 8 * (j >> 2) + 4 * h + (j & 3);
        if (r < nrow) dst[(long long)r * n_cand] = acc[j];
      }
    }
  };
  float4 y0[8], y1[8];
  int blk = w;
  load(blk, y0);
#pragma unroll 1
  for (; blk < nblk; blk += 8) {
    load(blk + 4, y1);
    __builtin_amdgcn_sched_barrier(0);  // the loads issue before the block's MFMAs
    compute(blk, y0);
    if (blk + 4 >= nblk) break;  // uniform
    load(blk + 8, y0);
    __builtin_amdgcn_sched_barrier(0);
    compute(blk + 4, y1);
  }
}

// Sums over key blocks for 32 rows of one head (one row group of one head per workgroup),
// then the per-row vector math. Waves 0..3 accumulate dims 16c..16c+15 of w @ v_bar as
// two v_mfma_f32_16x16x4_f32 chains over k (rows 0..15 and 16..31; lane l supplies
// A[row l%16][k 4s + l/16] and B[k 4s + l/16][column l%16]); in wave 4, lane r < 32 adds
// row r's weights one at a time in k order (fmaf(w, 1, acc) is the rounded sum acc + w).
// A and V go through LDS in chunks of 64 key blocks, two chunks' loads in flight.
//  SETUP: w = big(P) over k < kb_p; vq = big(w @ V), tm = big(sum w), X = Mvq =
//         big(Mb vq), tq = big(sum big(Mvq_i vq_i)).
//  OBJ:   w = big(P) on the drop set of k < n_cand; g = big(sum_Pd) vq - big(Pd @ V),
//         Mg = M g, ||g||^2_M, K = max(tm - big(sum_Pd), 1e-6), J; X = big(Mg),
//         tqb = big(vq . Mg); track-best (the first round records J and the set).
//  FINAL: J of the final set; track-best keeps the better of it and the best round's;
//         rank_key and obj of the result.
template <int MODE>
__global__ __launch_bounds__(320) void k_rs_pv(RsPvArgs a) {
  // two chunk buffers (the operands w and V); after the sums the same LDS holds M, the
  // sums and the per-row vectors
  __shared__ __align__(16) float Al[PV_NBUF][PV_ROWS * PV_LDA];
  __shared__ __align__(16) float Vl[PV_NBUF][PV_KC * PV_LDV];
  static_assert(64 * PV_LDM <= PV_NBUF * PV_KC * PV_LDV, "M fits the V buffers");
  static_assert(2 * PV_ROWS * PV_LDC <= PV_NBUF * PV_ROWS * PV_LDA, "C and G fit the A buffers");
  float* Cl = &Al[0][0];                     // after the sums: w @ V | sum w, then M vq / M g
  float* Gl = &Al[0][0] + PV_ROWS * PV_LDC;  // vq (setup) / g (objective)
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware order (workgroup L runs on XCD L % 8): with a multiple of 8 heads, XCD x takes
  // heads x, x + 8, ... whole, so each XCD's L2 holds the V of only its own heads
  const int G = cdiv(a.q_blk, PV_ROWS), BH = gridDim.x / G, L = blockIdx.x;
  int bh, grp;
  if ((BH & 7) == 0) {
    const int j = L >> 3;
    bh = (L & 7) + 8 * (j / G);
    grp = j % G;
  } else {
    bh = L / G;
    grp = L % G;
  }
  const int g0 = grp * PV_ROWS;
  const bool big = a.flags & RS_BF16;
  const int kend = MODE == RS_PV_SETUP ? a.kb_p : a.n_cand;
  const long long rowbase = (long long)bh * a.q_blk;
  const float* Vh = a.Vt + (long long)bh * a.kb64 * 64;
  // Chunk loads: thread t takes row (t % 256)/8 of the group, key blocks 8(t%8)..+7 of the
  // chunk (zero past kend, outside the drop set, and for rows past q_blk; stored in operand
  // order as four pairs), and V float4s t, t + 320, t + 640 and min(t + 960, 1023) of the
  // chunk's 64 dims of 16 float4s (already in operand order in Vt); threads
  // 256.. repeat what threads 0.. load and store (the same values to the same places). The
  // loads of chunk c are issued two chunks ahead into register set c & 1 and waited for
  // only when the chunk is stored to LDS, after the MFMAs of chunk c - 1; rounding and
  // masking happen at the store. Every load and store is unconditional (past the last
  // chunk they repeat it), so the waits the compiler places are the ones per chunk.
  // Addresses are uniform bases plus 32-bit lane offsets.
  const int lm = (tid & 255) >> 3, lk = 8 * (tid & 7);
  const bool lrow_ok = g0 + lm < a.q_blk;
  const int lmc = min(lm, a.q_blk - 1 - g0);  // clamped row: every load stays in the matrix
  const char* Ag = reinterpret_cast<const char*>(a.A + (rowbase + g0) * a.kb_p);
  const int dstr = rs_dstride(a.n_cand);
  const char* Dg = reinterpret_cast<const char*>(a.drop + (rowbase + g0) * dstr);
  const unsigned a_row = 4u * (unsigned)(lmc * a.kb_p), d_row = (unsigned)(lmc * dstr);
  const char* Vg = reinterpret_cast<const char*>(Vh);
  float x0_0 = 0.0f, x1_0 = 0.0f, x2_0 = 0.0f, x3_0 = 0.0f, x4_0 = 0.0f, x5_0 = 0.0f, x6_0 = 0.0f, x7_0 = 0.0f;
  float x0_1 = 0.0f, x1_1 = 0.0f, x2_1 = 0.0f, x3_1 = 0.0f, x4_1 = 0.0f, x5_1 = 0.0f, x6_1 = 0.0f, x7_1 = 0.0f;
  uint2 dm_0 = make_uint2(0u, 0u), dm_1 = dm_0;
  int k0_0 = 0, k0_1 = 0;
  const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float4 v0_0 = z4, v1_0 = z4, v2_0 = z4, v3_0 = z4, v0_1 = z4, v1_1 = z4, v2_1 = z4, v3_1 = z4;
#define RS_PV_X(S, u)                                                                              \
  x##u##_##S = *reinterpret_cast<const float*>(Ag + (a_row + 4u * (unsigned)min(k0_##S + lk + (u), kend - 1)))
#define RS_PV_LOAD(ch, S)                                                                          \
  do {                                                                                             \
    k0_##S = min((ch), nch - 1) * PV_KC;                                                           \
    RS_PV_X(S, 0); RS_PV_X(S, 1); RS_PV_X(S, 2); RS_PV_X(S, 3);                                    \
    RS_PV_X(S, 4); RS_PV_X(S, 5); RS_PV_X(S, 6); RS_PV_X(S, 7);                                    \
    /* k0 + lk + 8 <= nch * 64 <= the row stride: in the row */                                    \
    if (MODE != RS_PV_SETUP)                                                                       \
      dm_##S = *reinterpret_cast<const uint2*>(Dg + (d_row + (unsigned)(k0_##S + lk)));            \
    const char* vb_ = Vg + 256u * (unsigned)k0_##S;                                                \
    v0_##S = *reinterpret_cast<const float4*>(vb_ + 16u * (unsigned)tid);                          \
    v1_##S = *reinterpret_cast<const float4*>(vb_ + 16u * (unsigned)(tid + 320));                  \
    v2_##S = *reinterpret_cast<const float4*>(vb_ + 16u * (unsigned)(tid + 640));                  \
    v3_##S = *reinterpret_cast<const float4*>(vb_ + 16u * (unsigned)min(tid + 960, 1023));         \
  } while (0)
#define RS_PV_W(S, u)                                                                              \
  ((lrow_ok & (k0_##S + lk + (u) < kend) &                                                         \
    (MODE == RS_PV_SETUP || ((((u) < 4 ? dm_##S.x : dm_##S.y) >> (8 * ((u) & 3))) & 0xffu)))       \
       ? rs_bf(x##u##_##S, big)                                                                    \
       : 0.0f)
#define RS_PV_STORE(S)                                                                             \
  do {                                                                                             \
    /* keys lk + j and lk + 4 + j sit at positions 16j + lk/4 and 16j + lk/4 + 1 */               \
    float* al_ = &Al[S][lm * PV_LDA + (lk >> 2)];                                                  \
    *reinterpret_cast<float2*>(al_) = make_float2(RS_PV_W(S, 0), RS_PV_W(S, 4));                   \
    *reinterpret_cast<float2*>(al_ + 16) = make_float2(RS_PV_W(S, 1), RS_PV_W(S, 5));              \
    *reinterpret_cast<float2*>(al_ + 32) = make_float2(RS_PV_W(S, 2), RS_PV_W(S, 6));              \
    *reinterpret_cast<float2*>(al_ + 48) = make_float2(RS_PV_W(S, 3), RS_PV_W(S, 7));              \
    float* vl_ = &Vl[S][0];                                                                        \
    *reinterpret_cast<float4*>(vl_ + pv_vofs(tid)) = v0_##S;                                       \
    *reinterpret_cast<float4*>(vl_ + pv_vofs(tid + 320)) = v1_##S;                                 \
    *reinterpret_cast<float4*>(vl_ + pv_vofs(tid + 640)) = v2_##S;                                 \
    *reinterpret_cast<float4*>(vl_ + pv_vofs(min(tid + 960, 1023))) = v3_##S;                      \
  } while (0)
  rs_f4v acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = acc;  // rows 0..15 and 16..31
  const int am = lane & 15, aq = lane >> 4;
  float wsum = 0.0f;  // wave 4, lane r < 32: row r's weight sum
#define RS_PV_STEP(x, x2, y)                                          \
  do {                                                                \
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc, 0, 0, 0);   \
    acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(x2, y, acc2, 0, 0, 0); \
  } while (0)
#define RS_PV_ADD4(a0, a1, a2, a3) \
  do {                             \
    wsum = wsum + (a0);            \
    wsum = wsum + (a1);            \
    wsum = wsum + (a2);            \
    wsum = wsum + (a3);            \
  } while (0)
#define RS_PV_MFMA(S)                                                                              \
  do {                                                                                             \
    if (w < 4) {                                                                                   \
      const float4* Ab = reinterpret_cast<const float4*>(&Al[S][am * PV_LDA + 16 * aq]);           \
      const float4* Ab2 = reinterpret_cast<const float4*>(&Al[S][(am + 16) * PV_LDA + 16 * aq]);   \
      const float4* Vc = reinterpret_cast<const float4*>(&Vl[S][(16 * w + am) * PV_LDV + 16 * aq]); \
      _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_) {                                           \
        const float4 x_ = Ab[q_], x2_ = Ab2[q_], y_ = Vc[q_];                                      \
        RS_PV_STEP(x_.x, x2_.x, y_.x);                                                             \
        RS_PV_STEP(x_.y, x2_.y, y_.y);                                                             \
        RS_PV_STEP(x_.z, x2_.z, y_.z);                                                             \
        RS_PV_STEP(x_.w, x2_.w, y_.w);                                                             \
      }                                                                                            \
    } else { /* keys 4s + j in order: positions 16j + s */                                         \
      const float* Ar = &Al[S][(lane & 31) * PV_LDA];                                              \
      _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_) {                                           \
        const float4 t0_ = *reinterpret_cast<const float4*>(Ar + 4 * q_);                          \
        const float4 t1_ = *reinterpret_cast<const float4*>(Ar + 16 + 4 * q_);                     \
        const float4 t2_ = *reinterpret_cast<const float4*>(Ar + 32 + 4 * q_);                     \
        const float4 t3_ = *reinterpret_cast<const float4*>(Ar + 48 + 4 * q_);                     \
        RS_PV_ADD4(t0_.x, t1_.x, t2_.x, t3_.x);                                                    \
        RS_PV_ADD4(t0_.y, t1_.y, t2_.y, t3_.y);                                                    \
        RS_PV_ADD4(t0_.z, t1_.z, t2_.z, t3_.z);                                                    \
        RS_PV_ADD4(t0_.w, t1_.w, t2_.w, t3_.w);                                                    \
      }                                                                                            \
    }                                                                                              \
  } while (0)
  // chunk c lives in LDS buffer c & 1 and register set c & 1; a buffer is rewritten only
  // after the barrier that ends the step which last read it. kend >= 1, and chunk rows
  // stay below kb64 (nch * 64 <= kb64).
  const int nch = cdiv(kend, PV_KC);
  RS_PV_LOAD(0, 0);
  RS_PV_LOAD(1, 1);
  RS_PV_STORE(0);
  __syncthreads();
  for (int ch = 0; ch < nch; ch += 2) {
    RS_PV_LOAD(ch + 2, 0);
    RS_PV_MFMA(0);
    RS_PV_STORE(1);
    __syncthreads();
    if (ch + 1 >= nch) break;  // uniform
    RS_PV_LOAD(ch + 3, 1);
    RS_PV_MFMA(1);
    RS_PV_STORE(0);
    __syncthreads();
  }
#undef RS_PV_X
#undef RS_PV_LOAD
#undef RS_PV_W
#undef RS_PV_STORE
#undef RS_PV_MFMA
#undef RS_PV_STEP
#undef RS_PV_ADD4
  // M into the V buffers (free after the last barrier of the sums), rounded in the setup
  float* Ml = &Vl[0][0];
  {
    const float* Mh = a.M + (long long)(bh % a.H) * 4096;
    for (int e = tid; e < 4096; e += 320) {
      const float mv = Mh[e];
      Ml[(e >> 6) * PV_LDM + (e & 63)] = MODE == RS_PV_SETUP ? rs_bf(mv, big) : mv;
    }
  }
  // lane l holds rows 4(l/16) + i (+16 in acc2), column l%16 of its wave's 16 columns
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * aq + i;
    if (w < 4) {
      Cl[r * PV_LDC + 16 * w + am] = acc[i];
      Cl[(r + 16) * PV_LDC + 16 * w + am] = acc2[i];
    }
  }
  if (w == 4 && lane < PV_ROWS) Cl[lane * PV_LDC + 64] = wsum;
  __syncthreads();
  // ---- per-row vector math: thread t < 256 is row t/8, outputs 8(t%8)..+7 ----------------
  constexpr int PU = 64 * PV_ROWS / 256;  // outputs per thread
  const int m = tid / (256 / PV_ROWS), r = g0 + m, i0 = PU * (tid % (256 / PV_ROWS));
  const bool live = tid < 256 && r < a.q_blk;
  const bool lead = live && i0 == 0;  // the row's scalar work
  const long long R = rowbase + r;
  float* sc = a.rsv + R * RS_NSCAL;
  if constexpr (MODE == RS_PV_SETUP) {
    if (live) {
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        const float v = rs_bf(Cl[m * PV_LDC + i0 + u], big);
        Gl[m * PV_LDC + i0 + u] = v;
        a.vq[R * 64 + i0 + u] = v;
      }
      if (lead) sc[RSV_TM] = rs_bf(Cl[m * PV_LDC + 64], big);
    }
    __syncthreads();
    float o[PU];
    if (live) {
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        float s = 0.0f;
#pragma unroll 8
        for (int j = 0; j < 64; ++j) s = fmaf(Ml[(i0 + u) * PV_LDM + j], Gl[m * PV_LDC + j], s);
        o[u] = rs_bf(s, big);
      }
    }
    __syncthreads();  // every read of Cl's sums is done
    if (live)
#pragma unroll
      for (int u = 0; u < PU; ++u) Cl[m * PV_LDC + i0 + u] = o[u];
    __syncthreads();
    if (lead) {
      float tq = 0.0f;
      for (int i = 0; i < 64; ++i) tq = tq + rs_bf(Cl[m * PV_LDC + i] * Gl[m * PV_LDC + i], big);
      sc[RSV_TQ] = rs_bf(tq, big);
    }
  } else {
    const bool track = a.flags & RS_TRACK_BEST, maxim = a.flags & RS_MAXIMIZE;
    float sp = 0.0f;
    if (live) {
      sp = rs_bf(Cl[m * PV_LDC + 64], big);
#pragma unroll
      for (int u = 0; u < PU; ++u)
        Gl[m * PV_LDC + i0 + u] = sp * a.vq[R * 64 + i0 + u] - rs_bf(Cl[m * PV_LDC + i0 + u], big);
    }
    __syncthreads();
    float o[PU];
    if (live) {
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        float s = 0.0f;
#pragma unroll 8
        for (int j = 0; j < 64; ++j) s = fmaf(Ml[(i0 + u) * PV_LDM + j], Gl[m * PV_LDC + j], s);
        o[u] = s;
      }
    }
    __syncthreads();  // every read of Cl's sums is done
    if (live)
#pragma unroll
      for (int u = 0; u < PU; ++u) Cl[m * PV_LDC + i0 + u] = o[u];
    __syncthreads();
    if (lead) {
      const float* g = &Gl[m * PV_LDC];
      const float* Mg = &Cl[m * PV_LDC];
      const float* vq = a.vq + R * 64;
      float gn = 0.0f;
      for (int d = 0; d < 64; ++d) gn = gn + g[d] * Mg[d];
      float K = sc[RSV_TM] - sp;
      K = K < 1e-6f ? 1e-6f : K;
      const float J = gn / (K * K);
      int f = 0;
      if constexpr (MODE == RS_PV_OBJ) {
        float tqr = 0.0f;
#pragma unroll 4
        for (int d = 0; d < 64; ++d) tqr = tqr + vq[d] * Mg[d];
        sc[RSV_TQB] = rs_bf(tqr, big);
        sc[RSV_GN] = gn;
        sc[RSV_K] = K;
        sc[RSV_J] = J;
        if (track) {  // this round's set becomes the best when it beats the best so far
          const float b = sc[RSV_BEST];
          f = a.first || (maxim ? J > b : J < b);
          if (f) sc[RSV_BEST] = J;
        }
      } else {
        float fin = J;
        if (track && !a.first) {
          const float b = sc[RSV_BEST];
          if (!(maxim ? J > b : J < b)) {  // the final set is not better: return the best one
            f = 1;
            fin = b;
          }
        }
        if (a.obj) a.obj[R] = fin;
      }
      sc[RSV_FLAG] = (float)f;
    }
  }
  if constexpr (MODE != RS_PV_FINAL) {
    __syncthreads();  // Cl holds every row's X
    rs_pv_products<MODE == RS_PV_OBJ>(Cl, a.Vb + (long long)bh * a.kb64 * 64, a.kb64, a.n_cand,
                                      min(PV_ROWS, a.q_blk - g0), a.T + (rowbase + g0) * a.n_cand, big, w, lane);
  }
}

// Two exact top-m selections of one wave at once, over disjoint sets of lane elements
// (slot i of a lane is in set (setb >> i) & 1 when valid): for each set the m[s] largest
// order keys, ties at the threshold taken in candidate-index order (slot-major, then lane).
// MSB-first radix select over four 8-bit digits; one pass over the slots per digit feeds
// both sets' 256-bin histograms (hist: 576 ints of the wave's LDS, the last 64 spare). A set whose threshold
// bin is taken whole stops descending (the same set as the full descent); a set with m <= 0
// selects nothing, one with no more than m valid elements selects them all.
template <int NPL>
__device__ __forceinline__ void rs_top_m_pair(const uint32_t (&key)[NPL], uint32_t valid, uint32_t setb, int m0,
                                              int m1, int lane, int* hist, uint32_t& sel0, uint32_t& sel1) {
  int n0 = 0, n1 = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool v = (valid >> i) & 1u, s1 = (setb >> i) & 1u;
    n0 += __popcll(__ballot(v && !s1));
    n1 += __popcll(__ballot(v && s1));
  }
  // per set: thr/need of the final pass (take all: thr 0, need n; take none: thr ~0, need 0)
  uint32_t thr0 = 0u, thr1 = 0u, pm0 = 0u, pm1 = 0u;
  int need0 = m0, need1 = m1;
  bool act0 = true, act1 = true;
  if (m0 <= 0) thr0 = ~0u, need0 = 0, act0 = false;
  else if (n0 <= m0) need0 = n0, act0 = false;
  if (m1 <= 0) thr1 = ~0u, need1 = 0, act1 = false;
  else if (n1 <= m1) need1 = n1, act1 = false;
  for (int shift = 24; shift >= 0 && (act0 || act1); shift -= 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) hist[lane + 64 * j] = 0;
    __builtin_amdgcn_wave_barrier();
    // every lane adds once per slot: an element outside the descent counts into the lane's
    // own spare bin 512 + lane (no branch; distinct spare addresses do not collide)
    const uint32_t a0 = act0 ? 1u : 0u, a1 = act1 ? 1u : 0u;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const uint32_t s1 = (setb >> i) & 1u;
      const uint32_t pm = s1 ? pm1 : pm0, th = s1 ? thr1 : thr0;
      const uint32_t in = ((valid >> i) & 1u) & (s1 ? a1 : a0) & ((key[i] & pm) == th ? 1u : 0u);
      atomicAdd(&hist[in ? (s1 << 8) + ((key[i] >> shift) & 255u) : 512u + lane], 1);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (!(s ? act1 : act0)) continue;  // uniform
      const int* hs = hist + 256 * s;
      const int need = s ? need1 : need0;
      const int h0 = hs[4 * lane], h1 = hs[4 * lane + 1], h2 = hs[4 * lane + 2], h3 = hs[4 * lane + 3];
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
      const int left = need - n_gt;
      if (s) {
        need1 = left, thr1 |= (uint32_t)digit << shift, pm1 |= 255u << shift, act1 = n_in != left;
      } else {
        need0 = left, thr0 |= (uint32_t)digit << shift, pm0 |= 255u << shift, act0 = n_in != left;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // keys above a set's threshold are taken; of its ties the first ones in index order, up to
  // need (ties are rare: the rank work runs only for slots that hold one)
  uint32_t take = 0u;
  int before0 = 0, before1 = 0;
  const unsigned long long lower = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const uint32_t v = (valid >> i) & 1u, s1 = (setb >> i) & 1u;
    const uint32_t thr = s1 ? thr1 : thr0;
    uint32_t t = v & (key[i] > thr ? 1u : 0u);
    const bool eq = v && key[i] == thr;
    const unsigned long long be = __ballot(eq);
    if (be) {  // uniform
      const unsigned long long b1 = be & __ballot(s1 != 0u), b0 = be & ~b1;
      const int rank = s1 ? before1 + __popcll(b1 & lower) : before0 + __popcll(b0 & lower);
      t |= (eq && rank < (s1 ? need1 : need0)) ? 1u : 0u;
      before0 += __popcll(b0);
      before1 += __popcll(b1);
    }
    take |= t << i;
  }
  sel1 = take & setb;
  sel0 = take & ~setb;
}

struct RsSelArgs {
  const float* T;      // [BH][q_blk][n_cand] raw candidate products v_k . X (k_rs_pv)
  const float* A;      // [BH][q_blk][kb_p] pooled map
  const float* termk;  // [BH][n_cand]
  const float* rsv;    // [BH][q_blk][RS_NSCAL]
  float* ssq;          // [BH][q_blk][n_cand] s^2 (written by INIT, read by the rounds)
  float* s_out;        // [BH][q_blk][n_cand] or null: s (INIT)
  uint8_t* drop;       // [BH][q_blk][n_cand]
  uint8_t* best;       // [BH][q_blk][n_cand] the track-best set
  const int* nts;      // [BH][q_blk]
  int q_blk, kb_p, n_cand, flags;
  float frac;  // the round's fraction of nts (rounds only)
};

// One wave per row (four rows of one head per workgroup); candidate k = lane + 64i in
// slot i (n_cand <= 64 NPL). The candidates' values come from the raw products T:
//  INIT:  cr = big(T) = big(Mvq . v_k), qd = big(big(tq - big(2 cr)) + term_k) (>= 0),
//         s = big(P big(sqrt(qd))), the cut key s/(1-P) (or s; negated under
//         invert_cut), ssq = big(s^2); keep the top min(nts, n_cand) cut keys, drop the
//         rest (projected.py:259-302, 756-790).
//  round: raw = big(P big(big(T) - tqb)) with T = v_k . big(Mg), the restore quality
//         knorm(G, K, 2 raw + s^2, +P) of dropped candidates and the compensate quality
//         knorm(G, K, s^2 - 2 raw, -P) of kept ones (sign-flipped under maximize); restore
//         the top cnt restore qualities and drop the top cnt compensate qualities,
//         cnt = min(pic, #dropped, #kept) with pic = rint(frac * nts), at least 1 on rows
//         with a beneficial restore and 0 on rows without (projected.py:903-1035,
//         fused_round.py:126-226).
template <int NPL, bool INIT>
__global__ __launch_bounds__(256) void k_rs_select(RsSelArgs a) {
  __shared__ int hist[4][576];  // per wave: two 256-bin histograms, then one spare bin per lane
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = blockIdx.x * 4 + w;
  if (r >= a.q_blk) return;  // wave-uniform; no workgroup barrier below
  const int bh = blockIdx.y, n = a.n_cand;
  const long long R = (long long)bh * a.q_blk + r;
  const bool big = a.flags & RS_BF16;
  const float* Tr = a.T + R * n;
  const float* Ar = a.A + R * a.kb_p;
  const float* sc = a.rsv + R * RS_NSCAL;
  uint8_t* dr = a.drop + R * rs_dstride(n);
  float* sr = a.ssq + R * n;
  // every slot's operands first (slots past n_cand read candidate n_cand - 1 and are masked)
  float tv[NPL], pv[NPL], xv[NPL];
  uint32_t cand = 0u;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int k = lane + 64 * i;
    if (k < n) cand |= 1u << i;
    const int kc = min(k, n - 1);
    tv[i] = Tr[kc];
    pv[i] = Ar[kc];
    xv[i] = INIT ? a.termk[(long long)bh * n + kc] : sr[kc];
  }
  uint32_t dropb = 0u;
  if constexpr (!INIT) {
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (dr[min(lane + 64 * i, n - 1)]) dropb |= 1u << i;
    dropb &= cand;
  }
  uint32_t key[NPL];
  float rmax = -__builtin_huge_valf();
  const float s0 = INIT ? sc[RSV_TQ] : sc[RSV_TQB];
  const float gn = INIT ? 0.0f : sc[RSV_GN], K = INIT ? 0.0f : sc[RSV_K];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int k = lane + 64 * i;
    const float x = rs_bf(tv[i], big);
    const float Pb = rs_bf(pv[i], big);
    if constexpr (INIT) {
      float qd = rs_bf(rs_bf(s0 - rs_bf(2.0f * x, big), big) + xv[i], big);
      qd = qd < 0.0f ? 0.0f : qd;
      const float sq = rs_bf(sqrtf(qd), big);
      const float s = rs_bf(Pb * sq, big);
      float om = rs_bf(1.0f - Pb, big);
      om = rs_bf(om < 1e-4f ? 1e-4f : om, big);
      const float scut = (a.flags & RS_NO_RENORM) ? s : rs_bf(s / om, big);
      if (k < n) {
        sr[k] = rs_bf(s * s, big);
        if (a.s_out) a.s_out[R * n + k] = s;
      }
      key[i] = rs_key((a.flags & RS_INVERT_CUT) ? -scut : scut);
    } else {
      const float raw = rs_bf(Pb * rs_bf(x - s0, big), big);
      const float ss = xv[i];
      const bool dropped = (dropb >> i) & 1u;
      // one quality per candidate: the arguments are selected, not the results
      const float dG = dropped ? 2.0f * raw + ss : ss - 2.0f * raw;
      float v = rs_knorm(gn, K, dG, dropped ? Pb : -Pb);
      if (a.flags & RS_MAXIMIZE) v = -v;
      key[i] = rs_key(v);
      if (dropped) rmax = fmaxf(rmax, v);
    }
  }
  const int nts = a.nts[R];
  uint32_t nd, sel0, sel1;
  if constexpr (INIT) {
    const int m = min(max(nts, 0), n);
    rs_top_m_pair<NPL>(key, cand, 0u, m, 0, lane, hist[w], sel0, sel1);
    nd = cand & ~sel0;
  } else {
    int n_drop = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) n_drop += __popcll(__ballot((dropb >> i) & 1u));
    const int n_kept = n - n_drop;
    rmax = wave_max(rmax);
    const bool beneficial = rmax > 0.0f;
    const int pic0 = (int)rintf(a.frac * (float)nts);
    int cnt = beneficial && pic0 < 1 ? 1 : pic0;
    cnt = min(cnt, n_drop);
    cnt = min(cnt, n_kept);
    if (!beneficial) cnt = 0;
    if ((a.flags & RS_TRACK_BEST) && sc[RSV_FLAG] != 0.0f) {  // record the set this round starts from
      uint8_t* br = a.best + R * rs_dstride(n);
#pragma unroll
      for (int i = 0; i < NPL; ++i)  // the row's padding past n (to its 64-byte stride) is never read
        if (64 * i < rs_dstride(n)) br[lane + 64 * i] = (uint8_t)((dropb >> i) & 1u);
    }
    // set 0: the dropped candidates (restore the top cnt), set 1: the kept (drop the top cnt)
    rs_top_m_pair<NPL>(key, cand, cand & ~dropb, cnt, cnt, lane, hist[w], sel0, sel1);
    nd = (dropb & ~sel0) | sel1;
  }
#pragma unroll
  for (int i = 0; i < NPL; ++i)  // uniform bound: the row's padding past n is never read
    if (64 * i < rs_dstride(n)) dr[lane + 64 * i] = (uint8_t)((nd >> i) & 1u);
}

// The keep set of each row, one wave per row: the final set, or under track-best the best
// round's set when that one was better (RSV_FLAG) -> rank_key 1 kept / 0 dropped.
__global__ __launch_bounds__(256) void k_rs_keep(const uint8_t* __restrict__ drop, const uint8_t* __restrict__ best,
                                                 const float* __restrict__ rsv, int q_blk, int n_cand,
                                                 float* __restrict__ rank_key) {
  const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= q_blk) return;
  const long long R = (long long)blockIdx.y * q_blk + r;
  const uint8_t* src = (rsv[R * RS_NSCAL + RSV_FLAG] != 0.0f ? best : drop) + R * rs_dstride(n_cand);
  float* dst = rank_key + R * n_cand;
  for (int k = lane; k < n_cand; k += 64) dst[k] = src[k] ? 0.0f : 1.0f;
}

// ---- workspace -------------------------------------------------------------------------
struct RsWs {
  float *Vb, *Vt, *termk, *vq, *rsv, *ssq, *T;
  uint8_t *drop, *best;
  long long bytes;
};
inline long long rs_al(long long b) { return (b + 255) & ~255LL; }
inline RsWs rs_ws(void* base, int BH, int q_blk, int kb_p, int n_cand) {
  const long long R = (long long)BH * q_blk, kb64 = (long long)cdiv(kb_p, 64) * 64;
  char* p = reinterpret_cast<char*>(base);
  long long off = 0;
  RsWs w;
  auto take = [&](long long bytes) -> char* {
    char* q = p ? p + off : nullptr;
    off += rs_al(bytes);
    return q;
  };
  w.Vb = reinterpret_cast<float*>(take((long long)BH * kb64 * 64 * 4));
  w.Vt = reinterpret_cast<float*>(take((long long)BH * kb64 * 64 * 4));
  w.termk = reinterpret_cast<float*>(take((long long)BH * n_cand * 4));
  w.vq = reinterpret_cast<float*>(take(R * 64 * 4));
  w.rsv = reinterpret_cast<float*>(take(R * RS_NSCAL * 4));
  w.ssq = reinterpret_cast<float*>(take(R * n_cand * 4));
  w.T = reinterpret_cast<float*>(take(R * n_cand * 4));
  w.drop = reinterpret_cast<uint8_t*>(take(R * rs_dstride(n_cand)));
  w.best = reinterpret_cast<uint8_t*>(take(R * rs_dstride(n_cand)));
  w.bytes = off;
  return w;
}

template <int NPL, bool INIT>
int rs_launch_select(int BH, const RsSelArgs& s, hipStream_t stream) {
  hipLaunchKernelGGL((k_rs_select<NPL, INIT>), dim3(cdiv(s.q_blk, 4), BH), dim3(256), 0, stream, s);
  RESS_LAUNCHED("k_rs_select");
  return 0;
}
template <bool INIT>
int rs_select(int BH, const RsSelArgs& s, hipStream_t stream) {
  const int npl = cdiv(s.n_cand, 64);
  if (npl <= 4) return rs_launch_select<4, INIT>(BH, s, stream);
  if (npl <= 8) return rs_launch_select<8, INIT>(BH, s, stream);
  if (npl <= 12) return rs_launch_select<12, INIT>(BH, s, stream);
  if (npl <= 16) return rs_launch_select<16, INIT>(BH, s, stream);
  if (npl <= 24) return rs_launch_select<24, INIT>(BH, s, stream);
  return rs_launch_select<32, INIT>(BH, s, stream);
}

template <int MODE>
int rs_pv(int BH, const RsPvArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(k_rs_pv<MODE>, dim3(cdiv(a.q_blk, PV_ROWS) * BH), dim3(320), 0, stream, a);
  RESS_LAUNCHED("k_rs_pv");
  return 0;
}

}  // namespace

// ============================================================================
// C ABI
// ============================================================================
RESS_API long long ress_restore_swap_workspace_size(int BH, int q_blk, int kb_p, int n_cand) {
  if (BH <= 0 || q_blk < 0 || kb_p <= 0 || n_cand <= 0) return 0;
  return rs_ws(nullptr, BH, q_blk, kb_p, n_cand).bytes;
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
// reference does. workspace: ress_restore_swap_workspace_size bytes, 256-byte aligned.
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
  RESS_REQUIRE(((uintptr_t)workspace & 255u) == 0, "ress_restore_swap: workspace must be 256-byte aligned");
  const long long need = ress_restore_swap_workspace_size(BH, q_blk, kb_p, n_cand);
  RESS_REQUIRE(workspace_bytes >= need, "ress_restore_swap: workspace of %lld bytes required", need);
  if (q_blk == 0) return 0;
  const RsWs ws = rs_ws(workspace, BH, q_blk, kb_p, n_cand);
  const int kb64 = cdiv(kb_p, 64) * 64;
  const int big = (flags & RS_BF16) ? 1 : 0;
  hipLaunchKernelGGL(k_rs_head, dim3(kb64 / 64, BH), dim3(256), 0, stream, (const float*)V, (const float*)M, H, kb_p,
                     kb64, n_cand, big, ws.Vb, ws.Vt, ws.termk);
  RESS_LAUNCHED("k_rs_head");
  RsPvArgs pa;
  pa.A = (const float*)A;
  pa.M = (const float*)M;
  pa.Vt = ws.Vt;
  pa.drop = ws.drop;
  pa.best = ws.best;
  pa.vq = ws.vq;
  pa.Vb = ws.Vb;
  pa.T = ws.T;
  pa.rsv = ws.rsv;
  pa.rank_key = (float*)rank_key;
  pa.obj = (float*)obj;
  pa.H = H;
  pa.q_blk = q_blk;
  pa.kb_p = kb_p;
  pa.kb64 = kb64;
  pa.n_cand = n_cand;
  pa.flags = flags;
  pa.first = 1;
  int rc = rs_pv<RS_PV_SETUP>(BH, pa, stream);
  if (rc) return rc;
  RsSelArgs sa{ws.T, (const float*)A, ws.termk, ws.rsv, ws.ssq, (float*)s_out, ws.drop, ws.best, (const int*)nts,
               q_blk, kb_p, n_cand, flags, 0.0f};
  if ((rc = rs_select<true>(BH, sa, stream))) return rc;
  double remaining = restore_frac;
  for (int it = 0; it < n_iters; ++it) {
    const double frac = remaining * decay;
    remaining -= frac;
    pa.first = it == 0;
    if ((rc = rs_pv<RS_PV_OBJ>(BH, pa, stream))) return rc;
    sa.frac = (float)frac;
    if ((rc = rs_select<false>(BH, sa, stream))) return rc;
  }
  pa.first = n_iters == 0;
  if ((rc = rs_pv<RS_PV_FINAL>(BH, pa, stream))) return rc;
  hipLaunchKernelGGL(k_rs_keep, dim3(cdiv(q_blk, 4), BH), dim3(256), 0, stream, ws.drop, ws.best, ws.rsv, q_blk,
                     n_cand, (float*)rank_key);
  RESS_LAUNCHED("k_rs_keep");
  return 0;
}
