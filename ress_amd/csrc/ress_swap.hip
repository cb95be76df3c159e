// ReSS restore-swap block ranking for gfx950.
//
// Replaces restore_swap_rank_by (reference src/ress/scoring/projected.py:395-1058) with
// the round body of scoring/fused_round.py (kept-mass-normalised objective
// J = ||g||^2_M / K^2, drift compensate, geometric schedule, >=1 floor on beneficial
// rows, track-best) and fused_topm's exact top-m (ties to the lowest index). Every
// (batch*head, query-block) row is independent; the rows advance together, round by
// round, as the reference's batched tensors do, and each round is two kernels:
//   k_rs_pw      for 16 rows per workgroup (four waves, one chain of the sums each), the
//                drop set's sum_Pd and Pd @ v_bar on the matrix cores with the operands
//                loaded in operand order (V straight from global memory, the map through
//                LDS), then per row g,
//                M g (matrix cores), ||g||^2_M, K and J (and track-best), then the
//                candidate products v_k . big(M g) of its rows on the matrix cores;
//   k_rs_select  one wave per row: the restore / compensate qualities from the products,
//                the round's counts and the two exact top-m selections in one radix pass.
// The setup is the same pair with the dense reference (P @ v_bar, M v_bar_query, the cut
// key s/(1-P)) and the initial cut; the last k_rs_pw applies track-best, k_rs_keep writes
// the keep set.
//
// Numerics (the same operation order as oracle/ress_oracle.c):
//  * With `big` (the recipe's _bf16) every value the reference keeps in bf16 is rounded
//    at the reference's points (quadratic_deviation projected.py:259-288,
//    dense_reference :313-356, the round :903-947, fused_round.py:176-226).
//  * SEQK4 (P @ v_bar and sum P of the dense reference, Pd @ v_bar and sum_Pd of a drop
//    set): four fp32 chains, chain c over the keys of the 64-block chunks c, c + 4,
//    c + 8, ... in increasing k, fmaf(w_k, v_k[d], acc) with w_k = big(P_k), or 0 outside
//    the drop set, and the weight sum as fmaf(w_k, 1, acc); the result is
//    (chain 0 + chain 1) + (chain 2 + chain 3). v_mfma_f32_16x16x4_f32 adds its four k
//    terms to the accumulator one fmaf at a time, in k order, on gfx950 (IEEE, subnormals
//    kept), so chained steps over k = 0..3, 4..7, ... of a chain's chunks are the chain;
//    fmaf(w, 1, acc) is the rounded sum acc + w, so the weight sum is a chain of adds. An
//    accumulator that starts at +0 never holds -0, so the zero terms (masked and padding
//    blocks) leave it bit for bit unchanged, and a chain with no chunk is +0.
//  * DOT64 (v_k . Mvq and v_k . big(Mg)): one sequential fmaf chain over d = 0..63
//    (v_mfma_f32_32x32x2_f32 steps over d = (0,1), (2,3), ..., as in mfma_gemm.h).
//  * The drop set's sums are formed afresh for every objective, as the reference
//    recomputes Pd @ v_bar each round (projected.py:903-907).
//  * The 64-term products and sums of M (M v_bar_query, M g, ||g||^2_M, the term_q sums,
//    and term_k once per head) are sequential fp32 chains in index order.
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
// Operand order of a 64-block chunk (drop / best rows, Vt): key 4s + j of the chunk at
// position 16j + s, so that lane 16j + r of a v_mfma_f32_16x16x4_f32 step s finds its key's
// byte (or value) among 16 consecutive ones.
__host__ __device__ __forceinline__ int rs_dpos(int k) { return (k & ~63) | ((k & 3) << 4) | ((k >> 2) & 15); }

// Per-row scalars of the workspace (RS_NSCAL floats per row).
// RSV_FLAG: after a round's objective, 1 when the round's set becomes the best so far;
// after the final objective, 1 when the best round's set is returned.
enum { RSV_TM = 0, RSV_TQ, RSV_TQB, RSV_GN, RSV_K, RSV_J, RSV_BEST, RSV_FLAG, RS_NSCAL = 8 };

// Per-head preparation, 64 key blocks per workgroup: Vb = big(V) [kb64][64] with dim d of a
// row at (d % 4) * 16 + d / 4 (the products' B operand; rows past kb_p zero), the same
// values per 64-block chunk in the sums' operand order Vt (key 4s + j at position 16j + s),
// both as fp32, or with `big` as the bf16 bits of the (bf16-valued) big(V): the same values
// in half the bytes;
// the head's M and big(M) in operand order (workgroup 0: the matvecs' B operand) and the key
// side of quadratic_deviation, termk[k] =
// big(sum_i big(big(Mb v_k)_i * v_ki)) with the product and the sum sequential in index
// order (the block goes through an LDS tile).
__global__ __launch_bounds__(256) void k_rs_head(const float* __restrict__ V, const float* __restrict__ M, int H,
                                                 int kb_p, int kb64, int n_cand, int big, float* __restrict__ Vb,
                                                 float* __restrict__ Vt, float* __restrict__ Mop,
                                                 float* __restrict__ termk) {
  __shared__ float MbT[64 * 64];  // MbT[j*64 + i] = big(M[i][j])
  __shared__ float tile[64][65];  // [key][dim], padded
  __shared__ float pt[64][65];    // [key][dim]: big(big(Mb v_k)_i * v_ki)
  const int k0 = blockIdx.x * 64, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float* Mh = M + (long long)(bh % H) * 4096;
  for (int e = tid; e < 4096; e += 256) MbT[(e & 63) * 64 + (e >> 6)] = rs_bf(Mh[e], big);
  if (blockIdx.x == 0) {  // this head's M in operand order, rounded and not
    float* mo = Mop + (long long)bh * 8192;
    for (int e = tid; e < 4096; e += 256) {
      const int o = (e & ~63) | ((e & 3) << 4) | ((e >> 2) & 15);
      mo[o] = rs_bf(Mh[e], big);
      mo[4096 + o] = Mh[e];
    }
  }
  for (int r = w; r < 64; r += 4) {  // rows of V: lane = dim; the grid covers kb64 rows exactly
    const int k = k0 + r;
    const float x = k < kb_p ? rs_bf(V[((long long)bh * kb_p + k) * 64 + lane], big) : 0.0f;
    const long long o = ((long long)bh * kb64 + k) * 64 + ((lane & 3) << 4) + (lane >> 2);  // dim d at (d % 4) * 16 + d / 4
    if (big)
      reinterpret_cast<uint16_t*>(Vb)[o] = (uint16_t)(__float_as_uint(x) >> 16);
    else
      Vb[o] = x;
    tile[r][lane] = x;
  }
  __syncthreads();
  {  // Vt[bh][chunk][dim][pos]: key 4s + j of the chunk at pos 16j + s
    const long long o = ((long long)bh * kb64 + k0) * 64;
    for (int e = tid; e < 4096; e += 256) {
      const int pos = e & 63;
      const float x = tile[4 * (pos & 15) + (pos >> 4)][e >> 6];
      if (big)
        reinterpret_cast<uint16_t*>(Vt)[o + e] = (uint16_t)(__float_as_uint(x) >> 16);
      else
        Vt[o + e] = x;
    }
  }
  // termk: Mb v_k for the block's 64 keys on the matrix cores, the sum over j in order
  // (wave w: keys 16w.., lane 16q + r supplies A = v[16w + r][4s + q] and, for dims tile c,
  // B = Mb[16c + r][4s + q]; lane l gets keys 16w + 4(l/16) + i, dim 16c + l%16), then
  // big(big(.) * v_ki) per (key, dim) and each key's sum over the dims in order (lanes < 16)
  {
    const int am = lane & 15, aq = lane >> 4;
    rs_f4v o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = rs_f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const float xa = tile[16 * w + am][4 * st + aq];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, MbT[(4 * st + aq) * 64 + 16 * c + am], o[c], 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * w + 4 * aq + i, d = 16 * c + am;
        pt[r][d] = rs_bf(rs_bf(o[c][i], big) * tile[r][d], big);
      }
    __builtin_amdgcn_wave_barrier();  // each wave reads back only its own keys
    const int k = k0 + 16 * w + lane;
    if (lane < 16 && k < n_cand) {
      float t = 0.0f;
      for (int i = 0; i < 64; ++i) t = t + pt[16 * w + lane][i];
      termk[(long long)bh * n_cand + k] = rs_bf(t, big);
    }
  }
}

struct RsPvArgs {
  const float* A;   // [BH][q_blk][kb_p] pooled map
  const float* Vt;  // [BH][kb64/64][64 dims][64] big(V) per chunk in operand order, zero past kb_p
  const float* Vb;  // [BH][kb64][64] big(V), zero rows past kb_p; dim d of a row at (d % 4) * 16 + d / 4
                    // (Vt, Vb: fp32, or bf16 bits when the k-wide tensors are bf16)
  const float* Mop;  // [BH][2][64][64]: big(M), then M, element j of row i at (j % 4) * 16 + j / 4
  uint8_t* drop;    // [BH][q_blk][rs_dstride] 1 = dropped, candidates at rs_dpos
  uint8_t* best;    // [BH][q_blk][rs_dstride] the track-best set, the same order
  float* vq;        // [BH][q_blk][64] big(v_bar_query)
  float* T;         // [BH][q_blk][n_cand] setup: v_k . big(Mb vq); rounds: v_k . big(M g)
  float* rsv;       // [BH][q_blk][RS_NSCAL]
  float* rank_key;  // [BH][q_blk][n_cand] final: 1 kept, 0 dropped
  float* obj;       // [BH][q_blk] final (optional): J of the returned set
  int H, q_blk, kb_p, kb64, n_cand, flags, first;
};

enum { RS_PV_SETUP = 0, RS_PV_OBJ = 1, RS_PV_FINAL = 2 };
// ---- k_rs_pw: four waves per 16 rows -------------------------------------------------
// The drop-set sums of 16 rows of one head per workgroup on the matrix cores
// (v_mfma_f32_16x16x4_f32), in the SEQK4 order: wave c runs chain c, the 64-block chunks
// c, c + 4, ... of the row, and the four chains are added as (c0 + c1) + (c2 + c3). Lane
// l = 16j + r supplies, at step s of a chunk, A = w[row r][key 4s + j] (the pooled map,
// masked by the drop bytes and rounded as it is read) and, for dims tile t, B =
// big(V)[key 4s + j][dim 16t + r], which Vt keeps at position 16j + s of dim 16t + r: four
// 16-byte global loads per tile and chunk, no LDS. The map's chunk is loaded a row per
// instruction (lane = key) into the wave's LDS tile and read back in operand order; the
// drop bytes of a lane's 16 keys are one 16-byte load. Each wave accumulates all four dims
// tiles and the weight sum (B = 1 in column 0); every accumulator takes its chain's k terms
// in order, and lane l ends with rows 4j + i of column r of each tile. A wave's chunks are
// loaded one ahead into two register sets used in turn; the waves never wait for each
// other until their chains end.
// After the sums the row vectors go through LDS as 16 x 64 row-major tiles: wave h adds
// the chains of, and computes, columns 16h.. of the matvecs M g (or big(M) vq) on the
// matrix cores (A = g[r][4s + j] from LDS, B = M[16h + r][4s + j] from Mop), wave 0's row
// lanes the scalar chains (||g||^2_M, tq, tqb), and waves 1..3 the candidate products in
// blocks of 16 (A = X[r][4s + j], B = big(V)[16b + r][4s + j], contiguous in Vb's layout).
constexpr int PW_ROWS = 16;
constexpr int PW_LD = 68;  // LDS tile row stride
constexpr int PW_NW = 4;   // waves per 16 rows = SEQK4 chains

// A lane's 16 values of V for one step range of a dims tile (or a candidate row): fp32 in
// four float4, or bf16 bits in two uint4 (BV); value st as an fp32 operand.
template <bool BV>
struct PwV;
template <>
struct PwV<false> {
  float4 v[4];
  __device__ __forceinline__ void load(const void* base, long long o) {  // o: offset of value 0, in values
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + o)[q];
  }
  __device__ __forceinline__ float at(int st) const {
    const float4 y = v[st >> 2];
    return (st & 3) == 0 ? y.x : (st & 3) == 1 ? y.y : (st & 3) == 2 ? y.z : y.w;
  }
};
template <>
struct PwV<true> {
  uint4 v[2];
  __device__ __forceinline__ void load(const void* base, long long o) {
#pragma unroll
    for (int q = 0; q < 2; ++q) v[q] = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + o)[q];
  }
  __device__ __forceinline__ float at(int st) const {
    const uint4 y = v[st >> 3];
    const int q = (st >> 1) & 3;
    const uint32_t w = q == 0 ? y.x : q == 1 ? y.y : q == 2 ? y.z : y.w;
    return __uint_as_float((st & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};

template <bool BV>
struct PwSet {
  float x[PW_ROWS];  // the chunk of the map rows: row e, key k0 + lane
  uint4 dm;
  PwV<BV> v[4];  // dims tile c
};

template <int MODE, bool BV>
__global__ __launch_bounds__(64 * PW_NW, BV ? 3 : 2) void k_rs_pw(RsPvArgs a) {
  __shared__ __align__(16) float T0[PW_ROWS * PW_LD];  // g (or vq in the setup)
  __shared__ __align__(16) float T1[PW_ROWS * PW_LD];  // M g (or X in the setup)
  __shared__ __align__(16) float T2[PW_ROWS * PW_LD];  // vq (rounds)
  __shared__ float spw[PW_NW][PW_ROWS];                // the chains' weight sums
  __shared__ __align__(16) float Aw[PW_NW][PW_ROWS * PW_LD];  // per wave: its chunk's map rows, then its chains
  const int tid = threadIdx.x, lane = tid & 63, am = lane & 15, aq = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware order (workgroup L runs on XCD L % 8): with a multiple of 8 heads, XCD x takes
  // heads x, x + 8, ... whole, so each XCD's L2 holds the V of only its own heads
  const int G = cdiv(a.q_blk, PW_ROWS), BH = gridDim.x / G, L = blockIdx.x;
  int bh, grp;
  if ((BH & 7) == 0) {
    const int jj = L >> 3;
    bh = (L & 7) + 8 * (jj / G);
    grp = jj % G;
  } else {
    bh = L / G;
    grp = L % G;
  }
  const int g0 = grp * PW_ROWS, nrow = min(PW_ROWS, a.q_blk - g0);
  const bool big = a.flags & RS_BF16;
  const int kend = MODE == RS_PV_SETUP ? a.kb_p : a.n_cand;
  const long long rowbase = (long long)bh * a.q_blk + g0;
  const int dstr = rs_dstride(a.n_cand);
  const bool rok = am < nrow;
  const int ra = min(am, nrow - 1);  // clamped row: every load stays in the matrix
  const uint8_t* Dr = a.drop + (rowbase + ra) * dstr;
  // the map's chunk is loaded a row per instruction (lane = key: one contiguous 256-byte
  // run; rows past nrow read row nrow - 1, keys past kend key kend - 1, both masked later)
  const float* A0 = a.A + rowbase * a.kb_p;
  // this lane's V: dims 16c + am, positions 16aq.. of each chunk
  const long long vo = (long long)bh * a.kb64 * 64 + am * 64 + aq * 16;
  const int nch = cdiv(kend, 64);
  float* aw = Aw[wv];
  auto load = [&](PwSet<BV>& S, int ch) {
    ch = min(ch, nch - 1);  // past the chain's end: a chunk in range, not used
    const int k0 = ch * 64;
#pragma unroll
    for (int e = 0; e < PW_ROWS; ++e) S.x[e] = A0[(long long)min(e, nrow - 1) * a.kb_p + min(k0 + lane, kend - 1)];
    if (MODE != RS_PV_SETUP) S.dm = *reinterpret_cast<const uint4*>(Dr + k0 + 16 * aq);
#pragma unroll
    for (int c = 0; c < 4; ++c) S.v[c].load(a.Vt, vo + (long long)ch * 4096 + c * 1024);
  };
  rs_f4v acc[5];  // [4]: the weight sum
#pragma unroll
  for (int t = 0; t < 5; ++t) acc[t] = rs_f4v{0.0f, 0.0f, 0.0f, 0.0f};
  const float one = am == 0 ? 1.0f : 0.0f;
  auto compute = [&](const PwSet<BV>& S, int ch) {
    const int k0 = ch * 64;
    const uint32_t dw[4] = {S.dm.x, S.dm.y, S.dm.z, S.dm.w};
    // through the wave's LDS tile into operand order: lane 16j + r reads keys 4s + j of row r
    // (bank (4r + 4s + j) mod 64: the 64 lanes of a step hit 64 banks). A wave's LDS accesses
    // complete in issue order, so the tile is rewritten only after the previous reads.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int e = 0; e < PW_ROWS; ++e) aw[e * PW_LD + lane] = S.x[e];
    __builtin_amdgcn_wave_barrier();
    float xs[16];
#pragma unroll
    for (int st = 0; st < 16; ++st) xs[st] = aw[am * PW_LD + 4 * st + aq];
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const bool in = rok && k0 + 4 * st + aq < kend &&
                      (MODE == RS_PV_SETUP || ((dw[st >> 2] >> (8 * (st & 3))) & 0xffu));
      const float x = in ? rs_bf(xs[st], big) : 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, S.v[c].at(st), acc[c], 0, 0, 0);
      acc[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, one, acc[4], 0, 0, 0);
    }
  };
  if (wv < nch) {  // uniform per wave: chain wv
    PwSet<BV> s0, s1;
    load(s0, wv);
#pragma unroll 1
    for (int ch = wv; ch < nch; ch += 2 * PW_NW) {
      load(s1, ch + PW_NW);
      __builtin_amdgcn_sched_barrier(0);
      compute(s0, ch);
      if (ch + PW_NW >= nch) break;  // uniform per wave
      load(s0, ch + 2 * PW_NW);
      __builtin_amdgcn_sched_barrier(0);
      compute(s1, ch + PW_NW);
    }
  }
  // ---- per-row vector math ----------------------------------------------------------
  // the chains into the waves' tiles (each wave's own reads of its tile are done), then
  // lane l of wave h adds them for rows 4(l/16) + i, column 16h + l%16
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) aw[(4 * aq + i) * PW_LD + 16 * c + am] = acc[c][i];
  if (am == 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) spw[wv][4 * aq + i] = acc[4][i];
  __syncthreads();
  const int cb = 16 * wv + am;  // this lane's column
  float cs[4];                  // the SEQK4 sums of rows 4aq + i, column cb
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int o = (4 * aq + i) * PW_LD + cb;
    cs[i] = (Aw[0][o] + Aw[1][o]) + (Aw[2][o] + Aw[3][o]);
  }
  auto wsum = [&](int r) { return (spw[0][r] + spw[1][r]) + (spw[2][r] + spw[3][r]); };
  const float* Mo = a.Mop + (long long)bh * 8192 + (MODE == RS_PV_SETUP ? 0 : 4096);
  float* scr = a.rsv + (rowbase + am) * RS_NSCAL;  // lane r < nrow: row r's scalars
  // this wave's columns of the 16 x 64 tile in T0 times M^T on the matrix cores,
  // out[r][i] = sum_j in order M[i][j] * T0[r][j]
  auto matvec = [&]() {
    rs_f4v o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 m4 = reinterpret_cast<const float4*>(Mo + cb * 64 + 16 * aq)[q];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float xa = T0[am * PW_LD + 4 * (4 * q + u) + aq];
        o = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, u == 0 ? m4.x : u == 1 ? m4.y : u == 2 ? m4.z : m4.w, o, 0, 0,
                                                  0);
      }
    }
    return o;
  };
  if constexpr (MODE == RS_PV_SETUP) {
    // vq = big(C) (T0 and the workspace), tm = big(sum w)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * aq + i;
      const float v = rs_bf(cs[i], big);
      T0[r * PW_LD + cb] = v;
      if (r < nrow) a.vq[(rowbase + r) * 64 + cb] = v;
    }
    if (wv == 0 && lane < nrow) scr[RSV_TM] = rs_bf(wsum(lane), big);
    __syncthreads();
    const rs_f4v mo = matvec();  // big(M) vq
#pragma unroll
    for (int i = 0; i < 4; ++i) T1[(4 * aq + i) * PW_LD + cb] = rs_bf(mo[i], big);  // X
    __syncthreads();
    if (wv == 0 && lane < nrow) {
      float tq = 0.0f;
      for (int i = 0; i < 64; ++i) tq = tq + rs_bf(T1[lane * PW_LD + i] * T0[lane * PW_LD + i], big);
      scr[RSV_TQ] = rs_bf(tq, big);
    }
  } else {
    const bool track = a.flags & RS_TRACK_BEST, maxim = a.flags & RS_MAXIMIZE;
    // g = big(sum w) vq - big(C)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * aq + i;
      const float vq = a.vq[(rowbase + min(r, nrow - 1)) * 64 + cb];
      T2[r * PW_LD + cb] = vq;
      T0[r * PW_LD + cb] = rs_bf(wsum(r), big) * vq - rs_bf(cs[i], big);
    }
    __syncthreads();
    const rs_f4v mo = matvec();  // M g
#pragma unroll
    for (int i = 0; i < 4; ++i) T1[(4 * aq + i) * PW_LD + cb] = mo[i];
    __syncthreads();
    if (wv == 0 && lane < nrow) {
      const float* g = &T0[lane * PW_LD];
      const float* Mg = &T1[lane * PW_LD];
      const float sp = rs_bf(wsum(lane), big);
      float gn = 0.0f;
      for (int d = 0; d < 64; ++d) gn = gn + g[d] * Mg[d];
      float K = scr[RSV_TM] - sp;
      K = K < 1e-6f ? 1e-6f : K;
      const float J = gn / (K * K);
      int f = 0;
      if constexpr (MODE == RS_PV_OBJ) {
        const float* vq = &T2[lane * PW_LD];
        float tqr = 0.0f;
        for (int d = 0; d < 64; ++d) tqr = tqr + vq[d] * Mg[d];
        scr[RSV_TQB] = rs_bf(tqr, big);
        scr[RSV_GN] = gn;
        scr[RSV_K] = K;
        scr[RSV_J] = J;
        if (track) {  // this round's set becomes the best when it beats the best so far
          const float b = scr[RSV_BEST];
          f = a.first || (maxim ? J > b : J < b);
          if (f) scr[RSV_BEST] = J;
        }
      } else {
        float fin = J;
        if (track && !a.first) {
          const float b = scr[RSV_BEST];
          if (!(maxim ? J > b : J < b)) {  // the final set is not better: return the best one
            f = 1;
            fin = b;
          }
        }
        if (a.obj) a.obj[rowbase + lane] = fin;
      }
      scr[RSV_FLAG] = (float)f;
    }
  }
  if constexpr (MODE != RS_PV_FINAL) {
    // ---- candidate products: T[r][k] = X[r] . big(V_k), blocks of 16
    float xa[16];
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const float x = T1[am * PW_LD + 4 * st + aq];
      xa[st] = MODE == RS_PV_OBJ ? rs_bf(x, big) : x;  // the setup's X is rounded already
    }
    const int nb = cdiv(a.n_cand, 16);
    const long long vbo = (long long)bh * a.kb64 * 64 + 16 * aq;
    float* Tg = a.T + rowbase * a.n_cand;
    auto loadb = [&](PwV<BV>& y, int b) { y.load(a.Vb, vbo + (long long)min(16 * min(b, nb - 1) + am, a.kb64 - 1) * 64); };
    auto block = [&](const PwV<BV>& y, int b) {
      rs_f4v o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 16; ++st) o = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[st], y.at(st), o, 0, 0, 0);
      const int col = 16 * b + am;
      if (col < a.n_cand)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * aq + i < nrow) Tg[(long long)(4 * aq + i) * a.n_cand + col] = o[i];
    };
    // wave 0's row lanes ran the scalar chains, so the other waves take the blocks
    constexpr int P0 = 1, PS = PW_NW - P0;
    PwV<BV> y0, y1;
    int b = wv - P0;
    if (b >= 0 && b < nb) {  // uniform
      loadb(y0, b);
#pragma unroll 1
      for (; b < nb; b += 2 * PS) {
        loadb(y1, b + PS);
        __builtin_amdgcn_sched_barrier(0);
        block(y0, b);
        if (b + PS >= nb) break;  // uniform
        loadb(y0, b + 2 * PS);
        __builtin_amdgcn_sched_barrier(0);
        block(y1, b + PS);
      }
    }
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
  const float* T;      // [BH][q_blk][n_cand] raw candidate products v_k . X (k_rs_pw)
  const float* A;      // [BH][q_blk][kb_p] pooled map
  const float* termk;  // [BH][n_cand]
  const float* rsv;    // [BH][q_blk][RS_NSCAL]
  float* ssq;          // [BH][q_blk][n_cand] s^2 (written by INIT, read by the rounds)
  float* s_out;        // [BH][q_blk][n_cand] or null: s (INIT)
  uint8_t* drop;       // [BH][q_blk][rs_dstride] candidates at rs_dpos
  uint8_t* best;       // [BH][q_blk][rs_dstride] the track-best set, the same order
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
  const float* xr = INIT ? a.termk + (long long)bh * n : sr;
  float tv[NPL], pv[NPL], xv[NPL];
  uint32_t cand = 0u;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int k = lane + 64 * i;
    if (k < n) cand |= 1u << i;
    const unsigned kc = (unsigned)min(k, n - 1);
    tv[i] = at_u32(Tr, kc);
    pv[i] = at_u32(Ar, kc);
    xv[i] = at_u32(xr, kc);
  }
  uint32_t dropb = 0u;
  if constexpr (!INIT) {
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (at_u32(dr, (unsigned)rs_dpos(min(lane + 64 * i, n - 1)))) dropb |= 1u << i;
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
        at_u32(sr, (unsigned)k) = rs_bf(s * s, big);
        if (a.s_out) at_u32(a.s_out + R * n, (unsigned)k) = s;
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
        if (64 * i < rs_dstride(n)) at_u32(br, (unsigned)rs_dpos(lane + 64 * i)) = (uint8_t)((dropb >> i) & 1u);
    }
    // set 0: the dropped candidates (restore the top cnt), set 1: the kept (drop the top cnt)
    rs_top_m_pair<NPL>(key, cand, cand & ~dropb, cnt, cnt, lane, hist[w], sel0, sel1);
    nd = (dropb & ~sel0) | sel1;
  }
#pragma unroll
  for (int i = 0; i < NPL; ++i)  // uniform bound: the row's padding past n is never read
    if (64 * i < rs_dstride(n)) at_u32(dr, (unsigned)rs_dpos(lane + 64 * i)) = (uint8_t)((nd >> i) & 1u);
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
  for (int k = lane; k < n_cand; k += 64) dst[k] = src[rs_dpos(k)] ? 0.0f : 1.0f;
}

// ---- workspace -------------------------------------------------------------------------
struct RsWs {
  float *Vb, *Vt, *Mop, *termk, *vq, *rsv, *ssq, *T;
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
  w.Mop = reinterpret_cast<float*>(take((long long)BH * 8192 * 4));
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
  const dim3 grid(cdiv(a.q_blk, PW_ROWS) * BH), block(64 * PW_NW);
  if (a.flags & RS_BF16)  // k_rs_head stored big(V) as bf16 bits
    hipLaunchKernelGGL((k_rs_pw<MODE, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((k_rs_pw<MODE, false>), grid, block, 0, stream, a);
  RESS_LAUNCHED("k_rs_pw");
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
                     kb64, n_cand, big, ws.Vb, ws.Vt, ws.Mop, ws.termk);
  RESS_LAUNCHED("k_rs_head");
  RsPvArgs pa;
  pa.A = (const float*)A;
  pa.Vt = ws.Vt;
  pa.drop = ws.drop;
  pa.best = ws.best;
  pa.vq = ws.vq;
  pa.Vb = ws.Vb;
  pa.Mop = ws.Mop;
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
