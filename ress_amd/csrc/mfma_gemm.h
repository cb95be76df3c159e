// fp32 GEMM over 64-dim rows on the matrix cores: for every (bh, r, c) with
// r_begin <= r < r_end, c < nb, acc = DOT64(a[bh][r], b[bh][c]), the sequential fmaf chain
// over d = 0..63 exactly (v_mfma_f32_32x32x2_f32 adds its two k terms to the accumulator as
// fmaf(a1, b1, fmaf(a0, b0, c)) on gfx950, IEEE with subnormals kept; 32 chained steps over
// k = (0,1), (2,3), ... are the chain). The caller's epilogue receives each 128 x 128 tile.
//
// A workgroup of 4 waves takes a 128-row tile and walks column tiles of 128 (tiles
// blockIdx.x, blockIdx.x + gridDim.x, ..., at most the epilogue's kWalk). Wave w holds rows 32w..32w+31
// of the A operand in registers for the whole walk and computes them against all 128
// columns of each tile (4 column sub-tiles of 32). Step s takes dim 2s + l/32 of row l%32
// from lane l, so B tiles sit in LDS with each row's 64 dims split into the even dims
// (floats 0..31) and the odd dims (32..63): a lane's 32 values are one contiguous run, read
// as 8 float4s; the 68-float row stride puts 16 consecutive rows' float4 reads in distinct
// banks. B tiles are double-buffered: the next tile's loads are in flight during the MFMAs.
#pragma once
#include "common.h"

constexpr int G64_T = 128;
constexpr int G64_LD = 68;
typedef float g64_f16v __attribute__((ext_vector_type(16)));

// The tile a workgroup hands to its epilogue: rows r0.., columns c0.. of head bh; lane
// element j of accumulator ct is row r0 + lrow + 8(j/4) + j%4, column c0 + 32ct + rl.
struct G64Tile {
  int bh, r0, c0, lrow, rl;
};

// a [bh][na][64], b rows c of head bh at b + bh * b_head + 64c.
template <class Epi>
__global__ __launch_bounds__(256) void k_gemm64(const float* __restrict__ a, const float* __restrict__ b, int na,
                                                int nb, long long b_head, int r_begin, int r_end, Epi epi) {
  constexpr int NB = Epi::kWalk > 1 ? 2 : 1;  // B buffers: a walk double-buffers its tiles
  __shared__ __align__(16) float bl[NB][G64_T * G64_LD];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = r_begin + blockIdx.y * G64_T, bh = blockIdx.z, h = lane >> 5, rl = lane & 31;
  const int ntile = cdiv(nb, G64_T);
  const float* bhd = b + (long long)bh * b_head;
  // B tile loads: 2048 float4 chunks, chunk f = row f/16, dims 4(f%16)..+3; rows past the
  // matrix read its last row (zeroed when written to LDS; their outputs are not stored)
  float4 ys[8];
  auto load_b = [&](int t) {
    const int c0 = t * G64_T;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i;
      ys[i] = reinterpret_cast<const float4*>(bhd + (long long)min(c0 + (f >> 4), nb - 1) * 64)[f & 15];
    }
  };
  auto store_b = [&](int t, float* dst) {
    const int c0 = t * G64_T;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + 256 * i, r = f >> 4, q = f & 15;
      const float4 y = c0 + r < nb ? ys[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      // dims 4q and 4q+2 go to even positions 2q, 2q+1; dims 4q+1 and 4q+3 to the odd half
      *reinterpret_cast<float2*>(dst + r * G64_LD + 2 * q) = make_float2(y.x, y.z);
      *reinterpret_cast<float2*>(dst + r * G64_LD + 32 + 2 * q) = make_float2(y.y, y.w);
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
  constexpr int BCT = 32 * G64_LD / 4;  // float4s between column sub-tiles
#pragma unroll 1
  for (int it = 0;; ++it) {
    const int tn = t + (int)gridDim.x;
    const bool more = it + 1 < Epi::kWalk && tn < ntile;  // uniform
    if (more) load_b(tn);
    const float4* bp = reinterpret_cast<const float4*>(bl[it & (NB - 1)] + rl * G64_LD + 32 * h);
    g64_f16v acc[4];
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
    epi(G64Tile{bh, r0, t * G64_T, lrow, rl}, na, nb, r_end, acc);
    if (!more) break;
    // buffer (it+1)&1 was last read in the previous iteration, which every wave finished
    // before the barrier that ended it
    store_b(tn, bl[(it + 1) & (NB - 1)]);
    __syncthreads();
    t = tn;
  }
}

// The plain epilogue: S[bh][r][c] = acc * scale, row-major with nb columns.
template <int WALK = 4>
struct G64Store {
  static constexpr int kWalk = WALK;  // column tiles per workgroup (the A rows stay in registers)
  float* S;
  float scale;
  __device__ __forceinline__ void operator()(const G64Tile& t, int na, int nb, int r_end,
                                             const g64_f16v (&acc)[4]) const {
    // byte offsets from the (uniform) tile origin (below 2^31: 128 rows of at most 2^21
    // floats), unsigned so that the stores take the scalar-base + 32-bit offset form
    char* tile = reinterpret_cast<char*>(S + ((long long)t.bh * na + t.r0) * nb + t.c0);
    if (t.r0 + G64_T <= r_end && t.c0 + G64_T <= nb) {  // whole tile (uniform): no per-store test
      unsigned lofs = 4u * (unsigned)(t.lrow * nb + t.rl);
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
      int rlim = r_end - t.r0 - t.lrow, clim = nb - t.c0 - t.rl;
      unsigned lofs = 4u * (unsigned)(t.lrow * nb + t.rl);
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
  }
};

// grid of k_gemm64 for rows [r_begin, r_end) and nb columns over BH heads, `walk` column
// tiles per workgroup (the epilogue's kWalk)
inline dim3 g64_grid(int BH, int nb, int r_begin, int r_end, int walk) {
  return dim3(cdiv(cdiv(nb, G64_T), walk), cdiv(r_end - r_begin, G64_T), BH);
}
