// Shared device-side definitions for libress_hip (gfx950 / CDNA4).
//
// Numerics contract. Every kernel that feeds a block map (pooling, the pooled
// softmax, the CDF budget, the HeSS reallocation, top-k selection, restore-swap)
// fixes its floating-point evaluation order so that the result is a pure
// function of the inputs. The orders are:
//
//   SUM8x(T)   block pooling over T tokens with 8 token lanes:
//              p_j = ((0 + x[j]) + x[8+j]) + x[16+j] ...   for j = 0..7
//              (only the block's valid tokens, in increasing token order)
//              total = ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7))
//   SUM64(n)   row sums: p_l = sequential sum of x[i] for i = l, l+64, l+128 ...
//              for l = 0..63, then a butterfly: at offsets 1,2,4,8,16,32 every
//              partial becomes partial[l] + partial[l ^ off].
//   DOT64      pooled dot products: acc = fmaf(a[d], b[d], acc), d = 0..63, from 0.
//              On gfx950 v_mfma_f32_32x32x2_f32 adds its two k terms to the
//              accumulator as fmaf(a1, b1, fmaf(a0, b0, c)), IEEE with subnormals
//              kept (checked bit for bit against that chain on the GPU, random and
//              subnormal operands), so 32 chained steps over k = (0,1), (2,3), ...
//              are DOT64 exactly (scores_gemm).
//   SEQ        sequential sums in index order (CDF prefix sums, HeSS head sums,
//              the key mean over blocks).
//
// Division and square root are IEEE correctly rounded (hipcc's default
// -fhip-fp32-correctly-rounded-divide-sqrt), and every file is compiled with
// -ffp-contract=off so no multiply-add is fused unless written as fmaf().
// ress_expf is Cody-Waite argument reduction plus a degree-7 Taylor polynomial
// evaluated by Horner's rule; it is written out here (not the device libm) so
// its bits are fixed.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#define RESS_API extern "C" __attribute__((visibility("default")))

// Element i of a row through a 32-bit byte offset from the row's base. With a uniform base
// the access takes the scalar-base + zero-extended vector-offset form; a plain base[i]
// forms a 64-bit address per lane with a VALU add (i*sizeof(T) is computed in 64 bits).
// The row must span less than 4 GiB.
template <class T>
__device__ __forceinline__ T& at_u32(T* base, unsigned i) {
  return *reinterpret_cast<T*>(reinterpret_cast<char*>(const_cast<std::remove_const_t<T>*>(base)) +
                               i * (unsigned)sizeof(T));
}

// ---- error reporting (defined in capi.hip) --------------------------------
void ress_set_error(const char* fmt, ...);

#define RESS_REQUIRE(cond, ...)        \
  do {                                 \
    if (!(cond)) {                     \
      ress_set_error(__VA_ARGS__);     \
      return -1;                       \
    }                                  \
  } while (0)

#define RESS_LAUNCHED(name)                                                   \
  do {                                                                        \
    hipError_t _e = hipGetLastError();                                        \
    if (_e != hipSuccess) {                                                   \
      ress_set_error("%s: launch failed: %s", name, hipGetErrorString(_e));   \
      return -2;                                                              \
    }                                                                         \
  } while (0)

// ---- geometry --------------------------------------------------------------
// Token layout of one (batch, head) sequence as the backbone produces it:
// frames of P tokens, the first S of each frame special (camera/register),
// the remaining HW patch tokens. The kernels address tokens in "kernel order":
// patch tokens first (frame-major), then special tokens (frame-major), which is
// the reference's cat([k_patch, k_special]) (attention.py:405-406). S == 0 is the
// plain full-sequence layout (kernel order == storage order).
struct TokenMap {
  int P;    // tokens per frame in storage
  int S;    // special tokens per frame
  int HW;   // patch tokens per frame (P - S)
  int T_p;  // total patch tokens (frames * HW)
  int T_s;  // total special tokens (frames * S)
  // Patch order within a frame (null: storage order). The kernels' patch token j of a frame
  // is the frame's patch token perm[j] in storage, so blocks are formed in this order (the
  // reference's hilbert_permute, src/ress/models/hilbert.py:128-162, read in place instead
  // of a permuted copy). perm must be a permutation of 0..HW-1; entries are clamped into
  // range so a bad table cannot address outside the frame.
  const int* perm;
};

__device__ __forceinline__ int patch_to_storage(int p, const TokenMap& m) {
  const int f = p / m.HW, j = p - f * m.HW;
  return f * m.P + m.S + (m.perm ? min(max(m.perm[j], 0), m.HW - 1) : j);
}
__device__ __forceinline__ int special_to_storage(int s, const TokenMap& m) {
  int f = s / m.S;
  return f * m.P + (s - f * m.S);
}
// kernel key index -> storage index
__device__ __forceinline__ int key_to_storage(int kk, const TokenMap& m) {
  return kk < m.T_p ? patch_to_storage(kk, m) : special_to_storage(kk - m.T_p, m);
}

// ---- bf16 ------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ void unpack_bf16x8(const uint4& r, float x[8]) {
  x[0] = bf16_lo(r.x); x[1] = bf16_hi(r.x);
  x[2] = bf16_lo(r.y); x[3] = bf16_hi(r.y);
  x[4] = bf16_lo(r.z); x[5] = bf16_hi(r.z);
  x[6] = bf16_lo(r.w); x[7] = bf16_hi(r.w);
}
// two floats -> packed fp16 pair (round to nearest even), lo in bits 0..15
__device__ __forceinline__ uint32_t f32x2_to_f16_bits(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}
// fp32 -> bf16, round to nearest even, a NaN made quiet with its payload's high bits kept:
// the bits of ((u + 0x7fff + ((u >> 16) & 1)) >> 16) for numbers and ((u >> 16) | 0x40) for
// NaNs. gfx950's v_cvt_pk_bf16_f32 (the __bf16 conversion) gives exactly these bits for
// every one of the 2^32 inputs (checked exhaustively on the device, subnormals included).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(f32_to_bf16_bits(f) << 16);
}

// ---- exp -------------------------------------------------------------------
// e^x = 2^n * e^r, n = rint(x*log2(e)), r = x - n*ln2 (two-constant Cody-Waite
// split of ln2), e^r by the Taylor series to degree 7 (|r| <= 0.347 keeps the
// truncation error below 0.05 ulp).
__device__ __forceinline__ float ress_expf(float x) {
  if (x != x) return x;
  if (x > 0x1.62e42ep+6f) return __builtin_huge_valf();
  if (x < -0x1.9fe368p+6f) return 0.0f;
  float n = rintf(x * 0x1.715476p+0f);
  float r = fmaf(-n, 0x1.62e4p-1f, x);
  r = fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0x1p-1f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) return (p * 2.0f) * 0x1p127f;
  if (ni < -126) return (p * __int_as_float((ni + 127 + 64) << 23)) * 0x1p-64f;
  return p * __int_as_float((ni + 127) << 23);
}

// ---- strided (B, H, T, D) operands ----------------------------------------
struct Strides {  // element strides of a (B, H, T, D) tensor in any layout
  long long b, h, t;
  int H;
};
__device__ __forceinline__ long long bh_offset(int bh, const Strides& s) {
  return (long long)(bh / s.H) * s.b + (long long)(bh % s.H) * s.h;
}

// ---- int8 packing ------------------------------------------------------------
__device__ __forceinline__ uint2 pack_i8x8(const int c[8]) {
  // byte permutes (v_perm_b32: selector bytes 0-3 take the second operand's bytes, 4-7
  // the first's, 0x0c a zero byte): the low bytes of c[0..3] in order, then of c[4..7]
  uint32_t w[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)c[4 * h + 1], (uint32_t)c[4 * h], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)c[4 * h + 3], (uint32_t)c[4 * h + 2], 0x0c0c0400u);
    w[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  }
  return make_uint2(w[0], w[1]);
}

// ---- order keys ------------------------------------------------------------
// Order-preserving fp32 -> uint32 (unsigned compare == float compare; -0 == +0;
// NaN above +inf).
__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---- per-block int8 quantiser ---------------------------------------------
// scale = amax/127; q = trunc(x/scale + 0.5*sign) (round half away from zero),
// the published SageAttention per-block rule. A block whose amax is 0 has scale
// 0 and all-zero codes.
__device__ __forceinline__ int quant_i8(float x, float scale) {
  if (scale == 0.0f) return 0;
  float y = x / scale;
  y = y + (y >= 0.0f ? 0.5f : -0.5f);
  return (int)y;
}
// quant_i8 without a division per element: rcp = 1/scale (IEEE, once per block). y = x*rcp
// is within 2^-15 of x/scale for the codes' range (|x/scale| <= 127.5: two roundings of
// relative size 2^-24); the code is trunc(|y| + 0.5) with y's sign, so it can differ from
// quant_i8's only when |y| + 0.5 lies within that distance of an integer. Those elements
// (fraction within 2^-12 of an integer), NaN and infinities take quant_i8 itself, so the
// result is identical for every input.
__device__ __forceinline__ int quant_i8_rcp(float x, float scale, float rcp) {
  const float y = x * rcp;
  const float a = fabsf(y) + 0.5f;
  const float f = a - floorf(a);
  if (scale != 0.0f && f > 0x1p-12f && f < 1.0f - 0x1p-12f) {
    const int m = (int)a;
    return y >= 0.0f ? m : -m;
  }
  return quant_i8(x, scale);
}
// quant_i8_rcp over 8 elements: the fast codes of all 8, then, only if one of them is
// not trusted (or scale is 0), quant_i8 for those. Identical to quant_i8 per element, with
// one branch where quant_i8_rcp takes one per element. a = y + copysign(0.5, y) is
// sign(y) * (|y| + 0.5) with the same rounding, its truncation the code; the fraction of
// |a| (exact) must lie at least 2^-12 away from 0 and 1.
__device__ __forceinline__ void quant_i8x8_rcp(const float (&x)[8], float scale, float rcp, int (&c)[8]) {
  bool fast[8], all = scale != 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = x[i] * rcp;
    const float a = y + __builtin_copysignf(0.5f, y);
    const float f = __builtin_amdgcn_fractf(fabsf(a));
    fast[i] = fabsf(f - 0.5f) < 0.5f - 0x1p-12f;
    all = all && fast[i];
    c[i] = (int)a;
  }
  if (!all) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!(scale != 0.0f && fast[i])) c[i] = quant_i8(x[i], scale);
  }
}
// Two-term ("split") INT8: x ~ scale*hi + (scale/254)*lo. hi is the per-block code
// above; lo quantises the exact residual fmaf(-scale, hi, x) (|r| <= scale/2) with the
// scale scale/254, so |lo| <= 127.
__device__ __forceinline__ int quant_i8_lo(float x, float scale, int hi) {
  if (scale == 0.0f) return 0;
  return quant_i8(fmaf(-scale, (float)hi, x), scale / 254.0f);
}

// ---- wave scans and reductions (wave64, every lane active) -----------------
// DPP moves (GFX9 encodings): row_shr:n (0x110 + n) within 16-lane rows, row_bcast:15 /
// row_bcast:31 (0x142 / 0x143) carry lane 15 / 31 of a row pair into the rows the row mask
// selects. A lane without a source (or outside the row mask) gets `old`. Four row shifts
// and the two broadcasts make an inclusive scan over the 64 lanes; lane 63 then holds the
// whole reduction. Used for integer sums and for maxima / minima, which are exact in any
// order, so these return the same values as lane-shuffle trees without the LDS round trips
// of ds_bpermute. Float sums keep their shuffle trees (their order is part of the result).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xf, false);
}
template <typename Op>
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x, uint32_t identity, Op op) {
  x = op(x, dpp_u32<0x111, 0xf>(identity, x));
  x = op(x, dpp_u32<0x112, 0xf>(identity, x));
  x = op(x, dpp_u32<0x114, 0xf>(identity, x));
  x = op(x, dpp_u32<0x118, 0xf>(identity, x));
  x = op(x, dpp_u32<0x142, 0xa>(identity, x));
  x = op(x, dpp_u32<0x143, 0xc>(identity, x));
  return x;
}
__device__ __forceinline__ uint32_t lane63(uint32_t x) { return (uint32_t)__builtin_amdgcn_readlane((int)x, 63); }
// inclusive prefix sum over lanes 0..l
__device__ __forceinline__ int wave_scan_sum_i(int x) {
  return (int)wave_scan_u32((uint32_t)x, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
template <int C, int R>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const uint32_t lo = dpp_u32<C, R>(0u, (uint32_t)v), hi = dpp_u32<C, R>(0u, (uint32_t)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_scan_sum_u64(unsigned long long x) {
  x += dpp_u64<0x111, 0xf>(x);
  x += dpp_u64<0x112, 0xf>(x);
  x += dpp_u64<0x114, 0xf>(x);
  x += dpp_u64<0x118, 0xf>(x);
  x += dpp_u64<0x142, 0xa>(x);
  x += dpp_u64<0x143, 0xc>(x);
  return x;
}
__device__ __forceinline__ unsigned long long lane63_u64(unsigned long long x) {
  return ((unsigned long long)lane63((uint32_t)(x >> 32)) << 32) | lane63((uint32_t)x);
}
__device__ __forceinline__ float wave_max(float v) {
  const uint32_t r = wave_scan_u32(__float_as_uint(v), 0xff800000u,  // -inf
                                   [](uint32_t a, uint32_t b) { return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b))); });
  return __uint_as_float(lane63(r));
}
__device__ __forceinline__ int wave_sum_i(int v) { return (int)lane63((uint32_t)wave_scan_sum_i(v)); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return lane63(wave_scan_u32(v, ~0u, [](uint32_t a, uint32_t b) { return min(a, b); }));
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  return lane63(wave_scan_u32(v, 0u, [](uint32_t a, uint32_t b) { return a | b; }));
}
__device__ __forceinline__ uint32_t wave_and_u32(uint32_t v) {
  return lane63(wave_scan_u32(v, ~0u, [](uint32_t a, uint32_t b) { return a & b; }));
}
// The value of lane ^ J (J a power of two below 64) without the LDS: DPP quad permutes for
// 1 and 2, row shifts by 4 either way (the lane's bit 2 picks the direction), a rotate by
// 8 within the 16-lane row, and the gfx950 row swaps (v_permlane16_swap,
// v_permlane32_swap) for 16 and 32. The same partner as __shfl_xor(v, J), so butterflies
// built on it add the same pairs in the same order. The lane bits come from threadIdx.x:
// every kernel of this library runs one-dimensional workgroups.
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t a) {
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  } else if constexpr (J == 4) {
    const uint32_t below = (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0x114, 0xF, 0xF, false);  // row_shr:4
    const uint32_t above = (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0x104, 0xF, 0xF, false);  // row_shl:4
    return (threadIdx.x & 4) ? below : above;
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, a, false, false);
    return (threadIdx.x & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
  } else {
    static_assert(J == 32, "xor_lane: J is 1, 2, 4, 8, 16 or 32");
    const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
    return (threadIdx.x & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
  }
}
template <int J>
__device__ __forceinline__ float xor_lane_f(float a) {
  return __uint_as_float(xor_lane<J>(__float_as_uint(a)));
}
// the SUM64 butterfly over 64 lane partials
__device__ __forceinline__ float sum64_tree(float v) {
  v = v + xor_lane_f<1>(v);
  v = v + xor_lane_f<2>(v);
  v = v + xor_lane_f<4>(v);
  v = v + xor_lane_f<8>(v);
  v = v + xor_lane_f<16>(v);
  v = v + xor_lane_f<32>(v);
  return v;
}
// the SUM8x tree over token lanes j = lane>>3 (lane bits 3..5); lane shuffles (the LDS
// unit) for the HBM-bound prep pass, whose VALU is the busier unit
__device__ __forceinline__ float sum8_tree(float v) {
  v = v + __shfl_xor(v, 8, 64);
  v = v + __shfl_xor(v, 16, 64);
  v = v + __shfl_xor(v, 32, 64);
  return v;
}

__host__ __device__ constexpr __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// S[bh][r][c] = DOT64(a[bh][r], b[bh][c]) * scale for r_begin <= r < r_end (of na rows per
// head), c < nb (rows of 64 fp32, 16-byte aligned) on the matrix cores, bit-exact with the
// fmaf chain (scores.hip). Returns 0 or the RESS_LAUNCHED code.
int scores_gemm(const float* a, const float* b, int BH, int na, int nb, int r_begin, int r_end, float scale,
                float* S, hipStream_t stream);
