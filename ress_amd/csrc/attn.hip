// Block-sparse attention forward (INT8 QK^T, 16-bit PV) for gfx950.
//
// Replaces SpargeAttn's qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold
// as the reference calls it (src/ress/models/attention.py:238-241: HND layout, not
// causal, per-block Q/K scales, sm_scale = 1/sqrt(64), PV threshold disabled), and
// the special-query dense SDPA of attention.py:409 (special query blocks are rows
// whose LUT lists every key block).
//
//   O[q] = sum_k softmax_k( q_scale*k_scale*sm_scale * (Q8[q] . K8[k]) ) V[k]
//
// Work item = (batch*head, 128-query block); 256 threads = 4 waves of 32 queries.
// Per kept 64-key block:
//   S^T (64 keys x 32 queries) = K8 . Q8^T     4 x v_mfma_i32_32x32x32_i8
//   online softmax in the exp2 domain, scale folded into one fma per score
//   O^T (64 dims x 32 queries) += V^T . P^T    8 x v_mfma_f32_32x32x16_{bf16,f16}
// The S^T accumulator layout puts one query per lane, so P feeds the PV MFMA from
// registers; V is pre-packed (prep.hip) with keys permuted to match. K/V tiles are
// double-buffered in LDS. Work items are mapped XCD-major: hardware workgroup x runs
// on XCD x%8, and consecutive workgroups of one XCD walk the rows of one head so
// that head's K/V stay in that XCD's L2.
#include "common.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

struct AttnArgs {
  const int8_t* q_i8;      // [BH][q_blk_total][128][64]
  const int8_t* q_lo;      // split-INT8 residual codes (same layout) or null
  const int8_t* k_lo;      // split-INT8 residual codes [BH][kb_tot][64][64] or null
  const float* q_scale;    // [BH][q_blk_total]
  const int8_t* k_i8;      // [BH][kb_tot][64][64]
  const float* k_scale;    // [BH][kb_tot]
  const uint16_t* v_pack;  // [BH][kb_tot][64 dims][64 permuted keys]
  const int* lut;          // [BH][q_blk_total][kb_tot]
  const int* nvalid;       // [BH][q_blk_total]
  void* out;
  long long soB, soH, soT;
  int H, BH;
  int q_blk_p, q_blk_total, kb_tot, Tk;
  float sm_scale_log2e;
  TokenMap m;  // query rows: patch blocks via patch_to_storage, the rest via special_to_storage
};

enum { OUT_F32 = 0, OUT_BF16 = 1, OUT_F16 = 2 };

template <bool V_F16>
__device__ __forceinline__ v16f pv_mfma(const uint4& a, const uint4& b, v16f c) {
  if constexpr (V_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0,
                                                   0);
  }
}

template <bool V_F16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (V_F16) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
  } else {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
  }
}

// SPLIT: two-term INT8 Q and K (x ~ s*hi + s/254*lo). S = 254*(Qhi.Khi) + (Qhi.Klo + Qlo.Khi)
// in int32 (the lo.lo term, below 2^-16 relative, is dropped), 3 INT8 MFMAs per tile.
template <bool SPLIT, bool V_F16, int OUT>
__global__ __launch_bounds__(256, 2) void k_sparse_attn(AttnArgs a) {
  constexpr int KCH = SPLIT ? 512 : 256;  // 16-byte chunks of K per stage (hi [+ lo])
  constexpr int STAGE = KCH + 512;        // + V 8 KiB
  __shared__ __attribute__((aligned(16))) uint4 smem[2][STAGE];

  // ---- XCD-major work mapping -------------------------------------------
  const int x = blockIdx.x;
  const int xcd = x & 7, u = x >> 3;
  const int nh = (a.BH - xcd + 7) >> 3;  // heads whose rows this XCD runs
  const int q_blk_s = a.q_blk_total - a.q_blk_p;
  int bh, qb;
  if (u < nh * q_blk_s) {  // dense (special-query) rows first: they are the longest
    bh = xcd + 8 * (u / q_blk_s);
    qb = a.q_blk_p + u % q_blk_s;
  } else {
    const int v = u - nh * q_blk_s;
    const int hi = v / a.q_blk_p;
    if (hi >= nh) return;
    bh = xcd + 8 * hi;
    qb = v - hi * a.q_blk_p;
  }

  const long long row = (long long)bh * a.q_blk_total + qb;
  const int nv = a.nvalid[row];
  const int* lut = a.lut + row * a.kb_tot;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, qi = l & 31;

  const int8_t* qsrc = a.q_i8 + (row * 128 + 32 * w + qi) * 64 + 16 * g;
  const v4i qa0 = *reinterpret_cast<const v4i*>(qsrc);
  const v4i qa1 = *reinterpret_cast<const v4i*>(qsrc + 32);
  v4i ql0, ql1;
  if constexpr (SPLIT) {
    const int8_t* qlsrc = a.q_lo + (row * 128 + 32 * w + qi) * 64 + 16 * g;
    ql0 = *reinterpret_cast<const v4i*>(qlsrc);
    ql1 = *reinterpret_cast<const v4i*>(qlsrc + 32);
  }
  const float qs = a.q_scale[row] * a.sm_scale_log2e * (SPLIT ? (1.0f / 254.0f) : 1.0f);
  const float* ksc = a.k_scale + (long long)bh * a.kb_tot;
  const uint4* kbase_p = reinterpret_cast<const uint4*>(a.k_i8 + (long long)bh * a.kb_tot * 4096);
  const uint4* klbase_p = SPLIT ? reinterpret_cast<const uint4*>(a.k_lo + (long long)bh * a.kb_tot * 4096) : nullptr;
  const uint4* vbase_p = reinterpret_cast<const uint4*>(a.v_pack + (long long)bh * a.kb_tot * 4096);

  float m_run = -__builtin_huge_valf(), l_run = 0.0f;
  v16f o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.0f;

  uint4 r0, r1, r2, r3;
  if (nv > 0) {
    const int kb = lut[0];
    r0 = kbase_p[(long long)kb * 256 + tid];
    if constexpr (SPLIT) r3 = klbase_p[(long long)kb * 256 + tid];
    r1 = vbase_p[(long long)kb * 512 + tid];
    r2 = vbase_p[(long long)kb * 512 + 256 + tid];
    smem[0][tid] = r0;
    if constexpr (SPLIT) smem[0][256 + tid] = r3;
    smem[0][KCH + tid] = r1;
    smem[0][KCH + 256 + tid] = r2;
  }
  __syncthreads();

  for (int it = 0; it < nv; ++it) {
    const int buf = it & 1;
    const int kb = lut[it];
    const bool more = it + 1 < nv;
    if (more) {
      const int kn = lut[it + 1];
      r0 = kbase_p[(long long)kn * 256 + tid];
      if constexpr (SPLIT) r3 = klbase_p[(long long)kn * 256 + tid];
      r1 = vbase_p[(long long)kn * 512 + tid];
      r2 = vbase_p[(long long)kn * 512 + 256 + tid];
    }
    const int8_t* sk = reinterpret_cast<const int8_t*>(&smem[buf][0]);
    const int8_t* skl = sk + 4096;
    const uint16_t* sv = reinterpret_cast<const uint16_t*>(&smem[buf][KCH]);

    // ---- S^T = K . Q^T --------------------------------------------------
    v16i s0, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0;
    {
      const v4i k00 = *reinterpret_cast<const v4i*>(sk + qi * 64 + 16 * g);
      const v4i k01 = *reinterpret_cast<const v4i*>(sk + qi * 64 + 32 + 16 * g);
      const v4i k10 = *reinterpret_cast<const v4i*>(sk + (32 + qi) * 64 + 16 * g);
      const v4i k11 = *reinterpret_cast<const v4i*>(sk + (32 + qi) * 64 + 32 + 16 * g);
      s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k00, qa0, s0, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k01, qa1, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k10, qa0, s1, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k11, qa1, s1, 0, 0, 0);
      if constexpr (SPLIT) {
        v16i b0, b1;
#pragma unroll
        for (int r = 0; r < 16; ++r) b0[r] = b1[r] = 0;
        const v4i l00 = *reinterpret_cast<const v4i*>(skl + qi * 64 + 16 * g);
        const v4i l01 = *reinterpret_cast<const v4i*>(skl + qi * 64 + 32 + 16 * g);
        const v4i l10 = *reinterpret_cast<const v4i*>(skl + (32 + qi) * 64 + 16 * g);
        const v4i l11 = *reinterpret_cast<const v4i*>(skl + (32 + qi) * 64 + 32 + 16 * g);
        b0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k00, ql0, b0, 0, 0, 0);
        b0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k01, ql1, b0, 0, 0, 0);
        b0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(l00, qa0, b0, 0, 0, 0);
        b0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(l01, qa1, b0, 0, 0, 0);
        b1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k10, ql0, b1, 0, 0, 0);
        b1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k11, ql1, b1, 0, 0, 0);
        b1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(l10, qa0, b1, 0, 0, 0);
        b1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(l11, qa1, b1, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s0[r] = s0[r] * 254 + b0[r];
          s1[r] = s1[r] * 254 + b1[r];
        }
      }
    }

    // ---- online softmax (exp2 domain) -----------------------------------
    // lane holds query qi; register r of tile t is key 32t + 8(r/4) + 4g + r%4
    const float c = qs * ksc[kb];
    const int key0 = kb * 64;
    const int nk = min(64, a.Tk - key0);
    int imax = -2147483647 - 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = 8 * (r >> 2) + 4 * g + (r & 3);
      if (kr < nk) imax = max(imax, s0[r]);
      if (kr + 32 < nk) imax = max(imax, s1[r]);
    }
    imax = max(imax, __shfl_xor(imax, 32, 64));
    const float m_new = fmaxf(m_run, (float)imax * c);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float p0[16], p1[16];
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = 8 * (r >> 2) + 4 * g + (r & 3);
      p0[r] = kr < nk ? __builtin_amdgcn_exp2f(fmaf((float)s0[r], c, -m_new)) : 0.0f;
      p1[r] = kr + 32 < nk ? __builtin_amdgcn_exp2f(fmaf((float)s1[r], c, -m_new)) : 0.0f;
      psum += p0[r] + p1[r];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o0[r] *= alpha;
      o1[r] *= alpha;
    }

    // ---- O^T += V^T . P^T -----------------------------------------------
    // MFMA s covers keys 16s..16s+15: tile s/2, registers 8(s%2)..+7
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float* ps = (s < 2) ? p0 : p1;
      const int rb = 8 * (s & 1);
      uint4 pb;
      pb.x = pack2<V_F16>(ps[rb + 0], ps[rb + 1]);
      pb.y = pack2<V_F16>(ps[rb + 2], ps[rb + 3]);
      pb.z = pack2<V_F16>(ps[rb + 4], ps[rb + 5]);
      pb.w = pack2<V_F16>(ps[rb + 6], ps[rb + 7]);
      const uint4 va0 = *reinterpret_cast<const uint4*>(sv + qi * 64 + 16 * s + 8 * g);
      const uint4 va1 = *reinterpret_cast<const uint4*>(sv + (32 + qi) * 64 + 16 * s + 8 * g);
      o0 = pv_mfma<V_F16>(va0, pb, o0);
      o1 = pv_mfma<V_F16>(va1, pb, o1);
    }

    if (more) {
      smem[buf ^ 1][tid] = r0;
      if constexpr (SPLIT) smem[buf ^ 1][256 + tid] = r3;
      smem[buf ^ 1][KCH + tid] = r1;
      smem[buf ^ 1][KCH + 256 + tid] = r2;
    }
    __syncthreads();
  }

  // ---- epilogue ------------------------------------------------------------
  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = (nv > 0 && lt > 0.0f) ? 1.0f / lt : 0.0f;
  const bool special = qb >= a.q_blk_p;
  const int qbase = special ? (qb - a.q_blk_p) * 128 : qb * 128;
  const int cnt_q = min(128, (special ? a.m.T_s : a.m.T_p) - qbase);
  const int qrow = 32 * w + qi;
  if (qrow >= cnt_q) return;
  const int tok = special ? special_to_storage(qbase + qrow, a.m) : patch_to_storage(qbase + qrow, a.m);
  const long long off = (long long)(bh / a.H) * a.soB + (long long)(bh % a.H) * a.soH + (long long)tok * a.soT;
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const v16f& o = n ? o1 : o0;
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      const int d0 = 32 * n + 8 * a4 + 4 * g;
      const float y0 = o[4 * a4 + 0] * inv, y1 = o[4 * a4 + 1] * inv;
      const float y2 = o[4 * a4 + 2] * inv, y3 = o[4 * a4 + 3] * inv;
      if constexpr (OUT == OUT_F32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + off + d0) = make_float4(y0, y1, y2, y3);
      } else {
        constexpr bool F16 = OUT == OUT_F16;
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + off + d0) =
            make_uint2(pack2<F16>(y0, y1), pack2<F16>(y2, y3));
      }
    }
  }
}

// Plain (B,H,Tk,64) 16-bit V -> packed [BH][kb][64 dims][64 permuted keys].
__global__ __launch_bounds__(64) void k_pack_v(const uint16_t* __restrict__ v, long long svB, long long svH,
                                               long long svT, int H, int Tk, int kb_tot, uint16_t* __restrict__ v_pack) {
  __shared__ uint16_t vt[64 * 64];
  const int kb = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  const int j = lane >> 3, dg = lane & 7;
  const uint16_t* src = v + (long long)(bh / H) * svB + (long long)(bh % H) * svH + dg * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int t = 8 * i + j;
    uint4 rv = make_uint4(0u, 0u, 0u, 0u);
    if (kb * 64 + t < Tk) rv = *reinterpret_cast<const uint4*>(src + (long long)(kb * 64 + t) * svT);
    const int uu = t & 15;
    const int pos = (t & ~15) + 8 * ((uu >> 2) & 1) + 4 * (uu >> 3) + (uu & 3);
    const uint32_t wv[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      vt[(dg * 8 + 2 * c) * 64 + pos] = (uint16_t)(wv[c] & 0xffffu);
      vt[(dg * 8 + 2 * c + 1) * 64 + pos] = (uint16_t)(wv[c] >> 16);
    }
  }
  __syncthreads();
  uint4* dst = reinterpret_cast<uint4*>(v_pack + ((long long)bh * kb_tot + kb) * 4096);
  const uint4* s4 = reinterpret_cast<const uint4*>(vt);
#pragma unroll
  for (int i = 0; i < 8; ++i) dst[i * 64 + lane] = s4[i * 64 + lane];
}

// ============================================================================
// C ABI
// ============================================================================
template <bool SPLIT, bool V_F16>
static int launch_attn(const AttnArgs& a, int out_dtype, hipStream_t stream) {
  const int per_xcd = ((a.BH + 7) / 8) * a.q_blk_total;
  const dim3 grid(8 * per_xcd), block(256);
  switch (out_dtype) {
    case OUT_F32: hipLaunchKernelGGL((k_sparse_attn<SPLIT, V_F16, OUT_F32>), grid, block, 0, stream, a); break;
    case OUT_BF16: hipLaunchKernelGGL((k_sparse_attn<SPLIT, V_F16, OUT_BF16>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((k_sparse_attn<SPLIT, V_F16, OUT_F16>), grid, block, 0, stream, a); break;
  }
  RESS_LAUNCHED("k_sparse_attn");
  return 0;
}

static int attn_common(const void* q_i8, const void* q_lo, const void* q_scale, const void* k_i8, const void* k_lo,
                       const void* k_scale, const void* v_pack, int v_f16, const void* lut, const void* nvalid, int B,
                       int H, TokenMap m, int Tk, float sm_scale, void* out, int out_dtype, long long soB,
                       long long soH, long long soT, hipStream_t stream) {
  RESS_REQUIRE(q_i8 && q_scale && k_i8 && k_scale && v_pack && lut && nvalid && out, "sparse attention: null pointer");
  RESS_REQUIRE((q_lo == nullptr) == (k_lo == nullptr), "sparse attention: give both q_lo and k_lo, or neither");
  RESS_REQUIRE(((uintptr_t)q_i8 & 15u) == 0 && ((uintptr_t)k_i8 & 15u) == 0 && ((uintptr_t)v_pack & 15u) == 0 &&
                   ((uintptr_t)q_lo & 15u) == 0 && ((uintptr_t)k_lo & 15u) == 0,
               "sparse attention: q_i8/q_lo/k_i8/k_lo/v_pack must be 16-byte aligned");
  RESS_REQUIRE(out_dtype >= 0 && out_dtype <= 2, "sparse attention: out_dtype must be 0 (f32), 1 (bf16) or 2 (f16)");
  const int align = out_dtype == OUT_F32 ? 16 : 8;
  RESS_REQUIRE(((uintptr_t)out % align) == 0 && soT % 4 == 0 && soH % 4 == 0 && soB % 4 == 0,
               "sparse attention: output must be %d-byte aligned with strides a multiple of 4", align);
  AttnArgs a;
  a.q_i8 = (const int8_t*)q_i8;
  a.q_lo = (const int8_t*)q_lo;
  a.k_lo = (const int8_t*)k_lo;
  a.q_scale = (const float*)q_scale;
  a.k_i8 = (const int8_t*)k_i8;
  a.k_scale = (const float*)k_scale;
  a.v_pack = (const uint16_t*)v_pack;
  a.lut = (const int*)lut;
  a.nvalid = (const int*)nvalid;
  a.out = out;
  a.soB = soB;
  a.soH = soH;
  a.soT = soT;
  a.H = H;
  a.BH = B * H;
  a.q_blk_p = cdiv(m.T_p, 128);
  a.q_blk_total = a.q_blk_p + cdiv(m.T_s, 128);
  a.kb_tot = cdiv(Tk, 64);
  a.Tk = Tk;
  a.sm_scale_log2e = sm_scale * 1.4426950408889634f;
  a.m = m;
  if (q_lo) return v_f16 ? launch_attn<true, true>(a, out_dtype, stream) : launch_attn<true, false>(a, out_dtype, stream);
  return v_f16 ? launch_attn<false, true>(a, out_dtype, stream) : launch_attn<false, false>(a, out_dtype, stream);
}

// Fused-path attention over the ReSS token split: queries are the patch tokens
// (q-blocks 0..ceil(T_p/128)-1, sparse LUT rows) then the special tokens (dense
// rows); keys are cat(patch, special). The output is written in storage order
// (B,H,frames*P,64) with element strides soB/soH/soT, i.e. the reference's
// combine_special_and_patch (src/ress/models/qkv.py:71-81) is fused in. With q_lo/k_lo
// (split-INT8 residual codes from ress_prep_qkv) QK^T is evaluated as a two-term INT8
// product; without them it is the single-term per-block INT8 product of the reference.
RESS_API int ress_sparse_attn_fwd(const void* q_i8, const void* q_lo, const void* q_scale, const void* k_i8,
                                  const void* k_lo, const void* k_scale, const void* v_pack, int v_f16, const void* lut,
                                  const void* nvalid, int B, int H, int frames, int P, int S, float sm_scale, void* out,
                                  int out_dtype, long long soB, long long soH, long long soT, hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && frames > 0 && P > S && S >= 0, "ress_sparse_attn_fwd: bad geometry");
  TokenMap m;
  m.P = P;
  m.S = S;
  m.HW = P - S;
  m.T_p = frames * (P - S);
  m.T_s = frames * S;
  return attn_common(q_i8, q_lo, q_scale, k_i8, k_lo, k_scale, v_pack, v_f16, lut, nvalid, B, H, m, frames * P,
                     sm_scale, out, out_dtype, soB, soH, soT, stream);
}

RESS_API long long ress_qattn_workspace_size(int B, int H, int Tk) {
  return (long long)B * H * cdiv(Tk, 64) * 4096 * 2;
}

// Mirror of SpargeAttn's qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold
// (call site reference src/ress/models/attention.py:238-241). q_i8 (B,H,Tq,64) and
// k_i8 (B,H,Tk,64) int8 contiguous with rows allocated up to the next multiple of
// 128 / 64 (the blocked layout ress_per_block_int8 writes); v (B,H,Tk,64) fp16
// (v_f16=1) or bf16 with strides; lut/valid_block_num [B*H][ceil(Tq/128)][ceil(Tk/64)];
// q_scale [B*H][ceil(Tq/128)], k_scale [B*H][ceil(Tk/64)]; o (B,H,Tq,64) with strides.
// Supported: tensor_layout 1 (HND), is_causal 0, qk_quant_gran 1 (per block),
// return_pv_count 0, pv_threshold disabled (>= 1e9, the reference passes 1e10).
// workspace: ress_qattn_workspace_size(B,H,Tk) bytes for the packed V.
RESS_API int ress_qattn_block_sparse_fwd(const void* q_i8, const void* k_i8, const void* v, int v_f16, void* o,
                                         int o_dtype, const void* lut, const void* valid_block_num,
                                         const float* pv_threshold_host, const void* q_scale, const void* k_scale,
                                         int B, int H, int Tq, int Tk, long long svB, long long svH, long long svT,
                                         long long soB, long long soH, long long soT, int tensor_layout, int is_causal,
                                         int qk_quant_gran, float sm_scale, int return_pv_count, void* workspace,
                                         long long workspace_bytes, hipStream_t stream) {
  RESS_REQUIRE(tensor_layout == 1, "ress_qattn_block_sparse_fwd: only tensor_layout=1 (HND) is supported");
  RESS_REQUIRE(is_causal == 0, "ress_qattn_block_sparse_fwd: is_causal must be 0");
  RESS_REQUIRE(qk_quant_gran == 1, "ress_qattn_block_sparse_fwd: only per-block quantisation (qk_quant_gran=1)");
  RESS_REQUIRE(return_pv_count == 0, "ress_qattn_block_sparse_fwd: return_pv_count must be 0");
  if (pv_threshold_host)
    for (int h = 0; h < H; ++h)
      RESS_REQUIRE(pv_threshold_host[h] >= 1e9f,
                   "ress_qattn_block_sparse_fwd: PV-threshold skipping is not implemented (got %g; the reference "
                   "passes 1e10 = disabled)",
                   (double)pv_threshold_host[h]);
  RESS_REQUIRE(B > 0 && H > 0 && Tq > 0 && Tk > 0, "ress_qattn_block_sparse_fwd: bad geometry");
  RESS_REQUIRE(v && workspace && workspace_bytes >= ress_qattn_workspace_size(B, H, Tk),
               "ress_qattn_block_sparse_fwd: workspace of %lld bytes required", ress_qattn_workspace_size(B, H, Tk));
  RESS_REQUIRE(((uintptr_t)v & 15u) == 0 && svT % 8 == 0 && svH % 8 == 0 && svB % 8 == 0,
               "ress_qattn_block_sparse_fwd: v must be 16-byte aligned with strides a multiple of 8");
  const int kb_tot = cdiv(Tk, 64);
  hipLaunchKernelGGL(k_pack_v, dim3(kb_tot, B * H), dim3(64), 0, stream, (const uint16_t*)v, svB, svH, svT, H, Tk,
                     kb_tot, (uint16_t*)workspace);
  RESS_LAUNCHED("k_pack_v");
  TokenMap m;
  m.P = Tq;
  m.S = 0;
  m.HW = Tq;
  m.T_p = Tq;
  m.T_s = 0;
  return attn_common(q_i8, nullptr, q_scale, k_i8, nullptr, k_scale, workspace, v_f16, lut, valid_block_num, B, H, m,
                     Tk, sm_scale, o, o_dtype, soB, soH, soT, stream);
}
