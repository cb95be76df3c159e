// Block preparation: mean pooling, per-block INT8 quantisation of Q and K, and
// packing of V into the attention kernel's MFMA-ready layout.
//
// Replaces, for the block-sparse path:
//   * predict_attention's avg_pool1d of Q (128) and K (64), ceil mode, a partial
//     block divided by its valid count  (reference src/ress/models/attention.py:82-100)
//   * block_mean_value's pool of V (64)                     (attention.py:103-109)
//   * km = key.mean(dim=-2) and per_block_int8(q, k - km)   (attention.py:231-233,
//     SpargeAttn quant_per_block with external/patches/spargeattn.patch:38-41:
//     Q is quantised with sm_scale = 1)
//
// One wave (64 lanes) per (block, batch*head). Lane l owns dims 8*(l&7)..+7 of
// token lane j = l>>3; a block of T tokens is read in T/8 coalesced 1 KiB rows.
#include "common.h"

// hi (and, if lo_dst is set, split lo) codes of 8 values -> two 8-byte stores
// (quant_i8 / quant_i8_lo through the division-free quant_i8_rcp: identical codes)
__device__ __forceinline__ void store_codes(const float x[8], float scale, int8_t* hi_dst, int8_t* lo_dst) {
  int hi[8], lo[8];
  const float rc = scale != 0.0f ? 1.0f / scale : 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) hi[c] = quant_i8_rcp(x[c], scale, rc);
  *reinterpret_cast<uint2*>(hi_dst) = pack_i8x8(hi);
  if (lo_dst) {
    const float s2 = scale / 254.0f;
    const float rc2 = s2 != 0.0f ? 1.0f / s2 : 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) lo[c] = scale == 0.0f ? 0 : quant_i8_rcp(fmaf(-scale, (float)hi[c], x[c]), s2, rc2);
    *reinterpret_cast<uint2*>(lo_dst) = pack_i8x8(lo);
  }
}

// ----------------------------------------------------------------------------
// Q blocks: kernel q-blocks 0..q_blk_p-1 hold patch queries, q_blk_p.. the
// special queries. Writes q_i8 [BH][q_blk_total][128][64], q_scale [BH][q_blk_total]
// and, for patch blocks, pooled_q [BH][q_blk_p][64].
__device__ __forceinline__ void prep_q_block(int qb, int bh, const uint16_t* __restrict__ q, const Strides& sq,
                                             const TokenMap& m, int q_blk_p, int q_blk_total,
                                             int8_t* __restrict__ q_i8, int8_t* __restrict__ q_lo,
                                             float* __restrict__ q_scale, float* __restrict__ pooled_q) {
  const int lane = threadIdx.x;
  const int j = lane >> 3, dg = lane & 7;
  const bool special = qb >= q_blk_p;
  const int base = special ? (qb - q_blk_p) * 128 : qb * 128;
  const int cnt = min(128, (special ? m.T_s : m.T_p) - base);
  const uint16_t* src = q + bh_offset(bh, sq) + dg * 8;

  uint4 raw[16];
  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = 8 * i + j;
    raw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (t < cnt) {
      const int tok = special ? special_to_storage(base + t, m) : patch_to_storage(base + t, m);
      raw[i] = *reinterpret_cast<const uint4*>(src + (long long)tok * sq.t);
      float x[8];
      unpack_bf16x8(raw[i], x);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        acc[c] = acc[c] + x[c];
        amax = fmaxf(amax, fabsf(x[c]));
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = sum8_tree(acc[c]);
  if (!special && j == 0) {
    float* pq = pooled_q + ((long long)bh * q_blk_p + qb) * 64 + dg * 8;
#pragma unroll
    for (int c = 0; c < 8; ++c) pq[c] = acc[c] / (float)cnt;
  }
  if (!q_i8) return;  // pooling only (the bf16 attention operands read Q directly)
  amax = wave_max(amax);
  const float scale = amax / 127.0f;
  if (lane == 0) q_scale[(long long)bh * q_blk_total + qb] = scale;
  const long long off = (((long long)bh * q_blk_total + qb) * 128) * 64 + dg * 8;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float x[8];
    unpack_bf16x8(raw[i], x);
    const int r = (8 * i + j) * 64;
    store_codes(x, scale, q_i8 + off + r, q_lo ? q_lo + off + r : nullptr);
  }
}
__global__ __launch_bounds__(64) void k_prep_q(const uint16_t* __restrict__ q, Strides sq, TokenMap m,
                                               int q_blk_p, int q_blk_total, int8_t* __restrict__ q_i8,
                                               int8_t* __restrict__ q_lo, float* __restrict__ q_scale,
                                               float* __restrict__ pooled_q) {
  prep_q_block(blockIdx.x, blockIdx.y, q, sq, m, q_blk_p, q_blk_total, q_i8, q_lo, q_scale, pooled_q);
}

// ----------------------------------------------------------------------------
// K/V blocks over the kernel key grid (patch keys then special keys).
//  ksum   [BH][kb_tot][64]  full-block K sums (SUM8x), for the key mean (or null)
//  k_pack [BH][kb_tot][64 keys][64] fp16 row-major K blocks (or null); a bf16 value is
//         exact in fp16 unless below 2^-14 in magnitude (the subnormal range) or above 65504
//  k_norm [BH][kb_tot]  the block's largest key norm sqrt(sum_d k_d^2) (or null): per key
//         an fmaf chain over each lane's 8 dims, the tree of the 8 lanes, sqrtf; then the max
//  pooled_k [BH][kb_pool][64]  K means of the scoring grid: the patch keys only (kb_pool =
//                              kb_p), or every key in kernel order (kb_pool = kb_tot; the
//                              sink-mass map, attention.py:78, 451-452)
//  pooled_v [BH][kb_pool][64]  V means over the same grid (ReSS's v_bar)
//  v_pack [BH][kb_tot][64 dims][64 keys]  bf16, keys permuted inside every group of
//         16 as 0-3,8-11,4-7,12-15 so that one 16-byte read per lane is an MFMA
//         operand; keys past the sequence end are zero.
__device__ __forceinline__ void prep_kv_block(int kb, int bh, const uint16_t* __restrict__ k,
                                              const uint16_t* __restrict__ v, const Strides& sk, const Strides& sv,
                                              const TokenMap& m, int Tk, int kb_tot, int kb_p,
                                              float* __restrict__ ksum, float* __restrict__ pooled_k,
                                              float* __restrict__ pooled_v, uint16_t* __restrict__ v_pack,
                                              uint16_t* __restrict__ k_pack, float* __restrict__ k_norm,
                                              uint16_t* __restrict__ vt, int T_pool) {
  const int lane = threadIdx.x;
  const int j = lane >> 3, dg = lane & 7;
  const int base = kb * 64;
  const int cnt = min(64, Tk - base);
  const int cnt_p = min(64, T_pool - base);  // <= 0 past the pooled keys
  const uint16_t* ksrc = k + bh_offset(bh, sk) + dg * 8;
  const uint16_t* vsrc = v + bh_offset(bh, sv) + dg * 8;

  float ka[8], kp[8], vp[8];
  float nmax = 0.0f;  // largest key norm of this lane's keys (lane group j holds key t's 64 dims)
#pragma unroll
  for (int c = 0; c < 8; ++c) ka[c] = kp[c] = vp[c] = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int t = 8 * i + j;
    uint4 rv = make_uint4(0u, 0u, 0u, 0u), rk = rv, rk16 = rv;
    float ss = 0.0f;
    if (t < cnt) {
      const int tok = key_to_storage(base + t, m);
      rk = *reinterpret_cast<const uint4*>(ksrc + (long long)tok * sk.t);
      rv = *reinterpret_cast<const uint4*>(vsrc + (long long)tok * sv.t);
      float xk[8], xv[8];
      unpack_bf16x8(rk, xk);
      unpack_bf16x8(rv, xv);
      if (k_pack) {
        rk16.x = f32x2_to_f16_bits(xk[0], xk[1]);
        rk16.y = f32x2_to_f16_bits(xk[2], xk[3]);
        rk16.z = f32x2_to_f16_bits(xk[4], xk[5]);
        rk16.w = f32x2_to_f16_bits(xk[6], xk[7]);
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) ss = fmaf(xk[c], xk[c], ss);
      if (k_norm) {  // an element fp16 cannot hold (|x| >= 65520 rounds to inf): the key's norm is inf
        bool over = false;
#pragma unroll
        for (int c = 0; c < 8; ++c) over |= !(fabsf(xk[c]) < 65520.0f);
        if (over) ss = __builtin_huge_valf();
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) ka[c] = ka[c] + xk[c];
      if (t < cnt_p) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          kp[c] = kp[c] + xk[c];
          vp[c] = vp[c] + xv[c];
        }
      }
    }
    if (k_pack)  // row-major fp16 K block, zero past the sequence end
      *reinterpret_cast<uint4*>(k_pack + (((long long)bh * kb_tot + kb) * 64 + t) * 64 + dg * 8) = rk16;
    if (k_norm) {  // key t's squared norm: the tree of the 8 dim-group lanes of group j
      ss = ss + __shfl_xor(ss, 1, 64);
      ss = ss + __shfl_xor(ss, 2, 64);
      ss = ss + __shfl_xor(ss, 4, 64);
      nmax = fmaxf(nmax, sqrtf(ss));
    }
    // transpose into LDS: vt[dim][perm(key)]
    const int u = t & 15;
    const int pos = (t & ~15) + 8 * ((u >> 2) & 1) + 4 * (u >> 3) + (u & 3);
    const uint32_t w[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      vt[(dg * 8 + 2 * c) * 64 + pos] = (uint16_t)(w[c] & 0xffffu);
      vt[(dg * 8 + 2 * c + 1) * 64 + pos] = (uint16_t)(w[c] >> 16);
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    ka[c] = sum8_tree(ka[c]);
    kp[c] = sum8_tree(kp[c]);
    vp[c] = sum8_tree(vp[c]);
  }
  if (k_norm) {
    nmax = fmaxf(nmax, __shfl_xor(nmax, 8, 64));
    nmax = fmaxf(nmax, __shfl_xor(nmax, 16, 64));
    nmax = fmaxf(nmax, __shfl_xor(nmax, 32, 64));
    if (lane == 0) k_norm[(long long)bh * kb_tot + kb] = nmax;
  }
  if (j == 0) {
    if (ksum) {
      float* ks = ksum + ((long long)bh * kb_tot + kb) * 64 + dg * 8;
#pragma unroll
      for (int c = 0; c < 8; ++c) ks[c] = ka[c];
    }
    if (kb < kb_p) {
      float* pk = pooled_k + ((long long)bh * kb_p + kb) * 64 + dg * 8;
      float* pv = pooled_v + ((long long)bh * kb_p + kb) * 64 + dg * 8;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        pk[c] = kp[c] / (float)cnt_p;
        pv[c] = vp[c] / (float)cnt_p;
      }
    }
  }
  __syncthreads();
  // 8 KiB out, 128 B per lane
  uint4* dst = reinterpret_cast<uint4*>(v_pack + ((long long)bh * kb_tot + kb) * 4096);
  const uint4* s4 = reinterpret_cast<const uint4*>(vt);
#pragma unroll
  for (int i = 0; i < 8; ++i) dst[i * 64 + lane] = s4[i * 64 + lane];
}
__global__ __launch_bounds__(64) void k_prep_kv(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                Strides sk, Strides sv, TokenMap m, int Tk, int kb_tot, int kb_p,
                                                float* __restrict__ ksum, float* __restrict__ pooled_k,
                                                float* __restrict__ pooled_v, uint16_t* __restrict__ v_pack,
                                                uint16_t* __restrict__ k_pack, float* __restrict__ k_norm) {
  __shared__ uint16_t vt[64 * 64];
  prep_kv_block(blockIdx.x, blockIdx.y, k, v, sk, sv, m, Tk, kb_tot, kb_p, ksum, pooled_k, pooled_v, v_pack, k_pack,
                k_norm, vt, m.T_p);
}

// The layer's Q blocks and K/V blocks in one launch (they are independent): x < nqb is Q
// block x, the rest K/V block x - nqb. The K/V pools cover the first T_pool keys in kernel
// order (T_p: the patch keys; Tk: every key) in kb_pool blocks.
__global__ __launch_bounds__(64) void k_prep_qkv(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                 const uint16_t* __restrict__ v, Strides sq, Strides sk, Strides sv,
                                                 TokenMap m, int nqb, int q_blk_p, int q_blk_total, int Tk, int kb_tot,
                                                 int kb_p, int8_t* __restrict__ q_i8, int8_t* __restrict__ q_lo,
                                                 float* __restrict__ q_scale, float* __restrict__ pooled_q,
                                                 float* __restrict__ ksum, float* __restrict__ pooled_k,
                                                 float* __restrict__ pooled_v, uint16_t* __restrict__ v_pack,
                                                 uint16_t* __restrict__ k_pack, float* __restrict__ k_norm,
                                                 int T_pool) {
  __shared__ uint16_t vt[64 * 64];
  if ((int)blockIdx.x < nqb)
    prep_q_block(blockIdx.x, blockIdx.y, q, sq, m, q_blk_p, q_blk_total, q_i8, q_lo, q_scale, pooled_q);
  else
    prep_kv_block(blockIdx.x - nqb, blockIdx.y, k, v, sk, sv, m, Tk, kb_tot, kb_p, ksum, pooled_k, pooled_v, v_pack,
                  k_pack, k_norm, vt, T_pool);
}

// key mean over all Tk keys: km[d] = SEQ-sum of the block sums / Tk. The loads are
// issued 16 at a time so the serial add chain is not a chain of memory latencies.
__global__ __launch_bounds__(64) void k_key_mean(const float* __restrict__ ksum, int kb_tot, int Tk,
                                                 float* __restrict__ km) {
  const int bh = blockIdx.x, d = threadIdx.x;
  const float* s = ksum + (long long)bh * kb_tot * 64 + d;
  float acc = 0.0f;
  int b = 0;
  for (; b + 16 <= kb_tot; b += 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = s[(long long)(b + j) * 64];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc = acc + v[j];
  }
  for (; b < kb_tot; ++b) acc = acc + s[(long long)b * 64];
  km[(long long)bh * 64 + d] = acc / (float)Tk;
}

// K quantisation after smoothing: x = k - km (fp32), per 64-key block.
// k_i8 [BH][kb_tot][64 keys][64], k_scale [BH][kb_tot]. km may be null (no smoothing).
__global__ __launch_bounds__(64) void k_quant_k(const uint16_t* __restrict__ k, Strides sk, TokenMap m, int Tk,
                                                int kb_tot, const float* __restrict__ km, int8_t* __restrict__ k_i8,
                                                int8_t* __restrict__ k_lo, float* __restrict__ k_scale) {
  const int kb = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  const int j = lane >> 3, dg = lane & 7;
  const int base = kb * 64;
  const int cnt = min(64, Tk - base);
  const uint16_t* src = k + bh_offset(bh, sk) + dg * 8;
  float mean[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) mean[c] = km ? km[(long long)bh * 64 + dg * 8 + c] : 0.0f;
  float x[8][8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int t = 8 * i + j;
    uint4 r = make_uint4(0u, 0u, 0u, 0u);
    if (t < cnt) r = *reinterpret_cast<const uint4*>(src + (long long)key_to_storage(base + t, m) * sk.t);
    unpack_bf16x8(r, x[i]);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      x[i][c] = (t < cnt) ? x[i][c] - mean[c] : 0.0f;
      amax = fmaxf(amax, fabsf(x[i][c]));
    }
  }
  amax = wave_max(amax);
  const float scale = amax / 127.0f;
  if (lane == 0) k_scale[(long long)bh * kb_tot + kb] = scale;
  const long long off = ((long long)bh * kb_tot + kb) * 4096 + dg * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (8 * i + j) * 64;
    store_codes(x[i], scale, k_i8 + off + r, k_lo ? k_lo + off + r : nullptr);
  }
}

// ============================================================================
// C ABI
// ============================================================================
static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static TokenMap make_map(int frames, int P, int S, const int* perm = nullptr) {
  TokenMap m;
  m.P = P;
  m.S = S;
  m.HW = P - S;
  m.T_p = frames * (P - S);
  m.T_s = frames * S;
  m.perm = perm;
  return m;
}

// Fused preparation of one layer's Q/K/V for the ReSS forward (reference
// attention.py:398-491 + 226-233). Inputs are the backbone's bf16 Q/K/V in storage
// order with element strides (sB, sH, sT); D = 64 with unit stride.
//  * INT8 operands (q_i8 and k_i8 set): codes, scales, key mean; q_lo/k_lo (same
//    layouts as q_i8/k_i8) receive the split-INT8 residual codes, or are null.
//  * 16-bit operands (q_i8 and k_i8 null): the pools, v_pack, k_pack and, in k_scale,
//    each key block's largest key norm (k_norm of k_prep_kv) are written; q_lo,
//    q_scale, k_lo, ksum and km are unused (may be null).
// k_pack [BH][kb_tot][64 keys][64] fp16 (keys in kernel order, zero-padded) is
// written whenever it is non-null. patch_order: null, or HW = P-S int32 in device memory,
// the frame's patch tokens in the order blocks are formed (the Hilbert order of
// hilbert_permute), read in place; the same table must go to the attention call.
// pool_all: 0 pools K and V over the patch keys (kb_p blocks), 1 over every key in kernel
// order (kb_tot blocks: the sink-mass map of attention.py:78, 451-452 and its v_bar).
RESS_API int ress_prep_qkv(const void* q, const void* k, const void* v, int B, int H, int frames, int P, int S,
                           const int* patch_order, long long sqB, long long sqH, long long sqT, long long skB, long long skH, long long skT,
                           long long svB, long long svH, long long svT, void* q_i8, void* q_lo, void* q_scale,
                           void* pooled_q, void* k_i8, void* k_lo, void* k_scale, void* pooled_k, void* pooled_v,
                           void* v_pack, void* k_pack, void* ksum, void* km, int pool_all, hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && frames > 0 && P > S && S >= 0, "ress_prep_qkv: bad geometry B=%d H=%d F=%d P=%d S=%d",
               B, H, frames, P, S);
  RESS_REQUIRE(pool_all == 0 || pool_all == 1, "ress_prep_qkv: pool_all must be 0 or 1");
  RESS_REQUIRE(q && k && v && pooled_q && pooled_k && pooled_v && v_pack, "ress_prep_qkv: null pointer");
  const bool quant = q_i8 != nullptr;
  RESS_REQUIRE((q_i8 == nullptr) == (k_i8 == nullptr), "ress_prep_qkv: give both q_i8 and k_i8, or neither");
  RESS_REQUIRE(!quant || (q_scale && k_scale && ksum && km), "ress_prep_qkv: INT8 operands need q_scale, k_scale, ksum, km");
  RESS_REQUIRE(quant || (k_pack && k_scale), "ress_prep_qkv: 16-bit operands need k_pack and k_scale");
  RESS_REQUIRE(quant || (!q_lo && !k_lo), "ress_prep_qkv: q_lo/k_lo need the INT8 operands");
  RESS_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(v_pack) && aligned16(q_i8) && aligned16(k_i8) &&
                   aligned16(q_lo) && aligned16(k_lo) && aligned16(k_pack),
               "ress_prep_qkv: tensors must be 16-byte aligned");
  RESS_REQUIRE(sqT % 8 == 0 && skT % 8 == 0 && svT % 8 == 0 && sqH % 8 == 0 && skH % 8 == 0 && svH % 8 == 0 &&
                   sqB % 8 == 0 && skB % 8 == 0 && svB % 8 == 0,
               "ress_prep_qkv: strides must be multiples of 8 elements");
  TokenMap m = make_map(frames, P, S, patch_order);
  const int Tk = frames * P;
  const int BH = B * H;
  const int q_blk_p = cdiv(m.T_p, 128), q_blk_s = cdiv(m.T_s, 128);
  const int kb_tot = cdiv(Tk, 64), kb_p = cdiv(m.T_p, 64);
  Strides sq{sqB, sqH, sqT, H}, sk{skB, skH, skT, H}, sv{svB, svH, svT, H};
  // without codes only the patch blocks (the pooled ones) have Q work
  const int nqb = quant ? q_blk_p + q_blk_s : q_blk_p;
  hipLaunchKernelGGL(k_prep_qkv, dim3(nqb + kb_tot, BH), dim3(64), 0, stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, sq, sk, sv, m, nqb, q_blk_p, q_blk_p + q_blk_s, Tk, kb_tot,
                     pool_all ? kb_tot : kb_p,
                     (int8_t*)q_i8, (int8_t*)q_lo, (float*)q_scale, (float*)pooled_q,
                     (float*)(quant ? ksum : nullptr), (float*)pooled_k, (float*)pooled_v, (uint16_t*)v_pack,
                     (uint16_t*)k_pack, (float*)(quant ? nullptr : k_scale), pool_all ? Tk : m.T_p);
  RESS_LAUNCHED("k_prep_qkv");
  if (!quant) return 0;
  hipLaunchKernelGGL(k_key_mean, dim3(BH), dim3(64), 0, stream, (const float*)ksum, kb_tot, Tk, (float*)km);
  RESS_LAUNCHED("k_key_mean");
  hipLaunchKernelGGL(k_quant_k, dim3(kb_tot, BH), dim3(64), 0, stream, (const uint16_t*)k, sk, m, Tk, kb_tot,
                     (const float*)km, (int8_t*)k_i8, (int8_t*)k_lo, (float*)k_scale);
  RESS_LAUNCHED("k_quant_k");
  return 0;
}

// Mirror of SpargeAttn's per_block_int8(q, k) as the reference calls it
// (attention.py:232, with the patched Q scale of spargeattn.patch:38-41): plain
// sequences of Tq / Tk tokens, Q blocks of 128, K blocks of 64, optional key mean
// km [B*H][64] subtracted from K first (null = none). Outputs use the attention
// kernel's blocked layout: q_i8 [BH][ceil(Tq/128)][128][64],
// k_i8 [BH][ceil(Tk/64)][64][64], scales [BH][nblk].
RESS_API int ress_per_block_int8(const void* q, const void* k, const void* km, int B, int H, int Tq, int Tk,
                                 long long sqB, long long sqH, long long sqT, long long skB, long long skH,
                                 long long skT, void* q_i8, void* q_scale, void* k_i8, void* k_scale, void* pooled_q,
                                 hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && Tq > 0 && Tk > 0, "ress_per_block_int8: bad geometry");
  RESS_REQUIRE(q && k && q_i8 && q_scale && k_i8 && k_scale && pooled_q, "ress_per_block_int8: null pointer");
  RESS_REQUIRE(aligned16(q) && aligned16(k) && aligned16(q_i8) && aligned16(k_i8),
               "ress_per_block_int8: tensors must be 16-byte aligned");
  RESS_REQUIRE(sqT % 8 == 0 && skT % 8 == 0 && sqH % 8 == 0 && skH % 8 == 0 && sqB % 8 == 0 && skB % 8 == 0,
               "ress_per_block_int8: strides must be multiples of 8 elements");
  const int BH = B * H;
  TokenMap mq = make_map(1, Tq, 0), mk = make_map(1, Tk, 0);
  Strides sq{sqB, sqH, sqT, H}, sk{skB, skH, skT, H};
  const int nq = cdiv(Tq, 128), nk = cdiv(Tk, 64);
  hipLaunchKernelGGL(k_prep_q, dim3(nq, BH), dim3(64), 0, stream, (const uint16_t*)q, sq, mq, nq, nq, (int8_t*)q_i8,
                     (int8_t*)nullptr, (float*)q_scale, (float*)pooled_q);
  RESS_LAUNCHED("k_prep_q");
  hipLaunchKernelGGL(k_quant_k, dim3(nk, BH), dim3(64), 0, stream, (const uint16_t*)k, sk, mk, Tk, nk,
                     (const float*)km, (int8_t*)k_i8, (int8_t*)nullptr, (float*)k_scale);
  RESS_LAUNCHED("k_quant_k");
  return 0;
}

// Key mean of a plain (B,H,Tk,64) bf16 tensor (reference attention.py:231), via the
// same SUM8x block sums and SEQ block order as the fused path. ksum is workspace
// [BH][ceil(Tk/64)][64] fp32; the pooled/packed outputs of the block pass go to
// pooled_k [BH][ceil(Tk/64)][64], pooled_v (same) and v_pack [BH][ceil(Tk/64)][4096] bf16.
RESS_API int ress_prep_kv_plain(const void* k, const void* v, int B, int H, int Tk, long long skB, long long skH,
                                long long skT, long long svB, long long svH, long long svT, void* ksum, void* km,
                                void* pooled_k, void* pooled_v, void* v_pack, hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && Tk > 0, "ress_prep_kv_plain: bad geometry");
  RESS_REQUIRE(k && v && ksum && km && pooled_k && pooled_v && v_pack, "ress_prep_kv_plain: null pointer");
  RESS_REQUIRE(aligned16(k) && aligned16(v) && aligned16(v_pack), "ress_prep_kv_plain: tensors must be 16-byte aligned");
  RESS_REQUIRE(skT % 8 == 0 && svT % 8 == 0 && skH % 8 == 0 && svH % 8 == 0 && skB % 8 == 0 && svB % 8 == 0,
               "ress_prep_kv_plain: strides must be multiples of 8 elements");
  const int BH = B * H, nk = cdiv(Tk, 64);
  TokenMap mk = make_map(1, Tk, 0);
  Strides sk{skB, skH, skT, H}, sv{svB, svH, svT, H};
  hipLaunchKernelGGL(k_prep_kv, dim3(nk, BH), dim3(64), 0, stream, (const uint16_t*)k, (const uint16_t*)v, sk, sv, mk,
                     Tk, nk, nk, (float*)ksum, (float*)pooled_k, (float*)pooled_v, (uint16_t*)v_pack,
                     (uint16_t*)nullptr, (float*)nullptr);
  RESS_LAUNCHED("k_prep_kv");
  hipLaunchKernelGGL(k_key_mean, dim3(BH), dim3(64), 0, stream, (const float*)ksum, nk, Tk, (float*)km);
  RESS_LAUNCHED("k_key_mean");
  return 0;
}
