/* CPU oracle for the ReSS / HeSS block-sparse global-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C on host arrays, the
 * reference algorithm (libary753/ReSS) for every stage the GPU library implements,
 * under the same numerics contract (fixed evaluation orders, IEEE division, no
 * contraction: build with -ffp-contract=off):
 *   SUM8x  block pooling: per token lane j = t mod 8 a sequential sum over its
 *          tokens, then ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7))
 *   SUM64  row sums: 64 strided sequential partials, then an xor butterfly
 *   DOT64  sequential fmaf over the 64 dims
 *   SEQ    sequential sums in index order
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it, and
 * only as the checker. The product library never links or calls it.
 *
 * Tensors are contiguous row-major. bf16 values are passed as uint16_t bit patterns.
 * Rows (heads, query blocks) are independent; the loops over them run under OpenMP, which
 * changes no row's arithmetic.
 */
#define _GNU_SOURCE /* qsort_r */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf16f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t fbits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bitsf(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline int cdiv(int a, int b) { return (a + b - 1) / b; }

/* ---- exp: Cody-Waite reduction, degree-7 Taylor polynomial (Horner) ---------- */
float oracle_expf(float x) {
  if (x != x) return x;
  if (x > 0x1.62e42ep+6f) return INFINITY;
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
  if (ni < -126) return (p * bitsf((uint32_t)(ni + 127 + 64) << 23)) * 0x1p-64f;
  return p * bitsf((uint32_t)(ni + 127) << 23);
}

/* ---- bf16 rounding (round to nearest even) ------------------------------------ */
float oracle_round_bf16(float f) {
  uint32_t u = fbits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bitsf(((u >> 16) | 0x40u) << 16);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bitsf((u >> 16) << 16);
}

/* ---- order key ------------------------------------------------------------------ */
static inline uint32_t order_key(float x) {
  uint32_t u = fbits(x);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* ---- geometry: storage order <-> kernel order ------------------------------------ */
typedef struct {
  int P, S, HW, T_p, T_s;
} tokmap;
static tokmap mkmap(int frames, int P, int S) {
  tokmap m = {P, S, P - S, frames * (P - S), frames * S};
  return m;
}
static inline int patch_st(int p, const tokmap* m) { return (p / m->HW) * m->P + m->S + p % m->HW; }
static inline int special_st(int s, const tokmap* m) { return (s / m->S) * m->P + s % m->S; }
static inline int key_st(int kk, const tokmap* m) { return kk < m->T_p ? patch_st(kk, m) : special_st(kk - m->T_p, m); }

/* SUM8x over the rows[] (count cnt) of a (tokens, 64) bf16 matrix, for one dim d */
static float sum8x(const uint16_t* x, const int* rows, int cnt, int d) {
  float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int t = 0; t < cnt; ++t) p[t & 7] = p[t & 7] + bf16f(x[(long long)rows[t] * 64 + d]);
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

/* per-block quantiser: SageAttention quant_per_block (scale = amax/127, round half
 * away from zero), Q with sm_scale = 1 (external/patches/spargeattn.patch:38-41) */
static inline int8_t quant(float x, float scale) {
  if (scale == 0.0f) return 0;
  float y = x / scale;
  y = y + (y >= 0.0f ? 0.5f : -0.5f);
  return (int8_t)(int)y;
}
/* split-INT8 residual code: x ~ scale*hi + (scale/254)*lo, residual fmaf(-scale, hi, x) */
static inline int8_t quant_lo(float x, float scale, int8_t hi) {
  if (scale == 0.0f) return 0;
  return quant(fmaf(-scale, (float)hi, x), scale / 254.0f);
}

/* ---- preparation ------------------------------------------------------------------
 * Follows src/ress/models/qkv.py:60-68 + tokens.py:8-52 (patch/special split, kernel
 * key order cat(patch, special), attention.py:405-406), predict_attention's avg pools
 * (attention.py:90-96; ceil mode, a partial block divided by its valid count),
 * block_mean_value (attention.py:103-109), km = key.mean(-2) and
 * per_block_int8(q, k - km) (attention.py:231-233), all in fp32; k_norm[BH][kb_tot] the
 * 16-bit attention's per-block largest key norm: per key an fmaf chain over each group
 * of 8 dims, the tree ((g0+g1)+(g2+g3))+((g4+g5)+(g6+g7)), sqrtf; the max over the block.
 * q,k,v: (BH, frames*P, 64) bf16. Output layouts as ress_prep_qkv (include/ress_hip.h). */
void oracle_prep_qkv(const uint16_t* q, const uint16_t* k, const uint16_t* v, int BH, int frames, int P, int S,
                     int8_t* q_i8, int8_t* q_lo, float* q_scale, float* pooled_q, int8_t* k_i8, int8_t* k_lo,
                     float* k_scale, float* pooled_k, float* pooled_v, uint16_t* v_pack, float* ksum, float* km,
                     float* k_norm, int pool_all) {
  tokmap m = mkmap(frames, P, S);
  const int N = frames * P, Tk = N;
  const int qbp = cdiv(m.T_p, 128), qbs = cdiv(m.T_s, 128), qbt = qbp + qbs;
  const int kbt = cdiv(Tk, 64);
  /* the pooled grid: the patch keys, or every key in kernel order (pool_all) */
  const int T_pool = pool_all ? Tk : m.T_p, kbp = cdiv(T_pool, 64);
#pragma omp parallel for schedule(dynamic, 1)
  for (int bh = 0; bh < BH; ++bh) {
    int rows[128];
    const uint16_t* qh = q + (long long)bh * N * 64;
    const uint16_t* kh = k + (long long)bh * N * 64;
    const uint16_t* vh = v + (long long)bh * N * 64;
    /* Q blocks */
    for (int qb = 0; qb < qbt; ++qb) {
      const int special = qb >= qbp;
      const int base = special ? (qb - qbp) * 128 : qb * 128;
      const int cnt = (special ? m.T_s : m.T_p) - base < 128 ? (special ? m.T_s : m.T_p) - base : 128;
      for (int t = 0; t < cnt; ++t) rows[t] = special ? special_st(base + t, &m) : patch_st(base + t, &m);
      float amax = 0.0f;
      for (int t = 0; t < cnt; ++t)
        for (int d = 0; d < 64; ++d) amax = fmaxf(amax, fabsf(bf16f(qh[(long long)rows[t] * 64 + d])));
      const float scale = amax / 127.0f;
      q_scale[(long long)bh * qbt + qb] = scale;
      if (!special)
        for (int d = 0; d < 64; ++d)
          pooled_q[((long long)bh * qbp + qb) * 64 + d] = sum8x(qh, rows, cnt, d) / (float)cnt;
      int8_t* dst = q_i8 + ((long long)bh * qbt + qb) * 128 * 64;
      int8_t* dlo = q_lo + ((long long)bh * qbt + qb) * 128 * 64;
      for (int t = 0; t < 128; ++t)
        for (int d = 0; d < 64; ++d) {
          const float x = t < cnt ? bf16f(qh[(long long)rows[t] * 64 + d]) : 0.0f;
          dst[t * 64 + d] = quant(x, scale);
          dlo[t * 64 + d] = quant_lo(x, scale, dst[t * 64 + d]);
        }
    }
    /* K/V blocks over the kernel key grid */
    for (int kb = 0; kb < kbt; ++kb) {
      const int base = kb * 64;
      const int cnt = Tk - base < 64 ? Tk - base : 64;
      int cnt_p = T_pool - base < 64 ? T_pool - base : 64;
      if (cnt_p < 0) cnt_p = 0;
      for (int t = 0; t < cnt; ++t) rows[t] = key_st(base + t, &m);
      for (int d = 0; d < 64; ++d) {
        ksum[((long long)bh * kbt + kb) * 64 + d] = sum8x(kh, rows, cnt, d);
        if (kb < kbp) {
          pooled_k[((long long)bh * kbp + kb) * 64 + d] = sum8x(kh, rows, cnt_p, d) / (float)cnt_p;
          pooled_v[((long long)bh * kbp + kb) * 64 + d] = sum8x(vh, rows, cnt_p, d) / (float)cnt_p;
        }
      }
      float nmax = 0.0f;
      for (int t = 0; t < cnt; ++t) {
        float g8[8];
        int over = 0;  // an element fp16 cannot hold (|x| >= 65520 rounds to inf): the norm is inf
        for (int grp = 0; grp < 8; ++grp) {
          float ss = 0.0f;
          for (int c = 0; c < 8; ++c) {
            const float x = bf16f(kh[(long long)rows[t] * 64 + 8 * grp + c]);
            ss = fmaf(x, x, ss);
            over |= !(fabsf(x) < 65520.0f);
          }
          g8[grp] = ss;
        }
        const float n = over ? INFINITY
                             : sqrtf(((g8[0] + g8[1]) + (g8[2] + g8[3])) + ((g8[4] + g8[5]) + (g8[6] + g8[7])));
        nmax = fmaxf(nmax, n);
      }
      k_norm[(long long)bh * kbt + kb] = nmax;
      uint16_t* vp = v_pack + ((long long)bh * kbt + kb) * 4096;
      for (int t = 0; t < 64; ++t) {
        const int u = t & 15;
        const int pos = (t & ~15) + 8 * ((u >> 2) & 1) + 4 * (u >> 3) + (u & 3);
        for (int d = 0; d < 64; ++d) vp[d * 64 + pos] = t < cnt ? vh[(long long)rows[t] * 64 + d] : 0;
      }
    }
    /* key mean: SEQ over block sums / Tk */
    for (int d = 0; d < 64; ++d) {
      float acc = 0.0f;
      for (int kb = 0; kb < kbt; ++kb) acc = acc + ksum[((long long)bh * kbt + kb) * 64 + d];
      km[(long long)bh * 64 + d] = acc / (float)Tk;
    }
    /* K quantisation of k - km */
    for (int kb = 0; kb < kbt; ++kb) {
      const int base = kb * 64;
      const int cnt = Tk - base < 64 ? Tk - base : 64;
      float amax = 0.0f;
      for (int t = 0; t < cnt; ++t) {
        const int r = key_st(base + t, &m);
        for (int d = 0; d < 64; ++d)
          amax = fmaxf(amax, fabsf(bf16f(kh[(long long)r * 64 + d]) - km[(long long)bh * 64 + d]));
      }
      const float scale = amax / 127.0f;
      k_scale[(long long)bh * kbt + kb] = scale;
      int8_t* dst = k_i8 + ((long long)bh * kbt + kb) * 4096;
      int8_t* dlo = k_lo + ((long long)bh * kbt + kb) * 4096;
      for (int t = 0; t < 64; ++t) {
        const int r = t < cnt ? key_st(base + t, &m) : 0;
        for (int d = 0; d < 64; ++d) {
          const float x = t < cnt ? bf16f(kh[(long long)r * 64 + d]) - km[(long long)bh * 64 + d] : 0.0f;
          dst[t * 64 + d] = quant(x, scale);
          dlo[t * 64 + d] = quant_lo(x, scale, dst[t * 64 + d]);
        }
      }
    }
  }
}

/* ---- pooled map -----------------------------------------------------------------------
 * predict_attention's pooled GEMM + softmax (src/ress/models/attention.py:98-100) and
 * attn_cond = attn_pooled / clamp(rowsum(attn_pooled), 1e-6) (attention.py:457,473). */
static float sum64(const float* x, int n) {
  float part[64];
  for (int l = 0; l < 64; ++l) {
    float a = 0.0f;
    for (int i = l; i < n; i += 64) a = a + x[i];
    part[l] = a;
  }
  for (int off = 1; off < 64; off <<= 1) {
    float nx[64];
    for (int l = 0; l < 64; ++l) nx[l] = part[l] + part[l ^ off];
    memcpy(part, nx, sizeof(part));
  }
  return part[0];
}

void oracle_pooled_scores(const float* pooled_q, const float* pooled_k, int BH, int q_blk, int kb_p, int n_cand,
                          float scale, float* attn_full, float* attn_cond) {
#pragma omp parallel
  {
  float* s = (float*)malloc(sizeof(float) * (kb_p > 0 ? kb_p : 1));
#pragma omp for schedule(dynamic, 4)
  for (long long row = 0; row < (long long)BH * q_blk; ++row) {
      const int bh = (int)(row / q_blk), qb = (int)(row % q_blk);
      const float* pq = pooled_q + ((long long)bh * q_blk + qb) * 64;
      float m = -INFINITY;
      for (int kb = 0; kb < kb_p; ++kb) {
        const float* pk = pooled_k + ((long long)bh * kb_p + kb) * 64;
        float acc = 0.0f;
        for (int d = 0; d < 64; ++d) acc = fmaf(pq[d], pk[d], acc);
        s[kb] = acc * scale;
        m = fmaxf(m, s[kb]);
      }
      for (int kb = 0; kb < kb_p; ++kb) s[kb] = oracle_expf(s[kb] - m);
      const float total = sum64(s, kb_p);
      float* full = attn_full + ((long long)bh * q_blk + qb) * kb_p;
      for (int kb = 0; kb < kb_p; ++kb) full[kb] = s[kb] / total;
      float rs = sum64(full, n_cand);
      rs = fmaxf(rs, 0x1.0c6f7ap-20f);
      float* cond = attn_cond + ((long long)bh * q_blk + qb) * n_cand;
      for (int kb = 0; kb < n_cand; ++kb) cond[kb] = full[kb] / rs;
    }
  free(s);
  }
}

/* ---- baseline budget ------------------------------------------------------------------
 * compute_baseline_num_to_select (src/ress/models/attention.py:268-293): with a CDF
 * threshold, sort each row descending, SEQ cumsum, count of prefix sums <= fp32(tau)+1e-5
 * (searchsorted right=True); with a sparse ratio, topk = int(k*(1-sr)) (passed in) and the
 * larger of the two counts. cdf < 0 / topk < 0 disable the respective cut. */
static int cmp_desc(const void* a, const void* b) {
  float x = *(const float*)a, y = *(const float*)b;
  return (x < y) - (x > y);
}
void oracle_baseline_budget(const float* attn_cond, long long rows, int n, float cdf_threshold, int topk, int* out) {
  const float thr = cdf_threshold + 0x1.4f8b58p-17f;
#pragma omp parallel
  {
  float* v = (float*)malloc(sizeof(float) * (n > 0 ? n : 1));
#pragma omp for schedule(dynamic, 16)
  for (long long r = 0; r < rows; ++r) {
    if (cdf_threshold < 0.0f) {
      out[r] = topk;
      continue;
    }
    memcpy(v, attn_cond + r * n, sizeof(float) * n);
    qsort(v, n, sizeof(float), cmp_desc);
    float c = 0.0f;
    int count = 0;
    for (int i = 0; i < n; ++i) {
      c = c + v[i];
      if (c <= thr) ++count;
    }
    out[r] = count > topk ? count : topk;
  }
  free(v);
  }
}

/* ---- HeSS head reallocation -----------------------------------------------------------
 * adjust_attention_selection (src/ress/budget/_proportional.py:49-115) with
 * floor_frac=None, per (batch, q-block) column over heads, fp32, SEQ head sums:
 * ideal = scores_norm*total; adjusted = (1-beta)*nts + beta*ideal; repeat
 * {excess = clamp(adj - max, 0); stop if non-finite or sum <= 0; adj = min(adj, max);
 * w = adj*(adj<max); adj += w/(sum(w)+1e-9)*sum(excess)}; floor(min(adj, max)).
 * Then the floor min_select. Returns the largest iteration count, or -1 if a column
 * did not converge within max_iters. */
int oracle_head_budget(const int* baseline, int B, int H, int q_blk, const float* scores_norm, double beta,
                       int max_val, int max_iters, int min_select, int* out) {
  const float omb = (float)(1.0 - beta), bf = (float)beta, maxv = (float)max_val;
  int worst = 0;
  float* adj = (float*)malloc(sizeof(float) * H);
  float* w = (float*)malloc(sizeof(float) * H);
  for (int b = 0; b < B; ++b)
    for (int qb = 0; qb < q_blk; ++qb) {
      const int* base = baseline + (long long)b * H * q_blk + qb;
      int* dst = out + (long long)b * H * q_blk + qb;
      if (!scores_norm) {
        for (int h = 0; h < H; ++h) {
          int c = base[(long long)h * q_blk];
          dst[(long long)h * q_blk] = c < min_select ? min_select : c;
        }
        continue;
      }
      long long total = 0;
      for (int h = 0; h < H; ++h) total += base[(long long)h * q_blk];
      for (int h = 0; h < H; ++h) adj[h] = omb * (float)base[(long long)h * q_blk] + bf * (scores_norm[h] * (float)total);
      int it = 0;
      for (; it < max_iters; ++it) {
        float esum = 0.0f;
        int finite = 1;
        for (int h = 0; h < H; ++h) {
          float d = adj[h] - maxv;
          float ex = d < 0.0f ? 0.0f : d;
          finite = finite && (ex - ex == 0.0f);
          esum = esum + ex;
        }
        if (!finite || !(esum > 0.0f)) break;
        float wsum = 0.0f;
        for (int h = 0; h < H; ++h) {
          adj[h] = adj[h] > maxv ? maxv : adj[h];
          w[h] = adj[h] * (adj[h] < maxv ? 1.0f : 0.0f);
          wsum = wsum + w[h];
        }
        const float den = wsum + 0x1.12e0bep-30f;
        for (int h = 0; h < H; ++h) adj[h] = adj[h] + (w[h] / den) * esum;
      }
      if (it >= max_iters) worst = -1;
      else if (worst >= 0 && it > worst) worst = it;
      for (int h = 0; h < H; ++h) {
        float a = adj[h] > maxv ? maxv : adj[h];
        int c = (int)floorf(a);
        dst[(long long)h * q_blk] = c < min_select ? min_select : c;
      }
    }
  free(adj);
  free(w);
  return worst;
}

/* ---- selection --------------------------------------------------------------------------
 * build_block_mask (src/ress/models/attention.py:147-174): keep the top max(n, min_select)
 * (at most n_cand) candidates of each row, order (value desc, index asc) -- brute force by
 * sorting indices -- then the trailing sink columns (always kept) and any leading
 * attention_sink columns (external/patches/spargeattn.patch:61-65). LUT = ascending kept
 * columns (block_map_lut_triton, attention.py:224). Rows q_blk_sel..q_blk_total-1 are dense. */
static int cmp_rank(const void* a, const void* b, void* ctx) {
  const float* keys = (const float*)ctx;
  int i = *(const int*)a, j = *(const int*)b;
  uint32_t ki = order_key(keys[i]), kj = order_key(keys[j]);
  if (ki != kj) return ki > kj ? -1 : 1;
  return (i > j) - (i < j);
}
void oracle_select_blocks(const float* rank_key, const int* counts, int BH, int q_blk_sel, int q_blk_total,
                          int n_cand, int kb_tot, int sink_lead, int min_select, uint8_t* map, int* lut, int* nvalid) {
#pragma omp parallel
  {
  int* idx = (int*)malloc(sizeof(int) * (n_cand > 0 ? n_cand : 1));
  uint8_t* keep = (uint8_t*)malloc(kb_tot);
#pragma omp for schedule(dynamic, 4)
  for (long long row = 0; row < (long long)BH * q_blk_total; ++row) {
      const int bh = (int)(row / q_blk_total), qb = (int)(row % q_blk_total);
      if (qb >= q_blk_sel) {
        for (int c = 0; c < kb_tot; ++c) keep[c] = 1;
      } else {
        const long long srow = (long long)bh * q_blk_sel + qb;
        int n = counts[srow];
        n = n < min_select ? min_select : n;
        n = n < 0 ? 0 : (n > n_cand ? n_cand : n);
        for (int i = 0; i < n_cand; ++i) idx[i] = i;
        qsort_r(idx, n_cand, sizeof(int), cmp_rank, (void*)(rank_key + srow * n_cand));
        memset(keep, 0, kb_tot);
        for (int i = 0; i < n; ++i) keep[idx[i]] = 1;
        for (int c = n_cand; c < kb_tot; ++c) keep[c] = 1;
        for (int c = 0; c < sink_lead && c < kb_tot; ++c) keep[c] = 1;
        if (map) memcpy(map + srow * kb_tot, keep, kb_tot);
      }
      const long long lrow = (long long)bh * q_blk_total + qb;
      int pos = 0;
      for (int c = 0; c < kb_tot; ++c)
        if (keep[c]) lut[lrow * kb_tot + pos++] = c;
      nvalid[lrow] = pos;
    }
  free(idx);
  free(keep);
  }
}

/* vectorised helpers for tests */
void oracle_expf_array(const float* x, float* y, long long n) {
  for (long long i = 0; i < n; ++i) y[i] = oracle_expf(x[i]);
}
void oracle_round_bf16_array(const float* x, float* y, long long n) {
  for (long long i = 0; i < n; ++i) y[i] = oracle_round_bf16(x[i]);
}

/* ---- ReSS restore-swap ---------------------------------------------------------------
 * restore_swap_rank_by (src/ress/scoring/projected.py:395-1058) with the round body of
 * scoring/fused_round.py:_round_kernel (kept-mass-normalised objective J = ||g||^2_M / K^2,
 * drift compensate) and fused_topm's exact top-m (ties to the lowest index). One (head,
 * query-block) row at a time; rows are independent.
 *
 * Numerics. `big` (flag RS_BF16) is the dtype of the k-wide tensors: every value the
 * reference stores in bf16 is rounded here (bf), at the same points (quadratic_deviation
 * projected.py:259-288, dense_reference :313-356, the round :903-947, fused_round.py
 * :176-226). The reference leaves GEMM / sum accumulation orders to torch-CUDA; this
 * restatement fixes them, in the same order as the GPU kernels:
 *  - SEQK4, the sums over key blocks (P @ v_bar and sum P of the dense reference, Pd @ v_bar
 *    and sum_Pd of a drop set): four fp32 chains, chain c over the key blocks of the
 *    64-block chunks c, c + 4, c + 8, ... (k / 64 = c mod 4) in increasing k,
 *    fmaf(w_k, v_k[d], acc) with w_k = P_k, or 0 for a block outside the set (the zero
 *    terms are part of the chain), and the weight sum as fmaf(w_k, 1, acc); the result is
 *    (chain 0 + chain 1) + (chain 2 + chain 3);
 *  - DOT64, the per-candidate products v_k . Mvq and v_k . big(Mg): one sequential fmaf
 *    chain over d = 0..63;
 *  - the drop set's sum_Pd and Pd @ v_bar are formed afresh by SEQK4 for every objective
 *    (the reference recomputes Pd @ v_bar each round, projected.py:903-907);
 *  - every other sum and 64-term product (M v_bar_query, M g, ||g||^2_M, term_q, term_k)
 *    is a sequential fp32 chain in index order.
 * The GPU evaluates SEQK4 (one chain per wave) and DOT64 on the matrix cores (v_mfma_f32_16x16x4_f32 /
 * v_mfma_f32_32x32x2_f32 add their k terms to the accumulator one fmaf at a time, in k
 * order, on gfx950).
 *
 * A [H][q_blk][kb_p]  pooled map over the patch key blocks (attn_full), fp32
 * V [H][kb_p][64]     block-mean values (v_bar_full), fp32
 * M [H][64][64]       M_h = W_O^h^T W_O^h (identity for the _nowo recipes), fp32
 * nts [H][q_blk]      kept budget per row (after the min-2 floor)
 * keep [H][q_blk][n_cand]  out: 1 = kept candidate
 * obj  [H][q_blk]     out (optional): J of the returned set (fp32, this order)
 * s_out [H][q_blk][n_cand] out (optional): s = P*sqrt(d^T M d) (the rank_by base)
 * flags: 1 bf16 k-wide tensors, 2 track_best, 4 maximize, 8 invert_cut, 16 renormalize
 * off (the cut ranks s instead of s/(1-P)). Returns 0. */
#define RS_BF16 1
#define RS_TRACK_BEST 2
#define RS_MAXIMIZE 4
#define RS_INVERT_CUT 8
#define RS_NO_RENORM 16

static inline float rs_bf(float x, int big) { return big ? oracle_round_bf16(x) : x; }
/* fused_topm's order key: sign-bit flip for non-negatives, complement for negatives */
static inline uint32_t rs_key(float x) {
  uint32_t u = fbits(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
static int cmp_rs(const void* a, const void* b, void* ctx) {
  const uint32_t* keys = (const uint32_t*)ctx;
  int i = *(const int*)a, j = *(const int*)b;
  if (keys[i] != keys[j]) return keys[i] > keys[j] ? -1 : 1;
  return (i > j) - (i < j);
}
/* top-m of key among valid (ties: lowest index) -> sel[] = 1 */
static void rs_top_m(const float* q, const uint8_t* valid, int n, int m, uint8_t* sel, uint32_t* keys, int* idx) {
  int c = 0;
  for (int i = 0; i < n; ++i) {
    sel[i] = 0;
    keys[i] = rs_key(q[i]);
    if (valid[i]) idx[c++] = i;
  }
  qsort_r(idx, c, sizeof(int), cmp_rs, keys);
  for (int i = 0; i < m && i < c; ++i) sel[idx[i]] = 1;
}
/* kept_mass_norm_quality (projected.py:191-211), grouping ((G*u)*(2K+u))/(K*K) - dG, / Kn^2 */
static inline float rs_knorm(float G, float K, float dG, float u) {
  float Kn = K + u;
  Kn = Kn < 1e-6f ? 1e-6f : Kn;
  const float a = G * u;
  const float b = 2.0f * K + u;
  return (a * b / (K * K) - dG) / (Kn * Kn);
}

/* SEQK4 over k < n (use NULL: every k; else w_k = 0 where use[k] == 0): chain c = (k / 64)
 * mod 4 takes the fmaf terms w_k * V[k][d] (and w_k for the weight sum) in increasing k;
 * dot[d] = (chain 0 + chain 1) + (chain 2 + chain 3), *sum likewise */
static void rs_seqk(const float* P, const uint8_t* use, const float* Vb, int n, float* dot, float* sum) {
  float acc[4][64], sp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < 4; ++c)
    for (int d = 0; d < 64; ++d) acc[c][d] = 0.0f;
  for (int k = 0; k < n; ++k) {
    const int c = (k >> 6) & 3;
    const float w = (use && !use[k]) ? 0.0f : P[k];
    sp[c] = fmaf(w, 1.0f, sp[c]);
    for (int d = 0; d < 64; ++d) acc[c][d] = fmaf(w, Vb[(long long)k * 64 + d], acc[c][d]);
  }
  for (int d = 0; d < 64; ++d) dot[d] = (acc[0][d] + acc[1][d]) + (acc[2][d] + acc[3][d]);
  *sum = (sp[0] + sp[1]) + (sp[2] + sp[3]);
}
/* DOT64 of a and b (64 values each) */
static float rs_dot64(const float* a, const float* b) {
  float s = 0.0f;
  for (int d = 0; d < 64; ++d) s = fmaf(a[d], b[d], s);
  return s;
}

/* The objective state of a drop set: unrounded sum_Pd and Pd @ v_bar. */
typedef struct {
  float sp;
  float mv[64];
} rs_state;
static void rs_state_of(rs_state* st, const float* Pb, const uint8_t* drop, const float* Vb, int n_cand) {
  rs_seqk(Pb, drop, Vb, n_cand, st->mv, &st->sp);
}

/* g, Mg, ||g||^2_M, K and J of a state (projected.py:859-868 / 903-918) */
static float rs_objective(const rs_state* st, const float* M32, const float* vq, float tm, int big, float* g,
                          float* Mg, float* gn_out, float* K_out, float* sumpd_out) {
  const float* mv = st->mv;
  float sp = rs_bf(st->sp, big);
  for (int d = 0; d < 64; ++d) g[d] = sp * vq[d] - rs_bf(mv[d], big);
  for (int i = 0; i < 64; ++i) {
    float a = 0.0f;
    for (int j = 0; j < 64; ++j) a = fmaf(M32[i * 64 + j], g[j], a);
    Mg[i] = a;
  }
  float gn = 0.0f;
  for (int d = 0; d < 64; ++d) gn = gn + g[d] * Mg[d];
  float K = tm - sp;
  K = K < 1e-6f ? 1e-6f : K;
  *gn_out = gn;
  *K_out = K;
  *sumpd_out = sp;
  return gn / (K * K);
}

/* Per-head preparation: bf16-rounded M and V (when big) and the key side of
 * quadratic_deviation, term_k = big(sum_i big(big(M v_k)_i * v_ki)) (projected.py:282-284). */
static void rs_head_setup(const float* M32, const float* Vh, int kb_p, int n_cand, int big, float* Mb, float* Vb,
                          float* termk) {
  for (int i = 0; i < 4096; ++i) Mb[i] = rs_bf(M32[i], big);
  for (long long i = 0; i < (long long)kb_p * 64; ++i) Vb[i] = rs_bf(Vh[i], big);
#pragma omp parallel for schedule(static)
  for (int k = 0; k < n_cand; ++k) {
    float tk = 0.0f;
    for (int i = 0; i < 64; ++i) {
      float a = 0.0f;
      for (int j = 0; j < 64; ++j) a = fmaf(Mb[i * 64 + j], Vb[(long long)k * 64 + j], a);
      tk = tk + rs_bf(rs_bf(a, big) * Vb[(long long)k * 64 + i], big);
    }
    termk[k] = rs_bf(tk, big);
  }
}

/* Per-row scores: dense_reference (projected.py:313-356: v_bar_query = P @ v_bar, total mass),
 * quadratic_deviation's query side and cross term (:259-288), s = P*sqrt(quad), the cut key
 * s/(1-P).clamp(1e-4) (or s when renorm is off) and s^2 (:780-783). */
static void rs_row_setup(const float* Arow, const float* Mb, const float* Vb, const float* termk, int kb_p, int n_cand,
                         int big, int renorm, float* Pb, float* vq, float* tm_out, float* s, float* scut, float* ssq) {
  for (int k = 0; k < kb_p; ++k) Pb[k] = rs_bf(Arow[k], big);
  float tm;
  rs_seqk(Pb, NULL, Vb, kb_p, vq, &tm);
  *tm_out = rs_bf(tm, big);
  for (int d = 0; d < 64; ++d) vq[d] = rs_bf(vq[d], big);
  float Mvq[64], tq = 0.0f;
  for (int i = 0; i < 64; ++i) {
    float a = 0.0f;
    for (int j = 0; j < 64; ++j) a = fmaf(Mb[i * 64 + j], vq[j], a);
    Mvq[i] = rs_bf(a, big);
  }
  for (int i = 0; i < 64; ++i) tq = tq + rs_bf(Mvq[i] * vq[i], big);
  tq = rs_bf(tq, big);
  for (int k = 0; k < n_cand; ++k) {
    const float cr = rs_bf(rs_dot64(Mvq, Vb + (long long)k * 64), big);
    float qd = rs_bf(rs_bf(tq - rs_bf(2.0f * cr, big), big) + termk[k], big);
    qd = qd < 0.0f ? 0.0f : qd;
    const float sq = rs_bf(sqrtf(qd), big);
    s[k] = rs_bf(Pb[k] * sq, big);
    float om = rs_bf(1.0f - Pb[k], big);
    om = rs_bf(om < 1e-4f ? 1e-4f : om, big);
    scut[k] = renorm ? rs_bf(s[k] / om, big) : s[k];
    ssq[k] = rs_bf(s[k] * s[k], big);
  }
}

/* One round's marginals for the current drop set (projected.py:903-947, fused_round.py
 * :170-226): J = ||g||^2_M / K^2, and per candidate k the knorm quality of restoring it
 * (dG = 2 raw + s^2, u = +P_k) and of dropping it (dG = s^2 - 2 raw, u = -P_k), with
 * raw = big(P_k * big(v_k.Mg - v_bar_query.Mg)). rq/cq are written for every candidate
 * (not masked by the drop set, not sign-flipped); returns J. */
static float rs_round_qualities(const float* Pb, const rs_state* st, const float* Vb, const float* M32,
                                const float* vq, float tm, const float* ssq, int n_cand, int big, float* rq,
                                float* cq) {
  float g[64], Mg[64], gn, K, sp;
  const float J = rs_objective(st, M32, vq, tm, big, g, Mg, &gn, &K, &sp);
  float tqr = 0.0f, Mgb[64];
  for (int d = 0; d < 64; ++d) tqr = tqr + vq[d] * Mg[d];
  const float tqb = rs_bf(tqr, big);
  for (int d = 0; d < 64; ++d) Mgb[d] = rs_bf(Mg[d], big);
  for (int k = 0; k < n_cand; ++k) {
    const float tk = rs_bf(rs_dot64(Vb + (long long)k * 64, Mgb), big);
    const float raw = rs_bf(Pb[k] * rs_bf(tk - tqb, big), big);
    rq[k] = rs_knorm(gn, K, 2.0f * raw + ssq[k], Pb[k]);
    cq[k] = rs_knorm(gn, K, ssq[k] - 2.0f * raw, -Pb[k]);
  }
  return J;
}

/* Per-row scratch of oracle_restore_swap (one per thread). */
typedef struct {
  float *Pb, *s, *scut, *ssq, *rq, *cq;
  uint8_t *drop, *best, *sel, *sel2, *valid;
  uint32_t* keys;
  int* idx;
} rs_scratch;

static void rs_scratch_alloc(rs_scratch* w, int kb_p, int n_cand) {
  const size_t n = (size_t)(n_cand > 0 ? n_cand : 1);
  w->Pb = (float*)malloc(sizeof(float) * (size_t)(kb_p > 0 ? kb_p : 1));
  w->s = (float*)malloc(sizeof(float) * n);
  w->scut = (float*)malloc(sizeof(float) * n);
  w->ssq = (float*)malloc(sizeof(float) * n);
  w->rq = (float*)malloc(sizeof(float) * n);
  w->cq = (float*)malloc(sizeof(float) * n);
  w->drop = (uint8_t*)malloc(n);
  w->best = (uint8_t*)malloc(n);
  w->sel = (uint8_t*)malloc(n);
  w->sel2 = (uint8_t*)malloc(n);
  w->valid = (uint8_t*)malloc(n);
  w->keys = (uint32_t*)malloc(sizeof(uint32_t) * n);
  w->idx = (int*)malloc(sizeof(int) * n);
}

static void rs_scratch_free(rs_scratch* w) {
  free(w->Pb); free(w->s); free(w->scut); free(w->ssq); free(w->rq); free(w->cq);
  free(w->drop); free(w->best); free(w->sel); free(w->sel2); free(w->valid); free(w->keys); free(w->idx);
}

/* One (head, query-block) row: initial cut, n_iters rounds, track-best (projected.py:756-1058). */
static void rs_row(const float* Arow, const float* Mb, const float* Vb, const float* termk, const float* M32, int nts_row,
                   int kb_p, int n_cand, int n_iters, double restore_frac, double decay, int flags, rs_scratch* w,
                   uint8_t* keep_row, float* obj, float* s_row) {
  const int big = (flags & RS_BF16) != 0, track = (flags & RS_TRACK_BEST) != 0;
  const int renorm = (flags & RS_NO_RENORM) == 0;
  const int maxim = (flags & RS_MAXIMIZE) != 0, inv = (flags & RS_INVERT_CUT) != 0;
  float *Pb = w->Pb, *s = w->s, *scut = w->scut, *ssq = w->ssq, *rq = w->rq, *cq = w->cq;
  uint8_t *drop = w->drop, *best = w->best, *sel = w->sel, *sel2 = w->sel2, *valid = w->valid;
  float vq[64], tm;
  rs_row_setup(Arow, Mb, Vb, termk, kb_p, n_cand, big, renorm, Pb, vq, &tm, s, scut, ssq);
  if (s_row)
    for (int k = 0; k < n_cand; ++k) s_row[k] = s[k];
  /* initial one-shot cut: keep the top min(nts, n_cand) by s_cut (lowest under invert_cut) */
  int nkeep = nts_row;
  nkeep = nkeep < 0 ? 0 : (nkeep > n_cand ? n_cand : nkeep);
  for (int k = 0; k < n_cand; ++k) {
    valid[k] = 1;
    rq[k] = inv ? -scut[k] : scut[k];
  }
  rs_top_m(rq, valid, n_cand, nkeep, sel, w->keys, w->idx);
  for (int k = 0; k < n_cand; ++k) drop[k] = !sel[k];
  float g[64], Mg[64], gn, K, sp;
  rs_state st;
  rs_state_of(&st, Pb, drop, Vb, n_cand);
  float best_obj = 0.0f;
  if (track) {
    best_obj = rs_objective(&st, M32, vq, tm, big, g, Mg, &gn, &K, &sp);
    memcpy(best, drop, (size_t)n_cand);
  }
  double remaining = restore_frac;
  for (int it = 0; it < n_iters; ++it) {
    const double frac = remaining * decay;
    remaining -= frac;
    const int pic0 = (int)rintf((float)frac * (float)nts_row);
    const float J = rs_round_qualities(Pb, &st, Vb, M32, vq, tm, ssq, n_cand, big, rq, cq);
    if (track) {
      const int better = maxim ? J > best_obj : J < best_obj;
      if (better) {
        best_obj = J;
        memcpy(best, drop, (size_t)n_cand);
      }
    }
    int n_drop = 0, n_kept = 0;
    float rmax = -INFINITY;
    for (int k = 0; k < n_cand; ++k) {
      const float r = maxim ? -rq[k] : rq[k];
      const float c = maxim ? -cq[k] : cq[k];
      rq[k] = drop[k] ? r : -INFINITY;
      cq[k] = drop[k] ? -INFINITY : c;
      if (drop[k]) {
        ++n_drop;
        rmax = rq[k] > rmax ? rq[k] : rmax;
      } else {
        ++n_kept;
      }
    }
    const int beneficial = rmax > 0.0f;
    int pic = pic0;
    if (beneficial && pic < 1) pic = 1;
    int cnt = pic < n_drop ? pic : n_drop;
    cnt = cnt < n_kept ? cnt : n_kept;
    if (!beneficial) cnt = 0;
    for (int k = 0; k < n_cand; ++k) valid[k] = drop[k];
    rs_top_m(rq, valid, n_cand, cnt, sel, w->keys, w->idx);
    for (int k = 0; k < n_cand; ++k) valid[k] = !drop[k];
    rs_top_m(cq, valid, n_cand, cnt, sel2, w->keys, w->idx);
    for (int k = 0; k < n_cand; ++k) drop[k] = (uint8_t)((drop[k] && !sel[k]) || sel2[k]);
    rs_state_of(&st, Pb, drop, Vb, n_cand);
  }
  float fin = 0.0f;
  if (track || obj) fin = rs_objective(&st, M32, vq, tm, big, g, Mg, &gn, &K, &sp);
  if (track) {
    const int better = maxim ? fin > best_obj : fin < best_obj;
    if (!better) {
      memcpy(drop, best, (size_t)n_cand);
      fin = best_obj;
    }
  }
  if (obj) *obj = fin;
  for (int k = 0; k < n_cand; ++k) keep_row[k] = (uint8_t)!drop[k];
}

int oracle_restore_swap(const float* A, const float* V, const float* M, const int* nts, int H, int q_blk, int kb_p,
                        int n_cand, int n_iters, double restore_frac, double decay, int flags, uint8_t* keep,
                        float* obj_out, float* s_out) {
  const int big = (flags & RS_BF16) != 0;
  float* Vb = (float*)malloc(sizeof(float) * (size_t)(kb_p > 0 ? kb_p : 1) * 64);
  float* Mb = (float*)malloc(sizeof(float) * 64 * 64);
  float* termk = (float*)malloc(sizeof(float) * (size_t)(kb_p > 0 ? kb_p : 1));
  for (int h = 0; h < H; ++h) {
    const float* M32 = M + (long long)h * 4096;
    rs_head_setup(M32, V + (long long)h * kb_p * 64, kb_p, n_cand, big, Mb, Vb, termk);
#pragma omp parallel
    {
      rs_scratch w;
      rs_scratch_alloc(&w, kb_p, n_cand);
#pragma omp for schedule(dynamic, 1)
      for (int q = 0; q < q_blk; ++q) {
        const long long row = (long long)h * q_blk + q;
        rs_row(A + row * kb_p, Mb, Vb, termk, M32, nts[row], kb_p, n_cand, n_iters, restore_frac, decay, flags, &w,
               keep + row * n_cand, obj_out ? obj_out + row : NULL, s_out ? s_out + row * n_cand : NULL);
      }
      rs_scratch_free(&w);
    }
  }
  free(Vb); free(Mb); free(termk);
  return 0;
}

/* The quantities oracle_restore_swap ranks by, for a caller-given drop set, through the same
 * helpers (for checks against first principles): s and the initial cut's key scut
 * [H][q_blk][n_cand], J [H][q_blk] of the drop set, and the round marginals rq / cq
 * [H][q_blk][n_cand] (rs_round_qualities: every candidate, unmasked, minimisation sign).
 * drop [H][q_blk][n_cand] uint8, 1 = dropped.
 * flags as for oracle_restore_swap (only RS_BF16 and RS_NO_RENORM matter here). */
int oracle_rs_probe(const float* A, const float* V, const float* M, const uint8_t* drop, int H, int q_blk, int kb_p,
                    int n_cand, int flags, float* s_out, float* scut_out, float* J_out, float* rq_out,
                    float* cq_out) {
  const int big = (flags & RS_BF16) != 0, renorm = (flags & RS_NO_RENORM) == 0;
  float* Vb = (float*)malloc(sizeof(float) * (size_t)kb_p * 64);
  float* Mb = (float*)malloc(sizeof(float) * 64 * 64);
  float* termk = (float*)malloc(sizeof(float) * (size_t)kb_p);
  float* Pb = (float*)malloc(sizeof(float) * (size_t)kb_p);
  float* ssq = (float*)malloc(sizeof(float) * (size_t)n_cand);
  for (int h = 0; h < H; ++h) {
    const float* M32 = M + (long long)h * 4096;
    rs_head_setup(M32, V + (long long)h * kb_p * 64, kb_p, n_cand, big, Mb, Vb, termk);
    for (int q = 0; q < q_blk; ++q) {
      const long long row = (long long)h * q_blk + q;
      float vq[64], tm;
      rs_row_setup(A + row * kb_p, Mb, Vb, termk, kb_p, n_cand, big, renorm, Pb, vq, &tm, s_out + row * n_cand,
                   scut_out + row * n_cand, ssq);
      rs_state st;
      rs_state_of(&st, Pb, drop + row * n_cand, Vb, n_cand);
      J_out[row] = rs_round_qualities(Pb, &st, Vb, M32, vq, tm, ssq, n_cand, big, rq_out + row * n_cand,
                                      cq_out + row * n_cand);
    }
  }
  free(Vb); free(Mb); free(termk); free(Pb); free(ssq);
  return 0;
}

/* ---- SpargeAttn-convention block map (meansim) ----------------------------------------
 * get_block_map_meansim_fuse_quant as the reference patches it (external/patches/
 * spargeattn.patch:54-66: attention_sink = a count of leading tokens, forcing its
 * ceil(s/64) leading key blocks; Q quantised with sm_scale = 1, the scale of
 * quant_per_block, :38-41). SpargeAttn itself is not in the reference; this is the
 * build's restatement (parity unpinned against SpargeAttn):
 *  per block (Q 128, K 64 tokens; K smoothed by km when given), x the fp32 values:
 *    pooled  = mean_t x_t   (token lane r < 32 sums rows r, r+32, ... in order, tree8 over
 *              lanes 8w..8w+7, then (W0 + W1) + (W2 + W3); rows past the end add 0)
 *    sim     = ||sum_t x_t/||x_t|| ||^2 / n^2, the mean pairwise cosine similarity
 *              (self pairs included; a zero row contributes 0); similar = sim > simthreshd1[h]
 *    codes   = the per-block INT8 quantiser (scale = amax/127)
 *  per (head, q-block) row: scores = DOT64(pooled_q, pooled_k)/8 over the similar K
 *  blocks (the others -inf), softmax (ress exp, SUM64 sum), keep the top-n by (p desc,
 *  index asc) with n = #{prefix sums of the sorted p <= cdfthreshd[h]}, the prefix sums
 *  taken exactly over q = floor(p * 2^50) (uint64) against floor(min(th, 8192) * 2^50), then force on
 *  the non-similar K blocks, every block of a non-similar Q row, and the sinks.
 * q, k: (BH, T, 64) bf16; km [BH][64] or NULL; simth, cdfth [H].
 * Outputs: map [BH][nq][nk] uint8, q_i8 [BH][nq*128][64], q_scale [BH][nq],
 * k_i8 [BH][nk*64][64], k_scale [BH][nk], pooled_q [BH][nq][64], pooled_k [BH][nk][64],
 * sim_q [BH][nq], sim_k [BH][nk] uint8. */
static inline float tree8(const float* p) { return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])); }

static void ms_block(const uint16_t* x, const float* km, int T, int b, int BS, float th, float* pooled, uint8_t* sim,
                     int8_t* codes, float* scale_out) {
  const int base = b * BS, cnt = T - base < BS ? T - base : BS;
  float xs[128][64], xh[128][64];
  float amax = 0.0f;
  for (int t = 0; t < cnt; ++t) {
    float part[8];
    for (int d = 0; d < 64; ++d) {
      float v = bf16f(x[(long long)(base + t) * 64 + d]);
      if (km) v = v - km[d];
      xs[t][d] = v;
      const float av = fabsf(v);
      amax = av > amax ? av : amax;
    }
    for (int g = 0; g < 8; ++g) {
      float a = 0.0f;
      for (int c = 0; c < 8; ++c) a = fmaf(xs[t][8 * g + c], xs[t][8 * g + c], a);
      part[g] = a;
    }
    const float n2 = tree8(part);
    const float inv = n2 > 0.0f ? 1.0f / sqrtf(n2) : 0.0f;
    for (int d = 0; d < 64; ++d) xh[t][d] = xs[t][d] * inv;
  }
  /* per dim, over the BS padded rows (zeros past cnt): token lane r < 32 adds rows r + 32p
   * in p order, lanes 8w..8w+7 combine by tree8, the four groups as (W0 + W1) + (W2 + W3) */
  float ssum[64];
  for (int d = 0; d < 64; ++d) {
    float wp[4], wh[4];
    for (int w = 0; w < 4; ++w) {
      float lp[8], lh[8];
      for (int tl = 0; tl < 8; ++tl) {
        float a = 0.0f, h = 0.0f;
        for (int t = 8 * w + tl; t < BS; t += 32) {
          a = a + (t < cnt ? xs[t][d] : 0.0f);
          h = h + (t < cnt ? xh[t][d] : 0.0f);
        }
        lp[tl] = a;
        lh[tl] = h;
      }
      wp[w] = tree8(lp);
      wh[w] = tree8(lh);
    }
    pooled[d] = ((wp[0] + wp[1]) + (wp[2] + wp[3])) / (float)cnt;
    ssum[d] = (wh[0] + wh[1]) + (wh[2] + wh[3]);
  }
  float part[8];
  for (int g = 0; g < 8; ++g) {
    float a = 0.0f;
    for (int c = 0; c < 8; ++c) a = fmaf(ssum[8 * g + c], ssum[8 * g + c], a);
    part[g] = a;
  }
  const float s = tree8(part) / ((float)cnt * (float)cnt);
  *sim = s > th;
  const float scale = amax / 127.0f;
  *scale_out = scale;
  for (int t = 0; t < BS; ++t)
    for (int d = 0; d < 64; ++d) codes[t * 64 + d] = t < cnt ? quant(xs[t][d], scale) : 0;
}

static const float* g_ms_p;
static int cmp_ms(const void* a, const void* b) {
  const int i = *(const int*)a, j = *(const int*)b;
  const uint32_t ki = order_key(g_ms_p[i]), kj = order_key(g_ms_p[j]);
  if (ki != kj) return ki > kj ? -1 : 1;
  return (i > j) - (i < j);
}

void oracle_meansim_map(const uint16_t* q, const uint16_t* k, const float* km, int BH, int H, int Tq, int Tk,
                        const float* simth, const float* cdfth, int attention_sink, uint8_t* map, int8_t* q_i8,
                        float* q_scale, int8_t* k_i8, float* k_scale, float* pooled_q, float* pooled_k, uint8_t* sim_q,
                        uint8_t* sim_k) {
  const int nq = cdiv(Tq, 128), nk = cdiv(Tk, 64);
  float* sc = (float*)malloc(sizeof(float) * nk);
  int* idx = (int*)malloc(sizeof(int) * nk);
  const int n_sink = attention_sink > 0 ? cdiv(attention_sink, 64) : 0;
  for (int bh = 0; bh < BH; ++bh) {
    const int h = bh % H;
    for (int b = 0; b < nq; ++b)
      ms_block(q + (long long)bh * Tq * 64, NULL, Tq, b, 128, simth[h], pooled_q + ((long long)bh * nq + b) * 64,
               sim_q + (long long)bh * nq + b, q_i8 + ((long long)bh * nq + b) * 128 * 64, q_scale + (long long)bh * nq + b);
    for (int b = 0; b < nk; ++b)
      ms_block(k + (long long)bh * Tk * 64, km ? km + (long long)bh * 64 : NULL, Tk, b, 64, simth[h],
               pooled_k + ((long long)bh * nk + b) * 64, sim_k + (long long)bh * nk + b,
               k_i8 + ((long long)bh * nk + b) * 64 * 64, k_scale + (long long)bh * nk + b);
    for (int r = 0; r < nq; ++r) {
      uint8_t* row = map + ((long long)bh * nq + r) * nk;
      const float* pq = pooled_q + ((long long)bh * nq + r) * 64;
      float mx = -INFINITY;
      for (int c = 0; c < nk; ++c) {
        if (!sim_k[(long long)bh * nk + c]) {
          sc[c] = -INFINITY;
          continue;
        }
        const float* pk = pooled_k + ((long long)bh * nk + c) * 64;
        float a = 0.0f;
        for (int d = 0; d < 64; ++d) a = fmaf(pq[d], pk[d], a);
        sc[c] = a * 0.125f;
        mx = sc[c] > mx ? sc[c] : mx;
      }
      memset(row, 0, nk);
      if (mx > -INFINITY) {
        for (int c = 0; c < nk; ++c) sc[c] = sc[c] == -INFINITY ? 0.0f : oracle_expf(sc[c] - mx);
        const float sum = sum64(sc, nk);
        for (int c = 0; c < nk; ++c) sc[c] = sc[c] / sum;
        for (int c = 0; c < nk; ++c) idx[c] = c;
        g_ms_p = sc;
        qsort(idx, nk, sizeof(int), cmp_ms);
        /* n = #{k : S_k <= T}: S_k the exact sum of the k largest q = floor(p * 2^50) (uint64),
           T = floor(min(cdfth, 8192) * 2^50); a negative (or NaN) threshold keeps none */
        int n = 0;
        const float th = cdfth[h];
        if (th >= 0.0f) {
          const uint64_t T = (uint64_t)((double)(th < 8192.0f ? th : 8192.0f) * 1125899906842624.0);
          uint64_t cum = 0;
          for (int i = 0; i < nk; ++i) {
            cum += (uint64_t)((double)sc[idx[i]] * 1125899906842624.0);
            if (cum <= T) n = i + 1;
            else break;
          }
        }
        for (int i = 0; i < n; ++i) row[idx[i]] = 1;
      }
      for (int c = 0; c < nk; ++c)
        if (!sim_k[(long long)bh * nk + c] || !sim_q[(long long)bh * nq + r] || c < n_sink) row[c] = 1;
    }
  }
  free(sc);
  free(idx);
}
