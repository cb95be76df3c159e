// Block-sparse attention forward for gfx950: QK^T on 16-bit (fp16) or INT8 operands,
// online softmax, PV on bf16 (or fp16) MFMAs.
//
// Replaces SpargeAttn's qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold
// as the reference calls it (src/ress/models/attention.py:238-241: HND layout, not
// causal, per-block Q/K scales, sm_scale = 1/sqrt(64), PV threshold disabled), and
// the special-query dense SDPA of attention.py:409 (special query blocks are rows
// whose LUT lists every key block).
//
//   O[q] = sum_k softmax_k( sm_scale * (Q[q] . K[k]) ) V[k]
//
// Work item = (batch*head, 128-query block). Per kept 64-key block:
//   S^T = K . Q^T      v_mfma_f32_32x32x16_f16 (16-bit mode), or
//                      v_mfma_i32_32x32x32_i8 (INT8 modes, 1 or 3 per tile)
//   softmax in the exp2 domain: P = exp2(logit) directly on bounded 16-bit rows, else a
//   lazily rescaled running max with the scale folded into one fma
//   O^T (64 dims x 32 queries) += V^T . P^T    v_mfma_f32_32x32x16_{bf16,f16}
// 16-bit mode: 512 threads = 8 waves, wave w takes query group w/2 (32 queries) and key
// half w%2 of every block; the two halves merge through LDS when the row ends. INT8 modes:
// 256 threads = 4 waves of 32 queries, both key tiles per wave.
// The S^T accumulator layout puts one query per lane, so P feeds the PV MFMA from
// registers; V is pre-packed (prep.hip) with keys permuted to match. K/V tiles go
// through LDS stages filled by LDS-DMA several blocks ahead. The kernels are persistent:
// each XCD walks its own range of rows (see k_attn_schedule) so a head's K/V stay in its L2.
#include "common.h"

#include <mutex>
#include <type_traits>

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
  const uint16_t* q_bf;    // QK_F16: the bf16 queries, (B,H,T,64) storage order, strides sqB/sqH/sqT
  long long sqB, sqH, sqT;
  const uint16_t* k_pack;  // QK_F16: [BH][kb_tot][64 keys][64] fp16
  const float* k_norm;     // QK_F16: [BH][kb_tot] the block's largest key norm
  const int* lut;          // [BH][q_blk_total][kb_tot]
  const int* nvalid;       // [BH][q_blk_total]
  void* out;
  long long soB, soH, soT;
  int H, BH;
  int q_blk_p, q_blk_total, kb_tot, Tk;
  float sm_scale_log2e;
  int* sched;   // the row schedule written by k_attn_schedule (header of the sched workspace)
  float* part;  // key-range parts of the split rows (rest of the sched workspace)
  int split_L;  // rows split at the end of each XCD's range
  int chunks;   // patch-row order: 1 head-major, RESS_ROW_CHUNKS chunk-major (item_to_row)
  TokenMap m;   // query rows: patch blocks via patch_to_storage, the rest via special_to_storage
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

// LDS layout of one stage: K hi tile (4 KiB, 64 rows x 4 chunks of 16 B), [K lo
// tile], V^T tile (8 KiB, 64 rows x 8 chunks). Chunks are XOR-swizzled so that the
// b128 reads of any 8 or 16 consecutive lanes (consecutive rows, same logical chunk)
// fall in distinct bank groups:
//   K: chunk c of row r at 4r + (c ^ (((r >> 1) ^ (r >> 3)) & 3))
//   V: chunk c of row r at 8r + (c ^ ((r ^ (r >> 3)) & 7))
__device__ __forceinline__ int k_slot(int r, int c) { return 4 * r + (c ^ (((r >> 1) ^ (r >> 3)) & 3)); }
__device__ __forceinline__ int v_slot(int r, int c) { return 8 * r + (c ^ ((r ^ (r >> 3)) & 7)); }

// 16 bytes per lane, global -> LDS without a register round trip (buffer_load_dwordx4 ...
// lds): lane i of the wave writes lds_base + 16*i (lds_base uniform, taken from M0) with the
// bytes at soffset + voffset from the descriptor's base. The stage loads address a head's
// blocks through one descriptor per operand: the block offset is the scalar soffset and the
// lane's chunk a 32-bit voffset, so a DMA costs no VALU address arithmetic (the flat form's
// 64-bit lane addresses cost two VALU ops per load in the 16-bit loop).
#define RESS_BUF_DWORD3 0x00020000  // raw (untyped) buffer: descriptor word 3 of the gfx9 family
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, RESS_BUF_DWORD3);
}
__device__ __forceinline__ void buf_lds16(__amdgpu_buffer_rsrc_t rsrc, unsigned voffset, int soffset, void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds_base, 16, (int)voffset,
                                           soffset, 0, 0);
}
__device__ __forceinline__ void wait_lds_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Barrier between pipeline steps. __syncthreads() would also wait for every outstanding
// global access (vmcnt(0)), i.e. for the DMA just started two blocks ahead. Here the
// DMA the next step reads has been waited for explicitly (wait_lds_dma_but), this
// wave's LDS reads are complete (lgkmcnt(0)), and the empty asm statements keep the
// compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// all but the newest N vector-memory operations of this wave complete (loads retire in
// issue order): waits for older stages while the newest stage's DMA stays in flight
template <int N>
__device__ __forceinline__ void wait_lds_dma_but() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

template <bool V_F16>
__device__ __forceinline__ uint32_t cvt_pair(float a, float b) {
  const v2f x = {a, b};
  if constexpr (V_F16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2h));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2bf));
}
// a.x + a.y of a packed 16-bit pair accumulated in fp32
template <bool V_F16>
__device__ __forceinline__ float dot2_acc(uint32_t p, float acc) {
  if constexpr (V_F16) {
    const v2h ones = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, p), ones, acc, false);
  } else {
    const v2bf ones = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, p), ones, acc, false);
  }
}

// Reductions over the lane pair (l, l^32) that share a query row, without LDS:
// v_permlane32_swap exchanges the two 32-lane halves.
__device__ __forceinline__ int pair_max(int x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return max((int)r[0], (int)r[1]);
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float((int)r[0]) + __int_as_float((int)r[1]);
}

// ---- work schedule ---------------------------------------------------------
// Rows are items: first the dense special rows of every head, then the patch rows
// head-major (chunk-major for very large K/V, see item_to_row). The schedule cuts the
// item list into 8 contiguous ranges of equal work (kept blocks + a fixed per-row cost),
// one per XCD, so each XCD walks few heads (their K/V stay in its L2) and all XCDs
// finish together. The dense rows (every key block,
// several times a patch row) lead so they start at once: in head-major order the dense
// row of a head in the middle of a range would start late and end long after the rest.
//   sched[0..8]   range bounds (sched[j] .. sched[j+1]-1 belong to XCD j)
//   sched[16..23] per-XCD next-item counters (atomically advanced by the kernel)
//   sched[24]     operand status of the 16-bit kernel: RESS_F16_KEY_RANGE |
//                 RESS_F16_QUERY_RANGE when a key / query element was outside fp16's range
#define RESS_F16_KEY_RANGE 1
#define RESS_F16_QUERY_RANGE 2
#define RESS_SCHED_INTS 32
#define RESS_ROW_COST 2
// Tail split. Workgroups run out of rows one by one at the end of a range; the spread of
// their end times is about one row's duration. The last RESS_SPLIT_ROWS rows of each
// range (half the workgroups of an XCD; measured best) therefore run as RESS_SPLIT_PARTS parts over
// consecutive slices of their kept blocks. A part leaves its unnormalised O, running max
// and row sum in a slot of the workspace (RESS_PART_FLOATS floats, register order), and
// k_attn_merge combines the parts of each split row and writes it.
#define RESS_SPLIT_ROWS 32
#define RESS_SPLIT_PARTS 3
#define RESS_PART_FLOATS (256 * 32 + 2 * 256)
#define RESS_SCHED_HDR_BYTES 256

// Patch-row order. Head-major (chunks = 1): each XCD's range holds whole heads, whose K/V
// its L2 then serves. Chunk-major (chunks = RESS_ROW_CHUNKS): chunk c is q-blocks
// [c*q/8, (c+1)*q/8) of every head, so range x is about chunk x of every head and all
// XCDs walk the heads together: the K/V being read at any time is one head's, which the
// memory-side cache can hold when all heads' K/V cannot (the host picks it above
// RESS_CHUNK_MIN_KV bytes of K/V).
#define RESS_ROW_CHUNKS 8
#define RESS_CHUNK_MIN_KV (512LL << 20)
__device__ __forceinline__ void item_to_row(int i, int BH, int q_blk_p, int q_blk_total, int chunks, int& bh,
                                            int& qb) {
  const int qs = q_blk_total - q_blk_p;  // special (dense) q-blocks per head
  const int ns = BH * qs;
  if (i < ns) {
    bh = i / qs;
    qb = q_blk_p + (i - bh * qs);
  } else if (chunks == 1) {
    const int j = i - ns;
    bh = j / q_blk_p;
    qb = j - bh * q_blk_p;
  } else {  // the first chunk whose end passes j (empty chunks are passed over)
    const int j = i - ns;
    int c = 0;
    while (c < chunks - 1 && j >= BH * ((c + 1) * q_blk_p / chunks)) ++c;
    const int lo = c * q_blk_p / chunks, sz = (c + 1) * q_blk_p / chunks - lo, jj = j - BH * lo;
    bh = jj / sz;
    qb = lo + (jj - bh * sz);
  }
}

__global__ __launch_bounds__(1024) void k_attn_schedule(const int* __restrict__ nvalid, int BH, int q_blk_p,
                                                        int q_blk_total, int chunks, int* __restrict__ sched) {
  __shared__ long long wtot[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int n = BH * q_blk_total;
  const int per = (n + 1023) / 1024;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
  long long s = 0;
  for (int i = i0; i < i1; ++i) {
    int bh, qb;
    item_to_row(i, BH, q_blk_p, q_blk_total, chunks, bh, qb);
    s += nvalid[(long long)bh * q_blk_total + qb] + RESS_ROW_COST;
  }
  if (tid < 9) sched[tid] = tid == 0 ? 0 : n;
  if (tid == 9) sched[24] = 0;  // operand status, set by the 16-bit kernel
  // inclusive scan of the threads' sums: lane shuffles within each wave, then the 16 wave
  // totals through LDS (one barrier)
  long long incl = (long long)wave_scan_sum_u64((unsigned long long)s);
  if (lane == 63) wtot[wv] = incl;
  __syncthreads();
  long long W = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const long long t = wtot[k];
    incl += k < wv ? t : 0;
    W += t;
  }
  long long run = incl - s;  // exclusive prefix of this thread's first item
  long long prev = -1;            // exclusive prefix of item i-1
  if (i0 > 0 && i0 < n) {
    int bh, qb;
    item_to_row(i0 - 1, BH, q_blk_p, q_blk_total, chunks, bh, qb);
    prev = run - (nvalid[(long long)bh * q_blk_total + qb] + RESS_ROW_COST);
  }
  for (int i = i0; i < i1; ++i) {
    // item i starts range j if its exclusive prefix is the first to reach j*W/8
    for (int j = 1; j < 8; ++j)
      if (run * 8 >= (long long)j * W && prev * 8 < (long long)j * W) sched[j] = i;
    int bh, qb;
    item_to_row(i, BH, q_blk_p, q_blk_total, chunks, bh, qb);
    prev = run;
    run += nvalid[(long long)bh * q_blk_total + qb] + RESS_ROW_COST;
  }
  __syncthreads();
  if (tid < 8) sched[16 + tid] = sched[tid];
}

// The running max is moved (and O, l rescaled) only when a row's block max exceeds it
// by more than this many log2 units, so P stays below 2^8; the final O / l is exact.
#define RESS_RESCALE_LOG2 8.0f

// QK^T operand modes.
//  QK_I8    single-term per-block INT8 (the reference's SpargeAttn quantiser)
//  QK_I8X2  two-term INT8, x ~ s*hi + s/254*lo: S = 254*(hi.hi) + hi.lo + lo.hi in
//           int32 (the lo.lo term, below 2^-16 relative, is dropped)
//  QK_F16   16-bit operands: fp16 K blocks, the bf16 queries converted to fp16 per row
//           (pre-scaled on bounded rows), fp32 accumulation (see attn_row_f16)
enum { QK_I8 = 0, QK_I8X2 = 1, QK_F16 = 2 };

// INT8 modes. Q operand of one lane (query qi, half g), four 16-byte registers: [0],[1]
// = hi codes of dims 16g..16g+15 and 32+16g..; [2],[3] = lo codes. K operand LDS slots of
// one lane for tile t (key 32t+qi): ks[0], ks[1] = hi chunks g and 2+g (lo chunks at +256
// slots).
template <int QK>
__device__ __forceinline__ void k_slots(int row, int g, int ks[4]) {
  ks[0] = k_slot(row, g);
  ks[1] = k_slot(row, 2 + g);
  ks[2] = ks[3] = 0;
}

__device__ __forceinline__ float pair_maxf(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float((int)r[0]), __int_as_float((int)r[1]));
}

// INT8 modes: S^T for one 32-key tile (keys 32t.. of the stage) as floats, plus the
// tile's max score (in S units). Register r is key 32t + 8(r/4) + 4g + r%4 of the block.
// nkt = valid keys in the tile (MASK only): masked scores are the lowest int, which exp2
// maps to 0.
template <int QK, bool MASK>
__device__ __forceinline__ void qk_tile(const uint4* __restrict__ sk, int nkt, const int (&ks)[4],
                                        const uint4 (&qv)[4], int g, float (&s)[16], float& tmax) {
  static_assert(QK != QK_F16, "qk_tile is the INT8 modes' QK^T");
  {
    const v4i kx0 = __builtin_bit_cast(v4i, sk[ks[0]]);
    const v4i kx1 = __builtin_bit_cast(v4i, sk[ks[1]]);
    const v4i qa0 = __builtin_bit_cast(v4i, qv[0]), qa1 = __builtin_bit_cast(v4i, qv[1]);
    v16i sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0;
    sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kx0, qa0, sacc, 0, 0, 0);
    sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kx1, qa1, sacc, 0, 0, 0);
    if constexpr (QK == QK_I8X2) {
      // scale the hi.hi partial (|hi.hi| <= 64*127*127 < 2^23, so a 24-bit multiply is
      // exact), then let the cross-term MFMAs accumulate on top of it
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = __mul24(sacc[r], 254);
      const v4i lx0 = __builtin_bit_cast(v4i, sk[256 + ks[0]]);
      const v4i lx1 = __builtin_bit_cast(v4i, sk[256 + ks[1]]);
      const v4i ql0 = __builtin_bit_cast(v4i, qv[2]), ql1 = __builtin_bit_cast(v4i, qv[3]);
      sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kx0, ql0, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kx1, ql1, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(lx0, qa0, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(lx1, qa1, sacc, 0, 0, 0);
    }
    if constexpr (MASK) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + 4 * g + (r & 3) >= nkt) sacc[r] = -2147483647 - 1;
    }
    int mx = max(sacc[0], sacc[1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) mx = max(mx, max(sacc[r], sacc[r + 1]));
    tmax = (float)mx;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = (float)sacc[r];
  }
}

// P = exp2(S*c - m) for one tile, row sum, O^T += V^T P^T (2 MFMAs per output half).
template <bool V_F16, bool MASK>
__device__ __forceinline__ void pv_tile(const uint4* __restrict__ sv, int t, int nkt, const float (&s)[16], float c,
                                        float nm, int g, int qi, float& l_run, v16f& o0, v16f& o1) {
  float p[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(fmaf(s[r], c, nm));
  if constexpr (MASK) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (8 * (r >> 2) + 4 * g + (r & 3) >= nkt) p[r] = 0.0f;
  }
  // MFMA s = 2t + h covers keys 16s..16s+15, registers 8h..8h+7. The row sum
  // accumulates the same rounded P the MFMA consumes.
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint4 pb;
    pb.x = cvt_pair<V_F16>(p[8 * h + 0], p[8 * h + 1]);
    pb.y = cvt_pair<V_F16>(p[8 * h + 2], p[8 * h + 3]);
    pb.z = cvt_pair<V_F16>(p[8 * h + 4], p[8 * h + 5]);
    pb.w = cvt_pair<V_F16>(p[8 * h + 6], p[8 * h + 7]);
    l_run = dot2_acc<V_F16>(pb.x, l_run);
    l_run = dot2_acc<V_F16>(pb.y, l_run);
    l_run = dot2_acc<V_F16>(pb.z, l_run);
    l_run = dot2_acc<V_F16>(pb.w, l_run);
    const int sidx = 2 * t + h;
    const uint4 va0 = sv[v_slot(qi, 2 * sidx + g)];
    const uint4 va1 = sv[v_slot(32 + qi, 2 * sidx + g)];
    o0 = pv_mfma<V_F16>(va0, pb, o0);
    o1 = pv_mfma<V_F16>(va1, pb, o1);
  }
}

// INT8 modes: one 64-key block as two 32-key online-softmax steps (S^T tile -> running
// max with lazy rescale -> P -> O^T += V^T P^T), one S accumulator live at a time.
template <int QK, bool V_F16, bool MASK>
__device__ __forceinline__ void attn_block_i8(const uint4* __restrict__ stage, int kch, int nk, float c,
                                              const int (&ks0)[4], const int (&ks1)[4], const uint4 (&qv)[4], int g,
                                              int qi, float& m_run, float& l_run, v16f& o0, v16f& o1) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float sc[16], tmax;
    qk_tile<QK, MASK>(stage, nk - 32 * t, t ? ks1 : ks0, qv, g, sc, tmax);
    const float bmax = (float)pair_max((int)tmax) * c;
    const bool need = bmax > m_run + RESS_RESCALE_LOG2;
    if (__any(need)) {
      const float m_new = need ? bmax : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        o0[r] *= alpha;
        o1[r] *= alpha;
      }
    }
    pv_tile<V_F16, MASK>(stage + kch, t, nk - 32 * t, sc, c, -m_run, g, qi, l_run, o0, o1);
  }
}

// 16-bit mode (QK_F16). K blocks are fp16 (exact for bf16 keys above the fp16 subnormal
// range); the row's queries are converted to fp16 in registers when the row starts. A row
// runs one of two ways, chosen per row (the same for every wave of the workgroup):
//  * bounded: Q' = fp16(q * sm_scale * log2 e). Every logit of the row (log2 units) lies
//    in [-m0, m0], m0 = |Q'| * (the largest key norm of the row's kept blocks). When
//    m0 <= RESS_BOUND_MAX, P = exp2(logit) itself is in [2^-64, 2^64]: no offset, no scale,
//    no row max, no rescale. The row sum and O = sum P v stay below 2^82 * max|v| (fp32
//    overflows at 2^128), and the largest P of the row is at least 2^-64.
//  * running max (rows whose m0 exceeds RESS_BOUND_MAX, or is not finite): Q = fp16(q),
//    exact, the scale folded into one fma per score and the lazy-rescale running max.
#define RESS_BOUND_MAX 64.0f

// P of one 32-key tile (16 scores per lane) -> l_run and O^T += V^T P^T (2 MFMAs per
// output half). MFMA s = 2t + h covers keys 16s..16s+15, registers 8h..8h+7; the row sum
// accumulates the same rounded P the MFMA consumes.
__device__ __forceinline__ void pv_tile_bf16(const float (&p)[16], const uint4 (&vv)[4], float& l_run, v16f& o0,
                                             v16f& o1) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint4 pb;
    pb.x = cvt_pair<false>(p[8 * h + 0], p[8 * h + 1]);
    pb.y = cvt_pair<false>(p[8 * h + 2], p[8 * h + 3]);
    pb.z = cvt_pair<false>(p[8 * h + 4], p[8 * h + 5]);
    pb.w = cvt_pair<false>(p[8 * h + 6], p[8 * h + 7]);
    l_run = dot2_acc<false>(pb.x, l_run);
    l_run = dot2_acc<false>(pb.y, l_run);
    l_run = dot2_acc<false>(pb.z, l_run);
    l_run = dot2_acc<false>(pb.w, l_run);
    o0 = pv_mfma<false>(vv[2 * h], pb, o0);
    o1 = pv_mfma<false>(vv[2 * h + 1], pb, o1);
  }
}

// K chunks (16 B) per stage of the INT8 modes: hi 256 [+ lo 256].
template <int QK>
struct StageShape {
  static_assert(QK != QK_F16, "the 16-bit mode runs attn_row_f16");
  static constexpr int KCH = QK == QK_I8 ? 256 : 512;
  static constexpr int STAGE = KCH + 512;  // + V^T 8 KiB
  static constexpr int DMA = QK == QK_I8 ? 3 : 4;  // LDS-DMA instructions per lane per stage
};

// Output of one finished row (query block qb of head bh) for the lane's query of query
// group w (queries 32w..32w+31): O / row sum, in the output dtype at the row's storage
// positions. o0/o1 hold O^T in the PV MFMA's register order.
template <int OUT>
__device__ __forceinline__ void store_row(const AttnArgs& a, int bh, int qb, const v16f& o0, const v16f& o1,
                                          float l_run, int w) {
  const int l = threadIdx.x & 63, g = l >> 5, qi = l & 31;
  const bool special = qb >= a.q_blk_p;
  const int qbase = special ? (qb - a.q_blk_p) * 128 : qb * 128;
  const int cnt_q = min(128, (special ? a.m.T_s : a.m.T_p) - qbase);
  const int qrow = 32 * w + qi;
  const float lt = pair_sum(l_run);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
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

// One row of the INT8 modes (query block qb of head bh) over its kept blocks
// kb_lo..kb_hi-1 (LUT positions). part_out null: the whole row, written to the output;
// otherwise one part of a split row, left in part_out for k_attn_merge.
template <int QK, bool V_F16, int OUT>
__device__ __forceinline__ void sparse_attn_row(const AttnArgs& a, const int* __restrict__ lut_all,
                                                const float* __restrict__ k_scale, uint4* __restrict__ s0,
                                                uint4* __restrict__ s1, uint4* __restrict__ s2, int bh, int qb,
                                                int kb_lo, int kb_hi, float* __restrict__ part_out) {
  constexpr int KCH = StageShape<QK>::KCH;
  constexpr int DMA = StageShape<QK>::DMA;
  const long long row = (long long)bh * a.q_blk_total + qb;
  const int nv = kb_hi - kb_lo;
  const int* lut = lut_all + row * a.kb_tot + kb_lo;
  // the wave index is wave-uniform: held in an SGPR, the LDS-DMA destinations (m0) are
  // scalar arithmetic
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, g = l >> 5, qi = l & 31;
  const bool special = qb >= a.q_blk_p;
  const int qbase = special ? (qb - a.q_blk_p) * 128 : qb * 128;
  const int cnt_q = min(128, (special ? a.m.T_s : a.m.T_p) - qbase);
  const int qrow = 32 * w + qi;

  uint4 qv[4];  // Q operand (see k_slots)
  {
    const int8_t* qsrc = a.q_i8 + (row * 128 + qrow) * 64 + 16 * g;
    qv[0] = *reinterpret_cast<const uint4*>(qsrc);
    qv[1] = *reinterpret_cast<const uint4*>(qsrc + 32);
    qv[2] = qv[0];
    qv[3] = qv[1];
    if constexpr (QK == QK_I8X2) {
      const int8_t* qlsrc = a.q_lo + (row * 128 + qrow) * 64 + 16 * g;
      qv[2] = *reinterpret_cast<const uint4*>(qlsrc);
      qv[3] = *reinterpret_cast<const uint4*>(qlsrc + 32);
    }
  }
  // this row's logit scale (times log2 e); the block's k_scale is multiplied in per block
  const float qs = a.q_scale[row] * a.sm_scale_log2e * (QK == QK_I8X2 ? (1.0f / 254.0f) : 1.0f);
  const float* ksc = k_scale + (long long)bh * a.kb_tot;
  auto block_scale = [&](int kb) -> float { return qs * ksc[kb]; };

  // Stage loads are LDS-DMA: lane l of wave w fills 16-byte slots 64w+l (K hi, K lo) and
  // 128w+l, 128w+64+l (V), so it fetches the global chunk that the swizzle places there
  // (the XOR swizzles are their own inverse), through the head's buffer descriptors.
  const unsigned kslot = 64 * w + l;
  const unsigned ksrc = 16 * (4 * (kslot >> 2) + ((kslot & 3) ^ ((((kslot >> 2) >> 1) ^ ((kslot >> 2) >> 3)) & 3)));
  const unsigned vslot0 = 128 * w + l, vslot1 = vslot0 + 64;
  const unsigned vsrc0 = 16 * (8 * (vslot0 >> 3) + ((vslot0 & 7) ^ (((vslot0 >> 3) ^ (vslot0 >> 6)) & 7)));
  const unsigned vsrc1 = 16 * (8 * (vslot1 >> 3) + ((vslot1 & 7) ^ (((vslot1 >> 3) ^ (vslot1 >> 6)) & 7)));
  const __amdgpu_buffer_rsrc_t krs =
      head_rsrc(reinterpret_cast<const char*>(a.k_i8) + (long long)bh * a.kb_tot * 4096, a.kb_tot * 4096);
  const __amdgpu_buffer_rsrc_t klrs =
      head_rsrc(QK == QK_I8X2 ? reinterpret_cast<const char*>(a.k_lo) + (long long)bh * a.kb_tot * 4096
                              : reinterpret_cast<const char*>(a.k_i8),
                QK == QK_I8X2 ? a.kb_tot * 4096 : 0);
  const __amdgpu_buffer_rsrc_t vrs =
      head_rsrc(reinterpret_cast<const char*>(a.v_pack) + (long long)bh * a.kb_tot * 8192, a.kb_tot * 8192);
  auto stage_load = [&](uint4* stage, int kb) {
    char* base = reinterpret_cast<char*>(stage);
    buf_lds16(krs, ksrc, kb * 4096, base + 1024 * w);
    if constexpr (QK == QK_I8X2) buf_lds16(klrs, ksrc, kb * 4096, base + 4096 + 1024 * w);
    buf_lds16(vrs, vsrc0, kb * 8192, base + 16 * KCH + 2048 * w);
    buf_lds16(vrs, vsrc1, kb * 8192, base + 16 * KCH + 2048 * w + 1024);
  };
  // LDS sources of this lane's K operands, per tile
  int ks0[4], ks1[4];
  k_slots<QK>(qi, g, ks0);
  k_slots<QK>(32 + qi, g, ks1);

  float m_run = -__builtin_huge_valf(), l_run = 0.0f;  // running max (log2 units), row sum
  v16f o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.0f;
  // Only the sequence's last key block can be partial; LUTs are ascending, so if it is
  // kept it is the last entry. Full blocks run unmasked, the partial one is peeled off.
  const bool tail_partial = nv > 0 && (a.Tk & 63) != 0 && lut[nv - 1] == a.kb_tot - 1;

  auto block = [&](const uint4* cur, int nk, float cb, auto mask_tag) {
    constexpr bool M = decltype(mask_tag)::value;
    attn_block_i8<QK, V_F16, M>(cur, KCH, nk, cb, ks0, ks1, qv, g, qi, m_run, l_run, o0, o1);
  };

  // Three stages: block i lives in stage i % 3 and is fetched two steps ahead, so each
  // DMA has two blocks of compute to land in.
  if (nv > 0) stage_load(s0, lut[0]);
  if (nv > 1) {
    stage_load(s1, lut[1]);
    wait_lds_dma_but<DMA>();
  } else {
    wait_lds_dma();
  }
  __syncthreads();

  // LUT entries are read two steps before their DMA is issued (kb1, kb2 = blocks it+1,
  // it+2 at the start of step it), so no step waits on a scalar load; the scale of the
  // next block is read one step ahead.
  int kb = nv > 0 ? lut[0] : 0;
  int kb1 = nv > 1 ? lut[1] : 0;
  int kb2 = nv > 2 ? lut[2] : 0;
  float c = nv > 0 ? block_scale(kb) : 0.0f;
  const int nv_full = nv - (tail_partial ? 1 : 0);

  // One kept block: start the DMA of block it+2 into `ahead`, consume `cur`, then wait
  // for block it+1 (the newest DMA may stay in flight). The stages are distinct LDS
  // objects and the loop is unrolled by three, so the compiler can see that no DMA
  // writes the stage being read and does not wait for it before the LDS reads. The
  // stage `ahead` was last read in step it-1, which every wave has left (barrier).
  auto step = [&](const uint4* cur, uint4* ahead, int it) {
    const bool fetch = it + 2 < nv;
    if (fetch) stage_load(ahead, kb2);
    const float cn = it + 1 < nv ? block_scale(kb1) : 0.0f;
    block(cur, 64, c, std::false_type{});
    // issued after the block's LDS reads, so their waits do not include this load
    __builtin_amdgcn_sched_barrier(0);
    const int kb3 = it + 3 < nv ? lut[it + 3] : 0;
    kb = kb1;
    kb1 = kb2;
    kb2 = kb3;
    c = cn;
    if (fetch) wait_lds_dma_but<DMA>();
    else wait_lds_dma();
    stage_barrier();
  };
  int it = 0;
  for (; it + 3 <= nv_full; it += 3) {
    step(s0, s2, it);
    step(s1, s0, it + 1);
    step(s2, s1, it + 2);
  }
  if (it < nv_full) step(s0, s2, it++);
  if (it < nv_full) step(s1, s0, it++);
  if (tail_partial) {  // kb / c already hold the last block's index and scale
    const int st = it % 3;
    const uint4* cur = st == 0 ? s0 : (st == 1 ? s1 : s2);
    const int nk = a.Tk - kb * 64;
    block(cur, nk, c, std::true_type{});
    __syncthreads();  // the next row's prologue overwrites this stage
  }

  // ---- epilogue ------------------------------------------------------------
  if (part_out) {  // unnormalised O, running max and row sum of this part, in register order
    float4* po = reinterpret_cast<float4*>(part_out);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      po[q * 256 + tid] = make_float4(o0[4 * q], o0[4 * q + 1], o0[4 * q + 2], o0[4 * q + 3]);
      po[(4 + q) * 256 + tid] = make_float4(o1[4 * q], o1[4 * q + 1], o1[4 * q + 2], o1[4 * q + 3]);
    }
    part_out[8192 + tid] = m_run;
    part_out[8448 + tid] = l_run;
    return;
  }
  store_row<OUT>(a, bh, qb, o0, o1, l_run, threadIdx.x >> 6);
}

// Resident workgroups per CU (= waves per SIMD) of the INT8 kernel.
#define RESS_I8_OCCUPANCY 3

template <int QK, bool V_F16, int OUT>
__global__ __launch_bounds__(256, RESS_I8_OCCUPANCY) void k_sparse_attn(AttnArgs a, const int* __restrict__ lut,
                                                        const int* __restrict__ nvalid,
                                                        const float* __restrict__ k_scale) {
  constexpr int STAGE = StageShape<QK>::STAGE;
  __shared__ __attribute__((aligned(16))) uint4 stage0[STAGE];
  __shared__ __attribute__((aligned(16))) uint4 stage1[STAGE];
  __shared__ __attribute__((aligned(16))) uint4 stage2[STAGE];
  __shared__ int s_item;

  // ---- persistent loop over this XCD's range of rows ------------------------
  // positions b0 .. full_end-1 are whole rows; the last Lx rows of the range follow as
  // RESS_SPLIT_PARTS consecutive positions each (part s of row j at full_end + S*j + s)
  const int xcd = blockIdx.x & 7;
  const int b1 = a.sched[xcd + 1];
  const int Lx = min(a.split_L, b1 - a.sched[xcd]);
  const int full_end = b1 - Lx;
  const int item_end = full_end + Lx * RESS_SPLIT_PARTS;
  for (;;) {
    if (threadIdx.x == 0) s_item = atomicAdd(&a.sched[16 + xcd], 1);
    __syncthreads();
    const int pos = __builtin_amdgcn_readfirstlane(s_item);
    __syncthreads();
    if (pos >= item_end) break;
    int bh, qb;
    if (pos < full_end) {
      item_to_row(pos, a.BH, a.q_blk_p, a.q_blk_total, a.chunks, bh, qb);
      const int nv = nvalid[(long long)bh * a.q_blk_total + qb];
      sparse_attn_row<QK, V_F16, OUT>(a, lut, k_scale, stage0, stage1, stage2, bh, qb, 0, nv, nullptr);
    } else {
      const int j = (pos - full_end) / RESS_SPLIT_PARTS, part = pos - full_end - j * RESS_SPLIT_PARTS;
      item_to_row(full_end + j, a.BH, a.q_blk_p, a.q_blk_total, a.chunks, bh, qb);
      const int nv = nvalid[(long long)bh * a.q_blk_total + qb];
      float* slot = a.part + ((long long)(xcd * a.split_L + j) * RESS_SPLIT_PARTS + part) * RESS_PART_FLOATS;
      sparse_attn_row<QK, V_F16, OUT>(a, lut, k_scale, stage0, stage1, stage2, bh, qb, nv * part / RESS_SPLIT_PARTS,
                                      nv * (part + 1) / RESS_SPLIT_PARTS, slot);
    }
  }
}

// ---- 16-bit mode: eight waves per row ---------------------------------------------------
// Wave w takes the 32 queries 32*(w>>1).. of the row (query group) and the 32 keys
// 32*(w&1).. of every kept block (key half), with its own (m, l, O); when the row ends the
// two key halves of each query group are merged through LDS. With 64 KiB of LDS stages and
// at most 128 VGPRs a workgroup, two workgroups share a CU: four waves per SIMD, so one
// wave's LDS and MFMA latencies are covered by three others. K/V go through four LDS stages
// filled by LDS-DMA three blocks ahead (each wave moves 2 of the 32 16-byte chunks a lane
// moves per stage).
#define RESS_F16_WAVES 8
#define RESS_F16_STAGE 1024  // 16-byte chunks per stage: K block 512, V^T block 512

// S^T (32 keys x 32 queries) of this wave's key half: 4 MFMAs over the 64 dims. The four K
// operand reads go out before the first MFMA.
__device__ __forceinline__ v16f qk_half_f16(const uint4* __restrict__ stage, const int (&kofs)[4],
                                            const uint4 (&qv)[4]) {
  uint4 k[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) k[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(stage) + kofs[j]);
  __builtin_amdgcn_sched_barrier(0);
  v16f z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.0f;
  v16f acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, k[0]), __builtin_bit_cast(v8h, qv[0]), z, 0,
                                                    0, 0);
#pragma unroll
  for (int j = 1; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, k[j]), __builtin_bit_cast(v8h, qv[j]), acc, 0,
                                                 0, 0);
  return acc;
}

// Softmax and PV of one key half (32 keys, 16 scores per lane; register r is key
// 32*kh + 8(r/4) + 4g + r%4 of the block). BD: bounded row, P = exp2(S); otherwise the
// running max with lazy rescale and P = exp2(S*c - m). nk = valid keys of the block (MASK).
template <bool BD, bool MASK>
__device__ __forceinline__ void sv_half(const uint4* __restrict__ stage, const int (&vofs)[4], int kh, int nk, float c,
                                        const v16f& sacc, int g, float& m_run, float& l_run, v16f& o0, v16f& o1) {
  uint4 vv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) vv[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(stage) + vofs[j]);
  float x[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    x[r] = sacc[r];
    if constexpr (MASK) {
      if (32 * kh + 8 * (r >> 2) + 4 * g + (r & 3) >= nk) x[r] = -__builtin_huge_valf();
    }
  }
  float p[16];
  if constexpr (BD) {
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(x[r]);
  } else {
    float ma = fmaxf(fmaxf(x[0], x[1]), x[2]), mb = fmaxf(fmaxf(x[8], x[9]), x[10]);
    ma = fmaxf(fmaxf(ma, x[3]), x[4]);
    mb = fmaxf(fmaxf(mb, x[11]), x[12]);
    ma = fmaxf(fmaxf(ma, x[5]), x[6]);
    mb = fmaxf(fmaxf(mb, x[13]), x[14]);
    ma = fmaxf(fmaxf(ma, x[7]), mb);
    const float bmax = pair_maxf(fmaxf(ma, x[15])) * c;
    const bool need = bmax > m_run + RESS_RESCALE_LOG2;
    if (__any(need)) {
      const float m_new = need ? bmax : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        o0[r] *= alpha;
        o1[r] *= alpha;
      }
    }
    const float nm = -m_run;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(fmaf(x[r], c, nm));
  }
  pv_tile_bf16(p, vv, l_run, o0, o1);
}

// One row (query block qb of head bh) over its kept blocks kb_lo..kb_hi-1 (LUT positions),
// 16-bit operands, 512 threads. part_out null: the whole row, written to the output;
// otherwise one part of a split row, left in part_out for k_attn_merge (written by the
// even waves, query group qg at threads 64*qg + lane of the 256-thread part layout).
template <int OUT>
__device__ __forceinline__ void attn_row_f16(const AttnArgs& a, const int* __restrict__ lut_all,
                                             const int* __restrict__ nvalid_all, uint4* __restrict__ s0,
                                             uint4* __restrict__ s1, uint4* __restrict__ s2, uint4* __restrict__ s3,
                                             int* __restrict__ vote, int bh, int qb, int kb_lo, int kb_hi,
                                             float* __restrict__ part_out) {
  constexpr int DMA = 2;  // LDS-DMA instructions per lane per stage
  const long long row = (long long)bh * a.q_blk_total + qb;
  const int nv = kb_hi - kb_lo;
  const int* lut = lut_all + row * a.kb_tot + kb_lo;
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, g = l >> 5, qi = l & 31;
  const int qg = w >> 1, kh = w & 1;
  const bool special = qb >= a.q_blk_p;
  const int qbase = special ? (qb - a.q_blk_p) * 128 : qb * 128;
  const int cnt_q = min(128, (special ? a.m.T_s : a.m.T_p) - qbase);
  const int qrow = 32 * qg + qi;

  // ---- Q operand (dims 16j+8g..16j+8g+7 of the lane's query) and the row's path -------
  uint4 qraw[4], qv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) qraw[j] = make_uint4(0u, 0u, 0u, 0u);
  if (qrow < cnt_q) {
    const int tok = special ? special_to_storage(qbase + qrow, a.m) : patch_to_storage(qbase + qrow, a.m);
    const uint16_t* src =
        a.q_bf + (long long)(bh / a.H) * a.sqB + (long long)(bh % a.H) * a.sqH + (long long)tok * a.sqT + 8 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) qraw[j] = *reinterpret_cast<const uint4*>(src + 16 * j);
  }
  const float c = a.sm_scale_log2e;
  float qq = 0.0f;  // |Q'|^2 over this lane's 32 dims, Q' = fp16(q * c)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float x[8];
    unpack_bf16x8(qraw[j], x);
    uint32_t w4[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const _Float16 h0 = (_Float16)(x[2 * cc] * c), h1 = (_Float16)(x[2 * cc + 1] * c);
      const float f0 = (float)h0, f1 = (float)h1;
      qq = fmaf(f0, f0, qq);
      qq = fmaf(f1, f1, qq);
      w4[cc] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    }
    qv[j] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
  // the largest key norm over the whole row's kept blocks (every part of a split row sees
  // the same bound), times |Q'|: the row's logit bound in log2 units
  {
    const int* lut_row = lut_all + row * a.kb_tot;
    const int nv_row = nvalid_all[row];
    const float* kn = a.k_norm + (long long)bh * a.kb_tot;
    float kmax = 0.0f;
    for (int i = l; i < nv_row; i += 64) kmax = fmaxf(kmax, kn[lut_row[i]]);
    kmax = wave_max(kmax);
    const float m0 = sqrtf(pair_sum(qq)) * kmax;
    // the vote runs with every lane active (each lane pair holds one query of the wave's
    // 32); NaN fails the test
    const int over = __any(!(m0 <= RESS_BOUND_MAX)) ? 1 : 0;
    if (l == 0) vote[w] = over;
    // operands fp16 cannot hold (|x| >= 65520): an infinite key norm (prep's marker) or a
    // query element; the row's result is not meaningful and the caller is told so
    bool q_over = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x[8];
      unpack_bf16x8(qraw[j], x);
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) q_over |= !(fabsf(x[cc]) < 65520.0f);
    }
    const int bad = (!(kmax < __builtin_huge_valf()) ? RESS_F16_KEY_RANGE : 0) | (__any(q_over) ? RESS_F16_QUERY_RANGE : 0);
    if (bad && l == 0) atomicOr(&a.sched[24], bad);
  }
  __syncthreads();
  int any_over = 0;
#pragma unroll
  for (int i = 0; i < RESS_F16_WAVES; ++i) any_over |= vote[i];
  const bool bounded = __builtin_amdgcn_readfirstlane(any_over) == 0;  // the same in every lane
  if (!bounded) {  // running-max row: the exact fp16 queries, the scale applied per score
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x[8];
      unpack_bf16x8(qraw[j], x);
      qv[j] = make_uint4(f32x2_to_f16_bits(x[0], x[1]), f32x2_to_f16_bits(x[2], x[3]), f32x2_to_f16_bits(x[4], x[5]),
                         f32x2_to_f16_bits(x[6], x[7]));
    }
  }

  // ---- stage loads: lane l of wave w fills 16-byte slot 64w+l of the K block and of the V^T
  // block, fetching the chunk the XOR swizzle places there (its own inverse)
  const unsigned slot = 64 * w + l;
  const unsigned src = 16 * (8 * (slot >> 3) + ((slot & 7) ^ (((slot >> 3) ^ (slot >> 6)) & 7)));
  const __amdgpu_buffer_rsrc_t krs =
      head_rsrc(reinterpret_cast<const char*>(a.k_pack) + (long long)bh * a.kb_tot * 8192, a.kb_tot * 8192);
  const __amdgpu_buffer_rsrc_t vrs =
      head_rsrc(reinterpret_cast<const char*>(a.v_pack) + (long long)bh * a.kb_tot * 8192, a.kb_tot * 8192);
  auto stage_load = [&](uint4* stage, int kb) {
    char* base = reinterpret_cast<char*>(stage) + 1024 * w;
    buf_lds16(krs, src, kb * 8192, base);
    buf_lds16(vrs, src, kb * 8192, base + 8192);
  };
  // LDS byte offsets of this lane's operands within a stage: K chunk 2j+g of key 32kh+qi;
  // V^T chunks 4kh+2h+g of dims qi and 32+qi (the V^T block starts 8 KiB into the stage)
  int kofs[4], vofs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kofs[j] = 16 * v_slot(32 * kh + qi, 2 * j + g);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    vofs[2 * h] = 8192 + 16 * v_slot(qi, 4 * kh + 2 * h + g);
    vofs[2 * h + 1] = 8192 + 16 * v_slot(32 + qi, 4 * kh + 2 * h + g);
  }

  float m_run = bounded ? 0.0f : -__builtin_huge_valf(), l_run = 0.0f;
  v16f o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.0f;
  // only the sequence's last key block can be partial; LUTs are ascending, so if it is kept
  // it is the last entry, which runs masked after the loop
  const bool tail_partial = nv > 0 && (a.Tk & 63) != 0 && lut[nv - 1] == a.kb_tot - 1;

  auto run = [&](auto bounded_tag) {
    constexpr bool BD = decltype(bounded_tag)::value;
    // Block i lives in stage i % 4. Step i issues the DMA of block i+3 into the stage block
    // i-1 used, computes block i, and waits for block i+1 (blocks i+2, i+3 may stay in
    // flight). The loop is unrolled by four over distinct LDS arrays, so the compiler sees
    // that no DMA writes a stage being read.
    if (nv > 0) stage_load(s0, lut[0]);
    if (nv > 1) stage_load(s1, lut[1]);
    if (nv > 2) stage_load(s2, lut[2]);
    if (nv > 2) wait_lds_dma_but<2 * DMA>();
    else if (nv > 1) wait_lds_dma_but<DMA>();
    else wait_lds_dma();
    __syncthreads();
    int kb3 = nv > 3 ? lut[3] : 0;
    auto block = [&](const uint4* cur, int nk, auto mask_tag) {
      constexpr bool MK = decltype(mask_tag)::value;
      // the lane's byte offsets pass through an empty asm every block: the compiler then
      // adds the stage's address as the ds_read immediate instead of keeping one set of
      // offsets per stage live, which would not fit the 128 VGPRs
      asm volatile("" : "+v"(kofs[0]), "+v"(kofs[1]), "+v"(kofs[2]), "+v"(kofs[3]), "+v"(vofs[0]), "+v"(vofs[1]),
                   "+v"(vofs[2]), "+v"(vofs[3]));
      const v16f sacc = qk_half_f16(cur, kofs, qv);
      sv_half<BD, MK>(cur, vofs, kh, nk, c, sacc, g, m_run, l_run, o0, o1);
    };
    auto step = [&](const uint4* cur, uint4* ahead, int it) {
      const bool fetch = it + 3 < nv;
      const int kb4 = it + 4 < nv ? lut[it + 4] : 0;
      if (fetch) stage_load(ahead, kb3);
      block(cur, 64, std::false_type{});
      kb3 = kb4;
      if (fetch) wait_lds_dma_but<2 * DMA>();
      else if (it + 2 < nv) wait_lds_dma_but<DMA>();
      else wait_lds_dma();
      stage_barrier();
    };
    const int last = nv - 1;  // the final block runs after the loop (masked if partial)
    int it = 0;
    for (; it + 4 <= last; it += 4) {
      step(s0, s3, it);
      step(s1, s0, it + 1);
      step(s2, s1, it + 2);
      step(s3, s2, it + 3);
    }
    if (it < last) step(s0, s3, it++);
    if (it < last) step(s1, s0, it++);
    if (it < last) step(s2, s1, it++);
    if (nv > 0) {
      const int st = it & 3;
      const uint4* cur = st == 0 ? s0 : (st == 1 ? s1 : (st == 2 ? s2 : s3));
      if (tail_partial) block(cur, a.Tk - lut[last] * 64, std::true_type{});
      else block(cur, 64, std::false_type{});
    }
  };
  if (bounded) run(std::true_type{});
  else run(std::false_type{});

  // ---- merge the two key halves of each query group through LDS (the stages are free once
  // every wave has read its last block); the even wave of a group finishes the row
  __syncthreads();
  float* xs = reinterpret_cast<float*>(qg == 0 ? s0 : (qg == 1 ? s1 : (qg == 2 ? s2 : s3)));
  if (kh == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      xs[r * 64 + l] = o0[r];
      xs[(16 + r) * 64 + l] = o1[r];
    }
    xs[32 * 64 + l] = m_run;
    xs[33 * 64 + l] = l_run;
  }
  __syncthreads();
  if (kh == 0) {
    const float mo = xs[32 * 64 + l], lo = xs[33 * 64 + l];
    const float mm = fmaxf(m_run, mo);
    const float fe = m_run == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(m_run - mm);
    const float fo = mo == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(mo - mm);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o0[r] = fmaf(fo, xs[r * 64 + l], o0[r] * fe);
      o1[r] = fmaf(fo, xs[(16 + r) * 64 + l], o1[r] * fe);
    }
    m_run = mm;
    l_run = fmaf(fo, lo, l_run * fe);
    if (part_out) {  // unnormalised O, running max and row sum of this part, in register order
      const int t4 = 64 * qg + l;
      float4* po = reinterpret_cast<float4*>(part_out);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        po[q * 256 + t4] = make_float4(o0[4 * q], o0[4 * q + 1], o0[4 * q + 2], o0[4 * q + 3]);
        po[(4 + q) * 256 + t4] = make_float4(o1[4 * q], o1[4 * q + 1], o1[4 * q + 2], o1[4 * q + 3]);
      }
      part_out[8192 + t4] = m_run;
      part_out[8448 + t4] = l_run;
    } else {
      store_row<OUT>(a, bh, qb, o0, o1, l_run, qg);
    }
  }
  __syncthreads();  // the next row's prologue overwrites the stages
}

// The persistent 16-bit kernel: the row loop of k_sparse_attn with eight waves per row.
template <int OUT>
__global__ __launch_bounds__(512, 4) void k_sparse_attn_f16(AttnArgs a, const int* __restrict__ lut,
                                                            const int* __restrict__ nvalid) {
  __shared__ __attribute__((aligned(16))) uint4 stage0[RESS_F16_STAGE];
  __shared__ __attribute__((aligned(16))) uint4 stage1[RESS_F16_STAGE];
  __shared__ __attribute__((aligned(16))) uint4 stage2[RESS_F16_STAGE];
  __shared__ __attribute__((aligned(16))) uint4 stage3[RESS_F16_STAGE];
  __shared__ int s_item;
  __shared__ int s_vote[RESS_F16_WAVES];
  const int xcd = blockIdx.x & 7;
  const int b1 = a.sched[xcd + 1];
  const int Lx = min(a.split_L, b1 - a.sched[xcd]);
  const int full_end = b1 - Lx;
  const int item_end = full_end + Lx * RESS_SPLIT_PARTS;
  for (;;) {
    if (threadIdx.x == 0) s_item = atomicAdd(&a.sched[16 + xcd], 1);
    __syncthreads();
    const int pos = __builtin_amdgcn_readfirstlane(s_item);
    __syncthreads();
    if (pos >= item_end) break;
    // a whole row, or part `part` of split row j (one call site: one inlined copy of the row)
    const bool split = pos >= full_end;
    const int j = split ? (pos - full_end) / RESS_SPLIT_PARTS : 0;
    const int part = split ? pos - full_end - j * RESS_SPLIT_PARTS : 0;
    int bh, qb;
    item_to_row(split ? full_end + j : pos, a.BH, a.q_blk_p, a.q_blk_total, a.chunks, bh, qb);
    const int nv = nvalid[(long long)bh * a.q_blk_total + qb];
    float* slot =
        split ? a.part + ((long long)(xcd * a.split_L + j) * RESS_SPLIT_PARTS + part) * RESS_PART_FLOATS : nullptr;
    const int lo = split ? nv * part / RESS_SPLIT_PARTS : 0;
    const int hi = split ? nv * (part + 1) / RESS_SPLIT_PARTS : nv;
    attn_row_f16<OUT>(a, lut, nvalid, stage0, stage1, stage2, stage3, s_vote, bh, qb, lo, hi, slot);
  }
}

// The split rows: combine the parts' (O, m, l) (m in log2 units; an empty part has
// m = -inf, l = 0, O = 0) and write the row. One workgroup per slot (XCD range x, row j).
template <int OUT>
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a) {
  const int L = a.split_L, slot = blockIdx.x, x = slot / L, j = slot - x * L;
  const int b1 = a.sched[x + 1];
  const int Lx = min(L, b1 - a.sched[x]);
  if (j >= Lx) return;
  int bh, qb;
  item_to_row(b1 - Lx + j, a.BH, a.q_blk_p, a.q_blk_total, a.chunks, bh, qb);
  const int tid = threadIdx.x;
  const float* base = a.part + (long long)slot * RESS_SPLIT_PARTS * RESS_PART_FLOATS;
  float m = -__builtin_huge_valf();
#pragma unroll
  for (int s = 0; s < RESS_SPLIT_PARTS; ++s) m = fmaxf(m, base[s * RESS_PART_FLOATS + 8192 + tid]);
  v16f o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.0f;
  float l_run = 0.0f;
#pragma unroll
  for (int s = 0; s < RESS_SPLIT_PARTS; ++s) {
    const float* ps = base + s * RESS_PART_FLOATS;
    const float ms = ps[8192 + tid];
    const float f = ms == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(ms - m);
    l_run = fmaf(f, ps[8448 + tid], l_run);
    const float4* po = reinterpret_cast<const float4*>(ps);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 u = po[q * 256 + tid], v = po[(4 + q) * 256 + tid];
      o0[4 * q] = fmaf(f, u.x, o0[4 * q]);
      o0[4 * q + 1] = fmaf(f, u.y, o0[4 * q + 1]);
      o0[4 * q + 2] = fmaf(f, u.z, o0[4 * q + 2]);
      o0[4 * q + 3] = fmaf(f, u.w, o0[4 * q + 3]);
      o1[4 * q] = fmaf(f, v.x, o1[4 * q]);
      o1[4 * q + 1] = fmaf(f, v.y, o1[4 * q + 1]);
      o1[4 * q + 2] = fmaf(f, v.z, o1[4 * q + 2]);
      o1[4 * q + 3] = fmaf(f, v.w, o1[4 * q + 3]);
    }
  }
  store_row<OUT>(a, bh, qb, o0, o1, l_run, tid >> 6);
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
static int g_cu_count[64];

template <int QK, bool V_F16>
static int launch_attn(const AttnArgs& a, int out_dtype, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (g_cu_count[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    g_cu_count[dev] = cus;
  }
  hipLaunchKernelGGL(k_attn_schedule, dim3(1), dim3(1024), 0, stream, a.nvalid, a.BH, a.q_blk_p, a.q_blk_total,
                     a.chunks, a.sched);
  RESS_LAUNCHED("k_attn_schedule");
  const dim3 block(256);
  if constexpr (QK == QK_F16) {
    // persistent: two 512-thread workgroups per CU, a multiple of the 8 XCDs
    const dim3 grid(8 * ((2 * g_cu_count[dev] + 7) / 8)), fblock(64 * RESS_F16_WAVES);
    switch (out_dtype) {
      case OUT_F32:
        hipLaunchKernelGGL(k_sparse_attn_f16<OUT_F32>, grid, fblock, 0, stream, a, a.lut, a.nvalid);
        break;
      case OUT_BF16:
        hipLaunchKernelGGL(k_sparse_attn_f16<OUT_BF16>, grid, fblock, 0, stream, a, a.lut, a.nvalid);
        break;
      default:
        hipLaunchKernelGGL(k_sparse_attn_f16<OUT_F16>, grid, fblock, 0, stream, a, a.lut, a.nvalid);
        break;
    }
    RESS_LAUNCHED("k_sparse_attn_f16");
  } else {
    // persistent: RESS_I8_OCCUPANCY resident workgroups per CU, a multiple of the 8 XCDs
    const dim3 grid(8 * ((RESS_I8_OCCUPANCY * g_cu_count[dev] + 7) / 8));
    switch (out_dtype) {
      case OUT_F32:
        hipLaunchKernelGGL((k_sparse_attn<QK, V_F16, OUT_F32>), grid, block, 0, stream, a, a.lut, a.nvalid, a.k_scale);
        break;
      case OUT_BF16:
        hipLaunchKernelGGL((k_sparse_attn<QK, V_F16, OUT_BF16>), grid, block, 0, stream, a, a.lut, a.nvalid, a.k_scale);
        break;
      default:
        hipLaunchKernelGGL((k_sparse_attn<QK, V_F16, OUT_F16>), grid, block, 0, stream, a, a.lut, a.nvalid, a.k_scale);
        break;
    }
    RESS_LAUNCHED("k_sparse_attn");
  }
  const dim3 mgrid(8 * a.split_L);
  switch (out_dtype) {
    case OUT_F32:
      hipLaunchKernelGGL(k_attn_merge<OUT_F32>, mgrid, block, 0, stream, a);
      break;
    case OUT_BF16:
      hipLaunchKernelGGL(k_attn_merge<OUT_BF16>, mgrid, block, 0, stream, a);
      break;
    default:
      hipLaunchKernelGGL(k_attn_merge<OUT_F16>, mgrid, block, 0, stream, a);
      break;
  }
  RESS_LAUNCHED("k_attn_merge");
  return 0;
}

// rows split at the end of each XCD's range for n rows in all (at most one range's worth)
static int split_rows(long long n) { return (int)(n < RESS_SPLIT_ROWS ? n : RESS_SPLIT_ROWS); }

static bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Shared argument checks and fields; the QK operands are filled in by the caller.
static int attn_args(AttnArgs& a, const void* v_pack, const void* lut, const void* nvalid, int B, int H, TokenMap m,
                     int Tk, float sm_scale, void* out, int out_dtype, long long soB, long long soH, long long soT,
                     void* sched) {
  RESS_REQUIRE(v_pack && lut && nvalid && out && sched, "sparse attention: null pointer");
  RESS_REQUIRE(al16(v_pack) && al16(sched), "sparse attention: v_pack and sched must be 16-byte aligned");
  RESS_REQUIRE(out_dtype >= 0 && out_dtype <= 2, "sparse attention: out_dtype must be 0 (f32), 1 (bf16) or 2 (f16)");
  const int align = out_dtype == OUT_F32 ? 16 : 8;
  RESS_REQUIRE(((uintptr_t)out % align) == 0 && soT % 4 == 0 && soH % 4 == 0 && soB % 4 == 0,
               "sparse attention: output must be %d-byte aligned with strides a multiple of 4", align);
  a = AttnArgs{};
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
  // the kernels address a head's blocks (8 KiB each) through buffer descriptors with a
  // 32-bit size and scalar byte offsets
  RESS_REQUIRE((long long)a.kb_tot * 8192 <= 0x7fffffffLL,
               "sparse attention: %d key blocks per head exceed the 2 GiB a head's K/V blocks may span", a.kb_tot);
  a.Tk = Tk;
  a.sm_scale_log2e = sm_scale * 1.4426950408889634f;
  a.sched = (int*)sched;
  a.split_L = split_rows((long long)a.BH * a.q_blk_total);
  // chunk-major rows when the heads' K/V (16 KiB per key block in the 16-bit layout) exceeds
  // what the memory-side cache holds: measured 3.8% faster at 200 frames (1.1 GB), slower
  // at 16 and 64 frames (88 / 352 MB)
  a.chunks = (long long)a.BH * a.kb_tot * 16384 > RESS_CHUNK_MIN_KV ? RESS_ROW_CHUNKS : 1;
  a.part = reinterpret_cast<float*>(reinterpret_cast<char*>(sched) + RESS_SCHED_HDR_BYTES);
  a.m = m;
  return 0;
}

static int attn_common(const void* q_i8, const void* q_lo, const void* q_scale, const void* k_i8, const void* k_lo,
                       const void* k_scale, const void* v_pack, int v_f16, const void* lut, const void* nvalid, int B,
                       int H, TokenMap m, int Tk, float sm_scale, void* out, int out_dtype, long long soB,
                       long long soH, long long soT, void* sched, hipStream_t stream) {
  RESS_REQUIRE(q_i8 && q_scale && k_i8 && k_scale, "sparse attention: null pointer");
  RESS_REQUIRE((q_lo == nullptr) == (k_lo == nullptr), "sparse attention: give both q_lo and k_lo, or neither");
  RESS_REQUIRE(al16(q_i8) && al16(k_i8) && al16(q_lo) && al16(k_lo),
               "sparse attention: q_i8/q_lo/k_i8/k_lo must be 16-byte aligned");
  AttnArgs a;
  if (attn_args(a, v_pack, lut, nvalid, B, H, m, Tk, sm_scale, out, out_dtype, soB, soH, soT, sched)) return -1;
  a.q_i8 = (const int8_t*)q_i8;
  a.q_lo = (const int8_t*)q_lo;
  a.k_lo = (const int8_t*)k_lo;
  a.q_scale = (const float*)q_scale;
  a.k_i8 = (const int8_t*)k_i8;
  a.k_scale = (const float*)k_scale;
  if (q_lo)
    return v_f16 ? launch_attn<QK_I8X2, true>(a, out_dtype, stream) : launch_attn<QK_I8X2, false>(a, out_dtype, stream);
  return v_f16 ? launch_attn<QK_I8, true>(a, out_dtype, stream) : launch_attn<QK_I8, false>(a, out_dtype, stream);
}

static TokenMap layer_map(int frames, int P, int S, const int* perm) {
  TokenMap m;
  m.P = P;
  m.S = S;
  m.HW = P - S;
  m.T_p = frames * (P - S);
  m.T_s = frames * S;
  m.perm = perm;
  return m;
}

// Fused-path attention over the ReSS token split: queries are the patch tokens
// (q-blocks 0..ceil(T_p/128)-1, sparse LUT rows) then the special tokens (dense
// rows); keys are cat(patch, special). The output is written in storage order
// (B,H,frames*P,64) with element strides soB/soH/soT, i.e. the reference's
// combine_special_and_patch (src/ress/models/qkv.py:71-81) is fused in. With q_lo/k_lo
// (split-INT8 residual codes from ress_prep_qkv) QK^T is evaluated as a two-term INT8
// product; without them it is the single-term per-block INT8 product of the reference.
// sched: ress_attn_sched_bytes(B, H, frames*P) bytes of 16-byte aligned device workspace.
// patch_order: the table given to ress_prep_qkv (or null), so rows are read and written at
// the storage positions of the patch order the blocks were formed in.
RESS_API int ress_sparse_attn_fwd(const void* q_i8, const void* q_lo, const void* q_scale, const void* k_i8,
                                  const void* k_lo, const void* k_scale, const void* v_pack, int v_f16, const void* lut,
                                  const void* nvalid, int B, int H, int frames, int P, int S, const int* patch_order,
                                  float sm_scale, void* out,
                                  int out_dtype, long long soB, long long soH, long long soT, void* sched,
                                  hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && frames > 0 && P > S && S >= 0, "ress_sparse_attn_fwd: bad geometry");
  return attn_common(q_i8, q_lo, q_scale, k_i8, k_lo, k_scale, v_pack, v_f16, lut, nvalid, B, H,
                     layer_map(frames, P, S, patch_order), frames * P, sm_scale, out, out_dtype, soB, soH, soT, sched,
                     stream);
}

// The same fused-path attention with QK^T on 16-bit operands (fp32 accumulation): q is
// the layer's bf16 query tensor (B,H,frames*P,64) in storage order with element strides
// sqB/sqH/sqT, converted to fp16 per row in registers; k_pack the fp16 key blocks and
// k_norm the per-block largest key norms ress_prep_qkv writes (16-bit operands), v_pack
// its packed bf16 V. A row whose logit bound |q'| * max key norm is at most
// RESS_BOUND_MAX for every query runs with pre-scaled fp16 queries, P = exp2(logit) (no offset, no running max);
// other rows use exact fp16 queries and the running max (see attn_row_f16). patch_order:
// as for ress_sparse_attn_fwd.
RESS_API int ress_sparse_attn_fwd_f16(const void* q, long long sqB, long long sqH, long long sqT, const void* k_pack,
                                      const void* k_norm, const void* v_pack, const void* lut, const void* nvalid,
                                      int B, int H, int frames, int P, int S, const int* patch_order, float sm_scale,
                                      void* out,
                                      int out_dtype, long long soB, long long soH, long long soT, void* sched,
                                      hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && frames > 0 && P > S && S >= 0, "ress_sparse_attn_fwd_f16: bad geometry");
  RESS_REQUIRE(q && k_pack && k_norm, "ress_sparse_attn_fwd_f16: null pointer");
  RESS_REQUIRE(al16(q) && al16(k_pack) && sqT % 8 == 0 && sqH % 8 == 0 && sqB % 8 == 0,
               "ress_sparse_attn_fwd_f16: q/k_pack must be 16-byte aligned, q strides a multiple of 8");
  AttnArgs a;
  if (attn_args(a, v_pack, lut, nvalid, B, H, layer_map(frames, P, S, patch_order), frames * P, sm_scale, out,
                out_dtype, soB, soH, soT, sched))
    return -1;
  a.q_bf = (const uint16_t*)q;
  a.sqB = sqB;
  a.sqH = sqH;
  a.sqT = sqT;
  a.k_pack = (const uint16_t*)k_pack;
  a.k_norm = (const float*)k_norm;
  return launch_attn<QK_F16, false>(a, out_dtype, stream);
}

static long long qattn_vpack_bytes(int B, int H, int Tk) { return (long long)B * H * cdiv(Tk, 64) * 4096 * 2; }
// Mirror workspace: [status 256 B][packed V][checked LUT][checked nvalid][row schedule], each
// part 256-byte aligned.
static long long round256(long long x) { return (x + 255) / 256 * 256; }
static long long qattn_lut_bytes(int B, int H, int Tq, int Tk) {
  return round256((long long)B * H * cdiv(Tq, 128) * cdiv(Tk, 64) * 4);
}
static long long qattn_nv_bytes(int B, int H, int Tq) { return round256((long long)B * H * cdiv(Tq, 128) * 4); }

// Status bits of the SpargeAttn mirror (word 0 of its workspace), set on the device.
#define RESS_QATTN_BAD_NVALID 1    // a valid_block_num outside [0, ceil(Tk/64)]
#define RESS_QATTN_BAD_LUT 2       // a listed block outside [0, ceil(Tk/64)) or not strictly ascending
#define RESS_QATTN_PV_THRESHOLD 4  // a pv_threshold below 1e9 (PV skipping is not implemented)

__global__ void k_qattn_status_clear(int* status) {
  if (threadIdx.x == 0) status[0] = 0;
}

// Checks one (batch*head, q-block) row of a caller-supplied LUT and copies it clamped into
// range (listed blocks to [0, nk), the count to [0, nk]), so the attention kernel reads in
// bounds whatever the caller passed; what was wrong is OR-ed into *status for the host to
// report. One wave per row.
__global__ __launch_bounds__(64) void k_qattn_check(const int* __restrict__ lut, const int* __restrict__ nvalid,
                                                    const float* __restrict__ pv_threshold, int H, int nq, int nk,
                                                    int* __restrict__ lut_out, int* __restrict__ nv_out,
                                                    int* __restrict__ status) {
  const int qb = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  const long long row = (long long)bh * nq + qb;
  const int nv = nvalid[row];
  const int nvc = min(max(nv, 0), nk);
  int bad = (nv < 0 || nv > nk) ? RESS_QATTN_BAD_NVALID : 0;
  const float thr = pv_threshold ? pv_threshold[bh % H] : 1e10f;
  if (!(thr >= 1e9f)) bad |= RESS_QATTN_PV_THRESHOLD;  // NaN included
  const int* src = lut + row * nk;
  int* dst = lut_out + row * nk;
  bool lut_bad = false;
  for (int i = lane; i < nk; i += 64) {
    const int e = src[i];
    dst[i] = min(max(e, 0), nk - 1);
    if (i < nvc) lut_bad |= e < 0 || e >= nk || (i > 0 && e <= src[i - 1]);
  }
  if (__any(lut_bad)) bad |= RESS_QATTN_BAD_LUT;
  if (lane == 0) {
    nv_out[row] = nvc;
    if (bad) atomicOr(status, bad);
  }
}

// Workspace of the attention entry points for B*H heads of Tq query rows: the row
// schedule (header) and the parts of the rows split at the end of each XCD's range
// (at most RESS_SPLIT_ROWS rows per range, RESS_SPLIT_PARTS parts of RESS_PART_FLOATS
// floats each). The fused path's patch/special split can add one query block per head.
RESS_API long long ress_attn_sched_bytes(int B, int H, int Tq) {
  if (B <= 0 || H <= 0 || Tq < 0) return -1;
  const long long n = (long long)B * H * (cdiv(Tq, 128) + 1);
  return RESS_SCHED_HDR_BYTES + 8LL * split_rows(n) * RESS_SPLIT_PARTS * RESS_PART_FLOATS * 4;
}

RESS_API long long ress_qattn_workspace_size(int B, int H, int Tq, int Tk) {
  if (B <= 0 || H <= 0 || Tq < 0 || Tk < 0) return -1;
  return 256 + round256(qattn_vpack_bytes(B, H, Tk)) + qattn_lut_bytes(B, H, Tq, Tk) + qattn_nv_bytes(B, H, Tq) +
         ress_attn_sched_bytes(B, H, Tq);
}

// Mirror of SpargeAttn's qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold
// (call site reference src/ress/models/attention.py:238-241). q_i8 (B,H,Tq,64) and
// k_i8 (B,H,Tk,64) int8 contiguous with rows allocated up to the next multiple of
// 128 / 64 (the blocked layout ress_per_block_int8 writes); v (B,H,Tk,64) fp16
// (v_f16=1) or bf16 with strides; lut/valid_block_num [B*H][ceil(Tq/128)][ceil(Tk/64)];
// q_scale [B*H][ceil(Tq/128)], k_scale [B*H][ceil(Tk/64)]; o (B,H,Tq,64) with strides.
// Supported: tensor_layout 1 (HND), is_causal 0, qk_quant_gran 1 (per block),
// return_pv_count 0, pv_threshold disabled (>= 1e9, the reference passes 1e10).
// pv_threshold: H floats in device memory (or null = disabled), read on the device.
// workspace: ress_qattn_workspace_size(B,H,Tq,Tk) bytes: a status word (int32 at offset 0),
// packed V, the checked LUT copy, the row schedule. The status word gets the
// RESS_QATTN_* bits of what was wrong with lut / valid_block_num / pv_threshold; the call
// itself never synchronises, so the caller reads the word when it next synchronises.
RESS_API int ress_qattn_block_sparse_fwd(const void* q_i8, const void* k_i8, const void* v, int v_f16, void* o,
                                         int o_dtype, const void* lut, const void* valid_block_num,
                                         const float* pv_threshold, const void* q_scale, const void* k_scale,
                                         int B, int H, int Tq, int Tk, long long svB, long long svH, long long svT,
                                         long long soB, long long soH, long long soT, int tensor_layout, int is_causal,
                                         int qk_quant_gran, float sm_scale, int return_pv_count, void* workspace,
                                         long long workspace_bytes, hipStream_t stream) {
  RESS_REQUIRE(tensor_layout == 1, "ress_qattn_block_sparse_fwd: only tensor_layout=1 (HND) is supported");
  RESS_REQUIRE(is_causal == 0, "ress_qattn_block_sparse_fwd: is_causal must be 0");
  RESS_REQUIRE(qk_quant_gran == 1, "ress_qattn_block_sparse_fwd: only per-block quantisation (qk_quant_gran=1)");
  RESS_REQUIRE(return_pv_count == 0, "ress_qattn_block_sparse_fwd: return_pv_count must be 0");
  RESS_REQUIRE(B > 0 && H > 0 && Tq > 0 && Tk > 0, "ress_qattn_block_sparse_fwd: bad geometry");
  RESS_REQUIRE(lut && valid_block_num, "ress_qattn_block_sparse_fwd: null lut / valid_block_num");
  RESS_REQUIRE(v && workspace && workspace_bytes >= ress_qattn_workspace_size(B, H, Tq, Tk),
               "ress_qattn_block_sparse_fwd: workspace of %lld bytes required",
               ress_qattn_workspace_size(B, H, Tq, Tk));
  RESS_REQUIRE(((uintptr_t)v & 15u) == 0 && svT % 8 == 0 && svH % 8 == 0 && svB % 8 == 0,
               "ress_qattn_block_sparse_fwd: v must be 16-byte aligned with strides a multiple of 8");
  const int kb_tot = cdiv(Tk, 64), nq = cdiv(Tq, 128);
  char* ws = (char*)workspace;
  int* status = (int*)ws;
  char* vpack = ws + 256;
  int* lut_c = (int*)(vpack + round256(qattn_vpack_bytes(B, H, Tk)));
  int* nv_c = (int*)((char*)lut_c + qattn_lut_bytes(B, H, Tq, Tk));
  char* sched = (char*)nv_c + qattn_nv_bytes(B, H, Tq);
  hipLaunchKernelGGL(k_qattn_status_clear, dim3(1), dim3(64), 0, stream, status);
  RESS_LAUNCHED("k_qattn_status_clear");
  hipLaunchKernelGGL(k_qattn_check, dim3(nq, B * H), dim3(64), 0, stream, (const int*)lut, (const int*)valid_block_num,
                     pv_threshold, H, nq, kb_tot, lut_c, nv_c, status);
  RESS_LAUNCHED("k_qattn_check");
  hipLaunchKernelGGL(k_pack_v, dim3(kb_tot, B * H), dim3(64), 0, stream, (const uint16_t*)v, svB, svH, svT, H, Tk,
                     kb_tot, (uint16_t*)vpack);
  RESS_LAUNCHED("k_pack_v");
  TokenMap m;
  m.P = Tq;
  m.S = 0;
  m.HW = Tq;
  m.T_p = Tq;
  m.T_s = 0;
  m.perm = nullptr;
  return attn_common(q_i8, nullptr, q_scale, k_i8, nullptr, k_scale, vpack, v_f16, lut_c, nv_c, B, H, m, Tk, sm_scale,
                     o, o_dtype, soB, soH, soT, sched, stream);
}

// ---- allocation-free variant of ress_sparse_attn_fwd_f16 --------------------------------
// For callers that cannot allocate device memory (code under graph capture, serving loops,
// harnesses that forbid hipMalloc): the launch's scratch -- the row schedule and the parts
// of the split rows, ress_attn_sched_bytes(...) bytes, at most RESS_NOALLOC_SCRATCH_BYTES
// for any shape -- lives in this file-scope device array instead of a caller workspace.
// Each device holds its own copy for the life of the process. Every call on a device
// uses that device's copy, so calls that overlap on one device (other streams, other
// threads) race; the schedule kernel rewrites the counters at the start of every launch,
// so nothing needs clearing between calls.
#define RESS_NOALLOC_SCRATCH_BYTES \
  (RESS_SCHED_HDR_BYTES + 8LL * RESS_SPLIT_ROWS * RESS_SPLIT_PARTS * RESS_PART_FLOATS * 4)
static __device__ __align__(256) unsigned char scratch[RESS_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` per device, looked up once with that device current (the
// array's host-side name is not a device address).
static std::mutex g_scratch_mu;
static void* g_scratch_addr[64];

static int scratch_address(void** out) {
  int dev = -1;
  RESS_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64,
               "ress_sparse_attn_fwd_f16_noalloc: no usable current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    RESS_REQUIRE(e == hipSuccess && p != nullptr,
                 "ress_sparse_attn_fwd_f16_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                 hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return 0;
}

RESS_API long long ress_noalloc_scratch_bytes(void) { return RESS_NOALLOC_SCRATCH_BYTES; }

// Device address of the current device's operand-status word (int32) inside `scratch`:
// word 24 of the schedule header, which every ress_sparse_attn_fwd_f16_noalloc call clears
// when it starts and sets to RESS_F16_KEY_RANGE | RESS_F16_QUERY_RANGE for a key / query
// element outside fp16's range. Read it (a 4-byte device-to-host copy) after the call has
// completed and before the next call on the device.
RESS_API int ress_noalloc_status_address(void** out) {
  RESS_REQUIRE(out != nullptr, "ress_noalloc_status_address: null output pointer");
  void* base = nullptr;
  if (scratch_address(&base) != 0) return -1;
  *out = reinterpret_cast<int*>(base) + 24;
  return 0;
}

RESS_API int ress_sparse_attn_fwd_f16_noalloc(const void* q, long long sqB, long long sqH, long long sqT,
                                              const void* k_pack, const void* k_norm, const void* v_pack,
                                              const void* lut, const void* nvalid, int B, int H, int frames, int P,
                                              int S, const int* patch_order, float sm_scale, void* out, int out_dtype,
                                              long long soB, long long soH, long long soT, hipStream_t stream) {
  RESS_REQUIRE(B > 0 && H > 0 && frames > 0 && P > S && S >= 0, "ress_sparse_attn_fwd_f16_noalloc: bad geometry");
  const long long need = ress_attn_sched_bytes(B, H, frames * P);
  RESS_REQUIRE(need > 0 && need <= RESS_NOALLOC_SCRATCH_BYTES,
               "ress_sparse_attn_fwd_f16_noalloc: this shape needs %lld bytes of scratch, the static array holds %lld",
               need, (long long)RESS_NOALLOC_SCRATCH_BYTES);
  void* sched = nullptr;
  if (scratch_address(&sched) != 0) return -1;
  return ress_sparse_attn_fwd_f16(q, sqB, sqH, sqT, k_pack, k_norm, v_pack, lut, nvalid, B, H, frames, P, S,
                                  patch_order, sm_scale, out, out_dtype, soB, soH, soT, sched, stream);
}
