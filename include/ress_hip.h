/* libress_hip: MI355X (gfx950) kernels for ReSS / HeSS block-sparse global attention.
 *
 * Every entry point is a plain C function: device pointers and sizes in, an int
 * status out (0 = ok, -1 = bad argument, -2 = launch failure; the message is in
 * ress_last_error(), thread-local). Nothing here allocates device memory or
 * synchronises: work is enqueued on `stream` (hipStream_t; 0 = the null stream)
 * and buffers are owned by the caller. Tensors are row-major; "BH" is batch*heads.
 * Head dim is 64 throughout. Citations are to the reference repository
 * (libary753/ReSS) and to the SpargeAttn functions it binds.
 */
#ifndef RESS_HIP_H
#define RESS_HIP_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- library ------------------------------------------------------------- */
const char* ress_last_error(void);
int ress_abi_version(void);
/* Self-check of the device's bf16 rounding (no counterpart in the reference; for tests and
 * for callers that want to confirm a device before trusting bit-exact bf16 results). Every
 * kernel here rounds fp32 to bf16 with the device's conversion instruction, which stands
 * for round-to-nearest-even with NaNs made quiet ((u >> 16) | 0x40) -- the rounding of
 * torch's .to(bfloat16) for numbers. For the fp32 bit patterns first .. first+count-1
 * (count <= 2^32), adds the number of patterns whose conversion differs to out[0] and
 * lowers out[1] to the lowest such pattern: out is two uint64 in device memory, which the
 * caller sets to {0, ~0} first. */
int ress_bf16_selfcheck(unsigned int first, unsigned long long count, void* out, hipStream_t stream);

/* ---- block preparation (prep.hip) ---------------------------------------- */

/* Fused Q/K/V preparation for one ReSS global-attention layer.
 * Replaces: compute_patch_qkv's patch/special split (src/ress/models/qkv.py:60-68,
 * tokens.py:8-52), predict_attention's avg pools (src/ress/models/attention.py:90-96),
 * block_mean_value (attention.py:103-109), km = key.mean(-2) and
 * per_block_int8(q, k - km) (attention.py:231-233; SpargeAttn quant_per_block with
 * external/patches/spargeattn.patch:38-41).
 * q/k/v: bf16 (B,H,frames*P,64) in storage order (per frame S special then P-S patch
 * tokens), element strides (sB,sH,sT). Outputs:
 *   q_i8 [BH][qb_p+qb_s][128][64] int8, q_scale [BH][qb_p+qb_s] f32,
 *   pooled_q [BH][qb_p][64] f32                 qb_p = ceil(T_p/128), qb_s = ceil(T_s/128)
 *   k_i8 [BH][kb_tot][64][64] int8, k_scale [BH][kb_tot] f32   kb_tot = ceil(frames*P/64)
 *   pooled_k, pooled_v [BH][kb_p][64] f32       kb_p = ceil(T_p/64) (patch keys only), or
 *                  [BH][kb_tot][64] with pool_all = 1 (every key in kernel order: the
 *                  sink-mass map, RESS_SINK_MASS, src/ress/models/attention.py:78, 451-452)
 *   v_pack [BH][kb_tot][4096] bf16, ksum [BH][kb_tot][64] f32, km [BH][64] f32
 *   q_lo / k_lo (optional, layouts of q_i8 / k_i8): split-INT8 residual codes, x ~
 *   scale*hi + scale/254*lo, used by ress_sparse_attn_fwd for a two-term INT8 QK^T.
 *   k_pack [BH][kb_tot][64][64] fp16 (optional): the K blocks for ress_sparse_attn_fwd_f16
 *   (a bf16 key is exact in fp16 unless below 2^-14 in magnitude or above 65504).
 * q_i8 = k_i8 = NULL selects the 16-bit operands: pooled_q/k/v, v_pack, k_pack and
 * k_scale (both required) are written, k_scale [BH][kb_tot] receiving each key block's
 * largest key norm; q_lo, q_scale, k_lo, ksum, km are unused.
 * patch_order: NULL, or P-S int32 in device memory, a permutation of the frame's patch
 * tokens: block position j of every frame holds the frame's patch token patch_order[j]
 * (replaces the gather of hilbert_permute, src/ress/models/hilbert.py:128-162, and its
 * .contiguous() copy: the tokens are read in place). Give the attention call the same table. */
int ress_prep_qkv(const void* q, const void* k, const void* v, int B, int H, int frames, int P, int S,
                  const int* patch_order, long long sqB, long long sqH, long long sqT, long long skB, long long skH, long long skT,
                  long long svB, long long svH, long long svT, void* q_i8, void* q_lo, void* q_scale,
                  void* pooled_q, void* k_i8, void* k_lo, void* k_scale, void* pooled_k, void* pooled_v,
                  void* v_pack, void* k_pack, void* ksum, void* km, int pool_all, hipStream_t stream);

/* Replaces SpargeAttn per_block_int8(q, k) (call site src/ress/models/attention.py:232,
 * patched Q scale spargeattn.patch:38-41). km [BH][64] optional (NULL = no smoothing).
 * Outputs in the blocked layouts of ress_prep_qkv; pooled_q [BH][ceil(Tq/128)][64]. */
int ress_per_block_int8(const void* q, const void* k, const void* km, int B, int H, int Tq, int Tk,
                        long long sqB, long long sqH, long long sqT, long long skB, long long skH,
                        long long skT, void* q_i8, void* q_scale, void* k_i8, void* k_scale, void* pooled_q,
                        hipStream_t stream);

/* Key mean + K/V block pass of a plain (B,H,Tk,64) bf16 sequence (the key mean of
 * src/ress/models/attention.py:231; block_mean_value attention.py:103-109). */
int ress_prep_kv_plain(const void* k, const void* v, int B, int H, int Tk, long long skB, long long skH,
                       long long skT, long long svB, long long svH, long long svT, void* ksum, void* km,
                       void* pooled_k, void* pooled_v, void* v_pack, hipStream_t stream);

/* ---- pooled map (scores.hip) --------------------------------------------- */

/* Replaces predict_attention's pooled GEMM + softmax (src/ress/models/attention.py:98-100)
 * and attn_cond = attn_pooled / clamp(rowsum, 1e-6) (attention.py:457,473).
 * attn_full [BH][q_blk][kb_p], attn_cond [BH][q_blk][n_cand] f32. */
int ress_pooled_scores(const void* pooled_q, const void* pooled_k, int BH, int q_blk, int kb_p, int n_cand,
                       float scale, void* attn_full, void* attn_cond, hipStream_t stream);

/* ---- budgets (budget.hip) ------------------------------------------------- */

/* Replaces compute_baseline_num_to_select (src/ress/models/attention.py:268-293):
 * cdf_threshold < 0 disables the CDF cut, topk < 0 the sparse-ratio floor
 * (topk = int(k_blk*(1-sr)) in host double arithmetic). out [rows] int32. */
int ress_baseline_budget(const void* attn_cond, long long rows, int n, float cdf_threshold, int topk,
                         void* out_counts, hipStream_t stream);

/* Replaces adjust_attention_selection (src/ress/budget/_proportional.py:49-115) as
 * HessBudget.num_to_select calls it (src/ress/budget/hess.py:92-100), plus a floor.
 * baseline/out [B][H][q_blk] int32 (may alias); scores_norm [H] f32 or NULL (no
 * reallocation); iters_out [B][q_blk] int32 or NULL (-1 = did not converge). */
int ress_head_budget(const void* baseline, int B, int H, int q_blk, const void* scores_norm, double beta,
                     int max_val, int max_iters, int min_select, void* out_counts, void* iters_out,
                     hipStream_t stream);

/* ---- selection (select.hip) ------------------------------------------------ */

/* Replaces build_block_mask (src/ress/models/attention.py:147-174) with the
 * MIN_NUM_TO_SELECT floor (attention.py:525), SpargeAttn block_map_lut_triton
 * (attention.py:224) and leading attention_sink forcing (spargeattn.patch:61-65).
 * rank_key [BH][q_blk_sel][n_cand] f32, counts [BH][q_blk_sel] int32; rows
 * q_blk_sel..q_blk_total-1 are dense. map [BH][q_blk_sel][kb_tot] uint8 (or NULL),
 * lut [BH][q_blk_total][kb_tot] int32 (ascending kept block indices), nvalid
 * [BH][q_blk_total] int32. */
int ress_select_blocks(const void* rank_key, const void* counts, int BH, int q_blk_sel, int q_blk_total,
                       int n_cand, int kb_tot, int sink_lead, int min_select, void* map, void* lut,
                       void* nvalid, hipStream_t stream);

/* Replaces SpargeAttn fill_block_map_triton (src/ress/models/attention.py:168):
 * map[r, sorted_idx[r, :counts[r]]] = 1. map [rows][k] uint8, int64 counts/indices. */
int ress_fill_block_map(void* map, const void* counts, const void* sorted_idx, long long rows, int k,
                        hipStream_t stream);

/* Replaces SpargeAttn block_map_lut_triton (src/ress/models/attention.py:224):
 * map [rows][k] uint8 -> lut [rows][k] int32 (ascending), nvalid [rows]. */
int ress_block_map_lut(const void* map, long long rows, int k, void* lut, void* nvalid, hipStream_t stream);

/* ---- QKV preparation (qkv.hip) ------------------------------------------------ */

/* Replaces compute_patch_qkv's q_norm / k_norm and RoPE (src/ress/models/qkv.py:60-68)
 * for modules with LayerNorm(64) q/k norms and the rotate-half 2D RoPE (first 32 head
 * dims by row, last 32 by column, base^(-2i/32)): qkv (B,T,3*nh*64) bf16 (the qkv
 * Linear's output), LayerNorm weights/biases [64] bf16, pos (B,T,2) int64 or NULL (no
 * rotation) -> q, k, v (B,nh,T,64) bf16. v is copied exactly; q and k match the torch
 * modules to one bf16 rounding (hardware sine/cosine for |pos| <= 256, the library
 * functions beyond). */
int ress_qk_norm_rope(const void* qkv, int B, int T, int nh, const void* q_weight, const void* q_bias,
                      const void* k_weight, const void* k_bias, float eps, const void* pos, float rope_base,
                      void* q_out, void* k_out, void* v_out, hipStream_t stream);

/* ---- SpargeAttn meansim block map (meansim.hip) --------------------------- */

/* Replaces get_block_map_meansim_fuse_quant (SpargeAttn spas_sage_attn/utils.py as
 * patched by external/patches/spargeattn.patch:50-67; attention_sink = a count of
 * leading tokens forcing its ceil(sink/64) leading key blocks, :63-65; Q quantised with
 * sm_scale = 1, :38-41). q (B,H,Tq,64), k (B,H,Tk,64) bf16 with element strides, km
 * [B*H][64] f32 or NULL, simthreshd1 / cdfthreshd [H] f32 (device). Outputs: map
 * [B*H][nq][nk] uint8 (nq = ceil(Tq/128), nk = ceil(Tk/64) <= 6144), q_i8
 * [B*H][nq*128][64], q_scale [B*H][nq], k_i8 [B*H][nk*64][64], k_scale [B*H][nk], and the
 * intermediate pooled_q [B*H][nq][64], pooled_k [B*H][nk][64] f32, sim_q [B*H][nq],
 * sim_k [B*H][nk] uint8 (1 = similar block). Non-causal only. The CDF cut keeps the n
 * largest probabilities of a row (ties to the lowest index), n = the number of prefix sums
 * of the descending probabilities that are <= cdfthreshd[h], the sums taken exactly over
 * floor(p * 2^50) in uint64 against floor(min(cdfthreshd, 8192) * 2^50) (n = 0 for a
 * negative threshold): a value-only definition, within 2^-37 of the real-number sums. */
int ress_meansim_block_map(const void* q, const void* k, const void* km, int B, int H, int Tq, int Tk,
                           long long sqB, long long sqH, long long sqT, long long skB, long long skH, long long skT,
                           const void* simthreshd1, const void* cdfthreshd, int attention_sink, void* map, void* q_i8,
                           void* q_scale, void* k_i8, void* k_scale, void* pooled_q, void* pooled_k, void* sim_q,
                           void* sim_k, void* workspace, long long workspace_bytes, hipStream_t stream);

/* Bytes of ress_meansim_block_map's optional workspace (16-byte aligned): the fp32 scores
 * of every row when rows are long (nk > 1024), computed by one matrix-core GEMM; 0 for
 * shorter rows. With workspace = NULL long rows compute their own scores (slower; the same
 * map). */
long long ress_meansim_workspace_size(int B, int H, int Tq, int Tk);

/* ---- ReSS restore-swap (ress_swap.hip) ------------------------------------ */

/* Replaces restore_swap_rank_by (src/ress/scoring/projected.py:395-1058) with its fused
 * round body (src/ress/scoring/fused_round.py, fused_topm.py), as ress_attention_forward
 * calls it for the restore_swap* criteria (src/ress/models/attention.py:545-566).
 * A [BH][q_blk][kb_p] pooled map (attn_full), V [BH][kb_p][64] block means (v_bar_full),
 * M [H][64][64] (head bh % H), nts [BH][q_blk] kept budgets. Out: rank_key
 * [BH][q_blk][n_cand] = 1 kept / 0 dropped (its top-nts is the keep set), obj [BH][q_blk]
 * (optional) J of the returned set, s_out [BH][q_blk][n_cand] (optional) the scores
 * s = P*sqrt(d^T M d). flags: 1 bf16 k-wide tensors, 2 track_best, 4 maximize, 8
 * invert_cut, 16 renormalize off. kb_p <= 2048. */
long long ress_restore_swap_workspace_size(int BH, int q_blk, int kb_p, int n_cand);
int ress_restore_swap(const void* A, const void* V, const void* M, const void* nts, int BH, int H, int q_blk, int kb_p,
                      int n_cand, int n_iters, double restore_frac, double decay, int flags, void* rank_key, void* obj,
                      void* s_out, void* workspace, long long workspace_bytes, hipStream_t stream);

/* ---- attention (attn.hip) ----------------------------------------------- */

/* Fused-path attention (src/ress/models/attention.py:404-412 special queries dense,
 * :625 run_block_sparse_kernel, :652 combine_special_and_patch): inputs from
 * ress_prep_qkv + ress_select_blocks; out (B,H,frames*P,64) in storage order,
 * out_dtype 0 f32 / 1 bf16 / 2 f16, element strides soB/soH/soT. q_lo/k_lo both NULL: the
 * reference's single-term per-block INT8 QK^T; both set: the two-term split product.
 * sched: ress_attn_sched_bytes(B, H, frames*P) bytes of 16-byte aligned device workspace
 * (the persistent kernel's row schedule and the parts of the rows it splits; rewritten by
 * every call, so calls that overlap must not share it). */
long long ress_attn_sched_bytes(int B, int H, int Tq);
int ress_sparse_attn_fwd(const void* q_i8, const void* q_lo, const void* q_scale, const void* k_i8,
                         const void* k_lo, const void* k_scale, const void* v_pack, int v_f16, const void* lut,
                         const void* nvalid, int B, int H, int frames, int P, int S, const int* patch_order,
                         float sm_scale, void* out, int out_dtype, long long soB, long long soH, long long soT,
                         void* sched, hipStream_t stream);

/* The fused-path attention of ress_sparse_attn_fwd (same reference lines) with QK^T on
 * 16-bit operands (fp16 MFMA, fp32 accumulation) instead of INT8 codes: q is the layer's
 * bf16 (B,H,frames*P,64) query tensor in storage order with element strides
 * sqB/sqH/sqT, converted to fp16 per row in registers; k_pack (fp16), k_norm (the k_scale
 * output of the 16-bit mode: per-block largest key norms) and v_pack come from
 * ress_prep_qkv. A row whose logit bound |q*sm_scale*log2 e| * max key norm is at most 64
 * (log2 units) for every one of its queries runs with the pre-scaled queries rounded to fp16
 * and P = exp2(logit) taken directly (no offset, no running max); other rows use the exact
 * fp16 queries and a running max.
 * sched, patch_order: as for ress_sparse_attn_fwd (patch_order: the table given to
 * ress_prep_qkv; each row is read and written at the storage positions of its tokens).
 * After the call, int32 word 24 of sched (byte 96) is 1 if a key and 2 if a query element
 * (or 3 if both) lay outside fp16's range (|x| >= 65520, which bf16 can hold and fp16
 * cannot): those rows are not meaningful and the caller should use the INT8 entry point.
 * ress_prep_qkv marks such a key block by an infinite k_norm. */
int ress_sparse_attn_fwd_f16(const void* q, long long sqB, long long sqH, long long sqT, const void* k_pack,
                             const void* k_norm, const void* v_pack, const void* lut, const void* nvalid, int B,
                             int H, int frames, int P, int S, const int* patch_order, float sm_scale, void* out,
                             int out_dtype, long long soB, long long soH, long long soT, void* sched,
                             hipStream_t stream);

/* Allocation-free variant of ress_sparse_attn_fwd_f16 (same arguments without `sched`,
 * same kernels and results). No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The launch's scratch (row schedule and split-row parts) lives in a
 * static device array of ress_noalloc_scratch_bytes() bytes (about 26.7 MB) that each device
 * holds for the life of the process; every shape fits in it, and a shape that did not would be
 * rejected (-1). Calls on one device share that array: calls that overlap on a device (other
 * streams or threads) race. Nothing is allocated, freed or synchronised. */
long long ress_noalloc_scratch_bytes(void);
int ress_sparse_attn_fwd_f16_noalloc(const void* q, long long sqB, long long sqH, long long sqT, const void* k_pack,
                                     const void* k_norm, const void* v_pack, const void* lut, const void* nvalid,
                                     int B, int H, int frames, int P, int S, const int* patch_order, float sm_scale,
                                     void* out, int out_dtype,
                                     long long soB, long long soH, long long soT, hipStream_t stream);
/* The fp16 operand-range report of ress_sparse_attn_fwd_f16_noalloc (no counterpart in the
 * reference; for the same callers). ress_sparse_attn_fwd_f16 reports a key / query element
 * outside fp16's range (|x| >= 65520) in word 24 of its `sched` workspace; the noalloc call
 * keeps that word in its static array, whose device address (an int32, for the current
 * device) this returns in *out. Each call clears the word when it starts and ORs in 1 (a
 * key) or 2 (a query); read it after the call has completed and before the next call on the
 * device. Looks the address up once per device; allocates nothing. */
int ress_noalloc_status_address(void** out);

/* Replaces SpargeAttn qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold
 * (call src/ress/models/attention.py:238-241) with the same argument meaning; see
 * attn.hip for the supported flag values. pv_threshold: H floats in device memory (or
 * null), read on the device. workspace: ress_qattn_workspace_size(B,H,Tq,Tk) bytes,
 * 16-byte aligned: a status word (int32 at offset 0), packed V, a checked copy of the LUT,
 * the attention's sched workspace. The LUT contract is SpargeAttn's: per row, nvalid in
 * [0, ceil(Tk/64)] and that many strictly ascending block indices below ceil(Tk/64). The
 * call checks it on the device without synchronising: the attention runs on a copy
 * clamped into range, and the status word gets 1 (an nvalid out of range), 2 (a listed
 * block out of range or not ascending) or 4 (a pv_threshold below 1e9: PV-threshold skipping
 * is not implemented), OR-ed, for the caller to read at its next synchronisation. */
long long ress_qattn_workspace_size(int B, int H, int Tq, int Tk);
int ress_qattn_block_sparse_fwd(const void* q_i8, const void* k_i8, const void* v, int v_f16, void* o,
                                int o_dtype, const void* lut, const void* valid_block_num,
                                const float* pv_threshold, const void* q_scale, const void* k_scale,
                                int B, int H, int Tq, int Tk, long long svB, long long svH, long long svT,
                                long long soB, long long soH, long long soT, int tensor_layout, int is_causal,
                                int qk_quant_gran, float sm_scale, int return_pv_count, void* workspace,
                                long long workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* RESS_HIP_H */
