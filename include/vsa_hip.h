/* C ABI of the MI355X (gfx950) VSA / VSA2 block-sparse attention path (same library: libechosparse_hip.so).
 *
 * Conventions as in echosparse_hip.h: caller-owned device pointers, plain sizes, the HIP stream last, no
 * allocation and no synchronisation inside, an es_status return and es_last_error_string() on failure.
 * vsa_attn_fwd, vsa_attn_bwd_kv, vsa_attn_bwd_q, vsa_rep_attn_fwd and vsa_rep_attn_bwd_q balance their row blocks
 * over the XCDs through counters in a 64-slot ring of device memory per source file, one slot per kernel launch;
 * a launch that takes a slot waits (on its stream) for the slot's previous launch, so uncaptured launches may overlap
 * freely; launches recorded in a stream capture use a second ring of 64 slots and do not wait, so graph replays may
 * overlap uncaptured launches but not each other.
 * Layouts (row-major):
 *   tokens q, k, v, o, gate, dO      [BH, L, 128] bf16 (fp16: the _f16 twins), L = NB * 64, valid-first
 *                                    64-token blocks
 *   D (every entry point)            the logical head dim, 64 or 128: rows are always 128 columns wide and a
 *                                    D = 64 caller zero-fills columns 64..127 (they add exact zeros to every dot
 *                                    product and come out zero); D sets the softmax scale 1 / sqrt(D). The fine
 *                                    attention entry points (vsa_attn_*) run a D = 64 kernel variant that reads
 *                                    and computes on the first 64 columns only
 *   blk_cnt                          [NB] int32, valid tokens per block (1..64)
 *   router pools qr, kr, vr          [BH, Lr_pad, 128] bf16, Lr_pad = ceil64(NB * 64 / R)
 *   block means qc, kc, vc           [BH, NBc_pad, 128] bf16, NBc_pad = ceil64(NB)
 *   lse                              [BH, L] float32, natural log; -inf on rows with nothing to attend
 *   CSR selection                    ptr [BH, NB + 1] int32 absolute offsets into idx [nnz] int32;
 *                                    q2k rows list kv blocks ascending, k2q columns list query blocks ascending
 * Each entry point cites the reference function it replaces (paths relative to the reference tree).
 */
#ifndef VSA_HIP_H
#define VSA_HIP_H

#include "echosparse_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- pooling and fusion */

/* Router group means of R tokens (qr / kr / vr, each may be NULL; empty groups are 0) and whole-block means
 * (qc / kc / vc) over the valid tokens of each block. Padding rows of the outputs are not written.
 * Replaces csrc/vsa/vsa2_api.cpp:73-97 pool_fwd (kernel csrc/vsa/router/pool.cu:16-51). */
int vsa_pool(const void* q, const void* k, const void* v, const int* blk_cnt, void* qr, void* kr, void* vr,
             void* qc, void* kc, void* vc, int BH, int L, int D, int R, hipStream_t stream);

/* o = valid ? o_f + act(gate) * o_c[blk] : 0. gate_mode 0 = no gate (act = 1), 1 = per token [BH, L],
 * 2 = elementwise [BH, L, D]; gate_act 0 = tanh, 1 = identity. o_c is [BH, NBc_pad, D].
 * Replaces csrc/vsa/vsa2_api.cpp fuse_fwd (kernel csrc/vsa/fuse.cu:43-80). */
int vsa_fuse_fwd(const void* of, const void* oc, const void* gate, void* o, const int* blk_cnt, int BH, int L,
                 int D, int NBc_pad, int gate_mode, int gate_act, hipStream_t stream);

/* dO_f = valid ? dO : 0 (dout_f may be NULL), delta_f = rowsum(dO_f * O_f) [BH, L] fp32,
 * dO_c[blk] = sum over valid rows of act(gate) * dO (bf16), delta_c = <dO_c, O_c> [BH, NBc_pad] fp32,
 * dgate = act'(gate) * <dO, O_c> (mode 1, [BH, L]) or act'(gate) * dO * O_c (mode 2), 0 on padding rows.
 * Replaces csrc/vsa/vsa2_api.cpp fuse_bwd (kernel csrc/vsa/fuse.cu:82-166). */
int vsa_fuse_bwd(const void* dout, const void* of, const void* oc, const void* gate, void* dout_f, float* delta_f,
                 void* dout_c, float* delta_c, void* dgate, const int* blk_cnt, int BH, int L, int D, int NBc_pad,
                 int gate_mode, int gate_act, hipStream_t stream);

/* out = valid ? acc + add[blk] / blk_cnt[blk] : 0 in bf16; acc fp32 [BH, L, D] and add fp32 [BH, add_nb, D]
 * may each be NULL. Replaces csrc/vsa/vsa2_api.cpp finalize (kernel csrc/vsa/fuse.cu:168-210). */
int vsa_finalize(const float* acc, const float* add, int add_nb, void* out, const int* blk_cnt, int BH, int L,
                 int D, hipStream_t stream);

/* ---------------------------------------------------------------- fine block-sparse attention */

/* O and lse (natural) of every query block over its q2k list, key columns >= blk_cnt masked; padding query rows and
 * empty lists give O = 0, lse = -inf. Replaces csrc/vsa/vsa2_api.cpp:318-348 attn_fwd (kernel
 * csrc/vsa/generic/attn_fwd.cu:32-313). */
int vsa_attn_fwd(const void* q, const void* k, const void* v, const int* row_ptr, const int* col_idx,
                 const int* blk_cnt, void* out, float* lse, int BH, int L, int D, hipStream_t stream);

/* The forward over planned (row, beg, end, slot) tasks (tasks [max_tasks, 4], device count info[0]): slot < 0
 * writes O / lse, slot >= 0 an fp32 normalized partial part_o [slot, 64, D] and its log2 lse part_lse [slot, 64].
 * Replaces csrc/vsa/vsa2_api.cpp:524-555 attn_fwd_tasks (attn_fwd.cu:216-237). */
int vsa_attn_fwd_tasks(const void* q, const void* k, const void* v, const int* col_idx, const int* blk_cnt,
                       const int* tasks, const int* info, int max_tasks, void* out, float* lse, float* part_o,
                       float* part_lse, int BH, int L, int D, hipStream_t stream);

/* KV-owner backward over the k2q lists: dK, dV (bf16, or fp32 when out_fp32) plus the optional per-block
 * gradients add_dk / add_dv [BH, add_nb, D] fp32 spread as add / blk_cnt; padding rows 0. delta = rowsum(dO * O).
 * Replaces csrc/vsa/vsa2_api.cpp:353-416 attn_bwd (kernel csrc/vsa/generic/attn_bwd.cu:136-380); dQ comes from
 * vsa_attn_bwd_q (no atomics). */
int vsa_attn_bwd_kv(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                    const float* delta, const int* k2q_ptr, const int* k2q_idx, const int* blk_cnt,
                    const float* add_dk, const float* add_dv, int add_nb, void* dk, void* dv, int out_fp32, int BH,
                    int L, int D, hipStream_t stream);

/* KV-owner backward over planned k2q tasks: direct tasks write dK / dV like vsa_attn_bwd_kv, split chunks fp32
 * partials part_dk / part_dv [slot, 64, D] (no add) for vsa_split_merge_sum.
 * Replaces csrc/vsa/vsa2_api.cpp:624-685 attn_bwd_tasks. */
int vsa_attn_bwd_kv_tasks(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                          const float* delta, const int* k2q_idx, const int* blk_cnt, const int* tasks,
                          const int* info, int max_tasks, const float* add_dk, const float* add_dv, int add_nb,
                          void* dk, void* dv, float* part_dk, float* part_dv, int BH, int L, int D,
                          hipStream_t stream);

/* Q-owner dQ over the q2k lists, deterministic: dq (bf16, + add_dq / blk_cnt, padding rows 0) or, when dq_acc is
 * given instead, dq_acc += dQ on valid rows (fp32). Replaces csrc/vsa/vsa2_api.cpp:419-457 attn_bwd_q (kernel
 * attn_bwd.cu:382-476). */
int vsa_attn_bwd_q(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                   const float* delta, const int* q2k_ptr, const int* q2k_idx, const int* blk_cnt,
                   const float* add_dq, int add_nb, void* dq, float* dq_acc, int BH, int L, int D,
                   hipStream_t stream);

/* Q-owner dQ over planned q2k tasks (split chunks: fp32 partials part_dq [slot, 64, D]).
 * Replaces csrc/vsa/vsa2_api.cpp:687-730 attn_bwd_q_tasks. */
int vsa_attn_bwd_q_tasks(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                         const float* delta, const int* q2k_idx, const int* blk_cnt, const int* tasks,
                         const int* info, int max_tasks, const float* add_dq, int add_nb, void* dq, float* part_dq,
                         int BH, int L, int D, hipStream_t stream);

/* ---------------------------------------------------------------- routers and selections */

/* Bytes of device workspace vsa_route_rows / vsa_row_topk / vsa_global_topk / vsa_csr_transpose need. */
size_t vsa_topk_workspace(int bh_count, int NB);

/* Whole-block scores S = rnd(rnd(qc . kc) / sqrt(D)) (bf16) of (b, h) rows bh0 .. bh0 + bh_count - 1 into
 * scores [bh_count, NB, NB]. Replaces csrc/vsa/vsa2_api.cpp:244-260 block_scores (csrc/vsa/router/scores.cu). */
int vsa_block_scores(const void* qc, const void* kc, void* scores, int NB, int NBc_pad, int bh0, int bh_count, int D,
                     hipStream_t stream);

/* Original-VSA router: the block scores and exactly K blocks per row (score desc, ties to the smaller index,
 * -0 == +0) into the q2k / k2q CSR of rows bh0 .. (offsets (b * NB + i) * K). NB <= 8192.
 * Replaces csrc/vsa/vsa2_api.cpp:284-315 route_rows (topk.cu:621-685). */
int vsa_route_rows(const void* qc, const void* kc, int NB, int NBc_pad, int bh0, int bh_count, int K, int D,
                   int* q2k_ptr, int* q2k_idx, int* k2q_ptr, int* k2q_idx, void* workspace, size_t workspace_bytes,
                   hipStream_t stream);

/* The per-row top-K of given bf16 scores [bh_count, NB, NB]. Replaces csrc/vsa/vsa2_api.cpp:262-282
 * row_topk_into. */
int vsa_row_topk(const void* scores, int NB, int bh0, int bh_count, int K, int* q2k_ptr, int* q2k_idx,
                 int* k2q_ptr, int* k2q_idx, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* VSA2 PSP router pass 1: lse2 [BH, Lr_pad] (log2) of every pooled query row over all valid pooled keys.
 * Replaces csrc/vsa/vsa2_api.cpp:122-135 router_lse (csrc/vsa/router/router.cu). */
int vsa_router_lse(const void* qr, const void* kr, const int* blk_cnt, float* lse2, int NB, int R, int BH, int D,
                   hipStream_t stream);

/* VSA2 PSP router pass 2: block scores [bh_count, NB, NB] fp32, row_norm 0 = valid_groups, 1 = paper.
 * Replaces csrc/vsa/vsa2_api.cpp:137-155 router_scores. */
int vsa_router_scores(const void* qr, const void* kr, const float* lse2, const int* blk_cnt, float* scores, int NB,
                      int R, int row_norm, int bh0, int bh_count, int D, hipStream_t stream);

/* Exact global top-k of fp32 scores [bh_count, NB, NB]: k = min(budget, NB^2) entries per (b, h), score desc then
 * flat index asc, into the CSR of rows bh0 .. (offsets b * k), and (bits_out != NULL) the selection bitmap rows
 * bits_out [BH, NB, ceil(NB / 32)] of those (b, h). NB <= 46340 (NB^2 < 2^31).
 * Replaces csrc/vsa/vsa2_api.cpp:157-178 global_topk_into (topk.cu:69-578). */
int vsa_global_topk(const float* scores, int NB, int bh0, int bh_count, long long budget, int* q2k_ptr, int* q2k_idx,
                    int* k2q_ptr, int* k2q_idx, unsigned* bits_out, void* workspace, size_t workspace_bytes,
                    hipStream_t stream);

/* Transposed CSR (column lists, ascending) of rows bh0 .. with the same absolute base per (b, h). No reference
 * counterpart as an entry point: the reference builds k2q only inside its routers (topk.cu:405-459); this serves
 * selections given by the caller. */
int vsa_csr_transpose(const int* ptr, const int* idx, int NB, int bh0, int bh_count, int* out_ptr, int* out_idx,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- split-KV */

/* Device-side task plan of a CSR list ptr [BH, NB + 1]: tasks [BH * NB + max_slots, 4], merges
 * [max(1, min(BH * NB, max_slots / 2)), 4], info [8]; budget < 0 = unlimited.
 * Replaces csrc/vsa/vsa2_api.cpp:464-508 split_plan (csrc/vsa/split.cu:36-95). */
int vsa_split_plan(const int* ptr, int BH, int NB, int chunk, int max_slots, int min_len, double rel_mean,
                   double tail_frac, int resident, int budget, int* tasks, int* merges, int* info,
                   hipStream_t stream);

/* Ordered LSE merge of the forward partials of every split row into o / lse.
 * Replaces csrc/vsa/vsa2_api.cpp:557-583 split_merge_fwd (split.cu:117-155). */
int vsa_split_merge_fwd(const float* part_o, const float* part_lse, const int* merges, const int* info,
                        int max_merges, const int* blk_cnt, void* o, float* lse, int BH, int L, int D, int mask_rows,
                        hipStream_t stream);

/* Ordered sum of backward partials plus add / cnt into out (bf16, or out_f32).
 * Replaces csrc/vsa/vsa2_api.cpp:586-620 split_merge_sum (split.cu:157-200). */
int vsa_split_merge_sum(const float* part, const int* merges, const int* info, int max_merges, const float* add,
                        int add_nb, const int* blk_cnt, void* out, float* out_f32, int BH, int L, int D,
                        hipStream_t stream);

/* ---------------------------------------------------------------- VSA2 three-tier representatives */

/* Representative tables: k_mid / v_mid [BH, ceil64(NB * RM), D] = means of the RM contiguous 64 / RM-token groups
 * of every block (row blk * RM + g), k_tail / v_tail [BH, ceil64(NB), D] = block means, lc_mid [NB * RM] and
 * lc_tail [NB] = log2 of the valid tokens (-inf: empty group); padding rows are not written. Replaces
 * experiments/vsa2_representative/csrc/rep/rep_api.cpp rep_build (rep_pool.cu:23-57). */
int vsa_rep_build(const void* k, const void* v, const int* blk_cnt, void* k_mid, void* v_mid, float* lc_mid,
                  void* k_tail, void* v_tail, float* lc_tail, int BH, int L, int D, int RM, hipStream_t stream);

/* Seeded k-means tier-B tables (the three-tier benchmark construction; no reference counterpart, whose tables are contiguous means):
 * every block's valid keys clustered into RM groups by `iters` Lloyd rounds from seed tokens drawn with `seed`;
 * k_mid / v_mid rows (blk * RM + c, as vsa_rep_build) = the clusters' key / value means (zero when empty),
 * lc_mid / counts [BH, NB * RM] per head = log2 cluster sizes (-inf when empty) / sizes, labels [BH, L] uint8 =
 * each valid token's cluster (255 on padding). Float32 in a fixed order, no fused multiply-add (bit-exact against
 * oracle/vsa_ref.py kmeans_tables). The tail tables come from vsa_rep_build. */
int vsa_rep_build_kmeans(const void* k, const void* v, const int* blk_cnt, void* k_mid, void* v_mid, float* lc_mid,
                         int* counts, uint8_t* labels, int BH, int L, int D, int RM, int iters, unsigned seed,
                         hipStream_t stream);

/* Per-query-block tiers (the three-tier benchmark construction's split; the reference splits by global budgets, rep_api.cpp
 * route_tiers): for every row i of the fp32 scores [bh_count, NB, NB] of (b, h) rows bh0.., the ka (tier A) and
 * kab (tiers A and B) best blocks, score desc, ties to the smaller index, -0 == +0, as ascending CSR lists with
 * offsets (bh * NB + i) * K and as selection bitmaps [BH, NB, ceil(NB / 32)]. 0 <= ka <= kab <= NB <= 8192. */
int vsa_row_tiers(const float* scores, int NB, int bh0, int bh_count, int ka, int kab, int* a_ptr, int* a_idx,
                  int* ab_ptr, int* ab_idx, unsigned* bits_a, unsigned* bits_ab, hipStream_t stream);

/* Three-tier forward: one softmax over the tier-A tokens (q2k CSR), the tier-B representatives (bits_ab & ~bits_a)
 * and the tier-C means (~bits_ab), each representative column with + log2(count); O bf16, lse natural. phases:
 * 1 | 2 | 4 selects the tiers. lc_mid_stride: 0 when lc_mid is one [NB * RM] table for every head, NB * RM when
 * it is per head (k-means tables). NB <= 8192 (every three-tier entry point). Replaces rep_api.cpp rep_attn_fwd
 * (rep_attn_fwd.cu:37). */
int vsa_rep_attn_fwd(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                     const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                     const int* q2k_ptr, const int* q2k_idx, const unsigned* bits_a, const unsigned* bits_ab,
                     const int* blk_cnt, void* out, float* lse, int BH, int L, int D, int RM, int phases,
                     hipStream_t stream);

/* dQ of the three-tier attention (deterministic, no atomics), + dq_acc (fp32, optional) + add_dq / blk_cnt
 * (optional); padding rows 0. Replaces the dQ part of rep_api.cpp rep_attn_bwd_q (rep_attn_bwd.cu:141). */
int vsa_rep_attn_bwd_q(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                       const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                       const void* dout, const float* lse, const float* delta, const int* q2k_ptr,
                       const int* q2k_idx, const unsigned* bits_a, const unsigned* bits_ab, const int* blk_cnt,
                       const float* add_dq, int add_nb, const float* dq_acc, void* dq, int BH, int L, int D, int RM,
                       int phases, hipStream_t stream);

/* dK / dV of one representative table (tier 2: the mid table over tier B, tier 4: the tail table over tier C),
 * accumulated into dk_tab / dv_tab (fp32, the table's row layout) by a KV-owner pass: no atomics, deterministic.
 * Replaces the representative dK / dV atomics of rep_api.cpp rep_attn_bwd_q (rep_attn_bwd.cu:141). */
int vsa_rep_bwd_tables(const void* q, const void* dout, const void* k_tab, const void* v_tab, const float* lc,
                       int lc_stride, const float* lse, const float* delta, const unsigned* bits_a, const unsigned* bits_ab,
                       float* dk_tab, float* dv_tab, int BH, int L, int D, int RM, int tier, hipStream_t stream);

/* dK, dV (bf16) = acc (fp32 tier-A token gradients, optional) + dk_mid[group] / c_group + dk_tail[blk] / c_blk on
 * valid rows, 0 on padding; group = the token's contiguous group, or with labels / mid_counts (k-means tables,
 * both or neither) its cluster and that cluster's size. Replaces rep_api.cpp rep_unpool (rep_pool.cu:59-88). */
int vsa_rep_unpool(const float* acc_k, const float* acc_v, const float* dk_mid, const float* dv_mid,
                   const float* dk_tail, const float* dv_tail, const int* blk_cnt, const uint8_t* labels,
                   const int* mid_counts, void* dk, void* dv, int BH, int L,
                   int D, int RM, hipStream_t stream);

/* out [BH, L] = rowsum(x * y) on valid rows, 0 on padding. Replaces rep_api.cpp row_dot (rep_pool.cu:90-112). */
int vsa_row_dot(const void* x, const void* y, const int* blk_cnt, float* out, int BH, int L, int D,
                hipStream_t stream);

/* Tier-B CSR lists: the A|B lists without the tier-A columns, b_ptr = ab_ptr - a_ptr. Replaces
 * rep_pool.cu:114-140 tier_b_lists. */
int vsa_tier_b_lists(const int* ab_ptr, const int* ab_idx, const int* a_ptr, const unsigned* bits_a, int* b_ptr,
                     int* b_idx, int BH, int NB, hipStream_t stream);

/* ---------------------------------------------------------------- fp16 token tensors
 * Every entry point above that reads or writes token tensors (q, k, v, o, gate, dO, pools, block means, scores,
 * tier tables, gradients) has an fp16 twin with the suffix _f16 and the same arguments: the same kernels built for
 * fp16 storage and v_mfma_f32_32x32x16_f16 (fp32 accumulation), as the reference dispatches its kernels on the
 * tensor dtype (csrc/vsa/vsa2_api.cpp:51). Entry points without token tensors (vsa_topk_workspace,
 * vsa_global_topk, vsa_csr_transpose, vsa_split_plan, vsa_tier_b_lists, vsa_row_tiers) serve both. */
int vsa_pool_f16(const void* q, const void* k, const void* v, const int* blk_cnt, void* qr, void* kr, void* vr,
                 void* qc, void* kc, void* vc, int BH, int L, int D, int R, hipStream_t stream);
int vsa_fuse_fwd_f16(const void* of, const void* oc, const void* gate, void* o, const int* blk_cnt, int BH, int L,
                     int D, int NBc_pad, int gate_mode, int gate_act, hipStream_t stream);
int vsa_fuse_bwd_f16(const void* dout, const void* of, const void* oc, const void* gate, void* dout_f, float* delta_f,
                     void* dout_c, float* delta_c, void* dgate, const int* blk_cnt, int BH, int L, int D, int NBc_pad,
                     int gate_mode, int gate_act, hipStream_t stream);
int vsa_finalize_f16(const float* acc, const float* add, int add_nb, void* out, const int* blk_cnt, int BH, int L,
                     int D, hipStream_t stream);
int vsa_attn_fwd_f16(const void* q, const void* k, const void* v, const int* row_ptr, const int* col_idx,
                     const int* blk_cnt, void* out, float* lse, int BH, int L, int D, hipStream_t stream);
int vsa_attn_fwd_tasks_f16(const void* q, const void* k, const void* v, const int* col_idx, const int* blk_cnt,
                           const int* tasks, const int* info, int max_tasks, void* out, float* lse, float* part_o,
                           float* part_lse, int BH, int L, int D, hipStream_t stream);
int vsa_attn_bwd_kv_f16(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                        const float* delta, const int* k2q_ptr, const int* k2q_idx, const int* blk_cnt,
                        const float* add_dk, const float* add_dv, int add_nb, void* dk, void* dv, int out_fp32, int BH,
                        int L, int D, hipStream_t stream);
int vsa_attn_bwd_kv_tasks_f16(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                              const float* delta, const int* k2q_idx, const int* blk_cnt, const int* tasks,
                              const int* info, int max_tasks, const float* add_dk, const float* add_dv, int add_nb,
                              void* dk, void* dv, float* part_dk, float* part_dv, int BH, int L, int D,
                              hipStream_t stream);
int vsa_attn_bwd_q_f16(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                       const float* delta, const int* q2k_ptr, const int* q2k_idx, const int* blk_cnt,
                       const float* add_dq, int add_nb, void* dq, float* dq_acc, int BH, int L, int D,
                       hipStream_t stream);
int vsa_attn_bwd_q_tasks_f16(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                             const float* delta, const int* q2k_idx, const int* blk_cnt, const int* tasks,
                             const int* info, int max_tasks, const float* add_dq, int add_nb, void* dq, float* part_dq,
                             int BH, int L, int D, hipStream_t stream);
int vsa_block_scores_f16(const void* qc, const void* kc, void* scores, int NB, int NBc_pad, int bh0, int bh_count, int D,
                         hipStream_t stream);
int vsa_route_rows_f16(const void* qc, const void* kc, int NB, int NBc_pad, int bh0, int bh_count, int K, int D,
                       int* q2k_ptr, int* q2k_idx, int* k2q_ptr, int* k2q_idx, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);
int vsa_row_topk_f16(const void* scores, int NB, int bh0, int bh_count, int K, int* q2k_ptr, int* q2k_idx,
                     int* k2q_ptr, int* k2q_idx, void* workspace, size_t workspace_bytes, hipStream_t stream);
int vsa_router_lse_f16(const void* qr, const void* kr, const int* blk_cnt, float* lse2, int NB, int R, int BH, int D,
                       hipStream_t stream);
int vsa_router_scores_f16(const void* qr, const void* kr, const float* lse2, const int* blk_cnt, float* scores, int NB,
                          int R, int row_norm, int bh0, int bh_count, int D, hipStream_t stream);
int vsa_split_merge_fwd_f16(const float* part_o, const float* part_lse, const int* merges, const int* info,
                            int max_merges, const int* blk_cnt, void* o, float* lse, int BH, int L, int D, int mask_rows,
                            hipStream_t stream);
int vsa_split_merge_sum_f16(const float* part, const int* merges, const int* info, int max_merges, const float* add,
                            int add_nb, const int* blk_cnt, void* out, float* out_f32, int BH, int L, int D,
                            hipStream_t stream);
int vsa_rep_build_f16(const void* k, const void* v, const int* blk_cnt, void* k_mid, void* v_mid, float* lc_mid,
                      void* k_tail, void* v_tail, float* lc_tail, int BH, int L, int D, int RM, hipStream_t stream);
int vsa_rep_attn_fwd_f16(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                         const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                         const int* q2k_ptr, const int* q2k_idx, const unsigned* bits_a, const unsigned* bits_ab,
                         const int* blk_cnt, void* out, float* lse, int BH, int L, int D, int RM, int phases,
                         hipStream_t stream);
int vsa_rep_attn_bwd_q_f16(const void* q, const void* k, const void* v, const void* k_mid, const void* v_mid,
                           const float* lc_mid, int lc_mid_stride, const void* k_tail, const void* v_tail, const float* lc_tail,
                           const void* dout, const float* lse, const float* delta, const int* q2k_ptr,
                           const int* q2k_idx, const unsigned* bits_a, const unsigned* bits_ab, const int* blk_cnt,
                           const float* add_dq, int add_nb, const float* dq_acc, void* dq, int BH, int L, int D, int RM,
                           int phases, hipStream_t stream);
int vsa_rep_bwd_tables_f16(const void* q, const void* dout, const void* k_tab, const void* v_tab, const float* lc,
                           int lc_stride, const float* lse, const float* delta, const unsigned* bits_a, const unsigned* bits_ab,
                           float* dk_tab, float* dv_tab, int BH, int L, int D, int RM, int tier, hipStream_t stream);
int vsa_rep_build_kmeans_f16(const void* k, const void* v, const int* blk_cnt, void* k_mid, void* v_mid,
                             float* lc_mid, int* counts, uint8_t* labels, int BH, int L, int D, int RM, int iters,
                             unsigned seed, hipStream_t stream);
int vsa_rep_unpool_f16(const float* acc_k, const float* acc_v, const float* dk_mid, const float* dv_mid,
                       const float* dk_tail, const float* dv_tail, const int* blk_cnt, const uint8_t* labels,
                       const int* mid_counts, void* dk, void* dv, int BH, int L,
                       int D, int RM, hipStream_t stream);
int vsa_row_dot_f16(const void* x, const void* y, const int* blk_cnt, float* out, int BH, int L, int D,
                    hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
