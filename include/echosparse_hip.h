/* C ABI of the MI355X (gfx950) block-sparse attention hot path: libechosparse_hip.so.
 *
 * Every entry point takes caller-owned device pointers (no allocation inside), plain sizes and the HIP stream to
 * enqueue on, never synchronises, and returns an es_status; on failure es_last_error_string() holds a message.
 * es_block_attention, es_sparse_attention, es_dense_attention and es_dense_attention_kv balance their tiles over
 * the XCDs through counters in a ring of 64 slots of device memory, one slot per call: any number of such calls
 * may overlap on one GPU (a call waits on its stream for the previous user of its slot). Calls recorded in a stream
 * capture take slots from a second ring of 64 without waiting: graph replays may overlap uncaptured calls, not each
 * other.
 * Tensor layouts are the reference's (shapes in row-major order):
 *   q, k, v            (L, H, D) bf16, D = 128                       token-major, as echosparse passes them
 *   offset, lse        (nq * 128, H) float32, log2 units, 1e30 for rows >= L
 *   mass (map)         (H, nq, nb) float32
 *   keep               (H, nq, nb) uint8
 *   counts, *_counts   (nq, H) int32
 *   blocks, means      (nq, H, nk) int32 (ascending block ids, nk >= nb)
 *   refine             (nq, H, rw) int32 padded with nb
 *   exact / skip bits  (H, nq, nw) int32, bit (j % 32) of word (j / 32) = block j
 *   k_mean, v_mean     (nb, H, D) bf16
 *   k_rep, v_rep       (H, (nb + 1) * 4, D) bf16, block nb is an empty sentinel
 *   log_counts         (H, (nb + 1) * 4) float32
 *   scale_exact/_skip  (H, nq) float32
 * with nq = ceil(L / 128) query tiles and nb = ceil(L / 64) kv blocks. Each entry point cites the reference
 * function it replaces (paths relative to the reference tree).
 */
#ifndef ECHOSPARSE_HIP_H
#define ECHOSPARSE_HIP_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ES_ABI_VERSION 2  /* 2: lc_mid_stride, lc_stride, and the k-means labels / mid_counts of vsa_rep_unpool */

enum es_status {
  ES_OK = 0,
  ES_ERR_INVALID = 1,     /* bad pointer, size or shape */
  ES_ERR_UNSUPPORTED = 2, /* valid but not supported here (e.g. D != 128) */
  ES_ERR_LAUNCH = 3       /* the HIP launch failed */
};

/* Message of the last failed call on this host thread. */
const char* es_last_error_string(void);
int es_abi_version(void);

/* ---------------------------------------------------------------- EchoSparse fixed-offset attention */

/* Full step: every listed 64-token block at the fixed offset, the per-block mass map (mass may be NULL), O, the
 * new log2 LSE and the per-tile flag. Replaces echosparse/kernels/sm90.py:118-127 block_attention. */
int es_block_attention(const void* q, const void* k, const void* v, void* out, const int* counts,
                       const int* blocks, int nk, const float* offset, float* lse, int* flags, float* mass,
                       float threshold, int L, int H, int D, hipStream_t stream);

/* Sparse step: listed blocks exactly, listed mean blocks through k_mean/v_mean (bias log2 of the block length),
 * listed refined blocks through four representatives each (bias log_counts), one softmax at the fixed offset.
 * Only the first `tiles` query tiles are computed (the caller applies launched_tiles to the rest).
 * Replaces echosparse/kernels/sm90.py:130-144 sparse_attention (kernel sm90.py:54-115). */
int es_sparse_attention(const void* q, const void* k, const void* v, const void* k_mean, const void* v_mean,
                        const int* means, const int* mean_counts, void* out, const int* counts, const int* blocks,
                        int nk, const float* offset, float* lse, int* flags, const int* refine,
                        const int* refine_counts, int rw, const void* k_rep, const void* v_rep,
                        const float* log_counts, float* mass, float threshold, int tiles, int L, int H, int D,
                        hipStream_t stream);

/* Online-softmax recompute over the block list for the tiles whose flag is set; writes O and the log2 LSE.
 * Replaces echosparse/kernels/sm120.py:143-180 exact_fallback (triton_ops.py:202-248). */
int es_exact_fallback(const void* q, const void* k, const void* v, void* out, const int* counts,
                      const int* blocks, int nk, float* lse, const int* flags, int L, int H, int D,
                      hipStream_t stream);

/* Block-mean compensation of the keep == 0 blocks for flagged tiles, in place on out and lse.
 * Replaces echosparse/kernels/triton_ops.py:251-295 compensate_fallback. */
int es_compensate_fallback(const void* q, const void* k_mean, const void* v_mean, const uint8_t* keep, float* lse,
                           void* out, const int* flags, int L, int H, int D, hipStream_t stream);

/* Dense attention (every key) with its log2 LSE in the (nq * 128, H) offset layout (1e30 past L).
 * Replaces the FlashAttention-4 call of echosparse/attention.py:33-35 / backends.py:50-59 (dense steps and the
 * LSE that seeds the offsets, attention.py:284-287). */
int es_dense_attention(const void* q, const void* k, const void* v, void* out, float* lse2, int L, int H, int D,
                       hipStream_t stream);

/* Dense attention of Lq query rows (q, out: (Lq, H, 128)) over Lk key rows (k, v: (Lk, H, 128)); log2 LSE as
 * above over the query rows. The other FlashAttention-4 calls of the pipeline integrations: Wan cross-attention
 * (echosparse/models/wan.py:26-28), the text query rows of HunyuanVideo (models/hunyuan_video.py:71) and the
 * prefix rows of MiniMax-H3 (models/minimax_h3.py:85, 92). */
int es_dense_attention_kv(const void* q, const void* k, const void* v, void* out, float* lse2, int Lq, int Lk,
                          int H, int D, hipStream_t stream);

/* ---------------------------------------------------------------- EchoSparse map, scales and plans */

/* Mean key and value of every 64-token block (tail divided by its token count), bf16.
 * Replaces echosparse/kernels/triton_ops.py:21-40 block_means. */
int es_block_means(const void* k, const void* v, void* k_mean, void* v_mean, int L, int H, int D,
                   hipStream_t stream);

/* Mass estimates of the skipped blocks (written into mass where keep == 0) and the per-tile scales.
 * offset = this step's prior, lse = this step's new LSE.
 * Replaces echosparse/kernels/triton_ops.py:122-177 estimate_skipped (sm120.py:183-250 computes the same). */
int es_estimate_skipped(const void* q, const void* k_mean, const uint8_t* keep, const float* offset,
                        const float* lse, float* mass, float* scale_exact, float* scale_skip, int L, int H, int D,
                        hipStream_t stream);

/* Scales after a full step; resets lse rows >= L to 1e30.
 * Replaces echosparse/kernels/triton_ops.py:180-199 full_step_scales. */
int es_full_step_scales(const float* offset, float* lse, float* scale_exact, float* scale_skip, int L, int H,
                        hipStream_t stream);

/* Top-k blocks per (tile, head) by scaled block probability plus forced (own blocks +-1, sink) blocks, the
 * refine list (top-r skipped blocks by raw map, index tie cut) and the skip bit mask. Bit-exact.
 * Replaces echosparse/kernels/triton_ops.py:57-119 select_blocks. */
int es_select_blocks(const float* mass, const uint8_t* keep_prev, const float* scale_exact,
                     const float* scale_skip, uint8_t* keep, int* counts, int* blocks, const int* flags,
                     int* skip_bits, int nw, int* refine, int rw, int k, int r, int L, int H, int sink,
                     hipStream_t stream);

/* keep -> exact bit mask (bits past nb set). Replaces echosparse/kernels/sm120.py:258-273 pack_plan. */
int es_pack_plan(const uint8_t* keep, int* exact_bits, int nw, int H, int nq, int nb, hipStream_t stream);

/* Bit plans -> keep, exact list, refine list (padded with nb), mean list and their counts.
 * Replaces echosparse/kernels/sm120.py:276-305 rebuild_plan. */
int es_rebuild_plan(const int* exact_bits, const int* skip_bits, int nw, uint8_t* keep, int* counts, int* blocks,
                    int* refine, int* refine_counts, int rw, int* means, int* mean_counts, int H, int nq, int nb,
                    hipStream_t stream);

/* ---------------------------------------------------------------- representatives */

/* Bytes of device workspace es_representatives needs for (L, H, D). */
size_t es_representatives_workspace(int L, int H, int D);

/* Four representatives per block by weighted Lloyd k-means in the query metric, with log2 cluster sizes, and
 * (when k_mean != NULL) the block means. k_rep / v_rep / log_counts must hold the empty sentinel block nb
 * (zeros, -inf) from the caller's initialisation; it is not written.
 * Replaces echosparse/kernels/representatives.py:131-166 Representatives.build (kernels :22-128). */
int es_representatives(const void* q, const void* k, const void* v, void* k_rep, void* v_rep, float* log_counts,
                       void* k_mean, void* v_mean, void* workspace, size_t workspace_bytes, int iters, int L,
                       int H, int D, hipStream_t stream);

/* es_representatives without a workspace argument, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. Same kernels and
 * results as es_representatives; the workspace is a 48 MiB device array inside the library (one per GPU, held
 * until the process ends), so it calls no allocator. Rejects (ES_ERR_UNSUPPORTED) any (L, H) whose
 * es_representatives_workspace exceeds es_representatives_noalloc_limit() bytes (Wan2.1-14B, L = 75 600 and
 * H = 40, needs 44 MB). Calls that overlap on one GPU share the array and race: serialise them. */
size_t es_representatives_noalloc_limit(void);
int es_representatives_noalloc(const void* q, const void* k, const void* v, void* k_rep, void* v_rep,
                               float* log_counts, void* k_mean, void* v_mean, int iters, int L, int H, int D,
                               hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
