/*
 * dsa_amd.h -- C ABI of the MI355X (gfx950) DeepSeek Sparse Attention forward.
 *
 * One shared library, libdsa_amd.so, built with hipcc for gfx950 only.  Every
 * entry point:
 *   - takes plain device pointers, sizes and a hipStream_t passed as void*
 *     (NULL = the legacy default stream);
 *   - enqueues its kernels on that stream and returns without synchronising;
 *   - never allocates, frees or synchronises device memory;
 *   - returns DSA_OK (0), a negative code for an argument the caller got wrong
 *     (the Python layer raises AssertionError, as the reference's asserts do),
 *     or a positive code for a HIP runtime failure (RuntimeError);
 *   - records a message for any non-zero return, read back with
 *     dsa_last_error() on the same thread.
 * Arguments are validated before any HIP call, so a wrong argument is reported
 * without touching a GPU.
 *
 * Layouts are dense row-major (C-contiguous), as the reference wrappers make
 * them with .contiguous() before launching:
 *   q_idx [B,T,HI,DI]   k_idx [B,T,DI]   w_idx [B,T,HI]        (dtype below)
 *   Q,K   [B,T,HQ,DQ]   V     [B,T,HQ,DV]                     (dtype below)
 *   scores [B,T,T] fp32 (row stride ld >= T)   thr [B*T] fp32   O [B,T,HQ,DV] fp32
 */
#ifndef DSA_AMD_H
#define DSA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of q_idx/k_idx/w_idx and Q/K/V.  Arithmetic is fp32 in every
 * case: 16-bit inputs feed MFMA with fp32 accumulation (products are exact),
 * fp32 inputs use the fp32 MFMA.  Outputs are always fp32, as the reference's
 * Triton wrappers allocate them (dsa_attention.py:210, :309). */
enum dsa_dtype { DSA_F32 = 0, DSA_BF16 = 1, DSA_F16 = 2,
                 /* dsa_indexer_scores only: q_idx/k_idx OCP FP8 E4M3
                  * (torch.float8_e4m3fn, unscaled), w_idx fp32.  Products are
                  * exact in the fp32 accumulator of the fp8 MFMA. */
                 DSA_FP8 = 3 };

enum dsa_status {
  DSA_OK = 0,
  DSA_EINVAL = -1,       /* bad size, null pointer, k out of range, ...     */
  DSA_EUNSUPPORTED = -2, /* a shape this build has no kernel for            */
  DSA_EHIP = 1           /* a HIP runtime call failed (message says which)  */
};

/* Thread-local text of the last non-zero return on this thread. */
const char* dsa_last_error(void);

/* Library version string ("dsa_amd <semver> gfx950"). */
const char* dsa_version(void);

/*
 * Lightning indexer scores.
 *   scores[b,t,s] = sum_j w[b,t,j] * ReLU(<q[b,t,j,:], k[b,s,:]>)   for s <= t
 *   scores[b,t,s] = -inf                                              for s >  t
 * The upper triangle (s > t) is written only when write_upper != 0; the
 * internal split pipeline skips it because nothing reads it.
 * Replaces: _indexer_score_kernel + indexer_scores_triton,
 *           reference lightning_indexer.py:54-125 (torch form :26-33).
 * Constraints: B,T >= 1; 1 <= HI <= 256; DI in {16,32,64,128,256} (fp32) or
 *              {32,64,128,256} (bf16/fp16) or {64,128,256} (fp8, with
 *              ceil(HI/4) * (16*DI + 64) <= 160 KiB, e.g. HI*DI <= 32768
 *              for HI a multiple of 4 and DI >= 128); ld >= T.
 */
int dsa_indexer_scores(const void* q_idx, const void* k_idx, const void* w_idx,
                       int dtype, int64_t B, int64_t T, int HI, int DI,
                       float* scores, int64_t ld, int write_upper,
                       void* stream);

/*
 * dsa_indexer_scores for q_idx / k_idx / w_idx whose consecutive tokens are
 * ldq / ldk / ldw elements apart (a batch element spans T such rows), e.g.
 * the three column ranges of one projection GEMM's output [B*T, HI*DI+DI+HI],
 * read in place.  ldq >= HI*DI, ldk >= DI, ldw >= HI; ldq and ldk (in bytes)
 * and the q_idx / k_idx pointers 16-byte aligned; T*ldk < 2^31.
 * No reference counterpart: it fuses the front end of indexer_triton
 * (reference lightning_indexer.py:128-130, projection :36-47), whose three
 * separate projections produce packed tensors.
 */
int dsa_indexer_scores_strided(const void* q_idx, const void* k_idx, const void* w_idx,
                               int dtype, int64_t B, int64_t T, int HI, int DI,
                               int64_t ldq, int64_t ldk, int64_t ldw,
                               float* scores, int64_t ld, int write_upper,
                               void* stream);

/*
 * FP8 (E4M3) indexer with quantisation scales: q_idx and k_idx as e4m3 with
 * a positive fp32 scale per (token, head) of q_idx and per token of k_idx,
 * the layout of a block-128 (per head row) activation quantisation:
 *   scores[b,t,s] = sum_j w[b,t,j] * ReLU(q_scale[b,t,j] * k_scale[b,s] *
 *                                         <q8[b,t,j,:], k8[b,s,:]>)   for s <= t
 * (-inf above the diagonal when write_upper).  With positive scales this is
 * the indexer of the dequantised q and k; q_scale is folded into w and
 * k_scale multiplies each finished score, so the MFMA work is the unscaled
 * fp8 kernel's.  Either scale pointer may be NULL (scale 1).
 *   q_scale [B,T,HI] fp32, k_scale [B,T] fp32 (contiguous, 4-byte aligned);
 *   w_idx [B,T,HI] fp32.  Other arguments and constraints as
 *   dsa_indexer_scores with dtype DSA_FP8.
 * Scales must be positive and finite (a zero or negative scale does not
 * commute with the ReLU); quantisation scales (amax / 448) are.
 * Replaces: the scaling and dequantisation inside the indexer that the
 *   reference lists as its FP8 follow-up (DEVLOG.md:203-205); the indexer
 *   itself is lightning_indexer.py:54-125.
 */
int dsa_indexer_scores_fp8_scaled(const void* q_idx, const void* k_idx, const void* w_idx,
                                  const float* q_scale, const float* k_scale, int64_t B,
                                  int64_t T, int HI, int DI, float* scores, int64_t ld,
                                  int write_upper, void* stream);

/*
 * Per-row k-th largest ("top-K threshold") with an optional exactly-k index set.
 *   thr[r] = k-th largest of row r, ties counted (torch.topk(x,k).values[...,-1]).
 *   idx[r*k .. r*k+k) (optional, may be NULL) = the k positions a stable
 *   descending sort of row r puts first -- every entry above thr[r] plus the
 *   lowest-index entries equal to thr[r] -- written in ascending index order.
 * causal_T == 0: every row has n valid entries.
 * causal_T  > 0: row r is query t = r % causal_T of a [B,T,T] score matrix;
 *   only its first t+1 entries are read and the rest count as -inf, exactly as
 *   the reference's masked full row (dsa_attention.py:41-44): rows with
 *   t+1 < k get thr = -inf.
 * -0.0 and +0.0 compare equal; NaN ranks above +inf (as in torch.topk).
 * Replaces: topk_threshold / topk_threshold_batch_merge, reference
 *   topk_avx512.cpp:226-264, and scores.topk(...)[..., -1:] at
 *   dsa_attention.py:343-344 (and the in-kernel tl.sort at :151-155).
 * Constraints: rows >= 0; 1 <= k <= n; ld >= n; n < 2^31.
 */
int dsa_topk_threshold(const float* scores, int64_t rows, int64_t n, int64_t ld,
                       int k, int64_t causal_T, float* thr, int32_t* idx,
                       void* stream);

/*
 * Sparse attention restricted to keys whose indexer score passes a threshold.
 *   sel(b,t,s) = (s <= t) && (scores[b,t,s] >= thr[b*T+t])   (ties kept)
 *   O[b,t,h,:] = sum_{s in sel} softmax_s(<Q[b,t,h],K[b,s,h]> * scale) V[b,s,h,:]
 * Rows that select nothing (only possible for a NaN or +inf threshold) get
 * O = NaN, the 0/0 of a softmax over an all -inf row, as in the reference's
 * kernel and torch path.  The threshold may come from anywhere (the reference's hybrid path
 * computes it on the CPU, dsa_hybrid.py:61-66).
 * Replaces: _sparse_attn_kernel + sparse_attention_with_threshold_triton,
 *           reference dsa_attention.py:234-324.
 * Kernels (chosen by shape, same sel and O): per-query gathers (fp32 rows
 *   of HQ*DQ = 128 elements with Q, K, V and out 16-byte aligned load two
 *   keys per wave instruction, one per half-wave; the sums then run in
 *   another order, so results differ from the one-key form in the last
 *   bits); rows wider than one wave holds (fp32 HQ*D > 1024, 16-bit > 2048)
 *   in head chunks;
 *   the tile kernel below for 16-bit DQ = DV in {64,128} at T >= 4096 or on
 *   wide rows; the staged kernel below for fp32 rows of HQ*DQ = 512 at
 *   T >= 3072 when B*ceil(T/64) is at least the compute-unit count.
 * Constraints: HQ, DQ, DV powers of two; a single head of at most 64*16
 *   (fp32) or 64*32 (16-bit) elements; T*HQ*max(DQ,DV)*bytes < 4 GiB;
 *   ld >= T.
 */
int dsa_sparse_attn_threshold(const float* scores, int64_t ld, const float* thr,
                              const void* Q, const void* K, const void* V,
                              int dtype, int64_t B, int64_t T, int HQ, int DQ,
                              int DV, float scale, float* out, void* stream);

/*
 * dsa_sparse_attn_threshold with a device workspace: where it takes the
 * staged kernel, that kernel splits the causal keys of its long query tiles
 * into chunks run by separate blocks (the blocks then stream about the same
 * number of keys each) and a second launch combines the chunks' partial
 * softmax sums.  workspace_bytes below what
 * dsa_sparse_attn_workspace_bytes(0, ...) returns (or a null or
 * non-16-byte-aligned workspace) runs without the split, as
 * dsa_sparse_attn_threshold does.  The workspace is device memory of the
 * stream's device that no other work uses until the launches complete; its
 * contents on entry do not matter.  Same sel and O (the chunks' sums are
 * combined in another order: results differ in the last bits).
 * Replaces: sparse_attention_with_threshold_triton's launch,
 *           reference dsa_attention.py:234-324 (same contract as above);
 *           the workspace has no counterpart there.
 */
int dsa_sparse_attn_threshold_ws(const float* scores, int64_t ld, const float* thr,
                                 const void* Q, const void* K, const void* V,
                                 int dtype, int64_t B, int64_t T, int HQ, int DQ,
                                 int DV, float scale, float* out, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes with which dsa_sparse_attn_threshold_ws (staged = 0) or
 * dsa_sparse_attn_threshold_staged_ws (staged = 1) splits the staged
 * kernel's long tiles on the current device (the split follows its
 * compute-unit count); 0 when that call uses no workspace for the shape.
 * No counterpart in the reference (its Triton launch allocates nothing).
 */
int64_t dsa_sparse_attn_workspace_bytes(int staged, int dtype, int64_t B, int64_t T, int HQ,
                                        int DQ, int DV, int64_t ld);

/*
 * dsa_sparse_attn_threshold computed as dense-masked MFMA tiles: the same
 * sel and O, evaluated over the causal triangle in 128-query x 64-key tiles
 * with the selection as a mask, so every K/V tile a block loads serves 128
 * queries.  dsa_sparse_attn_threshold switches to it by itself for
 * T >= 4096 when the shape qualifies; this entry point runs it at any T.
 * P is rounded to the 16-bit input type for the P.V product (fp32
 * accumulation), inside the 16-bit tolerance.
 * Replaces: _sparse_attn_kernel + sparse_attention_with_threshold_triton,
 *           reference dsa_attention.py:234-324 (same contract as above).
 * Constraints: bf16/fp16 Q/K/V; DQ = DV in {64,128}; 1 <= HQ <= 1024;
 *   ld >= T; Q, K, V, out 16-byte aligned.  Other shapes return
 *   DSA_EUNSUPPORTED.
 */
int dsa_sparse_attn_threshold_tiled(const float* scores, int64_t ld, const float* thr,
                                    const void* Q, const void* K, const void* V,
                                    int dtype, int64_t B, int64_t T, int HQ, int DQ,
                                    int DV, float scale, float* out, void* stream);

/*
 * dsa_sparse_attn_threshold with each block's causal K/V rows staged through
 * LDS: a block takes 64 consecutive queries and streams their causal keys
 * once, in tiles of 16 keys copied by DMA, and every wave computes its
 * queries' selected pairs from LDS -- nearby queries select over the same
 * key range, so the K/V bytes read from L2/MALL drop by the block's query
 * count compared with per-query gathers.  Blocks run longest first.
 * dsa_sparse_attn_threshold switches to it by itself for fp32 rows of
 * HQ*DQ = 512 at T >= 3072 when B*ceil(T/64) is at least the compute-unit
 * count (other shapes measured faster with the gathers); this entry point
 * runs it at any T.  Same sel and O, fp32 arithmetic (the softmax sums in a
 * different order than the gathers).  Without a workspace every block
 * streams its tile's whole causal range; the _ws form below splits long
 * ranges.
 * Replaces: _sparse_attn_kernel + sparse_attention_with_threshold_triton,
 *           reference dsa_attention.py:234-324 (same contract as above).
 * Constraints: DQ = DV; HQ*DQ = 256 or 512 (fp32) or 512 (bf16/fp16) with
 *   DQ a multiple of HQ*DQ/64; ld >= T; T*ld*4 < 2^31 (one batch element's
 *   score rows are addressed with 32-bit offsets); Q, K, V, out 16-byte
 *   aligned.  Other shapes return DSA_EUNSUPPORTED.
 */
int dsa_sparse_attn_threshold_staged(const float* scores, int64_t ld, const float* thr,
                                     const void* Q, const void* K, const void* V,
                                     int dtype, int64_t B, int64_t T, int HQ, int DQ,
                                     int DV, float scale, float* out, void* stream);

/*
 * dsa_sparse_attn_threshold_staged with the workspace of
 * dsa_sparse_attn_threshold_ws (size from
 * dsa_sparse_attn_workspace_bytes(1, ...)): long key ranges are split into
 * chunks, and a second launch combines them.
 * Replaces: as dsa_sparse_attn_threshold_staged; the workspace has no
 *           counterpart in the reference.
 */
int dsa_sparse_attn_threshold_staged_ws(const float* scores, int64_t ld, const float* thr,
                                        const void* Q, const void* K, const void* V,
                                        int dtype, int64_t B, int64_t T, int HQ, int DQ,
                                        int DV, float scale, float* out, void* workspace,
                                        int64_t workspace_bytes, void* stream);

/*
 * Selection bitmask of the threshold selection, for dsa_sparse_attn_mask.
 * Row (b, t) of `mask` (ldm 64-bit words per row, ldm >= ceil(T/64)):
 * bit i of word w is set iff key s = 64w + i has s <= t and
 * scores[b,t,s] >= thr[b*T+t] (NaN scores or thresholds select nothing) --
 * the selection dsa_sparse_attn_threshold applies.  Words 0 ..
 * min(ceil(T/64)-1, (t|127)/64) of each row are written (those past the
 * causal range are 0): every word dsa_sparse_attn_mask reads for that row.
 * Replaces: the `scores >= thr` mask of _sparse_attn_kernel,
 *           reference dsa_attention.py:265-290, computed once per (t, s)
 *           instead of once per (t, s, head) -- no reference counterpart as
 *           a separate call.
 * Constraints: ld >= T; mask 8-byte aligned.
 */
int dsa_selection_mask(const float* scores, int64_t ld, const float* thr, int64_t B,
                       int64_t T, uint64_t* mask, int64_t ldm, void* stream);

/*
 * dsa_topk_threshold (causal, causal_T = T, rows = B*T, n = T) and
 * dsa_selection_mask of its thresholds in one call: the same thr and mask,
 * bit for bit.  Where the select's single-pass kernel serves the rows (rows
 * above 4096 entries), that kernel writes each row's bitmask words as soon as
 * it has the row's threshold: from the flag bitmap it keeps of the row (rows
 * up to 16384 entries), else by re-reading the row it has just streamed;
 * other shapes run the two launches.  This is the
 * split forward's select step when its attention runs on tiles.
 * Replaces: scores.topk(...)[..., -1:] at dsa_attention.py:343-344 followed
 *           by the `scores >= thr` selection of _sparse_attn_kernel
 *           (dsa_attention.py:265-290); no reference counterpart as one call.
 * Constraints: 1 <= k <= T < 2^31; B*T < 2^31; ld >= T;
 *   ldm >= ceil(T/64); mask 8-byte aligned.
 */
int dsa_topk_threshold_mask(const float* scores, int64_t B, int64_t T, int64_t ld, int k,
                            float* thr, uint64_t* mask, int64_t ldm, void* stream);

/*
 * Sparse attention with the selection read from a dsa_selection_mask
 * bitmask: the dense-masked MFMA tile kernel, which reads 1 bit per
 * (query, key) instead of a 4-byte score (per head).  Together with
 * dsa_selection_mask the same result, bit for bit, as the tile kernel of
 * dsa_sparse_attn_threshold / dsa_sparse_attn_threshold_tiled on the same
 * scores and thresholds.
 * Replaces: _sparse_attn_kernel + sparse_attention_with_threshold_triton
 *           (reference dsa_attention.py:234-324) where it runs on tiles.
 * Constraints: bf16/fp16; DQ = DV in {64, 128}; ldm >= ceil(T/64),
 *   ldm < 2^21; T*HQ*D*2 < 4 GiB; Q, K, V, out 16-byte aligned, mask
 *   8-byte aligned.  Other shapes return DSA_EUNSUPPORTED.
 */
int dsa_sparse_attn_mask(const uint64_t* mask, int64_t ldm, const void* Q, const void* K,
                         const void* V, int dtype, int64_t B, int64_t T, int HQ, int DQ,
                         int DV, float scale, float* out, void* stream);

/*
 * dsa_selection_mask + dsa_sparse_attn_mask in one call that allocates
 * nothing: the bitmask goes into a static device array of the library
 * (32 MiB per GPU the library runs on, held until the process ends), so
 * the caller passes only what dsa_sparse_attn_threshold takes.  Same output,
 * bit for bit, as that pair (and as the tile kernel of
 * dsa_sparse_attn_threshold_tiled).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).
 * Limit: B*T*ceil(T/64) <= 2^22 (B=1, T=16384 fits); larger inputs return
 *   DSA_EINVAL.  Shapes: those of dsa_sparse_attn_mask (bf16/fp16,
 *   DQ = DV in {64, 128}); ld >= T.  Calls that overlap in time on one GPU
 *   share the array and race; the device is the current one.
 * Graph capture: a device's first call looks up the array's address
 *   (hipGetSymbolAddress), so make that first call eagerly, outside any
 *   capture; later calls enqueue kernels only (no memset, no allocation)
 *   and may be captured.
 */
int dsa_sparse_attn_mask_noalloc(const float* scores, int64_t ld, const float* thr,
                                 const void* Q, const void* K, const void* V, int dtype,
                                 int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                 float* out, void* stream);

/*
 * 1 if dsa_sparse_attn_threshold runs this shape on the tile kernel (so
 * dsa_selection_mask + dsa_sparse_attn_mask apply and give its result),
 * else 0.  Pure function of the arguments.
 */
int dsa_sparse_attn_uses_mask(int dtype, int64_t T, int HQ, int DQ, int DV);

/*
 * Fused DSA forward for T <= 2048: indexer -> per-row radix select ->
 * sparse attention in one kernel; the score rows live in LDS only.
 * Same result as dsa_indexer_scores + dsa_topk_threshold(k = min(top_k,T),
 * causal) + dsa_sparse_attn_threshold (the attention gathers as that entry's
 * per-query gathers do, two keys per load under the same conditions).
 * Replaces: _dsa_fused_kernel + dsa_attention_triton,
 *           reference dsa_attention.py:96-227.
 * Constraints: 1 <= T <= 2048; 1 <= top_k; the indexer's and the sparse
 *   attention's head/dim constraints.
 */
int dsa_fused_forward(const void* q_idx, const void* k_idx, const void* w_idx,
                      const void* Q, const void* K, const void* V, int dtype,
                      int64_t B, int64_t T, int HI, int DI, int HQ, int DQ,
                      int DV, int top_k, float scale, float* out, void* stream);

/* Largest T dsa_fused_forward accepts (2048). */
int64_t dsa_fused_max_T(void);

#ifdef __cplusplus
}
#endif

#endif /* DSA_AMD_H */
