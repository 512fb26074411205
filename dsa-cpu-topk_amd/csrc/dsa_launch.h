// dsa_launch.h -- internal host-side launchers (C++ linkage, not exported).
// capi.cpp validates arguments and then calls these; each one enqueues its
// kernels on `stream` and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

// Radix-select: thr[r] = k-th largest of row r, optional exactly-k indices.
hipError_t launch_topk(const float* scores, int64_t rows, int64_t n, int64_t ld, int k,
                       int64_t causal_T, float* thr, int32_t* idx, hipStream_t stream);
// Causal thresholds of a [B,T,T] score matrix plus the rows' selection
// bitmask (what launch_selection_mask writes), in one pass over the scores
// where the bracket kernel serves the rows; otherwise the two launches.
hipError_t launch_topk_mask(const float* scores, int64_t B, int64_t T, int64_t ld, int k,
                            float* thr, uint64_t* mask, int64_t ldm, hipStream_t stream);

// Lightning indexer.  dtype: 0 f32, 1 bf16, 2 f16, 3 fp8 e4m3 (w fp32).
// ldq / ldk / ldw: elements from one token's q / k / w row to the next
// (HI*DI, DI, HI for packed tensors; a batch element spans T rows).
// dtype 3 only: q_scale [B*T, HI] and k_scale [B*T] fp32 positive scales
// (either may be null), I = sum_j w * ReLU(q_scale*k_scale*<q8, k8>).
hipError_t launch_indexer(const void* q, const void* k, const void* w, int dtype, int64_t B,
                          int64_t T, int HI, int DI, int64_t ldq, int64_t ldk, int64_t ldw,
                          float* scores, int64_t ld, int write_upper, hipStream_t stream,
                          const float* q_scale = nullptr, const float* k_scale = nullptr);
bool indexer_supported(int dtype, int DI);
bool indexer_fp8_fits(int HI, int DI);  // the fp8 kernel's 4-query tile fits LDS

// Threshold-driven sparse attention.  ws / ws_bytes: device workspace for
// the staged kernel's split tiles (sparse_attn_workspace_bytes; null or too
// small: the staged kernel runs every tile as one chunk).
hipError_t launch_sparse_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, int DV, float scale, float* out, void* ws,
                              int64_t ws_bytes, hipStream_t stream);
// Workspace bytes with which launch_sparse_attn (staged = false) or
// launch_staged_attn (staged = true) splits the staged kernel's long tiles;
// 0 when that launch uses no workspace for this shape.
int64_t sparse_attn_workspace_bytes(bool staged, int dtype, int64_t B, int64_t T, int HQ, int DQ,
                                    int DV, int64_t ld);
bool sparse_attn_supported(int dtype, int HQ, int DQ, int DV);
// The per-query gather kernel alone (launch_sparse_attn may pick tiles), and
// whether it splits a row into head chunks for this shape.
hipError_t launch_sparse_attn_gather(const float* scores, int64_t ld, const float* thr,
                                     const void* Q, const void* K, const void* V, int dtype,
                                     int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                     float* out, hipStream_t stream);
bool sparse_attn_chunked(int dtype, int HQ, int DQ, int DV);

// The same attention as dense-masked MFMA tiles (tile_attn.hip).  The
// threshold entry point switches to it at T >= kTiledMinT when it applies.
constexpr int64_t kTiledMinT = 4096;
// The tile kernel addresses 128 score rows (fp32) with 32-bit byte offsets.
constexpr int64_t kTileMaxLd = (int64_t{1} << 22) - 1;
// Whether launch_sparse_attn takes the tile kernel for this shape (16-bit,
// DQ = DV in {64, 128}, and T >= kTiledMinT or heads too wide to gather).
bool sparse_attn_uses_tiles(int dtype, int64_t T, int HQ, int DQ, int DV);
bool tile_attn_supported(int dtype, int HQ, int DQ, int DV, const void* Q, const void* K,
                         const void* V);
hipError_t launch_tile_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                            const void* K, const void* V, int dtype, int64_t B, int64_t T, int HQ,
                            int D, float scale, float* out, hipStream_t stream);
// The tile kernel reading its selection from a bitmask (selection_mask),
// and the kernel that builds that bitmask from scores and thresholds.
hipError_t launch_tile_attn_mask(const uint64_t* mask, int64_t ldm, const void* Q, const void* K,
                                 const void* V, int dtype, int64_t B, int64_t T, int HQ, int D,
                                 float scale, float* out, hipStream_t stream);
hipError_t launch_selection_mask(const float* scores, int64_t ld, const float* thr, int64_t B,
                                 int64_t T, uint64_t* mask, int64_t ldm, hipStream_t stream);
// The bitmask path with the bitmask in a static per-GPU array of
// kScratchWords words (32 MiB: B*T*ceil(T/64) <= 2^22, e.g. B=1, T=16384).
constexpr int64_t kScratchWords = int64_t{1} << 22;
hipError_t launch_sparse_attn_mask_noalloc(const float* scores, int64_t ld, const float* thr,
                                           const void* Q, const void* K, const void* V, int dtype,
                                           int64_t B, int64_t T, int HQ, int D, float scale,
                                           float* out, hipStream_t stream);

// The same attention with each block's causal K/V rows staged through LDS
// (staged_attn.hip): rows of 64*E elements, DQ = DV, E in {4, 8} for fp32
// and 8 for 16-bit.  The threshold entry point switches to it at
// T >= kStagedMinT when it applies and the tile kernel does not.
constexpr int64_t kStagedMinT = 3072;
bool staged_attn_supported(int dtype, int HQ, int DQ, int DV);
// Whether the threshold entry point takes the staged kernel: fp32 rows of
// 512 elements (E = 8) only, T >= kStagedMinT, and either a workspace for
// split key ranges (`split`) or at least half a block of tile pairs per
// compute unit.  For fp32 rows of 256 elements and 16-bit rows the per-query
// gathers measured faster on MI355X (B=2, T=4096, HQ=4, D=64, k=256: 0.17
// against 0.30 ms split; bf16 HQ=8 at T=3072: 0.15 against 0.30).
bool staged_attn_auto(int dtype, int64_t B, int64_t T, int HQ, int DQ, int DV, bool split);
// Compute units of the current device (cached per thread), 0 if unknown.
int device_cus();
// Its score copies address one batch element's [T, ld] rows with 32-bit
// buffer offsets.
constexpr int64_t kStagedMaxScoreBytes = int64_t{1} << 31;
inline bool staged_attn_fits(int64_t T, int64_t ld) { return T * ld * 4 < kStagedMaxScoreBytes; }
// Work items (64-query tile, key chunk) of one batch element, passed in the
// kernel arguments.
constexpr int kStagedMaxItems = 896;
// How the staged kernel assigns its blocks.  kStagedPairs: each block takes
// the 32-query tiles p and ntile-1-p and streams their causal keys.
// kStagedGroups: each block takes a 64-query group (queries 64m ..
// 64m+63) and streams its causal keys.  kStagedSplit: each block takes a
// 64-query group and a chunk of at most CK of its causal keys; groups
// q_split .. q_split + nsplit - 1 are split, into at most ncmax chunks, and
// their partial sums take ws_bytes of workspace (part_bytes of rows, then
// the per-head running max and sum).  The first two use no workspace.
enum { kStagedPairs = 0, kStagedGroups = 1, kStagedSplit = 2 };
struct StagedPlan {
  int mode;
  int CK;
  int q_split;
  int nsplit;
  int ncmax;
  int64_t part_bytes;
  int64_t ws_bytes;
};
StagedPlan staged_attn_plan(int64_t B, int64_t T, int HQ, int DQ, bool split);
hipError_t launch_staged_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, float scale, float* out, void* ws, int64_t ws_bytes,
                              hipStream_t stream);

// Fused forward for T <= kFusedMaxT.
constexpr int64_t kFusedMaxT = 2048;
hipError_t launch_fused(const void* qi, const void* ki, const void* wi, const void* Q,
                        const void* K, const void* V, int dtype, int64_t B, int64_t T, int HI,
                        int DI, int HQ, int DQ, int DV, int top_k, float scale, float* out,
                        hipStream_t stream);

}  // namespace dsa
