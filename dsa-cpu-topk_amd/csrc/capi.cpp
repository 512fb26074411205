// capi.cpp -- the exported C ABI (include/dsa_amd.h): argument validation,
// error reporting and dispatch to the gfx950 launchers.
//
// Every check runs before the first HIP call, so invalid arguments are
// reported (negative status + message) on a machine without a GPU.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/dsa_amd.h"
#include "dsa_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return DSA_OK;
  return fail(DSA_EHIP, "%s: HIP error %d (%s)", what, static_cast<int>(e), hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
bool dtype_ok(int d) { return d == DSA_F32 || d == DSA_BF16 || d == DSA_F16; }

// Elements of a 16-bit or 32-bit tensor fit the 32-bit indices some kernels use.
constexpr int64_t kMaxElems = (int64_t{1} << 31) - 1;

int check_indexer(const void* q, const void* k, const void* w, int dtype, int64_t B, int64_t T,
                  int HI, int DI, const float* scores, int64_t ld) {
  if (!dtype_ok(dtype) && dtype != DSA_FP8) return fail(DSA_EINVAL, "indexer: unknown dtype %d", dtype);
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "indexer: negative size B=%lld T=%lld", (long long)B, (long long)T);
  if (T > kMaxElems) return fail(DSA_EINVAL, "indexer: T=%lld too large", (long long)T);
  // the kernels index one batch element's k_idx rows with 32-bit offsets
  if (T * static_cast<int64_t>(DI > 0 ? DI : 0) > kMaxElems)
    return fail(DSA_EINVAL, "indexer: T*DI = %lld must be < 2^31", (long long)(T * static_cast<int64_t>(DI)));
  if (HI < 1 || HI > 256) return fail(DSA_EINVAL, "indexer: HI=%d outside [1,256]", HI);
  if (ld < T) return fail(DSA_EINVAL, "indexer: ld=%lld < T=%lld", (long long)ld, (long long)T);
  if (!dsa::indexer_supported(dtype, DI))
    return fail(DSA_EUNSUPPORTED, "indexer: DI=%d unsupported for dtype %d (fp32: 16..256, 16-bit: 32..256, fp8: 64..256, powers of two)", DI, dtype);
  if (dtype == DSA_FP8 && !dsa::indexer_fp8_fits(HI, DI))
    return fail(DSA_EUNSUPPORTED, "indexer: fp8 q tile of HI=%d DI=%d exceeds LDS (ceil(HI/4)*(16*DI+64) <= 160 KiB)", HI, DI);
  if (B * T == 0) return DSA_OK;
  if (!q || !k || !w || !scores) return fail(DSA_EINVAL, "indexer: null pointer");
  if (!aligned16(q) || !aligned16(k)) return fail(DSA_EINVAL, "indexer: q_idx/k_idx must be 16-byte aligned");
  if (B * T * HI * static_cast<int64_t>(DI) > (int64_t{1} << 40)) return fail(DSA_EINVAL, "indexer: q_idx too large");
  return DSA_OK;
}

int check_attn(int dtype, int64_t B, int64_t T, int HQ, int DQ, int DV, const void* Q,
               const void* K, const void* V, const float* out, const char* who) {
  if (!dtype_ok(dtype)) return fail(DSA_EINVAL, "%s: unknown dtype %d", who, dtype);
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "%s: negative size", who);
  if (T > kMaxElems) return fail(DSA_EINVAL, "%s: T=%lld too large", who, (long long)T);
  if (!pow2(HQ) || !pow2(DQ) || !pow2(DV))
    return fail(DSA_EINVAL, "%s: HQ=%d DQ=%d DV=%d must be powers of 2", who, HQ, DQ, DV);
  if (!dsa::sparse_attn_supported(dtype, HQ, DQ, DV))
    return fail(DSA_EUNSUPPORTED, "%s: no kernel for HQ=%d DQ=%d DV=%d dtype %d", who, HQ, DQ, DV, dtype);
  // the gathers address one batch element's K/V rows with 32-bit byte offsets
  const int64_t esize = dtype == DSA_F32 ? 4 : 2;
  if (T * HQ * static_cast<int64_t>(DQ > DV ? DQ : DV) * esize > (int64_t{1} << 32) - 1)
    return fail(DSA_EINVAL, "%s: T*HQ*max(DQ,DV) = %lld elements of %lld bytes must be < 4 GiB", who,
                (long long)(T * HQ * static_cast<int64_t>(DQ > DV ? DQ : DV)), (long long)esize);
  if (B * ((T + 3) / 4) * static_cast<int64_t>(HQ) > (int64_t{1} << 32) - 1)
    return fail(DSA_EINVAL, "%s: B*T*HQ too large for one launch", who);
  if (B * T == 0) return DSA_OK;
  if (!Q || !K || !V || !out) return fail(DSA_EINVAL, "%s: null pointer", who);
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(out))
    return fail(DSA_EINVAL, "%s: Q/K/V/out must be 16-byte aligned", who);
  return DSA_OK;
}

}  // namespace

extern "C" {

const char* dsa_last_error(void) { return g_err; }

const char* dsa_version(void) { return "dsa_amd 0.1.0 gfx950"; }

int64_t dsa_fused_max_T(void) { return dsa::kFusedMaxT; }

int dsa_indexer_scores(const void* q_idx, const void* k_idx, const void* w_idx, int dtype,
                       int64_t B, int64_t T, int HI, int DI, float* scores, int64_t ld,
                       int write_upper, void* stream) {
  int rc = check_indexer(q_idx, k_idx, w_idx, dtype, B, T, HI, DI, scores, ld);
  if (rc != DSA_OK || B * T == 0) return rc;
  return hip_status(dsa::launch_indexer(q_idx, k_idx, w_idx, dtype, B, T, HI, DI,
                                        static_cast<int64_t>(HI) * DI, DI, HI, scores, ld,
                                        write_upper, static_cast<hipStream_t>(stream)),
                    "dsa_indexer_scores");
}

int dsa_indexer_scores_strided(const void* q_idx, const void* k_idx, const void* w_idx,
                               int dtype, int64_t B, int64_t T, int HI, int DI, int64_t ldq,
                               int64_t ldk, int64_t ldw, float* scores, int64_t ld,
                               int write_upper, void* stream) {
  int rc = check_indexer(q_idx, k_idx, w_idx, dtype, B, T, HI, DI, scores, ld);
  if (rc != DSA_OK) return rc;
  if (ldq < static_cast<int64_t>(HI) * DI || ldk < DI || ldw < HI)
    return fail(DSA_EINVAL, "indexer: row strides ldq=%lld ldk=%lld ldw=%lld below HI*DI=%lld, DI=%d, HI=%d",
                (long long)ldq, (long long)ldk, (long long)ldw, (long long)HI * DI, DI, HI);
  const int64_t esize = dtype == DSA_F32 ? 4 : dtype == DSA_FP8 ? 1 : 2;
  if ((ldq * esize) % 16 != 0 || (ldk * esize) % 16 != 0)
    return fail(DSA_EINVAL, "indexer: ldq and ldk must be multiples of 16 bytes (ldq=%lld ldk=%lld elements)",
                (long long)ldq, (long long)ldk);
  if (T * ldk > kMaxElems) return fail(DSA_EINVAL, "indexer: T*ldk must be < 2^31");
  if (B * T == 0) return DSA_OK;
  return hip_status(dsa::launch_indexer(q_idx, k_idx, w_idx, dtype, B, T, HI, DI, ldq, ldk, ldw,
                                        scores, ld, write_upper, static_cast<hipStream_t>(stream)),
                    "dsa_indexer_scores_strided");
}

int dsa_indexer_scores_fp8_scaled(const void* q_idx, const void* k_idx, const void* w_idx,
                                  const float* q_scale, const float* k_scale, int64_t B,
                                  int64_t T, int HI, int DI, float* scores, int64_t ld,
                                  int write_upper, void* stream) {
  int rc = check_indexer(q_idx, k_idx, w_idx, DSA_FP8, B, T, HI, DI, scores, ld);
  if (rc != DSA_OK || B * T == 0) return rc;
  if ((q_scale && (reinterpret_cast<uintptr_t>(q_scale) & 3u)) ||
      (k_scale && (reinterpret_cast<uintptr_t>(k_scale) & 3u)))
    return fail(DSA_EINVAL, "indexer_fp8_scaled: scales must be 4-byte aligned fp32");
  return hip_status(dsa::launch_indexer(q_idx, k_idx, w_idx, DSA_FP8, B, T, HI, DI,
                                        static_cast<int64_t>(HI) * DI, DI, HI, scores, ld,
                                        write_upper, static_cast<hipStream_t>(stream), q_scale,
                                        k_scale),
                    "dsa_indexer_scores_fp8_scaled");
}

int dsa_topk_threshold(const float* scores, int64_t rows, int64_t n, int64_t ld, int k,
                       int64_t causal_T, float* thr, int32_t* idx, void* stream) {
  if (rows < 0 || n < 0) return fail(DSA_EINVAL, "topk: negative size rows=%lld n=%lld", (long long)rows, (long long)n);
  if (k <= 0) return fail(DSA_EINVAL, "topk: k must be > 0 (got %d)", k);
  if (k > n) return fail(DSA_EINVAL, "topk: k must be <= N (k=%d, N=%lld)", k, (long long)n);
  if (n > kMaxElems) return fail(DSA_EINVAL, "topk: row length %lld >= 2^31", (long long)n);
  if (rows > kMaxElems) return fail(DSA_EINVAL, "topk: %lld rows >= 2^31", (long long)rows);
  if (ld < n) return fail(DSA_EINVAL, "topk: ld=%lld < N=%lld", (long long)ld, (long long)n);
  if (causal_T < 0) return fail(DSA_EINVAL, "topk: causal_T=%lld < 0", (long long)causal_T);
  if (causal_T > 0) {
    if (causal_T > n) return fail(DSA_EINVAL, "topk: causal_T=%lld > N=%lld", (long long)causal_T, (long long)n);
    if (rows % causal_T != 0) return fail(DSA_EINVAL, "topk: rows=%lld not a multiple of causal_T=%lld", (long long)rows, (long long)causal_T);
  }
  if (rows == 0) return DSA_OK;
  if (!scores || !thr) return fail(DSA_EINVAL, "topk: null pointer");
  return hip_status(dsa::launch_topk(scores, rows, n, ld, k, causal_T, thr, idx,
                                     static_cast<hipStream_t>(stream)),
                    "dsa_topk_threshold");
}

int dsa_topk_threshold_mask(const float* scores, int64_t B, int64_t T, int64_t ld, int k,
                            float* thr, uint64_t* mask, int64_t ldm, void* stream) {
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "topk_mask: negative size B=%lld T=%lld", (long long)B, (long long)T);
  if (k <= 0) return fail(DSA_EINVAL, "topk_mask: k must be > 0 (got %d)", k);
  if (k > T) return fail(DSA_EINVAL, "topk_mask: k must be <= T (k=%d, T=%lld)", k, (long long)T);
  if (T > kMaxElems) return fail(DSA_EINVAL, "topk_mask: T=%lld >= 2^31", (long long)T);
  if (ld < T) return fail(DSA_EINVAL, "topk_mask: ld=%lld < T=%lld", (long long)ld, (long long)T);
  if (ldm < (T + 63) / 64)
    return fail(DSA_EINVAL, "topk_mask: ldm=%lld < ceil(T/64)=%lld", (long long)ldm, (long long)((T + 63) / 64));
  if (B * T == 0) return DSA_OK;
  if (B * T > kMaxElems) return fail(DSA_EINVAL, "topk_mask: B*T=%lld rows >= 2^31", (long long)(B * T));
  if (!scores || !thr || !mask) return fail(DSA_EINVAL, "topk_mask: null pointer");
  if ((reinterpret_cast<uintptr_t>(mask) & 7u) != 0) return fail(DSA_EINVAL, "topk_mask: mask must be 8-byte aligned");
  return hip_status(dsa::launch_topk_mask(scores, B, T, ld, k, thr, mask, ldm,
                                          static_cast<hipStream_t>(stream)),
                    "dsa_topk_threshold_mask");
}

int dsa_sparse_attn_threshold_ws(const float* scores, int64_t ld, const float* thr,
                                 const void* Q, const void* K, const void* V, int dtype,
                                 int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                 float* out, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  int rc = check_attn(dtype, B, T, HQ, DQ, DV, Q, K, V, out, "sparse_attn");
  if (rc != DSA_OK) return rc;
  if (ld < T) return fail(DSA_EINVAL, "sparse_attn: ld=%lld < T=%lld", (long long)ld, (long long)T);
  if (!std::isfinite(scale)) return fail(DSA_EINVAL, "sparse_attn: scale must be finite");
  if (workspace_bytes < 0) return fail(DSA_EINVAL, "sparse_attn: negative workspace size");
  if (B * T == 0) return DSA_OK;
  if (!scores || !thr) return fail(DSA_EINVAL, "sparse_attn: null pointer");
  return hip_status(dsa::launch_sparse_attn(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, DV,
                                            scale, out, workspace, workspace_bytes,
                                            static_cast<hipStream_t>(stream)),
                    "dsa_sparse_attn_threshold");
}

int dsa_sparse_attn_threshold(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, int DV, float scale, float* out, void* stream) {
  return dsa_sparse_attn_threshold_ws(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, DV, scale,
                                      out, nullptr, 0, stream);
}

int64_t dsa_sparse_attn_workspace_bytes(int staged, int dtype, int64_t B, int64_t T, int HQ,
                                        int DQ, int DV, int64_t ld) {
  if (!dtype_ok(dtype) || B < 0 || T < 0 || T > kMaxElems || HQ < 1 || DQ < 1 || DV < 1 || ld < T)
    return 0;
  return dsa::sparse_attn_workspace_bytes(staged != 0, dtype, B, T, HQ, DQ, DV, ld);
}

int dsa_sparse_attn_threshold_tiled(const float* scores, int64_t ld, const float* thr,
                                    const void* Q, const void* K, const void* V, int dtype,
                                    int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                    float* out, void* stream) {
  if (!dtype_ok(dtype)) return fail(DSA_EINVAL, "sparse_attn_tiled: unknown dtype %d", dtype);
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "sparse_attn_tiled: negative size");
  if (T > kMaxElems) return fail(DSA_EINVAL, "sparse_attn_tiled: T=%lld too large", (long long)T);
  if (HQ < 1 || HQ > 1024) return fail(DSA_EINVAL, "sparse_attn_tiled: HQ=%d outside [1,1024]", HQ);
  if (ld < T) return fail(DSA_EINVAL, "sparse_attn_tiled: ld=%lld < T=%lld", (long long)ld, (long long)T);
  if (!std::isfinite(scale)) return fail(DSA_EINVAL, "sparse_attn_tiled: scale must be finite");
  if (dtype == DSA_F32 || DQ != DV || (DQ != 64 && DQ != 128))
    return fail(DSA_EUNSUPPORTED, "sparse_attn_tiled: needs bf16/fp16 and DQ = DV in {64,128} (dtype %d DQ=%d DV=%d)", dtype, DQ, DV);
  // the tile DMA addresses one batch element's K/V rows with 32-bit byte offsets
  if (T * HQ * static_cast<int64_t>(DQ) * 2 > (int64_t{1} << 32) - 1)
    return fail(DSA_EINVAL, "sparse_attn_tiled: T*HQ*D = %lld 16-bit elements must be < 4 GiB",
                (long long)(T * HQ * static_cast<int64_t>(DQ)));
  if (ld > dsa::kTileMaxLd) return fail(DSA_EINVAL, "sparse_attn_tiled: ld=%lld > %lld", (long long)ld, (long long)dsa::kTileMaxLd);
  if (B * T == 0) return DSA_OK;
  if (!scores || !thr || !Q || !K || !V || !out) return fail(DSA_EINVAL, "sparse_attn_tiled: null pointer");
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(out))
    return fail(DSA_EINVAL, "sparse_attn_tiled: Q/K/V/out must be 16-byte aligned");
  if (B * T * HQ * static_cast<int64_t>(DQ) > (int64_t{1} << 40)) return fail(DSA_EINVAL, "sparse_attn_tiled: Q too large");
  return hip_status(dsa::launch_tile_attn(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, scale,
                                          out, static_cast<hipStream_t>(stream)),
                    "dsa_sparse_attn_threshold_tiled");
}

int dsa_selection_mask(const float* scores, int64_t ld, const float* thr, int64_t B, int64_t T,
                       uint64_t* mask, int64_t ldm, void* stream) {
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "selection_mask: negative size");
  if (T > kMaxElems) return fail(DSA_EINVAL, "selection_mask: T=%lld too large", (long long)T);
  if (ld < T) return fail(DSA_EINVAL, "selection_mask: ld=%lld < T=%lld", (long long)ld, (long long)T);
  if (ldm < (T + 63) / 64)
    return fail(DSA_EINVAL, "selection_mask: ldm=%lld < ceil(T/64)=%lld", (long long)ldm, (long long)((T + 63) / 64));
  if ((B * T + 3) / 4 > (int64_t{1} << 31) - 1) return fail(DSA_EINVAL, "selection_mask: B*T too large for one launch");
  if (B * T == 0) return DSA_OK;
  if (!scores || !thr || !mask) return fail(DSA_EINVAL, "selection_mask: null pointer");
  if ((reinterpret_cast<uintptr_t>(mask) & 7u) != 0) return fail(DSA_EINVAL, "selection_mask: mask must be 8-byte aligned");
  return hip_status(dsa::launch_selection_mask(scores, ld, thr, B, T, mask, ldm,
                                               static_cast<hipStream_t>(stream)),
                    "dsa_selection_mask");
}

int dsa_sparse_attn_mask(const uint64_t* mask, int64_t ldm, const void* Q, const void* K,
                         const void* V, int dtype, int64_t B, int64_t T, int HQ, int DQ, int DV,
                         float scale, float* out, void* stream) {
  if (!dtype_ok(dtype)) return fail(DSA_EINVAL, "sparse_attn_mask: unknown dtype %d", dtype);
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "sparse_attn_mask: negative size");
  if (T > kMaxElems) return fail(DSA_EINVAL, "sparse_attn_mask: T=%lld too large", (long long)T);
  if (HQ < 1 || HQ > 1024) return fail(DSA_EINVAL, "sparse_attn_mask: HQ=%d outside [1,1024]", HQ);
  if (!std::isfinite(scale)) return fail(DSA_EINVAL, "sparse_attn_mask: scale must be finite");
  if (dtype == DSA_F32 || dtype == DSA_FP8 || DQ != DV || (DQ != 64 && DQ != 128))
    return fail(DSA_EUNSUPPORTED, "sparse_attn_mask: needs bf16/fp16 and DQ = DV in {64,128} (dtype %d DQ=%d DV=%d)", dtype, DQ, DV);
  if (ldm < (T + 63) / 64)
    return fail(DSA_EINVAL, "sparse_attn_mask: ldm=%lld < ceil(T/64)=%lld", (long long)ldm, (long long)((T + 63) / 64));
  // 128 mask rows are addressed with 32-bit byte offsets
  if (ldm > (int64_t{1} << 21) - 1) return fail(DSA_EINVAL, "sparse_attn_mask: ldm=%lld too large", (long long)ldm);
  if (T * HQ * static_cast<int64_t>(DQ) * 2 > (int64_t{1} << 32) - 1)
    return fail(DSA_EINVAL, "sparse_attn_mask: T*HQ*D = %lld 16-bit elements must be < 4 GiB",
                (long long)(T * HQ * static_cast<int64_t>(DQ)));
  if (B * T == 0) return DSA_OK;
  if (!mask || !Q || !K || !V || !out) return fail(DSA_EINVAL, "sparse_attn_mask: null pointer");
  if ((reinterpret_cast<uintptr_t>(mask) & 7u) != 0) return fail(DSA_EINVAL, "sparse_attn_mask: mask must be 8-byte aligned");
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(out))
    return fail(DSA_EINVAL, "sparse_attn_mask: Q/K/V/out must be 16-byte aligned");
  if (B * T * HQ * static_cast<int64_t>(DQ) > (int64_t{1} << 40)) return fail(DSA_EINVAL, "sparse_attn_mask: Q too large");
  return hip_status(dsa::launch_tile_attn_mask(mask, ldm, Q, K, V, dtype, B, T, HQ, DQ, scale, out,
                                               static_cast<hipStream_t>(stream)),
                    "dsa_sparse_attn_mask");
}

int dsa_sparse_attn_mask_noalloc(const float* scores, int64_t ld, const float* thr, const void* Q,
                                 const void* K, const void* V, int dtype, int64_t B, int64_t T,
                                 int HQ, int DQ, int DV, float scale, float* out, void* stream) {
  if (!dtype_ok(dtype)) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: unknown dtype %d", dtype);
  if (B < 0 || T < 0) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: negative size");
  if (T > kMaxElems) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: T=%lld too large", (long long)T);
  if (HQ < 1 || HQ > 1024) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: HQ=%d outside [1,1024]", HQ);
  if (!std::isfinite(scale)) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: scale must be finite");
  if (dtype == DSA_F32 || dtype == DSA_FP8 || DQ != DV || (DQ != 64 && DQ != 128))
    return fail(DSA_EUNSUPPORTED, "sparse_attn_mask_noalloc: needs bf16/fp16 and DQ = DV in {64,128} (dtype %d DQ=%d DV=%d)", dtype, DQ, DV);
  if (ld < T) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: ld=%lld < T=%lld", (long long)ld, (long long)T);
  const int64_t words = B * T * ((T + 63) / 64);
  if (words > dsa::kScratchWords)
    return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: the bitmask needs B*T*ceil(T/64) = %lld words, above the static scratch of %lld words (32 MiB); use dsa_selection_mask + dsa_sparse_attn_mask with a caller-allocated mask",
                (long long)words, (long long)dsa::kScratchWords);
  if (T * HQ * static_cast<int64_t>(DQ) * 2 > (int64_t{1} << 32) - 1)
    return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: T*HQ*D = %lld 16-bit elements must be < 4 GiB",
                (long long)(T * HQ * static_cast<int64_t>(DQ)));
  if (B * T == 0) return DSA_OK;
  if (!scores || !thr || !Q || !K || !V || !out) return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: null pointer");
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(out))
    return fail(DSA_EINVAL, "sparse_attn_mask_noalloc: Q/K/V/out must be 16-byte aligned");
  return hip_status(dsa::launch_sparse_attn_mask_noalloc(scores, ld, thr, Q, K, V, dtype, B, T, HQ,
                                                         DQ, scale, out,
                                                         static_cast<hipStream_t>(stream)),
                    "dsa_sparse_attn_mask_noalloc");
}

int dsa_sparse_attn_uses_mask(int dtype, int64_t T, int HQ, int DQ, int DV) {
  return dtype_ok(dtype) && dsa::sparse_attn_uses_tiles(dtype, T, HQ, DQ, DV) ? 1 : 0;
}

int dsa_sparse_attn_threshold_staged_ws(const float* scores, int64_t ld, const float* thr,
                                        const void* Q, const void* K, const void* V, int dtype,
                                        int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                        float* out, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
  int rc = check_attn(dtype, B, T, HQ, DQ, DV, Q, K, V, out, "sparse_attn_staged");
  if (rc != DSA_OK) return rc;
  if (!dsa::staged_attn_supported(dtype, HQ, DQ, DV))
    return fail(DSA_EUNSUPPORTED, "sparse_attn_staged: needs DQ = DV and HQ*DQ = 256 or 512 (fp32) / 512 (16-bit) (HQ=%d DQ=%d DV=%d dtype %d)", HQ, DQ, DV, dtype);
  if (ld < T) return fail(DSA_EINVAL, "sparse_attn_staged: ld=%lld < T=%lld", (long long)ld, (long long)T);
  if (!dsa::staged_attn_fits(T, ld))
    return fail(DSA_EUNSUPPORTED, "sparse_attn_staged: T*ld*4 = %lld bytes of scores per batch element, the limit is 2^31 (use dsa_sparse_attn_threshold)", (long long)(T * ld * 4));
  if (!std::isfinite(scale)) return fail(DSA_EINVAL, "sparse_attn_staged: scale must be finite");
  if (workspace_bytes < 0) return fail(DSA_EINVAL, "sparse_attn_staged: negative workspace size");
  if (B * T == 0) return DSA_OK;
  if (!scores || !thr) return fail(DSA_EINVAL, "sparse_attn_staged: null pointer");
  return hip_status(dsa::launch_staged_attn(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, scale,
                                            out, workspace, workspace_bytes,
                                            static_cast<hipStream_t>(stream)),
                    "dsa_sparse_attn_threshold_staged");
}

int dsa_sparse_attn_threshold_staged(const float* scores, int64_t ld, const float* thr,
                                     const void* Q, const void* K, const void* V, int dtype,
                                     int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                     float* out, void* stream) {
  return dsa_sparse_attn_threshold_staged_ws(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, DV,
                                             scale, out, nullptr, 0, stream);
}

int dsa_fused_forward(const void* q_idx, const void* k_idx, const void* w_idx, const void* Q,
                      const void* K, const void* V, int dtype, int64_t B, int64_t T, int HI,
                      int DI, int HQ, int DQ, int DV, int top_k, float scale, float* out,
                      void* stream) {
  if (T > dsa::kFusedMaxT)
    return fail(DSA_EUNSUPPORTED, "fused: T=%lld > %lld (use the split pipeline)", (long long)T, (long long)dsa::kFusedMaxT);
  if (top_k < 1) return fail(DSA_EINVAL, "fused: top_k must be >= 1 (got %d)", top_k);
  if (dtype == DSA_FP8) return fail(DSA_EINVAL, "fused: fp8 is an indexer-only dtype");
  int rc = check_indexer(q_idx, k_idx, w_idx, dtype, B, T, HI, DI, out, T);
  if (rc != DSA_OK) return rc;
  rc = check_attn(dtype, B, T, HQ, DQ, DV, Q, K, V, out, "fused");
  if (rc != DSA_OK) return rc;
  if (!std::isfinite(scale)) return fail(DSA_EINVAL, "fused: scale must be finite");
  if (B * T == 0) return DSA_OK;
  hipError_t e = dsa::launch_fused(q_idx, k_idx, w_idx, Q, K, V, dtype, B, T, HI, DI, HQ, DQ,
                                   DV, top_k, scale, out, static_cast<hipStream_t>(stream));
  if (e == hipErrorNotSupported)
    return fail(DSA_EUNSUPPORTED, "fused: no fused instance for dtype %d DI=%d HQ=%d DQ=%d DV=%d", dtype, DI, HQ, DQ, DV);
  return hip_status(e, "dsa_fused_forward");
}

}  // extern "C"
