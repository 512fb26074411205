// topk_cpu.cpp -- TEST INFRASTRUCTURE ONLY (oracle + timed CPU baseline).
//
// C++ restatement of the reference's CPU k-th-largest extension
// (topk_avx512.cpp:24-105 row kernels and OpenMP driver, :172-199 dispatch,
// :226-249 contract).  Contract: for every row of n fp32 values, the k-th
// largest counting ties (== torch.topk(row, k).values[-1]); 0 < k <= n.
//
// Algorithm (the reference's): keep the k largest values seen so far; scan 16
// values per step with one AVX-512 compare against the current k-th largest;
// only values strictly above it are compressed out and inserted -- into a
// descending array for k <= 32, into a binary min-heap otherwise.  Rows are
// split over OpenMP threads statically.  Built without -ffast-math because
// causal score rows hold -inf.
//
// C ABI (ctypes from oracle/native.py):
//   int oracle_topk_has_avx512(void);
//   int oracle_topk_threshold(const float* in, float* out, int64_t rows,
//                             int64_t n, int k, int nthreads, int use_avx512);
#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cstdint>
#include <functional>
#include <vector>

namespace {

// ---- top-k buffers ---------------------------------------------------------
// Sorted buffer: buf[0] >= ... >= buf[k-1]; buf[k-1] is the current k-th.
inline void sorted_push(float* buf, int k, float v) {
  if (!(v > buf[k - 1])) return;
  int i = k - 1;
  for (; i > 0 && buf[i - 1] < v; --i) buf[i] = buf[i - 1];
  buf[i] = v;
}

// Min-heap: heap[0] is the current k-th largest.
inline void heap_replace_top(float* heap, int k, float v) {
  int i = 0;
  for (;;) {
    int c = 2 * i + 1;
    if (c >= k) break;
    if (c + 1 < k && heap[c + 1] < heap[c]) ++c;
    if (!(heap[c] < v)) break;
    heap[i] = heap[c];
    i = c;
  }
  heap[i] = v;
}

struct SortedBuf {
  static void init(float* b, int k) { std::sort(b, b + k, std::greater<float>()); }
  static float kth(const float* b, int k) { return b[k - 1]; }
  static void push(float* b, int k, float v) { sorted_push(b, k, v); }
};
struct MinHeap {
  static void init(float* b, int k) { std::make_heap(b, b + k, std::greater<float>()); }
  static float kth(const float* b, int) { return b[0]; }
  static void push(float* b, int k, float v) {
    if (v > b[0]) heap_replace_top(b, k, v);
  }
};

template <class Buf>
float row_kth_scalar(const float* row, int64_t n, int k, float* buf) {
  std::copy(row, row + k, buf);
  Buf::init(buf, k);
  for (int64_t i = k; i < n; ++i) Buf::push(buf, k, row[i]);
  return Buf::kth(buf, k);
}

template <class Buf>
__attribute__((target("avx512f"))) float row_kth_avx512(const float* row, int64_t n, int k,
                                                        float* buf) {
  std::copy(row, row + k, buf);
  Buf::init(buf, k);
  alignas(64) float cand[16];
  int64_t i = k;
  for (; i + 16 <= n; i += 16) {
    const __m512 x = _mm512_loadu_ps(row + i);
    const __mmask16 above =
        _mm512_cmp_ps_mask(x, _mm512_set1_ps(Buf::kth(buf, k)), _CMP_GT_OQ);
    if (above == 0) continue;
    _mm512_mask_compressstoreu_ps(cand, above, x);
    const int m = __builtin_popcount(static_cast<unsigned>(above));
    for (int j = 0; j < m; ++j) Buf::push(buf, k, cand[j]);
  }
  for (; i < n; ++i) Buf::push(buf, k, row[i]);
  return Buf::kth(buf, k);
}

template <class Buf>
void run_rows(const float* in, float* out, int64_t rows, int64_t n, int k, int nthreads,
              bool avx) {
#pragma omp parallel num_threads(nthreads)
  {
    std::vector<float> buf(static_cast<size_t>(k));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const float* row = in + r * n;
      out[r] = avx ? row_kth_avx512<Buf>(row, n, k, buf.data())
                   : row_kth_scalar<Buf>(row, n, k, buf.data());
    }
  }
}

}  // namespace

extern "C" {

int oracle_topk_has_avx512(void) { return __builtin_cpu_supports("avx512f") ? 1 : 0; }

int oracle_topk_threshold(const float* in, float* out, int64_t rows, int64_t n, int k,
                          int nthreads, int use_avx512) {
  if (k <= 0 || k > n || rows < 0) return -1;
  if (nthreads < 1) nthreads = 1;
  const bool avx = use_avx512 != 0 && oracle_topk_has_avx512();
  if (k <= 32)
    run_rows<SortedBuf>(in, out, rows, n, k, nthreads, avx);
  else
    run_rows<MinHeap>(in, out, rows, n, k, nthreads, avx);
  return 0;
}

}  // extern "C"
