// topk_cpu.cpp -- host k-th-largest per row for the CPU-offload (hybrid) path.
//
// Replaces the reference's AVX-512 extension (topk_avx512.cpp:226-264,
// `topk_threshold` / `topk_threshold_batch_merge`), which dsa_hybrid.py:57-63
// runs on pinned host copies of the indexer scores.  Same contract: for each
// row of n fp32 values the k-th largest counting ties, i.e.
// torch.topk(row, k).values[-1], for 0 < k <= n.
//
// Method (this library's own):
//   * every value becomes an order-preserving uint32 key (-0 folded onto +0,
//     every NaN onto one key above +inf: torch.topk's order), so the whole
//     scan is integer compares and the result is exact for any input;
//   * the row is scanned 16 values per step (AVX-512) with one compare
//     against the running k-th largest; the keys of values above it are
//     compress-stored into a candidate buffer (no per-value branch or
//     insertion);
//   * when the buffer is nearly full, a selection (nth_element) keeps its k
//     largest and raises the running k-th key to the buffer's k-th.  A key
//     equal to the running k-th cannot change the k-th largest of the row
//     (k values at or above it are already held), so strict '>' is exact;
//   * at the end one selection over the buffer gives the k-th largest.
// The expected number of candidates for a row in random order is about
// k*ln(n/k), so the selections cost little next to the scan.
//
// Rows run in parallel on OpenMP threads.  In causal mode row r is query
// t = (row0 + r) % causal_T of a [.., T, T] score matrix: only its t+1
// entries s <= t are read and the others count as -inf (what the indexer
// writes there), so rows with t+1 < k give -inf.
//
// Hosts without AVX-512F run a scalar loop of the same method.  Built
// without -ffast-math (rows hold -inf) and without -march=native (the
// library must run on whichever host the GPU box has).
#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <vector>

#include "../../include/dsa_cpu.h"

namespace {

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// Order-preserving key: unsigned order of keys == numeric order of floats,
// -0 == +0, NaN above +inf.  -inf is 0x007FFFFF; key 0 never occurs.
inline uint32_t to_key(float f) {
  f = f + 0.0f;
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if (f != f) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
inline float from_key(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Key of every NaN (the largest key).
constexpr uint32_t kNaNKey = 0xffc00000u;

// Candidate buffer capacity for a given k: room for max(3k, 512) more keys
// between selections (rows of up to ~512 entries need no selection until
// the end; one vector selection over 512 keys costs less than several over
// fewer).
inline int64_t buf_cap(int k) { return static_cast<int64_t>(k) + std::max(512, 3 * k) + 16; }

// Keep the k largest of buf[0..cnt) in buf[0..k), buf[k-1] the k-th largest.
inline uint32_t shrink(uint32_t* buf, int64_t& cnt, int k) {
  std::nth_element(buf, buf + (k - 1), buf + cnt, std::greater<uint32_t>());
  cnt = k;
  return buf[k - 1];
}

float row_kth_scalar(const float* row, int64_t n, int k, uint32_t* buf, int64_t cap) {
  float thr = -INFINITY;  // as in row_kth_avx512
  int64_t cnt = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float x = row[i];
    if (!(x <= thr)) {
      buf[cnt++] = to_key(x);
      if (cnt == cap) {
        const uint32_t tk = shrink(buf, cnt, k);
        if (tk == kNaNKey) return from_key(tk);
        thr = from_key(tk);
      }
    }
  }
  if (cnt < k) return -INFINITY;
  std::nth_element(buf, buf + (k - 1), buf + cnt, std::greater<uint32_t>());
  return from_key(buf[k - 1]);
}

__attribute__((target("avx512f")))
inline __m512i keys16(__m512 x) {
  const __m512 z = _mm512_add_ps(x, _mm512_setzero_ps());        // -0 -> +0
  __m512i u = _mm512_castps_si512(z);
  const __mmask16 nan = _mm512_cmp_ps_mask(x, x, _CMP_UNORD_Q);
  u = _mm512_mask_mov_epi32(u, nan, _mm512_set1_epi32(0x7fc00000));
  const __mmask16 neg = _mm512_cmplt_epi32_mask(u, _mm512_setzero_si512());  // sign bit set
  // negative: ~u; non-negative: u | sign
  const __m512i pos = _mm512_or_si512(u, _mm512_set1_epi32(static_cast<int>(0x80000000u)));
  const __m512i ngt = _mm512_xor_si512(u, _mm512_set1_epi32(-1));
  return _mm512_mask_mov_epi32(pos, neg, ngt);
}

// k-th largest (1-based) of keys a[0..m) by quickselect with AVX-512
// partitions: each pass splits the keys around a pivot into "above" (to the
// front of b) and "below" (to the back of b) with two compress-stores per 16
// keys, counts the pivot's copies, and continues on the side holding rank k.
// a and b hold at least m + 16 keys each; a's contents are destroyed.
__attribute__((target("avx512f")))
uint32_t select_kth_avx512(uint32_t* a, uint32_t* b, int64_t m, int64_t k) {
  while (m > 48) {
    uint32_t p0 = a[0], p1 = a[m / 2], p2 = a[m - 1];  // median of three
    if (p0 > p1) std::swap(p0, p1);
    if (p1 > p2) std::swap(p1, p2);
    if (p0 > p1) std::swap(p0, p1);
    const __m512i vp = _mm512_set1_epi32(static_cast<int>(p1));
    int64_t ng = 0, nl = 0;
    int64_t i = 0;
    for (; i + 16 <= m; i += 16) {
      const __m512i v = _mm512_loadu_si512(a + i);
      const __mmask16 gt = _mm512_cmpgt_epu32_mask(v, vp);
      const __mmask16 lt = _mm512_cmplt_epu32_mask(v, vp);
      _mm512_mask_compressstoreu_epi32(b + ng, gt, v);
      ng += __builtin_popcount(static_cast<unsigned>(gt));
      _mm512_mask_compressstoreu_epi32(a + nl, lt, v);  // in place: lands at or before i
      nl += __builtin_popcount(static_cast<unsigned>(lt));
    }
    for (; i < m; ++i) {
      const uint32_t v = a[i];
      if (v > p1) b[ng++] = v;
      else if (v < p1) a[nl++] = v;
    }
    const int64_t ne = m - ng - nl;
    if (k <= ng) {
      std::swap(a, b);
      m = ng;
    } else if (k <= ng + ne) {
      return p1;
    } else {
      k -= ng + ne;
      m = nl;
    }
  }
  std::sort(a, a + m, std::greater<uint32_t>());
  return a[k - 1];
}

// Keep the k largest of buf[0..cnt): the keys above the k-th largest tk,
// then tk repeated up to k entries; returns tk.  w1, w2: scratch of cap keys.
__attribute__((target("avx512f")))
uint32_t shrink_avx512(uint32_t* buf, int64_t& cnt, int k, uint32_t* w1, uint32_t* w2) {
  std::memcpy(w1, buf, static_cast<size_t>(cnt) * 4);
  const uint32_t tk = select_kth_avx512(w1, w2, cnt, k);
  const __m512i vk = _mm512_set1_epi32(static_cast<int>(tk));
  int64_t g = 0, j = 0;
  for (; j + 16 <= cnt; j += 16) {
    const __m512i v = _mm512_loadu_si512(buf + j);
    const __mmask16 gt = _mm512_cmpgt_epu32_mask(v, vk);
    _mm512_mask_compressstoreu_epi32(buf + g, gt, v);  // in place: g <= j
    g += __builtin_popcount(static_cast<unsigned>(gt));
  }
  for (; j < cnt; ++j)
    if (buf[j] > tk) buf[g++] = buf[j];
  for (; g < k; ++g) buf[g] = tk;
  cnt = k;
  return tk;
}

__attribute__((target("avx512f")))
float row_kth_avx512(const float* row, int64_t n, int k, uint32_t* buf, int64_t cap,
                     uint32_t* w1, uint32_t* w2) {
  // The scan compares floats against the running k-th largest `thr` with
  // "not less-or-equal, unordered": true for x > thr and for NaN x, false for
  // -0 against +0 -- the key order, in one compare per 16 values.  Only the
  // admitted values are turned into keys.  Until a selection has run, thr is
  // -inf, so -inf values are never admitted: if fewer than k values are, the
  // rest of the row is -inf and so is the k-th largest.
  int64_t cnt = 0;
  __m512 vthr = _mm512_set1_ps(-INFINITY);
  int64_t i = 0;
  for (; i + 16 <= n; i += 16) {
    const __m512 x = _mm512_loadu_ps(row + i);
    const __mmask16 m = _mm512_cmp_ps_mask(x, vthr, _CMP_NLE_UQ);
    if (m == 0) continue;
    _mm512_mask_compressstoreu_epi32(buf + cnt, m, keys16(x));
    cnt += __builtin_popcount(static_cast<unsigned>(m));
    if (cnt > cap - 16) {
      const uint32_t tk = shrink_avx512(buf, cnt, k, w1, w2);
      if (tk == kNaNKey) return from_key(tk);  // k NaNs: nothing ranks higher
      vthr = _mm512_set1_ps(from_key(tk));
    }
  }
  if (i < n) {
    const __mmask16 tail = static_cast<__mmask16>((1u << (n - i)) - 1u);
    const __m512 x = _mm512_maskz_loadu_ps(tail, row + i);
    const __mmask16 m = _mm512_mask_cmp_ps_mask(tail, x, vthr, _CMP_NLE_UQ);
    _mm512_mask_compressstoreu_epi32(buf + cnt, m, keys16(x));
    cnt += __builtin_popcount(static_cast<unsigned>(m));
  }
  if (cnt < k) return -INFINITY;
  return from_key(select_kth_avx512(buf, w1, cnt, k));
}

// AVX-512F when the host has it, unless DSA_CPU_ISA=scalar is set in the
// environment (read once; tests use it to run the scalar loop on any host).
bool host_has_avx512() {
  static const bool has = [] {
    const char* isa = std::getenv("DSA_CPU_ISA");
    if (isa != nullptr && std::strcmp(isa, "scalar") == 0) return false;
    return static_cast<bool>(__builtin_cpu_supports("avx512f"));
  }();
  return has;
}

}  // namespace

extern "C" {

const char* dsa_cpu_last_error(void) { return g_err; }

int dsa_cpu_isa(void) { return host_has_avx512() ? DSA_CPU_ISA_AVX512 : DSA_CPU_ISA_SCALAR; }

int dsa_cpu_topk_threshold(const float* scores, int64_t rows, int64_t n, int64_t ld, int k,
                           int64_t causal_T, int64_t row0, float* thr, int nthreads) {
  if (rows < 0 || n < 0) return fail(DSA_CPU_EINVAL, "topk_cpu: negative size rows=%lld n=%lld", (long long)rows, (long long)n);
  if (k <= 0) return fail(DSA_CPU_EINVAL, "topk_cpu: k must be > 0 (got %d)", k);
  if (k > n) return fail(DSA_CPU_EINVAL, "topk_cpu: k must be <= N (k=%d, N=%lld)", k, (long long)n);
  if (ld < n) return fail(DSA_CPU_EINVAL, "topk_cpu: ld=%lld < N=%lld", (long long)ld, (long long)n);
  if (causal_T < 0) return fail(DSA_CPU_EINVAL, "topk_cpu: causal_T=%lld < 0", (long long)causal_T);
  if (causal_T > 0) {
    if (causal_T > n) return fail(DSA_CPU_EINVAL, "topk_cpu: causal_T=%lld > N=%lld", (long long)causal_T, (long long)n);
  }
  if (row0 < 0) return fail(DSA_CPU_EINVAL, "topk_cpu: row0=%lld < 0", (long long)row0);
  if (nthreads < 0) return fail(DSA_CPU_EINVAL, "topk_cpu: nthreads=%d < 0", nthreads);
  if (rows == 0) return DSA_CPU_OK;
  if (!scores || !thr) return fail(DSA_CPU_EINVAL, "topk_cpu: null pointer");

  const bool avx = host_has_avx512();
  const int64_t cap = buf_cap(k);
  // small inputs: no more threads than one per 8K entries (team start-up
  // costs more than the scan below that)
  const int64_t work = rows * (causal_T > 0 ? (n + 1) / 2 : n);
  const int nt = static_cast<int>(std::min<int64_t>(
      nthreads > 0 ? nthreads : omp_get_max_threads(), std::max<int64_t>(1, work >> 13)));
  // causal rows differ in length: hand rows out in small dynamic chunks
  const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(64, rows / (8 * std::max(nt, 1))));
  int status = DSA_CPU_OK;
#pragma omp parallel num_threads(nt)
  {
    std::vector<uint32_t> buf;
    try {
      buf.resize(static_cast<size_t>(3 * (cap + 16)));
    } catch (...) {
#pragma omp atomic write
      status = DSA_CPU_ENOMEM;
    }
#pragma omp barrier
    if (status == DSA_CPU_OK) {
#pragma omp for schedule(dynamic, chunk)
      for (int64_t r = 0; r < rows; ++r) {
        const float* row = scores + r * ld;
        int64_t nv = n;
        if (causal_T > 0) nv = (row0 + r) % causal_T + 1;
        if (nv < k) {
          thr[r] = -INFINITY;
          continue;
        }
        uint32_t* b0 = buf.data();
        thr[r] = avx ? row_kth_avx512(row, nv, k, b0, cap, b0 + cap + 16, b0 + 2 * (cap + 16))
                     : row_kth_scalar(row, nv, k, b0, cap);
      }
    }
  }
  if (status != DSA_CPU_OK) return fail(status, "topk_cpu: out of host memory for %lld-entry buffers", (long long)cap);
  return DSA_CPU_OK;
}

}  // extern "C"
