// topk.hip -- per-row k-th largest ("top-K threshold") by block radix-select.
//
// Contract (reference topk_avx512.cpp:226-249, dsa_attention.py:41-44):
// thr[r] is the k-th largest value of row r counting ties, i.e.
// torch.topk(row, k).values[-1].  Optionally also the exactly-k index set a
// stable descending sort puts first (lowest index wins ties), in ascending
// index order.
//
// Design (gfx950): one workgroup per row.  The row is read from HBM once,
// straight into registers as radix keys (V keys per thread, float4 loads,
// chunk-major so every load instruction is one contiguous 16*NT-byte span).
// Three MSD passes over 11/11/10-bit digits build a histogram in LDS with
// ds_add, and a block suffix-scan picks the digit that holds the k-th key; a
// pass whose chosen digit holds a single key ends the search early.  No
// global workspace, no second read of the row.  Rows longer than the
// register capacity (NT*V) stream from global memory once per pass.
//
// Causal mode (causal_T > 0): row r is query t = r % causal_T of a [B,T,T]
// score matrix; only entries s <= t are read and the rest count as -inf, so
// algorithmic traffic is 4*(t+1) bytes per row.  Blocks take rows longest
// first so the short tail of the triangle fills in at the end of the grid.
#include "dsa_device.h"
#include "dsa_launch.h"

namespace dsa {
namespace {

struct SelectArgs {
  const float* scores;
  int64_t rows;
  int64_t n;
  int64_t ld;
  int k;
  int64_t causal_T;
  float* thr;
  int32_t* idx;
};

constexpr int kMaxBins = 2048;

// Digit of pass p: pass 0 = key[31:21], pass 1 = key[20:10], pass 2 = key[9:0].
__device__ __forceinline__ int pass_shift(int p) { return p == 0 ? 21 : (p == 1 ? 10 : 0); }
__device__ __forceinline__ int pass_bits(int p) { return p == 2 ? 10 : 11; }

template <int NT, int V, bool VEC, bool STREAM>
__global__ __launch_bounds__(NT) void topk_rows_kernel(SelectArgs a) {
  static_assert(V % 4 == 0, "keys are loaded four at a time");
  static_assert(NT % kWave == 0 && NT <= 1024, "block shape");
  __shared__ uint32_t hist[kMaxBins];
  __shared__ uint32_t wsum[NT / kWave];
  __shared__ uint32_t info[4];

  const int tid = threadIdx.x;
  int64_t row, nvalid;
  if (a.causal_T > 0) {
    const int64_t nb = a.rows / a.causal_T;
    const int64_t i = blockIdx.x;
    const int64_t t = a.causal_T - 1 - i / nb;
    row = (i % nb) * a.causal_T + t;
    nvalid = t + 1;
  } else {
    row = blockIdx.x;
    nvalid = a.n;
  }
  const int k = a.k;
  const float* __restrict__ src = a.scores + row * a.ld;

  if (nvalid < k) {
    // Causal row with fewer than k real entries: the k-th largest of the full
    // row is one of the implicit -inf entries, and a stable sort puts the
    // real entries first, then the -inf ones in index order.
    if (tid == 0) a.thr[row] = -__builtin_huge_valf();
    if (a.idx != nullptr) {
      int32_t* out = a.idx + row * static_cast<int64_t>(k);
      for (int i = tid; i < k; i += NT) out[i] = i;
    }
    return;
  }

  // ---- load the row as keys (kKeyNone beyond nvalid) --------------------
  uint32_t key[STREAM ? 4 : V];
  auto load4 = [&](int64_t pos, uint32_t (&kk)[4]) {
    if (VEC) {
      if (pos < nvalid) {
        const float4 f = *reinterpret_cast<const float4*>(src + pos);
        kk[0] = float_to_key(f.x);
        kk[1] = (pos + 1 < nvalid) ? float_to_key(f.y) : kKeyNone;
        kk[2] = (pos + 2 < nvalid) ? float_to_key(f.z) : kKeyNone;
        kk[3] = (pos + 3 < nvalid) ? float_to_key(f.w) : kKeyNone;
      } else {
        kk[0] = kk[1] = kk[2] = kk[3] = kKeyNone;
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kk[c] = (pos + c < nvalid) ? float_to_key(src[pos + c]) : kKeyNone;
    }
  };
  const int64_t nchunks =
      STREAM ? (nvalid + 4 * NT - 1) / (4 * NT) : static_cast<int64_t>(V / 4);
  if (!STREAM) {
#pragma unroll
    for (int j = 0; j < V / 4; ++j) {
      uint32_t kk[4];
      load4((static_cast<int64_t>(j) * NT + tid) * 4, kk);
#pragma unroll
      for (int c = 0; c < 4; ++c) key[4 * j + c] = kk[c];
    }
  }
  // Calls f(pos, key) for each of this thread's elements (padding included).
  auto for_each = [&](auto&& f) {
    if (STREAM) {
      for (int64_t j = 0; j < nchunks; ++j) {
        const int64_t pos = (j * NT + tid) * 4;
        uint32_t kk[4];
        load4(pos, kk);
#pragma unroll
        for (int c = 0; c < 4; ++c) f(pos + c, kk[c]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < V / 4; ++j) {
        const int64_t pos = (static_cast<int64_t>(j) * NT + tid) * 4;
#pragma unroll
        for (int c = 0; c < 4; ++c) f(pos + c, key[4 * j + c]);
      }
    }
  };

  // ---- three radix passes -------------------------------------------------
  uint32_t prefix = 0;           // digits chosen so far
  uint32_t krem = static_cast<uint32_t>(k);  // rank still wanted inside the prefix
  uint32_t cnt_eq = 0;           // keys equal to the answer
  uint32_t thr_key = 0;
  bool found = false;
  for (int p = 0; p < 3 && !found; ++p) {
    const int shift = pass_shift(p);
    const int bits = pass_bits(p);
    const int nbins = 1 << bits;
    const int hi_shift = shift + bits;  // 32 on pass 0: no prefix test
    for (int b = tid; b < nbins; b += NT) hist[b] = 0u;
    __syncthreads();
    for_each([&](int64_t, uint32_t kk) {
      const bool in_prefix = (p == 0) || ((kk >> hi_shift) == prefix);
      if (kk != kKeyNone && in_prefix) atomicAdd(&hist[(kk >> shift) & (nbins - 1)], 1u);
    });
    __syncthreads();
    // Thread tid owns bins [tid*bpt, tid*bpt + bpt); find the bin where the
    // count of keys above it first reaches krem.
    const int bpt = (nbins + NT - 1) / NT;
    const int lo = tid * bpt;
    uint32_t local = 0;
    for (int i = 0; i < bpt; ++i)
      if (lo + i < nbins) local += hist[lo + i];
    uint32_t total;
    const uint32_t excl = block_exclusive_sum<NT>(local, wsum, total);
    const uint32_t above = total - excl - local;  // keys in bins owned by higher threads
    if (above < krem && above + local >= krem) {
      uint32_t cum = above;
      for (int i = bpt - 1; i >= 0; --i) {
        const int b = lo + i;
        if (b >= nbins) continue;
        const uint32_t c = hist[b];
        if (cum + c >= krem) {
          info[0] = static_cast<uint32_t>(b);
          info[1] = krem - cum;
          info[2] = c;
          break;
        }
        cum += c;
      }
    }
    __syncthreads();
    prefix = (prefix << bits) | info[0];
    krem = info[1];
    cnt_eq = info[2];
    if (p < 2 && cnt_eq == 1u) {
      // The chosen digit holds one key: it is the answer.
      for_each([&](int64_t, uint32_t kk) {
        if (kk != kKeyNone && (kk >> shift) == prefix) info[3] = kk;
      });
      __syncthreads();
      thr_key = info[3];
      found = true;
    }
  }
  if (!found) thr_key = prefix;
  if (tid == 0) a.thr[row] = key_to_float(thr_key);

  // ---- exactly-k index set, ascending index order -------------------------
  // Position of a selected element = (#keys above thr before it) +
  // min(#keys equal to thr before it, krem); ties beyond krem are dropped.
  if (a.idx != nullptr) {
    int32_t* out = a.idx + row * static_cast<int64_t>(k);
    uint32_t run_gt = 0, run_eq = 0;
    auto emit_chunk = [&](int64_t pos, const uint32_t (&kk)[4]) {
      uint32_t ngt = 0, neq = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        ngt += (kk[c] > thr_key) ? 1u : 0u;
        neq += (kk[c] == thr_key) ? 1u : 0u;
      }
      uint32_t tot;
      const uint32_t ex = block_exclusive_sum<NT>((neq << 16) | ngt, wsum, tot);
      uint32_t gt_before = run_gt + (ex & 0xffffu);
      uint32_t eq_before = run_eq + (ex >> 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (kk[c] > thr_key) {
          out[gt_before + (eq_before < krem ? eq_before : krem)] = static_cast<int32_t>(pos + c);
          ++gt_before;
        } else if (kk[c] == thr_key) {
          if (eq_before < krem) out[gt_before + eq_before] = static_cast<int32_t>(pos + c);
          ++eq_before;
        }
      }
      run_gt += tot & 0xffffu;
      run_eq += tot >> 16;
    };
    if (STREAM) {
      for (int64_t j = 0; j < nchunks; ++j) {
        const int64_t pos = (j * NT + tid) * 4;
        uint32_t kk[4];
        load4(pos, kk);
        emit_chunk(pos, kk);
      }
    } else {
#pragma unroll
      for (int j = 0; j < V / 4; ++j) {
        const uint32_t kk[4] = {key[4 * j], key[4 * j + 1], key[4 * j + 2], key[4 * j + 3]};
        emit_chunk((static_cast<int64_t>(j) * NT + tid) * 4, kk);
      }
    }
  }
}

template <int NT, int V, bool STREAM>
hipError_t launch_cfg(const SelectArgs& a, bool vec, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.rows));
  if (vec)
    hipLaunchKernelGGL((topk_rows_kernel<NT, V, true, STREAM>), grid, dim3(NT), 0, stream, a);
  else
    hipLaunchKernelGGL((topk_rows_kernel<NT, V, false, STREAM>), grid, dim3(NT), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_topk(const float* scores, int64_t rows, int64_t n, int64_t ld, int k,
                       int64_t causal_T, float* thr, int32_t* idx, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  SelectArgs a{scores, rows, n, ld, k, causal_T, thr, idx};
  const int64_t cap = causal_T > 0 ? (causal_T < n ? causal_T : n) : n;
  // float4 loads stay inside [0, n) of every row only when n, ld and the base
  // are all 16-byte granular.
  const bool vec = (n % 4 == 0) && (ld % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(scores) & 15u) == 0);
  if (cap <= 256) return launch_cfg<64, 4, false>(a, vec, stream);
  if (cap <= 512) return launch_cfg<128, 4, false>(a, vec, stream);
  if (cap <= 1024) return launch_cfg<256, 4, false>(a, vec, stream);
  if (cap <= 2048) return launch_cfg<256, 8, false>(a, vec, stream);
  if (cap <= 4096) return launch_cfg<512, 8, false>(a, vec, stream);
  if (cap <= 8192) return launch_cfg<1024, 8, false>(a, vec, stream);
  if (cap <= 16384) return launch_cfg<1024, 16, false>(a, vec, stream);
  if (cap <= 32768) return launch_cfg<1024, 32, false>(a, vec, stream);
  return launch_cfg<1024, 4, true>(a, vec, stream);
}

}  // namespace dsa
