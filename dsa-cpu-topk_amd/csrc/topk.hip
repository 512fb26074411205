// topk.hip -- per-row k-th largest ("top-K threshold") by block radix-select.
//
// Contract (reference topk_avx512.cpp:226-249, dsa_attention.py:41-44):
// thr[r] is the k-th largest value of row r counting ties, i.e.
// torch.topk(row, k).values[-1].  Optionally also the exactly-k index set a
// stable descending sort puts first (lowest index wins ties), in ascending
// index order.
//
// Design (gfx950): one workgroup per row, the row read from HBM exactly once
// straight into registers as order-preserving radix keys (V keys per thread,
// float4 loads, chunk-major so each load instruction is one contiguous
// 16*NT-byte span; chunks past the row's valid length are skipped
// block-uniformly).  Then MSD radix passes over 11/11/10-bit digits:
//   pass 1  histogram of key[31:21] in LDS (ds_add), block suffix-scan picks
//           the digit holding the k-th key;
//           if that digit holds <= kCandCap keys they are compacted into LDS
//           (one LDS atomic per wave) and passes 2-3 touch only them;
//   pass 2  key[20:10] of the keys in the chosen digit;
//   pass 3  key[9:0].
// When only thresholds are asked for, the candidates go to one wave instead
// (wave_select_cand: 8-bit passes with wave-level syncs only) and the other
// waves of the block exit, freeing their registers for the next rows.
// A digit holding a single key ends the search early.  Every barrier orders
// LDS only, so waves of other resident blocks keep their HBM loads in flight
// while this block histograms -- blocks are sized (<= 64 VGPRs) so that
// several rows per CU are in flight.
//
// Causal mode (causal_T > 0): row r is query t = r % causal_T of a [B,T,T]
// score matrix; only entries s <= t are read and the rest count as -inf, so
// algorithmic traffic is 4*(t+1) bytes per row.  Blocks take rows longest
// first so the short tail of the triangle fills in at the end of the grid.
//
// Rows longer than the largest register configuration use the streaming
// kernel (same passes, the row re-read from global memory on every pass).
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


// Digits of the streaming kernel: key[31:21], key[20:10], key[9:0].
constexpr int kP1 = 11;
constexpr int kS1 = 21;
constexpr int kB2 = 11;
constexpr int kS2 = 10;
constexpr int kB3 = 10;
constexpr int kBins = 2048;
constexpr int kCandCap = 2048;

__device__ __forceinline__ void row_of_block(const SelectArgs& a, int64_t& row,
                                             int64_t& nvalid) {
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
}

// Causal row with fewer than k real entries: the k-th largest of the full row
// is one of the implicit -inf entries, and a stable sort puts the real
// entries first, then the -inf ones in index order.
template <int NT>
__device__ __forceinline__ void emit_short_row(const SelectArgs& a, int64_t row) {
  if (threadIdx.x == 0) a.thr[row] = -__builtin_huge_valf();
  if (a.idx != nullptr) {
    int32_t* out = a.idx + row * static_cast<int64_t>(a.k);
    for (int i = threadIdx.x; i < a.k; i += NT) out[i] = i;
  }
}

template <int HI>
__device__ __forceinline__ bool in_prefix(uint32_t kk, uint32_t prefix) {
  if constexpr (HI >= 32) return true;
  else return (kk >> HI) == prefix;
}

// Finds the digit holding the krem-th largest key of an NB-bin histogram.
// Thread tid owns bins [tid*BPT, tid*BPT+BPT).  Ends with a barrier after
// which info[0] = digit, info[1] = rank of the wanted key inside the digit,
// info[2] = keys in the digit.
template <int NT, int NB>
__device__ __forceinline__ void find_digit(const uint32_t* hist, uint32_t krem, uint32_t* wsum,
                                           uint32_t* info) {
  constexpr int BPT = NB >= NT ? NB / NT : 1;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int lo = tid * BPT;
  uint32_t h[BPT];
  uint32_t local = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    h[i] = (lo + i < NB) ? hist[lo + i] : 0u;
    local += h[i];
  }
  const uint32_t incl = wave_inclusive_sum(local);
  if (lane == kWave - 1) wsum[wid] = incl;
  block_sync_lds();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) {
    const uint32_t s = wsum[w];
    base += (w < wid) ? s : 0u;
    tot += s;
  }
  const uint32_t above = tot - base - incl;  // keys in bins of higher threads
  if (above < krem && above + local >= krem) {
    uint32_t cum = above;
    bool done = false;
#pragma unroll
    for (int i = BPT - 1; i >= 0; --i) {
      if (!done && cum + h[i] >= krem) {
        info[0] = static_cast<uint32_t>(lo + i);
        info[1] = krem - cum;
        info[2] = h[i];
        done = true;
      }
      cum += h[i];
    }
  }
  block_sync_lds();
}

// One radix pass over the keys `visit` enumerates (keys equal to kKeyNone
// are skipped).  Returns true when the chosen digit holds a single key, whose
// value is then in thr_key.  COUNT_NONE: a first pass (HI = 32) may count
// kKeyNone (0) into digit 0 instead of testing for it -- no real key has a
// top digit of 0 (the smallest, -inf, is 0x007fffff), and with at least krem
// real keys the search never reaches digit 0.
template <int NT, int SHIFT, int BITS, bool COUNT_NONE = false, typename Visit>
__device__ __forceinline__ bool radix_pass(Visit&& visit, uint32_t* hist, uint32_t* wsum,
                                           uint32_t* info, uint32_t& prefix, uint32_t& krem,
                                           uint32_t& cnt, bool allow_unique,
                                           uint32_t& thr_key) {
  constexpr int NB = 1 << BITS;
  constexpr int HI = SHIFT + BITS;
  for (int b = threadIdx.x; b < NB; b += NT) hist[b] = 0u;
  block_sync_lds();
  static_assert(!COUNT_NONE || HI >= 32, "kKeyNone is in digit 0 only for the first digit");
  visit([&](uint32_t kk) {
    if constexpr (COUNT_NONE) {
      atomicAdd(&hist[kk >> SHIFT], 1u);
    } else {
      if (kk != kKeyNone && in_prefix<HI>(kk, prefix))
        atomicAdd(&hist[(kk >> SHIFT) & (NB - 1)], 1u);
    }
  });
  block_sync_lds();
  find_digit<NT, NB>(hist, krem, wsum, info);
  prefix = (prefix << BITS) | info[0];
  krem = info[1];
  cnt = info[2];
  if (allow_unique && cnt == 1u) {
    visit([&](uint32_t kk) {
      if (kk != kKeyNone && (kk >> SHIFT) == prefix) info[3] = kk;
    });
    block_sync_lds();
    thr_key = info[3];
    return true;
  }
  return false;
}

// Writes the exactly-k index set of a row whose keys `chunk(j, kk)` yields
// chunk by chunk (chunk j covers positions (j*NT + tid)*4 .. +3), in
// ascending index order.  Position of a selected element =
// #(keys > thr before it) + min(#(keys == thr before it), krem).
template <int NT, typename Chunk>
__device__ __forceinline__ void emit_indices(int32_t* out, int64_t nchunks, uint32_t thr_key,
                                             uint32_t krem, uint32_t* wsum, Chunk&& chunk) {
  const int tid = threadIdx.x;
  uint32_t run_gt = 0, run_eq = 0;
  for (int64_t j = 0; j < nchunks; ++j) {
    uint32_t kk[4];
    chunk(j, kk);
    const int64_t pos = (j * NT + tid) * 4;
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
  }
}

// k-th largest of n candidate keys in LDS that all share their bits above
// bit `low` (those bits are `prefix`), by one wave: MSD passes over at most 8
// of the remaining bits, each a 256-bin histogram in `hist` (wave-private
// LDS) built with ds_add and a wave suffix scan -- wave-level syncs only, no
// block barrier.  A digit holding a single key ends the search early.
__device__ __forceinline__ uint32_t wave_select_cand(const uint32_t* cand, uint32_t n,
                                                     uint32_t prefix, int low, uint32_t krem,
                                                     uint32_t* hist) {
  const int lane = threadIdx.x & (kWave - 1);
  int shift = low;
  while (shift > 0) {
    const int bits = shift >= 8 ? 8 : shift;
    shift -= bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int hi = shift + bits;  // may be 32: 64-bit shifts below
    reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    for (uint32_t i = lane; i < n; i += kWave) {
      const uint32_t kk = cand[i];
      if ((static_cast<uint64_t>(kk) >> hi) == prefix) atomicAdd(&hist[(kk >> shift) & mask], 1u);
    }
    wave_lds_sync();
    const uint4 h4 = reinterpret_cast<const uint4*>(hist)[lane];
    const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
    const uint32_t local = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = wave_inclusive_sum(local);
    const uint32_t total = wave_read_lane(incl, kWave - 1);
    const uint32_t above = total - incl;  // keys in higher lanes' bins
    const bool mine = above < krem && above + local >= krem;
    uint32_t digit = 0, knew = 0, cnt = 0;
    if (mine) {
      uint32_t cum = above;
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (cnt == 0u && cum + h[i] >= krem) {
          digit = 4u * lane + i;
          knew = krem - cum;
          cnt = h[i];
        }
        cum += h[i];
      }
    }
    const int src = __ffsll(static_cast<unsigned long long>(__ballot(mine))) - 1;
    prefix = (prefix << bits) | wave_read_lane(digit, src);
    krem = wave_read_lane(knew, src);
    cnt = wave_read_lane(cnt, src);
    wave_lds_sync();  // histogram reads done before the next pass clears it
    if (shift > 0 && cnt == 1u) {
      uint32_t hit = 0;
      for (uint32_t i = lane; i < n; i += kWave) {
        const uint32_t kk = cand[i];
        if ((kk >> shift) == prefix) hit = kk;
      }
      const uint64_t m = __ballot(hit != 0u);
      return wave_read_lane(hit, __ffsll(static_cast<unsigned long long>(m)) - 1);
    }
  }
  return prefix;
}

template <bool VEC>
__device__ __forceinline__ void load_keys4(const float* __restrict__ src, int64_t pos,
                                           int64_t nvalid, uint32_t (&kk)[4]) {
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
}

// ---------------------------------------------------------------------------
// Register-resident kernel: rows up to 4*NT*(V/4) entries; first digit P1 bits.
// ---------------------------------------------------------------------------
// Keys plus ~30 working registers fit 64 VGPRs up to V = 32: blocks of up to
// 512 threads ask for 8 waves per SIMD there, so that four rows share a CU.
template <int NT, int V, int P1, bool VEC>
__global__ __launch_bounds__(NT, (V <= 32 && NT <= 512) ? 8 : 4) void topk_reg_kernel(SelectArgs a) {
  static_assert(V % 4 == 0 && NT % kWave == 0 && NT <= 1024, "block shape");
  static_assert(P1 == 11 || P1 == 12, "first digit width");
  constexpr int NCH = V / 4;
  constexpr int S1 = 32 - P1;           // shift of digit 1
  constexpr int B2 = (S1 + 1) / 2;      // bits of digit 2
  constexpr int S2 = S1 - B2;           // shift of digit 2
  constexpr int B3 = S2;                // bits of digit 3 (shift 0)
  constexpr int NBINS = 1 << (P1 > B2 ? P1 : B2);
  __shared__ uint32_t hist[NBINS];
  __shared__ uint32_t cand[kCandCap];
  __shared__ uint32_t wsum[NT / kWave];
  __shared__ uint32_t info[4];
  __shared__ uint32_t ncand;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  int64_t row, nvalid;
  row_of_block(a, row, nvalid);
  const int k = a.k;
  if (nvalid < k) {
    emit_short_row<NT>(a, row);
    return;
  }
  const float* __restrict__ src = a.scores + row * a.ld;
  // chunks that hold any valid entry (block-uniform)
  const int nch = static_cast<int>(min(static_cast<int64_t>(NCH), (nvalid + 4 * NT - 1) / (4 * NT)));

  // All of the row's loads are issued before any is used: one memory round
  // trip per row.  Addresses are clamped into the row (the last float4, or the
  // last entry) instead of predicated, so no load sits behind a branch -- a
  // per-chunk branch made every load wait for the previous one.  Chunks past
  // nch read that one clamped address and are never visited.
  uint32_t key[V];
  {
    const int nv = static_cast<int>(nvalid);  // the host checks n < 2^31
    // 32-bit byte offsets from the row base (a register row is < 2^30 bytes),
    // so each load takes one offset register against the scalar base
    const char* row_bytes = reinterpret_cast<const char*>(src);
    float raw[V];
    if constexpr (VEC) {
      const int last4 = (nv - 1) & ~3;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int pos = (j * NT + tid) * 4;
        const uint32_t off = static_cast<uint32_t>(min(pos, last4)) * 4u;
        const float4 f = *reinterpret_cast<const float4*>(row_bytes + off);
        raw[4 * j] = f.x;
        raw[4 * j + 1] = f.y;
        raw[4 * j + 2] = f.z;
        raw[4 * j + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t off = static_cast<uint32_t>(min((j * NT + tid) * 4 + c, nv - 1)) * 4u;
          raw[4 * j + c] = *reinterpret_cast<const float*>(row_bytes + off);
        }
    }
    // Entries past the row become kKeyNone; only a chunk the row ends inside
    // needs the per-entry test (block-uniform branch after the conversion,
    // so no load is sunk into it).
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
#pragma unroll
      for (int c = 0; c < 4; ++c) key[4 * j + c] = float_to_key(raw[4 * j + c]);
      if ((j + 1) * NT * 4 > nv) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if ((j * NT + tid) * 4 + c >= nv) key[4 * j + c] = kKeyNone;
      }
    }
  }
  auto visit_regs = [&](auto&& f) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j < nch) {
#pragma unroll
        for (int c = 0; c < 4; ++c) f(key[4 * j + c]);
      }
    }
  };

  // The first pass tests for kKeyNone only in the chunk the row ends inside.
  auto visit_first = [&](auto&& f) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j < nch) {
        if ((j + 1) * NT * 4 <= nvalid) {
#pragma unroll
          for (int c = 0; c < 4; ++c) f(key[4 * j + c]);
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (key[4 * j + c] != kKeyNone) f(key[4 * j + c]);
        }
      }
    }
  };

  if (tid == 0) ncand = 0u;
  uint32_t prefix = 0, krem = static_cast<uint32_t>(k), cnt = 0, thr_key = 0;
  bool found = radix_pass<NT, S1, P1, true>(visit_first, hist, wsum, info, prefix, krem, cnt,
                                            true, thr_key);
  if (!found) {
    if (cnt <= static_cast<uint32_t>(kCandCap)) {
      // Compact the chosen digit's keys into LDS: per-lane count, wave scan,
      // one LDS atomic per wave for the wave's base.
      const uint32_t top = prefix;
      uint32_t mine = 0;
      visit_regs([&](uint32_t kk) { mine += ((kk >> S1) == top) ? 1u : 0u; });
      const uint32_t incl = wave_inclusive_sum(mine);
      const uint32_t wtot = wave_read_lane(incl, kWave - 1);
      uint32_t wbase = 0;
      if (lane == kWave - 1 && wtot != 0u) wbase = atomicAdd(&ncand, wtot);
      wbase = wave_read_lane(wbase, kWave - 1);
      uint32_t p = wbase + incl - mine;
      visit_regs([&](uint32_t kk) {
        if ((kk >> S1) == top) cand[p++] = kk;
      });
      block_sync_lds();
      const uint32_t n_c = cnt;
      if (a.idx == nullptr) {
        // Threshold only: one wave finishes on the candidates; the other
        // waves exit now, so their registers take the next rows' loads.
        if (tid >= kWave) return;
        const uint32_t tk = wave_select_cand(cand, n_c, prefix, S1, krem, hist);
        if (tid == 0) a.thr[row] = key_to_float(tk);
        return;
      }
      auto visit_cand = [&](auto&& f) {
        for (uint32_t i = tid; i < n_c; i += NT) f(cand[i]);
      };
      found = radix_pass<NT, S2, B2>(visit_cand, hist, wsum, info, prefix, krem, cnt, true,
                                     thr_key);
      if (!found) radix_pass<NT, 0, B3>(visit_cand, hist, wsum, info, prefix, krem, cnt, false,
                                        thr_key);
    } else {
      found = radix_pass<NT, S2, B2>(visit_regs, hist, wsum, info, prefix, krem, cnt, true,
                                     thr_key);
      if (!found) radix_pass<NT, 0, B3>(visit_regs, hist, wsum, info, prefix, krem, cnt, false,
                                        thr_key);
    }
    if (!found) thr_key = prefix;
  }
  if (tid == 0) a.thr[row] = key_to_float(thr_key);

  if (a.idx != nullptr) {
    int32_t* out = a.idx + row * static_cast<int64_t>(k);
    emit_indices<NT>(out, nch, thr_key, krem, wsum, [&](int64_t j, uint32_t(&kk)[4]) {
#pragma unroll
      for (int jj = 0; jj < NCH; ++jj)
        if (jj == j) {
#pragma unroll
          for (int c = 0; c < 4; ++c) kk[c] = key[4 * jj + c];
        }
    });
  }
}

// ---------------------------------------------------------------------------
// Streaming kernel: any row length; the row is re-read on every pass.
// ---------------------------------------------------------------------------
template <int NT, bool VEC>
__global__ __launch_bounds__(NT) void topk_stream_kernel(SelectArgs a) {
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t wsum[NT / kWave];
  __shared__ uint32_t info[4];

  const int tid = threadIdx.x;
  int64_t row, nvalid;
  row_of_block(a, row, nvalid);
  const int k = a.k;
  if (nvalid < k) {
    emit_short_row<NT>(a, row);
    return;
  }
  const float* __restrict__ src = a.scores + row * a.ld;
  const int64_t nchunks = (nvalid + 4 * NT - 1) / (4 * NT);
  auto chunk = [&](int64_t j, uint32_t(&kk)[4]) {
    load_keys4<VEC>(src, (j * NT + tid) * 4, nvalid, kk);
  };
  auto visit = [&](auto&& f) {
    for (int64_t j = 0; j < nchunks; ++j) {
      uint32_t kk[4];
      chunk(j, kk);
#pragma unroll
      for (int c = 0; c < 4; ++c) f(kk[c]);
    }
  };
  uint32_t prefix = 0, krem = static_cast<uint32_t>(k), cnt = 0, thr_key = 0;
  bool found = radix_pass<NT, kS1, kP1>(visit, hist, wsum, info, prefix, krem, cnt, true, thr_key);
  if (!found) found = radix_pass<NT, kS2, kB2>(visit, hist, wsum, info, prefix, krem, cnt, true,
                                             thr_key);
  if (!found) radix_pass<NT, 0, kB3>(visit, hist, wsum, info, prefix, krem, cnt, false, thr_key);
  if (!found) thr_key = prefix;
  if (tid == 0) a.thr[row] = key_to_float(thr_key);
  if (a.idx != nullptr)
    emit_indices<NT>(a.idx + row * static_cast<int64_t>(k), nchunks, thr_key, krem, wsum, chunk);
}

template <int NT, int V, int P1>
hipError_t launch_reg(const SelectArgs& a, bool vec, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.rows));
  if (vec)
    hipLaunchKernelGGL((topk_reg_kernel<NT, V, P1, true>), grid, dim3(NT), 0, stream, a);
  else
    hipLaunchKernelGGL((topk_reg_kernel<NT, V, P1, false>), grid, dim3(NT), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_stream(const SelectArgs& a, bool vec, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.rows));
  if (vec)
    hipLaunchKernelGGL((topk_stream_kernel<1024, true>), grid, dim3(1024), 0, stream, a);
  else
    hipLaunchKernelGGL((topk_stream_kernel<1024, false>), grid, dim3(1024), 0, stream, a);
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
  // Rows above 8K entries use a 12-bit first digit: hot digits of real
  // score rows spread over twice the bins (fewer same-address LDS atomics)
  // and the chosen digit leaves half the candidates.
  if (cap <= 512) return launch_reg<128, 4, 11>(a, vec, stream);
  if (cap <= 1024) return launch_reg<128, 8, 11>(a, vec, stream);
  if (cap <= 2048) return launch_reg<256, 8, 11>(a, vec, stream);
  if (cap <= 4096) return launch_reg<256, 16, 11>(a, vec, stream);
  if (cap <= 8192) return launch_reg<512, 16, 11>(a, vec, stream);
  if (cap <= 16384) return launch_reg<512, 32, 12>(a, vec, stream);
  if (cap <= 32768) return launch_reg<1024, 32, 12>(a, vec, stream);
  return launch_stream(a, vec, stream);
}

}  // namespace dsa
