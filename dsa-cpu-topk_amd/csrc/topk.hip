// topk.hip -- per-row k-th largest ("top-K threshold") by block radix-select.
//
// Contract (reference topk_avx512.cpp:226-249, dsa_attention.py:41-44):
// thr[r] is the k-th largest value of row r counting ties, i.e.
// torch.topk(row, k).values[-1].  Optionally also the exactly-k index set a
// stable descending sort puts first (lowest index wins ties), in ascending
// index order.
//
// Design (gfx950): one workgroup per row, the row read from HBM exactly once
// straight into registers (V values per thread, float4 loads, chunk-major so
// each load instruction is one contiguous 16*NT-byte span; chunks past the
// row's valid length are skipped block-uniformly).  Rows of up to 16 values
// per thread first try value bins: the row's min and max (one block
// reduction), a 512-bin histogram linear in value between them, the bin
// holding the k-th largest (usually a few values) appended to an LDS list and
// ranked by key in one wave.  Bins follow the data's density, so the
// histogram's LDS atomics rarely collide and the finish has a few values to
// rank; this takes fewer VALU instructions per value than the digit passes
// below (config 3's causal rows of 1..4096: 44 -> 34.9 us; with no 64-bit
// division per row, 32.4 us).  A bin of more than
// kCandCap values (heavy ties) and longer register rows take MSD radix passes
// over order-preserving keys, 11/11/10-bit digits:
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
#include <cmath>

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
  int64_t nbatch;  // rows / causal_T in causal mode (set by the host)
  // Causal rows only, threshold-only bracket kernel: also the row's
  // selection bitmask (the words selection_mask_kernel writes), ldm words
  // per row; null: none.
  uint64_t* mask = nullptr;
  int64_t ldm = 0;
};

// Row r of the 1-D causal order: q = r / nb (rows longest first), r % nb
// the batch element; 32-bit arithmetic when the grid allows it (r is
// wave-uniform, so this is scalar work).
__device__ __forceinline__ void causal_div(int64_t r, int64_t nb, int64_t& q, int64_t& m) {
  if (r <= 0xffffffffll && nb <= 0xffffffffll) {
    const uint32_t q32 = static_cast<uint32_t>(r) / static_cast<uint32_t>(nb);
    q = q32;
    m = static_cast<uint32_t>(r) - q32 * static_cast<uint32_t>(nb);
  } else {
    q = r / nb;
    m = r % nb;
  }
}


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
  if (a.causal_T > 0 && gridDim.y > 1) {
    // 2-D causal grid (batch element fastest, then rows longest first): the
    // same order as the 1-D mapping below, without a 64-bit division.
    const int64_t t = a.causal_T - 1 - static_cast<int64_t>(blockIdx.y);
    row = static_cast<int64_t>(blockIdx.x) * a.causal_T + t;
    nvalid = t + 1;
  } else if (a.causal_T > 0) {
    int64_t q, m;
    causal_div(blockIdx.x, a.nbatch, q, m);
    const int64_t t = a.causal_T - 1 - q;
    row = m * a.causal_T + t;
    nvalid = t + 1;
  } else {
    row = blockIdx.x;
    nvalid = a.n;
  }
}

// Causal row with fewer than k real entries: the k-th largest of the full row
// is one of the implicit -inf entries, and a stable sort puts the real
// entries first, then the -inf ones in index order.
// Selection bitmask of causal row `row` (query t, T = causal_T) for the
// threshold th, once the block knows it: word w holds keys 64w .. 64w+63,
// bit i set iff key 64w+i <= t and its score >= th (a NaN score or threshold
// selects nothing); words 0 .. min(ceil(T/64)-1, (t|127)/64) are written,
// those past the causal range as 0 -- what selection_mask_kernel writes
// (tile_attn.hip), here from the row the block has just streamed: the
// re-read misses L2 but comes mostly from the MALL (config 4: 537 MB in
// ~60 us, above HBM's peak rate), not HBM.  The block's waves split
// the row's groups of 64 words; lane u of a wave keeps word 64c + u of its
// group c, so each group is one coalesced 512-byte store.
template <int NT>
__device__ __forceinline__ void emit_mask_row(const SelectArgs& a, int64_t row, int t,
                                              float th) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int T = static_cast<int>(a.causal_T);
  const float* __restrict__ srow = a.scores + row * a.ld;
  uint64_t* __restrict__ mrow = a.mask + row * a.ldm;
  const int W = (T + 63) / 64;
  const int nw = min(W, ((t | 127) >> 6) + 1);
  constexpr int U = 16;  // loads in flight per lane
  for (int c = 64 * wid; c < nw; c += 64 * NW) {
    const int nu = min(64, nw - c);
    uint64_t mine = 0;
    for (int u = 0; u < nu; u += U) {
      float v[U];
#pragma unroll
      for (int e = 0; e < U; ++e) v[e] = srow[min(64 * (c + u + e) + lane, t)];  // in the row
#pragma unroll
      for (int e = 0; e < U; ++e) {
        const uint64_t bits = ballot(64 * (c + u + e) + lane <= t && v[e] >= th);
        mine = (lane == u + e) ? bits : mine;
      }
    }
    if (lane < nu) mrow[c + lane] = mine;
  }
}

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

// Finds the digits holding the r[q]-th largest keys of an NB-bin histogram
// (one suffix scan for all R ranks).  Thread tid owns bins [tid*BPT,
// tid*BPT+BPT).  Ends with a barrier after which, for each q, info[3q] =
// digit, info[3q+1] = rank of the wanted key inside the digit, info[3q+2] =
// keys in the digit.  REV: the histogram is stored highest digit first
// (hist[NB-1-d] counts digit d).
template <int NT, int NB, int R, bool REV = false>
__device__ __forceinline__ void find_digits(const uint32_t* hist, const uint32_t (&r)[R],
                                            uint32_t* wsum, uint32_t* info) {
  constexpr int BPT = NB >= NT ? NB / NT : 1;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int lo = tid * BPT;
  uint32_t h[BPT];
  uint32_t local = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    h[i] = (lo + i < NB) ? hist[REV ? NB - 1 - (lo + i) : lo + i] : 0u;
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
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const uint32_t want = r[q];
    if (above < want && above + local >= want) {
      uint32_t cum = above;
      bool done = false;
#pragma unroll
      for (int i = BPT - 1; i >= 0; --i) {
        if (!done && cum + h[i] >= want) {
          info[3 * q] = static_cast<uint32_t>(lo + i);
          info[3 * q + 1] = want - cum;
          info[3 * q + 2] = h[i];
          done = true;
        }
        cum += h[i];
      }
    }
  }
  block_sync_lds();
}

template <int NT, int NB, bool REV = false>
__device__ __forceinline__ void find_digit(const uint32_t* hist, uint32_t krem, uint32_t* wsum,
                                           uint32_t* info) {
  const uint32_t r[1] = {krem};
  find_digits<NT, NB, 1, REV>(hist, r, wsum, info);
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

// krem-th largest of candidate keys that all share their bits above bit
// `low` (those bits are `prefix`), by one wave.  visit(f) calls f(key) for
// this lane's share of the candidates (in LDS), so every pass re-reads them.
// MSD passes over at most 8 of the remaining bits, each a 256-bin histogram
// in `hist` (wave-private LDS) built with ds_add and a wave suffix scan --
// wave-level syncs only, no block barrier.  A digit holding a single key
// ends the search early.
template <typename Visit>
__device__ __forceinline__ uint32_t wave_select_keys(Visit&& visit, uint32_t prefix, int low,
                                                     uint32_t krem, uint32_t* hist) {
  const int lane = threadIdx.x & (kWave - 1);
  int shift = low;
  while (shift > 0) {
    const int bits = shift >= 8 ? 8 : shift;
    shift -= bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int hi = shift + bits;  // may be 32: 64-bit shifts below
    reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    visit([&](uint32_t kk) {
      if ((static_cast<uint64_t>(kk) >> hi) == prefix) atomicAdd(&hist[(kk >> shift) & mask], 1u);
    });
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
      visit([&](uint32_t kk) {
        if ((kk >> shift) == prefix) hit = kk;
      });
      const uint64_t m = __ballot(hit != 0u);
      return wave_read_lane(hit, __ffsll(static_cast<unsigned long long>(m)) - 1);
    }
  }
  return prefix;
}

// wave_select_keys over n candidates stored contiguously at cand.
__device__ __forceinline__ uint32_t wave_select_cand(const uint32_t* cand, uint32_t n,
                                                     uint32_t prefix, int low, uint32_t krem,
                                                     uint32_t* hist) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  return wave_select_keys(
      [&](auto&& f) {
        for (uint32_t i = lane; i < n; i += kWave) f(cand[i]);
      },
      prefix, low, krem, hist);
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
  __shared__ __align__(16) uint32_t hist[NBINS];
  constexpr int CAP = kCandCap;
  __shared__ uint32_t cand[CAP];
  __shared__ uint32_t wsum[NT / kWave];
  __shared__ uint32_t info[4];
  __shared__ uint32_t ncand;
  __shared__ float red[3 * (NT / kWave)];

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
  // The row as float bit patterns (key order is formed only where needed).
  uint32_t key[V];
  const int nv = static_cast<int>(nvalid);  // the host checks n < 2^31
  {
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
#pragma unroll
    for (int j = 0; j < V; ++j) key[j] = __float_as_uint(raw[j]);
  }
  // f(x, i) for every valid entry: x its value, i its register (chunks past
  // nch hold clamped duplicates; only the chunk the row ends inside tests
  // positions).
  auto visit_vals = [&](auto&& f) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j < nch) {
        if ((j + 1) * NT * 4 <= nv) {
#pragma unroll
          for (int c = 0; c < 4; ++c) f(__uint_as_float(key[4 * j + c]), 4 * j + c);
        } else {
          const int p0 = (j * NT + tid) * 4;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (p0 + c < nv) f(__uint_as_float(key[4 * j + c]), 4 * j + c);
        }
      }
    }
  };
  // Registers -> radix keys in place; entries past the row become kKeyNone
  // (only a chunk the row ends inside needs the per-entry test).
  auto to_keys = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
#pragma unroll
      for (int c = 0; c < 4; ++c) key[4 * j + c] = float_to_key(__uint_as_float(key[4 * j + c]));
      if ((j + 1) * NT * 4 > nv) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if ((j * NT + tid) * 4 + c >= nv) key[4 * j + c] = kKeyNone;
      }
    }
  };
  auto visit_regs = [&](auto&& f) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j < nch) {
#pragma unroll
        for (int c = 0; c < 4; ++c) f(key[4 * j + c]);
      }
    }
  };

  uint32_t thr_key = 0, krem = 0;
  bool keys_in_regs = false, done = false;
  if (tid == 0) ncand = 0u;
  // Rows of up to 16 values per thread search by value bins first; longer
  // register rows (32 per thread) have no registers to spare for it and go
  // straight to the radix passes.
  if constexpr (V <= 16) {
  // Stage 1: the row's min and max (block reduction; min and max ignore NaN);
  // the histogram is cleared meanwhile.
  constexpr int NW = NT / kWave;
  const int wid = tid / kWave;
  constexpr int NBV = 512;  // value bins
  for (int b = tid; b < NBV / 4; b += NT) reinterpret_cast<uint4*>(hist)[b] = make_uint4(0u, 0u, 0u, 0u);
  float lo = __builtin_huge_valf(), hi = -__builtin_huge_valf();
  visit_vals([&](float x, int) {
    lo = fminf(lo, x);
    hi = fmaxf(hi, x);
  });
  auto block_range = [&]() __attribute__((always_inline)) {
    lo = wave_extreme_f32<false>(lo);
    hi = wave_extreme_f32<true>(hi);
    if (lane == 0) {
      red[wid] = lo;
      red[NW + wid] = hi;
    }
    block_sync_lds();
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      lo = fminf(lo, red[w]);
      hi = fmaxf(hi, red[NW + w]);
    }
  };
  block_range();
  if (!(lo > -__builtin_huge_valf()) || !(hi < __builtin_huge_valf())) {
    // An infinite value (block-uniform, rare): the finite range instead.
    block_sync_lds();  // every wave has read red
    lo = __builtin_huge_valf();
    hi = -__builtin_huge_valf();
    visit_vals([&](float x, int) {
      const bool fin = fabsf(x) <= __FLT_MAX__;
      lo = fminf(lo, fin ? x : __builtin_huge_valf());
      hi = fmaxf(hi, fin ? x : -__builtin_huge_valf());
    });
    block_range();
  }
  // Stage 2: NBV bins linear in value between lo and hi.  Bins follow the
  // data's density, so the histogram's ds_adds rarely collide, and the bin
  // holding the k-th largest usually holds a few values.  Bins only steer
  // the search: the candidates are ranked by key, so the result is exact for
  // any input.  Bins are counted from the top: c = med3((hi - x)*scale, 0,
  // top) is monotone (decreasing) in the key order with no test for special
  // values -- +inf lands in c = 0, and NaN too (med3 with a NaN operand
  // returns the minimum of the other two, 0, and so does the conversion of a
  // NaN); -inf in c = top.  A degenerate range (one finite value, none, or a
  // span that overflows) keeps scale = 1: the values then crowd the end
  // bins, which only costs the fallback below.  Each value's c is kept, two
  // per register, for the compaction.
  constexpr float kTop = static_cast<float>(NBV - 1);
  float scale = static_cast<float>(NBV) / (hi - lo);
  if (!(hi > lo) || !(scale > 0.0f && scale <= __FLT_MAX__)) {
    scale = 1.0f;
    if (!(fabsf(hi) <= __FLT_MAX__)) hi = 0.0f;
  }
  // (hi - x)*scale in one rounding: monotone in x
  const float hoff = hi * scale;
  auto bin_of = [&](float x) __attribute__((always_inline)) -> uint32_t {
    return static_cast<uint32_t>(
        __builtin_amdgcn_fmed3f(__builtin_fmaf(x, -scale, hoff), 0.0f, kTop));
  };
  uint32_t bp[V / 2];
#pragma unroll
  for (int i = 0; i < V / 2; ++i) bp[i] = 0u;
  visit_vals([&](float x, int i) {
    const uint32_t c = bin_of(x);
    atomicAdd(&hist[c], 1u);
    bp[i >> 1] |= c << (16 * (i & 1));
  });
  auto bin_at = [&](int i) __attribute__((always_inline)) {
    return (bp[i >> 1] >> (16 * (i & 1))) & 0xffffu;
  };
  block_sync_lds();
  find_digit<NT, NBV, true>(hist, static_cast<uint32_t>(k), wsum, info);
  const uint32_t csel = NBV - 1 - info[0], brank = info[1], bcnt = info[2];
  if (bcnt <= static_cast<uint32_t>(CAP)) {
    // Stage 3: the chosen bin's values (a few, usually), as keys, appended
    // to an LDS list in any order, then ranked by one wave: pairwise when
    // they fit a wave, else 8-bit radix passes.
    visit_vals([&](float x, int i) {
      if (bin_at(i) == csel) cand[atomicAdd(&ncand, 1u)] = float_to_key(x);
    });
    block_sync_lds();
    // Threshold only: the other waves exit now, so their registers take the
    // next rows' loads.
    if (a.idx == nullptr && tid >= kWave) return;
    if (tid < kWave) {
      uint32_t tk, ngt;
      if (bcnt <= static_cast<uint32_t>(kWave)) {
        const uint32_t mk = lane < static_cast<int>(bcnt) ? cand[lane] : 0u;
        uint32_t gt = 0, ge = 0;
        for (uint32_t j = 0; j < bcnt; ++j) {
          const uint32_t o = wave_read_lane(mk, static_cast<int>(j));  // lane j's key, no LDS read
          gt += (o > mk) ? 1u : 0u;
          ge += (o >= mk) ? 1u : 0u;
        }
        const bool hit = lane < static_cast<int>(bcnt) && gt < brank && ge >= brank;
        const int src = __ffsll(static_cast<unsigned long long>(ballot(hit))) - 1;
        tk = wave_read_lane(mk, src);
        ngt = wave_read_lane(gt, src);
      } else {
        tk = wave_select_cand(cand, bcnt, 0u, 32, brank, hist);
        uint32_t g = 0;
        for (uint32_t i = lane; i < bcnt; i += kWave) g += (cand[i] > tk) ? 1u : 0u;
        ngt = wave_read_lane(wave_inclusive_sum(g), kWave - 1);
      }
      if (a.idx == nullptr) {
        if (tid == 0) a.thr[row] = key_to_float(tk);
        return;
      }
      if (tid == 0) {
        info[0] = tk;
        info[1] = brank - ngt;  // rank of the wanted key among the keys equal to it
      }
    }
    block_sync_lds();
    thr_key = info[0];
    krem = info[1];
    done = true;
  }
  }  // V <= 16
  if (!done) {
    // A bin of more than CAP values (heavy ties, or a row whose values
    // sit at the ends of a huge range), or rows of 32 values per thread: MSD
    // radix passes over the keys in registers, 11/11/10 (or 12/10/10) bits.
    to_keys();
    keys_in_regs = true;
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
    uint32_t prefix = 0, cnt = 0;
    krem = static_cast<uint32_t>(k);
    bool found = radix_pass<NT, S1, P1, true>(visit_first, hist, wsum, info, prefix, krem, cnt,
                                              true, thr_key);
    if (!found) {
      if (cnt <= static_cast<uint32_t>(CAP)) {
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
  }
  if (tid == 0) a.thr[row] = key_to_float(thr_key);

  if (a.idx != nullptr) {
    if (!keys_in_regs) to_keys();
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
// Exact k-th largest key of the nvalid entries at src by three radix passes
// that each re-read the row; krem is left at the rank of the wanted key among
// the keys equal to it.  hist: kBins words of LDS.
template <int NT, bool VEC>
__device__ __forceinline__ uint32_t stream_select(const float* __restrict__ src, int64_t nvalid,
                                                  int k, uint32_t* hist, uint32_t* wsum,
                                                  uint32_t* info, uint32_t& krem) {
  const int tid = threadIdx.x;
  const int64_t nchunks = (nvalid + 4 * NT - 1) / (4 * NT);
  auto visit = [&](auto&& f) {
    for (int64_t j = 0; j < nchunks; ++j) {
      uint32_t kk[4];
      load_keys4<VEC>(src, (j * NT + tid) * 4, nvalid, kk);
#pragma unroll
      for (int c = 0; c < 4; ++c) f(kk[c]);
    }
  };
  uint32_t prefix = 0, cnt = 0, thr_key = 0;
  krem = static_cast<uint32_t>(k);
  bool found = radix_pass<NT, kS1, kP1>(visit, hist, wsum, info, prefix, krem, cnt, true, thr_key);
  if (!found) found = radix_pass<NT, kS2, kB2>(visit, hist, wsum, info, prefix, krem, cnt, true,
                                             thr_key);
  if (!found) radix_pass<NT, 0, kB3>(visit, hist, wsum, info, prefix, krem, cnt, false, thr_key);
  return found ? thr_key : prefix;
}

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
  uint32_t krem;
  const uint32_t thr_key = stream_select<NT, VEC>(src, nvalid, k, hist, wsum, info, krem);
  if (tid == 0) a.thr[row] = key_to_float(thr_key);
  if (a.idx != nullptr) {
    const int64_t nchunks = (nvalid + 4 * NT - 1) / (4 * NT);
    emit_indices<NT>(a.idx + row * static_cast<int64_t>(k), nchunks, thr_key, krem, wsum,
                     [&](int64_t j, uint32_t(&kk)[4]) {
                       load_keys4<VEC>(src, (j * NT + tid) * 4, nvalid, kk);
                     });
  }
}

// ---------------------------------------------------------------------------
// Bracket kernel: thresholds of long rows in one pass over the row.
// ---------------------------------------------------------------------------
constexpr int kBrBins = 1024;    // sample histogram: value bins over the sample's range
constexpr int kFinBins = 256;    // finishing wave's value bins over the kept values
constexpr int kFinGather = 64;   // kept values of one finishing bin ranked in registers

// A sample of four 4*NT-entry chunks spread evenly over the row is held in
// registers and ranked approximately: one LDS histogram over kBrBins bins
// linear in VALUE between the sample's minimum and maximum (bins follow the
// data's density, so ds_add rarely collides).  With m of the row's n entries
// in the sample, the row's k-th largest sits near sample rank e = k*m/n; the
// bins holding sample ranks e - delta and e + delta (delta = five standard
// deviations of that rank, plus 2), widened by a bin each side, give a value
// interval [lo, hi).  The rest of the row then streams through once,
// compared as floats: each thread counts its values below hi (NaN is not)
// and keeps those in [lo, hi) in its own LDS column -- every value is
// written to the column's next free slot and the slot index advances only
// when the value is kept, so there is no branch and no atomic per value.
// These sets are intervals of the key order (NaN largest, -0 == +0), so the
// interval only steers the search and exactness comes from the check: with
// above = n - (values below hi), when above < k <= above + kept the row's
// k-th largest is the (k - above)-th largest kept value; otherwise (the
// sample missed, or a column or the kept list outgrew LDS) the row is
// selected exactly by the streaming radix passes.  The kept values are then
// compacted into one list and one wave finishes: a histogram of them over
// kFinBins value bins between their minimum and maximum, then the few values
// of the bin holding the wanted rank are ranked against each other in
// registers (a bin holding more than kFinGather, i.e. heavy ties, takes
// radix passes over the kept keys).  A row of at most four chunks is its own
// sample (delta = 0).
//
// IDX (rows of at most 16 chunks): the exactly-k index set too, from the
// same single read of the row.  While streaming, each thread records which
// of its entries lie above the interval (certainly selected: abv, bit 4j+c
// for position (j*NT+tid)*4+c) and which it kept (kpt, same bit order).
// Its kept values sit in its column in streaming order: the sample chunks'
// first, then the other chunks', each group in position order, so the s-th
// kept value is the s-th set bit of kpt over the sample chunks' nibbles,
// then over the rest.  Once the threshold is known, each thread sorts its
// kept values into above / equal to it; the flags go to an LDS bitmap in
// position order, and one block-wide scan over 64-position ranges places
// every selected entry at #(above before it) + min(#(equal before it), k -
// #above), ascending positions -- emit_indices' rule without a pass per
// chunk.  MASK (the same rows): the bitmap's words are the bitmask.
// Eight blocks per CU (at most 64 VGPRs; the LDS columns allow eight): at
// config 4 thresholds 101 -> 98 us, with indices 156 -> 152, the bitmask
// 129 -> 127 against six (the bitmask and index forms spill a few SGPRs).
template <int NT, bool IDX, bool MASK = false>
__global__ __launch_bounds__(NT, 8) void topk_bracket_kernel(SelectArgs a) {
  // IDX: exactly-k indices; MASK: the selection bitmask (a.mask), both from
  // the row's flag bitmap below.
  static_assert(!(IDX && MASK), "one output mode");
  constexpr bool FLAGS = IDX || MASK;
  constexpr int NW = NT / kWave;
  constexpr int CH = 4 * NT;  // entries per chunk (one float4 per thread)
  constexpr int CAP = 19;     // LDS column slots per thread
  static_assert(NT == 256 && kBrBins == 4 * NT, "layout below assumes 4 waves of 4 bins");
  static_assert(CAP * NT >= kCandCap + kFinBins + kFinGather, "finish fits the columns");
  // IDX: the flag bitmap (16*NT bytes) sits past the finishing wave's LDS;
  // k indices of up to kIdxStage are staged in the columns' LDS afterwards.
  constexpr int kIdxMapWord = (kCandCap + kFinBins + kFinGather + 3) & ~3;
  constexpr int kIdxStage = CAP * NT;
  static_assert(!FLAGS || kIdxMapWord + 16 * NT / 4 <= CAP * NT, "the flag bitmap fits the columns");
  // lds: sample histogram [0, kBrBins), then per-thread columns (slot s of
  // thread t at s*NT + t), then the compacted kept list [0, n_kept) with the
  // finishing wave's histogram and gather list at kCandCap.
  __shared__ __align__(16) uint32_t lds[CAP * NT];
  __shared__ uint32_t wsum[NW];
  __shared__ uint32_t info[6];
  __shared__ float wext[2 * NW];
  __shared__ uint32_t wcnt[NW], wbad[NW];
  __shared__ float rsh[1];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  int64_t row, nvalid;
  row_of_block(a, row, nvalid);
  const int k = a.k;
  // (mask: causal rows, so the query is t = nvalid - 1; a.mask is uniform)
  if (nvalid < k) {
    emit_short_row<NT>(a, row);
    if (!IDX && a.mask != nullptr) emit_mask_row<NT>(a, row, static_cast<int>(nvalid) - 1, -__builtin_huge_valf());
    return;
  }
  const float* __restrict__ src = a.scores + row * a.ld;
  const char* row_bytes = reinterpret_cast<const char*>(src);
  const int nv = static_cast<int>(nvalid);  // the host keeps rows below 2^20 entries
  const int last4 = (nv - 1) & ~3;
  const int nc = (nv + CH - 1) / CH;
  const bool whole = nc <= 4;
  // Clamped float4 load of chunk j: no load behind a branch.
  auto load4 = [&](int j) -> float4 {
    const uint32_t off = static_cast<uint32_t>(min((j * NT + tid) * 4, last4)) * 4u;
    return *reinterpret_cast<const float4*>(row_bytes + off);
  };
  auto sample_chunk = [&](int s) { return whole ? s : (s * nc) / 4; };
  // Sample entry i of this thread lies inside the row (always, unless whole).
  auto sample_in = [&](int i) { return (sample_chunk(i / 4) * NT + tid) * 4 + (i & 3) < nv; };

  float sv[16];
  {
    float4 f[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = load4(sample_chunk(s));
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sv[4 * s] = f[s].x;
      sv[4 * s + 1] = f[s].y;
      sv[4 * s + 2] = f[s].z;
      sv[4 * s + 3] = f[s].w;
    }
  }
  uint32_t r1 = static_cast<uint32_t>(k), r2 = static_cast<uint32_t>(k);
  if (!whole) {
    const float frac = static_cast<float>(4 * CH) / static_cast<float>(nv);
    const float e = static_cast<float>(k) * frac;
    const float delta = 5.0f * sqrtf(e * (1.0f - frac)) + 2.0f;
    r1 = static_cast<uint32_t>(max(1.0f, floorf(e - delta)));
    r2 = static_cast<uint32_t>(min(static_cast<float>(4 * CH), ceilf(e + delta)));
  }

  // Range of the sample (NaN ignored by fmax/fmin; entries past the row
  // become NaN here).  An infinite end is replaced by the finite range.
  auto block_range = [&](bool finite_only, float& vmin, float& vmax) {
    float hi = -__builtin_huge_valf(), lo = __builtin_huge_valf();
    // (two copies on the block-uniform `whole`: only rows that are their
    // own sample test each entry against the row's end)
    auto extend = [&](float v) {
      if (finite_only) v = fabsf(v) <= __FLT_MAX__ ? v : __builtin_nanf("");
      hi = fmaxf(hi, v);
      lo = fminf(lo, v);
    };
    if (whole) {
#pragma unroll
      for (int i = 0; i < 16; ++i) extend(sample_in(i) ? sv[i] : __builtin_nanf(""));
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) extend(sv[i]);
    }
    hi = wave_extreme_f32<true>(hi);
    lo = wave_extreme_f32<false>(lo);
    if (lane == 0) {
      wext[wid] = hi;
      wext[NW + wid] = lo;
    }
    block_sync_lds();
    vmax = -__builtin_huge_valf();
    vmin = __builtin_huge_valf();
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      vmax = fmaxf(vmax, wext[w]);
      vmin = fminf(vmin, wext[NW + w]);
    }
  };
#pragma unroll
  for (int q = 0; q < kBrBins / (4 * NT); ++q)
    reinterpret_cast<uint4*>(lds)[q * NT + tid] = make_uint4(0u, 0u, 0u, 0u);
  float vmin, vmax;
  block_range(false, vmin, vmax);
  if (!(vmax < __builtin_huge_valf()) || !(vmin > -__builtin_huge_valf())) {
    block_sync_lds();  // every wave has read wext
    block_range(true, vmin, vmax);
  }
  // No finite value, a single one, or a range that overflows: one bin.
  const float range = vmax - vmin;
  float scale = static_cast<float>(kBrBins) / range;
  if (!(range > 0.0f) || !(scale <= __FLT_MAX__)) {
    scale = 0.0f;
    vmin = 0.0f;
  }
  if (whole) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (sample_in(i)) atomicAdd(&lds[value_bin(sv[i], vmin, scale, kBrBins - 1)], 1u);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) atomicAdd(&lds[value_bin(sv[i], vmin, scale, kBrBins - 1)], 1u);
  }
  block_sync_lds();
  {
    const uint32_t r[2] = {r1, r2};
    find_digits<NT, kBrBins, 2>(lds, r, wsum, info);
  }
  // Value interval [flo, fhi) covering bins b2 .. b1 (b1 >= b2) and one bin
  // either side (bin edges below are recomputed, not the binning's own
  // rounding); the end bins reach out to -inf and +inf.
  const int b1 = min(static_cast<int>(info[0]) + 1, kBrBins - 1);
  const int b2 = max(static_cast<int>(info[3]) - 1, 0);
  const float flo = b2 == 0 ? -__builtin_huge_valf() : vmin + static_cast<float>(b2) / scale;
  const float fhi = b1 == kBrBins - 1 ? __builtin_huge_valf()
                                      : vmin + static_cast<float>(b1 + 1) / scale;

  // Classify.  find_digits' closing barrier ordered every histogram read.
  uint32_t below = 0, kc = 0;  // this thread: valid values below fhi; kept
  bool bad = false;            // wave-uniform: a column came near CAP
  uint32_t* col = lds + tid;
  uint64_t abv = 0, kpt = 0;   // FLAGS: entries above the interval; kept entries
  // Streams one value: counts it below fhi, keeps it in the column if in
  // [flo, fhi).  FLAGS: kp = kept; ab = above the interval -- indices rank
  // NaN first (torch.topk's order), so for them every valid value not below
  // fhi; the bitmask selects by score >= thr, which no NaN passes, so for it
  // the values >= fhi.  Each flag is one compare (or one reused) and a
  // select of its bit in record(), not a packed code unpacked again.
  struct Took {
    bool kp, ab;
  };
  auto take = [&](float v, bool valid) -> Took {
    const bool lt = valid && v < fhi;
    const bool kp = lt && !(v < flo);
    col[kc * NT] = __float_as_uint(v);  // the next free slot; kept only if kc advances
    below += lt ? 1u : 0u;
    kc += kp ? 1u : 0u;
    return Took{kp, MASK ? (valid && v >= fhi) : (valid && !lt)};
  };
  // FLAGS: a chunk's 4 results into the masks (chunk j).
  auto record = [&](const Took (&r)[4], int j) {
    if constexpr (FLAGS) {
      const uint32_t nk = (r[0].kp ? 1u : 0u) | (r[1].kp ? 2u : 0u) | (r[2].kp ? 4u : 0u) | (r[3].kp ? 8u : 0u);
      const uint32_t na = (r[0].ab ? 1u : 0u) | (r[1].ab ? 2u : 0u) | (r[2].ab ? 4u : 0u) | (r[3].ab ? 8u : 0u);
      abv |= static_cast<uint64_t>(na) << (4 * j);
      kpt |= static_cast<uint64_t>(nk) << (4 * j);
    } else {
      (void)r; (void)j;
    }
  };
  // Before every 4 values: a column with fewer than 4 free slots stops the
  // wave (the row then takes the exact passes).
  auto room = [&]() {
    bad = bad || ballot(kc > static_cast<uint32_t>(CAP - 4)) != 0u;
    return !bad;
  };
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (room()) {
      Took r[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] = take(sv[4 * s + c], !whole || sample_in(4 * s + c));
      record(r, sample_chunk(s));
    }
  }

  auto chunk_of = [&](int u) {  // u-th chunk that is not a sample chunk
    int j = u;
#pragma unroll
    for (int s = 0; s < 4; ++s) j += ((s * nc) / 4 <= j) ? 1 : 0;
    return j;
  };
  if (!whole && !bad) {
    // Chunks outside the sample, 4 per step, the next step's loads in flight
    // while this step's values are classified.
    const int ns = nc - 4;
    const int nsteps = (ns + 3) / 4;
    float4 cur[4];
    int jc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      jc[q] = chunk_of(min(q, ns - 1));
      cur[q] = load4(jc[q]);
    }
    for (int it = 0; it < nsteps; ++it) {
      float4 nxt[4];
      int jn[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        jn[q] = chunk_of(min(4 * (it + 1) + q, ns - 1));
        nxt[q] = load4(jn[q]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float fv[4] = {cur[q].x, cur[q].y, cur[q].z, cur[q].w};
        if (4 * it + q < ns && room()) {  // else a repeated load past the last chunk
          Took r[4];
          if ((jc[q] + 1) * CH <= nv) {
#pragma unroll
            for (int c = 0; c < 4; ++c) r[c] = take(fv[c], true);
          } else {
            const int p0 = (jc[q] * NT + tid) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c) r[c] = take(fv[c], p0 + c < nv);
          }
          record(r, jc[q]);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cur[q] = nxt[q];
        jc[q] = jn[q];
      }
    }
  }

  // Block totals: values below fhi and kept, and whether a column filled.
  {
    const uint32_t wb = wave_read_lane(wave_inclusive_sum((below << 12) | kc), kWave - 1);
    if (lane == 0) {
      wcnt[wid] = wb;
      wbad[wid] = bad ? 1u : 0u;
    }
  }
  // Kept values to registers before the columns are overwritten by the list.
  uint32_t mine[CAP];
#pragma unroll
  for (int s = 0; s < CAP; ++s) mine[s] = col[s * NT];
  uint32_t ktot;
  const uint32_t kbase = block_exclusive_sum<NT>(kc, wsum, ktot);  // its barriers order the reads
  uint32_t tot_below = 0;
  bool any_bad = false;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    tot_below += wcnt[w] >> 12;
    any_bad = any_bad || wbad[w] != 0u;
  }
  const uint32_t ku = static_cast<uint32_t>(k);
  const uint32_t tot_above = static_cast<uint32_t>(nv) - tot_below;
  if (!any_bad && ktot <= static_cast<uint32_t>(kCandCap) && tot_above < ku &&
      ku <= tot_above + ktot) {
#pragma unroll
    for (int s = 0; s < CAP; ++s)
      if (static_cast<uint32_t>(s) < kc) lds[kbase + s] = mine[s];
    // FLAGS: the row's flags as an LDS bitmap in position order, past what
    // the finishing wave uses: byte j*NT+t holds positions (j*NT+t)*4 .. +3,
    // above the threshold in the low nibble, equal to it in the high one.
    uint8_t* fb = reinterpret_cast<uint8_t*>(lds + kIdxMapWord);
    // MASK: before the other waves exit, every thread writes its "above"
    // bits into the LDS bitmap (byte j*NT+t: positions (j*NT+t)*4 .. +3) and,
    // next to each of its kept values in the list, that value's bit in the
    // bitmap; wave 0 then finishes the threshold alone and sets the bits of
    // the kept values at or above it.  (Waves held at a barrier while wave 0
    // finishes cost more streaming throughput than wave 0's longer tail:
    // config 4, 9 us.  Leaving only each thread's flag words and list range
    // and having wave 0 expand them into the bitmask was no faster: 130 us
    // either way, the work moved into the tail.)  The s-th kept value of a
    // thread is the s-th set bit of its kept mask over the sample chunks'
    // nibbles, then over the rest.
    uint16_t* posl = reinterpret_cast<uint16_t*>(lds + kIdxMapWord + 16 * NT / 4);
    static_assert(!MASK || kIdxMapWord + 16 * NT / 4 + kCandCap / 2 <= CAP * NT, "the bit list fits");
    if constexpr (MASK) {
#pragma unroll
      for (int j = 0; j < 16; ++j) fb[j * NT + tid] = static_cast<uint8_t>((abv >> (4 * j)) & 15u);
      uint64_t smask = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) smask |= uint64_t{15} << (4 * sample_chunk(q));
      // Two walks, one per group (a single walk that switches groups when
      // the first runs out costs 4 us more at config 4).
      uint16_t* pl = posl + kbase;
      auto walk = [&](uint64_t m) {
        while (m != 0u) {
          const int bp = static_cast<int>(__builtin_ctzll(m));
          m &= m - 1u;
          // bit (bp & 3) of byte (bp >> 2) * NT + tid
          *pl++ = static_cast<uint16_t>(((((bp >> 2) * NT + tid)) << 3) | (bp & 3));
        }
      };
      walk(kpt & smask);
      walk(kpt & ~smask);
    }
    block_sync_lds();
    if (MASK && wid != 0) return;
    // The low nibbles of 16 bytes whose high nibbles are 0 -> 64 bits (the
    // bitmap's 64 positions, byte i's at bits 4i .. 4i+3): one shift and OR
    // puts two bytes' nibbles side by side, and a byte permute takes those
    // of four bytes (config 4: bitmask 2 us faster than a mask and a shift
    // per nibble, the index form 3-4 us with the walks below).
    auto pack_nibbles = [](uint4 v) {
      auto pack2 = [](uint32_t lo, uint32_t hi) {
        return __builtin_amdgcn_perm(hi | (hi >> 4), lo | (lo >> 4), 0x06040200u);
      };
      return static_cast<uint64_t>(pack2(v.x, v.y)) | (static_cast<uint64_t>(pack2(v.z, v.w)) << 32);
    };
    if (wid == 0) {  // one wave finishes on the kept list
      const uint32_t krem = ku - tot_above;
      // (MASK: four LDS reads in flight per step -- config 4 bitmask 1 us
      // faster, thresholds and indices 1-2 us slower; the steps are
      // wave-uniform, so a ballot inside f sees every lane that still has a
      // value)
      auto visit_kept = [&](auto&& f) {
        uint32_t b = 0;
        for (; MASK && b + 4 * kWave <= ktot; b += 4 * kWave) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = __uint_as_float(lds[b + q * kWave + lane]);
#pragma unroll
          for (int q = 0; q < 4; ++q) f(v[q]);
        }
        for (uint32_t i = b + lane; i < ktot; i += kWave) f(__uint_as_float(lds[i]));
      };
      // Value bins over the kept values' own range (all below fhi, so NaN is
      // never kept; -inf may be).
      float khi = -__builtin_huge_valf(), klo = __builtin_huge_valf();
      visit_kept([&](float v) {
        khi = fmaxf(khi, v);
        klo = fminf(klo, v);
      });
      khi = wave_extreme_f32<true>(khi);
      klo = wave_extreme_f32<false>(klo);
      const float krange = khi - klo;
      const float ks = static_cast<float>(kFinBins) / krange;
      // Bins need a finite range (klo > -inf); else all equal or -inf kept.
      const bool binned = krange > 0.0f && krange <= __FLT_MAX__ && ks <= __FLT_MAX__;
      uint32_t* fh = lds + kCandCap;
      reinterpret_cast<uint4*>(fh)[lane] = make_uint4(0u, 0u, 0u, 0u);
      wave_lds_sync();
      if (binned) visit_kept([&](float v) { atomicAdd(&fh[value_bin(v, klo, ks, kFinBins - 1)], 1u); });
      else if (lane == 0) fh[0] = ktot;  // one bin: the radix passes below
      wave_lds_sync();
      // Suffix scan over the bins (4 per lane) for the bin holding rank krem.
      const uint4 h4 = reinterpret_cast<const uint4*>(fh)[lane];
      const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
      const uint32_t local = h[0] + h[1] + h[2] + h[3];
      const uint32_t incl = wave_inclusive_sum(local);
      const uint32_t abv = wave_read_lane(incl, kWave - 1) - incl;
      const bool here = abv < krem && abv + local >= krem;
      uint32_t bsel = 0, brank = 0, bcnt = 0;
      if (here) {
        uint32_t cum = abv;
  #pragma unroll
        for (int i = 3; i >= 0; --i) {
          if (bcnt == 0u && cum + h[i] >= krem) {
            bsel = 4u * lane + i;
            brank = krem - cum;
            bcnt = h[i];
          }
          cum += h[i];
        }
      }
      const int srcl = __ffsll(static_cast<unsigned long long>(ballot(here))) - 1;
      bsel = wave_read_lane(bsel, srcl);
      brank = wave_read_lane(brank, srcl);
      bcnt = wave_read_lane(bcnt, srcl);
      float res;
      if (binned && bcnt <= static_cast<uint32_t>(kFinGather)) {
        // Gather the chosen bin's values, then rank them against each other:
        // the wanted one has fewer than brank greater and at least brank
        // greater-or-equal.
        uint32_t* gl = fh + kFinBins;
        uint32_t ng = 0;
        visit_kept([&](float v) {
          const bool in = value_bin(v, klo, ks, kFinBins - 1) == static_cast<int>(bsel);
          const uint64_t m = ballot(in);
          if (in) gl[ng + lanes_below(m)] = __float_as_uint(v);
          ng += popc64(m);
        });
        wave_lds_sync();
        const float mv = lane < static_cast<int>(bcnt) ? __uint_as_float(gl[lane]) : 0.0f;
        uint32_t gt = 0, ge = 0;
        for (uint32_t j = 0; j < bcnt; ++j) {
          const float o = __int_as_float(wave_read_lane(__float_as_int(mv), static_cast<int>(j)));
          gt += (o > mv) ? 1u : 0u;
          ge += (o >= mv) ? 1u : 0u;
        }
        const bool hit = lane < static_cast<int>(bcnt) && gt < brank && ge >= brank;
        res = __int_as_float(wave_read_lane(
            __float_as_int(mv), __ffsll(static_cast<unsigned long long>(ballot(hit))) - 1));
      } else {
        // Heavy ties or no finite range: exact radix passes over the kept keys.
        const uint32_t tk = wave_select_keys(
            [&](auto&& f) { visit_kept([&](float v) { f(float_to_key(v)); }); }, 0u, 32, krem, fh);
        res = key_to_float(tk);
      }
      if (lane == 0) {
        a.thr[row] = res + 0.0f;  // -0 reported as +0, as the key order does
        rsh[0] = res + 0.0f;
      }
      if constexpr (MASK) {
        // the kept values at or above thr set their bits
        const float thr = res + 0.0f;
        uint32_t* fbw = reinterpret_cast<uint32_t*>(fb);
        uint32_t b = 0;
        for (; b + 4 * kWave <= ktot; b += 4 * kWave) {
          float v[4];
          uint32_t p[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            v[q] = __uint_as_float(lds[b + q * kWave + lane]);
            p[q] = posl[b + q * kWave + lane];
          }
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (v[q] >= thr) atomicOr(&fbw[p[q] >> 5], 1u << (p[q] & 31u));
        }
        for (uint32_t i = b + lane; i < ktot; i += kWave) {
          if (__uint_as_float(lds[i]) >= thr) {
            const uint32_t pb = posl[i];
            atomicOr(&fbw[pb >> 5], 1u << (pb & 31u));
          }
        }
        wave_lds_sync();
        // words past the row hold no flags, so the words up to the end of
        // the row's 128-query block are 0 there
        const int nw = min(static_cast<int>((a.causal_T + 63) / 64), (((nv - 1) | 127) >> 6) + 1);
#pragma unroll
        for (int q = 0; q < NW; ++q) {
          const int w = lane + kWave * q;
          if (w < nw) a.mask[row * a.ldm + w] = pack_nibbles(reinterpret_cast<const uint4*>(fb)[w]);
        }
      }
    }  // wave 0
    if constexpr (IDX) {
      block_sync_lds();
      const float thr = rsh[0];
      // This thread's kept values (its kc entries of the kept list) above /
      // equal to thr: the s-th is the s-th set bit of kpt over the sample
      // chunks' nibbles, then over the other chunks'.
      uint64_t smask = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) smask |= uint64_t{15} << (4 * sample_chunk(q));
      uint64_t gt = abv, eq = 0;
      uint32_t s = kbase;
      auto walk = [&](uint64_t m) {  // one walk per group, as for the bitmask
        while (m != 0u) {
          const uint64_t bit = m & (0u - m);
          m ^= bit;
          const float v = __uint_as_float(lds[s++]);
          gt |= v > thr ? bit : 0u;
          eq |= v == thr ? bit : 0u;
        }
      };
      walk(kpt & smask);
      walk(kpt & ~smask);
#pragma unroll
      for (int j = 0; j < 16; ++j)
        fb[j * NT + tid] = static_cast<uint8_t>(((gt >> (4 * j)) & 15u) | (((eq >> (4 * j)) & 15u) << 4));
      block_sync_lds();
      // Thread t takes positions [64t, 64t+64): one scan of its (above,
      // equal) counts places them, and it walks its set bits only.  The k
      // indices are staged in LDS and written out coalesced.
      const uint4 fv = reinterpret_cast<const uint4*>(fb)[tid];
      constexpr uint32_t kLo = 0x0f0f0f0fu;  // "above" in the low nibbles, "equal" in the high
      const uint64_t G = pack_nibbles(make_uint4(fv.x & kLo, fv.y & kLo, fv.z & kLo, fv.w & kLo));
      const uint64_t Eq = pack_nibbles(make_uint4((fv.x >> 4) & kLo, (fv.y >> 4) & kLo,
                                                  (fv.z >> 4) & kLo, (fv.w >> 4) & kLo));
      {
        uint32_t tot;
        const uint32_t ex = block_exclusive_sum<NT>(
            static_cast<uint32_t>(__builtin_popcountll(G)) |
                (static_cast<uint32_t>(__builtin_popcountll(Eq)) << 16),
            wsum, tot);  // its barriers also order the bitmap reads before the staging
        const uint32_t kq = ku - (tot & 0xffffu);  // equal values taken, lowest positions first
        int32_t* out = a.idx + row * static_cast<int64_t>(k);
        const bool staged = k <= kIdxStage;
        int32_t* so = reinterpret_cast<int32_t*>(lds);
        uint32_t gb = ex & 0xffffu, eb = ex >> 16;
        if ((tot >> 16) <= kq) {
          // Every equal value is taken (the usual case): an entry's slot is its
          // rank among the selected ones.
          uint32_t slot = gb + eb;
  #pragma unroll
          for (int h = 0; h < 2; ++h) {
            for (uint32_t m = static_cast<uint32_t>((G | Eq) >> (32 * h)); m != 0u; m &= m - 1u) {
              const int32_t pos = 64 * tid + 32 * h + static_cast<int32_t>(__builtin_ctz(m));
              if (staged) so[slot] = pos;
              else out[slot] = pos;
              ++slot;
            }
          }
        } else {
          for (uint64_t m = G | Eq; m != 0u; m &= m - 1u) {
            const int bp = static_cast<int>(__builtin_ctzll(m));
            const int32_t pos = 64 * tid + bp;
            int32_t slot = -1;
            if ((G >> bp) & 1u) {
              slot = static_cast<int32_t>(gb + (eb < kq ? eb : kq));
              ++gb;
            } else {
              if (eb < kq) slot = static_cast<int32_t>(gb + eb);
              ++eb;
            }
            if (slot >= 0) {
              if (staged) so[slot] = pos;
              else out[slot] = pos;
            }
          }
        }
        if (staged) {
          block_sync_lds();
          // 16-byte stores when the row allows them; streamed past the caches
          // (the index rows are not re-read by this kernel)
          typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
          if ((k & 3) == 0 && (reinterpret_cast<uintptr_t>(a.idx) & 15u) == 0u) {
            const i32x4* s4 = reinterpret_cast<const i32x4*>(so);
            i32x4* o4 = reinterpret_cast<i32x4*>(out);
            for (int i = tid; i < k / 4; i += NT) __builtin_nontemporal_store(s4[i], o4 + i);
          } else {
            for (int i = tid; i < k; i += NT) out[i] = so[i];
          }
        }
      }
    }
    if (!FLAGS && a.mask != nullptr) {
      block_sync_lds();  // wave 0's threshold in rsh
      emit_mask_row<NT>(a, row, nv - 1, rsh[0]);
    }
    return;
  }
  uint32_t krem;
  const uint32_t tk = stream_select<NT, true>(src, nvalid, k, lds, wsum, info, krem);
  if (tid == 0) a.thr[row] = key_to_float(tk);
  if (!IDX && a.mask != nullptr) emit_mask_row<NT>(a, row, nv - 1, key_to_float(tk));
  if constexpr (IDX) {
    const int64_t nchunks = (nvalid + 4 * NT - 1) / (4 * NT);
    emit_indices<NT>(a.idx + row * static_cast<int64_t>(k), nchunks, tk, krem, wsum,
                     [&](int64_t j, uint32_t(&kk)[4]) {
                       load_keys4<true>(src, (j * NT + tid) * 4, nvalid, kk);
                     });
  }
}

// ---------------------------------------------------------------------------
// Wave kernel: thresholds of rows up to 64*V entries, one wave per row.
// ---------------------------------------------------------------------------
// The row is held in registers (V values per lane, float4 loads issued
// before the first use); no block barrier is involved, so a CU holds many
// rows at once.  The k-th largest is found from the row's finite min and max
// (DPP), a 256-bin LDS histogram linear in value between them, counted from
// the top (+inf and NaN in the first bin, -inf in the last), a prefix scan
// for the bin holding rank k, then that bin's few values gathered and ranked
// against each other by key (NaN largest, -0 == +0).  A bin of more than 64
// values (heavy ties) takes 8-bit radix passes over its keys instead.  Bins
// only steer the search: ranking by key makes the result exact for any
// input.  The kernel is bound by instruction issue more than by HBM, so each
// value costs one min/max, one fma + med3 + convert for its bin (kept, 8 bits
// each, for the gather) and one LDS add (config 2 standalone: 222 -> 177 us,
// 60 -> 75% of HBM peak).
template <int V>
__global__ __launch_bounds__(256, V <= 16 ? 8 : (V <= 32 ? 6 : 4)) void topk_wave_kernel(
    SelectArgs a) {
  static_assert(V % 4 == 0 && V >= 4 && V <= 64, "values per lane");
  constexpr int NCH = V / 4;  // float4 chunks per lane; chunk j covers 256 entries
  __shared__ __align__(16) uint32_t whist[4][256];
  __shared__ uint32_t wgl[4][kWave];
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t rid = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  if (rid >= a.rows) return;  // no block-level synchronisation below
  int64_t row, nvalid;
  if (a.causal_T > 0) {  // longest rows first
    int64_t q, r;
    causal_div(rid, a.nbatch, q, r);
    const int64_t t = a.causal_T - 1 - q;
    row = r * a.causal_T + t;
    nvalid = t + 1;
  } else {
    row = rid;
    nvalid = a.n;
  }
  const int k = a.k;
  if (nvalid < k) {
    if (lane == 0) a.thr[row] = -__builtin_huge_valf();
    return;
  }
  uint32_t* hist = whist[wid];
  uint32_t* gl = wgl[wid];
  const int nv = static_cast<int>(nvalid);  // <= 64*V
  const int nch = (nv + 4 * kWave - 1) / (4 * kWave);  // chunks holding valid entries
  float v[V];
  {
    const char* rb = reinterpret_cast<const char*>(a.scores + row * a.ld);
    const int last4 = (nv - 1) & ~3;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const uint32_t off = static_cast<uint32_t>(min((j * kWave + lane) * 4, last4)) * 4u;
      const float4 f = *reinterpret_cast<const float4*>(rb + off);
      v[4 * j] = f.x;
      v[4 * j + 1] = f.y;
      v[4 * j + 2] = f.z;
      v[4 * j + 3] = f.w;
    }
  }
  // f(x, i) for every valid entry (i: its register index).
  auto visit = [&](auto&& f) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j < nch) {
        if ((j + 1) * 4 * kWave <= nv) {
#pragma unroll
          for (int c = 0; c < 4; ++c) f(v[4 * j + c], 4 * j + c);
        } else {
          const int p0 = (j * kWave + lane) * 4;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (p0 + c < nv) f(v[4 * j + c], 4 * j + c);
        }
      }
    }
  };
  // The bin of `hist` (256 bins, 4 per lane) holding the want-th largest
  // counted entry: its index, the rank inside it and its count (uniform).
  auto pick = [&](uint32_t want, uint32_t& bin, uint32_t& rank, uint32_t& cnt) {
    const uint4 h4 = reinterpret_cast<const uint4*>(hist)[lane];
    const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
    const uint32_t local = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = wave_inclusive_sum(local);
    const uint32_t abv = wave_read_lane(incl, kWave - 1) - incl;  // in higher lanes' bins
    const bool here = abv < want && abv + local >= want;
    bin = rank = cnt = 0;
    if (here) {
      uint32_t cum = abv;
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (cnt == 0u && cum + h[i] >= want) {
          bin = 4u * lane + i;
          rank = want - cum;
          cnt = h[i];
        }
        cum += h[i];
      }
    }
    const int src = __ffsll(static_cast<unsigned long long>(ballot(here))) - 1;
    bin = wave_read_lane(bin, src);
    rank = wave_read_lane(rank, src);
    cnt = wave_read_lane(cnt, src);
  };
  // As pick, for bins counted from the top (bin 0 holds the largest values).
  auto pick_top = [&](uint32_t want, uint32_t& bin, uint32_t& rank, uint32_t& cnt) {
    const uint4 h4 = reinterpret_cast<const uint4*>(hist)[lane];
    const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
    const uint32_t local = h[0] + h[1] + h[2] + h[3];
    const uint32_t abv = wave_inclusive_sum(local) - local;  // in lower lanes' bins
    const bool here = abv < want && abv + local >= want;
    bin = rank = cnt = 0;
    if (here) {
      uint32_t cum = abv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (cnt == 0u && cum + h[i] >= want) {
          bin = 4u * lane + i;
          rank = want - cum;
          cnt = h[i];
        }
        cum += h[i];
      }
    }
    const int src = __ffsll(static_cast<unsigned long long>(ballot(here))) - 1;
    bin = wave_read_lane(bin, src);
    rank = wave_read_lane(rank, src);
    cnt = wave_read_lane(cnt, src);
  };
  // The row's min and max (fminf / fmaxf ignore NaN); a row holding an
  // infinite value (wave-uniform, rare) takes its finite range instead.
  float lo = __builtin_huge_valf(), hi = -__builtin_huge_valf();
  visit([&](float x, int) {
    lo = fminf(lo, x);
    hi = fmaxf(hi, x);
  });
  lo = wave_extreme_f32<false>(lo);
  hi = wave_extreme_f32<true>(hi);
  if (!(lo > -__builtin_huge_valf()) || !(hi < __builtin_huge_valf())) {
    lo = __builtin_huge_valf();
    hi = -__builtin_huge_valf();
    visit([&](float x, int) {
      const bool fin = fabsf(x) <= __FLT_MAX__;
      lo = fminf(lo, fin ? x : __builtin_huge_valf());
      hi = fmaxf(hi, fin ? x : -__builtin_huge_valf());
    });
    lo = wave_extreme_f32<false>(lo);
    hi = wave_extreme_f32<true>(hi);
  }
  // 256 bins linear in value, counted from the top: c = med3((hi - x)*scale,
  // 0, 255), the product and difference in one rounding (fma), is monotone
  // (decreasing) in key order with no test for special values -- +inf lands
  // in c = 0, and so does NaN (med3 with a NaN operand returns the minimum of
  // the other two, and every NaN is the largest key); -inf in c = 255.  A
  // degenerate range (one finite value, none, or a span that overflows)
  // keeps scale = 1: the values then crowd the end bins, which only costs
  // the heavy-tie path below.  Each value's bin is kept, four per register,
  // for the gather.
  float scale = 256.0f / (hi - lo);
  if (!(hi > lo) || !(scale > 0.0f && scale <= __FLT_MAX__)) {
    scale = 1.0f;
    if (!(fabsf(hi) <= __FLT_MAX__)) hi = 0.0f;
  }
  const float hoff = hi * scale;
  auto bin_of = [&](float x) -> uint32_t {
    return static_cast<uint32_t>(__builtin_amdgcn_fmed3f(__builtin_fmaf(x, -scale, hoff), 0.0f, 255.0f));
  };
  reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
  wave_lds_sync();
  uint32_t bp[V / 4];
#pragma unroll
  for (int i = 0; i < V / 4; ++i) bp[i] = 0u;
  visit([&](float x, int i) {
    const uint32_t c = bin_of(x);
    atomicAdd(&hist[c], 1u);
    bp[i >> 2] |= c << (8 * (i & 3));
  });
  wave_lds_sync();
  uint32_t bsel, brank, bcnt;
  pick_top(static_cast<uint32_t>(k), bsel, brank, bcnt);
  uint32_t tk;
  if (bcnt <= static_cast<uint32_t>(kWave)) {
    // The chosen bin's values (a few, usually), as keys, compacted into the
    // wave's list; register slots where no lane matches cost one compare.
    uint32_t ng = 0;
    visit([&](float x, int i) {
      const bool in = ((bp[i >> 2] >> (8 * (i & 3))) & 255u) == bsel;
      const uint64_t m = ballot(in);
      if (m != 0u) {
        if (in) gl[ng + lanes_below(m)] = float_to_key(x);
        ng += popc64(m);
      }
    });
    wave_lds_sync();
    const uint32_t mk = lane < static_cast<int>(bcnt) ? gl[lane] : 0u;
    uint32_t gt = 0, ge = 0;
    for (uint32_t j = 0; j < bcnt; ++j) {
      const uint32_t o = wave_read_lane(mk, static_cast<int>(j));  // lane j's key, no LDS read
      gt += (o > mk) ? 1u : 0u;
      ge += (o >= mk) ? 1u : 0u;
    }
    const bool hit = lane < static_cast<int>(bcnt) && gt < brank && ge >= brank;
    tk = wave_read_lane(mk, __ffsll(static_cast<unsigned long long>(ballot(hit))) - 1);
  } else {
    // Heavy ties.  Often every value of the chosen bin is the same (the
    // exact zeros of a score row whose weights are all negative, say): that
    // value is then the k-th largest, and the bin's least and greatest keys,
    // from the registers, show it without touching memory.
    uint32_t kmin = ~0u, kmax = 0u;
    visit([&](float x, int i) {
      if (((bp[i >> 2] >> (8 * (i & 3))) & 255u) == bsel) {
        const uint32_t key = float_to_key(x);
        kmin = min(kmin, key);
        kmax = max(kmax, key);
      }
    });
    kmin = wave_extreme_u32<false>(kmin);
    kmax = wave_extreme_u32<true>(kmax);
    if (kmin == kmax) {
      tk = kmin;
    } else {
      // Otherwise 8-bit radix passes over the keys of the chosen bin's
      // entries, tracked as a per-lane bit mask of entry slots.  Rows of up
      // to 16 values per lane keep their values in registers for them (a
      // launch of short rows ends with its slowest row, and a pass that
      // re-reads memory costs an L2 round trip: config 1's select 10.3 ->
      // 7.3 us); longer rows re-read the row (from L2: it was just read), so
      // this rare path costs the common one no registers.
      const char* rb = reinterpret_cast<const char*>(a.scores + row * a.ld);
      const int last4 = (nv - 1) & ~3;
      auto reload = [&](auto&& f) {  // f(key, slot) for every valid entry
        if constexpr (V <= 16) {
          visit(f);
          return;
        }
        for (int j = 0; j < nch; ++j) {
          const int p0 = (j * kWave + lane) * 4;
          const uint32_t off = static_cast<uint32_t>(min(p0, last4)) * 4u;
          const float4 q4 = *reinterpret_cast<const float4*>(rb + off);
          const float xs[4] = {q4.x, q4.y, q4.z, q4.w};
  #pragma unroll
          for (int c = 0; c < 4; ++c)
            if (p0 + c < nv) f(xs[c], 4 * j + c);
        }
      };
      uint64_t cm = 0;
      reload([&](float x, int i) {
        if (bin_of(x) == bsel) cm |= uint64_t{1} << i;
      });
      uint32_t prefix = 0, kr = brank, cnt = 0;
      int sh = 24;
      for (; sh >= 0; sh -= 8) {
        wave_lds_sync();  // previous reads of hist done
        reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
        wave_lds_sync();
        reload([&](float x, int i) {
          if ((cm >> i) & 1u) atomicAdd(&hist[(float_to_key(x) >> sh) & 255u], 1u);
        });
        wave_lds_sync();
        uint32_t d, knew;
        pick(kr, d, knew, cnt);
        reload([&](float x, int i) {
          if (((float_to_key(x) >> sh) & 255u) != d) cm &= ~(uint64_t{1} << i);
        });
        prefix = (prefix << 8) | d;
        kr = knew;
        if (cnt == 1u) break;
      }
      if (cnt == 1u && sh > 0) {  // one candidate left: its full key
        uint32_t mine = 0;
        reload([&](float x, int i) {
          if ((cm >> i) & 1u) mine = float_to_key(x);
        });
        tk = wave_read_lane(mine, __ffsll(static_cast<unsigned long long>(ballot(cm != 0u))) - 1);
      } else {
        tk = prefix;
      }
    }
  }
  if (lane == 0) a.thr[row] = key_to_float(tk);
}

template <int V>
hipError_t launch_wave(const SelectArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  hipLaunchKernelGGL((topk_wave_kernel<V>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int NT, int V, int P1>
hipError_t launch_reg(const SelectArgs& a, bool vec, hipStream_t stream) {
  // Causal rows: a 2-D grid (batch element, row) whose blocks need no
  // division to find their row (register rows are at most 32768 long, so
  // causal_T fits the grid's y range).
  const int64_t nb = a.nbatch;
  const bool two_d = a.causal_T > 1 && a.causal_T <= 65535 && nb <= 0x7fffffff;
  const dim3 grid = two_d ? dim3(static_cast<unsigned>(nb), static_cast<unsigned>(a.causal_T))
                          : dim3(static_cast<unsigned>(a.rows));
  if (vec)
    hipLaunchKernelGGL((topk_reg_kernel<NT, V, P1, true>), grid, dim3(NT), 0, stream, a);
  else
    hipLaunchKernelGGL((topk_reg_kernel<NT, V, P1, false>), grid, dim3(NT), 0, stream, a);
  return hipGetLastError();
}

// The bracket kernel pays off when the keys it keeps fit LDS with room to
// spare: expected kept keys at the longest row, (2*delta + 1) sample ranks
// scaled by n/m, at most half of kCandCap.
constexpr int64_t kBracketIdxMaxN = 16 * 4 * 256;

bool bracket_fits(int64_t cap, int k) {
  if (cap <= 4096 || cap > (int64_t{1} << 20)) return false;
  const double frac = 4096.0 / static_cast<double>(cap);
  const double e = static_cast<double>(k) * frac;
  const double delta = 5.0 * std::sqrt(e * (1.0 - frac)) + 2.0;
  return (2.0 * delta + 1.0) / frac <= 0.5 * kCandCap;
}

hipError_t launch_bracket(const SelectArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.rows));
  if (a.idx != nullptr)
    hipLaunchKernelGGL((topk_bracket_kernel<256, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((topk_bracket_kernel<256, false>), grid, dim3(256), 0, stream, a);
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
  SelectArgs a{scores, rows, n, ld, k, causal_T, thr, idx, causal_T > 0 ? rows / causal_T : 0};
  const int64_t cap = causal_T > 0 ? (causal_T < n ? causal_T : n) : n;
  // float4 loads stay inside [0, n) of every row only when n, ld and the base
  // are all 16-byte granular.
  const bool vec = (n % 4 == 0) && (ld % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(scores) & 15u) == 0);
  // Rows above 8K entries use a 12-bit first digit: hot digits of real
  // score rows spread over twice the bins (fewer same-address LDS atomics)
  // and the chosen digit leaves half the candidates.
  // Rows above 4K entries: one pass over HBM (bracket kernel);
  // threshold-only rows up to 2K entries: one wave per row, the row in registers (config 2
  // standalone: 284 -> 177 us; at 4K entries, 64 registers of row per lane
  // leave 4 waves per SIMD and the block kernel is faster: 43 vs 45 us).
  // With indices: rows of at most 16 chunks (the per-thread position masks
  // are 64 bits).
  if (vec && bracket_fits(cap, k) && (idx == nullptr || cap <= kBracketIdxMaxN))
    return launch_bracket(a, stream);
  if (idx == nullptr && vec && cap <= 2048) {
    if (cap <= 512) return launch_wave<8>(a, stream);
    if (cap <= 1024) return launch_wave<16>(a, stream);
    return launch_wave<32>(a, stream);
  }
  if (cap <= 512) return launch_reg<128, 4, 11>(a, vec, stream);
  if (cap <= 1024) return launch_reg<128, 8, 11>(a, vec, stream);
  if (cap <= 2048) return launch_reg<256, 8, 11>(a, vec, stream);
  if (cap <= 4096) return launch_reg<256, 16, 11>(a, vec, stream);
  if (cap <= 8192) return launch_reg<512, 16, 11>(a, vec, stream);
  if (cap <= 16384) return launch_reg<512, 32, 12>(a, vec, stream);
  if (cap <= 32768) return launch_reg<1024, 32, 12>(a, vec, stream);
  return launch_stream(a, vec, stream);
}

hipError_t launch_topk_mask(const float* scores, int64_t B, int64_t T, int64_t ld, int k,
                            float* thr, uint64_t* mask, int64_t ldm, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const int64_t rows = B * T;
  const bool vec = (T % 4 == 0) && (ld % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(scores) & 15u) == 0);
  if (vec && bracket_fits(T, k)) {
    // The rows the bracket kernel would select anyway: it writes each row's
    // bitmask words as soon as it has the threshold (config 4: the mask
    // kernel's second 537 MB read of the scores goes).  Rows of up to 16
    // chunks take the words from the flag bitmap the index output uses (no
    // second read of the row at all); longer rows re-read it.
    SelectArgs a{scores, rows, T, ld, k, T, thr, nullptr, B};
    a.mask = mask;
    a.ldm = ldm;
    if (T <= kBracketIdxMaxN)
      hipLaunchKernelGGL((topk_bracket_kernel<256, false, true>), dim3(static_cast<unsigned>(rows)),
                         dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((topk_bracket_kernel<256, false>), dim3(static_cast<unsigned>(rows)),
                         dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  const hipError_t e = launch_topk(scores, rows, T, ld, k, T, thr, nullptr, stream);
  if (e != hipSuccess) return e;
  return launch_selection_mask(scores, ld, thr, B, T, mask, ldm, stream);
}

}  // namespace dsa
