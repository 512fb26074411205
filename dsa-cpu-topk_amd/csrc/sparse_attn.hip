// sparse_attn.hip -- threshold-driven sparse attention (gfx950).
//
// Replaces _sparse_attn_kernel + sparse_attention_with_threshold_triton
// (reference dsa_attention.py:234-324) and is the last stage of the split
// forward and of the precomputed-threshold path (dsa_hybrid.py:66).  The
// reference loads every K/V row of the prefix and masks; this kernel reads
// only the score row and the selected K/V rows (attn_tile.h; fp32 rows of
// 128 elements two keys per wave load, attend_query_pair).
//
// Block = 4 waves = 4 consecutive queries of one batch element.  Blocks run
// longest query first, spread evenly over the XCDs (causal_block_tile).
// Rows wider than one wave's registers hold (more than 16 fp32 or 32 16-bit
// elements per lane) are split into head chunks: each block then takes one
// chunk of its 4 queries' heads, and the chunks of a tile are adjacent
// blocks (they read the same score rows, one after another, from L2).
//
// For long rows (T >= kTiledMinT) with 16-bit inputs and DQ = DV in {64,
// 128}, launch_sparse_attn hands over to the dense-masked MFMA tile kernel
// (tile_attn.hip): there every query selects a large share of a long row and
// per-query gathers would re-read the same K/V rows thousands of times.
#include "attn_tile.h"
#include "dsa_launch.h"

namespace dsa {
namespace {

struct AttnArgs {
  const float* scores;
  int64_t ld;
  const float* thr;
  const void* Q;
  const void* K;
  const void* V;
  int64_t B;
  int T;
  int HQ, DQ, DV;
  float scale_log2;
  float* out;
  int vec;
  int HQc;     // heads per chunk
  int nchunk;  // HQ / HQc
};

// PAIR: fp32 rows of 128 elements gathered two keys per wave load
// (attend_query_pair); the host takes it for whole rows (no head chunks)
// with DQ % 4 == 0 and Q, K, V and out 16-byte aligned.
template <typename Tag, int EK, int EV, bool PAIR = false>
__global__ __launch_bounds__(256) void sparse_attn_kernel(AttnArgs a) {
  static_assert(!PAIR || (std::is_same_v<Tag, F32> && EK == 2 && EV == 2), "rows of 128 fp32");
  using raw = typename Tag::raw;
  __shared__ __align__(16) int lists[4][kListCap];
  const int wave = threadIdx.x >> 6;
  const int T = a.T;
  const int tiles = (T + 3) >> 2;
  const int chunk = static_cast<int>(blockIdx.x % static_cast<uint32_t>(a.nchunk));
  int64_t b;
  int tile;
  causal_block_tile(blockIdx.x / static_cast<uint32_t>(a.nchunk), a.B, tiles, b, tile);
  const int t = tile * 4 + wave;
  if (t >= T) return;
  const int64_t EQ = static_cast<int64_t>(a.HQ) * a.DQ;
  const int64_t EVt = static_cast<int64_t>(a.HQ) * a.DV;
  const int64_t cq = static_cast<int64_t>(chunk) * a.HQc * a.DQ;  // chunk's first element
  const int64_t cv = static_cast<int64_t>(chunk) * a.HQc * a.DV;
  const raw* Q = static_cast<const raw*>(a.Q) + b * T * EQ + cq;
  const raw* K = static_cast<const raw*>(a.K) + b * T * EQ + cq;
  const raw* V = static_cast<const raw*>(a.V) + b * T * EVt + cv;
  const int64_t qrow = b * T + t;
  const float* srow = a.scores + qrow * a.ld;
  const float thr = a.thr[qrow];
  const bool vec = a.vec != 0;
  auto load4 = [&](int s, float(&sv)[4]) {
    if (vec) {
      const float4 f = *reinterpret_cast<const float4*>(srow + s);
      sv[0] = f.x; sv[1] = f.y; sv[2] = f.z; sv[3] = f.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) sv[c] = (s + c <= t) ? srow[s + c] : 0.f;
    }
  };
  if constexpr (PAIR)
    attend_query_pair(Q, K, V, t, a.DQ, a.scale_log2, thr, load4, lists[wave],
                      a.out + qrow * EVt);
  else
    attend_query<Tag, EK, EV>(Q, K, V, t, a.HQc, a.DQ, a.DV, a.scale_log2, thr, load4, lists[wave],
                              a.out + qrow * EVt + cv, nullptr, static_cast<int>(EQ),
                              static_cast<int>(EVt));
}

template <typename Tag, int EK, int EV, bool PAIR = false>
hipError_t launch(const AttnArgs& a, hipStream_t stream) {
  const int64_t nblk = a.B * ((a.T + 3) / 4) * a.nchunk;
  hipLaunchKernelGGL((sparse_attn_kernel<Tag, EK, EV, PAIR>), dim3(static_cast<unsigned>(nblk)),
                     dim3(256), 0, stream, a);
  return hipGetLastError();
}

// (EK, EV) pairs with an instance: equal, or one a factor 2 from the other.
#define DSA_ATTN_PAIRS(X, Tag) \
  X(Tag, 1, 1) X(Tag, 1, 2) X(Tag, 2, 1) X(Tag, 2, 2) X(Tag, 2, 4) X(Tag, 4, 2) X(Tag, 4, 4) \
  X(Tag, 4, 8) X(Tag, 8, 4) X(Tag, 8, 8) X(Tag, 8, 16) X(Tag, 16, 8) X(Tag, 16, 16)
#define DSA_ATTN_PAIRS16(X, Tag) \
  DSA_ATTN_PAIRS(X, Tag) X(Tag, 16, 32) X(Tag, 32, 16) X(Tag, 32, 32)

#define DSA_ATTN_CASE(Tag, ek, ev) \
  if (EK == ek && EV == ev) return launch<Tag, ek, ev>(a, stream);
#define DSA_ATTN_HAS(Tag, ek, ev) \
  if (EK == ek && EV == ev) return true;

int elems_per_lane(int HQ, int D) {
  const int e = HQ * D / kWave;
  return e < 1 ? 1 : e;
}

bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Largest slice a lane holds: 16 fp32 or 32 16-bit elements (64 bytes).
int max_elems(int dtype) { return dtype == 0 ? 16 : 32; }

// Head chunks a row is split into so that a chunk's K and V rows fit one
// wave at <= max_elems per lane (1 when the whole row fits).
int head_chunks(int dtype, int HQ, int DQ, int DV) {
  const int64_t width = static_cast<int64_t>(HQ) * (DQ > DV ? DQ : DV);
  const int64_t cap = static_cast<int64_t>(kWave) * max_elems(dtype);
  int n = 1;
  while (width / n > cap && n < HQ) n *= 2;
  return n;
}

}  // namespace

bool sparse_attn_chunked(int dtype, int HQ, int DQ, int DV) {
  return head_chunks(dtype, HQ, DQ, DV) > 1;
}

bool sparse_attn_supported(int dtype, int HQ, int DQ, int DV) {
  if (!pow2(HQ) || !pow2(DQ) || !pow2(DV)) return false;
  const int HQc = HQ / head_chunks(dtype, HQ, DQ, DV);
  const int EK = elems_per_lane(HQc, DQ), EV = elems_per_lane(HQc, DV);
  if (EK > max_elems(dtype) || EV > max_elems(dtype)) return false;
  if (EK > DQ || EV > DV) return false;  // a lane's slice must stay inside one head
  if (dtype == 0) {
    DSA_ATTN_PAIRS(DSA_ATTN_HAS, F32)
  } else if (dtype == 1 || dtype == 2) {
    DSA_ATTN_PAIRS16(DSA_ATTN_HAS, BF16)
  }
  return false;
}

bool sparse_attn_uses_tiles(int dtype, int64_t T, int HQ, int DQ, int DV) {
  if ((dtype != 1 && dtype != 2) || DQ != DV || (DQ != 64 && DQ != 128) || HQ < 1) return false;
  return T >= kTiledMinT || head_chunks(dtype, HQ, DQ, DV) > 1;
}

hipError_t launch_sparse_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, int DV, float scale, float* out, void* ws,
                              int64_t ws_bytes, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  // Dense-masked tiles for long rows, and for rows whose gathers would need
  // head chunks (each chunk re-reads the score row and the list).
  if (sparse_attn_uses_tiles(dtype, T, HQ, DQ, DV) && ld <= kTileMaxLd &&
      tile_attn_supported(dtype, HQ, DQ, DV, Q, K, V))
    return launch_tile_attn(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, scale, out, stream);
  // Long rows whose K/V rows a wave holds in one slice: each block streams
  // its causal keys once through LDS instead of gathering per query.
  const int64_t need = sparse_attn_workspace_bytes(false, dtype, B, T, HQ, DQ, DV, ld);
  const bool split = need > 0 && ws != nullptr && ws_bytes >= need &&
                     (reinterpret_cast<uintptr_t>(ws) & 15u) == 0;
  if (staged_attn_auto(dtype, B, T, HQ, DQ, DV, split) && staged_attn_fits(T, ld))
    return launch_staged_attn(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, scale, out, ws,
                              ws_bytes, stream);
  return launch_sparse_attn_gather(scores, ld, thr, Q, K, V, dtype, B, T, HQ, DQ, DV, scale,
                                   out, stream);
}

int64_t sparse_attn_workspace_bytes(bool staged, int dtype, int64_t B, int64_t T, int HQ, int DQ,
                                    int DV, int64_t ld) {
  if (B <= 0 || T <= 0 || !staged_attn_supported(dtype, HQ, DQ, DV) || !staged_attn_fits(T, ld))
    return 0;
  if (!staged && (sparse_attn_uses_tiles(dtype, T, HQ, DQ, DV) ||
                  !staged_attn_auto(dtype, B, T, HQ, DQ, DV, true)))
    return 0;
  return staged_attn_plan(B, T, HQ, DQ, true).ws_bytes;
}

hipError_t launch_sparse_attn_gather(const float* scores, int64_t ld, const float* thr,
                                     const void* Q, const void* K, const void* V, int dtype,
                                     int64_t B, int64_t T, int HQ, int DQ, int DV, float scale,
                                     float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const int nchunk = head_chunks(dtype, HQ, DQ, DV);
  const int HQc = HQ / nchunk;
  const bool vec = (ld % 4 == 0) && ((reinterpret_cast<uintptr_t>(scores) & 15u) == 0);
  AttnArgs a{scores, ld, thr, Q, K, V, B, static_cast<int>(T), HQ, DQ, DV,
             scale * 1.4426950408889634f, out, vec ? 1 : 0, HQc, nchunk};
  const int EK = elems_per_lane(HQc, DQ), EV = elems_per_lane(HQc, DV);
  // Two keys per gather instruction for whole fp32 rows of 128 elements.
  if (dtype == 0 && nchunk == 1 && HQ * DQ == 128 && DQ == DV && DQ % 4 == 0 &&
      ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) |
        reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0)
    return launch<F32, 2, 2, true>(a, stream);
  if (dtype == 0) {
    DSA_ATTN_PAIRS(DSA_ATTN_CASE, F32)
  } else if (dtype == 1) {
    DSA_ATTN_PAIRS16(DSA_ATTN_CASE, BF16)
  } else if (dtype == 2) {
    DSA_ATTN_PAIRS16(DSA_ATTN_CASE, F16)
  }
  return hipErrorInvalidValue;
}

}  // namespace dsa
