// indexer.hip -- standalone lightning-indexer scores [B,T,T] fp32 (gfx950 MFMA).
//
// Replaces _indexer_score_kernel + indexer_scores_triton
// (reference lightning_indexer.py:54-125).  Same output: causal scores, -inf
// above the diagonal (written only on request -- the public drop-in asks for
// it because callers check it, the internal split pipeline does not).
//
// Grid: x = (batch, 16-query tile), y = 256-key chunk.  Each of the 4 waves
// owns 4 queries of the tile and walks the chunk in super-blocks of 16*KB
// keys (indexer_tile.h).  Chunks wholly above the diagonal do no MFMA work;
// they only write -inf when asked, which is what the reference's kernel
// computes for those tiles anyway (lightning_indexer.py:92-94).
#include "dsa_launch.h"
#include "indexer_tile.h"

namespace dsa {
namespace {

constexpr int kChunk = 256;

struct IndexerArgs {
  const void* q;
  const void* k;
  const void* w;
  int64_t B;
  int T;
  int HI;
  float* scores;
  int64_t ld;
  int write_upper;
};

template <typename Tag, int DI, int KB>
__global__ __launch_bounds__(256) void indexer_kernel(IndexerArgs a) {
  static_assert(kChunk % (16 * KB) == 0, "chunk is whole super-blocks");
  using raw = typename Tag::raw;
  const int T = a.T;
  const int ntile = (T + 15) >> 4;
  const int64_t b = blockIdx.x / ntile;
  const int tile = blockIdx.x % ntile;
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int g = lane >> 4, r16 = lane & 15;
  const int t0 = tile * 16 + wave * 4;
  if (t0 >= T) return;  // no block-level synchronisation below
  const int c0 = blockIdx.y * kChunk;
  const int c1 = (c0 + kChunk < T) ? c0 + kChunk : T;

  const raw* q = static_cast<const raw*>(a.q) + b * T * static_cast<int64_t>(a.HI) * DI;
  const raw* k = static_cast<const raw*>(a.k) + b * T * static_cast<int64_t>(DI);
  const raw* w = static_cast<const raw*>(a.w) + b * T * static_cast<int64_t>(a.HI);
  float* out = a.scores + (b * T) * a.ld;
  const float ninf = -__builtin_huge_valf();
  const int tq = t0 + g;  // this lane's output query

  // Keys this wave must compute: [c0, min(c1, t0 + 4)).
  const int s_end = (t0 + 4 < c1) ? t0 + 4 : c1;
  int done_end = c0;
  if (s_end > c0) {
    indexer_rows<Tag, DI, KB>(q, k, w, T, a.HI, t0, c0, s_end, [&](int s0, const float(&sc)[KB]) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int s = s0 + 16 * kb + r16;
        if (tq < T && s < c1 && (s <= tq || a.write_upper))
          out[static_cast<int64_t>(tq) * a.ld + s] = (s <= tq) ? sc[kb] : ninf;
      }
    });
    const int span = s_end - c0;
    done_end = c0 + ((span + 16 * KB - 1) / (16 * KB)) * (16 * KB);
  }
  if (a.write_upper && tq < T) {
    for (int s = done_end + r16; s < c1; s += 16) out[static_cast<int64_t>(tq) * a.ld + s] = ninf;
  }
}

template <typename Tag, int DI, int KB>
hipError_t launch(const IndexerArgs& a, hipStream_t stream) {
  const int ntile = (a.T + 15) / 16;
  const dim3 grid(static_cast<unsigned>(a.B * ntile), static_cast<unsigned>((a.T + kChunk - 1) / kChunk));
  hipLaunchKernelGGL((indexer_kernel<Tag, DI, KB>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename Tag>
hipError_t dispatch_di(const IndexerArgs& a, int DI, hipStream_t stream) {
  if constexpr (Tag::kBytes == 4) {
    switch (DI) {
      case 16: return launch<Tag, 16, 4>(a, stream);
      case 32: return launch<Tag, 32, 4>(a, stream);
      case 64: return launch<Tag, 64, 4>(a, stream);
      case 128: return launch<Tag, 128, 2>(a, stream);
      case 256: return launch<Tag, 256, 1>(a, stream);
    }
  } else {
    switch (DI) {
      case 32: return launch<Tag, 32, 4>(a, stream);
      case 64: return launch<Tag, 64, 4>(a, stream);
      case 128: return launch<Tag, 128, 4>(a, stream);
      case 256: return launch<Tag, 256, 2>(a, stream);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool indexer_supported(int dtype, int DI) {
  if (dtype == 0) return DI == 16 || DI == 32 || DI == 64 || DI == 128 || DI == 256;
  if (dtype == 1 || dtype == 2) return DI == 32 || DI == 64 || DI == 128 || DI == 256;
  return false;
}

hipError_t launch_indexer(const void* q, const void* k, const void* w, int dtype, int64_t B,
                          int64_t T, int HI, int DI, float* scores, int64_t ld,
                          int write_upper, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  IndexerArgs a{q, k, w, B, static_cast<int>(T), HI, scores, ld, write_upper};
  switch (dtype) {
    case 0: return dispatch_di<F32>(a, DI, stream);
    case 1: return dispatch_di<BF16>(a, DI, stream);
    case 2: return dispatch_di<F16>(a, DI, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace dsa
