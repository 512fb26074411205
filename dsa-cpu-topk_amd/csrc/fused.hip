// fused.hip -- whole DSA forward in one kernel for T <= 2048 (gfx950).
//
// Replaces _dsa_fused_kernel + dsa_attention_triton (reference
// dsa_attention.py:96-227).  A block of 8 waves owns QB = 16 consecutive
// queries (8 when 16-query blocks would leave compute units idle):
//   1. lightning indexer on MFMA: each wave computes the score rows of 8
//      (DI <= 32) or 4 queries over a part of their causal key range, into
//      LDS rows shared by the block;
//   -- one block barrier --
//   2. each wave takes QB/8 rows: the k_eff-th largest by a value-bin
//      histogram (wave_select.h), then sparse attention over keys with
//      score >= thr (attn_tile.h).
// The score rows never touch HBM.  Splitting the indexer's key range over
// several waves and giving each wave one or two rows multiplies the waves
// that hide the gathers' memory latency, at the same MFMA work.  Blocks run
// longest queries first, spread evenly over the XCDs, or, when the grid is
// resident two blocks per CU, one long and one short tile per CU
// (block_tile).
//
// LDS per block: QB score rows of RS floats, RS = round_up(T,32) + 16 (the
// +16 puts consecutive rows on different banks for the MFMA epilogue
// stores), plus a 256-bin histogram and a 512-entry key list per wave, and
// each row's score range (min, max, non-finite flag per key part), which the
// indexer's epilogue gathers so that the select starts at its histogram.
#include "attn_tile.h"
#include "dsa_launch.h"
#include "indexer_tile.h"
#include "wave_select.h"

namespace dsa {
namespace {

struct FusedArgs {
  const void* qi;
  const void* ki;
  const void* wi;
  const void* Q;
  const void* K;
  const void* V;
  int64_t B;
  int T;
  int HI, HQ, DQ, DV;
  int keff;
  float scale_log2;
  float* out;
  int RS;
  int pair_cus;  // > 0: pair long and short tiles on each CU (see block_tile)
};

int row_stride(int T) { return ((T + 31) / 32) * 32 + 16; }

// Block -> (batch element, 16-query tile).  By default longest tiles first
// (causal_block_tile).  When the whole grid is resident with two blocks per
// CU (pair_cus = the CU count, a multiple of B), block i and block
// i + pair_cus share a CU (workgroups go round-robin over the XCDs and then
// over each XCD's CUs): the first pair_cus blocks take the longest tiles in
// descending order and the rest the shortest in ascending order, so every CU
// holds one long and one short tile and the CUs' work evens out.  The batch
// element stays bid % B in both halves, so each XCD keeps its batch
// elements' K/V rows in its L2.
__device__ __forceinline__ void block_tile(uint32_t bid, int64_t B, int tiles, int pair_cus,
                                           int64_t& b, int& tile) {
  if (pair_cus > 0) {
    const uint32_t cus = static_cast<uint32_t>(pair_cus);
    const uint32_t j = bid < cus ? bid : bid - cus;
    b = static_cast<int64_t>(j) % B;
    tile = bid < cus ? tiles - 1 - static_cast<int>(j / B) : static_cast<int>(j / B);
  } else {
    causal_block_tile(bid, B, tiles, b, tile);
  }
}
constexpr int kFusedWaves = 8;
// Per (row, key part): the minimum, maximum and non-finite flag of the
// row's causal scores, gathered by the indexer for the select (rows x parts
// is at most 64).
constexpr int kRangeWords = 64 * 3;
size_t fused_lds_bytes(int T, int QB) {
  return static_cast<size_t>(QB) * row_stride(T) * 4 + kFusedWaves * 256 * 4 +
         kFusedWaves * kListCap * 4 + kRangeWords * 4;
}

// Narrow indexer rows (DI <= 64) ask for 4 waves per SIMD (<= 128 VGPRs): the
// whole grid of a T = 512 problem is then resident at once.
// QB queries per block (16, or 8 when 16-query blocks would leave CUs idle):
// each wave finishes QB/8 rows.
// PAIR: fp32 attention rows of 128 elements gathered two keys per wave load
// (attend_query_pair); the host takes it when DQ % 4 == 0 and Q, K, V and
// out are 16-byte aligned.
template <typename Tag, int DI, int KB, int EK, int EV, int QB, bool PAIR>
__global__ __launch_bounds__(64 * kFusedWaves, DI <= 64 ? 4 : 1) void fused_kernel(FusedArgs a) {
  static_assert(QB == 8 || QB == 16, "8 or 16 queries per block");
  static_assert(!PAIR || (std::is_same_v<Tag, F32> && EK == 2 && EV == 2), "rows of 128 fp32");
  constexpr int RPW = QB / kFusedWaves;  // rows per wave
  using raw = typename Tag::raw;
  extern __shared__ __align__(16) float smem[];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int g = lane >> 4, r16 = lane & 15;
  const int T = a.T;
  const int RS = a.RS;
  const int tiles = (T + QB - 1) / QB;
  int64_t b;
  int tile;
  block_tile(blockIdx.x, a.B, tiles, a.pair_cus, b, tile);

  float* rows = smem;  // QB score rows
  uint32_t* hist = reinterpret_cast<uint32_t*>(smem + QB * RS) + wave * 256;
  int* list = reinterpret_cast<int*>(smem + QB * RS + kFusedWaves * 256) + wave * kListCap;
  float* rng = smem + QB * RS + kFusedWaves * 256 + kFusedWaves * kListCap;

  const raw* qi = static_cast<const raw*>(a.qi) + b * T * static_cast<int64_t>(a.HI) * DI;
  const raw* ki = static_cast<const raw*>(a.ki) + b * T * static_cast<int64_t>(DI);
  const raw* wi = static_cast<const raw*>(a.wi) + b * T * static_cast<int64_t>(a.HI);

  // 1. indexer: the block's QB queries in groups of 4*QGN, each group's
  //    causal key range [0, min(T, tg + 4*QGN)) split into NPART parts of
  //    whole super-blocks; wave w takes group w % NGRP and part w / NGRP.
  //    Narrow rows (DI <= 32, attention slices of <= 4 elements per lane)
  //    take 8-query groups, so every key block a wave loads serves 8
  //    queries; the others keep 4-query groups within 128 VGPRs.
  constexpr int QGN = (DI <= 32 && EK <= 4) ? 2 : 1;  // 4-query groups per wave
  constexpr int NGRP = QB / (4 * QGN);   // query groups per block
  constexpr int NPART = kFusedWaves / NGRP;
  {
    const int grp = wave % NGRP, part = wave / NGRP;
    const int tg = tile * QB + grp * 4 * QGN;
    if (tg < T) {
      constexpr int SB = 16 * KB;
      const int s_end = (tg + 4 * QGN < T) ? tg + 4 * QGN : T;
      const int nsb = (s_end + SB - 1) / SB;
      const int s_lo = ((part * nsb) / NPART) * SB;
      const int s_hi = min(((part + 1) * nsb / NPART) * SB, s_end);
      float lo[QGN], hi[QGN], bad[QGN];
#pragma unroll
      for (int qg = 0; qg < QGN; ++qg) {
        lo[qg] = __builtin_huge_valf();
        hi[qg] = -__builtin_huge_valf();
        bad[qg] = 0.0f;
      }
      auto take = [&](int qg, int s0, const float (&sc)[KB]) {
        float* qrow_p = rows + (grp * 4 * QGN + qg * 4 + g) * RS;
        const int qrow = tg + qg * 4 + g;  // the query of these scores
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int s = s0 + 16 * kb + r16;
          const float v = sc[kb];
          if (s < T) qrow_p[s] = v;
          if (s <= qrow && s < T) {
            lo[qg] = fminf(lo[qg], v);
            hi[qg] = fmaxf(hi[qg], v);
            bad[qg] = fabsf(v) <= __FLT_MAX__ ? bad[qg] : 1.0f;
          }
        }
      };
      if (s_lo < s_hi) {
        if constexpr (QGN == 1) {
          indexer_rows<Tag, DI, KB, 1>(qi, ki, wi, T, a.HI, static_cast<int64_t>(a.HI) * DI, DI,
                                       a.HI, tg, s_lo, s_hi,
                                       [&](int s0, const float(&sc)[KB]) { take(0, s0, sc); });
        } else {
          indexer_rows<Tag, DI, KB, QGN>(qi, ki, wi, T, a.HI, static_cast<int64_t>(a.HI) * DI,
                                         DI, a.HI, tg, s_lo, s_hi,
                                         [&](int s0, const float(&sc)[QGN][KB]) {
#pragma unroll
                                           for (int qg = 0; qg < QGN; ++qg) take(qg, s0, sc[qg]);
                                         });
        }
      }
      // over the 16 lanes that hold each row's keys
#pragma unroll
      for (int qg = 0; qg < QGN; ++qg) {
        lo[qg] = fminf(lo[qg], dpp_partner<8>(lo[qg]));
        lo[qg] = fminf(lo[qg], dpp_partner<4>(lo[qg]));
        lo[qg] = fminf(lo[qg], dpp_partner<2>(lo[qg]));
        lo[qg] = fminf(lo[qg], dpp_partner<1>(lo[qg]));
        hi[qg] = fmaxf(hi[qg], dpp_partner<8>(hi[qg]));
        hi[qg] = fmaxf(hi[qg], dpp_partner<4>(hi[qg]));
        hi[qg] = fmaxf(hi[qg], dpp_partner<2>(hi[qg]));
        hi[qg] = fmaxf(hi[qg], dpp_partner<1>(hi[qg]));
        bad[qg] = fmaxf(bad[qg], dpp_partner<8>(bad[qg]));
        bad[qg] = fmaxf(bad[qg], dpp_partner<4>(bad[qg]));
        bad[qg] = fmaxf(bad[qg], dpp_partner<2>(bad[qg]));
        bad[qg] = fmaxf(bad[qg], dpp_partner<1>(bad[qg]));
        if (r16 == 0) {
          float* slot = rng + ((grp * 4 * QGN + qg * 4 + g) * NPART + part) * 3;
          slot[0] = lo[qg];
          slot[1] = hi[qg];
          slot[2] = bad[qg];
        }
      }
    }
  }
  block_sync_lds();

  const int64_t EQ = static_cast<int64_t>(a.HQ) * a.DQ;
  const int64_t EVt = static_cast<int64_t>(a.HQ) * a.DV;
  const raw* Q = static_cast<const raw*>(a.Q) + b * T * EQ;
  const raw* K = static_cast<const raw*>(a.K) + b * T * EQ;
  const raw* V = static_cast<const raw*>(a.V) + b * T * EVt;

  // 2. rows 2w, 2w+1 of the block.  Both query rows are loaded first, so
  // their latency hides behind the first row's select.
  constexpr int QE = PAIR ? 4 : EK;  // query elements per lane
  float qpre[RPW][QE];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int t = min(tile * QB + RPW * wave + rr, T - 1);
    if constexpr (PAIR) load_query_pair(Q, t, a.scale_log2, qpre[rr]);
    else load_query<Tag, EK>(Q, t, static_cast<int>(EQ), a.scale_log2, qpre[rr]);
  }
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = RPW * wave + rr;
    const int t = tile * QB + r;
    if (t >= T) break;
    const float* row = rows + r * RS;
    // threshold: k_eff-th largest of the full row, whose s > t entries are
    // -inf (dsa_attention.py:41-44).
    const int n = t + 1;
    const float* rq = rng + r * NPART * 3;  // the row's NPART key parts
    float rlo = rq[0], rhi = rq[1], rb = rq[2];
#pragma unroll
    for (int p = 1; p < NPART; ++p) {
      rlo = fminf(rlo, rq[3 * p]);
      rhi = fmaxf(rhi, rq[3 * p + 1]);
      rb = fmaxf(rb, rq[3 * p + 2]);
    }
    const bool rbad = rb != 0.0f;
    const float thr = (n < a.keff) ? -__builtin_huge_valf()
                                   : wave_select_kth_bins(row, n, a.keff, hist,
                                                          reinterpret_cast<uint32_t*>(list),
                                                          rlo, rhi, rbad);
    // attention over keys with score >= thr.
    auto load4 = [&](int s, float(&sv)[4]) {
      const float4 f = *reinterpret_cast<const float4*>(row + s);
      sv[0] = f.x; sv[1] = f.y; sv[2] = f.z; sv[3] = f.w;
    };
    if constexpr (PAIR)
      attend_query_pair(Q, K, V, t, a.DQ, a.scale_log2, thr, load4, list,
                        a.out + (b * T + t) * EVt, qpre[rr]);
    else
      attend_query<Tag, EK, EV, true>(Q, K, V, t, a.HQ, a.DQ, a.DV, a.scale_log2, thr, load4, list,
                                      a.out + (b * T + t) * EVt, qpre[rr]);
  }
}

template <typename Tag, int DI, int KB, int EK, int EV, int QB, bool PAIR>
hipError_t launch(const FusedArgs& a, hipStream_t stream) {
  const size_t lds = fused_lds_bytes(a.T, QB);
  auto kern = fused_kernel<Tag, DI, KB, EK, EV, QB, PAIR>;
  // Raise the dynamic-LDS limit of this instance once, to what T = 2048 needs.
  // A runtime that does not need (or know) the attribute may refuse it; the
  // launch below then reports any real shortfall itself.
  static const bool attr_set = [&] {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
        static_cast<int>(fused_lds_bytes(static_cast<int>(kFusedMaxT), QB)));
    if (e != hipSuccess) (void)hipGetLastError();
    return e == hipSuccess;
  }();
  (void)attr_set;
  const int64_t nblk = a.B * ((a.T + QB - 1) / QB);
  FusedArgs args = a;
  args.pair_cus = 0;
  // Resident blocks per CU of this instance at this LDS size (host query,
  // cached per thread for the last device and size seen).
  const int cus = device_cus();
  thread_local int c_cus = 0, c_per_cu = 0;
  thread_local size_t c_lds = 0;
  if (cus > 0 && (cus != c_cus || lds != c_lds)) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(kern), 64 * kFusedWaves, lds) != hipSuccess) {
      (void)hipGetLastError();  // the default order needs no figure
      per_cu = 0;
    }
    c_cus = cus;
    c_lds = lds;
    c_per_cu = per_cu;
  }
  if (cus > 0 && c_per_cu == 2 && nblk > cus && nblk <= 2 * static_cast<int64_t>(cus) &&
      cus % a.B == 0)
    args.pair_cus = cus;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nblk)), dim3(64 * kFusedWaves), lds, stream,
                     args);
  return hipGetLastError();
}

int elems_per_lane(int HQ, int D) {
  const int e = HQ * D / kWave;
  return e < 1 ? 1 : e;
}

// 16-query blocks unless they would leave compute units idle (fewer blocks
// than CUs): then 8-query blocks, one row per wave, twice the blocks.
// pair: fp32 rows of 128 elements may take attend_query_pair.
template <typename Tag, int DI, int KB, int EK>
hipError_t launch_qb(const FusedArgs& a, bool pair, hipStream_t stream) {
  const int cus = device_cus();
  const bool qb8 = cus > 0 && a.B * ((a.T + 15) / 16) < cus;
  if constexpr (std::is_same_v<Tag, F32> && EK == 2) {
    if (pair) {
      if (qb8) return launch<Tag, DI, KB, EK, EK, 8, true>(a, stream);
      return launch<Tag, DI, KB, EK, EK, 16, true>(a, stream);
    }
  }
  if (qb8) return launch<Tag, DI, KB, EK, EK, 8, false>(a, stream);
  return launch<Tag, DI, KB, EK, EK, 16, false>(a, stream);
}

#define DSA_FUSED_EK(Tag, di, kb)                                              \
  switch (EK) {                                                                \
    case 1: return launch_qb<Tag, di, kb, 1>(a, pair, stream);                 \
    case 2: return launch_qb<Tag, di, kb, 2>(a, pair, stream);                 \
    case 4: return launch_qb<Tag, di, kb, 4>(a, pair, stream);                 \
    case 8: return launch_qb<Tag, di, kb, 8>(a, pair, stream);                 \
  }                                                                            \
  break;

}  // namespace

// Compute units of the current device (cached per thread), 0 if unknown.
int device_cus() {
  thread_local int c_dev = -1, c_cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (dev != c_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    c_dev = dev;
    c_cus = cus;
  }
  return c_cus;
}

hipError_t launch_fused(const void* qi, const void* ki, const void* wi, const void* Q,
                        const void* K, const void* V, int dtype, int64_t B, int64_t T, int HI,
                        int DI, int HQ, int DQ, int DV, int top_k, float scale, float* out,
                        hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const int keff = top_k < T ? top_k : static_cast<int>(T);
  FusedArgs a{qi, ki, wi, Q, K, V, B, static_cast<int>(T), HI, HQ, DQ, DV, keff,
              scale * 1.4426950408889634f, out, row_stride(static_cast<int>(T)), 0};
  const int EK = elems_per_lane(HQ, DQ);
  if (elems_per_lane(HQ, DV) != EK) return hipErrorNotSupported;
  // Two keys per gather instruction for fp32 rows of 128 elements.
  const bool pair = dtype == 0 && HQ * DQ == 128 && DQ == DV && DQ % 4 == 0 &&
                    ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) |
                      reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  // Key blocks per indexer super-block (KB): fp32 rows take 2 (config 1:
  // 34.0 us against 35.1 at 4 and 34.4 at 1), DI = 64 takes 1 to stay within
  // 128 VGPRs without scratch.
  if (dtype == 0) {
    switch (DI) {
      case 16: DSA_FUSED_EK(F32, 16, 2)
      case 32: DSA_FUSED_EK(F32, 32, 2)
      case 64: DSA_FUSED_EK(F32, 64, 1)
      case 128: DSA_FUSED_EK(F32, 128, 2)
    }
  } else if (dtype == 1) {
    switch (DI) {
      case 32: DSA_FUSED_EK(BF16, 32, 4)
      case 64: DSA_FUSED_EK(BF16, 64, 4)
      case 128: DSA_FUSED_EK(BF16, 128, 4)
    }
  }
  return hipErrorNotSupported;
}

}  // namespace dsa
