// fused.hip -- whole DSA forward in one kernel for T <= 2048 (gfx950).
//
// Replaces _dsa_fused_kernel + dsa_attention_triton (reference
// dsa_attention.py:96-227).  Per wave, for its 4 queries:
//   1. lightning indexer on MFMA over keys [0, t0+4)  -> score rows in LDS
//   2. per row, radix-select the k_eff-th largest (wave_select.h)
//   3. per row, sparse attention over keys with score >= thr (attn_tile.h)
// The score rows never touch HBM.  The 4 waves of a block hold 16
// consecutive queries and share nothing but L1, so there is no block barrier;
// blocks run longest queries first, spread evenly over the XCDs
// (causal_block_tile).
//
// LDS per block: 16 score rows of RS floats, RS = round_up(T,32) + 16 (the
// +16 puts consecutive rows on different banks for the MFMA epilogue
// stores), plus a 256-bin histogram and a 512-entry key list per wave.
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
};

int row_stride(int T) { return ((T + 31) / 32) * 32 + 16; }
size_t fused_lds_bytes(int T) {
  return static_cast<size_t>(16) * row_stride(T) * 4 + 4 * 256 * 4 + 4 * kListCap * 4;
}

template <typename Tag, int DI, int KB, int EK, int EV>
__global__ __launch_bounds__(256) void fused_kernel(FusedArgs a) {
  using raw = typename Tag::raw;
  extern __shared__ __align__(16) float smem[];
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int g = lane >> 4, r16 = lane & 15;
  const int T = a.T;
  const int RS = a.RS;
  const int tiles = (T + 15) >> 4;
  int64_t b;
  int tile;
  causal_block_tile(blockIdx.x, a.B, tiles, b, tile);
  const int t0 = tile * 16 + wave * 4;
  if (t0 >= T) return;

  float* rows = smem + wave * 4 * RS;
  uint32_t* hist = reinterpret_cast<uint32_t*>(smem + 16 * RS) + wave * 256;
  int* list = reinterpret_cast<int*>(smem + 16 * RS + 4 * 256) + wave * kListCap;

  const raw* qi = static_cast<const raw*>(a.qi) + b * T * static_cast<int64_t>(a.HI) * DI;
  const raw* ki = static_cast<const raw*>(a.ki) + b * T * static_cast<int64_t>(DI);
  const raw* wi = static_cast<const raw*>(a.wi) + b * T * static_cast<int64_t>(a.HI);

  // 1. indexer rows t0..t0+3 over keys [0, min(T, t0+4)).
  const int s_end = (t0 + 4 < T) ? t0 + 4 : T;
  indexer_rows<Tag, DI, KB>(qi, ki, wi, T, a.HI, t0, 0, s_end, [&](int s0, const float(&sc)[KB]) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int s = s0 + 16 * kb + r16;
      if (s < T) rows[g * RS + s] = sc[kb];
    }
  });
  wave_lds_sync();

  const int64_t EQ = static_cast<int64_t>(a.HQ) * a.DQ;
  const int64_t EVt = static_cast<int64_t>(a.HQ) * a.DV;
  const raw* Q = static_cast<const raw*>(a.Q) + b * T * EQ;
  const raw* K = static_cast<const raw*>(a.K) + b * T * EQ;
  const raw* V = static_cast<const raw*>(a.V) + b * T * EVt;

  for (int r = 0; r < 4; ++r) {
    const int t = t0 + r;
    if (t >= T) break;
    const float* row = rows + r * RS;
    // 2. threshold: k_eff-th largest of the full row, whose s > t entries
    //    are -inf (dsa_attention.py:41-44).
    const int n = t + 1;
    const float thr = (n < a.keff) ? -__builtin_huge_valf() : wave_select_kth(row, n, a.keff, hist);
    // 3. attention over keys with score >= thr.
    attend_query<Tag, EK, EV>(
        Q, K, V, t, a.HQ, a.DQ, a.DV, a.scale_log2, thr,
        [&](int s, float(&sv)[4]) {
          const float4 f = *reinterpret_cast<const float4*>(row + s);
          sv[0] = f.x; sv[1] = f.y; sv[2] = f.z; sv[3] = f.w;
        },
        list, a.out + (b * T + t) * EVt);
  }
}

template <typename Tag, int DI, int KB, int EK, int EV>
hipError_t launch(const FusedArgs& a, hipStream_t stream) {
  const size_t lds = fused_lds_bytes(a.T);
  auto kern = fused_kernel<Tag, DI, KB, EK, EV>;
  // Raise the dynamic-LDS limit of this instance once, to what T = 2048 needs.
  // A runtime that does not need (or know) the attribute may refuse it; the
  // launch below then reports any real shortfall itself.
  static const bool attr_set = [&] {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
        static_cast<int>(fused_lds_bytes(static_cast<int>(kFusedMaxT))));
    if (e != hipSuccess) (void)hipGetLastError();
    return e == hipSuccess;
  }();
  (void)attr_set;
  const int64_t nblk = a.B * ((a.T + 15) / 16);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nblk)), dim3(256), lds, stream, a);
  return hipGetLastError();
}

int elems_per_lane(int HQ, int D) {
  const int e = HQ * D / kWave;
  return e < 1 ? 1 : e;
}

#define DSA_FUSED_EK(Tag, di, kb)                                              \
  switch (EK) {                                                                \
    case 1: return launch<Tag, di, kb, 1, 1>(a, stream);                       \
    case 2: return launch<Tag, di, kb, 2, 2>(a, stream);                       \
    case 4: return launch<Tag, di, kb, 4, 4>(a, stream);                       \
    case 8: return launch<Tag, di, kb, 8, 8>(a, stream);                       \
  }                                                                            \
  break;

}  // namespace

hipError_t launch_fused(const void* qi, const void* ki, const void* wi, const void* Q,
                        const void* K, const void* V, int dtype, int64_t B, int64_t T, int HI,
                        int DI, int HQ, int DQ, int DV, int top_k, float scale, float* out,
                        hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const int keff = top_k < T ? top_k : static_cast<int>(T);
  FusedArgs a{qi, ki, wi, Q, K, V, B, static_cast<int>(T), HI, HQ, DQ, DV, keff,
              scale * 1.4426950408889634f, out, row_stride(static_cast<int>(T))};
  const int EK = elems_per_lane(HQ, DQ);
  if (elems_per_lane(HQ, DV) != EK) return hipErrorNotSupported;
  if (dtype == 0) {
    switch (DI) {
      case 16: DSA_FUSED_EK(F32, 16, 4)
      case 32: DSA_FUSED_EK(F32, 32, 4)
      case 64: DSA_FUSED_EK(F32, 64, 4)
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
