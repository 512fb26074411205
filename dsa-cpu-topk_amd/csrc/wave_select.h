// wave_select.h -- k-th largest of one LDS-resident score row, one wave.
//
// Replaces the fused reference kernel's tl.sort(...)[TOP_K-1]
// (dsa_attention.py:151-155): same value (the k-th largest counting ties)
// without sorting.  Four MSD radix passes over 8-bit digits of the
// order-preserving key; each pass is a 256-bin LDS histogram built with
// ds_add by the wave, then a wave suffix-scan over the bins (4 per lane)
// finds the digit holding the k-th key.  A digit that holds a single key ends
// the search early.  The row is re-read from LDS on every pass, so no
// register array scales with T.
#pragma once

#include "dsa_device.h"

namespace dsa {

// row: n (>= k >= 1) valid scores in LDS, 16-byte aligned.  hist: 256 words
// of LDS private to this wave.  Returns the k-th largest value.
__device__ __forceinline__ float wave_select_kth(const float* row, int n, int k,
                                                 uint32_t* hist) {
  const int lane = lane_id();
  uint32_t prefix = 0;
  uint32_t krem = static_cast<uint32_t>(k);
  for (int p = 0; p < 4; ++p) {
    const int shift = 24 - 8 * p;
    reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    for (int s = 4 * lane; s < n; s += 4 * kWave) {
      const float4 f = *reinterpret_cast<const float4*>(row + s);
      const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t kk = float_to_key(fv[c]);
        const bool in = (s + c < n) && (p == 0 || (kk >> (shift + 8)) == prefix);
        if (in) atomicAdd(&hist[(kk >> shift) & 255u], 1u);
      }
    }
    wave_lds_sync();
    const uint4 h4 = reinterpret_cast<const uint4*>(hist)[lane];
    const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
    const uint32_t local = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = wave_inclusive_sum(local);
    const uint32_t total = wave_read_lane(incl, kWave - 1);
    const uint32_t above = total - incl;  // keys in higher lanes' bins
    const bool mine = above < krem && above + local >= krem;
    uint32_t bucket = 0, knew = 0, cnt = 0;
    if (mine) {
      uint32_t cum = above;
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (cnt == 0u && cum + h[i] >= krem) {
          bucket = 4u * lane + i;
          knew = krem - cum;
          cnt = h[i];
        }
        cum += h[i];
      }
    }
    const uint64_t who = __ballot(mine);
    const int src = __ffsll(static_cast<unsigned long long>(who)) - 1;  // uniform
    bucket = wave_read_lane(bucket, src);
    knew = wave_read_lane(knew, src);
    cnt = wave_read_lane(cnt, src);
    prefix = (prefix << 8) | bucket;
    krem = knew;
    wave_lds_sync();  // histogram reads done before the next pass clears it
    if (p < 3 && cnt == 1u) {
      // The digit holds one key; fetch it.
      uint32_t hit = 0;
      for (int s = 4 * lane; s < n; s += 4 * kWave) {
        const float4 f = *reinterpret_cast<const float4*>(row + s);
        const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t kk = float_to_key(fv[c]);
          if ((s + c < n) && (kk >> shift) == prefix) hit = kk;
        }
      }
      const uint64_t m = __ballot(hit != 0u);
      return key_to_float(wave_read_lane(hit, __ffsll(static_cast<unsigned long long>(m)) - 1));
    }
  }
  return key_to_float(prefix);
}

}  // namespace dsa
