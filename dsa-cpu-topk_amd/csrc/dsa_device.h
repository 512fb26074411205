// dsa_device.h -- device helpers shared by the gfx950 DSA kernels.
//
// Wave64 primitives, the order-preserving float -> uint32 radix key, MFMA
// operand types, and typed loads.  Written for CDNA4 (gfx950) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Storage tags for the three input element types.  Arithmetic is fp32 always.
struct F32 { using raw = float; static constexpr int kBytes = 4; };
struct BF16 { using raw = uint16_t; static constexpr int kBytes = 2; };
struct F16 { using raw = uint16_t; static constexpr int kBytes = 2; };
// OCP FP8 E4M3 (torch.float8_e4m3fn), gfx950's native fp8: the indexer's
// q/k only (products on the fp8 MFMA, weights and sums fp32).
struct FP8 { using raw = uint8_t; static constexpr int kBytes = 1; };

__device__ __forceinline__ float to_f32(F32, float x) { return x; }
__device__ __forceinline__ float to_f32(BF16, uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
__device__ __forceinline__ float to_f32(F16, uint16_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, x));
}

// ---------------------------------------------------------------------------
// Radix keys.  Unsigned order of the key equals the numeric order of the
// float, with -0.0 folded onto +0.0 (IEEE '>=' treats them as equal, and the
// reference selects with '>=': dsa_attention.py:46) and every NaN folded onto
// one positive quiet NaN that ranks above +inf (torch.topk's NaN order).
// -inf maps to 0x007FFFFF, the smallest key a float can produce; key 0 is
// therefore free and marks "no element" (padding, masked positions).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t float_to_key(float f) {
  f = f + 0.0f;  // IEEE: -0.0 + 0.0 = +0.0; every other value (and NaN-ness) unchanged
  uint32_t u = __float_as_uint(f);
  u = (f != f) ? 0x7fc00000u : u;
  // negative: flip every bit; non-negative: set the sign bit
  return u ^ (static_cast<uint32_t>(static_cast<int32_t>(u) >> 31) | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
constexpr uint32_t kKeyNone = 0u;

// ---------------------------------------------------------------------------
// Wave64 primitives.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Orders this wave's LDS traffic: everything issued before is visible to every
// lane of the wave after.  (A wave's LDS instructions complete in order; the
// fence makes the compiler wait for them and not move accesses across.)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// DPP lane move within the wave (no LDS traffic).  Lanes whose source falls
// outside the pattern, or whose row is masked off, read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes (32-bit integer types): four
// row_shr steps scan each 16-lane row, then row_bcast:15 and row_bcast:31
// carry row totals into the rows above.
template <typename T>
__device__ __forceinline__ T wave_inclusive_sum(T x) {
  static_assert(sizeof(T) == 4, "32-bit lanes");
  uint32_t v = static_cast<uint32_t>(x);
  v += dpp_u32<0x111>(v);        // row_shr:1
  v += dpp_u32<0x112>(v);        // row_shr:2
  v += dpp_u32<0x114>(v);        // row_shr:4
  v += dpp_u32<0x118>(v);        // row_shr:8
  v += dpp_u32<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_u32<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
  return static_cast<T>(v);
}

// Maximum and minimum of a float over the 64 lanes by the scan's DPP steps
// (a lane with no source keeps its own value); the result is read from lane
// 63.  NaN inputs are the caller's to exclude.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_keep_f32(float v) {
  const int b = __float_as_int(v);
  return __int_as_float(__builtin_amdgcn_update_dpp(b, b, CTRL, ROW_MASK, 0xf, false));
}
template <bool MAX>
__device__ __forceinline__ float wave_extreme_f32(float v) {
  auto op = [](float x, float y) { return MAX ? fmaxf(x, y) : fminf(x, y); };
  v = op(v, dpp_keep_f32<0x111>(v));
  v = op(v, dpp_keep_f32<0x112>(v));
  v = op(v, dpp_keep_f32<0x114>(v));
  v = op(v, dpp_keep_f32<0x118>(v));
  v = op(v, dpp_keep_f32<0x142, 0xa>(v));
  v = op(v, dpp_keep_f32<0x143, 0xc>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// The same for unsigned integers (the wave's least or greatest key).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_keep_u32(uint32_t v) {
  const int b = static_cast<int>(v);
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(b, b, CTRL, ROW_MASK, 0xf, false));
}
template <bool MAX>
__device__ __forceinline__ uint32_t wave_extreme_u32(uint32_t v) {
  auto op = [](uint32_t x, uint32_t y) { return MAX ? max(x, y) : min(x, y); };
  v = op(v, dpp_keep_u32<0x111>(v));
  v = op(v, dpp_keep_u32<0x112>(v));
  v = op(v, dpp_keep_u32<0x114>(v));
  v = op(v, dpp_keep_u32<0x118>(v));
  v = op(v, dpp_keep_u32<0x142, 0xa>(v));
  v = op(v, dpp_keep_u32<0x143, 0xc>(v));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// DPP lane moves of a float inside 16-lane rows (VALU, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// A partner lane for butterfly step W (1, 2, 4 or 8): its bit log2(W)
// differs from this lane's and its bits above, within the 16-lane row, are
// the same (mirrors, so the bits below differ too: steps whose data layout
// depends only on bits already combined do not care).
template <int W>
__device__ __forceinline__ float dpp_partner(float v) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8, "step inside a row");
  if constexpr (W == 8) return dpp_f32<0x140>(v);       // row_mirror: i <-> 15-i
  else if constexpr (W == 4) return dpp_f32<0x141>(v);  // row_half_mirror: i <-> 7-i
  else if constexpr (W == 2) return dpp_f32<0x1B>(v);   // quad_perm [3,2,1,0]
  else return dpp_f32<0xB1>(v);                          // quad_perm [1,0,3,2]
}
// Lane u of this lane's aligned group of G lanes (G in 2, 4, 8, 16).
template <int G, int U>
__device__ __forceinline__ float group_bcast(float v) {
  static_assert(U >= 0 && U < G, "lane inside the group");
  if constexpr (G == 16) {
    return dpp_f32<0x150 + U>(v);  // row_newbcast:U
  } else if constexpr (G == 8) {
    const float lo = dpp_f32<0x150 + U>(v), hi = dpp_f32<0x158 + U>(v);
    return (lane_id() & 8) ? hi : lo;
  } else if constexpr (G == 4) {
    return dpp_f32<U | (U << 2) | (U << 4) | (U << 6)>(v);  // quad_perm [U,U,U,U]
  } else {
    return dpp_f32<U | (U << 2) | ((U + 2) << 4) | ((U + 2) << 6)>(v);  // [U,U,U+2,U+2]
  }
}

// Max / sum of v over the lane pairs {l, l^32} and {l, l^16}, on the VALU
// (v_permlane32_swap / v_permlane16_swap of v with itself: the two results
// hold, for every lane l, v[l & ~M] and v[l | M], M = 32 or 16).
// max(x, 0) on the bit pattern: a float with the sign bit set is a negative
// int32.  One integer max instead of the canonicalising float max the
// compiler emits for fmaxf on values it cannot prove canonical (MFMA
// results); -0.0 maps to +0.0, a NaN with the sign bit clear stays NaN.
__device__ __forceinline__ float relu_f32(float x) {
  return __int_as_float(max(__float_as_int(x), 0));
}

__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Value of lane `src` (uniform) broadcast to the wave.
template <typename T>
__device__ __forceinline__ T wave_read_lane(T x, int src) {
  static_assert(sizeof(T) == 4, "32-bit lanes");
  return static_cast<T>(__builtin_amdgcn_readlane(static_cast<int>(x), src));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Bin of v among top + 1 bins linear in value: (v - lo) * scale clamped to
// [0, top].  For finite lo and scale >= 0 it is monotone non-decreasing in v
// (each rounding step is monotone, then a clamp and a truncation), and -0
// and +0 share a bin.
__device__ __forceinline__ int value_bin(float v, float lo, float scale, float top) {
  return static_cast<int>(__builtin_amdgcn_fmed3f((v - lo) * scale, 0.0f, top));
}

// Lanes whose predicate holds, as a 64-bit mask (the compare's own lane mask;
// HIP's __ballot takes an int and re-materialises it).
__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

__device__ __forceinline__ uint32_t popc64(uint64_t m) {
  return static_cast<uint32_t>(__popcll(m));
}
// Number of set bits of m below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

// Workgroup barrier that orders LDS traffic only.  __syncthreads() also
// fences global memory, which makes every wave drain its outstanding global
// loads at the barrier; kernels whose threads exchange data through LDS alone
// use this one so that prefetched loads stay in flight across it.
__device__ __forceinline__ void block_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block-wide exclusive prefix sum in thread order (NT threads, NT % 64 == 0).
// wsum must hold NT/64 words of LDS.  Contains two LDS-only barriers.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_sum(uint32_t v, uint32_t* wsum,
                                                        uint32_t& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const uint32_t incl = wave_inclusive_sum(v);
  if (lane == kWave - 1) wsum[wid] = incl;
  block_sync_lds();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) {
    const uint32_t s = wsum[w];
    base += (w < wid) ? s : 0u;
    tot += s;
  }
  block_sync_lds();
  total = tot;
  return base + incl - v;
}

// ---------------------------------------------------------------------------
// Typed vector loads: N consecutive elements starting at p (N*bytes a multiple
// of 16 and p 16-byte aligned when vec is true) converted to fp32.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&out)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const float4 v = *reinterpret_cast<const float4*>(p + i);
      out[i] = v.x; out[i + 1] = v.y; out[i + 2] = v.z; out[i + 3] = v.w;
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      const float2 v = *reinterpret_cast<const float2*>(p + i);
      out[i] = v.x; out[i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = p[i];
  }
}

template <typename Tag, int N>
__device__ __forceinline__ void load_cvt(const typename Tag::raw* __restrict__ p, float (&out)[N]) {
  if constexpr (Tag::kBytes == 4) {
    load_f32<N>(reinterpret_cast<const float*>(p), out);
  } else {
    if constexpr (N % 8 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(p + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          out[i + 2 * j] = to_f32(Tag{}, static_cast<uint16_t>(w[j] & 0xffffu));
          out[i + 2 * j + 1] = to_f32(Tag{}, static_cast<uint16_t>(w[j] >> 16));
        }
      }
    } else if constexpr (N % 2 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 2) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(p + i);
        out[i] = to_f32(Tag{}, static_cast<uint16_t>(w & 0xffffu));
        out[i + 1] = to_f32(Tag{}, static_cast<uint16_t>(w >> 16));
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) out[i] = to_f32(Tag{}, p[i]);
    }
  }
}

// Buffer resource over rows s1 .. T-1 of a [T, rowbytes] array (`base` is
// row 0).  Its size ends at row T, so buffer reads at or past row T are
// range-checked by the hardware and return zeros without touching memory;
// with s1 >= T every read does.  Word 3 is the raw-buffer configuration of
// CDNA (untyped dword access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const char* base, int64_t s1, int64_t T,
                                                           uint32_t rowbytes) {
  const uint64_t rem = s1 >= T ? 0ull : static_cast<uint64_t>(T - s1) * rowbytes;
  const int nrec = rem > 0xffffffffull ? -1 : static_cast<int>(static_cast<uint32_t>(rem));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base + s1 * rowbytes), 0, nrec,
                                           0x00020000);
}

// Block order for causal work whose cost grows with the query tile.
// Workgroups are dispatched in index order, round-robin over the 8 XCDs
// (block i starts on XCD i % 8).  Index order here is: tiles longest first,
// batch element fastest.  So every XCD receives the same mix of long and
// short tiles (a contiguous tile range per XCD would leave the XCD holding
// the last rows of a causal triangle with up to 2x the average work), and
// when B is a multiple of 8 each XCD receives B/8 whole batch elements, whose
// K/V rows then stay in that XCD's L2.
__device__ __forceinline__ void causal_block_tile(uint32_t bid, int64_t B, int ntile,
                                                  int64_t& b, int& tile) {
  b = static_cast<int64_t>(bid) % B;
  tile = ntile - 1 - static_cast<int>(static_cast<int64_t>(bid) / B);
}

}  // namespace dsa
