// tile_attn.hip -- threshold-masked attention on MFMA tiles, for long rows (gfx950).
//
// Same result as sparse_attn.hip (reference dsa_attention.py:234-324):
//   sel(t,s) = s <= t && scores[t,s] >= thr[t]
//   O[t,h,:] = sum_{s in sel} softmax_s(<Q[t,h],K[s,h]> * scale) V[s,h,:]
// but computed densely over the causal triangle with the selection applied
// as a mask.  When each query selects a large share of a long row (config 4:
// k = 2048 of up to 16384 keys, every 64x64 tile holds selected pairs), the
// per-query gather re-reads 16 MB of K/V rows per query from L2/MALL; here a
// block of 128 queries shares every K/V tile it loads, and both products run
// on MFMA.
//
// Block = 4 waves = 128 consecutive queries of one (batch element, head);
// wave w owns queries t0+32w .. t0+32w+31 (two 16-query MFMA column tiles).
// Key tiles of 64 keys are staged in LDS (K as [key][d], V transposed as
// [d][key]), double-buffered with one barrier per tile.
//
// The products are computed transposed, so that no lane exchanges are needed
// between them (16x16x32 MFMA: A[m][k] lane l holds m = l%16, k-slots
// 8(l/16)..+7; B[k][n] lane l holds n = l%16, the same k-slots; D[m][n] lane
// l holds n = l%16, m = 4(l/16)+r):
//   S^T = K . Q^T   A = K rows (LDS), B = Q^T (registers, loaded once)
//                   -> lane l: query l%16, keys 4(l/16)+r of each 16-key tile
//   softmax state (running max m, normaliser l) is per query = per lane
//   O^T = V^T . P^T A = V^T rows (LDS), B = P^T straight from the S^T
//                   registers: the 8 k-slots of lane group g are keys
//                   {4g..4g+3} of key tile 2j and of key tile 2j+1; V^T reads
//                   use the same key order
//                   -> lane l: query l%16, dims 4(l/16)+r of each 16-dim tile
// P is rounded to the input's 16-bit type for the second product (the
// reference multiplies fp32 probabilities; the difference is far inside the
// 16-bit tolerance); everything else is fp32.  Rows that select nothing get
// 0/0 = NaN, as the reference.
#include "dsa_device.h"
#include "dsa_launch.h"

namespace dsa {
namespace {

constexpr int kTQ = 128;  // queries per block
constexpr int kKT = 64;   // keys per LDS tile
constexpr int kNT = 256;  // threads per block

struct TileArgs {
  const float* scores;
  int64_t ld;
  const float* thr;
  const void* Q;
  const void* K;
  const void* V;
  int64_t B;
  int T;
  int HQ;
  float scale_log2;
  float* out;
  int vec;  // score rows 16-byte aligned with ld % 4 == 0: float4 loads
};

template <typename Tag>
struct Mfma16x16x32;

template <>
struct Mfma16x16x32<BF16> {
  static __device__ __forceinline__ f32x4 run(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {  // one v_cvt_pk_bf16_f32
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
  }
};

template <>
struct Mfma16x16x32<F16> {
  static __device__ __forceinline__ f32x4 run(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
  }
};

template <typename Tag, int D>
__global__ __launch_bounds__(kNT, 2) void tile_attn_kernel(TileArgs a) {
  static_assert(D % 32 == 0 && D <= 128, "head dim");
  using M = Mfma16x16x32<Tag>;
  constexpr int KS = D + 8;        // K tile row stride (elements): +16 B keeps b128 reads conflict-free
  constexpr int VS = kKT + 4;      // V^T tile row stride (elements): +8 B likewise for b64 reads
  constexpr int KTILE = kKT * KS;  // elements per K tile
  constexpr int VTILE = D * VS;    // elements per V^T tile
  constexpr int NKS = D / 32;      // k-steps of the first product
  constexpr int NDT = D / 16;      // 16-dim output tiles
  constexpr int PPR = D / 8;       // 16-byte pieces per K/V row
  constexpr int KCH = kKT * PPR / kNT;        // K pieces per thread per tile
  constexpr int VCH = (kKT / 2) * PPR / kNT;  // V piece pairs per thread per tile
  static_assert(KCH >= 1 && VCH >= 1, "tile staging");
  __shared__ __align__(16) uint16_t lds[2 * (KTILE + VTILE)];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = lane_id();
  const int g = lane >> 4, c16 = lane & 15;
  const int T = a.T;
  const int HQ = a.HQ;

  // Block -> (tile, batch, head): tiles longest first, then batch, head fastest.
  const int ntile = (T + kTQ - 1) / kTQ;
  const int64_t per_tile = a.B * HQ;
  const int tile = ntile - 1 - static_cast<int>(blockIdx.x / per_tile);
  const int64_t bh = blockIdx.x % per_tile;
  const int64_t b = bh / HQ;
  const int h = static_cast<int>(bh % HQ);
  const int t0 = tile * kTQ;
  const int tw = t0 + 32 * wave;  // first query of this wave

  const int64_t rowE = static_cast<int64_t>(HQ) * D;  // elements per Q/K/V row
  const uint16_t* Qb = static_cast<const uint16_t*>(a.Q) + b * T * rowE + static_cast<int64_t>(h) * D;
  const uint16_t* Kb = static_cast<const uint16_t*>(a.K) + b * T * rowE + static_cast<int64_t>(h) * D;
  const uint16_t* Vb = static_cast<const uint16_t*>(a.V) + b * T * rowE + static_cast<int64_t>(h) * D;

  // Q^T fragments: qf[qt][ks] = Q[query tw+16qt+c16][dims 32ks+8g .. +8].
  uint4 qf[2][NKS];
  int tq[2];
  float thr[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    tq[qt] = tw + 16 * qt + c16;
    const int tl = min(tq[qt], T - 1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qf[qt][ks] = *reinterpret_cast<const uint4*>(Qb + tl * rowE + 32 * ks + 8 * g);
    thr[qt] = a.thr[b * T + tl];
  }
  const float* srow[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) srow[qt] = a.scores + (b * T + min(tq[qt], T - 1)) * a.ld;

  float m[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};
  float l[2] = {0.f, 0.f};
  f32x4 o[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) o[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int s_hi = min(T, t0 + kTQ);          // keys [0, s_hi) can be causal in this block
  const int nkt = (s_hi + kKT - 1) / kKT;
  const int wave_last = min(tw + 31, T - 1);  // last query of this wave

  // Global -> registers (prefetch) -> LDS staging of key tile kt.  Rows past
  // T are clamped to T-1: they are never causal for any query.
  u32x4 kreg[KCH];  // native vectors: a uint4 struct array here stays in scratch memory
  u32x4 vreg[VCH][2];
  auto gload = [&](int kt) {
    const int s0 = kt * kKT;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + kNT * i;
      const int s = min(s0 + c / PPR, T - 1);
      kreg[i] = *reinterpret_cast<const u32x4*>(Kb + s * rowE + 8 * (c % PPR));
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int c = tid + kNT * i;
      const int s = s0 + 2 * (c / PPR);
      vreg[i][0] = *reinterpret_cast<const u32x4*>(Vb + min(s, T - 1) * rowE + 8 * (c % PPR));
      vreg[i][1] = *reinterpret_cast<const u32x4*>(Vb + min(s + 1, T - 1) * rowE + 8 * (c % PPR));
    }
  };
  auto swrite = [&](int buf) {
    uint16_t* kl = lds + buf * (KTILE + VTILE);
    uint16_t* vl = kl + KTILE;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + kNT * i;
      *reinterpret_cast<u32x4*>(kl + (c / PPR) * KS + 8 * (c % PPR)) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int c = tid + kNT * i;
      const int kp = c / PPR, d0 = 8 * (c % PPR);
      const u32x4 w0 = vreg[i][0], w1 = vreg[i][1];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t lo = (w0[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        const uint32_t hi = (w1[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        *reinterpret_cast<uint32_t*>(vl + (d0 + e) * VS + 2 * kp) = lo | (hi << 16);
      }
    }
  };

  gload(0);
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    swrite(buf);
    block_sync_lds();
    gload(min(kt + 1, nkt - 1));  // unconditional: keeps the prefetch registers out of memory
    const int s0 = kt * kKT;
    if (s0 > wave_last) continue;  // the whole tile is above this wave's diagonal

    // Selection of this wave's 32 x 64 tile, as a per-entry bias word:
    // 0.0f where (query tq[qt], key s0 + 16j + 4g + r) is selected, all-ones
    // (a NaN) where not.  st + bias is st or NaN, which fmaxf skips, and
    // v_bfi(bias, -inf, st) is st or -inf: both exact for any st, NaN and
    // +-inf logits of unselected keys included (the reference masks them to
    // -inf before its softmax).
    const bool inner = (s0 + kKT - 1 <= tw) && (tw + 31 < T);  // no causal or row-end test
    uint32_t bias[2][4][4];
    bool any = false;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = s0 + 16 * j + 4 * g;
        const float* sp = srow[qt] + s;
        float v4[4];
        if (inner) {
          if (a.vec) {
            const float4 f = *reinterpret_cast<const float4*>(sp);
            v4[0] = f.x; v4[1] = f.y; v4[2] = f.z; v4[3] = f.w;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) v4[r] = sp[r];
          }
        } else {
          // entries past the query (or past T) are never read: they may lie past the row
#pragma unroll
          for (int r = 0; r < 4; ++r) v4[r] = (s + r <= tq[qt] && tq[qt] < T) ? sp[r] : -__builtin_nanf("");
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool on = v4[r] >= thr[qt];  // NaN scores and NaN thresholds select nothing
          bias[qt][j][r] = on ? 0u : 0xffffffffu;
          any |= on;
        }
      }
    }
    if (__ballot(any) == 0) continue;  // nothing selected in this wave's tile

    const uint16_t* kl = lds + buf * (KTILE + VTILE);
    const uint16_t* vl = kl + KTILE;

    // S^T = K . Q^T
    f32x4 st[4][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) st[j][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const uint4 ka = *reinterpret_cast<const uint4*>(kl + (16 * j + c16) * KS + 32 * ks + 8 * g);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) st[j][qt] = M::run(ka, qf[qt][ks], st[j][qt]);
      }
    }

    // Online softmax per query, log2 domain.  The running max moves only
    // when a tile's max exceeds it by more than 2^8 (probabilities stay
    // <= 256, far from overflow in fp32 and exact in scale for 16-bit), so
    // the O rescale is skipped on almost every tile.
    uint4 pf[2][2];
    bool grow = false;
    float alpha[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[j][qt][r] + __uint_as_float(bias[qt][j][r]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float m_blk = mx * a.scale_log2;
      const bool up = m_blk > m[qt] + 8.f;
      const float m_new = up ? m_blk : m[qt];
      alpha[qt] = up ? exp2f(m[qt] - m_new) : 1.f;   // m = -inf: alpha = 0 on an empty O
      grow |= up && (m[qt] != -__builtin_huge_valf());
      m[qt] = m_new;
      const float m_use = (m_new == -__builtin_huge_valf()) ? 0.f : m_new;
      float p[4][4];
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = __uint_as_float((bias[qt][j][r] & 0xff800000u) |
                                          (~bias[qt][j][r] & __float_as_uint(st[j][qt][r])));
          p[j][r] = __builtin_amdgcn_exp2f(fmaf(x, a.scale_log2, -m_use));  // bare v_exp_f32
          ps += p[j][r];
        }
      l[qt] = fmaf(l[qt], alpha[qt], ps);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        pf[qt][jj] = make_uint4(M::pack(p[2 * jj][0], p[2 * jj][1]), M::pack(p[2 * jj][2], p[2 * jj][3]),
                                M::pack(p[2 * jj + 1][0], p[2 * jj + 1][1]),
                                M::pack(p[2 * jj + 1][2], p[2 * jj + 1][3]));
    }
    if (__ballot(grow) != 0) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[dt][qt][r] *= alpha[qt];
    }

    // O^T += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint16_t* vr = vl + (16 * dt + c16) * VS + 32 * jj + 4 * g;
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
        const uint4 va = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[dt][qt] = M::run(va, pf[qt][jj], o[dt][qt]);
      }
    }
  }

  // O = O^T / l, lane l: query tq[qt], dims 16dt + 4g .. +3.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float lt = l[qt];
    lt += __shfl_xor(lt, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    const float inv = 1.f / lt;  // lt == 0 only if nothing passed: NaN, as the reference
    if (tq[qt] < T) {
      float* orow = a.out + ((b * T + tq[qt]) * HQ + h) * static_cast<int64_t>(D);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 v = o[dt][qt];
        *reinterpret_cast<float4*>(orow + 16 * dt + 4 * g) =
            make_float4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
      }
    }
  }
}

template <typename Tag, int D>
hipError_t launch(const TileArgs& a, hipStream_t stream) {
  const int64_t nblk = a.B * a.HQ * ((a.T + kTQ - 1) / kTQ);
  hipLaunchKernelGGL((tile_attn_kernel<Tag, D>), dim3(static_cast<unsigned>(nblk)), dim3(kNT), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

bool tile_attn_supported(int dtype, int HQ, int DQ, int DV, const void* Q, const void* K,
                         const void* V) {
  if (dtype != 1 && dtype != 2) return false;
  if (DQ != DV || (DQ != 64 && DQ != 128)) return false;
  if (HQ < 1) return false;
  for (const void* p : {Q, K, V})
    if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0) return false;
  return true;
}

hipError_t launch_tile_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                            const void* K, const void* V, int dtype, int64_t B, int64_t T, int HQ,
                            int D, float scale, float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const bool vec = (ld % 4 == 0) && ((reinterpret_cast<uintptr_t>(scores) & 15u) == 0);
  TileArgs a{scores, ld, thr, Q, K, V, B, static_cast<int>(T), HQ,
             scale * 1.4426950408889634f, out, vec ? 1 : 0};
  if (dtype == 1) {
    if (D == 64) return launch<BF16, 64>(a, stream);
    if (D == 128) return launch<BF16, 128>(a, stream);
  } else if (dtype == 2) {
    if (D == 64) return launch<F16, 64>(a, stream);
    if (D == 128) return launch<F16, 128>(a, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace dsa
