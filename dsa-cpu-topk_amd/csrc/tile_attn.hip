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
// Key tiles of 64 keys are copied HBM -> LDS by the DMA path
// (global_load_lds_dwordx4: no registers, no LDS store instructions), K and
// V both as plain [key][d] rows, double-buffered with one barrier per tile.
// Rows are stored with their 16-byte chunks XOR-swizzled by row so that
// every LDS read pattern below hits distinct banks.
//
// The products are computed transposed, so that no lane exchanges are needed
// between them (16x16x32 MFMA: A[m][k] lane l holds m = l%16, k-slots
// 8(l/16)..+7; B[k][n] lane l holds n = l%16, the same k-slots; D[m][n] lane
// l holds n = l%16, m = 4(l/16)+r):
//   S^T = K . Q^T   A = K rows (LDS), B = Q^T (registers, loaded once)
//                   -> lane l: query l%16, keys 4(l/16)+r of each 16-key tile
//   softmax state (running max m, normaliser l) is per query = per lane
//   O^T = V^T . P^T A = V^T (from the [key][d] V rows by the transposing
//                   LDS read ds_read_b64_tr_b16: within each 16-lane group,
//                   lane i's element s is element i%4 of the 8 bytes lane
//                   4s+i/4 addressed, so lanes addressing rows key0+4g+j/4,
//                   dims 16dt+4(j%4) receive d = 16dt+i, keys key0+4g+s),
//                   B = P^T straight from the S^T registers: the 8 k-slots of
//                   lane group g are keys {4g..4g+3} of key tile 2j and of
//                   key tile 2j+1
//                   -> lane l: query l%16, dims 4(l/16)+r of each 16-dim tile
// P is rounded to the input's 16-bit type for the second product and for
// the softmax normaliser, which is one more MFMA per fragment (ones . P^T),
// so numerator and denominator sum the same probabilities (the reference
// uses fp32 probabilities; the difference is far inside the 16-bit
// tolerance); everything else is fp32.  Rows that select nothing get
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
  int vec;  // score rows 16-byte aligned with ld % 4 == 0: float4 loads (ld >= 4 then)
};

template <typename Tag>
struct Mfma16x16x32;

template <>
struct Mfma16x16x32<BF16> {
  static __device__ __forceinline__ f32x4 run(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static constexpr uint32_t kOnes = 0x3f803f80u;  // two bf16 1.0
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {  // one v_cvt_pk_bf16_f32
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
  }
};

template <>
struct Mfma16x16x32<F16> {
  static __device__ __forceinline__ f32x4 run(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static constexpr uint32_t kOnes = 0x3c003c00u;  // two f16 1.0
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define DSA_LDS __attribute__((address_space(3)))

// One K or V tile in LDS: 64 rows of D 16-bit elements, 16-byte chunk c of
// row r stored at chunk position c ^ swz(r).
template <int D>
struct TileLds {
  static constexpr int NCH = D / 8;  // 16-byte chunks per row
  static constexpr int BYTES = kKT * D * 2;
  // K is read as 16-byte A fragments by 16 consecutive rows at one chunk:
  // row % NCH spreads them over NCH chunk positions.
  static __device__ __forceinline__ int swz_k(int r) { return r & (NCH - 1); }
  // V is read by the transposing 8-byte reads: 4 consecutive rows at one
  // chunk pair {2m, 2m+1} per 16-lane group; 2*(r % (NCH/2)) keeps the pair
  // together and moves it per row.
  static __device__ __forceinline__ int swz_v(int r) { return (2 * r) & (NCH - 1); }
};

// Issue this wave's share of the DMA of one tile (rows s0 .. s0+63 of a
// [T, HQ*D] tensor, this head's D columns) into `dst`.  Rows past T are
// clamped to T-1 (never causal for any query).  Completion is awaited with
// vmcnt before the barrier that publishes the tile.
template <int D, bool IS_K>
__device__ __forceinline__ void dma_tile(const uint16_t* __restrict__ src, int64_t rowE, int s0,
                                         int T, DSA_LDS uint8_t* dst, int wave, int lane) {
  using L = TileLds<D>;
  constexpr int PER_WAVE = L::BYTES / 1024 / (kNT / kWave);  // 1 KiB DMA instructions per wave
  // 32-bit byte offsets against the uniform base (the host keeps a batch
  // element's K and V under 4 GiB)
  const char* base = reinterpret_cast<const char*>(src);
  const uint32_t rowbytes = static_cast<uint32_t>(rowE) * 2u;
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int ins = wave * PER_WAVE + i;
    const int P = ins * 64 + lane;  // physical chunk index this lane fills
    const int r = P / L::NCH, pc = P % L::NCH;
    const int lc = pc ^ (IS_K ? L::swz_k(r) : L::swz_v(r));
    const uint32_t s = static_cast<uint32_t>(min(s0 + r, T - 1));
    const uint32_t off = s * rowbytes + 16u * static_cast<uint32_t>(lc);
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint16_t*>(base + off),
                                     dst + ins * 1024, 16, 0, 0);
  }
}

__device__ __forceinline__ void wait_dma_and_sync() {
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  block_sync_lds();
}

template <typename Tag, int D, bool VEC>
__global__ __launch_bounds__(kNT, 2) void tile_attn_kernel(TileArgs a) {
  static_assert(D == 64 || D == 128, "head dim");
  using M = Mfma16x16x32<Tag>;
  using L = TileLds<D>;
  constexpr int NKS = D / 32;  // k-steps of the first product
  constexpr int NDT = D / 16;  // 16-dim output tiles
  // Two buffers per operand, as separate objects: the compiler then knows a
  // DMA into one buffer does not alias reads of the other, and keeps the
  // next tile's DMA in flight while the current tile is read.
  __shared__ __align__(16) uint8_t k0[L::BYTES], k1[L::BYTES], v0[L::BYTES], v1[L::BYTES];

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

  const int s_hi = min(T, t0 + kTQ);          // keys [0, s_hi) can be causal in this block
  const int nkt = (s_hi + kKT - 1) / kKT;
  const int wave_last = min(tw + 31, T - 1);  // last query of this wave

  DSA_LDS uint8_t* kb[2] = {(DSA_LDS uint8_t*)k0, (DSA_LDS uint8_t*)k1};
  DSA_LDS uint8_t* vb[2] = {(DSA_LDS uint8_t*)v0, (DSA_LDS uint8_t*)v1};
  dma_tile<D, true>(Kb, rowE, 0, T, kb[0], wave, lane);
  dma_tile<D, false>(Vb, rowE, 0, T, vb[0], wave, lane);

  // Q^T fragments: qf[qt][ks] = Q[query tw+16qt+c16][dims 32ks+8g .. +8].
  u32x4 qf[2][NKS];
  int tq[2];
  float thr[2];
  const float* srow[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    tq[qt] = tw + 16 * qt + c16;
    const int tl = min(tq[qt], T - 1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qf[qt][ks] = *reinterpret_cast<const u32x4*>(Qb + tl * rowE + 32 * ks + 8 * g);
    thr[qt] = a.thr[b * T + tl];
    srow[qt] = a.scores + (b * T + tl) * a.ld;
  }

  float m[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};
  // Softmax normaliser per query as an MFMA accumulator: ones . P^T sums the
  // tile's (16-bit) probabilities over all 64 keys of the tile, the same
  // values the O product uses; every register of a query's lanes holds it.
  f32x4 lacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  const u32x4 ones = u32x4{M::kOnes, M::kOnes, M::kOnes, M::kOnes};
  f32x4 o[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) o[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Per-lane LDS read offsets within a tile (the swizzles depend on the row
  // only through c16 (K) and 4g + c16/4 (V), so they are loop invariant).
  int kofs[NKS], vofs[NDT];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) kofs[ks] = c16 * (2 * D) + 16 * ((4 * ks + g) ^ L::swz_k(c16));
  {
    const int vr = 4 * g + (c16 >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      vofs[dt] = vr * (2 * D) + 16 * ((2 * dt + ((c16 & 3) >> 1)) ^ L::swz_v(vr)) + 8 * (c16 & 1);
  }

  // This wave's scores of key tile kt: sv[qt][j][r] = scores[tq[qt]][s0 +
  // 16j + 4g + r].  Always the same loads (addresses clamped into the row;
  // entries that are not causal are masked in compute), with no branches:
  // loads complete in order, so with a fixed count the mask waits for these
  // loads only and not for the next tile's DMA issued behind them.
  const int64_t s_clamp = VEC ? a.ld - 4 : a.ld - 1;
  auto load_scores = [&](int kt, float (&sv)[2][4][4]) {
    const int s0 = kt * kKT;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = s0 + 16 * j + 4 * g;
        if constexpr (VEC) {
          const float4 f = *reinterpret_cast<const float4*>(srow[qt] + min<int64_t>(s, s_clamp));
          sv[qt][j][0] = f.x; sv[qt][j][1] = f.y; sv[qt][j][2] = f.z; sv[qt][j][3] = f.w;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[qt][j][r] = srow[qt][min<int64_t>(s + r, s_clamp)];
        }
      }
    }
  };

  // Selection of this wave's 32 x 64 tile: sel[qt][j][r] for (query
  // tq[qt], key s0 + 16j + 4g + r).  Kept as lane masks (one compare each)
  // and applied once per entry in compute, as a select of the logit or
  // -inf -- exact for any logit, NaN and +-inf of unselected keys included
  // (the reference masks them to -inf before its softmax).  Returns whether
  // the wave has work in the tile.  Bitwise & and | keep it branch-free.
  auto make_sel = [&](int kt, const float (&sv)[2][4][4], bool (&sel)[2][4][4]) {
    const int s0 = kt * kKT;
    const bool inner = (s0 + kKT - 1 <= tw) && (tw + 31 < T);  // every entry causal
    bool any = false;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // key s0 + 16j + 4g + r is causal for query tq iff 16j + r <= tq - s0 - 4g:
      // one compare against a constant per entry
      const int dq = (tq[qt] < T) ? tq[qt] - s0 - 4 * g : -1;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // NaN scores and thresholds select nothing
          sel[qt][j][r] = (inner | (16 * j + r <= dq)) & (sv[qt][j][r] >= thr[qt]);
          any |= sel[qt][j][r];
        }
    }
    return s0 <= wave_last && __ballot(any) != 0;
  };

  // Everything one wave does with key tile kt, staged in (kl, vl).
  auto compute = [&](const bool (&sel)[2][4][4], const DSA_LDS uint8_t* kl,
                     const DSA_LDS uint8_t* vl) {
    // S^T = K . Q^T; A fragment = K row 16j+c16, chunk 4ks+g (swizzled):
    // byte offset kofs[ks] + 16j rows (swz_k(16j+c16) = swz_k(c16)).
    f32x4 st[4][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) st[j][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const u32x4 ka = *reinterpret_cast<const DSA_LDS u32x4*>(kl + kofs[ks] + 16 * j * (2 * D));
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) st[j][qt] = M::run(ka, qf[qt][ks], st[j][qt]);
      }
    }

    // Online softmax per query, log2 domain.  The running max moves only
    // when a tile's max exceeds it by more than 2^8 (probabilities stay
    // <= 256, far from overflow in fp32 and exact in scale for 16-bit), so
    // the O rescale is skipped on almost every tile.
    u32x4 pf[2][2];
    bool grow = false;
    float alpha[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // masked logits: the logit where selected, -inf where not
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st[j][qt][r] = sel[qt][j][r] ? st[j][qt][r] : -__builtin_huge_valf();
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[j][qt][r]);
      mx = max_xor32(max_xor16(mx));  // over the 4 lane groups (VALU lane swaps)
      const float m_blk = mx * a.scale_log2;
      const bool up = m_blk > m[qt] + 8.f;
      const float m_new = up ? m_blk : m[qt];
      alpha[qt] = up ? exp2f(m[qt] - m_new) : 1.f;   // m = -inf: alpha = 0 on an empty O
      grow |= up && (m[qt] != -__builtin_huge_valf());
      m[qt] = m_new;
      const float m_use = (m_new == -__builtin_huge_valf()) ? 0.f : m_new;
      float p[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)  // bare v_exp_f32; exp2(-inf) = 0 for unselected keys
          p[j][r] = __builtin_amdgcn_exp2f(fmaf(st[j][qt][r], a.scale_log2, -m_use));
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        pf[qt][jj] = u32x4{M::pack(p[2 * jj][0], p[2 * jj][1]), M::pack(p[2 * jj][2], p[2 * jj][3]),
                           M::pack(p[2 * jj + 1][0], p[2 * jj + 1][1]),
                           M::pack(p[2 * jj + 1][2], p[2 * jj + 1][3])};
    }
    if (__ballot(grow) != 0) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[dt][qt][r] *= alpha[qt];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int r = 0; r < 4; ++r) lacc[qt][r] *= alpha[qt];
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) lacc[qt] = M::run(ones, pf[qt][jj], lacc[qt]);

    // O^T += V^T . P^T.  Lane (g, j=c16) addresses V row key0 + 4g + j/4,
    // dims 16dt + 4(j%4) .. +3; rows key0 + 16 and + 32 keep the swizzle, so
    // byte offset vofs[dt] + (32jj + 16h) rows.
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const DSA_LDS uint8_t* va = vl + vofs[dt] + 32 * jj * (2 * D);
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((DSA_LDS s16x4*)va);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((DSA_LDS s16x4*)(va + 16 * (2 * D)));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        const u32x4 vfrag = u32x4{l2.x, l2.y, h2.x, h2.y};
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[dt][qt] = M::run(vfrag, pf[qt][jj], o[dt][qt]);
      }
    }
  };

  // Per tile: scores -> mask (waits for the score loads), then the next
  // tile's DMA is issued (so nothing below waits for it), then the products.
  wait_dma_and_sync();
  float sv[2][4][4];
  bool sel[2][4][4];
  for (int kt = 0; kt < nkt; kt += 2) {
    // tile kt in buffers 0 (DMA'd before the barrier above); tile kt+1 -> buffers 1
    load_scores(kt, sv);
    bool act = make_sel(kt, sv, sel);
    if (kt + 1 < nkt) {
      dma_tile<D, true>(Kb, rowE, (kt + 1) * kKT, T, kb[1], wave, lane);
      dma_tile<D, false>(Vb, rowE, (kt + 1) * kKT, T, vb[1], wave, lane);
    }
    if (act) compute(sel, kb[0], vb[0]);
    wait_dma_and_sync();
    if (kt + 1 >= nkt) break;
    load_scores(kt + 1, sv);
    act = make_sel(kt + 1, sv, sel);
    if (kt + 2 < nkt) {
      dma_tile<D, true>(Kb, rowE, (kt + 2) * kKT, T, kb[0], wave, lane);
      dma_tile<D, false>(Vb, rowE, (kt + 2) * kKT, T, vb[0], wave, lane);
    }
    if (act) compute(sel, kb[1], vb[1]);
    wait_dma_and_sync();
  }

  // O = O^T / l, lane l: query tq[qt], dims 16dt + 4g .. +3.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float inv = 1.f / lacc[qt][0];  // lt == 0 only if nothing passed: NaN, as the reference
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
  if (a.vec)
    hipLaunchKernelGGL((tile_attn_kernel<Tag, D, true>), dim3(static_cast<unsigned>(nblk)),
                       dim3(kNT), 0, stream, a);
  else
    hipLaunchKernelGGL((tile_attn_kernel<Tag, D, false>), dim3(static_cast<unsigned>(nblk)),
                       dim3(kNT), 0, stream, a);
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
