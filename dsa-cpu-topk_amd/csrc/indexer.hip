// indexer.hip -- standalone lightning-indexer scores [B,T,T] fp32 (gfx950 MFMA).
//
// Replaces _indexer_score_kernel + indexer_scores_triton
// (reference lightning_indexer.py:54-125).  Same output: causal scores, -inf
// above the diagonal (written only on request -- the public drop-in asks for
// it because callers check it, the internal split pipeline does not).
//
// Two kernels:
//
// indexer_qtile_kernel (query-stationary; used whenever a 4-query tile of q
//   fits in LDS).  A block owns TQ = 4*NQ consecutive queries of one batch
//   element.  It stages their q rows (all heads) into LDS once, already in
//   MFMA fragment order, so every later A-operand read is one conflict-free
//   ds_read_b128 per lane, and their w rows next to them.  Its 16 waves (4
//   per SIMD: the q tile fills the CU's LDS, so one block is all a CU holds;
//   8 for fp8 at DI <= 64)
//   then split the causal key range [0, t0+TQ) into super-blocks of 16*KB
//   keys, load each super-block's k rows straight into B-operand registers,
//   and run all TQ queries x HI heads against it.  q is read from HBM
//   exactly once; k (B*T*DI elements) is re-read from L2 / MALL once per
//   query tile.
//
// indexer_kernel (register-streaming; fallback for very wide q rows).  Grid
//   x = (batch, 16-query tile), y = 256-key chunk; each wave owns 4 queries
//   and walks its chunk with indexer_rows (indexer_tile.h).
//
// Both skip key blocks wholly above the diagonal (no MFMA work there); they
// only write -inf when asked, which is what the reference's kernel computes
// for those tiles anyway (lightning_indexer.py:92-94).
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
  int64_t ldq, ldk, ldw;  // elements from one token's q / k / w row to the next
  // fp8 only (either may be null): per (token, head) scales of q [B*T, HI]
  // and per token scales of k [B*T], fp32, positive.
  const float* q_scale;
  const float* k_scale;
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

  const raw* q = static_cast<const raw*>(a.q) + b * T * a.ldq;
  const raw* k = static_cast<const raw*>(a.k) + b * T * a.ldk;
  const raw* w = static_cast<const raw*>(a.w) + b * T * a.ldw;
  float* out = a.scores + (b * T) * a.ld;
  const float ninf = -__builtin_huge_valf();
  const int tq = t0 + g;  // this lane's output query

  // Keys this wave must compute: [c0, min(c1, t0 + 4)).
  const int s_end = (t0 + 4 < c1) ? t0 + 4 : c1;
  int done_end = c0;
  if (s_end > c0) {
    indexer_rows<Tag, DI, KB>(q, k, w, T, a.HI, a.ldq, a.ldk, a.ldw, t0, c0, s_end,
                              [&](int s0, const float(&sc)[KB]) {
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

// ---------------------------------------------------------------------------
// Query-stationary kernel.
// ---------------------------------------------------------------------------
// Waves per block.  16 = 4 per SIMD, which caps a wave at 128 registers: one
// super-block of B operands (64 for 16-bit DI = 128), no second set to
// prefetch into -- the SIMD's other three waves cover a wave's key-row
// latency instead (8 waves with two register sets ping-ponged: config 4
// 1.68 -> 1.56 ms; fp8 1.0 -> 0.89 ms at DI = 128).  fp8 at DI <= 64 does
// half-padded MFMAs on 16-register operand sets, and there 8 waves with the
// ping-pong stay faster (0.76 vs 0.80 ms at T = 16384, HI = 64).
template <typename Tag, int DI, int NQ>
constexpr int qtile_waves() { return (__is_same(Tag, FP8) && DI <= 64) ? 8 : 16; }
#ifndef DSA_QTILE_MAX_NQ
#define DSA_QTILE_MAX_NQ 4
#endif
constexpr size_t kQTileLds = 160 * 1024;  // q + w tile budget per block (all of a CU's LDS)

// 16-byte chunks of one lane's DI/4-element operand slice.
template <typename Tag, int DI>
constexpr int lane_chunks() { return (DI / 4) * Tag::kBytes / 16; }

// One 16-byte A chunk against the matching chunk of a key block's B slice.
template <typename Tag, int E>
__device__ __forceinline__ f32x4 mfma_chunk(const uint4& a, const Slice<Tag, E>& b, int c,
                                            f32x4 acc) {
  if constexpr (Tag::kBytes == 4) {
    const float av[4] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z),
                         __uint_as_float(a.w)};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], b.v[4 * c + j], acc, 0, 0, 0);
    return acc;
  } else if constexpr (__is_same(Tag, BF16)) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b.v[c]), acc, 0,
                                                   0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b.v[c]), acc, 0, 0,
                                                  0);
  }
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

// fp8: chunks c and c+1 of A (a0, a1) against the same chunks of a key
// block's B slice on v_mfma_f32_16x16x128_f8f6f4 (E4M3 x E4M3, unscaled).  A
// slice of one chunk (DI = 64) is padded with zeros.
template <int E>
__device__ __forceinline__ f32x4 mfma_fp8(const uint4& a0, const uint4& a1,
                                          const Slice<FP8, E>& b, int c, f32x4 acc) {
  constexpr int NC = E / 16;
  const uint4 b0 = b.v[c];
  const uint4 b1 = (c + 1 < NC) ? b.v[c + 1 < NC ? c + 1 : c] : make_uint4(0u, 0u, 0u, 0u);
  const i32x8 av = {static_cast<int>(a0.x), static_cast<int>(a0.y), static_cast<int>(a0.z),
                    static_cast<int>(a0.w), static_cast<int>(a1.x), static_cast<int>(a1.y),
                    static_cast<int>(a1.z), static_cast<int>(a1.w)};
  const i32x8 bv = {static_cast<int>(b0.x), static_cast<int>(b0.y), static_cast<int>(b0.z),
                    static_cast<int>(b0.w), static_cast<int>(b1.x), static_cast<int>(b1.y),
                    static_cast<int>(b1.z), static_cast<int>(b1.w)};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 0, 0, 0, 0, 0, 0);
}

// The indexer weights w: the input type, except fp32 alongside fp8 q/k.
template <typename Tag>
struct WeightT { using raw = typename Tag::raw; static constexpr bool kF32 = Tag::kBytes == 4; };
template <>
struct WeightT<FP8> { using raw = float; static constexpr bool kF32 = true; };
template <typename Tag>
__device__ __forceinline__ float weight_f32(typename WeightT<Tag>::raw x) {
  if constexpr (WeightT<Tag>::kF32) return x;
  else return to_f32(Tag{}, x);
}

struct QTileShape {
  int nq;   // quads (4 queries) per block
  int nhg;  // head groups of 4 (HI rounded up)
};

template <typename Tag, int DI>
size_t qtile_lds_bytes(QTileShape sh) {
  return static_cast<size_t>(sh.nq) * sh.nhg * (lane_chunks<Tag, DI>() * 1024 + 64);
}

// LDS layout:
//   qf[quad][hg][chunk][lane] : uint4   A fragment of lane `lane`: row r16 =
//       (query 4*quad + r16/4, head 4*hg + r16%4), chunk `chunk` of the
//       lane group's DI slice (lane/16 owns dims [lane/16*DI/4, ...))
//   wf[quad][hg][g][4]        : float   w of query 4*quad+g, heads 4hg..4hg+3
// KS: fp8 with scales.  Positive scales factor out of the ReLU,
//   w * ReLU(qs*ks*<q8,k8>) = (w*qs) * ks * ReLU(<q8,k8>),
// so q's scale is folded into w when w is staged and k's multiplies each
// finished score (loaded with the key block it belongs to).
template <typename Tag, int DI, int KB, int NQ, bool KS = false>
__global__ __launch_bounds__((64 * qtile_waves<Tag, DI, NQ>())) void indexer_qtile_kernel(
    IndexerArgs a) {
  constexpr int NW = qtile_waves<Tag, DI, NQ>();
  using raw = typename Tag::raw;
  using S = Slice<Tag, DI / 4>;
  constexpr int NCH = lane_chunks<Tag, DI>();
  constexpr int E = DI / 4;
  constexpr int EPC = 16 / Tag::kBytes;  // elements per 16-byte chunk
  extern __shared__ __align__(16) uint4 lds[];
  const int T = a.T;
  const int HI = a.HI;
  const int nhg = (HI + 3) >> 2;
  constexpr int TQ = 4 * NQ;
  const int ntile = (T + TQ - 1) / TQ;
  int64_t b;
  int tile;
  causal_block_tile(blockIdx.x, a.B, ntile, b, tile);  // longest rows first
  const int t0 = tile * TQ;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = lane_id();
  const int g = lane >> 4, r16 = lane & 15;

  const raw* q = static_cast<const raw*>(a.q) + b * T * a.ldq;
  const raw* k = static_cast<const raw*>(a.k) + b * T * a.ldk;
  using wraw = typename WeightT<Tag>::raw;
  const wraw* w = static_cast<const wraw*>(a.w) + b * T * a.ldw;
  float* out = a.scores + (b * T) * a.ld;

  uint4* qf = lds;
  float* wf = reinterpret_cast<float*>(lds + static_cast<size_t>(NQ) * nhg * NCH * 64);

  // Stage q: one 16-byte chunk per thread-iteration, coalesced along DI.
  {
    const int hp4 = 4 * nhg;
    const int per_t = hp4 * (DI / EPC);
    const int total = TQ * per_t;
    for (int u = tid; u < total; u += 64 * NW) {
      const int tl = u / per_t;
      const int rem = u - tl * per_t;
      const int h = rem / (DI / EPC);
      const int d0 = (rem - h * (DI / EPC)) * EPC;
      const int t = t0 + tl;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (t < T && h < HI)
        v = *reinterpret_cast<const uint4*>(q + static_cast<int64_t>(t) * a.ldq + h * DI + d0);
      const int gg = d0 / E;
      const int c = (d0 - gg * E) / EPC;
      const int ln = gg * 16 + 4 * (tl & 3) + (h & 3);
      qf[((static_cast<size_t>(tl >> 2) * nhg + (h >> 2)) * NCH + c) * 64 + ln] = v;
    }
    for (int u = tid; u < TQ * hp4; u += 64 * NW) {
      const int tl = u / hp4;
      const int h = u - tl * hp4;
      const int t = t0 + tl;
      float wv = (t < T && h < HI) ? weight_f32<Tag>(w[static_cast<int64_t>(t) * a.ldw + h]) : 0.f;
      if constexpr (KS) {
        if (a.q_scale != nullptr && t < T && h < HI) wv *= a.q_scale[(b * T + t) * HI + h];
      }
      wf[((tl >> 2) * nhg + (h >> 2)) * 16 + (tl & 3) * 4 + (h & 3)] = wv;
    }
  }
  __syncthreads();

  const float ninf = -__builtin_huge_valf();
  const int t_end = (t0 + TQ < T) ? t0 + TQ : T;  // keys [0, t_end) can be causal
  constexpr int SB = 16 * KB;
  const int nsb = (t_end + SB - 1) / SB;

  // k rows of super-block sb into B registers.  Rows past T are clamped to
  // row T-1: their scores are never stored.
  // k's scales of a super-block: one load per lane (lane l holds key
  // s0 + l % SB), spread to the lanes that store each key by row swaps.
  const float* ksc = KS && a.k_scale != nullptr ? a.k_scale + b * T : nullptr;
  auto load_b = [&](int sbi, S (&bk)[KB], float& ksr) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int s = min(sbi * SB + 16 * kb + r16, T - 1);
      bk[kb].load(k + static_cast<int64_t>(s) * a.ldk + g * E);
    }
    if constexpr (KS) ksr = ksc != nullptr ? ksc[min(sbi * SB + (lane % SB), T - 1)] : 1.f;
  };
  // ks[kb] = scale of key s0 + 16kb + r16, from lane 16kb + r16's load
  auto spread_ks = [&](float ksr, float (&ks)[KB]) {
    if constexpr (!KS) {
      (void)ksr;
      (void)ks;
    } else if constexpr (KB == 4) {
      const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(ksr), __float_as_uint(ksr),
                                                      false, false);  // rows {0,1} / {2,3} of l
      const auto lo = __builtin_amdgcn_permlane16_swap(x[0], x[0], false, false);
      const auto hi = __builtin_amdgcn_permlane16_swap(x[1], x[1], false, false);
      ks[0] = __uint_as_float(lo[0]);
      ks[1] = __uint_as_float(lo[1]);
      ks[2] = __uint_as_float(hi[0]);
      ks[3] = __uint_as_float(hi[1]);
    } else {
      static_assert(KB == 2, "fp8 super-blocks are 2 or 4 key blocks");
      const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(ksr), __float_as_uint(ksr),
                                                      false, false);
      ks[0] = __uint_as_float(x[0]);
      ks[1] = __uint_as_float(x[1]);
    }
  };

  // All NQ quads against one super-block.  The head-group loop holds no
  // stores: a loop with stores and no loads makes the compiler drain every
  // outstanding load (the prefetch included) before entering it.
  auto compute = [&](int sbi, const S (&bk)[KB], float ksr) {
    const int s0 = sbi * SB;
    float sc[NQ][KB];
#pragma unroll
    for (int qd = 0; qd < NQ; ++qd)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sc[qd][kb] = 0.f;
    const uint4* qa = qf + lane;
    const float4* wq = reinterpret_cast<const float4*>(wf) + g;
    for (int hg = 0; hg < nhg; ++hg) {
#pragma unroll
      for (int qd = 0; qd < NQ; ++qd) {
        f32x4 acc[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        // 16-bit: the unit's MFMAs at raised priority, its ReLU.w epilogue at
        // the normal one, so a SIMD's waves with MFMAs to issue go first and
        // the epilogues fill in behind (config 4: 1.54-1.60 -> 1.52-1.57 ms;
        // fp32 unchanged, so left as is).
        if constexpr (Tag::kBytes == 2) __builtin_amdgcn_s_setprio(1);
        if constexpr (__is_same(Tag, FP8)) {
#pragma unroll
          for (int c = 0; c < NCH; c += 2) {
            const uint4 a0 = qa[((qd * nhg + hg) * NCH + c) * 64];
            const uint4 a1 = (c + 1 < NCH) ? qa[((qd * nhg + hg) * NCH + (c + 1 < NCH ? c + 1 : c)) * 64]
                                           : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc[kb] = mfma_fp8<E>(a0, a1, bk[kb], c, acc[kb]);
          }
        } else if constexpr (Tag::kBytes == 2 && NCH <= 4 && NQ <= 2) {
          // All of the unit's A fragments read before its MFMAs (a scheduling
          // fence keeps them together): one LDS latency per unit, not one per
          // chunk (config 4 1.56 -> 1.51 ms; fp32 is faster without it, and
          // wider rows or four quads would spill the 128 registers).
          uint4 av[NCH];
#pragma unroll
          for (int c = 0; c < NCH; ++c) av[c] = qa[((qd * nhg + hg) * NCH + c) * 64];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc[kb] = mfma_chunk<Tag, E>(av[c], bk[kb], c, acc[kb]);
        } else {
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
            const uint4 av = qa[((qd * nhg + hg) * NCH + c) * 64];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc[kb] = mfma_chunk<Tag, E>(av, bk[kb], c, acc[kb]);
          }
        }
        if constexpr (Tag::kBytes == 2) __builtin_amdgcn_s_setprio(0);
        const float4 wv = wq[(qd * nhg + hg) * 4];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sc[qd][kb] = fmaf(wv.x, relu_f32(acc[kb][0]), sc[qd][kb]);
          sc[qd][kb] = fmaf(wv.y, relu_f32(acc[kb][1]), sc[qd][kb]);
          sc[qd][kb] = fmaf(wv.z, relu_f32(acc[kb][2]), sc[qd][kb]);
          sc[qd][kb] = fmaf(wv.w, relu_f32(acc[kb][3]), sc[qd][kb]);
        }
      }
    }
    float ks[KB];
    if constexpr (KS) spread_ks(ksr, ks);
#pragma unroll
    for (int qd = 0; qd < NQ; ++qd) {
      const int tq = t0 + 4 * qd + g;  // this lane's output query
      if (tq < T) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int s = s0 + 16 * kb + r16;
          float v = sc[qd][kb];
          if constexpr (KS) v *= ks[kb];
          if (s < T && (s <= tq || a.write_upper))
            out[static_cast<int64_t>(tq) * a.ld + s] = (s <= tq) ? v : ninf;
        }
      }
    }
  };

  if constexpr (NW == 16) {
    // One register set per wave: a super-block's rows load, then its
    // products run; the SIMD's other waves issue MFMAs while this one waits
    // on L2.
    S bk[KB];
    float ksr = 1.f;  // k's scale (KS only; otherwise unused)
    for (int sb = wave; sb < nsb; sb += NW) {
      load_b(sb, bk, ksr);
      compute(sb, bk, ksr);
    }
  } else {
    // Two register sets ping-pong: the next super-block's rows load during
    // this one's products.  Super-blocks past the last one load row T-1's
    // clamp like rows past T (never stored); unconditional loads keep the
    // wait counts exact, so the prefetch stays in flight during the MFMAs.
    const int last = nsb - 1;
    S b0[KB], b1[KB];
    float k0s = 1.f, k1s = 1.f;  // k's scales (KS only; otherwise unused)
    int sb = wave;
    load_b(min(sb, last), b0, k0s);
    while (sb < nsb) {
      load_b(min(sb + NW, last), b1, k1s);
      compute(sb, b0, k0s);
      sb += NW;
      if (sb >= nsb) break;
      load_b(min(sb + NW, last), b0, k0s);
      compute(sb, b1, k1s);
      sb += NW;
    }
  }

  // Keys past the last super-block are above the diagonal for every query.
  if (a.write_upper) {
    const int s_lo = nsb * SB;
    const int width = T - s_lo;
    if (width > 0) {
      for (int tl = wave; tl < TQ; tl += NW) {
        const int t = t0 + tl;
        if (t >= T) break;
        for (int s = s_lo + lane; s < T; s += 64) out[static_cast<int64_t>(t) * a.ld + s] = ninf;
      }
    }
  }
}

template <typename Tag, int DI, int KB, int NQ, bool KS = false>
hipError_t launch_qtile(const IndexerArgs& a, QTileShape sh, hipStream_t stream) {
  auto kern = indexer_qtile_kernel<Tag, DI, KB, NQ, KS>;
  const size_t lds = qtile_lds_bytes<Tag, DI>(sh);
  static const bool attr_set = [&] {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(kQTileLds));
    if (e != hipSuccess) (void)hipGetLastError();
    return e == hipSuccess;
  }();
  (void)attr_set;
  const int64_t nblk = a.B * ((a.T + 4 * NQ - 1) / (4 * NQ));
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nblk)), dim3(64 * qtile_waves<Tag, DI, NQ>()), lds, stream,
                     a);
  return hipGetLastError();
}

// Largest quad count (<= DSA_QTILE_MAX_NQ) whose q + w tile fits the LDS
// budget; 0 when one quad does not fit.
template <typename Tag, int DI>
QTileShape pick_qtile(const IndexerArgs& a) {
  QTileShape sh{0, (a.HI + 3) / 4};
  for (int nq = DSA_QTILE_MAX_NQ; nq >= 1; nq >>= 1) {
    if (qtile_lds_bytes<Tag, DI>(QTileShape{nq, sh.nhg}) <= kQTileLds) {
      sh.nq = nq;
      break;
    }
  }
  return sh;
}

template <typename Tag, int DI, int KB>
hipError_t launch_stream(const IndexerArgs& a, hipStream_t stream);

template <typename Tag, int DI, int KB>
hipError_t launch(const IndexerArgs& a, hipStream_t stream) {
  const QTileShape sh = pick_qtile<Tag, DI>(a);
  if constexpr (__is_same(Tag, FP8)) {
    if (a.q_scale != nullptr || a.k_scale != nullptr) {
      switch (sh.nq) {
        case 4: return launch_qtile<Tag, DI, KB, 4, true>(a, sh, stream);
        case 2: return launch_qtile<Tag, DI, KB, 2, true>(a, sh, stream);
        case 1: return launch_qtile<Tag, DI, KB, 1, true>(a, sh, stream);
      }
      return hipErrorNotSupported;
    }
  }
  switch (sh.nq) {
    case 4: return launch_qtile<Tag, DI, KB, 4>(a, sh, stream);
    case 2: return launch_qtile<Tag, DI, KB, 2>(a, sh, stream);
    case 1: return launch_qtile<Tag, DI, KB, 1>(a, sh, stream);
  }
  if constexpr (__is_same(Tag, FP8)) return hipErrorNotSupported;  // no streaming fp8 kernel
  else return launch_stream<Tag, DI, KB>(a, stream);
}

template <typename Tag, int DI, int KB>
hipError_t launch_stream(const IndexerArgs& a, hipStream_t stream) {
  const int ntile = (a.T + 15) / 16;
  const dim3 grid(static_cast<unsigned>(a.B * ntile), static_cast<unsigned>((a.T + kChunk - 1) / kChunk));
  hipLaunchKernelGGL((indexer_kernel<Tag, DI, KB>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename Tag>
hipError_t dispatch_di(const IndexerArgs& a, int DI, hipStream_t stream) {
  if constexpr (__is_same(Tag, FP8)) {
    switch (DI) {
      case 64: return launch<Tag, 64, 4>(a, stream);
      case 128: return launch<Tag, 128, 4>(a, stream);
      case 256: return launch<Tag, 256, 2>(a, stream);
    }
  } else if constexpr (Tag::kBytes == 4) {
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
  if (dtype == 3) return DI == 64 || DI == 128 || DI == 256;
  return false;
}

bool indexer_fp8_fits(int HI, int DI) {
  // one 4-query tile of fp8 q (16 rows of DI bytes per head group) plus its w
  // fits the LDS budget; fp8 has no streaming kernel to fall back on
  const int nhg = (HI + 3) / 4;
  return static_cast<size_t>(nhg) * (16 * DI + 64) <= kQTileLds;
}

hipError_t launch_indexer(const void* q, const void* k, const void* w, int dtype, int64_t B,
                          int64_t T, int HI, int DI, int64_t ldq, int64_t ldk, int64_t ldw,
                          float* scores, int64_t ld, int write_upper, hipStream_t stream,
                          const float* q_scale, const float* k_scale) {
  if (B == 0 || T == 0) return hipSuccess;
  if ((q_scale != nullptr || k_scale != nullptr) && dtype != 3) return hipErrorInvalidValue;
  IndexerArgs a{q, k, w, B, static_cast<int>(T), HI, scores, ld, write_upper, ldq, ldk, ldw,
                q_scale, k_scale};
  switch (dtype) {
    case 0: return dispatch_di<F32>(a, DI, stream);
    case 1: return dispatch_di<BF16>(a, DI, stream);
    case 2: return dispatch_di<F16>(a, DI, stream);
    case 3: return dispatch_di<FP8>(a, DI, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace dsa
