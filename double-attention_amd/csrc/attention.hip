// Flash-tiled outer attention with the map mix fused in.
//
// Replaces routed_attention_reference (reference src/double_attention/ops.py:65-93),
// its Triton forward (triton_kernels.py:674-811, 2022-2090) and the map combine
// of SharedDictionaryAttention.forward (modules.py:265-272):
//   O_s = softmax(gamma_s * q_s k_s^T, causal) V          for every outer map s
//   Y   = sum_s alpha_s O_s,  alpha = softmax(map_mix_logits)   (mix mode)
// or every O_s written to its own slot (per-map mode, used by the concat
// combine and by the operator-level API).
//
// A workgroup of NW waves (2 or 4) owns 32*NW query rows of one sequence and
// a slice of DS value features; every wave owns 32 queries (two 16-column MFMA
// blocks) and the whole slice, so no score tile is formed twice inside a
// workgroup.  The value width is split over workgroups (DS <= 128) to keep a
// wave's accumulators small enough for two waves per SIMD.  A wave walks the
// (map, 32-key tile) sequence up to the causal bound in the transposed domain:
//   S^T[key, q] = sum_r K[key, r] Q^T[r, q]      (A = key rows from LDS, B = queries in VGPRs)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P in VGPRs)
// so P never leaves registers, and every A fragment read from LDS feeds two
// MFMAs (the two query blocks).  Key and V^T tiles are double-buffered in
// padded LDS tiles (da_tile.h) filled by global->LDS DMA; the loads of the next
// tile are spread through the score loop, so no wave stalls on a full memory
// queue in one burst.  V^T arrives from the projection GEMM in 32-token tiles
// (element (b, d, t) at b*stride_b + (t/32)*32*D + 32*d + t%32), so each
// slice of a V tile is one contiguous block.  gamma_s = exp(clamp(log scale))
// and the mix weights are computed on the device: a forward never
// synchronizes with the host.
//
// Element types: TQ for the routed queries/keys (fp16 on the module path: they
// are unit vectors), TV for V, the probabilities and the output.
#include <algorithm>
#include <type_traits>

#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kKeyTile = 32;
constexpr int kAttnQW = 32;     // queries per wave

struct AttnParams {
  const void* q;
  const void* k;
  int64_t qk_stride_b, qk_stride_t, map_stride;
  int map_repeat;
  const void* vt;
  int64_t vt_stride_b;
  int S, T, D;
  int n_qt, n_slices;
  int chunk_tiles;     // > 0: split long causal key ranges into chunks of this many key tiles
  int n_items;         // workgroups per (sequence, slice): sum over query tiles of their chunks
  float* part;         // per item: [QT][DS] unnormalized outputs, then [QT] reference m, [QT] sums l
  const void* scales;
  int scales_dtype;
  float scale_mult;
  const void* mix_logits;
  int mix_dtype;
  int flags;
  float score_bound;   // > 0: |q . k| <= score_bound for every raw score
  void* out;
  int64_t out_stride_b, out_stride_t, out_stride_s;
};

__device__ __forceinline__ float map_gamma(const AttnParams& p, int s) {
  float v = load_scalar(p.scales, p.scales_dtype, s);
  if (p.flags & kAttnScalesAreLog) v = expf(fminf(fmaxf(v, kLogScaleMin), kLogScaleMax));
  return v * p.scale_mult;
}

__device__ __forceinline__ float map_weight(const AttnParams& p, int s) {
  if (!(p.flags & kAttnMix)) return 1.f;
  if (p.mix_logits == nullptr) return 1.f / static_cast<float>(p.S);
  float mx = -INFINITY;
  for (int i = 0; i < p.S; ++i) mx = fmaxf(mx, load_scalar(p.mix_logits, p.mix_dtype, i));
  float den = 0.f;
  for (int i = 0; i < p.S; ++i) den += expf(load_scalar(p.mix_logits, p.mix_dtype, i) - mx);
  return expf(load_scalar(p.mix_logits, p.mix_dtype, s) - mx) / den;
}

// Store DC accumulator columns (value features d0 .. d0+DC-1) of query t.
template <typename T, int DC>
__device__ __forceinline__ void store_rows(const AttnParams& p, int b, int s, int t, int g, int d0,
                                           const f32x4* acc, float w) {
  T* orow = static_cast<T*>(p.out) + b * p.out_stride_b + static_cast<int64_t>(t) * p.out_stride_t +
            s * p.out_stride_s + d0;
#pragma unroll
  for (int db = 0; db < DC / 16; ++db) {
    typename Elem<T>::v4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<T>(acc[db][i] * w);
    *reinterpret_cast<typename Elem<T>::v4*>(orow + db * 16 + 4 * g) = o;
  }
}

// Key tiles of query tile qt (QT queries) and the chunks they are split into.
__device__ __forceinline__ int key_tiles_of(const AttnParams& p, int qt, int QT) {
  if (!(p.flags & kAttnCausal)) return (p.T + kKeyTile - 1) / kKeyTile;
  return (min(qt * QT + QT, p.T) - 1) / kKeyTile + 1;
}
__device__ __forceinline__ int chunks_of(const AttnParams& p, int qt, int QT) {
  return p.chunk_tiles > 0 ? (key_tiles_of(p, qt, QT) + p.chunk_tiles - 1) / p.chunk_tiles : 1;
}
// Items (query tile x key chunk) of query tiles qt .. n_qt-1, which come
// first in the heaviest-first order.  With chunking the tiles are QT = 64
// queries = 2 key tiles, so a full causal tile t has 2(t+1) key tiles and
// ceil((t+1)/h) chunks (h = chunk_tiles/2), whose prefix sums have a closed
// form: sum_{q=1..n} ceil(q/h) = h a(a+1)/2 + r(a+1), n = a h + r.
__device__ __forceinline__ int ceil_sum(int n, int h) {
  const int a = n / h;
  const int r = n - a * h;
  return h * a * (a + 1) / 2 + r * (a + 1);
}
__device__ __forceinline__ int items_from(const AttnParams& p, int qt, int QT) {
  if (qt >= p.n_qt) return 0;
  if (p.chunk_tiles == 0) return p.n_qt - qt;
  if (!(p.flags & kAttnCausal)) return (p.n_qt - qt) * chunks_of(p, 0, QT);
  const int last = p.n_qt - 1;   // the last tile may be partial
  return ceil_sum(last, p.chunk_tiles / 2) - ceil_sum(qt, p.chunk_tiles / 2) + chunks_of(p, last, QT);
}
// Work item y of a (sequence, slice): returns its query tile; `chunk`,
// `n_chunks` and `first` (the item index of the tile's chunk 0) describe its
// place.  Binary search on the decreasing items_from.
__device__ __forceinline__ int decode_item(const AttnParams& p, int y, int QT, int& chunk, int& n_chunks, int& first) {
  int lo = 0, hi = p.n_qt - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (items_from(p, mid, QT) > y) lo = mid;
    else hi = mid - 1;
  }
  first = items_from(p, lo + 1, QT);
  n_chunks = chunks_of(p, lo, QT);
  chunk = y - first;
  return lo;
}

template <int RP, int DS, int NW>
struct AttnTile {
  typedef PaddedTile<kKeyTile, RP / 8, true> KT;    // keys (blocked rows)
  typedef PaddedTile<DS, kKeyTile / 8, false> VT;   // V^T rows: DS features x 4 chunks
  static constexpr int KPW = (KT::LOADS + NW - 1) / NW;   // key loads per wave
  static constexpr int VPW = (VT::LOADS + NW - 1) / NW;   // V^T loads per wave
  static constexpr int BYTES = KT::BYTES + VT::BYTES;     // one stage: a key tile, then a V^T tile
};

// The tile sequence u = 0 .. total-1 runs over (map s, key tile kt), u = s*n_kt + kt.
// Stage buffer u%2 holds the keys of tile u+1 and the V^T of tile u, so step u
// forms the scores of tile u+1 (MFMA) while it turns the scores of tile u into
// probabilities (VALU) and accumulates P(u) V(u) (MFMA): the softmax of one
// tile runs in the shadow of the next tile's score MFMAs.
template <typename TQ, typename TV, int RP, int DS, int NW, bool MULTI>
__global__ __launch_bounds__(NW * 64, 1) void attention_kernel(AttnParams p) {
  typedef AttnTile<RP, DS, NW> Tile;
  typedef typename Tile::KT KT;
  typedef typename Tile::VT VT;
  typedef typename Elem<TQ>::v8 q8;
  typedef typename Elem<TV>::v8 v8;
  constexpr int KS = RP / 32;
  constexpr int NB = DS / 16;    // accumulator blocks per query block
  constexpr int NL = Tile::KPW + Tile::VPW;
  constexpr int QT = NW * kAttnQW;
  __shared__ __attribute__((aligned(1024))) char lds0[Tile::BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  // blockIdx.y = work item (query tile and key chunk), heaviest first;
  // x = (sequence, slice).
  int chunk, n_chunks, first_item;
  const int qt = decode_item(p, static_cast<int>(blockIdx.y), QT, chunk, n_chunks, first_item);
  const int b = static_cast<int>(blockIdx.x) / p.n_slices;
  const int ds0 = (static_cast<int>(blockIdx.x) - b * p.n_slices) * DS;   // first feature of the slice
  const int q0 = qt * QT;
  const int qw0 = q0 + wave * kAttnQW;                       // this wave's first query
  const bool causal = p.flags & kAttnCausal;
  // Key tiles [kt_begin, kt_begin + n_kt) of every map.
  const int kt_all = key_tiles_of(p, qt, QT);
  const int kt_begin = p.chunk_tiles > 0 ? chunk * p.chunk_tiles : 0;
  const int n_kt = p.chunk_tiles > 0 ? min(p.chunk_tiles, kt_all - kt_begin) : kt_all;
  const int total = p.S * n_kt;

  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b;
  const char* kbase = reinterpret_cast<const char*>(static_cast<const TQ*>(p.k) + b * p.qk_stride_b);
  // Feature d of a 32-token V^T tile sits at 32*d, so the slice is one block.
  const char* vbase = reinterpret_cast<const char*>(static_cast<const TV*>(p.vt) + b * p.vt_stride_b + 32 * ds0);
  const int kstride = static_cast<int>(p.qk_stride_t) * static_cast<int>(sizeof(TQ));   // bytes per key row

  // Per-lane DMA sources of this wave's loads: key load i fills wave load
  // i*NW + wave of the key tile ((row << 16) | byte offset of the chunk; rows
  // are clamped to the last key when the tile is issued), V^T load i the same
  // wave load of the V^T tile (byte offset inside the tile).  Wave loads past a tile's end re-load the data of wave
  // load 0 into slot 0 of that tile.
  uint32_t kdesc[Tile::KPW], vdesc[Tile::VPW];
#pragma unroll
  for (int i = 0; i < Tile::KPW; ++i) {
    int row, ck;
    const int j = i * NW + wave;
    KT::slot_chunk((j < KT::LOADS ? j : 0) * 64 + lane, row, ck);
    kdesc[i] = (static_cast<uint32_t>(row) << 16) | static_cast<uint32_t>(ck * 16);
  }
#pragma unroll
  for (int i = 0; i < Tile::VPW; ++i) {
    int row, ck;
    const int j = i * NW + wave;
    VT::slot_chunk((j < VT::LOADS ? j : 0) * 64 + lane, row, ck);
    vdesc[i] = static_cast<uint32_t>((row * kKeyTile + ck * 8) * sizeof(TV));
  }
  auto slot_of = [&](int n) {
    if (n < Tile::KPW) {
      const int j = n * NW + wave;
      return j < KT::LOADS ? j * 1024 : 0;
    }
    const int j = (n - Tile::KPW) * NW + wave;
    return KT::BYTES + (j < VT::LOADS ? j * 1024 : 0);
  };
  // DMA sources of tile u: key rows (keys past the end re-read the last one)
  // and the V^T tile.
  struct Src {
    const char* k;
    const char* v;
    int last;
  };
  auto source = [&](int uk, int uv) {
    const int sk = uk / n_kt;
    const int k0 = (kt_begin + uk - sk * n_kt) * kKeyTile;
    const int64_t off = static_cast<int64_t>(sk / p.map_repeat) * p.map_stride * static_cast<int64_t>(sizeof(TQ));
    const int v0 = (kt_begin + uv - (uv / n_kt) * n_kt) * kKeyTile;
    return Src{kbase + static_cast<int64_t>(k0) * kstride + off,
               vbase + static_cast<int64_t>(v0) * p.D * static_cast<int64_t>(sizeof(TV)), p.T - 1 - k0};
  };
  auto issue_one = [&](char* buf, const Src& src, int n) {
    if (n < Tile::KPW) {
      const int row = min(static_cast<int>(kdesc[n] >> 16), src.last);
      dma16(src.k + static_cast<uint32_t>(row * kstride + static_cast<int>(kdesc[n] & 0xFFFFu)), buf + slot_of(n));
    } else {
      dma16(src.v + vdesc[n - Tile::KPW], buf + slot_of(n));
    }
  };

  f32x4 acc[2][NB];
  f32x4 yacc[MULTI ? 2 : 1][MULTI ? NB : 1];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      acc[cb][i] = zero4();
      if constexpr (MULTI) yacc[cb][i] = zero4();
    }
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_part[2] = {0.f, 0.f};
  q8 qf[2][KS];

  // Query fragments of map s; returns the map's score multiplier (log2
  // domain).  The rescale test compares maxima of raw scores, so a negative
  // score scale is folded into the queries instead (negation is exact).
  auto load_map = [&](int s) {
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride;
    const float gamma = map_gamma(p, s);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        qf[cb][kk] = tq < p.T ? load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + off + kk * 32 + 8 * g)
                              : zero8<TQ>();
        if (gamma < 0.f) qf[cb][kk] = -qf[cb][kk];
      }
    }
    return fabsf(gamma) * kLog2e;
  };

  const int kfrag = KT::offset(c, g);
  const int vfrag = KT::BYTES + VT::offset(c, g);

  // Scores of 32 keys x 32 queries from a key tile in LDS: four independent
  // accumulator chains, each key fragment feeding both query blocks.  With
  // DMA, the loads of the next stage are spread between the fragment reads.
  auto scores = [&](const char* kt_lds, f32x4 (&st)[2][2], auto with_dma, char* nxt, const Src& src) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) st[cb][0] = st[cb][1] = zero4();
    const char* kf = kt_lds + kfrag;
    // Key fragments are read in groups of KG steps (2*KG reads in flight),
    // then consumed: LDS latency is paid once per group, and the group size
    // bounds the registers the reads hold.
    constexpr int KG = KS < 4 ? KS : 4;
#pragma unroll
    for (int k0 = 0; k0 < KS; k0 += KG) {
      q8 kfr[KG][2];
#pragma unroll
      for (int kk = 0; kk < KG; ++kk) {
        kfr[kk][0] = lds_v8<TQ>(kf + KT::offset(0, (k0 + kk) * 4));
        kfr[kk][1] = lds_v8<TQ>(kf + KT::offset(16, (k0 + kk) * 4));
      }
#pragma unroll
      for (int kk = 0; kk < KG; ++kk) {
        if constexpr (decltype(with_dma)::value) {
#pragma unroll
          for (int n = 0; n < NL; ++n)
            if (n * KS / NL == k0 + kk) issue_one(nxt, src, n);
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          st[cb][0] = Elem<TQ>::mma(kfr[kk][0], qf[cb][k0 + kk], st[cb][0]);
          st[cb][1] = Elem<TQ>::mma(kfr[kk][1], qf[cb][k0 + kk], st[cb][1]);
        }
      }
    }
  };

  // Prologue: keys of tile 0 into stage 1's key slot, stage 0 = {K(1), V(0)}.
  float sc = load_map(0);
  float sc_next = sc;
  {
    const Src s0 = source(0, 0);
#pragma unroll
    for (int n = 0; n < Tile::KPW; ++n) issue_one(lds1, s0, n);
    const Src s1 = source(min(1, total - 1), 0);
#pragma unroll
    for (int n = 0; n < NL; ++n) issue_one(lds0, s1, n);
  }
  wait_vmem();
  __syncthreads();
  f32x4 st_prev[2][2];
  scores(lds1, st_prev, std::false_type{}, nullptr, Src{});

  // One pipelined step u = s*n_kt + kt.  FIXED: every score is bounded by
  // score_bound, so exponents use the fixed reference score_bound*sc (all
  // probabilities <= 1) and the accumulators are never rescaled; otherwise the
  // lazy online rescale runs.
  auto step = [&](auto fixed, int u, int s, int kt) {
    constexpr bool FIXED = decltype(fixed)::value;
    char* cur = (u & 1) ? lds1 : lds0;
    char* nxt = (u & 1) ? lds0 : lds1;
    const int k0 = (kt_begin + kt) * kKeyTile;
    // Tile u + 1 opens map s + 1: its queries are needed by this step's scores.
    if (kt == n_kt - 1 && s + 1 < p.S) sc_next = load_map(s + 1);
    // Stage u + 1 = {K(u + 2), V(u + 1)}, clamped at the end of the sequence.
    const Src src = source(min(u + 2, total - 1), min(u + 1, total - 1));

    // What may branch comes before the barrier: the causal / end mask
    // (diagonal and last tiles only) and the rescale test.  What follows it is
    // one straight block, so the compiler can interleave the exponentials of
    // tile u with the score MFMAs of tile u + 1.
    if ((causal && k0 + kKeyTile - 1 > qw0) || k0 + kKeyTile > p.T) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int tq = qw0 + cb * 16 + c;
        const int kmax = min(causal ? tq : p.T - 1, p.T - 1);   // last key this query sees
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k0 + 8 * g + 4 * kb + i > kmax) st_prev[cb][kb][i] = -INFINITY;
      }
    }
    float m_use[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      if constexpr (FIXED) {
        m_use[cb] = -p.score_bound * sc;
      } else {
        const float lmax =
            fmaxf(fmaxf(fmaxf(st_prev[cb][0][0], st_prev[cb][0][1]), fmaxf(st_prev[cb][0][2], st_prev[cb][0][3])),
                  fmaxf(fmaxf(st_prev[cb][1][0], st_prev[cb][1][1]), fmaxf(st_prev[cb][1][2], st_prev[cb][1][3])));
        lazy_rescale<NB>(lmax, sc, m_run[cb], l_part[cb], acc[cb]);
        m_use[cb] = m_run[cb] == -INFINITY ? 0.f : -m_run[cb];   // negated; 0 while fully masked
      }
    }

    wait_vmem();
    __syncthreads();

    f32x4 st_new[2][2];
    scores(cur, st_new, std::true_type{}, nxt, src);

    // Probabilities of tile u: lane (c, g) holds keys k0 + 8g + 4kb + i for
    // query qw0 + 16cb + c.
    v8 pb[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(st_prev[cb][kb][i], sc, m_use[cb]));
          st_prev[cb][kb][i] = pr;
          psum += pr;
        }
      }
      l_part[cb] += psum;
      pb[cb] = pack_blocked<TV>(st_prev[cb][0], st_prev[cb][1]);   // keys k0 + 8g + e
    }

    // O^T += V^T(u) P^T(u).
    const char* vf = cur + vfrag;
    constexpr int VG = NB < 4 ? NB : 4;
#pragma unroll
    for (int d0 = 0; d0 < NB; d0 += VG) {
      v8 vfr[VG];
#pragma unroll
      for (int db = 0; db < VG; ++db) vfr[db] = lds_v8<TV>(vf + VT::offset((d0 + db) * 16, 0));
#pragma unroll
      for (int db = 0; db < VG; ++db) {
        acc[0][d0 + db] = Elem<TV>::mma(vfr[db], pb[0], acc[0][d0 + db]);
        acc[1][d0 + db] = Elem<TV>::mma(vfr[db], pb[1], acc[1][d0 + db]);
      }
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      st_prev[cb][0] = st_new[cb][0];
      st_prev[cb][1] = st_new[cb][1];
    }
  };

  for (int s = 0; s < p.S; ++s) {
    // The fixed reference keeps every probability within the range of the
    // operand type: bf16 holds 2^-120 .. 1 exactly in exponent; fp16 does not.
    const bool fixed = p.score_bound > 0.f && sizeof(TV) == 2 && !std::is_same<TV, _Float16>::value &&
                       2.f * p.score_bound * sc <= 120.f;
    const int u0 = s * n_kt;
    if (fixed) {
      for (int kt = 0; kt < n_kt; ++kt) step(std::true_type{}, u0 + kt, s, kt);
    } else {
      for (int kt = 0; kt < n_kt; ++kt) step(std::false_type{}, u0 + kt, s, kt);
    }
    const float wmap = map_weight(p, s);
    // A chunk of a split key range (one map) stores its normalized outputs,
    // reference and row sums in fp32 for the merge kernel; otherwise the map's
    // output goes to its slot (or into the mix).
    const bool partial = n_chunks > 1;
    float* part = p.part + (static_cast<int64_t>(blockIdx.x) * p.n_items + blockIdx.y) * (QT * (DS + 2));
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const float l = group_sum(l_part[cb]);
      const float w = (partial ? 1.f : wmap) / (l > 0.f ? l : 1.f);
      const int ql = wave * kAttnQW + cb * 16 + c;
      const int tq = q0 + ql;
      if constexpr (MULTI) {
#pragma unroll
        for (int i = 0; i < NB; ++i) yacc[cb][i] += acc[cb][i] * w;
      } else {
        TV* orow = static_cast<TV*>(p.out) + b * p.out_stride_b + static_cast<int64_t>(tq) * p.out_stride_t +
                   ((p.flags & kAttnMix) ? 0 : s) * p.out_stride_s + ds0;
#pragma unroll
        for (int db = 0; db < NB; ++db) {
          const f32x4 v = acc[cb][db] * w;
          if (partial) {
            *reinterpret_cast<f32x4*>(part + ql * DS + db * 16 + 4 * g) = v;
          } else if (tq < p.T) {
            typename Elem<TV>::v4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = static_cast<TV>(v[r]);
            *reinterpret_cast<typename Elem<TV>::v4*>(orow + db * 16 + 4 * g) = o;
          }
        }
        if (partial && g == 0) {
          part[QT * DS + ql] = fixed ? p.score_bound * sc : m_run[cb];
          part[QT * DS + QT + ql] = l;
        }
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) acc[cb][i] = zero4();
      m_run[cb] = -INFINITY;
      l_part[cb] = 0.f;
    }
    sc = sc_next;
  }

  if constexpr (MULTI) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
      if (tq < p.T) store_rows<TV, DS>(p, b, 0, tq, g, ds0, yacc[cb], 1.f);
    }
  }
  // The last step's (redundant) stage loads must land before the workgroup's
  // LDS is released.
  wait_vmem();
}

// Merge of split key ranges: out = sum_c 2^(m_c - M) l_c o_c / sum_c 2^(m_c - M) l_c,
// o_c = O_c / l_c the chunk's normalized output, M = max_c m_c, per query row
// (one map, weight 1).  Each wave takes one query row, its lanes covering
// consecutive features, so every partial row is read by one coalesced sweep.
template <typename TV, int DS>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnParams p) {
  constexpr int QT = 2 * kAttnQW;
  const int qt = p.n_qt - 1 - static_cast<int>(blockIdx.y);
  const int n_ch = chunks_of(p, qt, QT);
  if (n_ch <= 1) return;   // written directly by its only item
  const int first = items_from(p, qt + 1, QT);
  const int b = static_cast<int>(blockIdx.x) / p.n_slices;
  const int ds0 = (static_cast<int>(blockIdx.x) - b * p.n_slices) * DS;
  constexpr int ITEM = QT * (DS + 2);
  const float* part = p.part + (static_cast<int64_t>(blockIdx.x) * p.n_items + first) * ITEM;
  const int lane = lane_id();
  // blockIdx.z picks four query rows of the tile, one per wave.
  {
    const int ql = static_cast<int>(blockIdx.z) * 4 + (static_cast<int>(threadIdx.x) >> 6);
    const int tq = qt * QT + ql;
    if (tq >= p.T) return;
    float M = -INFINITY;
    for (int c = 0; c < n_ch; ++c) M = fmaxf(M, part[c * ITEM + QT * DS + ql]);
    f32x4 o[DS / 256 > 0 ? DS / 256 : 1];
#pragma unroll
    for (int k = 0; k < (DS / 256 > 0 ? DS / 256 : 1); ++k) o[k] = zero4();
    float den = 0.f;
    for (int c = 0; c < n_ch; ++c) {
      const float m = part[c * ITEM + QT * DS + ql];
      const float wl = (m == -INFINITY ? 0.f : exp2f(m - M)) * part[c * ITEM + QT * DS + QT + ql];
      den += wl;
#pragma unroll
      for (int k = 0; k < (DS / 256 > 0 ? DS / 256 : 1); ++k) {
        const int d4 = (k * 64 + lane) * 4;
        if (d4 < DS) o[k] += wl * *reinterpret_cast<const f32x4*>(part + c * ITEM + ql * DS + d4);
      }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    TV* orow = static_cast<TV*>(p.out) + b * p.out_stride_b + static_cast<int64_t>(tq) * p.out_stride_t + ds0;
#pragma unroll
    for (int k = 0; k < (DS / 256 > 0 ? DS / 256 : 1); ++k) {
      const int d4 = (k * 64 + lane) * 4;
      if (d4 < DS) {
        typename Elem<TV>::v4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = static_cast<TV>(o[k][i] * inv);
        *reinterpret_cast<typename Elem<TV>::v4*>(orow + d4) = v;
      }
    }
  }
}

template <typename TQ, typename TV, int RP, int DS, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, const AttnPlan& plan, AttnParams& p, hipStream_t s) {
  p.n_slices = a.D / DS;
  p.n_qt = plan.n_qt;
  p.chunk_tiles = plan.chunk_tiles;
  p.n_items = plan.n_items;
  hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, 2, MULTI>), dim3(a.B * p.n_slices, plan.n_items), dim3(128),
                     0, s, p);
  if constexpr (!MULTI) {
    if (plan.chunk_tiles > 0)
      hipLaunchKernelGGL((attention_merge_kernel<TV, DS>), dim3(a.B * p.n_slices, plan.n_qt, 2 * kAttnQW / 4),
                         dim3(256), 0, s, p);
  }
}

template <typename TQ, typename TV, int RP>
static void launch_attn_1(const AttentionArgs& a, const AttnPlan& plan, AttnParams& p, hipStream_t s) {
  const bool multi = (a.flags & kAttnMix) && a.S > 1;
  if (plan.ds == 64) {
    if (multi) launch_attn_3<TQ, TV, RP, 64, true>(a, plan, p, s);
    else launch_attn_3<TQ, TV, RP, 64, false>(a, plan, p, s);
  } else if (plan.ds == 128) {
    if (multi) launch_attn_3<TQ, TV, RP, 128, true>(a, plan, p, s);
    else launch_attn_3<TQ, TV, RP, 128, false>(a, plan, p, s);
  } else {
    if constexpr (RP < 512) launch_attn_3<TQ, TV, RP, 256, false>(a, plan, p, s);
  }
}

template <typename TQ, typename TV>
static void launch_attn_0(const AttentionArgs& a, const AttnPlan& plan, AttnParams& p, hipStream_t s) {
  switch (a.RP) {
    case 64: launch_attn_1<TQ, TV, 64>(a, plan, p, s); break;
    case 128: launch_attn_1<TQ, TV, 128>(a, plan, p, s); break;
    case 256: launch_attn_1<TQ, TV, 256>(a, plan, p, s); break;
    default: launch_attn_1<TQ, TV, 512>(a, plan, p, s); break;
  }
}

// Key tiles of query tile qt of `length` tokens (host copy of key_tiles_of).
static int64_t host_key_tiles(int64_t qt, int64_t qtile, int64_t length, bool causal) {
  if (!causal) return (length + kKeyTile - 1) / kKeyTile;
  return (std::min(qt * qtile + qtile, length) - 1) / kKeyTile + 1;
}

AttnPlan plan_attention(int64_t B, int64_t S, int64_t T, int64_t D, int64_t RP, bool multi, bool causal,
                        bool allow_split) {
  AttnPlan plan{};
  const int64_t qtile = 2 * kAttnQW;
  plan.n_qt = static_cast<int>((T + qtile - 1) / qtile);
  // Value slice: as wide as possible (one score tile serves more value columns
  // and the softmax is shared by more MFMAs) while the grid keeps at least 256
  // workgroups.  The register budget caps it at 256 features, and at 128 with
  // the map mix (a second accumulator set) or 512-wide scores.
  const int64_t tiles = B * plan.n_qt;
  int64_t ds = std::min<int64_t>(D, (multi || RP == 512) ? 128 : 256);
  while (ds > 128 && tiles * (D / ds) < 256) ds /= 2;
  plan.ds = static_cast<int>(ds);
  const int64_t slices = D / ds;
  plan.n_items = plan.n_qt;
  plan.chunk_tiles = 0;
  // Long key ranges (one map only) on a grid that cannot fill the chip twice:
  // split them into chunks so that the grid holds enough workgroups for every
  // SIMD and the causal staircase is cut into pieces of similar length.
  // Chunks keep >= 32 key tiles: below that the partials' traffic and the
  // merge cost more than the balance gains.
  const int64_t most = host_key_tiles(plan.n_qt - 1, qtile, T, causal);
  if (allow_split && S == 1 && B * slices * plan.n_qt < 512 && most >= 64) {
    for (int64_t kc = 256; kc >= 32; kc /= 2) {
      if (kc >= most) continue;
      int64_t items = 0;
      for (int64_t qt = 0; qt < plan.n_qt; ++qt) items += (host_key_tiles(qt, qtile, T, causal) + kc - 1) / kc;
      plan.chunk_tiles = static_cast<int>(kc);
      plan.n_items = static_cast<int>(items);
      if (B * slices * items >= 512) break;
    }
  }
  plan.part_bytes = plan.chunk_tiles > 0 ? B * slices * plan.n_items * qtile * (ds + 2) * 4 : 0;
  return plan;
}

void launch_routed_attention(const AttentionArgs& a, void* partials, hipStream_t stream) {
  if (a.T == 0 || a.B == 0) return;
  const AttnPlan plan = plan_attention(a.B, a.S, a.T, a.D, a.RP, (a.flags & kAttnMix) && a.S > 1,
                                       a.flags & kAttnCausal, partials != nullptr);
  AttnParams p;
  p.part = static_cast<float*>(partials);
  p.q = a.q;
  p.k = a.k;
  p.qk_stride_b = a.qk_stride_b;
  p.qk_stride_t = a.qk_stride_t;
  p.map_stride = a.map_stride;
  p.map_repeat = a.map_repeat;
  p.vt = a.vt;
  p.vt_stride_b = a.vt_stride_b;
  p.S = a.S;
  p.T = a.T;
  p.D = static_cast<int>(a.D);
  p.scales = a.scales;
  p.scales_dtype = a.scales_dtype;
  p.scale_mult = a.scale_mult;
  p.mix_logits = a.mix_logits;
  p.mix_dtype = a.mix_dtype;
  p.flags = a.flags;
  p.score_bound = a.score_bound;
  p.out = a.out;
  p.out_stride_b = a.out_stride_b;
  p.out_stride_t = a.out_stride_t;
  p.out_stride_s = a.out_stride_s;
  if (a.qk_dtype == kF16 && a.v_dtype == kBF16) launch_attn_0<_Float16, __bf16>(a, plan, p, stream);
  else if (a.qk_dtype == kF16) launch_attn_0<_Float16, _Float16>(a, plan, p, stream);
  else launch_attn_0<__bf16, __bf16>(a, plan, p, stream);
}

}  // namespace da
