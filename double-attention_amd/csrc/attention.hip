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
constexpr int kAttnStages = 2; // stage buffers of the key/V^T ring

struct AttnParams {
  const void* q;
  const void* k;
  int64_t qk_stride_b, qk_stride_t, map_stride;
  int map_repeat;
  const void* vt;
  int64_t vt_stride_b;
  int S, T, D;
  int n_qt, n_slices;
  // Stream split (one map only): the key tiles of all query tiles of a
  // (sequence, slice), query tile by query tile, form one stream that
  // workgroup y covers from tile y*stream_len on, stream_len tiles.  0: one
  // workgroup per query tile, every map.
  int stream_len;
  int n_seg;           // workgroups per (sequence, slice) in the stream split
  float* part;         // per workgroup, two pieces: [QT][DS] normalized outputs, [QT] reference m, [QT] sums l
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

// Key tiles of query tile qt (QT queries).
__device__ __forceinline__ int key_tiles_of(const AttnParams& p, int qt, int QT) {
  if (!(p.flags & kAttnCausal)) return (p.T + kKeyTile - 1) / kKeyTile;
  return (min(qt * QT + QT, p.T) - 1) / kKeyTile + 1;
}
// The stream split orders the query tiles of a (sequence, slice) in pairs
// qt, n_qt-1-qt (0, n_qt-1, 1, n_qt-2, ...): a short causal tile next to a
// long one, so every run of the stream holds few units (each unit switch
// reloads the queries).  Stream unit i is query tile stream_qt(i).
__device__ __forceinline__ int stream_qt(const AttnParams& p, int i) {
  return (i & 1) ? p.n_qt - 1 - (i >> 1) : (i >> 1);
}
__device__ __forceinline__ int stream_index(const AttnParams& p, int qt) {
  return 2 * qt <= p.n_qt - 1 ? 2 * qt : 2 * (p.n_qt - 1 - qt) + 1;
}
// Key tiles of every pair (PS) and the shortfall d of pair 0, whose second
// tile is the last query tile (it may be partial): causal full tiles hold
// QT/32 (qt+1) key tiles, so a pair holds (QT/32)(n_qt+1).
__device__ __forceinline__ void stream_pairs(const AttnParams& p, int QT, int64_t& PS, int64_t& d) {
  if (!(p.flags & kAttnCausal)) {
    PS = 2 * static_cast<int64_t>(key_tiles_of(p, 0, QT));
    d = 0;
  } else {
    PS = static_cast<int64_t>(QT / kKeyTile) * (p.n_qt + 1);
    d = static_cast<int64_t>(QT / kKeyTile) * p.n_qt - key_tiles_of(p, p.n_qt - 1, QT);
  }
}
// Stream position of unit i's first key tile.
__device__ __forceinline__ int64_t tiles_before(const AttnParams& p, int i, int QT) {
  int64_t PS, d;
  stream_pairs(p, QT, PS, d);
  const int j = i >> 1;
  int64_t pos = static_cast<int64_t>(j) * PS - (j > 0 ? d : 0);
  if (i & 1) pos += key_tiles_of(p, j, QT);
  return pos;
}
// Stream unit holding stream tile gt.
__device__ __forceinline__ int stream_unit(const AttnParams& p, int64_t gt, int QT) {
  int64_t PS, d;
  stream_pairs(p, QT, PS, d);
  int64_t j = gt < PS - d ? 0 : 1 + (gt - (PS - d)) / PS;
  j = min<int64_t>(j, (p.n_qt - 1) / 2);
  int i = static_cast<int>(2 * j);
  if (i + 1 < p.n_qt && gt >= tiles_before(p, i + 1, QT)) ++i;
  return i;
}

template <int RP, int DS, int NW>
struct AttnTile {
  typedef PaddedTile<kKeyTile, RP / 8, true> KT;    // keys (blocked rows)
  typedef PaddedTile<DS, kKeyTile / 8, false> VT;   // V^T rows: DS features x 4 chunks
  static constexpr int KPW = (KT::LOADS + NW - 1) / NW;   // key loads per wave
  static constexpr int VPW = (VT::LOADS + NW - 1) / NW;   // V^T loads per wave
  static constexpr int BYTES = KT::BYTES + VT::BYTES;     // one stage: a key tile, then a V^T tile
};

// A workgroup walks a run of key tiles u = 0 .. total-1 (the maps of one
// query tile, or a stretch of the stream split).  A ring of NST stage buffers: stage u (buffer u % NST) holds the keys of tile
// u+1 and the V^T of tile u, so step u forms the scores of tile u+1 (MFMA)
// while it turns the scores of tile u into probabilities (VALU) and
// accumulates P(u) V(u) (MFMA): the softmax of one tile runs in the shadow of
// the next tile's score MFMAs.  Step u also issues stage u+NST-1 into the
// buffer stage u-1 used, so every stage has NST-1 steps to land.
template <typename TQ, typename TV, int RP, int DS, int NW, int NST, bool MULTI>
__global__ __launch_bounds__(NW * 64, 1) void attention_kernel(AttnParams p) {
  static_assert(NST == 2 || NST == 3, "two or three stage buffers");
  typedef AttnTile<RP, DS, NW> Tile;
  typedef typename Tile::KT KT;
  typedef typename Tile::VT VT;
  typedef typename Elem<TQ>::v8 q8;
  typedef typename Elem<TV>::v8 v8;
  constexpr int KS = RP / 32;
  constexpr int NB = DS / 16;    // accumulator blocks per query block
  constexpr int NL = Tile::KPW + Tile::VPW;
  constexpr int QT = NW * kAttnQW;
  __shared__ __attribute__((aligned(1024))) char lds[NST * Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int b = static_cast<int>(blockIdx.x) / p.n_slices;
  const int ds0 = (static_cast<int>(blockIdx.x) - b * p.n_slices) * DS;   // first feature of the slice
  const bool causal = p.flags & kAttnCausal;
  // The workgroup's work is a run of `total` key tiles over consecutive
  // units: maps s of query tile n_qt-1-y (heaviest first), or in the stream
  // split the query tiles of stream tiles [y*stream_len, ...).  The run starts
  // at key tile kt_first of unit unit_first.
  const bool stream = p.stream_len > 0;
  const int qt_maps = p.n_qt - 1 - static_cast<int>(blockIdx.y);
  const int n_kt_maps = key_tiles_of(p, qt_maps, QT);
  int unit_first = 0, kt_first = 0, total;
  if (stream) {
    const int64_t g0 = static_cast<int64_t>(blockIdx.y) * p.stream_len;
    const int last = p.n_qt - 1;
    const int64_t all = tiles_before(p, last, QT) + key_tiles_of(p, stream_qt(p, last), QT);
    unit_first = stream_unit(p, g0, QT);
    kt_first = static_cast<int>(g0 - tiles_before(p, unit_first, QT));
    total = static_cast<int>(min<int64_t>(p.stream_len, all - g0));
  } else {
    total = p.S * n_kt_maps;
  }
  // Units: key tiles, query tile and map.
  auto unit_tiles = [&](int unit) { return stream ? key_tiles_of(p, stream_qt(p, unit), QT) : n_kt_maps; };
  auto unit_qt = [&](int unit) { return stream ? stream_qt(p, unit) : qt_maps; };
  auto unit_map = [&](int unit) { return stream ? 0 : unit; };

  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b;
  const char* kbase = reinterpret_cast<const char*>(static_cast<const TQ*>(p.k) + b * p.qk_stride_b);
  // Feature d of a 32-token V^T tile sits at 32*d, so the slice is one block.
  const char* vbase = reinterpret_cast<const char*>(static_cast<const TV*>(p.vt) + b * p.vt_stride_b + 32 * ds0);
  const int kstride = static_cast<int>(p.qk_stride_t) * static_cast<int>(sizeof(TQ));   // bytes per key row

  // Per-lane DMA sources of this wave's loads: key load i fills wave load
  // i*NW + wave of the key tile (koff: byte offset of the lane's chunk from
  // row 0; kchunk: the chunk's offset inside its row, so that rows past the
  // last key clamp to it as min(koff, last*kstride + kchunk)), V^T load i the
  // same wave load of the V^T tile (byte offset inside the tile).  Wave loads
  // past a tile's end re-load the data of wave load 0 into slot 0 of that tile.
  uint32_t koff[Tile::KPW], kchunk[Tile::KPW], vdesc[Tile::VPW];
#pragma unroll
  for (int i = 0; i < Tile::KPW; ++i) {
    int row, ck;
    const int j = i * NW + wave;
    KT::slot_chunk((j < KT::LOADS ? j : 0) * 64 + lane, row, ck);
    kchunk[i] = static_cast<uint32_t>(ck * 16);
    koff[i] = static_cast<uint32_t>(row * kstride) + kchunk[i];
  }
#pragma unroll
  for (int i = 0; i < Tile::VPW; ++i) {
    int row, ck;
    const int j = i * NW + wave;
    VT::slot_chunk((j < VT::LOADS ? j : 0) * 64 + lane, row, ck);
    vdesc[i] = static_cast<uint32_t>((row * kKeyTile + ck * 8) * sizeof(TV));
  }
  // LDS slot of this wave's load n inside a stage (key loads first): a
  // constant plus wave*1024, except for the wave loads past a tile's end.
  const int wave_slot = wave * 1024;
  auto slot_of = [&](int n) {
    if (n < Tile::KPW) {
      if (n * NW + NW - 1 < KT::LOADS) return n * NW * 1024 + wave_slot;
      return n * NW + wave < KT::LOADS ? n * NW * 1024 + wave_slot : 0;
    }
    const int i = n - Tile::KPW;
    if (i * NW + NW - 1 < VT::LOADS) return KT::BYTES + i * NW * 1024 + wave_slot;
    return KT::BYTES + (i * NW + wave < VT::LOADS ? i * NW * 1024 + wave_slot : 0);
  };
  // DMA sources of one stage: row 0 of a key tile, the last key row it may
  // read (rows past the end re-read it) and the V^T tile.
  struct Src {
    const char* k;
    const char* v;
    int last;
  };
  // Cursors over the key tiles and V^T tiles still to be loaded, in run
  // order; each issue takes the next one, and past the end of the run the
  // last tile is loaded again.  Key tiles follow the map's branch: maps s and
  // s+1 share it while (s+1) % map_repeat != 0.
  const int64_t ktile_bytes = static_cast<int64_t>(kKeyTile) * kstride;
  const int64_t vtile_bytes = static_cast<int64_t>(kKeyTile) * p.D * static_cast<int64_t>(sizeof(TV));
  const int64_t kmap_bytes = p.map_stride * static_cast<int64_t>(sizeof(TQ));
  // Each cursor: unit, key tile, the unit's tile count, advances left, and
  // the tile's address (keys: also the last row it may read).
  struct Cursor {
    int unit, kt, n, left;
  };
  Cursor kc{unit_first, kt_first, unit_tiles(unit_first), total - 1};
  Cursor vc = kc;
  const char* kmap = kbase;       // row 0 of the key cursor's map
  const char* kptr = kbase + kt_first * ktile_bytes;
  int klast = p.T - 1 - kt_first * kKeyTile;
  int krep = 0;
  const char* vptr = vbase + kt_first * vtile_bytes;
  // Advances a cursor; true when it moved to the next unit (at key tile 0).
  auto advance = [&](Cursor& cu) {
    if (cu.left == 0) return false;
    --cu.left;
    if (++cu.kt == cu.n) {
      cu.kt = 0;
      cu.n = unit_tiles(++cu.unit);
      return true;
    }
    return false;
  };
  auto next_key = [&]() {
    const Src src{kptr, nullptr, klast};
    if (kc.left > 0) {
      if (advance(kc)) {
        if (!stream && ++krep == p.map_repeat) {
          krep = 0;
          kmap += kmap_bytes;
        }
        kptr = kmap;
        klast = p.T - 1;
      } else {
        kptr += ktile_bytes;
        klast -= kKeyTile;
      }
    }
    return src;
  };
  auto next_value = [&]() {
    const char* v = vptr;
    if (vc.left > 0) vptr = advance(vc) ? vbase : vptr + vtile_bytes;
    return v;
  };
  auto issue_one = [&](char* buf, const Src& src, int n) {
    if (n < Tile::KPW) {
      const uint32_t lim = static_cast<uint32_t>(src.last * kstride) + kchunk[n];
      dma16(uniform_ptr(src.k) + min(koff[n], lim), buf + slot_of(n));
    } else {
      dma16(uniform_ptr(src.v) + vdesc[n - Tile::KPW], buf + slot_of(n));
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

  // Query fragments of map s for the wave's queries qw .. qw+31; returns the
  // map's score multiplier (log2 domain).  The rescale test compares maxima
  // of raw scores, so a negative score scale is folded into the queries
  // instead (negation is exact).
  auto load_queries = [&](int s, int qw) {
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride;
    const float gamma = map_gamma(p, s);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw + cb * 16 + c;
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

  // Prologue: keys of tile 0 into the last buffer's key slot, stages
  // 0 .. NST-2 = {K(j+1), V(j)} into buffers 0 .. NST-2; the queries of map 0
  // load meanwhile (one memory round trip for both).
  {
    const Src s0 = next_key();
#pragma unroll
    for (int n = 0; n < Tile::KPW; ++n) issue_one(lds + (NST - 1) * Tile::BYTES, s0, n);
#pragma unroll
    for (int j = 0; j < NST - 1; ++j) {
      Src sj = next_key();
      sj.v = next_value();
#pragma unroll
      for (int n = 0; n < NL; ++n) issue_one(lds + j * Tile::BYTES, sj, n);
    }
  }
  int qw0 = unit_qt(unit_first) * QT + wave * kAttnQW;   // this wave's first query in the current unit
  float sc = load_queries(unit_map(unit_first), qw0);
  float sc_next = sc;
  wait_vmem();
  __syncthreads();
  f32x4 st_prev[2][2];
  scores(lds + (NST - 1) * Tile::BYTES, st_prev, std::false_type{}, nullptr, Src{});
  int cur_off = 0;                              // buffer of stage u
  int nxt_off = (NST - 1) * Tile::BYTES;        // buffer of stage u-1: target of stage u+NST-1

  // One pipelined step: tile u is key tile kt of the current unit.  FIXED:
  // every score is bounded by score_bound, so exponents use the fixed
  // reference score_bound*sc (all probabilities <= 1) and the accumulators
  // are never rescaled; otherwise the lazy online rescale runs.  `opens`:
  // tile u+1 is the first of unit `next`, whose queries this step's scores
  // need.
  auto step = [&](auto fixed, int kt, bool opens, int next) {
    constexpr bool FIXED = decltype(fixed)::value;
    char* cur = lds + cur_off;
    char* nxt = lds + nxt_off;
    const int k0 = kt * kKeyTile;
    if (opens) sc_next = load_queries(unit_map(next), unit_qt(next) * QT + wave * kAttnQW);
    // Stage u + NST - 1 = {K(u + NST), V(u + NST - 1)}.
    Src src = next_key();
    src.v = next_value();

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

    // Stage u has landed once at most the NST - 2 later stages are in flight.
    wait_vmem_at_most<(NST - 2) * NL>();
    __syncthreads();

    // Fragment reads come before the stage loads in program order where the
    // registers allow: the loads write LDS, so the compiler keeps every later
    // LDS read behind them.  Up to eight key steps and eight V^T blocks are
    // read up front; 512-wide scores read their keys in groups of four steps,
    // each two steps ahead of its first use, and their V^T blocks after the
    // scores.  The loads are spread over the second half of the score MFMAs.
    constexpr int KG = KS <= 8 ? KS : 4;
    constexpr int KLEAD = 2;
    constexpr int VA = KS <= 8 ? (NB < 8 ? NB : 8) : 0;
    const char* kf = cur + kfrag;
    const char* vf = cur + vfrag;
    q8 kfr[KS][2];
    v8 vfr[NB];
    auto read_keys = [&](int kk) {
      kfr[kk][0] = lds_v8<TQ>(kf + KT::offset(0, kk * 4));
      kfr[kk][1] = lds_v8<TQ>(kf + KT::offset(16, kk * 4));
    };
#pragma unroll
    for (int kk = 0; kk < KG; ++kk) read_keys(kk);
#pragma unroll
    for (int db = 0; db < VA; ++db) vfr[db] = lds_v8<TV>(vf + VT::offset(db * 16, 0));

    f32x4 st_new[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) st_new[cb][0] = st_new[cb][1] = zero4();
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (KG < KS && kk + KLEAD >= KG && kk + KLEAD < KS && (kk + KLEAD) % KG == 0) {
#pragma unroll
        for (int k2 = kk + KLEAD; k2 < kk + KLEAD + KG; ++k2) read_keys(k2);
      }
      constexpr int D0 = KS / 2;
#pragma unroll
      for (int n = 0; n < NL; ++n)
        if (kk >= D0 && D0 + n * (KS - D0) / NL == kk) issue_one(nxt, src, n);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        st_new[cb][0] = Elem<TQ>::mma(kfr[kk][0], qf[cb][kk], st_new[cb][0]);
        st_new[cb][1] = Elem<TQ>::mma(kfr[kk][1], qf[cb][kk], st_new[cb][1]);
      }
    }
#pragma unroll
    for (int db = VA; db < NB; ++db) vfr[db] = lds_v8<TV>(vf + VT::offset(db * 16, 0));

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
#pragma unroll
    for (int db = 0; db < NB; ++db) {
      acc[0][db] = Elem<TV>::mma(vfr[db], pb[0], acc[0][db]);
      acc[1][db] = Elem<TV>::mma(vfr[db], pb[1], acc[1][db]);
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      st_prev[cb][0] = st_new[cb][0];
      st_prev[cb][1] = st_new[cb][1];
    }
    nxt_off = cur_off;
    cur_off = cur_off + Tile::BYTES == NST * Tile::BYTES ? 0 : cur_off + Tile::BYTES;
  };

  int unit = unit_first, kt_start = kt_first, left = total;
  while (left > 0) {
    const int n_unit = unit_tiles(unit);
    const int n_here = min(n_unit - kt_start, left);
    const bool more = left > n_here;
    const int s = unit_map(unit);
    // The fixed reference keeps every probability within the range of the
    // operand type: bf16 holds 2^-120 .. 1 exactly in exponent; fp16 does not.
    const bool fixed = p.score_bound > 0.f && sizeof(TV) == 2 && !std::is_same<TV, _Float16>::value &&
                       2.f * p.score_bound * sc <= 120.f;
    if (fixed) {
      for (int i = 0; i < n_here; ++i) step(std::true_type{}, kt_start + i, more && i == n_here - 1, unit + 1);
    } else {
      for (int i = 0; i < n_here; ++i) step(std::false_type{}, kt_start + i, more && i == n_here - 1, unit + 1);
    }
    const float wmap = map_weight(p, s);
    // A piece of a query tile's key range (stream split) stores its normalized
    // outputs, reference and row sums in fp32 for the merge kernel: slot 0 if
    // it is the run's first unit, else slot 1.  Otherwise the unit's output
    // goes to its slot (or into the mix).
    const bool partial = kt_start > 0 || n_here < n_unit;
    float* part = p.part + ((static_cast<int64_t>(blockIdx.x) * p.n_seg + blockIdx.y) * 2 + (unit == unit_first ? 0 : 1)) *
                               (QT * (DS + 2));
    const int q0 = unit_qt(unit) * QT;
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
    left -= n_here;
    ++unit;
    kt_start = 0;
    qw0 = unit_qt(unit) * QT + wave * kAttnQW;
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

// Merge of a query tile split over stream workgroups: out = sum_c 2^(m_c - M)
// l_c o_c / sum_c 2^(m_c - M) l_c over its pieces c, o_c the piece's
// normalized output, M = max_c m_c, per query row (one map, weight 1).  The
// tile's first stream tile is P; its pieces sit in workgroups y0 = P / L ..
// y1 = (P + n - 1) / L, in slot 1 of y0 when the tile does not open y0's run,
// else slot 0.  Each wave takes one query row, its lanes covering consecutive
// features, so every partial row is read by one coalesced sweep.
template <typename TV, int DS, int QT>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnParams p) {
  const int qt = static_cast<int>(blockIdx.y);
  const int64_t P = tiles_before(p, stream_index(p, qt), QT);
  const int n = key_tiles_of(p, qt, QT);
  const int y0 = static_cast<int>(P / p.stream_len);
  const int y1 = static_cast<int>((P + n - 1) / p.stream_len);
  if (y0 == y1) return;   // written directly by its workgroup
  const int b = static_cast<int>(blockIdx.x) / p.n_slices;
  const int ds0 = (static_cast<int>(blockIdx.x) - b * p.n_slices) * DS;
  constexpr int ITEM = QT * (DS + 2);
  auto piece = [&](int y) {
    const int slot = (y == y0 && P != static_cast<int64_t>(y0) * p.stream_len) ? 1 : 0;
    return p.part + ((static_cast<int64_t>(blockIdx.x) * p.n_seg + y) * 2 + slot) * ITEM;
  };
  const int lane = lane_id();
  // blockIdx.z picks four query rows of the tile, one per wave.
  const int ql = static_cast<int>(blockIdx.z) * 4 + (static_cast<int>(threadIdx.x) >> 6);
  const int tq = qt * QT + ql;
  if (tq >= p.T) return;
  constexpr int NV = DS / 256 > 0 ? DS / 256 : 1;   // 4-feature vectors per lane
  float M = -INFINITY;
  for (int y = y0; y <= y1; ++y) M = fmaxf(M, piece(y)[QT * DS + ql]);
  f32x4 o[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) o[k] = zero4();
  float den = 0.f;
  for (int y = y0; y <= y1; ++y) {
    const float* pc = piece(y);
    const float m = pc[QT * DS + ql];
    const float wl = (m == -INFINITY ? 0.f : exp2f(m - M)) * pc[QT * DS + QT + ql];
    den += wl;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int d4 = (k * 64 + lane) * 4;
      if (d4 < DS) o[k] += wl * *reinterpret_cast<const f32x4*>(pc + ql * DS + d4);
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  TV* orow = static_cast<TV*>(p.out) + b * p.out_stride_b + static_cast<int64_t>(tq) * p.out_stride_t + ds0;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int d4 = (k * 64 + lane) * 4;
    if (d4 < DS) {
      typename Elem<TV>::v4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = static_cast<TV>(o[k][i] * inv);
      *reinterpret_cast<typename Elem<TV>::v4*>(orow + d4) = v;
    }
  }
}

template <typename TQ, typename TV, int RP, int DS, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, const AttnPlan& plan, AttnParams& p, hipStream_t s) {
  // 512-wide scores take a whole CU's LDS per workgroup: four waves (128
  // queries) share each key / V^T tile so every SIMD is busy.
  constexpr int NW = RP == 512 ? 4 : 2;
  constexpr int QT = NW * kAttnQW;
  p.n_slices = a.D / DS;
  p.n_qt = plan.n_qt;
  p.stream_len = plan.stream_len;
  p.n_seg = plan.n_seg;
  const int gy = plan.stream_len > 0 ? plan.n_seg : plan.n_qt;
  hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, NW, kAttnStages, MULTI>), dim3(a.B * p.n_slices, gy),
                     dim3(NW * 64), 0, s, p);
  if constexpr (!MULTI) {
    if (plan.stream_len > 0)
      hipLaunchKernelGGL((attention_merge_kernel<TV, DS, QT>), dim3(a.B * p.n_slices, plan.n_qt, QT / 4), dim3(256), 0,
                         s, p);
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

// Host copy of key_tiles_of, and the key tiles of all query tiles.
static int64_t host_key_tiles(int64_t qt, int64_t qtile, int64_t length, bool causal) {
  if (!causal) return (length + kKeyTile - 1) / kKeyTile;
  return (std::min(qt * qtile + qtile, length) - 1) / kKeyTile + 1;
}
static int64_t host_all_tiles(int64_t n_qt, int64_t qtile, int64_t length, bool causal) {
  if (!causal) return n_qt * host_key_tiles(0, qtile, length, false);
  return qtile / kKeyTile * (n_qt - 1) * n_qt / 2 + host_key_tiles(n_qt - 1, qtile, length, true);
}

// MI355X: 256 CUs of 160 KiB LDS; every attention variant holds more than 256
// registers per lane, so a SIMD runs one wave.
constexpr int64_t kCUs = 256;
constexpr int64_t kLdsBytes = 160 * 1024;

AttnPlan plan_attention(int64_t B, int64_t S, int64_t T, int64_t D, int64_t RP, bool multi, bool causal,
                        bool allow_split) {
  AttnPlan plan{};
  const int64_t nw = RP == 512 ? 4 : 2;
  const int64_t qtile = nw * kAttnQW;
  plan.nw = static_cast<int>(nw);
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
  // Stream split (one map only): when the longest query tile holds more key
  // tiles than an even share of the whole problem over the workgroups that
  // run at once, cut every (sequence, slice)'s stream of key tiles into runs
  // of that share (at least 16 tiles, so the prologue and the partials stay
  // small next to the run).
  const int64_t stage = (RP / 8 + 1) * 32 * 16 + ds * 5 * 16;   // one key + V^T stage, padded
  const int64_t stage_bytes = (stage + 1023) / 1024 * 1024;
  const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(4 / nw, kLdsBytes / (kAttnStages * stage_bytes)));
  const int64_t last = plan.n_qt - 1;
  const int64_t stream_all = host_all_tiles(plan.n_qt, qtile, T, causal);
  const int64_t longest = host_key_tiles(last, qtile, T, causal);
  const int64_t share = std::max<int64_t>(16, (B * slices * stream_all + kCUs * per_cu - 1) / (kCUs * per_cu));
  plan.stream_len = 0;
  plan.n_seg = 0;
  if (allow_split && S == 1 && !multi && longest > share) {
    plan.stream_len = static_cast<int>(share);
    plan.n_seg = static_cast<int>((stream_all + share - 1) / share);
  }
  plan.part_bytes = plan.stream_len > 0 ? B * slices * plan.n_seg * 2 * qtile * (ds + 2) * 4 : 0;
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
