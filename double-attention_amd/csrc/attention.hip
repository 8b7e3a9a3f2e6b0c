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
// A workgroup of NW waves (2 or 4) owns 32*NW/SUB query rows of one sequence
// (SUB sub-streams share the same queries, below) and a slice of DS value
// features; every wave owns 32 queries (two 16-column MFMA blocks) and the
// whole slice, so no score tile is formed twice inside a sub-stream.  The
// value width is split over workgroups (DS <= 128), which bounds a wave's O^T
// accumulators and multiplies the workgroups of small grids; the variants the
// module uses still hold more than 256 registers per lane (query, key and
// score fragments beside the accumulators), one wave per SIMD.  A wave walks the
// (map, 32-key tile) sequence up to the causal bound in the transposed domain:
//   S^T[key, q] = sum_r K[key, r] Q^T[r, q]      (A = key rows from LDS, B = queries in VGPRs)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P in VGPRs)
// so P never leaves registers, and every A fragment read from LDS feeds two
// MFMAs (the two query blocks).  Key and V^T tiles are double-buffered in
// XOR-swizzled LDS tiles (da_tile.h) filled by global->LDS DMA; the loads of the next
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
  // Stream split (one map, or the map mix): the key tiles of every (query
  // tile, map) unit of a (sequence, slice) form one stream that workgroup y
  // covers from tile y*stream_len on, stream_len tiles.  0: one workgroup per
  // query tile, every map.
  int stream_len;
  int n_seg;           // workgroups per (sequence, slice) in the stream split
  // Per workgroup of the stream split, slots of attn_slot_bytes(QT, DS, es)
  // bytes: two unit pieces ([QT][DS] normalized outputs, es bytes each, then
  // [QT] reference m and [QT] sums l in fp32) and, with the map mix, two
  // partial mixes ([QT][DS] outputs).  es is 2 (the value dtype; the outputs
  // are bounded by max |V|) unless the call asks for fp32 outputs (4).
  char* part;
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

// Piece element bytes of a call, and the bytes of one slot.
__host__ __device__ inline int attn_piece_bytes(int flags) { return (flags & kAttnOutF32) ? 4 : 2; }
__host__ __device__ inline int64_t attn_slot_bytes(int QT, int DS, int es) {
  return static_cast<int64_t>(QT) * DS * es + 8 * static_cast<int64_t>(QT);
}

// Store four normalized outputs of a piece (or a partial mix) at element
// offset `at`, in fp32 or in the value dtype.
template <typename TV, int es>
__device__ __forceinline__ void store_piece4(char* slot, int at, f32x4 v) {
  if constexpr (es == 4) {
    *reinterpret_cast<f32x4*>(slot + 4 * at) = v;
  } else {
    typename Elem<TV>::v4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<TV>(v[i]);
    *reinterpret_cast<typename Elem<TV>::v4*>(slot + 2 * at) = o;
  }
}
template <typename TV, int es>
__device__ __forceinline__ f32x4 load_piece4(const char* slot, int at) {
  if constexpr (es == 4) return *reinterpret_cast<const f32x4*>(slot + 4 * at);
  const typename Elem<TV>::v4 v = *reinterpret_cast<const typename Elem<TV>::v4*>(slot + 2 * at);
  return f32x4{static_cast<float>(v[0]), static_cast<float>(v[1]), static_cast<float>(v[2]), static_cast<float>(v[3])};
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
  const int64_t at = b * p.out_stride_b + static_cast<int64_t>(t) * p.out_stride_t + s * p.out_stride_s + d0;
  if (p.flags & kAttnOutF32) {
    float* orow = static_cast<float*>(p.out) + at;
#pragma unroll
    for (int db = 0; db < DC / 16; ++db) *reinterpret_cast<f32x4*>(orow + db * 16 + 4 * g) = acc[db] * w;
    return;
  }
  T* orow = static_cast<T*>(p.out) + at;
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
// Query-tile stream index holding query-tile stream tile gt.
__device__ __forceinline__ int stream_unit(const AttnParams& p, int64_t gt, int QT) {
  int64_t PS, d;
  stream_pairs(p, QT, PS, d);
  int64_t j = gt < PS - d ? 0 : 1 + (gt - (PS - d)) / PS;
  j = min<int64_t>(j, (p.n_qt - 1) / 2);
  int i = static_cast<int>(2 * j);
  if (i + 1 < p.n_qt && gt >= tiles_before(p, i + 1, QT)) ++i;
  return i;
}

// With S maps every query tile contributes S consecutive units (its maps in
// order), so unit u = qi*S + s of query-tile stream index qi starts at
// S * tiles_before(qi) + s * (key tiles of the query tile).
__device__ __forceinline__ int64_t unit_start(const AttnParams& p, int u, int QT) {
  const int qi = u / p.S;
  const int s = u - qi * p.S;
  return p.S * tiles_before(p, qi, QT) + static_cast<int64_t>(s) * key_tiles_of(p, stream_qt(p, qi), QT);
}
__device__ __forceinline__ int unit_of_tile(const AttnParams& p, int64_t gt, int QT) {
  const int qi = stream_unit(p, gt / p.S, QT);
  const int64_t a = p.S * tiles_before(p, qi, QT);
  return qi * p.S + static_cast<int>((gt - a) / key_tiles_of(p, stream_qt(p, qi), QT));
}

template <int RP, int DS, int NW>
struct AttnTile {
  typedef XorTile<kKeyTile, RP / 8, true> KT;       // keys (blocked rows)
  typedef XorTile<DS, 4, false> VT;                 // V^T rows: DS features x 4 chunks (32 tokens)
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
//
// SUB = 2 splits a workgroup's run between two sub-streams of NW/2 waves each
// (the same queries): with one map the even and odd key tiles, with several
// maps the even and odd maps.  Each sub-stream has its own key / V^T tiles in
// every stage and the two step in lockstep (the shorter one pads with fully
// masked tiles); at the end the odd sub-stream hands its accumulators over
// LDS to the even one, which merges and stores.  A small grid so keeps every
// SIMD of a CU busy, and long map mixes finish in half the steps.
template <typename TQ, typename TV, int RP, int DS, int NW, int NST, bool MULTI, int SUB, int PIECE = 2>
__global__ __launch_bounds__(NW * 64, 1) void attention_kernel(AttnParams p) {
  static_assert(NST == 2 || NST == 3, "two or three stage buffers");
  static_assert(SUB == 1 || SUB == 2, "one or two sub-streams");
  constexpr int NQW = NW / SUB;   // waves of one sub-stream (its query waves)
  typedef AttnTile<RP, DS, NQW> Tile;
  typedef typename Tile::KT KT;
  typedef typename Tile::VT VT;
  typedef typename Elem<TQ>::v8 q8;
  typedef typename Elem<TV>::v8 v8;
  constexpr int KS = RP / 32;
  constexpr int NB = DS / 16;    // accumulator blocks per query block
  constexpr int NL = Tile::KPW + Tile::VPW;
  constexpr int QT = NQW * kAttnQW;
  constexpr int SBYTES = SUB * Tile::BYTES;   // one stage: each sub-stream's key tile and V^T tile
  __shared__ __attribute__((aligned(1024))) char lds[NST * SBYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  // Per-map constants, lane s holding map s (S <= 64; lanes past S repeat
  // map S-1): the raw score scale and mix logit.  Issued first and without
  // branches, so their round trip overlaps the set-up.
  const int map_lane = min(lane, p.S - 1);
  ScalarHalves scale_raw = fetch_scalar(p.scales, p.scales_dtype, map_lane);
  const bool mix_logits = (p.flags & kAttnMix) && p.mix_logits != nullptr;
  ScalarHalves mix_raw = fetch_scalar(mix_logits ? p.mix_logits : p.scales,
                                      mix_logits ? p.mix_dtype : p.scales_dtype, map_lane);
  auto lane_value = [](float v, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i)); };
  // Score scale gamma_s (clamped exp of the log scale, times scale_mult) and
  // mix weight alpha_s (softmax of the logits, or 1/S) of map s.
  auto gamma_of = [&](int s) {
    float v = lane_value(scalar_value(scale_raw, p.scales_dtype), s);
    if (p.flags & kAttnScalesAreLog) v = expf(fminf(fmaxf(v, kLogScaleMin), kLogScaleMax));
    return v * p.scale_mult;
  };
  auto weight_of = [&](int s) {
    if (!(p.flags & kAttnMix)) return 1.f;
    if (!mix_logits) return 1.f / static_cast<float>(p.S);
    const float logit = scalar_value(mix_raw, p.mix_dtype);
    float mx = -INFINITY;
    for (int i = 0; i < p.S; ++i) mx = fmaxf(mx, lane_value(logit, i));
    float den = 0.f;
    for (int i = 0; i < p.S; ++i) den += expf(lane_value(logit, i) - mx);
    return expf(lane_value(logit, s) - mx) / den;
  };
  const int sub = SUB == 1 ? 0 : uniform_wave() / NQW;
  const int wave = uniform_wave() - sub * NQW;    // query wave inside the sub-stream
  char* const lds_sub = lds + sub * Tile::BYTES;  // the sub-stream's share of stage 0
  // XCD-aware placement: workgroups are dispatched x-fastest and dealt to
  // the XCDs round-robin, so each XCD takes one contiguous range of the
  // logical order (sequence, y, slice): the workgroups of a sequence share an
  // XCD, whose L2 then fetches its key and V^T tiles once.  gx = b*n_slices +
  // slice and gy take the roles of the grid's x and y.
  const int n_wg = static_cast<int>(gridDim.x * gridDim.y);
  const int wg = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x);
  const int xcd = wg % kXcds, per_xcd = n_wg / kXcds, rem_xcd = n_wg % kXcds;
  const int logical = xcd * per_xcd + min(xcd, rem_xcd) + wg / kXcds;
  const int gy_b = logical / p.n_slices;
  const int gy = gy_b % static_cast<int>(gridDim.y);
  const int b = gy_b / static_cast<int>(gridDim.y);
  const int gx = b * p.n_slices + (logical - gy_b * p.n_slices);
  const int ds0 = (gx - b * p.n_slices) * DS;   // first feature of the slice
  const bool causal = p.flags & kAttnCausal;
  // The workgroup's work is a run of `total` key tiles over consecutive
  // units: maps s of query tile n_qt-1-y (heaviest first), or in the stream
  // split the query tiles of stream tiles [y*stream_len, ...).  The run starts
  // at key tile kt_first of unit unit_first.
  const bool stream = SUB == 1 && p.stream_len > 0;
  const int qt_maps = p.n_qt - 1 - gy;
  const int n_kt_maps = key_tiles_of(p, qt_maps, QT);
  // Sub-streams of one map step over every second key tile (kt_stride 2).
  const bool split_tiles = SUB == 2 && p.S == 1;
  const int kt_stride = split_tiles ? 2 : 1;
  int unit_first = 0, kt_first = 0, total, real;
  if (SUB == 2) {
    // Both sub-streams take `total` steps; the first `real` are theirs.  A
    // sub-stream without a tile of its own points its loads at tile 0.
    if (split_tiles) {
      kt_first = min(sub, n_kt_maps - 1);
      total = (n_kt_maps + 1) / 2;
      real = (n_kt_maps - sub + 1) / 2;
    } else {
      total = (p.S + 1) / 2 * n_kt_maps;
      real = (p.S - sub + 1) / 2 * n_kt_maps;
    }
  } else if (stream) {
    const int64_t g0 = static_cast<int64_t>(gy) * p.stream_len;
    const int last = p.n_qt - 1;
    const int64_t all = p.S * (tiles_before(p, last, QT) + key_tiles_of(p, stream_qt(p, last), QT));
    unit_first = unit_of_tile(p, g0, QT);
    kt_first = static_cast<int>(g0 - unit_start(p, unit_first, QT));
    total = static_cast<int>(min<int64_t>(p.stream_len, all - g0));
    real = total;
  } else {
    total = p.S * n_kt_maps;
    real = total;
  }
  // Units: tiles (of this sub-stream), query tile and map.
  auto unit_qt = [&](int unit) { return stream ? stream_qt(p, p.S == 1 ? unit : unit / p.S) : qt_maps; };
  auto unit_tiles = [&](int unit) {
    return stream ? key_tiles_of(p, unit_qt(unit), QT) : split_tiles ? real : n_kt_maps;
  };
  auto unit_map = [&](int unit) {
    if (stream) return p.S == 1 ? 0 : unit % p.S;
    return SUB == 2 ? min(sub + 2 * unit, p.S - 1) : unit;
  };

  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b;
  const char* kbase = reinterpret_cast<const char*>(static_cast<const TQ*>(p.k) + b * p.qk_stride_b);
  // Feature d of a 32-token V^T tile sits at 32*d, so the slice is one block.
  const char* vbase = reinterpret_cast<const char*>(static_cast<const TV*>(p.vt) + b * p.vt_stride_b + 32 * ds0);
  const int kstride = static_cast<int>(p.qk_stride_t) * static_cast<int>(sizeof(TQ));   // bytes per key row

  // Per-lane DMA sources of this wave's loads: key load i fills wave load
  // i*NQW + wave of the key tile (koff: byte offset of the lane's chunk from
  // row 0; kchunk: the chunk's offset inside its row, so that rows past the
  // last key clamp to it as min(koff, last*kstride + kchunk)), V^T load i the
  // same wave load of the V^T tile (byte offset inside the tile).  Wave loads
  // past a tile's end re-load the data of wave load 0 into slot 0 of that tile.
  uint32_t koff[Tile::KPW], kchunk[Tile::KPW], vdesc[Tile::VPW];
#pragma unroll
  for (int i = 0; i < Tile::KPW; ++i) {
    int row, ck;
    const int j = i * NQW + wave;
    KT::slot_chunk((j < KT::LOADS ? j : 0) * 64 + lane, row, ck);
    kchunk[i] = static_cast<uint32_t>(ck * 16);
    koff[i] = static_cast<uint32_t>(row * kstride) + kchunk[i];
  }
#pragma unroll
  for (int i = 0; i < Tile::VPW; ++i) {
    int row, ck;
    const int j = i * NQW + wave;
    VT::slot_chunk((j < VT::LOADS ? j : 0) * 64 + lane, row, ck);
    vdesc[i] = static_cast<uint32_t>((row * kKeyTile + ck * 8) * sizeof(TV));
  }
  // LDS slot of this wave's load n inside a stage (key loads first): a
  // constant plus wave*1024, except for the wave loads past a tile's end.
  const int wave_slot = wave * 1024;
  auto slot_of = [&](int n) {
    if (n < Tile::KPW) {
      if (n * NQW + NQW - 1 < KT::LOADS) return n * NQW * 1024 + wave_slot;
      return n * NQW + wave < KT::LOADS ? n * NQW * 1024 + wave_slot : 0;
    }
    const int i = n - Tile::KPW;
    if (i * NQW + NQW - 1 < VT::LOADS) return KT::BYTES + i * NQW * 1024 + wave_slot;
    return KT::BYTES + (i * NQW + wave < VT::LOADS ? i * NQW * 1024 + wave_slot : 0);
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
  // One cursor walks the run's tiles in order: unit, key tile, the unit's
  // tile count, advances left (past the end of the run the last tile is
  // loaded again), and the tile's key row 0, last readable key row and V^T
  // tile.  A stage pairs the keys of one tile with the V^T of the tile before
  // (vlag).
  int cu_unit = unit_first, cu_kt = 0, cu_n = unit_tiles(unit_first), cu_left = real - 1;
  if (!split_tiles) cu_kt = kt_first;
  // Row 0 of a unit's key tiles: the map's branch (maps s and s+1 share it
  // while (s+1) % map_repeat != 0).
  auto key_row0 = [&](int unit) { return kbase + (unit_map(unit) / p.map_repeat) * kmap_bytes; };
  const char* kptr = key_row0(unit_first) + kt_first * ktile_bytes;
  const char* vptr = vbase + kt_first * vtile_bytes;
  const char* vlag = vptr;
  int klast = p.T - 1 - kt_first * kKeyTile;
  auto take = [&]() {
    const Src src{kptr, vlag, klast};
    vlag = vptr;
    if (cu_left > 0) {
      --cu_left;
      if (++cu_kt < cu_n) {
        kptr += kt_stride * ktile_bytes;
        vptr += kt_stride * vtile_bytes;
        klast -= kt_stride * kKeyTile;
      } else {
        cu_kt = 0;
        cu_n = unit_tiles(++cu_unit);
        kptr = key_row0(cu_unit);
        vptr = vbase;
        klast = p.T - 1;
      }
    }
    return src;
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

  // Query fragments of map s for the wave's queries qw .. qw+31 (fetch),
  // then the map's score multiplier in the log2 domain (finish).  The
  // rescale test compares maxima of raw scores, so a negative score scale is
  // folded into the queries instead (negation is exact).
  // Queries past the last token repeat its row: their outputs are never
  // stored, and the loads need no branch.
  auto fetch_queries = [&](int s, int qw) {
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = min(qw + cb * 16 + c, p.T - 1);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        qf[cb][kk] = load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + off + kk * 32 + 8 * g);
    }
  };
  auto finish_queries = [&](int s) {
    const float gamma = gamma_of(s);
    if (gamma < 0.f) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) qf[cb][kk] = -qf[cb][kk];
    }
    return fabsf(gamma) * kLog2e;
  };
  auto load_queries = [&](int s, int qw) {
    fetch_queries(s, qw);
    return finish_queries(s);
  };

  // Key fragment of chunk group kk, row block kb: one of four per-lane bases
  // plus an immediate (da_tile.h); V^T block db: a per-lane base plus 1 KiB
  // per block.
  constexpr int KB = KS < 4 ? KS : 4;
  int kfrag[KB];
#pragma unroll
  for (int k = 0; k < KB; ++k) kfrag[k] = KT::base(c, g, k);
  auto key_frag = [&](const char* tile, int kk, int kb) {
    return lds_v8<TQ>(tile + kfrag[kk & 3] + 256 * (kk >> 2) + kb * KT::ROW_BLOCK);
  };
  const int vfrag = KT::BYTES + VT::offset(c, g);

  // Scores of 32 keys x 32 queries from a key tile in LDS: four independent
  // accumulator chains, each key fragment feeding both query blocks.  With
  // DMA, the loads of the next stage are spread between the fragment reads.
  auto scores = [&](const char* kt_lds, f32x4 (&st)[2][2], auto with_dma, char* nxt, const Src& src) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) st[cb][0] = st[cb][1] = zero4();
    const char* kf = kt_lds;
    // Key fragments are read in groups of KG steps (2*KG reads in flight),
    // then consumed: LDS latency is paid once per group, and the group size
    // bounds the registers the reads hold.
    constexpr int KG = KS < 4 ? KS : 4;
#pragma unroll
    for (int k0 = 0; k0 < KS; k0 += KG) {
      q8 kfr[KG][2];
#pragma unroll
      for (int kk = 0; kk < KG; ++kk) {
        kfr[kk][0] = key_frag(kf, k0 + kk, 0);
        kfr[kk][1] = key_frag(kf, k0 + kk, 1);
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

  // Prologue: the queries of the first unit, keys of tile 0 into the last
  // buffer's key slot and stages 0 .. NST-2 = {K(j+1), V(j)} into buffers
  // 0 .. NST-2, all in one memory round trip.
  int qw0 = unit_qt(unit_first) * QT + wave * kAttnQW;   // this wave's first query in the current unit
  fetch_queries(unit_map(unit_first), qw0);
  {
    const Src s0 = take();
#pragma unroll
    for (int n = 0; n < Tile::KPW; ++n) issue_one(lds_sub + (NST - 1) * SBYTES, s0, n);
#pragma unroll
    for (int j = 0; j < NST - 1; ++j) {
      const Src sj = take();
#pragma unroll
      for (int n = 0; n < NL; ++n) issue_one(lds_sub + j * SBYTES, sj, n);
    }
  }
  // Nothing that uses a loaded value moves above the loads' issue: with DMA
  // in flight, an early use would wait for every load.
  __builtin_amdgcn_sched_barrier(0);
  wait_vmem();
  float sc = finish_queries(unit_map(unit_first));
  float sc_next = sc;
  __syncthreads();
  f32x4 st_prev[2][2];
  scores(lds_sub + (NST - 1) * SBYTES, st_prev, std::false_type{}, nullptr, Src{});
  int cur_off = 0;                              // buffer of stage u
  int nxt_off = (NST - 1) * SBYTES;             // buffer of stage u-1: target of stage u+NST-1

  // One pipelined step: tile u is key tile kt of the current unit.  FIXED:
  // every score is bounded by score_bound, so exponents use the fixed
  // reference score_bound*sc (all probabilities <= 1) and the accumulators
  // are never rescaled; otherwise the lazy online rescale runs.  `opens`:
  // tile u+1 is the first of unit `next`, whose queries this step's scores
  // need.
  auto step = [&](auto fixed, int kt, bool opens, int next, bool pad = false) {
    constexpr bool FIXED = decltype(fixed)::value;
    char* cur = lds_sub + cur_off;
    char* nxt = lds_sub + nxt_off;
    const int k0 = kt * kKeyTile;
    if (opens) sc_next = load_queries(unit_map(next), unit_qt(next) * QT + wave * kAttnQW);
    // Stage u + NST - 1 = {K(u + NST), V(u + NST - 1)}.
    const Src src = take();

    // What may branch comes before the barrier: the causal / end mask
    // (diagonal and last tiles only) and the rescale test.  What follows it is
    // one straight block, so the compiler can interleave the exponentials of
    // tile u with the score MFMAs of tile u + 1.
    if ((causal && k0 + kKeyTile - 1 > qw0) || k0 + kKeyTile > p.T || pad) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int tq = qw0 + cb * 16 + c;
        // Last key this query sees; a padding step of a sub-stream sees none.
        const int kmax = pad ? -1 : min(causal ? tq : p.T - 1, p.T - 1);
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
    // LDS read behind them.  Key fragments are read two chunk steps at a
    // time, two steps ahead of their MFMAs, so few reads are waited for at
    // once (against reading up to eight steps up front, the attention kernel
    // at C1/C2/C3/C5 went about 16.3/71/76.2/100 -> 15.7/69.5/74.2/98.8 us);
    // up to eight V^T blocks are read up front, after the scores for 512-wide
    // scores.  The next stage's loads are spread over the score MFMAs.
    constexpr int KG = KS < 2 ? KS : 2;
    constexpr int KLEAD = 2;
    constexpr int KIN = KS < (KG > KLEAD ? KG : KLEAD) ? KS : (KG > KLEAD ? KG : KLEAD);   // steps read up front
    constexpr int VA = KS <= 8 ? (NB < 8 ? NB : 8) : 0;
    const char* kf = cur;
    const char* vf = cur + vfrag;
    q8 kfr[KS][2];
    v8 vfr[NB];
    auto read_keys = [&](int kk) {
      kfr[kk][0] = key_frag(kf, kk, 0);
      kfr[kk][1] = key_frag(kf, kk, 1);
    };
#pragma unroll
    for (int kk = 0; kk < KIN; ++kk) read_keys(kk);
#pragma unroll
    for (int db = 0; db < VA; ++db) vfr[db] = lds_v8<TV>(vf + db * 1024);

    f32x4 st_new[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) st_new[cb][0] = st_new[cb][1] = zero4();
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (KIN < KS && kk + KLEAD >= KIN && kk + KLEAD < KS && (kk + KLEAD) % KG == 0) {
#pragma unroll
        for (int k2 = kk + KLEAD; k2 < kk + KLEAD + KG; ++k2) read_keys(k2);
      }
      // The next stage's loads start at chunk step D0: over the whole score
      // loop for 256-wide scores, over its second half otherwise (measured:
      // from step 0 the C1 and C5 attention ran 15.7 -> 15.4 and 99.8 -> 95.7
      // us, C2 and C3 (128- and 512-wide scores) about 0.8 us slower).
      constexpr int D0 = KS == 8 ? 0 : KS / 2;
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
    for (int db = VA; db < NB; ++db) vfr[db] = lds_v8<TV>(vf + db * 1024);

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
    cur_off = cur_off + SBYTES == NST * SBYTES ? 0 : cur_off + SBYTES;
  };

  // Slots of this workgroup's partial results (stream split); PIECE is
  // attn_piece_bytes(p.flags), a template argument so that only the piece
  // store of the call's type is compiled into the loop.
  constexpr int es = PIECE;
  const int64_t slot_bytes = attn_slot_bytes(QT, DS, es);
  char* slots = p.part + static_cast<int64_t>(gx * p.n_seg + gy) * (MULTI ? 4 : 2) * slot_bytes;
  // The fixed reference keeps every probability within the range of the
  // operand type: bf16 holds 2^-120 .. 1 exactly in exponent; fp16 does not.
  auto fixed_for = [&](float scale) {
    return p.score_bound > 0.f && sizeof(TV) == 2 && !std::is_same<TV, _Float16>::value &&
           2.f * p.score_bound * scale <= 120.f;
  };
  // Sub-streams of one map keep their accumulators for the final merge.
  const bool keep = SUB == 2 && split_tiles;
  int unit = unit_first, kt_start = split_tiles ? 0 : kt_first, left = real;
  // The run holds the current query tile from its first map's first tile on.
  bool qt_from_start = unit_map(unit_first) == 0 && kt_first == 0;
  while (left > 0) {
    const int n_unit = unit_tiles(unit);
    const int n_here = min(n_unit - kt_start, left);
    const bool more = left > n_here;
    const int s = unit_map(unit);
    const int qt = unit_qt(unit);
    const bool fixed = fixed_for(sc);
    if (fixed) {
      for (int i = 0; i < n_here; ++i)
        step(std::true_type{}, split_tiles ? sub + 2 * i : kt_start + i, more && i == n_here - 1, unit + 1);
    } else {
      for (int i = 0; i < n_here; ++i)
        step(std::false_type{}, split_tiles ? sub + 2 * i : kt_start + i, more && i == n_here - 1, unit + 1);
    }
    if (keep) break;
    const float wmap = weight_of(s);
    // A piece of a unit's key range (stream split) stores its normalized
    // outputs (16-bit, or fp32 for fp32 outputs), reference and row sum
    // (fp32) for the merge kernel: slot 0 if it is the run's first unit, else
    // slot 1.  A whole unit goes to its output slot, or with the map mix
    // into the query tile's mix.
    const bool partial = stream && (kt_start > 0 || n_here < n_unit);
    char* piece = slots + (unit == unit_first ? 0 : 1) * slot_bytes;
    float* piece_stats = reinterpret_cast<float*>(piece + static_cast<int64_t>(QT) * DS * es);
    const int q0 = qt * QT;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const float l = group_sum(l_part[cb]);
      const float w = (partial ? 1.f : wmap) / (l > 0.f ? l : 1.f);
      const int ql = wave * kAttnQW + cb * 16 + c;
      const int tq = q0 + ql;
      if (partial) {
#pragma unroll
        for (int db = 0; db < NB; ++db) store_piece4<TV, es>(piece, ql * DS + db * 16 + 4 * g, acc[cb][db] * w);
        if (g == 0) {
          piece_stats[ql] = fixed ? p.score_bound * sc : m_run[cb];
          piece_stats[QT + ql] = l;
        }
      } else if constexpr (MULTI) {
#pragma unroll
        for (int i = 0; i < NB; ++i) yacc[cb][i] += acc[cb][i] * w;
      } else if (tq < p.T) {
        store_rows<TV, DS>(p, b, (p.flags & kAttnMix) ? 0 : s, tq, g, ds0, acc[cb], w);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) acc[cb][i] = zero4();
      m_run[cb] = -INFINITY;
      l_part[cb] = 0.f;
    }
    if constexpr (MULTI && SUB == 1) {
      // The query tile ends here (in this run): a tile the run holds whole is
      // stored; otherwise its partial mix goes to mix slot 0 (the run's first
      // query tile) or 1 for the merge kernel.
      if (!more || unit_qt(unit + 1) != qt) {
        const bool whole = qt_from_start && s == p.S - 1 && !partial;
        char* mix = slots + (2 + (qt == unit_qt(unit_first) ? 0 : 1)) * slot_bytes;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int ql = wave * kAttnQW + cb * 16 + c;
          if (whole) {
            if (q0 + ql < p.T) store_rows<TV, DS>(p, b, 0, q0 + ql, g, ds0, yacc[cb], 1.f);
          } else {
#pragma unroll
            for (int db = 0; db < NB; ++db) store_piece4<TV, es>(mix, ql * DS + db * 16 + 4 * g, yacc[cb][db]);
          }
#pragma unroll
          for (int i = 0; i < NB; ++i) yacc[cb][i] = zero4();
        }
        qt_from_start = true;
      }
    }
    sc = sc_next;
    left -= n_here;
    ++unit;
    kt_start = 0;
    qw0 = unit_qt(unit) * QT + wave * kAttnQW;
  }

  if constexpr (SUB == 2) {
    // Padding steps of the shorter sub-stream (every score masked).
    const int n_pad = total - real;
    if (fixed_for(sc)) {
      for (int i = 0; i < n_pad; ++i) step(std::true_type{}, 0, false, 0, true);
    } else {
      for (int i = 0; i < n_pad; ++i) step(std::false_type{}, 0, false, 0, true);
    }
    if (keep || MULTI) {
      // The odd sub-stream hands its accumulators (the map's unnormalized
      // outputs with their references and row sums, or the mix) to the even
      // one through LDS, in the lanes' own order.
      wait_vmem();
      __syncthreads();
      constexpr int XW = 2 * NB * 256 + 256;   // floats per query wave
      static_assert(NQW * XW * 4 <= NST * SBYTES, "the hand-over fits the stage buffers");
      float* xch = reinterpret_cast<float*>(lds) + wave * XW;
      if (sub == 1) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
          for (int db = 0; db < NB; ++db)
            *reinterpret_cast<f32x4*>(xch + ((cb * NB + db) * 64 + lane) * 4) = MULTI ? yacc[cb][db] : acc[cb][db];
          xch[2 * NB * 256 + lane * 4 + cb] = m_run[cb];
          xch[2 * NB * 256 + lane * 4 + 2 + cb] = l_part[cb];
        }
      }
      __syncthreads();
      if (sub == 0) {
        const bool fixed = fixed_for(sc);
        const float wmap = weight_of(0);
        const int q0 = qt_maps * QT;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int ql = wave * kAttnQW + cb * 16 + c;
          if constexpr (MULTI) {
#pragma unroll
            for (int db = 0; db < NB; ++db)
              yacc[cb][db] += *reinterpret_cast<const f32x4*>(xch + ((cb * NB + db) * 64 + lane) * 4);
            if (q0 + ql < p.T) store_rows<TV, DS>(p, b, 0, q0 + ql, g, ds0, yacc[cb], 1.f);
          } else {
            // With the fixed reference both sub-streams share it; online,
            // each scales to the larger running maximum.
            const float m1 = xch[2 * NB * 256 + lane * 4 + cb];
            const float l1 = xch[2 * NB * 256 + lane * 4 + 2 + cb];
            float f0 = 1.f, f1 = 1.f;
            if (!fixed) {
              const float M = fmaxf(m_run[cb], m1);
              f0 = m_run[cb] == -INFINITY ? 0.f : exp2f(m_run[cb] - M);
              f1 = m1 == -INFINITY ? 0.f : exp2f(m1 - M);
            }
            const float l = group_sum(l_part[cb] * f0 + l1 * f1);
            const float w = wmap / (l > 0.f ? l : 1.f);
            if (q0 + ql < p.T) {
              f32x4 o[NB];
#pragma unroll
              for (int db = 0; db < NB; ++db)
                o[db] = acc[cb][db] * f0 + *reinterpret_cast<const f32x4*>(xch + ((cb * NB + db) * 64 + lane) * 4) * f1;
              store_rows<TV, DS>(p, b, 0, q0 + ql, g, ds0, o, w);
            }
          }
        }
      }
    }
  }
  // The last step's (redundant) stage loads must land before the workgroup's
  // LDS is released.
  wait_vmem();
}

// Merge of a query tile split over stream workgroups.  The tile's S units
// (maps) cover stream tiles [A, A + S n); a unit split over workgroups ya ..
// yb merges as O = sum_c 2^(m_c - M) l_c o_c / sum_c 2^(m_c - M) l_c over its
// pieces c (o_c normalized, M = max_c m_c), per query row.  Its piece sits in
// slot 1 of ya when the unit does not open ya's run, else in slot 0.  With
// the map mix the output is sum_s alpha_s O_s over the split units plus the
// partial mixes of the whole units, one per workgroup ya .. yb of the tile
// (slot rule as for pieces, offset by two slots).  A workgroup takes 32 query
// rows of the tile, each wave eight of them; the lanes cover consecutive
// features, so a partial row is one coalesced sweep, and the loads of a
// piece's eight rows are issued together.
template <typename TV, int DS, int QT, bool MULTI, int PIECE>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnParams p) {
  const int qt = static_cast<int>(blockIdx.y);
  const int64_t L = p.stream_len;
  const int64_t A = p.S * tiles_before(p, stream_index(p, qt), QT);
  const int n = key_tiles_of(p, qt, QT);
  const int y0 = static_cast<int>(A / L);
  const int y1 = static_cast<int>((A + static_cast<int64_t>(p.S) * n - 1) / L);
  if (y0 == y1) return;   // written directly by its workgroup
  const int b = static_cast<int>(blockIdx.x) / p.n_slices;
  const int ds0 = (static_cast<int>(blockIdx.x) - b * p.n_slices) * DS;
  constexpr int es = PIECE;
  const int64_t slot_bytes = attn_slot_bytes(QT, DS, es);
  constexpr int NSLOT = MULTI ? 4 : 2;
  auto slot = [&](int y, int64_t start, int k) -> const char* {
    const int first = (y == static_cast<int>(start / L) && start != (start / L) * L) ? 1 : 0;
    return p.part + ((static_cast<int64_t>(blockIdx.x) * p.n_seg + y) * NSLOT + k + first) * slot_bytes;
  };
  const int lane = lane_id();
  constexpr int RW = 8;                             // query rows per wave
  static_assert(QT % 32 == 0, "32 rows per workgroup");
  // blockIdx.z picks 32 rows of the tile; rows past T are merged (their
  // pieces lie inside the slots) but not stored.
  const int q_base = static_cast<int>(blockIdx.z) * 32 + (static_cast<int>(threadIdx.x) >> 6) * RW;
  constexpr int NV = DS / 256 > 0 ? DS / 256 : 1;   // 4-feature vectors per lane
  f32x4 out[RW][NV];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int k = 0; k < NV; ++k) out[r][k] = zero4();
  if constexpr (MULTI) {
    for (int y = y0; y <= y1; ++y) {
      const char* mix = slot(y, A, 2);
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int d4 = (k * 64 + lane) * 4;
          if (d4 < DS) out[r][k] += load_piece4<TV, es>(mix, (q_base + r) * DS + d4);
        }
    }
  }
  for (int s = 0; s < p.S; ++s) {
    const int64_t start = A + static_cast<int64_t>(s) * n;
    const int ya = static_cast<int>(start / L);
    const int yb = static_cast<int>((start + n - 1) / L);
    if (ya == yb) continue;   // whole in one run: stored or in that run's mix
    // One pass with a running maximum per row: a piece's loads (references,
    // row sums, values of all eight rows) are issued together.
    float M[RW], den[RW];
    f32x4 o[RW][NV];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      M[r] = -INFINITY;
      den[r] = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k) o[r][k] = zero4();
    }
    for (int y = ya; y <= yb; ++y) {
      const char* pc = slot(y, start, 0);
      const float* stats = reinterpret_cast<const float*>(pc + static_cast<int64_t>(QT) * DS * es);
      float m[RW], l[RW];
      f32x4 v[RW][NV];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        m[r] = stats[q_base + r];
        l[r] = stats[QT + q_base + r];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int d4 = min((k * 64 + lane) * 4, DS - 4);
          v[r][k] = load_piece4<TV, es>(pc, (q_base + r) * DS + d4);
        }
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        if (m[r] == -INFINITY) continue;   // a piece with every key masked
        const float Mn = fmaxf(M[r], m[r]);
        const float f_old = M[r] == -INFINITY ? 0.f : exp2f(M[r] - Mn);
        const float wl = exp2f(m[r] - Mn) * l[r];
        den[r] = den[r] * f_old + wl;
#pragma unroll
        for (int k = 0; k < NV; ++k) o[r][k] = o[r][k] * f_old + v[r][k] * wl;
        M[r] = Mn;
      }
    }
    const float wmap = MULTI ? map_weight(p, s) : 1.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float w = wmap * (den[r] > 0.f ? 1.f / den[r] : 0.f);
#pragma unroll
      for (int k = 0; k < NV; ++k) out[r][k] += o[r][k] * w;
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int tq = qt * QT + q_base + r;
    if (tq >= p.T) continue;
    const int64_t at = b * p.out_stride_b + static_cast<int64_t>(tq) * p.out_stride_t + ds0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int d4 = (k * 64 + lane) * 4;
      if (d4 < DS) {
        if (p.flags & kAttnOutF32) {
          *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + at + d4) = out[r][k];
        } else {
          typename Elem<TV>::v4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = static_cast<TV>(out[r][k][i]);
          *reinterpret_cast<typename Elem<TV>::v4*>(static_cast<TV*>(p.out) + at + d4) = v;
        }
      }
    }
  }
}

// Short sequences (T <= 64): one workgroup per (sequence, map group, value
// slice) loads all of its keys and its V^T slice once -- no key-tile loop,
// no stage ring, no online softmax -- and each wave computes the scores of
// its 32 queries against at most two key tiles, the exact row softmax
// (maximum and sum over the row in registers) and P V.  Wave w takes map
// slot w / 2 of the group and query block w % 2; with the map mix the waves
// of slot 1 hand alpha_s O_s to those of slot 0 through LDS.  The kernel's
// code is a fraction of the general one's: with two steps per sequence the
// general kernel's first pass through its loop is most of its time.
template <typename TQ, typename TV, int RP, int DS, int NMAP>
__global__ __launch_bounds__(128 * NMAP, 1) void attention_short_kernel(AttnParams p) {
  static_assert(NMAP == 1 || NMAP == 2, "one or two map slots");
  typedef XorTile<kKeyTile, RP / 8, true> KT;   // keys (blocked rows)
  typedef XorTile<DS, 4, false> VT;             // V^T rows: DS features x 32 tokens
  typedef typename Elem<TQ>::v8 q8;
  constexpr int NW = 2 * NMAP;
  constexpr int KS = RP / 32;
  constexpr int NB = DS / 16;
  constexpr int KBYTES = 2 * KT::BYTES;          // one map slot's two key tiles
  constexpr int VOFF = NMAP * KBYTES;            // the two V^T tiles follow the keys
  constexpr int LOADS = NMAP * 2 * KT::LOADS + 2 * VT::LOADS;   // wave loads of the workgroup
  static_assert(LOADS % NW == 0, "every wave issues the same number of loads");
  // The map hand-over (after every wave has read its tiles) reuses the LDS.
  constexpr int XBYTES = NMAP == 2 ? 2 * 2 * NB * 256 * 4 : 0;
  constexpr int LDS_BYTES = VOFF + 2 * VT::BYTES > XBYTES ? VOFF + 2 * VT::BYTES : XBYTES;
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int mslot = wave >> 1;
  const int qb = wave & 1;
  const bool causal = p.flags & kAttnCausal;
  const bool mix = p.flags & kAttnMix;
  // Workgroups of one sequence are consecutive in the logical order and so
  // share an XCD (dispatch deals workgroups to the XCDs round-robin).
  const int n_wg = static_cast<int>(gridDim.x);
  const int wg = static_cast<int>(blockIdx.x);
  const int xcd = wg % kXcds, per_xcd = n_wg / kXcds, rem_xcd = n_wg % kXcds;
  const int logical = xcd * per_xcd + min(xcd, rem_xcd) + wg / kXcds;
  const int n_mg = (p.S + NMAP - 1) / NMAP;
  const int b = logical / (n_mg * p.n_slices);
  const int mg = (logical / p.n_slices) % n_mg;
  const int slice = logical % p.n_slices;
  const int ds0 = slice * DS;
  auto map_of = [&](int ms) { return min(mg * NMAP + ms, p.S - 1); };
  const int s = map_of(mslot);
  const bool real_map = mg * NMAP + mslot < p.S;   // a missing slot repeats the last map and stores nothing

  // Per-map scalars, lane i holding map min(i, S-1), issued first.
  const int map_lane = min(lane, p.S - 1);
  const ScalarHalves scale_raw = fetch_scalar(p.scales, p.scales_dtype, map_lane);
  const bool mix_logits = mix && p.mix_logits != nullptr;
  const ScalarHalves mix_raw = fetch_scalar(mix_logits ? p.mix_logits : p.scales,
                                            mix_logits ? p.mix_dtype : p.scales_dtype, map_lane);

  // Query fragments of this wave's map and block (rows past T repeat row
  // T-1; their outputs are never stored).
  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b + (s / p.map_repeat) * p.map_stride;
  q8 qf[2][KS];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int tq = min(32 * qb + 16 * cb + c, p.T - 1);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qf[cb][kk] = load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + kk * 32 + 8 * g);
  }
  // The workgroup's keys (both tiles of every map slot; rows past T read
  // row T-1) and V^T tiles, by global->LDS DMA, spread over the waves.
  const int kstride = static_cast<int>(p.qk_stride_t) * static_cast<int>(sizeof(TQ));
  const char* vbase =
      reinterpret_cast<const char*>(static_cast<const TV*>(p.vt) + b * p.vt_stride_b + 32 * ds0);
#pragma unroll
  for (int i = 0; i < LOADS / NW; ++i) {
    const int j = i * NW + wave;
    int row, ck;
    if (j < NMAP * 2 * KT::LOADS) {
      const int ms = j / (2 * KT::LOADS);
      const int kt = (j / KT::LOADS) % 2;
      const int jj = j % KT::LOADS;
      KT::slot_chunk(jj * 64 + lane, row, ck);
      const int key = min(kt * kKeyTile + row, p.T - 1);
      const char* kb = reinterpret_cast<const char*>(static_cast<const TQ*>(p.k) + b * p.qk_stride_b +
                                                     (map_of(ms) / p.map_repeat) * p.map_stride);
      dma16(uniform_ptr(kb) + static_cast<uint32_t>(key * kstride + ck * 16),
            lds + ms * KBYTES + kt * KT::BYTES + jj * 1024);
    } else {
      const int v = j - NMAP * 2 * KT::LOADS;
      const int kt = v / VT::LOADS;
      const int jj = v % VT::LOADS;
      VT::slot_chunk(jj * 64 + lane, row, ck);
      dma16(uniform_ptr(vbase + static_cast<int64_t>(kt) * kKeyTile * p.D * sizeof(TV)) +
                static_cast<uint32_t>((row * kKeyTile + ck * 8) * sizeof(TV)),
            lds + VOFF + kt * VT::BYTES + jj * 1024);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vmem();

  auto lane_value = [](float v, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i)); };
  float gamma = lane_value(scalar_value(scale_raw, p.scales_dtype), s);
  if (p.flags & kAttnScalesAreLog) gamma = expf(fminf(fmaxf(gamma, kLogScaleMin), kLogScaleMax));
  gamma *= p.scale_mult;
  float weight = 1.f;
  if (mix) {
    if (!mix_logits) {
      weight = 1.f / static_cast<float>(p.S);
    } else {
      const float logit = scalar_value(mix_raw, p.mix_dtype);
      float mx = -INFINITY;
      for (int i = 0; i < p.S; ++i) mx = fmaxf(mx, lane_value(logit, i));
      float den = 0.f;
      for (int i = 0; i < p.S; ++i) den += expf(lane_value(logit, i) - mx);
      weight = expf(lane_value(logit, s) - mx) / den;
    }
  }
  // A negative scale folds into the queries (exact), so row maxima of raw
  // scores are maxima of scaled ones.
  if (gamma < 0.f) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) qf[cb][kk] = -qf[cb][kk];
  }
  const float sc = fabsf(gamma) * kLog2e;
  __syncthreads();

  // Scores: lane (c, g) of block (kt, cb, kb) holds key 32kt + 8g + 4kb + e
  // for query 32qb + 16cb + c.  Query block qb sees key tiles 0 .. qb when
  // causal; tile 1 exists when T > 32.
  const char* kl = lds + mslot * KBYTES;
  int kfrag[KS < 4 ? KS : 4];
#pragma unroll
  for (int k = 0; k < (KS < 4 ? KS : 4); ++k) kfrag[k] = KT::base(c, g, k);
  const int n_kt = p.T > kKeyTile && (!causal || qb == 1) ? 2 : 1;
  f32x4 st[2][2][2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) st[kt][cb][0] = st[kt][cb][1] = zero4();
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    if (kt < n_kt) {
      const char* tile = kl + kt * KT::BYTES;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const q8 k0 = lds_v8<TQ>(tile + kfrag[kk & 3] + 256 * (kk >> 2));
        const q8 k1 = lds_v8<TQ>(tile + kfrag[kk & 3] + 256 * (kk >> 2) + KT::ROW_BLOCK);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          st[kt][cb][0] = Elem<TQ>::mma(k0, qf[cb][kk], st[kt][cb][0]);
          st[kt][cb][1] = Elem<TQ>::mma(k1, qf[cb][kk], st[kt][cb][1]);
        }
      }
    }
  }
  // Exact row softmax: the row maximum over the valid keys, exponentials
  // against it, the row sum; masked keys get probability zero.
  auto valid = [&](int kt, int cb, int kb, int e) {
    const int key = kt * kKeyTile + 8 * g + 4 * kb + e;
    const int tq = 32 * qb + 16 * cb + c;
    return kt < n_kt && key < p.T && (!causal || key <= tq);
  };
  typename Elem<TV>::v8 pb[2][2];
  float inv_l[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    float m = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (valid(kt, cb, kb, e)) m = fmaxf(m, st[kt][cb][kb][e]);
    m = group_max(m) * sc;
    float l = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pr = valid(kt, cb, kb, e) ? __builtin_amdgcn_exp2f(__builtin_fmaf(st[kt][cb][kb][e], sc, -m)) : 0.f;
          st[kt][cb][kb][e] = pr;
          l += pr;
        }
    inv_l[cb] = 1.f / group_sum(l);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) pb[kt][cb] = pack_blocked<TV>(st[kt][cb][0], st[kt][cb][1]);
  }
  // O^T += V^T P^T over the key tiles.
  const char* vl = lds + VOFF + VT::offset(c, g);
  f32x4 acc[2][NB];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int db = 0; db < NB; ++db) acc[cb][db] = zero4();
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    if (kt < n_kt) {
#pragma unroll
      for (int db = 0; db < NB; ++db) {
        const typename Elem<TV>::v8 vf = lds_v8<TV>(vl + kt * VT::BYTES + db * 1024);
        acc[0][db] = Elem<TV>::mma(vf, pb[kt][0], acc[0][db]);
        acc[1][db] = Elem<TV>::mma(vf, pb[kt][1], acc[1][db]);
      }
    }
  }
  if (NMAP == 2 && mix) {
    // Slot 1 hands weight * O (normalized) to slot 0 of the same query block.
    __syncthreads();
    float* xch = reinterpret_cast<float*>(lds) + qb * (2 * NB * 256);
    if (mslot == 1) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int db = 0; db < NB; ++db)
          *reinterpret_cast<f32x4*>(xch + ((cb * NB + db) * 64 + lane) * 4) =
              real_map ? acc[cb][db] * (weight * inv_l[cb]) : zero4();
    }
    __syncthreads();
    if (mslot == 1) return;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = 32 * qb + 16 * cb + c;
      f32x4 o[NB];
#pragma unroll
      for (int db = 0; db < NB; ++db)
        o[db] = acc[cb][db] * (weight * inv_l[cb]) + *reinterpret_cast<const f32x4*>(xch + ((cb * NB + db) * 64 + lane) * 4);
      if (tq < p.T) store_rows<TV, DS>(p, b, 0, tq, g, ds0, o, 1.f);
    }
    return;
  }
  if (!real_map) return;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int tq = 32 * qb + 16 * cb + c;
    if (tq < p.T) store_rows<TV, DS>(p, b, mix ? 0 : s, tq, g, ds0, acc[cb], weight * inv_l[cb]);
  }
}

template <typename TQ, typename TV, int RP, int DS>
static void launch_attn_short(const AttentionArgs& a, AttnParams& p, hipStream_t s) {
  p.n_slices = a.D / DS;
  if (a.S == 1) {
    hipLaunchKernelGGL((attention_short_kernel<TQ, TV, RP, DS, 1>), dim3(a.B * p.n_slices), dim3(128), 0, s, p);
  } else {
    const int n_mg = (a.S + 1) / 2;
    hipLaunchKernelGGL((attention_short_kernel<TQ, TV, RP, DS, 2>), dim3(a.B * p.n_slices * n_mg), dim3(256), 0, s, p);
  }
}

template <typename TQ, typename TV, int RP, int DS, bool MULTI, int NW>
static void launch_attn_4(const AttentionArgs& a, const AttnPlan& plan, AttnParams& p, hipStream_t s) {
  constexpr int QT = NW * kAttnQW;
  if (plan.stream_len == 0) {
    hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, NW, kAttnStages, MULTI, 1>), dim3(a.B * p.n_slices, plan.n_qt),
                       dim3(NW * 64), 0, s, p);
    return;
  }
  // The stream split: pieces in the value dtype, or in fp32 when the call
  // asks for fp32 outputs.  plan_attention gives it four-wave workgroups
  // only (every key and V^T tile it stages serves 128 queries).
  if constexpr (NW == 4) {
    const dim3 grid(a.B * p.n_slices, plan.n_seg), merge(a.B * p.n_slices, plan.n_qt, QT / 32);
    if (attn_piece_bytes(a.flags) == 4) {
      hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, NW, kAttnStages, MULTI, 1, 4>), grid, dim3(NW * 64), 0, s, p);
      hipLaunchKernelGGL((attention_merge_kernel<TV, DS, QT, MULTI, 4>), merge, dim3(256), 0, s, p);
    } else {
      hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, NW, kAttnStages, MULTI, 1, 2>), grid, dim3(NW * 64), 0, s, p);
      hipLaunchKernelGGL((attention_merge_kernel<TV, DS, QT, MULTI, 2>), merge, dim3(256), 0, s, p);
    }
  }
}

template <typename TQ, typename TV, int RP, int DS, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, const AttnPlan& plan, AttnParams& p, hipStream_t s) {
  // Two waves per query tile (64 queries), or four (128 queries) sharing each
  // key / V^T tile: always for 512-wide scores, whose tiles take a whole CU's
  // LDS, and for the stream split of long problems, where the tile fill per
  // query halves.  Two sub-streams run four waves over 64 queries.
  p.n_slices = a.D / DS;
  p.n_qt = plan.n_qt;
  p.stream_len = plan.stream_len;
  p.n_seg = plan.n_seg;
  if constexpr (RP < 512) {
    if constexpr (DS <= 128) {
      if (plan.sub == 2) {
        hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, 4, kAttnStages, MULTI, 2>),
                           dim3(a.B * p.n_slices, plan.n_qt), dim3(256), 0, s, p);
        return;
      }
    }
    if (plan.nw == 2) {
      launch_attn_4<TQ, TV, RP, DS, MULTI, 2>(a, plan, p, s);
      return;
    }
  }
  launch_attn_4<TQ, TV, RP, DS, MULTI, 4>(a, plan, p, s);
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
                        bool allow_split, int piece_bytes) {
  AttnPlan plan{};
  const int64_t nw = RP == 512 ? 4 : 2;
  const int64_t qtile = nw * kAttnQW;
  plan.nw = static_cast<int>(nw);
  plan.n_qt = static_cast<int>((T + qtile - 1) / qtile);
  // Value slice: as wide as possible (one score tile serves more value columns
  // and the softmax is shared by more MFMAs) while the grid keeps at least 256
  // workgroups.  The register budget caps it at 256 features, and at 128 with
  // the map mix (a second accumulator set) or 512-wide scores; a slice width
  // (256, 128 or 64) divides D, which is a multiple of 64.
  const int64_t tiles = B * plan.n_qt;
  const int64_t cap = (multi || RP == 512) ? 128 : 256;
  int64_t ds = 64;
  for (int64_t w = 256; w > 64; w /= 2)
    if (w <= cap && D % w == 0) {
      ds = w;
      break;
    }
  while (ds > 128 && tiles * (D / ds) < 256) ds /= 2;
  plan.ds = static_cast<int>(ds);
  const int64_t slices = D / ds;
  // Work shape, by the steps of the slowest workgroup slot: with G
  // workgroups of at most h steps and W steps in all over C workgroups that
  // run at once, about max(h, W / C).
  //  - one workgroup per query tile (all maps);
  //  - the same with two sub-streams (scores narrower than 512): half the
  //    steps per workgroup, twice the LDS;
  //  - the stream split (one map, or the map mix): runs of an even share of
  //    all steps (at least 16, so the prologue and partials stay small next
  //    to a run), plus the partials' round trip through memory.
  auto concurrent = [&](int64_t waves, int64_t subs, int64_t width) {
    const int64_t stage = subs * (RP / 8 * 32 * 16 + width * 4 * 16);   // key + V^T tiles
    const int64_t stage_bytes = (stage + 1023) / 1024 * 1024;
    return kCUs * std::max<int64_t>(1, std::min<int64_t>(4 / waves, kLdsBytes / (kAttnStages * stage_bytes)));
  };
  const int64_t last = plan.n_qt - 1;
  const int64_t n_last = host_key_tiles(last, qtile, T, causal);
  const int64_t per_qt = S * n_last;   // the heaviest query tile
  const int64_t stream_all = S * host_all_tiles(plan.n_qt, qtile, T, causal);
  const int64_t work = B * slices * stream_all;
  const int64_t c1 = concurrent(nw, 1, ds);
  const int64_t span_maps = std::max(per_qt, (work + c1 - 1) / c1);
  int64_t best = span_maps;
  plan.sub = 1;
  plan.stream_len = 0;
  plan.n_seg = 0;
  if (RP < 512) {
    // Two sub-streams hold twice the accumulators: value slices of at most
    // 128 features.
    const int64_t ds2 = std::min<int64_t>(ds, 128);
    const int64_t c2 = concurrent(2 * nw, 2, ds2);
    const int64_t steps = S == 1 ? (n_last + 1) / 2 : (S + 1) / 2 * n_last;
    const int64_t span_sub = std::max(steps, (B * (D / ds2) * stream_all / 2 + c2 - 1) / c2);
    if (span_sub <= best) {
      best = span_sub;
      plan.sub = 2;
      plan.ds = static_cast<int>(ds2);
    }
  }
  const int64_t share = std::max<int64_t>(16, (work + c1 - 1) / c1);
  int64_t part_qtile = qtile;
  if (allow_split && (S == 1 || multi) && per_qt > share && share * 5 / 4 < best) {
    // The stream split runs four waves (128 queries) per workgroup: every key
    // and V^T tile it fills serves twice the queries.
    const int64_t q4 = 4 * kAttnQW;
    const int64_t n_qt4 = (T + q4 - 1) / q4;
    const int64_t all4 = S * host_all_tiles(n_qt4, q4, T, causal);
    const int64_t c4 = concurrent(4, 1, ds);
    const int64_t share4 = std::max<int64_t>(16, (B * slices * all4 + c4 - 1) / c4);
    plan.sub = 1;
    plan.nw = 4;
    plan.ds = static_cast<int>(ds);
    plan.n_qt = static_cast<int>(n_qt4);
    plan.stream_len = static_cast<int>(share4);
    plan.n_seg = static_cast<int>((all4 + share4 - 1) / share4);
    part_qtile = q4;
  }
  plan.part_bytes = plan.stream_len > 0 ? B * slices * plan.n_seg * (multi ? 4 : 2) *
                                              attn_slot_bytes(static_cast<int>(part_qtile), static_cast<int>(ds), piece_bytes)
                                        : 0;
  return plan;
}

template <typename TQ, typename TV, int RP>
static void launch_attn_short_d(const AttentionArgs& a, AttnParams& p, hipStream_t s) {
  if (a.D % 128 == 0) launch_attn_short<TQ, TV, RP, 128>(a, p, s);
  else launch_attn_short<TQ, TV, RP, 64>(a, p, s);
}

template <typename TQ, typename TV>
static void launch_attn_short_r(const AttentionArgs& a, AttnParams& p, hipStream_t s) {
  switch (a.RP) {
    case 64: launch_attn_short_d<TQ, TV, 64>(a, p, s); break;
    case 128: launch_attn_short_d<TQ, TV, 128>(a, p, s); break;
    default: launch_attn_short_d<TQ, TV, 256>(a, p, s); break;
  }
}

// The short-sequence kernel takes sequences of at most two key tiles with
// scores up to 256 wide; with the map mix, at most two maps (one workgroup
// holds every map of its sequence).
static bool attention_short_fits(const AttentionArgs& a) {
  return a.T <= 2 * kKeyTile && a.RP <= 256 && (a.S <= 2 || !(a.flags & kAttnMix));
}

void launch_routed_attention(const AttentionArgs& a, void* partials, hipStream_t stream) {
  if (a.T == 0 || a.B == 0) return;
  AttnParams p;
  p.part = static_cast<char*>(partials);
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
  if (attention_short_fits(a)) {
    p.n_qt = 1;
    p.stream_len = 0;
    p.n_seg = 0;
    if (a.qk_dtype == kF16 && a.v_dtype == kBF16) launch_attn_short_r<_Float16, __bf16>(a, p, stream);
    else if (a.qk_dtype == kF16) launch_attn_short_r<_Float16, _Float16>(a, p, stream);
    else launch_attn_short_r<__bf16, __bf16>(a, p, stream);
    return;
  }
  const AttnPlan plan = plan_attention(a.B, a.S, a.T, a.D, a.RP, (a.flags & kAttnMix) && a.S > 1,
                                       a.flags & kAttnCausal, partials != nullptr, attn_piece_bytes(a.flags));
  if (a.qk_dtype == kF16 && a.v_dtype == kBF16) launch_attn_0<_Float16, __bf16>(a, plan, p, stream);
  else if (a.qk_dtype == kF16) launch_attn_0<_Float16, _Float16>(a, plan, p, stream);
  else launch_attn_0<__bf16, __bf16>(a, plan, p, stream);
}

}  // namespace da
