// MFMA GEMM for the projections of SharedDictionaryAttention.
//
// Replaces the fused Q/K projection (reference src/double_attention/modules.py:143-157:
// cat(query.weight, key.weight) then F.linear), the value projection
// (modules.py:83,212) and the output projection (modules.py:117-121,272).
//
// Every launch computes one or two "segments" D[i, j] = sum_k P[i, k] Q[j, k]
// (+ bias), with both operands K-contiguous, as PyTorch stores x [N, d] and
// Linear weights [out, in].  The query and key weights are read as two stacked
// operands, so no concatenated weight is ever materialized.  Epilogues:
//   mode 0: out[j, i]                 -- features i of token j (Q/K projection,
//                                        output projection)
//   mode 1: V^T in 32-token tiles -- feature j of token t of sequence b at
//           out[b*vt_stride_b + (t/32)*32*J + 32*j + t%32], the layout the
//           attention kernel streams one contiguous tile at a time.  Rows i
//           run over B * Tp "virtual" tokens (t < Tp, the padded length);
//           tokens past T reuse the last real row, so the padding is finite.
// Tiles: 128 x 128 per workgroup when the launch has at least 512 of them
// (two per CU), else 96 x 128 where that fills one round of 512 workgroups
// and 64 x 128 would not, else 64 x 128 (twice the workgroups).  64-deep K stages sit
// in XOR-swizzled LDS tiles (da_tile.h, conflict-free MFMA operand reads)
// filled by global->LDS DMA, in a ring of two buffers (128- and 96-row
// tiles) or three (64-row tiles); each of the four waves owns a (BI/2) x 64
// block (BI/32 x 4 MFMA 16x16x32 blocks).
//
// A launch may also carry a dictionary normalization (dict_norm.h): its
// workgroups precede the GEMM tiles, so the module forward normalizes its bank
// while the projections run, without a launch of its own.
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"
#include "dict_norm.h"

namespace da {

// erf for the GELU epilogue: Abramowitz & Stegun, Handbook of Mathematical
// Functions, formula 7.1.26, erf(x) = 1 - (a1 t + ... + a5 t^5) e^(-x^2) with
// t = 1 / (1 + p x) for x >= 0 (odd extension), absolute error <= 1.5e-7, far
// below one rounding of the 16-bit outputs.  Branch-free: a reciprocal, an
// exponential and five FMAs, where the library erff takes several times the
// VALU work (the epilogue of a 4096 x 1536 GEMM runs it 6.3 million times).
__device__ __forceinline__ float erf_fast(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, ax, 1.f));
  float poly = __builtin_fmaf(t, 1.061405429f, -1.453152027f);
  poly = __builtin_fmaf(t, poly, 1.421413741f);
  poly = __builtin_fmaf(t, poly, -0.284496736f);
  poly = __builtin_fmaf(t, poly, 0.254829592f);
  poly *= t;
  const float y = 1.f - poly * __builtin_amdgcn_exp2f(-ax * ax * kLog2e);
  return copysignf(y, x);
}

constexpr int kBJ = 128;
constexpr int kBK = 64;
typedef XorTile<kBJ, kBK / 8, false> GemmTileQ;         // Q operand tile: 128 rows x 64 k

// Row tile of BI (128 or 64) P rows; the four waves form a 2 x 2 grid of
// (BI/2) x 64 output blocks.
template <int BI>
struct GemmCfg {
  typedef XorTile<BI, kBK / 8, false> TileP;
  static constexpr int LOADS = TileP::LOADS + GemmTileQ::LOADS;
  static constexpr int PER_WAVE = (LOADS + 3) / 4;      // wave loads per wave per stage
  static constexpr int NA = BI / 32;                    // 16-row MFMA blocks per wave
  static constexpr int STAGE = TileP::BYTES + GemmTileQ::BYTES;
};

struct GemmSeg {
  const void* p0;
  const void* p1;
  int64_t p_split;
  const void* q;
  int64_t I, J, K;
  const void* bias;
  int bias_dtype;
  int mode;
  void* out;
  int64_t ldo;
  int64_t T, Tp, vt_stride_b;
  int act;               // mode 0: kGemmActGelu applies the exact GELU after the bias
  const void* residual;  // mode 0: nullptr, or added to the output (same layout as out)
  int tiles_i, tiles_j, tiles;
};

struct GemmParams {
  GemmSeg seg[2];
  int nseg;
  int gemm_blocks;     // workgroups of GEMM tiles, after those that run `norm`
  NormJob norm;
};

// Virtual token i0 + off of the value segment as (sequence, token): the tile's
// first row is split once per workgroup (b0, t0 = i0 = b0*Tp + t0), and a row
// offset below 2*Tp (tiles are <= 128 rows, Tp >= 64) wraps at most twice.
struct VToken {
  int64_t b;
  int64_t t;
};
__device__ __forceinline__ VToken vtoken(int64_t b0, int64_t t0, int64_t off, int64_t Tp) {
  VToken v{b0, t0 + off};
  while (v.t >= Tp) {
    v.t -= Tp;
    ++v.b;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ const T* p_row(const GemmSeg& sg, int64_t i0, int64_t b0, int64_t t0, int off) {
  const T* p0 = static_cast<const T*>(sg.p0);
  if (sg.mode == 1) {     // virtual token i = b * Tp + t of the value segment
    VToken v = vtoken(b0, t0, off, sg.Tp);
    if (i0 + off >= sg.I) v = VToken{sg.I / sg.Tp - 1, sg.Tp - 1};   // rows of a partial last tile
    return p0 + (v.b * sg.T + min(v.t, sg.T - 1)) * sg.K;
  }
  const int64_t i = min(i0 + off, sg.I - 1);   // rows of a partial last tile are computed but never stored
  return i < sg.p_split ? p0 + i * sg.K : static_cast<const T*>(sg.p1) + (i - sg.p_split) * sg.K;
}

// EPI: kGemmActGelu applies GELU after the bias (mode 0); EPI_RES adds the
// segment's residual (mode 0).  Launches without either compile neither.
constexpr int kEpiResidual = 2;

template <typename T, int BI, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams prm) {
  typedef typename Elem<T>::v8 v8;
  typedef GemmCfg<BI> Cfg;
  typedef typename Cfg::TileP TileP;
  constexpr int STAGE = Cfg::STAGE;            // P tile, then Q tile
  constexpr int NA = Cfg::NA;
  // Stage buffers: three for 64-row tiles (two workgroups still share a
  // CU), two for 96- and 128-row tiles.
  constexpr int NST = BI == 64 ? 3 : 2;
  static_assert(2 * STAGE >= kNormLdsBytes, "a normalization workgroup reuses the stage buffers");
  __shared__ __attribute__((aligned(1024))) char lds[NST * STAGE];
  char* const lds0 = lds;
  char* const lds1 = lds + STAGE;

  // The normalization's workgroups come first: they start with the first
  // round of tiles instead of after it.
  const int n_norm = norm_blocks(prm.norm);
  if (static_cast<int>(blockIdx.x) < n_norm) {
    normalize_block(prm.norm, static_cast<int>(blockIdx.x), lds);
    return;
  }
  const int w = static_cast<int>(blockIdx.x) - n_norm;
  // XCD-aware order: workgroup w runs on XCD (w + n_norm) % kXcds
  // (round-robin dispatch), so the workgroups of one residue of w take one
  // contiguous range of tiles.  Inside a segment consecutive tiles share their
  // block of the larger operand, which the XCD's L2 then fetches once.
  const int xcd = w % kXcds;
  const int per = prm.gemm_blocks / kXcds, rem = prm.gemm_blocks % kXcds;
  int tile = xcd * per + min(xcd, rem) + w / kXcds;
  const int si = (prm.nseg > 1 && tile >= prm.seg[0].tiles) ? 1 : 0;
  if (si) tile -= prm.seg[0].tiles;
  const GemmSeg& sg = prm.seg[si];
  const bool i_fast = sg.tiles_i <= sg.tiles_j;
  const int64_t i0 = static_cast<int64_t>(i_fast ? tile % sg.tiles_i : tile / sg.tiles_j) * BI;
  const int64_t j0 = static_cast<int64_t>(i_fast ? tile / sg.tiles_i : tile % sg.tiles_j) * kBJ;
  // Value segment: the tile's first virtual token, split once (uniform).
  const int64_t b0 = sg.mode == 1 ? static_cast<int>(i0) / static_cast<int>(sg.Tp) : 0;   // rows fit in int
  const int64_t t0 = sg.mode == 1 ? i0 - b0 * sg.Tp : 0;

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int wi = wave & 1;
  const int wj = wave >> 1;
  const int K = static_cast<int>(sg.K);
  const int n_stages = (K + kBK - 1) / kBK;

  // This wave's DMA sources for stage k0 = 0: wave load j < TileP::LOADS
  // fills the P tile, the rest the Q tile; only the k offset moves between
  // stages.  A partial last round (j >= LOADS) re-loads wave load 0's data
  // into slot 0.
  const T* src[Cfg::PER_WAVE];
  int kchunk[Cfg::PER_WAVE];
  int slot[Cfg::PER_WAVE];
#pragma unroll
  for (int n = 0; n < Cfg::PER_WAVE; ++n) {
    const int j0w = n * 4 + wave;
    const int j = j0w < Cfg::LOADS ? j0w : 0;
    slot[n] = j * 1024;
    int r, ck;
    if (j < TileP::LOADS) {
      TileP::slot_chunk(j * 64 + lane, r, ck);
      src[n] = p_row<T>(sg, i0, b0, t0, r);
    } else {
      GemmTileQ::slot_chunk((j - TileP::LOADS) * 64 + lane, r, ck);
      src[n] = static_cast<const T*>(sg.q) + min(j0 + r, sg.J - 1) * sg.K;
    }
    kchunk[n] = ck * 8;
  }
  auto issue = [&](char* buf, int k0) {
    // Columns past K only occur in a final half stage that is never read.
    const bool tail = k0 + kBK > K;
#pragma unroll
    for (int n = 0; n < Cfg::PER_WAVE; ++n) {
      const int kc = tail ? min(k0 + kchunk[n], K - 8) : k0 + kchunk[n];
      dma16(src[n] + kc, buf + slot[n]);
    }
  };

  // Bias of this lane's outputs, fetched ahead of the K loop without
  // branches (clamped or dummy indices, valid addresses only), so the
  // epilogue finds it landed: slot a*4 + r holds i = ... + a*16 + 4g + r
  // (mode 0), slot b the j = ... + b*16 + c (mode 1).
  constexpr int WI = BI / 2;                 // i extent of a wave's block
  const bool has_bias = sg.bias != nullptr;
  const void* bsrc = has_bias ? sg.bias : sg.q;
  const int bdt = has_bias ? sg.bias_dtype : kF16;
  ScalarHalves bias_raw[NA * 4];
#pragma unroll
  for (int k = 0; k < NA * 4; ++k) {
    const int64_t i = min(i0 + wi * WI + (k / 4) * 16 + 4 * g + k % 4, sg.I - 1);
    const int64_t j = min(j0 + wj * 64 + (k % 4) * 16 + c, sg.J - 1);
    const int64_t idx = !has_bias ? 0 : sg.mode == 0 ? i : k < 4 ? j : 0;
    bias_raw[k] = fetch_scalar(bsrc, bdt, idx);
  }

  f32x4 acc[NA][4];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

  // Lane (c, g)'s fragment bases for chunk groups kk = 0, 1 (chunk 4kk + g of
  // its row); 16-row blocks add XorTile::ROW_BLOCK.
  const int afrag[2] = {TileP::base(wi * (BI / 2) + c, g, 0), TileP::base(wi * (BI / 2) + c, g, 1)};
  const int bfrag[2] = {TileP::BYTES + GemmTileQ::base(wj * 64 + c, g, 0),
                        TileP::BYTES + GemmTileQ::base(wj * 64 + c, g, 1)};

  // A ring of NST stage buffers: step st reads stage st (buffer st % NST) and
  // issues stage st + NST - 1 into the buffer stage st - 1 used, so a stage
  // has NST - 1 steps to land.  The step waits for its own stage only (the
  // later one stays in flight across the barrier), reads every fragment of
  // it (LDS latency paid once), issues the next stage, then runs the MFMAs.
  // A final half stage (K % 64 == 32) takes one 32-deep step.
  auto step = [&](int st, char* cur, char* nxt) {
    if (NST == 3 && st + 1 < n_stages) {
      wait_vmem_at_most<Cfg::PER_WAVE>();   // stage st + 1 may stay in flight
    } else {
      wait_vmem();
    }
    lds_barrier();
    const bool full = K - st * kBK >= kBK;
    v8 af[2][NA], bf[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kk == 1 && !full) break;
#pragma unroll
      for (int a = 0; a < NA; ++a) af[kk][a] = lds_v8<T>(cur + afrag[kk] + a * TileP::ROW_BLOCK);
#pragma unroll
      for (int b = 0; b < 4; ++b) bf[kk][b] = lds_v8<T>(cur + bfrag[kk] + b * GemmTileQ::ROW_BLOCK);
    }
    if (st + NST - 1 < n_stages) issue(nxt, (st + NST - 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kk == 1 && !full) break;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = Elem<T>::mma(af[kk][a], bf[kk][b], acc[a][b]);
    }
  };

  if constexpr (NST == 2) {
    issue(lds0, 0);
    int st = 0;
    for (; st + 1 < n_stages; st += 2) {
      step(st, lds0, lds1);
      step(st + 1, lds1, lds0);
    }
    if (st < n_stages) step(st, lds0, lds1);
  } else {
    char* const lds2 = lds + 2 * STAGE;
    issue(lds0, 0);
    if (n_stages > 1) issue(lds1, kBK);
    int st = 0;
    for (; st + 2 < n_stages; st += 3) {
      step(st, lds0, lds2);
      step(st + 1, lds1, lds0);
      step(st + 2, lds2, lds1);
    }
    if (st < n_stages) step(st, lds0, lds2);
    if (st + 1 < n_stages) step(st + 1, lds1, lds0);
  }

  // Epilogue.  Lane (c, g) holds D[i0 + wi*BI/2 + a*16 + 4g + r][j0 + wj*64 + b*16 + c],
  // r = 0..3: four consecutive i of one j.  Both output layouts run along i
  // for a fixed j (mode 0: out[j*ldo + i]; mode 1: 32-token runs of V^T), so
  // each wave stages its block in LDS as [j][i] rows and writes them back as
  // 16-byte chunks, eight lanes per 128-byte row segment.
  constexpr int ROWB = WI * 2 + 16;          // bytes per staged j row (padded)
  static_assert(64 * ROWB <= STAGE, "a wave's staging block must fit one stage buffer");
  __syncthreads();                           // every wave is done reading the stage buffers
  char* stage_w = (wave < 2 ? lds0 : lds1) + (wave & 1) * (STAGE / 2);
  static_assert(2 * 64 * ROWB <= STAGE, "two waves share one stage buffer");
  float bias_i[NA][4];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = i0 + wi * WI + a * 16 + 4 * g + r;
      bias_i[a][r] = (sg.mode == 0 && has_bias && i < sg.I) ? scalar_value(bias_raw[a * 4 + r], bdt) : 0.f;
    }
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t j = j0 + wj * 64 + b * 16 + c;
    const float bj = (sg.mode == 1 && has_bias && j < sg.J) ? scalar_value(bias_raw[b], bdt) : 0.f;
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      typename Elem<T>::v4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = acc[a][b][r] + bias_i[a][r] + bj;
        if constexpr ((EPI & kGemmActGelu) != 0) v = 0.5f * v * (1.f + erf_fast(v * 0.70710678118654752f));
        o[r] = static_cast<T>(v);
      }
      *reinterpret_cast<typename Elem<T>::v4*>(stage_w + (b * 16 + c) * ROWB + (a * 16 + 4 * g) * 2) = o;
    }
  }
  // Same-wave LDS round trip: the stores above complete before the loads below.
  T* out = static_cast<T*>(sg.out);
  constexpr int CHUNKS = WI / 8;             // 16-byte chunks per staged row
  constexpr int ROWS_PER_PASS = 64 / CHUNKS;   // 16, 10 or 8 rows (WI 32, 48, 64)
  constexpr int PASSES = (64 + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    const int jr = pass * ROWS_PER_PASS + lane / CHUNKS;   // staged row (j)
    // With 48-row blocks a pass covers 60 lanes' chunks and the last pass
    // 4 rows; other lanes have no chunk.
    if (lane >= ROWS_PER_PASS * CHUNKS || jr >= 64) continue;
    const int ic = (lane % CHUNKS) * 8;                     // first i of the chunk
    const int64_t j = j0 + wj * 64 + jr;
    const int64_t i = i0 + wi * WI + ic;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage_w + jr * ROWB + ic * 2);
    if (j >= sg.J || i >= sg.I) continue;
    if (sg.mode == 0) {
      T* dst = out + j * sg.ldo + i;
      const bool full = i + 8 <= sg.I;   // else I % 4 == 0: a last half chunk
      u32x4 w = v;
      if constexpr ((EPI & kEpiResidual) != 0) {
        // out = residual + (rounded) result, rounded again: the order of the
        // unfused `x + linear(...)` in the output dtype.
        const T* res = static_cast<const T*>(sg.residual) + j * sg.ldo + i;
        u32x4 rv = full ? *reinterpret_cast<const u32x4*>(res) : u32x4{reinterpret_cast<const uint2*>(res)->x,
                                                                    reinterpret_cast<const uint2*>(res)->y, 0u, 0u};
        const v8 a = __builtin_bit_cast(v8, v);
        const v8 b = __builtin_bit_cast(v8, rv);
        v8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = static_cast<T>(static_cast<float>(a[e]) + static_cast<float>(b[e]));
        w = __builtin_bit_cast(u32x4, o);
      }
      if (full) {
        store16B(dst, w);
      } else {
        *reinterpret_cast<uint2*>(dst) = uint2{w[0], w[1]};
      }
    } else {
      // Eight consecutive virtual tokens of one sequence and one 32-token
      // tile (Tp % 64 == 0, i % 8 == 0).
      const VToken vt = vtoken(b0, t0, i - i0, sg.Tp);
      store16B(out + vt.b * sg.vt_stride_b + (vt.t >> 5) * 32 * sg.J + 32 * j + (vt.t & 31), v);
    }
  }
}

template <int BI>
static int setup_gemm(const GemmSegment* segs, int nseg, GemmParams& prm) {
  prm.nseg = nseg;
  int total = 0;
  for (int s = 0; s < nseg; ++s) {
    GemmSeg& d = prm.seg[s];
    const GemmSegment& a = segs[s];
    d.p0 = a.p0;
    d.p1 = a.p1 ? a.p1 : a.p0;
    d.p_split = a.p1 ? a.p_split : a.I;
    d.q = a.q;
    d.mode = a.mode;
    d.T = a.T > 0 ? a.T : 1;
    d.Tp = a.Tp > 0 ? a.Tp : 1;
    // The value segment runs over B * Tp virtual tokens (a.I = B * T real ones).
    d.I = a.mode == 1 ? (a.I / d.T) * d.Tp : a.I;
    d.J = a.J;
    d.K = a.K;
    d.bias = a.bias;
    d.bias_dtype = a.bias_dtype;
    d.out = a.out;
    d.ldo = a.ldo;
    d.vt_stride_b = a.vt_stride_b;
    d.act = a.act;
    d.residual = a.residual;
    d.tiles_i = static_cast<int>((d.I + BI - 1) / BI);
    d.tiles_j = static_cast<int>((a.J + kBJ - 1) / kBJ);
    d.tiles = d.tiles_i * d.tiles_j;
    total += d.tiles;
  }
  if (nseg == 1) prm.seg[1] = prm.seg[0];
  return total;
}

template <typename T, int BI>
static void launch_gemm_k(const GemmParams& prm, int total, int nb, hipStream_t stream) {
  // Every segment of a launch shares its epilogue (only single-segment
  // launches ask for GELU or a residual).
  const int epi = (prm.seg[0].act == kGemmActGelu ? kGemmActGelu : 0) | (prm.seg[0].residual ? kEpiResidual : 0);
  const dim3 grid(static_cast<unsigned>(total + nb));
  switch (epi) {
    case 0: hipLaunchKernelGGL((gemm_kernel<T, BI, 0>), grid, dim3(256), 0, stream, prm); break;
    case kGemmActGelu: hipLaunchKernelGGL((gemm_kernel<T, BI, kGemmActGelu>), grid, dim3(256), 0, stream, prm); break;
    case kEpiResidual: hipLaunchKernelGGL((gemm_kernel<T, BI, kEpiResidual>), grid, dim3(256), 0, stream, prm); break;
    default:
      hipLaunchKernelGGL((gemm_kernel<T, BI, kGemmActGelu | kEpiResidual>), grid, dim3(256), 0, stream, prm);
      break;
  }
}

// 128-row tiles when the grid holds two workgroups per CU, else 64-row tiles
// (twice the workgroups, so two share every CU and hide each other's waits),
// or 96-row tiles where 64-row ones would need a second, partial round of
// the 512 workgroup slots and 96-row ones fill at least three quarters of
// one (e.g. 4096 x 512 -> 1536: 768 tiles of 64 rows, 512 of 96).
// `norm` (or nullptr) adds a dictionary normalization's workgroups.
constexpr int kGemmSlots = 512;   // two workgroups per CU
void launch_gemm(const GemmSegment* segs, int nseg, int dtype, hipStream_t stream, const NormJob* norm) {
  GemmParams prm;
  const int tiles128 = setup_gemm<128>(segs, nseg, prm);
  prm.norm = norm ? *norm : NormJob{};
  const int nb = norm_blocks(prm.norm);
  if (tiles128 + nb == 0) return;
  const bool f16 = dtype == kF16;
  if (tiles128 >= kGemmSlots) {
    prm.gemm_blocks = tiles128;
    f16 ? launch_gemm_k<_Float16, 128>(prm, tiles128, nb, stream) : launch_gemm_k<__bf16, 128>(prm, tiles128, nb, stream);
    return;
  }
  const int tiles96 = setup_gemm<96>(segs, nseg, prm);
  const int tiles64 = setup_gemm<64>(segs, nseg, prm);
  // (Plain linears only: the Q/K/V launch's V^T segment keeps 64-row tiles.)
  const bool plain = nseg == 1 && segs[0].mode == 0;
  if (plain && tiles64 + nb > kGemmSlots && tiles96 + nb <= kGemmSlots && 4 * (tiles96 + nb) >= 3 * kGemmSlots) {
    setup_gemm<96>(segs, nseg, prm);
    prm.gemm_blocks = tiles96;
    f16 ? launch_gemm_k<_Float16, 96>(prm, tiles96, nb, stream) : launch_gemm_k<__bf16, 96>(prm, tiles96, nb, stream);
    return;
  }
  prm.gemm_blocks = tiles64;
  f16 ? launch_gemm_k<_Float16, 64>(prm, tiles64, nb, stream) : launch_gemm_k<__bf16, 64>(prm, tiles64, nb, stream);
}

}  // namespace da
