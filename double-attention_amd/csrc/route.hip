// Fused dictionary route: one launch for all Q and K rows.
//
// Replaces dictionary_route_reference (reference src/double_attention/ops.py:16-62)
// and its Triton launcher dictionary_route_triton (triton_kernels.py:1984-2019)
// for the identity-activation / softmax-assignment case:
//   u = x / max(||x||, eps)                 (if normalize_input)
//   w = softmax_j(beta * <u, Dk[:, j]>)     over the M atoms
//   r = sum_j w_j Dv[:, j]
//   z = r / max(||r||, eps)                 (if normalize_output)
//
// The route is attention of every row against M "dictionary tokens" (keys =
// key atoms, values = value atoms), so it runs as a flash-style loop over atom
// tiles with an online softmax; no [rows, M] logits or weights reach memory.
// Work happens in the transposed domain so the softmax tile produced by the
// first MFMA is directly the B operand of the second:
//   S^T[j, c] = sum_r Dk^T[j, r] U^T[r, c]      (A = key atoms from LDS, B = rows in VGPRs)
//   O^T[r, c] += sum_j Dv[r, j] P^T[j, c]       (A = value atoms from LDS, B = P in VGPRs)
// The waves of a workgroup (or of each of its two sub-streams, below) share
// each dictionary tile, double-buffered in
// XOR-swizzled LDS tiles (da_tile.h) and filled by global->LDS DMA while the previous
// tile is multiplied.  Each wave owns 16 rows (one MFMA column block), so
// every dictionary fragment read from LDS feeds one MFMA and each wave reads
// the whole of every stage tile of its stream (SUB, below) from LDS.  The
// input scale beta/||x|| is applied before the single rounding of the unit
// row.
//
// Element types: TX = input rows, TK = key atoms and the normalized input (fp16
// when the input is L2-normalized, since |u_i| <= 1; else TX), value atoms and
// the softmax weights are fp16 (both bounded by 1), TO = output rows.  Value
// atoms are stored in 32-atom tiles: coordinate r of atom j at
// value[(j/32)*32*R + 32*r + j%32].
#include <type_traits>

#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kRouteWaves = 4;
constexpr int kRouteQW = 16;    // rows per wave (one MFMA column block)
constexpr int kRouteAT = 32;    // atoms per tile
constexpr int kRouteRows = kRouteWaves * kRouteQW;
// Fixed-reference mode keeps fp16 probabilities in [2^(kP16Lift - 2*beta*log2e), 2^kP16Lift].
constexpr float kP16Lift = 14.f;

template <int R, int NW>
struct RouteTile {
  typedef XorTile<kRouteAT, R / 8, true> KT;        // key atoms (blocked rows)
  typedef XorTile<R, 4, false> VT;                  // value coordinates x atoms (32 per row)
  static constexpr int KPW = (KT::LOADS + NW - 1) / NW;   // loads per wave of NW sharing a tile
  static constexpr int VPW = (VT::LOADS + NW - 1) / NW;
  static constexpr int BYTES = KT::BYTES + VT::BYTES;   // one stage: key atoms, then value atoms
};

// The atom tiles t = 0 .. n_tiles-1 are pipelined like the outer attention:
// stage buffer t%2 holds the key atoms of tile t+1 and the value atoms of tile
// t, so step t forms the logits of tile t+1 (MFMA) while it turns the logits
// of tile t into weights (VALU) and accumulates their reconstruction (MFMA).
//
// SUB = 2 runs two sub-streams of two waves over the same rows, the even and
// the odd atom tiles (the padded atom count is even in tiles), each with its
// own share of every stage; at the end the odd one hands its accumulators to
// the even one through LDS.  Few rows then still spread over every CU.
//
// VAR builds the variants of ops.py:41-61 in: 2 SiLU logits, standardized
// logits (a first pass over all atom tiles gathers each row's logit mean and
// variance, then the pipeline runs again) and the direct-SiLU assignment,
// whose weights need no softmax.
template <typename TX, typename TK, typename TO, int R, int SUB, bool VAR>
__global__ __launch_bounds__(kRouteWaves * 64, R >= 512 || SUB == 2 ? 1 : 2) void route_kernel(
    const TX* x, int64_t rows, int64_t x_stride, const TK* __restrict__ key_t,
    const _Float16* __restrict__ value, int M, int Mp, const void* __restrict__ beta_ptr,
    int beta_dtype, float beta_value, float eps, int flags, float silu_gain, float logit_scale, TO* out,
    int64_t out_stride) {
  // x and out may alias (in-place routing): every row is read into VGPRs by
  // its own wave before that wave writes it.
  static_assert(SUB == 1 || SUB == 2, "one or two sub-streams");
  constexpr int NQW = kRouteWaves / SUB;   // waves of one sub-stream (its row waves)
  typedef RouteTile<R, NQW> Tile;
  typedef typename Tile::KT KT;
  typedef typename Tile::VT VT;
  typedef typename Elem<TK>::v8 k8;
  constexpr int KS = R / 32;
  constexpr int RB = R / 16;           // output row blocks
  constexpr int NL = Tile::KPW + Tile::VPW;
  __shared__ __attribute__((aligned(1024))) char lds_all[2 * SUB * Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int sub = SUB == 1 ? 0 : uniform_wave() / NQW;
  const int wave = uniform_wave() - sub * NQW;
  // The sub-stream's share of the two stage buffers.
  char* const lds0 = lds_all + sub * Tile::BYTES;
  char* const lds1 = lds_all + (SUB + sub) * Tile::BYTES;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * NQW + wave) * kRouteQW;
  // This sub-stream's atom tiles are tile_of(t) = SUB*t + sub, t < n_tiles.
  const int n_tiles = Mp / kRouteAT / SUB;
  auto tile_of = [&](int t) { return SUB * t + sub; };

  // Per-lane DMA sources (byte offsets from the tile's first atom): key load i
  // fills wave load i*4 + wave of the key tile (rows of key_t), value load i
  // the same wave load of the value tile (32-atom tiles of the value bank).
  // Wave loads past a tile's end re-load the data of wave load 0 into slot 0.
  uint32_t kdesc[Tile::KPW], vdesc[Tile::VPW];
#pragma unroll
  for (int i = 0; i < Tile::KPW; ++i) {
    int row, ck;
    const int j = i * NQW + wave;
    KT::slot_chunk((j < KT::LOADS ? j : 0) * 64 + lane, row, ck);
    kdesc[i] = static_cast<uint32_t>((row * R + ck * 8) * sizeof(TK));
  }
#pragma unroll
  for (int i = 0; i < Tile::VPW; ++i) {
    int row, ck;
    const int j = i * NQW + wave;
    VT::slot_chunk((j < VT::LOADS ? j : 0) * 64 + lane, row, ck);
    vdesc[i] = static_cast<uint32_t>(((ck >> 2) * 32 * R + row * 32 + (ck & 3) * 8) * 2);
  }
  auto slot_of = [&](int n) {
    if (n < Tile::KPW) {
      const int j = n * NQW + wave;
      return j < KT::LOADS ? j * 1024 : 0;
    }
    const int j = (n - Tile::KPW) * NQW + wave;
    return KT::BYTES + (j < VT::LOADS ? j * 1024 : 0);
  };
  const char* kbytes = reinterpret_cast<const char*>(key_t);
  const char* vbytes = reinterpret_cast<const char*>(value);
  // Load n of this wave's share of stage {K(tk), V(tv)} (the sub-stream's
  // tiles tk, tv).
  auto issue_one = [&](char* buf, int tk, int tv, int n) {
    if (n < Tile::KPW) {
      dma16(kbytes + static_cast<int64_t>(tile_of(tk)) * kRouteAT * R * sizeof(TK) + kdesc[n], buf + slot_of(n));
    } else {
      dma16(vbytes + static_cast<int64_t>(tile_of(tv)) * kRouteAT * R * 2 + vdesc[n - Tile::KPW], buf + slot_of(n));
    }
  };

  // Prologue: beta and the wave's rows, then the DMA of the keys of tile 0
  // into stage 1's key slot and stage 0 = {K(1), V(0)}, all in one memory
  // round trip.  Rows past the end repeat the last row (never stored).
  const ScalarHalves beta_bits = fetch_scalar(beta_ptr ? beta_ptr : static_cast<const void*>(x),
                                              beta_ptr ? beta_dtype : kF32, 0);
  typename Elem<TX>::v8 xr[KS];
  {
    const int64_t row = min(row0 + c, rows - 1);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) xr[kk] = load8(x + row * x_stride + kk * 32 + 8 * g);
  }
#pragma unroll
  for (int n = 0; n < Tile::KPW; ++n) issue_one(lds1, 0, 0, n);
#pragma unroll
  for (int n = 0; n < NL; ++n) issue_one(lds0, min(1, n_tiles - 1), 0, n);
  // Nothing that uses a loaded value moves above the loads' issue: with DMA
  // in flight, an early use would wait for every load.
  __builtin_amdgcn_sched_barrier(0);
  wait_vmem();

  // Row fragments (B operands of the assignment contraction), kept in VGPRs.
  const float beta_raw = beta_ptr ? scalar_value(beta_bits, beta_dtype) : beta_value;
  const float beta = (flags & kRouteBetaIsLog) ? expf(fminf(fmaxf(beta_raw, kLogBetaMin), kLogBetaMax)) : beta_raw;
  // Logits -> log2-domain exponents.  Maxima are taken of raw logits, so a
  // negative beta is folded into the rows instead (exact).
  const float scale = fabsf(beta) * kLog2e;
  const float sign = beta < 0.f ? -1.f : 1.f;
  // Variants: the sign of beta folds into the rows only where the logits stay
  // linear in them; after a SiLU activation it multiplies the logits, and the
  // direct-SiLU assignment does not use beta.
  const bool silu_logits = VAR && (flags & kRouteSiluLogits);
  const bool standardize = VAR && (flags & kRouteStandardize);
  const bool direct = VAR && (flags & kRouteDirectSilu);
  const float row_sign = silu_logits || direct ? 1.f : sign;
  const float post_sign = silu_logits && !direct ? sign : 1.f;
  k8 xf[KS];
  {
    float ss = 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = static_cast<float>(xr[kk][e]);
        ss += v * v;
      }
    }
    ss = group_sum(ss);
    // With input normalization the unit row is rounded once to TK; otherwise
    // TK == TX and the raw row passes through unchanged.
    const float inv_norm = row_sign * ((flags & kRouteNormalizeInput) ? 1.f / fmaxf(sqrtf(ss), eps) : 1.f);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[kk][e] = static_cast<TK>(static_cast<float>(xr[kk][e]) * inv_norm);
  }

  f32x4 acc[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) acc[i] = zero4();
  float m_run = -INFINITY, l_part = 0.f;

  // Key fragment of chunk group kk, row block kb: one of four per-lane bases
  // plus an immediate (da_tile.h); value block rb: a per-lane base plus 1 KiB
  // per block.
  constexpr int KB = KS < 4 ? KS : 4;
  int kfrag[KB];
#pragma unroll
  for (int k = 0; k < KB; ++k) kfrag[k] = KT::base(c, g, k);
  auto key_frag = [&](const char* tile, int kk, int kb) {
    return lds_v8<TK>(tile + kfrag[kk & 3] + 256 * (kk >> 2) + kb * KT::ROW_BLOCK);
  };
  const int vfrag = KT::BYTES + VT::offset(c, g);

  // Logits of 32 atoms x 16 rows from a key tile in LDS: two accumulator
  // chains; fragments are read in groups (latency paid once per group) and
  // the next stage's loads are spread between them.
  auto logits = [&](const char* kt_lds, f32x4 (&st)[2], auto with_dma, char* nxt, int tk, int tv) {
    st[0] = st[1] = zero4();
    const char* kf = kt_lds;
    constexpr int KG = KS < 4 ? KS : 4;
#pragma unroll
    for (int k0 = 0; k0 < KS; k0 += KG) {
      k8 kfr[KG][2];
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
            if (n * KS / NL == k0 + kk) issue_one(nxt, tk, tv, n);
        }
        st[0] = Elem<TK>::mma(kfr[kk][0], xf[k0 + kk], st[0]);
        st[1] = Elem<TK>::mma(kfr[kk][1], xf[k0 + kk], st[1]);
      }
    }
  };

  __syncthreads();
  f32x4 st_prev[2];
  logits(lds1, st_prev, std::false_type{}, nullptr, 0, 0);

  // 2 SiLU(l) = 2 l / (1 + e^-l).
  auto silu2 = [](float v) { return 2.f * v / (1.f + __builtin_amdgcn_exp2f(-kLog2e * v)); };
  // Standardized logits: (l - mu) * cstd, cstd = logit_scale / sqrt(var + eps).
  float mu = 0.f, cstd = 1.f;
  if (standardize) {
    // First pass: the same pipeline over every atom tile, gathering the sum
    // and sum of squares of each row's (activated) logits over the M atoms.
    float s1 = 0.f, s2 = 0.f;
    for (int t = 0; t < n_tiles; ++t) {
      char* cur = (t & 1) ? lds1 : lds0;
      char* nxt = (t & 1) ? lds0 : lds1;
      const int j0 = tile_of(t) * kRouteAT;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = silu_logits ? silu2(st_prev[kb][i]) : st_prev[kb][i];
          if (j0 + 8 * g + 4 * kb + i < M) {
            s1 += v;
            s2 += v * v;
          }
        }
      wait_vmem();
      __syncthreads();
      logits(cur, st_prev, std::true_type{}, nxt, min(t + 2, n_tiles - 1), min(t + 1, n_tiles - 1));
    }
    s1 = group_sum(s1);
    s2 = group_sum(s2);
    wait_vmem();
    __syncthreads();
    if constexpr (SUB == 2) {
      // Each sub-stream saw half the atom tiles: exchange the partial sums.
      float* xs = reinterpret_cast<float*>(lds_all) + (sub * NQW + wave) * 128;
      xs[lane * 2] = s1;
      xs[lane * 2 + 1] = s2;
      __syncthreads();
      const float* other = reinterpret_cast<const float*>(lds_all) + ((1 - sub) * NQW + wave) * 128;
      s1 += other[lane * 2];
      s2 += other[lane * 2 + 1];
      __syncthreads();
    }
    mu = s1 / static_cast<float>(M);
    const float var = fmaxf(s2 / static_cast<float>(M) - mu * mu, 0.f);
    cstd = logit_scale / sqrtf(var + eps);
    // Second pass: the pipeline restarts at tile 0.
#pragma unroll
    for (int n = 0; n < Tile::KPW; ++n) issue_one(lds1, 0, 0, n);
#pragma unroll
    for (int n = 0; n < NL; ++n) issue_one(lds0, min(1, n_tiles - 1), 0, n);
    wait_vmem();
    __syncthreads();
    logits(lds1, st_prev, std::false_type{}, nullptr, 0, 0);
  }

  // Step modes.  kFixed: every logit is bounded by `bound` (unit rows and unit
  // key atoms, or standardized logits), so the exponents use the fixed
  // reference (bound |beta| - kP16Lift) log2e: weights stay in fp16's normal
  // range and the accumulators are never rescaled.  kLazy: the lazy online
  // rescale.  kDirect: direct-SiLU weights.
  constexpr int kLazy = 0, kFixed = 1, kDirect = 2;
  float bound = 1.f;
  bool bounded = (flags & kRouteNormalizeInput) && (flags & kRouteUnitKeys);
  if constexpr (VAR) {
    if (silu_logits) bound = 1.4621172f;   // max |2 SiLU(l)| over |l| <= 1
    if (standardize) {
      // |l - mu| <= sqrt(M - 1) * std for every atom.
      bound = sqrtf(static_cast<float>(M - 1)) * logit_scale;
      bounded = true;
    }
  }
  auto step = [&](auto mode, int t) {
    constexpr int MODE = decltype(mode)::value;
    char* cur = (t & 1) ? lds1 : lds0;
    char* nxt = (t & 1) ? lds0 : lds1;
    const int j0 = tile_of(t) * kRouteAT;
    if constexpr (VAR) {
      if (silu_logits || standardize || post_sign != 1.f) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = st_prev[kb][i];
            if (silu_logits) v = silu2(v);
            if (standardize) v = (v - mu) * cstd;
            st_prev[kb][i] = v * post_sign;
          }
      }
    }
    // Lane (c, g) holds atoms j0 + 8g + 4kb + i of row c; only the last tile
    // can hold padding atoms (weight zero).
    if (j0 + kRouteAT > M) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (j0 + 8 * g + 4 * kb + i >= M) st_prev[kb][i] = MODE == kDirect ? 0.f : -INFINITY;
    }
    float m_use = 0.f;
    if constexpr (MODE == kFixed) {
      m_use = kP16Lift - bound * scale;
    } else if constexpr (MODE == kLazy) {
      const float lmax = fmaxf(fmaxf(fmaxf(st_prev[0][0], st_prev[0][1]), fmaxf(st_prev[0][2], st_prev[0][3])),
                               fmaxf(fmaxf(st_prev[1][0], st_prev[1][1]), fmaxf(st_prev[1][2], st_prev[1][3])));
      lazy_rescale<RB>(lmax, scale, m_run, l_part, acc);
      // A sub-stream whose tiles so far are all padding (with at most 32
      // atoms, the odd one's only tile) keeps the reference at -inf: its
      // weights are exp2(-inf) = 0 and the merge gives it factor 0.
      m_use = m_run == -INFINITY ? 0.f : -m_run;
    }

    wait_vmem();
    __syncthreads();

    f32x4 st_new[2];
    logits(cur, st_new, std::true_type{}, nxt, min(t + 2, n_tiles - 1), min(t + 1, n_tiles - 1));

    if constexpr (MODE == kDirect) {
      // (2/g) SiLU(g l) = 2 l / (1 + e^(-g l)).
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = st_prev[kb][i];
          st_prev[kb][i] = 2.f * v / (1.f + __builtin_amdgcn_exp2f(-kLog2e * silu_gain * v));
        }
    } else {
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(st_prev[kb][i], scale, m_use));
          st_prev[kb][i] = pr;
          psum += pr;
        }
      l_part += psum;
    }
    const f16x8 pb = pack_blocked<_Float16>(st_prev[0], st_prev[1]);   // atoms j0 + 8g + e

    // O^T += Dv(t) P^T(t).
    const char* vf = cur + vfrag;
    constexpr int VG = RB < 8 ? RB : 8;
#pragma unroll
    for (int r0 = 0; r0 < RB; r0 += VG) {
      f16x8 vfr[VG];
#pragma unroll
      for (int rb = 0; rb < VG; ++rb) vfr[rb] = lds_v8<_Float16>(vf + (r0 + rb) * 1024);
#pragma unroll
      for (int rb = 0; rb < VG; ++rb) acc[r0 + rb] = Elem<_Float16>::mma(vfr[rb], pb, acc[r0 + rb]);
    }
    st_prev[0] = st_new[0];
    st_prev[1] = st_new[1];
  };

  const bool fixed = !direct && bounded && 2.f * bound * scale <= 2.f * kP16Lift;
  if (direct) {
    for (int t = 0; t < n_tiles; ++t) step(std::integral_constant<int, kDirect>{}, t);
  } else if (fixed) {
    for (int t = 0; t < n_tiles; ++t) step(std::integral_constant<int, kFixed>{}, t);
  } else {
    for (int t = 0; t < n_tiles; ++t) step(std::integral_constant<int, kLazy>{}, t);
  }

  if constexpr (SUB == 2) {
    // The odd sub-stream hands its accumulators (unnormalized outputs, their
    // reference and row sums) to the even one through LDS, in the lanes' own
    // order; with the fixed reference both share it, online each scales to
    // the larger running maximum.
    wait_vmem();
    __syncthreads();
    static_assert(NQW * (RB * 256 + 128) * 4 <= 2 * SUB * Tile::BYTES, "the hand-over fits the stage buffers");
    float* xch = reinterpret_cast<float*>(lds_all) + wave * (RB * 256 + 128);
    if (sub == 1) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) *reinterpret_cast<f32x4*>(xch + (rb * 64 + lane) * 4) = acc[rb];
      xch[RB * 256 + lane * 2] = m_run;
      xch[RB * 256 + lane * 2 + 1] = l_part;
    }
    __syncthreads();
    if (sub == 1) return;
    const float m1 = xch[RB * 256 + lane * 2];
    const float l1 = xch[RB * 256 + lane * 2 + 1];
    float f0 = 1.f, f1 = 1.f;
    if (!fixed && !direct) {
      const float M = fmaxf(m_run, m1);
      f0 = m_run == -INFINITY ? 0.f : exp2f(m_run - M);
      f1 = m1 == -INFINITY ? 0.f : exp2f(m1 - M);
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = acc[rb] * f0 + *reinterpret_cast<const f32x4*>(xch + (rb * 64 + lane) * 4) * f1;
    l_part = l_part * f0 + l1 * f1;
  }
  // r = O / l (direct-SiLU: r = O); z = r / max(||r||, eps).
  const float inv_l = direct ? 1.f : 1.f / group_sum(l_part);
  float out_scale = inv_l;
  if (flags & kRouteNormalizeOutput) {
    float rs = 0.f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = acc[rb][i] * inv_l;
        rs += v * v;
      }
    rs = group_sum(rs);
    out_scale = inv_l / fmaxf(sqrtf(rs), eps);
  }
  const int64_t row = row0 + c;
  if (row < rows) {
    TO* orow = out + row * out_stride;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      typename Elem<TO>::v4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = static_cast<TO>(acc[rb][i] * out_scale);
      *reinterpret_cast<typename Elem<TO>::v4*>(orow + rb * 16 + 4 * g) = o;
    }
  }
  // The last step's (redundant) stage loads must land before the workgroup's
  // LDS is released.
  wait_vmem();
}

template <typename TX, typename TK, typename TO, int R, int SUB, bool VAR>
static void launch_route_v(const RouteArgs& a, hipStream_t s) {
  constexpr int rows_per_block = kRouteRows / SUB;
  const int64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((route_kernel<TX, TK, TO, R, SUB, VAR>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kRouteWaves * 64), 0, s, static_cast<const TX*>(a.x), a.rows, a.x_stride,
                     static_cast<const TK*>(a.key_t), static_cast<const _Float16*>(a.value), a.M,
                     static_cast<int>(round_up(a.M, kAtomPad)), a.beta_ptr, a.beta_dtype, a.beta_value, a.eps,
                     a.flags, a.silu_gain, a.logit_scale, static_cast<TO*>(a.out), a.out_stride);
}

template <typename TX, typename TK, typename TO, int R, int SUB>
static void launch_route_s(const RouteArgs& a, hipStream_t s) {
  if (a.flags & (kRouteSiluLogits | kRouteStandardize | kRouteDirectSilu)) {
    launch_route_v<TX, TK, TO, R, SUB, true>(a, s);
  } else {
    launch_route_v<TX, TK, TO, R, SUB, false>(a, s);
  }
}

// Rows that do not give every CU (MI355X: 256) a workgroup of four row waves
// run as two sub-streams (two row waves each) over the even and odd atom
// tiles, up to 256-wide rows (the LDS holds four 512-wide stages only once).
constexpr int64_t kRouteCUs = 256;

template <typename TX, typename TK, typename TO, int R>
static void launch_route_r(const RouteArgs& a, hipStream_t s) {
  if constexpr (R <= 256) {
    if ((a.rows + kRouteRows - 1) / kRouteRows < kRouteCUs) {
      launch_route_s<TX, TK, TO, R, 2>(a, s);
      return;
    }
  }
  launch_route_s<TX, TK, TO, R, 1>(a, s);
}

template <typename TX, typename TK, typename TO>
static void launch_route_t(const RouteArgs& a, hipStream_t s) {
  switch (a.R) {
    case 64: launch_route_r<TX, TK, TO, 64>(a, s); break;
    case 128: launch_route_r<TX, TK, TO, 128>(a, s); break;
    case 256: launch_route_r<TX, TK, TO, 256>(a, s); break;
    default: launch_route_r<TX, TK, TO, 512>(a, s); break;
  }
}

void launch_dictionary_route(const RouteArgs& a, hipStream_t stream) {
  if (a.rows == 0) return;
  // Supported (x, key, out) type triples; the C ABI validates the request.
  if (a.x_dtype == kBF16) {
    if (a.key_dtype == kF16) {
      if (a.out_dtype == kF16) launch_route_t<__bf16, _Float16, _Float16>(a, stream);
      else launch_route_t<__bf16, _Float16, __bf16>(a, stream);
    } else {
      if (a.out_dtype == kF16) launch_route_t<__bf16, __bf16, _Float16>(a, stream);
      else launch_route_t<__bf16, __bf16, __bf16>(a, stream);
    }
  } else {
    launch_route_t<_Float16, _Float16, _Float16>(a, stream);
  }
}

}  // namespace da
