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
// A workgroup of four waves shares each dictionary tile, double-buffered in
// padded LDS tiles (da_tile.h) and filled by global->LDS DMA while the previous
// tile is multiplied.  Each wave owns QW rows (QW/16 MFMA column blocks), so
// every dictionary fragment read from LDS feeds QW/16 MFMAs.  The input scale
// beta/||x|| is applied before the single rounding of the unit row.
//
// Element types: TX = input rows, TK = key atoms and the normalized input (fp16
// when the input is L2-normalized, since |u_i| <= 1; else TX), value atoms and
// the softmax weights are fp16 (both bounded by 1), TO = output rows.  Value
// atoms are stored in 32-atom tiles: coordinate r of atom j at
// value[(j/32)*32*R + 32*r + j%32].
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kRouteWaves = 4;

template <int R>
struct RouteCfg {
  static constexpr int QW = 16;                   // rows per wave
  static constexpr int AT = 32;                   // atoms per tile
  typedef PaddedTile<AT, R / 8, true> KT;         // key atoms (blocked rows)
  typedef PaddedTile<R, AT / 8, false> VT;        // value coordinates x atoms
  static constexpr int LOADS = KT::LOADS + VT::LOADS;
  static constexpr int PER_WAVE = (LOADS + kRouteWaves - 1) / kRouteWaves;
  static constexpr int BYTES = LOADS * 1024;
  static constexpr int ROWS = kRouteWaves * QW;   // rows per workgroup
};

template <typename TX, typename TK, typename TO, int R>
__global__ __launch_bounds__(kRouteWaves * 64) void route_kernel(
    const TX* x, int64_t rows, int64_t x_stride, const TK* __restrict__ key_t,
    const _Float16* __restrict__ value, int M, int Mp, const void* __restrict__ beta_ptr,
    int beta_dtype, float beta_value, float eps, int flags, TO* out, int64_t out_stride) {
  // x and out may alias (in-place routing): every row is read into VGPRs by
  // its own wave before that wave writes it.
  typedef RouteCfg<R> Cfg;
  typedef typename Cfg::KT KT;
  typedef typename Cfg::VT VT;
  typedef typename Elem<TK>::v8 k8;
  constexpr int KS = R / 32;
  constexpr int AT = Cfg::AT;
  constexpr int CB = Cfg::QW / 16;   // column blocks per wave
  constexpr int NB = AT / 16;        // atom blocks per tile
  __shared__ __attribute__((aligned(1024))) char lds0[Cfg::BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[Cfg::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kRouteWaves + wave) * Cfg::QW;
  const int n_tiles = Mp / AT;

  // Per-lane DMA sources relative to the tile's atom offset: key atoms are
  // rows of key_t, value chunks live in 32-atom tiles.
  int desc[Cfg::PER_WAVE];
#pragma unroll
  for (int i = 0; i < Cfg::PER_WAVE; ++i) {
    const int j = i * kRouteWaves + wave;
    int row = 0, ck = 0;
    if (j < KT::LOADS) {
      KT::slot_chunk(j * 64 + lane, row, ck);
      desc[i] = row * R + ck * 8;
    } else if (j < Cfg::LOADS) {
      VT::slot_chunk((j - KT::LOADS) * 64 + lane, row, ck);
      desc[i] = (ck >> 2) * 32 * R + row * 32 + (ck & 3) * 8;
    } else {
      desc[i] = 0;
    }
  }
  auto issue = [&](char* buf, int t) {
    const int j0 = t * AT;
    const TK* ktile = key_t + static_cast<int64_t>(j0) * R;
    const _Float16* vtile = value + static_cast<int64_t>(j0) * R;   // 32-atom tiles: j0/32 * 32R
#pragma unroll
    for (int i = 0; i < Cfg::PER_WAVE; ++i) {
      const int j = i * kRouteWaves + wave;
      if (j < KT::LOADS) dma16(ktile + desc[i], buf + j * 1024);
      else if (j < Cfg::LOADS) dma16(vtile + desc[i], buf + j * 1024);
    }
  };
  issue(lds0, 0);

  // Row fragments (B operands of the assignment contraction), kept in VGPRs.
  const float beta_raw = beta_ptr ? load_scalar(beta_ptr, beta_dtype, 0) : beta_value;
  const float beta = (flags & kRouteBetaIsLog) ? expf(fminf(fmaxf(beta_raw, kLogBetaMin), kLogBetaMax)) : beta_raw;
  // Logits -> log2-domain exponents.  The rescale test compares maxima of raw
  // logits, so a negative beta is folded into the rows instead (exact).
  const float scale = fabsf(beta) * kLog2e;
  const float sign = beta < 0.f ? -1.f : 1.f;
  k8 xf[CB][KS];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int64_t row = row0 + cb * 16 + c;
    typename Elem<TX>::v8 xr[KS];
    float ss = 0.f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      xr[kk] = row < rows ? load8(x + row * x_stride + kk * 32 + 8 * g) : zero8<TX>();
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = static_cast<float>(xr[kk][e]);
        ss += v * v;
      }
    }
    ss = group_sum(ss);
    // With input normalization the unit row is rounded once to TK; otherwise
    // TK == TX and the raw row passes through unchanged.
    const float inv_norm = sign * ((flags & kRouteNormalizeInput) ? 1.f / fmaxf(sqrtf(ss), eps) : 1.f);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[cb][kk][e] = static_cast<TK>(static_cast<float>(xr[kk][e]) * inv_norm);
  }

  f32x4 acc[CB][R / 16];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int i = 0; i < R / 16; ++i) acc[cb][i] = zero4();
  float m_run[CB], l_part[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    m_run[cb] = -INFINITY;
    l_part[cb] = 0.f;
  }

  const int kfrag = KT::offset(c, g);
  const int vfrag = KT::BYTES + VT::offset(c, g);

  auto step = [&](int t, char* cur, char* nxt) {
    wait_vmem();
    __syncthreads();
    if (t + 1 < n_tiles) issue(nxt, t + 1);
    const int j0 = t * AT;

    // Logits: NB x CB independent accumulator chains; each key fragment
    // feeds all CB column blocks.
    f32x4 s[CB][NB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) s[cb][kb] = zero4();
    const char* kf = cur + kfrag;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      k8 a[NB];
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) a[kb] = lds_v8<TK>(kf + KT::offset(16 * kb, kk * 4));
#pragma unroll
      for (int kb = 0; kb < NB; ++kb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) s[cb][kb] = Elem<TK>::mma(a[kb], xf[cb][kk], s[cb][kb]);
    }
    // Lane (c, g) holds atoms j0 + 32*(kb/2) + 8g + 4*(kb%2) + i of row c;
    // only the last tile can hold padding atoms.
    if (j0 + AT > M) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (j0 + 32 * (kb >> 1) + 8 * g + 4 * (kb & 1) + i >= M) s[cb][kb][i] = -INFINITY;
    }
    f16x8 pb[CB][AT / 32];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      float lmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NB; ++kb)
        lmax = fmaxf(lmax, fmaxf(fmaxf(s[cb][kb][0], s[cb][kb][1]), fmaxf(s[cb][kb][2], s[cb][kb][3])));
      lazy_rescale<R / 16>(lmax, scale, m_run[cb], l_part[cb], acc[cb]);
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(s[cb][kb][i], scale, -m_run[cb]));
          s[cb][kb][i] = pr;
          psum += pr;
        }
      }
      l_part[cb] += psum;
#pragma unroll
      for (int w = 0; w < AT / 32; ++w) pb[cb][w] = pack_blocked<_Float16>(s[cb][2 * w], s[cb][2 * w + 1]);
    }

    const char* vf = cur + vfrag;
#pragma unroll
    for (int w = 0; w < AT / 32; ++w) {
#pragma unroll
      for (int rb = 0; rb < R / 16; ++rb) {
        const f16x8 a = lds_v8<_Float16>(vf + VT::offset(16 * rb, 4 * w));
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[cb][rb] = Elem<_Float16>::mma(a, pb[cb][w], acc[cb][rb]);
      }
    }
  };

  int t = 0;
  for (; t + 1 < n_tiles; t += 2) {
    step(t, lds0, lds1);
    step(t + 1, lds1, lds0);
  }
  if (t < n_tiles) step(t, lds0, lds1);

  // r = O / l; z = r / max(||r||, eps).
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const float inv_l = 1.f / group_sum(l_part[cb]);
    float out_scale = inv_l;
    if (flags & kRouteNormalizeOutput) {
      float rs = 0.f;
#pragma unroll
      for (int rb = 0; rb < R / 16; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = acc[cb][rb][i] * inv_l;
          rs += v * v;
        }
      rs = group_sum(rs);
      out_scale = inv_l / fmaxf(sqrtf(rs), eps);
    }
    const int64_t row = row0 + cb * 16 + c;
    if (row < rows) {
      TO* orow = out + row * out_stride;
#pragma unroll
      for (int rb = 0; rb < R / 16; ++rb) {
        typename Elem<TO>::v4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = static_cast<TO>(acc[cb][rb][i] * out_scale);
        *reinterpret_cast<typename Elem<TO>::v4*>(orow + rb * 16 + 4 * g) = o;
      }
    }
  }
}

template <typename TX, typename TK, typename TO, int R>
static void launch_route_r(const RouteArgs& a, hipStream_t s) {
  constexpr int ROWS = RouteCfg<R>::ROWS;
  const int64_t blocks = (a.rows + ROWS - 1) / ROWS;
  hipLaunchKernelGGL((route_kernel<TX, TK, TO, R>), dim3(static_cast<unsigned>(blocks)), dim3(kRouteWaves * 64), 0,
                     s, static_cast<const TX*>(a.x), a.rows, a.x_stride, static_cast<const TK*>(a.key_t),
                     static_cast<const _Float16*>(a.value), a.M, static_cast<int>(round_up(a.M, kAtomPad)),
                     a.beta_ptr, a.beta_dtype, a.beta_value, a.eps, a.flags, static_cast<TO*>(a.out),
                     a.out_stride);
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
