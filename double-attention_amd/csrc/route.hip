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
// One wave owns 16 rows; the four waves of a workgroup share each dictionary
// tile, which is double-buffered in LDS and filled by global->LDS DMA while the
// previous tile is multiplied.  The input scale beta/||x|| is applied before
// the single rounding of the unit row.
//
// Element types: TX = input rows, TK = key atoms and the normalized input (fp16
// when the input is L2-normalized, since |u_i| <= 1; else TX), value atoms and
// the softmax weights are fp16 (both bounded by 1), TO = output rows.
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

template <int R>
struct RouteTile {
  static constexpr int AT = R >= 512 ? 32 : 64;   // atoms per tile
  static constexpr int NCK = R / 8;              // chunks per key-atom row
  static constexpr int KCH = AT * NCK;
  static constexpr int VCK = AT / 8;             // chunks per value row
  static constexpr int VCH = R * VCK;
  static constexpr int BYTES = (KCH + VCH) * 16;
  static_assert(KCH % 256 == 0 && VCH % 256 == 0, "tile must split evenly over 256 lanes");
};

template <typename TX, typename TK, typename TO, int R>
__global__ __launch_bounds__(256) void route_kernel(
    const TX* x, int64_t rows, int64_t x_stride, const TK* __restrict__ key_t,
    const _Float16* __restrict__ value, int M, int Mp, const void* __restrict__ beta_ptr,
    int beta_dtype, float beta_value, float eps, int flags, TO* out, int64_t out_stride) {
  // x and out may alias (in-place routing): every row is read into VGPRs by
  // its own wave before that wave writes it.
  typedef RouteTile<R> Tile;
  typedef typename Elem<TK>::v8 k8;
  constexpr int KS = R / 32;
  constexpr int AT = Tile::AT;
  __shared__ __attribute__((aligned(1024))) char lds0[Tile::BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * 16 + c;
  const bool row_ok = row < rows;
  const int n_tiles = Mp / AT;

  auto issue = [&](char* buf, int j0) {
#pragma unroll
    for (int i = 0; i < Tile::KCH / 256; ++i) {
      const int j = i * 4 + wave;
      int a, ck;
      chunk_of<Tile::NCK, true>(j * 64 + lane, a, ck);
      dma16(key_t + static_cast<int64_t>(j0 + a) * R + ck * 8, buf + j * 1024);
    }
#pragma unroll
    for (int i = 0; i < Tile::VCH / 256; ++i) {
      const int j = i * 4 + wave;
      int r, ck;
      chunk_of<Tile::VCK, false>(j * 64 + lane, r, ck);
      dma16(value + static_cast<int64_t>(r) * Mp + j0 + ck * 8, buf + Tile::KCH * 16 + j * 1024);
    }
  };
  issue(lds0, 0);

  // Row fragment (B operand of the assignment contraction), kept in VGPRs.
  typename Elem<TX>::v8 xr[KS];
  float ss = 0.f;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    xr[kk] = row_ok ? load8(x + row * x_stride + kk * 32 + 8 * g) : zero8<TX>();
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = static_cast<float>(xr[kk][e]);
      ss += v * v;
    }
  }
  ss = group_sum(ss);
  float beta = beta_ptr ? load_scalar(beta_ptr, beta_dtype, 0) : beta_value;
  if (flags & kRouteBetaIsLog) beta = expf(fminf(fmaxf(beta, kLogBetaMin), kLogBetaMax));
  const bool norm_in = flags & kRouteNormalizeInput;
  const float inv_norm = norm_in ? 1.f / fmaxf(sqrtf(ss), eps) : 1.f;
  // With input normalization the unit row is rounded once to TK; otherwise
  // TK == TX and the raw row passes through unchanged.
  k8 xf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) xf[kk][e] = static_cast<TK>(static_cast<float>(xr[kk][e]) * inv_norm);
  const float scale = beta * kLog2e;   // logits -> log2-domain exponents

  f32x4 acc[R / 16];
#pragma unroll
  for (int i = 0; i < R / 16; ++i) acc[i] = zero4();
  float m_run = -INFINITY;
  float l_part = 0.f;   // this lane's share of the softmax denominator

  auto step = [&](int t, char* cur, char* nxt) {
    wait_vmem();
    __syncthreads();
    if (t + 1 < n_tiles) issue(nxt, (t + 1) * AT);
    const int j0 = t * AT;
    // Logits: AT/16 independent accumulator chains, fragments read from LDS
    // in batches ahead of their MFMAs.
    constexpr int NB = AT / 16;
    f32x4 s[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) s[kb] = zero4();
    {
      constexpr int KB = NB == 4 ? 2 : 4;   // k-steps per batch (8 fragments in flight)
#pragma unroll
      for (int kk0 = 0; kk0 < KS; kk0 += KB) {
        u32x4 a[KB][NB];
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
          for (int kb = 0; kb < NB; ++kb)
            a[i][kb] = lds_chunk<Tile::NCK, true>(cur, blocked_row(kb, c), (kk0 + i) * 4 + g);
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
          for (int kb = 0; kb < NB; ++kb) s[kb] = Elem<TK>::mma(as_v8<TK>(a[i][kb]), xf[kk0 + i], s[kb]);
      }
    }
    // Lane (c, g) holds atoms j0 + 32*(kb/2) + 8g + 4*(kb%2) + i of row c.
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < AT / 16; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int atom = j0 + 32 * (kb >> 1) + 8 * g + 4 * (kb & 1) + i;
        const float v = atom < M ? s[kb][i] * scale : -INFINITY;
        s[kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    lazy_rescale<R / 16>(group_max(tmax), m_run, l_part, acc);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < AT / 16; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = exp2f(s[kb][i] - m_run);
        s[kb][i] = pr;
        psum += pr;
      }
    }
    l_part += psum;
    const char* vtile = cur + Tile::KCH * 16;
    constexpr int RB = R / 16 < 8 ? R / 16 : 8;
#pragma unroll
    for (int w = 0; w < AT / 32; ++w) {
      const f16x8 pb = pack_blocked<_Float16>(s[2 * w], s[2 * w + 1]);   // atoms j0 + 32w + 8g + e
#pragma unroll
      for (int rb0 = 0; rb0 < R / 16; rb0 += RB) {
        u32x4 a[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) a[i] = lds_chunk<Tile::VCK, false>(vtile, (rb0 + i) * 16 + c, 4 * w + g);
#pragma unroll
        for (int i = 0; i < RB; ++i) acc[rb0 + i] = Elem<_Float16>::mma(as_v8<_Float16>(a[i]), pb, acc[rb0 + i]);
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
  const float inv_l = 1.f / group_sum(l_part);
  float out_scale = inv_l;
  if (flags & kRouteNormalizeOutput) {
    float rs = 0.f;
#pragma unroll
    for (int rb = 0; rb < R / 16; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = acc[rb][i] * inv_l;
        rs += v * v;
      }
    rs = group_sum(rs);
    out_scale = inv_l / fmaxf(sqrtf(rs), eps);
  }
  if (row_ok) {
    TO* orow = out + row * out_stride;
#pragma unroll
    for (int rb = 0; rb < R / 16; ++rb) {
      typename Elem<TO>::v4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = static_cast<TO>(acc[rb][i] * out_scale);
      *reinterpret_cast<typename Elem<TO>::v4*>(orow + rb * 16 + 4 * g) = o;
    }
  }
}

template <typename TX, typename TK, typename TO, int R>
static void launch_route_r(const RouteArgs& a, hipStream_t s) {
  const int64_t blocks = (a.rows + 63) / 64;
  hipLaunchKernelGGL((route_kernel<TX, TK, TO, R>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                     static_cast<const TX*>(a.x), a.rows, a.x_stride, static_cast<const TK*>(a.key_t),
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
