// Fused dictionary route: one launch per Q/K row set.
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
// key atoms, values = value atoms), so it runs as a flash-style loop over
// 64-atom tiles with an online softmax; no [rows, M] logits or weights ever
// reach memory.  Work is done in the transposed domain so that the softmax
// tile produced by the first MFMA is directly the B operand of the second:
//   S^T[j, c] = sum_r Dk^T[j, r] X^T[r, c]      (A = key atoms from LDS, B = rows in VGPRs)
//   O^T[r, c] += sum_j Dv[r, j] P^T[j, c]       (A = value atoms from LDS, B = P in VGPRs)
// One wave owns 16 rows (the 16 MFMA columns); a workgroup of NW waves shares
// each dictionary tile through LDS.  The per-row input scale beta/||x|| is
// applied to the fp32 logits, so the input is never re-rounded after
// normalization.
#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kRouteAtomTile = 64;
constexpr int kRouteKeyPad = 8;    // elements of padding per key-atom row in LDS
constexpr int kRouteValPad = 8;    // elements of padding per value row in LDS

template <typename T, int R, int NW>
__global__ __launch_bounds__(NW * 64) void route_kernel(
    const T* x, int64_t rows, int64_t x_stride, const T* __restrict__ key_t,
    const T* __restrict__ value, int M, int Mp, const void* __restrict__ beta_ptr, int beta_dtype,
    float beta_value, float eps, int flags, T* out, int64_t out_stride) {
  // x and out may alias (in-place routing); every row is read into VGPRs by
  // its own wave before that wave writes it.
  typedef typename Elem<T>::v8 v8;
  constexpr int KS = R / 32;                     // 32-wide k steps over the routing dim
  constexpr int KROW = R + kRouteKeyPad;         // LDS row pitch of a key atom
  constexpr int VROW = kRouteAtomTile + kRouteValPad;
  __shared__ __attribute__((aligned(16))) T ks[kRouteAtomTile * KROW];
  __shared__ __attribute__((aligned(16))) T vs[R * VROW];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * NW + wave_id()) * 16 + c;
  const bool row_ok = row < rows;

  // Row fragment (B operand of the assignment contraction), kept in VGPRs.
  v8 xf[KS];
  float ss = 0.f;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    xf[kk] = row_ok ? load8(x + row * x_stride + kk * 32 + 8 * g) : zero8<T>();
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = static_cast<float>(xf[kk][e]);
      ss += v * v;
    }
  }
  ss = group_sum(ss);

  float beta = beta_ptr ? load_scalar(beta_ptr, beta_dtype, 0) : beta_value;
  if (flags & kRouteBetaIsLog) beta = expf(fminf(fmaxf(beta, kLogBetaMin), kLogBetaMax));
  const float inv_norm = (flags & kRouteNormalizeInput) ? 1.f / fmaxf(sqrtf(ss), eps) : 1.f;
  const float scale = beta * inv_norm * kLog2e;   // logits -> log2-domain softmax exponents

  f32x4 acc[R / 16];
#pragma unroll
  for (int i = 0; i < R / 16; ++i) acc[i] = zero4();
  float m_run = -INFINITY;
  float l_part = 0.f;   // this lane's share of the softmax denominator

  for (int j0 = 0; j0 < Mp; j0 += kRouteAtomTile) {
    __syncthreads();
    // Stage the key tile [64 atoms, R] and the value tile [R, 64 atoms].
    for (int ch = threadIdx.x; ch < kRouteAtomTile * (R / 8); ch += NW * 64) {
      const int a = ch / (R / 8);
      const int k8 = ch % (R / 8);
      store16B(&ks[a * KROW + k8 * 8], load16B(key_t + static_cast<int64_t>(j0 + a) * R + k8 * 8));
    }
    for (int ch = threadIdx.x; ch < R * (kRouteAtomTile / 8); ch += NW * 64) {
      const int r = ch / (kRouteAtomTile / 8);
      const int a8 = ch % (kRouteAtomTile / 8);
      store16B(&vs[r * VROW + a8 * 8], load16B(value + static_cast<int64_t>(r) * Mp + j0 + a8 * 8));
    }
    __syncthreads();

    // Assignment logits for 64 atoms x 16 rows.
    f32x4 s[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 t = zero4();
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        t = Elem<T>::mma(load8(&ks[(b * 16 + c) * KROW + kk * 32 + 8 * g]), xf[kk], t);
      s[b] = t;
    }

    float tmax = -INFINITY;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int atom = j0 + b * 16 + 4 * g + i;
        const float v = atom < M ? s[b][i] * scale : -INFINITY;
        s[b][i] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    const float m_new = fmaxf(m_run, group_max(tmax));
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = exp2f(s[b][i] - m_new);
        s[b][i] = p;
        psum += p;
      }
    }
    l_part = l_part * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < R / 16; ++i) acc[i] *= alpha;

    const v8 p0 = pack_blocked<T>(s[0], s[1]);
    const v8 p1 = pack_blocked<T>(s[2], s[3]);
#pragma unroll
    for (int rb = 0; rb < R / 16; ++rb) {
      const T* vrow = &vs[(rb * 16 + c) * VROW];
      acc[rb] = Elem<T>::mma(load_blocked<T>(vrow, g), p0, acc[rb]);
      acc[rb] = Elem<T>::mma(load_blocked<T>(vrow + 32, g), p1, acc[rb]);
    }
  }

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
    T* orow = out + row * out_stride;
#pragma unroll
    for (int rb = 0; rb < R / 16; ++rb) {
      typename Elem<T>::v4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = static_cast<T>(acc[rb][i] * out_scale);
      *reinterpret_cast<typename Elem<T>::v4*>(orow + rb * 16 + 4 * g) = o;
    }
  }
}

template <typename T, int R>
static void launch_route_r(const RouteArgs& a, hipStream_t s) {
  constexpr int NW = 4;
  const int64_t blocks = (a.rows + NW * 16 - 1) / (NW * 16);
  hipLaunchKernelGGL((route_kernel<T, R, NW>), dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), 0,
                     s, static_cast<const T*>(a.x), a.rows, a.x_stride,
                     static_cast<const T*>(a.key_t), static_cast<const T*>(a.value), a.M,
                     round_up(a.M, kAtomPad), a.beta_ptr, a.beta_dtype, a.beta_value, a.eps,
                     a.flags, static_cast<T*>(a.out), a.out_stride);
}

template <typename T>
static void launch_route_t(const RouteArgs& a, hipStream_t s) {
  switch (a.R) {
    case 64: launch_route_r<T, 64>(a, s); break;
    case 128: launch_route_r<T, 128>(a, s); break;
    case 256: launch_route_r<T, 256>(a, s); break;
    default: launch_route_r<T, 512>(a, s); break;
  }
}

void launch_dictionary_route(const RouteArgs& a, hipStream_t stream) {
  if (a.rows == 0) return;
  if (a.dtype == kF16) launch_route_t<_Float16>(a, stream);
  else launch_route_t<__bf16>(a, stream);
}

}  // namespace da
