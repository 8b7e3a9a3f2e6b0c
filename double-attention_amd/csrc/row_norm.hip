// Row L2 normalization and its backward: the route's input and output norms
// (F.normalize(x, dim=-1, eps) at reference src/double_attention/ops.py:39 and
// :62; the reference's Triton path has them as _row_l2_normalize /
// _row_l2_normalize_backward, triton_kernels.py:30-45, 553-586).
//
// One wave per row, four rows per workgroup, no barriers.  Each lane takes
// four consecutive elements per 256-element stretch of the row (one 8- or
// 16-byte load per operand), the row sums meet with wave_sum, and a second
// pass over the row (its lines are still in L1/L2) writes the result rounded
// once from fp32:
//   forward   y  = x i,                                 i = 1 / max(|x|, eps)
//   backward  dx = h i - x (<x, h> i^3 [|x| > eps])      (h = dL/dy)
// The backward equals (h - y <y, h>) / |x| where |x| > eps and h / eps
// elsewhere, the gradient of F.normalize.
#include "da_common.h"
#include "da_launch.h"

namespace da {

namespace {

constexpr int kRowWaves = 4;

template <typename T>
struct Quad;
template <>
struct Quad<float> {
  typedef f32x4 V;
};
template <>
struct Quad<_Float16> {
  typedef f16x4 V;
};
template <>
struct Quad<__bf16> {
  typedef bf16x4 V;
};

template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&f)[4]) {
  const typename Quad<T>::V v = *reinterpret_cast<const typename Quad<T>::V*>(p);
  f[0] = static_cast<float>(v[0]);
  f[1] = static_cast<float>(v[1]);
  f[2] = static_cast<float>(v[2]);
  f[3] = static_cast<float>(v[3]);
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float (&f)[4]) {
  typename Quad<T>::V v;
  v[0] = static_cast<T>(f[0]);
  v[1] = static_cast<T>(f[1]);
  v[2] = static_cast<T>(f[2]);
  v[3] = static_cast<T>(f[3]);
  *reinterpret_cast<typename Quad<T>::V*>(p) = v;
}

template <typename TX, typename TO>
__global__ __launch_bounds__(64 * kRowWaves) void row_normalize_kernel(RowNormArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;   // whole waves only: the kernel has no barrier
  const int lane = lane_id();
  const TX* x = static_cast<const TX*>(a.x) + row * a.ld_x;
  TO* y = static_cast<TO*>(a.out) + row * a.ld_out;
  float ss = 0.f;
  for (int c = 4 * lane; c < a.R; c += 256) {
    float f[4];
    load4(x + c, f);
    ss += f[0] * f[0] + f[1] * f[1] + f[2] * f[2] + f[3] * f[3];
  }
  const float inv = 1.f / fmaxf(sqrtf(wave_sum(ss)), a.eps);
  for (int c = 4 * lane; c < a.R; c += 256) {
    float f[4];
    load4(x + c, f);
    f[0] *= inv;
    f[1] *= inv;
    f[2] *= inv;
    f[3] *= inv;
    store4(y + c, f);
  }
}

// SPLIT: the 16-bit result at columns [0, R) and its rounding residual
// (the fp32 value minus the rounded one, rounded) at [R, 2R) of the row.
template <typename TX, typename TG, typename TO, bool SPLIT>
__global__ __launch_bounds__(64 * kRowWaves) void row_normalize_backward_kernel(RowNormArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int lane = lane_id();
  const TX* x = static_cast<const TX*>(a.x) + row * a.ld_x;
  const TG* h = static_cast<const TG*>(a.grad) + row * a.ld_grad;
  TO* dx = static_cast<TO*>(a.out) + row * a.ld_out;
  float ss = 0.f, dot = 0.f;
  for (int c = 4 * lane; c < a.R; c += 256) {
    float f[4], g[4];
    load4(x + c, f);
    load4(h + c, g);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ss += f[e] * f[e];
      dot += f[e] * g[e];
    }
  }
  const float norm = sqrtf(wave_sum(ss));
  dot = wave_sum(dot);
  const float inv = 1.f / fmaxf(norm, a.eps);
  const float coef = norm > a.eps ? dot * inv * inv * inv : 0.f;
  for (int c = 4 * lane; c < a.R; c += 256) {
    float f[4], g[4];
    load4(x + c, f);
    load4(h + c, g);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = g[e] * inv - f[e] * coef;
    store4(dx + c, f);
    if constexpr (SPLIT) {
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] -= static_cast<float>(static_cast<TO>(f[e]));
      store4(dx + a.R + c, f);
    }
  }
}

template <typename TX>
void launch_fwd(const RowNormArgs& a, dim3 grid, hipStream_t s) {
  if (a.out_dtype == kF32) hipLaunchKernelGGL((row_normalize_kernel<TX, float>), grid, dim3(64 * kRowWaves), 0, s, a);
  else if (a.out_dtype == kF16) hipLaunchKernelGGL((row_normalize_kernel<TX, _Float16>), grid, dim3(64 * kRowWaves), 0, s, a);
  else hipLaunchKernelGGL((row_normalize_kernel<TX, __bf16>), grid, dim3(64 * kRowWaves), 0, s, a);
}

template <typename TX, typename TG>
void launch_bwd_g(const RowNormArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(64 * kRowWaves);
  const bool split = a.out_dtype & kOutSplit;
  const int dt = a.out_dtype & ~kOutSplit;
  if (dt == kF32) hipLaunchKernelGGL((row_normalize_backward_kernel<TX, TG, float, false>), grid, block, 0, s, a);
  else if (dt == kF16 && split) hipLaunchKernelGGL((row_normalize_backward_kernel<TX, TG, _Float16, true>), grid, block, 0, s, a);
  else if (dt == kF16) hipLaunchKernelGGL((row_normalize_backward_kernel<TX, TG, _Float16, false>), grid, block, 0, s, a);
  else if (split) hipLaunchKernelGGL((row_normalize_backward_kernel<TX, TG, __bf16, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((row_normalize_backward_kernel<TX, TG, __bf16, false>), grid, block, 0, s, a);
}

template <typename TX>
void launch_bwd(const RowNormArgs& a, dim3 grid, hipStream_t s) {
  if (a.grad_dtype == kF32) launch_bwd_g<TX, float>(a, grid, s);
  else if (a.grad_dtype == kF16) launch_bwd_g<TX, _Float16>(a, grid, s);
  else launch_bwd_g<TX, __bf16>(a, grid, s);
}

}  // namespace

void launch_row_normalize(const RowNormArgs& a, bool backward, hipStream_t stream) {
  if (a.rows == 0) return;
  const dim3 grid(static_cast<unsigned>((a.rows + kRowWaves - 1) / kRowWaves));
  if (backward) {
    if (a.x_dtype == kF32) launch_bwd<float>(a, grid, stream);
    else if (a.x_dtype == kF16) launch_bwd<_Float16>(a, grid, stream);
    else launch_bwd<__bf16>(a, grid, stream);
  } else {
    if (a.x_dtype == kF32) launch_fwd<float>(a, grid, stream);
    else if (a.x_dtype == kF16) launch_fwd<_Float16>(a, grid, stream);
    else launch_fwd<__bf16>(a, grid, stream);
  }
}

}  // namespace da
