// LayerNorm of the blocks and the LM head (nn.LayerNorm in modules.py:311, 313
// and 440 of the reference: attention_norm, feedforward_norm, final_norm,
// applied at :340, :344, :454): y = (x - mean) / sqrt(var + eps) * weight + bias over the last
// dimension, biased variance, statistics in fp32, one rounding to the
// activation dtype.  One wave per row; each lane holds up to CH 16-byte
// chunks of the row in registers, so the row is read from memory once.
#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kLnRowsPerBlock = 4;

// Eight parameters of a chunk as floats (weight / bias of param dtype pdt).
__device__ __forceinline__ void load_params8(const void* p, int pdt, int64_t i0, float (&o)[8], float dflt) {
  if (p == nullptr) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = dflt;
  } else if (pdt == kF32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i0);
    const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = a[e];
      o[e + 4] = b[e];
    }
  } else if (pdt == kF16) {
    const auto v = load8(static_cast<const _Float16*>(p) + i0);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(v[e]);
  } else {
    const auto v = load8(static_cast<const __bf16*>(p) + i0);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(v[e]);
  }
}

template <typename T, int CH>
__global__ __launch_bounds__(64 * kLnRowsPerBlock) void layer_norm_kernel(const T* x, int64_t rows, int dim,
                                                                          const void* weight, const void* bias,
                                                                          int pdt, float eps, T* out) {
  const int lane = lane_id();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kLnRowsPerBlock + threadIdx.x / 64;
  if (row >= rows) return;   // whole waves
  const int nch = dim / 8;
  const T* xr = x + row * dim;
  // Every chunk load is issued before any is used: lanes past the row's
  // chunks re-read its last chunk and drop it.
  typename Elem<T>::v8 raw[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) raw[k] = load8(xr + min(lane + 64 * k, nch - 1) * 8);
  float v[CH][8];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const bool valid = lane + 64 * k < nch;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[k][e] = valid ? static_cast<float>(raw[k][e]) : 0.f;
      sum += v[k][e];
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(dim);
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const bool valid = lane + 64 * k < nch;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = v[k][e] - mean;
      sq += valid ? d * d : 0.f;
    }
  }
  const float rstd = 1.f / sqrtf(wave_sum(sq) / static_cast<float>(dim) + eps);
  T* orow = out + row * dim;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int ci = lane + 64 * k;
    if (ci >= nch) break;
    float w[8], b[8];
    load_params8(weight, pdt, static_cast<int64_t>(ci) * 8, w, 1.f);
    load_params8(bias, pdt, static_cast<int64_t>(ci) * 8, b, 0.f);
    typename Elem<T>::v8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<T>((v[k][e] - mean) * rstd * w[e] + b[e]);
    store16B(orow + ci * 8, __builtin_bit_cast(u32x4, o));
  }
}

template <typename T>
static void launch_ln_t(const void* x, int64_t rows, int dim, const void* w, const void* b, int pdt, float eps,
                        void* out, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock));
  const dim3 block(64 * kLnRowsPerBlock);
  const int nch = dim / 8;
  const T* xt = static_cast<const T*>(x);
  T* ot = static_cast<T*>(out);
  if (nch <= 64) hipLaunchKernelGGL((layer_norm_kernel<T, 1>), grid, block, 0, s, xt, rows, dim, w, b, pdt, eps, ot);
  else if (nch <= 128) hipLaunchKernelGGL((layer_norm_kernel<T, 2>), grid, block, 0, s, xt, rows, dim, w, b, pdt, eps, ot);
  else if (nch <= 256) hipLaunchKernelGGL((layer_norm_kernel<T, 4>), grid, block, 0, s, xt, rows, dim, w, b, pdt, eps, ot);
  else hipLaunchKernelGGL((layer_norm_kernel<T, 8>), grid, block, 0, s, xt, rows, dim, w, b, pdt, eps, ot);
}

void launch_layer_norm(const void* x, int64_t rows, int dim, const void* weight, const void* bias, int param_dtype,
                       float eps, int dtype, void* out, hipStream_t stream) {
  if (rows == 0) return;
  if (dtype == kF16) launch_ln_t<_Float16>(x, rows, dim, weight, bias, param_dtype, eps, out, stream);
  else launch_ln_t<__bf16>(x, rows, dim, weight, bias, param_dtype, eps, out, stream);
}

}  // namespace da
