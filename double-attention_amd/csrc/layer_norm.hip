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

// Backward of the LayerNorm above at dy = dL/dy, the statistics formed again
// from x (fp32, two passes as the forward forms them):
//   xh = (x - mean) rstd,  g = dy w,
//   dx = rstd (g - mean(g) - xh mean(g xh))                 (one rounding)
//   dw += sum over rows of dy xh,  db += sum over rows of dy (fp32)
// A wave takes rows wave, wave + W, ... (W = waves in the grid), each row
// held in registers, the next row's loads issued before this row's sums.
// The row sums take two rounds of wave reductions, two independent sums
// each: (sum x, sum g), then (sum (x - mean)^2, sum g (x - mean)).  The
// parameter gradients stay in the lanes' registers over the wave's rows,
// meet across the workgroup's waves in LDS and leave as one fp32 atomic add
// per workgroup and column into one of kLnParamCopies copies (the caller
// zeroes them and adds the copies up).
template <typename T, int CH>
__global__ __launch_bounds__(64 * kLnRowsPerBlock) void layer_norm_backward_kernel(
    const T* x, const T* dy, int64_t rows, int dim, const void* weight, int pdt, float eps, T* dx, float* dparams) {
  extern __shared__ float part[];   // [2][dim]: weight, then bias gradients
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int nch = dim / 8;
  const float inv_dim = 1.f / static_cast<float>(dim);
  float w[CH][8], gw[CH][8], gb[CH][8];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    load_params8(weight, pdt, static_cast<int64_t>(min(lane + 64 * k, nch - 1)) * 8, w[k], 1.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) gw[k][e] = gb[k][e] = 0.f;
  }
  const int64_t step = static_cast<int64_t>(gridDim.x) * kLnRowsPerBlock;
  typename Elem<T>::v8 rx[CH], rg[CH];
  auto load_row = [&](int64_t row) {
    const int64_t r = min(row, rows - 1);
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int64_t c = static_cast<int64_t>(min(lane + 64 * k, nch - 1)) * 8;
      rx[k] = load8(x + r * dim + c);
      rg[k] = load8(dy + r * dim + c);
    }
  };
  int64_t row = static_cast<int64_t>(blockIdx.x) * kLnRowsPerBlock + wave;
  if (row < rows) load_row(row);
  for (; row < rows; row += step) {
    float v[CH][8], g[CH][8];
    float sx = 0.f, sg = 0.f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const bool valid = lane + 64 * k < nch;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[k][e] = valid ? static_cast<float>(rx[k][e]) : 0.f;
        const float d = valid ? static_cast<float>(rg[k][e]) : 0.f;
        gb[k][e] += d;
        g[k][e] = d;
        sg += d * w[k][e];
        sx += v[k][e];
      }
    }
    load_row(row + step);   // the next row (clamped past the last) while this one is reduced
    __builtin_amdgcn_sched_barrier(0);
    const float mean = wave_sum(sx) * inv_dim;
    const float a = wave_sum(sg) * inv_dim;
    float sq = 0.f, sgx = 0.f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const bool valid = lane + 64 * k < nch;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = valid ? v[k][e] - mean : 0.f;
        v[k][e] = d;
        sq += d * d;
        sgx += g[k][e] * w[k][e] * d;
      }
    }
    const float rstd = 1.f / sqrtf(wave_sum(sq) * inv_dim + eps);
    const float bq = wave_sum(sgx) * inv_dim * rstd;   // mean(g xh)
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int ci = lane + 64 * k;
      typename Elem<T>::v8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = v[k][e] * rstd;
        gw[k][e] += g[k][e] * xh;
        o[e] = static_cast<T>(rstd * (g[k][e] * w[k][e] - a - xh * bq));
      }
      if (ci < nch) store16B(dx + row * dim + ci * 8, __builtin_bit_cast(u32x4, o));
    }
  }
  // Parameter gradients: the workgroup's waves add theirs into one LDS copy
  // in turn, then one atomic add per workgroup and column.
  for (int q = 0; q < kLnRowsPerBlock; ++q) {
    if (wave == q) {
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int ci = lane + 64 * k;
        if (ci >= nch) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float* pw = part + ci * 8 + e;
          float* pb = part + dim + ci * 8 + e;
          *pw = q == 0 ? gw[k][e] : *pw + gw[k][e];
          *pb = q == 0 ? gb[k][e] : *pb + gb[k][e];
        }
      }
    }
    __syncthreads();
  }
  // Copy blockIdx % kLnParamCopies of the sums: each address takes
  // 1 / kLnParamCopies of the workgroups' adds.
  float* copy = dparams + static_cast<int64_t>(blockIdx.x % kLnParamCopies) * 2 * dim;
  for (int i = static_cast<int>(threadIdx.x); i < 2 * dim; i += 64 * kLnRowsPerBlock) unsafeAtomicAdd(copy + i, part[i]);
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

template <typename T>
static void launch_ln_bwd_t(const void* x, const void* dy, int64_t rows, int dim, const void* w, int pdt, float eps,
                            void* dx, float* dparams, hipStream_t s) {
  // One workgroup per CU, each wave then looping over its rows (more
  // workgroups add atomic adds per column faster than they add speed).
  const int64_t blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
  const dim3 grid(static_cast<unsigned>(blocks < 256 ? blocks : 256));
  const dim3 block(64 * kLnRowsPerBlock);
  const size_t lds = 2 * static_cast<size_t>(dim) * sizeof(float);   // <= 32 KiB
  const int nch = dim / 8;
  const T* xt = static_cast<const T*>(x);
  const T* gt = static_cast<const T*>(dy);
  T* ot = static_cast<T*>(dx);
  if (nch <= 64)
    hipLaunchKernelGGL((layer_norm_backward_kernel<T, 1>), grid, block, lds, s, xt, gt, rows, dim, w, pdt, eps, ot, dparams);
  else if (nch <= 128)
    hipLaunchKernelGGL((layer_norm_backward_kernel<T, 2>), grid, block, lds, s, xt, gt, rows, dim, w, pdt, eps, ot, dparams);
  else if (nch <= 256)
    hipLaunchKernelGGL((layer_norm_backward_kernel<T, 4>), grid, block, lds, s, xt, gt, rows, dim, w, pdt, eps, ot, dparams);
  else
    hipLaunchKernelGGL((layer_norm_backward_kernel<T, 8>), grid, block, lds, s, xt, gt, rows, dim, w, pdt, eps, ot, dparams);
}

void launch_layer_norm_backward(const void* x, const void* dy, int64_t rows, int dim, const void* weight,
                                int param_dtype, float eps, int dtype, void* dx, float* dparams, hipStream_t stream) {
  if (rows == 0) return;
  if (dtype == kF16) launch_ln_bwd_t<_Float16>(x, dy, rows, dim, weight, param_dtype, eps, dx, dparams, stream);
  else launch_ln_bwd_t<__bf16>(x, dy, rows, dim, weight, param_dtype, eps, dx, dparams, stream);
}

void launch_layer_norm(const void* x, int64_t rows, int dim, const void* weight, const void* bias, int param_dtype,
                       float eps, int dtype, void* out, hipStream_t stream) {
  if (rows == 0) return;
  if (dtype == kF16) launch_ln_t<_Float16>(x, rows, dim, weight, bias, param_dtype, eps, out, stream);
  else launch_ln_t<__bf16>(x, rows, dim, weight, bias, param_dtype, eps, out, stream);
}

}  // namespace da
