// Map combine of the training path and its backward, and the sum of split-K
// partial products.  The map combine is the weighted sum over
// the outer maps (the reference's map_combine "weighted_sum",
// src/double_attention/modules.py:265-272, combined = einsum("s,bstd->btd",
// softmax(map_mix_logits), map_output)) over per-map outputs the attention
// kernel wrote in fp32, and its gradient.
//   forward   out[b, t, :]      = sum_s w_s O[b, s, t, :]           (fp32 sum, one rounding)
//   backward  dO[b, s, t, :]    = round(w_s dY[b, t, :])             (per map, 16-bit)
//             wsum[s]          += sum_{b, t, d} O[b, s, t, d] dY[b, t, d]   (fp32)
// wsum is the gradient at the weights themselves; the softmax's backward to
// the logits is left to the caller.  Both passes are HBM-bound: a thread
// takes 8 consecutive features of one token (16- and 32-byte accesses) with
// every map's loads issued before they are used, in a grid-stride loop over
// the tokens' chunks; the backward's per-map sums meet per workgroup in LDS
// and leave as one atomic add per workgroup and map.
// The partial sum adds the fp32 partial products of a split-K GEMM (the
// training path's weight gradients) and rounds the sum once to 16 bits.
#include <algorithm>

#include "da_common.h"
#include "da_launch.h"

namespace da {

namespace {

constexpr int kMixThreads = 256;

template <typename T>
__device__ __forceinline__ void to_float8(const typename Elem<T>::v8& v, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = static_cast<float>(v[e]);
}

template <typename T>
__device__ __forceinline__ void store8f(T* p, const float (&f)[8]) {
  typename Elem<T>::v8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = static_cast<T>(f[e]);
  *reinterpret_cast<typename Elem<T>::v8*>(p) = v;
}

__device__ __forceinline__ void load_f32x8(const float* p, float (&f)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
}

template <typename TO, int S>
__global__ __launch_bounds__(kMixThreads) void map_combine_kernel(MapCombineArgs a) {
  const int64_t per_row = a.D / 8;
  const int64_t n = a.rows * per_row;
  float w[S];
#pragma unroll
  for (int s = 0; s < S; ++s) w[s] = a.weights[s];
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kMixThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kMixThreads) {
    const int64_t row = i / per_row, c8 = (i - row * per_row) * 8;
    const int64_t b = row / a.T, t = row - b * a.T;
    const float* o = a.maps + ((b * S) * a.T + t) * a.D + c8;
    float x[S][8];
#pragma unroll
    for (int s = 0; s < S; ++s) load_f32x8(o + static_cast<int64_t>(s) * a.T * a.D, x[s]);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[e] = w[0] * x[0][e];
#pragma unroll
      for (int s = 1; s < S; ++s) acc[e] += w[s] * x[s][e];
    }
    store8f(static_cast<TO*>(a.out) + row * a.D + c8, acc);
  }
}

template <typename TG, int S>
__global__ __launch_bounds__(kMixThreads) void map_combine_backward_kernel(MapCombineArgs a) {
  __shared__ float red[S][kMixThreads / 64];
  const int64_t per_row = a.D / 8;
  const int64_t n = a.rows * per_row;
  float w[S], part[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    w[s] = a.weights[s];
    part[s] = 0.f;
  }
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kMixThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kMixThreads) {
    const int64_t row = i / per_row, c8 = (i - row * per_row) * 8;
    const int64_t b = row / a.T, t = row - b * a.T;
    float g[8];
    to_float8<TG>(load8(static_cast<const TG*>(a.grad) + row * a.D + c8), g);
    const int64_t first = ((b * S) * a.T + t) * a.D + c8;
    float x[S][8];
#pragma unroll
    for (int s = 0; s < S; ++s) load_f32x8(a.maps + first + static_cast<int64_t>(s) * a.T * a.D, x[s]);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float d[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d[e] = w[s] * g[e];
        part[s] += x[s][e] * g[e];
      }
      store8f(static_cast<TG*>(a.grad_maps) + first + static_cast<int64_t>(s) * a.T * a.D, d);
    }
  }
  const int lane = lane_id(), wave = static_cast<int>(threadIdx.x) >> 6;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float v = wave_sum(part[s]);
    if (lane == 0) red[s][wave] = v;
  }
  __syncthreads();
  if (threadIdx.x < S) {
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < kMixThreads / 64; ++k) v += red[threadIdx.x][k];
    unsafeAtomicAdd(a.weight_sums + threadIdx.x, v);
  }
}

// Workgroups: enough to fill the chip a few times over, each thread then
// looping over a few chunks (fewer workgroups means fewer atomic adds).
unsigned mix_grid(int64_t n) {
  const int64_t blocks = (n + kMixThreads - 1) / kMixThreads;
  return static_cast<unsigned>(blocks < 2048 ? (blocks > 0 ? blocks : 1) : 2048);
}

template <typename T, int S>
void launch_s(const MapCombineArgs& a, bool backward, hipStream_t stream) {
  // The backward's S per-map sums take one atomic add per workgroup each:
  // 256 workgroups (a few chunks per thread) keep those adds few.
  const unsigned grid = backward ? std::min(mix_grid(a.rows * (a.D / 8)), 256u) : mix_grid(a.rows * (a.D / 8));
  if (backward) hipLaunchKernelGGL((map_combine_backward_kernel<T, S>), dim3(grid), dim3(kMixThreads), 0, stream, a);
  else hipLaunchKernelGGL((map_combine_kernel<T, S>), dim3(grid), dim3(kMixThreads), 0, stream, a);
}

template <typename T>
void launch_t(const MapCombineArgs& a, bool backward, hipStream_t stream) {
  switch (a.S) {
    case 1: launch_s<T, 1>(a, backward, stream); break;
    case 2: launch_s<T, 2>(a, backward, stream); break;
    case 3: launch_s<T, 3>(a, backward, stream); break;
    case 4: launch_s<T, 4>(a, backward, stream); break;
    case 5: launch_s<T, 5>(a, backward, stream); break;
    case 6: launch_s<T, 6>(a, backward, stream); break;
    case 7: launch_s<T, 7>(a, backward, stream); break;
    default: launch_s<T, 8>(a, backward, stream); break;
  }
}

// out[i] = sum_c partials[c n + i] (fp32, in order c = 0, 1, ...), rounded once
// to TO: eight elements per thread; with C > 0 partials known at compile time
// every partial's loads are issued together, C = 0 loops over `count`.
template <typename TO, int C>
__global__ __launch_bounds__(kMixThreads) void sum_partials_kernel(const float* partials, int count, int64_t n,
                                                                   TO* out) {
  const int64_t n8 = n / 8;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kMixThreads + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * kMixThreads) {
    float acc[8];
    if constexpr (C > 0) {
      float x[C][8];
#pragma unroll
      for (int c = 0; c < C; ++c) load_f32x8(partials + static_cast<int64_t>(c) * n + 8 * i, x[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] = x[0][e];
#pragma unroll
        for (int c = 1; c < C; ++c) acc[e] += x[c][e];
      }
    } else {
      float x[8];
      load_f32x8(partials + 8 * i, acc);
      for (int c = 1; c < count; ++c) {
        load_f32x8(partials + static_cast<int64_t>(c) * n + 8 * i, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += x[e];
      }
    }
    store8f(out + 8 * i, acc);
  }
}

template <typename TO>
void launch_sum_partials_t(const float* partials, int count, int64_t n, TO* out, hipStream_t stream) {
  const dim3 grid(mix_grid(n / 8)), block(kMixThreads);
  switch (count) {
    case 1: hipLaunchKernelGGL((sum_partials_kernel<TO, 1>), grid, block, 0, stream, partials, count, n, out); break;
    case 2: hipLaunchKernelGGL((sum_partials_kernel<TO, 2>), grid, block, 0, stream, partials, count, n, out); break;
    case 4: hipLaunchKernelGGL((sum_partials_kernel<TO, 4>), grid, block, 0, stream, partials, count, n, out); break;
    case 8: hipLaunchKernelGGL((sum_partials_kernel<TO, 8>), grid, block, 0, stream, partials, count, n, out); break;
    default: hipLaunchKernelGGL((sum_partials_kernel<TO, 0>), grid, block, 0, stream, partials, count, n, out); break;
  }
}

}  // namespace

void launch_sum_partials(const float* partials, int count, int64_t n, void* out, int out_dtype, hipStream_t stream) {
  if (n == 0) return;
  if (out_dtype == kF16) launch_sum_partials_t(partials, count, n, static_cast<_Float16*>(out), stream);
  else launch_sum_partials_t(partials, count, n, static_cast<__bf16*>(out), stream);
}

void launch_map_combine(const MapCombineArgs& a, bool backward, hipStream_t stream) {
  if (a.rows == 0) return;
  if (a.dtype == kF16) launch_t<_Float16>(a, backward, stream);
  else launch_t<__bf16>(a, backward, stream);
}

}  // namespace da
