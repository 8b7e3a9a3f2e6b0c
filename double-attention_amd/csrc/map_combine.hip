// Map combine of the training path and its backward: the weighted sum over
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
  const unsigned grid = mix_grid(a.rows * (a.D / 8));
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

}  // namespace

void launch_map_combine(const MapCombineArgs& a, bool backward, hipStream_t stream) {
  if (a.rows == 0) return;
  if (a.dtype == kF16) launch_t<_Float16>(a, backward, stream);
  else launch_t<__bf16>(a, backward, stream);
}

}  // namespace da
