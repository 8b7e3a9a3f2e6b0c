// Once-per-bank dictionary normalization as a launch of its own (the module
// forward runs the same work inside its projection launch); the work and the
// layouts are described in dict_norm.h.
#include "dict_norm.h"

namespace da {

__global__ __launch_bounds__(256) void dict_normalize_kernel(NormJob job) {
  __shared__ __attribute__((aligned(16))) char lds[kNormLdsBytes];
  normalize_block(job, static_cast<int>(blockIdx.x), lds);
}

void launch_dictionary_normalize(const void* raw_key, const void* raw_value, int in_dtype, int R,
                                 int M, float eps, void* key_t, int key_dtype, void* value,
                                 void* value_rows, hipStream_t stream) {
  const NormJob job{raw_key, raw_value, in_dtype, R, M, static_cast<int>(round_up(M, kAtomPad)), eps,
                    key_t, key_dtype, value, value_rows};
  hipLaunchKernelGGL(dict_normalize_kernel, dim3(norm_blocks(job)), dim3(256), 0, stream, job);
}

// Backward of the column normalization (F.normalize over dim 0 under
// autograd, reference modules.py:45-48).  Atom j with raw column v and
// gradient h at the normalized atom (for a tied bank, the sum of its key and
// value gradients) gets
//   dv = h i - v (<v, h> i^3 [|v| > eps]),   i = 1 / max(|v|, eps),
// i.e. (h - n <n, h>) / |v| with n = v / |v|, and h / eps for |v| <= eps.
// A block holds 64 atoms, one per lane, so every row access is one coalesced
// 64-wide load; its 16 waves split the routing coordinates, the two column
// sums meet in LDS, and each wave writes its own coordinates (second reads
// hit L2: the bank is a few MB).  blockIdx.y picks the key or value bank.
constexpr int kNormBwdWaves = 16;

template <typename T>
__global__ __launch_bounds__(64 * kNormBwdWaves) void dict_normalize_backward_kernel(NormBwdArgs a) {
  __shared__ float part[2][kNormBwdWaves][64];
  const int lane = lane_id();
  const int w = static_cast<int>(threadIdx.x) >> 6;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool value_bank = blockIdx.y == 1;
  const T* raw = static_cast<const T*>(value_bank ? a.raw_value : a.raw_key);
  const float* g1 = value_bank ? a.grad_value : a.grad_key;
  const float* g2 = (!value_bank && !a.raw_value) ? a.grad_value : nullptr;
  T* out = static_cast<T*>(value_bank ? a.d_value : a.d_key);
  const bool live = j < a.M;
  float ss = 0.f, dot = 0.f;
  if (live) {
    for (int r = w; r < a.R; r += kNormBwdWaves) {
      const int64_t i = static_cast<int64_t>(r) * a.M + j;
      const float v = static_cast<float>(raw[i]);
      const float h = (g1 ? g1[i] : 0.f) + (g2 ? g2[i] : 0.f);
      ss += v * v;
      dot += v * h;
    }
  }
  part[0][w][lane] = ss;
  part[1][w][lane] = dot;
  __syncthreads();
  ss = 0.f;
  dot = 0.f;
#pragma unroll
  for (int k = 0; k < kNormBwdWaves; ++k) {
    ss += part[0][k][lane];
    dot += part[1][k][lane];
  }
  if (!live) return;
  const float norm = sqrtf(ss);
  const float inv = 1.f / fmaxf(norm, a.eps);
  const float coef = norm > a.eps ? dot * inv * inv * inv : 0.f;
  for (int r = w; r < a.R; r += kNormBwdWaves) {
    const int64_t i = static_cast<int64_t>(r) * a.M + j;
    const float v = static_cast<float>(raw[i]);
    const float h = (g1 ? g1[i] : 0.f) + (g2 ? g2[i] : 0.f);
    out[i] = static_cast<T>(h * inv - v * coef);
  }
}

void launch_dictionary_normalize_backward(const NormBwdArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.M + 63) / 64), (a.raw_value && a.d_value) ? 2u : 1u);
  const dim3 block(64 * kNormBwdWaves);
  if (a.dtype == kF32) {
    hipLaunchKernelGGL(dict_normalize_backward_kernel<float>, grid, block, 0, stream, a);
  } else if (a.dtype == kF16) {
    hipLaunchKernelGGL(dict_normalize_backward_kernel<_Float16>, grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL(dict_normalize_backward_kernel<__bf16>, grid, block, 0, stream, a);
  }
}

}  // namespace da
