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
// A block holds 64 atoms, one per lane, so every row access of the bank is
// one coalesced 64-wide load; its 16 waves split the routing coordinates, the
// two column sums meet in LDS, and each wave writes its own coordinates
// (second reads hit L2: the bank is a few MB).  Atom-major gradients (the
// route backward's [atoms, R] rows) are first copied into an LDS tile
// [R][64] with coalesced 16-byte loads of the block's 64 contiguous rows,
// since read in place their lanes would sit 4R bytes apart.  blockIdx.y picks
// the key or value bank.
constexpr int kNormBwdWaves = 16;
constexpr int kNormBwdPitch = 65;       // floats per coordinate row of the LDS tile
constexpr int kNormBwdTileMaxR = 512;   // coordinates the tile holds (133 KiB)

template <typename T, bool ATOM_MAJOR>
__global__ __launch_bounds__(64 * kNormBwdWaves) void dict_normalize_backward_kernel(NormBwdArgs a) {
  __shared__ float tile[ATOM_MAJOR ? kNormBwdTileMaxR * kNormBwdPitch : 1];   // [R][kNormBwdPitch]
  __shared__ float part[2][kNormBwdWaves][64];
  const int lane = lane_id();
  const int w = static_cast<int>(threadIdx.x) >> 6;
  const int64_t j0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t j = j0 + lane;
  const bool value_bank = blockIdx.y == 1;
  const T* raw = static_cast<const T*>(value_bank ? a.raw_value : a.raw_key);
  const float* g1 = value_bank ? a.grad_value : a.grad_key;
  const float* g2 = (!value_bank && !a.raw_value) ? a.grad_value : nullptr;
  T* out = static_cast<T*>(value_bank ? a.d_value : a.d_key);
  const bool live = j < a.M;
  if constexpr (ATOM_MAJOR) {
    // Rows j0 .. j0+63 of the [M, R] gradients (pitch g_ld_j) as 16-byte
    // chunks: chunk c of atom jj holds coordinates 4c .. 4c+3.
    const int chunks = a.R / 4;
    const int atoms = static_cast<int>(min<int64_t>(64, a.M - j0));
    for (int idx = static_cast<int>(threadIdx.x); idx < atoms * chunks; idx += 64 * kNormBwdWaves) {
      const int jj = idx / chunks, c = idx - jj * chunks;
      const int64_t off = (j0 + jj) * a.g_ld_j + 4 * c;
      f32x4 h = g1 ? *reinterpret_cast<const f32x4*>(g1 + off) : zero4();
      if (g2) {
        const f32x4 h2 = *reinterpret_cast<const f32x4*>(g2 + off);
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] += h2[e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[(4 * c + e) * kNormBwdPitch + jj] = h[e];
    }
    __syncthreads();
  }
  auto grad_at = [&](int r) {
    if constexpr (ATOM_MAJOR) {
      return tile[r * kNormBwdPitch + lane];
    } else {
      const int64_t gi = static_cast<int64_t>(r) * a.g_ld_r + j * a.g_ld_j;
      return (g1 ? g1[gi] : 0.f) + (g2 ? g2[gi] : 0.f);
    }
  };
  float ss = 0.f, dot = 0.f;
  if (live) {
    for (int r = w; r < a.R; r += kNormBwdWaves) {
      const float v = static_cast<float>(raw[static_cast<int64_t>(r) * a.M + j]);
      const float h = grad_at(r);
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
    out[i] = static_cast<T>(grad_at(r) * inv - v * coef);
  }
}

template <typename T>
static void launch_norm_bwd(const NormBwdArgs& a, dim3 grid, hipStream_t stream) {
  const dim3 block(64 * kNormBwdWaves);
  // The tile path: atom-major rows of 16-byte chunks that fit the tile.
  auto aligned16 = [](const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool tile = a.g_ld_r == 1 && a.R > 1 && a.R % 4 == 0 && a.R <= kNormBwdTileMaxR && a.g_ld_j % 4 == 0 &&
                    aligned16(a.grad_key) && aligned16(a.grad_value);
  if (tile) {
    hipLaunchKernelGGL((dict_normalize_backward_kernel<T, true>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((dict_normalize_backward_kernel<T, false>), grid, block, 0, stream, a);
  }
}

void launch_dictionary_normalize_backward(const NormBwdArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.M + 63) / 64), (a.raw_value && a.d_value) ? 2u : 1u);
  if (a.dtype == kF32) launch_norm_bwd<float>(a, grid, stream);
  else if (a.dtype == kF16) launch_norm_bwd<_Float16>(a, grid, stream);
  else launch_norm_bwd<__bf16>(a, grid, stream);
}

}  // namespace da
