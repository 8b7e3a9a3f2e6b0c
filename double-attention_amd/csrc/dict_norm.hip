// Once-per-bank dictionary normalization.
//
// Replaces SharedDictionaryBank.normalized (reference
// src/double_attention/modules.py:45-48): every atom (column j of the
// [R, M] raw bank) is divided by max(||column||_2, eps), the semantics of
// F.normalize(dim=0).  The tied bank (raw_value == nullptr) uses the key atoms
// for reconstruction as well (modules.py:47).
//
// Output layouts are the ones the fused route kernel reads, padded to
// Mp = round_up(M, 64) atoms with zero atoms in the padding:
//   key_t  [Mp, R]  atom-major (row j = normalized key atom j)
//   value  [R, Mp]  routing-dim-major (row r = coordinate r of every value atom)
// The sums of squares are accumulated in fp32; each output is rounded once.
#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kNormCols = 32;     // atoms per workgroup
constexpr int kNormGroups = 8;    // row groups per workgroup (256 threads)

template <typename Tin, typename Tout>
__global__ __launch_bounds__(256) void dict_normalize_kernel(
    const Tin* __restrict__ raw_key, const Tin* __restrict__ raw_value, int R, int M, int Mp,
    float eps, Tout* __restrict__ key_t, Tout* __restrict__ value) {
  const int which = blockIdx.y;  // 0: key bank, 1: value bank (untied only)
  const Tin* src = which == 0 ? raw_key : raw_value;
  const bool write_key = which == 0;
  const bool write_value = which == 1 || raw_value == nullptr;

  const int jj = threadIdx.x % kNormCols;
  const int rg = threadIdx.x / kNormCols;
  const int j = blockIdx.x * kNormCols + jj;
  const bool valid = j < M;

  __shared__ float partial[kNormGroups][kNormCols];
  __shared__ float scale_s[kNormCols];

  float ss = 0.f;
  if (valid) {
    for (int r = rg; r < R; r += kNormGroups) {
      const float v = static_cast<float>(src[static_cast<int64_t>(r) * M + j]);
      ss += v * v;
    }
  }
  partial[rg][jj] = ss;
  __syncthreads();
  if (rg == 0) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kNormGroups; ++i) t += partial[i][jj];
    scale_s[jj] = valid ? 1.f / fmaxf(sqrtf(t), eps) : 0.f;
  }
  __syncthreads();
  const float scale = scale_s[jj];

  if (write_value && j < Mp) {
    for (int r = rg; r < R; r += kNormGroups) {
      const float v = valid ? static_cast<float>(src[static_cast<int64_t>(r) * M + j]) : 0.f;
      value[static_cast<int64_t>(r) * Mp + j] = static_cast<Tout>(v * scale);
    }
  }
  if (write_key && j < Mp) {
    // Thread (jj, rg) writes a contiguous run of R / kNormGroups coordinates
    // of atom j, eight at a time (R is a multiple of 64, so runs are 16B
    // aligned and whole).
    const int run = R / kNormGroups;
    Tout* dst = key_t + static_cast<int64_t>(j) * R + rg * run;
    for (int r0 = 0; r0 < run; r0 += 8) {
      Tout buf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = rg * run + r0 + e;
        const float v = valid ? static_cast<float>(src[static_cast<int64_t>(r) * M + j]) : 0.f;
        buf[e] = static_cast<Tout>(v * scale);
      }
      store16B(dst + r0, *reinterpret_cast<const u32x4*>(buf));
    }
  }
}

template <typename Tin, typename Tout>
static void launch_norm(const void* rk, const void* rv, int R, int M, int Mp, float eps, void* kt,
                        void* v, hipStream_t s) {
  dim3 grid(Mp / kNormCols, rv ? 2 : 1);
  hipLaunchKernelGGL((dict_normalize_kernel<Tin, Tout>), grid, dim3(256), 0, s,
                     static_cast<const Tin*>(rk), static_cast<const Tin*>(rv), R, M, Mp, eps,
                     static_cast<Tout*>(kt), static_cast<Tout*>(v));
}

template <typename Tout>
static void dispatch_in(int in_dtype, const void* rk, const void* rv, int R, int M, int Mp, float eps,
                        void* kt, void* v, hipStream_t s) {
  if (in_dtype == kF32) launch_norm<float, Tout>(rk, rv, R, M, Mp, eps, kt, v, s);
  else if (in_dtype == kF16) launch_norm<_Float16, Tout>(rk, rv, R, M, Mp, eps, kt, v, s);
  else launch_norm<__bf16, Tout>(rk, rv, R, M, Mp, eps, kt, v, s);
}

void launch_dictionary_normalize(const void* raw_key, const void* raw_value, int in_dtype, int R,
                                 int M, float eps, void* key_t, void* value, int out_dtype,
                                 hipStream_t stream) {
  const int Mp = round_up(M, kAtomPad);
  if (out_dtype == kF16)
    dispatch_in<_Float16>(in_dtype, raw_key, raw_value, R, M, Mp, eps, key_t, value, stream);
  else
    dispatch_in<__bf16>(in_dtype, raw_key, raw_value, R, M, Mp, eps, key_t, value, stream);
}

}  // namespace da
