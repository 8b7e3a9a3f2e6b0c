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
//   key_t  [Mp, R]  atom-major, element type TK
//   value  32-atom tiles, fp16 (normalized atoms are bounded by 1): coordinate
//          r of atom j at value[(j/32)*32*R + 32*r + j%32]
//   value_rows (optional) [R, Mp] fp16, coordinate-major: the [R, M] bank of
//          the module API, written by the same pass so no copy kernel is needed
// A workgroup owns 32 atoms: it reads each column once into registers (fp32),
// reduces the sums of squares through LDS, writes the value layout directly
// and the atom-major key layout through an LDS transpose, so every global
// store is a full 16-byte chunk or a coalesced row segment.
#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kNormCols = 32;     // atoms per workgroup
constexpr int kNormGroups = 8;    // row groups per workgroup (256 threads)

template <typename Tin, typename TK, int R>
__global__ __launch_bounds__(256) void dict_normalize_kernel(
    const Tin* __restrict__ raw_key, const Tin* __restrict__ raw_value, int M, int Mp, float eps,
    TK* __restrict__ key_t, _Float16* __restrict__ value, _Float16* __restrict__ value_rows) {
  constexpr int PER = R / kNormGroups;
  const int which = blockIdx.y;  // 0: key bank, 1: value bank (untied only)
  const Tin* src = which == 0 ? raw_key : raw_value;
  const bool write_key = which == 0;
  const bool write_value = which == 1 || raw_value == nullptr;

  const int jj = threadIdx.x % kNormCols;
  const int rg = threadIdx.x / kNormCols;
  const int j0 = blockIdx.x * kNormCols;
  const int j = j0 + jj;
  const bool valid = j < M;

  __shared__ float partial[kNormGroups][kNormCols];
  __shared__ float scale_s[kNormCols];
  __shared__ __attribute__((aligned(16))) TK tile[kNormCols][R + 8];

  float v[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int r = rg + i * kNormGroups;
    v[i] = valid ? static_cast<float>(src[static_cast<int64_t>(r) * M + j]) : 0.f;
    ss += v[i] * v[i];
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

  if (write_value) {
    // The workgroup's 32 atoms are exactly one value tile.
    _Float16* vtile = value + static_cast<int64_t>(j0) * R;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = rg + i * kNormGroups;
      const _Float16 h = static_cast<_Float16>(v[i] * scale);
      vtile[r * kNormCols + jj] = h;
      if (value_rows) value_rows[static_cast<int64_t>(r) * Mp + j] = h;
    }
  }
  if (write_key) {
#pragma unroll
    for (int i = 0; i < PER; ++i) tile[jj][rg + i * kNormGroups] = static_cast<TK>(v[i] * scale);
    __syncthreads();
    // 32 atoms x R coordinates = 32 * R / 8 chunks of 16 bytes.
    for (int ch = threadIdx.x; ch < kNormCols * (R / 8); ch += 256) {
      const int a = ch / (R / 8);
      const int r8 = (ch % (R / 8)) * 8;
      store16B(key_t + static_cast<int64_t>(j0 + a) * R + r8, *reinterpret_cast<const u32x4*>(&tile[a][r8]));
    }
  }
}

template <typename Tin, typename TK, int R>
static void launch_norm(const void* rk, const void* rv, int M, int Mp, float eps, void* kt, void* v,
                        void* vr, hipStream_t s) {
  dim3 grid(Mp / kNormCols, rv ? 2 : 1);
  hipLaunchKernelGGL((dict_normalize_kernel<Tin, TK, R>), grid, dim3(256), 0, s,
                     static_cast<const Tin*>(rk), static_cast<const Tin*>(rv), M, Mp, eps,
                     static_cast<TK*>(kt), static_cast<_Float16*>(v), static_cast<_Float16*>(vr));
}

template <typename Tin, typename TK>
static void dispatch_r(int R, const void* rk, const void* rv, int M, int Mp, float eps, void* kt,
                       void* v, void* vr, hipStream_t s) {
  switch (R) {
    case 64: launch_norm<Tin, TK, 64>(rk, rv, M, Mp, eps, kt, v, vr, s); break;
    case 128: launch_norm<Tin, TK, 128>(rk, rv, M, Mp, eps, kt, v, vr, s); break;
    case 256: launch_norm<Tin, TK, 256>(rk, rv, M, Mp, eps, kt, v, vr, s); break;
    default: launch_norm<Tin, TK, 512>(rk, rv, M, Mp, eps, kt, v, vr, s); break;
  }
}

template <typename TK>
static void dispatch_in(int in_dtype, int R, const void* rk, const void* rv, int M, int Mp, float eps,
                        void* kt, void* v, void* vr, hipStream_t s) {
  if (in_dtype == kF32) dispatch_r<float, TK>(R, rk, rv, M, Mp, eps, kt, v, vr, s);
  else if (in_dtype == kF16) dispatch_r<_Float16, TK>(R, rk, rv, M, Mp, eps, kt, v, vr, s);
  else dispatch_r<__bf16, TK>(R, rk, rv, M, Mp, eps, kt, v, vr, s);
}

void launch_dictionary_normalize(const void* raw_key, const void* raw_value, int in_dtype, int R,
                                 int M, float eps, void* key_t, int key_dtype, void* value,
                                 void* value_rows, hipStream_t stream) {
  const int Mp = static_cast<int>(round_up(M, kAtomPad));
  if (key_dtype == kF16)
    dispatch_in<_Float16>(in_dtype, R, raw_key, raw_value, M, Mp, eps, key_t, value, value_rows, stream);
  else
    dispatch_in<__bf16>(in_dtype, R, raw_key, raw_value, M, Mp, eps, key_t, value, value_rows, stream);
}

}  // namespace da
