// Dictionary normalization work, shared by the standalone normalization
// kernel and the projection launch of the module forward (which runs it in
// extra workgroups beside the GEMM tiles, so the bank needs no launch of its
// own).
//
// Replaces SharedDictionaryBank.normalized (reference
// src/double_attention/modules.py:45-48): every atom (column j of the [R, M]
// raw bank) is divided by max(||column||_2, eps), the semantics of
// F.normalize(dim=0).  The tied bank (raw_value == nullptr) uses the key atoms
// for reconstruction as well (modules.py:47).
//
// Output layouts are the ones the fused route kernel reads, padded to
// Mp = round_up(M, 64) atoms with zero atoms in the padding:
//   key_t  [Mp, R]  atom-major, fp16 or bf16
//   value  32-atom tiles, fp16 (normalized atoms are bounded by 1): coordinate
//          r of atom j at value[(j/32)*32*R + 32*r + j%32]
//   value_rows (optional) [R, Mp] fp16, coordinate-major: the [R, M] bank of
//          the module API, written by the same pass so no copy kernel is needed
// A workgroup of 256 threads owns 32 atoms of one bank: it reads each column
// once into registers (fp32), reduces the sums of squares through LDS, writes
// the value layout directly and the atom-major key layout through an LDS
// transpose, so every global store is a full 16-byte chunk or a coalesced row
// segment.
#pragma once

#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kNormCols = 32;     // atoms per workgroup
constexpr int kNormGroups = 8;    // row groups per workgroup (256 threads)
constexpr int kNormMaxR = 512;
// LDS of one workgroup: [8][32] partial sums, [32] scales, then the [32][R+8]
// transposed key tile.
constexpr int kNormLdsBytes = (kNormGroups + 1) * kNormCols * 4 + kNormCols * (kNormMaxR + 8) * 2;

struct NormJob {
  const void* raw_key;     // [R, M]; nullptr: no job
  const void* raw_value;   // [R, M] or nullptr (tied bank)
  int raw_dtype;
  int R, M, Mp;
  float eps;
  void* key_t;
  int key_dtype;           // kF16 or kBF16
  void* value;
  void* value_rows;        // or nullptr
};

// Workgroups of a job: Mp/32 per bank.
__host__ __device__ inline int norm_blocks(const NormJob& j) {
  return j.raw_key ? (j.Mp / kNormCols) * (j.raw_value ? 2 : 1) : 0;
}

// Workgroup `block` of a job (blockDim.x == 256): atoms 32*block' .. of the key
// bank (block' = block < Mp/32) or of the value bank (block' = block - Mp/32).
template <typename Tin, int R>
__device__ __forceinline__ void normalize_block_t(const NormJob& job, int block, char* lds) {
  constexpr int PER = R / kNormGroups;
  const int per_bank = job.Mp / kNormCols;
  const int which = block >= per_bank ? 1 : 0;
  const int j0 = (block - which * per_bank) * kNormCols;
  const Tin* src = static_cast<const Tin*>(which ? job.raw_value : job.raw_key);
  const bool write_key = which == 0;
  const bool write_value = which == 1 || job.raw_value == nullptr;
  const int tid = static_cast<int>(threadIdx.x);
  const int jj = tid % kNormCols;
  const int rg = tid / kNormCols;
  const int j = j0 + jj;
  const bool valid = j < job.M;
  float* partial = reinterpret_cast<float*>(lds);         // [8][32]
  float* scale_s = partial + kNormGroups * kNormCols;     // [32]
  uint16_t* tile = reinterpret_cast<uint16_t*>(scale_s + kNormCols);   // [32][R + 8]

  // Every load is issued before any is used: padding atoms (j >= M) re-read
  // atom M-1 and are zeroed afterwards, so the loads need no branch.
  const int jc = min(j, job.M - 1);
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int r = rg + i * kNormGroups;
    v[i] = static_cast<float>(src[static_cast<int64_t>(r) * job.M + jc]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] = valid ? v[i] : 0.f;
    ss += v[i] * v[i];
  }
  partial[rg * kNormCols + jj] = ss;
  __syncthreads();
  if (rg == 0) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kNormGroups; ++i) t += partial[i * kNormCols + jj];
    scale_s[jj] = valid ? 1.f / fmaxf(sqrtf(t), job.eps) : 0.f;
  }
  __syncthreads();
  const float scale = scale_s[jj];

  if (write_value) {
    // The workgroup's 32 atoms are exactly one value tile.
    _Float16* vtile = static_cast<_Float16*>(job.value) + static_cast<int64_t>(j0) * R;
    _Float16* rows = static_cast<_Float16*>(job.value_rows);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = rg + i * kNormGroups;
      const _Float16 h = static_cast<_Float16>(v[i] * scale);
      vtile[r * kNormCols + jj] = h;
      if (rows) rows[static_cast<int64_t>(r) * job.Mp + j] = h;
    }
  }
  if (write_key) {
    constexpr int PITCH = R + 8;
    const bool bf = job.key_dtype == kBF16;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float x = v[i] * scale;
      tile[jj * PITCH + rg + i * kNormGroups] =
          bf ? __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)) : __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    __syncthreads();
    // 32 atoms x R coordinates = 32 * R / 8 chunks of 16 bytes.
    uint16_t* key_t = static_cast<uint16_t*>(job.key_t);
#pragma unroll
    for (int ch = tid; ch < kNormCols * (R / 8); ch += 256) {
      const int a = ch / (R / 8);
      const int r8 = (ch % (R / 8)) * 8;
      store16B(key_t + static_cast<int64_t>(j0 + a) * R + r8, *reinterpret_cast<const u32x4*>(tile + a * PITCH + r8));
    }
  }
}

template <typename Tin>
__device__ __forceinline__ void normalize_block_r(const NormJob& job, int block, char* lds) {
  switch (job.R) {
    case 64: normalize_block_t<Tin, 64>(job, block, lds); break;
    case 128: normalize_block_t<Tin, 128>(job, block, lds); break;
    case 256: normalize_block_t<Tin, 256>(job, block, lds); break;
    default: normalize_block_t<Tin, 512>(job, block, lds); break;
  }
}

__device__ __forceinline__ void normalize_block(const NormJob& job, int block, char* lds) {
  if (job.raw_dtype == kF32) normalize_block_r<float>(job, block, lds);
  else if (job.raw_dtype == kF16) normalize_block_r<_Float16>(job, block, lds);
  else normalize_block_r<__bf16>(job, block, lds);
}

}  // namespace da
