// LDS tile staging for gfx950: direct global->LDS DMA and swizzled layouts.
//
// Tiles are staged with global_load_lds_dwordx4: every lane names its own
// 16-byte global chunk and the wave writes 64 consecutive 16-byte LDS slots
// (slot = M0 base + 16 * lane).  Data never passes through VGPRs, so the next
// tile's loads run while the current tile is being multiplied.
//
// A tile is a row-major array of 16-byte chunks, `nck` chunks per row (nck a
// power of two).  Chunk (row, ck) lives in LDS slot row*nck + (ck ^ swz(row)).
// The swizzle makes each 16-lane group of a ds_read_b128 hit 16 distinct
// 16-byte bank groups, for the two row orders the kernels read in:
//   linear rows:  lanes c = 0..15 read rows base + c
//   blocked rows: lanes c = 0..15 read rows base + 8*(c/4) + (c%4)
// (the blocked order is the key/atom order that makes a score accumulator
// directly usable as the next MFMA's B operand; see da_common.h).
#pragma once

#include "da_common.h"

namespace da {

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void dma16(const void* src, void* lds_slot_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds_slot_base), 16, 0, 0);
}

// s_waitcnt vmcnt(0) only (gfx9 encoding: expcnt and lgkmcnt left at max).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <int NCK>
__device__ __forceinline__ int swz_linear(int row) {
  if constexpr (NCK >= 16) return row & 15;
  else return (row / (16 / NCK)) & (NCK - 1);
}

template <int NCK>
__device__ __forceinline__ int swz_blocked(int row) {
  if constexpr (NCK >= 16) return ((row >> 1) & 12) | (row & 3);
  else if constexpr (NCK == 8) return (((row >> 3) & 3) << 1) | ((row >> 1) & 1);
  else return swz_linear<NCK>(row);
}

template <int NCK, bool BLOCKED>
__device__ __forceinline__ int slot_of(int row, int ck) {
  return row * NCK + (ck ^ (BLOCKED ? swz_blocked<NCK>(row) : swz_linear<NCK>(row)));
}

// Inverse of slot_of: which (row, ck) a given LDS slot holds.
template <int NCK, bool BLOCKED>
__device__ __forceinline__ void chunk_of(int slot, int& row, int& ck) {
  row = slot / NCK;
  ck = (slot % NCK) ^ (BLOCKED ? swz_blocked<NCK>(row) : swz_linear<NCK>(row));
}

// 16-byte read of chunk (row, ck) from a tile starting at `tile`.
template <int NCK, bool BLOCKED>
__device__ __forceinline__ u32x4 lds_chunk(const char* tile, int row, int ck) {
  return *reinterpret_cast<const u32x4*>(tile + slot_of<NCK, BLOCKED>(row, ck) * 16);
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 as_v8(u32x4 v) {
  return __builtin_bit_cast(typename Elem<T>::v8, v);
}

// Row of the blocked order: MFMA block `kb` of a 32-row window, lane row c.
__device__ __forceinline__ int blocked_row(int kb, int c) {
  return 32 * (kb >> 1) + 8 * (c >> 2) + 4 * (kb & 1) + (c & 3);
}

__device__ __forceinline__ int uniform_wave() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

}  // namespace da
