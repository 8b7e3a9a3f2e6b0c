// LDS tile staging for gfx950: direct global->LDS DMA into padded tiles
// (PaddedTile, below) or XOR-swizzled tiles without padding (XorTile).
//
// Tiles are staged with global_load_lds_dwordx4: every lane names its own
// 16-byte global chunk and a wave writes 64 consecutive 16-byte LDS slots
// (slot = M0 base + 16 * lane).  Data never passes through VGPRs, so the next
// tile's loads run while the current tile is being multiplied.
//
// A PaddedTile is ROWS rows of NCK 16-byte chunks.  In LDS each row occupies
// NCK + 1 slots (one pad slot), so the 16 lanes of a ds_read_b128 that read
// 16 consecutive rows at one chunk position hit 16 distinct bank groups, and
// a lane's address for chunk k of row r is base + 16 * (r * (NCK + 1) + k):
// every fragment read of a kernel's inner loop is a per-lane base plus an
// immediate offset.  Pad slots are filled with a duplicate chunk and never
// read.
//
// "Blocked" tiles store their rows permuted inside each 32-row window:
// logical row 8a + 4h + i (a, i in 0..3, h in 0..1) sits at physical row
// 16h + 4a + i.  MFMA block kb = 2w + h of the window then reads physical rows
// 16 kb + c, c = 0..15 -- linear -- while its 16x16 accumulator holds logical
// rows 32w + 8g + 4h + i in lane group g: exactly the k order in which two
// stacked accumulator blocks form the next MFMA's B operand (da_common.h).
#pragma once

#include "da_common.h"

namespace da {

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void dma16(const void* src, void* lds_slot_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds_slot_base), 16, 0, 0);
}

// s_waitcnt vmcnt(0) only (gfx9 encoding: expcnt and lgkmcnt left at max).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): vmcnt is split over bits [3:0] and [15:14]; expcnt
// [6:4] and lgkmcnt [11:8] are left at their maxima (no wait).
template <int N>
__device__ __forceinline__ void wait_vmem_at_most() {
  static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup barrier for hand-offs through LDS: this wave's LDS accesses are
// complete (lgkmcnt(0)), then s_barrier.  Unlike __syncthreads, whose fence
// also waits for every vector memory operation (vmcnt(0)), it leaves
// global->LDS loads in flight, so a ring of stage buffers keeps its later
// stages loading across the barrier; the caller first waits for the stage it
// reads with wait_vmem_at_most.  The "memory" clobber keeps the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A wave-uniform pointer moved to SGPRs, so that an address built from it
// takes the scalar-base + 32-bit lane-offset form.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int uniform_wave() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

template <int ROWS, int NCK, bool BLOCKED>
struct PaddedTile {
  static_assert(!BLOCKED || ROWS % 32 == 0, "blocked tiles are made of 32-row windows");
  static constexpr int PITCH = NCK + 1;                 // slots per row
  static constexpr int SLOTS = ROWS * PITCH;
  static constexpr int LOADS = (SLOTS + 63) / 64;       // wave loads that fill the tile
  static constexpr int BYTES = LOADS * 1024;

  // Logical row held by physical row p.
  static __device__ __forceinline__ int logical_row(int p) {
    if constexpr (BLOCKED) return (p & ~31) + 8 * ((p >> 2) & 3) + 4 * ((p >> 4) & 1) + (p & 3);
    else return p;
  }

  // What slot `slot` holds: logical row and chunk; false for pad slots and the
  // tail of the last wave load (which then load a duplicate of chunk 0 of row 0).
  static __device__ __forceinline__ bool slot_chunk(int slot, int& row, int& ck) {
    const int p = slot / PITCH;
    ck = slot - p * PITCH;
    const bool real = ck < NCK && p < ROWS;
    row = real ? logical_row(p) : 0;
    if (!real) ck = 0;
    return real;
  }

  // Byte offset of (physical row, chunk).
  static __device__ __forceinline__ constexpr int offset(int prow, int ck) { return (prow * PITCH + ck) * 16; }
};

// Chunk permutation of an XOR-swizzled tile row (NCK chunks of 16 bytes).
template <int NCK>
__host__ __device__ constexpr int xor_swizzle(int p) {
  if constexpr (NCK >= 16) return p & 15;
  else if constexpr (NCK == 8) return (p >> 1) & 7;
  else return ((p >> 1) ^ (p >> 2)) & 3;   // NCK == 4
}

// A tile of ROWS rows of NCK 16-byte chunks with no padding: chunk ck of
// physical row p sits at slot p*NCK + (ck ^ xor_swizzle(p)).  gfx950's LDS
// serves a ds_read_b128 in four clocks (64 banks, 256 bytes per clock) when
// the 64 lanes' chunks spread over the banks; the MFMA operand reads -- lane
// (c, g) reading row c (or 16 + c) at chunk 4k + g -- then do: measured 205
// bytes per clock per CU with four waves, against 120 for a padded pitch or a
// row-XOR of fewer than 16 values, whose reads take four extra conflict
// clocks.  Rows 16 apart share the permutation, so
//   offset(p + 16m, ck) = offset(p, ck) + 256 m NCK,
// and for NCK >= 16 the chunk group k adds 256 (k >> 2) to the lane's base
// for k & 3: fragment reads are one of four per-lane bases plus an immediate.
// The global->LDS DMA writes whole 1 KiB wave loads of consecutive slots.
template <int ROWS, int NCK, bool BLOCKED>
struct XorTile {
  static_assert(NCK == 4 || NCK == 8 || NCK % 16 == 0, "4, 8 or a multiple of 16 chunks per row");
  static_assert(!BLOCKED || ROWS % 32 == 0, "blocked tiles are made of 32-row windows");
  static constexpr int SLOTS = ROWS * NCK;
  static_assert(SLOTS % 64 == 0, "whole wave loads");
  static constexpr int LOADS = SLOTS / 64;
  static constexpr int BYTES = LOADS * 1024;
  static constexpr int ROW_BLOCK = 16 * NCK * 16;   // bytes between rows p and p + 16

  static __device__ __forceinline__ int logical_row(int p) {
    if constexpr (BLOCKED) return (p & ~31) + 8 * ((p >> 2) & 3) + 4 * ((p >> 4) & 1) + (p & 3);
    else return p;
  }
  // What slot `slot` holds (every slot is real).
  static __device__ __forceinline__ bool slot_chunk(int slot, int& row, int& ck) {
    const int p = slot / NCK;
    ck = (slot - p * NCK) ^ xor_swizzle<NCK>(p);
    row = logical_row(p);
    return true;
  }
  // Byte offset of (physical row, chunk).
  static __device__ __forceinline__ constexpr int offset(int prow, int ck) {
    return (prow * NCK + (ck ^ xor_swizzle<NCK>(prow))) * 16;
  }
  // Lane (c, g)'s base for chunk group k (chunk 4k + g of row c): the read
  // of group k is at base(c, g, k & 3) + 256 (k >> 2).
  static __device__ __forceinline__ int base(int c, int g, int k) { return offset(c, 4 * k + g); }
};

template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 lds_v8(const char* p) {
  return *reinterpret_cast<const typename Elem<T>::v8*>(p);
}

}  // namespace da
