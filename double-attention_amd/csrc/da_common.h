// Shared device helpers for the gfx950 shared-dictionary attention kernels.
//
// Every contraction in this library runs on the CDNA4 16x16x32 MFMA
// (v_mfma_f32_16x16x32_{bf16,f16}).  Lane layout used throughout, for a wave of
// 64 lanes with lane = 16*g + c (g = lane/16 in 0..3, c = lane%16 in 0..15):
//   A operand (16 x 32):  lane supplies row c, eight k values "chunk g"
//   B operand (32 x 16):  lane supplies column c, eight k values "chunk g"
//   C/D (16 x 16 fp32):   lane holds column c, rows 4g .. 4g+3
// The hardware contracts A's element e of chunk g with B's element e of chunk
// g, so any assignment of the 32 k indices to (g, e) is valid as long as A and
// B use the same one.  Two assignments are used:
//   "linear":   k = 8g + e                         (operands read from memory)
//   "blocked":  k = 4g + e (e < 4), 16 + 4g + e-4  (e >= 4)
// The blocked one is exactly how two vertically stacked 16x16 accumulator
// blocks are spread over the lanes, so a softmax tile that was produced as an
// accumulator can be fed back as a B operand without leaving registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace da {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element-type traits: 16-bit storage type, 8- and 4-wide vectors, MFMA.
template <typename T> struct Elem;

template <> struct Elem<__bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Elem<_Float16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Scalar dtype codes shared with the C ABI (include/double_attention_hip.h).
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

__device__ __forceinline__ float load_scalar(const void* p, int dtype, int64_t i) {
  if (dtype == kF32) return static_cast<const float*>(p)[i];
  if (dtype == kF16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return static_cast<float>(static_cast<const __bf16*>(p)[i]);
}

// Element i of a scalar array in two steps: fetch_scalar issues two 16-bit
// loads without branching on the dtype (the second re-reads the first for
// 16-bit types), so their wait falls at the first use; scalar_value
// assembles and converts.
struct ScalarHalves {
  uint16_t lo, hi;
};
__device__ __forceinline__ ScalarHalves fetch_scalar(const void* p, int dtype, int64_t i) {
  const bool wide = dtype == kF32;
  const uint16_t* h = static_cast<const uint16_t*>(p) + (wide ? 2 * i : i);
  return ScalarHalves{h[0], h[wide ? 1 : 0]};
}
__device__ __forceinline__ float scalar_value(ScalarHalves v, int dtype) {
  const uint32_t lo = v.lo, hi = v.hi;
  if (dtype == kF32) return __uint_as_float(hi << 16 | lo);
  if (dtype == kF16) return static_cast<float>(__builtin_bit_cast(_Float16, v.lo));
  return __uint_as_float(lo << 16);
}

// MI355X: eight XCDs, each with its own L2; workgroups are dealt to them
// round-robin in dispatch order.
constexpr int kXcds = 8;

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Reductions across the four 16-lane rows (lanes c, c+16, c+32, c+48 hold the
// same accumulator column), with gfx950's v_permlane32_swap / v_permlane16_swap:
// swapping a value with itself leaves the two halves (rows) exchanged between
// the pair of results, so one VALU op pairs lane l with lane l^32 (l^16) and no
// LDS round trip is needed.
__device__ __forceinline__ void lane_pair32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void lane_pair16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// Sum over the 64 lanes of a wave.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ __forceinline__ float group_max(float v) {
  float a, b;
  lane_pair32(v, a, b);
  lane_pair16(fmaxf(a, b), a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float group_sum(float v) {
  float a, b;
  lane_pair32(v, a, b);
  lane_pair16(a + b, a, b);
  return a + b;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

constexpr float kLog2e = 1.4426950408889634f;

// Online-softmax bookkeeping with lazy rescaling, in the log2 domain.  Each
// lane holds raw scores of one accumulator column c; the exponent of a score s
// is s * scale - m, where m (column-uniform) is a running reference maximum.
// m only moves -- and the accumulators are rescaled -- when some score exceeds
// it by more than kRescaleSlack, so exponentials stay <= 2^kRescaleSlack
// (exact in fp16/bf16 operands) and most tiles skip both the rescale and the
// cross-lane maximum: the test uses each lane's own maximum, and only when
// the wave's ballot says some lane exceeded does it reduce the column maxima
// across the lane rows.  Columns that do not need it keep factor 1; the common
// factor 2^-m cancels in the final division by the row sum.
constexpr float kRescaleSlack = 8.f;

template <int N>
__device__ __forceinline__ void lazy_rescale(float lane_max, float scale, float& m_run, float& l_part,
                                             f32x4* acc) {
  if (__ballot(lane_max * scale > m_run + kRescaleSlack)) {
    const float tile_max = group_max(lane_max) * scale;
    const bool need = tile_max > m_run + kRescaleSlack;
    const float alpha = need ? exp2f(m_run - tile_max) : 1.f;
    if (need) m_run = tile_max;
    l_part *= alpha;
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] *= alpha;
  }
}

// Build a B operand (8 values of T) from two stacked 16x16 fp32 accumulator
// blocks using the "blocked" k assignment described above.
template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 pack_blocked(const f32x4& lo, const f32x4& hi) {
  typename Elem<T>::v8 r;
  r[0] = static_cast<T>(lo[0]);
  r[1] = static_cast<T>(lo[1]);
  r[2] = static_cast<T>(lo[2]);
  r[3] = static_cast<T>(lo[3]);
  r[4] = static_cast<T>(hi[0]);
  r[5] = static_cast<T>(hi[1]);
  r[6] = static_cast<T>(hi[2]);
  r[7] = static_cast<T>(hi[3]);
  return r;
}

// A operand with the "blocked" k assignment from a row-major 16-bit tile:
// elements [4g, 4g+4) and [16+4g, 16+4g+4) of the 32-wide k window at `row`.
template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 load_blocked(const T* row, int g) {
  typedef typename Elem<T>::v4 v4;
  v4 lo = *reinterpret_cast<const v4*>(row + 4 * g);
  v4 hi = *reinterpret_cast<const v4*>(row + 16 + 4 * g);
  typename Elem<T>::v8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 load8(const T* p) {
  return *reinterpret_cast<const typename Elem<T>::v8*>(p);
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 zero8() {
  typename Elem<T>::v8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = static_cast<T>(0.f);
  return r;
}

__device__ __forceinline__ u32x4 load16B(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void store16B(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

}  // namespace da
