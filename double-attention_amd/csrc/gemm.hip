// MFMA GEMM for the projections of SharedDictionaryAttention.
//
// Replaces the fused Q/K projection (reference src/double_attention/modules.py:143-157:
// cat(query.weight, key.weight) then F.linear), the value projection
// (modules.py:83,212) and the output projection (modules.py:117-121,272).
//
// Every launch computes one or two "segments" D[i, j] = sum_k P[i, k] Q[j, k]
// (+ bias), with both operands K-contiguous, as PyTorch stores x [N, d] and
// Linear weights [out, in].  The query and key weights are read as two stacked
// operands, so no concatenated weight is ever materialized.  Epilogues:
//   mode 0: out[j, i]                      -- Q/K features (i) of token j, or the output projection
//   mode 1: out[b, i_feature, t] (V^T)     -- value features in the token-contiguous
//                                             layout the attention kernel streams
// Tiles: 128 x 128 per workgroup, 64-wide K stages staged through LDS; each
// of the four waves owns a 64 x 64 quadrant (4 x 4 MFMA 16x16x32 blocks).
#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kBI = 128;
constexpr int kBJ = 128;
constexpr int kBK = 64;
constexpr int kGemmPad = 8;

struct GemmSeg {
  const void* p0;
  const void* p1;
  int64_t p_split;
  const void* q;
  int64_t I, J, K;
  const void* bias;
  int bias_dtype;
  int mode;
  void* out;
  int64_t ldo;
  int64_t T, Tp, vt_stride_b;
  int tiles_i, tiles;   // tiles along i, total tiles of this segment
};

struct GemmParams {
  GemmSeg seg[2];
  int nseg;
};

template <typename T>
__device__ __forceinline__ void stage_operand(T* lds, const T* p0, const T* p1, int64_t split,
                                              int64_t rows, int64_t K, int64_t r0, int k0) {
  // 128 rows x 64 k = 1024 chunks of 8 elements; 4 per thread.
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int ch = threadIdx.x + it * 256;
    const int r = ch >> 3;
    const int k8 = (ch & 7) * 8;
    const int64_t gr = r0 + r;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (gr < rows && k0 + k8 < K) {
      const T* src = gr < split ? p0 + gr * K : p1 + (gr - split) * K;
      v = load16B(src + k0 + k8);
    }
    store16B(lds + r * (kBK + kGemmPad) + k8, v);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams prm) {
  typedef typename Elem<T>::v8 v8;
  constexpr int ROW = kBK + kGemmPad;
  __shared__ __attribute__((aligned(16))) T as[kBI * ROW];
  __shared__ __attribute__((aligned(16))) T bs[kBJ * ROW];

  int tile = blockIdx.x;
  const int si = (prm.nseg > 1 && tile >= prm.seg[0].tiles) ? 1 : 0;
  if (si) tile -= prm.seg[0].tiles;
  const GemmSeg& sg = prm.seg[si];
  const int64_t i0 = static_cast<int64_t>(tile % sg.tiles_i) * kBI;
  const int64_t j0 = static_cast<int64_t>(tile / sg.tiles_i) * kBJ;

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wi = wave_id() & 1;
  const int wj = wave_id() >> 1;

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

  const T* p0 = static_cast<const T*>(sg.p0);
  const T* p1 = static_cast<const T*>(sg.p1 ? sg.p1 : sg.p0);
  const T* qq = static_cast<const T*>(sg.q);

  for (int k0 = 0; k0 < sg.K; k0 += kBK) {
    __syncthreads();
    stage_operand<T>(as, p0, p1, sg.p_split, sg.I, sg.K, i0, k0);
    stage_operand<T>(bs, qq, qq, sg.J, sg.J, sg.K, j0, k0);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      v8 af[4], bf[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) af[a] = load8(&as[(wi * 64 + a * 16 + c) * ROW + kk * 32 + 8 * g]);
#pragma unroll
      for (int b = 0; b < 4; ++b) bf[b] = load8(&bs[(wj * 64 + b * 16 + c) * ROW + kk * 32 + 8 * g]);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = Elem<T>::mma(af[a], bf[b], acc[a][b]);
    }
  }

  // Epilogue: lane holds D[i0 + wi*64 + a*16 + 4g + r][j0 + wj*64 + b*16 + c], r = 0..3.
  T* out = static_cast<T*>(sg.out);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t j = j0 + wj * 64 + b * 16 + c;
    if (j >= sg.J) continue;
    const float bj = (sg.mode == 1 && sg.bias) ? load_scalar(sg.bias, sg.bias_dtype, j) : 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int64_t i = i0 + wi * 64 + a * 16 + 4 * g;
      if (i >= sg.I) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float bi = 0.f;
        if (sg.mode == 0 && sg.bias && i + r < sg.I) bi = load_scalar(sg.bias, sg.bias_dtype, i + r);
        v[r] = acc[a][b][r] + bi + bj;
      }
      if (sg.mode == 0) {
        T* dst = out + j * sg.ldo + i;
        if (i + 4 <= sg.I) {
          typename Elem<T>::v4 o;
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = static_cast<T>(v[r]);
          *reinterpret_cast<typename Elem<T>::v4*>(dst) = o;
        } else {
          for (int r = 0; r < 4 && i + r < sg.I; ++r) dst[r] = static_cast<T>(v[r]);
        }
      } else {
        // i indexes tokens n = b*T + t, j indexes value features.
        const int64_t bb = i / sg.T;
        const int64_t t = i % sg.T;
        T* dst = out + bb * sg.vt_stride_b + j * sg.Tp + t;
        if (i + 4 <= sg.I && t + 4 <= sg.T && (sg.T % 4) == 0) {
          typename Elem<T>::v4 o;
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = static_cast<T>(v[r]);
          *reinterpret_cast<typename Elem<T>::v4*>(dst) = o;
        } else {
          for (int r = 0; r < 4 && i + r < sg.I; ++r) {
            const int64_t n = i + r;
            out[(n / sg.T) * sg.vt_stride_b + j * sg.Tp + (n % sg.T)] = static_cast<T>(v[r]);
          }
        }
      }
    }
  }
}

void launch_gemm(const GemmSegment* segs, int nseg, int dtype, hipStream_t stream) {
  GemmParams prm;
  prm.nseg = nseg;
  int total = 0;
  for (int s = 0; s < nseg; ++s) {
    GemmSeg& d = prm.seg[s];
    const GemmSegment& a = segs[s];
    d.p0 = a.p0;
    d.p1 = a.p1;
    d.p_split = a.p1 ? a.p_split : a.I;
    d.q = a.q;
    d.I = a.I;
    d.J = a.J;
    d.K = a.K;
    d.bias = a.bias;
    d.bias_dtype = a.bias_dtype;
    d.mode = a.mode;
    d.out = a.out;
    d.ldo = a.ldo;
    d.T = a.T > 0 ? a.T : 1;
    d.Tp = a.Tp;
    d.vt_stride_b = a.vt_stride_b;
    d.tiles_i = static_cast<int>((a.I + kBI - 1) / kBI);
    d.tiles = d.tiles_i * static_cast<int>((a.J + kBJ - 1) / kBJ);
    total += d.tiles;
  }
  if (nseg == 1) prm.seg[1] = prm.seg[0];
  if (total == 0) return;
  if (dtype == kF16) hipLaunchKernelGGL((gemm_kernel<_Float16>), dim3(total), dim3(256), 0, stream, prm);
  else hipLaunchKernelGGL((gemm_kernel<__bf16>), dim3(total), dim3(256), 0, stream, prm);
}

}  // namespace da
