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
//   mode 0: out[j, i]                 -- features i of token j (Q/K projection,
//                                        output projection)
//   mode 1: out[b, j_feature, t] (V^T) -- value features in the token-contiguous
//                                        layout the attention kernel streams.
//           Rows i run over B * Tp "virtual" tokens (t < Tp, the padded
//           length); tokens past T reuse the last real row, so the padding of
//           V^T is always finite.
// Tiles: 128 x 128 per workgroup, 64-wide K stages double-buffered in LDS and
// filled by global->LDS DMA; each of the four waves owns a 64 x 64 quadrant
// (4 x 4 MFMA 16x16x32 blocks).
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kBI = 128;
constexpr int kBJ = 128;
constexpr int kBK = 64;
constexpr int kGemmNck = kBK / 8;                        // chunks per tile row
constexpr int kGemmTileBytes = kBI * kBK * 2;            // one operand tile

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
  int tiles_i, tiles;
};

struct GemmParams {
  GemmSeg seg[2];
  int nseg;
};

template <typename T>
__device__ __forceinline__ const T* p_row(const GemmSeg& sg, int64_t i) {
  const T* p0 = static_cast<const T*>(sg.p0);
  i = min(i, sg.I - 1);   // rows of a partial last tile are computed but never stored
  if (sg.mode == 1) {   // virtual token i = b * Tp + t of the value segment
    const int64_t b = i / sg.Tp;
    const int64_t t = min(i % sg.Tp, sg.T - 1);
    return p0 + (b * sg.T + t) * sg.K;
  }
  return i < sg.p_split ? p0 + i * sg.K : static_cast<const T*>(sg.p1) + (i - sg.p_split) * sg.K;
}

template <typename T>
__device__ __forceinline__ void issue_stage(char* buf, const GemmSeg& sg, int64_t i0, int64_t j0, int k0,
                                            int wave, int lane) {
  const T* qq = static_cast<const T*>(sg.q);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int j = it * 4 + wave;
    int r, ck;
    chunk_of<kGemmNck, false>(j * 64 + lane, r, ck);
    // Columns past K only occur in a final half stage that is never read.
    const int kc = min(k0 + ck * 8, static_cast<int>(sg.K) - 8);
    dma16(p_row<T>(sg, i0 + r) + kc, buf + j * 1024);
    const int64_t jr = min(j0 + r, sg.J - 1);
    dma16(qq + jr * sg.K + kc, buf + kGemmTileBytes + j * 1024);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams prm) {
  typedef typename Elem<T>::v8 v8;
  __shared__ __attribute__((aligned(1024))) char lds0[2 * kGemmTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds1[2 * kGemmTileBytes];

  int tile = blockIdx.x;
  const int si = (prm.nseg > 1 && tile >= prm.seg[0].tiles) ? 1 : 0;
  if (si) tile -= prm.seg[0].tiles;
  const GemmSeg& sg = prm.seg[si];
  const int64_t i0 = static_cast<int64_t>(tile % sg.tiles_i) * kBI;
  const int64_t j0 = static_cast<int64_t>(tile / sg.tiles_i) * kBJ;

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int wi = wave & 1;
  const int wj = wave >> 1;
  const int K = static_cast<int>(sg.K);
  const int n_stages = (K + kBK - 1) / kBK;

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

  auto step = [&](int st, char* cur, char* nxt) {
    wait_vmem();
    __syncthreads();
    if (st + 1 < n_stages) issue_stage<T>(nxt, sg, i0, j0, (st + 1) * kBK, wave, lane);
    const int ksteps = min(kBK, K - st * kBK) / 32;
    for (int kk = 0; kk < ksteps; ++kk) {
      v8 af[4], bf[4];
#pragma unroll
      for (int a = 0; a < 4; ++a)
        af[a] = as_v8<T>(lds_chunk<kGemmNck, false>(cur, wi * 64 + a * 16 + c, kk * 4 + g));
#pragma unroll
      for (int b = 0; b < 4; ++b)
        bf[b] = as_v8<T>(lds_chunk<kGemmNck, false>(cur + kGemmTileBytes, wj * 64 + b * 16 + c, kk * 4 + g));
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = Elem<T>::mma(af[a], bf[b], acc[a][b]);
    }
  };

  issue_stage<T>(lds0, sg, i0, j0, 0, wave, lane);
  int st = 0;
  for (; st + 1 < n_stages; st += 2) {
    step(st, lds0, lds1);
    step(st + 1, lds1, lds0);
  }
  if (st < n_stages) step(st, lds0, lds1);

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
      typename Elem<T>::v4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float bi = 0.f;
        if (sg.mode == 0 && sg.bias && i + r < sg.I) bi = load_scalar(sg.bias, sg.bias_dtype, i + r);
        o[r] = static_cast<T>(acc[a][b][r] + bi + bj);
      }
      if (sg.mode == 0) {
        T* dst = out + j * sg.ldo + i;
        if (i + 4 <= sg.I) {
          *reinterpret_cast<typename Elem<T>::v4*>(dst) = o;
        } else {
          for (int r = 0; r < 4 && i + r < sg.I; ++r) dst[r] = o[r];
        }
      } else {
        // Four consecutive virtual tokens of one sequence (Tp % 64 == 0).
        const int64_t bb = i / sg.Tp;
        const int64_t t = i % sg.Tp;
        *reinterpret_cast<typename Elem<T>::v4*>(out + bb * sg.vt_stride_b + j * sg.Tp + t) = o;
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
    d.p1 = a.p1 ? a.p1 : a.p0;
    d.p_split = a.p1 ? a.p_split : a.I;
    d.q = a.q;
    d.mode = a.mode;
    d.T = a.T > 0 ? a.T : 1;
    d.Tp = a.Tp > 0 ? a.Tp : 1;
    // The value segment runs over B * Tp virtual tokens (a.I = B * T real ones).
    d.I = a.mode == 1 ? (a.I / d.T) * d.Tp : a.I;
    d.J = a.J;
    d.K = a.K;
    d.bias = a.bias;
    d.bias_dtype = a.bias_dtype;
    d.out = a.out;
    d.ldo = a.ldo;
    d.vt_stride_b = a.vt_stride_b;
    d.tiles_i = static_cast<int>((d.I + kBI - 1) / kBI);
    d.tiles = d.tiles_i * static_cast<int>((a.J + kBJ - 1) / kBJ);
    total += d.tiles;
  }
  if (nseg == 1) prm.seg[1] = prm.seg[0];
  if (total == 0) return;
  if (dtype == kF16) hipLaunchKernelGGL((gemm_kernel<_Float16>), dim3(total), dim3(256), 0, stream, prm);
  else hipLaunchKernelGGL((gemm_kernel<__bf16>), dim3(total), dim3(256), 0, stream, prm);
}

}  // namespace da
