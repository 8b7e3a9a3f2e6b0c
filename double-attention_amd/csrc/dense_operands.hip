// Operands of the dense outer-attention backward (the training path's
// library-GEMM backward for long sequences and wide scores, the products of
// the reference's attention backward, triton_kernels.py:2093-2263), formed in
// one pass over the score maps: for every (sequence, map) the [T, R] query
// and key rows q and k (strided views of the routed rows) become
//   key_t   [B*S, R, T]  K^T in the score dtype (the right operand of S = q k^T)
//   q_out   [B*S, T, R]  q in the value dtype    (the right operand of dk = dS^T q)
//   k_out   [B*S, T, R]  k in the value dtype    (the right operand of dq = dS k)
// A workgroup of 256 threads takes 32 tokens x 64 features of one map: one
// 16-byte chunk of q and of k per thread, stored converted, and k through an
// LDS tile for the transposed store (feature f of tokens t .. t+7 as one
// 16-byte chunk; element stores at a ragged end).
#include "da_common.h"
#include "da_launch.h"

namespace da {

namespace {

constexpr int kDoTokens = 32, kDoFeatures = 64;

template <typename TQ, typename TV>
__global__ __launch_bounds__(256) void dense_operands_kernel(DenseOperandArgs a) {
  constexpr int PITCH = kDoFeatures + 8;   // elements per LDS row (16 bytes of padding)
  __shared__ __attribute__((aligned(16))) uint16_t tile[kDoTokens * PITCH];
  const int tid = static_cast<int>(threadIdx.x);
  const int t0 = static_cast<int>(blockIdx.x) * kDoTokens;
  const int f0 = static_cast<int>(blockIdx.y) * kDoFeatures;
  const int bs = static_cast<int>(blockIdx.z);
  const int b = bs / a.S, s = bs - b * a.S;
  const int64_t base = b * a.stride_b + (s / a.map_repeat) * a.map_stride;
  // Thread -> (token r, chunk ch) of the 32 x 64 tile.
  const int r = tid >> 3, ch = tid & 7;
  const int t = min(t0 + r, a.T - 1);   // rows past the sequence re-read the last one, stored nowhere
  const int64_t src = base + static_cast<int64_t>(t) * a.stride_t + f0 + ch * 8;
  const typename Elem<TQ>::v8 qv = load8(static_cast<const TQ*>(a.q) + src);
  const typename Elem<TQ>::v8 kv = load8(static_cast<const TQ*>(a.k) + src);
  *reinterpret_cast<u32x4*>(tile + r * PITCH + ch * 8) = __builtin_bit_cast(u32x4, kv);
  if (t0 + r < a.T) {
    typename Elem<TV>::v8 qo, ko;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qo[e] = static_cast<TV>(static_cast<float>(qv[e]));
      ko[e] = static_cast<TV>(static_cast<float>(kv[e]));
    }
    const int64_t dst = (static_cast<int64_t>(bs) * a.T + t0 + r) * a.R + f0 + ch * 8;
    store16B(static_cast<TV*>(a.q_out) + dst, __builtin_bit_cast(u32x4, qo));
    store16B(static_cast<TV*>(a.k_out) + dst, __builtin_bit_cast(u32x4, ko));
  }
  __syncthreads();
  // Thread -> (feature f, tokens 8 tg .. 8 tg + 7) of the transposed tile.
  const int f = tid >> 2, tg = tid & 3;
  uint16_t* out = static_cast<uint16_t*>(a.key_t) + (static_cast<int64_t>(bs) * a.R + f0 + f) * a.T + t0 + 8 * tg;
  const int n = min(8, a.T - (t0 + 8 * tg));
  if (n == 8 && a.T % 8 == 0) {
    u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = static_cast<uint32_t>(tile[(8 * tg + 2 * j) * PITCH + f]) |
             (static_cast<uint32_t>(tile[(8 * tg + 2 * j + 1) * PITCH + f]) << 16);
    store16B(out, v);
  } else {
    for (int j = 0; j < n; ++j) out[j] = tile[(8 * tg + j) * PITCH + f];
  }
}

template <typename TQ>
void launch_t(const DenseOperandArgs& a, dim3 grid, hipStream_t s) {
  if (a.out_dtype == kF16) hipLaunchKernelGGL((dense_operands_kernel<TQ, _Float16>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((dense_operands_kernel<TQ, __bf16>), grid, dim3(256), 0, s, a);
}

}  // namespace

void launch_dense_operands(const DenseOperandArgs& a, hipStream_t stream) {
  if (a.B * a.S == 0 || a.T == 0) return;
  const dim3 grid(static_cast<unsigned>((a.T + kDoTokens - 1) / kDoTokens), static_cast<unsigned>(a.R / kDoFeatures),
                  static_cast<unsigned>(a.B * a.S));
  if (a.qk_dtype == kF16) launch_t<_Float16>(a, grid, stream);
  else launch_t<__bf16>(a, grid, stream);
}

}  // namespace da
