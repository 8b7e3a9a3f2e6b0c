// Flash-tiled outer attention with the map mix fused in.
//
// Replaces routed_attention_reference (reference src/double_attention/ops.py:65-93),
// its Triton forward (triton_kernels.py:674-811, 2022-2090) and the map combine
// of SharedDictionaryAttention.forward (modules.py:265-272):
//   O_s = softmax(gamma_s * q_s k_s^T, causal) V          for every outer map s
//   Y   = sum_s alpha_s O_s,  alpha = softmax(map_mix_logits)   (mix mode)
// or every O_s written to its own slot (per-map mode, used by the concat
// combine and by the operator-level API).
//
// One workgroup owns NW*16 query rows of one sequence and loops over the maps
// and over 64-key tiles up to the causal bound.  As in the route kernel, work
// happens in the transposed domain:
//   S^T[key, q] = sum_r K[key, r] Q^T[r, q]      (A = key rows from LDS, B = queries in VGPRs)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P in VGPRs)
// so P never leaves registers and the score tile is computed exactly once per
// (query tile, key tile) for the full value width D -- there is no per-D-block
// recomputation.  V arrives token-contiguous (V^T, [B, D, Tv]) straight from
// the projection GEMM's epilogue.  The temperatures gamma_s = exp(clamp(log
// scale)) and the mix weights are computed on the device from the parameter
// tensors, so a forward never synchronizes with the host.
#include "da_common.h"
#include "da_launch.h"

namespace da {

constexpr int kKeyTile = 64;
constexpr int kAttnKeyPad = 8;
constexpr int kAttnValPad = 8;

struct AttnParams {
  const void* q;
  const void* k;
  int64_t qk_stride_b, qk_stride_t, map_stride;
  int map_repeat;
  const void* vt;
  int64_t vt_stride_b, vt_stride_d;
  int S, T;
  const void* scales;
  int scales_dtype;
  float scale_mult;
  const void* mix_logits;
  int mix_dtype;
  int flags;
  void* out;
  int64_t out_stride_b, out_stride_t, out_stride_s;
};

__device__ __forceinline__ float map_gamma(const AttnParams& p, int s) {
  float v = load_scalar(p.scales, p.scales_dtype, s);
  if (p.flags & kAttnScalesAreLog) v = expf(fminf(fmaxf(v, kLogScaleMin), kLogScaleMax));
  return v * p.scale_mult;
}

__device__ __forceinline__ float map_weight(const AttnParams& p, int s) {
  if (!(p.flags & kAttnMix)) return 1.f;
  if (p.mix_logits == nullptr) return 1.f / static_cast<float>(p.S);
  float mx = -INFINITY;
  for (int i = 0; i < p.S; ++i) mx = fmaxf(mx, load_scalar(p.mix_logits, p.mix_dtype, i));
  float den = 0.f;
  for (int i = 0; i < p.S; ++i) den += expf(load_scalar(p.mix_logits, p.mix_dtype, i) - mx);
  return expf(load_scalar(p.mix_logits, p.mix_dtype, s) - mx) / den;
}

template <typename T, int D>
__device__ __forceinline__ void store_rows(const AttnParams& p, int b, int s, int t, int g,
                                           const f32x4* acc, float w) {
  T* orow = static_cast<T*>(p.out) + b * p.out_stride_b + static_cast<int64_t>(t) * p.out_stride_t +
            s * p.out_stride_s;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    typename Elem<T>::v4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<T>(acc[db][i] * w);
    *reinterpret_cast<typename Elem<T>::v4*>(orow + db * 16 + 4 * g) = o;
  }
}

template <typename T, int RP, int D, int NW, bool MULTI>
__global__ __launch_bounds__(NW * 64) void attention_kernel(AttnParams p) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KS = RP / 32;
  constexpr int KROW = RP + kAttnKeyPad;
  constexpr int VROW = kKeyTile + kAttnValPad;
  constexpr int QT = NW * 16;   // queries per workgroup
  __shared__ __attribute__((aligned(16))) T ks[kKeyTile * KROW];
  __shared__ __attribute__((aligned(16))) T vs[D * VROW];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int n_qt = (p.T + QT - 1) / QT;
  const int qt = n_qt - 1 - static_cast<int>(blockIdx.x);   // heaviest causal tiles first
  const int b = blockIdx.y;
  const int q0 = qt * QT;
  const int tq = q0 + wave_id() * 16 + c;                  // this lane's query token
  const bool q_ok = tq < p.T;
  const bool causal = p.flags & kAttnCausal;
  const int q_last = min(q0 + QT, p.T) - 1;
  const int n_kt = causal ? q_last / kKeyTile + 1 : (p.T + kKeyTile - 1) / kKeyTile;

  const T* qbase = static_cast<const T*>(p.q) + b * p.qk_stride_b;
  const T* kbase = static_cast<const T*>(p.k) + b * p.qk_stride_b;
  const T* vtb = static_cast<const T*>(p.vt) + b * p.vt_stride_b;

  f32x4 yacc[MULTI ? D / 16 : 1];
  if constexpr (MULTI) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) yacc[i] = zero4();
  }

  for (int s = 0; s < p.S; ++s) {
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride;
    const float sc = map_gamma(p, s) * kLog2e;
    v8 qf[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[kk] = q_ok ? load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + off + kk * 32 + 8 * g)
                    : zero8<T>();

    f32x4 acc[D / 16];
#pragma unroll
    for (int i = 0; i < D / 16; ++i) acc[i] = zero4();
    float m_run = -INFINITY;
    float l_part = 0.f;

    for (int kt = 0; kt < n_kt; ++kt) {
      const int k0 = kt * kKeyTile;
      __syncthreads();
      for (int ch = threadIdx.x; ch < kKeyTile * (RP / 8); ch += NW * 64) {
        const int a = ch / (RP / 8);
        const int k8 = ch % (RP / 8);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (k0 + a < p.T) v = load16B(kbase + static_cast<int64_t>(k0 + a) * p.qk_stride_t + off + k8 * 8);
        store16B(&ks[a * KROW + k8 * 8], v);
      }
      for (int ch = threadIdx.x; ch < D * (kKeyTile / 8); ch += NW * 64) {
        const int d = ch / (kKeyTile / 8);
        const int a8 = ch % (kKeyTile / 8);
        const int key = k0 + a8 * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (key < p.T) {
          v = load16B(vtb + d * p.vt_stride_d + key);
          if (key + 8 > p.T) {
            // Zero the tokens past the sequence end: P is zero there, but the
            // padding of V^T is never written and must not inject NaN/Inf.
            // Word w holds tokens key+2w (low half) and key+2w+1 (high half).
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const uint32_t lo = key + 2 * w < p.T ? 0x0000ffffu : 0u;
              const uint32_t hi = key + 2 * w + 1 < p.T ? 0xffff0000u : 0u;
              v[w] &= (lo | hi);
            }
          }
        }
        store16B(&vs[d * VROW + a8 * 8], v);
      }
      __syncthreads();

      f32x4 st[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        f32x4 t = zero4();
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
          t = Elem<T>::mma(load8(&ks[(kb * 16 + c) * KROW + kk * 32 + 8 * g]), qf[kk], t);
        st[kb] = t;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + kb * 16 + 4 * g + i;
          const bool ok = key < p.T && (!causal || key <= tq);
          const float v = ok ? st[kb][i] * sc : -INFINITY;
          st[kb][i] = v;
          tmax = fmaxf(tmax, v);
        }
      }
      const float m_new = fmaxf(m_run, group_max(tmax));
      const float m_use = m_new == -INFINITY ? 0.f : m_new;   // fully masked so far
      const float alpha = exp2f(m_run - m_use);
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = exp2f(st[kb][i] - m_use);
          st[kb][i] = pr;
          psum += pr;
        }
      }
      l_part = l_part * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) acc[i] *= alpha;

      const v8 p0 = pack_blocked<T>(st[0], st[1]);
      const v8 p1 = pack_blocked<T>(st[2], st[3]);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        const T* vrow = &vs[(db * 16 + c) * VROW];
        acc[db] = Elem<T>::mma(load_blocked<T>(vrow, g), p0, acc[db]);
        acc[db] = Elem<T>::mma(load_blocked<T>(vrow + 32, g), p1, acc[db]);
      }
    }

    const float l = group_sum(l_part);
    const float w = map_weight(p, s) / (l > 0.f ? l : 1.f);
    if constexpr (MULTI) {
#pragma unroll
      for (int i = 0; i < D / 16; ++i) yacc[i] += acc[i] * w;
    } else {
      if (q_ok) store_rows<T, D>(p, b, (p.flags & kAttnMix) ? 0 : s, tq, g, acc, w);
    }
  }
  if constexpr (MULTI) {
    if (q_ok) store_rows<T, D>(p, b, 0, tq, g, yacc, 1.f);
  }
}

template <typename T, int RP, int D, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  constexpr int NW = 4;
  const int n_qt = (a.T + NW * 16 - 1) / (NW * 16);
  hipLaunchKernelGGL((attention_kernel<T, RP, D, NW, MULTI>), dim3(n_qt, a.B), dim3(NW * 64), 0, s, p);
}

template <typename T, int RP, int D>
static void launch_attn_2(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  if ((a.flags & kAttnMix) && a.S > 1) launch_attn_3<T, RP, D, true>(a, p, s);
  else launch_attn_3<T, RP, D, false>(a, p, s);
}

template <typename T, int RP>
static void launch_attn_1(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  switch (a.D) {
    case 64: launch_attn_2<T, RP, 64>(a, p, s); break;
    case 128: launch_attn_2<T, RP, 128>(a, p, s); break;
    case 256: launch_attn_2<T, RP, 256>(a, p, s); break;
    default: launch_attn_2<T, RP, 512>(a, p, s); break;
  }
}

template <typename T>
static void launch_attn_0(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  switch (a.RP) {
    case 64: launch_attn_1<T, 64>(a, p, s); break;
    case 128: launch_attn_1<T, 128>(a, p, s); break;
    case 256: launch_attn_1<T, 256>(a, p, s); break;
    default: launch_attn_1<T, 512>(a, p, s); break;
  }
}

void launch_routed_attention(const AttentionArgs& a, hipStream_t stream) {
  if (a.T == 0 || a.B == 0) return;
  AttnParams p;
  p.q = a.q;
  p.k = a.k;
  p.qk_stride_b = a.qk_stride_b;
  p.qk_stride_t = a.qk_stride_t;
  p.map_stride = a.map_stride;
  p.map_repeat = a.map_repeat;
  p.vt = a.vt;
  p.vt_stride_b = a.vt_stride_b;
  p.vt_stride_d = a.vt_stride_d;
  p.S = a.S;
  p.T = a.T;
  p.scales = a.scales;
  p.scales_dtype = a.scales_dtype;
  p.scale_mult = a.scale_mult;
  p.mix_logits = a.mix_logits;
  p.mix_dtype = a.mix_dtype;
  p.flags = a.flags;
  p.out = a.out;
  p.out_stride_b = a.out_stride_b;
  p.out_stride_t = a.out_stride_t;
  p.out_stride_s = a.out_stride_s;
  if (a.dtype == kF16) launch_attn_0<_Float16>(a, p, stream);
  else launch_attn_0<__bf16>(a, p, stream);
}

}  // namespace da
