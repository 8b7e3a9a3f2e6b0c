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
// One workgroup (4 waves) owns 64 query rows of one sequence and walks the
// (map, 32-key tile) sequence up to the causal bound.  Work happens in the
// transposed domain:
//   S^T[key, q] = sum_r K[key, r] Q^T[r, q]      (A = key rows from LDS, B = queries in VGPRs)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P in VGPRs)
// so P never leaves registers and each score tile is computed once for the
// full value width D.  Key and V^T tiles are double-buffered in LDS and
// filled by global->LDS DMA while the previous tile is multiplied.  V comes
// token-contiguous (V^T, [B, D, Tv]) from the projection GEMM's epilogue.
// gamma_s = exp(clamp(log scale)) and the mix weights are computed on the
// device, so a forward never synchronizes with the host.
//
// Element types: TQ for the routed queries/keys (fp16 on the module path: they
// are unit vectors), TV for V and the probabilities (the model dtype).
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kKeyTile = 32;

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

template <typename TQ, typename TV, int RP, int D>
struct AttnTile {
  static constexpr int NCK = RP / 8;                  // 16B chunks per key row
  static constexpr int KCH = kKeyTile * NCK;          // chunks in the key tile
  static constexpr int VCK = kKeyTile / 8;            // chunks per V^T row (4)
  static constexpr int VCH = D * VCK;                 // chunks in the V^T tile
  static constexpr int BYTES = (KCH + VCH) * 16;
  static_assert(KCH % 256 == 0 && VCH % 256 == 0, "tile must split evenly over 256 lanes");

  // Issue the DMA of key tile [k0, k0+32) of map offset `off` into `buf`.
  static __device__ __forceinline__ void issue(char* buf, const TQ* kbase, const TV* vtb,
                                               const AttnParams& p, int64_t off, int k0, int wave,
                                               int lane) {
#pragma unroll
    for (int i = 0; i < KCH / 256; ++i) {
      const int j = i * 4 + wave;
      int row, ck;
      chunk_of<NCK, true>(j * 64 + lane, row, ck);
      // Rows past the sequence end are masked to -inf; any valid row will do.
      const int key = min(k0 + row, p.T - 1);
      dma16(kbase + static_cast<int64_t>(key) * p.qk_stride_t + off + ck * 8, buf + j * 1024);
    }
#pragma unroll
    for (int i = 0; i < VCH / 256; ++i) {
      const int j = i * 4 + wave;
      int d, ck;
      chunk_of<VCK, false>(j * 64 + lane, d, ck);
      int key = k0 + ck * 8;
      // Chunks wholly past the end read token 0 (their P is zero); a chunk
      // that straddles the end reads the V^T row padding, which the producer
      // keeps finite.
      if (key >= p.T) key = 0;
      dma16(vtb + d * p.vt_stride_d + key, buf + KCH * 16 + j * 1024);
    }
  }
};

template <typename TQ, typename TV, int RP, int D, bool MULTI>
__global__ __launch_bounds__(256) void attention_kernel(AttnParams p) {
  typedef AttnTile<TQ, TV, RP, D> Tile;
  typedef typename Elem<TQ>::v8 q8;
  constexpr int KS = RP / 32;
  constexpr int QT = 64;   // queries per workgroup
  __shared__ __attribute__((aligned(1024))) char lds0[Tile::BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int n_qt = (p.T + QT - 1) / QT;
  const int qt = n_qt - 1 - static_cast<int>(blockIdx.x);   // heaviest causal tiles first
  const int b = blockIdx.y;
  const int q0 = qt * QT;
  const int tq = q0 + wave * 16 + c;                       // this lane's query token
  const bool q_ok = tq < p.T;
  const bool causal = p.flags & kAttnCausal;
  const int q_last = min(q0 + QT, p.T) - 1;
  const int n_kt = causal ? q_last / kKeyTile + 1 : (p.T + kKeyTile - 1) / kKeyTile;
  const int total = p.S * n_kt;

  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b;
  const TQ* kbase = static_cast<const TQ*>(p.k) + b * p.qk_stride_b;
  const TV* vtb = static_cast<const TV*>(p.vt) + b * p.vt_stride_b;

  f32x4 yacc[MULTI ? D / 16 : 1];
  if constexpr (MULTI) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) yacc[i] = zero4();
  }
  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = zero4();
  float m_run = -INFINITY;
  float l_part = 0.f;
  q8 qf[KS];
  float sc = 0.f;

  auto map_offset = [&](int s) -> int64_t { return static_cast<int64_t>(s / p.map_repeat) * p.map_stride; };
  auto load_map = [&](int s) {
    const int64_t off = map_offset(s);
    sc = map_gamma(p, s) * kLog2e;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[kk] = q_ok ? load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + off + kk * 32 + 8 * g)
                    : zero8<TQ>();
  };

  // One pipeline step: tile u is resident in `cur`; prefetch u+1 into `nxt`.
  auto step = [&](int u, char* cur, char* nxt) {
    wait_vmem();
    __syncthreads();
    if (u + 1 < total) {
      const int s1 = (u + 1) / n_kt;
      Tile::issue(nxt, kbase, vtb, p, map_offset(s1), ((u + 1) - s1 * n_kt) * kKeyTile, wave, lane);
    }
    const int s = u / n_kt;
    const int kt = u - s * n_kt;
    const int k0 = kt * kKeyTile;

    // Scores: two independent accumulator chains (the two 16-key blocks),
    // fragments read from LDS in batches ahead of their MFMAs.
    f32x4 st[2] = {zero4(), zero4()};
    {
      const int row0 = blocked_row(0, c);
      const int row1 = blocked_row(1, c);
      constexpr int KB = KS < 4 ? KS : 4;
#pragma unroll
      for (int kk0 = 0; kk0 < KS; kk0 += KB) {
        u32x4 a0[KB], a1[KB];
#pragma unroll
        for (int i = 0; i < KB; ++i) {
          a0[i] = lds_chunk<Tile::NCK, true>(cur, row0, (kk0 + i) * 4 + g);
          a1[i] = lds_chunk<Tile::NCK, true>(cur, row1, (kk0 + i) * 4 + g);
        }
#pragma unroll
        for (int i = 0; i < KB; ++i) {
          st[0] = Elem<TQ>::mma(as_v8<TQ>(a0[i]), qf[kk0 + i], st[0]);
          st[1] = Elem<TQ>::mma(as_v8<TQ>(a1[i]), qf[kk0 + i], st[1]);
        }
      }
    }
    // Lane (c, g) now holds keys k0 + 8g + 4kb + i of query tq.
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = k0 + 8 * g + 4 * kb + i;
        const bool ok = key < p.T && (!causal || key <= tq);
        const float v = ok ? st[kb][i] * sc : -INFINITY;
        st[kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    lazy_rescale<D / 16>(group_max(tmax), m_run, l_part, acc);
    const float m_use = m_run == -INFINITY ? 0.f : m_run;   // fully masked so far
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = exp2f(st[kb][i] - m_use);
        st[kb][i] = pr;
        psum += pr;
      }
    }
    l_part += psum;
    const typename Elem<TV>::v8 pb = pack_blocked<TV>(st[0], st[1]);   // keys k0 + 8g + e
    const char* vtile = cur + Tile::KCH * 16;
    constexpr int DB = D / 16 < 8 ? D / 16 : 8;
#pragma unroll
    for (int db0 = 0; db0 < D / 16; db0 += DB) {
      u32x4 a[DB];
#pragma unroll
      for (int i = 0; i < DB; ++i) a[i] = lds_chunk<Tile::VCK, false>(vtile, (db0 + i) * 16 + c, g);
#pragma unroll
      for (int i = 0; i < DB; ++i) acc[db0 + i] = Elem<TV>::mma(as_v8<TV>(a[i]), pb, acc[db0 + i]);
    }

    if (kt == n_kt - 1) {   // map s complete
      const float l = group_sum(l_part);
      const float w = map_weight(p, s) / (l > 0.f ? l : 1.f);
      if constexpr (MULTI) {
#pragma unroll
        for (int i = 0; i < D / 16; ++i) yacc[i] += acc[i] * w;
      } else {
        if (q_ok) store_rows<TV, D>(p, b, (p.flags & kAttnMix) ? 0 : s, tq, g, acc, w);
      }
#pragma unroll
      for (int i = 0; i < D / 16; ++i) acc[i] = zero4();
      m_run = -INFINITY;
      l_part = 0.f;
      if (s + 1 < p.S) load_map(s + 1);
    }
  };

  load_map(0);
  Tile::issue(lds0, kbase, vtb, p, map_offset(0), 0, wave, lane);
  int u = 0;
  for (; u + 1 < total; u += 2) {
    step(u, lds0, lds1);
    step(u + 1, lds1, lds0);
  }
  if (u < total) step(u, lds0, lds1);

  if constexpr (MULTI) {
    if (q_ok) store_rows<TV, D>(p, b, 0, tq, g, yacc, 1.f);
  }
}

template <typename TQ, typename TV, int RP, int D, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  const int n_qt = (a.T + 63) / 64;
  hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, D, MULTI>), dim3(n_qt, a.B), dim3(256), 0, s, p);
}

template <typename TQ, typename TV, int RP, int D>
static void launch_attn_2(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  if ((a.flags & kAttnMix) && a.S > 1) launch_attn_3<TQ, TV, RP, D, true>(a, p, s);
  else launch_attn_3<TQ, TV, RP, D, false>(a, p, s);
}

template <typename TQ, typename TV, int RP>
static void launch_attn_1(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  switch (a.D) {
    case 64: launch_attn_2<TQ, TV, RP, 64>(a, p, s); break;
    case 128: launch_attn_2<TQ, TV, RP, 128>(a, p, s); break;
    case 256: launch_attn_2<TQ, TV, RP, 256>(a, p, s); break;
    default: launch_attn_2<TQ, TV, RP, 512>(a, p, s); break;
  }
}

template <typename TQ, typename TV>
static void launch_attn_0(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  switch (a.RP) {
    case 64: launch_attn_1<TQ, TV, 64>(a, p, s); break;
    case 128: launch_attn_1<TQ, TV, 128>(a, p, s); break;
    case 256: launch_attn_1<TQ, TV, 256>(a, p, s); break;
    default: launch_attn_1<TQ, TV, 512>(a, p, s); break;
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
  if (a.qk_dtype == kF16 && a.v_dtype == kBF16) launch_attn_0<_Float16, __bf16>(a, p, stream);
  else if (a.qk_dtype == kF16) launch_attn_0<_Float16, _Float16>(a, p, stream);
  else launch_attn_0<__bf16, __bf16>(a, p, stream);
}

}  // namespace da
