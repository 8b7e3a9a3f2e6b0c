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
// A workgroup of four waves owns 64 query rows of one sequence: wave w takes
// the 32 queries of group w%2 (two 16-column MFMA blocks) and half w/2 of the
// value width.  It walks the (map, 32-key tile) sequence up to the causal
// bound in the transposed domain:
//   S^T[key, q] = sum_r K[key, r] Q^T[r, q]      (A = key rows from LDS, B = queries in VGPRs)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P in VGPRs)
// so P never leaves registers, and every A fragment read from LDS feeds two
// MFMAs (the two query blocks).  Key and V^T tiles are double-buffered in
// padded LDS tiles (da_tile.h) filled by global->LDS DMA while the previous
// tile is multiplied.  V^T arrives from the projection GEMM in 32-token tiles
// (element (b, d, t) at b*stride_b + (t/32)*32*D + 32*d + t%32), so each V tile
// is one contiguous block.  gamma_s = exp(clamp(log scale)) and the mix
// weights are computed on the device: a forward never synchronizes with the
// host.
//
// Element types: TQ for the routed queries/keys (fp16 on the module path: they
// are unit vectors), TV for V, the probabilities and the output.
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kKeyTile = 32;
constexpr int kAttnWaves = 4;   // 2 query groups x 2 value halves
constexpr int kAttnQW = 32;     // queries per wave
constexpr int kAttnQT = 64;     // queries per workgroup

struct AttnParams {
  const void* q;
  const void* k;
  int64_t qk_stride_b, qk_stride_t, map_stride;
  int map_repeat;
  const void* vt;
  int64_t vt_stride_b;
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

// Store DC accumulator columns (value features d0 .. d0+DC-1) of query t.
template <typename T, int DC>
__device__ __forceinline__ void store_rows(const AttnParams& p, int b, int s, int t, int g, int d0,
                                           const f32x4* acc, float w) {
  T* orow = static_cast<T*>(p.out) + b * p.out_stride_b + static_cast<int64_t>(t) * p.out_stride_t +
            s * p.out_stride_s + d0;
#pragma unroll
  for (int db = 0; db < DC / 16; ++db) {
    typename Elem<T>::v4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<T>(acc[db][i] * w);
    *reinterpret_cast<typename Elem<T>::v4*>(orow + db * 16 + 4 * g) = o;
  }
}

template <int RP, int D>
struct AttnTile {
  typedef PaddedTile<kKeyTile, RP / 8, true> KT;    // keys (blocked rows)
  typedef PaddedTile<D, kKeyTile / 8, false> VT;    // V^T rows: D features x 4 chunks
  static constexpr int LOADS = KT::LOADS + VT::LOADS;
  static constexpr int PER_WAVE = (LOADS + kAttnWaves - 1) / kAttnWaves;
  static constexpr int BYTES = LOADS * 1024;        // K tile, then V^T tile
};

template <typename TQ, typename TV, int RP, int D, bool MULTI>
__global__ __launch_bounds__(kAttnWaves * 64) void attention_kernel(AttnParams p) {
  typedef AttnTile<RP, D> Tile;
  typedef typename Tile::KT KT;
  typedef typename Tile::VT VT;
  typedef typename Elem<TQ>::v8 q8;
  constexpr int KS = RP / 32;
  constexpr int DC = D / 2;      // value columns per wave
  constexpr int NB = DC / 16;    // accumulator blocks per query block
  __shared__ __attribute__((aligned(1024))) char lds0[Tile::BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  const int qg = wave & 1;
  const int d0 = (wave >> 1) * DC;
  const int n_qt = (p.T + kAttnQT - 1) / kAttnQT;
  const int qt = n_qt - 1 - static_cast<int>(blockIdx.x);   // heaviest causal tiles first
  const int b = blockIdx.y;
  const int q0 = qt * kAttnQT;
  const int qw0 = q0 + qg * kAttnQW;                         // this wave's first query
  const bool causal = p.flags & kAttnCausal;
  const int q_last = min(q0 + kAttnQT, p.T) - 1;
  const int n_kt = causal ? q_last / kKeyTile + 1 : (p.T + kKeyTile - 1) / kKeyTile;
  const int total = p.S * n_kt;

  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b;
  const TQ* kbase = static_cast<const TQ*>(p.k) + b * p.qk_stride_b;
  const TV* vtb = static_cast<const TV*>(p.vt) + b * p.vt_stride_b;

  // Per-lane DMA descriptors of this wave's share of a tile: key loads keep
  // (row, chunk*8) packed, V^T loads their element offset inside the tile.
  int desc[Tile::PER_WAVE];
#pragma unroll
  for (int i = 0; i < Tile::PER_WAVE; ++i) {
    const int j = i * kAttnWaves + wave;
    int row = 0, ck = 0;
    if (j < KT::LOADS) {
      KT::slot_chunk(j * 64 + lane, row, ck);
      desc[i] = (row << 16) | (ck * 8);
    } else if (j < Tile::LOADS) {
      VT::slot_chunk((j - KT::LOADS) * 64 + lane, row, ck);
      desc[i] = row * kKeyTile + ck * 8;
    } else {
      desc[i] = 0;
    }
  }
  auto issue = [&](char* buf, int u) {
    const int s = u / n_kt;
    const int k0 = (u - s * n_kt) * kKeyTile;
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride;
    const TQ* ktile = kbase + static_cast<int64_t>(k0) * p.qk_stride_t + off;
    const TV* vtile = vtb + static_cast<int64_t>(k0) * D;   // 32-token tile k0/32
    const int last = p.T - 1 - k0;                           // keys past the end re-read the last one
#pragma unroll
    for (int i = 0; i < Tile::PER_WAVE; ++i) {
      const int j = i * kAttnWaves + wave;
      if (j < KT::LOADS) {
        const int row = min(desc[i] >> 16, last);
        dma16(ktile + static_cast<int64_t>(row) * p.qk_stride_t + (desc[i] & 0xffff), buf + j * 1024);
      } else if (j < Tile::LOADS) {
        dma16(vtile + desc[i], buf + j * 1024);
      }
    }
  };

  f32x4 acc[2][NB];
  f32x4 yacc[MULTI ? 2 : 1][MULTI ? NB : 1];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      acc[cb][i] = zero4();
      if constexpr (MULTI) yacc[cb][i] = zero4();
    }
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_part[2] = {0.f, 0.f};
  q8 qf[2][KS];
  float sc = 0.f;

  auto load_map = [&](int s) {
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride;
    sc = map_gamma(p, s) * kLog2e;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        qf[cb][kk] = tq < p.T ? load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + off + kk * 32 + 8 * g)
                              : zero8<TQ>();
    }
  };

  // Lane-relative LDS bases of the fragment reads.
  const int kfrag = KT::offset(c, g);
  const int vfrag = KT::BYTES + VT::offset(d0 + c, g);

  auto step = [&](int u, char* cur, char* nxt) {
    wait_vmem();
    __syncthreads();
    if (u + 1 < total) issue(nxt, u + 1);
    const int s = u / n_kt;
    const int kt = u - s * n_kt;
    const int k0 = kt * kKeyTile;

    // Scores for 32 keys x 32 queries: four independent accumulator chains,
    // each key fragment feeding both query blocks.
    f32x4 st[2][2] = {{zero4(), zero4()}, {zero4(), zero4()}};
    const char* kf = cur + kfrag;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const q8 a0 = lds_v8<TQ>(kf + KT::offset(0, kk * 4));
      const q8 a1 = lds_v8<TQ>(kf + KT::offset(16, kk * 4));
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        st[cb][0] = Elem<TQ>::mma(a0, qf[cb][kk], st[cb][0]);
        st[cb][1] = Elem<TQ>::mma(a1, qf[cb][kk], st[cb][1]);
      }
    }
    // Lane (c, g) holds keys k0 + 8g + 4kb + i for query qw0 + 16cb + c.
    const bool masked = (causal && k0 + kKeyTile - 1 > qw0) || k0 + kKeyTile > p.T;
    typename Elem<TV>::v8 pb[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = st[cb][kb][i] * sc;
          if (masked) {
            const int key = k0 + 8 * g + 4 * kb + i;
            if (key >= p.T || (causal && key > tq)) v = -INFINITY;
          }
          st[cb][kb][i] = v;
          tmax = fmaxf(tmax, v);
        }
      }
      lazy_rescale<NB>(group_max(tmax), m_run[cb], l_part[cb], acc[cb]);
      const float m_use = m_run[cb] == -INFINITY ? 0.f : m_run[cb];   // fully masked so far
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(st[cb][kb][i] - m_use);
          st[cb][kb][i] = pr;
          psum += pr;
        }
      }
      l_part[cb] += psum;
      pb[cb] = pack_blocked<TV>(st[cb][0], st[cb][1]);   // keys k0 + 8g + e
    }

    const char* vf = cur + vfrag;
#pragma unroll
    for (int db = 0; db < NB; ++db) {
      const typename Elem<TV>::v8 a = lds_v8<TV>(vf + VT::offset(db * 16, 0));
      acc[0][db] = Elem<TV>::mma(a, pb[0], acc[0][db]);
      acc[1][db] = Elem<TV>::mma(a, pb[1], acc[1][db]);
    }

    if (kt == n_kt - 1) {   // map s complete
      const float wmap = map_weight(p, s);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const float l = group_sum(l_part[cb]);
        const float w = wmap / (l > 0.f ? l : 1.f);
        const int tq = qw0 + cb * 16 + c;
        if constexpr (MULTI) {
#pragma unroll
          for (int i = 0; i < NB; ++i) yacc[cb][i] += acc[cb][i] * w;
        } else {
          if (tq < p.T) store_rows<TV, DC>(p, b, (p.flags & kAttnMix) ? 0 : s, tq, g, d0, acc[cb], w);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) acc[cb][i] = zero4();
        m_run[cb] = -INFINITY;
        l_part[cb] = 0.f;
      }
      if (s + 1 < p.S) load_map(s + 1);
    }
  };

  load_map(0);
  issue(lds0, 0);
  int u = 0;
  for (; u + 1 < total; u += 2) {
    step(u, lds0, lds1);
    step(u + 1, lds1, lds0);
  }
  if (u < total) step(u, lds0, lds1);

  if constexpr (MULTI) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
      if (tq < p.T) store_rows<TV, DC>(p, b, 0, tq, g, d0, yacc[cb], 1.f);
    }
  }
}

template <typename TQ, typename TV, int RP, int D, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, const AttnParams& p, hipStream_t s) {
  const int n_qt = (a.T + kAttnQT - 1) / kAttnQT;
  hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, D, MULTI>), dim3(n_qt, a.B), dim3(kAttnWaves * 64), 0, s, p);
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
