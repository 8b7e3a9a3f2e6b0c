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
// A workgroup of NW waves (2 or 4) owns 32*NW query rows of one sequence and
// a slice of DS value features; every wave owns 32 queries (two 16-column MFMA
// blocks) and the whole slice, so no score tile is formed twice inside a
// workgroup.  The value width is split over workgroups (DS <= 128) to keep a
// wave's accumulators small enough for two waves per SIMD.  A wave walks the
// (map, 32-key tile) sequence up to the causal bound in the transposed domain:
//   S^T[key, q] = sum_r K[key, r] Q^T[r, q]      (A = key rows from LDS, B = queries in VGPRs)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P in VGPRs)
// so P never leaves registers, and every A fragment read from LDS feeds two
// MFMAs (the two query blocks).  Key and V^T tiles are double-buffered in
// padded LDS tiles (da_tile.h) filled by global->LDS DMA; the loads of the next
// tile are spread through the score loop, so no wave stalls on a full memory
// queue in one burst.  V^T arrives from the projection GEMM in 32-token tiles
// (element (b, d, t) at b*stride_b + (t/32)*32*D + 32*d + t%32), so each
// slice of a V tile is one contiguous block.  gamma_s = exp(clamp(log scale))
// and the mix weights are computed on the device: a forward never
// synchronizes with the host.
//
// Element types: TQ for the routed queries/keys (fp16 on the module path: they
// are unit vectors), TV for V, the probabilities and the output.
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

constexpr int kKeyTile = 32;
constexpr int kAttnQW = 32;     // queries per wave

struct AttnParams {
  const void* q;
  const void* k;
  int64_t qk_stride_b, qk_stride_t, map_stride;
  int map_repeat;
  const void* vt;
  int64_t vt_stride_b;
  int S, T, D;
  int n_qt, n_slices;
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

template <int RP, int DS, int NW>
struct AttnTile {
  typedef PaddedTile<kKeyTile, RP / 8, true> KT;    // keys (blocked rows)
  typedef PaddedTile<DS, kKeyTile / 8, false> VT;   // V^T rows: DS features x 4 chunks
  static constexpr int KPW = (KT::LOADS + NW - 1) / NW;   // key loads per wave
  static constexpr int VPW = (VT::LOADS + NW - 1) / NW;   // V^T loads per wave
  static constexpr int BYTES = KT::BYTES + VT::BYTES;     // K tile, then V^T tile
};

template <typename TQ, typename TV, int RP, int DS, int NW, bool MULTI>
__global__ __launch_bounds__(NW * 64, 1) void attention_kernel(AttnParams p) {
  typedef AttnTile<RP, DS, NW> Tile;
  typedef typename Tile::KT KT;
  typedef typename Tile::VT VT;
  typedef typename Elem<TQ>::v8 q8;
  typedef typename Elem<TV>::v8 v8;
  constexpr int KS = RP / 32;
  constexpr int NB = DS / 16;    // accumulator blocks per query block
  constexpr int NL = Tile::KPW + Tile::VPW;
  constexpr int QT = NW * kAttnQW;
  __shared__ __attribute__((aligned(1024))) char lds0[Tile::BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[Tile::BYTES];

  const int lane = lane_id();
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wave = uniform_wave();
  // blockIdx.y ranks query tiles heaviest (causal) first; x = (sequence, slice).
  const int qt = p.n_qt - 1 - static_cast<int>(blockIdx.y);
  const int b = static_cast<int>(blockIdx.x) / p.n_slices;
  const int ds0 = (static_cast<int>(blockIdx.x) - b * p.n_slices) * DS;   // first feature of the slice
  const int q0 = qt * QT;
  const int qw0 = q0 + wave * kAttnQW;                       // this wave's first query
  const bool causal = p.flags & kAttnCausal;
  const int q_last = min(q0 + QT, p.T) - 1;
  const int n_kt = causal ? q_last / kKeyTile + 1 : (p.T + kKeyTile - 1) / kKeyTile;
  const int total = p.S * n_kt;

  const TQ* qbase = static_cast<const TQ*>(p.q) + b * p.qk_stride_b;
  const char* kbase = reinterpret_cast<const char*>(static_cast<const TQ*>(p.k) + b * p.qk_stride_b);
  // Feature d of a 32-token V^T tile sits at 32*d, so the slice is one block.
  const char* vbase = reinterpret_cast<const char*>(static_cast<const TV*>(p.vt) + b * p.vt_stride_b + 32 * ds0);
  const int kstride = static_cast<int>(p.qk_stride_t) * static_cast<int>(sizeof(TQ));   // bytes per key row

  // Per-lane DMA sources of this wave's loads, as byte offsets from the tile's
  // base: key load i fills wave load i*NW + wave of the key tile (row in the
  // top five bits, for clamping the last tile), V^T load i the same wave load
  // of the V^T tile.  Out-of-range wave loads of a partial last round re-load
  // slot data of load 0 into their own slots, which nothing reads.
  uint32_t kdesc[Tile::KPW], vdesc[Tile::VPW];
#pragma unroll
  for (int i = 0; i < Tile::KPW; ++i) {
    int row, ck;
    const int j = i * NW + wave;
    KT::slot_chunk((j < KT::LOADS ? j : 0) * 64 + lane, row, ck);
    kdesc[i] = (static_cast<uint32_t>(row) << 27) | static_cast<uint32_t>(row * kstride + ck * 16);
  }
#pragma unroll
  for (int i = 0; i < Tile::VPW; ++i) {
    int row, ck;
    const int j = i * NW + wave;
    VT::slot_chunk((j < VT::LOADS ? j : 0) * 64 + lane, row, ck);
    vdesc[i] = static_cast<uint32_t>((row * kKeyTile + ck * 8) * sizeof(TV));
  }
  // LDS slot of load n (K loads first); loads past a tile's end rewrite slot 0.
  auto slot_of = [&](int n) {
    if (n < Tile::KPW) {
      const int j = n * NW + wave;
      return j < KT::LOADS ? j * 1024 : 0;
    }
    const int j = (n - Tile::KPW) * NW + wave;
    return KT::BYTES + (j < VT::LOADS ? j * 1024 : 0);
  };
  // Tile u = (map s, key tile kt): byte bases and the clamp row (keys past the
  // end re-read the last one; only the final key tile has any).
  struct Src {
    const char* k;
    const char* v;
    int last;
  };
  auto source = [&](int s, int kt) {
    const int k0 = kt * kKeyTile;
    const int64_t off = static_cast<int64_t>(s / p.map_repeat) * p.map_stride * static_cast<int64_t>(sizeof(TQ));
    return Src{kbase + static_cast<int64_t>(k0) * kstride + off,
               vbase + static_cast<int64_t>(k0) * p.D * static_cast<int64_t>(sizeof(TV)), p.T - 1 - k0};
  };
  auto issue_one = [&](char* buf, const Src& src, int n) {
    if (n < Tile::KPW) {
      uint32_t off = kdesc[n] & 0x07FFFFFFu;
      if (src.last < kKeyTile - 1) {
        const int over = static_cast<int>(kdesc[n] >> 27) - src.last;
        if (over > 0) off -= static_cast<uint32_t>(over * kstride);
      }
      dma16(src.k + off, buf + slot_of(n));
    } else {
      dma16(src.v + vdesc[n - Tile::KPW], buf + slot_of(n));
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
    // The rescale test compares maxima of raw scores, so a negative score
    // scale is folded into the queries instead (negation is exact).
    const float gamma = map_gamma(p, s);
    sc = fabsf(gamma) * kLog2e;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        qf[cb][kk] = tq < p.T ? load8(qbase + static_cast<int64_t>(tq) * p.qk_stride_t + off + kk * 32 + 8 * g)
                              : zero8<TQ>();
        if (gamma < 0.f) qf[cb][kk] = -qf[cb][kk];
      }
    }
  };

  // Lane-relative LDS offsets of the fragment reads.
  const int kfrag = KT::offset(c, g);
  const int vfrag = KT::BYTES + VT::offset(c, g);

  load_map(0);
  {
    const Src src0 = source(0, 0);
#pragma unroll
    for (int n = 0; n < NL; ++n) issue_one(lds0, src0, n);
  }

  int s = 0, kt = 0;
  for (int u = 0; u < total; ++u) {
    char* cur = (u & 1) ? lds1 : lds0;
    char* nxt = (u & 1) ? lds0 : lds1;
    // Tile u + 1; the last step reloads its own tile into the idle buffer.
    int s_n = s, kt_n = kt + 1;
    if (kt_n == n_kt) {
      kt_n = 0;
      ++s_n;
    }
    if (s_n == p.S) {
      s_n = s;
      kt_n = kt;
    }
    const Src src = source(s_n, kt_n);
    const int k0 = kt * kKeyTile;

    wait_vmem();
    __syncthreads();

    if (!(causal && k0 > qw0 + kAttnQW - 1)) {   // else the tile lies above this wave's causal bound
      // Scores for 32 keys x 32 queries: four independent accumulator chains,
      // each key fragment feeding both query blocks; the next tile's loads are
      // spread between the fragment reads.
      f32x4 st[2][2] = {{zero4(), zero4()}, {zero4(), zero4()}};
      const char* kf = cur + kfrag;
      // Software pipeline: the fragments of step kk + 1 are read while the
      // MFMAs of step kk run; scheduling barriers keep the compiler from
      // hoisting every read (which would cost the second wave per SIMD).
      q8 a0 = lds_v8<TQ>(kf + KT::offset(0, 0));
      q8 a1 = lds_v8<TQ>(kf + KT::offset(16, 0));
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        q8 n0 = a0, n1 = a1;
        if (kk + 1 < KS) {
          n0 = lds_v8<TQ>(kf + KT::offset(0, (kk + 1) * 4));
          n1 = lds_v8<TQ>(kf + KT::offset(16, (kk + 1) * 4));
        }
#pragma unroll
        for (int n = 0; n < NL; ++n)
          if (n * KS / NL == kk) issue_one(nxt, src, n);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          st[cb][0] = Elem<TQ>::mma(a0, qf[cb][kk], st[cb][0]);
          st[cb][1] = Elem<TQ>::mma(a1, qf[cb][kk], st[cb][1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        a0 = n0;
        a1 = n1;
      }
      // The first V^T fragments do not depend on the scores: read them before
      // the softmax.
      const char* vf = cur + vfrag;
      v8 va = lds_v8<TV>(vf + VT::offset(0, 0));
      v8 vb = lds_v8<TV>(vf + VT::offset(NB > 1 ? 16 : 0, 0));

      // Lane (c, g) holds keys k0 + 8g + 4kb + i for query qw0 + 16cb + c.
      // Only tiles on the causal diagonal or past the end carry masked keys.
      if ((causal && k0 + kKeyTile - 1 > qw0) || k0 + kKeyTile > p.T) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int tq = qw0 + cb * 16 + c;
          const int kmax = min(causal ? tq : p.T - 1, p.T - 1);   // last key this query sees
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (k0 + 8 * g + 4 * kb + i > kmax) st[cb][kb][i] = -INFINITY;
        }
      }
      v8 pb[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const float lmax = fmaxf(fmaxf(fmaxf(st[cb][0][0], st[cb][0][1]), fmaxf(st[cb][0][2], st[cb][0][3])),
                                 fmaxf(fmaxf(st[cb][1][0], st[cb][1][1]), fmaxf(st[cb][1][2], st[cb][1][3])));
        lazy_rescale<NB>(lmax, sc, m_run[cb], l_part[cb], acc[cb]);
        const float m_use = m_run[cb] == -INFINITY ? 0.f : m_run[cb];   // fully masked so far
        float psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(st[cb][kb][i], sc, -m_use));
            st[cb][kb][i] = pr;
            psum += pr;
          }
        }
        l_part[cb] += psum;
        pb[cb] = pack_blocked<TV>(st[cb][0], st[cb][1]);   // keys k0 + 8g + e
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < NB; ++db) {
        v8 vn = vb;
        if (db + 2 < NB) vn = lds_v8<TV>(vf + VT::offset((db + 2) * 16, 0));
        acc[0][db] = Elem<TV>::mma(va, pb[0], acc[0][db]);
        acc[1][db] = Elem<TV>::mma(va, pb[1], acc[1][db]);
        __builtin_amdgcn_sched_barrier(0);
        va = vb;
        vb = vn;
      }
    } else {
#pragma unroll
      for (int n = 0; n < NL; ++n) issue_one(nxt, src, n);
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
          if (tq < p.T) store_rows<TV, DS>(p, b, (p.flags & kAttnMix) ? 0 : s, tq, g, ds0, acc[cb], w);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) acc[cb][i] = zero4();
        m_run[cb] = -INFINITY;
        l_part[cb] = 0.f;
      }
      if (s + 1 < p.S) load_map(s + 1);
      kt = 0;
      ++s;
    } else {
      ++kt;
    }
  }

  if constexpr (MULTI) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int tq = qw0 + cb * 16 + c;
      if (tq < p.T) store_rows<TV, DS>(p, b, 0, tq, g, ds0, yacc[cb], 1.f);
    }
  }
}

// Workgroups of four waves when there are enough of them to fill the chip
// twice over, else of two waves (more, smaller workgroups).
template <typename TQ, typename TV, int RP, int DS, bool MULTI>
static void launch_attn_3(const AttentionArgs& a, AttnParams& p, hipStream_t s) {
  p.n_slices = a.D / DS;
  const int64_t wg4 = static_cast<int64_t>(a.B) * p.n_slices * ((a.T + 127) / 128);
  if (wg4 >= 512) {
    p.n_qt = static_cast<int>((a.T + 127) / 128);
    hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, 4, MULTI>), dim3(a.B * p.n_slices, p.n_qt), dim3(256), 0,
                       s, p);
  } else {
    p.n_qt = static_cast<int>((a.T + 63) / 64);
    hipLaunchKernelGGL((attention_kernel<TQ, TV, RP, DS, 2, MULTI>), dim3(a.B * p.n_slices, p.n_qt), dim3(128), 0,
                       s, p);
  }
}

// Value slice per workgroup: 128 features (64 when the value width is 64).
template <typename TQ, typename TV, int RP>
static void launch_attn_1(const AttentionArgs& a, AttnParams& p, hipStream_t s) {
  const bool multi = (a.flags & kAttnMix) && a.S > 1;
  if (a.D == 64) {
    if (multi) launch_attn_3<TQ, TV, RP, 64, true>(a, p, s);
    else launch_attn_3<TQ, TV, RP, 64, false>(a, p, s);
  } else {
    if (multi) launch_attn_3<TQ, TV, RP, 128, true>(a, p, s);
    else launch_attn_3<TQ, TV, RP, 128, false>(a, p, s);
  }
}

template <typename TQ, typename TV>
static void launch_attn_0(const AttentionArgs& a, AttnParams& p, hipStream_t s) {
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
  p.D = static_cast<int>(a.D);
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
