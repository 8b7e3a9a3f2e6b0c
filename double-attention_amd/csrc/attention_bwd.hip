// Backward of the outer routed attention (ops.py:65-93), per score map:
// given the forward's inputs, the per-row log-sum-exp and dO, it forms
//   dV = P^T dO,  dP = dO V^T,  dS = P (dP - rowsum(dO . O)),
//   dQ = gamma dS K,  dK = gamma dS^T Q,  dgamma = sum dS . (Q K^T),
// the flash-attention backward (the reference's Triton kernels compute the
// same products, triton_kernels.py:814-1278 and 2093-2263).
//
// attention_lse_kernel: per query row, LSE2 = m + log2(l) over its keys with
// p = 2^(s gamma log2e - LSE2), one wave per 32 queries, key fragments read
// straight from global memory.
//
// attention_bwd_kernel: one workgroup per (sequence x map, 32-key tile), four
// waves.  The key tile (and each wave's share of V and K^T) stays resident;
// the workgroup walks the query tiles that see its keys, staging Q, Q^T, dO
// and dO^T tiles in LDS.  Every wave forms the full 32 x 32 S^T and P^T; the
// dP^T contraction over the value features is split over the waves and summed
// through LDS; P^T, dS^T and dS go through LDS into the layouts the last three
// products read.  dV (shared by the maps) and dQ (shared by the key tiles)
// accumulate with fp32 atomics, dK is stored once.
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

namespace {

constexpr int kBwdTile = 32;   // keys per workgroup, queries per step

struct BwdParams {
  const void* q;        // [BS][T][RP] routed queries (score dtype)
  const void* k;        // [BS][T][RP] routed keys
  const void* qt;       // [BS][Tp/32][RP][32] Q^T tiles
  const void* kt;       // [BS][Tp/32][RP][32] K^T tiles
  const void* v;        // [B][T][D] values
  const void* dout;     // [BS][T][D] output gradient
  const void* doutt;    // [BS][Tp/32][D][32] its transposed tiles
  float* lse2;          // [BS][T] (written by the LSE pass)
  const float* dvec;    // [BS][T] rowsum(dO . O)
  const float* gamma;   // [S] score scales
  float* dq;            // [BS][T][RP] (accumulated)
  float* dk;            // [BS][T][RP]
  float* dv;            // [B][T][D] (accumulated)
  float* dgamma;        // [S] (accumulated)
  int S, T, Tp, RP, D;
  int causal;
};

// LDS tile pitches (bytes): row-major tiles get one 16-byte pad chunk per
// row, transposed 32-token tiles a 16-byte pad on their 64-byte rows, so the
// 16-byte fragment reads of 8 consecutive lanes hit distinct bank groups.
__host__ __device__ constexpr int row_pitch(int width) { return width * 2 + 16; }
constexpr int kTPitch = 80;

}  // namespace

template <typename TQ, int RP>
__global__ __launch_bounds__(256) void attention_lse_kernel(BwdParams p) {
  typedef typename Elem<TQ>::v8 q8;
  constexpr int KS = RP / 32;
  const int lane = lane_id();
  const int c = lane & 15, g = lane >> 4;
  const int bs = static_cast<int>(blockIdx.y);
  const int q0 = (static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x) / 64) * kBwdTile;
  if (q0 >= p.T) return;   // whole waves
  const int s = bs % p.S;
  const float sc = p.gamma[s] * kLog2e;
  const TQ* qb = static_cast<const TQ*>(p.q) + static_cast<int64_t>(bs) * p.T * RP;
  const TQ* kbase = static_cast<const TQ*>(p.k) + static_cast<int64_t>(bs) * p.T * RP;
  q8 qf[2][KS];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[cb][kk] = load8(qb + static_cast<int64_t>(min(q0 + cb * 16 + c, p.T - 1)) * RP + kk * 32 + 8 * g);
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  const int k_end = p.causal ? min(q0 + kBwdTile, p.T) : p.T;
  for (int k0 = 0; k0 < k_end; k0 += kBwdTile) {
    f32x4 st[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const TQ* krow = kbase + static_cast<int64_t>(min(k0 + kb * 16 + c, p.T - 1)) * RP + 8 * g;
      q8 kf[KS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) kf[kk] = load8(krow + kk * 32);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        st[kb][cb] = zero4();
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) st[kb][cb] = Elem<TQ>::mma(kf[kk], qf[cb][kk], st[kb][cb]);
      }
    }
    // Lane (c, g) holds keys k0 + 16kb + 4g + i of query q0 + 16cb + c.
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int q = q0 + cb * 16 + c;
      float t[8];
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + kb * 16 + 4 * g + i;
          const bool live = key < p.T && (!p.causal || key <= q);
          t[kb * 4 + i] = live ? st[kb][cb][i] * sc : -INFINITY;
          mx = fmaxf(mx, t[kb * 4 + i]);
        }
      mx = group_max(mx);
      const float mn = fmaxf(m[cb], mx);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += mn == -INFINITY ? 0.f : exp2f(t[e] - mn);
      sum = group_sum(sum);
      l[cb] = (m[cb] == -INFINITY ? 0.f : l[cb] * exp2f(m[cb] - mn)) + sum;
      m[cb] = mn;
    }
  }
  if (g == 0) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int q = q0 + cb * 16 + c;
      if (q < p.T) p.lse2[static_cast<int64_t>(bs) * p.T + q] = m[cb] + log2f(l[cb]);
    }
  }
}

template <typename TQ, typename TV, int RP, int D>
__global__ __launch_bounds__(256, 1) void attention_bwd_kernel(BwdParams p) {
  typedef typename Elem<TQ>::v8 q8;
  typedef typename Elem<TV>::v8 v8;
  constexpr int KS = RP / 32;                  // 32-deep steps over the score width
  constexpr int DC = D / 32;                   // 32-deep chunks of the value width
  constexpr int MYDC = (DC + 3) / 4;           // chunks per wave (round robin)
  constexpr int DB = D / 16 / 4;               // 16-wide dV column blocks per wave
  constexpr int RB = RP / 16 / 4;              // 16-wide dK / dQ column blocks per wave
  static_assert(D / 16 % 4 == 0 && RP / 16 % 4 == 0, "widths of at least 64");
  constexpr int KP = row_pitch(RP), VP = row_pitch(D);
  // LDS: key tile, Q tile, Q^T tile, dO tile, dO^T tile, P^T, dS^T, dS,
  // the dP^T partials of the four waves, LSE2 and rowsum rows.
  constexpr int OFF_K = 0;
  constexpr int OFF_Q = OFF_K + kBwdTile * KP;
  constexpr int OFF_QT = OFF_Q + kBwdTile * KP;
  constexpr int OFF_DO = OFF_QT + RP * kTPitch;
  constexpr int OFF_DOT = OFF_DO + kBwdTile * VP;
  constexpr int OFF_PT = OFF_DOT + D * kTPitch;
  constexpr int OFF_DST = OFF_PT + kBwdTile * kTPitch;
  constexpr int OFF_DS = OFF_DST + kBwdTile * kTPitch;
  constexpr int OFF_RED = OFF_DS + kBwdTile * kTPitch;
  constexpr int OFF_ROW = OFF_RED + 4 * 64 * 16 * 4;
  constexpr int LDS_BYTES = OFF_ROW + 2 * kBwdTile * 4;
  static_assert(LDS_BYTES <= 160 * 1024, "the tiles fit the LDS");
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];

  const int lane = lane_id();
  const int c = lane & 15, g = lane >> 4;
  const int wave = uniform_wave();
  const int tid = static_cast<int>(threadIdx.x);
  const int bs = static_cast<int>(blockIdx.y);
  const int b = bs / p.S, s = bs - b * p.S;
  const int k0 = static_cast<int>(blockIdx.x) * kBwdTile;
  const float gamma = p.gamma[s];
  const float sc = gamma * kLog2e;
  const TQ* qb = static_cast<const TQ*>(p.q) + static_cast<int64_t>(bs) * p.T * RP;
  const TQ* kbase = static_cast<const TQ*>(p.k) + static_cast<int64_t>(bs) * p.T * RP;
  const TQ* qtb = static_cast<const TQ*>(p.qt) + static_cast<int64_t>(bs) * p.Tp * RP;
  const TQ* ktb = static_cast<const TQ*>(p.kt) + static_cast<int64_t>(bs) * p.Tp * RP;
  const TV* vb = static_cast<const TV*>(p.v) + static_cast<int64_t>(b) * p.T * D;
  const TV* dob = static_cast<const TV*>(p.dout) + static_cast<int64_t>(bs) * p.T * D;
  const TV* dotb = static_cast<const TV*>(p.doutt) + static_cast<int64_t>(bs) * p.Tp * D;

  // Resident: the key tile (rows past T repeat row T-1; their P is masked to
  // zero), this wave's V chunks (A operands of dP^T) and K^T blocks (B
  // operands of dQ).
  for (int ch = tid; ch < kBwdTile * RP / 8; ch += 256) {
    const int r = ch / (RP / 8), c8 = (ch % (RP / 8)) * 8;
    *reinterpret_cast<u32x4*>(lds + OFF_K + r * KP + c8 * 2) =
        *reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(min(k0 + r, p.T - 1)) * RP + c8);
  }
  v8 vf[MYDC][2];
#pragma unroll
  for (int j = 0; j < MYDC; ++j) {
    const int chunk = min(wave + 4 * j, DC - 1);   // waves past the last chunk repeat it (unused)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      vf[j][kb] = load8(vb + static_cast<int64_t>(min(k0 + kb * 16 + c, p.T - 1)) * D + chunk * 32 + 8 * g);
  }
  q8 ktf[RB];
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const int r = (wave + 4 * j) * 16 + c;
    ktf[j] = load8(ktb + (static_cast<int64_t>(k0 / 32) * RP + r) * 32 + 8 * g);
  }

  f32x4 dv_acc[2][DB], dk_acc[2][RB];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int j = 0; j < DB; ++j) dv_acc[kb][j] = zero4();
#pragma unroll
    for (int j = 0; j < RB; ++j) dk_acc[kb][j] = zero4();
  }
  float dgamma = 0.f;
  const int n_qt = (p.T + kBwdTile - 1) / kBwdTile;
  const int qt_first = p.causal ? static_cast<int>(blockIdx.x) : 0;
  float* red = reinterpret_cast<float*>(lds + OFF_RED);
  float* rowv = reinterpret_cast<float*>(lds + OFF_ROW);

  for (int qt = qt_first; qt < n_qt; ++qt) {
    const int q0 = qt * kBwdTile;
    __syncthreads();   // the previous step is done with every staged tile
    for (int ch = tid; ch < kBwdTile * RP / 8; ch += 256) {
      const int r = ch / (RP / 8), c8 = (ch % (RP / 8)) * 8;
      *reinterpret_cast<u32x4*>(lds + OFF_Q + r * KP + c8 * 2) =
          *reinterpret_cast<const u32x4*>(qb + static_cast<int64_t>(min(q0 + r, p.T - 1)) * RP + c8);
    }
    for (int ch = tid; ch < RP * 4; ch += 256) {
      const int r = ch / 4, c8 = (ch % 4) * 8;
      *reinterpret_cast<u32x4*>(lds + OFF_QT + r * kTPitch + c8 * 2) =
          *reinterpret_cast<const u32x4*>(qtb + (static_cast<int64_t>(qt) * RP + r) * 32 + c8);
    }
    for (int ch = tid; ch < kBwdTile * D / 8; ch += 256) {
      const int r = ch / (D / 8), c8 = (ch % (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(lds + OFF_DO + r * VP + c8 * 2) =
          *reinterpret_cast<const u32x4*>(dob + static_cast<int64_t>(min(q0 + r, p.T - 1)) * D + c8);
    }
    for (int ch = tid; ch < D * 4; ch += 256) {
      const int r = ch / 4, c8 = (ch % 4) * 8;
      *reinterpret_cast<u32x4*>(lds + OFF_DOT + r * kTPitch + c8 * 2) =
          *reinterpret_cast<const u32x4*>(dotb + (static_cast<int64_t>(qt) * D + r) * 32 + c8);
    }
    if (tid < 2 * kBwdTile) {
      const int q = q0 + (tid & 31);
      const float* src = tid < kBwdTile ? p.lse2 : p.dvec;
      rowv[tid] = q < p.T ? src[static_cast<int64_t>(bs) * p.T + q] : 0.f;
    }
    __syncthreads();

    // S^T (keys x queries), every wave in full: A = key rows, B = query rows.
    f32x4 st[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) st[kb][cb] = zero4();
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      q8 kf[2], qf[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        kf[h] = *reinterpret_cast<const q8*>(lds + OFF_K + (h * 16 + c) * KP + (kk * 32 + 8 * g) * 2);
        qf[h] = *reinterpret_cast<const q8*>(lds + OFF_Q + (h * 16 + c) * KP + (kk * 32 + 8 * g) * 2);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) st[kb][cb] = Elem<TQ>::mma(kf[kb], qf[cb], st[kb][cb]);
    }
    // P^T: lane (c, g) element i is key k0 + 16kb + 4g + i, query q0 + 16cb + c.
    f32x4 pt[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int q = q0 + cb * 16 + c;
      const float lse = rowv[cb * 16 + c];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + kb * 16 + 4 * g + i;
          const bool live = q < p.T && key < p.T && (!p.causal || key <= q);
          pt[kb][cb][i] = live ? exp2f(st[kb][cb][i] * sc - lse) : 0.f;
        }
    }
    // dP^T = V dO^T over this wave's value chunks, summed over the waves.
    f32x4 dpt[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) dpt[kb][cb] = zero4();
#pragma unroll
    for (int j = 0; j < MYDC; ++j) {
      const int chunk = wave + 4 * j;
      if (chunk >= DC) break;
      v8 df[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        df[cb] = *reinterpret_cast<const v8*>(lds + OFF_DO + (cb * 16 + c) * VP + (chunk * 32 + 8 * g) * 2);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) dpt[kb][cb] = Elem<TV>::mma(vf[j][kb], df[cb], dpt[kb][cb]);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        *reinterpret_cast<f32x4*>(red + ((wave * 64 + lane) * 4 + kb * 2 + cb) * 4) = dpt[kb][cb];
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        f32x4 sum = zero4();
#pragma unroll
        for (int w = 0; w < 4; ++w) sum += *reinterpret_cast<const f32x4*>(red + ((w * 64 + lane) * 4 + kb * 2 + cb) * 4);
        dpt[kb][cb] = sum;
      }
    // dS^T = P^T (dP^T - rowsum(dO . O)).
    f32x4 dst[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const float dvq = rowv[kBwdTile + cb * 16 + c];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[kb][cb][i] = pt[kb][cb][i] * (dpt[kb][cb][i] - dvq);
    }
    // Wave w owns block (kb, cb) = (w >> 1, w & 1): it writes P^T and dS^T as
    // [key][query] rows and dS as [query][key] rows, and adds dS . raw scores
    // of that block to dgamma.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        if (kb * 2 + cb != wave) continue;
        TV* ptl = reinterpret_cast<TV*>(lds + OFF_PT);
        TQ* dstl = reinterpret_cast<TQ*>(lds + OFF_DST);
        typename Elem<TQ>::v4 dsq;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb * 16 + 4 * g + i, q = cb * 16 + c;
          ptl[key * (kTPitch / 2) + q] = static_cast<TV>(pt[kb][cb][i]);
          dstl[key * (kTPitch / 2) + q] = static_cast<TQ>(dst[kb][cb][i]);
          dsq[i] = static_cast<TQ>(dst[kb][cb][i]);
          dgamma += dst[kb][cb][i] * st[kb][cb][i];
        }
        *reinterpret_cast<typename Elem<TQ>::v4*>(lds + OFF_DS + (cb * 16 + c) * kTPitch + (kb * 16 + 4 * g) * 2) = dsq;
      }
    __syncthreads();

    // dV += P^T dO (B: dO^T rows), dK += dS^T Q (B: Q^T rows), dQ = dS K.
    v8 pa[2];
    q8 da[2], dsa[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      pa[h] = *reinterpret_cast<const v8*>(lds + OFF_PT + (h * 16 + c) * kTPitch + 8 * g * 2);
      da[h] = *reinterpret_cast<const q8*>(lds + OFF_DST + (h * 16 + c) * kTPitch + 8 * g * 2);
      dsa[h] = *reinterpret_cast<const q8*>(lds + OFF_DS + (h * 16 + c) * kTPitch + 8 * g * 2);
    }
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      const int d = (wave + 4 * j) * 16 + c;
      const v8 bf = *reinterpret_cast<const v8*>(lds + OFF_DOT + d * kTPitch + 8 * g * 2);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) dv_acc[kb][j] = Elem<TV>::mma(pa[kb], bf, dv_acc[kb][j]);
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int r = (wave + 4 * j) * 16 + c;
      const q8 bf = *reinterpret_cast<const q8*>(lds + OFF_QT + r * kTPitch + 8 * g * 2);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) dk_acc[kb][j] = Elem<TQ>::mma(da[kb], bf, dk_acc[kb][j]);
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int r0 = (wave + 4 * j) * 16;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const f32x4 dqv = Elem<TQ>::mma(dsa[cb], ktf[j], zero4());
        // Lane (c, g) element i: query q0 + 16cb + 4g + i, feature r0 + c.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = q0 + cb * 16 + 4 * g + i;
          if (q < p.T)
            unsafeAtomicAdd(p.dq + (static_cast<int64_t>(bs) * p.T + q) * RP + r0 + c, dqv[i] * gamma);
        }
      }
    }
  }

  // dK rows of this tile; dV accumulates over the maps; dgamma over tiles.
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = k0 + kb * 16 + 4 * g + i;
      if (key >= p.T) continue;
#pragma unroll
      for (int j = 0; j < RB; ++j)
        p.dk[(static_cast<int64_t>(bs) * p.T + key) * RP + (wave + 4 * j) * 16 + c] = dk_acc[kb][j][i] * gamma;
#pragma unroll
      for (int j = 0; j < DB; ++j)
        unsafeAtomicAdd(p.dv + (static_cast<int64_t>(b) * p.T + key) * D + (wave + 4 * j) * 16 + c, dv_acc[kb][j][i]);
    }
  dgamma = wave_sum(dgamma);
  if (lane == 0) unsafeAtomicAdd(p.dgamma + s, dgamma);
}

template <typename TQ, typename TV, int RP>
static void launch_bwd_r(const BwdParams& p, int B, hipStream_t stream) {
  const int n_kt = (p.T + kBwdTile - 1) / kBwdTile;
  const dim3 lse_grid(static_cast<unsigned>((n_kt + 3) / 4), static_cast<unsigned>(B * p.S));
  hipLaunchKernelGGL((attention_lse_kernel<TQ, RP>), lse_grid, dim3(256), 0, stream, p);
  const dim3 grid(static_cast<unsigned>(n_kt), static_cast<unsigned>(B * p.S));
  switch (p.D) {
    case 64: hipLaunchKernelGGL((attention_bwd_kernel<TQ, TV, RP, 64>), grid, dim3(256), 0, stream, p); break;
    case 128: hipLaunchKernelGGL((attention_bwd_kernel<TQ, TV, RP, 128>), grid, dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((attention_bwd_kernel<TQ, TV, RP, 256>), grid, dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL((attention_bwd_kernel<TQ, TV, RP, 512>), grid, dim3(256), 0, stream, p); break;
  }
}

template <typename TQ, typename TV>
static void launch_bwd_t(const BwdParams& p, int B, hipStream_t stream) {
  switch (p.RP) {
    case 64: launch_bwd_r<TQ, TV, 64>(p, B, stream); break;
    case 128: launch_bwd_r<TQ, TV, 128>(p, B, stream); break;
    default: launch_bwd_r<TQ, TV, 256>(p, B, stream); break;
  }
}

void launch_routed_attention_backward(const AttentionBwdArgs& a, hipStream_t stream) {
  BwdParams p{a.q, a.k, a.qt, a.kt, a.v, a.dout, a.doutt, a.lse2, a.dvec, a.gamma, a.dq, a.dk, a.dv, a.dgamma,
              a.S, a.T, static_cast<int>(round_up(a.T, kKeyPad)), a.RP, a.D, a.causal ? 1 : 0};
  if (a.qk_dtype == kF16) {
    if (a.v_dtype == kBF16) launch_bwd_t<_Float16, __bf16>(p, a.B, stream);
    else launch_bwd_t<_Float16, _Float16>(p, a.B, stream);
  } else {
    launch_bwd_t<__bf16, __bf16>(p, a.B, stream);
  }
}

}  // namespace da
