// Backward of the outer routed attention (ops.py:65-93), per score map:
// given the forward's inputs and output O and dO, it forms
//   dV = sum_s P^T dO,  dP = dO V^T,  dS = P (dP - rowsum(dO . O)),
//   dQ = gamma dS K,  dK = gamma dS^T Q,  dgamma = sum dS . (Q K^T),
// the flash-attention backward (the reference's Triton kernels compute the
// same products, triton_kernels.py:814-1278 and 2093-2263).
//
// Three launches:
//   attention_bwd_prep_kernel  two workgroups per (sequence x map, 32-token
//       tile): one forms Q^T, K^T and dO^T in 32-token tiles (zero past the
//       length) and rowsum(dO . O), the other the value rows (from V^T
//       tiles) and the zeroes of the accumulated gradients;
//   attention_lse_kernel       one workgroup per 32-query tile; its four
//       waves split the key tiles and merge (max, sum) through LDS into
//       LSE2 = m + log2(l) with p = 2^(s gamma log2e - LSE2);
//   attention_bwd_kernel       one workgroup per (64-key tile, run of query
//       tiles); wave w owns keys 16w..16w+15 of the tile.
//
// In the main kernel S = Q K^T and dP = dO V^T come out of the MFMA with
// lane (c, g) holding queries 4g..4g+3 and 16+4g..16+4g+3 of key c.  Those
// eight values are exactly the eight contraction elements a lane supplies to
// a 16x16x32 MFMA whose contraction runs over the 32 queries in that order,
// so P and dS feed dV += P^T dO and dK += dS^T Q straight from registers; the
// B operands read the matching two 8-byte pieces of the dO^T and Q^T tile
// rows.  Only dQ = dS K needs dS with the query as the row, through LDS.
// dQ accumulates over key tiles and dK, dV over query runs (and dV over the
// maps) with fp32 atomics.
#include <type_traits>

#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

namespace {

constexpr int kQTile = 32;    // queries per step (and tokens per transposed tile)
constexpr int kKTile = 64;    // keys per workgroup (16 per wave)

struct BwdParams {
  // Query row t of (sequence b, map s) at q + b q_sb + (s / rep) q_ms + t q_st
  // (elements, score dtype), key rows alike; grad_query and grad_key (fp32)
  // use the same strides.  Contiguous [BS][T][RP] rows are q_sb = S T RP,
  // q_ms = T RP, q_st = RP, rep = 1.
  const void* q;
  const void* k;
  const void* v;        // [B] x v_sb: [Tk][D] value rows (or the prep's copy in vrows)
  const void* out;      // [BS][T][D] forward output, out_dtype
  const void* dout;     // [BS][T][D] output gradient
  void* qt;             // [BS][Tp/32][RP][32] Q^T tiles (workspace)
  void* kt;             // [BS][Tkp/32][RP][32] K^T tiles
  void* doutt;          // [BS][Tp/32][D][32] dO^T tiles
  float* lse2;          // [BS][T]
  float* dvec;          // [BS][T] rowsum(dO . O)
  const void* scales;   // [S] score scales (or their logs), scales_dtype
  float* dq;
  float* dk;
  float* dv;            // [B][Tk][D]
  float* dv_sum;        // [D] column sums of dv over every sequence and key, or nullptr
  float* dv_copies;     // [kDvCopies][D] workspace: the LSE pass's partial column sums
  // With ds_out set the main kernel writes gamma dS (score dtype, rounded
  // once) as rows [BS][T] of ds_ld elements, keys 0 .. Tkp-1, instead of
  // forming dQ = gamma dS K with atomics (dq is then not touched).
  void* ds_out;
  int64_t ds_ld;
  int v_dtype;          // kF16 or kBF16: the element type of dout
  float* dgamma;        // [S] d loss / d scales[s] (of the logs with scales_log)
  int64_t q_sb, q_st, q_ms;
  int64_t k_sb, k_st, k_ms;
  int rep;
  int64_t v_sb;         // elements between sequences' value rows
  // Values given as V^T tiles [B] x vt_sb: [Tkp/32][D][32] (16-bit, vt_dtype):
  // the prep kernel writes them as rows [B][Tkp][D] (TV) into vrows.
  const void* vt;
  int64_t vt_sb;
  int vt_dtype;
  void* vrows;
  int scales_dtype;
  int scales_log;       // gamma = exp(clamp(scales[s], log_lo, log_hi))
  float log_lo, log_hi;
  float scale_mult;     // every gamma times this
  int S, T, Tp, RP, D;
  int Tk, Tkp;          // keys (== T when causal) and their padded count
  int causal;
  int out_dtype;        // kF32, kF16 or kBF16
  int qchunk;           // query tiles per workgroup of the main kernel
  int n_chunks;         // query runs per key tile
};

// LDS pitches (bytes): row-major tiles get one 16-byte pad chunk per row,
// transposed 32-token tiles a 16-byte pad on their 64-byte rows.
__host__ __device__ constexpr int row_pitch(int width) { return width * 2 + 16; }
constexpr int kTPitch = 80;
constexpr int kDsPitch = kKTile * 2 + 16;

// First query / key row of sequence x map bs (elements).
__device__ __forceinline__ int64_t q_rows0(const BwdParams& p, int bs) {
  const int b = bs / p.S, s = bs - b * p.S;
  return b * p.q_sb + (s / p.rep) * p.q_ms;
}
__device__ __forceinline__ int64_t k_rows0(const BwdParams& p, int bs) {
  const int b = bs / p.S, s = bs - b * p.S;
  return b * p.k_sb + (s / p.rep) * p.k_ms;
}

// The score scale of map s as the kernels apply it: scales[s] (or the
// clamped exponential of the log) times scale_mult.
__device__ __forceinline__ float bwd_gamma(const BwdParams& p, int s) {
  float v = load_scalar(p.scales, p.scales_dtype, s);
  if (p.scales_log) v = expf(fminf(fmaxf(v, p.log_lo), p.log_hi));
  return v * p.scale_mult;
}

// Factor from sum dS (q . k) (the gradient at the applied scale) to the
// gradient at scales[s]: scale_mult, or for a log, the applied scale where the
// clamp passes the gradient (log_lo <= scales[s] <= log_hi) and 0 elsewhere.
__device__ __forceinline__ float bwd_dscale_factor(const BwdParams& p, int s) {
  const float v = load_scalar(p.scales, p.scales_dtype, s);
  if (!p.scales_log) return p.scale_mult;
  return v >= p.log_lo && v <= p.log_hi ? expf(v) * p.scale_mult : 0.f;
}

}  // namespace

// Eight 16-bit elements of dtype `dt` (kF16 or kBF16) as floats.
__device__ __forceinline__ void halves_to_float(u32x4 v, int dt, float (&y)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint16_t e = static_cast<uint16_t>(v[j / 2] >> (16 * (j % 2)));
    y[j] = dt == kBF16 ? __uint_as_float(static_cast<uint32_t>(e) << 16)
                       : static_cast<float>(__builtin_bit_cast(_Float16, e));
  }
}

template <typename TQ, typename TV, int RP, int D>
__global__ __launch_bounds__(256) void attention_bwd_prep_kernel(BwdParams p) {
  // Two workgroups per (sequence x map, 32-token tile), blockIdx.z = 0 and
  // 1.  Part 0: the tile's Q, K and dO rows become the Q^T, K^T and dO^T
  // tiles, and the rows' rowsum(dO . O); every global load is issued first
  // (one memory round trip) and the rows meet in LDS behind one barrier
  // (LDS 32 x (2 row_pitch(RP) + row_pitch(D)) bytes).  Part 1: the V^T tile
  // (values given as tiles) becomes value rows through the same LDS, and
  // the accumulated gradients of the tile's rows are zeroed.  (One workgroup
  // doing both took 15.2 us against 14.2 at 8 x 512 tokens, R 256, D 512.)
  constexpr int PQ = row_pitch(RP), PD = row_pitch(D);
  constexpr int NQ = kQTile * RP / 8 / 256;   // 16-byte chunks per thread of a Q or K tile
  constexpr int ND = kQTile * D / 8 / 256;    // of a dO tile, and of a V^T tile (D rows x 4 chunks)
  static_assert(NQ >= 1 && ND >= 1 && kQTile * RP / 8 % 256 == 0 && kQTile * D / 8 % 256 == 0, "whole chunks per thread");
  constexpr int OFF_K = kQTile * PQ, OFF_D = 2 * kQTile * PQ;
  __shared__ __attribute__((aligned(16))) char lds[OFF_D + kQTile * PD];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  const int wave = uniform_wave();
  const int bs = static_cast<int>(blockIdx.y);
  const int b = bs / p.S, s = bs - b * p.S;
  const int tile = static_cast<int>(blockIdx.x);
  const int t0 = tile * kQTile;
  const int64_t tiles = p.Tp / kQTile, ktiles = p.Tkp / kQTile;
  const int64_t rows = static_cast<int64_t>(bs) * p.T;
  const int64_t q0 = q_rows0(p, bs), k0 = k_rows0(p, bs);
  const bool has_q = tile < tiles, has_k = tile < ktiles;   // uniform
  const bool has_v = p.vt != nullptr && s == 0 && has_k;

  if (blockIdx.z == 0) {   // part 0: transposes and sums; part 1: V rows and zeroing
  // 1. Loads.  Rows clamp into their tensors (a tile past the queries or keys
  // re-reads the last row and stores nothing), so the Q, K and dO loads need
  // no branch; O is loaded as two 16-byte halves of a chunk whatever its
  // dtype (a 16-bit chunk reads its 16 bytes twice).
  const TQ* qsrc = static_cast<const TQ*>(p.q) + q0;
  const TQ* ksrc = static_cast<const TQ*>(p.k) + k0;
  const TV* dsrc = static_cast<const TV*>(p.dout) + rows * D;
  u32x4 qv[NQ], kv[NQ], dv8[ND];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int ch = tid + 256 * i, r = ch / (RP / 8), c8 = (ch % (RP / 8)) * 8;
    qv[i] = load16B(qsrc + static_cast<int64_t>(min(t0 + r, p.T - 1)) * p.q_st + c8);
    kv[i] = load16B(ksrc + static_cast<int64_t>(min(t0 + r, p.Tk - 1)) * p.k_st + c8);
  }
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int ch = tid + 256 * i, r = ch / (D / 8), c8 = (ch % (D / 8)) * 8;
    dv8[i] = load16B(dsrc + static_cast<int64_t>(min(t0 + r, p.T - 1)) * D + c8);
  }
  // rowsum(dO . O): wave w takes rows w, w + 4, ..., lane l chunk l of the
  // row (D / 8 <= 64 chunks).
  constexpr int OC = D / 8;
  const int es = p.out_dtype == kF32 ? 4 : 2;
  const char* obase = static_cast<const char*>(p.out);
  u32x4 oa[kQTile / 4], ob[kQTile / 4];
#pragma unroll
  for (int j = 0; j < kQTile / 4; ++j) {
    const int t = min(t0 + wave + 4 * j, p.T - 1);
    const char* at = obase + ((rows + t) * D + min(lane, OC - 1) * 8) * es;
    oa[j] = load16B(at);
    ob[j] = load16B(at + (es == 4 ? 16 : 0));
  }
  // 2. The rows into LDS (zero past the sequence).
  const u32x4 zv = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int ch = tid + 256 * i, r = ch / (RP / 8), c8 = (ch % (RP / 8)) * 8;
    store16B(lds + r * PQ + c8 * 2, t0 + r < p.T ? qv[i] : zv);
    store16B(lds + OFF_K + r * PQ + c8 * 2, t0 + r < p.Tk ? kv[i] : zv);
  }
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int ch = tid + 256 * i, r = ch / (D / 8), c8 = (ch % (D / 8)) * 8;
    store16B(lds + OFF_D + r * PD + c8 * 2, t0 + r < p.T ? dv8[i] : zv);
  }
  __syncthreads();

  // 3. Transposed tiles: feature f of tokens t8 .. t8+7 as one 16-byte chunk.
  auto transposed = [&](int off, int pitch, int width, void* dst) {
    for (int ch = tid; ch < width * 4; ch += 256) {
      const int f = ch / 4, t8 = (ch % 4) * 8;
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = *reinterpret_cast<const uint16_t*>(lds + off + (t8 + 2 * j) * pitch + f * 2);
        const uint32_t hi = *reinterpret_cast<const uint16_t*>(lds + off + (t8 + 2 * j + 1) * pitch + f * 2);
        v[j] = lo | (hi << 16);
      }
      store16B(static_cast<uint16_t*>(dst) + f * kQTile + t8, v);
    }
  };
  if (has_q) transposed(0, PQ, RP, static_cast<TQ*>(p.qt) + (bs * tiles + tile) * RP * kQTile);
  if (has_k) transposed(OFF_K, PQ, RP, static_cast<TQ*>(p.kt) + (bs * ktiles + tile) * RP * kQTile);
  if (has_q) transposed(OFF_D, PD, D, static_cast<TV*>(p.doutt) + (bs * tiles + tile) * D * kQTile);

  // 4. rowsum(dO . O), O in fp32 (out_dtype) keeping this sum free of O's
  // 16-bit rounding, which would otherwise reach every dS = P (dP - rowsum)
  // of the row (and the scale gradient's sum over them).
#pragma unroll
  for (int j = 0; j < kQTile / 4; ++j) {
    const int r = wave + 4 * j, t = t0 + r;
    if (t >= p.T) break;   // uniform over the wave
    float acc = 0.f;
    if (lane < OC) {
      float x[8], y[8];
      halves_to_float(load16B(lds + OFF_D + r * PD + lane * 16), std::is_same<TV, __bf16>::value ? kBF16 : kF16, x);
      if (es == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y[e] = __uint_as_float(oa[j][e]);
          y[4 + e] = __uint_as_float(ob[j][e]);
        }
      } else {
        halves_to_float(oa[j], p.out_dtype, y);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += x[e] * y[e];
    }
    acc = wave_sum(acc);
    if (lane == 0) p.dvec[rows + t] = acc;
  }

    return;
  }

  // 5. The V^T tile transposed into value rows of TV, through the dO region.
  if (has_v) {
    u32x4 vv[ND];
    const uint16_t* vsrc = static_cast<const uint16_t*>(p.vt) + b * p.vt_sb + static_cast<int64_t>(tile) * D * kQTile;
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int ch = tid + 256 * i, f = ch / 4, t8 = (ch % 4) * 8;
      vv[i] = load16B(vsrc + f * kQTile + t8);
    }
    const bool same = p.vt_dtype == (std::is_same<TV, __bf16>::value ? kBF16 : kF16);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int ch = tid + 256 * i, f = ch / 4, t8 = (ch % 4) * 8;
      float y[8];
      halves_to_float(vv[i], p.vt_dtype, y);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint16_t e = same ? static_cast<uint16_t>(vv[i][j / 2] >> (16 * (j % 2)))
                                : __builtin_bit_cast(uint16_t, static_cast<TV>(y[j]));
        *reinterpret_cast<uint16_t*>(lds + OFF_D + (t8 + j) * PD + f * 2) = e;
      }
    }
    __syncthreads();
    TV* vdst = static_cast<TV*>(p.vrows) + (static_cast<int64_t>(b) * p.Tkp + t0) * D;
    for (int ch = tid; ch < kQTile * D / 8; ch += 256) {
      const int r = ch / (D / 8), c8 = (ch % (D / 8)) * 8;
      store16B(vdst + static_cast<int64_t>(r) * D + c8, load16B(lds + OFF_D + r * PD + c8 * 2));
    }
  }

  // Zero the accumulated gradients of this tile's query and key rows.
  const f32x4 z = zero4();
  const int q_rows = p.ds_out ? 0 : max(0, min(kQTile, p.T - t0)), k_rows = max(0, min(kQTile, p.Tk - t0));
  for (int i = tid; i < q_rows * RP / 4; i += 256) {
    const int r = i / (RP / 4), c4 = i - r * (RP / 4);
    reinterpret_cast<f32x4*>(p.dq + q0 + (t0 + r) * p.q_st)[c4] = z;
  }
  for (int i = tid; i < k_rows * RP / 4; i += 256) {
    const int r = i / (RP / 4), c4 = i - r * (RP / 4);
    reinterpret_cast<f32x4*>(p.dk + k0 + (t0 + r) * p.k_st)[c4] = z;
  }
  if (s == 0)
    for (int i = tid; i < k_rows * D / 4; i += 256)
      reinterpret_cast<f32x4*>(p.dv + (static_cast<int64_t>(b) * p.Tk + t0) * D)[i] = z;
  if (bs == 0 && tile == 0 && tid < p.S) p.dgamma[tid] = 0.f;
  if (p.dv_sum && bs == 0 && tile == 0)
    for (int i = tid; i < kDvCopies * D; i += 256) p.dv_copies[i] = 0.f;
}

template <typename TQ, int RP>
__global__ __launch_bounds__(256) void attention_lse_kernel(BwdParams p) {
  typedef typename Elem<TQ>::v8 q8;
  constexpr int KS = RP / 32;
  __shared__ float part[4][2][kQTile];
  const int lane = lane_id();
  const int c = lane & 15, g = lane >> 4;
  const int wave = uniform_wave();
  const int bs = static_cast<int>(blockIdx.y);
  const int q0 = static_cast<int>(blockIdx.x) * kQTile;
  const float sc = bwd_gamma(p, bs % p.S) * kLog2e;
  // Summed over the keys, dV = P^T dO gives the column sums of dO over the
  // queries (every row of P sums to one).  With dv_sum set this workgroup
  // adds those of its 32 rows of dO: one column pair per thread (D <= 512),
  // each row a coalesced pass.  The loads are issued here and summed after
  // the key loop, and the adds (into one of kDvCopies copies of the D sums)
  // come at the end, when the workgroups of a causal staircase finish at
  // different times.  Rows past the sequence re-read its last row and are
  // dropped.
  const int tid0 = static_cast<int>(threadIdx.x);
  const bool col_sums = p.dv_sum != nullptr && tid0 < p.D / 2;
  const int last_row = min(kQTile, p.T - q0) - 1;
  uint32_t dorow[kQTile];
  if (col_sums) {
    const uint32_t* rows = static_cast<const uint32_t*>(p.dout) + (static_cast<int64_t>(bs) * p.T + q0) * (p.D / 2);
#pragma unroll
    for (int r = 0; r < kQTile; ++r) dorow[r] = rows[static_cast<int64_t>(min(r, last_row)) * (p.D / 2) + tid0];
  }
  const TQ* qb = static_cast<const TQ*>(p.q) + q_rows0(p, bs);
  const TQ* kbase = static_cast<const TQ*>(p.k) + k_rows0(p, bs);
  q8 qf[2][KS];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[cb][kk] = load8(qb + static_cast<int64_t>(min(q0 + cb * 16 + c, p.T - 1)) * p.q_st + kk * 32 + 8 * g);
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  const int k_end = p.causal ? min(q0 + kQTile, p.Tk) : p.Tk;
  for (int k0 = wave * kQTile; k0 < k_end; k0 += 4 * kQTile) {
    f32x4 st[2][2];
    // Both key blocks' fragments are loaded before the first MFMA (one
    // memory round trip per tile; the scheduling barrier keeps the second
    // block's loads ahead of the first block's products).
    q8 kf[2][KS];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const TQ* krow = kbase + static_cast<int64_t>(min(k0 + kb * 16 + c, p.Tk - 1)) * p.k_st + 8 * g;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) kf[kb][kk] = load8(krow + kk * 32);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        st[kb][cb] = zero4();
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) st[kb][cb] = Elem<TQ>::mma(kf[kb][kk], qf[cb][kk], st[kb][cb]);
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
          const bool live = key < p.Tk && (!p.causal || key <= q);
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
      part[wave][0][cb * 16 + c] = m[cb];
      part[wave][1][cb * 16 + c] = l[cb];
    }
  }
  __syncthreads();
  const int tid = static_cast<int>(threadIdx.x);
  if (tid < kQTile) {
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mm = fmaxf(mm, part[w][0][tid]);
    float ll = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (part[w][0][tid] != -INFINITY) ll += part[w][1][tid] * exp2f(part[w][0][tid] - mm);
    const int q = q0 + tid;
    if (q < p.T) p.lse2[static_cast<int64_t>(bs) * p.T + q] = mm + log2f(ll);
  }
  if (col_sums) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int r = 0; r < kQTile; ++r) {
      const uint32_t x = r <= last_row ? dorow[r] : 0u;
      if (p.v_dtype == kBF16) {
        s0 += __uint_as_float(x << 16);
        s1 += __uint_as_float(x & 0xffff0000u);
      } else {
        s0 += static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x)));
        s1 += static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x >> 16)));
      }
    }
    // Workgroups spread their adds over kDvCopies copies of the sums (one
    // address per copy takes 1 / kDvCopies of the adds); the main kernel
    // adds the copies up.
    float* copy = p.dv_copies + static_cast<int64_t>((blockIdx.x + blockIdx.y) % kDvCopies) * p.D;
    unsafeAtomicAdd(copy + 2 * tid0, s0);
    unsafeAtomicAdd(copy + 2 * tid0 + 1, s1);
  }
}

// SPLIT = 2 (512-wide scores): two workgroups per (key tile, query run),
// each forming S, P, dP and dS in full but accumulating half of the dV, dK
// and dQ columns, so the accumulators fit the register file.
template <typename TQ, typename TV, int RP, int D, int SPLIT>
__global__ __launch_bounds__(256, 1) void attention_bwd_kernel(BwdParams p) {
  typedef typename Elem<TQ>::v8 q8;
  typedef typename Elem<TV>::v8 v8;
  typedef typename Elem<TQ>::v4 q4;
  typedef typename Elem<TV>::v4 v4;
  constexpr int KS = RP / 32;       // 32-deep steps over the score width
  constexpr int DC = D / 32;        // 32-deep steps over the value width
  constexpr int NV = D / 16 / SPLIT;    // 16-wide dV column blocks of this workgroup
  constexpr int NK = RP / 16 / SPLIT;   // 16-wide dK column blocks
  constexpr int GV = NV < 8 ? NV : 8, GK = NK < 8 ? NK : 8;   // B operands per read group
  constexpr int RB = RP / 64 / SPLIT;   // dQ column blocks per wave
  static_assert(RB >= 1 && NV >= 1, "the split needs wide scores and values");
  constexpr int QP = row_pitch(RP), VP = row_pitch(D);
  // Staged per step by LDS DMA: Q and dO rows, Q^T and dO^T tile rows, each
  // row followed by one 16-byte pad slot (so QP, VP and kTPitch pitches).
  typedef PaddedTile<kQTile, RP / 8, false> QRows;
  typedef PaddedTile<RP / SPLIT, 4, false> QCols;   // Q^T rows of this workgroup's dK columns
  typedef PaddedTile<kQTile, D / 8, false> DRows;
  typedef PaddedTile<D / SPLIT, 4, false> DCols;    // dO^T rows of its dV columns
  static_assert(QRows::PITCH * 16 == QP && DRows::PITCH * 16 == VP && QCols::PITCH * 16 == kTPitch, "pitches");
  constexpr int OFF_Q = 0;
  constexpr int OFF_QT = OFF_Q + QRows::BYTES;
  constexpr int OFF_DO = OFF_QT + QCols::BYTES;
  constexpr int OFF_DOT = OFF_DO + DRows::BYTES;
  constexpr int OFF_DS = OFF_DOT + DCols::BYTES;
  constexpr int OFF_ROW = OFF_DS + kQTile * kDsPitch;
  constexpr int LDS_BYTES = OFF_ROW + 2 * kQTile * 4;
  static_assert(LDS_BYTES <= 160 * 1024, "the tiles fit the LDS");
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];

  const int lane = lane_id();
  const int c = lane & 15, g = lane >> 4;
  const int wave = uniform_wave();
  const int tid = static_cast<int>(threadIdx.x);
  // The value bias's gradient: the LSE pass's copies of the column sums of
  // dO, added up by one workgroup (before any return).
  if (p.dv_sum && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = tid; i < D; i += 256) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < kDvCopies; ++k) t += p.dv_copies[k * D + i];
      p.dv_sum[i] = t;
    }
  // Workgroups go round-robin over the XCDs; each XCD takes a contiguous run
  // of the logical order (sequence, query run, key tile), so the workgroups
  // that run together on one XCD stage nearly the same query tiles from its L2.
  const int n_wg = static_cast<int>(gridDim.x * gridDim.y);
  const int wg = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x);
  const int xcd = wg % kXcds, per_xcd = n_wg / kXcds, rem_xcd = n_wg % kXcds;
  const int logical = xcd * per_xcd + min(xcd, rem_xcd) + wg / kXcds;
  const int n_kt = static_cast<int>(gridDim.x) / (p.n_chunks * SPLIT);
  const int bs = logical / static_cast<int>(gridDim.x);
  const int rest_h = logical - bs * static_cast<int>(gridDim.x);
  const int half = rest_h % SPLIT;                  // which column half
  const int rest = rest_h / SPLIT;
  const int r_base = half * (RP / SPLIT), d_base = half * (D / SPLIT);
  const int chunk = rest / n_kt;
  const int kt = rest - chunk * n_kt;
  const int b = bs / p.S, s = bs - b * p.S;
  const int k0 = kt * kKTile;
  const int n_qt = (p.T + kQTile - 1) / kQTile;
  const int qt_begin = (p.causal ? k0 / kQTile : 0) + chunk * p.qchunk;
  if (qt_begin >= n_qt) return;   // whole workgroup, before any barrier
  const int qt_end = min(n_qt, qt_begin + p.qchunk);
  const float gamma = bwd_gamma(p, s);
  const float sc = gamma * kLog2e;
  const int64_t tiles = p.Tp / kQTile;
  const int64_t qrows0 = q_rows0(p, bs), krows0 = k_rows0(p, bs);
  const TQ* qb = static_cast<const TQ*>(p.q) + qrows0;
  const TQ* kbase = static_cast<const TQ*>(p.k) + krows0;
  const TQ* qtb = static_cast<const TQ*>(p.qt) + bs * tiles * RP * kQTile;
  const TQ* ktb = static_cast<const TQ*>(p.kt) + bs * static_cast<int64_t>(p.Tkp / kQTile) * RP * kQTile;
  const TV* vb = static_cast<const TV*>(p.v) + static_cast<int64_t>(b) * p.v_sb;
  const TV* dob = static_cast<const TV*>(p.dout) + static_cast<int64_t>(bs) * p.T * D;
  const TV* dotb = static_cast<const TV*>(p.doutt) + bs * tiles * D * kQTile;

  // Resident per wave: its 16 keys as B operands of S (K rows) and dP
  // (V rows), and K^T of all 64 keys for its dQ columns.
  const int kw = k0 + wave * 16;
  const int krow = min(kw + c, p.Tk - 1);
  q8 kf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) kf[kk] = load8(kbase + static_cast<int64_t>(krow) * p.k_st + kk * 32 + 8 * g);
  v8 vf[DC];
#pragma unroll
  for (int j = 0; j < DC; ++j) vf[j] = load8(vb + static_cast<int64_t>(krow) * D + j * 32 + 8 * g);
  q8 ktf[RB][2];
#pragma unroll
  for (int j = 0; j < RB; ++j)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      ktf[j][ks] = load8(ktb + ((k0 / kQTile + ks) * RP + r_base + (wave + 4 * j) * 16 + c) * static_cast<int64_t>(kQTile) + 8 * g);

  f32x4 dv_acc[NV], dk_acc[NK];
#pragma unroll
  for (int j = 0; j < NV; ++j) dv_acc[j] = zero4();
#pragma unroll
  for (int j = 0; j < NK; ++j) dk_acc[j] = zero4();
  float dgamma = 0.f;
  const float* rowv = reinterpret_cast<const float*>(lds + OFF_ROW);
  const int key = kw + c;

  // Step qt's tiles: the row statistics into a register (every thread loads
  // one, at a clamped index), then the tile DMAs, wave w taking wave loads
  // w, w+4, ...  The register load is older than the DMAs, so its use after
  // the step's vmcnt(0) wait needs nothing more.
  float row_stat = 0.f;
  auto issue = [&](int qt) {
    const int q0 = qt * kQTile;
    const float* src = (tid & 63) < kQTile ? p.lse2 : p.dvec;
    row_stat = src[static_cast<int64_t>(bs) * p.T + min(q0 + (tid & (kQTile - 1)), p.T - 1)];
    for (int L = wave; L < QRows::LOADS; L += 4) {
      int r, ck;
      QRows::slot_chunk(L * 64 + lane, r, ck);
      dma16(qb + static_cast<int64_t>(min(q0 + r, p.T - 1)) * p.q_st + ck * 8, lds + OFF_Q + L * 1024);
    }
    for (int L = wave; L < QCols::LOADS; L += 4) {
      int r, ck;
      QCols::slot_chunk(L * 64 + lane, r, ck);
      dma16(qtb + (static_cast<int64_t>(qt) * RP + r_base + r) * kQTile + ck * 8, lds + OFF_QT + L * 1024);
    }
    for (int L = wave; L < DRows::LOADS; L += 4) {
      int r, ck;
      DRows::slot_chunk(L * 64 + lane, r, ck);
      dma16(dob + static_cast<int64_t>(min(q0 + r, p.T - 1)) * D + ck * 8, lds + OFF_DO + L * 1024);
    }
    for (int L = wave; L < DCols::LOADS; L += 4) {
      int r, ck;
      DCols::slot_chunk(L * 64 + lane, r, ck);
      dma16(dotb + (static_cast<int64_t>(qt) * D + d_base + r) * kQTile + ck * 8, lds + OFF_DOT + L * 1024);
    }
  };
  issue(qt_begin);

  for (int qt = qt_begin; qt < qt_end; ++qt) {
    const int q0 = qt * kQTile;
    wait_vmem();   // this step's DMAs (and the previous step's atomics)
    if (tid < 2 * kQTile)
      reinterpret_cast<float*>(lds + OFF_ROW)[tid] = q0 + (tid & (kQTile - 1)) < p.T ? row_stat : 0.f;
    __syncthreads();

    // S = Q K^T and dP = dO V^T for this wave's keys: lane (c, g) element i
    // of block cb is query q0 + 16cb + 4g + i, key kw + c.
    f32x4 sv[2] = {zero4(), zero4()}, dp[2] = {zero4(), zero4()};
    // Groups of four contraction steps: the eight A reads of both query
    // blocks, then their eight MFMAs alternating between the two blocks.
    constexpr int GS = KS < 4 ? KS : 4;
#pragma unroll
    for (int k0 = 0; k0 < KS; k0 += GS) {
      q8 a[GS][2];
#pragma unroll
      for (int kk = 0; kk < GS; ++kk)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          a[kk][cb] = *reinterpret_cast<const q8*>(lds + OFF_Q + (cb * 16 + c) * QP + ((k0 + kk) * 32 + 8 * g) * 2);
#pragma unroll
      for (int kk = 0; kk < GS; ++kk)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) sv[cb] = Elem<TQ>::mma(a[kk][cb], kf[k0 + kk], sv[cb]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * GS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * GS, 0);
    }
    constexpr int GD = DC < 4 ? DC : 4;
#pragma unroll
    for (int j0 = 0; j0 < DC; j0 += GD) {
      v8 a[GD][2];
#pragma unroll
      for (int j = 0; j < GD; ++j)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          a[j][cb] = *reinterpret_cast<const v8*>(lds + OFF_DO + (cb * 16 + c) * VP + ((j0 + j) * 32 + 8 * g) * 2);
#pragma unroll
      for (int j = 0; j < GD; ++j)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) dp[cb] = Elem<TV>::mma(a[j][cb], vf[j0 + j], dp[cb]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * GD, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * GD, 0);
    }
    // P, dS = P (dP - rowsum(dO . O)); contraction element 4cb + i.
    v8 pa;
    q8 dsa;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ql = cb * 16 + 4 * g + i;
        const int q = q0 + ql;
        const bool live = q < p.T && key < p.Tk && (!p.causal || key <= q);
        const float pr = live ? exp2f(sv[cb][i] * sc - rowv[ql]) : 0.f;
        const float ds = pr * (dp[cb][i] - rowv[kQTile + ql]);
        dgamma += ds * sv[cb][i];
        pa[cb * 4 + i] = static_cast<TV>(pr);
        dsa[cb * 4 + i] = static_cast<TQ>(ds);
        // gamma dS for ds_out, rounded once (the LDS tile is free: every
        // wave passed this step's first barrier after reading it last).
        if (p.ds_out)
          *reinterpret_cast<TQ*>(lds + OFF_DS + ql * kDsPitch + (wave * 16 + c) * 2) = static_cast<TQ>(ds * gamma);
      }
    // dV += P^T dO and dK += dS^T Q; B rows read the same query order.  The
    // B operands go in groups of eight: eight LDS reads, then eight MFMAs,
    // so the reads of a group overlap instead of each waiting in turn.
#pragma unroll
    for (int j0 = 0; j0 < NV; j0 += GV) {
      v8 bf[GV];
#pragma unroll
      for (int j = 0; j < GV; ++j) {
        const char* row = lds + OFF_DOT + ((j0 + j) * 16 + c) * kTPitch;
        const v4 lo = *reinterpret_cast<const v4*>(row + 8 * g);
        const v4 hi = *reinterpret_cast<const v4*>(row + 32 + 8 * g);
        bf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int j = 0; j < GV; ++j) dv_acc[j0 + j] = Elem<TV>::mma(pa, bf[j], dv_acc[j0 + j]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * GV, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, GV, 0);
    }
#pragma unroll
    for (int j0 = 0; j0 < NK; j0 += GK) {
      q8 bf[GK];
#pragma unroll
      for (int j = 0; j < GK; ++j) {
        const char* row = lds + OFF_QT + ((j0 + j) * 16 + c) * kTPitch;
        const q4 lo = *reinterpret_cast<const q4*>(row + 8 * g);
        const q4 hi = *reinterpret_cast<const q4*>(row + 32 + 8 * g);
        bf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int j = 0; j < GK; ++j) dk_acc[j0 + j] = Elem<TQ>::mma(dsa, bf[j], dk_acc[j0 + j]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * GK, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, GK, 0);
    }
    // dS with the query as the row, for dQ (ds_out: written above).
    if (!p.ds_out) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<TQ*>(lds + OFF_DS + ((e >> 2) * 16 + 4 * g + (e & 3)) * kDsPitch + (wave * 16 + c) * 2) = dsa[e];
    }
    __syncthreads();   // dS of all four waves is in LDS; the staged tiles are free
    if (qt + 1 < qt_end) issue(qt + 1);
    if (p.ds_out) {
      // 32 query rows x 64 keys: one 16-byte chunk per thread, eight per row.
      const int row = tid >> 3, ch = tid & 7;
      if (q0 + row < p.T)
        store16B(static_cast<TQ*>(p.ds_out) + (static_cast<int64_t>(bs) * p.T + q0 + row) * p.ds_ld + k0 + ch * 8,
                 *reinterpret_cast<const u32x4*>(lds + OFF_DS + row * kDsPitch + ch * 16));
      continue;
    }

    // dQ = dS K over the 64 keys, this wave's 16-column blocks.
    q8 dsf[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        dsf[cb][ks] = *reinterpret_cast<const q8*>(lds + OFF_DS + (cb * 16 + c) * kDsPitch + (ks * 32 + 8 * g) * 2);
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int r = r_base + (wave + 4 * j) * 16 + c;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) acc = Elem<TQ>::mma(dsf[cb][ks], ktf[j][ks], acc);
        // Lane (c, g) element i: query q0 + 16cb + 4g + i, feature r.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = q0 + cb * 16 + 4 * g + i;
          if (q < p.T) unsafeAtomicAdd(p.dq + qrows0 + q * p.q_st + r, acc[i] * gamma);
        }
      }
    }
  }

  // dK and dV rows of this wave's keys: lane (c, g) element i is key
  // kw + 4g + i, column 16j + c.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kr = kw + 4 * g + i;
    if (kr >= p.Tk) continue;
#pragma unroll
    for (int j = 0; j < NK; ++j)
      unsafeAtomicAdd(p.dk + krows0 + kr * p.k_st + r_base + j * 16 + c, dk_acc[j][i] * gamma);
#pragma unroll
    for (int j = 0; j < NV; ++j)
      unsafeAtomicAdd(p.dv + (static_cast<int64_t>(b) * p.Tk + kr) * D + d_base + j * 16 + c, dv_acc[j][i]);
  }
  dgamma = wave_sum(dgamma);
  if (lane == 0 && half == 0) unsafeAtomicAdd(p.dgamma + s, dgamma * bwd_dscale_factor(p, s));
}

namespace {

// Query tiles per main-kernel workgroup: the longest run (at most 16 tiles
// for causal attention, 32 without a mask) that still gives at least 256
// non-empty workgroups without a mask, 128 with one.  Every workgroup ends
// with 64 x (RP + D) atomic adds of its dK and dV rows, so shorter runs than
// that cost more in atomics than they gain in balance.  Measured: the route
// backward at 16384 rows x 1024 atoms 333 us with runs of at most 16 tiles,
// 304 us with 32, and 32768 rows x 128-wide rows 307 / 288 (64-tile runs
// leave 32768 rows on 256 workgroups: 347 us); the causal C2 outer attention
// 0.403 / 0.416 ms with runs of 16 / 32.  For causal key ranges the 256
// workgroups left C1 (8 x 512 tokens) with runs of two query tiles: 122 us,
// against 95 us with the 160 workgroups of four-tile runs (C4 92 / 74 us;
// 96 workgroups at C1: 149 us); without a mask 128 workgroups were slower
// at 8192 rows x 512 atoms (182 / 171 us).
int pick_qchunk(int B_S, int T, int Tk, bool causal) {
  const int n_qt = (T + kQTile - 1) / kQTile;
  const int n_kt = (Tk + kKTile - 1) / kKTile;
  const int64_t min_wgs = causal ? 128 : 256;
  for (int qc = causal ? 16 : 32; qc > 1; qc /= 2) {
    int64_t wgs = 0;
    for (int kt = 0; kt < n_kt; ++kt) {
      const int steps = causal ? n_qt - kt * (kKTile / kQTile) : n_qt;
      wgs += (steps + qc - 1) / qc;
    }
    if (wgs * B_S >= min_wgs) return qc;
  }
  return 1;
}

}  // namespace

template <typename TQ, typename TV, int RP, int D>
static void launch_bwd_d(BwdParams p, int B, hipStream_t stream) {
  const unsigned bs = static_cast<unsigned>(B * p.S);
  hipLaunchKernelGGL((attention_bwd_prep_kernel<TQ, TV, RP, D>),
                     dim3(static_cast<unsigned>(max(p.Tp, p.Tkp) / kQTile), bs, 2), dim3(256), 0, stream, p);
  const int n_qt = (p.T + kQTile - 1) / kQTile;
  hipLaunchKernelGGL((attention_lse_kernel<TQ, RP>), dim3(static_cast<unsigned>(n_qt), bs), dim3(256), 0, stream, p);
  p.qchunk = pick_qchunk(B * p.S, p.T, p.Tk, p.causal != 0);
  p.n_chunks = (n_qt + p.qchunk - 1) / p.qchunk;
  const int n_kt = (p.Tk + kKTile - 1) / kKTile;
  // 512-wide scores split their columns over two workgroups (the
  // accumulators and resident K fragments would not fit one wave otherwise).
  constexpr int SPLIT = RP == 512 ? 2 : 1;
  hipLaunchKernelGGL((attention_bwd_kernel<TQ, TV, RP, D, SPLIT>),
                     dim3(static_cast<unsigned>(n_kt * p.n_chunks * SPLIT), bs), dim3(256), 0, stream, p);
}

template <typename TQ, typename TV, int RP>
static void launch_bwd_r(const BwdParams& p, int B, hipStream_t stream) {
  switch (p.D) {
    case 64: launch_bwd_d<TQ, TV, RP, 64>(p, B, stream); break;
    case 128: launch_bwd_d<TQ, TV, RP, 128>(p, B, stream); break;
    case 256: launch_bwd_d<TQ, TV, RP, 256>(p, B, stream); break;
    default: launch_bwd_d<TQ, TV, RP, 512>(p, B, stream); break;
  }
}

template <typename TQ, typename TV>
static void launch_bwd_t(const BwdParams& p, int B, hipStream_t stream) {
  switch (p.RP) {
    case 64: launch_bwd_r<TQ, TV, 64>(p, B, stream); break;
    case 128: launch_bwd_r<TQ, TV, 128>(p, B, stream); break;
    case 256: launch_bwd_r<TQ, TV, 256>(p, B, stream); break;
    default: launch_bwd_r<TQ, TV, 512>(p, B, stream); break;
  }
}

AttentionBwdLayout attention_bwd_layout(int64_t B, int64_t S, int64_t T, int64_t Tk, int64_t RP, int64_t D) {
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  const int64_t BS = B * S, Tp = round_up(T, kKeyPad), Tkp = round_up(Tk, kKeyPad);
  AttentionBwdLayout l;
  l.qt = 0;
  l.kt = l.qt + up(BS * Tp * RP * 2);
  l.doutt = l.kt + up(BS * Tkp * RP * 2);
  l.lse2 = l.doutt + up(BS * Tp * D * 2);
  l.dvec = l.lse2 + up(BS * T * 4);
  l.vrows = l.dvec + up(BS * T * 4);
  l.dv_copies = l.vrows + up(B * Tkp * D * 2);
  l.bytes = l.dv_copies + up(kDvCopies * D * 4);
  return l;
}

void launch_routed_attention_backward(const AttentionBwdArgs& a, void* workspace, hipStream_t stream) {
  const AttentionBwdLayout l = attention_bwd_layout(a.B, a.S, a.T, a.Tk, a.RP, a.D);
  char* ws = static_cast<char*>(workspace);
  const int64_t Tkp = round_up(a.Tk, kKeyPad);
  BwdParams p{a.q, a.k, a.vt ? static_cast<const void*>(ws + l.vrows) : a.v, a.out, a.dout, ws + l.qt, ws + l.kt, ws + l.doutt,
              reinterpret_cast<float*>(ws + l.lse2), reinterpret_cast<float*>(ws + l.dvec), a.scales,
              a.dq, a.dk, a.dv, a.dv_sum, reinterpret_cast<float*>(ws + l.dv_copies), a.ds_out, a.ds_ld, a.v_dtype, a.dgamma,
              a.q_stride_b, a.q_stride_t, a.q_map_stride, a.k_stride_b, a.k_stride_t, a.k_map_stride,
              a.map_repeat, a.vt ? Tkp * a.D : static_cast<int64_t>(a.Tk) * a.D, a.vt, a.vt_stride_b, a.vt_dtype,
              ws + l.vrows, a.scales_dtype, a.scales_log ? 1 : 0, a.log_lo, a.log_hi, a.scale_mult,
              a.S, a.T, static_cast<int>(round_up(a.T, kKeyPad)), a.RP, a.D,
              a.Tk, static_cast<int>(Tkp), a.causal ? 1 : 0, a.out_dtype, 1, 1};
  if (a.qk_dtype == kF16) {
    if (a.v_dtype == kBF16) launch_bwd_t<_Float16, __bf16>(p, a.B, stream);
    else launch_bwd_t<_Float16, _Float16>(p, a.B, stream);
  } else {
    launch_bwd_t<__bf16, __bf16>(p, a.B, stream);
  }
}

}  // namespace da
