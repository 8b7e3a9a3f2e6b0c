// Row-wise backward of the dictionary route's assignment, for every variant.
//
// Replaces the reference's _row_scaled_softmax_backward_kernel
// (src/double_attention/triton_kernels.py:589-671, launched at :1480) and the
// direct-SiLU branch of _DictionaryRouteFunction.backward (:1940-1948): the
// step between the two GEMM pairs of the route backward.  Per row, from the
// raw logits l_j = <u, Dk_j> and dW_j = <dr, Dv_j> (fp32, written by GEMMs),
// it forms the forward weights of ops.py:41-61 again and returns the gradient
// at the raw logits, the weights (for dDv = dr^T W) and the row's share of
// d beta:
//   a0 = l                   or 2 SiLU(l)                    (activation)
//   a  = a0                  or s (a0 - mean a0) / sqrt(var a0 + eps)   (standardize)
//   w  = softmax_j(beta a)   or (2/g) SiLU(g a)              (assignment)
//   softmax: d(beta a_j) = w_j (dW_j - sum_k w_k dW_k); da = beta d(beta a);
//            d beta = sum_j d(beta a_j) a_j
//   direct:  da_j = dW_j 2 SiLU'(g a_j)
//   standardize: with c = (a0 - mean) isd, dc = s da:
//            da0 = isd (dc - mean dc - c mean(dc c))
//   SiLU activation: dl = da0 2 SiLU'(l),  SiLU'(x) = sig(x) (1 + x (1 - sig(x)))
// One wave per row, the row's atoms strided over the lanes and held in VGPRs
// (NPL per lane, M <= 64 NPL <= 4096), so every reduction is a wave reduction
// and the two inputs are read once, coalesced; rows of up to 16384 atoms are
// shared by a workgroup's four waves (their sums meet in LDS), and longer rows
// take the multi-pass kernel below.  The outer attention's backward uses
// the same kernel for its softmax (scores as logits, dP as dW, gamma as beta,
// a causal row length).
#include "da_common.h"
#include "da_launch.h"
#include "da_tile.h"

namespace da {

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + __expf(-x)); }

// The scale of the assignment from the beta argument: beta itself, or
// exp(clamp(.)) of a log with kRouteBetaIsLog (log beta, window ln .05 ..
// ln 64) or kRouteBetaIsLogScale (log gamma, window ln .25 .. ln 1024).
__device__ __forceinline__ bool beta_log_window(int flags, float& lo, float& hi) {
  if (flags & kRouteBetaIsLog) {
    lo = kLogBetaMin;
    hi = kLogBetaMax;
    return true;
  }
  if (flags & kRouteBetaIsLogScale) {
    lo = kLogScaleMin;
    hi = kLogScaleMax;
    return true;
  }
  return false;
}
__device__ __forceinline__ float beta_from(int flags, float beta_raw) {
  float lo, hi;
  return beta_log_window(flags, lo, hi) ? expf(fminf(fmaxf(beta_raw, lo), hi)) : beta_raw;
}
// With a log argument the row's d beta term is written at the log: times
// beta where the clamp passes the gradient, zero outside its window.
__device__ __forceinline__ float dbeta_at(int flags, float dbeta, float beta_raw, float beta) {
  float lo, hi;
  if (!beta_log_window(flags, lo, hi)) return dbeta;
  return beta_raw >= lo && beta_raw <= hi ? dbeta * beta : 0.f;
}

// WPR waves per row: with WPR = 1 a workgroup's four waves take four rows;
// with WPR = 4 its waves share one row (column j at wave j / 64 % 4), and the
// row sums meet in LDS.
template <typename TO, int NPL, int WPR>
__global__ __launch_bounds__(256) void route_backward_rows_kernel(RouteBwdRowsArgs a) {
  static_assert(WPR == 1 || WPR == 4, "one wave per row, or the workgroup's four");
  constexpr int STRIDE = 64 * WPR;   // columns between a lane's consecutive elements
  __shared__ float red[2][WPR];
  const int lane = lane_id();
  const int wave = uniform_wave();
  const int64_t row = WPR == 1 ? static_cast<int64_t>(blockIdx.x) * 4 + wave : static_cast<int64_t>(blockIdx.x);
  if (row >= a.rows) return;   // whole waves (WPR 1), or the whole workgroup
  const int col0 = (WPR == 1 ? 0 : wave * 64) + lane;
  // Sum or maximum over the row: the wave's lanes, then (WPR 4) the four
  // waves through one of two LDS slots in turn, so one barrier per call.
  int slot = 0;
  auto row_reduce = [&](float v, bool is_max) {
    v = is_max ? wave_max64(v) : wave_sum64(v);
    if constexpr (WPR > 1) {
      if (lane == 0) red[slot][wave] = v;
      __syncthreads();
      v = red[slot][0];
#pragma unroll
      for (int i = 1; i < WPR; ++i) v = is_max ? fmaxf(v, red[slot][i]) : v + red[slot][i];
      slot ^= 1;
    }
    return v;
  };
  // With causal_period P, row r (token r % P of its sequence) keeps columns
  // j <= r % P; the others get zero weight and gradient.
  const int M = a.causal_period ? min(a.atoms, static_cast<int>(row % a.causal_period) + 1) : a.atoms;
  const float* lrow = a.logits + row * a.ld_in;
  const float* grow = a.grad_weights + row * a.ld_in;
  const bool silu_logits = a.flags & kRouteSiluLogits;
  const bool standardize = a.flags & kRouteStandardize;
  const bool direct = a.flags & kRouteDirectSilu;

  // beta of this row: one value, or entry (row / beta_period) % beta_count.
  const int64_t beta_index = a.beta_count > 1 ? (row / a.beta_period) % a.beta_count : 0;
  const ScalarHalves beta_bits = fetch_scalar(a.beta_ptr ? a.beta_ptr : static_cast<const void*>(a.logits),
                                              a.beta_ptr ? a.beta_dtype : kF32, a.beta_ptr ? beta_index : 0);
  float l[NPL], g[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = col0 + STRIDE * i;
    l[i] = j < M ? lrow[j] : 0.f;
    g[i] = j < M ? grow[j] : 0.f;
  }
  const float beta_raw = a.beta_ptr ? scalar_value(beta_bits, a.beta_dtype) : a.beta_value;
  const float beta = beta_from(a.flags, beta_raw);
  const float inv_m = 1.f / static_cast<float>(M);

  // Activation, then standardization: c holds the standardized value
  // (before the scale s), a the assignment logits.
  float c[NPL], w[NPL];
  float isd = 1.f;
#pragma unroll
  for (int i = 0; i < NPL; ++i) c[i] = silu_logits ? 2.f * l[i] * sigmoidf(l[i]) : l[i];
  if (standardize) {
    float s1 = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) s1 += col0 + STRIDE * i < M ? c[i] : 0.f;
    const float mean = row_reduce(s1, false) * inv_m;
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      c[i] = col0 + STRIDE * i < M ? c[i] - mean : 0.f;
      s2 += c[i] * c[i];
    }
    isd = rsqrtf(row_reduce(s2, false) * inv_m + a.eps);
#pragma unroll
    for (int i = 0; i < NPL; ++i) c[i] *= isd;
  }
  const float s = standardize ? a.logit_scale : 1.f;

  // Assignment weights and the gradient at the assignment logits (into g).
  float dbeta = 0.f;
  if (direct) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float x = a.silu_gain * (c[i] * s);
      const float sg = sigmoidf(x);
      w[i] = (2.f / a.silu_gain) * x * sg;
      g[i] *= 2.f * sg * (1.f + x * (1.f - sg));
    }
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      if (col0 + STRIDE * i < M) mx = fmaxf(mx, beta * (c[i] * s));
    mx = row_reduce(mx, true);
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      w[i] = col0 + STRIDE * i < M ? __expf(beta * (c[i] * s) - mx) : 0.f;
      z += w[i];
    }
    const float inv_z = 1.f / row_reduce(z, false);
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      w[i] *= inv_z;
      d += w[i] * g[i];
    }
    d = row_reduce(d, false);
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float dsc = w[i] * (g[i] - d);   // gradient at beta a_j
      dbeta += dsc * (c[i] * s);
      g[i] = beta * dsc;
    }
    dbeta = row_reduce(dbeta, false);
  }
  if (standardize) {
    float m1 = 0.f, m2 = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      g[i] *= s;
      m1 += g[i];
      m2 += g[i] * c[i];
    }
    m1 = row_reduce(m1, false) * inv_m;
    m2 = row_reduce(m2, false) * inv_m;
#pragma unroll
    for (int i = 0; i < NPL; ++i) g[i] = isd * (g[i] - m1 - c[i] * m2);
  }
  if (silu_logits) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float sg = sigmoidf(l[i]);
      g[i] *= 2.f * sg * (1.f + l[i] * (1.f - sg));
    }
  }

  TO* dl_row = static_cast<TO*>(a.grad_logits) + row * a.ld_out;
  TO* w_row = static_cast<TO*>(a.weights) + row * a.ld_out;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = col0 + STRIDE * i;
    if (j < a.atoms) {
      dl_row[j] = static_cast<TO>(j < M ? g[i] : 0.f);
      w_row[j] = static_cast<TO>(j < M ? w[i] : 0.f);
    }
  }
  if (a.dbeta_rows && lane == 0 && (WPR == 1 || wave == 0)) a.dbeta_rows[row] = direct ? 0.f : dbeta_at(a.flags, dbeta, beta_raw, beta);
}

// Rows longer than the register-held kernels' 16384 columns: the same algebra
// in passes over the row, each re-reading the fp32 inputs (written just
// before by the GEMMs) 1024 columns at a time and forming the forward values
// again: the standardization's mean, then its variance; the softmax's
// maximum, normalizer and sum_j w_j dW_j in one pass with a running maximum
// per lane; then d beta and the standardization's backward sums; then the
// outputs.  One wave per row, as above.
template <typename TO>
__global__ __launch_bounds__(256) void route_backward_long_rows_kernel(RouteBwdRowsArgs a) {
  constexpr int CH = 16;        // columns per lane in one chunk
  constexpr int CW = 64 * CH;   // columns per chunk
  const int lane = lane_id();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + uniform_wave();
  if (row >= a.rows) return;   // whole waves
  const int M = a.causal_period ? min(a.atoms, static_cast<int>(row % a.causal_period) + 1) : a.atoms;
  const float* lrow = a.logits + row * a.ld_in;
  const float* grow = a.grad_weights + row * a.ld_in;
  const bool silu_logits = a.flags & kRouteSiluLogits;
  const bool standardize = a.flags & kRouteStandardize;
  const bool direct = a.flags & kRouteDirectSilu;
  const int64_t beta_index = a.beta_count > 1 ? (row / a.beta_period) % a.beta_count : 0;
  const ScalarHalves beta_bits = fetch_scalar(a.beta_ptr ? a.beta_ptr : static_cast<const void*>(a.logits),
                                              a.beta_ptr ? a.beta_dtype : kF32, a.beta_ptr ? beta_index : 0);
  const float beta_raw = a.beta_ptr ? scalar_value(beta_bits, a.beta_dtype) : a.beta_value;
  const float beta = beta_from(a.flags, beta_raw);
  const float inv_m = 1.f / static_cast<float>(M);
  auto act = [&](float x) { return silu_logits ? 2.f * x * sigmoidf(x) : x; };

  // Standardization statistics (two passes: the mean, then the spread).
  float mean = 0.f, isd = 1.f;
  if (standardize) {
    float s1 = 0.f;
    for (int j0 = 0; j0 < M; j0 += CW) {
      float v[CH];
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int j = j0 + lane + 64 * i;
        v[i] = j < M ? act(lrow[j]) : 0.f;
      }
#pragma unroll
      for (int i = 0; i < CH; ++i) s1 += v[i];
    }
    mean = wave_sum64(s1) * inv_m;
    float s2 = 0.f;
    for (int j0 = 0; j0 < M; j0 += CW) {
      float v[CH];
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int j = j0 + lane + 64 * i;
        v[i] = j < M ? act(lrow[j]) - mean : 0.f;
      }
#pragma unroll
      for (int i = 0; i < CH; ++i) s2 += v[i] * v[i];
    }
    isd = rsqrtf(wave_sum64(s2) * inv_m + a.eps);
  }
  const float s = standardize ? a.logit_scale : 1.f;
  auto cval = [&](float x) { return standardize ? (act(x) - mean) * isd : act(x); };

  // Softmax statistics: maximum, normalizer and sum_j w_j dW_j (running
  // maximum per lane, merged over the wave at the end).
  float mx = 0.f, inv_z = 0.f, d = 0.f;
  if (!direct) {
    float m_l = -INFINITY, z_l = 0.f, dn_l = 0.f;
    for (int j0 = 0; j0 < M; j0 += CW) {
      float x[CH], gv[CH];
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int j = j0 + lane + 64 * i;
        x[i] = j < M ? beta * (cval(lrow[j]) * s) : -INFINITY;
        gv[i] = j < M ? grow[j] : 0.f;
      }
      float cm = m_l;
#pragma unroll
      for (int i = 0; i < CH; ++i) cm = fmaxf(cm, x[i]);
      if (cm > m_l) {
        const float f = m_l == -INFINITY ? 0.f : __expf(m_l - cm);
        z_l *= f;
        dn_l *= f;
        m_l = cm;
      }
      if (m_l != -INFINITY) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const float e = x[i] == -INFINITY ? 0.f : __expf(x[i] - m_l);
          z_l += e;
          dn_l += e * gv[i];
        }
      }
    }
    mx = wave_max64(m_l);
    const float f = m_l == -INFINITY ? 0.f : __expf(m_l - mx);
    inv_z = 1.f / wave_sum64(z_l * f);
    d = wave_sum64(dn_l * f) * inv_z;
  }

  // Per column: the weight and the gradient at the assignment logits (times
  // s), and the column's d beta term.
  auto column = [&](float lj, float gj, float& wj, float& cj, float& db) {
    cj = cval(lj);
    if (direct) {
      const float x = a.silu_gain * (cj * s);
      const float sg = sigmoidf(x);
      wj = (2.f / a.silu_gain) * x * sg;
      db = 0.f;
      return gj * 2.f * sg * (1.f + x * (1.f - sg)) * s;
    }
    wj = __expf(beta * (cj * s) - mx) * inv_z;
    const float dsc = wj * (gj - d);
    db = dsc * (cj * s);
    return beta * dsc * s;
  };

  // d beta and the standardization's backward sums.
  float dbeta = 0.f, m1 = 0.f, m2 = 0.f;
  if (!direct || standardize) {
    for (int j0 = 0; j0 < M; j0 += CW) {
      float lv[CH], gv[CH];
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int j = j0 + lane + 64 * i;
        lv[i] = j < M ? lrow[j] : 0.f;
        gv[i] = j < M ? grow[j] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        if (j0 + lane + 64 * i < M) {
          float wj, cj, db;
          const float gs = column(lv[i], gv[i], wj, cj, db);
          dbeta += db;
          m1 += gs;
          m2 += gs * cj;
        }
      }
    }
    dbeta = wave_sum64(dbeta);
    m1 = wave_sum64(m1) * inv_m;
    m2 = wave_sum64(m2) * inv_m;
  }

  // Outputs.
  TO* dl_row = static_cast<TO*>(a.grad_logits) + row * a.ld_out;
  TO* w_row = static_cast<TO*>(a.weights) + row * a.ld_out;
  for (int j0 = 0; j0 < a.atoms; j0 += CW) {
    float lv[CH], gv[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int j = j0 + lane + 64 * i;
      lv[i] = j < M ? lrow[j] : 0.f;
      gv[i] = j < M ? grow[j] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int j = j0 + lane + 64 * i;
      if (j < a.atoms) {
        float wj = 0.f, gj = 0.f;
        if (j < M) {
          float cj, db;
          gj = column(lv[i], gv[i], wj, cj, db);
          if (standardize) gj = isd * (gj - m1 - cj * m2);
          if (silu_logits) {
            const float sg = sigmoidf(lv[i]);
            gj *= 2.f * sg * (1.f + lv[i] * (1.f - sg));
          }
        }
        dl_row[j] = static_cast<TO>(gj);
        w_row[j] = static_cast<TO>(wj);
      }
    }
  }
  if (a.dbeta_rows && lane == 0) a.dbeta_rows[row] = direct ? 0.f : dbeta_at(a.flags, dbeta, beta_raw, beta);
}

template <typename TO>
static void launch_route_bwd_rows_t(const RouteBwdRowsArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  // Up to 4096 columns one wave holds a row; up to 16384 the workgroup's four
  // waves share it (32 or 64 columns per lane); longer rows take passes.
  const dim3 per_row(static_cast<unsigned>(a.rows));
  if (a.atoms > 16384) {
    hipLaunchKernelGGL((route_backward_long_rows_kernel<TO>), grid, dim3(256), 0, s, a);
  } else if (a.atoms > 8192) {
    hipLaunchKernelGGL((route_backward_rows_kernel<TO, 64, 4>), per_row, dim3(256), 0, s, a);
  } else if (a.atoms > 4096) {
    hipLaunchKernelGGL((route_backward_rows_kernel<TO, 32, 4>), per_row, dim3(256), 0, s, a);
  } else if (a.atoms <= 512) {
    hipLaunchKernelGGL((route_backward_rows_kernel<TO, 8, 1>), grid, dim3(256), 0, s, a);
  } else if (a.atoms <= 1024) {
    hipLaunchKernelGGL((route_backward_rows_kernel<TO, 16, 1>), grid, dim3(256), 0, s, a);
  } else if (a.atoms <= 2048) {
    hipLaunchKernelGGL((route_backward_rows_kernel<TO, 32, 1>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((route_backward_rows_kernel<TO, 64, 1>), grid, dim3(256), 0, s, a);
  }
}

void launch_route_backward_rows(const RouteBwdRowsArgs& a, hipStream_t stream) {
  if (a.rows == 0) return;
  if (a.out_dtype == kBF16) {
    launch_route_bwd_rows_t<__bf16>(a, stream);
  } else {
    launch_route_bwd_rows_t<_Float16>(a, stream);
  }
}

}  // namespace da
