// Host-side launch interfaces between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace da {

constexpr int kAtomPad = 64;   // dictionary atoms are padded to a multiple of this
constexpr int kKeyPad = 64;    // V^T rows are padded to a multiple of this many tokens

// Clamp bounds of the reference's temperatures (modules.py:130-132, ops.py:160-161).
constexpr float kLogBetaMin = -2.995732273553991f;   // ln 0.05
constexpr float kLogBetaMax = 4.1588830833596715f;   // ln 64
constexpr float kLogScaleMin = -1.3862943611198906f; // ln 0.25
constexpr float kLogScaleMax = 6.931471805599453f;   // ln 1024

// Route flags (mirrored in include/double_attention_hip.h).
enum : int {
  kRouteNormalizeInput = 1,
  kRouteNormalizeOutput = 2,
  kRouteBetaIsLog = 4,
  kRouteUnitKeys = 8,
  kRouteSiluLogits = 16,    // logits -> 2 SiLU(logits)                        (ops.py:41-44)
  kRouteStandardize = 32,   // logits -> (logits - mean) / std * logit_scale   (ops.py:47-55)
  kRouteDirectSilu = 64,    // weights = (2/g) SiLU(g logits), no softmax      (ops.py:58-59)
  kRouteBetaIsLogScale = 128,   // row backward only: beta holds log gamma, the
                                // outer attention's temperature (clamp window
                                // kLogScaleMin .. kLogScaleMax)
};

// Attention flags.
enum : int {
  kAttnCausal = 1,
  kAttnScalesAreLog = 2,
  kAttnMix = 4,   // weighted sum over maps into one output; else one output per map
  kAttnOutF32 = 8,   // outputs in fp32 (else in the value dtype)
};

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

struct RouteArgs {
  const void* x;
  int64_t rows;
  int64_t x_stride;
  int x_dtype;
  int R;
  const void* key_t;
  int key_dtype;
  const void* value;    // fp16
  int M;
  const void* beta_ptr;
  int beta_dtype;
  float beta_value;
  float eps;
  int flags;
  float silu_gain;      // g of kRouteDirectSilu
  float logit_scale;    // scale of kRouteStandardize
  void* out;
  int64_t out_stride;
  int out_dtype;
};

struct AttentionArgs {
  const void* q;
  const void* k;
  int64_t qk_stride_b, qk_stride_t;   // element strides of a routed row
  int64_t map_stride;                 // elements between the first branches of consecutive maps
  int map_repeat;                     // maps sharing one branch (S > H repeat)
  int RP;                             // score width R' of one map
  const void* vt;                     // V^T in 32-token tiles: (b, d, t) at b*vt_stride_b + (t/32)*32*D + 32*d + t%32
  int64_t vt_stride_b;
  int B, S, T, D;
  const void* scales;
  int scales_dtype;
  float scale_mult;                   // extra factor on every score scale (RMS-sum groups)
  const void* mix_logits;             // [S] map-mix logits or nullptr (uniform)
  int mix_dtype;
  int flags;
  float score_bound;                  // > 0: |q . k| <= score_bound for every raw score (e.g. unit rows)
  int qk_dtype;                       // routed queries/keys
  int v_dtype;                        // V, probabilities and the output
  void* out;
  int64_t out_stride_b, out_stride_t, out_stride_s;
};

// Backward of the outer attention, per score map (see attention_bwd.hip).
struct AttentionBwdArgs {
  // Query row t of (sequence b, map s) at q + b*q_stride_b +
  // (s / map_repeat)*q_map_stride + t*q_stride_t (elements, qk_dtype), key
  // rows alike; dq and dk (fp32) use the same strides.
  const void* q;
  const void* k;
  int64_t q_stride_b, q_stride_t, q_map_stride;
  int64_t k_stride_b, k_stride_t, k_map_stride;
  int map_repeat;
  const void* v;         // [B][Tk][D] values, v_dtype; or, with vt set, the V^T tiles
  const void* vt;        // [B] x vt_stride_b: [Tkp/32][D][32], 16-bit of vt_dtype
  int64_t vt_stride_b;
  int vt_dtype;
  const void* out;       // [B*S][T][D] forward output, out_dtype
  const void* dout;      // [B*S][T][D] output gradient, v_dtype
  const void* scales;    // [S] score scales, scales_dtype
  int scales_dtype;
  bool scales_log;       // scales hold logs: gamma = exp(clamp(., log_lo, log_hi))
  float log_lo, log_hi;
  float scale_mult;      // every gamma times this
  float* dq;
  float* dk;
  float* dv;             // [B][Tk][D]
  float* dv_sum;         // [D] column sums of dv, or nullptr
  void* ds_out;          // gamma dS rows [B*S*T][ds_ld] (qk_dtype) instead of dq, or nullptr
  int64_t ds_ld;
  float* dgamma;         // [S] gradient at scales[s] (at the log with scales_log)
  int B, S, T, RP, D;
  int Tk;                // keys per sequence (== T when causal)
  bool causal;
  int out_dtype;         // kF32, kF16 or kBF16
  int qk_dtype, v_dtype;
};
// Byte offsets of the backward's workspace pieces (256-byte aligned).
struct AttentionBwdLayout {
  int64_t qt, kt, doutt, lse2, dvec, vrows, dv_copies, bytes;
};
// Copies of the value bias's gradient the LSE pass's workgroups spread
// their atomic adds over.
constexpr int kDvCopies = 8;
AttentionBwdLayout attention_bwd_layout(int64_t B, int64_t S, int64_t T, int64_t Tk, int64_t RP, int64_t D);
void launch_routed_attention_backward(const AttentionBwdArgs& a, void* workspace, hipStream_t stream);

struct GemmSegment {
  // D[i, j] = sum_k P[i, k] Q[j, k]; P rows may come from two stacked matrices
  // (rows [0, split) from p0, rows [split, I) from p1).
  const void* p0;
  const void* p1;
  int64_t p_split;
  const void* q;
  int64_t I, J, K;
  const void* bias;       // nullptr or [I] (mode rows) / [J] (mode vt)
  int bias_dtype;
  int mode;               // 0: out[j, i] (row-major by j), 1: V^T layout
  void* out;
  int64_t ldo;            // mode 0: row pitch of out (elements)
  // mode 1: I counts the B*T real tokens; token t of sequence b, feature j
  // goes to out[b*vt_stride_b + (t/32)*32*J + 32*j + t%32] (32-token tiles),
  // and tokens T..Tp-1 are filled too.
  int64_t T, Tp, vt_stride_b;
  // mode 0 only: kGemmActGelu applies GELU (erf form) after the bias, and a
  // non-null residual (same layout as out) is added to the rounded result.
  int act;
  const void* residual;
};

enum : int { kGemmActNone = 0, kGemmActGelu = 1 };

void launch_dictionary_normalize(const void* raw_key, const void* raw_value, int in_dtype, int R,
                                 int M, float eps, void* key_t, int key_dtype, void* value,
                                 void* value_rows, hipStream_t stream);
void launch_dictionary_route(const RouteArgs& a, hipStream_t stream);
// Backward of the column normalization (dict_norm.hip).  Banks [R, M]
// row-major of one dtype; gradients fp32 [R, M]; raw_value NULL = tied bank
// (the key gradient plus grad_value, when given, flows into d_key).
struct NormBwdArgs {
  const void* raw_key; const void* raw_value; int dtype;
  int R; int64_t M; float eps;
  const float* grad_key; const float* grad_value;
  int64_t g_ld_r, g_ld_j;   // gradient element (r, j) at r * g_ld_r + j * g_ld_j
  void* d_key; void* d_value;
};
void launch_dictionary_normalize_backward(const NormBwdArgs& a, hipStream_t stream);

// Row L2 normalization and its backward (row_norm.hip).  R % 4 == 0; row
// pitches multiples of 4 elements; x, grad and out aligned to 4 elements.
// Arithmetic in fp32 whatever the element types.
// Row-normalize backward output: a 16-bit dtype or'd with kOutSplit writes
// the rounded gradient and its rounding residual side by side.
constexpr int kOutSplit = 0x100;
struct RowNormArgs {
  const void* x; int x_dtype; int64_t ld_x;
  int64_t rows; int R; float eps;
  const void* grad; int grad_dtype; int64_t ld_grad;   // backward only: dL/dy
  void* out; int out_dtype; int64_t ld_out;
};
void launch_row_normalize(const RowNormArgs& a, bool backward, hipStream_t stream);

// Row-wise backward of the route's assignment (route_bwd.hip).
struct RouteBwdRowsArgs {
  const float* logits;        // [rows, ld_in] raw logits <u, Dk_j>
  const float* grad_weights;  // [rows, ld_in] <dr, Dv_j>
  int64_t rows;
  int atoms;                  // M <= kRouteBwdRowsMaxAtoms
  int64_t causal_period;      // 0, or row r keeps columns j <= r % causal_period
  int64_t ld_in;
  const void* beta_ptr;
  int beta_dtype;
  float beta_value;
  int beta_count;             // entries of beta_ptr: row r takes (r / beta_period) % beta_count
  int64_t beta_period;
  int flags;                  // kRouteBetaIsLog and the variant bits
  float silu_gain, logit_scale, eps;
  void* grad_logits;          // [rows, ld_out] out_dtype
  void* weights;              // [rows, ld_out] out_dtype
  int64_t ld_out;
  int out_dtype;
  float* dbeta_rows;          // [rows] or nullptr
};
// Rows of up to 16384 columns are held in registers (one wave up to 4096,
// a workgroup's four waves above); longer rows take a multi-pass kernel.
constexpr int kRouteBwdRowsMaxAtoms = 1 << 24;
void launch_route_backward_rows(const RouteBwdRowsArgs& a, hipStream_t stream);

// Map combine of the training path (map_combine.hip): out = sum_s w_s O_s
// over per-map fp32 outputs O [B, S, T, D]; backward grad_maps = w_s dY (dtype)
// and weight_sums[s] += <O_s, dY> (fp32 atomics; zeroed by the caller).
struct MapCombineArgs {
  const float* maps;      // [B, S, T, D] fp32
  const float* weights;   // [S] fp32
  int64_t rows;           // B * T
  int64_t T;
  int S, D;               // S <= 8, D a multiple of 8
  int dtype;              // kF16 or kBF16: out, or grad and grad_maps
  void* out;              // [B, T, D] (forward)
  const void* grad;       // [B, T, D] (backward)
  void* grad_maps;        // [B, S, T, D] (backward)
  float* weight_sums;     // [S] (backward)
};
constexpr int kMapCombineMaxMaps = 8;
void launch_map_combine(const MapCombineArgs& a, bool backward, hipStream_t stream);
// out[i] = sum_c partials[c * n + i] rounded once to out_dtype (kF16 / kBF16); n % 8 == 0.
void launch_sum_partials(const float* partials, int count, int64_t n, void* out, int out_dtype, hipStream_t stream);

// Operands of the dense attention backward (dense_operands.hip): from the
// score maps (row (b, s, t) at q/k + b*stride_b + (s/map_repeat)*map_stride +
// t*stride_t, R elements) K^T [B*S, R, T] in qk_dtype and q, k [B*S, T, R] in
// out_dtype.  R a multiple of 64.
struct DenseOperandArgs {
  const void* q;
  const void* k;
  int64_t stride_b, stride_t, map_stride;
  int map_repeat;
  int qk_dtype;
  int B, S, T, R;
  void* key_t;
  void* q_out;
  void* k_out;
  int out_dtype;
};
void launch_dense_operands(const DenseOperandArgs& a, hipStream_t stream);

// LayerNorm over the last dimension (dim a multiple of 8, at most 4096).
void launch_layer_norm(const void* x, int64_t rows, int dim, const void* weight, const void* bias, int param_dtype,
                       float eps, int dtype, void* out, hipStream_t stream);
// Its backward: dx (dtype) and the fp32 parameter gradients added into
// dparams [kLnParamCopies][2 * dim] (weight then bias; zeroed by the caller,
// the gradients are the sums over the copies).
constexpr int kLnParamCopies = 8;
void launch_layer_norm_backward(const void* x, const void* dy, int64_t rows, int dim, const void* weight,
                                int param_dtype, float eps, int dtype, void* dx, float* dparams, hipStream_t stream);
// Launch shape of the attention for a problem: value slice width, waves per
// query tile, sub-streams, query tiles, the stream split of long key ranges (run length, 0
// = none; runs per sequence and slice) and the bytes of partials it needs
// with piece outputs of piece_bytes (2: 16-bit, 4: fp32 for fp32 outputs).
struct AttnPlan {
  int ds;
  int nw;
  int sub;          // sub-streams per workgroup (1 or 2)
  int n_qt;
  int stream_len;
  int n_seg;
  int64_t part_bytes;
};
AttnPlan plan_attention(int64_t B, int64_t S, int64_t T, int64_t D, int64_t RP, bool multi, bool causal,
                        bool allow_split, int piece_bytes);
// `partials`: plan.part_bytes of device scratch (plan with allow_split), or
// nullptr to run without key-range splitting.
void launch_routed_attention(const AttentionArgs& a, void* partials, hipStream_t stream);
struct NormJob;
// `norm`: a dictionary normalization run by extra workgroups of the same
// launch, or nullptr.
void launch_gemm(const GemmSegment* segs, int nseg, int dtype, hipStream_t stream, const NormJob* norm = nullptr);

}  // namespace da
