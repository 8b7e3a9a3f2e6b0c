/*
 * C ABI of the MI355X (gfx950) shared-dictionary attention forward path.
 *
 * Every entry point takes plain device pointers, element counts and strides,
 * a dtype code and the HIP stream to enqueue on.  Nothing here allocates,
 * frees or synchronizes: the caller owns every buffer (including the
 * workspace of da_shared_dictionary_attention_forward) and the stream order.
 * Scalars that the reference keeps as device tensors (beta, the score scales,
 * the map-mix logits) are passed as device pointers and read on the device,
 * so no entry point needs a host round trip.
 *
 * Return value: 0 on success, a negative DA_ERR_* code otherwise; the
 * message of the last failure on the calling thread is da_last_error().
 * Argument checks run before anything is enqueued, so a failed call leaves
 * the stream untouched.
 *
 * Reference interfaces replaced (paths relative to the reference repository
 * Ahnd6474/double-attention):
 *   da_dictionary_normalize   SharedDictionaryBank.normalized        src/double_attention/modules.py:45-48
 *   da_dictionary_normalize_backward
 *                             autograd of SharedDictionaryBank.normalized  src/double_attention/modules.py:45-48
 *   da_row_normalize          F.normalize of the route's rows        src/double_attention/ops.py:39, 62; triton_kernels.py:1286-1308
 *   da_row_normalize_backward _row_l2_normalize_backward             src/double_attention/triton_kernels.py:553-586, 1410-1440
 *   da_dictionary_route       dictionary_route_triton / _reference   src/double_attention/triton_kernels.py:1984-2019, ops.py:16-62
 *   da_dictionary_route_backward_rows
 *                             _row_scaled_softmax_backward_kernel    src/double_attention/triton_kernels.py:589-671, 1480
 *                             + direct-SiLU backward branch          src/double_attention/triton_kernels.py:1940-1948
 *   da_routed_attention       routed_attention_triton / _reference   src/double_attention/triton_kernels.py:2290-2305, ops.py:65-93
 *                             + map combine                          src/double_attention/modules.py:265-272
 *   da_routed_attention_backward, da_routed_attention_backward_ex, da_attention_backward_workspace_bytes
 *                             backward of routed_attention_triton    src/double_attention/triton_kernels.py:2093-2263, 2290-2305
 *                             (_ex: on the score maps as views of the routed rows, with the
 *                             temperature clamp's backward,          src/double_attention/modules.py:242-263, ops.py:160-161)
 *   da_qkv_projection         _project_query_key + self.value        src/double_attention/modules.py:143-157, 212
 *   da_linear                 self.output                            src/double_attention/modules.py:117-121, 272
 *   da_linear_ex              DoubleAttentionBlock.feedforward       src/double_attention/modules.py:318-330, 343-346
 *                             + the block's residual adds
 *   da_layer_norm, da_layer_norm_backward
 *                             attention_norm / feedforward_norm /    src/double_attention/modules.py:311, 313, 440
 *                             final_norm (nn.LayerNorm) and its autograd backward
 *   da_sum_partials           (split-K weight gradients of the training path; no reference counterpart)
 *   da_dense_attention_operands
 *                             operands of the dense attention backward src/double_attention/triton_kernels.py:2093-2263
 *   da_map_combine, da_map_combine_backward
 *                             map_combine "weighted_sum" (einsum      src/double_attention/modules.py:265-272
 *                             over the per-map outputs) and its backward
 *   da_shared_dictionary_attention_forward
 *                             SharedDictionaryAttention.forward      src/double_attention/modules.py:190-291
 */
#ifndef DOUBLE_ATTENTION_HIP_H
#define DOUBLE_ATTENTION_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* da_stream_t; /* hipStream_t; NULL = default stream */

/* dtype codes */
#define DA_F32 0
#define DA_F16 1
#define DA_BF16 2
#define DA_OUT_SPLIT 0x100 /* or'd into a 16-bit out_dtype: see da_row_normalize_backward */

/* error codes */
#define DA_OK 0
#define DA_ERR_INVALID_ARGUMENT (-1)
#define DA_ERR_UNSUPPORTED (-2)
#define DA_ERR_ALIGNMENT (-3)
#define DA_ERR_LAUNCH (-4)
#define DA_ERR_WORKSPACE (-5)

/* da_dictionary_route flags */
#define DA_ROUTE_NORMALIZE_INPUT 1  /* u = x / max(||x||, eps) before the assignment   */
#define DA_ROUTE_NORMALIZE_OUTPUT 2 /* z = r / max(||r||, eps) after the reconstruction */
#define DA_ROUTE_BETA_IS_LOG 4      /* *beta is log_beta: use exp(clamp(., ln .05, ln 64)) */
#define DA_ROUTE_UNIT_KEYS 8        /* key atoms have L2 norm <= 1 (a normalized bank): with
                                       DA_ROUTE_NORMALIZE_INPUT every logit is bounded by |beta|,
                                       which lets the kernel skip online-softmax rescaling */
#define DA_ROUTE_SILU_LOGITS 16     /* logits -> 2 SiLU(logits)           (activation "silu", ops.py:41-44) */
#define DA_ROUTE_STANDARDIZE 32     /* logits -> (logits - mean) / sqrt(var + eps) * logit_scale over the
                                       atoms (standardize_logits, ops.py:47-55): two passes */
#define DA_ROUTE_DIRECT_SILU 64     /* weights = (2/silu_gain) SiLU(silu_gain logits) instead of
                                       softmax(beta logits) (assignment "silu", ops.py:56-59) */
#define DA_ROUTE_BETA_IS_LOG_SCALE 128 /* da_dictionary_route_backward_rows only: *beta holds
                                       log_score_scales, exp(clamp(., ln .25, ln 1024)) (the
                                       outer attention's temperatures, ops.py:160-161) */

/* da_routed_attention flags */
#define DA_ATTN_CAUSAL 1
#define DA_ATTN_SCALES_ARE_LOG 2    /* scales are log_score_scales: exp(clamp(., ln .25, ln 1024)) */
#define DA_ATTN_MIX 4               /* alpha-weighted sum of the maps into one output */
#define DA_ATTN_OUT_F32 8           /* out holds fp32 values (forward: written so; backward: read so) */

/* da_shared_dictionary_attention_forward flags */
#define DA_SDA_NORMALIZE_INPUT 1
#define DA_SDA_NORMALIZE_OUTPUT 2
#define DA_SDA_CAUSAL 4
#define DA_SDA_CONCAT 8             /* map_combine == "concat" */
#define DA_SDA_UNIT_KEYS 16         /* key_t holds atoms of L2 norm <= 1 (da_dictionary_normalize
                                       output): the route may then bound its logits by |beta|
                                       (DA_ROUTE_UNIT_KEYS).  Implied when raw_key is set (the call
                                       normalizes the bank itself); never set it for a bank whose
                                       atoms were not normalized. */

/* ABI version of this header (bumped on any signature or semantics change). */
int da_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* da_last_error(void);

/* Atoms after padding: the route layouts hold round_up(atoms, 64) atoms. */
int64_t da_padded_atoms(int64_t atoms);

/* Tokens after padding: V^T rows hold round_up(length, 64) tokens. */
int64_t da_padded_length(int64_t length);

/*
 * Column-normalize one dictionary bank (modules.py:45-48).
 *   raw_key, raw_value: [routing_dim, atoms] row-major, dtype raw_dtype
 *                       (raw_value NULL = tied bank: key atoms serve both roles)
 *   key_t:  out [da_padded_atoms(atoms), routing_dim]   atom-major, key_dtype
 *   value:  out, fp16, 32-atom tiles: coordinate r of atom j at
 *           value[(j/32)*32*routing_dim + 32*r + j%32]
 *           (da_padded_atoms(atoms) * routing_dim elements)
 *   value_rows: NULL, or out [routing_dim, da_padded_atoms(atoms)] fp16, the
 *           same value atoms coordinate-major (written by the same pass)
 * Atom j becomes raw[:, j] / max(||raw[:, j]||, eps); padding atoms are zero.
 * routing_dim must be 64, 128, 256 or 512; key_dtype DA_F16 or DA_BF16.
 */
int da_dictionary_normalize(const void* raw_key, const void* raw_value, int raw_dtype,
                            int64_t routing_dim, int64_t atoms, float eps, void* key_t,
                            int key_dtype, void* value, void* value_rows, da_stream_t stream);

/*
 * Backward of da_dictionary_normalize (F.normalize(raw, dim=0) under autograd,
 * modules.py:45-48): gradients at the raw bank from gradients at the
 * normalized atoms.
 *   raw_key, raw_value: [routing_dim, atoms] row-major, raw_dtype (raw_value
 *           NULL = tied bank)
 *   grad_key, grad_value: fp32 gradients at the normalized key and value
 *           atoms, coordinate r of atom j at [r * grad_ld_r + j * grad_ld_j]
 *           (grad_ld_r = atoms, grad_ld_j = 1 for [routing_dim, atoms] rows;
 *           grad_ld_r = 1, grad_ld_j = routing_dim for the atom-major
 *           [atoms, routing_dim] gradients of the route backward); grad_value
 *           may be NULL (zero).  For a tied bank both flow into the key atoms.
 *   d_raw_key, d_raw_value: out, [routing_dim, atoms] raw_dtype (d_raw_value
 *           NULL = not wanted; must be NULL for a tied bank)
 * Atom j with raw column v and gradient h gets (h - n <n, h>) / |v| with
 * n = v / |v| where |v| > eps, and h / eps elsewhere.
 */
int da_dictionary_normalize_backward(const void* raw_key, const void* raw_value, int raw_dtype,
                                     int64_t routing_dim, int64_t atoms, float eps, const float* grad_key,
                                     const float* grad_value, int64_t grad_ld_r, int64_t grad_ld_j,
                                     void* d_raw_key, void* d_raw_value, da_stream_t stream);

/*
 * Row L2 normalization, F.normalize(x, dim=-1, eps) (ops.py:39, :62; the
 * reference's Triton _row_l2_normalize, triton_kernels.py:30-45, 1286-1308):
 *   out[i, :] = x[i, :] / max(|x[i, :]|, eps), computed in fp32 and rounded
 *   once to out_dtype.
 *   x: [rows, width] with row pitch ld_x, x_dtype; out: [rows, width], pitch
 *   ld_out, out_dtype.  width, ld_x and ld_out multiples of 4; x and out
 *   aligned to 4 elements.
 */
int da_row_normalize(const void* x, int x_dtype, int64_t rows, int64_t width, int64_t ld_x, float eps, void* out,
                     int out_dtype, int64_t ld_out, da_stream_t stream);

/*
 * Backward of da_row_normalize (autograd of F.normalize; the reference's
 * _row_l2_normalize_backward, triton_kernels.py:553-586, 1410-1440): from x
 * and grad = dL/dout (grad_dtype, pitch ld_grad), grad_x = (grad - y <y,
 * grad>) / |x| with y = x / |x| where |x| > eps, grad / eps elsewhere; fp32
 * arithmetic, rounded once to out_dtype.  Same layout rules as
 * da_row_normalize, grad included.  out_dtype DA_F16 or DA_BF16 or'd with
 * DA_OUT_SPLIT writes each row's 16-bit result at columns [0, width) and its
 * rounding residual (the fp32 value minus the rounded one, rounded) at
 * [width, 2 width), with ld_out >= 2 width: a 16-bit operand pair that carries
 * the gradient to about 16 significant bits through a GEMM with fp32
 * accumulation.
 */
int da_row_normalize_backward(const void* x, int x_dtype, int64_t rows, int64_t width, int64_t ld_x, float eps,
                              const void* grad, int grad_dtype, int64_t ld_grad, void* grad_x, int out_dtype,
                              int64_t ld_out, da_stream_t stream);

/*
 * Fused dictionary route (ops.py:16-62), for any number of rows:
 *   z = N_out( sum_j w_j Dv_j ),  w = softmax(beta l) or (2/g) SiLU(g l),
 *   l_j = Std(Act(<N_in(x), Dk_j>)) with the optional 2 SiLU activation and
 *   standardization over the atoms (the DA_ROUTE_* variant flags).
 *   x:   rows x routing_dim, row pitch x_row_stride (elements), x_dtype
 *   key_t (key_dtype), value (fp16): the layouts of da_dictionary_normalize.
 *        key_dtype is DA_F16, or x_dtype; without DA_ROUTE_NORMALIZE_INPUT it
 *        must equal x_dtype (raw rows are not range-limited).
 *   beta: device scalar of beta_dtype, or NULL to use beta_value (unused by
 *        DA_ROUTE_DIRECT_SILU)
 *   silu_gain: g of DA_ROUTE_DIRECT_SILU (> 0); logit_scale: the scale of
 *        DA_ROUTE_STANDARDIZE (> 0; the reference's default is routing_dim^-1/2)
 *   out: rows x routing_dim, row pitch out_row_stride, out_dtype (DA_F16 or
 *        x_dtype); may alias x when the pitches match (each row is read
 *        completely before it is written).  A DA_F16 x needs DA_F16 keys and out.
 */
int da_dictionary_route(const void* x, int64_t rows, int64_t routing_dim, int64_t x_row_stride,
                        int x_dtype, const void* key_t, int key_dtype, const void* value,
                        int64_t atoms, const void* beta, int beta_dtype, float beta_value,
                        float eps, int flags, float silu_gain, float logit_scale, void* out,
                        int64_t out_row_stride, int out_dtype, da_stream_t stream);

/*
 * Row-wise backward of the route's assignment, every variant.  Replaces the
 * reference's _row_scaled_softmax_backward_kernel (triton_kernels.py:589-671,
 * launched at :1480) and the direct-SiLU branch of
 * _DictionaryRouteFunction.backward (triton_kernels.py:1940-1948).
 *   logits:       rows x atoms (row pitch ld_in, fp32), l_j = <N_in(x), Dk_j>
 *   grad_weights: rows x atoms (pitch ld_in, fp32), <dr, Dv_j> for the
 *                 gradient dr at the unnormalized reconstruction
 *   beta, beta_dtype, beta_value, flags (DA_ROUTE_BETA_IS_LOG and the
 *   variant bits), silu_gain, logit_scale, eps: as da_dictionary_route
 * Writes, per row, the gradient at the raw logits (grad_logits) and the
 * assignment weights (weights), rows x atoms with pitch ld_out in out_dtype
 * (DA_F16 or DA_BF16), and the row's share of d beta to dbeta_rows[row]
 * (fp32; 0 for DA_ROUTE_DIRECT_SILU; may be NULL); with DA_ROUTE_BETA_IS_LOG
 * or DA_ROUTE_BETA_IS_LOG_SCALE the share of the gradient at the log (beta
 * times the share inside the clamp's window, zero outside it).  atoms <= 2^24 (rows of
 * up to 16384 atoms are held in registers, longer rows are passed over several
 * times).
 * causal_period > 0 limits row r to columns j <= r % causal_period (zeros
 * written past them), and beta may hold beta_count (<= 64) values, row r
 * taking entry (r / beta_period) % beta_count: the outer attention's softmax
 * backward, with scores as logits, dP = dO V^T as grad_weights and the maps'
 * gammas as beta (rows ordered batch, map, token).  The GEMMs
 * around it (logits, grad_weights, then dN_in(x) = grad_logits Dk^T,
 * dDk = N_in(x)^T grad_logits, dDv = dr^T weights) are plain library GEMMs.
 */
int da_dictionary_route_backward_rows(const float* logits, const float* grad_weights, int64_t rows,
                                      int64_t atoms, int64_t causal_period, int64_t ld_in, const void* beta,
                                      int beta_dtype, float beta_value, int64_t beta_count, int64_t beta_period,
                                      int flags, float silu_gain, float logit_scale, float eps,
                                      void* grad_logits, void* weights, int64_t ld_out, int out_dtype,
                                      float* dbeta_rows, da_stream_t stream);

/*
 * Flash outer attention over `maps` score maps (ops.py:65-93) with the map
 * combine of modules.py:265-272 fused in.
 *   query/key row of (batch b, token t, map s) starts at
 *       base + b*stride_b + t*stride_t + (s / map_repeat) * map_stride
 *     and holds score_dim elements.
 *   value_t: V^T in 32-token tiles, element (b, d, t) at
 *     value_t[b*vt_stride_b + (t/32)*32*value_dim + 32*d + t%32];
 *     vt_stride_b >= value_dim * da_padded_length(length).
 *   scales: [maps] device tensor (gamma_s, or log gamma_s with
 *     DA_ATTN_SCALES_ARE_LOG); every gamma is multiplied by scale_mult.
 *   DA_ATTN_MIX: out(b, t) = sum_s alpha_s O_s(b, t), alpha = softmax(mix_logits)
 *     (uniform 1/maps if mix_logits is NULL); else O_s(b, t) goes to
 *     out + b*out_stride_b + t*out_stride_t + s*out_stride_s.
 *   workspace: NULL, or >= da_attention_workspace_bytes(...) bytes, 256-byte
 *     aligned (scratch for split key ranges; see below).
 *   score_bound: 0, or an upper bound on |q . k| over all raw query/key rows
 *     (1 for L2-normalized rows).  With a bound, maps whose scaled bound fits
 *     the probability type skip the online-softmax rescaling (bf16 V only).
 * maps <= 64.  score_dim must be 64, 128, 256 or 512; value_dim a multiple of
 * 64 in [64, 4096].  Element types:
 *   (qk_dtype, v_dtype) in {(F16, BF16), (F16, F16), (BF16, BF16)}; the output
 *   has v_dtype, or fp32 with DA_ATTN_OUT_F32 (strides then count floats, and
 *   out must be 16-byte aligned).
 *   V^T padding tokens (length .. padded length - 1) must hold finite values.
 */
int da_routed_attention(const void* query, const void* key, int64_t stride_b, int64_t stride_t,
                        int64_t map_stride, int64_t map_repeat, int64_t score_dim,
                        const void* value_t, int64_t vt_stride_b,
                        int64_t batch, int64_t maps, int64_t length, int64_t value_dim,
                        const void* scales, int scales_dtype, float scale_mult,
                        const void* mix_logits, int mix_dtype, int flags, float score_bound,
                        int qk_dtype, int v_dtype, void* out, int64_t out_stride_b,
                        int64_t out_stride_t, int64_t out_stride_s, void* workspace,
                        int64_t workspace_bytes, da_stream_t stream);

/* Scratch bytes da_routed_attention can use (0 if it needs none): fp32
 * partials of long causal key ranges split over workgroups and merged by a
 * second kernel.  Passing a NULL workspace is always allowed (no splitting). */
int64_t da_attention_workspace_bytes(int64_t batch, int64_t maps, int64_t length, int64_t score_dim,
                                     int64_t value_dim, int flags);

/*
 * Backward of the per-map outer attention (no map mix): with
 *   P_s = softmax(scales[s] * q_s k_s^T, causal mask),  out_s = P_s v,
 * given dO_s = d loss / d out_s it writes the gradients of q, k, v and
 * scales (the products of triton_kernels.py:2093-2263 behind the autograd
 * function of triton_kernels.py:2290-2305; reference math ops.py:65-93).
 *   query:       [batch*maps, length, score_dim], qk_dtype
 *   key:         [batch*maps, key_length, score_dim], qk_dtype (key_length == length
 *                for causal; other lengths serve cross attention such as the
 *                dictionary route, where the atoms are the keys and values)
 *   value:       [batch, key_length, value_dim], v_dtype
 *   out:         [batch*maps, length, value_dim], v_dtype (the forward output),
 *                or fp32 with DA_ATTN_OUT_F32 (rowsum(dO . O) then sees no
 *                16-bit rounding of O)
 *   grad_out:    [batch*maps, length, value_dim], v_dtype
 *   scales:      [maps] fp32 score scales (already exponentiated)
 *   workspace:   >= da_attention_backward_workspace_bytes(...) bytes,
 *                256-byte aligned (transposed tiles, row statistics)
 *   grad_query:  [batch*maps, length, score_dim] fp32
 *   grad_key:    [batch*maps, key_length, score_dim] fp32
 *   grad_value:  [batch, key_length, value_dim] fp32 (summed over the maps)
 *   grad_scales: [maps] fp32
 *   score_dim and value_dim in {64, 128, 256, 512}; flags:
 *   DA_ATTN_CAUSAL and DA_ATTN_OUT_F32.  The gradients are zeroed and then accumulated with
 *   fp32 atomics, so their last bits vary between runs.
 */
int64_t da_attention_backward_workspace_bytes(int64_t batch, int64_t maps, int64_t length, int64_t key_length,
                                              int64_t score_dim, int64_t value_dim);
int da_routed_attention_backward(const void* query, const void* key, const void* value, const void* out,
                                 const void* grad_out, const float* scales, int64_t batch, int64_t maps,
                                 int64_t length, int64_t key_length, int64_t score_dim, int64_t value_dim,
                                 int flags, int qk_dtype, int v_dtype, void* workspace, int64_t workspace_bytes,
                                 float* grad_query, float* grad_key, float* grad_value, float* grad_scales,
                                 da_stream_t stream);

/*
 * da_routed_attention_backward on strided query and key rows, with score
 * scales in any dtype or as logs.  Query row t of (sequence b, map s) starts
 * at query + b*query_stride_b + (s / map_repeat)*query_map_stride +
 * t*query_stride_t elements (key rows alike), so the score maps can be views
 * of the module's routed [batch, length, 2, branches, routing_dim] rows
 * (modules.py:242-247 reads them through assemble_score_maps): map_repeat
 * maps sharing one branch (outer_maps > qk_branches), or query_map_stride =
 * score_dim with score_dim = group * routing_dim for grouped branches
 * (qk_branches > outer_maps, with scale_mult = group^-1/2 in place of the
 * group^-1/4 factor on both operands).  grad_query and grad_key are fp32 with
 * the strides of query and key (every map's rows are zeroed, then
 * accumulated: maps sharing rows add up); they must not overlap each other.
 * Strides are multiples of 8, stride_t >= score_dim, and maps a multiple of
 * map_repeat.
 * The applied scale of map s is scales[s] * scale_mult, or with
 * DA_ATTN_SCALES_ARE_LOG exp(clamp(scales[s], log_min, log_max)) *
 * scale_mult; grad_scales[s] is the gradient at scales[s], which for logs
 * is zero outside [log_min, log_max] (the clamp's backward).
 * The values come as rows (value, v_dtype) or, with value NULL, as the
 * forward's V^T tiles (value_t: sequence b at value_t + b*value_t_stride_b
 * elements, [padded key_length / 32][value_dim][32], 16-bit of
 * value_t_dtype, converted to v_dtype; padding tokens finite, as
 * da_routed_attention requires).  out has out_dtype (DA_F32, DA_F16 or
 * DA_BF16) whatever v_dtype is.  grad_value_sum (optional, [value_dim]
 * fp32) receives the column sums of grad_value over every sequence and key:
 * the gradient of a bias added to the values.  With grad_scores set
 * (qk_dtype, rows of grad_scores_ld >= key_length padded to a multiple of 64,
 * 16-byte aligned) the gradient at the scaled scores, scale * dS, is written
 * there as [batch*maps*length] rows (padding keys zero) instead of
 * grad_query = scale * dS K, which is then not touched (may be NULL): a
 * caller with few keys per query (the dictionary route) forms it with one
 * GEMM instead of one atomic add per key tile.  flags: DA_ATTN_CAUSAL and
 * DA_ATTN_SCALES_ARE_LOG.  Everything else is as for
 * da_routed_attention_backward (whose workspace size serves both).
 */
typedef struct da_attention_backward_args {
  const void* query;
  int64_t query_stride_b, query_stride_t, query_map_stride;
  const void* key;
  int64_t key_stride_b, key_stride_t, key_map_stride;
  int64_t map_repeat;
  const void* value;        /* [batch, key_length, value_dim], or NULL: value_t */
  const void* value_t;
  int64_t value_t_stride_b;
  int value_t_dtype;
  const void* out;          /* [batch*maps, length, value_dim], out_dtype */
  int out_dtype;
  const void* grad_out;     /* [batch*maps, length, value_dim] */
  const void* scales;       /* [maps], scales_dtype */
  int scales_dtype;
  float scale_mult;
  float log_min, log_max;   /* with DA_ATTN_SCALES_ARE_LOG */
  int64_t batch, maps, length, key_length, score_dim, value_dim;
  int flags;                /* DA_ATTN_CAUSAL, DA_ATTN_SCALES_ARE_LOG */
  int qk_dtype, v_dtype;
  void* workspace;
  int64_t workspace_bytes;
  float* grad_query;
  float* grad_key;
  float* grad_value;        /* [batch, key_length, value_dim] */
  float* grad_scales;       /* [maps] */
  float* grad_value_sum;    /* [value_dim] or NULL */
  void* grad_scores;        /* [batch*maps*length, grad_scores_ld], qk_dtype, or NULL */
  int64_t grad_scores_ld;
} da_attention_backward_args;

int da_routed_attention_backward_ex(const da_attention_backward_args* args, da_stream_t stream);

/*
 * Q/K and V projections in one launch (modules.py:143-157 and 212):
 *   qk_out [tokens, 2*qk_width] = x @ [wq; wk]^T   (row n: query features, then key features)
 *   value_t (b, f, t)           = (x @ wv^T + bv)[b*length + t, f], in the 32-token
 *                                 tile layout of da_routed_attention
 *   x: [tokens, model_dim] with tokens = batch*length; wq, wk: [qk_width, model_dim];
 *   wv: [value_dim, model_dim]; bv: [value_dim] of bias_dtype or NULL.
 *   vt_stride_b per sequence (>= value_dim * vt_pitch); vt_pitch (a multiple
 *   of 64, >= length) tokens are written per sequence, the padding ones with
 *   finite values.
 */
int da_qkv_projection(const void* x, int64_t tokens, int64_t model_dim, int64_t length,
                      const void* wq, const void* wk, int64_t qk_width, const void* wv,
                      const void* bv, int64_t value_dim, int bias_dtype, int dtype, void* qk_out,
                      void* value_t, int64_t vt_stride_b, int64_t vt_pitch, da_stream_t stream);

/* out [rows, out_features] = x [rows, in_features] @ weight^T (+ bias) */
int da_linear(const void* x, int64_t rows, int64_t in_features, const void* weight,
              int64_t out_features, const void* bias, int bias_dtype, int dtype, void* out,
              da_stream_t stream);

/* Activations of da_linear_ex. */
#define DA_ACT_NONE 0
#define DA_ACT_GELU 1               /* exact (erf) GELU, nn.GELU()'s default */

/*
 * The block's feed-forward linears with their neighbours fused in
 * (modules.py:318-330, 343-346: Linear -> GELU -> Linear, then x + ...):
 *   out = act(x @ weight^T + bias), rounded to dtype, then + residual
 *   (residual: NULL or [rows, out_features] like out, added to the rounded
 *   result and rounded again, as the unfused `x + linear(...)` does).
 */
int da_linear_ex(const void* x, int64_t rows, int64_t in_features, const void* weight, int64_t out_features,
                 const void* bias, int bias_dtype, int dtype, int activation, const void* residual, void* out,
                 da_stream_t stream);

/*
 * LayerNorm over the last dimension (nn.LayerNorm of modules.py:311, 313, 440;
 * applied at :340, :344, :454): out = (x - mean) / sqrt(var + eps) * weight +
 * bias, biased variance, fp32 statistics.  x, out: [rows, dim] of dtype;
 * weight, bias: [dim] of param_dtype, or NULL (1 and 0).  dim a multiple of 8,
 * at most 4096; pointers 16-byte aligned.
 */
int da_layer_norm(const void* x, int64_t rows, int64_t dim, const void* weight, const void* bias, int param_dtype,
                  float eps, int dtype, void* out, da_stream_t stream);

/*
 * Backward of da_layer_norm (autograd of nn.LayerNorm) at grad = dL/dout
 * ([rows, dim] of dtype): the statistics are formed again from x in fp32;
 * grad_x = rstd (g - mean(g) - xh mean(g xh)) with xh = (x - mean) rstd and
 * g = grad weight (weight of param_dtype, or NULL for 1), rounded once to
 * dtype.  grad_params is [8][2 dim] fp32, zeroed by the caller: the rows'
 * sums of grad xh (the weight's gradient) and of grad (the bias's) are added
 * into its eight copies (fp32 atomic adds spread over the copies), and the
 * gradients are the sums over the copies: weight columns [0, dim), bias
 * columns [dim, 2 dim) of each copy (da_sum_partials adds them and rounds to
 * 16 bits in one launch).  Same layout rules as da_layer_norm.
 */
int da_layer_norm_backward(const void* x, const void* grad, int64_t rows, int64_t dim, const void* weight,
                           int param_dtype, float eps, int dtype, void* grad_x, float* grad_params, da_stream_t stream);

/*
 * The weighted map combine (modules.py:265-272: einsum("s,bstd->btd", w,
 * map_output)) over fp32 per-map outputs, as the training path keeps them:
 *   maps: [batch, n_maps, length, width] fp32, contiguous, 16-byte aligned
 *   weights: [n_maps] fp32 (device), n_maps in [1, 8]; width a multiple of 8
 *   out[b, t, :] = sum_s weights[s] maps[b, s, t, :], fp32 sum rounded once to
 *   out_dtype (DA_F16 or DA_BF16), [batch, length, width], 16-byte aligned.
 * Its backward at grad = dL/dout ([batch, length, width], grad_dtype):
 *   grad_maps[b, s, t, :] = weights[s] grad[b, t, :] rounded to grad_dtype
 *   ([batch, n_maps, length, width]), and weight_sums[s] += sum over b, t and
 *   the features of maps[b, s, t, :] grad[b, t, :] (fp32 atomic adds: the
 *   caller zeroes weight_sums; the gradient at the weights themselves).
 */
int da_map_combine(const float* maps, int64_t batch, int64_t n_maps, int64_t length, int64_t width,
                   const float* weights, void* out, int out_dtype, da_stream_t stream);

/*
 * Operands of the dense outer-attention backward (library GEMMs around
 * da_dictionary_route_backward_rows for long sequences and wide scores; the
 * products of the reference's attention backward, triton_kernels.py:2093-2263)
 * in one pass over the score maps.  Row (b, s, t) of query and key starts at
 *   base + b*stride_b + (s / map_repeat)*map_stride + t*stride_t
 * and holds score_dim elements of qk_dtype (strides in elements, multiples of
 * 8).  Writes key_t [batch*maps, score_dim, length] (K^T, qk_dtype) and
 * query_out, key_out [batch*maps, length, score_dim] (out_dtype): the right
 * operands of S = q k^T, dk = dS^T q and dq = dS k.  score_dim a multiple of
 * 64 up to 4096, batch*maps <= 65535, pointers 16-byte aligned.
 */
int da_dense_attention_operands(const void* query, const void* key, int64_t stride_b, int64_t stride_t,
                                int64_t map_stride, int64_t map_repeat, int qk_dtype, int64_t batch, int64_t maps,
                                int64_t length, int64_t score_dim, void* key_t, void* query_out, void* key_out,
                                int out_dtype, da_stream_t stream);

/*
 * out[i] = sum over c < count of partials[c * n + i], summed in fp32 in order
 * and rounded once to out_dtype (DA_F16 or DA_BF16): the split-K partial
 * products of the training path's weight gradients (no counterpart in the
 * reference, whose autograd forms them in one GEMM).  n a multiple of 8,
 * count in [1, 1024], pointers 16-byte aligned.
 */
int da_sum_partials(const float* partials, int64_t count, int64_t n, void* out, int out_dtype, da_stream_t stream);
int da_map_combine_backward(const float* maps, int64_t batch, int64_t n_maps, int64_t length, int64_t width,
                            const float* weights, const void* grad, int grad_dtype, void* grad_maps,
                            float* weight_sums, da_stream_t stream);

/* Whole SharedDictionaryAttention forward (modules.py:190-291): model_dim a
 * multiple of 64 in [64, 4096], routing_dim (and the grouped score width) in
 * {64, 128, 256, 512}. */
typedef struct da_sda_forward_args {
  const void* x;            /* [batch, length, model_dim] */
  int64_t batch, length, model_dim;
  int64_t qk_branches, outer_maps, routing_dim, atoms;
  const void* wq;           /* query.weight [qk_branches*routing_dim, model_dim] */
  const void* wk;           /* key.weight */
  const void* wv;           /* value.weight [model_dim, model_dim] */
  const void* bv;           /* value.bias [model_dim] or NULL */
  const void* wo;           /* output.weight [model_dim, model_dim or maps*model_dim] or NULL (identity) */
  const void* key_t;        /* normalized bank, da_dictionary_normalize layouts (written by
                               this call when raw_key is set) */
  const void* value;
  const void* log_beta;     /* scalar */
  const void* log_score_scales; /* [outer_maps] */
  const void* map_mix_logits;   /* [outer_maps] or NULL */
  int param_dtype;          /* dtype of bias and of the three scalar tensors */
  int dtype;                /* activation / weight dtype: DA_F16 or DA_BF16 */
  float eps;
  int flags;                /* DA_SDA_* */
  void* workspace;          /* da_sda_workspace_bytes(...) bytes, 256-byte aligned */
  int64_t workspace_bytes;
  void* out;                /* [batch, length, model_dim] */
  /* Optional: the raw bank (da_dictionary_normalize's raw_key / raw_value /
   * raw_dtype).  When raw_key is non-NULL the call normalizes it into key_t
   * and value first, inside its projection launch (no launch of its own). */
  const void* raw_key;
  const void* raw_value;
  int raw_dtype;
  /* Route variants: DA_ROUTE_SILU_LOGITS | DA_ROUTE_STANDARDIZE |
   * DA_ROUTE_DIRECT_SILU bits (0 = identity activation, softmax assignment),
   * with their silu_gain and logit_scale as for da_dictionary_route. */
  int route_variant;
  float silu_gain;
  float logit_scale;
  /* Optional: [batch, length, model_dim] added to the output projection's
   * rounded result (the block's residual `x + attention(...)`, modules.py:
   * 338-342); needs wo and 16-byte alignment.  NULL: none. */
  const void* residual;
} da_sda_forward_args;

/* Workspace layout (byte offsets, each 256-aligned):
 *   routed [tokens, 2*qk_width]   Q/K projections, routed in place (fp16 out)
 *   value_t [batch, padded_length/32, model_dim, 32]  (32-token tiles)
 *   mixed  [tokens, model_dim or maps*model_dim] (only with an output projection)
 *   then, with one outer map, fp32 partial results of the attention over
 *   chunks of long causal key ranges (merged by a second kernel). */
int64_t da_sda_workspace_bytes(int64_t batch, int64_t length, int64_t model_dim,
                               int64_t qk_width, int64_t outer_maps, int concat,
                               int has_output_projection);
int64_t da_sda_workspace_offset(int64_t batch, int64_t length, int64_t model_dim,
                                int64_t qk_width, int which /* 0 routed, 1 value_t, 2 mixed */);

int da_shared_dictionary_attention_forward(const da_sda_forward_args* args, da_stream_t stream);

/*
 * Allocation-free variant of da_shared_dictionary_attention_forward.  It has
 * no counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  args->workspace and args->workspace_bytes are
 * ignored; the workspace is a library-owned device array of
 * DA_NOALLOC_SCRATCH_BYTES per GPU (each GPU the library runs on holds it
 * until the process ends), found once per device on its first call there;
 * the call uses the array of the device `stream` launches on (the current
 * device for the null stream).
 * Problems whose da_sda_workspace_bytes exceed it fail with DA_ERR_WORKSPACE.
 * The call itself allocates nothing.  Every call on one GPU shares that GPU's
 * array, which keeps the last call's contents: calls that overlap on one GPU
 * (other streams, other threads) race, so serialize them.  The caller still
 * owns x, the weights, the bank layouts and out.
 */
#define DA_NOALLOC_SCRATCH_BYTES (128LL << 20)
int da_shared_dictionary_attention_forward_noalloc(const da_sda_forward_args* args, da_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DOUBLE_ATTENTION_HIP_H */
