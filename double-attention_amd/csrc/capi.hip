// C ABI entry points (declared in include/double_attention_hip.h).
//
// Each entry point validates its arguments on the host, then enqueues the
// kernels on the caller's stream.  Nothing is allocated, freed or
// synchronized here.  Validation failures return before any launch so the
// stream is untouched; launch failures are reported from hipGetLastError.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/double_attention_hip.h"
#include "da_launch.h"
#include "dict_norm.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }
bool pow2_width(int64_t v) { return v == 64 || v == 128 || v == 256 || v == 512; }
// The attention forward takes value (model) widths that are multiples of 64:
// its value slices are 64, 128 or 256 features wide.
constexpr int64_t kMaxValueDim = 4096;
bool half_dtype(int d) { return d == DA_F16 || d == DA_BF16; }
bool any_dtype(int d) { return d == DA_F32 || d == DA_F16 || d == DA_BF16; }

int ok() {
  g_error.clear();
  return DA_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_error.clear();
  return DA_OK;
}

constexpr int64_t kAlign = 256;
int64_t align_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

constexpr int kRouteFlagMask = DA_ROUTE_NORMALIZE_INPUT | DA_ROUTE_NORMALIZE_OUTPUT | DA_ROUTE_BETA_IS_LOG |
                               DA_ROUTE_UNIT_KEYS | DA_ROUTE_SILU_LOGITS | DA_ROUTE_STANDARDIZE |
                               DA_ROUTE_DIRECT_SILU;
constexpr int kRouteVariantMask = DA_ROUTE_SILU_LOGITS | DA_ROUTE_STANDARDIZE | DA_ROUTE_DIRECT_SILU;

int validate_route(const void* x, int64_t rows, int64_t R, int64_t xs, int x_dtype, const void* kt,
                   int key_dtype, const void* v, int64_t atoms, const void* beta, int beta_dtype,
                   int flags, float silu_gain, float logit_scale, const void* out, int64_t os, int out_dtype) {
  if (flags & ~kRouteFlagMask) return fail(DA_ERR_INVALID_ARGUMENT, "route: unknown flag bits 0x%x", flags);
  if ((flags & DA_ROUTE_DIRECT_SILU) && !(silu_gain > 0.f && std::isfinite(silu_gain)))
    return fail(DA_ERR_INVALID_ARGUMENT, "route: silu_gain must be positive and finite");
  if ((flags & DA_ROUTE_STANDARDIZE) && !(logit_scale > 0.f && std::isfinite(logit_scale)))
    return fail(DA_ERR_INVALID_ARGUMENT, "route: logit_scale must be positive and finite");
  if (!half_dtype(x_dtype) || !half_dtype(key_dtype) || !half_dtype(out_dtype))
    return fail(DA_ERR_INVALID_ARGUMENT, "route: element types must be DA_F16 or DA_BF16");
  if (key_dtype != DA_F16 && key_dtype != x_dtype)
    return fail(DA_ERR_UNSUPPORTED, "route: key_dtype must be DA_F16 or x_dtype");
  if (!(flags & DA_ROUTE_NORMALIZE_INPUT) && key_dtype != x_dtype)
    return fail(DA_ERR_UNSUPPORTED, "route: without input normalization key_dtype must equal x_dtype");
  if (out_dtype != DA_F16 && out_dtype != x_dtype)
    return fail(DA_ERR_UNSUPPORTED, "route: out_dtype must be DA_F16 or x_dtype");
  if (!pow2_width(R)) return fail(DA_ERR_UNSUPPORTED, "route: routing_dim %lld not in {64,128,256,512}", (long long)R);
  if (rows < 0 || atoms < 1 || atoms > (1 << 24)) return fail(DA_ERR_INVALID_ARGUMENT, "route: bad rows/atoms");
  if (rows == 0) return DA_OK;
  if (!x || !kt || !v || !out) return fail(DA_ERR_INVALID_ARGUMENT, "route: null pointer");
  if (beta && !any_dtype(beta_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "route: bad beta dtype");
  if (!aligned(x, 16) || !aligned(kt, 16) || !aligned(v, 16) || !aligned(out, 16))
    return fail(DA_ERR_ALIGNMENT, "route: tensors must be 16-byte aligned");
  if (xs < R || xs % 8 || os < R || os % 8)
    return fail(DA_ERR_ALIGNMENT, "route: row strides must be >= routing_dim and multiples of 8");
  if ((rows + 63) / 64 > 0x7fffffffLL) return fail(DA_ERR_UNSUPPORTED, "route: too many rows");
  return DA_OK;
}

int validate_attention(const void* q, const void* k, int64_t sb, int64_t st, int64_t ms, int64_t rep,
                       int64_t RP, const void* vt, int64_t vsb, int64_t B, int64_t S,
                       int64_t T, int64_t D, const void* scales, int scales_dtype,
                       const void* mix, int mix_dtype, int qk_dtype, int v_dtype, const void* out,
                       int64_t ob, int64_t ot, int64_t os) {
  const bool types_ok = (qk_dtype == DA_F16 && (v_dtype == DA_BF16 || v_dtype == DA_F16)) ||
                        (qk_dtype == DA_BF16 && v_dtype == DA_BF16);
  if (!types_ok)
    return fail(DA_ERR_UNSUPPORTED, "attention: (qk_dtype, v_dtype) must be (F16,BF16), (F16,F16) or (BF16,BF16)");
  if (!pow2_width(RP)) return fail(DA_ERR_UNSUPPORTED, "attention: score_dim %lld not in {64,128,256,512}", (long long)RP);
  if (D < 64 || D > kMaxValueDim || D % 64)
    return fail(DA_ERR_UNSUPPORTED, "attention: value_dim %lld must be a multiple of 64 in [64, %lld]", (long long)D,
                (long long)kMaxValueDim);
  if (B < 0 || T < 0 || S < 1 || rep < 1 || B > 65535 || T > (1LL << 30))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention: bad batch/maps/length/map_repeat");
  if (S > 64) return fail(DA_ERR_UNSUPPORTED, "attention: at most 64 maps (got %lld)", (long long)S);
  if (B == 0 || T == 0) return DA_OK;
  if (!q || !k || !vt || !scales || !out) return fail(DA_ERR_INVALID_ARGUMENT, "attention: null pointer");
  if (!any_dtype(scales_dtype) || (mix && !any_dtype(mix_dtype)))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention: bad scalar dtype");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(vt, 16) || !aligned(out, 8))
    return fail(DA_ERR_ALIGNMENT, "attention: q/k/value_t must be 16-byte and out 8-byte aligned");
  if (sb % 8 || st % 8 || ms % 8 || st < RP)
    return fail(DA_ERR_ALIGNMENT, "attention: q/k strides must be multiples of 8 and stride_t >= score_dim");
  if (vsb % 8 || (B > 1 && vsb < D * da::round_up(T, da::kKeyPad)))
    return fail(DA_ERR_ALIGNMENT, "attention: vt_stride_b must be a multiple of 8 and >= value_dim * padded length");
  if (ob % 4 || ot % 4 || os % 4) return fail(DA_ERR_ALIGNMENT, "attention: out strides must be multiples of 4");
  return DA_OK;
}

}  // namespace

extern "C" {

static_assert(DA_OUT_SPLIT == da::kOutSplit, "split-output flag");
static_assert(DA_ROUTE_BETA_IS_LOG_SCALE == da::kRouteBetaIsLogScale, "route flag");

int da_abi_version(void) { return 19; }

const char* da_last_error(void) { return g_error.c_str(); }

int64_t da_padded_atoms(int64_t atoms) { return da::round_up(atoms, da::kAtomPad); }

int64_t da_padded_length(int64_t length) { return da::round_up(length, da::kKeyPad); }

int da_dictionary_normalize(const void* raw_key, const void* raw_value, int raw_dtype,
                            int64_t routing_dim, int64_t atoms, float eps, void* key_t,
                            int key_dtype, void* value, void* value_rows, da_stream_t stream) {
  if (!any_dtype(raw_dtype) || !half_dtype(key_dtype))
    return fail(DA_ERR_INVALID_ARGUMENT, "normalize: bad dtype");
  if (!pow2_width(routing_dim))
    return fail(DA_ERR_UNSUPPORTED, "normalize: routing_dim %lld not in {64,128,256,512}", (long long)routing_dim);
  if (atoms < 1 || atoms > (1 << 24)) return fail(DA_ERR_INVALID_ARGUMENT, "normalize: bad atom count");
  if (!raw_key || !key_t || !value) return fail(DA_ERR_INVALID_ARGUMENT, "normalize: null pointer");
  if (!aligned(key_t, 16) || !aligned(value, 16) || !aligned(value_rows, 16))
    return fail(DA_ERR_ALIGNMENT, "normalize: outputs must be 16-byte aligned");
  da::launch_dictionary_normalize(raw_key, raw_value, raw_dtype, static_cast<int>(routing_dim),
                                  static_cast<int>(atoms), eps, key_t, key_dtype, value, value_rows,
                                  reinterpret_cast<hipStream_t>(stream));
  return check_launch("normalize");
}

int da_dictionary_normalize_backward(const void* raw_key, const void* raw_value, int raw_dtype,
                                     int64_t routing_dim, int64_t atoms, float eps, const float* grad_key,
                                     const float* grad_value, int64_t grad_ld_r, int64_t grad_ld_j,
                                     void* d_raw_key, void* d_raw_value, da_stream_t stream) {
  if (!any_dtype(raw_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: bad dtype");
  if (routing_dim < 1 || routing_dim > (1 << 16))
    return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: routing_dim %lld out of range", (long long)routing_dim);
  if (atoms < 1 || atoms > (1 << 24)) return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: bad atom count");
  if (!(eps >= 0.f)) return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: eps must be >= 0");
  if (!raw_key || !grad_key || !d_raw_key) return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: null pointer");
  if (!raw_value && d_raw_value)
    return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: d_raw_value given for a tied bank");
  // Each atom's coordinates must be distinct elements: one stride 1 and the
  // other covering the first's range.
  const bool coord_major = grad_ld_j == 1 && grad_ld_r >= atoms;
  const bool atom_major = grad_ld_r == 1 && grad_ld_j >= routing_dim;
  if (!coord_major && !atom_major)
    return fail(DA_ERR_INVALID_ARGUMENT, "normalize backward: gradient strides (%lld, %lld) must be (>= atoms, 1) or "
                "(1, >= routing_dim)", (long long)grad_ld_r, (long long)grad_ld_j);
  const da::NormBwdArgs a{raw_key, raw_value, raw_dtype, static_cast<int>(routing_dim), atoms, eps,
                          grad_key, grad_value, grad_ld_r, grad_ld_j, d_raw_key, d_raw_value};
  da::launch_dictionary_normalize_backward(a, reinterpret_cast<hipStream_t>(stream));
  return check_launch("normalize backward");
}

namespace {

int validate_row_norm(const char* what, const void* x, int x_dtype, int64_t rows, int64_t width, int64_t ld_x,
                      float eps, const void* grad, int grad_dtype, int64_t ld_grad, bool backward, const void* out,
                      int out_dtype, int64_t ld_out) {
  // DA_OUT_SPLIT (backward only, 16-bit outputs): head and residual side by
  // side, so the output row spans 2 x width.
  const bool split = backward && (out_dtype & DA_OUT_SPLIT);
  if (split) {
    out_dtype &= ~DA_OUT_SPLIT;
    if (out_dtype != DA_F16 && out_dtype != DA_BF16)
      return fail(DA_ERR_INVALID_ARGUMENT, "%s: DA_OUT_SPLIT needs a 16-bit output", what);
    if (ld_out < 2 * width) return fail(DA_ERR_ALIGNMENT, "%s: DA_OUT_SPLIT needs ld_out >= 2 width", what);
  }
  if (!any_dtype(x_dtype) || !any_dtype(out_dtype) || (backward && !any_dtype(grad_dtype)))
    return fail(DA_ERR_INVALID_ARGUMENT, "%s: bad dtype", what);
  if (rows < 0 || rows > 0x7fffffffLL * 4) return fail(DA_ERR_INVALID_ARGUMENT, "%s: bad row count", what);
  if (width < 4 || width > (1 << 20) || width % 4)
    return fail(DA_ERR_UNSUPPORTED, "%s: width %lld must be a positive multiple of 4", what, (long long)width);
  if (!(eps >= 0.f)) return fail(DA_ERR_INVALID_ARGUMENT, "%s: eps must be >= 0", what);
  if (!x || !out || (backward && !grad)) return fail(DA_ERR_INVALID_ARGUMENT, "%s: null pointer", what);
  if (ld_x < width || ld_out < width || (backward && ld_grad < width) || ld_x % 4 || ld_out % 4 ||
      (backward && ld_grad % 4))
    return fail(DA_ERR_ALIGNMENT, "%s: row pitches must be >= width and multiples of 4", what);
  const auto elem = [](int d) { return d == DA_F32 ? 4 : 2; };
  if (reinterpret_cast<uintptr_t>(x) % (4 * elem(x_dtype)) || reinterpret_cast<uintptr_t>(out) % (4 * elem(out_dtype)) ||
      (backward && reinterpret_cast<uintptr_t>(grad) % (4 * elem(grad_dtype))))
    return fail(DA_ERR_ALIGNMENT, "%s: tensors must be aligned to 4 elements", what);
  return 0;
}

}  // namespace

int da_row_normalize(const void* x, int x_dtype, int64_t rows, int64_t width, int64_t ld_x, float eps, void* out,
                     int out_dtype, int64_t ld_out, da_stream_t stream) {
  int rc = validate_row_norm("row normalize", x, x_dtype, rows, width, ld_x, eps, nullptr, DA_F32, 0, false, out,
                             out_dtype, ld_out);
  if (rc) return rc;
  if (rows == 0) return ok();
  const da::RowNormArgs a{x, x_dtype, ld_x, rows, static_cast<int>(width), eps, nullptr, DA_F32, 0, out, out_dtype,
                          ld_out};
  da::launch_row_normalize(a, false, reinterpret_cast<hipStream_t>(stream));
  return check_launch("row normalize");
}

int da_row_normalize_backward(const void* x, int x_dtype, int64_t rows, int64_t width, int64_t ld_x, float eps,
                              const void* grad, int grad_dtype, int64_t ld_grad, void* grad_x, int out_dtype,
                              int64_t ld_out, da_stream_t stream) {
  int rc = validate_row_norm("row normalize backward", x, x_dtype, rows, width, ld_x, eps, grad, grad_dtype, ld_grad,
                             true, grad_x, out_dtype, ld_out);
  if (rc) return rc;
  if (rows == 0) return ok();
  const da::RowNormArgs a{x, x_dtype, ld_x, rows, static_cast<int>(width), eps, grad, grad_dtype, ld_grad, grad_x,
                          out_dtype, ld_out};
  da::launch_row_normalize(a, true, reinterpret_cast<hipStream_t>(stream));
  return check_launch("row normalize backward");
}

int da_dictionary_route(const void* x, int64_t rows, int64_t routing_dim, int64_t x_row_stride,
                        int x_dtype, const void* key_t, int key_dtype, const void* value,
                        int64_t atoms, const void* beta, int beta_dtype, float beta_value,
                        float eps, int flags, float silu_gain, float logit_scale, void* out,
                        int64_t out_row_stride, int out_dtype, da_stream_t stream) {
  int rc = validate_route(x, rows, routing_dim, x_row_stride, x_dtype, key_t, key_dtype, value, atoms,
                          beta, beta_dtype, flags, silu_gain, logit_scale, out, out_row_stride, out_dtype);
  if (rc) return rc;
  if (rows == 0) return ok();
  da::RouteArgs a{x, rows, x_row_stride, x_dtype, static_cast<int>(routing_dim), key_t, key_dtype,
                  value, static_cast<int>(atoms), beta, beta_dtype, beta_value, eps, flags, silu_gain,
                  logit_scale, out, out_row_stride, out_dtype};
  da::launch_dictionary_route(a, reinterpret_cast<hipStream_t>(stream));
  return check_launch("route");
}

int da_dictionary_route_backward_rows(const float* logits, const float* grad_weights, int64_t rows,
                                      int64_t atoms, int64_t causal_period, int64_t ld_in, const void* beta,
                                      int beta_dtype, float beta_value, int64_t beta_count, int64_t beta_period,
                                      int flags, float silu_gain, float logit_scale, float eps,
                                      void* grad_logits, void* weights, int64_t ld_out, int out_dtype,
                                      float* dbeta_rows, da_stream_t stream) {
  constexpr int kBwdRowsFlags = DA_ROUTE_BETA_IS_LOG | DA_ROUTE_BETA_IS_LOG_SCALE | DA_ROUTE_SILU_LOGITS |
                                DA_ROUTE_STANDARDIZE | DA_ROUTE_DIRECT_SILU;
  if (flags & ~kBwdRowsFlags)
    return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: unknown flag bits 0x%x", flags);
  if ((flags & DA_ROUTE_BETA_IS_LOG) && (flags & DA_ROUTE_BETA_IS_LOG_SCALE))
    return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: DA_ROUTE_BETA_IS_LOG and _LOG_SCALE exclude each other");
  if ((flags & DA_ROUTE_DIRECT_SILU) && !(silu_gain > 0.f && std::isfinite(silu_gain)))
    return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: silu_gain must be positive and finite");
  if ((flags & DA_ROUTE_STANDARDIZE) && !(logit_scale > 0.f && std::isfinite(logit_scale)))
    return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: logit_scale must be positive and finite");
  if (!half_dtype(out_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: out_dtype must be DA_F16 or DA_BF16");
  if (rows < 0 || atoms < 1) return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: bad rows/atoms");
  if (atoms > da::kRouteBwdRowsMaxAtoms)
    return fail(DA_ERR_UNSUPPORTED, "route backward rows: at most %d atoms (got %lld)", da::kRouteBwdRowsMaxAtoms,
                (long long)atoms);
  if (ld_in < atoms || ld_out < atoms) return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: row pitches < atoms");
  if (causal_period < 0) return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: causal_period must be >= 0");
  if (beta_count < 1 || beta_count > 64 || (beta_count > 1 && (beta_period < 1 || !beta)))
    return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: beta_count in [1, 64] with a positive beta_period");
  if (rows == 0) return ok();
  if (!logits || !grad_weights || !grad_logits || !weights)
    return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: null pointer");
  if (beta && !any_dtype(beta_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "route backward rows: bad beta dtype");
  if ((rows + 3) / 4 > 0x7fffffffLL) return fail(DA_ERR_UNSUPPORTED, "route backward rows: too many rows");
  da::RouteBwdRowsArgs a{logits, grad_weights, rows, static_cast<int>(atoms), causal_period, ld_in, beta, beta_dtype,
                         beta_value, static_cast<int>(beta_count), beta_count > 1 ? beta_period : 1,
                         flags, silu_gain, logit_scale, eps, grad_logits, weights, ld_out, out_dtype, dbeta_rows};
  da::launch_route_backward_rows(a, reinterpret_cast<hipStream_t>(stream));
  return check_launch("route backward rows");
}

int64_t da_attention_workspace_bytes(int64_t batch, int64_t maps, int64_t length, int64_t score_dim,
                                     int64_t value_dim, int flags) {
  if (batch < 1 || maps < 1 || length < 1 || value_dim < 1) return 0;
  const bool multi = (flags & DA_ATTN_MIX) && maps > 1;
  return align_up(da::plan_attention(batch, maps, length, value_dim, score_dim, multi, flags & DA_ATTN_CAUSAL, true,
                                     (flags & DA_ATTN_OUT_F32) ? 4 : 2)
                      .part_bytes);
}

int da_routed_attention(const void* query, const void* key, int64_t stride_b, int64_t stride_t,
                        int64_t map_stride, int64_t map_repeat, int64_t score_dim,
                        const void* value_t, int64_t vt_stride_b,
                        int64_t batch, int64_t maps, int64_t length, int64_t value_dim,
                        const void* scales, int scales_dtype, float scale_mult,
                        const void* mix_logits, int mix_dtype, int flags, float score_bound,
                        int qk_dtype, int v_dtype, void* out, int64_t out_stride_b,
                        int64_t out_stride_t, int64_t out_stride_s, void* workspace,
                        int64_t workspace_bytes, da_stream_t stream) {
  int rc = validate_attention(query, key, stride_b, stride_t, map_stride, map_repeat, score_dim,
                              value_t, vt_stride_b, batch, maps, length, value_dim,
                              scales, scales_dtype, mix_logits, mix_dtype, qk_dtype, v_dtype, out,
                              out_stride_b, out_stride_t, out_stride_s);
  if (rc) return rc;
  if (!(score_bound >= 0.f) || std::isinf(score_bound))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention: score_bound must be finite and >= 0");
  if (flags & ~(DA_ATTN_CAUSAL | DA_ATTN_SCALES_ARE_LOG | DA_ATTN_MIX | DA_ATTN_OUT_F32))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention: unknown flag bits 0x%x", flags);
  // fp32 outputs are written as 16-byte vectors of four floats.
  if ((flags & DA_ATTN_OUT_F32) && !aligned(out, 16))
    return fail(DA_ERR_ALIGNMENT, "attention: fp32 out (DA_ATTN_OUT_F32) must be 16-byte aligned");
  const int64_t need = da_attention_workspace_bytes(batch, maps, length, score_dim, value_dim, flags);
  if (workspace && need > 0) {
    if (!aligned(workspace, 256)) return fail(DA_ERR_ALIGNMENT, "attention: workspace must be 256-byte aligned");
    if (workspace_bytes < need)
      return fail(DA_ERR_WORKSPACE, "attention: workspace of %lld bytes < %lld required",
                  (long long)workspace_bytes, (long long)need);
  }
  if (batch == 0 || length == 0) return ok();
  da::AttentionArgs a;
  a.q = query;
  a.k = key;
  a.qk_stride_b = stride_b;
  a.qk_stride_t = stride_t;
  a.map_stride = map_stride;
  a.map_repeat = static_cast<int>(map_repeat);
  a.RP = static_cast<int>(score_dim);
  a.vt = value_t;
  a.vt_stride_b = vt_stride_b;
  a.B = static_cast<int>(batch);
  a.S = static_cast<int>(maps);
  a.T = static_cast<int>(length);
  a.D = static_cast<int>(value_dim);
  a.scales = scales;
  a.scales_dtype = scales_dtype;
  a.scale_mult = scale_mult;
  a.mix_logits = mix_logits;
  a.mix_dtype = mix_dtype;
  a.flags = flags;
  a.score_bound = score_bound;
  a.qk_dtype = qk_dtype;
  a.v_dtype = v_dtype;
  a.out = out;
  a.out_stride_b = out_stride_b;
  a.out_stride_t = out_stride_t;
  a.out_stride_s = out_stride_s;
  da::launch_routed_attention(a, need > 0 ? workspace : nullptr, reinterpret_cast<hipStream_t>(stream));
  return check_launch("attention");
}

int64_t da_attention_backward_workspace_bytes(int64_t batch, int64_t maps, int64_t length, int64_t key_length,
                                              int64_t score_dim, int64_t value_dim) {
  if (batch < 1 || maps < 1 || length < 1 || key_length < 1 || score_dim < 1 || value_dim < 1) return 0;
  return da::attention_bwd_layout(batch, maps, length, key_length, score_dim, value_dim).bytes;
}

int da_routed_attention_backward_ex(const da_attention_backward_args* args, da_stream_t stream) {
  if (!args) return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: null args");
  const da_attention_backward_args& x = *args;
  const int qk_dtype = x.qk_dtype, v_dtype = x.v_dtype, flags = x.flags;
  const bool types_ok = (qk_dtype == DA_F16 && (v_dtype == DA_BF16 || v_dtype == DA_F16)) ||
                        (qk_dtype == DA_BF16 && v_dtype == DA_BF16);
  if (!types_ok)
    return fail(DA_ERR_UNSUPPORTED,
                "attention backward: (qk_dtype, v_dtype) must be (F16,BF16), (F16,F16) or (BF16,BF16)");
  if (flags & ~(DA_ATTN_CAUSAL | DA_ATTN_SCALES_ARE_LOG))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: unknown flag bits 0x%x", flags);
  if (!any_dtype(x.out_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: bad out dtype");
  if (!x.value && !(half_dtype(x.value_t_dtype) && x.value_t_stride_b >= 0 && x.value_t_stride_b % 8 == 0))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: V^T tiles need a 16-bit dtype and a stride_b multiple of 8");
  if (!pow2_width(x.score_dim))
    return fail(DA_ERR_UNSUPPORTED, "attention backward: score_dim %lld not in {64,128,256,512}", (long long)x.score_dim);
  if (!pow2_width(x.value_dim))
    return fail(DA_ERR_UNSUPPORTED, "attention backward: value_dim %lld not in {64,128,256,512}", (long long)x.value_dim);
  const int64_t batch = x.batch, maps = x.maps, length = x.length, key_length = x.key_length;
  if (batch < 0 || length < 0 || key_length < 0 || maps < 1 || maps > 64 || batch * maps > 65535 ||
      length > (1LL << 24) || key_length > (1LL << 24))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: bad batch/maps/length/key_length");
  if (x.map_repeat < 1 || maps % x.map_repeat)
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: maps must be a multiple of map_repeat >= 1");
  if ((flags & DA_ATTN_CAUSAL) && key_length != length)
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: a causal mask needs key_length == length");
  if (!any_dtype(x.scales_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: bad scales dtype");
  if (!(x.scale_mult > 0.f) || std::isinf(x.scale_mult))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: scale_mult must be finite and > 0");
  if ((flags & DA_ATTN_SCALES_ARE_LOG) &&
      !(x.log_min <= x.log_max && std::isfinite(x.log_min) && std::isfinite(x.log_max)))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: log_min <= log_max must be finite");
  const int64_t qs[] = {x.query_stride_b, x.query_stride_t, x.query_map_stride,
                        x.key_stride_b, x.key_stride_t, x.key_map_stride};
  for (int64_t st : qs)
    if (st < 0 || st % 8) return fail(DA_ERR_ALIGNMENT, "attention backward: strides must be multiples of 8");
  if (x.query_stride_t < x.score_dim || x.key_stride_t < x.score_dim)
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: stride_t must be >= score_dim");
  if (batch == 0 || length == 0) return ok();
  if (key_length == 0) return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: queries need at least one key");
  if (x.grad_scores && (x.grad_scores_ld < da::round_up(key_length, da::kKeyPad) || x.grad_scores_ld % 8 ||
                        !aligned(x.grad_scores, 16)))
    return fail(DA_ERR_ALIGNMENT, "attention backward: grad_scores needs a 16-byte aligned buffer and a row pitch "
                "that is a multiple of 8 of at least the padded key count");
  const void* values = x.value ? x.value : x.value_t;
  // grad_scores replaces grad_query.
  const void* dq = x.grad_scores ? x.grad_scores : static_cast<const void*>(x.grad_query);
  const void* ptrs[] = {x.query, x.key, values, x.out, x.grad_out, x.scales, x.workspace, dq,
                        x.grad_key, x.grad_value, x.grad_scales};
  for (const void* ptr : ptrs)
    if (!ptr) return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: null pointer");
  const void* halves[] = {x.query, x.key, values, x.out, x.grad_out};
  for (const void* ptr : halves)
    if (!aligned(ptr, 16)) return fail(DA_ERR_ALIGNMENT, "attention backward: half-precision tensors must be 16-byte aligned");
  const void* f32[] = {dq, x.grad_key, x.grad_value};
  for (const void* ptr : f32)
    if (!aligned(ptr, 16)) return fail(DA_ERR_ALIGNMENT, "attention backward: gradients must be 16-byte aligned");
  if (!aligned(x.scales, x.scales_dtype == DA_F32 ? 4 : 2) || !aligned(x.grad_scales, 4) ||
      !aligned(x.grad_value_sum, 4))
    return fail(DA_ERR_ALIGNMENT, "attention backward: scales must be aligned to their element size");
  if (!aligned(x.workspace, 256)) return fail(DA_ERR_ALIGNMENT, "attention backward: workspace must be 256-byte aligned");
  const int64_t need =
      da_attention_backward_workspace_bytes(batch, maps, length, key_length, x.score_dim, x.value_dim);
  if (x.workspace_bytes < need)
    return fail(DA_ERR_WORKSPACE, "attention backward: workspace of %lld bytes < %lld required",
                (long long)x.workspace_bytes, (long long)need);
  da::AttentionBwdArgs a;
  a.q = x.query;
  a.k = x.key;
  a.q_stride_b = x.query_stride_b;
  a.q_stride_t = x.query_stride_t;
  a.q_map_stride = x.query_map_stride;
  a.k_stride_b = x.key_stride_b;
  a.k_stride_t = x.key_stride_t;
  a.k_map_stride = x.key_map_stride;
  a.map_repeat = static_cast<int>(x.map_repeat);
  a.v = x.value;
  a.vt = x.value ? nullptr : x.value_t;
  a.vt_stride_b = x.value_t_stride_b;
  a.vt_dtype = x.value_t_dtype;
  a.out = x.out;
  a.out_dtype = x.out_dtype;
  a.dout = x.grad_out;
  a.scales = x.scales;
  a.scales_dtype = x.scales_dtype;
  a.scales_log = (flags & DA_ATTN_SCALES_ARE_LOG) != 0;
  a.log_lo = x.log_min;
  a.log_hi = x.log_max;
  a.scale_mult = x.scale_mult;
  a.dq = x.grad_query;
  a.dk = x.grad_key;
  a.dv = x.grad_value;
  a.dv_sum = x.grad_value_sum;
  a.ds_out = x.grad_scores;
  a.ds_ld = x.grad_scores_ld;
  a.dgamma = x.grad_scales;
  a.B = static_cast<int>(batch);
  a.S = static_cast<int>(maps);
  a.T = static_cast<int>(length);
  a.Tk = static_cast<int>(key_length);
  a.RP = static_cast<int>(x.score_dim);
  a.D = static_cast<int>(x.value_dim);
  a.causal = (flags & DA_ATTN_CAUSAL) != 0;
  a.qk_dtype = qk_dtype;
  a.v_dtype = v_dtype;
  da::launch_routed_attention_backward(a, x.workspace, reinterpret_cast<hipStream_t>(stream));
  return check_launch("attention backward");
}

int da_routed_attention_backward(const void* query, const void* key, const void* value, const void* out,
                                 const void* grad_out, const float* scales, int64_t batch, int64_t maps,
                                 int64_t length, int64_t key_length, int64_t score_dim, int64_t value_dim,
                                 int flags, int qk_dtype, int v_dtype, void* workspace, int64_t workspace_bytes,
                                 float* grad_query, float* grad_key, float* grad_value, float* grad_scales,
                                 da_stream_t stream) {
  // Contiguous [batch*maps, length, score_dim] rows, value rows and fp32 scales.
  if (flags & ~(DA_ATTN_CAUSAL | DA_ATTN_OUT_F32))
    return fail(DA_ERR_INVALID_ARGUMENT, "attention backward: unknown flag bits 0x%x", flags);
  da_attention_backward_args x{};
  x.query = query;
  x.query_stride_t = score_dim;
  x.query_map_stride = length * score_dim;
  x.query_stride_b = maps * length * score_dim;
  x.key = key;
  x.key_stride_t = score_dim;
  x.key_map_stride = key_length * score_dim;
  x.key_stride_b = maps * key_length * score_dim;
  x.map_repeat = 1;
  x.value = value;
  x.out = out;
  x.out_dtype = (flags & DA_ATTN_OUT_F32) ? DA_F32 : v_dtype;
  x.grad_out = grad_out;
  x.scales = scales;
  x.scales_dtype = DA_F32;
  x.scale_mult = 1.f;
  x.batch = batch;
  x.maps = maps;
  x.length = length;
  x.key_length = key_length;
  x.score_dim = score_dim;
  x.value_dim = value_dim;
  x.flags = flags & DA_ATTN_CAUSAL;
  x.qk_dtype = qk_dtype;
  x.v_dtype = v_dtype;
  x.workspace = workspace;
  x.workspace_bytes = workspace_bytes;
  x.grad_query = grad_query;
  x.grad_key = grad_key;
  x.grad_value = grad_value;
  x.grad_scales = grad_scales;
  return da_routed_attention_backward_ex(&x, stream);
}

static int validate_gemm_common(const char* what, const void* x, int64_t rows, int64_t K, int dtype) {
  if (!half_dtype(dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "%s: dtype must be DA_F16 or DA_BF16", what);
  if (rows < 0 || K < 32 || K % 32) return fail(DA_ERR_UNSUPPORTED, "%s: in_features must be a positive multiple of 32", what);
  if (!x || !aligned(x, 16)) return fail(DA_ERR_ALIGNMENT, "%s: input must be non-null and 16-byte aligned", what);
  return DA_OK;
}

int da_qkv_projection(const void* x, int64_t tokens, int64_t model_dim, int64_t length,
                      const void* wq, const void* wk, int64_t qk_width, const void* wv,
                      const void* bv, int64_t value_dim, int bias_dtype, int dtype, void* qk_out,
                      void* value_t, int64_t vt_stride_b, int64_t vt_pitch, da_stream_t stream) {
  int rc = validate_gemm_common("projection", x, tokens, model_dim, dtype);
  if (rc) return rc;
  if (length < 1 || tokens % length) return fail(DA_ERR_INVALID_ARGUMENT, "projection: tokens must be a multiple of length");
  if (qk_width < 8 || qk_width % 8 || value_dim < 4 || value_dim % 4)
    return fail(DA_ERR_UNSUPPORTED, "projection: qk_width must be a multiple of 8 and value_dim of 4");
  if (!wq || !wk || !wv || !qk_out || !value_t) return fail(DA_ERR_INVALID_ARGUMENT, "projection: null pointer");
  if (!aligned(wq, 16) || !aligned(wk, 16) || !aligned(wv, 16) || !aligned(qk_out, 16) || !aligned(value_t, 16))
    return fail(DA_ERR_ALIGNMENT, "projection: tensors must be 16-byte aligned");
  if (bv && !any_dtype(bias_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "projection: bad bias dtype");
  if (vt_pitch < length || vt_pitch % da::kKeyPad || vt_stride_b < value_dim * vt_pitch || vt_stride_b % 8)
    return fail(DA_ERR_ALIGNMENT, "projection: vt_pitch must be a multiple of 64 and >= length");
  da::GemmSegment segs[2];
  segs[0] = da::GemmSegment{wq, wk, qk_width, x, 2 * qk_width, tokens, model_dim, nullptr, 0, 0,
                            qk_out, 2 * qk_width, 0, 0, 0};
  segs[1] = da::GemmSegment{x, nullptr, 0, wv, tokens, value_dim, model_dim, bv, bias_dtype, 1,
                            value_t, 0, length, vt_pitch, vt_stride_b};
  da::launch_gemm(segs, 2, dtype, reinterpret_cast<hipStream_t>(stream));
  return check_launch("projection");
}

int da_linear(const void* x, int64_t rows, int64_t in_features, const void* weight,
              int64_t out_features, const void* bias, int bias_dtype, int dtype, void* out,
              da_stream_t stream) {
  int rc = validate_gemm_common("linear", x, rows, in_features, dtype);
  if (rc) return rc;
  if (out_features < 4 || out_features % 4) return fail(DA_ERR_UNSUPPORTED, "linear: out_features must be a multiple of 4");
  if (!weight || !out || !aligned(weight, 16) || !aligned(out, 8))
    return fail(DA_ERR_ALIGNMENT, "linear: weight/out must be non-null and aligned");
  if (bias && !any_dtype(bias_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "linear: bad bias dtype");
  da::GemmSegment seg{weight, nullptr, 0, x, out_features, rows, in_features, bias, bias_dtype, 0,
                      out, out_features, 0, 0, 0};
  da::launch_gemm(&seg, 1, dtype, reinterpret_cast<hipStream_t>(stream));
  return check_launch("linear");
}

int da_linear_ex(const void* x, int64_t rows, int64_t in_features, const void* weight, int64_t out_features,
                 const void* bias, int bias_dtype, int dtype, int activation, const void* residual, void* out,
                 da_stream_t stream) {
  if (activation != DA_ACT_NONE && activation != DA_ACT_GELU)
    return fail(DA_ERR_INVALID_ARGUMENT, "linear: unknown activation %d", activation);
  if (residual && !aligned(residual, 8)) return fail(DA_ERR_ALIGNMENT, "linear: residual must be 8-byte aligned");
  int rc = validate_gemm_common("linear", x, rows, in_features, dtype);
  if (rc) return rc;
  if (out_features < 4 || out_features % 4) return fail(DA_ERR_UNSUPPORTED, "linear: out_features must be a multiple of 4");
  if (!weight || !out || !aligned(weight, 16) || !aligned(out, 8))
    return fail(DA_ERR_ALIGNMENT, "linear: weight/out must be non-null and aligned");
  if (bias && !any_dtype(bias_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "linear: bad bias dtype");
  da::GemmSegment seg{weight, nullptr, 0, x, out_features, rows, in_features, bias, bias_dtype, 0,
                      out, out_features, 0, 0, 0, activation == DA_ACT_GELU ? da::kGemmActGelu : da::kGemmActNone,
                      residual};
  da::launch_gemm(&seg, 1, dtype, reinterpret_cast<hipStream_t>(stream));
  return check_launch("linear");
}

int da_layer_norm(const void* x, int64_t rows, int64_t dim, const void* weight, const void* bias, int param_dtype,
                  float eps, int dtype, void* out, da_stream_t stream) {
  if (!half_dtype(dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm: dtype must be DA_F16 or DA_BF16");
  if ((weight || bias) && !any_dtype(param_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm: bad parameter dtype");
  if (rows < 0 || dim < 8 || dim % 8 || dim > 4096)
    return fail(DA_ERR_UNSUPPORTED, "layer_norm: dim must be a multiple of 8 in [8, 4096]");
  if (rows == 0) return ok();
  if (!x || !out || !aligned(x, 16) || !aligned(out, 16) || !aligned(weight, 16) || !aligned(bias, 16))
    return fail(DA_ERR_ALIGNMENT, "layer_norm: x, out, weight and bias must be 16-byte aligned");
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm: bad eps");
  da::launch_layer_norm(x, rows, static_cast<int>(dim), weight, bias, param_dtype, eps, dtype, out,
                        reinterpret_cast<hipStream_t>(stream));
  return check_launch("layer_norm");
}

namespace {

int validate_map_combine(const char* what, const float* maps, int64_t batch, int64_t n_maps, int64_t length,
                         int64_t width, const float* weights, int dtype) {
  if (!half_dtype(dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "%s: dtype must be DA_F16 or DA_BF16", what);
  if (batch < 0 || length < 0 || n_maps < 1 || n_maps > da::kMapCombineMaxMaps)
    return fail(DA_ERR_UNSUPPORTED, "%s: maps must be in [1, %d] and sizes >= 0", what, da::kMapCombineMaxMaps);
  if (width < 8 || width % 8 || width > (1 << 20))
    return fail(DA_ERR_UNSUPPORTED, "%s: width must be a positive multiple of 8", what);
  if (!maps || !weights) return fail(DA_ERR_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned(maps, 16)) return fail(DA_ERR_ALIGNMENT, "%s: the map outputs must be 16-byte aligned", what);
  return 0;
}

}  // namespace

int da_map_combine(const float* maps, int64_t batch, int64_t n_maps, int64_t length, int64_t width,
                   const float* weights, void* out, int out_dtype, da_stream_t stream) {
  int rc = validate_map_combine("map combine", maps, batch, n_maps, length, width, weights, out_dtype);
  if (rc) return rc;
  if (batch * length == 0) return ok();
  if (!out) return fail(DA_ERR_INVALID_ARGUMENT, "map combine: null pointer");
  if (!aligned(out, 16)) return fail(DA_ERR_ALIGNMENT, "map combine: out must be 16-byte aligned");
  const da::MapCombineArgs a{maps, weights, batch * length, length, static_cast<int>(n_maps), static_cast<int>(width),
                             out_dtype, out, nullptr, nullptr, nullptr};
  da::launch_map_combine(a, false, reinterpret_cast<hipStream_t>(stream));
  return check_launch("map combine");
}

int da_map_combine_backward(const float* maps, int64_t batch, int64_t n_maps, int64_t length, int64_t width,
                            const float* weights, const void* grad, int grad_dtype, void* grad_maps,
                            float* weight_sums, da_stream_t stream) {
  int rc = validate_map_combine("map combine backward", maps, batch, n_maps, length, width, weights, grad_dtype);
  if (rc) return rc;
  if (batch * length == 0) return ok();
  if (!grad || !grad_maps || !weight_sums) return fail(DA_ERR_INVALID_ARGUMENT, "map combine backward: null pointer");
  if (!aligned(grad, 16) || !aligned(grad_maps, 16))
    return fail(DA_ERR_ALIGNMENT, "map combine backward: grad and grad_maps must be 16-byte aligned");
  const da::MapCombineArgs a{maps, weights, batch * length, length, static_cast<int>(n_maps), static_cast<int>(width),
                             grad_dtype, nullptr, grad, grad_maps, weight_sums};
  da::launch_map_combine(a, true, reinterpret_cast<hipStream_t>(stream));
  return check_launch("map combine backward");
}

int da_dense_attention_operands(const void* query, const void* key, int64_t stride_b, int64_t stride_t,
                                int64_t map_stride, int64_t map_repeat, int qk_dtype, int64_t batch, int64_t maps,
                                int64_t length, int64_t score_dim, void* key_t, void* query_out, void* key_out,
                                int out_dtype, da_stream_t stream) {
  if (!half_dtype(qk_dtype) || !half_dtype(out_dtype))
    return fail(DA_ERR_INVALID_ARGUMENT, "dense operands: dtypes must be DA_F16 or DA_BF16");
  if (batch < 0 || maps < 1 || maps > 65535 || length < 0 || batch * maps > 65535 || map_repeat < 1)
    return fail(DA_ERR_INVALID_ARGUMENT, "dense operands: bad batch, maps, length or map_repeat");
  if (score_dim < 64 || score_dim % 64 || score_dim > 4096)
    return fail(DA_ERR_UNSUPPORTED, "dense operands: score_dim must be a multiple of 64 up to 4096");
  if (batch == 0 || length == 0) return ok();
  if (!query || !key || !key_t || !query_out || !key_out)
    return fail(DA_ERR_INVALID_ARGUMENT, "dense operands: null pointer");
  if (stride_b % 8 || stride_t % 8 || map_stride % 8 || stride_t < score_dim || !aligned(query, 16) ||
      !aligned(key, 16) || !aligned(key_t, 16) || !aligned(query_out, 16) || !aligned(key_out, 16))
    return fail(DA_ERR_ALIGNMENT, "dense operands: strides must be multiples of 8 (stride_t >= score_dim), "
                "pointers 16-byte aligned");
  const da::DenseOperandArgs a{query, key, stride_b, stride_t, map_stride, static_cast<int>(map_repeat), qk_dtype,
                               static_cast<int>(batch), static_cast<int>(maps), static_cast<int>(length),
                               static_cast<int>(score_dim), key_t, query_out, key_out, out_dtype};
  da::launch_dense_operands(a, reinterpret_cast<hipStream_t>(stream));
  return check_launch("dense operands");
}

int da_sum_partials(const float* partials, int64_t count, int64_t n, void* out, int out_dtype, da_stream_t stream) {
  if (!half_dtype(out_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "sum partials: out_dtype must be DA_F16 or DA_BF16");
  if (count < 1 || count > 1024 || n < 0 || n % 8)
    return fail(DA_ERR_UNSUPPORTED, "sum partials: count must be in [1, 1024] and n a multiple of 8");
  if (n == 0) return ok();
  if (!partials || !out) return fail(DA_ERR_INVALID_ARGUMENT, "sum partials: null pointer");
  if (!aligned(partials, 16) || !aligned(out, 16))
    return fail(DA_ERR_ALIGNMENT, "sum partials: partials and out must be 16-byte aligned");
  da::launch_sum_partials(partials, static_cast<int>(count), n, out, out_dtype, reinterpret_cast<hipStream_t>(stream));
  return check_launch("sum partials");
}

int da_layer_norm_backward(const void* x, const void* grad, int64_t rows, int64_t dim, const void* weight,
                           int param_dtype, float eps, int dtype, void* grad_x, float* grad_params, da_stream_t stream) {
  if (!half_dtype(dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm backward: dtype must be DA_F16 or DA_BF16");
  if (weight && !any_dtype(param_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm backward: bad parameter dtype");
  if (rows < 0 || dim < 8 || dim % 8 || dim > 4096)
    return fail(DA_ERR_UNSUPPORTED, "layer_norm backward: dim must be a multiple of 8 in [8, 4096]");
  if (rows == 0) return ok();
  if (!x || !grad || !grad_x || !grad_params) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm backward: null pointer");
  if (!aligned(x, 16) || !aligned(grad, 16) || !aligned(grad_x, 16) || !aligned(weight, 16))
    return fail(DA_ERR_ALIGNMENT, "layer_norm backward: x, grad, grad_x and weight must be 16-byte aligned");
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(DA_ERR_INVALID_ARGUMENT, "layer_norm backward: bad eps");
  da::launch_layer_norm_backward(x, grad, rows, static_cast<int>(dim), weight, param_dtype, eps, dtype, grad_x,
                                 grad_params, reinterpret_cast<hipStream_t>(stream));
  return check_launch("layer_norm backward");
}

int64_t da_sda_workspace_offset(int64_t batch, int64_t length, int64_t model_dim, int64_t qk_width,
                                int which) {
  const int64_t tokens = batch * length;
  const int64_t routed = align_up(tokens * 2 * qk_width * 2);
  const int64_t vt = align_up(batch * model_dim * da::round_up(length, da::kKeyPad) * 2);
  if (which <= 0) return 0;
  if (which == 1) return routed;
  return routed + vt;
}

// Split-key partials of the outer attention (one map only: then the score
// width equals qk_width); the larger of the causal and non-causal plans.
static int64_t attention_partial_bytes(int64_t batch, int64_t length, int64_t model_dim, int64_t qk_width,
                                       int64_t outer_maps) {
  if (outer_maps != 1) return 0;
  const da::AttnPlan causal = da::plan_attention(batch, 1, length, model_dim, qk_width, false, true, true, 2);
  const da::AttnPlan full = da::plan_attention(batch, 1, length, model_dim, qk_width, false, false, true, 2);
  return align_up(std::max(causal.part_bytes, full.part_bytes));
}

int64_t da_sda_workspace_bytes(int64_t batch, int64_t length, int64_t model_dim, int64_t qk_width,
                               int64_t outer_maps, int concat, int has_output_projection) {
  const int64_t tokens = batch * length;
  const int64_t mixed =
      has_output_projection ? align_up(tokens * (concat ? outer_maps : 1) * model_dim * 2) : 0;
  return da_sda_workspace_offset(batch, length, model_dim, qk_width, 2) + mixed +
         attention_partial_bytes(batch, length, model_dim, qk_width, outer_maps);
}

int da_shared_dictionary_attention_forward(const da_sda_forward_args* a, da_stream_t stream) {
  if (!a) return fail(DA_ERR_INVALID_ARGUMENT, "forward: null args");
  const int64_t B = a->batch, T = a->length, d = a->model_dim;
  const int64_t H = a->qk_branches, S = a->outer_maps, R = a->routing_dim;
  if (B < 1 || T < 1 || d < 1 || H < 1 || S < 1 || R < 1 || a->atoms < 1)
    return fail(DA_ERR_INVALID_ARGUMENT, "forward: sizes must be positive");
  if ((H > S ? H % S : S % H) != 0) return fail(DA_ERR_INVALID_ARGUMENT, "forward: branches and maps must divide one another");
  if (S > 64) return fail(DA_ERR_UNSUPPORTED, "forward: at most 64 maps (got %lld)", (long long)S);
  if (!half_dtype(a->dtype) || !any_dtype(a->param_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "forward: bad dtype");
  if (!a->x || !a->wq || !a->wk || !a->wv || !a->key_t || !a->value || !a->log_beta ||
      !a->log_score_scales || !a->out || !a->workspace)
    return fail(DA_ERR_INVALID_ARGUMENT, "forward: null pointer");
  const bool concat = a->flags & DA_SDA_CONCAT;
  if (concat && !a->wo) return fail(DA_ERR_INVALID_ARGUMENT, "forward: concat combine needs an output projection");
  if (!aligned(a->workspace, 256)) return fail(DA_ERR_ALIGNMENT, "forward: workspace must be 256-byte aligned");
  const int64_t need = da_sda_workspace_bytes(B, T, d, H * R, S, concat, a->wo != nullptr);
  if (a->workspace_bytes < need)
    return fail(DA_ERR_WORKSPACE, "forward: workspace of %lld bytes < %lld required",
                (long long)a->workspace_bytes, (long long)need);
  const int64_t W = H * R;
  const int64_t group = H > S ? H / S : 1;
  const int64_t RP = group * R;
  const int64_t Tp = da::round_up(T, da::kKeyPad);
  char* ws = static_cast<char*>(a->workspace);
  void* routed = ws;
  void* vt = ws + da_sda_workspace_offset(B, T, d, W, 1);
  void* mixed = a->wo ? ws + da_sda_workspace_offset(B, T, d, W, 2) : a->out;
  const int64_t mixed_bytes = a->wo ? align_up(B * T * (concat ? S : 1) * d * 2) : 0;
  void* partials = attention_partial_bytes(B, T, d, W, S) > 0
                       ? ws + da_sda_workspace_offset(B, T, d, W, 2) + mixed_bytes
                       : nullptr;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  // Validate every stage before enqueueing the first one.
  int rc = validate_gemm_common("forward/projection", a->x, B * T, d, a->dtype);
  if (rc) return rc;
  if (W % 8) return fail(DA_ERR_UNSUPPORTED, "forward: qk width must be a multiple of 8");
  const bool norm_in = a->flags & DA_SDA_NORMALIZE_INPUT;
  const int key_dtype = norm_in ? DA_F16 : a->dtype;
  // Unit key atoms bound every logit by |beta| (fixed-reference softmax); that
  // holds only for a bank this call normalizes or one the caller says came
  // from da_dictionary_normalize.  Any other bank takes the online softmax.
  if (a->flags & ~(DA_SDA_NORMALIZE_INPUT | DA_SDA_NORMALIZE_OUTPUT | DA_SDA_CAUSAL | DA_SDA_CONCAT | DA_SDA_UNIT_KEYS))
    return fail(DA_ERR_INVALID_ARGUMENT, "forward: unknown flag bits 0x%x", a->flags);
  int rflags = da::kRouteBetaIsLog;
  if (a->raw_key || (a->flags & DA_SDA_UNIT_KEYS)) rflags |= da::kRouteUnitKeys;
  if (norm_in) rflags |= da::kRouteNormalizeInput;
  if (a->flags & DA_SDA_NORMALIZE_OUTPUT) rflags |= da::kRouteNormalizeOutput;
  if (a->route_variant & ~kRouteVariantMask)
    return fail(DA_ERR_INVALID_ARGUMENT, "forward: route_variant holds bits other than DA_ROUTE_SILU_LOGITS, "
                "DA_ROUTE_STANDARDIZE and DA_ROUTE_DIRECT_SILU");
  rflags |= a->route_variant;
  rc = validate_route(routed, B * T * 2 * H, R, R, a->dtype, a->key_t, key_dtype, a->value, a->atoms,
                      a->log_beta, a->param_dtype, rflags, a->silu_gain, a->logit_scale, routed, R, DA_F16);
  if (rc) return rc;
  const int64_t ot = concat ? S * d : d;
  rc = validate_attention(routed, static_cast<char*>(routed) + W * 2, T * 2 * W, 2 * W,
                          H > S ? RP : R, 1, RP, vt, d * Tp, B, S, T, d, a->log_score_scales,
                          a->param_dtype, a->map_mix_logits, a->param_dtype, DA_F16, a->dtype,
                          mixed, T * ot, ot, concat ? d : 0);
  if (rc) return rc;
  if (a->wo) {
    rc = validate_gemm_common("forward/output", mixed, B * T, ot, a->dtype);
    if (rc) return rc;
    if (d % 4) return fail(DA_ERR_UNSUPPORTED, "forward: model_dim must be a multiple of 4");
  }
  if (a->residual && (!a->wo || !aligned(a->residual, 16)))
    return fail(DA_ERR_UNSUPPORTED, "forward: a residual needs the output projection and 16-byte alignment");
  if (!aligned(a->wq, 16) || !aligned(a->wk, 16) || !aligned(a->wv, 16) || (a->wo && !aligned(a->wo, 16)) ||
      !aligned(a->out, 16))
    return fail(DA_ERR_ALIGNMENT, "forward: weights and output must be 16-byte aligned");
  // The bank's normalization, when asked for, rides in the projection launch.
  da::NormJob norm{};
  if (a->raw_key) {
    if (!any_dtype(a->raw_dtype)) return fail(DA_ERR_INVALID_ARGUMENT, "forward: bad raw bank dtype");
    if (!pow2_width(R)) return fail(DA_ERR_UNSUPPORTED, "forward: routing_dim %lld not in {64,128,256,512}", (long long)R);
    if (a->atoms > (1 << 24)) return fail(DA_ERR_INVALID_ARGUMENT, "forward: bad atom count");
    if (!aligned(a->key_t, 16) || !aligned(a->value, 16))
      return fail(DA_ERR_ALIGNMENT, "forward: bank layouts must be 16-byte aligned");
    norm = da::NormJob{a->raw_key, a->raw_value, a->raw_dtype, static_cast<int>(R), static_cast<int>(a->atoms),
                       static_cast<int>(da::round_up(a->atoms, da::kAtomPad)), a->eps, const_cast<void*>(a->key_t),
                       key_dtype, const_cast<void*>(a->value), nullptr};
  }

  // 1. Q/K projections (route rows) and V^T with bias.
  da::GemmSegment proj[2];
  proj[0] = da::GemmSegment{a->wq, a->wk, W, a->x, 2 * W, B * T, d, nullptr, 0, 0, routed, 2 * W, 0, 0, 0};
  proj[1] = da::GemmSegment{a->x, nullptr, 0, a->wv, B * T, d, d, a->bv, a->param_dtype, 1, vt, 0, T, Tp, d * Tp};
  da::launch_gemm(proj, 2, a->dtype, s, a->raw_key ? &norm : nullptr);
  // 2. Route all Q and K rows in place: [tokens, 2, H, R] is [tokens*2H, R].
  //    The routed rows are written as fp16 (unit vectors, or convex
  //    combinations of unit atoms without output normalization).
  da::RouteArgs ra{routed, B * T * 2 * H, R, a->dtype, static_cast<int>(R), a->key_t, key_dtype,
                   a->value, static_cast<int>(a->atoms), a->log_beta, a->param_dtype, 0.f, a->eps,
                   rflags, a->silu_gain, a->logit_scale, routed, R, DA_F16};
  da::launch_dictionary_route(ra, s);
  // 3. Outer attention over the S maps, mixed (or concatenated).
  da::AttentionArgs at;
  at.q = routed;
  at.k = static_cast<char*>(routed) + W * 2;
  at.qk_stride_b = T * 2 * W;
  at.qk_stride_t = 2 * W;
  at.map_stride = H > S ? RP : R;
  at.map_repeat = static_cast<int>(S > H ? S / H : 1);
  at.RP = static_cast<int>(RP);
  at.vt = vt;
  at.vt_stride_b = d * Tp;
  at.B = static_cast<int>(B);
  at.S = static_cast<int>(S);
  at.T = static_cast<int>(T);
  at.D = static_cast<int>(d);
  at.scales = a->log_score_scales;
  at.scales_dtype = a->param_dtype;
  at.scale_mult = group > 1 ? static_cast<float>(1.0 / std::sqrt(static_cast<double>(group))) : 1.f;
  at.mix_logits = a->map_mix_logits;
  at.mix_dtype = a->param_dtype;
  at.flags = da::kAttnScalesAreLog | ((a->flags & DA_SDA_CAUSAL) ? da::kAttnCausal : 0) |
             (concat ? 0 : da::kAttnMix);
  // Output-normalized routed rows are unit vectors (fp16 rounding aside), so a
  // grouped score q'.k' = sum of `group` unit dot products is at most `group`.
  at.score_bound = (a->flags & DA_SDA_NORMALIZE_OUTPUT) ? 1.01f * static_cast<float>(group) : 0.f;
  at.qk_dtype = DA_F16;
  at.v_dtype = a->dtype;
  at.out = mixed;
  at.out_stride_b = T * ot;
  at.out_stride_t = ot;
  at.out_stride_s = concat ? d : 0;
  da::launch_routed_attention(at, partials, s);
  // 4. Output projection.
  if (a->wo) {
    da::GemmSegment o{a->wo, nullptr, 0, mixed, d, B * T, ot, nullptr, 0, 0, a->out, d, 0, 0, 0, da::kGemmActNone,
                      a->residual};
    da::launch_gemm(&o, 1, a->dtype, s);
  }
  return check_launch("forward");
}

}  // extern "C"

// Scratch of the allocation-free forward: one array per GPU, held until the
// process ends.  Host code never passes `scratch` itself to a kernel (on the
// host it names a shadow variable, not device memory): each device's address
// comes from hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) char scratch[DA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch of the device that `stream` launches on (the current device
// for the null stream): each GPU holds its own copy of the array, at its own
// address, which hipGetSymbolAddress returns with that device current.
int scratch_of_stream_device(hipStream_t stream, void** out) {
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return fail(DA_ERR_LAUNCH, "noalloc forward: hipGetDevice: %s", hipGetErrorString(e));
  int dev = current;
  if (stream) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return fail(DA_ERR_LAUNCH, "noalloc forward: hipStreamGetDevice: %s", hipGetErrorString(e));
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(DA_ERR_UNSUPPORTED, "noalloc forward: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    if (dev != current) {
      e = hipSetDevice(dev);
      if (e != hipSuccess) return fail(DA_ERR_LAUNCH, "noalloc forward: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t restore = dev != current ? hipSetDevice(current) : hipSuccess;
    if (e != hipSuccess || !ptr)
      return fail(DA_ERR_LAUNCH, "noalloc forward: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    if (restore != hipSuccess)
      return fail(DA_ERR_LAUNCH, "noalloc forward: hipSetDevice(%d): %s", current, hipGetErrorString(restore));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DA_OK;
}
}  // namespace

extern "C" int da_shared_dictionary_attention_forward_noalloc(const da_sda_forward_args* args, da_stream_t stream) {
  if (!args) return fail(DA_ERR_INVALID_ARGUMENT, "noalloc forward: null args");
  if (args->batch < 1 || args->length < 1 || args->model_dim < 1 || args->qk_branches < 1 || args->routing_dim < 1 ||
      args->outer_maps < 1)
    return fail(DA_ERR_INVALID_ARGUMENT, "noalloc forward: sizes must be positive");
  const int64_t need = da_sda_workspace_bytes(args->batch, args->length, args->model_dim,
                                              args->qk_branches * args->routing_dim, args->outer_maps,
                                              (args->flags & DA_SDA_CONCAT) != 0, args->wo != nullptr);
  if (need > DA_NOALLOC_SCRATCH_BYTES)
    return fail(DA_ERR_WORKSPACE,
                "noalloc forward: the problem needs %lld bytes of scratch, more than the %lld-byte per-GPU array "
                "(use da_shared_dictionary_attention_forward with a workspace)",
                (long long)need, (long long)DA_NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  const int rc = scratch_of_stream_device(reinterpret_cast<hipStream_t>(stream), &ptr);
  if (rc) return rc;
  // Nothing in the workspace needs to start at zero: every byte a kernel
  // reads was written earlier in the same call.
  da_sda_forward_args local = *args;
  local.workspace = ptr;
  local.workspace_bytes = DA_NOALLOC_SCRATCH_BYTES;
  return da_shared_dictionary_attention_forward(&local, stream);
}
