"""Shared-dictionary attention modules with a gfx950 ``backend="hip"`` forward.

The module tree, parameter names, buffer names and construction order follow
the reference (``src/double_attention/modules.py:25-460``): checkpoints load
unchanged, and a seeded construction consumes the RNG in the same order, so
default-initialized weights are identical.  The HIP forward
(``SharedDictionaryAttention._hip_forward``) replaces the projection,
route, outer attention and map combine with one C call into the gfx950
library; LayerNorm, FFN, embeddings and the LM head stay PyTorch ops.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .config import DoubleAttentionConfig
from .ops import (
    assemble_score_maps,
    dictionary_route_reference,
    resolve_backend,
    routed_attention_reference,
    score_scale_from_log,
)

# Reference switch (modules.py:22): one GEMM over cat(Wq, Wk) instead of two.
FUSED_QUERY_KEY_PROJECTION = True


class SharedDictionaryBank(nn.Module):
    """Routing dictionary shared by several attention layers (``modules.py:25-54``).

    ``raw_key`` (and ``raw_value`` when untied) are ``[routing_dim, atoms]``
    and drawn ``N(0, 1/routing_dim)``.  A tied bank registers ``raw_value`` as
    ``None`` and reconstructs with the key atoms.
    """

    def __init__(self, routing_dim: int, dictionary_size: int, *, untied: bool = True) -> None:
        super().__init__()
        self.routing_dim = routing_dim
        self.dictionary_size = dictionary_size
        self.untied = untied
        std = routing_dim ** -0.5
        self.raw_key = nn.Parameter(torch.randn(routing_dim, dictionary_size) * std)
        if untied:
            self.raw_value = nn.Parameter(torch.randn(routing_dim, dictionary_size) * std)
        else:
            self.register_parameter("raw_value", None)

    def normalized(self, eps: float = 1e-6) -> tuple[Tensor, Tensor]:
        """Unit-norm atoms ``(key, value)``; a tied bank returns one tensor twice."""

        key = F.normalize(self.raw_key, dim=0, eps=eps)
        value = key if self.raw_value is None else F.normalize(self.raw_value, dim=0, eps=eps)
        return key, value

    def normalized_hip(self, eps: float = 1e-6, key_dtype: torch.dtype = torch.float16) -> tuple[Tensor, Tensor]:
        """``normalized`` computed by the gfx950 kernel, in the route layouts.

        One launch covers both banks of an untied dictionary.  The returned
        ``[R, M]`` tensors are views that the HIP route reads without a copy
        (key atoms in ``key_dtype``, value atoms in fp16).
        """

        from .hip_ops import dictionary_normalize_hip

        return dictionary_normalize_hip(self.raw_key, self.raw_value, eps, key_dtype)

    def extra_repr(self) -> str:
        return (
            f"routing_dim={self.routing_dim}, dictionary_size={self.dictionary_size}, "
            f"untied={self.untied}"
        )


@dataclass
class DoubleAttentionAux:
    """Intermediate tensors of one forward (``modules.py:57-65``)."""

    routing_query: Tensor
    routing_key: Tensor
    score_query: Tensor
    score_key: Tensor
    score_scales: Tensor
    map_weights: Tensor
    backend: str


class _Spec(NamedTuple):
    is_cuda: bool
    dtype: torch.dtype


def _compute_dtype(x: Tensor, weight: Tensor) -> torch.dtype:
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return weight.dtype if x.dtype == weight.dtype else torch.promote_types(x.dtype, weight.dtype)


def _hip_covers(config: DoubleAttentionConfig) -> bool:
    """Whether the HIP kernels cover this configuration (``backend="auto"``
    takes the torch path for one they do not; ``"hip"`` raises instead)."""

    from . import hip_ops

    try:
        hip_ops.check_module_supported(config)
    except NotImplementedError:
        return False
    return True


class SharedDictionaryAttention(nn.Module):
    """Routing/content-decoupled attention (``modules.py:68-291``).

    ``config.backend`` picks the implementation: ``"torch"`` (the PyTorch
    composition, any shape), ``"hip"`` (the gfx950 kernels; raises
    ``NotImplementedError`` for a configuration they do not cover) or
    ``"auto"`` (the kernels when they cover the call, else torch).  Limits of
    the kernels (``hip_ops.check_module_supported``):

    * ``routing_dim`` in {64, 128, 256, 512}, ``model_dim`` a multiple of 64
      from 64 to 4096 (every preset); a grouped score width
      ``(qk_branches // outer_maps) * routing_dim`` of at most 512; at most 64
      outer maps;
    * ``dictionary_activation`` "identity" or "silu", ``dictionary_assignment``
      "softmax" or "silu"; any number of atoms and rows;
    * 16-bit compute (bf16 or fp16 inputs, or autocast) on a ROCm device.

    Training on ``"hip"`` runs the native backward for every covered forward
    (any bank size); only model widths above 512 whose score matrices do not
    fit the dense attention backward take the outer attention's gradients
    from autograd of the torch composition.
    """

    def __init__(
        self,
        config: DoubleAttentionConfig,
        *,
        bank: SharedDictionaryBank | None = None,
        create_bank: bool = True,
    ) -> None:
        super().__init__()
        self.config = config
        width = config.qk_branches * config.routing_dim
        # Registration order matters: it fixes the default-init RNG stream.
        self.query = nn.Linear(config.model_dim, width, bias=False)
        self.key = nn.Linear(config.model_dim, width, bias=False)
        self.value = nn.Linear(config.model_dim, config.model_dim, bias=config.value_bias)
        if bank is None and create_bank:
            bank = SharedDictionaryBank(
                config.routing_dim, config.dictionary_size, untied=config.untied_dictionary
            )
        self.bank = bank

        log_scale = math.log(config.initial_score_scale)
        if config.outer_maps == 1:
            scales = torch.tensor([log_scale])
        else:
            # A small deterministic spread breaks the symmetry between maps
            # that share one Q/K branch (modules.py:101-105).
            scales = log_scale + torch.linspace(-0.05, 0.05, config.outer_maps)
        self.log_score_scales = nn.Parameter(scales)
        log_beta = torch.tensor(math.log(config.beta))
        if config.learnable_beta:
            self.log_beta = nn.Parameter(log_beta)
        else:
            self.register_buffer("log_beta", log_beta, persistent=True)

        if config.map_combine == "weighted_sum":
            if config.outer_maps > 1:
                self.map_mix_logits = nn.Parameter(torch.zeros(config.outer_maps))
            else:
                self.register_parameter("map_mix_logits", None)
            self.output = (
                nn.Linear(config.model_dim, config.model_dim, bias=False)
                if config.output_projection
                else nn.Identity()
            )
        else:
            self.register_parameter("map_mix_logits", None)
            self.output = nn.Linear(config.outer_maps * config.model_dim, config.model_dim, bias=False)

    @property
    def beta(self) -> Tensor:
        return self.log_beta.clamp(math.log(0.05), math.log(64.0)).exp()

    # ---- PyTorch path -----------------------------------------------------

    def _project_branches(self, projection: nn.Linear, x: Tensor) -> Tensor:
        batch, length, _ = x.shape
        return self._reshape_branches(projection(x), batch, length)

    def _reshape_branches(self, result: Tensor, batch: int, length: int) -> Tensor:
        shaped = result.view(batch, length, self.config.qk_branches, self.config.routing_dim)
        return shaped.permute(0, 2, 1, 3).contiguous()

    def _project_query_key(self, x: Tensor) -> tuple[Tensor, Tensor]:
        if not FUSED_QUERY_KEY_PROJECTION:
            return self._project_branches(self.query, x), self._project_branches(self.key, x)
        batch, length, _ = x.shape
        fused = F.linear(x, torch.cat((self.query.weight, self.key.weight), dim=0))
        query, key = fused.split(self.config.total_qk_width, dim=-1)
        return self._reshape_branches(query, batch, length), self._reshape_branches(key, batch, length)

    def _route(self, x: Tensor, dictionary_key: Tensor, dictionary_value: Tensor) -> Tensor:
        cfg = self.config
        return dictionary_route_reference(
            x, dictionary_key, dictionary_value, self.beta, cfg.eps,
            cfg.dictionary_activation, cfg.dictionary_assignment, cfg.dictionary_silu_gain,
            cfg.standardize_dictionary_logits, cfg.standardized_logit_scale,
            cfg.normalize_routing_input, cfg.normalize_routing_output,
        )

    def _combine(self, x: Tensor, map_output: Tensor) -> tuple[Tensor, Tensor]:
        if self.config.map_combine == "weighted_sum":
            if self.map_mix_logits is None:
                return self.output(map_output[:, 0]), x.new_ones(1)
            weights = torch.softmax(self.map_mix_logits, dim=0).to(map_output.dtype)
            factors = weights.float()
            # The weighted map sum in fp32, rounded once (as einsum's fp32
            # accumulation does), without einsum's internal transposed bmm.
            combined = (map_output.float() * factors[None, :, None, None]).sum(1).to(map_output.dtype)
            return self.output(combined), weights
        weights = x.new_full((self.config.outer_maps,), 1.0 / self.config.outer_maps)
        return self.output(map_output.permute(0, 2, 1, 3).flatten(2)), weights

    def _torch_forward(
        self,
        x: Tensor,
        dictionary_key: Tensor,
        dictionary_value: Tensor,
        return_aux: bool,
    ) -> Tensor | tuple[Tensor, DoubleAttentionAux]:
        query, key = self._project_query_key(x)
        dense_value = self.value(x)
        # Under AMP the masters stay fp32 while projections are fp16/bf16;
        # route in the projection dtype (modules.py:226-231).
        if dictionary_key.dtype != query.dtype:
            dictionary_key = dictionary_key.to(query.dtype)
            dictionary_value = dictionary_value.to(query.dtype)
        # Q and K tokens route together, as one batch of rows (modules.py:236-241).
        pair = torch.cat((query, key), dim=2)
        routed = self._route(pair, dictionary_key, dictionary_value)
        routed_query, routed_key = routed.split(x.shape[1], dim=2)
        score_query, score_key = assemble_score_maps(routed_query, routed_key, self.config.outer_maps)
        scales = score_scale_from_log(self.log_score_scales)
        map_output = routed_attention_reference(score_query, score_key, dense_value, scales, self.config.causal)
        output, weights = self._combine(x, map_output)
        if not return_aux:
            return output
        return output, DoubleAttentionAux(
            routing_query=routed_query,
            routing_key=routed_key,
            score_query=score_query,
            score_key=score_key,
            score_scales=scales,
            map_weights=weights,
            backend="torch",
        )

    # ---- HIP path ---------------------------------------------------------

    def _hip_forward(
        self,
        x: Tensor,
        bank: SharedDictionaryBank,
        normalized_dictionary: tuple[Tensor, Tensor] | None,
        dtype: torch.dtype,
        return_aux: bool,
    ) -> Tensor | tuple[Tensor, DoubleAttentionAux]:
        from . import hip_ops

        hip_ops.check_module_supported(self.config)
        needs_grad = torch.is_grad_enabled() and (
            x.requires_grad or any(p.requires_grad for p in self.parameters())
            or (normalized_dictionary is not None and any(t.requires_grad for t in normalized_dictionary))
            or any(p.requires_grad for p in bank.parameters())
        )
        if needs_grad:
            return _HipModuleFunction.run(self, x, bank, normalized_dictionary, dtype, return_aux)
        result = self._hip_call(x, bank, normalized_dictionary, dtype, want_routed=return_aux)
        if not return_aux:
            return result.output
        return result.output, self._hip_aux(result.routed, dtype)

    def _hip_call(
        self,
        x: Tensor,
        bank: SharedDictionaryBank,
        normalized_dictionary: tuple[Tensor, Tensor] | None,
        dtype: torch.dtype,
        residual: Tensor | None = None,
        want_routed: bool = True,
    ):
        """The fused forward (no autograd); ``residual`` is added to its output.
        ``want_routed`` False skips the routed-rows view (only the output is used)."""

        from . import hip_ops

        key_dtype = hip_ops.route_key_dtype(self.config.normalize_routing_input, dtype)
        if normalized_dictionary is None:
            # The forward normalizes its own bank inside its projection launch.
            layout = hip_ops.own_bank_layout(bank, key_dtype)
            return hip_ops.shared_dictionary_attention_hip(
                self, x, layout, dtype, raw_bank=(bank.raw_key, bank.raw_value), residual=residual,
                want_routed=want_routed,
            )
        layout = hip_ops.route_layout(*normalized_dictionary, key_dtype)
        return hip_ops.shared_dictionary_attention_hip(self, x, layout, dtype, residual=residual,
                                                       want_routed=want_routed)

    def _hip_inference_dtype(self, x: Tensor, bank: SharedDictionaryBank) -> torch.dtype | None:
        """The compute dtype when a forward of ``x`` would run the HIP kernels
        without autograd (else None)."""

        cfg = self.config
        if cfg.backend == "torch" or x.ndim != 3 or x.shape[-1] != cfg.model_dim:
            return None
        dtype = _compute_dtype(x, self.query.weight)
        if resolve_backend(cfg.backend, (_Spec(x.is_cuda, dtype),)) != "hip":  # type: ignore[arg-type]
            return None
        if cfg.backend == "auto" and not _hip_covers(cfg):
            return None
        if torch.is_grad_enabled() and (
            x.requires_grad
            or any(p.requires_grad for p in self.parameters())
            or any(p.requires_grad for p in bank.parameters())
        ):
            return None
        return dtype

    def _hip_aux(self, routed: Tensor, dtype: torch.dtype) -> DoubleAttentionAux:
        # routed: [B, T, 2, H, R] (fp16) -> [B, H, T, R] for queries and keys,
        # in the activation dtype like the PyTorch path's aux tensors.
        routed = routed.to(dtype)
        routed_query = routed[:, :, 0].permute(0, 2, 1, 3)
        routed_key = routed[:, :, 1].permute(0, 2, 1, 3)
        score_query, score_key = assemble_score_maps(routed_query, routed_key, self.config.outer_maps)
        scales = score_scale_from_log(self.log_score_scales)
        if self.config.map_combine == "weighted_sum":
            weights = (
                routed.new_ones(1)
                if self.map_mix_logits is None
                else torch.softmax(self.map_mix_logits, dim=0).to(routed.dtype)
            )
        else:
            weights = routed.new_full((self.config.outer_maps,), 1.0 / self.config.outer_maps)
        return DoubleAttentionAux(
            routing_query=routed_query,
            routing_key=routed_key,
            score_query=score_query,
            score_key=score_key,
            score_scales=scales,
            map_weights=weights,
            backend="hip",
        )

    # ---- entry point -------------------------------------------------------

    def forward(
        self,
        x: Tensor,
        *,
        bank: SharedDictionaryBank | None = None,
        normalized_dictionary: tuple[Tensor, Tensor] | None = None,
        return_aux: bool = False,
    ) -> Tensor | tuple[Tensor, DoubleAttentionAux]:
        cfg = self.config
        if x.ndim != 3 or x.shape[-1] != cfg.model_dim:
            raise ValueError(f"expected x with shape [B, T, {cfg.model_dim}], got {tuple(x.shape)}")
        active = bank if bank is not None else self.bank
        if active is None:
            raise ValueError("no dictionary bank supplied")
        if active.routing_dim != cfg.routing_dim or active.dictionary_size != cfg.dictionary_size:
            raise ValueError("dictionary bank dimensions do not match the attention config")
        if normalized_dictionary is not None:
            expected = (cfg.routing_dim, cfg.dictionary_size)
            if normalized_dictionary[0].shape != expected or normalized_dictionary[1].shape != expected:
                raise ValueError("normalized dictionary dimensions do not match attention config")

        if cfg.backend != "torch":
            dtype = _compute_dtype(x, self.query.weight)
            spec = _Spec(x.is_cuda, dtype)
            if resolve_backend(cfg.backend, (spec,)) == "hip" and (cfg.backend == "hip" or _hip_covers(cfg)):  # type: ignore[arg-type]
                return self._hip_forward(x, active, normalized_dictionary, dtype, return_aux)

        if normalized_dictionary is None:
            dictionary_key, dictionary_value = active.normalized(cfg.eps)
        else:
            dictionary_key, dictionary_value = normalized_dictionary
        return self._torch_forward(x, dictionary_key, dictionary_value, return_aux)


class _HipModuleFunction(torch.autograd.Function):
    """HIP forward and native backward of one ``SharedDictionaryAttention`` call.

    Inputs are ``x``, the normalized dictionary or the raw bank parameters,
    and every module parameter, so autograd routes gradients to all of them.
    With the raw bank (a module's own bank whose route backward is native)
    the forward normalizes it in one launch straight into the route layouts,
    and the backward returns the gradients at the raw atoms through
    ``da_dictionary_normalize_backward``.
    The forward runs the library's stages one launch each (Q/K/V projection,
    route, per-map attention, map combine, output projection) and keeps what
    the backward needs: the pre-route rows, the routed rows, the per-map
    attention outputs, the combined maps and the V^T tiles.  The backward
    then runs no forward again: the output projection's GEMMs, the map
    combine's backward, the native attention backward, the score-map
    assembly's backward, the native route backward and the projection GEMMs
    (reference modules.py:190-291 and its autograd).
    """

    @staticmethod
    def run(module, x, bank, normalized_dictionary, dtype, return_aux):
        from . import hip_ops

        cfg = module.config
        params = [p for p in module.parameters()]
        raw_bank = (
            normalized_dictionary is None
            and x.is_cuda
            and hip_ops.route_backward_is_native(
                cfg.routing_dim, bank.dictionary_size, dtype, hip_ops.RouteVariant.of_config(cfg)
            )
        )
        if raw_bank:
            dictionary = (bank.raw_key, bank.raw_value)
        elif normalized_dictionary is None:
            dictionary = bank.normalized(cfg.eps)
            if dictionary[0] is dictionary[1]:
                dictionary = (dictionary[0], dictionary[0].view_as(dictionary[0]))
        else:
            dictionary = normalized_dictionary
        out = _HipModuleFunction.apply(module, (dtype, raw_bank), x, dictionary[0], dictionary[1], *params)
        if not return_aux:
            return out
        with torch.no_grad():
            key_dtype = hip_ops.route_key_dtype(cfg.normalize_routing_input, dtype)
            if raw_bank:
                layout = hip_ops.own_bank_layout(bank, key_dtype)
                result = hip_ops.shared_dictionary_attention_hip(
                    module, x, layout, dtype, raw_bank=(bank.raw_key, bank.raw_value)
                )
            else:
                layout = hip_ops.route_layout(dictionary[0], dictionary[1], key_dtype)
                result = hip_ops.shared_dictionary_attention_hip(module, x, layout, dtype)
        return out, module._hip_aux(result.routed, dtype)

    @staticmethod
    def forward(ctx, module, spec, x, dictionary_key, dictionary_value, *params):  # type: ignore[override]
        from . import hip_ops

        dtype, raw_bank = spec
        ctx.raw_bank = raw_bank
        raw_key = raw_value = None
        if raw_bank:
            raw_key, raw_value = dictionary_key, dictionary_value
            dictionary_key, dictionary_value = hip_ops.dictionary_normalize_hip(
                raw_key, raw_value, module.config.eps,
                hip_ops.route_key_dtype(module.config.normalize_routing_input, dtype),
            )

        cfg = module.config
        batch, length, model_dim = x.shape
        branches, maps, routing_dim = cfg.qk_branches, cfg.outer_maps, cfg.routing_dim

        def cast(t: Tensor) -> Tensor:
            return hip_ops._aligned(t.detach().to(dtype))

        xc = cast(x)
        qk, vt = hip_ops.qkv_projection_hip(
            xc, cast(module.query.weight), cast(module.key.weight), cast(module.value.weight), module.value.bias
        )
        key_dtype = hip_ops.route_key_dtype(cfg.normalize_routing_input, dtype)
        layout = hip_ops.route_layout(dictionary_key, dictionary_value, key_dtype)
        variant = hip_ops.RouteVariant.of_config(cfg)
        # beta and the score scales are formed from their logs in the kernels
        # (the clamped exponentials of modules.py:130-132 and ops.py:160-161).
        log_beta = module.log_beta.detach()
        # Q and K rows route together, as [B, T, 2, H, R] rows, fp16 out (the
        # attention's operand type for bounded rows).  The route stops before
        # its output norm: the backward needs that reconstruction r, and the
        # norm is one row normalization here.
        recon = hip_ops._route_forward(
            qk.view(-1, routing_dim), layout, log_beta, cfg.eps, cfg.normalize_routing_input, False, variant,
            out_dtype=torch.float16, beta_is_log=True,
        )
        if cfg.normalize_routing_output:
            # F.normalize in fp32, one rounding to fp16.
            routed = hip_ops._row_normalize(recon, cfg.eps, torch.float16)
        else:
            routed = recon
        group = branches // maps if branches > maps else 1
        bound = 1.01 * group if cfg.normalize_routing_output else 0.0
        # fp32 per-map outputs: the combine sums them before one rounding (as
        # the fused forward's in-kernel mix), and the backward's rowsum(dO . O)
        # and map-mix gradient read them unrounded.  The score maps are views
        # of the routed rows (no assembled copies).
        map_output = hip_ops._attention_forward_rows(
            routed.view(batch, length, 2, branches, routing_dim), branches, maps, vt, module.log_score_scales,
            cfg.causal, bound,
        )
        factors = None
        if cfg.map_combine == "weighted_sum":
            if module.map_mix_logits is None:
                mixed = map_output[:, 0].to(dtype)
            else:
                # The weights rounded to the map dtype, the sum in fp32 (as _combine).
                factors = torch.softmax(module.map_mix_logits.detach(), dim=0).to(dtype).float()
                if hip_ops.map_combine_supported(map_output):
                    mixed = hip_ops.map_combine(map_output, factors, dtype)
                else:
                    mixed = (map_output.float() * factors[None, :, None, None]).sum(1).to(dtype)
        else:
            mixed = map_output.permute(0, 2, 1, 3).reshape(batch, length, maps * model_dim).to(dtype)
        mixed = hip_ops._aligned(mixed)
        output_weight = cast(module.output.weight) if isinstance(module.output, nn.Linear) else None
        out = mixed if output_weight is None else hip_ops.linear_hip(mixed, output_weight)
        ctx.module = module
        ctx.dtype = dtype
        ctx.param_names = [name for name, _ in module.named_parameters()]
        ctx.x_dtype = x.dtype
        ctx.save_for_backward(xc, qk, recon, routed, map_output, mixed, vt, log_beta, dictionary_key,
                              dictionary_value, factors if factors is not None else torch.empty(0), raw_key,
                              raw_value, *params)
        return out

    @staticmethod
    def _score_maps(routed: Tensor, batch: int, length: int, branches: int, maps: int, routing_dim: int):
        rows = routed.view(batch, length, 2, branches, routing_dim)
        return assemble_score_maps(rows[:, :, 0].transpose(1, 2), rows[:, :, 1].transpose(1, 2), maps)

    @staticmethod
    def backward(ctx, grad):  # type: ignore[override]
        from . import hip_ops
        from .hip_ops import _mm_tn_f32

        module = ctx.module
        cfg = module.config
        dtype = ctx.dtype
        (xc, qk, recon, routed, map_output, mixed, vt, log_beta, dk, dv, factors, raw_key, raw_value,
         *params) = ctx.saved_tensors
        named = dict(zip(ctx.param_names, params))
        batch, length, model_dim = xc.shape
        branches, maps, routing_dim = cfg.qk_branches, cfg.outer_maps, cfg.routing_dim
        width = branches * routing_dim
        tokens = batch * length
        grads: dict[str, Tensor] = {}

        def wants(name: str) -> bool:
            return name in named and named[name].requires_grad

        # Output projection.
        g = grad.reshape(tokens, -1).to(dtype)
        mixed2d = mixed.reshape(tokens, -1)
        if isinstance(module.output, nn.Linear):
            d_mixed = torch.mm(g, named["output.weight"].detach().to(dtype))
            if wants("output.weight"):
                grads["output.weight"] = _mm_tn_f32(g, mixed2d, named["output.weight"].dtype)
        else:
            d_mixed = g
        # Map combine.
        if cfg.map_combine == "weighted_sum":
            if module.map_mix_logits is None:
                d_maps = d_mixed.view(batch, 1, length, model_dim)
            else:
                # The per-map sums dY . O_s in fp32 throughout: they are large
                # and nearly equal, and the softmax backward differences them
                # (dY enters the fp32 product as its exact fp32 value).
                # alpha_s dY is rounded once (bf16 x bf16 products are exact
                # in fp32).  One pass over the map outputs when the kernel
                # takes them.
                if hip_ops.map_combine_supported(map_output):
                    d_maps, per_map = hip_ops.map_combine_backward(
                        map_output, factors, d_mixed.view(batch, length, model_dim))
                else:
                    per_map = (map_output * d_mixed.view(batch, 1, length, model_dim)).sum(dim=(0, 2, 3))
                    d_maps = d_mixed.view(batch, 1, length, model_dim) * factors.to(dtype).view(1, maps, 1, 1)
                if wants("map_mix_logits"):
                    alpha = torch.softmax(module.map_mix_logits.detach().float(), dim=0)
                    grads["map_mix_logits"] = alpha * (per_map - (alpha * per_map).sum())
        else:
            d_maps = d_mixed.view(batch, length, maps, model_dim).transpose(1, 2)
        # Outer attention.  dq and dk stay fp32 (no rounding, no cast): the
        # route backward takes fp32 gradient rows.
        log_scales = named["log_score_scales"]
        d_value_sums = None
        if hip_ops.rows_backward_supported(batch, length, branches, maps, routing_dim, model_dim):
            # The key-tile kernels read the score maps as views of the routed
            # rows and write their gradients into [B, T, 2, H, R] (the
            # assembly's backward), with the temperature clamp's backward.
            d_rows_qk, d_value, d_log_scales, d_value_sums = hip_ops.attention_gradients_rows(
                routed.view(batch, length, 2, branches, routing_dim), branches, maps, vt, log_scales,
                map_output, d_maps, cfg.causal,
            )
            if wants("log_score_scales"):
                grads["log_score_scales"] = d_log_scales
            d_routed = d_rows_qk.view(-1, routing_dim)
        else:
            score_query, score_key = _HipModuleFunction._score_maps(
                routed, batch, length, branches, maps, routing_dim
            )
            if hip_ops._dense_fits(batch, maps, length, score_query.shape[-1], model_dim):
                # The dense backward lays the V^T tiles out as V^T itself, and
                # its row kernel takes the log temperatures with their clamp
                # (the scale gradient comes back at the logs).
                d_sq, d_sk, d_value, d_log_scales = hip_ops._attention_backward_dense(
                    score_query, score_key, None, log_scales.detach(), d_maps, cfg.causal, torch.float32,
                    value_t=vt, scales_are_log=True,
                )
            else:
                # The temperatures as the forward kernel formed them: fp32
                # exponentials of the clamped logs.
                log32 = log_scales.detach().float()
                scales = log32.clamp(*hip_ops.LOG_SCALE_RANGE).exp()
                padded = vt.shape[1] * 32
                value_rows = vt.transpose(2, 3).reshape(batch, padded, model_dim)[:, :length]
                d_sq, d_sk, d_value, d_scales = hip_ops.attention_gradients(
                    score_query, score_key, value_rows, scales, map_output, d_maps, cfg.causal,
                    qk_grad_dtype=torch.float32,
                )
                # The clamp passes the gradient only inside its window.
                inside = (log32 >= hip_ops.LOG_SCALE_RANGE[0]) & (log32 <= hip_ops.LOG_SCALE_RANGE[1])
                d_log_scales = d_scales.float() * scales * inside
            if wants("log_score_scales"):
                grads["log_score_scales"] = d_log_scales
            # Score-map assembly (views, grouping or repetition of the branches).
            if branches == maps:
                d_rq, d_rk = d_sq, d_sk
            else:
                # The assembly is linear (scales, concatenation, repetition):
                # its backward runs on fp32 copies of the rows, so the fp32
                # dq/dk reach the route backward unrounded.
                with torch.enable_grad():
                    rows = routed.view(batch, length, 2, branches, routing_dim)
                    rq = rows[:, :, 0].transpose(1, 2).detach().float().requires_grad_()
                    rk = rows[:, :, 1].transpose(1, 2).detach().float().requires_grad_()
                    sq, sk = assemble_score_maps(rq, rk, maps)
                    d_rq, d_rk = torch.autograd.grad((sq, sk), (rq, rk), (d_sq.float(), d_sk.float()))
            d_routed = torch.stack((d_rq.transpose(1, 2), d_rk.transpose(1, 2)), dim=2).reshape(-1, routing_dim)
        # Route.
        variant = hip_ops.RouteVariant.of_config(cfg)
        # With the raw bank the gradients at the normalized atoms stay fp32
        # for the normalization's backward; a tied bank's key atoms take both.
        need_key, need_value = ctx.needs_input_grad[3], ctx.needs_input_grad[4]
        if ctx.raw_bank and raw_value is None:
            need_value = need_key
        d_rows, d_key, d_val, d_beta = hip_ops.route_gradients(
            qk.view(-1, routing_dim), dk, dv, log_beta, cfg.eps, cfg.normalize_routing_input,
            cfg.normalize_routing_output, variant, d_routed, (True, need_key, need_value, wants("log_beta")), recon,
            torch.float32 if ctx.raw_bank else None, beta_is_log=True,
        )
        if ctx.raw_bank and (need_key or need_value):
            d_key, d_val = hip_ops.dictionary_normalize_backward_hip(raw_key, raw_value, d_key, d_val, cfg.eps)
            if not ctx.needs_input_grad[3]:
                d_key = None
            if not ctx.needs_input_grad[4]:
                d_val = None
        if wants("log_beta") and d_beta is not None:
            # At the log, through the clamp (the route backward's beta_is_log).
            grads["log_beta"] = d_beta
        # Q/K/V projections.
        x2d = xc.reshape(tokens, model_dim)
        d_qk = d_rows.reshape(tokens, 2 * width).to(dtype)
        d_v = d_value.reshape(tokens, model_dim).to(dtype)
        dx = None
        if ctx.needs_input_grad[2]:
            dx = torch.mm(d_v, named["value.weight"].detach().to(dtype))
            dx.addmm_(d_qk[:, :width], named["query.weight"].detach().to(dtype))
            dx.addmm_(d_qk[:, width:], named["key.weight"].detach().to(dtype))
            dx = dx.view(batch, length, model_dim).to(ctx.x_dtype)
        if wants("query.weight") and wants("key.weight"):
            wq_dtype, wk_dtype = named["query.weight"].dtype, named["key.weight"].dtype
            d_wqk = _mm_tn_f32(d_qk, x2d, wq_dtype if wq_dtype == wk_dtype else torch.float32)
            grads["query.weight"], grads["key.weight"] = d_wqk[:width], d_wqk[width:]
        elif wants("query.weight"):
            grads["query.weight"] = _mm_tn_f32(d_qk[:, :width], x2d, named["query.weight"].dtype)
        elif wants("key.weight"):
            grads["key.weight"] = _mm_tn_f32(d_qk[:, width:], x2d, named["key.weight"].dtype)
        if wants("value.weight"):
            grads["value.weight"] = _mm_tn_f32(d_v, x2d, named["value.weight"].dtype)
        if wants("value.bias"):
            grads["value.bias"] = (
                d_value_sums.to(named["value.bias"].dtype) if d_value_sums is not None
                else hip_ops.column_sums(d_v, named["value.bias"].dtype)
            )
        tail = [
            grads[name].to(named[name].dtype).reshape(named[name].shape) if name in grads else None
            for name in ctx.param_names
        ]
        return (None, None, dx, d_key, d_val, *tail)


class _HipLayerNormFunction(torch.autograd.Function):
    """``nn.LayerNorm`` over the last dimension (the blocks' and the LM's
    norms, reference ``modules.py:311, 313, 440``) on the library's LayerNorm
    kernel, with its native backward (``da_layer_norm_backward``: dx and the
    parameter gradients in one pass over x and dY)."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps):  # type: ignore[override]
        from . import hip_ops

        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        ctx.param_dtypes = (weight.dtype if weight is not None else None, bias.dtype if bias is not None else None)
        return hip_ops.layer_norm_hip(x, weight, bias, eps)

    @staticmethod
    def backward(ctx, grad):  # type: ignore[override]
        from . import hip_ops

        x, weight = ctx.saved_tensors
        wd, bd = ctx.param_dtypes
        # One cast for both parameter gradients when they share a dtype.
        dx, d_weight, d_bias = hip_ops.layer_norm_backward_hip(
            x, grad, weight, ctx.eps, params_dtype=wd if wd is not None and wd == bd else torch.float32)
        return (dx if ctx.needs_input_grad[0] else None,
                d_weight.to(wd) if wd is not None and ctx.needs_input_grad[1] else None,
                d_bias.to(bd) if bd is not None and ctx.needs_input_grad[2] else None, None)


def _hip_layer_norm_applies(norm: nn.Module, x: Tensor, backend: str) -> bool:
    """Whether ``norm`` (an ``nn.LayerNorm``) runs as ``_HipLayerNormFunction``
    on x: a 16-bit CUDA input whose backend resolves to HIP, one normalized
    dimension (a multiple of 8 up to 4096), weight and bias both present or
    both absent in one dtype."""

    if backend == "torch" or not isinstance(norm, nn.LayerNorm) or len(norm.normalized_shape) != 1:
        return False
    if x.dtype not in (torch.float16, torch.bfloat16) or not x.is_cuda or torch.is_autocast_enabled("cuda"):
        return False
    dim = norm.normalized_shape[0]
    if dim % 8 or dim > 4096 or x.shape[-1] != dim:
        return False
    if (norm.weight is None) != (norm.bias is None):
        return False
    if norm.weight is not None and norm.weight.dtype != norm.bias.dtype:
        return False
    return resolve_backend(backend, (_Spec(True, x.dtype),)) == "hip"  # type: ignore[arg-type]


def _layer_norm(norm: nn.LayerNorm, x: Tensor, backend: str) -> Tensor:
    if _hip_layer_norm_applies(norm, x, backend):
        return _HipLayerNormFunction.apply(x, norm.weight, norm.bias, norm.eps)
    return norm(x)


class _HipFeedForwardFunction(torch.autograd.Function):
    """``x + W2 GELU(W1 h + b1) + b2`` (the block's feed-forward and its
    residual add, reference ``modules.py:318-330, 343-346``) on the library's
    GEMM, with a native backward.

    Forward: z = W1 h + b1 (one GEMM, bias in its epilogue), u = GELU(z)
    (exact, ``nn.GELU()``), y = W2 u + b2 + x (one GEMM, bias and residual in
    its epilogue); z and u are kept.  Backward: dU = dY W2, dZ = dU GELU'(z),
    dH = dZ W1, the weight gradients as split-K library products rounded once
    and the bias gradients as column sums (library GEMVs), where torch's
    autograd would reduce the 16-bit gradients over the rows.
    """

    @staticmethod
    def forward(ctx, x, h, w1, b1, w2, b2):  # type: ignore[override]
        from . import hip_ops

        dtype = x.dtype
        cast = lambda t: t if t is None or t.dtype == dtype else t.to(dtype)  # noqa: E731
        z = hip_ops.linear_hip(h, cast(w1.detach()), b1.detach() if b1 is not None else None)
        u = F.gelu(z)
        y = hip_ops.linear_hip(u, cast(w2.detach()), b2.detach() if b2 is not None else None, residual=x.detach())
        ctx.save_for_backward(h, z, u, w1, w2)
        ctx.has_bias = (b1 is not None, b2 is not None)
        ctx.bias_dtypes = (b1.dtype if b1 is not None else None, b2.dtype if b2 is not None else None)
        return y

    @staticmethod
    def backward(ctx, grad):  # type: ignore[override]
        from . import hip_ops

        h, z, u, w1, w2 = ctx.saved_tensors
        dtype = z.dtype
        rows = z.numel() // z.shape[-1]
        dy = grad.reshape(rows, -1).to(dtype)
        h2, z2, u2 = h.reshape(rows, -1), z.reshape(rows, -1), u.reshape(rows, -1)
        du = torch.mm(dy, w2.detach().to(dtype))
        d_w2 = hip_ops._mm_tn_f32(dy, u2, w2.dtype) if ctx.needs_input_grad[4] else None
        d_b2 = hip_ops.column_sums(dy, ctx.bias_dtypes[1]) if ctx.has_bias[1] and ctx.needs_input_grad[5] else None
        dz = torch.ops.aten.gelu_backward(du, z2)
        d_w1 = hip_ops._mm_tn_f32(dz, h2, w1.dtype) if ctx.needs_input_grad[2] else None
        d_b1 = hip_ops.column_sums(dz, ctx.bias_dtypes[0]) if ctx.has_bias[0] and ctx.needs_input_grad[3] else None
        dh = torch.mm(dz, w1.detach().to(dtype)).view(h.shape) if ctx.needs_input_grad[1] else None
        dx = grad if ctx.needs_input_grad[0] else None
        return dx, dh, d_w1, d_b1, d_w2, d_b2


class DoubleAttentionBlock(nn.Module):
    """Pre-norm transformer block around ``SharedDictionaryAttention`` (``modules.py:294-356``)."""

    def __init__(
        self,
        config: DoubleAttentionConfig,
        *,
        feedforward_dim: int | None = None,
        dropout: float = 0.0,
    ) -> None:
        super().__init__()
        feedforward_dim = feedforward_dim or 3 * config.model_dim
        if config.q_dictionary_feedforward:
            if config.qk_branches != 1:
                raise ValueError("Q-dictionary FFN requires exactly one Q branch")
            if feedforward_dim != config.dictionary_size:
                raise ValueError("Q-dictionary FFN requires feedforward_dim == dictionary_size")
        self.attention_norm = nn.LayerNorm(config.model_dim)
        self.attention = SharedDictionaryAttention(config, create_bank=False)
        self.feedforward_norm = nn.LayerNorm(config.model_dim)
        # The Q-dictionary FFN keeps the standard FFN's module indices; only
        # feedforward[0] (the expansion) is replaced by Dk^T Q (modules.py:314-323).
        first = nn.Identity() if config.q_dictionary_feedforward else nn.Linear(config.model_dim, feedforward_dim)
        self.feedforward = nn.Sequential(
            first,
            nn.GELU(),
            nn.Linear(feedforward_dim, config.model_dim),
            nn.Dropout(dropout),
        )

    def _hip_block(
        self,
        x: Tensor,
        bank: SharedDictionaryBank,
        normalized_dictionary: tuple[Tensor, Tensor] | None,
    ) -> Tensor | None:
        """The block on the HIP kernels, without autograd, or None.

        LayerNorms run as the library's LayerNorm kernel; the residual adds
        ride in the epilogues of the attention's output projection and of the
        FFN's second linear; the FFN's GELU rides in its first linear.  The
        Q-dictionary FFN expands on the library's GEMM against the normalized
        key atoms.
        """

        from . import hip_ops

        attention = self.attention
        dtype = attention._hip_inference_dtype(x, bank)
        if dtype is None or x.dtype != dtype or not isinstance(attention.output, nn.Linear):
            return None
        if self.training and any(isinstance(m, nn.Dropout) and m.p > 0 for m in self.feedforward):
            return None
        if normalized_dictionary is not None and any(t.requires_grad for t in normalized_dictionary):
            return None
        hip_ops.check_module_supported(attention.config)
        x = x.contiguous()
        norm1 = self.attention_norm
        hidden = hip_ops.layer_norm_hip(x, norm1.weight, norm1.bias, norm1.eps)
        x = attention._hip_call(hidden, bank, normalized_dictionary, dtype, residual=x, want_routed=False).output
        norm2 = self.feedforward_norm
        normalized_x = hip_ops.layer_norm_hip(x, norm2.weight, norm2.bias, norm2.eps)
        if attention.config.q_dictionary_feedforward:
            return self._q_dictionary_feedforward_hip(x, normalized_x, bank, normalized_dictionary, dtype)
        first, second = self.feedforward[0], self.feedforward[2]
        expanded = hip_ops.linear_hip(normalized_x, first.weight, first.bias, activation="gelu")
        return hip_ops.linear_hip(expanded, second.weight, second.bias, residual=x)

    def _q_dictionary_feedforward_hip(
        self,
        x: Tensor,
        normalized_x: Tensor,
        bank: SharedDictionaryBank,
        normalized_dictionary: tuple[Tensor, Tensor] | None,
        dtype: torch.dtype,
    ) -> Tensor:
        """The Q-dictionary FFN (``modules.py:546``) on the library's GEMM: the
        query projection, the expansion against the normalized key atoms with
        GELU in its epilogue, then the second linear with the residual add."""

        from . import hip_ops

        if normalized_dictionary is None:
            dictionary_key, _ = bank.normalized(self.attention.config.eps)
        else:
            dictionary_key, _ = normalized_dictionary
        query = hip_ops.linear_hip(normalized_x, self.attention.query.weight.to(dtype))
        atoms_by_dim = hip_ops._aligned(dictionary_key.detach().t().to(dtype))   # [atoms, R]
        hidden = hip_ops.linear_hip(query, atoms_by_dim, activation="gelu")
        second = self.feedforward[2]
        return hip_ops.linear_hip(hidden, second.weight.to(dtype), second.bias, residual=x)

    def _q_dictionary_feedforward(
        self,
        x: Tensor,
        normalized_x: Tensor,
        bank: SharedDictionaryBank,
        normalized_dictionary: tuple[Tensor, Tensor] | None,
    ) -> Tensor:
        if normalized_dictionary is None:
            dictionary_key, _ = bank.normalized(self.attention.config.eps)
        else:
            dictionary_key, _ = normalized_dictionary
        query = self.attention.query(normalized_x)
        if dictionary_key.dtype != query.dtype:
            dictionary_key = dictionary_key.to(query.dtype)
        hidden = F.linear(query, dictionary_key.transpose(0, 1).contiguous())
        return x + self.feedforward(hidden)

    def forward(
        self,
        x: Tensor,
        bank: SharedDictionaryBank,
        *,
        normalized_dictionary: tuple[Tensor, Tensor] | None = None,
    ) -> Tensor:
        fused = self._hip_block(x, bank, normalized_dictionary)
        if fused is not None:
            return fused
        backend = self.attention.config.backend
        x = x + self.attention(
            _layer_norm(self.attention_norm, x, backend), bank=bank, normalized_dictionary=normalized_dictionary
        )
        normalized_x = _layer_norm(self.feedforward_norm, x, backend)
        if not self.attention.config.q_dictionary_feedforward:
            if self._hip_feedforward_applies(x, normalized_x):
                first, second = self.feedforward[0], self.feedforward[2]
                return _HipFeedForwardFunction.apply(x, normalized_x, first.weight, first.bias, second.weight,
                                                     second.bias)
            return x + self.feedforward(normalized_x)
        return self._q_dictionary_feedforward(x, normalized_x, bank, normalized_dictionary)

    def _hip_feedforward_applies(self, x: Tensor, normalized_x: Tensor) -> bool:
        """Whether the feed-forward runs as ``_HipFeedForwardFunction``: the
        attention's backend resolves to HIP for this input, the activations
        are 16-bit with the parameters in their dtype or fp32, and no dropout
        is active (eval, or p = 0)."""

        cfg = self.attention.config
        first, second = self.feedforward[0], self.feedforward[2]
        if cfg.backend == "torch" or not isinstance(first, nn.Linear) or not isinstance(second, nn.Linear):
            return False
        if self.training and self.feedforward[3].p > 0:
            return False
        dtype = x.dtype
        if dtype not in (torch.float16, torch.bfloat16) or normalized_x.dtype != dtype or not x.is_cuda:
            return False
        if torch.is_autocast_enabled("cuda"):
            return False
        if any(p.dtype not in (dtype, torch.float32) for p in (first.weight, second.weight)):
            return False
        if first.in_features % 32 or second.in_features % 32 or first.out_features % 4 or second.out_features % 4:
            return False
        return resolve_backend(cfg.backend, (_Spec(True, dtype),)) == "hip"  # type: ignore[arg-type]


class DoubleAttentionStack(nn.Module):
    """Blocks sharing global or stage-wise banks (``modules.py:359-412``)."""

    def __init__(
        self,
        config: DoubleAttentionConfig,
        num_layers: int,
        *,
        dictionary_group_size: int | None = None,
        feedforward_dim: int | None = None,
        dropout: float = 0.0,
    ) -> None:
        super().__init__()
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        group_size = dictionary_group_size or num_layers
        if group_size <= 0:
            raise ValueError("dictionary_group_size must be positive")
        self.config = config
        self.num_layers = num_layers
        self.dictionary_group_size = group_size
        self.banks = nn.ModuleList(
            SharedDictionaryBank(config.routing_dim, config.dictionary_size, untied=config.untied_dictionary)
            for _ in range(math.ceil(num_layers / group_size))
        )
        self.blocks = nn.ModuleList(
            DoubleAttentionBlock(config, feedforward_dim=feedforward_dim, dropout=dropout)
            for _ in range(num_layers)
        )

    def _normalize_banks(self, x: Tensor) -> tuple[tuple[Tensor, Tensor], ...]:
        # Each bank is normalized once per forward and reused by every block
        # of its group (modules.py:398-404).  On the HIP path that is one
        # kernel launch per bank, already in the route layouts.
        cfg = self.config
        if cfg.backend != "torch" and not torch.is_grad_enabled():
            attention = self.blocks[0].attention
            dtype = _compute_dtype(x, attention.query.weight)
            if resolve_backend(cfg.backend, (_Spec(x.is_cuda, dtype),)) == "hip":  # type: ignore[arg-type]
                from . import hip_ops

                hip_ops.check_module_supported(cfg)
                key_dtype = hip_ops.route_key_dtype(cfg.normalize_routing_input, dtype)
                return tuple(bank.normalized_hip(cfg.eps, key_dtype) for bank in self.banks)
        return tuple(bank.normalized(cfg.eps) for bank in self.banks)

    def forward(self, x: Tensor) -> Tensor:
        dictionaries = self._normalize_banks(x)
        for index, block in enumerate(self.blocks):
            bank_index = min(index // self.dictionary_group_size, len(self.banks) - 1)
            x = block(x, self.banks[bank_index], normalized_dictionary=dictionaries[bank_index])
        return x


class DoubleAttentionLM(nn.Module):
    """Causal LM over a ``DoubleAttentionStack`` (``modules.py:415-460``)."""

    def __init__(
        self,
        vocab_size: int,
        max_sequence_length: int,
        config: DoubleAttentionConfig,
        num_layers: int,
        *,
        dictionary_group_size: int | None = None,
        feedforward_dim: int | None = None,
        dropout: float = 0.0,
    ) -> None:
        super().__init__()
        self.max_sequence_length = max_sequence_length
        self.token_embedding = nn.Embedding(vocab_size, config.model_dim)
        self.position_embedding = nn.Embedding(max_sequence_length, config.model_dim)
        self.stack = DoubleAttentionStack(
            config,
            num_layers,
            dictionary_group_size=dictionary_group_size,
            feedforward_dim=feedforward_dim,
            dropout=dropout,
        )
        self.final_norm = nn.LayerNorm(config.model_dim)
        # Built (consuming its init draws) and then tied to the embedding.
        self.lm_head = nn.Linear(config.model_dim, vocab_size, bias=False)
        self.lm_head.weight = self.token_embedding.weight

    def _final_norm(self, hidden: Tensor) -> Tensor:
        # On the HIP path the final LayerNorm is the library's kernel (with
        # its native backward when training).
        attention = self.stack.blocks[0].attention
        needs_grad = torch.is_grad_enabled() and any(p.requires_grad for p in self.final_norm.parameters())
        if not needs_grad and attention._hip_inference_dtype(hidden, self.stack.banks[0]) == hidden.dtype:
            from . import hip_ops

            return hip_ops.layer_norm_hip(hidden, self.final_norm.weight, self.final_norm.bias, self.final_norm.eps)
        return _layer_norm(self.final_norm, hidden, attention.config.backend)

    def forward(self, token_ids: Tensor, targets: Tensor | None = None) -> tuple[Tensor, Tensor | None]:
        if token_ids.ndim != 2:
            raise ValueError("token_ids must have shape [B, T]")
        length = token_ids.shape[1]
        if length > self.max_sequence_length:
            raise ValueError(
                f"sequence length {length} exceeds configured maximum {self.max_sequence_length}"
            )
        # Positions 0 .. length-1 of the plain position table are its first
        # `length` rows (reference modules.py:452-453 gathers them with an
        # arange): the same values and gradients without an index tensor or
        # a gather launch.
        hidden = self.token_embedding(token_ids) + self.position_embedding.weight[:length][None]
        logits = self.lm_head(self._final_norm(self.stack(hidden)))
        loss = None
        if targets is not None:
            if targets.shape != token_ids.shape:
                raise ValueError("targets must match token_ids shape")
            loss = F.cross_entropy(logits.flatten(0, 1), targets.flatten())
        return logits, loss
