"""CPU oracle for the shared-dictionary attention forward path.

TEST INFRASTRUCTURE ONLY.  This package is a NumPy restatement of the
reference's PyTorch math (Ahnd6474/double-attention, ``src/double_attention/
ops.py`` and ``modules.py``).  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker or the timed CPU baseline -- never as an implementation the product
path calls.  The product (``double-attention_amd/double_attention``) never
imports it.

Functions and what pins them (each check is in ``tests/test_oracle.py``):

* ``l2_normalize``            closed form; zero vector stays zero; unit norms.
* ``bank_normalized``         unit column norms; tied bank returns one array.
* ``bank_normalized_backward``
                              central finite differences in fp64 of both
                              banks, tied and untied, with a column below eps
                              (the closed form h / eps there).
* ``dictionary_route``        zero input -> normalized mean atom; huge beta ->
                              the argmax atom; one-atom bank; input-scale
                              invariance; atom-permutation invariance; scalar
                              fp64 loop brute force; golden module vectors.
* ``dictionary_route_backward``
                              central finite differences in fp64 of every
                              input (x, both banks, beta) with both norms on
                              and off.
* ``routed_attention``        first causal row = V[0]; all-equal keys ->
                              causal running mean; probabilities sum to one;
                              causal prefix invariance; brute-force loop.
* ``routed_attention_backward``
                              central finite differences of a scalar loss in
                              fp64 for every input; dV = P^T dO sums over maps;
                              zero output gradient -> zero gradients.
* ``assemble_score_maps``     RMS-sum identity q'.k' = sum_g q_g.k_g / sqrt(g);
                              repeat layout; shapes.
* ``assemble_score_maps_backward`` / ``shared_dictionary_attention_backward``
                              central finite differences in fp64 of x and of
                              every module parameter (log beta included) for
                              ten layouts: untied and tied banks, the map mix,
                              grouped and repeated branches, concat, no output
                              projection or bias, non-causal, the route
                              variants.
* ``shared_dictionary_attention`` / ``double_attention_lm``
                              golden vectors written by the reference's own
                              PyTorch path (``tests/golden/make_golden.py``)
                              and parameter-count fixtures from the reference's
                              run records.
"""

from .sda import (
    assemble_score_maps,
    assemble_score_maps_backward,
    bank_normalized,
    bank_normalized_backward,
    beta_from_log,
    dictionary_route,
    dictionary_route_backward,
    double_attention_lm,
    gelu,
    l2_normalize,
    layer_norm,
    routed_attention,
    routed_attention_backward,
    score_scale_from_log,
    shared_dictionary_attention,
    shared_dictionary_attention_backward,
)

__all__ = [
    "assemble_score_maps",
    "assemble_score_maps_backward",
    "bank_normalized",
    "bank_normalized_backward",
    "beta_from_log",
    "dictionary_route",
    "dictionary_route_backward",
    "double_attention_lm",
    "gelu",
    "l2_normalize",
    "layer_norm",
    "routed_attention",
    "routed_attention_backward",
    "score_scale_from_log",
    "shared_dictionary_attention",
    "shared_dictionary_attention_backward",
]
