"""The GM-convolution over a node's geodesic neighbourhood on the HIP path.

Restates the reference's ``nn/convolution.py``:

* ``SO2Convolution`` (:94-470): ``y_i = sum_j c(v_ij) w_ij V(v_ij)
  rho(g_{i<-j}) x_j`` with the aggregation window ``c``, the tangent-space
  quadrature weight ``w``, an optional division by each target's window mass
  (``normalize``), an optional pointwise self-intertwiner added after the sum,
  and ``forward_chunked`` over target ranges holding whole neighbourhoods.
  ``depthwise=True`` takes :class:`~gm_attention_amd.nn.depthwise.SO2DepthwiseKernel`
  through the fused depthwise op (reference ``_aggregate_fused``, :432-441),
  with the radial heads evaluated inside the walk where the kernel allows
  (``depthwise_radial``);
  the general kernel runs in the factored order through the fused factored
  aggregate (:310-330), with the window weights as the aggregation weights.

A layer whose fused op is not enabled raises: the reference's eager branch
(gather, per-edge messages, weighted segment sum) is this build's parity
oracle, not a product path.
"""

from __future__ import annotations

import functools
from collections.abc import Sequence

import torch
import torch.utils.checkpoint
from torch import Tensor, nn

from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.nn import depthwise_radial, fused_attention, fused_factored, kernels
from gm_attention_amd.nn.attention import gather_to_edges, sum_partials, weighted_segment_sum
from gm_attention_amd.nn.depthwise import SO2DepthwiseKernel, stacked_coefficients
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.nn.linear import SO2Linear
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

evaluate_aggregation_window = fused_attention.evaluate_aggregation_window


def _checkpointed(module: nn.Module, compute):
    if module.training and torch.is_grad_enabled():
        return torch.utils.checkpoint.checkpoint(compute, use_reentrant=False)
    return compute()


class SO2Convolution(nn.Module):
    """A gauge-equivariant convolution over each node's geodesic neighbourhood (:94-269)."""

    def __init__(self, field_type_in: SO2FieldType, field_type_out: SO2FieldType, *, cutoff: float,
                 window: str = "hard", self_interaction: str = "none", depthwise: bool = False,
                 normalize: bool = False, n_radial_basis: int = 8, radial_hidden_features: Sequence[int] = (16,),
                 radial_basis: str = "gaussian", bias: bool = True, eps: float = 1e-12, dtype=None,
                 device=None) -> None:
        super().__init__()
        if window not in ("hard", "quartic"):
            raise ValueError(f"window must be 'hard' or 'quartic', got {window!r}.")
        if not eps > 0:
            raise ValueError(f"eps must be positive, got {eps}.")
        if depthwise and field_type_in != field_type_out:
            raise ValueError("a depthwise convolution maps every irrep copy to itself, so its input and output "
                             f"types must agree; got {field_type_in!r} -> {field_type_out!r}.")
        if self_interaction not in ("none", "linear"):
            raise ValueError(f"self_interaction must be 'none' or 'linear', got {self_interaction!r}.")
        self.field_type_in = field_type_in
        self.field_type_out = field_type_out
        self.cutoff = float(cutoff)
        self.window = window
        self.self_interaction = self_interaction
        self.depthwise = bool(depthwise)
        self.normalize = bool(normalize)
        self.eps = float(eps)
        self.kernel: SO2SteerableKernel | SO2DepthwiseKernel
        if depthwise:
            self.kernel = SO2DepthwiseKernel(field_type_in, cutoff=cutoff, n_radial_basis=n_radial_basis,
                                             radial_hidden_features=radial_hidden_features,
                                             radial_basis=radial_basis, bias=bias, dtype=dtype, device=device)
        else:
            self.kernel = SO2SteerableKernel(field_type_in, field_type_out, cutoff=cutoff,
                                             n_radial_basis=n_radial_basis,
                                             radial_hidden_features=radial_hidden_features,
                                             radial_basis=radial_basis, bias=bias, dtype=dtype, device=device)
        self.self_linear = (SO2Linear(field_type_in, field_type_out, bias=False, dtype=dtype, device=device)
                            if self_interaction == "linear" else None)

    def _check(self, x: SO2FeatureField, edges):
        if isinstance(edges, SphericalDiscretization):
            edges = edges.edges_within(self.cutoff)
        if x.field_type != self.field_type_in:
            raise ValueError(f"Expected a field of type {self.field_type_in!r}, got {x.field_type!r}.")
        n_nodes = edges.row_ptr.shape[0] - 1
        if tuple(x.batch_shape) != (n_nodes,):
            raise ValueError(f"x.batch_shape must equal (n_nodes,) = ({n_nodes},), inferred from edges.row_ptr, "
                             f"got {tuple(x.batch_shape)}.")
        return edges

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        edges = self._check(x, edges)
        return self._finish(x, self._aggregate(x, edges))

    def _aggregate(self, x: SO2FeatureField, edges, products=None, groups=None) -> dict[int, Tensor]:
        if self.depthwise:
            if fused_attention.enabled_depthwise(self, x, edges):
                return self._aggregate_fused(x, edges)
            # the reference's eager path (convolution.py:297-308): per-edge messages, weighted segment sums
            g = fused_attention.geometry(edges, self.cutoff, self.window, x.dtype)
            messages = self.kernel(gather_to_edges(x, edges.source_index), edges)
            return weighted_segment_sum(g.aggregation_weights(self.normalize, self.eps), messages.coefficients,
                                        edges.row_ptr)
        kernel = self.kernel
        assert isinstance(kernel, SO2SteerableKernel)
        g = fused_attention.geometry(edges, self.cutoff, self.window, x.dtype)
        weights = g.aggregation_weights(self.normalize, self.eps)
        if not kernels.factored_enabled():  # the per-edge readout through the fused pair terms
            messages = kernel(gather_to_edges(x, edges.source_index), edges)
            return weighted_segment_sum(weights, messages.coefficients, edges.row_ptr)
        return kernel.forward_factored_aggregated(x, edges, weights, products, groups).coefficients

    def _aggregate_fused(self, x: SO2FeatureField, edges) -> dict[int, Tensor]:
        """The depthwise aggregation as one fused op per direction: the radial
        heads evaluated inside the walk where the kernel is eligible
        (``depthwise_radial``), else on the coefficients the heads give per
        edge by torch products (the reference's split)."""
        kernel = self.kernel
        assert isinstance(kernel, SO2DepthwiseKernel)
        kernel.validate_edges(edges)
        if depthwise_radial.eligible(kernel, x, edges):
            flat = depthwise_radial.forward(self, x._rows(), edges)
            return SO2FeatureField.from_flat(self.field_type_out, flat).coefficients
        rc, cc = stacked_coefficients([kernel], edges)
        flat = fused_attention.forward_depthwise(self, x._rows(), rc, cc, edges)
        return SO2FeatureField.from_flat(self.field_type_out, flat).coefficients

    def forward_chunked(self, x: SO2FeatureField, edges, *, chunk_size: int) -> SO2FeatureField:
        """:meth:`forward` over consecutive ranges of at most ``chunk_size``
        targets with their whole neighbourhoods (reference :357-430), the node
        mixes of a general kernel formed once; under training each range is
        recomputed in the backward rather than kept."""
        edges = self._check(x, edges)
        factored = isinstance(self.kernel, SO2SteerableKernel) and kernels.factored_enabled()
        products = self.kernel.node_products(x) if factored else None

        def part(chunk):
            groups = fused_factored.groups_for(chunk, chunk.source_index) if factored else None
            return _checkpointed(self, functools.partial(self._aggregate, x, chunk, products, groups))

        partials = [part(chunk) for chunk in edges.chunks(chunk_size)]
        return self._finish(x, sum_partials(partials) if partials else self._aggregate(x, edges))

    def _finish(self, x: SO2FeatureField, outputs: dict[int, Tensor]) -> SO2FeatureField:
        aggregated = SO2FeatureField(self.field_type_out, outputs)
        if self.self_linear is None:
            return aggregated
        pointwise = self.self_linear(x)
        return SO2FeatureField(self.field_type_out,
                               {f: aggregated[f] + pointwise[f] for f in self.field_type_out.frequencies})

    def extra_repr(self) -> str:
        return (f"field_type_in={self.field_type_in!r}, field_type_out={self.field_type_out!r}, "
                f"cutoff={self.cutoff:.6g}, window={self.window!r}, self_interaction={self.self_interaction!r}, "
                f"depthwise={self.depthwise}, normalize={self.normalize}")
