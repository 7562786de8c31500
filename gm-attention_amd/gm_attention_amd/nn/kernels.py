"""The steerable value kernel whose factored evaluation runs on the HIP path.

Restates the parts of the reference's ``nn/kernels.py`` the fused path needs:

* ``_GaussianRadialBasis`` (:191-231): ``exp(-((s - mu_k) / sigma)^2 / 2)`` of
  ``s = (r / cutoff)^2`` over centres ``linspace(0, 1, n)``, width the spacing;
* ``SO2SteerableKernel`` (:234-397): the radial trunk (``Linear`` + ``SiLU`` per
  hidden width), the complex readout head laid out as consecutive
  ``(n, m, role)`` ranges of ``2 b_m a_n`` reals (rows ``(b_m, a_n, re/im)``;
  ``linear`` for every pair but ``(0, 0)``, ``antilinear`` for ``n, m >= 1``),
  the real head of the ``(0, 0)`` block, and each role's radial power
  (``|m - n|`` linear, ``m + n`` antilinear);
* ``_blocks`` / ``_block_weights`` / ``_input_vector_key`` /
  ``node_products`` (:496-603): ``Z_t(j) = W_t v_j`` for every block and
  ``t = 0..T`` (the bias on ``t = 0``), the blocks that read one node vector
  as one product;
* ``forward_factored`` / ``forward_factored_aggregated`` (:645-732) through the
  fused factored op (``fused_factored.forward`` / ``forward_aggregated``);
* ``forward`` / ``validate_call`` (:421-476) on an edge-shaped field: the
  per-edge readout ``_forward_general`` (:752-915) through the fused pair
  terms (``fused_pairs.forward_general``).

A call the fused ops decline (CPU tensors, a ``GM_FUSED_*`` switch at
``"0"``, a plan beyond the kernels' bounds) runs the same numbers in torch
(``eager_ops``), as the reference falls back to its eager branches.
"""

from __future__ import annotations

import itertools
import math
import os
from collections.abc import Sequence

import torch
from torch import Tensor, nn

from gm_attention_amd.representations import so2
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

#: ``GM_FACTORED_KERNEL``: the layers evaluate their value kernels in the factored order
#: (reference kernels.py:39-46).  The default is ``"1"`` (the reference's is ``"0"``, the per-edge
#: readout): the factored order is the one the north-star shape fits in memory (the readout
#: materialises (E, 2 b a) coefficients per head); ``"0"`` selects the readout through the fused pair
#: terms.  Both orders compute the same function to summation order.
FACTORED = os.environ.get("GM_FACTORED_KERNEL", "1") != "0"


def factored_enabled() -> bool:
    return FACTORED


class GaussianRadialBasis(nn.Module):
    centers: Tensor

    def __init__(self, n_basis: int, cutoff: float, *, dtype=None, device=None) -> None:
        super().__init__()
        if n_basis < 1:
            raise ValueError(f"n_basis must be at least 1, got {n_basis}.")
        if not (math.isfinite(cutoff) and cutoff > 0.0):
            raise ValueError(f"cutoff must be finite and positive, got {cutoff}.")
        self.cutoff = float(cutoff)
        self.n_basis = n_basis
        self.width = 1.0 / max(n_basis - 1, 1)
        self.register_buffer("centers", torch.linspace(0.0, 1.0, n_basis, dtype=dtype, device=device))

    def forward(self, r: Tensor) -> Tensor:
        normalized = r / self.cutoff
        s = normalized * normalized
        difference = s.unsqueeze(-1) - self.centers
        return torch.exp(-0.5 * (difference / self.width) ** 2)


class SO2SteerableKernel(nn.Module):
    """A gauge-equivariant value kernel ``field_type_in -> field_type_out``."""

    def __init__(self, field_type_in: SO2FieldType, field_type_out: SO2FieldType, *, cutoff: float,
                 n_radial_basis: int = 8, radial_hidden_features: Sequence[int] = (16,), radial_basis: str = "gaussian",
                 bias: bool = True, dtype=None, device=None) -> None:
        super().__init__()
        if radial_basis != "gaussian":
            raise ValueError(f"radial_basis must be 'gaussian', got {radial_basis!r}.")
        self.field_type_in = field_type_in
        self.field_type_out = field_type_out
        self.pairs = tuple((n, m) for n in field_type_in.frequencies for m in field_type_out.frequencies)
        self.radial_basis = GaussianRadialBasis(n_radial_basis, cutoff, dtype=dtype, device=device)
        widths = [n_radial_basis, *radial_hidden_features]
        if any(w < 1 for w in widths[1:]):
            raise ValueError(f"radial_hidden_features must contain only positive widths, got {tuple(radial_hidden_features)}.")
        layers: list[nn.Module] = []
        for a, b in itertools.pairwise(widths):
            layers += [nn.Linear(a, b, bias=bias, dtype=dtype, device=device), nn.SiLU()]
        self.radial_trunk = nn.Sequential(*layers)
        trunk_width = widths[-1]

        self._pair_ranges: dict[tuple[int, int, str], slice] = {}
        self._coefficient_order: list[tuple[int, int, str]] = []
        self._coefficient_widths: list[int] = []
        self._pair_powers: dict[tuple[int, int, str], int] = {}
        real_width = 0
        offset = 0
        for n, m in self.pairs:
            a_n, b_m = field_type_in.multiplicity(n), field_type_out.multiplicity(m)
            if n == 0 and m == 0:
                real_width = b_m * a_n
                continue
            width = 2 * b_m * a_n
            for role, power in (("linear", abs(m - n)), ("antilinear", m + n)):
                if role == "antilinear" and not (n >= 1 and m >= 1):
                    continue
                self._pair_ranges[(n, m, role)] = slice(offset, offset + width)
                self._coefficient_order.append((n, m, role))
                self._coefficient_widths.append(width)
                self._pair_powers[(n, m, role)] = power
                offset += width
        self.complex_head = nn.Linear(trunk_width, offset, bias=bias, dtype=dtype, device=device) if offset else None
        self.real_head = nn.Linear(trunk_width, real_width, bias=bias, dtype=dtype, device=device) if real_width else None

    def validate_call(self, x: SO2FeatureField, edges) -> None:
        """The checks of :meth:`forward` (:444-476): the input type, one
        gathered feature per edge, harmonics tabulated to the top frequency pair."""
        if x.field_type != self.field_type_in:
            raise ValueError(f"Expected a field of type {self.field_type_in!r}, got {x.field_type!r}.")
        if tuple(x.batch_shape) != (edges.n_edges,):
            raise ValueError(f"x.batch_shape must equal (edges.n_edges,) = ({edges.n_edges},), got "
                             f"{tuple(x.batch_shape)}. Gather node features to edge shape (e.g. via "
                             "edges.source_index) before calling this kernel.")
        required = self.field_type_in.max_frequency + self.field_type_out.max_frequency
        if edges.max_frequency < required:
            raise ValueError(f"edges tabulates harmonics up to order {edges.max_frequency}, but connecting frequency "
                             f"{self.field_type_in.max_frequency} to {self.field_type_out.max_frequency} needs "
                             f"order {required}.")

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        """One message per edge from the source features gathered to edge
        shape (:421-442): the per-edge readout through the fused pair terms."""
        from gm_attention_amd.nn import fused_pairs

        self.validate_call(x, edges)
        if fused_pairs.enabled(self, x, edges):
            return fused_pairs.forward_general(self, x, edges)
        from gm_attention_amd.nn import eager_ops

        return SO2FeatureField(self.field_type_out, eager_ops.readout(self, x, edges))

    # ---- the factored evaluation's pieces

    def _blocks(self) -> list[tuple[int, int, str]]:
        """Every coefficient block, the real ``(0, 0)`` block first (kernels.py:496-504)."""
        return ([(0, 0, "real")] if self.real_head is not None else []) + list(self._coefficient_order)

    def readout_parameters(self) -> list[Tensor | None]:
        """The readout heads' parameters in a fixed order: the real head's
        weight and bias, then the complex head's (a bias may be None)."""
        real = self.real_head
        return [real.weight if real is not None else None, real.bias if real is not None else None,
                self.complex_head.weight, self.complex_head.bias]

    def _block_weights(self, block: tuple[int, int, str], params: list[Tensor | None] | None = None) -> Tensor:
        """``(W_0 = bias, W_1..W_T)`` of one block as ``(b_m, a_n, T + 1)``
        (kernels.py:506-536): complex for the phase-carrying blocks.  ``params``
        stands in for the readout parameters (``readout_parameters`` order)."""
        n, m, role = block
        real_w, real_b, cw, cb = self.readout_parameters() if params is None else params
        a_n, b_m = self.field_type_in.multiplicity(n), self.field_type_out.multiplicity(m)
        if role == "real":
            columns = real_w.reshape(b_m, a_n, -1)
            bias = real_b.reshape(b_m, a_n) if real_b is not None else columns.new_zeros(b_m, a_n)
            return torch.cat([bias.unsqueeze(-1), columns], dim=-1)
        rows = self._pair_ranges[block]
        weight = cw[rows]
        columns = so2.as_complex(weight.reshape(b_m, a_n, 2, -1).permute(0, 1, 3, 2).contiguous())
        if cb is not None:
            bias = so2.as_complex(cb[rows].reshape(b_m, a_n, 2).contiguous())
        else:
            bias = columns.new_zeros(b_m, a_n)
        return torch.cat([bias.unsqueeze(-1), columns], dim=-1)

    @staticmethod
    def _input_vector_key(block: tuple[int, int, str]) -> tuple[int, str]:
        """The node vector a block reads: ``x_0`` (real or promoted), ``x_n``,
        or ``conj(x_n)`` for the antilinear blocks and the rows onto 0 (kernels.py:538-546)."""
        n, m, role = block
        if role == "real":
            return (0, "real")
        if n == 0:
            return (0, "plain")
        return (n, "conj" if (m == 0 or role == "antilinear") else "plain")

    def node_vector_groups(self) -> list[tuple[tuple[int, str], list[tuple[int, int, str]]]]:
        """The blocks grouped by the node vector they read, in block order."""
        groups: dict[tuple[int, str], list[tuple[int, int, str]]] = {}
        for block in self._blocks():
            groups.setdefault(self._input_vector_key(block), []).append(block)
        return list(groups.items())

    def node_products(self, x: SO2FeatureField) -> dict[tuple[int, int, str], Tensor]:
        """``W_t v_j`` per block, ``(n_nodes, T + 1, b_m)`` (complex but for the
        real block), one product per node vector (kernels.py:575-603)."""
        if x.field_type != self.field_type_in:
            raise ValueError(f"Expected a field of type {self.field_type_in!r}, got {x.field_type!r}.")
        from gm_attention_amd.nn import node_products as np_op

        return np_op.node_products(self, x)

    def _trunk_hidden(self, distances: Tensor) -> Tensor:
        """The radial trunk's features on the edges, ``(n_edges, T)`` (kernels.py:605-607)."""
        hidden = self.radial_basis(distances)
        for layer in self.radial_trunk:
            hidden = layer(hidden)
        return hidden

    def forward_factored(self, x: SO2FeatureField, edges, products=None, groups=None) -> SO2FeatureField:
        """The messages on the edges through the fused factored op (kernels.py:645-697)."""
        from gm_attention_amd.nn import eager_ops, fused_factored

        if fused_factored.enabled(self, x, edges):
            return fused_factored.forward(self, x, edges, products, groups)
        return SO2FeatureField.from_flat(self.field_type_out, eager_ops.factored_rows(self, x, edges, products))

    def forward_factored_aggregated(self, x: SO2FeatureField, edges, weights: Tensor, products=None,
                                    groups=None) -> SO2FeatureField:
        """Each target's weighted sum of its messages through the fused op (kernels.py:699-732)."""
        from gm_attention_amd.nn import eager_ops, fused_factored

        if fused_factored.enabled(self, x, edges):
            if products is None:  # float32 rows on the grouped kernels where a share of the output copies fits
                shares = fused_factored.forward_aggregated_shares(self, x, edges, weights, groups)
                if shares is not None:
                    return shares
            return fused_factored.forward_aggregated(self, x, edges, weights, products, groups)
        rows = eager_ops.factored_rows(self, x, edges, products)
        return SO2FeatureField.from_flat(self.field_type_out,
                                         eager_ops.segment_sum(weights.to(rows.dtype).unsqueeze(-1) * rows,
                                                               edges.row_ptr))
