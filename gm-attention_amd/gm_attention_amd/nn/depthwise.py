"""The depthwise (per-copy) steerable kernel whose aggregation runs on the HIP path.

Restates the reference's ``nn/depthwise.py``:

* ``SO2DepthwiseKernel`` (:44-193): one steerable kernel per irrep copy of
  ``field_type``; per copy ``a`` of frequency ``n`` the message is
  ``C_a(r) x_a`` at ``n = 0`` and ``A_a(r) z + (r/c)^{2n} B_a(r) e^{2 i n phi}
  conj(z)`` above it (``z`` the transported copy).  The radial functions are
  heads over one shared trunk: a real head of ``a_0`` outputs and a complex
  head of ``sum_n 4 a_n`` outputs laid out per frequency as ``(2, a_n, 2)``
  = (A | B, copy, re/im) (:106-127, 175-191);
* ``stacked_coefficients`` (:206-238): every kernel's ``(rc, cc)`` readouts of
  one radial embedding on a leading kernel axis, each kernel read out by its
  own trunk and heads.

The per-edge message form (``SO2DepthwiseKernel.forward`` on edge-shaped
fields, :147-193) is the eager path (``eager_ops.depthwise_messages``); the
layer (``convolution.SO2Convolution``) evaluates the kernel through the fused
depthwise op and takes the eager path only for calls the op declines.
"""

from __future__ import annotations

from collections.abc import Sequence
import torch
from torch import Tensor, nn

from gm_attention_amd.discretization.edge_geometry import cutoff_tolerance
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FieldType


class SO2DepthwiseKernel(nn.Module):
    """One steerable kernel per irrep copy, ``field_type -> field_type`` (:44-145)."""

    def __init__(self, field_type: SO2FieldType, *, cutoff: float, n_radial_basis: int = 8,
                 radial_hidden_features: Sequence[int] = (16,), radial_basis: str = "gaussian", bias: bool = True,
                 dtype: torch.dtype | None = None, device: torch.device | str | None = None) -> None:
        super().__init__()
        if not isinstance(field_type, SO2FieldType):
            raise TypeError(f"field_type must be an SO2FieldType, got {type(field_type).__name__}.")
        self.field_type = field_type
        self.field_type_in = field_type
        self.field_type_out = field_type
        # the radial embedding and trunk of a scalar 1 -> 1 steerable kernel: identical construction
        template = SO2SteerableKernel(SO2FieldType({0: 1}), SO2FieldType({0: 1}), cutoff=cutoff,
                                      n_radial_basis=n_radial_basis, radial_hidden_features=radial_hidden_features,
                                      radial_basis=radial_basis, bias=bias, dtype=dtype, device=device)
        self.radial_basis = template.radial_basis
        self.radial_trunk = template.radial_trunk
        trunk_width = [n_radial_basis, *radial_hidden_features][-1]
        scalar_width = field_type.multiplicity(0) if 0 in field_type else 0
        self._complex_frequencies = [f for f in field_type.frequencies if f != 0]
        self._complex_widths = [4 * field_type.multiplicity(f) for f in self._complex_frequencies]
        complex_width = sum(self._complex_widths)
        self.real_head = (nn.Linear(trunk_width, scalar_width, bias=bias, dtype=dtype, device=device)
                          if scalar_width > 0 else None)
        self.complex_head = (nn.Linear(trunk_width, complex_width, bias=bias, dtype=dtype, device=device)
                             if complex_width > 0 else None)
        self._validated_edge_geometry_ids: set[int] = set()

    @property
    def cutoff(self) -> float:
        return float(self.radial_basis.cutoff)

    def validate_edges(self, edges) -> None:
        """Harmonics tabulated to twice the top frequency; no edge beyond the
        cutoff (checked once per edge set) (:129-145)."""
        required = 2 * self.field_type.max_frequency
        if edges.max_frequency < required:
            raise ValueError(f"edges tabulates harmonics up to order {edges.max_frequency}, but a depthwise kernel "
                             f"at frequency {self.field_type.max_frequency} needs order {required}.")
        if edges.distances.numel() > 0 and id(edges) not in self._validated_edge_geometry_ids:
            maximum = float(edges.distances.max())
            if maximum > self.cutoff + cutoff_tolerance(edges.distances.dtype):
                raise ValueError(f"edges contains a distance ({maximum:.6g}) beyond this kernel's cutoff "
                                 f"({self.cutoff:.6g}).")
            self._validated_edge_geometry_ids.add(id(edges))

    def radial_readouts(self, embedding: Tensor) -> tuple[Tensor | None, Tensor | None]:
        """The real head's ``(E, a_0)`` and the complex head's ``(E, sum 4 a_n)``
        outputs on a radial embedding of the edges: the trunk's features once
        (its ``Linear`` + ``SiLU`` modules in order), then each head's ``Linear``."""
        features = self.radial_trunk(embedding)
        return tuple(None if head is None else head(features)  # type: ignore[return-value]
                     for head in (self.real_head, self.complex_head))

    def forward(self, x, edges):
        """One message per edge from the source features gathered to edge shape
        (:147-193): ``C x_0`` on the scalars, ``A z + (r/c)^{2n} e^{2 i n phi}
        B conj(z)`` per copy of frequency n (``z`` the transported copy)."""
        from gm_attention_amd.nn import eager_ops
        from gm_attention_amd.representations.field_type import SO2FeatureField

        if x.field_type != self.field_type:
            raise ValueError(f"Expected a field of type {self.field_type!r}, got {x.field_type!r}.")
        if tuple(x.batch_shape) != (edges.n_edges,):
            raise ValueError(f"x.batch_shape must equal (edges.n_edges,) = ({edges.n_edges},), got "
                             f"{tuple(x.batch_shape)}.")
        self.validate_edges(edges)
        return SO2FeatureField(self.field_type, eager_ops.depthwise_messages(self, x, edges))

    def extra_repr(self) -> str:
        return f"field_type={self.field_type!r}, cutoff={self.cutoff:.6g}"


def stacked_coefficients(kernels: Sequence[SO2DepthwiseKernel], edges) -> tuple[Tensor | None, Tensor | None]:
    """Every kernel's ``rc (K, E, a_0)`` and ``cc (K, E, sum 4 a_n)`` on the
    edges, kernels on the leading axis (reference :206-238); ``None`` for a
    head the type does not have.  The kernels of one layer share the radial
    basis (one cutoff), so the edges' embedding is evaluated once and read
    out by each kernel's own modules (:meth:`SO2DepthwiseKernel.radial_readouts`);
    a single kernel's readouts gain the kernel axis as a view."""
    for kernel in kernels:
        kernel.validate_edges(edges)
    with torch.profiler.record_function("gm::depthwise/readouts"):
        embedding = kernels[0].radial_basis(edges.distances)
        readouts = [kernel.radial_readouts(embedding) for kernel in kernels]
    heads = []
    for which in range(2):
        parts = [r[which] for r in readouts]
        if parts[0] is None:
            heads.append(None)
        else:
            heads.append(parts[0].unsqueeze(0) if len(parts) == 1 else torch.stack(parts))
    return heads[0], heads[1]
