"""Field types and the flat layout of SO(2)-steerable fields.

Restates ``representations/field_type.py`` of the reference: an
``SO2FieldType`` is the multiplicity of each frequency (ascending, zeros
dropped; :27-137), ``slices`` gives each frequency's range in the flat vector
(:238-255), and ``SO2FeatureField.{from_flat,to_flat}`` pack frequency 0
first and then each frequency's ``(a_n, 2)`` pairs, the copy index outside the
pair index (:426-488).  ``gauge_transform`` applies ``rho(r_{-theta})``
(:519-537).
"""

from __future__ import annotations

from collections.abc import Iterable, Mapping

import torch
from torch import Tensor

from gm_attention_amd.representations import so2


class SO2FieldType:
    __slots__ = ("_frequencies", "_multiplicities")

    def __init__(self, multiplicities: Mapping[int, int] | Iterable[tuple[int, int]]) -> None:
        raw = list(multiplicities.items()) if isinstance(multiplicities, Mapping) else [tuple(i) for i in multiplicities]
        seen: set[int] = set()
        items: list[tuple[int, int]] = []
        for frequency, multiplicity in raw:
            so2.irrep_dimension(frequency)
            if multiplicity < 0:
                raise ValueError(f"A multiplicity must be nonnegative, got {multiplicity} for frequency {frequency}.")
            if frequency in seen:
                raise ValueError(f"Frequency {frequency} was specified more than once.")
            seen.add(frequency)
            if multiplicity > 0:
                items.append((int(frequency), int(multiplicity)))
        if not items:
            raise ValueError("A field type must contain at least one frequency with nonzero multiplicity.")
        items.sort()
        self._frequencies = tuple(f for f, _ in items)
        self._multiplicities = tuple(m for _, m in items)

    @property
    def frequencies(self) -> tuple[int, ...]:
        return self._frequencies

    @property
    def multiplicities(self) -> tuple[int, ...]:
        return self._multiplicities

    @property
    def dimension(self) -> int:
        return sum(m * so2.irrep_dimension(f) for f, m in self.items())

    @property
    def max_frequency(self) -> int:
        return self._frequencies[-1]

    def multiplicity(self, frequency: int) -> int:
        if frequency not in self._frequencies:
            return 0
        return self._multiplicities[self._frequencies.index(frequency)]

    def items(self) -> tuple[tuple[int, int], ...]:
        return tuple(zip(self._frequencies, self._multiplicities))

    def scaled(self, factor: int) -> SO2FieldType:
        return SO2FieldType({f: factor * m for f, m in self.items()})

    def slices(self) -> dict[int, slice]:
        out: dict[int, slice] = {}
        start = 0
        for frequency, multiplicity in self.items():
            stop = start + multiplicity * so2.irrep_dimension(frequency)
            out[frequency] = slice(start, stop)
            start = stop
        return out

    def common_frequencies(self, other: SO2FieldType) -> tuple[int, ...]:
        return tuple(f for f in self._frequencies if f in set(other.frequencies))

    def __contains__(self, frequency: object) -> bool:
        return frequency in self._frequencies

    def __len__(self) -> int:
        return len(self._frequencies)

    def __eq__(self, other: object) -> bool:
        if not isinstance(other, SO2FieldType):
            return NotImplemented
        return self._frequencies == other._frequencies and self._multiplicities == other._multiplicities

    def __hash__(self) -> int:
        return hash((self._frequencies, self._multiplicities))

    def __repr__(self) -> str:
        body = ", ".join(f"{f}: {m}" for f, m in self.items())
        return f"SO2FieldType({{{body}}}, dimension={self.dimension})"


class SO2FeatureField:
    """Per-frequency coefficients: ``(*batch, a_0)`` at 0, ``(*batch, a_n, 2)`` above."""

    __slots__ = ("coefficients", "field_type", "_flat")

    def __init__(self, field_type: SO2FieldType, coefficients: Mapping[int, Tensor]) -> None:
        if set(coefficients) != set(field_type.frequencies):
            raise ValueError(
                f"coefficients must supply exactly the frequencies of the field type {sorted(field_type.frequencies)}, "
                f"got {sorted(coefficients)}."
            )
        for frequency, multiplicity in field_type.items():
            t = coefficients[frequency]
            trailing = (multiplicity,) if frequency == 0 else (multiplicity, 2)
            if tuple(t.shape[-len(trailing):]) != trailing:
                raise ValueError(
                    f"coefficients[{frequency}] must have shape (*batch_shape, {', '.join(map(str, trailing))}), "
                    f"got {tuple(t.shape)}."
                )
        self.field_type = field_type
        self.coefficients = dict(coefficients)
        self._flat = None

    @classmethod
    def from_flat(cls, field_type: SO2FieldType, flat: Tensor) -> SO2FeatureField:
        if flat.ndim == 0 or flat.shape[-1] != field_type.dimension:
            raise ValueError(f"flat must have shape (*batch_shape, {field_type.dimension}), got {tuple(flat.shape)}.")
        out: dict[int, Tensor] = {}
        for frequency, multiplicity in field_type.items():
            block = flat[..., field_type.slices()[frequency]]
            out[frequency] = block if frequency == 0 else block.unflatten(-1, (multiplicity, 2))
        field = cls(field_type, out)
        field._flat = (flat, out)  # to_flat hands the rows back while the coefficients are these views
        return field

    def to_flat(self) -> Tensor:
        """The flat rows (frequency 0, then each frequency's ``(a_n, 2)`` pairs)
        as a new tensor (reference field_type.py:472-488)."""
        blocks = [self.coefficients[f] if f == 0 else self.coefficients[f].flatten(-2) for f in self.field_type.frequencies]
        return torch.cat(blocks, dim=-1)

    def _rows(self) -> Tensor:
        """The flat rows for the package's own read-only use: the tensor the
        field was made from by ``from_flat`` while its coefficients are still
        the views of it (no copy), otherwise :meth:`to_flat`.  Callers must not
        write into the result."""
        if self._flat is not None:
            flat, views = self._flat
            if all(self.coefficients[f] is v for f, v in views.items()):
                return flat
        return self.to_flat()

    def apply_rotation(self, angles: Tensor) -> SO2FeatureField:
        return SO2FeatureField(self.field_type, {
            f: so2.rotate_irrep_coefficients(f, t, angles.unsqueeze(-1)) for f, t in self.coefficients.items()
        })

    def gauge_transform(self, angles: Tensor) -> SO2FeatureField:
        """The field in the gauge ``E' = E r(theta)``: coefficients by ``rho(r_{-theta})``."""
        return self.apply_rotation(-angles)

    @property
    def frequencies(self) -> tuple[int, ...]:
        return self.field_type.frequencies

    @property
    def batch_shape(self) -> torch.Size:
        f = self.field_type.frequencies[0]
        t = self.coefficients[f]
        return t.shape[: t.ndim - (1 if f == 0 else 2)]

    @property
    def dtype(self) -> torch.dtype:
        return self.coefficients[self.field_type.frequencies[0]].dtype

    @property
    def device(self) -> torch.device:
        return self.coefficients[self.field_type.frequencies[0]].device

    def __getitem__(self, frequency: int) -> Tensor:
        return self.coefficients[frequency]

    def to(self, device=None, dtype=None) -> SO2FeatureField:
        return SO2FeatureField(self.field_type, {f: t.to(device=device, dtype=dtype) for f, t in self.coefficients.items()})
