"""Real SO(2) irreps in complex form: ``rho_n(r_theta)`` acts on a frequency-n
pair ``(x, y) = x + iy`` as multiplication by ``exp(i n theta)``.

Restates ``representations/so2.py`` of the reference (``complex_dtype``
:73-81, ``phase_powers`` :167-213, ``as_complex`` :216-263, ``as_real``
:266-289, ``rotate_irrep_coefficients`` :292-327).
"""

from __future__ import annotations

import torch
from torch import Tensor

_COMPLEX = {torch.float32: torch.complex64, torch.float64: torch.complex128}


def irrep_dimension(frequency: int) -> int:
    if frequency < 0:
        raise ValueError(f"An SO(2) irrep frequency must be nonnegative, got {frequency}.")
    return 1 if frequency == 0 else 2


def complex_dtype(real_dtype: torch.dtype) -> torch.dtype:
    if real_dtype not in _COMPLEX:
        raise TypeError(f"Representation arithmetic supports torch.float32 and torch.float64, got {real_dtype}.")
    return _COMPLEX[real_dtype]


def phase_powers(angles: Tensor, max_frequency: int) -> Tensor:
    """``exp(i k theta)`` for k = 0..max_frequency, ``(..., max_frequency + 1)``,
    as one ``torch.polar`` over ``theta (x) (0..K)`` (reference so2.py:205-213)."""
    exponents = torch.arange(max_frequency + 1, dtype=angles.dtype, device=angles.device)
    scaled = angles.unsqueeze(-1) * exponents
    return torch.polar(torch.ones_like(scaled), scaled)


def as_complex(coefficients: Tensor) -> Tensor:
    coefficients = coefficients.contiguous()
    if coefficients.storage_offset() % 2 != 0:
        coefficients = coefficients.clone()
    return torch.view_as_complex(coefficients)


def as_real(values: Tensor) -> Tensor:
    return torch.view_as_real(values.contiguous())


def rotate_irrep_coefficients(frequency: int, coefficients: Tensor, angles: Tensor) -> Tensor:
    """The bare action ``rho_n(r_theta)`` on ``(..., 2)`` coefficients (identity at n = 0)."""
    if frequency == 0:
        return coefficients
    phase = torch.polar(torch.ones_like(angles), frequency * angles)
    return as_real(as_complex(coefficients) * phase)
