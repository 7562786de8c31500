"""The factored kernel's node-side channel mixing, ``Z_t(j) = W_t v_j``, as
real matrix products.

The reference forms it as one complex ``einsum("ja,bat->jtb")`` per node
vector (``nn/kernels.py:575-603``).  Here every node vector's blocks become
one real matrix ``M`` of ``(width of the vector's reals, K * sum b_m * 2)``
that encodes the complex product and the conjugation of the input, so the
mixing is one dense real product ``X_n M`` over the node field's frequency-n
columns (``x_0`` or the ``(a_n, 2)`` pairs of ``x_n``).  ``M`` is built from
the kernel's parameters by differentiable torch ops, so the parameters'
gradients follow from autograd on the product.
"""

from __future__ import annotations

import torch
from torch import Tensor

from gm_attention_amd.representations import so2
from gm_attention_amd.representations.field_type import SO2FeatureField


def mixing_matrix(weights: Tensor, kind: str) -> Tensor:
    """The real ``M`` with ``X M = (re, im)`` of ``sum_a v_a W[b, a, t]`` laid out
    ``(t, b, re/im)``: ``weights`` is ``(sum b, a, K)``, complex (real for the
    real block); ``kind`` is ``"real"``, ``"plain"`` (``v = x_0`` or ``x_n``) or
    ``"conj"`` (``v = conj(x_n)``), and ``promote`` marks a real ``x_0`` read by
    complex blocks."""
    b, a, k = weights.shape
    if kind == "real":
        return weights.permute(1, 2, 0).reshape(a, k * b)  # (a, t, b)
    wr, wi = weights.real.permute(1, 2, 0), weights.imag.permute(1, 2, 0)  # (a, t, b)
    if kind == "promote":  # real x_0 times complex W
        return torch.stack([wr, wi], dim=-1).reshape(a, k * b * 2)
    sign = -1.0 if kind == "conj" else 1.0  # d/d(imag part): (-Wi, Wr) for v, (Wi, -Wr) for conj(v)
    # row 2a is the input's real part, row 2a + 1 its imaginary part
    from_real = torch.stack([wr, wi], dim=-1)  # (a, t, b, 2)
    from_imag = torch.stack([-sign * wi, sign * wr], dim=-1)
    return torch.stack([from_real, from_imag], dim=1).reshape(2 * a, k * b * 2)


def node_products(kernel, x: SO2FeatureField) -> dict[tuple[int, int, str], Tensor]:
    """``(n_nodes, K, b_m)`` per block, complex except the real block."""
    products: dict[tuple[int, int, str], Tensor] = {}
    n_nodes = x.batch_shape[0]
    with torch.profiler.record_function("gm::kernel/node_products"):
        for (n, kind), blocks in kernel.node_vector_groups():
            weights = torch.cat([kernel._block_weights(b) for b in blocks], dim=0)  # (sum b, a_n, K)
            k = weights.shape[-1]
            widths = [kernel.field_type_out.multiplicity(m) for _, m, _ in blocks]
            if kind == "real":
                vector = x[0]
                mixed = (vector @ mixing_matrix(weights, "real").to(vector.dtype)).reshape(n_nodes, k, -1)
            else:
                if n == 0:
                    vector, mode = x[0], "promote"
                else:
                    vector, mode = x[n].reshape(n_nodes, -1), kind
                flat = vector @ mixing_matrix(weights, mode).to(vector.dtype)
                mixed = so2.as_complex(flat.reshape(n_nodes, k, -1, 2))
            for block, piece in zip(blocks, torch.split(mixed, widths, dim=-1), strict=True):
                products[block] = piece
    return products
