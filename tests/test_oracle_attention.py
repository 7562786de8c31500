"""Pins the oracle's softmax and depthwise restatements (oracle/eager.py)
against the reference's own compiled CPU arithmetic (oracle/_ref), the
committed golden vectors, closed forms and finite differences."""

import math

import pytest
import torch

import problems
from oracle import eager, ref

FIELD = {0: 8, 1: 8, 2: 8}


def _needs_ref():
    if not ref.available():
        pytest.skip("oracle/_ref not built (needs the reference checkout)")


def _softmax_case(window="quartic", heads=4, field=FIELD, nlat=12, nlon=24, seed=0):
    t = problems.tables(nlat, nlon, window=window)
    p, desc, scale = problems.attention_layout(field, heads)
    D = p.width
    q = problems.normal((t.n_nodes, D), seed)
    k = problems.normal((t.n_nodes, D), seed + 1)
    return t, p, desc, scale, q, k


@pytest.mark.parametrize("window", ["hard", "quartic"])
@pytest.mark.parametrize("heads,field", [(4, FIELD), (2, {0: 6, 1: 4, 2: 2}), (1, {0: 3, 2: 2})])
def test_softmax_oracle_matches_the_compiled_reference(window, heads, field):
    _needs_ref()
    t, p, desc, scale, q, k = _softmax_case(window, heads, field)
    alpha = eager.softmax_op(q, k, t.transport, t.bias, t.inside, p.rows, t.row_ptr, t.source, heads, scale)
    expected = ref.softmax_forward(q, k, t.transport, t.bias, t.inside, desc, t.row_ptr, t.source, heads, scale)
    torch.testing.assert_close(alpha, expected, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("heads,field", [(4, FIELD), (2, {0: 6, 1: 4, 2: 2})])
def test_softmax_oracle_gradients_match_the_compiled_reference(heads, field):
    _needs_ref()
    t, p, desc, scale, q, k = _softmax_case("quartic", heads, field)
    q.requires_grad_(True)
    k.requires_grad_(True)
    alpha = eager.softmax_op(q, k, t.transport, t.bias, t.inside, p.rows, t.row_ptr, t.source, heads, scale)
    dalpha = problems.normal(alpha.shape, 7)
    dq, dk = torch.autograd.grad(alpha, (q, k), dalpha)
    rdq, rdk = ref.softmax_backward(dalpha, q.detach(), k.detach(), t.transport, desc, t.row_ptr, t.source,
                                    alpha.detach(), heads, scale)
    torch.testing.assert_close(dq, rdq, rtol=1e-11, atol=1e-13)
    torch.testing.assert_close(dk, rdk, rtol=1e-11, atol=1e-13)


def test_softmax_oracle_is_a_partition_of_unity_and_passes_gradcheck():
    t = problems.tables(5, 8, window="quartic", rows=1.5)
    p, desc, scale = problems.attention_layout({0: 2, 1: 2, 2: 2}, 2)
    q = problems.normal((t.n_nodes, p.width), 3).requires_grad_(True)
    k = problems.normal((t.n_nodes, p.width), 4).requires_grad_(True)

    def f(q, k):
        return eager.softmax_op(q, k, t.transport, t.bias, t.inside, p.rows, t.row_ptr, t.source, 2, scale)

    alpha = f(q, k)
    sums = torch.segment_reduce(alpha, "sum", offsets=t.row_ptr, axis=0)
    torch.testing.assert_close(sums, torch.ones_like(sums), rtol=0, atol=1e-12)
    assert bool((alpha[t.inside == 0] == 0).all())
    assert torch.autograd.gradcheck(f, (q, k), eps=1e-6, atol=1e-7)


def test_softmax_shift_is_taken_over_the_window_alone():
    """The reference's float32 boundary case (tests/nn/test_fused_attention.py:376-409):
    an out-of-window edge whose score beats the self-loop's by more than
    -log(tiny) must not set the shift.  Scores 225 (self) and 450 (edge at the
    cutoff, quartic window 0)."""
    q = torch.tensor([[15.0], [30.0]])
    row_ptr = torch.tensor([0, 2, 3])
    source = torch.tensor([0, 1, 1])
    tiny = torch.finfo(torch.float32).tiny
    window = torch.tensor([1.0, 0.0, 1.0])
    bias = torch.log(window.clamp_min(tiny))
    inside = (window > 0).to(torch.uint8)
    transport = torch.zeros(3, 3, 2)
    transport[:, :, 0] = 1.0
    rows = ((0, 1, 0, 0, 1),)
    alpha = eager.softmax_op(q, q, transport, bias, inside, rows, row_ptr, source, 1, 1.0)
    assert torch.equal(alpha, torch.tensor([[1.0], [0.0], [1.0]]))


@pytest.mark.parametrize("field", [{0: 4, 1: 4, 2: 4}, {0: 3, 1: 2}, {1: 2, 2: 1}])
def test_depthwise_oracle_matches_the_compiled_reference(field):
    _needs_ref()
    t = problems.tables(10, 20, window="quartic")
    p, desc = problems.depthwise_layout(field)
    E = t.source.shape[0]
    v = problems.normal((t.n_nodes, p.width), 1).requires_grad_(True)
    rc = problems.normal((1, E, p.a_0), 2).requires_grad_(True)
    cc = problems.normal((1, E, p.complex_width), 3).requires_grad_(True)
    out = eager.conv_op(v, rc, cc, t.transport, t.angular, t.rho, t.weights, p.rows, t.row_ptr, t.source)
    expected = ref.conv_forward(v.detach(), rc.detach(), cc.detach(), t.transport, t.angular, t.rho, t.weights, desc,
                                t.row_ptr, t.source, p.a_0, p.complex_width)
    torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-13)
    g = problems.normal(out.shape, 4)
    grads = torch.autograd.grad(out, (v, rc, cc), g, allow_unused=True, materialize_grads=True)
    rgrads = ref.conv_backward(g, v.detach(), rc.detach(), cc.detach(), t.transport, t.angular, t.rho, t.weights,
                               desc, t.row_ptr, t.source, p.a_0, p.complex_width)
    for mine, theirs in zip(grads, rgrads):
        torch.testing.assert_close(mine, theirs, rtol=1e-11, atol=1e-12)


def test_depthwise_oracle_at_the_origin_is_the_per_copy_intertwiner():
    """At r = 0 (a self-loop) the antilinear term vanishes: m = A z on complex
    copies and rc x on scalars (depthwise.py:17-19)."""
    p, desc = problems.depthwise_layout({0: 1, 1: 1})
    v = torch.tensor([[2.0, 1.0, -1.0]], dtype=torch.float64)
    rc = torch.tensor([[[3.0]]], dtype=torch.float64)
    cc = torch.tensor([[[0.5, 0.25, 7.0, 9.0]]], dtype=torch.float64)  # A = 0.5 + 0.25i, B = 7 + 9i
    transport = torch.zeros(1, 3, 2, dtype=torch.float64)
    transport[:, :, 0] = 1.0
    out = eager.conv_op(v, rc, cc, transport, transport, torch.zeros(1, dtype=torch.float64),
                        torch.ones(1, dtype=torch.float64), p.rows, torch.tensor([0, 1]), torch.tensor([0]))
    z = complex(1.0, -1.0) * complex(0.5, 0.25)
    torch.testing.assert_close(out, torch.tensor([[6.0, z.real, z.imag]], dtype=torch.float64))
