"""The grouped factored kernels' lane-owned slot tables (gm_factored_lane_tables,
host only), checked on the CPU: which plans take them, that they cover every
packed column exactly once, and that the lane kernels' arithmetic replayed
in float64 from the tables (lane q of an edge's four lanes, slot by slot:
u = Z0 + sum_t h_t Z_t at the slot's columns, V = F u with F from the
rho-scaled angular entry and the transport entry, outputs summed over their
consecutive slots) reproduces the oracle's rows (oracle.eager.factored_rows,
the reference's eager forward_factored)."""

import math

import pytest
import torch

from gm_attention_amd import _native
from gm_attention_amd.nn import fused_factored
from gm_attention_amd.nn.attention import SO2MHSA
from gm_attention_amd.representations.field_type import SO2FieldType
from oracle import eager

ACTIVE, REAL, SCALAR, FLUSH, ACONJ, TCONJ = 1 << 7, 1 << 8, 1 << 9, 1 << 10, 1 << 14, 1 << 18


def heads(field, n_heads):
    torch.manual_seed(0)
    mhsa = SO2MHSA(SO2FieldType(field), n_heads, cutoff=0.3, window="hard", dtype=torch.float64)
    kernels = [h.value for h in mhsa.heads]
    hp = fused_factored.heads_plan(kernels[0])
    _, pa, pt = fused_factored.grouped_eligible(hp, torch.float32, 17)
    desc = torch.tensor([list(r) for r in hp.desc_rows], dtype=torch.int32)
    return hp.plan, desc, pa, pt


def tables(field, n_heads):
    plan, desc, pa, pt = heads(field, n_heads)
    n, slot, slotcol = _native.lane_tables(desc, plan.wc, plan.wr, plan.d_out, pa, pt)
    return plan, desc, pa, pt, n, slot, slotcol


@pytest.mark.parametrize("field,n_heads,slots", [
    ({0: 32, 1: 32, 2: 32}, 8, 13),   # the benchmark layer: four copies per frequency and head
    ({0: 16, 1: 16, 2: 16}, 4, 13),
    ({0: 16, 1: 8, 2: 8}, 2, 16),      # eight scalar copies: the scalar output group twice
    ({0: 8, 1: 8}, 2, 5),
])
def test_plans_in_fours_take_the_lane_tables(field, n_heads, slots):
    plan, desc, pa, pt, n, slot, slotcol = tables(field, n_heads)
    assert n == slots
    assert all(w & ACTIVE for w in slot[:n]) and not any(slot[n:])
    assert slot[n - 1] & FLUSH
    C = 2 * plan.wc + plan.wr
    used = [c for c in slotcol if c != 0xFF]
    assert sorted(used) == list(range(C)), "every packed column in exactly one slot column"


@pytest.mark.parametrize("field,n_heads", [({0: 8, 1: 8, 2: 8}, 4), ({0: 6, 1: 3}, 3), ({0: 4, 1: 4, 2: 4}, 2)])
def test_other_plans_take_the_generic_kernels(field, n_heads):
    assert tables(field, n_heads)[4] == 0


def replay(h, Z, ang, tra, rho, slot, slotcol, n, pa, d_out):
    """The lane kernels' forward for edges of one source, from the tables."""
    E = h.shape[0]
    ht = torch.cat([torch.ones(E, 1, dtype=h.dtype), h], dim=1)  # (E, 17)
    out = torch.full((E, d_out), math.nan, dtype=h.dtype)
    NT = (n + 1) // 2
    for q in range(4):
        sr = torch.zeros(E, dtype=h.dtype)
        si = torch.zeros(E, dtype=h.dtype)
        for s in range(2 * NT):
            w = slot[s]
            sc = 16 * (s // 2) + 4 * q + 2 * (s % 2)
            u = [ht @ Z[:, slotcol[sc + c]] if slotcol[sc + c] != 0xFF else torch.zeros(E, dtype=h.dtype)
                 for c in (0, 1)]
            ai, ti = (w >> 11) & 7, (w >> 15) & 7
            A = torch.polar(rho ** ai, ai * ang)
            T = torch.polar(torch.ones_like(rho), (ti - pa) * tra)
            A = A.conj() if w & ACONJ else A
            T = T.conj() if w & TCONJ else T
            v = (A * T) * torch.complex(u[0], u[1])
            sr, si = sr + v.real, si + v.imag
            if w & FLUSH:
                ob = w & 0x7F
                if w & SCALAR:
                    assert torch.isnan(out[:, ob + q]).all()
                    out[:, ob + q] = sr
                else:
                    assert torch.isnan(out[:, ob + 2 * q: ob + 2 * q + 2]).all()
                    out[:, ob + 2 * q], out[:, ob + 2 * q + 1] = sr, si
                sr, si = torch.zeros_like(sr), torch.zeros_like(si)
    return out


@pytest.mark.parametrize("field,n_heads", [({0: 32, 1: 32, 2: 32}, 8), ({0: 16, 1: 8, 2: 8}, 2), ({0: 8, 1: 8}, 2)])
def test_replayed_lane_arithmetic_matches_the_oracle_rows(field, n_heads):
    plan, desc, pa, pt, n, slot, slotcol = tables(field, n_heads)
    assert n > 0
    g = torch.Generator().manual_seed(3)
    E, K, C = 40, 17, 2 * plan.wc + plan.wr
    h = torch.randn(E, K - 1, dtype=torch.float64, generator=g)
    Z = torch.randn(K, C, dtype=torch.float64, generator=g)
    ang = torch.rand(E, dtype=torch.float64, generator=g) * 2 * math.pi
    tra = (torch.rand(E, dtype=torch.float64, generator=g) - 0.5) * 2 * math.pi
    rho = torch.rand(E, dtype=torch.float64, generator=g)
    orders = torch.arange(8, dtype=torch.float64)
    angular = torch.view_as_real(torch.polar(torch.ones(E, 8, dtype=torch.float64), ang[:, None] * orders))
    transport = torch.view_as_real(torch.polar(torch.ones(E, 8, dtype=torch.float64), tra[:, None] * orders))
    zc = Z[:, :2 * plan.wc].reshape(1, K, plan.wc, 2)
    zr = Z[:, 2 * plan.wc:].reshape(1, K, plan.wr)
    want = eager.factored_rows(h, zc, zr, angular, transport, rho, [tuple(int(v) for v in r) for r in desc.tolist()],
                               torch.zeros(E, dtype=torch.long), plan.d_out)
    got = replay(h, Z, ang, tra, rho, slot, slotcol, n, pa, plan.d_out)
    assert not torch.isnan(got).any(), "every output written"
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
