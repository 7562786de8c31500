"""Head shares (fused_factored.SubHead / heads_mixing(split) / share_columns) and
channel groups (depthwise_radial.channel_groups / Packing(group)) on the CPU.

A value head too wide for the grouped kernels runs as shares of its output
copies.  Replaying the descriptor semantics the kernels implement (rows of
``F_b (sum_t h~_t Z_t)`` per block, ``F_b = e^{i a phi} e^{i s gamma} rho^p``)
in float64 on the shares' mixes, and putting the shares side by side with
``share_columns``, must give every head's rows as the eager path computes
them (nn/eager_ops.factored_rows, itself checked against the oracle).  The
depthwise groups must partition the copies, read exactly the layout's
columns and map readout rows one-to-one onto the full kernel's rows."""

import pytest
import torch

import problems
from gm_attention_amd.nn import depthwise_radial, eager_ops, fused_factored
from gm_attention_amd.nn.attention import SO2MHSA
from gm_attention_amd.nn.convolution import SO2Convolution
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType


def _phase(table, order):
    column = table[:, abs(order)]
    return column.conj() if order < 0 else column


def replay_rows(hp, mixes, share, n_shares, h, x_edges_source, edges, cutoff):
    """One share's rows ``(E, d_out)`` from the heads' mix arrays: the packed
    complex columns are every input frequency's complex columns in group
    order, the real block's columns follow (the layout the kernels read)."""
    p = hp.plan
    N = mixes[0].shape[0]
    K = h.shape[1] + 1
    zc, zr = [], []
    for (n, _blocks, cw, rw), mix in zip(hp.groups, mixes, strict=True):
        view = mix.reshape(N, n_shares, K, cw + rw)[:, share]
        zc.append(view[..., :cw])
        zr.append(view[..., cw:])
    zc = torch.cat(zc, dim=-1)
    zr = torch.cat(zr, dim=-1)
    hk = torch.cat([torch.ones_like(h[:, :1]), h], dim=1)  # (E, K)
    rho = edges.distances / cutoff
    E = h.shape[0]
    rows = h.new_zeros(E, p.d_out)
    for kind, zo, bm, ang, tr, power, out, take_real in hp.desc_rows:
        if kind == 0:
            z = zr.index_select(0, x_edges_source)  # (E, K, wr)
            rows[:, out:out + bm] += torch.einsum("et,etb->eb", hk, z[..., :bm])
            continue
        pairs = zc[..., 2 * zo:2 * (zo + bm)].reshape(N, K, bm, 2)
        z = torch.view_as_complex(pairs.contiguous()).index_select(0, x_edges_source)
        combined = torch.einsum("et,etb->eb", hk.to(z.dtype), z)
        factor = _phase(edges.angular_phases, ang) * _phase(edges.transport_phases, tr)
        if power:
            factor = factor * rho.pow(power).to(factor.dtype)
        term = factor.unsqueeze(-1) * combined
        if take_real:
            rows[:, out:out + bm] += term.real
        else:
            rows[:, out:out + 2 * bm] += torch.view_as_real(term).reshape(E, 2 * bm)
    return rows


@pytest.mark.parametrize("field,n_heads,split", [({0: 16, 1: 16, 2: 16}, 2, 2), ({0: 8, 1: 16, 2: 8}, 1, 4),
                                                 ({0: 4, 2: 8}, 1, 2)])
def test_shares_side_by_side_are_the_heads_rows(field, n_heads, split):
    disc = problems.discretization(8, 16)
    edges = disc.edge_geometry
    torch.manual_seed(3)
    mhsa = SO2MHSA(SO2FieldType(field), n_heads, cutoff=disc.coverage_radius, dtype=torch.float64)
    with torch.no_grad():
        for p in mhsa.parameters():
            p.add_(0.1 * torch.randn_like(p))
    kernels = [h.value for h in mhsa.heads]
    x = SO2FeatureField.from_flat(mhsa.field_type_in, problems.normal((disc.n_nodes, mhsa.field_type_in.dimension), 4))
    unit = fused_factored.sub_head(kernels[0], split)
    assert unit.field_type_out.dimension * split == kernels[0].field_type_out.dimension
    hp = fused_factored.heads_plan(unit)
    mats = fused_factored.heads_mixing(kernels, hp, split)
    mixes = [v @ m for v, m in zip(fused_factored.node_vectors(x, hp), mats, strict=True)]
    shares = []
    for v in range(n_heads * split):
        kernel = kernels[v // split]
        h = kernel._trunk_hidden(edges.distances)
        shares.append(replay_rows(hp, mixes, v, n_heads * split, h, edges.source_index, edges,
                                  kernel.radial_basis.cutoff))
    side = torch.stack(shares, dim=1).reshape(edges.n_edges, -1)
    got = side.index_select(1, fused_factored.share_columns(kernels[0], split, n_heads, torch.device("cpu")))
    got = got.reshape(edges.n_edges, n_heads, -1)
    for head, kernel in enumerate(kernels):
        want = eager_ops.factored_rows(kernel, x, edges)
        torch.testing.assert_close(got[:, head], want, rtol=1e-11, atol=1e-12)


def test_the_c5_heads_split_in_two():
    """{0: 64, 1: 64, 2: 64} in 8 heads and {0: 128, 1: 128, 2: 128} in 16: heads
    of {0: 8, 1: 8, 2: 8} (packed width 200) run as two shares of the headline
    layer's shape (48 complex, 4 real columns)."""
    for field, n_heads in (({0: 64, 1: 64, 2: 64}, 8), ({0: 128, 1: 128, 2: 128}, 16)):
        mhsa = SO2MHSA(SO2FieldType(field), n_heads, cutoff=0.1, dtype=torch.float32)
        kernel = mhsa.heads[0].value
        assert fused_factored.head_split(kernel, 17) == 2
        p = fused_factored.heads_plan(fused_factored.sub_head(kernel, 2)).plan
        assert (p.wc, p.wr, p.d_out) == (48, 4, 20)


@pytest.mark.parametrize("field,groups", [({0: 64, 1: 64, 2: 64}, 2), ({0: 128, 1: 128, 2: 128}, 4),
                                          ({0: 32, 1: 32, 2: 32}, None), ({0: 36, 1: 4}, ())])
def test_depthwise_channel_groups_partition_the_copies(field, groups):
    ft = SO2FieldType(field)
    got = depthwise_radial.channel_groups(ft)
    if groups is None or groups == ():
        assert got == groups
        return
    assert len(got) == groups
    conv = SO2Convolution(ft, ft, cutoff=0.1, depthwise=True, dtype=torch.float32)
    kernel = conv.kernel
    n_rows = ft.multiplicity(0) + sum(4 * m for n, m in ft.items() if n != 0)  # real rows, then complex rows
    cols, rows = [], []
    for g in got:
        p = depthwise_radial.packing(kernel, torch.device("cpu"), g)
        assert p.a0 <= 16 * depthwise_radial.NS and p.tiles.shape[1] <= depthwise_radial.NC
        cols.append(p.columns)
        rows.append(p.rowmap[p.rowmap != n_rows])  # row n_rows is the zero row padding the tiles
        # the tiles point at whole copies of the group's own layout
        assert int(p.tiles[1].max()) + 8 <= p.columns.shape[0]
    cols, rows = torch.cat(cols), torch.cat(rows)
    assert torch.equal(cols.sort().values, torch.arange(ft.dimension))
    assert torch.equal(rows.sort().values, torch.arange(n_rows))
