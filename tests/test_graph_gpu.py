"""The layer's forward captured in a HIP graph (torch.cuda.CUDAGraph): every
native entry point it calls launches on the current stream, allocates only
through torch and neither synchronises nor sets memory, so a capture replays
the eager kernels.  Each replay, with eager steps and synchronisations between
replays, must equal the eager forward bit for bit (the kernels are
deterministic): C1's configuration (4 heads, {0:16,1:16,2:16}, 32x64, one
sample) and the headline's heads on a small grid."""

import pytest
import torch

import problems
from gm_attention_amd.nn.attention import SO2MHSA
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nlat,nlon,batch,heads,field", [
    (32, 64, 1, 4, {0: 16, 1: 16, 2: 16}),
    (16, 32, 2, 8, {0: 32, 1: 32, 2: 32}),
])
def test_forward_graph_replays_equal_the_eager_forward(nlat, nlon, batch, heads, field, cuda):
    disc = problems.discretization(nlat, nlon)
    edges = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes).to(cuda, torch.float32)
    ft = SO2FieldType(field)
    torch.manual_seed(0)
    mhsa = SO2MHSA(ft, heads, cutoff=disc.coverage_radius, window="hard", batched=True, dtype=torch.float32,
                   device=cuda)
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, ft.dimension), 3).float().to(cuda)

    def forward():
        return mhsa(SO2FeatureField.from_flat(ft, x), edges)._rows()

    print(f"graph {nlat}x{nlon} B={batch} H={heads}", flush=True)
    with torch.no_grad():
        want = forward().clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                forward()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = forward()
        for replay in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), f"replay {replay}"
            eager = forward()  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(eager, want)
