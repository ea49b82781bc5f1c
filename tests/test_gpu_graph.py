"""HIP-graph capture of the cells' forward.

Every entry point enqueues its kernels on the caller's stream and neither
allocates, synchronises nor clears memory with hipMemsetAsync, so a cell's
forward can be captured once (torch.cuda.graph, the HIP graph API underneath)
and replayed: the launch-bound small configurations then pay one graph launch
per layer call instead of one host round trip per kernel.  A captured forward
must replay to the eager result bit for bit, replay after replay, with new
input contents copied into the static input and eager work (other forwards,
host synchronisations) between the replays.
"""
import pytest

from tests.gpu_util import print_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cells():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cssm_amd import cells as c
    return c


# (name, cell kwargs, input shape, input dtype): the power-of-two and the small-plane gated scans,
# the fused 32 x 32 GDN core with the frame-sequential qkv projection, and the three-kernel GDN core
CASES = [
    ("gated_32", dict(channels=16, kernel_size=7), (2, 3, 32, 32, 16), torch.float32),
    ("gated_14_bf16", dict(channels=32, kernel_size=5, expand=2, short_conv_size=0, short_conv_spatial_size=0),
     (4, 1, 14, 14, 32), torch.bfloat16),
    ("gdn_32", dict(channels=16, delta_key_dim=4, gate_type="factored", kernel_size=7, short_conv_size=4),
     (1, 8, 32, 32, 16), torch.float32),
    ("gdn_16", dict(channels=8, delta_key_dim=2, gate_type="channel", kernel_size=5, short_conv_size=3),
     (2, 3, 16, 16, 8), torch.float32),
]


@pytest.mark.parametrize("name,kw,shape,dtype", CASES, ids=[c[0] for c in CASES])
def test_cell_forward_replays_from_a_graph(cells, name, kw, shape, dtype):
    print_case(test="graph_replay", case=name, shape=shape)
    cls = cells.GatedCSSM if name.startswith("gated") else cells.GatedDeltaNetCSSM
    cell = cls(**kw)
    variables = cell.init(3, shape)
    g = torch.Generator(device="cuda").manual_seed(5)
    xs = [torch.randn(shape, generator=g, device="cuda").to(dtype) for _ in range(3)]
    static_x = xs[0].clone()
    # warm up on a side stream (the derived weights are computed and cached eagerly, as torch's
    # capture recipe asks); default stream priority
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            cell.apply(variables, static_x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = cell.apply(variables, static_x)
    torch.cuda.synchronize()
    for i, x in enumerate(xs + xs[::-1]):
        ref = cell.apply(variables, x)          # eager work between the replays
        torch.cuda.synchronize()
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y, ref), f"{name}: replay {i} differs from the eager forward"


def test_entry_points_enqueue_on_the_current_stream(cells):
    """The raw stream handle the bindings pass is torch's current stream, on a side stream too
    (what graph capture and multi-stream callers rely on)."""
    from cssm_amd import spectral as S
    assert S._stream() == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert S._stream() == side.cuda_stream
    assert S._stream() == torch.cuda.current_stream().cuda_stream
