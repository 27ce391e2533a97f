"""The HIP graph builder against the torch-operation builder, table by table.

Both builders order stably (ties keep edge / node order), so the tables must be
identical (integer work: bit-exact).  Cases follow the reference's graph tests
(``tests/lunatp/test_make_graph.py:9-55``) plus empty, isolated-node, hub and
full config-2 graphs.
"""

import pytest
import torch

from lunaequivariance_amd import make_graph
from lunaequivariance_amd.workloads import periodic_radius_graph

pytestmark = pytest.mark.gpu
DEV = "cuda"


def tables(graph):
    seg = graph.source_segments
    return {
        "src": graph.src, "dst": graph.dst, "dst_rowptr": graph.dst_rowptr, "src_rowptr": graph.src_rowptr,
        "edge_ids_by_src": graph.edge_ids_by_src, "edge_ids_by_dst": graph.edge_ids_by_dst,
        "node_order": graph.node_order, "source_node_order": graph.source_node_order,
        "node_tiers": graph.node_tiers, "seg_nodes": seg.nodes, "seg_begin": seg.begin, "seg_end": seg.end,
        "seg_rowptr": seg.rowptr, "seg_order": seg.order,
    }


def assert_same_graph(src, dst, num_nodes=None):
    print(f"graph: edges={src.numel()} num_nodes={num_nodes} dtype={src.dtype}", flush=True)
    ref = make_graph(src.cpu(), dst.cpu(), num_nodes)
    dev = make_graph(src.to(DEV), dst.to(DEV), num_nodes)
    assert dev.num_nodes == ref.num_nodes
    for name, expected in tables(ref).items():
        actual = tables(dev)[name]
        assert actual.is_cuda and actual.dtype == torch.int32, name
        assert torch.equal(actual.cpu(), expected.to(torch.int32)), name
    return dev


def random_graph(num_nodes, num_edges, seed, hub=None, dtype=torch.int64):
    gen = torch.Generator().manual_seed(seed)
    src = torch.randint(0, num_nodes, (num_edges,), generator=gen)
    dst = torch.randint(0, num_nodes, (num_edges,), generator=gen)
    if hub is not None:
        src[: num_edges // 2] = hub
    dst, order = torch.sort(dst, stable=True)
    return src[order].to(dtype), dst.to(dtype)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_reference_cases(dtype):
    assert_same_graph(torch.tensor([2, 0, 1], dtype=dtype), torch.tensor([0, 1, 2], dtype=dtype), 4)
    assert_same_graph(torch.tensor([2, 0, 1, 0], dtype=dtype), torch.tensor([0, 1, 1, 2], dtype=dtype), 3)
    graph = assert_same_graph(torch.tensor([2, 0, 1, 0], dtype=dtype), torch.tensor([0, 1, 1, 2], dtype=dtype), 4)
    assert graph.src_rowptr.tolist() == [0, 2, 3, 4, 4]
    assert graph.dst_rowptr.tolist() == [0, 1, 3, 4, 4]


def test_empty_and_isolated():
    empty = torch.zeros(0, dtype=torch.int64)
    assert_same_graph(empty, empty, 0)
    assert_same_graph(empty, empty, 5)
    assert_same_graph(torch.zeros(10, dtype=torch.int64), torch.zeros(10, dtype=torch.int64))
    assert_same_graph(torch.tensor([0, 3]), torch.tensor([1, 1]), 9)


@pytest.mark.parametrize("num_nodes,num_edges,hub", [
    (1000, 16000, None),     # config 1 shape
    (3000, 20000, 7),        # one source with 10,000 out-edges (many segments, several sort tiles)
    (70000, 50000, None),    # more nodes than edges; node ids beyond 16 bits
    (17, 5000, 3),           # dense multigraph
])
def test_random_graphs(num_nodes, num_edges, hub):
    for dtype in (torch.int32, torch.int64):
        assert_same_graph(*random_graph(num_nodes, num_edges, num_nodes + num_edges, hub, dtype), num_nodes)


def test_config2_graph():
    src, dst, *_ = periodic_radius_graph(20000, 0.1, 5.0, seed=0)
    assert_same_graph(src, dst, 20000)


def test_errors_match_the_host_path():
    with pytest.raises(ValueError, match="num_nodes=2.*at least 4"):
        make_graph(torch.tensor([3], device=DEV), torch.tensor([0], device=DEV), 2)
    with pytest.raises(ValueError, match="nonnegative"):
        make_graph(torch.tensor([-1], device=DEV), torch.tensor([0], device=DEV), 2)
    with pytest.raises(ValueError, match="sorted"):
        make_graph(torch.tensor([0, 1], device=DEV), torch.tensor([1, 0], device=DEV), 2)
    graph = make_graph(torch.tensor([0, 1], device=DEV), torch.tensor([0, 1], device=DEV))
    assert graph.num_nodes == 2
