"""Graph construction, ordering and ownership (``tests/lunatp/test_make_graph.py:9-55``)."""

import pytest
import torch

from lunaequivariance_amd import make_graph


def test_destination_sorted_endpoints_are_preserved():
    src = torch.tensor([2, 0, 1])
    dst = torch.tensor([0, 1, 2])
    graph = make_graph(src, dst, 4)
    assert torch.equal(graph.dst, dst.to(graph.dst.dtype))
    assert torch.equal(graph.src, src.to(graph.src.dtype))
    assert graph.dst_rowptr.tolist() == [0, 1, 2, 3, 3]


def test_invalid_graph_includes_values():
    with pytest.raises(ValueError, match="num_nodes=2.*at least 4"):
        make_graph(torch.tensor([3]), torch.tensor([0]), 2)
    with pytest.raises(ValueError, match="nonnegative"):
        make_graph(torch.tensor([-1]), torch.tensor([0]), 2)
    with pytest.raises(ValueError, match="sorted"):
        make_graph(torch.tensor([0, 1]), torch.tensor([1, 0]), 2)
    with pytest.raises(TypeError):
        make_graph(torch.tensor([0.0]), torch.tensor([0.0]), 1)
    with pytest.raises(ValueError, match="equal shape"):
        make_graph(torch.tensor([0, 1]), torch.tensor([0]), 2)


def test_source_edge_order_is_generated():
    src = torch.tensor([2, 0, 1, 0])
    dst = torch.tensor([0, 1, 1, 2])
    graph = make_graph(src, dst, 3)
    assert graph.dst.tolist() == [0, 1, 1, 2]
    assert graph.src[graph.edge_ids_by_src.long()].tolist() == [0, 0, 1, 2]
    assert graph.src_rowptr.tolist() == [0, 2, 3, 4]


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_generated_graph_tables_and_input_ownership(dtype):
    src = torch.tensor([2, 0, 1, 0], dtype=dtype)
    dst = torch.tensor([0, 1, 1, 2], dtype=dtype)
    graph = make_graph(src, dst, 4)
    assert graph.src_rowptr.tolist() == [0, 2, 3, 4, 4]
    assert graph.dst_rowptr.tolist() == [0, 1, 3, 4, 4]
    assert graph.edge_ids_by_src.sort().values.tolist() == [0, 1, 2, 3]
    assert graph.src[graph.edge_ids_by_src.long()].tolist() == [0, 0, 1, 2]
    assert graph.edge_ids_by_dst.tolist() == [0, 1, 2, 3]
    for rowptr, order in ((graph.dst_rowptr, graph.node_order), (graph.src_rowptr, graph.source_node_order)):
        assert order.sort().values.tolist() == [0, 1, 2, 3]
        assert rowptr.diff()[order.long()].tolist() == [2, 1, 1, 0]
    assert graph.src.data_ptr() != src.data_ptr()
    assert graph.dst.data_ptr() != dst.data_ptr()
    src.zero_()
    dst.zero_()
    assert graph.src.tolist() == [2, 0, 1, 0]
    assert graph.dst.tolist() == [0, 1, 1, 2]


def test_stable_source_permutation_and_column_shapes():
    """Equal sources keep destination order; [E, 1] inputs are accepted."""
    src = torch.tensor([[1], [0], [1], [1], [0]])
    dst = torch.tensor([[0], [0], [1], [2], [2]])
    graph = make_graph(src, dst)
    assert graph.num_nodes == 3
    assert graph.edge_ids_by_src.tolist() == [1, 4, 0, 2, 3]


def test_empty_graph_and_segments():
    empty = torch.zeros(0, dtype=torch.int64)
    graph = make_graph(empty, empty, 5)
    assert graph.dst_rowptr.tolist() == [0] * 6
    assert graph.node_tiers.tolist() == [5, 5, 5]
    assert graph.source_segments.nodes.tolist() == [0, 1, 2, 3, 4]
    assert make_graph(empty, empty).num_nodes == 0


def test_source_segments_split_long_rows():
    """Rows longer than 32 edges are cut into 32-edge segments (uvu_conv/graph.py:38-99)."""
    src = torch.cat([torch.zeros(70, dtype=torch.int64), torch.ones(5, dtype=torch.int64)])
    dst = torch.arange(75)
    graph = make_graph(src, dst, 75)
    seg = graph.source_segments
    assert seg.rowptr[:3].tolist() == [0, 3, 4]
    assert (seg.end - seg.begin)[:4].tolist() == [32, 32, 6, 5]
    assert seg.nodes[:4].tolist() == [0, 0, 0, 1]
    assert seg.order[:2].tolist() == [0, 1]


def test_node_tiers():
    """Prefix lengths of node_order covering a quarter, half and three quarters of the edges."""
    dst = torch.tensor([0] * 8 + [1] * 4 + [2] * 2 + [3] * 2)
    src = torch.zeros(16, dtype=torch.int64)
    graph = make_graph(src, dst, 4)
    assert graph.node_order.tolist() == [0, 1, 2, 3]
    assert graph.node_tiers.tolist() == [1, 1, 2]
