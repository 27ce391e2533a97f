"""Dispatcher operators and torch.compile (``tests/lunatp/test_uvu_conv.py:1272-1329`` analogue)."""

import pytest
import torch

import lunaequivariance_amd as lunaeq
from lunaequivariance_amd import ops
from lunaequivariance_amd.workloads import mace_irreps
from tests.test_uvu_conv_gpu import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def problem(dtype=torch.float32, channels=8, lmax=2, nodes=12, edges=50, seed=0):
    in1, sh, out, instructions = mace_irreps(channels, lmax)
    conv = lunaeq.TensorProductConv(in1, sh, out, instructions, internal_weights=False, shared_weights=False,
                                    dtype=dtype)
    gen = torch.Generator().manual_seed(seed)
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.sort(torch.randint(nodes, (edges,), generator=gen))[0]
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    x = torch.randn(nodes, conv.irreps_in1.dim, generator=gen, dtype=dtype).to(DEV).requires_grad_()
    y = torch.randn(edges, conv.irreps_in2.dim, generator=gen, dtype=dtype).to(DEV).requires_grad_()
    w = torch.randn(edges, conv.weight_numel, generator=gen, dtype=dtype).to(DEV).requires_grad_()
    return conv, graph, x, y, w


def test_opcheck_forward_and_backward():
    conv, graph, x, y, w = problem()
    tables = ops.graph_tables(graph)
    config = conv.op.torch_config
    torch.library.opcheck(torch.ops.lunaeq_amd.uvu_conv_forward.default,
                          (x, y, w, None, tables, graph.num_nodes, False, config))
    g = torch.randn(graph.num_nodes, conv.irreps_out.dim, device=DEV)
    torch.library.opcheck(torch.ops.lunaeq_amd.uvu_conv_backward.default,
                          (x.detach(), y.detach(), w.detach(), None, g, None, tables, graph.num_nodes,
                           [True, True, True, False], config))


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_module_matches_eager(backend):
    """Forward and first order (aot_autograd does not support double backward)."""
    conv, graph, x, y, w = problem()

    def layer(a, b, c):
        return conv(a, b, c, graph=graph)

    torch._dynamo.reset()
    compiled = torch.compile(layer, backend=backend, fullgraph=True)
    eager_out = layer(x, y, w)
    out = compiled(x, y, w)
    assert_close(out, eager_out.double(), torch.float32, "compiled forward")
    seed = torch.randn_like(out)
    first_e = torch.autograd.grad(eager_out, (x, y, w), seed)
    first_c = torch.autograd.grad(out, (x, y, w), seed)
    for a, b in zip(first_c, first_e):
        assert_close(a, b.double(), torch.float32, "compiled first order")


def test_dispatcher_ops_differentiate_to_second_order():
    """Outside compilation the operators' own autograd composes second order."""
    conv, graph, x, y, w = problem(seed=3)
    tables = ops.graph_tables(graph)
    out, _ = torch.ops.lunaeq_amd.uvu_conv_forward(x, y, w, None, tables, graph.num_nodes, False,
                                                   conv.op.torch_config)
    eager = conv(x, y, w, graph=graph)
    assert_close(out, eager.double(), torch.float32, "op forward")
    seed = torch.randn_like(out)
    first_o = torch.autograd.grad(out, (x, y, w), seed, create_graph=True)
    first_e = torch.autograd.grad(eager, (x, y, w), seed, create_graph=True)
    dirs = [torch.randn_like(t) for t in first_e]
    second_o = torch.autograd.grad(first_o, (x, y, w), dirs)
    second_e = torch.autograd.grad(first_e, (x, y, w), dirs)
    for a, b in zip(second_o, second_e):
        assert_close(a, b.double(), torch.float32, "op second order")


def other_mode_problem(mode, seed=0, nodes=10, edges=40):
    ir = "8x0e+8x1o+8x2e"
    edge = ir if mode == "uuu" else "1x0e+1x1o+1x2e"
    a, b = lunaeq.Irreps(ir), lunaeq.Irreps(edge)
    instructions = [(i, j, k, mode, True) for i, (m, p) in enumerate(a) for j, (n, q) in enumerate(b)
                    for k, (o, r) in enumerate(a) if r in p * q and (mode != "uuu" or m == n == o)]
    conv = lunaeq.TensorProductConv(ir, edge, ir, instructions, internal_weights=False,
                                    shared_weights=mode == "uvw")
    gen = torch.Generator().manual_seed(seed)
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.sort(torch.randint(nodes, (edges,), generator=gen))[0]
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    x = torch.randn(nodes, a.dim, generator=gen).to(DEV).requires_grad_()
    y = torch.randn(edges, b.dim, generator=gen).to(DEV).requires_grad_()
    wshape = (conv.weight_numel,) if mode == "uvw" else (edges, conv.weight_numel)
    w = torch.randn(wshape, generator=gen).to(DEV).requires_grad_()
    return conv, graph, x, y, w


@pytest.mark.parametrize("mode", ["uuu", "uvw"])
def test_compiled_uuu_and_uvw_match_eager(mode):
    """UUU runs through lunaeq_amd::uuu_conv_*, the shared-weight UVW aggregation through
    lunaeq_amd::uvu_conv_* plus library GEMMs; compiled forward and first order equal eager."""
    conv, graph, x, y, w = other_mode_problem(mode)

    def layer(a, b, c):
        return conv(a, b, c, graph=graph)

    torch._dynamo.reset()
    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    eager_out = layer(x, y, w)
    out = compiled(x, y, w)
    assert_close(out, eager_out.double(), torch.float32, f"{mode} compiled forward")
    seed = torch.randn_like(out)
    for a, b in zip(torch.autograd.grad(out, (x, y, w), seed), torch.autograd.grad(eager_out, (x, y, w), seed)):
        assert_close(a, b.double(), torch.float32, f"{mode} compiled first order")


def test_opcheck_uuu():
    conv, graph, x, y, w = other_mode_problem("uuu", seed=2)
    tables = ops.graph_tables(graph)
    config = conv.op.torch_config
    torch.library.opcheck(torch.ops.lunaeq_amd.uuu_conv_forward.default,
                          (x, y, w, None, tables, graph.num_nodes, False, config))
    g = torch.randn(graph.num_nodes, conv.irreps_out.dim, device=DEV)
    torch.library.opcheck(torch.ops.lunaeq_amd.uuu_conv_backward.default,
                          (x.detach(), y.detach(), w.detach(), None, g, None, tables, graph.num_nodes,
                           [True, True, True, False], config))


def test_uuu_dispatcher_ops_second_order_with_unweighted_paths():
    """The dispatcher ops' double backward substitutes weight directions through the
    weight-linear operator (unweighted paths make the product affine in w)."""
    ir = "8x0e+8x1o"
    a = lunaeq.Irreps(ir)
    paths = [(i, j, k, "uuu", n % 2 == 0)
             for n, (i, j, k) in enumerate((i, j, k) for i, (_, p) in enumerate(a) for j, (_, q) in enumerate(a)
                                          for k, (_, r) in enumerate(a) if r in p * q)]
    conv = lunaeq.TensorProductConv(ir, ir, ir, paths, internal_weights=False, shared_weights=False)
    gen = torch.Generator().manual_seed(5)
    nodes, edges = 9, 30
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.sort(torch.randint(nodes, (edges,), generator=gen))[0]
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    x = torch.randn(nodes, a.dim, generator=gen).to(DEV).requires_grad_()
    y = torch.randn(edges, a.dim, generator=gen).to(DEV).requires_grad_()
    w = torch.randn(edges, conv.weight_numel, generator=gen).to(DEV).requires_grad_()
    out, _ = torch.ops.lunaeq_amd.uuu_conv_forward(x, y, w, None, ops.graph_tables(graph), nodes, False,
                                                   conv.op.torch_config)
    eager = conv(x, y, w, graph=graph)
    assert_close(out, eager.double(), torch.float32, "uuu op forward")
    seed = torch.randn_like(out)
    first_o = torch.autograd.grad(out, (x, y, w), seed, create_graph=True)
    first_e = torch.autograd.grad(eager, (x, y, w), seed, create_graph=True)
    dirs = [torch.randn_like(t) for t in first_e]
    for a_, b_ in zip(torch.autograd.grad(first_o, (x, y, w), dirs), torch.autograd.grad(first_e, (x, y, w), dirs)):
        assert_close(a_, b_.double(), torch.float32, "uuu op second order")
