"""luna_uvu_conv_bwd_noalloc (static device scratch, no allocation) against
luna_uvu_conv_bwd (caller workspace), both called through the C-ABI: identical
outputs on two calls in a row, the second with a smaller problem, and a clear
error for a problem whose workspace exceeds the scratch array."""

import ctypes

import pytest
import torch

import lunaequivariance_amd as lunaeq
from lunaequivariance_amd import _native
from lunaequivariance_amd.workloads import mace_irreps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_conv(dtype, channels=16, lmax=2):
    in1, sh, out, ins = mace_irreps(channels, lmax)
    return lunaeq.TensorProductConv(in1, sh, out, ins, internal_weights=False, shared_weights=False, dtype=dtype)


def problem(conv, nodes, edges, seed, dtype, env):
    gen = torch.Generator().manual_seed(seed)
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.sort(torch.randint(nodes, (edges,), generator=gen))[0]
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    x = torch.randn(nodes, conv.irreps_in1.dim, generator=gen, dtype=dtype).to(DEV)
    y = torch.randn(edges, conv.irreps_in2.dim, generator=gen, dtype=dtype).to(DEV)
    w = torch.randn(edges, conv.weight_numel, generator=gen, dtype=dtype).to(DEV)
    g = torch.randn(nodes, conv.irreps_out.dim, generator=gen, dtype=dtype).to(DEV)
    e = torch.randn(edges, generator=gen, dtype=dtype).to(DEV) if env else None
    gl0 = torch.randn(edges, conv.op.l0_dim, generator=gen, dtype=dtype).to(DEV) if env else None
    return graph, x, y, w, g, e, gl0


def outputs(conv, graph, x, dtype, env):
    N, E = graph.num_nodes, graph.num_edges
    gx = torch.full((N, conv.irreps_in1.dim), float("nan"), device=DEV, dtype=dtype)
    gy = torch.full((E, conv.irreps_in2.dim), float("nan"), device=DEV, dtype=dtype)
    gw = torch.full((E, conv.weight_numel), float("nan"), device=DEV, dtype=dtype)
    ge = torch.full((E,), float("nan"), device=DEV, dtype=dtype) if env else None
    return gx, gy, gw, ge


def common_args(conv, graph, x, y, w, g, e, gl0, outs):
    p = _native.ptr
    return [conv.op.plan.handle, x.data_ptr(), y.data_ptr(), w.data_ptr(), p(e), g.data_ptr(), p(gl0),
            graph.src.data_ptr(), graph.dst_rowptr.data_ptr(), graph.node_order.data_ptr(),
            graph.src_rowptr.data_ptr(), graph.edge_ids_by_src.data_ptr(), *[p(t) for t in outs]]


def run_with_workspace(conv, graph, x, y, w, g, e, gl0, dtype, env):
    lib = _native.lib()
    outs = outputs(conv, graph, x, dtype, env)
    size = ctypes.c_size_t()
    _native.check(lib.luna_uvu_conv_bwd_workspace(conv.op.plan.handle, graph.num_nodes, graph.num_edges,
                                                  ctypes.byref(size)), "workspace")
    workspace = torch.empty(size.value, device=DEV, dtype=torch.uint8)
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.luna_uvu_conv_bwd(*common_args(conv, graph, x, y, w, g, e, gl0, outs),
                                        workspace.data_ptr(), size.value, graph.num_nodes, graph.num_edges,
                                        stream), "luna_uvu_conv_bwd")
    torch.cuda.synchronize()
    return outs


def run_noalloc(conv, graph, x, y, w, g, e, gl0, dtype, env):
    lib = _native.lib()
    outs = outputs(conv, graph, x, dtype, env)
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.luna_uvu_conv_bwd_noalloc(*common_args(conv, graph, x, y, w, g, e, gl0, outs),
                                                graph.num_nodes, graph.num_edges, stream),
                  "luna_uvu_conv_bwd_noalloc")
    torch.cuda.synchronize()
    return outs


def assert_same(a, b, what):
    for name, s, t in zip(("gx", "gy", "gw", "genv"), a, b):
        if s is None:
            assert t is None
            continue
        assert not torch.isnan(t).any(), f"{what}: {name} not fully written"
        assert torch.equal(s, t), f"{what}: {name} differs (max {(s - t).abs().max().item():.3e})"


@pytest.mark.parametrize("dtype,env", [(torch.float32, False), (torch.float32, True), (torch.float64, True)])
def test_noalloc_matches_workspace_entry_point(dtype, env):
    conv = make_conv(dtype)
    first = problem(conv, 60, 900, 1, dtype, env)
    second = problem(conv, 23, 170, 2, dtype, env)
    assert conv.op.plan is not None
    for label, case in (("first call", first), ("second, smaller call", second)):
        expected = run_with_workspace(conv, *case, dtype, env)
        actual = run_noalloc(conv, *case, dtype, env)
        assert_same(expected, actual, label)


def test_noalloc_uses_no_torch_allocation_and_rejects_oversized_problems():
    conv = make_conv(torch.float32)
    case = problem(conv, 30, 300, 3, torch.float32, False)
    outs = outputs(conv, case[0], case[1], torch.float32, False)
    lib = _native.lib()
    before = torch.cuda.memory_allocated()
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.luna_uvu_conv_bwd_noalloc(*common_args(conv, *case, outs), 30, 300, stream), "noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    limit = lib.luna_uvu_conv_bwd_noalloc_limit()
    assert limit == 64 << 20
    size = ctypes.c_size_t()
    big = 2_000_000
    _native.check(lib.luna_uvu_conv_bwd_workspace(conv.op.plan.handle, 1000, big, ctypes.byref(size)), "ws")
    assert size.value > limit
    status = lib.luna_uvu_conv_bwd_noalloc(conv.op.plan.handle, *([None] * 15), 1000, big, None)
    assert status != 0
    message = lib.luna_last_error().decode()
    assert "static scratch" in message and str(big) in message
