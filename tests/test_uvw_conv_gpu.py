"""GPU parity of the UVW convolution (HIP aggregation + per-path GEMMs) against the fp64 oracle.

Tolerance as for the UVU tests: max error <= rtol * max|reference| + atol with
(1e-5, 1e-7) in fp32 and (1e-11, 1e-14) in fp64.  Cases follow the reference's
UVW conv tests (``tests/lunatp/test_uvw_conv.py``): shared and per-edge weights
through third order, envelopes, several edge channels, internal weights, empty
graphs.
"""

import pytest
import torch

import lunaequivariance_amd as lunaeq
from oracle.uvu_conv import conv as oracle_conv
from tests.test_uvu_conv_gpu import DEV, assert_close, random_graph

pytestmark = pytest.mark.gpu


def uvw_paths(in1, in2, out):
    a, b, c = lunaeq.Irreps(in1), lunaeq.Irreps(in2), lunaeq.Irreps(out)
    return [(i, j, k, "uvw", True) for i, (_, x) in enumerate(a) for j, (_, y) in enumerate(b)
            for k, (_, z) in enumerate(c) if z in x * y]


def check(in1, in2, out, nodes, edges, dtype, shared, seed, env=False, orders=3):
    print(f"uvw conv: {in1} x {in2} -> {out} nodes={nodes} edges={edges} {dtype} shared={shared} env={env}",
          flush=True)
    ins = uvw_paths(in1, in2, out)
    module = lunaeq.TensorProductConv(in1, in2, out, ins, internal_weights=False, shared_weights=shared,
                                      dtype=dtype)
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(nodes, module.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(edges, module.irreps_in2.dim, generator=gen, dtype=torch.float64)
    wshape = (module.weight_numel,) if shared else (edges, module.weight_numel)
    w = torch.randn(wshape, generator=gen, dtype=torch.float64)
    src, dst = random_graph(nodes, edges, gen)
    e = torch.rand(edges, generator=gen, dtype=torch.float64) if env else None
    refs = [t.clone().requires_grad_() for t in (x, y, w)] + ([e.clone().requires_grad_()] if env else [])
    wexp = refs[2].expand(edges, -1) if shared else refs[2]
    ref = oracle_conv(in1, in2, out, ins, refs[0], refs[1], wexp, src, dst, nodes, env=refs[3] if env else None)
    devs = [t.to(DEV, dtype).requires_grad_() for t in (x, y, w)] + ([e.to(DEV, dtype).requires_grad_()] if env else [])
    graph = module.create_graph(src.to(DEV), dst.to(DEV), nodes)
    act = module(devs[0], devs[1], devs[2], graph=graph, env=devs[3] if env else None)
    assert_close(act, ref, dtype, "forward")
    if orders < 1:
        return
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    rg, dg = g.clone().requires_grad_(), g.to(DEV, dtype).requires_grad_()
    ref1 = torch.autograd.grad(ref, refs, rg, create_graph=True)
    act1 = torch.autograd.grad(act, devs, dg, create_graph=True)
    for n, (a, r) in enumerate(zip(act1, ref1)):
        assert_close(a, r, dtype, f"first-order {n}")
    if orders < 2:
        return
    dirs = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in ref1]
    ref2 = torch.autograd.grad(ref1, refs + [rg], dirs, create_graph=True, allow_unused=True)
    act2 = torch.autograd.grad(act1, devs + [dg], [d.to(DEV, dtype) for d in dirs], create_graph=True,
                               allow_unused=True)
    for n, (a, r) in enumerate(zip(act2, ref2)):
        if r is None:
            assert a is None or not a.count_nonzero()
            continue
        assert_close(torch.zeros_like(r) if a is None else a, r, dtype, f"second-order {n}")
    if orders < 3:
        return
    pairs = [(a, r) for a, r in zip(act2, ref2) if r is not None and r.requires_grad and a is not None]
    seeds = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for _, r in pairs]
    ref3 = torch.autograd.grad([r for _, r in pairs], refs + [rg], seeds, allow_unused=True)
    act3 = torch.autograd.grad([a for a, _ in pairs], devs + [dg], [s.to(DEV, dtype) for s in seeds],
                               allow_unused=True)
    for n, (a, r) in enumerate(zip(act3, ref3)):
        if r is None:
            assert a is None or not a.count_nonzero()
            continue
        assert_close(torch.zeros_like(r) if a is None else a, r, dtype, f"third-order {n}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shared", [False, True])
def test_reference_problem_all_orders(dtype, shared):
    """The reference's problem: 32x0e+32x1o x 1x0e+1x1o -> 32x0e+32x1o, 7 nodes, 19 edges."""
    check("32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o", 7, 19, dtype, shared, 731)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shared", [False, True])
def test_envelope_all_orders(dtype, shared):
    check("8x0e+8x1o+4x2e", "1x0e+1x1o+1x2e", "8x0e+8x1o+4x2e", 9, 40, dtype, shared, 17, env=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shared", [False, True])
def test_several_edge_channels_and_distinct_multiplicities(dtype, shared):
    """Edge irreps with several channels, output multiplicities unlike the input's, uncovered outputs."""
    check("4x0e+3x1o", "2x0e+3x1o", "5x0e+2x1o+2x2e+1x1e", 6, 25, dtype, shared, 29, env=True, orders=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_wide_channels(dtype):
    check("96x0e+96x1o", "1x0e+1x1o", "96x0e+96x1o", 30, 150, dtype, True, 3, orders=1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shared", [False, True])
def test_empty_graph(dtype, shared):
    ins = uvw_paths("4x0e+4x1o", "1x0e+1x1o", "4x0e+4x1o")
    module = lunaeq.TensorProductConv("4x0e+4x1o", "1x0e+1x1o", "4x0e+4x1o", ins, internal_weights=False,
                                      shared_weights=shared, dtype=dtype)
    x = torch.randn(5, 16, device=DEV, dtype=dtype, requires_grad=True)
    y = torch.randn(0, 4, device=DEV, dtype=dtype, requires_grad=True)
    w = torch.randn((module.weight_numel,) if shared else (0, module.weight_numel), device=DEV, dtype=dtype,
                    requires_grad=True)
    empty = torch.zeros(0, dtype=torch.int64, device=DEV)
    out = module(x, y, w, graph=module.create_graph(empty, empty, 5))
    assert out.shape == (5, 16) and not out.count_nonzero()
    for value, grad in zip((x, y, w), torch.autograd.grad(out.sum(), (x, y, w))):
        assert grad.shape == value.shape and not grad.count_nonzero()


def test_internal_weights_train():
    """Internal shared weights are the module's parameter and receive gradients."""
    ins = uvw_paths("2x1o", "2x1o", "2x0e")
    module = lunaeq.TensorProductConv("2x1o", "2x1o", "2x0e", ins, internal_weights=True, shared_weights=True,
                                      dtype=torch.float64).to(DEV)
    gen = torch.Generator().manual_seed(42)
    x = torch.randn(3, 6, generator=gen, dtype=torch.float64)
    y = torch.randn(4, 6, generator=gen, dtype=torch.float64)
    src, dst = torch.tensor([1, 2, 0, 1]), torch.tensor([0, 0, 1, 2])
    graph = module.create_graph(src.to(DEV), dst.to(DEV), 3)
    out = module(x.to(DEV), y.to(DEV), graph=graph)
    weight = module.weight.detach().cpu().clone().requires_grad_()
    ref = oracle_conv("2x1o", "2x1o", "2x0e", ins, x, y, weight.expand(4, -1), src, dst, 3)
    assert_close(out, ref, torch.float64, "internal forward")
    out.sum().backward()
    (gw,) = torch.autograd.grad(ref.sum(), weight)
    assert_close(module.weight.grad, gw, torch.float64, "internal weight gradient")


@pytest.mark.parametrize("mode", ["uvu", "uuu", "uvw"])
def test_zero_nodes(mode):
    """A graph with no nodes and no edges gives empty outputs and gradients in every mode."""
    ir = "4x0e+4x1o"
    edge = ir if mode == "uuu" else "1x0e+1x1o"
    a, b = lunaeq.Irreps(ir), lunaeq.Irreps(edge)
    ins = [(i, j, k, mode, True) for i, (m, p) in enumerate(a) for j, (n, q) in enumerate(b)
           for k, (o, r) in enumerate(a) if r in p * q and (mode != "uuu" or m == n == o)]
    module = lunaeq.TensorProductConv(ir, edge, ir, ins, internal_weights=False, shared_weights=False)
    empty = torch.zeros(0, dtype=torch.int64, device=DEV)
    graph = module.create_graph(empty, empty, 0)
    x = torch.randn(0, a.dim, device=DEV, requires_grad=True)
    y = torch.randn(0, b.dim, device=DEV, requires_grad=True)
    w = torch.randn(0, module.weight_numel, device=DEV, requires_grad=True)
    out = module(x, y, w, graph=graph)
    assert out.shape == (0, a.dim)
    grads = torch.autograd.grad(out.sum(), (x, y, w), allow_unused=True)
    for value, grad in zip((x, y, w), grads):
        assert grad is None or grad.shape == value.shape
