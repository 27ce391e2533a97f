"""GPU parity of the HIP UUU convolution against the fp64 CPU oracle.

Same tolerance as the UVU tests: max error <= rtol * max|reference| + atol with
(rtol, atol) = (1e-5, 1e-7) for fp32 and (1e-11, 1e-14) for fp64.  Cases follow
the reference's UUU conv tests (``tests/lunatp/test_uuu_conv.py``: forward,
derivatives through third order, empty graphs, fp64 gradcheck, shared weights)
plus channel counts that exercise the several-edges-per-wave lanes (8, 32),
several chunks (96, 130), unweighted paths, env and scalar features, and
configurations whose backward is cut into several launches.
"""

import pytest
import torch

import lunaequivariance_amd as lunaeq
from oracle.uvu_conv import conv as oracle_conv
from tests.test_uvu_conv_gpu import DEV, assert_close, check_orders, random_graph

pytestmark = pytest.mark.gpu


def uuu_paths(in1, in2, out, unweighted=()):
    a, b, c = lunaeq.Irreps(in1), lunaeq.Irreps(in2), lunaeq.Irreps(out)
    paths = [(i, j, k, "uuu", True) for i, (m, x) in enumerate(a) for j, (n, y) in enumerate(b)
             for k, (o, z) in enumerate(c) if z in x * y and m == n == o]
    return [p[:4] + (False,) if n in unweighted else p for n, p in enumerate(paths)]


def irreps(channels, lmax):
    return "+".join(f"{channels}x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(lmax + 1))


def make(in1, in2, out, instructions, dtype):
    return lunaeq.TensorProductConv(in1, in2, out, instructions, internal_weights=False,
                                    shared_weights=False, dtype=dtype)


def run_case(in1, in2, out, instructions, nodes, edges, dtype, seed, env=False, l0=False, orders=3):
    print(f"uuu case: {in1} x {in2} -> {out} nodes={nodes} edges={edges} {dtype} env={env} l0={l0}",
          flush=True)
    gen = torch.Generator().manual_seed(seed)
    conv = make(in1, in2, out, instructions, dtype)
    x = torch.randn(nodes, conv.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(edges, conv.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(edges, conv.weight_numel, generator=gen, dtype=torch.float64)
    src, dst = random_graph(nodes, edges, gen)
    e = torch.rand(edges, generator=gen, dtype=torch.float64) if env else None
    check_orders(conv, in1, in2, out, instructions, x, y, w, src, dst, nodes, dtype, gen, env=e, l0=l0,
                 orders=orders)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_reference_problem_all_orders(dtype):
    """The reference's UUU conv problem: 32x0e+32x1o on both inputs, all paths, 7 nodes, 19 edges."""
    ir = "32x0e+32x1o"
    run_case(ir, ir, ir, uuu_paths(ir, ir, ir), 7, 19, dtype, 731)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_docs_dot_product_closed_form(dtype):
    """8x1o x 8x1o -> 8x0e (docs/operators/tensor_product.md:108-130): msg = w * <x_u, y_u> / sqrt(3)."""
    gen = torch.Generator().manual_seed(0)
    conv = make("8x1o", "8x1o", "8x0e", [(0, 0, 0, "uuu", True)], dtype)
    x = torch.randn(10, 24, generator=gen, dtype=torch.float64)
    y = torch.randn(40, 24, generator=gen, dtype=torch.float64)
    w = torch.randn(40, 8, generator=gen, dtype=torch.float64)
    src = torch.randint(10, (40,), generator=gen)
    dst = torch.arange(10).repeat_interleave(4)
    msg = (x[src].reshape(40, 8, 3) * y.reshape(40, 8, 3)).sum(-1) * w / 3 ** 0.5
    expected = torch.zeros(10, 8, dtype=torch.float64).index_add(0, dst, msg)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), 10)
    out = conv(x.to(DEV, dtype), y.to(DEV, dtype), w.to(DEV, dtype), graph=graph)
    assert_close(out, expected, dtype, "closed form")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("channels", [1, 8, 33, 96, 130])
def test_channel_counts(dtype, channels):
    """Several edges per wave (1, 8, 33 channels) and several 64-channel chunks (96, 130)."""
    ir = irreps(channels, 1)
    run_case(ir, ir, ir, uuu_paths(ir, ir, ir), 23, 90, dtype, channels, orders=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("env,l0", [(True, False), (False, True), (True, True)])
def test_envelope_and_scalar_features(dtype, env, l0):
    ir = "16x0e+16x1o+16x2e"
    run_case(ir, ir, ir, uuu_paths(ir, ir, ir), 11, 60, dtype, 5, env=env, l0=l0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_unweighted_and_mixed_paths(dtype):
    """has_weight=False paths use weight 1 and own no weight columns (only UUU allows them)."""
    ir = "16x0e+16x1o"
    paths = uuu_paths(ir, ir, ir, unweighted=(0, 3))
    run_case(ir, ir, ir, paths, 9, 40, dtype, 11, env=True, l0=True)
    # No weighted path at all: weight_numel == 0 and the weight is never used.
    unweighted = [p[:4] + (False,) for p in paths]
    conv = make(ir, ir, ir, unweighted, dtype)
    assert conv.weight_numel == 0
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(9, 64, generator=gen, dtype=torch.float64, requires_grad=True)
    y = torch.randn(40, 64, generator=gen, dtype=torch.float64, requires_grad=True)
    src, dst = random_graph(9, 40, gen)
    ref = oracle_conv(ir, ir, ir, unweighted, x, y, torch.zeros(40, 0, dtype=torch.float64), src, dst, 9)
    dx, dy = (t.detach().to(DEV, dtype).requires_grad_() for t in (x, y))
    out = conv(dx, dy, None, graph=conv.create_graph(src.to(DEV), dst.to(DEV), 9))
    assert_close(out, ref, dtype, "unweighted forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    for a, r, what in zip(torch.autograd.grad(out, (dx, dy), g.to(DEV, dtype)),
                          torch.autograd.grad(ref, (x, y), g), ("gx", "gy")):
        assert_close(a, r, dtype, "unweighted " + what)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("lmax", [2, 3])
def test_full_irreps(dtype, lmax):
    """Every allowed path up to lmax on 64 channels (the reference's UUU benchmark layout)."""
    ir = irreps(64, lmax)
    run_case(ir, ir, ir, uuu_paths(ir, ir, ir), 30, 200, dtype, lmax, env=lmax == 3, orders=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_distinct_irreps_and_channel_counts(dtype):
    """Different x / y / out layouts, blocks of different channel counts, uncovered outputs."""
    in1, in2, out = "8x0e+24x1o+8x2e", "8x1o+24x0e+8x2e", "8x1o+24x1o+8x0e+3x0e"
    run_case(in1, in2, out, uuu_paths(in1, in2, out), 13, 70, dtype, 21, env=True, l0=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_backward_cut_into_phases(dtype):
    """lmax 4 on 64 channels exceeds one wave body's register estimate: the backward
    runs its input blocks in several launches that add into the shared gy blocks."""
    ir = irreps(64, 4)
    run_case(ir, ir, ir, uuu_paths(ir, ir, ir), 12, 50, dtype, 4, env=True, orders=1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_empty_graph_and_isolated_nodes(dtype):
    ir = "32x0e+32x1o"
    conv = make(ir, ir, ir, uuu_paths(ir, ir, ir), dtype)
    x = torch.randn(7, conv.irreps_in1.dim, device=DEV, dtype=dtype, requires_grad=True)
    y = torch.randn(0, conv.irreps_in2.dim, device=DEV, dtype=dtype, requires_grad=True)
    w = torch.randn(0, conv.weight_numel, device=DEV, dtype=dtype, requires_grad=True)
    empty = torch.zeros(0, dtype=torch.int64, device=DEV)
    out = conv(x, y, w, graph=conv.create_graph(empty, empty, 7))
    assert out.shape == (7, conv.irreps_out.dim) and not out.count_nonzero()
    for value, grad in zip((x, y, w), torch.autograd.grad(out.sum(), (x, y, w))):
        assert grad.shape == value.shape and not grad.count_nonzero()
    # Nodes 1, 3, 5 have neither in- nor out-edges.
    src, dst = torch.tensor([0, 2, 4, 6, 0]), torch.tensor([0, 0, 2, 4, 6])
    gen = torch.Generator().manual_seed(3)
    xs = torch.randn(7, conv.irreps_in1.dim, generator=gen, dtype=torch.float64)
    ys = torch.randn(5, conv.irreps_in2.dim, generator=gen, dtype=torch.float64)
    ws = torch.randn(5, conv.weight_numel, generator=gen, dtype=torch.float64)
    check_orders(conv, ir, ir, ir, uuu_paths(ir, ir, ir), xs, ys, ws, src, dst, 7, dtype, gen, orders=2)


def test_shared_and_absent_weights():
    """Shared weights [weight_numel] expand to every edge; weight=None needs weight_numel == 0."""
    ir = "16x0e+16x1o"
    paths = uuu_paths(ir, ir, ir)
    conv = make(ir, ir, ir, paths, torch.float64)
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(6, conv.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(20, conv.irreps_in2.dim, generator=gen, dtype=torch.float64)
    shared = torch.randn(conv.weight_numel, generator=gen, dtype=torch.float64)
    src, dst = random_graph(6, 20, gen)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), 6)
    sw = shared.to(DEV).requires_grad_()
    out = conv(x.to(DEV), y.to(DEV), sw, graph=graph)
    ref_w = shared.clone().requires_grad_()
    ref = oracle_conv(ir, ir, ir, paths, x, y, ref_w.expand(20, -1), src, dst, 6)
    assert_close(out, ref, torch.float64, "shared forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    (gw,) = torch.autograd.grad(out, sw, g.to(DEV))
    (rw,) = torch.autograd.grad(ref, ref_w, g)
    assert_close(gw, rw, torch.float64, "shared weight gradient")
    with pytest.raises(ValueError, match="requires weights"):
        conv(x.to(DEV), y.to(DEV), None, graph=graph)
    unweighted = [p[:4] + (False,) for p in paths]
    free = make(ir, ir, ir, unweighted, torch.float64)
    assert free.weight_numel == 0
    out = free(x.to(DEV), y.to(DEV), None, graph=graph)
    ref = oracle_conv(ir, ir, ir, unweighted, x, y, torch.zeros(20, 0, dtype=torch.float64), src, dst, 6)
    assert_close(out, ref, torch.float64, "unweighted forward")


def test_fp64_gradcheck():
    ir = "4x0e+4x1o"
    conv = make(ir, ir, ir, uuu_paths(ir, ir, ir), torch.float64)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(5, conv.irreps_in1.dim, generator=gen, dtype=torch.float64).to(DEV).requires_grad_()
    y = torch.randn(12, conv.irreps_in2.dim, generator=gen, dtype=torch.float64).to(DEV).requires_grad_()
    w = torch.randn(12, conv.weight_numel, generator=gen, dtype=torch.float64).to(DEV).requires_grad_()
    src, dst = random_graph(5, 12, gen)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), 5)
    fn = lambda a, b, c: conv(a, b, c, graph=graph)  # noqa: E731
    assert torch.autograd.gradcheck(fn, (x, y, w), eps=1e-6, atol=1e-5, rtol=1e-4, nondet_tol=1e-12)
    assert torch.autograd.gradgradcheck(fn, (x, y, w), eps=1e-6, atol=1e-5, rtol=1e-4, nondet_tol=1e-12)


def test_prebuilt_metadata_and_compile_op():
    """mode="uuu" metadata, prepare_tensor_product(convolution=True) and the dispatcher op."""
    from lunaequivariance_amd import ops
    from lunaequivariance_amd.uuu_conv import build_uuu_conv_metadata

    ir = "16x0e+16x1o"
    paths = uuu_paths(ir, ir, ir)
    tp = lunaeq.TensorProductConfig(ir, ir, ir, paths, internal_weights=False, shared_weights=False)
    meta = build_uuu_conv_metadata(tp)
    conv = lunaeq.TensorProductConv(meta, mode="uuu")
    prepared = lunaeq.prepare_tensor_product(ir, ir, ir, paths, convolution=True)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(6, 64, generator=gen).to(DEV)
    y = torch.randn(20, 64, generator=gen).to(DEV)
    w = torch.randn(20, tp.weight_numel, generator=gen).to(DEV)
    src, dst = random_graph(6, 20, gen)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), 6)
    a = conv(x, y, w, graph=graph)
    b = lunaeq.tensor_product_conv(x, y, w, graph=graph, config=prepared)
    c, _ = torch.ops.lunatp.uuu_conv_forward.default(x, y, w, None, ops.graph_tables(graph), 6, False,
                                                 prepared.torch_config)
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("nodes", [300, 3000, 9000])
def test_waves_per_node(dtype, nodes):
    """Few nodes give each node several waves (8 at 300 nodes, 4 at 3,000) that
    split its edges and sum through LDS; 9,000 nodes run one wave per node."""
    ir = "16x0e+16x1o"
    run_case(ir, ir, ir, uuu_paths(ir, ir, ir), nodes, 4 * nodes, dtype, nodes, env=True, orders=1)
