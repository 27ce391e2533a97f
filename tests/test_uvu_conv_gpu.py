"""GPU parity of the HIP UVU convolution against the fp64 CPU oracle.

Tolerance (written here, used everywhere): the maximum absolute error must
not exceed ``rtol * max|reference| + atol`` with (rtol, atol) = (1e-5, 1e-7)
for fp32 and (1e-11, 1e-14) for fp64.  Reference tests use the same
max-norm form (``tests/testing_utils.py:14-41``).
"""

import pytest
import torch

import lunaequivariance_amd as lunaeq
from oracle.uvu_conv import uvu_conv
from tests.conftest import all_uvu_instructions, mace_irreps

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-7), torch.float64: (1e-11, 1e-14)}
DEV = "cuda"


def assert_close(actual, reference, dtype, what=""):
    assert actual.shape == reference.shape, what
    if reference.numel() == 0:
        return
    rtol, atol = TOL[dtype]
    err = (actual.detach().double().cpu() - reference.detach().double().cpu()).abs().max().item()
    limit = rtol * reference.detach().abs().max().item() + atol
    assert err <= limit, f"{what}: max error {err:.3e} > {limit:.3e}"


def make_conv(in1, in2, out, instructions, dtype):
    return lunaeq.TensorProductConv(in1, in2, out, instructions, internal_weights=False,
                                    shared_weights=False, dtype=dtype)


def random_graph(nodes, edges, gen):
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.sort(torch.randint(nodes, (edges,), generator=gen))[0]
    return src, dst


def inputs(conv, nodes, edges, dtype, gen):
    x = torch.randn(nodes, conv.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(edges, conv.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(edges, conv.weight_numel, generator=gen, dtype=torch.float64)
    return x, y, w


def check_orders(conv, in1, in2, out, instructions, x, y, w, src, dst, nodes, dtype, gen,
                 env=None, l0=False, orders=3, normalization=None):
    """Forward and derivatives up to ``orders`` against the oracle's autograd."""
    ref_args = [t.clone().requires_grad_() for t in (x, y, w)]
    ref_env = None if env is None else env.clone().requires_grad_()
    ref = uvu_conv(in1, in2, out, instructions, *ref_args, src, dst, nodes, env=ref_env, return_l0=l0,
                   normalization=normalization)
    ref = ref if isinstance(ref, tuple) else (ref,)
    dev_args = [t.to(DEV, dtype).requires_grad_() for t in (x, y, w)]
    dev_env = None if env is None else env.to(DEV, dtype).requires_grad_()
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    act = conv(*dev_args, graph=graph, env=dev_env, return_l0_feat=l0)
    act = act if isinstance(act, tuple) else (act,)
    for a, r in zip(act, ref):
        assert_close(a, r, dtype, "forward")
    if orders < 1:
        return
    ref_in = ref_args + ([ref_env] if ref_env is not None else [])
    dev_in = dev_args + ([dev_env] if dev_env is not None else [])
    seeds = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in ref]
    ref_seeds = [s.clone().requires_grad_() for s in seeds]
    dev_seeds = [s.to(DEV, dtype).requires_grad_() for s in seeds]
    ref_first = torch.autograd.grad(ref, ref_in, ref_seeds, create_graph=orders > 1)
    dev_first = torch.autograd.grad(act, dev_in, dev_seeds, create_graph=orders > 1)
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert_close(a, r, dtype, f"first-order grad {n}")
    if orders < 2:
        return
    dirs = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in ref_first]
    ref_dirs = [d.clone().requires_grad_() for d in dirs]
    dev_dirs = [d.to(DEV, dtype).requires_grad_() for d in dirs]
    ref_second = torch.autograd.grad(ref_first, ref_in + ref_seeds, ref_dirs, create_graph=orders > 2,
                                     allow_unused=True)
    dev_second = torch.autograd.grad(dev_first, dev_in + dev_seeds, dev_dirs, create_graph=orders > 2,
                                     allow_unused=True)
    for n, (a, r) in enumerate(zip(dev_second, ref_second)):
        if r is None:
            assert a is None or not a.count_nonzero()
            continue
        assert_close(torch.zeros_like(r) if a is None else a, r, dtype, f"second-order grad {n}")
    if orders < 3:
        return
    pairs = [(a, r) for a, r in zip(dev_second, ref_second) if r is not None and r.requires_grad]
    s2 = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for _, r in pairs]
    targets_ref = ref_in + ref_seeds + ref_dirs
    targets_dev = dev_in + dev_seeds + dev_dirs
    ref_third = torch.autograd.grad([r for _, r in pairs], targets_ref, s2, allow_unused=True)
    dev_third = torch.autograd.grad([a for a, _ in pairs], targets_dev, [s.to(DEV, dtype) for s in s2],
                                    allow_unused=True)
    for n, (a, r) in enumerate(zip(dev_third, ref_third)):
        if r is None:
            assert a is None or not a.count_nonzero()
            continue
        assert_close(torch.zeros_like(r) if a is None else a, r, dtype, f"third-order grad {n}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_reference_problem_all_orders(make_problem, dtype):
    tp, instructions, x, y, w, src, dst = make_problem()
    conv = lunaeq.TensorProductConv(tp, dtype=dtype)
    gen = torch.Generator().manual_seed(5)
    check_orders(conv, "32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o", instructions, x, y, w, src, dst,
                 7, dtype, gen)


def test_config1_closed_form():
    """32x1o x 1x1o -> 32x0e: message = w * <x_src, y> / sqrt(3) (examples/basic_uvu_conv.py:33-41)."""
    gen = torch.Generator().manual_seed(0)
    conv = make_conv("32x1o", "1x1o", "32x0e", [(0, 0, 0, "uvu", True)], torch.float32)
    nodes, edges = 1000, 16000
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.arange(nodes).repeat_interleave(16)
    x = torch.randn(nodes, 96, generator=gen, dtype=torch.float64)
    v = torch.randn(edges, 3, generator=gen, dtype=torch.float64)
    y = v / v.norm(dim=1, keepdim=True)
    w = torch.randn(edges, 32, generator=gen, dtype=torch.float64)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    out = conv(x.to(DEV, torch.float32), y.to(DEV, torch.float32), w.to(DEV, torch.float32), graph=graph)
    msg = (x[src].reshape(edges, 32, 3) * y[:, None, :]).sum(-1) * w / 3 ** 0.5
    ref = torch.zeros(nodes, 32, dtype=torch.float64).index_add(0, dst, msg)
    assert_close(out, ref, torch.float32, "config 1")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("env_shape", [None, (19,), (19, 1)])
@pytest.mark.parametrize("l0", [False, True])
def test_envelope_and_scalar_features(make_problem, dtype, env_shape, l0):
    tp, instructions, x, y, w, src, dst = make_problem()
    conv = lunaeq.TensorProductConv(tp, dtype=dtype)
    gen = torch.Generator().manual_seed(11)
    env = None if env_shape is None else torch.rand(env_shape, generator=gen, dtype=torch.float64)
    check_orders(conv, "32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o", instructions, x, y, w, src, dst,
                 7, dtype, gen, env=env, l0=l0, orders=2)


def shape_problem(channels):
    """``tests/lunatp/test_uvu_conv.py:378-452``: edge multiplicity > 1, repeated
    instructions and two instructions summed into one output block."""
    in1 = f"{channels}x0e + {channels}x1o + 1x2e"
    in2 = "2x0e + 3x1o + 1x2e"
    out = f"{channels}x0e + {channels}x1o + 1x2e"
    instructions = [(0, 0, 0, "uvu", True), (0, 0, 0, "uvu", True), (1, 1, 0, "uvu", True),
                    (0, 1, 1, "uvu", True), (1, 0, 1, "uvu", True)]
    src = torch.tensor([1, 0, 1, 2, 0, 1, 2, 0, 1])
    dst = torch.tensor([0, 0, 0, 1, 1, 1, 2, 2, 2])
    return in1, in2, out, instructions, src, dst


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("channels", [1, 33, 1025])
@pytest.mark.parametrize("feature", ["ordinary", "envelope", "l0"])
def test_nonunit_edge_multiplicity(dtype, channels, feature):
    in1, in2, out, instructions, src, dst = shape_problem(channels)
    conv = make_conv(in1, in2, out, instructions, dtype)
    gen = torch.Generator().manual_seed(72619)
    x, y, w = inputs(conv, 5, 9, dtype, gen)
    env = torch.randn(9, 1, generator=gen, dtype=torch.float64) if feature == "envelope" else None
    check_orders(conv, in1, in2, out, instructions, x, y, w, src, dst, 5, dtype, gen, env=env,
                 l0=feature == "l0", orders=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_empty_graph(dtype):
    conv = make_conv("32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o",
                     all_uvu_instructions("32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o"), dtype)
    x = torch.randn(7, conv.irreps_in1.dim, device=DEV, dtype=dtype, requires_grad=True)
    y = torch.randn(0, 4, device=DEV, dtype=dtype, requires_grad=True)
    w = torch.randn(0, conv.weight_numel, device=DEV, dtype=dtype, requires_grad=True)
    empty = torch.zeros(0, dtype=torch.int64, device=DEV)
    graph = conv.create_graph(empty, empty, 7)
    out = conv(x, y, w, graph=graph)
    assert out.shape == (7, conv.irreps_out.dim) and not out.count_nonzero()
    grads = torch.autograd.grad(out.sum(), (x, y, w))
    for value, grad in zip((x, y, w), grads):
        assert grad.shape == value.shape and not grad.count_nonzero()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("lmax", [2, 3])
def test_mace_style_paths(dtype, lmax):
    """All uvu paths up to lmax (one output block per path), 16 channels, random graph."""
    in1, sh, out, instructions = mace_irreps(16, lmax)
    conv = make_conv(in1, sh, out, instructions, dtype)
    gen = torch.Generator().manual_seed(3)
    nodes, edges = 40, 300
    src, dst = random_graph(nodes, edges, gen)
    x, y, w = inputs(conv, nodes, edges, dtype, gen)
    check_orders(conv, in1, sh, out, instructions, x, y, w, src, dst, nodes, dtype, gen, orders=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_merged_outputs_collision(dtype):
    """MACE with merged outputs: several instructions sum into one output block."""
    in1, sh = "8x0e+8x1o+8x2e", "1x0e+1x1o+1x2e"
    out = "8x0e+8x1o+8x2e+8x1e+8x2o"
    instructions = all_uvu_instructions(in1, sh, out)
    conv = make_conv(in1, sh, out, instructions, dtype)
    assert conv.op.plan.info.fwd_needs_zero
    gen = torch.Generator().manual_seed(4)
    nodes, edges = 30, 200
    src, dst = random_graph(nodes, edges, gen)
    x, y, w = inputs(conv, nodes, edges, dtype, gen)
    check_orders(conv, in1, sh, out, instructions, x, y, w, src, dst, nodes, dtype, gen, orders=2)


def test_isolated_nodes_and_unsorted_sources():
    """Nodes with no in- or out-edges produce zero rows and zero gradients."""
    dtype = torch.float32
    in1, sh, out, instructions = mace_irreps(8, 2)
    conv = make_conv(in1, sh, out, instructions, dtype)
    gen = torch.Generator().manual_seed(9)
    nodes = 50
    src = torch.randint(0, 10, (60,), generator=gen)
    dst = torch.sort(torch.randint(20, 30, (60,), generator=gen))[0]
    x, y, w = inputs(conv, nodes, 60, dtype, gen)
    check_orders(conv, in1, sh, out, instructions, x, y, w, src, dst, nodes, dtype, gen, orders=1)


def test_non_default_stream():
    dtype = torch.float32
    in1, sh, out, instructions = mace_irreps(8, 1)
    conv = make_conv(in1, sh, out, instructions, dtype)
    gen = torch.Generator().manual_seed(1)
    src, dst = random_graph(20, 100, gen)
    x, y, w = inputs(conv, 20, 100, dtype, gen)
    ref = uvu_conv(in1, sh, out, instructions, x, y, w, src, dst, 20)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), 20)
    stream = torch.cuda.Stream()
    xd, yd, wd = (t.to(DEV, dtype) for t in (x, y, w))
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        result = conv(xd, yd, wd, graph=graph)
    stream.synchronize()
    assert_close(result, ref, dtype, "non-default stream")


def load_golden(name):
    import json
    from pathlib import Path

    import numpy as np

    data = np.load(Path(__file__).resolve().parent / "golden" / f"{name}.npz")
    meta = json.loads(str(data["meta"]))
    meta["instructions"] = [tuple(i) for i in meta["instructions"]]
    return meta, {k: torch.tensor(data[k]) for k in data.files if k != "meta"}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("name", ["reference_problem", "config1_small", "multi_edge_env", "lmax3_paths",
                                  "uuu_reference", "uvw_reference"])
def test_golden_fixtures(name, dtype):
    """HIP forward, first and second order against the committed oracle fixtures."""
    meta, t = load_golden(name)
    conv = make_conv(meta["in1"], meta["in2"], meta["out"], meta["instructions"], dtype)
    graph = conv.create_graph(t["src"].to(DEV), t["dst"].to(DEV), meta["nodes"])
    leaves = [t[k].to(DEV, dtype).requires_grad_() for k in ("x", "y", "w")]
    env = t["env"].to(DEV, dtype) if "env" in t else None
    out = conv(*leaves, graph=graph, env=env)
    assert_close(out, t["out"], dtype, "forward")
    first = torch.autograd.grad(out, leaves, t["g"].to(DEV, dtype), create_graph=True)
    for a, k in zip(first, ("gx", "gy", "gw")):
        assert_close(a, t[k], dtype, k)
    second = torch.autograd.grad(first, leaves, tuple(t[k].to(DEV, dtype) for k in ("rx", "ry", "rw")))
    for a, k in zip(second, ("hx", "hy", "hw")):
        assert_close(a, t[k], dtype, k)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_full_size_sampled_rows(dtype):
    """Config 2 (fp32) / config 3 (fp64) at full size: outputs and gradients of
    sampled nodes and edges against the oracle evaluated on just those rows,
    plus exact linearity of the forward in the weights."""
    from lunaequivariance_amd.workloads import mace_irreps, periodic_radius_graph, spherical_harmonics

    in1, sh, out, instructions = mace_irreps(128, 3)
    conv = make_conv(in1, sh, out, instructions, dtype)
    N = 20000
    src, dst, _, vec, _ = periodic_radius_graph(N, 0.1, 5.0, seed=0, device=DEV)
    E = src.numel()
    assert E > 1_000_000
    graph = conv.create_graph(src, dst, N)
    gen = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(N, conv.irreps_in1.dim, device=DEV, dtype=dtype, generator=gen).requires_grad_()
    y = spherical_harmonics(3, vec).to(dtype).requires_grad_()
    w = (torch.randn(E, conv.weight_numel, device=DEV, dtype=dtype, generator=gen) / 34 ** 0.5).requires_grad_()
    g = torch.randn(N, conv.irreps_out.dim, device=DEV, dtype=dtype, generator=gen)
    result = conv(x, y, w, graph=graph)
    gx, gy, gw = torch.autograd.grad(result, (x, y, w), g)
    with torch.no_grad():
        doubled = conv(x, y, 2 * w, graph=graph)
        assert torch.equal(doubled, 2 * result), "forward is not exactly linear in w"
    pick = torch.randperm(N, generator=torch.Generator().manual_seed(1))[:12]
    src_c, dst_c = src.cpu(), dst.cpu()
    x64, y64, w64, g64 = (t.detach().double().cpu() for t in (x, y, w, g))
    # Destination rows: forward, gw and gy of their in-edges.
    for node in pick.tolist():
        edges = torch.nonzero(dst_c == node).flatten()
        local_dst = torch.zeros(len(edges), dtype=torch.long)
        leaves = [x64.clone().requires_grad_(), y64[edges].clone().requires_grad_(),
                  w64[edges].clone().requires_grad_()]
        ref = uvu_conv(in1, sh, out, instructions, leaves[0], leaves[1], leaves[2], src_c[edges], local_dst, 1)
        assert_close(result[node:node + 1], ref, dtype, f"out[{node}]")
        rgx, rgy, rgw = torch.autograd.grad(ref, leaves, g64[node:node + 1])
        assert_close(gy[edges.to(DEV)], rgy, dtype, f"gy of edges into {node}")
        assert_close(gw[edges.to(DEV)], rgw, dtype, f"gw of edges into {node}")
    # Source rows: gx sums the messages of a node's out-edges.
    for node in pick[:4].tolist():
        edges = torch.nonzero(src_c == node).flatten()
        targets, local_dst = torch.unique(dst_c[edges], return_inverse=True)
        xs = x64.clone().requires_grad_()
        ref = uvu_conv(in1, sh, out, instructions, xs, y64[edges], w64[edges], src_c[edges], local_dst,
                       len(targets))
        (rgx,) = torch.autograd.grad(ref, xs, g64[targets])
        assert_close(gx[node:node + 1], rgx[node:node + 1], dtype, f"gx[{node}]")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_lmax3_split_groups_with_envelope_and_scalar_features(dtype):
    """The lmax-3 layout, whose fp64 backward splits input blocks into two path
    subsets that combine their gy partials (env column included) in LDS, with an
    envelope and the scalar-path features (gl0 enters the per-edge seeds)."""
    in1, sh, out, instructions = mace_irreps(16, 3)
    conv = make_conv(in1, sh, out, instructions, dtype)
    gen = torch.Generator().manual_seed(33)
    nodes, edges = 30, 200
    src, dst = random_graph(nodes, edges, gen)
    x, y, w = inputs(conv, nodes, edges, dtype, gen)
    env = torch.rand(edges, 1, generator=gen, dtype=torch.float64)
    check_orders(conv, in1, sh, out, instructions, x, y, w, src, dst, nodes, dtype, gen, env=env, l0=True,
                 orders=2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_wide_mixed_width_edge_channels(dtype):
    """Blocks of 65,537 and 65,601 channels, several edge channels, a repeated
    instruction, env with zeros and scalar features (``tests/lunatp/test_uvu_conv.py:500-575``)."""
    in1, sh = "65537x0e+65601x1o+1x2e", "2x0e+3x1o+1x2e"
    out = "65537x0e+65601x0e+65537x1o+65601x1o+1x2e"
    instructions = [(0, 0, 0, "uvu", True), (0, 0, 0, "uvu", True), (1, 1, 1, "uvu", True),
                    (0, 1, 2, "uvu", True), (1, 0, 3, "uvu", True)]
    conv = make_conv(in1, sh, out, instructions, dtype)
    gen = torch.Generator().manual_seed(92671)
    src, dst = torch.tensor([1, 0, 1, 0]), torch.tensor([0, 0, 1, 1])
    x, y, w = inputs(conv, 3, 4, dtype, gen)
    env = torch.tensor([0.0, 0.5, -1.0, 0.0], dtype=torch.float64)
    check_orders(conv, in1, sh, out, instructions, x, y, w, src, dst, 3, dtype, gen, env=env, l0=True, orders=2)


def test_graph_capture_replays():
    """Forward and first-order backward captured in a HIP graph and replayed with new
    inputs each time, every replay against eager (``tests/lunatp/test_uvu_conv.py:933-995``)."""
    dtype = torch.float32
    in1, sh, out, instructions = mace_irreps(16, 2)
    conv = make_conv(in1, sh, out, instructions, dtype)
    gen = torch.Generator().manual_seed(12)
    src, dst = random_graph(40, 300, gen)
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), 40)
    x, y, w = (t.to(DEV, dtype) for t in inputs(conv, 40, 300, dtype, gen))
    g = torch.randn(40, conv.irreps_out.dim, generator=gen).to(DEV)
    sx, sy, sw, sg = (t.clone().requires_grad_(t is not g) if t is not g else t.clone() for t in (x, y, w, g))

    def step():
        o = conv(sx, sy, sw, graph=graph)
        return (o, *torch.autograd.grad(o, (sx, sy, sw), sg))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    captured = torch.cuda.CUDAGraph()
    with torch.cuda.graph(captured):
        static = step()
    for replay in range(3):
        nx, ny, nw, ng = (torch.randn(t.shape, generator=gen).to(DEV) for t in (x, y, w, g))
        with torch.no_grad():
            sx.copy_(nx)
            sy.copy_(ny)
            sw.copy_(nw)
            sg.copy_(ng)
        captured.replay()
        torch.cuda.synchronize()
        ex, ey, ew = (t.clone().requires_grad_() for t in (nx, ny, nw))
        eo = conv(ex, ey, ew, graph=graph)
        expected = (eo, *torch.autograd.grad(eo, (ex, ey, ew), ng))
        for n, (a, b) in enumerate(zip(static, expected)):
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-6), f"replay {replay}, output {n}"


@pytest.mark.parametrize("irrep_norm,path_norm", [("norm", "path"), ("component", "none"), ("none", "element")])
def test_nondefault_normalisation_and_variances(irrep_norm, path_norm):
    """Path weights from non-default normalisation and non-unit variances
    (src/lunatp/utils/layout.py:323-370) reach the kernels: parity to second order."""
    in1, sh, out = "8x0e+8x1o+8x2e", "2x0e+2x1o", "8x0e+8x1o+8x2e+8x1e"
    instructions = all_uvu_instructions(in1, sh, out)
    variances = dict(in1_var=[0.5, 2.0, 3.0], in2_var=[1.5, 0.25], out_var=[2.0, 0.5, 4.0, 1.25])
    norm = dict(irrep_normalization=irrep_norm, path_normalization=path_norm)
    conv = lunaeq.TensorProductConv(in1, sh, out, instructions, internal_weights=False, shared_weights=False,
                                    dtype=torch.float32, **norm, **variances)
    gen = torch.Generator().manual_seed(21)
    nodes, edges = 9, 40
    src, dst = random_graph(nodes, edges, gen)
    x, y, w = inputs(conv, nodes, edges, torch.float32, gen)
    check_orders(conv, in1, sh, out, instructions, x, y, w, src, dst, nodes, torch.float32, gen, orders=2,
                 normalization=dict(norm, **variances))


def test_cfg4_layout_force_training_small():
    """Config 4's layer (64 channels, lmax 3, every uvu path, fp32): forward, first order
    and the force-training double backward d<ry, gy>/d(x, w) against the oracle."""
    from lunaequivariance_amd.workloads import mace_irreps

    in1, sh, out, instructions = mace_irreps(64, 3)
    conv = make_conv(in1, sh, out, instructions, torch.float32)
    gen = torch.Generator().manual_seed(44)
    nodes, edges = 11, 70
    src, dst = random_graph(nodes, edges, gen)
    x, y, w = inputs(conv, nodes, edges, torch.float32, gen)
    g = torch.randn(nodes, conv.irreps_out.dim, generator=gen, dtype=torch.float64)
    ry = torch.randn(edges, conv.irreps_in2.dim, generator=gen, dtype=torch.float64)
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ref = uvu_conv(in1, sh, out, instructions, *ref_in, src, dst, nodes)
    rgx, rgy, rgw = torch.autograd.grad(ref, ref_in, g, create_graph=True)
    rhx, rhw = torch.autograd.grad(rgy, (ref_in[0], ref_in[2]), ry)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    graph = conv.create_graph(src.to(DEV), dst.to(DEV), nodes)
    act = conv(*dev_in, graph=graph)
    gx, gy, gw = torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32), create_graph=True)
    hx, hw = torch.autograd.grad(gy, (dev_in[0], dev_in[2]), ry.to(DEV, torch.float32))
    for a, r, name in ((act, ref, "out"), (gx, rgx, "gx"), (gy, rgy, "gy"), (gw, rgw, "gw"),
                       (hx, rhx, "hx"), (hw, rhw, "hw")):
        assert_close(a, r, torch.float32, name)


def test_cfg4_full_size_sampled_rows():
    """Config 4 at full size (10,000 atoms, ~520k edges, 64 channels, fp32): the bench's
    force-training step, checked on sampled destination rows (out, gy, gw, hw) and
    source rows (gx, hx) against the oracle evaluated on just those rows."""
    from lunaequivariance_amd.workloads import mace_irreps, periodic_radius_graph, spherical_harmonics

    dtype = torch.float32
    in1, sh, out, instructions = mace_irreps(64, 3)
    conv = make_conv(in1, sh, out, instructions, dtype)
    N = 10000
    src, dst, _, vec, _ = periodic_radius_graph(N, 0.1, 5.0, seed=0, device=DEV)
    E = src.numel()
    assert 500_000 < E < 545_000
    graph = conv.create_graph(src, dst, N)
    gen = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(N, conv.irreps_in1.dim, device=DEV, dtype=dtype, generator=gen).requires_grad_()
    y = spherical_harmonics(3, vec).to(dtype).requires_grad_()
    w = (torch.randn(E, conv.weight_numel, device=DEV, dtype=dtype, generator=gen) / 34 ** 0.5).requires_grad_()
    g = torch.randn(N, conv.irreps_out.dim, device=DEV, dtype=dtype, generator=gen)
    ry = torch.randn(E, conv.irreps_in2.dim, device=DEV, dtype=dtype, generator=gen)
    result = conv(x, y, w, graph=graph)
    gx, gy, gw = torch.autograd.grad(result, (x, y, w), g, create_graph=True)
    hx, hw = torch.autograd.grad(gy, (x, w), ry)
    pick = torch.randperm(N, generator=torch.Generator().manual_seed(2))[:8]
    src_c, dst_c = src.cpu(), dst.cpu()
    x64, y64, w64, g64, ry64 = (t.detach().double().cpu() for t in (x, y, w, g, ry))
    for node in pick.tolist():
        edges = torch.nonzero(dst_c == node).flatten()
        local_dst = torch.zeros(len(edges), dtype=torch.long)
        leaves = [x64.clone().requires_grad_(), y64[edges].clone().requires_grad_(),
                  w64[edges].clone().requires_grad_()]
        ref = uvu_conv(in1, sh, out, instructions, *leaves, src_c[edges], local_dst, 1)
        assert_close(result[node:node + 1], ref, dtype, f"out[{node}]")
        rgx, rgy, rgw = torch.autograd.grad(ref, leaves, g64[node:node + 1], create_graph=True)
        assert_close(gy[edges.to(DEV)], rgy, dtype, f"gy of edges into {node}")
        assert_close(gw[edges.to(DEV)], rgw, dtype, f"gw of edges into {node}")
        (rhw,) = torch.autograd.grad(rgy, leaves[2], ry64[edges])
        assert_close(hw[edges.to(DEV)], rhw, dtype, f"hw of edges into {node}")
    for node in pick[:4].tolist():
        edges = torch.nonzero(src_c == node).flatten()
        targets, local_dst = torch.unique(dst_c[edges], return_inverse=True)
        xs = x64.clone().requires_grad_()
        ys = y64[edges].clone().requires_grad_()
        ref = uvu_conv(in1, sh, out, instructions, xs, ys, w64[edges], src_c[edges], local_dst, len(targets))
        rgx, rgy = torch.autograd.grad(ref, (xs, ys), g64[targets], create_graph=True)
        assert_close(gx[node:node + 1], rgx[node:node + 1], dtype, f"gx[{node}]")
        (rhx,) = torch.autograd.grad(rgy, xs, ry64[edges])
        assert_close(hx[node:node + 1], rhx[node:node + 1], dtype, f"hx[{node}]")
