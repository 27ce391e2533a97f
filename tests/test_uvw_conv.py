"""UVW convolution on the CPU: the oracle's uvw branch against fixed facts and the lowering.

The oracle's uvw conv branch is pinned by its scalar-loop brute force, by the
identity "convolution over a graph in which every edge has its own
destination = the row-wise UVW product" against the separately pinned
``oracle/uvw.py`` (itself pinned by tests/test_oracle_uvw.py), by linearity
(shared weights = the shared row repeated per edge), rotation equivariance
and gradcheck / gradgradcheck.
"""

import numpy as np
import pytest
import torch

from oracle.uvu_conv import brute_force, conv, parse_irreps
from oracle.uvw import uvw_tensor_product
from tests.test_oracle_conv import block_diag_d, rotation


def uvw_paths(in1, in2, out):
    from lunaequivariance_amd import Irreps

    a, b, c = Irreps(in1), Irreps(in2), Irreps(out)
    return [(i, j, k, "uvw", True) for i, (_, x) in enumerate(a) for j, (_, y) in enumerate(b)
            for k, (_, z) in enumerate(c) if z in x * y]


def dims(*texts):
    return [sum(m * (2 * l + 1) for m, l, _ in parse_irreps(t)) for t in texts]


def weight_numel(in1, in2, out, instructions):
    a, b, c = parse_irreps(in1), parse_irreps(in2), parse_irreps(out)
    return sum(a[i][0] * b[j][0] * c[k][0] for i, j, k, *_ in instructions)


def problem(in1, in2, out, instructions, nodes, edges, seed):
    gen = torch.Generator().manual_seed(seed)
    d1, d2, _ = dims(in1, in2, out)
    x = torch.randn(nodes, d1, generator=gen, dtype=torch.float64)
    y = torch.randn(edges, d2, generator=gen, dtype=torch.float64)
    w = torch.randn(edges, weight_numel(in1, in2, out, instructions), generator=gen, dtype=torch.float64)
    src = torch.randint(nodes, (edges,), generator=gen)
    dst = torch.sort(torch.randint(nodes, (edges,), generator=gen))[0]
    return x, y, w, src, dst


IN1, IN2, OUT = "3x0e+2x1o", "2x0e+1x1o", "2x0e+3x1o+1x2e"


def test_oracle_matches_brute_force():
    ins = uvw_paths(IN1, IN2, OUT)
    x, y, w, src, dst = problem(IN1, IN2, OUT, ins, 4, 9, 0)
    dense = conv(IN1, IN2, OUT, ins, x, y, w, src, dst, 4)
    loops = brute_force(IN1, IN2, OUT, ins, x, y, w, src.numpy(), dst.numpy(), 4)
    assert np.allclose(dense.numpy(), loops, atol=1e-12)


def test_edge_own_destination_is_the_row_product():
    ins = uvw_paths(IN1, IN2, OUT)
    x, y, w, _, _ = problem(IN1, IN2, OUT, ins, 6, 6, 1)
    shared = w[0]
    ident = torch.arange(6)
    out = conv(IN1, IN2, OUT, ins, x, y, shared.expand(6, -1), ident, ident, 6)
    rows = uvw_tensor_product(IN1, IN2, OUT, ins, x, y, shared)
    assert torch.allclose(out, rows, atol=1e-12)


def test_oracle_equivariance_and_gradients():
    ins = uvw_paths(IN1, IN2, OUT)
    x, y, w, src, dst = problem(IN1, IN2, OUT, ins, 5, 12, 2)
    R = rotation(5)
    rng = np.random.default_rng(6)
    D1, D2, D3 = (block_diag_d(t, R, rng) for t in (IN1, IN2, OUT))
    out = conv(IN1, IN2, OUT, ins, x, y, w, src, dst, 5)
    rotated = conv(IN1, IN2, OUT, ins, x @ D1.T, y @ D2.T, w, src, dst, 5)
    assert torch.allclose(rotated, out @ D3.T, atol=1e-10)
    small = "1x0e+1x1o"
    ins = uvw_paths(small, small, small)
    x, y, w, src, dst = problem(small, small, small, ins, 3, 5, 3)
    leaves = [t.clone().requires_grad_() for t in (x, y, w)]
    env = torch.rand(5, dtype=torch.float64, requires_grad=True)
    fn = lambda a, b, c, e: conv(small, small, small, ins, a, b, c, src, dst, 3, env=e)  # noqa: E731
    assert torch.autograd.gradcheck(fn, (*leaves, env))
    assert torch.autograd.gradgradcheck(fn, (*leaves, env))


def test_lowering_and_dispatch():
    import lunaequivariance_amd as lunaeq
    from lunaequivariance_amd.uvw_conv import LunaTPUVWConv

    ins = uvw_paths(IN1, IN2, OUT)
    op = lunaeq.prepare_tensor_product(IN1, IN2, OUT, ins, convolution=True)
    assert isinstance(op, LunaTPUVWConv) and op.weight_mode == "external"
    assert op.weight_numel == weight_numel(IN1, IN2, OUT, ins)
    # one aggregation block per (path, edge channel): mul1 * d3 columns each
    a, b, c = parse_irreps(IN1), parse_irreps(IN2), parse_irreps(OUT)
    expected = sum(a[i][0] * b[j][0] * (2 * c[k][1] + 1) for i, j, k, *_ in ins)
    assert op.aggregate_dim == expected
    assert op.agg.spec.startswith("LUNAUVU2") and op.agg.spec.split("\n")[0].endswith(" 1")
    shared = lunaeq.prepare_tensor_product(IN1, IN2, OUT, ins, convolution=True, shared_weights=True)
    assert shared.weight_mode == "shared"
    module = lunaeq.TensorProductConv("2x0e", "2x0e", "2x0e", [(0, 0, 0, "uvw", True)], dtype=torch.float64)
    assert module.internal_weights and module.shared_weights and module.mode == "uvw_conv"
    assert module.weight is dict(module.named_parameters())["tp.weight"]
    assert module.weight.dtype == torch.float64 and module.op.compute_dtype == torch.float64
    module.float()
    assert module.op.compute_dtype == torch.float32


def test_split_k_weight_gradient(monkeypatch):
    """The node-level GEMM's weight gradient is split over K; values and higher
    derivatives equal the plain product's."""
    from lunaequivariance_amd import uvw_conv
    from lunaequivariance_amd.uvw_conv import _RowsTimesWeight, _split_k_tn

    gen = torch.Generator().manual_seed(9)
    a = torch.randn(10001, 30, generator=gen, dtype=torch.float64)
    b = torch.randn(10001, 7, generator=gen, dtype=torch.float64)
    assert torch.allclose(_split_k_tn(a, b), a.t() @ b, atol=1e-11)
    monkeypatch.setattr(uvw_conv, "SPLIT_K_MIN_ROWS", 16)
    rows = torch.randn(53, 3, generator=gen, dtype=torch.float64, requires_grad=True)
    weight = torch.randn(3, 2, generator=gen, dtype=torch.float64, requires_grad=True)
    assert torch.allclose(_split_k_tn(rows, rows[:, :2]), rows.t() @ rows[:, :2], atol=1e-12)
    assert torch.autograd.gradcheck(_RowsTimesWeight.apply, (rows, weight))
    assert torch.autograd.gradgradcheck(_RowsTimesWeight.apply, (rows, weight))
