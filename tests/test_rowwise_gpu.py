"""Row-wise UVU and UUU tensor products (convolution kernels over the identity graph)
against the fp64 oracle (the convolution oracle with row b's edge going from and to b).

Tolerance as for the convolution tests.  Cases follow the reference's
``tests/lunatp/test_uvu.py`` / ``test_uuu.py`` modes: per-row and shared weights,
internal weights, unweighted UUU paths, fp32 and fp64, two derivative orders.
"""

import pytest
import torch

import lunaequivariance_amd as lunaeq
from oracle.uvu_conv import conv as oracle_conv
from tests.test_uvu_conv_gpu import DEV, assert_close

pytestmark = pytest.mark.gpu


def paths(mode, in1, in2, out, unweighted=()):
    a, b, c = lunaeq.Irreps(in1), lunaeq.Irreps(in2), lunaeq.Irreps(out)
    found = [(i, j, k, mode, True) for i, (m, x) in enumerate(a) for j, (n, y) in enumerate(b)
             for k, (o, z) in enumerate(c) if z in x * y and (mode != "uuu" or m == n == o)]
    return [p[:4] + (False,) if n in unweighted else p for n, p in enumerate(found)]


CASES = {
    "uvu": ("16x0e+16x1o", "1x0e+1x1o", "16x0e+16x1o"),
    "uuu": ("16x0e+16x1o+8x2e", "16x0e+16x1o+8x2e", "16x0e+16x1o+8x2e"),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("mode", ["uvu", "uuu"])
def test_rowwise_two_orders(mode, shared, dtype):
    in1, in2, out = CASES[mode]
    ins = paths(mode, in1, in2, out, unweighted=(1,) if mode == "uuu" else ())
    tp = lunaeq.TensorProduct(in1, in2, out, ins, shared_weights=shared, internal_weights=False, dtype=dtype)
    assert tp.op.compute_dtype == dtype
    rows = 45
    gen = torch.Generator().manual_seed(rows + shared)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn((tp.weight_numel,) if shared else (rows, tp.weight_numel), generator=gen, dtype=torch.float64)
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ids = torch.arange(rows)
    ref = oracle_conv(in1, in2, out, ins, ref_in[0], ref_in[1],
                      ref_in[2].expand(rows, -1) if shared else ref_in[2], ids, ids, rows)
    dev_in = [t.to(DEV, dtype).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert_close(act, ref, dtype, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g, create_graph=True)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, dtype), create_graph=True)
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert_close(a, r, dtype, f"first-order {n}")
    dirs = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in ref_first]
    ref_second = torch.autograd.grad(ref_first, ref_in, dirs, allow_unused=True)
    dev_second = torch.autograd.grad(dev_first, dev_in, [d.to(DEV, dtype) for d in dirs], allow_unused=True)
    for n, (a, r) in enumerate(zip(dev_second, ref_second)):
        if r is None:
            assert a is None or not a.count_nonzero()
            continue
        assert_close(torch.zeros_like(r) if a is None else a, r, dtype, f"second-order {n}")


def test_rowwise_internal_weights_and_functional():
    in1, in2, out = CASES["uuu"]
    ins = paths("uuu", in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, ins, shared_weights=True, internal_weights=True).to(DEV)
    x = torch.randn(20, tp.irreps_in1.dim, device=DEV)
    y = torch.randn(20, tp.irreps_in2.dim, device=DEV)
    out_t = tp(x, y)
    ids = torch.arange(20)
    ref = oracle_conv(in1, in2, out, ins, x.double().cpu(), y.double().cpu(),
                      tp.weight.detach().double().cpu().expand(20, -1), ids, ids, 20)
    assert_close(out_t, ref, torch.float32, "internal weights")
    out_t.sum().backward()
    assert tp.weight.grad is not None and tp.weight.grad.shape == tp.weight.shape
    op = lunaeq.prepare_tensor_product(in1, in2, out, ins, shared_weights=True)
    again = lunaeq.tensor_product(x, y, tp.weight.detach(), config=op)
    assert_close(again, ref, torch.float32, "functional")


def test_uuu_batch_broadcasting():
    """UUU broadcasts leading dimensions (docs/operators/tensor_product.md:108-130 example shapes)."""
    ins = [(0, 0, 0, "uuu", True)]
    tp = lunaeq.TensorProduct("8x1o", "8x1o", "8x0e", ins, shared_weights=False, internal_weights=False)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(4, 1, 24, generator=gen)
    y = torch.randn(1, 3, 24, generator=gen)
    w = torch.randn(4, 3, 8, generator=gen)
    out = tp(x.to(DEV), y.to(DEV), w.to(DEV))
    assert out.shape == (4, 3, 8)
    expected = (x.reshape(4, 1, 8, 3) * y.reshape(1, 3, 8, 3)).sum(-1) * w / 3 ** 0.5
    assert_close(out, expected.double(), torch.float32, "broadcast")


@pytest.mark.parametrize("rows", [0, 1])
@pytest.mark.parametrize("mode", ["uvu", "uuu"])
def test_rowwise_tiny_batches(mode, rows):
    """No rows and one row, shared weights: outputs and first-order gradients."""
    in1, in2, out = CASES[mode]
    ins = paths(mode, in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, ins, shared_weights=True, internal_weights=False)
    gen = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64)
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ids = torch.arange(rows)
    ref = oracle_conv(in1, in2, out, ins, ref_in[0], ref_in[1], ref_in[2].expand(rows, -1), ids, ids, rows)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert act.shape == (rows, tp.irreps_out.dim)
    assert_close(act, ref, torch.float32, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32))
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert a.shape == r.shape
        assert_close(a, r, torch.float32, f"first-order {n}")
